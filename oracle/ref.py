"""ctypes driver of the reference C runtime built into oracle/_ref/libv3ref.so (TEST INFRASTRUCTURE ONLY).

The library is runtime/vault3.c compiled from the reference tree by oracle/Makefile with the shim
in oracle/ref_shim.c.  It is an independent oracle for the whole decode step: Q8_0/Q4_0 row dots
(runtime/vault3.c:499-602), attention (:1958-2032), boundary re-basing and segment eviction
(:1833-1915, 2076-2105), scorer and habituation (:961-977, 2201-2216).
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_ref", "libv3ref.so")


def available() -> bool:
    return os.path.exists(LIB)


def build() -> bool:
    """Build oracle/_ref/libv3ref.so when the reference tree is present; True if the library exists."""
    import subprocess
    if os.path.isdir("/root/reference/runtime"):
        subprocess.run(["make", "-s", "-C", HERE], check=True)
    return available()


_lib = None


def _load():
    global _lib
    if _lib is None:
        lib = C.CDLL(LIB)
        lib.ref_open.restype = C.c_void_p
        lib.ref_open.argtypes = [C.c_char_p, C.c_uint64, C.c_int, C.POINTER(C.c_int)]
        lib.ref_close.argtypes = [C.c_void_p]
        lib.ref_reset.argtypes = [C.c_void_p]
        lib.ref_set_threads.argtypes = [C.c_void_p, C.c_int]
        lib.ref_set_pinned.argtypes = [C.c_void_p, C.c_uint32]
        lib.ref_set_pinned.restype = C.c_int
        lib.ref_step.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p]
        lib.ref_vocab.argtypes = [C.c_void_p]
        lib.ref_vocab.restype = C.c_uint32
        lib.ref_arena_bytes.argtypes = [C.c_void_p]
        lib.ref_arena_bytes.restype = C.c_uint64
        lib.ref_state_info.argtypes = [C.c_void_p] + [C.c_void_p] * 4
        lib.ref_mem_pos.argtypes = [C.c_void_p, C.c_void_p]
        lib.ref_seed_long_context.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint64]
        lib.ref_state_field.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p]
        lib.ref_state_field.restype = C.c_int64
        lib.ref_seed_long_context.restype = C.c_int
        lib.v3_argmax.restype = C.c_uint32
        lib.v3_argmax.argtypes = [C.c_void_p, C.c_uint32]
        lib.v3_sample_topk.restype = C.c_uint32
        lib.v3_sample_topk.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.c_float, C.POINTER(C.c_uint64)]
        lib.ref_state_flags.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]
        lib.ref_set_seg_budget.argtypes = [C.c_void_p, C.c_uint32]
        lib.ref_set_seg_budget.restype = C.c_int
        lib.ref_res_state.argtypes = [C.c_void_p] + [C.c_void_p] * 5
        lib.ref_rings.argtypes = [C.c_void_p] + [C.c_void_p] * 3
        lib.ref_model.restype = C.c_void_p
        lib.ref_model.argtypes = [C.c_void_p]
        lib.ref_gov_size.restype = C.c_uint64
        lib.v3_gov_init.argtypes = [C.c_void_p]
        lib.v3_gov_reset_stream.argtypes = [C.c_void_p]
        lib.v3_gov_add_rule.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t]
        lib.v3_gov_add_rule.restype = C.c_int
        lib.v3_gov_arm_system.argtypes = [C.c_void_p, C.c_char_p, C.c_size_t]
        lib.v3_govern_logits.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
        lib.v3_gov_commit.argtypes = [C.c_void_p, C.c_void_p, C.c_uint32]
        lib.ref_res_load_bank.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32]
        lib.ref_res_load_bank.restype = C.c_int
        lib.ref_res_update.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint64, C.c_uint32,
                                       C.c_void_p, C.c_void_p, C.c_void_p]
        lib.ref_res_update.restype = C.c_int
        lib.ref_spoof.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint64, C.c_uint32]
        lib.ref_spoof.restype = C.c_int
        lib.ref_math.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_uint64]
        lib.ref_seg_update.argtypes = [C.c_void_p, C.c_uint64, C.c_uint32, C.c_uint32, C.c_uint32] + \
            [C.c_void_p] * 3 + [C.c_uint32] + [C.c_void_p] * 9
        lib.ref_seg_update.restype = C.c_int
        _lib = lib
    return _lib


class RefRuntime:
    def __init__(self, vlt3_bytes: bytes, threads: int = 1, verify: bool = True):
        lib = _load()
        err = C.c_int(0)
        self._h = lib.ref_open(vlt3_bytes, len(vlt3_bytes), 1 if verify else 0, C.byref(err))
        if not self._h:
            e = RuntimeError(f"v3_load / v3_state_init failed: {err.value}")
            e.code = err.value
            raise e
        self.vocab = lib.ref_vocab(self._h)
        self.threads = threads
        lib.ref_set_threads(self._h, threads)

    def close(self):
        if getattr(self, "_h", None) and _lib is not None:
            _lib.ref_close(self._h)
        self._h = None

    __del__ = close

    def reset(self):
        _load().ref_reset(self._h)

    def set_pinned(self, n: int) -> None:
        rc = _load().ref_set_pinned(self._h, n)
        if rc:
            raise RuntimeError(f"v3_set_pinned: {rc}")

    def step(self, tok: int, out: np.ndarray | None = None) -> np.ndarray:
        if out is None:
            out = np.empty(self.vocab, dtype=np.float32)
        _load().ref_step(self._h, int(tok), out.ctypes.data)
        return out

    def info(self):
        pos, n_pin, mem, off = C.c_uint64(), C.c_uint32(), C.c_uint32(), C.c_uint32()
        _load().ref_state_info(self._h, C.byref(pos), C.byref(n_pin), C.byref(mem), C.byref(off))
        return dict(pos=pos.value, n_pin=n_pin.value, mem_cnt=mem.value, seg_id_offset=off.value)

    def flags(self):
        lk, ba, nu = C.c_int(), C.c_int(), C.c_uint32()
        _load().ref_state_flags(self._h, C.byref(lk), C.byref(ba), C.byref(nu))
        return dict(pin_locked=bool(lk.value), seg_bias_active=int(ba.value), n_uniq_segs=nu.value)

    def res_state(self):
        """(mem_tok, mem_seg, arch, sup, hop1) over the bank's mem_cnt slots after the last step."""
        n = self.info()["mem_cnt"]
        t, g = np.zeros(max(1, n), dtype=np.uint32), np.zeros(max(1, n), dtype=np.uint32)
        a, s, h = (np.zeros(max(1, n), dtype=np.float32) for _ in range(3))
        _load().ref_res_state(self._h, t.ctypes.data, g.ctypes.data, a.ctypes.data, s.ctypes.data, h.ctypes.data)
        return t[:n], g[:n], a[:n], s[:n], h[:n]

    def rings(self, window: int):
        """(tok_prev, tok_cur, sc_cur) of the state (W slots each)."""
        p, c = np.zeros(window, dtype=np.uint32), np.zeros(window, dtype=np.uint32)
        sc = np.zeros(window, dtype=np.float32)
        _load().ref_rings(self._h, p.ctypes.data, c.ctypes.data, sc.ctypes.data)
        return p, c, sc

    def model_ptr(self) -> int:
        return _load().ref_model(self._h)

    def res_load_bank(self, mem_tok, mem_seg) -> int:
        """rebuild_shingle_index over a constructed bank; returns the number of distinct segments."""
        t = np.ascontiguousarray(mem_tok, dtype=np.uint32)
        g = np.ascontiguousarray(mem_seg, dtype=np.uint32)
        n = _load().ref_res_load_bank(self._h, t.ctypes.data, g.ctypes.data, t.size)
        if n < 0:
            raise RuntimeError("bank larger than the state's segment capacity")
        self._bank_n = t.size
        return n

    def res_update(self, tok_prev, tok_cur, c: int, pos: int, n_pin: int):
        """update_query_resonance on constructed rings: (mode, arch, sup, hop1) over the loaded bank."""
        p = np.ascontiguousarray(tok_prev, dtype=np.uint32)
        q = np.ascontiguousarray(tok_cur, dtype=np.uint32)
        n = max(1, getattr(self, "_bank_n", 0))
        a, s, h = (np.zeros(n, dtype=np.float32) for _ in range(3))
        mode = _load().ref_res_update(self._h, p.ctypes.data, q.ctypes.data, c, pos, n_pin, a.ctypes.data,
                                      s.ctypes.data, h.ctypes.data)
        m = getattr(self, "_bank_n", 0)
        return mode, a[:m], s[:m], h[:m]

    def spoof(self, tok_prev, tok_cur, c: int, pos: int, n_pin: int) -> bool:
        p = np.ascontiguousarray(tok_prev, dtype=np.uint32)
        q = np.ascontiguousarray(tok_cur, dtype=np.uint32)
        return bool(_load().ref_spoof(self._h, p.ctypes.data, q.ctypes.data, c, pos, n_pin))


    def set_seg_budget(self, budget: int) -> None:
        rc = _load().ref_set_seg_budget(self._h, budget)
        if rc:
            raise RuntimeError(f"v3_set_seg_budget: {rc}")

    def mem_pos(self) -> np.ndarray:
        n = self.info()["mem_cnt"]
        out = np.zeros(max(1, n), dtype=np.uint64)
        _load().ref_mem_pos(self._h, out.ctypes.data)
        return out[:n].astype(np.int64)

    FIELDS = ("k_prev", "k_cur", "v_prev", "v_cur", "kraw_prev", "kraw_cur", "k_sink_raw", "k_sink_rot",
              "v_sink", "k_seg_raw", "k_seg_rot", "v_seg")

    def state_field(self, layer: int, name: str, n_kv_heads: int, head_dim: int) -> np.ndarray:
        """One layer's KV field of the runtime state as a [G, rows, D] float32 copy."""
        lib = _load()
        f = self.FIELDS.index(name)
        rows = lib.ref_state_field(self._h, layer, f, None)
        if rows < 0:
            raise RuntimeError(f"ref_state_field({layer}, {name}) rejected")
        out = np.empty((n_kv_heads, rows, head_dim), dtype=np.float32)
        if rows:
            lib.ref_state_field(self._h, layer, f, out.ctypes.data)
        return out

    def seg_update(self, ev: int, n_pin: int, offset: int, budget: int, sc, seg, tok, mem_pos, mem_score, mem_tok,
                   mem_seg):
        """update_segment_bank on constructed rings and bank: ((pos, score, tok, seg) of the new bank,
        new seg-id offset)."""
        sc = np.ascontiguousarray(sc, dtype=np.float32)
        seg = np.ascontiguousarray(seg, dtype=np.uint32)
        tok = np.ascontiguousarray(tok, dtype=np.uint32)
        m = len(mem_pos)
        ip = np.zeros(max(1, m), np.uint64)
        isc = np.zeros(max(1, m), np.float32)
        it = np.zeros(max(1, m), np.uint32)
        ig = np.zeros(max(1, m), np.uint32)
        ip[:m], isc[:m], it[:m], ig[:m] = mem_pos, mem_score, mem_tok, mem_seg
        n = max(1, budget)
        op, osc, ot, og = np.zeros(n, np.uint64), np.zeros(n, np.float32), np.zeros(n, np.uint32), np.zeros(n, np.uint32)
        off = C.c_uint32()
        k = _load().ref_seg_update(self._h, ev, n_pin, offset, budget, sc.ctypes.data, seg.ctypes.data,
                                   tok.ctypes.data, m, ip.ctypes.data, isc.ctypes.data, it.ctypes.data, ig.ctypes.data,
                                   op.ctypes.data, osc.ctypes.data, ot.ctypes.data, og.ctypes.data, C.byref(off))
        if k < 0:
            raise RuntimeError("budget beyond the state's segment capacity")
        return (op[:k].astype(np.int64), osc[:k], ot[:k].astype(np.int64), og[:k].astype(np.int64)), off.value

    def seed_long_context(self, pos: int, n_pin: int, mem_cnt: int, seed: int = 0) -> None:
        rc = _load().ref_seed_long_context(self._h, pos, n_pin, mem_cnt, seed)
        if rc:
            raise RuntimeError("seed_long_context rejected the arguments")


class RefGovernor:
    """The reference's v3_governor (runtime/vault3.c:2888-3193) over a loaded runtime's model."""

    def __init__(self, rt: RefRuntime):
        lib = _load()
        self._rt = rt
        self._m = rt.model_ptr()
        self._buf = C.create_string_buffer(int(lib.ref_gov_size()))
        lib.v3_gov_init(self._buf)

    def arm_system(self, text: bytes) -> None:
        _load().v3_gov_arm_system(self._buf, text, len(text))

    def add_rule(self, pat: bytes) -> int:
        return int(_load().v3_gov_add_rule(self._buf, pat, len(pat)))

    def reset_stream(self) -> None:
        _load().v3_gov_reset_stream(self._buf)

    def govern_logits(self, logits: np.ndarray, top_k_guard: int = 0) -> np.ndarray:
        a = np.ascontiguousarray(logits, dtype=np.float32).copy()
        _load().v3_govern_logits(self._buf, self._m, a.ctypes.data, int(top_k_guard))
        return a

    def commit(self, tid: int) -> None:
        _load().v3_gov_commit(self._buf, self._m, int(tid))


def argmax(logits: np.ndarray) -> int:
    """The reference's v3_argmax (runtime/vault3.c:3198-3202) on one fp32 row."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    return int(_load().v3_argmax(a.ctypes.data, a.size))


def math(fn: str, x: np.ndarray) -> np.ndarray:
    """The reference's own v3_expf / v3_erff / v3_geluf (runtime/vault3.c:104-129), element-wise."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(a)
    _load().ref_math(("exp", "erf", "gelu").index(fn), a.ctypes.data, out.ctypes.data, a.size)
    return out


def sample_topk(logits: np.ndarray, k: int, temp: float, state: int):
    """The reference's v3_sample_topk (runtime/vault3.c:3204-3230): (index, new xorshift state)."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    st = C.c_uint64(state)
    idx = _load().v3_sample_topk(a.ctypes.data, a.size, k, float(temp), C.byref(st))
    return int(idx), int(st.value)
