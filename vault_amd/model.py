"""Drop-in VAULT v3 streaming model over the libvault_amd kernels.

Mirrors ``VAULTv3ForCausalLM`` / ``VAULTv3State`` of src/vault_v3_model.py (new_state :2159,
prefill :2163-2212, step :2214-2311, forward :2153) with the same argument meaning and state
fields; every projection, attention, RoPE, norm, KV-cache write, chunk-boundary re-base/re-rotation,
segment-bank compaction and scorer op is a call into the HIP library.  The auto-pin FSM runs on the
host (it decides on the prompt's first tokens); the segmenter, the segment rings and the top-B
eviction merge run on the device.

Token rules: with the token strings of a VLT3 file (``weights.tokens``) the segment-break tiers,
the system-role test and the newline id of the auto-pin rule come from the bytes, as in the C
runtime (runtime/vault3.c:937-959, 1920-1928, 2047); without them (a model built from tensors,
like the reference Python model offline) every tier is 0, the system role is
``cfg.system_tok_id`` and the newline id is 198 (src/vault_v3_model.py:2224-2252, 2260-2268).
Resonance and quarantine (runtime/vault3.c:1178-1831): with token strings and segment memory
(batch 1), the library's host unit (vault_amd/control.py) keeps a shingle index over the segment bank
(rebuilt after every bank merge, from the bank's tokens and segment ids read back once per W tokens)
and evaluates the query resonance of every step on host mirrors of the token rings; an active mode
writes the per-head bias rows of the state's two device bias buffers (layers [L/4, L/2) and
[L/2, L - L/14)), which the captured decode step reads on the segment span.  The spoof check
overwrites the step's segment score with -1e30.  Prefill chunks in which resonance is active at some
position run through the step path (the same launches as decoding), the others through the chunk
kernels with the quarantine applied to the chunk's scores.

Differences by design:
* The KV caches of all layers are single tensors [n_layers, B, G, n, D]; prev/cur are swapped by
  reference at chunk boundaries instead of copied (the reference copies cur into prev; the old cur
  content is never read before being overwritten).
* RoPE uses one device table of fp32 cos/sin rows computed from double-precision angles, as the C
  runtime does (runtime/vault3.c:840-849, 2126-2133).
* prefill() / forward() with batch > 1 and forward(mode="full") run the parallel form: every
  projection over all B * L tokens at once (MFMA GEMM), RoPE at absolute positions with the ring
  table's double-precision angles, and block_sliding_attention (or full causal attention) on the
  MFMA prefill kernel; batch-1 prefill / forward keep the chunk-recurrent form (segment memory).
"""
from __future__ import annotations

import gc
import math
from collections import OrderedDict
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from . import control, ops
from .attention import block_sliding_attention, causal_attention, rope_table_double
from .config import VAULTv3Config
from .weights import ModelWeights

V3_MAX_SINK = 512


def sink_capacity(cfg: VAULTv3Config) -> int:
    """Sink slots (runtime/vault3.c:706-710): min(W, 512), at least n_sink, at least 1."""
    return max(1, min(cfg.window, V3_MAX_SINK), cfg.n_sink)


class LayerView:
    """Per-layer views of the stacked caches, with the reference's LayerState field names."""

    _FIELDS = ("k_prev", "k_cur", "v_prev", "v_cur", "kraw_prev", "kraw_cur", "k_sink_raw", "k_sink_rot",
               "v_sink", "k_seg_raw", "k_seg_rot", "v_seg")

    def __init__(self, st: "VAULTv3State", li: int):
        self._st, self._li = st, li

    def __getattr__(self, name):
        if name in LayerView._FIELDS:
            return getattr(self._st, name)[self._li]
        raise AttributeError(name)


class StepIO:
    """Host inputs of the decode step and the device words the step's kernels read them from.

    The host writes each step's descriptor words (include/vault_amd.h VGX_STEP_*), token ids (their
    values, or the device address of a device tensor), logits address and, while a resonance mode is
    active, the bias vectors into one slot of a ring in pinned, device-coherent host memory; the
    step's first launch (ops.step_begin) reads the slot a device counter names and stores the words
    on the device, so a step makes no host-to-device copy.  Slots are taken in order, one per launch:
    a slot is rewritten only after the event recorded behind the launch that read it completed."""

    RING = 8

    def __init__(self, batch: int, device, n_heads: int = 0, bias_cap: int = 0):
        import ctypes
        lib = ops.L.load()
        self.batch, self.H, self.bias_cap = batch, n_heads, bias_cap
        self.slot_bytes = int(lib.vgx_step_slot_bytes(batch, n_heads, bias_cap))
        self.bias_off = int(lib.vgx_step_slot_bias_off(batch))
        ptr = ctypes.c_void_p()
        ops.L.check(lib.vgx_host_alloc(self.RING * self.slot_bytes, ctypes.byref(ptr)), "vgx_host_alloc")
        self.ring = int(ptr.value)
        self.host = np.ctypeslib.as_array((ctypes.c_uint8 * (self.RING * self.slot_bytes)).from_address(self.ring))
        self.host = self.host.reshape(self.RING, self.slot_bytes)
        # device words: descriptor [0, 16), slot counter [16, 20), logits address [24, 32), ids [64, ...)
        self.dev = torch.zeros(64 + 8 * batch, dtype=torch.uint8, device=device)
        self.step = self.dev[:16].view(torch.int32)
        self.counter = self.dev[16:20].view(torch.int32)
        self.out_ref = self.dev[24:32].view(torch.int64)
        self.ids = self.dev[64:].view(torch.int64)
        self.events: List[Optional[torch.cuda.Event]] = [None] * self.RING
        self.keep: List[Optional[torch.Tensor]] = [None] * self.RING    # device ids / logits a slot names
        self.i = 0

    def close(self) -> None:
        """Wait for the launches that read the ring, then free it."""
        if self.ring:
            for ev in self.events:
                if ev is not None:
                    ev.synchronize()
            ops.L.load().vgx_host_free(self.ring)
            self.ring, self.host = 0, None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def write(self, ids: torch.Tensor, slot: int, row: int, sink: int, n_cur: int,
              out: Optional[torch.Tensor] = None, bias: Optional[tuple] = None) -> None:
        """Fill the next slot: descriptor words, ids (host values, or the address of int64 device ids),
        the logits address ``out`` and ``bias`` = (row index [2, H] int8, vectors [3, M] fp32)."""
        k = self.i % self.RING
        if self.events[k] is not None:
            self.events[k].synchronize()
        h = self.host[k]
        h[0:16].view(np.int32)[:] = (slot, row, sink, n_cur)
        flags = 0
        if ids.is_cuda:
            d = ids if ids.dtype == torch.int64 and ids.is_contiguous() else ids.to(torch.int64).contiguous()
            h[ops.L.SLOT_IDS_ADDR:ops.L.SLOT_IDS_ADDR + 8].view(np.int64)[0] = d.data_ptr()
            flags |= ops.L.SLOTF_DEVICE_IDS
            self.keep[k] = d
        else:
            h[ops.L.SLOT_IDS:ops.L.SLOT_IDS + 8 * self.batch].view(np.int64)[:] = ids.numpy()
            self.keep[k] = None
        h[ops.L.SLOT_OUT_ADDR:ops.L.SLOT_OUT_ADDR + 8].view(np.int64)[0] = 0 if out is None else out.data_ptr()
        if bias is not None:
            rows, vec = bias
            o = self.bias_off
            h[o:o + 2 * self.H].view(np.int8)[:] = rows.reshape(-1)
            v = h[o + (2 * self.H + 15) // 16 * 16:o + (2 * self.H + 15) // 16 * 16 + 12 * self.bias_cap]
            v = v.view(np.float32).reshape(3, self.bias_cap)
            M = vec.shape[1]
            v[:, :M] = vec
            v[:, M:] = 0.0
            flags |= ops.L.SLOTF_BIAS
        h[ops.L.SLOT_FLAGS:ops.L.SLOT_FLAGS + 4].view(np.int32)[0] = flags

    def launched(self) -> None:
        """The launch that reads the slot of the last write is enqueued (on the current stream)."""
        ev = torch.cuda.Event()
        ev.record()
        self.events[self.i % self.RING] = ev
        self.i += 1

    def resync(self) -> None:
        """After a step that failed between write and launched: align the host's slot number with the
        device counter (whether or not the first launch ran)."""
        torch.cuda.synchronize(self.dev.device)
        c = int(self.counter.item())
        self.i += (c - self.i) % self.RING


class VAULTv3State:
    def __init__(self, cfg: VAULTv3Config, batch: int, device, kv_dtype=torch.float32, seg_budget: Optional[int] = None):
        self.cfg = cfg
        self.batch = batch
        self.device = torch.device(device)
        self.kv_dtype = kv_dtype
        self.pos = 0
        self.seg_budget = cfg.seg_budget if seg_budget is None else int(seg_budget)
        self.sink_cap = sink_capacity(cfg)
        self.n_pin = min(cfg.n_sink, cfg.window, self.sink_cap)
        self.pin_locked = not cfg.auto_pin_system
        self.saw_im_start = False
        self.awaiting_sys_nl = False
        W, G, D, L = cfg.window, cfg.n_kv_heads, cfg.head_dim, cfg.n_layers
        M_cap = max(1, self.seg_budget)
        z = lambda n: torch.zeros(L, batch, G, n, D, dtype=kv_dtype, device=self.device)
        self.k_prev, self.k_cur, self.v_prev, self.v_cur = z(W), z(W), z(W), z(W)
        self.kraw_prev, self.kraw_cur = z(W), z(W)
        self.k_sink_raw, self.k_sink_rot, self.v_sink = z(self.sink_cap), z(self.sink_cap), z(self.sink_cap)
        self.k_seg_raw, self.k_seg_rot, self.v_seg = z(M_cap), z(M_cap), z(M_cap)
        self._seg_tmp_k, self._seg_tmp_v = z(M_cap), z(M_cap)
        # Token and segment-id rings, segmenter state and the segment bank live on the device: the
        # decode step updates them (vgx_seg_step) and the chunk boundary merges the bank
        # (vgx_seg_evict) without a host round trip.  Host views below read them (a synchronisation).
        dev = self.device
        self.tok_prev = torch.zeros(batch, W, dtype=torch.int32, device=dev)
        self.tok_cur = torch.zeros(batch, W, dtype=torch.int32, device=dev)
        self.seg_prev_ids = torch.zeros(W, dtype=torch.int32, device=dev)
        self.seg_cur_ids = torch.zeros(W, dtype=torch.int32, device=dev)
        self.sc_prev = torch.zeros(W, dtype=torch.float32, device=dev)
        self.sc_cur = torch.zeros(W, dtype=torch.float32, device=dev)
        self.ctrl = torch.zeros(ops.L.SEG_WORDS, dtype=torch.int32, device=dev)     # VGX_SEG_* words
        self.bank_pos = torch.zeros(M_cap, dtype=torch.int64, device=dev)
        self.bank_score = torch.zeros(M_cap, dtype=torch.float32, device=dev)
        self.bank_tok = torch.zeros(M_cap, dtype=torch.int32, device=dev)
        self.bank_seg = torch.zeros(M_cap, dtype=torch.int32, device=dev)
        self.idx_old = torch.zeros(M_cap, dtype=torch.int32, device=dev)
        self.idx_new = torch.zeros(M_cap, dtype=torch.int32, device=dev)
        fd = max(1, len(cfg.seg_layers) * cfg.d_model)
        self.ema_ready = False
        self.seg_feat_ema = torch.zeros(fd, dtype=torch.float32, device=self.device)
        # resonance (batch 1 with token strings): host mirrors of the token rings, the shingle index and
        # the bias rows [H, bank capacity] of the early / late biased layers
        self.seg_bias_mode = 0
        self.seg_bias_active = False
        self.tok_prev_h = np.zeros(W, dtype=np.uint32)
        self.tok_cur_h = np.zeros(W, dtype=np.uint32)
        self.res: Optional[control.Resonance] = None
        self.bias_rows: Optional[tuple] = None     # the next step's bias rows for its slot (StepIO.write)
        self.bias_early: Optional[torch.Tensor] = None
        self.bias_late: Optional[torch.Tensor] = None
        self.graphs: "OrderedDict[tuple, tuple]" = OrderedDict()   # captured decode steps
        self._io: Optional[StepIO] = None

    # host views of the device bookkeeping (each reads the device: a synchronisation)
    def _word(self, i: int) -> int:
        return int(self.ctrl[i].item())

    @property
    def mem_cnt(self) -> int:
        return self._word(ops.L.SEG_MEM_CNT)

    @property
    def seg_id_offset(self) -> int:
        return self._word(ops.L.SEG_ID_OFFSET)

    @property
    def cur_seg_id(self) -> int:
        return self._word(ops.L.SEG_CUR_ID)

    @property
    def seg_len(self) -> int:
        return self._word(ops.L.SEG_LEN)

    @property
    def mem_pos(self) -> torch.Tensor:
        return self.bank_pos[:self.mem_cnt].cpu()

    @property
    def mem_score(self) -> torch.Tensor:
        return self.bank_score[:self.mem_cnt].cpu()

    @property
    def mem_tok(self) -> torch.Tensor:
        return self.bank_tok[:self.mem_cnt].to("cpu", torch.int64)

    @property
    def mem_seg(self) -> torch.Tensor:
        return self.bank_seg[:self.mem_cnt].to("cpu", torch.int64)

    @property
    def seg_head_bias(self) -> Optional[torch.Tensor]:
        """While a resonance mode is active: the (1, H, 1, M) per-head bias of the late biased layers on
        the bank's M slots (src/vault_v3_model.py:1629-1641, 1711-1716), a view of the device rows."""
        if not self.seg_bias_active or self.res is None:
            return None
        M = self.res.mem_cnt
        return self.bias_late[:, :M].reshape(1, -1, 1, M)

    @property
    def seg_head_bias_hop1(self) -> Optional[torch.Tensor]:
        """In mode 2: the (1, H, 1, M) hop-1 bias of the early biased layers, else None."""
        if self.seg_bias_mode != 2 or self.res is None:
            return None
        M = self.res.mem_cnt
        return self.bias_early[:, :M].reshape(1, -1, 1, M)

    @property
    def layers(self) -> List[LayerView]:
        """Per-layer views (built on access: a stored list would make a reference cycle, leaving the
        state to the cyclic garbage collector, which may run while a decode graph is captured)."""
        return [LayerView(self, li) for li in range(self.cfg.n_layers)]

    def step_io(self) -> StepIO:
        if self._io is None:
            cap = self.bias_early.shape[1] if self.bias_early is not None else 0
            self._io = StepIO(self.batch, self.device, self.cfg.n_heads if cap else 0, cap)
        return self._io

    def set_pinned(self, n_pin: int) -> None:
        cap = min(self.cfg.window, self.sink_cap)
        self.n_pin = max(0, min(int(n_pin), cap))
        self.pin_locked = True

    KV_FIELDS = ("k_prev", "k_cur", "v_prev", "v_cur", "kraw_prev", "kraw_cur", "k_sink_raw", "k_sink_rot",
                 "v_sink", "k_seg_raw", "k_seg_rot", "v_seg")

    def nbytes(self) -> int:
        return sum(getattr(self, n).numel() * getattr(self, n).element_size() for n in self.KV_FIELDS)

    def seed_long_context(self, pos: int, n_pin: int, mem_cnt: int, fill) -> None:
        """Put the state where a long stream leaves it: position ``pos`` (chunk index >= 2), ``n_pin``
        sinks locked, ``mem_cnt`` occupied segment-memory slots (mem_pos[i] = 8 i, segment i // 16,
        score 0), EMA ready.  ``fill(layer, field, shape)`` returns the host values of one layer's KV
        tensor (shape [B, G, n, D]).  Steps taken from here stay in the current chunk while
        pos % W < W - 1.  The fixed-size state makes this exactly the state a stream reaches, up to
        the values of the cached rows."""
        W = self.cfg.window
        if pos < 2 * W or n_pin > self.sink_cap or mem_cnt > max(0, self.seg_budget):
            raise ValueError("seed_long_context: pos < 2W, or n_pin / mem_cnt beyond capacity")
        for name in self.KV_FIELDS:
            t = getattr(self, name)
            for li in range(t.shape[0]):
                t[li].copy_(fill(li, name, tuple(t.shape[1:])).to(t.dtype))
        self.pos = int(pos)
        self.n_pin = int(n_pin)
        self.pin_locked = True
        i = torch.arange(mem_cnt, dtype=torch.int64)
        self.bank_pos[:mem_cnt].copy_(i * 8)
        self.bank_score.zero_()
        self.bank_tok.zero_()
        self.bank_seg[:mem_cnt].copy_((i // 16).to(torch.int32))
        self.ctrl.copy_(torch.tensor([mem_cnt, 0, 0, 0], dtype=torch.int32))
        self.ema_ready = True
        if self.res is not None:
            self.res.rebuild(self.bank_tok[:mem_cnt].cpu().numpy(), self.bank_seg[:mem_cnt].cpu().numpy())


class VAULTv3ForCausalLM:
    def __init__(self, weights: ModelWeights, kv_dtype: torch.dtype = torch.float32):
        self.w = weights
        self.cfg = weights.cfg
        self.device = weights.device
        self.kv_dtype = kv_dtype
        self.ws = ops.Workspace(self.device)
        self.ws_prefill = ops.Workspace(self.device)   # the chunk attention's key-range partials
        self.prefill_ws = ops.Workspace(self.device)
        self.tokens = weights.tokens
        vs = self.cfg.vocab_size
        self.tier_lut = self.tokens.tiers if self.tokens is not None else np.zeros(vs, dtype=np.uint8)
        self.tier_dev = torch.from_numpy(self.tier_lut.copy()).to(self.device) if self.tier_lut.any() else None
        self.use_graphs = True          # replay captured HIP graphs for decode steps
        # token strings for the host control unit (resonance, quarantine); none: those rules cannot fire
        self.ctl_tokens = control.TokenBytes(self.tokens.tokens) \
            if self.tokens is not None and self.tokens.has_strings else None
        self.head_class = control.head_classes(self.cfg.n_heads, self.cfg.n_kv_heads)
        self._table = None
        self._abs_table = None
        self._p0 = 0
        self._ensure_table(sink_capacity(self.cfg) + max(1, self.cfg.seg_budget))

    # ------------------------------------------------------------------ RoPE table
    def _ensure_table(self, neg: int) -> None:
        """Rows for positions [-neg, 2W): [cos(D/2) | sin(D/2)] fp32 from double-precision angles of a
        fp32 inverse frequency (runtime/vault3.c:840-849)."""
        c = self.cfg
        neg = max(neg, c.window)
        if self._table is not None and -self._p0 >= neg:
            return
        tab = rope_table_double(np.arange(-neg, 2 * c.window), c.head_dim, c.rope_theta)
        self._table = torch.from_numpy(tab).to(self.device)
        self._p0 = -neg

    def _abs_rows(self, L: int) -> torch.Tensor:
        """Table rows of absolute positions [0, L) (the parallel forms rotate at absolute positions),
        same arithmetic as the ring table; grown on demand."""
        if self._abs_table is None or self._abs_table.shape[0] < L:
            n = max(L, 2 * self.cfg.window)
            self._abs_table = torch.from_numpy(rope_table_double(np.arange(n), self.cfg.head_dim,
                                                                 self.cfg.rope_theta)).to(self.device)
        return self._abs_table

    def _rows(self, p: int) -> torch.Tensor:
        """Table rows starting at position p."""
        return self._table[p - self._p0:]

    # ------------------------------------------------------------------ API
    def new_state(self, batch: int = 1, seg_budget: Optional[int] = None) -> VAULTv3State:
        st = VAULTv3State(self.cfg, batch, self.device, self.kv_dtype, seg_budget=seg_budget)
        self._ensure_table(st.sink_cap + max(1, st.seg_budget))
        if self.ctl_tokens is not None and self._seg_active(st, batch):
            cfg = self.cfg
            st.res = control.Resonance(self.ctl_tokens, cfg.window, st.seg_budget, cfg.n_sink, cfg.im_start_id,
                                       cfg.im_end_id)
            st.bias_early = torch.zeros(cfg.n_heads, st.seg_budget, dtype=torch.float32, device=self.device)
            st.bias_late = torch.zeros_like(st.bias_early)
        return st

    def _seg_active(self, st: VAULTv3State, batch: int) -> bool:
        return self.w.scorer is not None and st.seg_budget > 0 and batch == 1

    @torch.no_grad()
    def step(self, token_ids: torch.Tensor, st: VAULTv3State, vault_on: bool = False) -> torch.Tensor:
        """token_ids: (B,) on the host or the device -> logits (B, V) fp32 on the device.  Mutates
        ``st``.  Device ids (e.g. ops.argmax of the previous logits) are not read on the host once the
        auto-pin prefix is decided (segmentation and the segment bank are updated on the device),
        except by the host resonance / quarantine rules of a model with token strings and segment
        memory, which read each id."""
        _ = vault_on
        ids = token_ids.reshape(-1)
        ids = ids if ids.is_cuda else ids.to("cpu", torch.int64)
        B = ids.numel()
        if B != st.batch:
            raise ValueError("batch size differs from the state's")
        return self._advance(st, ids, boundary=True)

    def _advance(self, st: VAULTv3State, ids: torch.Tensor, boundary: bool) -> torch.Tensor:
        """One token through the step path (runtime/vault3.c:2034-2222); ``boundary`` False when the
        caller has already crossed this chunk's boundary."""
        W = self.cfg.window
        B = ids.numel()
        pos = st.pos
        c = pos % W
        seg_active = self._seg_active(st, B)
        if not st.pin_locked and B == 1:
            self._auto_pin(st, int(ids[0]), pos)
        if boundary and c == 0 and pos > 0:
            self._boundary(st, seg_active)
        if st.res is not None:
            st.tok_cur_h[c] = int(ids[0])           # a host read when the id is on the device
            self._resonance(st, c, pos, seg_active)
        logits = self._decode(st, ids, pos, c, seg_active)
        if st.res is not None and seg_active and self._spoofed(st, c, pos):
            st.sc_cur[c:c + 1].fill_(-1.0e30)
        if seg_active:
            st.ema_ready = True
        st.pos = pos + 1
        return logits

    # ------------------------------------------------------------------ resonance / quarantine (host)
    def _resonance(self, st: VAULTv3State, c: int, pos: int, seg_active: bool, direct: bool = False) -> None:
        """This step's query resonance over the host rings.  An active mode sets the bias rows of the
        early / late biased layers (runtime/vault3.c:1976-1988): head h's late row is arch (class 1) or
        sup (class 2), its early row the same, or hop-1 in mode 2; zero for class 0.  They travel as
        a row index per head and the three vectors in the next decode step's slot (``st.bias_rows``),
        or with ``direct`` are copied into the device rows now."""
        mode = 0
        if seg_active and pos >= 2 * self.cfg.window and st.res.mem_cnt > 0:
            mode = st.res.update(st.tok_prev_h, st.tok_cur_h, c, pos, st.n_pin)
        st.seg_bias_mode = mode
        st.seg_bias_active = mode > 0
        st.bias_rows = None
        if mode:
            M = st.res.mem_cnt
            cls = np.asarray(self.head_class, dtype=np.int64)
            rows = np.full((2, self.cfg.n_heads), -1, dtype=np.int8)
            rows[1][cls > 0] = cls[cls > 0] - 1                 # 0 = arch, 1 = sup
            rows[0] = rows[1]
            if mode == 2:
                rows[0][cls > 0] = 2                             # hop-1
            vec = np.stack([st.res.arch[:M], st.res.sup[:M], st.res.hop1[:M]]).astype(np.float32)
            if direct:
                zero = np.zeros((1, M), dtype=np.float32)
                full = np.concatenate([vec, zero])
                st.bias_early[:, :M].copy_(torch.from_numpy(full[rows[0].astype(np.int64)]))
                st.bias_late[:, :M].copy_(torch.from_numpy(full[rows[1].astype(np.int64)]))
            else:
                st.bias_rows = (rows, vec)

    def _spoofed(self, st: VAULTv3State, c: int, pos: int, n_pin: Optional[int] = None) -> bool:
        cfg = self.cfg
        return control.spoof_check(self.ctl_tokens, st.tok_prev_h, st.tok_cur_h, cfg.window, c, pos,
                                   st.n_pin if n_pin is None else n_pin, cfg.n_sink)

    def _sync_bank(self, st: VAULTv3State) -> None:
        """Rebuild the shingle index from the device bank (after a merge: once per W tokens)."""
        M = st.mem_cnt
        st.res.rebuild(st.bank_tok[:M].cpu().numpy(), st.bank_seg[:M].cpu().numpy())

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, vault_on: bool = False,
                seg_budget: Optional[int] = None) -> Tuple[torch.Tensor, VAULTv3State]:
        """Prefill from position 0; returns last-token logits (B, V) and the streaming state."""
        _ = vault_on
        B, L = input_ids.shape
        bud = self.cfg.seg_budget if seg_budget is None else int(seg_budget)
        if B == 1:
            h, st, lg = self._chunk_recurrent(input_ids, bud, all_logits=False)
            return (self._logits(h) if h is not None else lg), st
        # batch > 1: the parallel sliding-window + sink prefill (src/vault_v3_model.py:2177-2212)
        h, st = self._forward_block(input_ids, mode="block", want_state=True, last_only=True)
        return self._logits(h), st

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor, mode: str = "block", vault_on: bool = False,
                seg_budget: Optional[int] = None) -> torch.Tensor:
        """Logits for every position, (B, L, V)."""
        _ = vault_on
        B, L = input_ids.shape
        bud = self.cfg.seg_budget if seg_budget is None else int(seg_budget)
        if B == 1 and mode == "block":
            _, _, lg = self._chunk_recurrent(input_ids, bud, all_logits=True)
            return lg.unsqueeze(0)
        # batch > 1, or full causal attention: the parallel form (src/vault_v3_model.py:2118-2151)
        h, _ = self._forward_block(input_ids, mode=mode, want_state=False, last_only=False)
        return self._logits(h).view(B, L, -1)

    __call__ = forward

    # ------------------------------------------------------------------ host control
    def _breaks(self, tid: int, seg_len: int) -> bool:
        """Whether a segment closes after this token (runtime/vault3.c:2109-2122;
        src/vault_v3_model.py:2260-2268): tier 1 from seg_min tokens on, tier 2 from
        max(seg_min, 2 seg_max / 3), tier 3 from max(seg_min, seg_max - 8), any token at seg_max."""
        cfg = self.cfg
        tr = int(self.tier_lut[tid]) if 0 <= tid < self.tier_lut.shape[0] else 0
        t2 = max(cfg.seg_min, (cfg.seg_max * 2) // 3)
        t3 = max(cfg.seg_min, cfg.seg_max - 8 if cfg.seg_max > 8 else cfg.seg_min)
        return (seg_len >= cfg.seg_max or (tr == 1 and seg_len >= cfg.seg_min) or (tr == 2 and seg_len >= t2)
                or (tr == 3 and seg_len >= t3))

    def _is_system_role(self, tid: int) -> bool:
        return self.tokens.is_system_role(tid) if self.tokens is not None else tid == self.cfg.system_tok_id

    @property
    def newline_id(self) -> int:
        return self.tokens.newline_id if self.tokens is not None else 198

    def _auto_pin(self, st: VAULTv3State, tid: int, pos: int) -> None:
        """Online ChatML system-prompt pinning (src/vault_v3_model.py:2224-2252)."""
        cfg = self.cfg
        limit = min(cfg.max_sink, cfg.window, st.sink_cap)
        if pos == 0:
            if tid == cfg.im_start_id and limit >= 2:
                st.saw_im_start = True
            else:
                st.pin_locked = True
        elif pos == 1 and st.saw_im_start:
            if not self._is_system_role(tid):
                st.saw_im_start = False
                st.pin_locked = True
        elif st.saw_im_start and pos < limit:
            if st.awaiting_sys_nl:
                st.n_pin = max(st.n_pin, pos + 1 if tid == self.newline_id else pos)
                st.pin_locked = True
                st.awaiting_sys_nl = False
            elif tid == cfg.im_end_id:
                st.n_pin = max(st.n_pin, pos + 1)
                if pos + 1 < limit:
                    st.awaiting_sys_nl = True
                else:
                    st.pin_locked = True
        elif pos >= limit:
            if st.saw_im_start and not st.awaiting_sys_nl:
                st.n_pin = max(st.n_pin, limit)
            st.pin_locked = True
            st.awaiting_sys_nl = False

    def _flat(self, t: torch.Tensor) -> torch.Tensor:
        """[L, B, G, n, D] -> [L*B*G, n, D] view."""
        return t.view(-1, t.shape[-2], t.shape[-1])

    def _boundary(self, st: VAULTv3State, seg_active: bool) -> None:
        """Chunk boundary at c == 0, pos > 0 (src/vault_v3_model.py:1858-1935)."""
        cfg = self.cfg
        W = cfg.window
        pos = st.pos
        if pos >= 2 * W and seg_active and st.seg_budget > 0:
            self._evict(st, pos // W - 2)
        st.k_prev, st.k_cur = st.k_cur, st.k_prev
        st.v_prev, st.v_cur = st.v_cur, st.v_prev
        st.kraw_prev, st.kraw_cur = st.kraw_cur, st.kraw_prev
        if pos >= 2 * W:
            kp = self._flat(st.k_prev)
            ops.rope_rotate(kp, kp, self._rows(-W), 0)
        st.tok_prev, st.tok_cur = st.tok_cur, st.tok_prev
        st.sc_prev, st.sc_cur = st.sc_cur, st.sc_prev
        st.seg_prev_ids, st.seg_cur_ids = st.seg_cur_ids, st.seg_prev_ids
        st.ctrl[ops.L.SEG_CUR_ID:ops.L.SEG_LEN + 1].zero_()
        if pos >= 2 * W:
            self._refresh_prefix(st, seg_active)
        if st.res is not None:
            st.tok_prev_h, st.tok_cur_h = st.tok_cur_h, st.tok_prev_h
            if pos >= 2 * W and seg_active and st.seg_budget > 0:
                self._sync_bank(st)

    def _refresh_prefix(self, st: VAULTv3State, seg_active: bool) -> None:
        """Segment keys at positions [-M, 0), sinks at [-(M+S), -M) (src/vault_v3_model.py:1842-1856),
        with the bank count M read on the device."""
        S = st.n_pin
        D = self.cfg.head_dim
        dyn = st.ctrl[ops.L.SEG_MEM_CNT:ops.L.SEG_MEM_CNT + 1]
        if seg_active:
            ops.rope_rotate_dyn(self._flat(st.k_seg_raw), self._flat(st.k_seg_rot), self._rows(0), D, dyn, 0, True)
            if S > 0:
                ops.rope_rotate_dyn(self._flat(st.k_sink_raw)[:, :S], self._flat(st.k_sink_rot)[:, :S], self._rows(0),
                                    D, dyn, -S, False)
        elif S > 0:
            ops.rope_rotate(self._flat(st.k_sink_raw)[:, :S], self._flat(st.k_sink_rot)[:, :S], self._rows(-S), D)

    def _evict(self, st: VAULTv3State, ev: int) -> None:
        """Segment-memory update for the evicted chunk `ev` (src/vault_v3_model.py:1865-1921;
        runtime/vault3.c:1833-1915), all on the device: quarantine, per-segment max with the
        -1e-6 * (seg id mod 16384) tie-break, exact top-B merge ordered by (score desc, position
        asc) (vgx_seg_evict), then the chronological compaction of the bank's keys / values from the
        old bank and the evicted chunk into the spare bank, which becomes the bank."""
        ops.seg_evict(st.sc_prev, st.seg_prev_ids, st.tok_prev[0], st.bank_pos, st.bank_score, st.bank_tok,
                      st.bank_seg, st.ctrl, ev, st.n_pin if ev == 0 else 0, st.seg_budget, st.idx_old, st.idx_new)
        for bank, tmp, src_prev in ((st.k_seg_raw, st._seg_tmp_k, st.kraw_prev), (st.v_seg, st._seg_tmp_v, st.v_prev)):
            ops.gather_rows_masked(self._flat(bank), self._flat(tmp), st.idx_old)
            ops.gather_rows_masked(self._flat(src_prev), self._flat(tmp), st.idx_new)
        st.k_seg_raw, st._seg_tmp_k = st._seg_tmp_k, st.k_seg_raw
        st.v_seg, st._seg_tmp_v = st._seg_tmp_v, st.v_seg

    # ------------------------------------------------------------------ decode step on the device
    def _decode(self, st: VAULTv3State, ids: torch.Tensor, pos: int, c: int, seg_active: bool) -> torch.Tensor:
        """One decode step on the device.  The position-dependent words (ring slot, RoPE row, sink
        slot, current-chunk length), the token ids, the logits address and the bias rows go through a
        slot of the pinned host ring that the step's first launch reads, so the launch sequence only
        depends on the chunk configuration; that sequence is captured once per configuration as a HIP
        graph and replayed at every position of the chunk (re-captured when the configuration changes:
        at most twice per W tokens).  GEMV batches (B < ops.GEMM_MIN_ROWS) write the logits straight
        into a fresh tensor named in the slot; larger batches copy them out of the graph's buffer."""
        cfg = self.cfg
        W, B = cfg.window, ids.numel()
        io = st.step_io()
        eff = W + c if pos >= W else c
        n_sk = st.n_pin if pos >= 2 * W else 0
        has_seg = pos >= 2 * W and seg_active       # the bank span, its length on the device
        n_prev = W if pos >= W else 0
        bias_on = bool(has_seg and st.seg_bias_active)
        ema_first = seg_active and not st.ema_ready
        indirect = B < ops.GEMM_MIN_ROWS
        spec = (B, n_sk, has_seg, n_prev, seg_active, ema_first, bias_on, indirect)
        out = torch.empty(B, self.w.embed.rows, dtype=torch.float32, device=self.device) if indirect else None
        if bias_on and st.bias_rows is None:
            raise RuntimeError("a resonance mode is active but this step's bias rows were not computed")
        io.write(ids, slot=c, row=eff - self._p0, sink=pos if pos < st.sink_cap else -1, n_cur=c + 1, out=out,
                 bias=st.bias_rows if bias_on else None)
        try:
            if not self.use_graphs:
                lg = self._decode_launch(st, spec)
                io.launched()
                return out if indirect else lg
            self._size_workspace(st)
            key = spec + tuple(t.data_ptr() for t in (st.k_prev, st.k_cur, st.v_prev, st.v_cur, st.kraw_cur,
                                                       st.k_seg_rot, st.v_seg, st.sc_cur, st.tok_cur, st.seg_cur_ids,
                                                       self._table, self.ws.buf,
                                                       ops.gemm_workspace(self.device).buf)) + \
                ((st.bias_early.data_ptr(), st.bias_late.data_ptr()) if bias_on else ())
            ent = st.graphs.get(key)
            if ent is None:
                # No destructor may run HIP calls while the stream captures: collect garbage now and keep
                # the collector off during the capture.
                gc.collect()
                gc_was_on = gc.isenabled()
                gc.disable()
                try:
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g):
                        lg = self._decode_launch(st, spec)
                finally:
                    if gc_was_on:
                        gc.enable()
                ent = (g, lg)
                st.graphs[key] = ent
                while len(st.graphs) > 8:
                    st.graphs.pop(next(iter(st.graphs)))
            ent[0].replay()
            io.launched()
        except BaseException:
            io.resync()
            raise
        return out if indirect else ent[1].clone()

    def _batch_qkv_fusable(self, B: int) -> bool:
        """Decode batches that run the small-batch GEMM (8..64 rows) on Q8_0 / Q4_0 q/k/v weights take
        the projections' K-split sums in the RoPE launch (ops.qkv_rope_batch)."""
        if not ops.GEMM_MIN_ROWS <= B <= 64:
            return False
        for lw in self.w.layers:
            if lw.wqkv.dtype not in (ops.Q8_0, ops.Q4_0) or lw.ln1.data_ptr() % 16:
                return False
            if lw.wq is not None and lw.wq.dtype not in (ops.Q8_0, ops.Q4_0):
                return False
        return True

    def _size_workspace(self, st: VAULTv3State) -> None:
        """Grow the workspaces before a capture (a captured graph holds their addresses): attention to
        the bound of any decode step of this batch size (the library's bound at its split cap), and
        the GEMM activation splits for batches that use the MFMA GEMM."""
        cfg = self.cfg
        lib = ops.L.load()
        # the most any decode step of this batch can need (the split count is capped, so a key count
        # beyond every state's capacity gives the bound)
        self.ws.get(int(lib.vgx_attn_decode_workspace_bytes(st.batch, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                                              1 << 24)))
        if st.batch >= ops.GEMM_MIN_ROWS:
            shapes = [(cfg.d_ff, cfg.d_model, ops.L.EPI_SWIGLU), (cfg.d_model, cfg.d_ff, ops.L.EPI_ACCUM),
                      ((cfg.n_heads + 2 * cfg.n_kv_heads) * cfg.head_dim, cfg.d_model, ops.L.EPI_STORE),
                      (cfg.d_model, cfg.n_heads * cfg.head_dim, ops.L.EPI_ACCUM),
                      (cfg.vocab_size, cfg.d_model, ops.L.EPI_STORE)]
            need = max(int(lib.vgx_qgemm_workspace_bytes(st.batch, r, c, e)) for r, c, e in shapes)
            if self._batch_qkv_fusable(st.batch):
                need = max([need] + [int(lib.vgx_qkv_rope_batch_workspace_bytes(
                    st.batch, cfg.d_model, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, sep)) for sep in (0, 1)])
            ops.gemm_workspace(self.device).get(need)

    def _decode_launch(self, st: VAULTv3State, spec: tuple) -> torch.Tensor:
        """Every kernel of one decode step (embedding -> 28 layers -> scorer -> LM head) for the chunk
        configuration ``spec``; position-dependent values are read from the step buffer."""
        B, n_sk, has_seg, n_prev, seg_active, ema_first, bias_on, indirect = spec
        cfg, w = self.cfg, self.w
        H, G, D, d = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.d_model
        HD, GD = H * D, G * D
        io = st.step_io()
        step, n_cur = io.step, io.step[ops.L.STEP_N_CUR:ops.L.STEP_N_CUR + 1]
        # the slot's words and ids onto the device, token ring and segmenter, and the embedding rows of
        # the ids [B, d], in one launch
        x = torch.empty(B, d, dtype=torch.float32, device=self.device)
        ops.step_begin(io.ring, io.RING, io.slot_bytes, io.counter, step, io.ids, io.out_ref if indirect else None,
                       st.tok_cur, st.seg_cur_ids if seg_active else None, st.ctrl if seg_active else None,
                       self.tier_dev, cfg.seg_min, cfg.seg_max,
                       bias=(st.bias_early, st.bias_late) if bias_on else None, embed=(w.embed, x))
        # bank span: its length is the device count (the bias rows cover the bank's capacity)
        m_dev = st.ctrl[ops.L.SEG_MEM_CNT:ops.L.SEG_MEM_CNT + 1]
        n_seg = st.k_seg_rot.shape[3] if has_seg else 0
        # rows [0, B) receive the scorer features, rows [B, 2B) the habituated ones (one LayerNorm launch)
        feats = torch.empty(2 * B, len(cfg.seg_layers) * d, dtype=torch.float32, device=self.device) \
            if seg_active else None
        ao = torch.empty(B, H, D, dtype=torch.float32, device=self.device)
        hbuf = torch.empty(B, cfg.d_ff, dtype=torch.float32, device=self.device)
        table = self._rows(self._p0)
        scale = 1.0 / math.sqrt(D)
        fused = B == 1 and all(lw.wq_rope is not None for lw in w.layers)
        batch_fused = not fused and self._batch_qkv_fusable(B)
        qbuf = torch.empty(B, H, D, dtype=torch.float32, device=self.device) if fused or batch_fused else None
        # the scorer rides in the down projections of the two layers after its last feature layer (their
        # launches leave CUs free), instead of launches of its own after the layers
        sides, h_sc = self._score_sides(st, feats, ema_first, step) if seg_active and fused else ({}, None)
        for li, lw in enumerate(w.layers):
            xc = None
            if seg_active and li in cfg.seg_layers:
                j = cfg.seg_layers.index(li)
                xc = feats[:B, j * d:(j + 1) * d]
                if not fused:
                    xc.copy_(x)
            if fused:
                # one launch: norm + q/k/v + bias + RoPE + ring / sink writes (+ the scorer feature copy)
                bkv = lw.bqkv[HD:] if lw.wq is None else lw.bqkv
                ops.qkv_rope_step(lw.wq_rope, lw.bq, lw.wkv_rope, bkv, x, (lw.ln1, cfg.rms_eps), table, D, step,
                                  qbuf, st.k_cur[li], st.kraw_cur[li], st.v_cur[li], st.k_sink_raw[li],
                                  st.v_sink[li], x_copy=xc)
                q = qbuf
            elif batch_fused:
                # projections as K-split partials, summed by the RoPE / ring-write launch
                ops.qkv_rope_batch(lw.wq, lw.bq if lw.wq is not None else None, lw.wqkv, lw.bqkv, x,
                                   (lw.ln1, cfg.rms_eps), table, D, step, qbuf, st.k_cur[li], st.kraw_cur[li],
                                   st.v_cur[li], st.k_sink_raw[li], st.v_sink[li])
                q = qbuf
            else:
                q, k, v = self._qkv(lw, x, B)
                ops.rope_qkv_write_step(q, k, v, table, D, step, st.k_cur[li], st.kraw_cur[li], st.v_cur[li],
                                        st.k_sink_raw[li], st.v_sink[li])
            spans = []
            if n_sk:
                spans.append((st.k_sink_rot[li][:, :, :n_sk], st.v_sink[li][:, :, :n_sk]))
            bias, bspan = None, -1
            if n_seg:
                bias = self._seg_bias(st, li) if bias_on else None
                bspan = len(spans)
                spans.append((st.k_seg_rot[li], st.v_seg[li], m_dev))
            if n_prev:
                spans.append((st.k_prev[li], st.v_prev[li]))
            spans.append((st.k_cur[li], st.v_cur[li], n_cur))
            ops.attn_decode(q, spans, out=ao, bias=bias, bias_span=bspan, scale=scale, ws=self.ws)
            ops.qlinear(lw.wo, ao.view(B, HD), out=x, accumulate=True)
            ops.qlinear_swiglu(lw.wgu, x, out=hbuf, norm=(lw.ln2, cfg.rms_eps))
            if li in sides:
                ops.qlinear_side(lw.wd, hbuf, x, True, sides[li])
            else:
                ops.qlinear(lw.wd, hbuf, out=x, accumulate=True)
        if seg_active and not sides:
            self._score(st, feats, T=1, c0=0, first=ema_first, out_index=step[ops.L.STEP_SLOT:ops.L.STEP_SLOT + 1])
        if indirect:
            ops.qlinear_indirect(self.w.embed, x, io.out_ref, norm=(self.w.norm, cfg.rms_eps))
            return None
        return self._logits(x)

    def _qkv(self, lw, x: torch.Tensor, N: int):
        """q [N,H,D], k [N,G,D], v [N,G,D] views of the fused RMSNorm + QKV projection outputs."""
        cfg = self.cfg
        H, G, D = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim
        HD, GD = H * D, G * D
        ln1 = (lw.ln1, cfg.rms_eps)
        if lw.wq is None:
            qkv = ops.qlinear(lw.wqkv, x, bias=lw.bqkv, norm=ln1)
            return qkv[:, :HD].view(N, H, D), qkv[:, HD:HD + GD].view(N, G, D), qkv[:, HD + GD:].view(N, G, D)
        q = ops.qlinear(lw.wq, x, bias=lw.bq, norm=ln1).view(N, H, D)
        kv = ops.qlinear(lw.wqkv, x, bias=lw.bqkv, norm=ln1)
        return q, kv[:, :GD].view(N, G, D), kv[:, GD:].view(N, G, D)

    # ------------------------------------------------------------------ device compute
    def _seg_bias(self, st: VAULTv3State, li: int) -> Optional[torch.Tensor]:
        """The bias rows of layer li on the segment span (runtime/vault3.c:1976-1988): the early buffer
        (hop-1 in mode 2, else arch / sup) in [L/4, L/2), the late one in [L/2, L - L/14), none
        elsewhere."""
        lo, mid, hi = control.biased_layers(self.cfg.n_layers)
        return st.bias_early if lo <= li < mid else st.bias_late if mid <= li < hi else None

    def _layers(self, x: torch.Tensor, st: VAULTv3State, pos: int, seg_active: bool,
                bias: Optional[Tuple[torch.Tensor, torch.Tensor]] = None) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Chunk prefill (batch 1): run all layers in place on x [N, d], the N tokens at slots [0, N)
        of chunk pos // W (src/vault_v3_model.py:2045-2096); ``bias``: the chunk's (early, late)
        resonance bias rows on the segment run (_chunk_bias), applied in the biased layers."""
        cfg, w = self.cfg, self.w
        W, H, G, D, d = cfg.window, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.d_model
        N = x.shape[0]
        HD = H * D
        ci = pos // W
        feats = None
        if seg_active:
            feats = torch.empty(2 * N, len(cfg.seg_layers) * d, dtype=torch.float32, device=self.device)
        n_sk = st.n_pin if ci >= 2 else 0
        n_seg = st.mem_cnt if (seg_active and ci >= 2) else 0
        n_prev = W if ci >= 1 else 0
        table, trs = self._rows(W if ci >= 1 else 0), D
        ao = torch.empty(N, H, D, dtype=torch.float32, device=self.device)
        hbuf = torch.empty(N, cfg.d_ff, dtype=torch.float32, device=self.device)
        scale = 1.0 / math.sqrt(D)
        mfma = D == 128 and H // G in (1, 2, 4, 6, 8)
        lo, mid, hi = control.biased_layers(cfg.n_layers)
        head_rows = [int(k) - 1 for k in self.head_class]          # arch heads row 0, sup heads row 1
        if bias is not None and not (mfma and n_seg == bias[1].shape[2]):
            raise RuntimeError("chunk bias needs the MFMA attention and one bias column per bank slot")
        for li, lw in enumerate(w.layers):
            if seg_active and li in cfg.seg_layers:
                j = cfg.seg_layers.index(li)
                feats[:N, j * d:(j + 1) * d].copy_(x)
            q, k, v = self._qkv(lw, x, N)
            kc, kr, vc = st.k_cur[li], st.kraw_cur[li], st.v_cur[li]          # [1, G, W, D]
            ks, vs = st.k_sink_raw[li], st.v_sink[li]                          # [1, G, S_cap, D]
            take = max(0, min(N, st.sink_cap - pos))
            ops.rope_qkv_write(q, k, v, table, trs, kc[0], kr[0], vc[0], D, kc.stride(1),
                               ks[0, :, pos] if take else None, vs[0, :, pos] if take else None, take,
                               D, ks.stride(1))
            spans = []
            if n_sk:
                spans.append((st.k_sink_rot[li][:, :, :n_sk], st.v_sink[li][:, :, :n_sk]))
            if n_seg:
                spans.append((st.k_seg_rot[li][:, :, :n_seg], st.v_seg[li][:, :, :n_seg]))
            if n_prev:
                spans.append((st.k_prev[li], st.v_prev[li]))
            spans.append((kc[:, :, :N], st.v_cur[li][:, :, :N]))
            if mfma:
                # block attention on MFMA (fp32 cache: K / V as bf16 hi + lo; runs are the [G, n, D] views
                # of batch entry 0)
                blk = {"q": q, "out": ao, "runs": [(k_[0], v_[0]) for k_, v_ in spans], "causal_base": 0}
                if bias is not None and lo <= li < hi:
                    blk.update(bias=bias[0] if li < mid else bias[1], bias_head_row=head_rows,
                               bias_run=1 if n_sk else 0)
                ops.attn_prefill([blk], H, G, scale, ws=self.ws_prefill)
            else:
                ops.attn_decode(q, spans, out=ao, scale=scale, ws=self.ws, causal_base=0)
            ops.qlinear(lw.wo, ao.view(N, HD), out=x, accumulate=True)
            ops.qlinear_swiglu(lw.wgu, x, out=hbuf, norm=(lw.ln2, cfg.rms_eps))
            ops.qlinear(lw.wd, hbuf, out=x, accumulate=True)
        return x, feats

    def _score_sides(self, st: VAULTv3State, feats: torch.Tensor, first: bool, step: torch.Tensor):
        """The decode token's scorer as the two jobs of ops.score_side, keyed by the layer whose down
        projection carries each (the two layers after the last feature layer; none when the model has
        no such layers or the scorer does not fit the jobs), and the fc1 output buffer they share (held
        by the caller until both are launched)."""
        cfg, sw = self.cfg, self.w.scorer
        l1 = max(cfg.seg_layers) + 1
        fd = feats.shape[1]
        if l1 + 1 >= len(self.w.layers) or fd > 5120 or sw.w1.dtype != ops.L.F32 or \
                not all(t.data_ptr() % 16 == 0 for t in (feats, st.seg_feat_ema, sw.ln_w, sw.ln_b)):
            return {}, None
        h = torch.empty(2, sw.w1.rows, dtype=torch.float32, device=self.device)
        idx = step[ops.L.STEP_SLOT:ops.L.STEP_SLOT + 1]
        args = (feats[0], st.seg_feat_ema, first, sw.w1, sw.b1, sw.ln_w, sw.ln_b, 1e-5, sw.w2, sw.b2, h,
                st.sc_cur[0:1], idx)
        return {l1: ops.score_side(1, *args), l1 + 1: ops.score_side(2, *args)}, h

    def _score(self, st: VAULTv3State, rows: torch.Tensor, T: int, c0: int, first: bool,
               out_index: Optional[torch.Tensor] = None) -> None:
        """Habituated segment scores of T tokens into sc_cur[c0:c0+T], shifted by the device slot
        ``out_index`` when given (src/vault_v3_model.py:1224-1247, 2294-2305).  rows: [2T, fd] with the
        features in rows[:T]; rows[T:] receive the habituated features, then both halves are
        LayerNormed in place."""
        sw = self.w.scorer
        fd = rows.shape[1]
        if T == 1 and fd <= 5120 and sw.w1.dtype == ops.L.F32 and \
                all(t.data_ptr() % 16 == 0 for t in (rows, st.seg_feat_ema, sw.ln_w, sw.ln_b)):
            # one token: the fc1 GEMV builds both LayerNormed rows itself, the tail updates the EMA
            ops.seg_score_step(rows[0], st.seg_feat_ema, first, sw.w1, sw.b1, sw.ln_w, sw.ln_b, 1e-5, sw.w2, sw.b2,
                               st.sc_cur[c0:c0 + 1], out_index=out_index)
            return
        ops.ema_habituate(rows[:T], rows[T:2 * T], st.seg_feat_ema, first)
        ops.layernorm(rows[:2 * T], sw.ln_w, sw.ln_b, 1e-5, rows[:2 * T])
        h1 = ops.qlinear(sw.w1, rows[:2 * T], bias=sw.b1)   # T = 1: both rows in one pass over the weights
        ops.seg_score_tail(h1, sw.w2, sw.b2, T, first, st.sc_cur[c0:c0 + T], out_index=out_index)

    def _logits(self, h: torch.Tensor) -> torch.Tensor:
        return ops.qlinear(self.w.embed, h, norm=(self.w.norm, self.cfg.rms_eps))

    def _forward_block(self, input_ids: torch.Tensor, mode: str, want_state: bool, last_only: bool):
        """Parallel form for B sequences of L tokens (src/vault_v3_model.py:1048-1061, 2118-2151,
        2177-2212): hidden states of every token (or of each sequence's last token) and, with
        ``want_state``, the streaming state the reference's batched prefill leaves (n_sink sinks
        pinned, no segment memory; ring rows re-rotated to their re-based positions)."""
        cfg, w = self.cfg, self.w
        B, L = input_ids.shape
        H, G, D, W = cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.window
        HD, N = H * D, B * L
        dev = self.device
        ids = input_ids.reshape(-1).to(dev, torch.int64)
        st = None
        if want_state:
            st = self.new_state(B, seg_budget=0)
            st.set_pinned(cfg.n_sink)
            n_pin = st.n_pin
        else:
            n_pin = max(0, min(cfg.n_sink, W, sink_capacity(cfg)))
        ns = min(n_pin, L)
        tab = self._abs_rows(L)
        mfma = D == 128 and H // G in (1, 2, 4, 6, 8)
        x = ops.embed(w.embed, ids, pad_row=0)                                 # [N, d]
        kr = torch.empty(B, G, L, D, dtype=torch.float32, device=dev)          # rotated keys
        vv = torch.empty(B, G, L, D, dtype=torch.float32, device=dev)          # values, same strides
        ao = torch.empty(B, L, H, D, dtype=torch.float32, device=dev)
        hbuf = torch.empty(N, cfg.d_ff, dtype=torch.float32, device=dev)
        # raw keys / values of the sink tokens: the state's sink slots, or scratch
        if st is None and ns:
            sk_all = torch.empty(B, G, ns, D, dtype=torch.float32, device=dev)
            sv_all = torch.empty_like(sk_all)
        last = (L - 1) // W
        cnt = L - last * W
        for li, lw in enumerate(w.layers):
            q, k, v = self._qkv(lw, x, N)                                      # k / v stay raw in place
            for b in range(B):
                r = slice(b * L, (b + 1) * L)
                if ns:
                    sk, sv = (st.k_sink_raw[li][b], st.v_sink[li][b]) if st is not None else (sk_all[b], sv_all[b])
                else:
                    sk = sv = None
                ops.rope_qkv_write(q[r], k[r], v[r], tab, D, kr[b], None, vv[b], D, L * D,
                                   sk, sv, ns, D, sk.stride(0) if sk is not None else 0)
            qv = q.view(B, L, H, D).permute(0, 2, 1, 3)
            aov = ao.permute(0, 2, 1, 3)
            full = mode == "full" or L <= 2 * W
            if mfma and full:
                causal_attention(qv, kr, vv, aov)
            elif mfma:
                block_sliding_attention(qv, kr, vv, W, k_raw=k.view(B, L, G, D).permute(0, 2, 1, 3),
                                        n_sink=n_pin, head_dim=D, rope_theta=cfg.rope_theta, out=aov,
                                        angles="double")
            else:
                sinks = None
                if ns and not full:
                    sinks = (st.k_sink_raw[li], st.v_sink[li]) if st is not None else (sk_all, sv_all)
                self._block_attn_split(q.view(B, L, H, D), kr, vv, sinks, ns, ao, full)
            if st is not None:
                self._fill_ring(st, li, k.view(B, L, G, D), v.view(B, L, G, D), last, cnt)
            ops.qlinear(lw.wo, ao.view(N, HD), out=x, accumulate=True)
            ops.qlinear_swiglu(lw.wgu, x, out=hbuf, norm=(lw.ln2, cfg.rms_eps))
            ops.qlinear(lw.wd, hbuf, out=x, accumulate=True)
        if st is not None:
            ids32 = input_ids.to(dev, torch.int32)
            st.tok_cur[:, :cnt].copy_(ids32[:, last * W:L])
            if last >= 1:
                st.tok_prev.copy_(ids32[:, (last - 1) * W:last * W])
            st.pos = L
            if L >= 2 * W:
                self._refresh_prefix(st, seg_active=False)
        h = x.view(B, L, -1)[:, L - 1] if last_only else x
        return h, st

    def _block_attn_split(self, q: torch.Tensor, kr: torch.Tensor, vv: torch.Tensor, sinks, ns: int,
                          ao: torch.Tensor, full: bool) -> None:
        """Block sliding-window (or, ``full``, causal) attention on the split-K decode kernel, for head
        sizes the MFMA prefill kernel does not take: per sequence and W-token query chunk, one call
        over [sinks re-rotated to (i-1)W - S + j | chunk i-1 | chunk i causal].  q / ao: [B, L, H, D];
        kr / vv: [B, G, L, D]; sinks: raw (keys, values) [B, G, >= ns, D] or None."""
        cfg = self.cfg
        B, L, H, D = q.shape
        G, W = kr.shape[1], cfg.window
        tab = self._abs_rows(L)
        # re-rotated sink keys, laid out like the sink values (a span's K and V share strides)
        rot = torch.empty_like(sinks[1][0]) if sinks is not None else None
        scale = 1.0 / math.sqrt(D)
        for b in range(B):
            for i in range((L + W - 1) // W):
                r0, r1 = i * W, min(L, (i + 1) * W)
                spans = []
                if full:
                    lo = 0
                else:
                    lo = max(0, r0 - W)
                    if i >= 2 and sinks is not None:
                        ops.rope_rotate(sinks[0][b][:, :ns], rot[:, :ns], tab[(i - 1) * W - ns:], D)
                        spans.append((rot[None, :, :ns], sinks[1][b][None, :, :ns]))
                if r0 > lo:
                    spans.append((kr[b:b + 1, :, lo:r0], vv[b:b + 1, :, lo:r0]))
                spans.append((kr[b:b + 1, :, r0:r1], vv[b:b + 1, :, r0:r1]))
                ops.attn_decode(q[b, r0:r1], spans, out=ao[b, r0:r1], scale=scale, ws=self.prefill_ws,
                                causal_base=0)

    def _fill_ring(self, st: VAULTv3State, li: int, k: torch.Tensor, v: torch.Tensor, last: int, cnt: int) -> None:
        """Ring rows of layer li after a parallel prefill (src/vault_v3_model.py:2197-2206): the last
        (partial) chunk into cur at re-based positions W + j (j if it is chunk 0), the chunk before
        it into prev at positions j; raw keys and values alongside.  k / v: [B, L, G, D] raw views."""
        W, D = self.cfg.window, self.cfg.head_dim
        for b in range(k.shape[0]):
            for c0, n, rot, raw, vd, row in ((last * W, cnt, st.k_cur, st.kraw_cur, st.v_cur, W if last >= 1 else 0),
                                             ((last - 1) * W, W, st.k_prev, st.kraw_prev, st.v_prev, 0)):
                if c0 < 0:
                    continue
                ops.rope_qkv_write(None, k[b, c0:c0 + n], v[b, c0:c0 + n], self._rows(row), D, rot[li][b],
                                   raw[li][b], vd[li][b], D, W * D)

    def _chunk_recurrent(self, input_ids: torch.Tensor, bud: int, all_logits: bool):
        """Chunk-recurrent prefill / forward for batch 1 (src/vault_v3_model.py:1938-2116)."""
        cfg = self.cfg
        W = cfg.window
        ids_all = input_ids.reshape(-1).to("cpu", torch.int64)
        L = ids_all.numel()
        st = self.new_state(1, seg_budget=bud)
        seg_active = self._seg_active(st, 1)
        limit = min(cfg.max_sink, W, st.sink_cap)
        pin_at = []                     # the pin count each early position saw (resonance, quarantine)
        for p in range(min(L, limit + 1)):
            if st.pin_locked:
                break
            self._auto_pin(st, int(ids_all[p]), p)
            pin_at.append(st.n_pin)
        n_pin_at = lambda p: pin_at[p] if p < len(pin_at) else st.n_pin
        outs = []                       # ("h", hidden rows) of chunk kernels, ("l", logits) of steps
        for ci in range((L + W - 1) // W):
            r0, r1 = ci * W, min(L, (ci + 1) * W)
            clen = r1 - r0
            st.pos = r0
            if ci > 0:
                self._boundary(st, seg_active)
            ch = ids_all[r0:r1]
            bias = None
            if st.res is not None:
                st.tok_cur_h[:clen] = ch.numpy().astype(np.uint32)
                if self._mfma_prefill():
                    # the per-position resonance biases of the chunk, added by the chunk attention
                    bias = self._chunk_bias(st, r0, clen, seg_active, n_pin_at)
                elif self._chunk_resonates(st, r0, clen, seg_active, n_pin_at):
                    # shapes the MFMA attention does not take: the step path, token by token
                    rows = [self._advance(st, ch[j:j + 1], boundary=False) for j in range(clen)]
                    outs.append(("l", torch.cat(rows, dim=0)))
                    continue
            st.tok_cur[0, :clen].copy_(ch.to(torch.int32))
            if seg_active:
                # the chunk's segment ids (host rule, the prompt is on the host), then the open
                # segment's id and length as the device segmenter continues from them
                seg = np.empty(clen, dtype=np.int32)
                s_loc, slen = 0, 0
                for j in range(clen):
                    seg[j] = s_loc
                    slen += 1
                    if j == W - 1 or self._breaks(int(ch[j]), slen):
                        s_loc += 1
                        slen = 0
                st.seg_cur_ids[:clen].copy_(torch.from_numpy(seg))
                st.ctrl[ops.L.SEG_CUR_ID:ops.L.SEG_LEN + 1].copy_(torch.tensor([s_loc, slen], dtype=torch.int32))
            x = ops.embed(self.w.embed, ch.to(self.device), pad_row=0)
            x, feats = self._layers(x, st, pos=r0, seg_active=seg_active, bias=bias)
            if seg_active:
                self._score(st, feats, T=clen, c0=0, first=not st.ema_ready)
                st.ema_ready = True
                if st.res is not None:
                    for j in range(clen):
                        if self._spoofed(st, j, r0 + j, n_pin_at(r0 + j)):
                            st.sc_cur[j:j + 1].fill_(-1.0e30)
            if st.res is not None:
                # the resonance fields as the step loop leaves them after the chunk's last token
                st.pos = r1 - 1
                self._resonance(st, clen - 1, r1 - 1, seg_active, direct=True)
            outs.append(("h", x if all_logits else x[-1:]))
        st.pos = L
        if not all_logits:
            kind, t = outs[-1]
            return (t[-1:] if kind == "h" else None), st, (None if kind == "h" else t[-1:])
        return None, st, torch.cat([self._logits(t) if kind == "h" else t for kind, t in outs], dim=0)

    def _mfma_prefill(self) -> bool:
        """Whether the chunk attention runs on the MFMA prefill kernel (head_dim 128, 1-8 heads per group)."""
        cfg = self.cfg
        return cfg.head_dim == 128 and cfg.n_heads // cfg.n_kv_heads in (1, 2, 4, 6, 8)

    def _chunk_bias(self, st: VAULTv3State, r0: int, clen: int, seg_active: bool, n_pin_at):
        """The chunk-level resonance bias (src/vault_v3_model.py:1718-1793): row j holds the biases the
        step rule gives position r0 + j (runtime/vault3.c:1426-1786, 1976-1988) over the segment bank,
        as (early, late) fp32 tensors [clen, 2, M]: row 0 for the arch heads, row 1 for the sup heads;
        late = (arch, sup), early = (hop1, hop1) at mode-2 positions, else as late; zero rows where the
        mode is 0.  None when no position of the chunk resonates."""
        if not seg_active or r0 < 2 * self.cfg.window or st.res.mem_cnt == 0:
            return None
        M = st.res.mem_cnt
        late = np.zeros((clen, 2, M), dtype=np.float32)
        early = None
        for j in range(clen):
            mode = st.res.update(st.tok_prev_h, st.tok_cur_h, j, r0 + j, n_pin_at(r0 + j))
            if not mode:
                continue
            late[j, 0] = st.res.arch[:M]
            late[j, 1] = st.res.sup[:M]
            if mode == 2:
                if early is None:
                    early = late.copy()
                early[j, 0] = st.res.hop1[:M]
                early[j, 1] = st.res.hop1[:M]
            elif early is not None:
                early[j] = late[j]
        if not late.any() and early is None:
            return None
        lt = torch.from_numpy(late).to(self.device)
        return (lt if early is None else torch.from_numpy(early).to(self.device)), lt

    def _chunk_resonates(self, st: VAULTv3State, r0: int, clen: int, seg_active: bool, n_pin_at) -> bool:
        """Whether the query resonance is active at some position of the chunk [r0, r0 + clen) (the
        host rings hold the previous chunk and this chunk's tokens)."""
        if not seg_active or r0 < 2 * self.cfg.window or st.res.mem_cnt == 0:
            return False
        return any(st.res.update(st.tok_prev_h, st.tok_cur_h, j, r0 + j, n_pin_at(r0 + j)) for j in range(clen))
