"""Float64 restatement of the VAULT v3 streaming decode step (TEST INFRASTRUCTURE ONLY).

Follows src/vault_v3_model.py (step :2214-2311, boundary :1858-1935, prefix re-rotation
:1842-1856, attention step :1072-1139, scorer :870-883) and runtime/vault3.c (v3_step :2034-2222,
update_segment_bank :1833-1915), with the token-byte rules of either reference (see
``OracleModel.__init__``); shingles, resonance biases and spoof quarantine are not modelled, so the
token strings of a comparison must produce no shingles (seg biases stay inactive).  RoPE uses the C runtime's angles (double-precision angle, fp32 cos/sin
of a fp32 inverse frequency, runtime/vault3.c:840-849, 2126-2133, 866-891) by default.

prefill() and forward() are sequences of step() calls: the reference asserts both equal the
step-by-step stream (tests/test_vault_v3.py:52-90).

Weights are given as a dict name -> float array (the dequantized fp32 weights).
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import numpy as np

from . import cmath
from . import rope as orope
from . import tokens as otok


def _gelu_c(x):
    """The C runtime's scorer GELU (runtime/vault3.c:118-129, 974: A&S 7.1.26 erf, fp32), which the
    segment scores follow; src/vault_v3_model.py:882 uses the exact erf (within 1.5e-7 of it)."""
    return cmath.geluf(np.asarray(x, dtype=np.float32)).astype(np.float64)


@dataclass
class OState:
    pos: int
    n_pin: int
    pin_locked: bool
    seg_budget: int
    k_prev: np.ndarray
    k_cur: np.ndarray
    v_prev: np.ndarray
    v_cur: np.ndarray
    kraw_prev: np.ndarray
    kraw_cur: np.ndarray
    k_sink_raw: np.ndarray
    k_sink_rot: np.ndarray
    v_sink: np.ndarray
    k_seg_raw: np.ndarray
    k_seg_rot: np.ndarray
    v_seg: np.ndarray
    saw_im_start: bool = False
    awaiting_sys_nl: bool = False
    tok_prev: np.ndarray = None
    tok_cur: np.ndarray = None
    sc_prev: np.ndarray = None
    sc_cur: np.ndarray = None
    seg_prev: np.ndarray = None
    seg_cur: np.ndarray = None
    seg_id_offset: int = 0
    cur_seg_id: int = 0
    seg_len: int = 0
    mem_pos: np.ndarray = field(default_factory=lambda: np.zeros(0, dtype=np.int64))
    mem_score: np.ndarray = field(default_factory=lambda: np.zeros(0))
    ema_ready: bool = False
    ema: Optional[np.ndarray] = None


def bf16_round(x: np.ndarray) -> np.ndarray:
    """float -> fp32 -> bf16 (round to nearest even) -> float64."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


class OracleModel:
    """kv="bf16" stores every cached key/value rounded to bf16 (the model's bf16 KV cache: keys are
    rotated in fp32 and rounded on store, raw keys and values rounded on store)."""

    def __init__(self, cfg, weights: Dict[str, np.ndarray], table=orope.table_c, kv: str = "fp32",
                 token_bytes=None, newline_id: int = 198):
        """token_bytes: per-id byte strings (the VLT3 file's VTOK) or None.  With them, break tiers
        and the system-role test follow the bytes and ``newline_id`` is the byte map's entry for
        '\n' (runtime/vault3.c:937-959, 1920-1928, 2047); without them every tier is 0, the system
        role is cfg.system_tok_id and the newline id 198 (src/vault_v3_model.py:2224-2268)."""
        self.cfg = cfg
        self.w = {k: np.asarray(v, dtype=np.float64) for k, v in weights.items()}
        self.table = table
        self.has_scorer = cfg.has_seg_scorer and "seg_scorer.ln.weight" in weights
        self._kv = bf16_round if kv == "bf16" else (lambda a: np.asarray(a, dtype=np.float64))
        self.token_bytes = token_bytes
        self.newline_id = newline_id if token_bytes is not None else 198

    def _bytes(self, tid: int) -> bytes:
        tb = self.token_bytes
        return tb[tid] if tb is not None and 0 <= tid < len(tb) else b""

    def _is_system(self, tid: int) -> bool:
        if self.token_bytes is None:
            return tid == self.cfg.system_tok_id
        return otok.system_role(self._bytes(tid))

    def _seg_break(self, tid: int, seg_len: int) -> bool:
        """runtime/vault3.c:2109-2122; src/vault_v3_model.py:2260-2268."""
        c = self.cfg
        tr = otok.tier(self._bytes(tid))
        t2 = max(c.seg_min, (c.seg_max * 2) // 3)
        t3 = max(c.seg_min, c.seg_max - 8 if c.seg_max > 8 else c.seg_min)
        return (seg_len >= c.seg_max or (tr == 1 and seg_len >= c.seg_min) or (tr == 2 and seg_len >= t2)
                or (tr == 3 and seg_len >= t3))

    # ------------------------------------------------------------------ state
    def new_state(self, seg_budget: Optional[int] = None) -> OState:
        c = self.cfg
        W, G, D, Lr = c.window, c.n_kv_heads, c.head_dim, c.n_layers
        S_cap = c.sink_cap
        bud = c.seg_budget if seg_budget is None else int(seg_budget)
        M_cap = max(1, bud)
        z = lambda n: np.zeros((Lr, G, n, D))
        st = OState(pos=0, n_pin=min(c.n_sink, W), pin_locked=not c.auto_pin_system, seg_budget=bud,
                    k_prev=z(W), k_cur=z(W), v_prev=z(W), v_cur=z(W), kraw_prev=z(W), kraw_cur=z(W),
                    k_sink_raw=z(S_cap), k_sink_rot=z(S_cap), v_sink=z(S_cap),
                    k_seg_raw=z(M_cap), k_seg_rot=z(M_cap), v_seg=z(M_cap))
        st.tok_prev = np.zeros(W, dtype=np.int64)
        st.tok_cur = np.zeros(W, dtype=np.int64)
        st.sc_prev = np.zeros(W)
        st.sc_cur = np.zeros(W)
        st.seg_prev = np.zeros(W, dtype=np.int64)
        st.seg_cur = np.zeros(W, dtype=np.int64)
        st.ema = np.zeros(max(1, len(c.seg_layers) * c.d_model))
        return st

    def set_pinned(self, st: OState, n: int) -> None:
        st.n_pin = max(0, min(int(n), self.cfg.window, st.k_sink_raw.shape[2]))
        st.pin_locked = True

    # ------------------------------------------------------------------ pieces
    def _cs(self, positions):
        c, s = self.table(positions, self.cfg.head_dim, self.cfg.rope_theta)
        return c.astype(np.float64), s.astype(np.float64)

    @staticmethod
    def _rms(x, g, eps):
        return g * (x / np.sqrt(np.mean(x * x) + eps))

    def _scorer(self, f):
        w = self.w
        mu = f.mean()
        var = ((f - mu) ** 2).mean()
        h = (f - mu) / np.sqrt(var + 1e-5) * w["seg_scorer.ln.weight"] + w["seg_scorer.ln.bias"]
        h = _gelu_c(w["seg_scorer.fc1.weight"] @ h + w["seg_scorer.fc1.bias"])
        return float(w["seg_scorer.fc2.weight"].reshape(-1) @ h + w["seg_scorer.fc2.bias"][0])

    def _auto_pin(self, st: OState, tid: int) -> None:
        """Online ChatML system-prompt pinning (src/vault_v3_model.py:2224-2252)."""
        c = self.cfg
        pos = st.pos
        limit = min(c.max_sink, c.window, st.k_sink_raw.shape[2])
        if pos == 0:
            if tid == c.im_start_id and limit >= 2:
                st.saw_im_start = True
            else:
                st.pin_locked = True
        elif pos == 1 and st.saw_im_start:
            if not self._is_system(tid):
                st.saw_im_start = False
                st.pin_locked = True
        elif st.saw_im_start and pos < limit:
            if st.awaiting_sys_nl:
                st.n_pin = max(st.n_pin, pos + 1 if tid == self.newline_id else pos)
                st.pin_locked = True
                st.awaiting_sys_nl = False
            elif tid == c.im_end_id:
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

    def _boundary(self, st: OState, seg_active: bool) -> None:
        """Chunk boundary at c == 0, pos > 0 (src/vault_v3_model.py:1858-1935; runtime/vault3.c:2076-2105)."""
        c = self.cfg
        W = c.window
        pos = st.pos
        if pos >= 2 * W and seg_active and st.seg_budget > 0:
            ev = pos // W - 2
            sc = st.sc_prev.copy()
            seg_ids = st.seg_prev
            bad = sc <= -1.0e29
            if bad.any():
                bad_seg = np.zeros(int(seg_ids.max()) + 1, dtype=bool)
                bad_seg[seg_ids[bad]] = True
                sc[bad_seg[seg_ids]] = -1.0e30
                st.sc_prev = sc
            n_loc = int(seg_ids.max()) + 1
            mx = np.full(n_loc, -np.inf)
            np.maximum.at(mx, seg_ids, sc)
            full_seg = seg_ids + st.seg_id_offset
            cand_all = mx[seg_ids] - 1e-6 * (full_seg % 16384).astype(np.float64)
            st.seg_id_offset += n_loc
            t0 = st.n_pin if ev == 0 else 0
            if t0 < W:
                t = np.arange(t0, W)
                ok = cand_all[t0:] > -1.0e29
                c_pos = ev * W + t[ok]
                c_sc = cand_all[t0:][ok]
                c_src = t[ok]
                M = st.mem_pos.size
                all_pos = np.concatenate([st.mem_pos, c_pos])
                all_sc = np.concatenate([st.mem_score, c_sc])
                if all_pos.size <= st.seg_budget:
                    win = np.arange(all_pos.size)
                else:
                    order = np.argsort(-all_sc, kind="stable")[:st.seg_budget]
                    win = np.sort(order)
                keep = win[win < M]
                add = win[win >= M] - M
                nk, na = keep.size, add.size
                old_k, old_v = st.k_seg_raw[:, :, keep].copy(), st.v_seg[:, :, keep].copy()
                st.k_seg_raw[:, :, :nk] = old_k
                st.v_seg[:, :, :nk] = old_v
                st.k_seg_raw[:, :, nk:nk + na] = st.kraw_prev[:, :, c_src[add]]
                st.v_seg[:, :, nk:nk + na] = st.v_prev[:, :, c_src[add]]
                st.mem_pos = all_pos[win]
                st.mem_score = all_sc[win]
        st.k_prev, st.k_cur = st.k_cur.copy(), st.k_prev
        st.v_prev, st.v_cur = st.v_cur.copy(), st.v_prev
        st.kraw_prev, st.kraw_cur = st.kraw_cur.copy(), st.kraw_prev
        if pos >= 2 * W:
            cs, sn = self._cs([-W])
            st.k_prev = self._kv(orope.rotate(st.k_prev, cs, sn))
        st.tok_prev, st.tok_cur = st.tok_cur.copy(), st.tok_prev
        st.sc_prev, st.sc_cur = st.sc_cur.copy(), st.sc_prev
        st.seg_prev, st.seg_cur = st.seg_cur.copy(), st.seg_prev
        st.cur_seg_id = 0
        st.seg_len = 0
        if pos >= 2 * W:
            self._refresh_prefix(st, seg_active)

    def _refresh_prefix(self, st: OState, seg_active: bool) -> None:
        """Segment keys at positions [-M, 0), sinks at [-(M+S), -M) (src/vault_v3_model.py:1842-1856)."""
        M = st.mem_pos.size if seg_active else 0
        S = st.n_pin
        if M:
            cs, sn = self._cs(np.arange(-M, 0))
            st.k_seg_rot[:, :, :M] = self._kv(orope.rotate(st.k_seg_raw[:, :, :M], cs, sn))
        if S:
            cs, sn = self._cs(np.arange(-(M + S), -M))
            st.k_sink_rot[:, :, :S] = self._kv(orope.rotate(st.k_sink_raw[:, :, :S], cs, sn))

    # ------------------------------------------------------------------ step
    def step(self, tok: int, st: OState) -> np.ndarray:
        c = self.cfg
        w = self.w
        W, D, H, G = c.window, c.head_dim, c.n_heads, c.n_kv_heads
        grp = H // G
        pos = st.pos
        cc = pos % W
        seg_active = self.has_scorer and st.seg_budget > 0
        if not st.pin_locked:
            self._auto_pin(st, tok)
        if cc == 0 and pos > 0:
            self._boundary(st, seg_active)
        st.tok_cur[cc] = tok
        if seg_active:
            st.seg_cur[cc] = st.cur_seg_id
            st.seg_len += 1
            if cc == W - 1 or self._seg_break(tok, st.seg_len):
                st.cur_seg_id += 1
                st.seg_len = 0
        eff = W + cc if pos >= W else cc
        cs, sn = self._cs([eff])
        x = w["embed_tokens.weight"][tok].copy()
        S_cap = st.k_sink_raw.shape[2]
        feats = []
        for li in range(c.n_layers):
            p = f"layers.{li}."
            if seg_active and li in c.seg_layers:
                feats.append((c.seg_layers.index(li), x.copy()))
            u = self._rms(x, w[p + "input_layernorm.weight"], c.rms_eps)
            q = (w[p + "self_attn.q_proj.weight"] @ u + w[p + "self_attn.q_proj.bias"]).reshape(H, D)
            k = (w[p + "self_attn.k_proj.weight"] @ u + w[p + "self_attn.k_proj.bias"]).reshape(G, D)
            v = (w[p + "self_attn.v_proj.weight"] @ u + w[p + "self_attn.v_proj.bias"]).reshape(G, D)
            qr = orope.rotate(q, cs, sn)
            kr = orope.rotate(k, cs, sn)
            st.k_cur[li, :, cc] = self._kv(kr)
            st.v_cur[li, :, cc] = self._kv(v)
            st.kraw_cur[li, :, cc] = self._kv(k)
            if pos < S_cap:
                st.k_sink_raw[li, :, pos] = self._kv(k)
                st.v_sink[li, :, pos] = self._kv(v)
            parts_k, parts_v = [], []
            if pos >= 2 * W:
                S = st.n_pin
                M = st.mem_pos.size if seg_active else 0
                parts_k += [st.k_sink_rot[li, :, :S], st.k_seg_rot[li, :, :M]]
                parts_v += [st.v_sink[li, :, :S], st.v_seg[li, :, :M]]
            if pos >= W:
                parts_k.append(st.k_prev[li])
                parts_v.append(st.v_prev[li])
            parts_k.append(st.k_cur[li, :, :cc + 1])
            parts_v.append(st.v_cur[li, :, :cc + 1])
            K = np.concatenate(parts_k, axis=1)
            V = np.concatenate(parts_v, axis=1)
            o = np.empty((H, D))
            for h in range(H):
                s = K[h // grp] @ qr[h] / math.sqrt(D)
                pr = np.exp(s - s.max())
                o[h] = (pr / pr.sum()) @ V[h // grp]
            x = x + w[p + "self_attn.o_proj.weight"] @ o.reshape(-1)
            u = self._rms(x, w[p + "post_attention_layernorm.weight"], c.rms_eps)
            g = w[p + "mlp.gate_proj.weight"] @ u
            up = w[p + "mlp.up_proj.weight"] @ u
            x = x + w[p + "mlp.down_proj.weight"] @ (g / (1.0 + np.exp(-g)) * up)
        if seg_active:
            f = np.concatenate([v for _, v in sorted(feats, key=lambda t: t[0])])
            raw = self._scorer(f)
            sc = raw
            if not st.ema_ready:
                st.ema = f.copy()
                st.ema_ready = True
            else:
                hab = self._scorer(f - 0.65 * st.ema)
                st.ema = 0.985 * st.ema + 0.015 * f
                sc = raw + 0.35 * max(0.0, hab - raw)
            st.sc_cur[cc] = sc
        st.pos = pos + 1
        h = self._rms(x, w["norm.weight"], c.rms_eps)
        return w["embed_tokens.weight"] @ h

    def forward_block(self, ids, mode: str = "block", n_pin: Optional[int] = None,
                      sink_pos=None) -> np.ndarray:
        """Logits of every position of one sequence by the parallel form (src/vault_v3_model.py:
        1048-1061, 2136-2151): RoPE at absolute positions, full causal attention when mode == "full"
        or L <= 2W, else block sliding-window attention with ``n_pin`` (default n_sink) sinks
        re-rotated to their virtual positions (``attention.block_sliding``; ``sink_pos`` replaces the
        position rule, for tests that plant a mistake)."""
        from . import attention as oatt
        c, w = self.cfg, self.w
        H, G, D, W = c.n_heads, c.n_kv_heads, c.head_dim, c.window
        ids = np.asarray(ids, dtype=np.int64)
        L = ids.size
        S = min(c.n_sink if n_pin is None else n_pin, L)
        x = w["embed_tokens.weight"][ids].copy()
        cs, sn = self._cs(np.arange(L))
        rms = lambda a, g: g * (a / np.sqrt(np.mean(a * a, axis=-1, keepdims=True) + c.rms_eps))
        rot = lambda a: np.transpose(orope.rotate(np.transpose(a, (1, 0, 2)), cs, sn), (1, 0, 2))
        kw = {} if sink_pos is None else {"sink_pos": sink_pos}
        for li in range(c.n_layers):
            p = f"layers.{li}."
            u = rms(x, w[p + "input_layernorm.weight"])
            q = (u @ w[p + "self_attn.q_proj.weight"].T + w[p + "self_attn.q_proj.bias"]).reshape(L, H, D)
            k = (u @ w[p + "self_attn.k_proj.weight"].T + w[p + "self_attn.k_proj.bias"]).reshape(L, G, D)
            v = (u @ w[p + "self_attn.v_proj.weight"].T + w[p + "self_attn.v_proj.bias"]).reshape(L, G, D)
            qr, kr = rot(q), rot(k)
            if mode == "full" or L <= 2 * W:
                o = oatt.chunk(qr, [], np.transpose(kr, (1, 0, 2)), np.transpose(v, (1, 0, 2)))
            else:
                o = oatt.block_sliding(qr, kr, v, k, W, S, c.rope_theta, table=self.table, **kw)
            x = x + o.reshape(L, H * D) @ w[p + "self_attn.o_proj.weight"].T
            u = rms(x, w[p + "post_attention_layernorm.weight"])
            g = u @ w[p + "mlp.gate_proj.weight"].T
            up = u @ w[p + "mlp.up_proj.weight"].T
            x = x + (g / (1.0 + np.exp(-g)) * up) @ w[p + "mlp.down_proj.weight"].T
        return rms(x, w["norm.weight"]) @ w["embed_tokens.weight"].T

    def stream(self, ids, st: Optional[OState] = None, positions=None) -> np.ndarray:
        """Logits for every token of ``ids`` stepped from ``st`` (a fresh state if None)."""
        st = st or self.new_state()
        out = [self.step(int(t), st) for t in ids]
        return np.stack(out)
