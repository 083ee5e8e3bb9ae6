"""Host control logic of the decode loop (libvault_amd's C++ unit, include/vault_amd.h
"host control logic"): segment-memory resonance, the authority-spoof quarantine and the output
governor.  The classes own their native handles; token strings come from a model's TokenTable.

Reference semantics: runtime/vault3.c:1034-1831 and 2814-3193; src/vault_v3_model.py:397-560
(CAAIGovernor) and 1249-1830 (resonance, spoof check).  The biased heads and layers follow
runtime/vault3.c:1976-1988: of each group of ``grp`` query heads, the first grp // 3 take no bias,
the next ones the arch bias and the last (grp - grp // 3) // 2 the sup bias, in layers
[L // 4, L - L // 14); in mode 2 the layers below L // 2 take the hop-1 bias on every biased head.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence, Tuple

import numpy as np
import torch

from . import _lib as L
from .tokens import TokenTable


def _u32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int64).astype(np.uint32))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


class TokenBytes:
    """Native copy of a model's token byte strings (vgx_tokens)."""

    def __init__(self, tokens: Sequence[bytes]):
        toks = [bytes(t) for t in tokens]
        off = np.zeros(len(toks) + 1, dtype=np.uint64)
        off[1:] = np.cumsum([len(t) for t in toks], dtype=np.uint64)
        pool = np.frombuffer(b"".join(toks) or b"\0", dtype=np.uint8)
        self._lib = L.load()
        self.n = len(toks)
        self.handle = self._lib.vgx_tokens_create(_ptr(pool), _ptr(off), self.n)
        if not self.handle:
            raise ValueError("vgx_tokens_create rejected the token table")

    @classmethod
    def of(cls, table: TokenTable) -> "TokenBytes":
        return cls(table.tokens)

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            self._lib.vgx_tokens_destroy(h)


def head_classes(n_heads: int, n_kv_heads: int) -> np.ndarray:
    """Per query head: 0 = no bias, 1 = arch, 2 = sup (runtime/vault3.c:1976-1988)."""
    grp = n_heads // n_kv_heads
    free_h = grp // 3
    arch_end = grp - (grp - free_h) // 2
    hr = np.arange(n_heads) % grp
    return np.where(hr < free_h, 0, np.where(hr < arch_end, 1, 2)).astype(np.int64)


def biased_layers(n_layers: int) -> Tuple[int, int, int]:
    """(first biased layer, first layer past the hop-1 range, end of the biased range)."""
    return n_layers // 4, n_layers // 2, n_layers - n_layers // 14


class Resonance:
    """Shingle index over one state's segment bank and the per-step query resonance."""

    def __init__(self, tokens: TokenBytes, window: int, seg_cap: int, n_sink: int, im_start_id: int, im_end_id: int):
        self._lib = L.load()
        self._tokens = tokens                      # kept alive: the handle reads its bytes
        self.seg_cap = int(seg_cap)
        self.handle = self._lib.vgx_res_create(tokens.handle, int(window), self.seg_cap, int(n_sink), int(im_start_id),
                                               int(im_end_id))
        if not self.handle:
            raise ValueError("vgx_res_create failed")
        self.mem_cnt = 0
        self.n_segs = 0
        self.arch = np.zeros(max(1, self.seg_cap), dtype=np.float32)
        self.sup = np.zeros_like(self.arch)
        self.hop1 = np.zeros_like(self.arch)

    def rebuild(self, mem_tok, mem_seg) -> int:
        t, s = _u32(mem_tok), _u32(mem_seg)
        if t.shape != s.shape:
            raise ValueError("mem_tok / mem_seg lengths differ")
        n = int(self._lib.vgx_res_rebuild(self.handle, _ptr(t), _ptr(s), t.size))
        L.check(min(n, 0), "vgx_res_rebuild")
        self.mem_cnt, self.n_segs = t.size, n
        return n

    def update(self, tok_prev, tok_cur, c: int, pos: int, n_pin: int) -> int:
        """Mode 0 / 1 / 2 of this step; self.arch / sup / hop1[:mem_cnt] hold the biases (hop1 in mode 2)."""
        p, q = _u32(tok_prev), _u32(tok_cur)
        m = int(self._lib.vgx_res_update(self.handle, _ptr(p), _ptr(q), int(c), int(pos), int(n_pin),
                                         _ptr(self.arch), _ptr(self.sup), _ptr(self.hop1)))
        L.check(min(m, 0), "vgx_res_update")
        return m

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            self._lib.vgx_res_destroy(h)


def spoof_check(tokens: TokenBytes, tok_prev, tok_cur, window: int, c: int, pos: int, n_pin: int, n_sink: int) -> bool:
    p, q = _u32(tok_prev), _u32(tok_cur)
    r = int(L.load().vgx_spoof_check(tokens.handle, _ptr(p), _ptr(q), int(window), int(c), int(pos), int(n_pin),
                                     int(n_sink)))
    L.check(min(r, 0), "vgx_spoof_check")
    return r == 1


class Governor:
    """Output governor (CAAIGovernor, src/vault_v3_model.py:397-560; runtime/vault3.c:2814-3193).

    ``govern_logits(logits)`` masks (-3.4e38) the candidates of a device logits row whose bytes would
    complete a rule; the candidates come from the device (ops.topk), the rule test runs here."""

    MASK = -3.4e38
    CAND = 256          # four passes over at most 64 candidates

    def __init__(self, tokens: TokenBytes, eos_id: int, im_start_id: int, im_end_id: int):
        self._lib = L.load()
        self._tokens = tokens
        self.handle = self._lib.vgx_gov_create(tokens.handle, int(eos_id), int(im_start_id), int(im_end_id))
        if not self.handle:
            raise ValueError("vgx_gov_create failed")
        self._masked = np.zeros(self.CAND, dtype=np.int64)

    @classmethod
    def from_system_prompt(cls, sys_text: str | bytes, tokens: TokenBytes, eos_id: int, im_start_id: int,
                           im_end_id: int) -> "Governor":
        g = cls(tokens, eos_id, im_start_id, im_end_id)
        g.arm_system(sys_text)
        return g

    def arm_system(self, sys_text: str | bytes) -> int:
        raw = sys_text.encode("utf-8") if isinstance(sys_text, str) else bytes(sys_text)
        buf = C.create_string_buffer(raw, len(raw))
        return int(self._lib.vgx_gov_arm_system(self.handle, buf, len(raw)))

    def add_rule(self, pat: str | bytes) -> int:
        raw = pat.encode("utf-8") if isinstance(pat, str) else bytes(pat)
        buf = C.create_string_buffer(raw, len(raw))
        return int(self._lib.vgx_gov_add_rule(self.handle, buf, len(raw)))

    @property
    def active(self) -> bool:
        return bool(self._lib.vgx_gov_active(self.handle))

    def reset_stream(self) -> None:
        self._lib.vgx_gov_reset_stream(self.handle)

    def commit(self, tid: int) -> None:
        L.check(self._lib.vgx_gov_commit(self.handle, int(tid)), "vgx_gov_commit")

    def screen(self, cand_idx, cand_val, top_k_guard: int, vocab: int) -> np.ndarray:
        """Ids to mask given the row's top candidates (value desc, index asc)."""
        i = np.ascontiguousarray(cand_idx, dtype=np.int64)
        v = np.ascontiguousarray(cand_val, dtype=np.float32)
        n = int(self._lib.vgx_gov_screen(self.handle, _ptr(i), _ptr(v), i.size, int(top_k_guard), int(vocab),
                                         _ptr(self._masked), self._masked.size))
        L.check(min(n, 0), "vgx_gov_screen")
        return self._masked[:n].copy()

    def govern_logits(self, logits: torch.Tensor, top_k_guard: int = 0, ws=None) -> np.ndarray:
        """Mask one device row [V] (or [1, V]) in place; returns the masked ids."""
        if not self.active:
            return self._masked[:0].copy()
        from . import ops
        row = logits.view(1, -1)
        idx, val = ops.topk(row, min(self.CAND, row.shape[1]), ws=ws)
        masked = self.screen(idx[0].cpu().numpy(), val[0].cpu().numpy(), top_k_guard, row.shape[1])
        if masked.size:
            row[0].index_fill_(0, torch.from_numpy(masked).to(row.device), self.MASK)
        return masked

    def __del__(self):
        h, self.handle = getattr(self, "handle", None), None
        if h:
            self._lib.vgx_gov_destroy(h)
