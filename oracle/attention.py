"""Attention oracles in float64 (TEST INFRASTRUCTURE ONLY).

``decode``: one query per (batch, head) over the concatenated key spans
[sink n_pin | segment memory M | prev W | cur c+1] with GQA (kv head g = h // (H/G)), scale
1/sqrt(D), and an optional additive fp32 bias on one span per head
(src/vault_v3_model.py:1098-1136 incl. _expand_kv :797-802; runtime/vault3.c:1958-2032).

``chunk``: a block of queries over prefix spans plus a causal current span, query t seeing
current keys j <= t (src/vault_v3_model.py:2029-2037, 2064-2093).

``block_sliding``: whole-sequence block sliding-window attention with re-rotated sinks: a query
in chunk i sees all of chunk i-1, chunk i causally, and for i >= 2 the first S keys re-rotated
to virtual positions (i-1)W - S + j (src/vault_v3_model.py:805-863).  Built as a dense masked
softmax from that visibility rule.
"""
from __future__ import annotations

import numpy as np

from . import rope as _rope


def _softmax_rows(s: np.ndarray) -> np.ndarray:
    m = np.max(s, axis=-1, keepdims=True)
    e = np.exp(s - m)
    return e / np.sum(e, axis=-1, keepdims=True)


def decode(q: np.ndarray, spans: list, bias: np.ndarray | None = None, bias_span: int = -1) -> np.ndarray:
    """q: [B, H, D]; spans: list of (K [B, G, n, D], V [B, G, n, D]); bias: [H, n_bias_span]."""
    q = np.asarray(q, dtype=np.float64)
    B, H, D = q.shape
    K = np.concatenate([np.asarray(k, dtype=np.float64) for k, _ in spans], axis=2)
    V = np.concatenate([np.asarray(v, dtype=np.float64) for _, v in spans], axis=2)
    G = K.shape[1]
    grp = H // G
    Ke = np.repeat(K, grp, axis=1)   # [B, H, n, D]
    Ve = np.repeat(V, grp, axis=1)
    s = np.einsum("bhd,bhnd->bhn", q, Ke) / np.sqrt(D)
    if bias is not None:
        off = sum(np.asarray(k).shape[2] for k, _ in spans[:bias_span])
        n_b = np.asarray(spans[bias_span][0]).shape[2]
        s[:, :, off:off + n_b] += np.asarray(bias, dtype=np.float64)[None, :, :n_b]
    p = _softmax_rows(s)
    return np.einsum("bhn,bhnd->bhd", p, Ve)


def chunk(q: np.ndarray, prefix: list, k_cur: np.ndarray, v_cur: np.ndarray, bias=None, bias_span=-1) -> np.ndarray:
    """q: [T, H, D]; prefix: list of (K [G, n, D], V [G, n, D]); k_cur/v_cur: [G, T, D] -> [T, H, D].
    ``bias`` on prefix run ``bias_span``: [H, n] (every query) or [T, H, n] (per query row: the
    chunk-level resonance bias added to the scores, src/vault_v3_model.py:2083-2090)."""
    q = np.asarray(q, dtype=np.float64)
    T, H, D = q.shape
    Ks = [np.asarray(k, dtype=np.float64) for k, _ in prefix] + [np.asarray(k_cur, dtype=np.float64)]
    Vs = [np.asarray(v, dtype=np.float64) for _, v in prefix] + [np.asarray(v_cur, dtype=np.float64)]
    K = np.concatenate(Ks, axis=1)
    V = np.concatenate(Vs, axis=1)
    G = K.shape[0]
    grp = H // G
    P = K.shape[1] - T
    Ke = np.repeat(K, grp, axis=0)
    Ve = np.repeat(V, grp, axis=0)
    s = np.einsum("thd,hnd->htn", q, Ke) / np.sqrt(D)
    if bias is not None:
        off = sum(np.asarray(k).shape[1] for k, _ in prefix[:bias_span])
        n_b = np.asarray(prefix[bias_span][0]).shape[1]
        b = np.asarray(bias, dtype=np.float64)
        s[:, :, off:off + n_b] += b[:, None, :n_b] if b.ndim == 2 else b.transpose(1, 0, 2)[:, :, :n_b]
    t = np.arange(T)[:, None]
    j = np.arange(P + T)[None, :]
    s = np.where((j <= P + t)[None], s, -np.inf)
    p = _softmax_rows(s)
    return np.einsum("htn,hnd->thd", p, Ve)


def sink_positions(i: int, W: int, S: int) -> np.ndarray:
    """Virtual positions of the S sinks for query chunk i >= 2 (src/vault_v3_model.py:805-809)."""
    return np.maximum(0, (i - 1) * W - S + np.arange(S))


def block_sliding(q: np.ndarray, k: np.ndarray, v: np.ndarray, k_raw: np.ndarray, W: int, S: int,
                  theta: float, table=_rope.table_torch, sink_store=None, sink_pos=sink_positions) -> np.ndarray:
    """q: [L, H, D] post-RoPE, k/v: [L, G, D] post-RoPE / values, k_raw: [L, G, D] pre-RoPE.
    ``sink_store``: applied to the re-rotated sink keys before use (a bf16 rounding, for callers whose
    re-rotated sinks are stored in bf16).  Returns [L, H, D]."""
    q = np.asarray(q, dtype=np.float64)
    L, H, D = q.shape
    G = k.shape[1]
    grp = H // G
    out = np.zeros((L, H, D))
    n = (L + W - 1) // W
    S = min(S, L)
    for i in range(n):
        r0, r1 = i * W, min(L, (i + 1) * W)
        lo = max(0, (i - 1) * W)
        keys = [np.asarray(k[lo:r1], dtype=np.float64)]
        vals = [np.asarray(v[lo:r1], dtype=np.float64)]
        if i >= 2 and S > 0:
            c, s_ = table(sink_pos(i, W, S), D, theta)
            ks = _rope.rotate(np.transpose(np.asarray(k_raw[:S], dtype=np.float64), (1, 0, 2)), c, s_)
            if sink_store is not None:
                ks = sink_store(ks)
            keys.insert(0, np.transpose(ks, (1, 0, 2)))
            vals.insert(0, np.asarray(v[:S], dtype=np.float64))
        K = np.concatenate(keys, axis=0)   # [nk, G, D]
        V = np.concatenate(vals, axis=0)
        nk = K.shape[0]
        Ke = np.repeat(K, grp, axis=1)
        Ve = np.repeat(V, grp, axis=1)
        qq = q[r0:r1]
        s = np.einsum("thd,nhd->htn", qq, Ke) / np.sqrt(D)
        T = r1 - r0
        P = nk - T
        t = np.arange(T)[:, None]
        j = np.arange(nk)[None, :]
        s = np.where((j <= P + t)[None], s, -np.inf)
        p = _softmax_rows(s)
        out[r0:r1] = np.einsum("htn,nhd->thd", p, Ve)
    return out
