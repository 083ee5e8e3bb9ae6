"""Segment-bank merge at a chunk boundary in the C runtime's fp32 arithmetic (TEST INFRASTRUCTURE ONLY).

Restates update_segment_bank with the quarantine before it (runtime/vault3.c:1833-1915, 2079-2088):
a score <= -1e29 marks its local segment, whose scores all become -1e30; per-segment maxima; tokens
t >= t0 of a segment whose maximum is > -1e29 become candidates at position ev*W + t with score
fp32(max - fp32(1e-6 * fp32(global seg id mod 16384))); the seg-id offset advances by the number of
local segments; unless t0 >= W, the bank and the candidates (positions ascending) compete on (score
desc, position asc) for ``budget`` slots, kept in chronological order.  The top-B selection is the
reference's sort-then-resort (a full ordering by np.lexsort here), independent of the device's
rank counting.
"""
from __future__ import annotations

import numpy as np


def evict(sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg, offset: int, ev: int, t0: int, budget: int):
    """Returns (sc after quarantine, new offset, new bank (pos, score, tok, seg), idx_old, idx_new) with
    idx_old[j] / idx_new[j] the source of new slot j (old bank slot / evicted-chunk row, else -1)."""
    sc = np.asarray(sc, dtype=np.float32).copy()
    seg = np.asarray(seg, dtype=np.int64)
    W = sc.size
    if np.any(sc <= np.float32(-1.0e29)):
        bad = np.zeros(W + 1, dtype=bool)
        bad[seg[sc <= np.float32(-1.0e29)]] = True
        sc[bad[seg]] = np.float32(-1.0e30)
    n_loc = int(seg.max()) + 1
    mx = np.full(n_loc, np.float32(-3.4e38), dtype=np.float32)
    np.maximum.at(mx, seg, sc)
    M = len(mem_pos)
    new_off = offset + n_loc
    keep_all = (np.asarray(mem_pos, np.int64), np.asarray(mem_score, np.float32), np.asarray(mem_tok, np.int64),
                np.asarray(mem_seg, np.int64))
    ident = np.arange(M, dtype=np.int64)
    if t0 >= W:
        return sc, new_off, keep_all, ident, np.full(M, -1, dtype=np.int64)
    t = np.arange(t0, W)
    smx = mx[seg[t]]
    ok = smx > np.float32(-1.0e29)
    t = t[ok]
    full = seg[t] + offset
    g = (full & 16383).astype(np.float32)
    c_sc = (smx[ok] - (np.float32(1e-6) * g).astype(np.float32)).astype(np.float32)
    pos = np.concatenate([keep_all[0], ev * W + t])
    score = np.concatenate([keep_all[1], c_sc]).astype(np.float32)
    toks = np.concatenate([keep_all[2], np.asarray(tok, np.int64)[t]])
    segs = np.concatenate([keep_all[3], full])
    src_old = np.concatenate([ident, np.full(t.size, -1)])
    src_new = np.concatenate([np.full(M, -1), t])
    n = pos.size
    if n > budget:
        order = np.lexsort((np.arange(n), -score.astype(np.float64)))[:budget]
        win = np.sort(order)
    else:
        win = np.arange(n)
    return sc, new_off, (pos[win], score[win], toks[win], segs[win]), src_old[win], src_new[win]
