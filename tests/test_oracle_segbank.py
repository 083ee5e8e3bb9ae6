"""The fp32 segment-bank merge restatement (oracle/segbank.py) checked by the properties that define
it (runtime/vault3.c:1833-1915): exactly min(budget, bank + candidates) winners, kept in chronological
order; every winner ranks above every loser by (score desc, position asc); quarantined segments
and the pinned prefix of chunk 0 contribute nothing; the seg-id offset advances by the local segment
count; and a bank that fits is kept whole.  The device merge is checked against it on the GPU, and
both are pinned end to end by the model's segment-memory slots against the reference runtime."""
import numpy as np
import pytest

from oracle import segbank


def _case(rng, W, M, levels, quarantine, ev=11):
    seg = np.sort(rng.integers(0, max(1, W // 5), W))
    seg = np.unique(seg, return_inverse=True)[1].astype(np.int64)          # consecutive local ids
    sc = (rng.integers(0, levels, W) / levels).astype(np.float32)           # few levels: many ties
    if quarantine:
        sc[rng.integers(0, W, 3)] = np.float32(-1.0e30)
    tok = rng.integers(0, 1000, W)
    mem_pos = np.sort(rng.choice(ev * W, M, replace=False)).astype(np.int64)    # before the evicted chunk
    mem_score = (rng.integers(0, levels, M) / levels).astype(np.float32)
    return sc, seg, tok, mem_pos, mem_score, rng.integers(0, 1000, M), rng.integers(0, 500, M)


@pytest.mark.parametrize("W,M,budget,levels,t0,quar", [
    (64, 0, 12, 4, 0, False), (64, 12, 12, 4, 0, True), (64, 30, 40, 1000, 5, False),
    (64, 10, 200, 8, 0, False), (1024, 1024, 1024, 16, 0, True), (1024, 700, 1024, 1 << 20, 512, False),
])
def test_merge_properties(W, M, budget, levels, t0, quar):
    rng = np.random.default_rng(W + M + budget + t0)
    sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg = _case(rng, W, M, levels, quar)
    ev = 11
    sc_q, off, (pos, score, toks, segs), idx_old, idx_new = segbank.evict(
        sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg, 100, ev, t0, budget)
    assert off == 100 + int(seg.max()) + 1
    bad_segs = set(seg[sc <= -1e29].tolist())
    assert all(sc_q[t] == np.float32(-1e30) for t in range(W) if seg[t] in bad_segs)
    # the full candidate list, in position order (bank first: its positions precede the chunk's)
    cand_t = [t for t in range(t0, W) if seg[t] not in bad_segs]
    n_tot = M + len(cand_t)
    assert len(pos) == min(budget, n_tot)
    assert np.all(np.diff(pos) > 0)                                         # chronological
    assert all(ev * W + t0 <= p < (ev + 1) * W for p, o in zip(pos, idx_old) if o < 0)
    for j in range(len(pos)):
        if idx_old[j] >= 0:
            assert idx_new[j] < 0 and mem_pos[idx_old[j]] == pos[j] and mem_score[idx_old[j]] == score[j]
        else:
            t = idx_new[j]
            assert pos[j] == ev * W + t and toks[j] == tok[t] and segs[j] == seg[t] + 100
            assert score[j] == np.float32(sc_q[seg == seg[t]].max() - np.float32(1e-6) * np.float32((seg[t] + 100) % 16384))
    if n_tot > budget:
        all_pos = np.concatenate([mem_pos, ev * W + np.asarray(cand_t, dtype=np.int64)])
        won = set(pos.tolist())
        key = {}
        for j, p in enumerate(mem_pos):
            key[int(p)] = (float(mem_score[j]), int(p))
        for t in cand_t:
            full = seg[t] + 100
            key[ev * W + t] = (float(np.float32(sc_q[seg == seg[t]].max() - np.float32(1e-6) * np.float32(full % 16384))),
                               ev * W + t)
        worst_win = min((key[int(p)][0], -key[int(p)][1]) for p in won)
        best_lose = max((key[int(p)][0], -key[int(p)][1]) for p in all_pos if int(p) not in won)
        assert worst_win > best_lose


def test_pinned_prefix_keeps_bank():
    rng = np.random.default_rng(5)
    sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg = _case(rng, 16, 6, 4, False)
    _, off, (pos, *_), idx_old, idx_new = segbank.evict(sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg, 7, 0, 16, 12)
    assert np.array_equal(pos, mem_pos) and np.array_equal(idx_old, np.arange(6)) and np.all(idx_new < 0)
    assert off == 7 + int(seg.max()) + 1
