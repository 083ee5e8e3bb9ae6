"""Device-resident decode control: the segment-bank merge (vgx_seg_evict) against the fp32 restatement
(oracle/segbank.py) on ties, quarantine, pinned prefixes and full banks over consecutive boundaries;
the step segmenter (vgx_seg_step) against the host rule; the masked gather and the device-count
rotation; next-token selection (vgx_argmax, vgx_sample_topk) against the reference runtime's own
v3_argmax / v3_sample_topk (runtime/vault3.c:3198-3230, compiled into oracle/_ref); and a greedy
decode loop fed by device ids equal to the host-id loop.  Integer results are compared exactly."""
import numpy as np
import pytest
import torch

from oracle import ref, segbank
from tests import modelgen
from tests.test_oracle_segbank import _case
from vault_amd import ops
from vault_amd.model import VAULTv3ForCausalLM
from vault_amd.weights import ModelWeights

pytestmark = pytest.mark.gpu


def _dev(a, dtype, dev):
    return torch.as_tensor(np.asarray(a)).to(dtype).to(dev)


@pytest.mark.parametrize("W,M,budget,levels,t0,quar", [
    (64, 0, 12, 4, 0, False), (64, 12, 12, 4, 0, True), (64, 30, 40, 1000, 5, False), (64, 10, 200, 8, 0, False),
    (1024, 1024, 1024, 16, 0, True), (1024, 700, 1024, 1 << 20, 512, False), (1024, 300, 1024, 3, 1024, False),
])
def test_seg_evict_matches_restatement(dev, W, M, budget, levels, t0, quar):
    rng = np.random.default_rng(W * 7 + M + t0)
    cap = max(budget, M)
    bank = [torch.zeros(cap, dtype=t, device=dev) for t in (torch.int64, torch.float32, torch.int32, torch.int32)]
    sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg = _case(rng, W, M, levels, quar)
    for b, a in zip(bank, (mem_pos, mem_score, mem_tok, mem_seg)):
        b[:M].copy_(torch.as_tensor(np.asarray(a)).to(b.dtype))
    ctrl = torch.tensor([M, 100, 0, 0], dtype=torch.int32, device=dev)
    idx_old = torch.zeros(budget, dtype=torch.int32, device=dev)
    idx_new = torch.zeros(budget, dtype=torch.int32, device=dev)
    sc_d = _dev(sc, torch.float32, dev)
    ops.seg_evict(sc_d, _dev(seg, torch.int32, dev), _dev(tok, torch.int32, dev), *bank, ctrl, 11, t0, budget,
                  idx_old, idx_new)
    sc_q, off, (pos, score, toks, segs), io, inew = segbank.evict(sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg,
                                                                   100, 11, t0, budget)
    K = len(pos)
    assert ctrl.tolist()[:2] == [K, off]
    assert np.array_equal(sc_d.cpu().numpy(), sc_q)
    assert np.array_equal(bank[0][:K].cpu().numpy(), pos)
    assert np.array_equal(bank[1][:K].cpu().numpy(), score)
    assert np.array_equal(bank[2][:K].cpu().numpy(), toks) and np.array_equal(bank[3][:K].cpu().numpy(), segs)
    assert np.array_equal(idx_old[:K].cpu().numpy(), io) and np.array_equal(idx_new[:K].cpu().numpy(), inew)
    if K < budget:
        assert (idx_old[K:] == -1).all() and (idx_new[K:] == -1).all()


@pytest.mark.parametrize("budget", [40, 31])
def test_seg_evict_nan_and_signed_zero_scores(dev, budget):
    """Bank scores that are NaN, +0 and -0 among ties: the ranking puts NaN last and -0 level with +0
    (index order breaks the tie), as the restatement's lexsort does, and keeps exactly `budget` winners."""
    rng = np.random.default_rng(budget)
    W, M = 64, 30
    sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg = _case(rng, W, M, 4, False)
    mem_score = np.asarray(mem_score, np.float32).copy()
    mem_score[[2, 7, 19]] = np.nan
    mem_score[[3, 11]] = 0.0
    mem_score[[5, 23]] = -0.0
    cap = max(budget, M)
    bank = [torch.zeros(cap, dtype=t, device=dev) for t in (torch.int64, torch.float32, torch.int32, torch.int32)]
    for b, a in zip(bank, (mem_pos, mem_score, mem_tok, mem_seg)):
        b[:M].copy_(torch.as_tensor(np.asarray(a)).to(b.dtype))
    ctrl = torch.tensor([M, 100, 0, 0], dtype=torch.int32, device=dev)
    idx_old = torch.zeros(budget, dtype=torch.int32, device=dev)
    idx_new = torch.zeros(budget, dtype=torch.int32, device=dev)
    ops.seg_evict(_dev(sc, torch.float32, dev), _dev(seg, torch.int32, dev), _dev(tok, torch.int32, dev), *bank, ctrl,
                  11, 0, budget, idx_old, idx_new)
    _, off, (pos, score, toks, segs), io, inew = segbank.evict(sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg,
                                                              100, 11, 0, budget)
    K = len(pos)
    assert K == budget and ctrl.tolist()[:2] == [K, off]
    assert np.array_equal(bank[0][:K].cpu().numpy(), pos)
    assert np.array_equal(bank[1][:K].cpu().numpy().view(np.uint32), score.view(np.uint32))
    assert np.array_equal(idx_old[:K].cpu().numpy(), io) and np.array_equal(idx_new[:K].cpu().numpy(), inew)


def test_seg_step_matches_host_rule(dev):
    cfg = modelgen.tiny_cfg(window=32, seg_min=3, seg_max=11)
    toks, bmap = modelgen.test_vocab(cfg)
    from vault_amd.tokens import TokenTable
    tiers = TokenTable(toks, bmap, cfg.vocab_size).tiers
    ids = np.random.default_rng(2).integers(0, cfg.vocab_size - 8, 200)
    W = cfg.window
    tok_cur = torch.zeros(1, W, dtype=torch.int32, device=dev)
    seg_cur = torch.zeros(W, dtype=torch.int32, device=dev)
    ctrl = torch.zeros(4, dtype=torch.int32, device=dev)
    step = torch.zeros(4, dtype=torch.int32, device=dev)
    tiers_d = torch.from_numpy(tiers).to(dev)
    cur = ln = 0
    t2 = max(cfg.seg_min, cfg.seg_max * 2 // 3)
    t3 = max(cfg.seg_min, cfg.seg_max - 8 if cfg.seg_max > 8 else cfg.seg_min)
    for p, tid in enumerate(ids):
        c = p % W
        if c == 0:
            ctrl[2:4].zero_()
            cur = ln = 0
        step[0] = c
        ops.seg_step(torch.tensor([int(tid)], device=dev), step, tok_cur, seg_cur, ctrl, tiers_d, cfg.seg_min,
                     cfg.seg_max)
        want_seg = cur
        ln += 1
        tr = int(tiers[tid])
        if c == W - 1 or ln >= cfg.seg_max or (tr == 1 and ln >= cfg.seg_min) or (tr == 2 and ln >= t2) or \
                (tr == 3 and ln >= t3):
            cur, ln = cur + 1, 0
        assert int(seg_cur[c]) == want_seg and int(tok_cur[0, c]) == int(tid), p
        assert ctrl[2:4].tolist() == [cur, ln], p


def test_masked_gather_and_dynamic_rotation(dev):
    rng = np.random.default_rng(4)
    O, n, D = 6, 20, 64
    src = torch.from_numpy(rng.standard_normal((O, n, D)).astype(np.float32)).to(dev)
    dst = torch.full((O, 16, D), 7.0, device=dev)
    idx = torch.tensor([3, -1, 0, 19, -1] + [-1] * 11, dtype=torch.int32, device=dev)
    ops.gather_rows_masked(src, dst, idx)
    d = dst.cpu().numpy()
    s = src.cpu().numpy()
    assert np.array_equal(d[:, 0], s[:, 3]) and np.array_equal(d[:, 2], s[:, 0]) and np.array_equal(d[:, 3], s[:, 19])
    assert (d[:, 1] == 7).all() and (d[:, 4:] == 7).all()
    # rows i < m rotated to positions i - m, against the fixed-offset rotation
    from vault_amd.attention import rope_table_double
    tab = torch.from_numpy(rope_table_double(np.arange(-40, 10), D, 1e6)).to(dev)
    t0 = tab[40:]
    m = torch.tensor([13], dtype=torch.int32, device=dev)
    out = torch.zeros_like(src)
    ops.rope_rotate_dyn(src, out, t0, D, m, 0, True)
    want = torch.zeros_like(src)
    ops.rope_rotate(src[:, :13], want[:, :13], tab[40 - 13:], D)
    assert torch.equal(out[:, :13], want[:, :13]) and (out[:, 13:] == 0).all()
    out2 = torch.zeros_like(src)
    ops.rope_rotate_dyn(src[:, :5], out2[:, :5], t0, D, m, -5, False)
    want2 = torch.zeros_like(src)
    ops.rope_rotate(src[:, :5], want2[:, :5], tab[40 - 18:], D)
    assert torch.equal(out2, want2)


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
def test_argmax_matches_reference(dev):
    rng = np.random.default_rng(8)
    V = 151665
    x = rng.standard_normal((9, V)).astype(np.float32)
    x[1, [5, 900, 150000]] = 40.0                         # ties: the first index
    x[2, :] = -np.inf
    x[3, 100] = np.nan
    x[3, 7] = 50.0
    x[4, 0] = -0.0
    x[4, 1:] = -1.0
    x[4, 3] = 0.0                                         # -0 then +0: equal, the first one wins
    x[5] = np.round(x[5])                                 # many ties
    got = ops.argmax(torch.from_numpy(x).to(dev)).cpu().numpy()
    want = np.array([ref.argmax(r) for r in x])
    assert np.array_equal(got, want)


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("k,temp", [(2, 1.0), (8, 0.7), (40, 1.3), (64, 0.5), (100, 1.0), (1, 1.0), (8, 0.0),
                                    (64, 3.0), (16, 0.05)])
def test_sample_topk_matches_reference(dev, k, temp):
    """The same index and the same new xorshift state as the reference's sampler on every row: the
    candidate weights use the runtime's own exp arithmetic, the sum runs in candidate order, and the
    draw walks the same cumulative weights.  Rows with tied maxima, rows of few distinct values (ties
    inside the top k, kept in index order) and a row whose weights reach the subnormal range."""
    rng = np.random.default_rng(k * 10 + int(temp * 10))
    B, V = 96, 151665
    x = (rng.standard_normal((B, V)) * 3).astype(np.float32)
    x[::7, 1000:1010] = x[::7].max(axis=1, keepdims=True)      # tied maxima
    x[64:80] = np.round(x[64:80])                               # many ties inside the top k
    x[80:88] = np.round(x[80:88] * 4) / 4
    x[88, :] = -200.0
    x[88, rng.integers(0, V, 70)] = rng.uniform(-200, 0, 70).astype(np.float32)   # weights down to e^-200/T
    states = rng.integers(0, 2**63, B, dtype=np.int64)
    states[0] = 0
    st_dev = torch.from_numpy(states.copy()).to(dev)
    got = ops.sample_topk(torch.from_numpy(x).to(dev), k, temp, st_dev).cpu().numpy()
    new_states = st_dev.cpu().numpy().view(np.uint64)
    for b in range(B):
        idx, s2 = ref.sample_topk(x[b], k, temp, int(np.uint64(states[b].view(np.uint64))))
        if temp > 0 and k > 1:
            assert int(new_states[b]) == s2, b
        assert int(got[b]) == idx, b


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("M,budget,ev,n_pin,seed", [(0, 8, 11, 0, 0), (8, 8, 11, 0, 1), (20, 24, 11, 5, 2),
                                                     (24, 24, 11, 0, 3), (5, 12, 11, 0, 4), (0, 24, 0, 3, 5),
                                                     (0, 6, 0, 17, 6), (0, 24, 0, 64, 7)])
def test_seg_evict_matches_runtime_on_near_ties(dev, M, budget, ev, n_pin, seed):
    """The device merge against the runtime's own update_segment_bank (runtime/vault3.c:1833-1915) on
    banks whose candidates nearly tie: maxima one ulp apart, equal maxima separated only by the
    -1e-6 * seg-id tie-break, bank scores equal to candidate scores (ranked by position)."""
    from tests.test_oracle_cmath import near_tie_case
    cfg = modelgen.tiny_cfg(window=64, seg_budget=24)
    _, blob, _ = modelgen.build(cfg, "q8_0", seed=1)
    rt = ref.RefRuntime(blob)
    rng = np.random.default_rng(seed)
    off = 100
    sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg = near_tie_case(rng, cfg.window, M, ev, off)
    (pos, score, toks, segs), new_off = rt.seg_update(ev, n_pin, off, budget, sc, seg, tok, mem_pos, mem_score,
                                                      mem_tok, mem_seg)
    cap = max(budget, M)
    bank = [torch.zeros(cap, dtype=t, device=dev) for t in (torch.int64, torch.float32, torch.int32, torch.int32)]
    for b, a in zip(bank, (mem_pos, mem_score, mem_tok, mem_seg)):
        b[:M].copy_(torch.as_tensor(np.asarray(a)).to(b.dtype))
    ctrl = torch.tensor([M, off, 0, 0], dtype=torch.int32, device=dev)
    idx_old = torch.zeros(budget, dtype=torch.int32, device=dev)
    idx_new = torch.zeros(budget, dtype=torch.int32, device=dev)
    ops.seg_evict(_dev(sc, torch.float32, dev), _dev(seg, torch.int32, dev), _dev(tok, torch.int32, dev), *bank, ctrl,
                  ev, n_pin if ev == 0 else 0, budget, idx_old, idx_new)
    K = len(pos)
    assert ctrl.tolist()[:2] == [K, new_off]
    assert np.array_equal(bank[0][:K].cpu().numpy(), pos)
    assert np.array_equal(bank[1][:K].cpu().numpy().view(np.uint32), score.view(np.uint32))
    assert np.array_equal(bank[2][:K].cpu().numpy(), toks) and np.array_equal(bank[3][:K].cpu().numpy(), segs)


@pytest.mark.parametrize("seg_budget", [12, 0])
def test_device_id_decode_loop(dev, seg_budget):
    """Greedy decoding with the next id taken on the device (ops.argmax, no host read) equals the loop
    that reads each id on the host, bit for bit, across chunk boundaries and segment-bank merges."""
    cfg = modelgen.tiny_cfg(head_dim=128, seg_budget=seg_budget)
    tensors, _, _ = modelgen.build(cfg, "q4_0", seed=9)
    w = ModelWeights.from_tensors(cfg, tensors, dev)
    ma, mb = VAULTv3ForCausalLM(w), VAULTv3ForCausalLM(w)
    sa, sb = ma.new_state(1), mb.new_state(1)
    ta = torch.tensor([5])
    tb = torch.tensor([5], device=dev)
    for i in range(120):
        la = ma.step(ta, sa)
        lb = mb.step(tb, sb)
        assert torch.equal(la, lb), i
        ta = torch.tensor([int(la[0].argmax())])
        tb = ops.argmax(lb)
        assert int(ta[0]) == int(tb[0]), i
    assert np.array_equal(sa.mem_pos.numpy(), sb.mem_pos.numpy())
