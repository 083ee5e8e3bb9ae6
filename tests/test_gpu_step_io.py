"""The decode step's host inputs through the pinned host ring (vgx_step_begin) and the GEMV whose output
address is read on the device (vgx_qlinear_indirect).

vgx_step_begin takes the place of vgx_seg_step plus the host-to-device copies of the step words, ids
and bias rows: its ring, segmenter, id and word results are compared exactly with vgx_seg_step run on
the same inputs, over host and device ids, ring wrap-around, a host that runs ahead of the device by
more slots than the ring holds, and bias rows (per-head row indices into three vectors, the bias
construction of runtime/vault3.c:1976-1988) expanded against numpy.  vgx_qlinear_indirect runs the
same kernels as vgx_qlinear_ex, so its outputs must be bit-identical, also from a captured graph
replayed into a different buffer each time."""
import numpy as np
import pytest
import torch

from oracle import codec
from tests import modelgen
from vault_amd import ops, vlt3
from vault_amd.model import StepIO

pytestmark = pytest.mark.gpu


def _tiers(cfg, dev):
    from vault_amd.tokens import TokenTable
    toks, bmap = modelgen.test_vocab(cfg)
    return torch.from_numpy(TokenTable(toks, bmap, cfg.vocab_size).tiers).to(dev)


def _begin(io, tok, seg, ctrl, tiers, cfg, out_ref=True, bias=None):
    ops.step_begin(io.ring, io.RING, io.slot_bytes, io.counter, io.step, io.ids, io.out_ref if out_ref else None,
                   tok, seg, ctrl, tiers, cfg.seg_min, cfg.seg_max, bias=bias)
    io.launched()


@pytest.mark.parametrize("B", [1, 5])
def test_step_begin_matches_seg_step(dev, B):
    cfg = modelgen.tiny_cfg(window=32, seg_min=3, seg_max=11)
    W = cfg.window
    tiers = _tiers(cfg, dev)
    rng = np.random.default_rng(B)
    io = StepIO(B, dev)
    seg1 = B == 1
    tok_a, tok_b = (torch.zeros(B, W, dtype=torch.int32, device=dev) for _ in range(2))
    seg_a, seg_b = (torch.zeros(W, dtype=torch.int32, device=dev) for _ in range(2))
    ctrl_a, ctrl_b = (torch.zeros(4, dtype=torch.int32, device=dev) for _ in range(2))
    step_b = torch.zeros(4, dtype=torch.int32, device=dev)
    for p in range(3 * W + 5):                      # ring slots reused many times, chunk wrap-around
        c = p % W
        if c == 0:
            ctrl_a[2:4].zero_()
            ctrl_b[2:4].zero_()
        ids = rng.integers(0, cfg.vocab_size - 8, B)
        host = p % 3 != 0
        t = torch.from_numpy(ids).to(torch.int64)
        out = torch.empty(B, 7, device=dev)
        words = [c, p + 7, p if p < 5 else -1, c + 1]
        io.write(t if host else t.to(dev), *words, out=out)
        _begin(io, tok_a, seg_a if seg1 else None, ctrl_a if seg1 else None, tiers, cfg)
        step_b.copy_(torch.tensor(words, dtype=torch.int32))
        ops.seg_step(t.to(dev), step_b, tok_b, seg_b if seg1 else None, ctrl_b if seg1 else None, tiers, cfg.seg_min,
                     cfg.seg_max)
        assert io.step.tolist() == words, p
        assert io.ids.tolist() == ids.tolist(), p
        assert int(io.out_ref[0]) == out.data_ptr(), p
        assert int(io.counter[0]) == (p + 1) % io.RING, p
        assert torch.equal(tok_a, tok_b), p
        assert torch.equal(seg_a, seg_b) and torch.equal(ctrl_a, ctrl_b), p
    io.close()


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.F32])
@pytest.mark.parametrize("B", [1, 3])
def test_step_begin_embed_equals_embed(dev, dt, B):
    """vgx_step_begin_embed: the step words, ids, ring and segmenter as vgx_step_begin, and the
    embedding rows of the ids it wrote equal vgx_embed_rows's (pad row 0) bit for bit, host and device
    ids, including ids out of the table's range (row 0)."""
    cfg = modelgen.tiny_cfg(window=32, seg_min=3, seg_max=11)
    W, rows, cols = cfg.window, 300, 96
    tiers = _tiers(cfg, dev)
    rng = np.random.default_rng(B + dt)
    raw = vlt3.synthetic_blocks(dt, rows, cols, rng) if dt != codec.F32 else \
        rng.standard_normal((rows, cols)).astype(np.float32).tobytes()
    table = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    io = StepIO(B, dev)
    tok_a, tok_b = (torch.zeros(B, W, dtype=torch.int32, device=dev) for _ in range(2))
    for p in range(2 * W + 3):
        ids = rng.integers(0, rows, B)
        if p % 5 == 0:
            ids[0] = rows + 7 if p % 10 == 0 else -3        # out of range: row 0
        t = torch.from_numpy(ids).to(torch.int64)
        words = [p % W, p + 7, -1, p % W + 1]
        io.write(t if p % 2 else t.to(dev), *words, out=torch.empty(B, 7, device=dev))
        x = torch.full((B, cols), float("nan"), device=dev)
        ops.step_begin(io.ring, io.RING, io.slot_bytes, io.counter, io.step, io.ids, None, tok_a, None, None, tiers,
                       cfg.seg_min, cfg.seg_max, embed=(table, x))
        io.launched()
        ref = ops.embed(table, io.ids, pad_row=0)
        step_b = torch.tensor(words, dtype=torch.int32, device=dev)
        ops.seg_step(t.to(dev), step_b, tok_b, None, None, tiers, cfg.seg_min, cfg.seg_max)
        torch.cuda.synchronize()
        assert io.step.tolist() == words and io.ids.tolist() == ids.tolist(), p
        assert torch.equal(tok_a, tok_b), p
        assert torch.equal(x, ref), p
    io.close()


def test_step_begin_host_runs_ahead(dev):
    """40 steps enqueued behind a long device job with no host synchronisation: the host waits for a
    slot's previous launch before rewriting it, so every launch reads its own step's ids."""
    cfg = modelgen.tiny_cfg(window=64)
    io = StepIO(2, dev)
    tok = torch.zeros(2, cfg.window, dtype=torch.int32, device=dev)
    got = torch.zeros(40, 2, dtype=torch.int64, device=dev)
    a = torch.randn(4096, 4096, device=dev) / 64
    torch.cuda.synchronize()
    b = a
    for _ in range(8):
        b = b @ a                                   # keeps the device busy while the host writes ahead
    want = []
    for p in range(40):
        ids = [1000 + p, 2000 + p]
        want.append(ids)
        io.write(torch.tensor(ids), p % cfg.window, 0, -1, p % cfg.window + 1)
        _begin(io, tok, None, None, None, cfg, out_ref=False)
        got[p].copy_(io.ids)
    torch.cuda.synchronize()
    assert got.tolist() == want
    assert tok[:, :40].tolist() == [[w[0] for w in want], [w[1] for w in want]]
    io.close()


@pytest.mark.parametrize("H,cap,M", [(12, 40, 33), (12, 1024, 1024), (7, 2500, 1900)])
def test_step_begin_bias_rows(dev, H, cap, M):
    cfg = modelgen.tiny_cfg(window=64)
    rng = np.random.default_rng(cap)
    io = StepIO(1, dev, H, cap)
    tok = torch.zeros(1, cfg.window, dtype=torch.int32, device=dev)
    early = torch.full((H, cap + 3), 7.0, device=dev)[:, :cap]       # a row stride above the capacity
    late = torch.full((H, cap + 3), 7.0, device=dev)[:, :cap]
    for it, m in enumerate((M, M // 2, M)):
        rows = rng.integers(-1, 3, (2, H)).astype(np.int8)
        vec = rng.standard_normal((3, m)).astype(np.float32)
        io.write(torch.tensor([it]), it, 0, -1, it + 1, bias=(rows, vec))
        _begin(io, tok, None, None, None, cfg, out_ref=False, bias=(early, late))
        full = np.concatenate([np.pad(vec, ((0, 0), (0, cap - m))), np.zeros((1, cap), np.float32)])
        assert np.array_equal(early.cpu().numpy(), full[rows[0].astype(np.int64)]), it
        assert np.array_equal(late.cpu().numpy(), full[rows[1].astype(np.int64)]), it
    # a slot without bias leaves the rows as they are
    before = early.clone()
    io.write(torch.tensor([9]), 3, 0, -1, 4)
    _begin(io, tok, None, None, None, cfg, out_ref=False, bias=(early, late))
    assert torch.equal(early, before)
    io.close()


def test_step_begin_rejects_bad_arguments(dev):
    cfg = modelgen.tiny_cfg(window=64)
    io = StepIO(1, dev)
    tok = torch.zeros(1, cfg.window, dtype=torch.int32, device=dev)
    lib = ops.L.load()
    args = [io.ring, io.RING, io.slot_bytes, io.counter.data_ptr(), io.step.data_ptr(), io.ids.data_ptr(), 1, None,
            tok.data_ptr(), cfg.window, None, None, None, 0, 3, 11, cfg.window, None, None, 0, 0, 0, None]
    for i, v, code in [(2, io.slot_bytes - 256, -1), (2, io.slot_bytes + 8, -1), (0, io.ring + 8, -11), (6, 0, -1),
                       (17, io.step.data_ptr(), -31)]:
        bad = list(args)
        bad[i] = v
        assert lib.vgx_step_begin(*bad) == code, i
    # a ring without room for the bias part
    early = torch.zeros(12, 64, device=dev)
    bias_args = list(args)
    bias_args[17:22] = [early.data_ptr(), early.data_ptr(), 12, 64, 64]
    assert lib.vgx_step_slot_bytes(1, 12, 64) > io.slot_bytes
    assert lib.vgx_step_begin(*bias_args) == -1
    io.close()


def _weight(dt, rows, cols, seed, dev):
    rng = np.random.default_rng(seed)
    if dt == codec.F32:
        raw = rng.standard_normal((rows, cols)).astype(np.float32).tobytes()
    elif dt in (codec.BF16, codec.F16):
        raw = vlt3.quantize(dt, rng.standard_normal((rows, cols)).astype(np.float32) * 0.05)
    else:
        raw = vlt3.synthetic_blocks(dt, rows, cols, rng)
    return ops.QWeight.from_blocks(dt, rows, cols, raw, dev)


@pytest.mark.parametrize("dt,rows,cols,B", [
    (dt, r, c, b) for dt in (codec.Q8_0, codec.Q4_0, codec.F32, codec.BF16, codec.F16)
    for r, c, b in ((1000, 256, 1), (517, 96, 3), (64, 1536, 2), (300, 64, 7))] + [(codec.Q8_0, 151665, 1536, 1)])
def test_qlinear_indirect_equals_direct(dev, dt, rows, cols, B):
    w = _weight(dt, rows, cols, rows + B, dev)
    x = torch.randn(B, cols, device=dev)
    nw = torch.rand(cols, device=dev) + 0.5
    want = ops.qlinear(w, x, norm=(nw, 1e-6))
    out = torch.full((B, rows), float("nan"), device=dev)
    addr = torch.tensor([out.data_ptr()], dtype=torch.int64, device=dev)
    ops.qlinear_indirect(w, x, addr, norm=(nw, 1e-6))
    assert torch.equal(out, want)


def test_qlinear_indirect_graph_replays_into_new_buffers(dev):
    """One captured launch, replayed five times with the address word (and the input) changed between
    replays and eager work in between: each replay fills its own buffer, equal to the eager GEMV."""
    w = _weight(codec.Q8_0, 4096, 1536, 3, dev)
    x = torch.randn(1, 1536, device=dev)
    addr = torch.zeros(1, dtype=torch.int64, device=dev)
    tmp = torch.empty(1, 4096, device=dev)
    addr.fill_(tmp.data_ptr())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.qlinear_indirect(w, x, addr)
    outs, wants = [], []
    for r in range(5):
        x.copy_(torch.randn(1, 1536, device=dev))
        o = torch.full((1, 4096), float("nan"), device=dev)
        addr.fill_(o.data_ptr())
        g.replay()
        wants.append(ops.qlinear(w, x))
        torch.cuda.synchronize()
        outs.append(o)
    for r in range(5):
        assert torch.equal(outs[r], wants[r]), r


@pytest.mark.parametrize("graphs", [True, False])
def test_step_ring_resyncs_after_failed_steps(dev, graphs):
    """The ring's host slot number follows the device counter through failures: a slot consumed by a
    launch whose host bookkeeping never ran (counter ahead), and a step that fails before its first launch
    (counter behind).  Decoding then continues bit-identical to an undisturbed state."""
    from vault_amd.model import VAULTv3ForCausalLM
    from vault_amd.weights import ModelWeights
    cfg = modelgen.tiny_cfg(head_dim=128, seg_budget=12)
    tensors, _, _ = modelgen.build(cfg, "q8_0", seed=4)
    w = ModelWeights.from_tensors(cfg, tensors, dev)
    ma, mb = VAULTv3ForCausalLM(w), VAULTv3ForCausalLM(w)
    ma.use_graphs = mb.use_graphs = graphs
    sa, sb = ma.new_state(1), mb.new_state(1)
    ids = np.random.default_rng(8).integers(0, cfg.vocab_size - 8, 70)
    io = sa.step_io()
    for i, t in enumerate(ids):
        if i == 5:
            # a slot consumed on the device without the host's bookkeeping
            tok = torch.zeros(1, cfg.window, dtype=torch.int32, device=dev)
            io.write(torch.tensor([7]), 0, 0, -1, 1)
            ops.step_begin(io.ring, io.RING, io.slot_bytes, io.counter, io.step, io.ids, None, tok, None, None, None,
                           cfg.seg_min, cfg.seg_max)
            io.resync()
            assert io.i % io.RING == int(io.counter[0])
        if i == 9:
            # a step that fails after its slot was written, before its first launch (a replayed graph never
            # calls ops.step_begin from the host: the workspace sizing before the replay fails instead)
            def failing(*a, **k):
                raise RuntimeError("planted failure")
            holder, name = (ma, "_size_workspace") if graphs else (ops, "step_begin")
            real = getattr(holder, name)
            setattr(holder, name, failing)
            try:
                with pytest.raises(RuntimeError, match="planted"):
                    ma.step(torch.tensor([int(t)]), sa)
            finally:
                setattr(holder, name, real)
            assert io.i % io.RING == int(io.counter[0]) and sa.pos == i
        la = ma.step(torch.tensor([int(t)]), sa)
        lb = mb.step(torch.tensor([int(t)]), sb)
        assert torch.equal(la, lb), i
