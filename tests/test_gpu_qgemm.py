"""GPU parity of the MFMA Q8_0 / Q4_0 GEMM (vgx_qgemm, used by ops.qlinear from 8 activation rows on)
against the fp64 oracle.

Bar: the GEMV accumulation bound of oracle.linalg.  Above 64 activation rows (the tiled kernels: fp16
hi + lo pieces of a power-of-two-scaled row, about 2^-22 relative per element) at the one-row GEMV's
relative term, 2e-6; up to 64 rows (the decode-batch kernels: bf16 hi + fp16 lo16 pieces, 2^-20) with
the relative term raised to 8e-6.  A dropped block, a wrong scale or a transposed operand is orders
of magnitude beyond either.  Shapes: the model's projections at prefill and
batched-decode row counts, ragged row and batch counts, every epilogue, with and without the fused
RMSNorm; an invariant check that the GEMM equals the GEMV row by row within the same bound.
"""
import numpy as np
import pytest
import torch

from oracle import codec, linalg
from vault_amd import _lib as L
from vault_amd import ops, vlt3

pytestmark = pytest.mark.gpu


def _blocks(dt, rows, cols, seed):
    rng = np.random.default_rng(seed)
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.05
    return vlt3.quantize(dt, w)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
@pytest.mark.parametrize("rows,cols,batch,epi,norm", [
    (1536, 1536, 16, "store", False), (2048, 1536, 300, "store", True), (1536, 8960, 37, "accum", False),
    (8960, 1536, 64, "swiglu", True), (13, 96, 9, "store", True), (256, 4608, 1024, "store", False),
    (2, 64, 8, "swiglu", False), (13, 96, 130, "store", True), (2, 64, 200, "swiglu", False),
    (1536, 8960, 200, "accum", False), (1536, 1536, 32, "accum", False), (1026, 1536, 27, "store", True),
    (1024, 1024, 20, "swiglu", True)])
def test_qgemm_matches_oracle(dev, dt, rows, cols, batch, epi, norm):
    rel = 2e-6 if batch > 64 else 8e-6
    rng = np.random.default_rng(rows + cols + batch)
    x = (rng.standard_normal((batch, cols)) * 2.0).astype(np.float32)
    g = rng.uniform(0.8, 1.2, cols).astype(np.float32)
    u = linalg.rmsnorm(x, g, 1e-6) if norm else x.astype(np.float64)
    nrm = (torch.from_numpy(g).to(dev), 1e-6) if norm else None
    xt = torch.from_numpy(x).to(dev)
    if epi == "swiglu":
        gate, up = _blocks(dt, rows, cols, 1), _blocks(dt, rows, cols, 2)
        w = ops.QWeight.gateup_from_blocks(dt, rows, cols, gate, up, dev)
        h = ops.qlinear_swiglu(w, xt, norm=nrm).cpu().numpy().astype(np.float64)
        gf, uf = codec.decode(dt, gate, rows, cols), codec.decode(dt, up, rows, cols)
        gg, uu = linalg.gemv(gf, u), linalg.gemv(uf, u)
        ref = linalg.swiglu(gg, uu)
        tg, tu = linalg.gemv_bound(gf, u, dt, rel=rel), linalg.gemv_bound(uf, u, dt, rel=rel)
        tol = 1.1 * np.abs(uu) * tg + np.abs(gg) * tu + 1e-6 * np.abs(ref) + 1e-30
        err = np.abs(h - ref)
        assert np.all(err <= tol), float((err / tol).max())
        return
    raw = _blocks(dt, rows, cols, 3)
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    wf = codec.decode(dt, raw, rows, cols)
    bias = rng.standard_normal(rows).astype(np.float32)
    ref = linalg.gemv(wf, u, bias)
    out = None
    if epi == "accum":
        y0 = rng.standard_normal((batch, rows)).astype(np.float32)
        ref = ref + y0
        out = torch.from_numpy(y0).to(dev)
    y = ops.qlinear(wq, xt, bias=torch.from_numpy(bias).to(dev), out=out, accumulate=epi == "accum",
                    norm=nrm).cpu().numpy().astype(np.float64)
    tol = linalg.gemv_bound(wf, u, dt, rel=rel) + np.abs(ref) * 2e-7
    err = np.abs(y - ref)
    assert np.all(err <= tol), float((err / tol).max())


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
@pytest.mark.parametrize("norm", [False, True])
def test_qgemm_row_magnitudes(dev, dt, norm):
    """The tiled kernels scale every activation row by its own power of two before splitting it into
    fp16 pieces: rows whose magnitudes span 1e-20 .. 1e20 (far outside fp16's range, and past the
    2^21 where a fixed-scale fp16 residual would overflow) and an all-zero row all meet the GEMV bar
    relative to their own magnitude (with the fused RMSNorm over 1e-15 .. 1e15, so that the fp32 sum of
    squares stays finite).  100 rows: the tiled path."""
    rows, cols, batch = 1536, 1536, 100
    rng = np.random.default_rng(77 + dt + norm)
    span = 15 if norm else 20          # with the norm, keep the fp32 sum of squares finite
    x = rng.standard_normal((batch, cols)) * 10.0 ** rng.uniform(-span, span, (batch, 1))
    x[7] = 0.0
    x = x.astype(np.float32)
    g = rng.uniform(0.8, 1.2, cols).astype(np.float32)
    u = linalg.rmsnorm(x, g, 1e-6) if norm else x.astype(np.float64)
    raw = _blocks(dt, rows, cols, 5)
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    wf = codec.decode(dt, raw, rows, cols)
    y = ops.qlinear(wq, torch.from_numpy(x).to(dev), norm=(torch.from_numpy(g).to(dev), 1e-6) if norm else None)
    y = y.cpu().numpy().astype(np.float64)
    ref = linalg.gemv(wf, u)
    tol = linalg.gemv_bound(wf, u, dt, rel=2e-6) + np.abs(ref) * 2e-7
    assert np.all(np.isfinite(y))
    assert np.all(y[7] == 0.0)
    err = np.abs(y - ref)
    assert np.all(err <= tol), float((err / tol).max())


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
@pytest.mark.parametrize("rows,cols,batch,epi,norm", [
    (8960, 1536, 1024, "swiglu", True), (10246, 512, 820, "accum", False), (10246, 512, 820, "store", True),
    (65541, 256, 40, "store", True), (65541, 256, 17, "accum", False), (65541, 768, 32, "store", True),
    (65541, 768, 20, "store", False), (65541, 1536, 32, "store", True), (1536, 8960, 300, "accum", False),
    (2048, 1536, 1000, "store", True)])
def test_qgemm_chunk_shapes_match_oracle(dev, dt, rows, cols, batch, epi, norm):
    """Many tiles: the gate/up pair of a full 1024-token prefill chunk (1120 tiles, three rounds of
    workgroups), 10246 x 512 over 820 activation rows (ragged rows and activation rows in the last
    tiles), K-split launches of 512 and more workgroups with ragged activation tiles (1536 x 8960 over
    300 rows: 36 tiles x 16 splits; 2048 x 1536 over 1000 rows: 128 tiles x 4 splits) on the LDS-DMA
    kernel, and LM-head-like tall weights (65541 rows, ragged; the stores over 768 and 1536 columns run
    on the persistent unsplit kernel, with 2 activation tiles per row group, the others on the 32-row
    tiles of the small-batch kernel).  Same bars as above."""
    test_qgemm_matches_oracle(dev, dt, rows, cols, batch, epi, norm)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
def test_qgemm_equals_gemv_rows(dev, dt):
    """The GEMM over 40 rows equals the batch-1 GEMV applied to each row (both vs the same bound)."""
    rows, cols, batch = 1536, 1536, 40
    raw = _blocks(dt, rows, cols, 4)
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    x = torch.randn(batch, cols, generator=torch.Generator().manual_seed(5)).to(dev)
    big = ops.qlinear(wq, x)
    one = torch.cat([ops.qlinear(wq, x[i:i + 1]) for i in range(batch)])
    wf = codec.decode(dt, raw, rows, cols)
    tol = torch.from_numpy(2 * linalg.gemv_bound(wf, x.cpu().numpy(), dt, rel=8e-6)).to(dev)
    assert bool(((big.double() - one.double()).abs() <= tol).all())


@pytest.mark.parametrize("epi,rows,cols", [("swiglu", 8960, 1536), ("accum", 1536, 8960), ("accum", 1536, 1536)])
def test_qgemm_fused_split_sum_replays(dev, epi, rows, cols):
    """Decode-batch Q4_0 projections whose K splits are summed by the last workgroup of each output tile
    (gate/up with the RMSNorm, down with the residual add, the o-projection on 64-row tiles, batch 32): eager calls one after another and
    replays of a captured graph, with eager work between the replays, give the same bits each time (the
    tile counters are back at zero after every call) and stay within the oracle bound."""
    rng = np.random.default_rng(rows + cols + 7)
    batch = 32
    x = torch.from_numpy((rng.standard_normal((batch, cols)) * 2.0).astype(np.float32)).to(dev)
    if epi == "swiglu":
        g = torch.from_numpy(rng.uniform(0.8, 1.2, cols).astype(np.float32)).to(dev)
        gate, up = _blocks(codec.Q4_0, rows, cols, 8), _blocks(codec.Q4_0, rows, cols, 9)
        w = ops.QWeight.gateup_from_blocks(codec.Q4_0, rows, cols, gate, up, dev)
        run = lambda out: ops.qlinear_swiglu(w, x, out=out, norm=(g, 1e-6))
        u = linalg.rmsnorm(x.cpu().numpy(), g.cpu().numpy(), 1e-6)
        gf, uf = codec.decode(codec.Q4_0, gate, rows, cols), codec.decode(codec.Q4_0, up, rows, cols)
        gg, uu = linalg.gemv(gf, u), linalg.gemv(uf, u)
        ref = linalg.swiglu(gg, uu)
        tol = 1.1 * np.abs(uu) * linalg.gemv_bound(gf, u, codec.Q4_0, rel=8e-6) + \
            np.abs(gg) * linalg.gemv_bound(uf, u, codec.Q4_0, rel=8e-6) + 1e-6 * np.abs(ref) + 1e-30
        y0 = torch.zeros(batch, rows, device=dev)
    else:
        raw = _blocks(codec.Q4_0, rows, cols, 10)
        w = ops.QWeight.from_blocks(codec.Q4_0, rows, cols, raw, dev)
        run = lambda out: ops.qlinear(w, x, out=out, accumulate=True)
        wf = codec.decode(codec.Q4_0, raw, rows, cols)
        y0 = torch.from_numpy(rng.standard_normal((batch, rows)).astype(np.float32)).to(dev)
        ref = linalg.gemv(wf, x.cpu().numpy()) + y0.cpu().numpy()
        tol = linalg.gemv_bound(wf, x.cpu().numpy(), codec.Q4_0, rel=8e-6) + np.abs(ref) * 2e-7
    eager = []
    for _ in range(3):
        out = y0.clone()
        run(out)
        eager.append(out)
    torch.cuda.synchronize()
    assert all(torch.equal(e, eager[0]) for e in eager[1:])
    assert np.all(np.abs(eager[0].cpu().numpy().astype(np.float64) - ref) <= tol)
    out = y0.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run(out)                      # workspace sized before the capture
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run(out)
    for i in range(3):
        out.copy_(y0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[0]), f"replay {i}"
        run(y0.clone())               # eager call between replays
        torch.cuda.synchronize()


@pytest.mark.parametrize("dt", [codec.Q4_0])
@pytest.mark.parametrize("rows,cols,batch", [(64, 7200, 8), (16, 4096, 8), (64, 7200, 200)])
def test_qgemm_k_split_edges(dev, dt, rows, cols, batch):
    """Few weight rows and long rows: the GEMM splits K over many workgroups (up to 16), including
    a possibly empty last split (225 blocks over 16 splits)."""
    rng = np.random.default_rng(rows + cols)
    raw = _blocks(dt, rows, cols, 6)
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    y = ops.qlinear(wq, torch.from_numpy(x).to(dev)).cpu().numpy().astype(np.float64)
    wf = codec.decode(dt, raw, rows, cols)
    ref = linalg.gemv(wf, x)
    tol = linalg.gemv_bound(wf, x, dt, rel=8e-6)
    assert np.all(np.abs(y - ref) <= tol)


@pytest.mark.parametrize("rows,cols,batch,epi", [
    (256, 4608, 2048, "store"), (130, 96, 77, "accum"), (64, 160, 300, "swiglu"), (13, 32, 40, "store")])
def test_f32_gemm_matches_oracle(dev, rows, cols, batch, epi):
    """F32 weights over many rows (the scorer's fc1 over a chunk: 4608 -> 256 on 2 x 1024 rows) run the
    fp32-MFMA GEMM; bar: the fp32 accumulation bound of the fp64 oracle."""
    rng = np.random.default_rng(rows * 7 + cols + batch)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    xt = torch.from_numpy(x).to(dev)
    if epi == "swiglu":
        g = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        u = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        w = ops.QWeight.gateup_from_blocks(codec.F32, rows, cols, g.tobytes(), u.tobytes(), dev)
        h = ops.qlinear_swiglu(w, xt).cpu().numpy().astype(np.float64)
        gg, uu = linalg.gemv(g.astype(np.float64), x), linalg.gemv(u.astype(np.float64), x)
        ref = linalg.swiglu(gg, uu)
        tg = linalg.gemv_bound(g, x, codec.F32, rel=8e-6)
        tu = linalg.gemv_bound(u, x, codec.F32, rel=8e-6)
        tol = 1.1 * np.abs(uu) * tg + np.abs(gg) * tu + 1e-6 * np.abs(ref) + 1e-30
        assert np.all(np.abs(h - ref) <= tol)
        return
    wm = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    wq = ops.QWeight.from_blocks(codec.F32, rows, cols, wm.tobytes(), dev)
    bias = rng.standard_normal(rows).astype(np.float32)
    ref = linalg.gemv(wm.astype(np.float64), x, bias)
    out = None
    if epi == "accum":
        y0 = rng.standard_normal((batch, rows)).astype(np.float32)
        ref = ref + y0
        out = torch.from_numpy(y0).to(dev)
    y = ops.qlinear(wq, xt, bias=torch.from_numpy(bias).to(dev), out=out,
                    accumulate=epi == "accum").cpu().numpy().astype(np.float64)
    tol = linalg.gemv_bound(wm, x, codec.F32, rel=8e-6) + np.abs(ref) * 2e-7
    assert np.all(np.abs(y - ref) <= tol), float((np.abs(y - ref) / tol).max())


def test_f32_gemm_rejects_rmsnorm(dev):
    lib = L.load()
    z = torch.zeros(1 << 16, device=dev)
    p = z.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    assert lib.vgx_qgemm(L.F32, p, 64, 64, p, 64, 100, p, 1e-6, None, p, 64, L.EPI_STORE, None, 0, s) < 0
