"""GPU parity of the Q8_0 / Q4_0 / F32 / BF16 / F16 weight kernels against the oracle.

Bars: packing round trip and dequantization bit-exact; GEMV within the fp32 accumulation bound
``oracle.linalg.gemv_bound`` of the fp64 oracle (a dropped term or a wrong scale is ~1e3x that
bound); SwiGLU within the same bound propagated through silu.
"""
import numpy as np
import pytest
import torch

from oracle import codec, linalg
from vault_amd import ops, vlt3

pytestmark = pytest.mark.gpu

BENCH_SHAPES = [(1536, 1536), (256, 1536), (8960, 1536), (1536, 8960)]


def _blocks(dt, rows, cols, seed, kind="synthetic"):
    rng = np.random.default_rng(seed)
    if dt == codec.F32:
        return rng.standard_normal((rows, cols)).astype(np.float32).tobytes()
    if dt in (codec.BF16, codec.F16):
        return vlt3.quantize(dt, rng.standard_normal((rows, cols)).astype(np.float32) * 0.05)
    if kind == "synthetic":
        return vlt3.synthetic_blocks(dt, rows, cols, rng)
    w = rng.standard_normal((rows, cols)).astype(np.float32) * 0.05
    return vlt3.quantize(dt, w)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.F32, codec.BF16, codec.F16])
@pytest.mark.parametrize("rows,cols", [(1, 32), (13, 96), (64, 1536), (1030, 8960)])
def test_pack_unpack_dequant_bit_exact(dev, dt, rows, cols):
    raw = _blocks(dt, rows, cols, seed=rows + cols, kind="quantized")
    w = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    back = w.unpack().cpu().numpy().tobytes()
    assert back == raw
    deq = w.dequant().cpu().numpy()
    ref = codec.decode(dt, raw, rows, cols)
    assert np.array_equal(deq.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.BF16, codec.F16])
def test_embed_rows(dev, dt):
    rows, cols = 301, 1536
    raw = _blocks(dt, rows, cols, seed=5, kind="quantized")
    w = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    ids = torch.tensor([0, 300, 7, 7, -1, 301, 5000], dtype=torch.int64)
    out = ops.embed(w, ids.to(dev), pad_row=3).cpu().numpy()
    ref = codec.decode(dt, raw, rows, cols)
    want = np.stack([ref[i] if 0 <= i < rows else ref[3] for i in ids.tolist()])
    assert np.array_equal(out, want)


def _check_gemv(dev, dt, rows, cols, batch, seed, kind="synthetic", bias=False, accumulate=False):
    raw = _blocks(dt, rows, cols, seed, kind)
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    wf = codec.decode(dt, raw, rows, cols)
    rng = np.random.default_rng(seed + 1)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    b = rng.standard_normal(rows).astype(np.float32) if bias else None
    y0 = rng.standard_normal((batch, rows)).astype(np.float32) if accumulate else None
    xt = torch.from_numpy(x).to(dev)
    bt = torch.from_numpy(b).to(dev) if bias else None
    out = torch.from_numpy(y0).to(dev) if accumulate else None
    y = ops.qlinear(wq, xt, bias=bt, out=out, accumulate=accumulate).cpu().numpy().astype(np.float64)
    ref = linalg.gemv(wf, x, b)
    if accumulate:
        ref = ref + y0
    tol = linalg.gemv_bound(wf, x, dt) + (np.abs(ref) * 2e-7 if (bias or accumulate) else 0)
    err = np.abs(y - ref)
    assert np.all(err <= tol), (float(err.max()), float((err / tol).max()))
    return err, tol


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.F32, codec.BF16, codec.F16])
@pytest.mark.parametrize("batch", [1, 2, 3, 4, 5, 16])
def test_gemv_small_ragged(dev, dt, batch):
    _check_gemv(dev, dt, 13, 96, batch, seed=11 * batch, kind="quantized")


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.BF16, codec.F16])
@pytest.mark.parametrize("rows,cols", BENCH_SHAPES)
@pytest.mark.parametrize("batch", [1, 16])
def test_gemv_benchmark_shapes(dev, dt, rows, cols, batch):
    _check_gemv(dev, dt, rows, cols, batch, seed=rows * 3 + cols + batch)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.BF16])
@pytest.mark.parametrize("batch", [1, 16])
def test_gemv_lm_head_shape(dev, dt, batch):
    """The tied LM head, 151665 x 1536, at batch 1 (one-row GEMV) and 16 (MFMA small-batch GEMM)."""
    _check_gemv(dev, dt, 151665, 1536, batch, seed=9 + batch)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.BF16])
@pytest.mark.parametrize("rows", [151665, 65540])
def test_gemv_tall_fused_rmsnorm(dev, dt, rows):
    """The LM head's own call: final RMSNorm fused into the one-row GEMV over tall 1536-column weights
    (the persistent streaming kernel; 65540 rows: a row count whose row-quads do not divide evenly
    among the waves), against oracle rmsnorm -> fp64 GEMV."""
    cols = 1536
    rng = np.random.default_rng(rows + 17)
    x = (rng.standard_normal((1, cols)) * 3.0).astype(np.float32)
    g = rng.uniform(0.8, 1.2, cols).astype(np.float32)
    u = linalg.rmsnorm(x, g, 1e-6)
    raw = _blocks(dt, rows, cols, seed=rows % 97)
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    wf = codec.decode(dt, raw, rows, cols)
    ref = linalg.gemv(wf, u)
    y = ops.qlinear(wq, torch.from_numpy(x).to(dev), norm=(torch.from_numpy(g).to(dev), 1e-6))
    y = y.cpu().numpy().astype(np.float64)
    tol = 2 * linalg.gemv_bound(wf, u, dt) + np.abs(ref) * 2e-7
    err = np.abs(y - ref)
    assert np.all(err <= tol), float((err / tol).max())


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
@pytest.mark.parametrize("rows,cols", [(1026, 8960), (1026, 1536), (6, 6400)])
def test_gemv_pieces_ragged(dev, dt, rows, cols):
    """One-row GEMV on 1 KB pieces at ragged shapes: an odd row-quad count (the last workgroup of two
    row-quads holds one), rows not a multiple of 4, a row length whose last piece is partial (200 blocks),
    with bias and with the residual add."""
    _check_gemv(dev, dt, rows, cols, 1, seed=rows + cols, kind="quantized", bias=True)
    _check_gemv(dev, dt, rows, cols, 1, seed=rows + cols + 1, kind="quantized", accumulate=True)


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("accumulate", [False, True])
def test_gemv_f32_scorer_shape(dev, batch, accumulate):
    """F32 weights at the segment scorer's fc1 shape (256 x 4608) with bias, one and two activation rows
    (the decode step's features and habituated features in one pass), store and accumulate."""
    _check_gemv(dev, codec.F32, 256, 4608, batch, seed=31 + batch, bias=True, accumulate=accumulate)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
def test_gemv_bias_and_residual(dev, dt):
    _check_gemv(dev, dt, 1536, 1536, 1, seed=21, kind="quantized", bias=True)
    _check_gemv(dev, dt, 1536, 1536, 3, seed=22, kind="quantized", accumulate=True)


def test_gemv_linearity(dev):
    """y(a x1 + x2) == a y(x1) + y(x2) within accumulation error (size-independent property)."""
    dt, rows, cols = codec.Q4_0, 8960, 1536
    wq = ops.QWeight.from_blocks(dt, rows, cols, _blocks(dt, rows, cols, 3), dev)
    g = torch.Generator(device="cpu").manual_seed(0)
    x1 = torch.randn(1, cols, generator=g).to(dev)
    x2 = torch.randn(1, cols, generator=g).to(dev)
    lhs = ops.qlinear(wq, 0.5 * x1 + x2).double()
    rhs = 0.5 * ops.qlinear(wq, x1).double() + ops.qlinear(wq, x2).double()
    assert torch.allclose(lhs, rhs, rtol=0, atol=1e-4 * float(rhs.abs().max()))


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
@pytest.mark.parametrize("rows,cols,batch", [(18, 64, 1), (8960, 1536, 1), (8960, 1536, 4), (8960, 1536, 7)])
def test_swiglu(dev, dt, rows, cols, batch):
    gate = _blocks(dt, rows, cols, seed=31, kind="quantized")
    up = _blocks(dt, rows, cols, seed=32, kind="quantized")
    w = ops.QWeight.gateup_from_blocks(dt, rows, cols, gate, up, dev)
    x = np.random.default_rng(33).standard_normal((batch, cols)).astype(np.float32)
    h = ops.qlinear_swiglu(w, torch.from_numpy(x).to(dev)).cpu().numpy().astype(np.float64)
    gf, uf = codec.decode(dt, gate, rows, cols), codec.decode(dt, up, rows, cols)
    g, u = linalg.gemv(gf, x), linalg.gemv(uf, x)
    ref = linalg.swiglu(g, u)
    tg, tu = linalg.gemv_bound(gf, x, dt), linalg.gemv_bound(uf, x, dt)
    # |d silu(g)u| <= |u| (1.1 |dg|) + |silu(g)| |du|
    tol = 1.1 * np.abs(u) * tg + np.abs(g) * tu + 1e-6 * np.abs(ref) + 1e-30
    err = np.abs(h - ref)
    assert np.all(err <= tol), float((err / tol).max())


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.F32])
@pytest.mark.parametrize("rows,cols,batch,epi", [(2048, 1536, 1, "store"), (1536, 8960, 2, "accum"),
                                                 (8960, 1536, 1, "swiglu"), (40000, 1536, 3, "store"),
                                                 (256, 4608, 4, "store"), (12, 64, 5, "swiglu")])
def test_gemv_fused_rmsnorm(dev, dt, rows, cols, batch, epi):
    """u = RMSNorm(x) staged inside the GEMV (row mode, split-K mode, several LDS chunks) against
    oracle rmsnorm -> fp64 GEMV; the norm's own fp32 rounding (relative 1e-6 of |u|) is folded into
    the accumulation bound."""
    rng = np.random.default_rng(rows + cols + batch)
    x = (rng.standard_normal((batch, cols)) * 3.0).astype(np.float32)
    g = rng.uniform(0.8, 1.2, cols).astype(np.float32)
    u = linalg.rmsnorm(x, g, 1e-6)
    xt, gt = torch.from_numpy(x).to(dev), torch.from_numpy(g).to(dev)
    if epi == "swiglu":
        gate = _blocks(dt, rows, cols, seed=41, kind="quantized")
        up = _blocks(dt, rows, cols, seed=42, kind="quantized")
        w = ops.QWeight.gateup_from_blocks(dt, rows, cols, gate, up, dev)
        h = ops.qlinear_swiglu(w, xt, norm=(gt, 1e-6)).cpu().numpy().astype(np.float64)
        gf, uf = codec.decode(dt, gate, rows, cols), codec.decode(dt, up, rows, cols)
        gg, uu = linalg.gemv(gf, u), linalg.gemv(uf, u)
        ref = linalg.swiglu(gg, uu)
        tg, tu = 2 * linalg.gemv_bound(gf, u, dt), 2 * linalg.gemv_bound(uf, u, dt)
        tol = 1.1 * np.abs(uu) * tg + np.abs(gg) * tu + 1e-6 * np.abs(ref) + 1e-30
        err = np.abs(h - ref)
        assert np.all(err <= tol), float((err / tol).max())
        return
    raw = _blocks(dt, rows, cols, seed=43, kind="quantized")
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
                    norm=(gt, 1e-6)).cpu().numpy().astype(np.float64)
    tol = 2 * linalg.gemv_bound(wf, u, dt) + np.abs(ref) * 2e-7
    err = np.abs(y - ref)
    assert np.all(err <= tol), float((err / tol).max())


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0])
def test_gemv_fused_rmsnorm_equals_separate(dev, dt):
    """Fused prologue == standalone RMSNorm kernel followed by the plain GEMV (same fp32 expression;
    only the order of the sum of squares may differ)."""
    rows, cols = 1536, 1536
    raw = _blocks(dt, rows, cols, seed=44, kind="quantized")
    wq = ops.QWeight.from_blocks(dt, rows, cols, raw, dev)
    g = torch.rand(cols, generator=torch.Generator().manual_seed(1)).to(dev) + 0.5
    x = torch.randn(2, cols, generator=torch.Generator().manual_seed(2)).to(dev)
    fused = ops.qlinear(wq, x, norm=(g, 1e-6))
    sep = ops.qlinear(wq, ops.rmsnorm(x, g, 1e-6))
    assert torch.allclose(fused, sep, rtol=0, atol=1e-5 * float(sep.abs().max()))


@pytest.mark.parametrize("dt", [codec.BF16, codec.F16])
@pytest.mark.parametrize("batch", [1, 3, 8, 40, 200])
def test_plain16_swiglu_and_norm(dev, dt, batch):
    """BF16 / F16 gate/up with the fused SwiGLU, and the projections with an RMSNorm prologue, over the
    GEMV (batch < 8) and the fp32 MFMA GEMM (batch >= 8, the norm applied by a separate launch)."""
    rows, cols = 512, 1536
    rng = np.random.default_rng(batch + dt)
    rg, ru = _blocks(dt, rows, cols, 1), _blocks(dt, rows, cols, 2)
    w = ops.QWeight.gateup_from_blocks(dt, rows, cols, rg, ru, dev)
    x = rng.standard_normal((batch, cols)).astype(np.float32)
    gamma = rng.uniform(0.8, 1.2, cols).astype(np.float32)
    u = linalg.rmsnorm(x, gamma, 1e-6)
    wg, wu = codec.decode(dt, rg, rows, cols), codec.decode(dt, ru, rows, cols)
    h = ops.qlinear_swiglu(w, torch.from_numpy(x).to(dev), norm=(torch.from_numpy(gamma).to(dev), 1e-6))
    g, up = linalg.gemv(wg, u), linalg.gemv(wu, u)
    ref = linalg.swiglu(g, up)
    tol = (2 * linalg.gemv_bound(wg, u, dt) * np.abs(up) + 2 * linalg.gemv_bound(wu, u, dt) * np.abs(g) +
           np.abs(ref) * 1e-6)
    err = np.abs(h.cpu().numpy().astype(np.float64) - ref)
    assert np.all(err <= tol), float((err / tol).max())
