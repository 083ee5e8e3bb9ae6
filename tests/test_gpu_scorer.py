"""GPU parity of the segment scorer's EMA habituation (vgx_ema_habituate) against the per-token rule of
the oracle model (oracle/model.py, restating src/vault_v3_model.py:2294-2305): the first token of a
stream sets ema = f; every later token gives hab = f - 0.65 ema (before the update) and
ema <- 0.985 ema + 0.015 f.  Chunk lengths that are and are not multiples of the kernel's 32-token
load batches.  Bar: fp32 recurrence against float64, 1e-5 relative to the feature scale (the
recurrence contracts, so rounding does not grow with T).
"""
import numpy as np
import pytest
import torch

from vault_amd import ops

pytestmark = pytest.mark.gpu


def _ref(f, ema0, first):
    f = f.astype(np.float64)
    T, fd = f.shape
    e = f[0].copy() if first else ema0.astype(np.float64).copy()
    hab = np.empty_like(f)
    for t in range(T):
        hab[t] = f[t] - 0.65 * e
        if not (first and t == 0):
            e = 0.985 * e + 0.015 * f[t]
    return hab, e


@pytest.mark.parametrize("T", [1, 33, 1000, 1024])
@pytest.mark.parametrize("first", [True, False])
def test_ema_habituate_matches_recurrence(dev, T, first):
    rng = np.random.default_rng(T + first)
    fd = 4608
    f = (rng.standard_normal((T, fd)) * 2.0).astype(np.float32)
    ema0 = rng.standard_normal(fd).astype(np.float32)
    ft = torch.from_numpy(f).to(dev)
    hab = torch.full((T, fd), float("nan"), device=dev)
    ema = torch.from_numpy(ema0).to(dev)
    ops.ema_habituate(ft, hab, ema, first)
    torch.cuda.synchronize()
    want_h, want_e = _ref(f, ema0, first)
    tol = 1e-5 * float(np.abs(f).max())
    got_h = hab.double().cpu().numpy()
    rows = slice(1, None) if first else slice(None)   # the first token's hab is not used by the model
    if got_h[rows].size:
        assert np.abs(got_h[rows] - want_h[rows]).max() <= tol
    assert np.abs(ema.double().cpu().numpy() - want_e).max() <= tol


@pytest.mark.skipif(not __import__("oracle.ref", fromlist=["ref"]).available(), reason="oracle/_ref not built")
def test_score_tail_gelu_is_the_runtimes(dev):
    """The scorer tail's GELU is the C runtime's v3_geluf (runtime/vault3.c:118-129, 974) bit for bit.
    With fc2 = e_0 and b2 = 0 the tail's score of token t is exactly gelu(h[t, 0]) (every other term
    adds zero, and the habituated row equals the raw one, so the combine adds zero; a -0 becomes +0 in
    that sum): 2^20 inputs over
    the range the hidden units take, the erf clamp at |x / sqrt 2| = 4 and both signs."""
    from oracle import ref
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.uniform(-8, 8, 1 << 19), rng.standard_normal(1 << 18) * 2,
                        np.linspace(5.6, 5.72, 1 << 17), -np.linspace(5.6, 5.72, 1 << 17)]).astype(np.float32)
    T, hidden = x.size, 64
    h = torch.zeros((2 * T, hidden), dtype=torch.float32, device=dev)
    xt = torch.from_numpy(x).to(dev)
    h[:T, 0] = xt
    h[T:, 0] = xt
    w2 = torch.zeros(hidden, dtype=torch.float32, device=dev)
    w2[0] = 1.0
    b2 = torch.zeros(1, dtype=torch.float32, device=dev)
    out = torch.empty(T, dtype=torch.float32, device=dev)
    ops.seg_score_tail(h, w2, b2, T, False, out)
    got = out.cpu().numpy()
    want = ref.math("gelu", x)
    # bit for bit, except that a -0 GELU (large negative x) enters the tail's sum as +0
    nz = want != 0
    assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))
    assert np.all(got[~nz] == 0)


@pytest.mark.parametrize("fd", [4608, 2688, 96])
@pytest.mark.parametrize("first", [True, False])
def test_score_step_equals_separate_launches(dev, fd, first):
    """vgx_seg_score_step (the decode token's scorer: the fc1 GEMV building both LayerNormed rows
    itself, then the tail with the EMA update) against the separate launches it replaces
    (vgx_ema_habituate, vgx_layernorm, the fc1 vgx_qlinear, vgx_seg_score_tail at T = 1): the score,
    the fc1 outputs and the EMA state equal bit for bit; the score lands at the slot a device index
    names; feature widths of the 1.5B model (3 x 1536), the 0.5B one (3 x 896) and a tiny one."""
    rng = np.random.default_rng(fd + first)
    hidden = 256
    f = torch.from_numpy((rng.standard_normal(fd) * 2.0).astype(np.float32)).to(dev)
    ema0 = torch.from_numpy(rng.standard_normal(fd).astype(np.float32)).to(dev)
    ln_w = torch.from_numpy(rng.uniform(0.8, 1.2, fd).astype(np.float32)).to(dev)
    ln_b = torch.from_numpy((rng.standard_normal(fd) * 0.05).astype(np.float32)).to(dev)
    w1m = (rng.standard_normal((hidden, fd)) * 0.02).astype(np.float32)
    w1 = ops.QWeight.from_blocks(ops.L.F32, hidden, fd, w1m.tobytes(), dev)
    b1 = torch.from_numpy((rng.standard_normal(hidden) * 0.02).astype(np.float32)).to(dev)
    w2 = torch.from_numpy((rng.standard_normal(hidden) * 0.02).astype(np.float32)).to(dev)
    b2 = torch.from_numpy((rng.standard_normal(1) * 0.02).astype(np.float32)).to(dev)
    # separate launches
    rows = torch.empty(2, fd, device=dev)
    rows[0] = f
    ema_a = ema0.clone()
    ops.ema_habituate(rows[:1], rows[1:2], ema_a, first)
    ops.layernorm(rows, ln_w, ln_b, 1e-5, rows)
    h_a = ops.qlinear(w1, rows, bias=b1)
    out_a = torch.full((8,), -7.0, device=dev)
    idx = torch.tensor([5], dtype=torch.int32, device=dev)
    ops.seg_score_tail(h_a, w2, b2, 1, first, out_a[0:1], out_index=idx)
    # one step
    ema_b = ema0.clone()
    out_b = torch.full((8,), -7.0, device=dev)
    ops.seg_score_step(f, ema_b, first, w1, b1, ln_w, ln_b, 1e-5, w2, b2, out_b[0:1], out_index=idx)
    torch.cuda.synchronize()
    assert torch.equal(out_a, out_b) and out_b[5].item() != -7.0
    assert torch.equal(ema_a, ema_b)


@pytest.mark.parametrize("dt,rows,cols", [(9, 1536, 8960), (8, 1536, 8960), (9, 1536, 1536), (9, 256, 1536)])
@pytest.mark.parametrize("first", [True, False])
def test_score_jobs_with_a_gemv(dev, dt, rows, cols, first):
    """vgx_qlinear_side: the scorer's two jobs carried by a batch-1 GEMV launch (the 16-wave pieces
    GEMV of the down projection's shapes, Q4_0 / Q8_0) or launched after it (other shapes).  The GEMV
    result (accumulated) equals vgx_qlinear's, the score and the EMA state equal vgx_seg_score_step's,
    all bit for bit."""
    from vault_amd import vlt3
    rng = np.random.default_rng(rows + cols + dt + first)
    fd, hidden = 4608, 256
    w = ops.QWeight.from_blocks(dt, rows, cols, vlt3.synthetic_blocks(dt, rows, cols, rng), dev)
    x = torch.from_numpy(rng.standard_normal((1, cols)).astype(np.float32)).to(dev)
    y0 = torch.from_numpy(rng.standard_normal((1, rows)).astype(np.float32)).to(dev)
    f = torch.from_numpy((rng.standard_normal(fd) * 2.0).astype(np.float32)).to(dev)
    ema0 = torch.from_numpy(rng.standard_normal(fd).astype(np.float32)).to(dev)
    ln_w = torch.from_numpy(rng.uniform(0.8, 1.2, fd).astype(np.float32)).to(dev)
    ln_b = torch.from_numpy((rng.standard_normal(fd) * 0.05).astype(np.float32)).to(dev)
    w1 = ops.QWeight.from_blocks(ops.L.F32, hidden, fd,
                                 (rng.standard_normal((hidden, fd)) * 0.02).astype(np.float32).tobytes(), dev)
    b1, w2 = (torch.from_numpy((rng.standard_normal(hidden) * 0.02).astype(np.float32)).to(dev) for _ in range(2))
    b2 = torch.from_numpy((rng.standard_normal(1) * 0.02).astype(np.float32)).to(dev)
    idx = torch.tensor([3], dtype=torch.int32, device=dev)
    # reference: the GEMV and the scorer step on their own
    y_a = y0.clone()
    ops.qlinear(w, x, out=y_a, accumulate=True)
    ema_a, out_a = ema0.clone(), torch.full((8,), -7.0, device=dev)
    ops.seg_score_step(f, ema_a, first, w1, b1, ln_w, ln_b, 1e-5, w2, b2, out_a[0:1], out_index=idx)
    # the jobs with the GEMV (phase 1 with one launch, phase 2 with the next)
    y_b = y0.clone()
    ema_b, out_b = ema0.clone(), torch.full((8,), -7.0, device=dev)
    h = torch.full((2, hidden), float("nan"), device=dev)
    args = (f, ema_b, first, w1, b1, ln_w, ln_b, 1e-5, w2, b2, h, out_b[0:1], idx)
    ops.qlinear_side(w, x, y_b, True, ops.score_side(1, *args))
    y_c = y_b.clone()
    ops.qlinear_side(w, x, y_c, True, ops.score_side(2, *args))
    torch.cuda.synchronize()
    assert torch.equal(y_a, y_b)
    assert torch.equal(out_a, out_b) and out_b[3].item() != -7.0
    assert torch.equal(ema_a, ema_b)
    y_d = y_a.clone()
    ops.qlinear(w, x, out=y_d, accumulate=True)
    assert torch.equal(y_c, y_d)

