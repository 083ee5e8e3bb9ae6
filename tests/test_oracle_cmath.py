"""The oracle's fp32 restatement of the reference runtime's exp / erf / GELU (oracle/cmath.py) against the
runtime's own functions (runtime/vault3.c:104-129, compiled into oracle/_ref), bit for bit, over dense
sweeps that cover the subnormal range of exp, the |z| > 4 clamp of erf and both signs; and the
segment-bank merge restatement (oracle/segbank.py) against the runtime's update_segment_bank
(:1833-1915) on near-tie banks: scores one ulp apart, equal maxima separated only by the seg-id
tie-break, and equal candidate scores ranked by position."""
import numpy as np
import pytest

from oracle import cmath, ref, segbank

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")


def _same_bits(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def test_expf_matches_runtime():
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.uniform(-110, 95, 1_000_000).astype(np.float32),
        np.linspace(-104, -85, 200_001, dtype=np.float32),             # subnormal results
        np.linspace(-1, 1, 100_001, dtype=np.float32),
        np.array([0.0, -0.0, 88.72, np.nextafter(88.72, 0, dtype=np.float32), -103.9,
                  np.nextafter(-103.9, 0, dtype=np.float32), 1e-30, -1e-30, np.inf, -np.inf], np.float32)])
    assert _same_bits(cmath.expf(x), ref.math("exp", x))


@pytest.mark.parametrize("fn", ["erf", "gelu"])
def test_erf_gelu_match_runtime(fn):
    rng = np.random.default_rng(2)
    x = np.concatenate([
        rng.uniform(-9, 9, 1_000_000).astype(np.float32),
        (rng.standard_normal(500_000) * 2).astype(np.float32),
        np.linspace(3.99, 4.01, 20_001, dtype=np.float32), np.linspace(-5.7, -5.6, 20_001, dtype=np.float32),
        np.array([0.0, -0.0, 4.0, -4.0, 1e-20, -1e-20, 1e-39], np.float32)])
    got = cmath.erff(x) if fn == "erf" else cmath.geluf(x)
    assert _same_bits(got, ref.math(fn, x))


def test_exact_erf_gelu_is_not_the_runtime():
    """The Python model's exact-erf GELU (src/vault_v3_model.py:882) differs from the runtime's in the
    last bits for most inputs, so the bit-exact checks above are able to tell the two apart."""
    from scipy.special import erf
    x = np.random.default_rng(3).uniform(-6, 6, 100_000).astype(np.float32)
    exact = (0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / np.sqrt(2)))).astype(np.float32)
    assert (exact != ref.math("gelu", x)).mean() > 0.3
    assert np.max(np.abs(exact - ref.math("gelu", x))) < 1e-6


def near_tie_case(rng, W, M, ev=11, offset=100):
    """Evicted-chunk rings and a bank whose candidates nearly tie: segment maxima drawn from a few values
    and their one-ulp neighbours, so the ranks hinge on single ulps, on the -1e-6 * seg-id tie-break and
    on positions."""
    seg = np.sort(rng.integers(0, max(1, W // 6), W))
    seg = np.unique(seg, return_inverse=True)[1].astype(np.int64)
    base = np.float32(rng.choice([0.25, 1.5, 3.0]))
    levels = np.array([base, np.nextafter(base, np.float32(9), dtype=np.float32),
                       np.nextafter(base, np.float32(-9), dtype=np.float32), base + np.float32(1e-6)], np.float32)
    sc = levels[rng.integers(0, levels.size, W)] - np.float32(0.5) * rng.integers(0, 2, W).astype(np.float32)
    tok = rng.integers(0, 1000, W)
    mem_pos = np.sort(rng.choice(ev * W, M, replace=False)).astype(np.int64)
    # bank scores equal to candidate scores (ties broken by position) and one ulp around them
    g = (seg[rng.integers(0, W, M)] + offset) % 16384
    mem_score = (levels[rng.integers(0, levels.size, M)] - (np.float32(1e-6) * g.astype(np.float32))).astype(np.float32)
    return sc.astype(np.float32), seg, tok, mem_pos, mem_score, rng.integers(0, 1000, M), rng.integers(0, 500, M)


@pytest.mark.parametrize("M,budget,ev,n_pin,seed", [(0, 8, 11, 0, 0), (8, 8, 11, 0, 1), (20, 24, 11, 5, 2),
                                                     (24, 24, 11, 0, 3), (5, 12, 11, 0, 4), (0, 24, 0, 3, 5),
                                                     (0, 6, 0, 17, 6), (0, 24, 0, 64, 7)])
def test_segbank_restatement_matches_runtime_on_near_ties(M, budget, ev, n_pin, seed):
    from tests import modelgen
    cfg = modelgen.tiny_cfg(window=64, seg_budget=24)
    _, blob, _ = modelgen.build(cfg, "q8_0", seed=1)
    rt = ref.RefRuntime(blob)
    rng = np.random.default_rng(seed)
    off = 100
    sc, seg, tok, mem_pos, mem_score, mem_tok, mem_seg = near_tie_case(rng, cfg.window, M, ev, off)
    (pos, score, toks, segs), new_off = rt.seg_update(ev, n_pin, off, budget, sc, seg, tok, mem_pos, mem_score,
                                                      mem_tok, mem_seg)
    _, o_off, (o_pos, o_score, o_toks, o_segs), _, _ = segbank.evict(sc, seg, tok, mem_pos, mem_score, mem_tok,
                                                                     mem_seg, off, ev, n_pin if ev == 0 else 0, budget)
    assert new_off == o_off
    assert np.array_equal(pos, o_pos) and _same_bits(score, o_score)
    assert np.array_equal(toks, o_toks) and np.array_equal(segs, o_segs)
