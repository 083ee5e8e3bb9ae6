"""Pins the attention and RoPE oracles (CPU).

* ``oracle.attention.decode`` / ``chunk`` against torch's scaled_dot_product_attention in float64
  (an independent implementation; torch is the reference's own attention backend,
  src/vault_v3_model.py:1136), with GQA expansion g = h // (H/G) (src/vault_v3_model.py:797-802).
* Closed-form special cases: a single key returns its value; identical keys return the mean of the
  values; a -inf bias on a span removes that span; decode == chunk with one query.
* ``oracle.attention.block_sliding`` equals full causal attention for L <= 2W and no sinks
  (tests/test_vault_v3.py:175-181 asserts the same of the reference), and for L > 2W equals
  per-chunk attention assembled from ``chunk`` with sinks re-rotated to (i-1)W - S + j
  (src/vault_v3_model.py:805-809, 849-856).
* ``oracle.rope``: R_0 = identity, norm preservation, R_a R_b = R_(a+b), relative-position invariance
  of q.k, and the two angle conventions agree to fp32 rounding at small positions
  (runtime/vault3.c:840-849 vs src/vault_v3_model.py:777-782).
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oatt
from oracle import rope as orope


def _sdpa(q, K, V, mask=None):
    """q [B,H,T,D], K/V [B,H,n,D] float64 torch; mask [T,n] bool (True = visible)."""
    return F.scaled_dot_product_attention(q, K, V, attn_mask=mask)


@pytest.mark.parametrize("lens,G,H", [([7], 2, 12), ([3, 0, 11, 5], 2, 12), ([16, 4], 1, 4), ([9, 9], 4, 8)])
def test_decode_matches_torch_sdpa(lens, G, H):
    rng = np.random.default_rng(sum(lens) + H)
    B, D = 2, 64
    spans = [(rng.standard_normal((B, G, n, D)), rng.standard_normal((B, G, n, D))) for n in lens]
    q = rng.standard_normal((B, H, D))
    got = oatt.decode(q, spans)
    K = np.concatenate([k for k, _ in spans], axis=2)
    V = np.concatenate([v for _, v in spans], axis=2)
    Ke = torch.from_numpy(np.repeat(K, H // G, axis=1))
    Ve = torch.from_numpy(np.repeat(V, H // G, axis=1))
    ref = _sdpa(torch.from_numpy(q)[:, :, None], Ke, Ve)[:, :, 0].numpy()
    assert np.abs(got - ref).max() < 1e-12


def test_decode_bias_matches_additive_mask():
    rng = np.random.default_rng(4)
    B, H, G, D = 1, 6, 2, 32
    spans = [(rng.standard_normal((B, G, n, D)), rng.standard_normal((B, G, n, D))) for n in (5, 8, 6)]
    q = rng.standard_normal((B, H, D))
    bias = rng.standard_normal((H, 8))
    got = oatt.decode(q, spans, bias=bias, bias_span=1)
    K = np.concatenate([k for k, _ in spans], axis=2)
    V = np.concatenate([v for _, v in spans], axis=2)
    full = np.zeros((H, 19))
    full[:, 5:13] = bias
    Ke = torch.from_numpy(np.repeat(K, H // G, axis=1))
    Ve = torch.from_numpy(np.repeat(V, H // G, axis=1))
    ref = _sdpa(torch.from_numpy(q)[:, :, None], Ke, Ve, torch.from_numpy(full)[None, :, None, :])[:, :, 0].numpy()
    assert np.abs(got - ref).max() < 1e-12


def test_decode_special_cases():
    rng = np.random.default_rng(5)
    B, H, G, D = 1, 4, 2, 16
    q = rng.standard_normal((B, H, D))
    k1, v1 = rng.standard_normal((B, G, 1, D)), rng.standard_normal((B, G, 1, D))
    out = oatt.decode(q, [(k1, v1)])
    assert np.allclose(out, np.repeat(v1[:, :, 0], H // G, axis=1), atol=1e-15)
    ks = np.repeat(k1, 9, axis=2)
    vs = rng.standard_normal((B, G, 9, D))
    out = oatt.decode(q, [(ks, vs)])
    assert np.allclose(out, np.repeat(vs.mean(axis=2), H // G, axis=1), atol=1e-12)
    a = (rng.standard_normal((B, G, 6, D)), rng.standard_normal((B, G, 6, D)))
    b = (rng.standard_normal((B, G, 4, D)), rng.standard_normal((B, G, 4, D)))
    out = oatt.decode(q, [a, b], bias=np.full((H, 6), -np.inf), bias_span=0)
    assert np.allclose(out, oatt.decode(q, [b]), atol=1e-14)


def test_chunk_matches_sdpa_and_decode():
    rng = np.random.default_rng(6)
    T, H, G, D, P = 7, 4, 2, 32, 10
    q = rng.standard_normal((T, H, D))
    pk, pv = rng.standard_normal((G, P, D)), rng.standard_normal((G, P, D))
    ck, cv = rng.standard_normal((G, T, D)), rng.standard_normal((G, T, D))
    got = oatt.chunk(q, [(pk, pv)], ck, cv)
    K = np.concatenate([pk, ck], axis=1)
    V = np.concatenate([pv, cv], axis=1)
    mask = torch.from_numpy(np.arange(P + T)[None, :] <= P + np.arange(T)[:, None])
    ref = _sdpa(torch.from_numpy(q.transpose(1, 0, 2))[None], torch.from_numpy(np.repeat(K, H // G, 0))[None],
                torch.from_numpy(np.repeat(V, H // G, 0))[None], mask)[0].numpy().transpose(1, 0, 2)
    assert np.abs(got - ref).max() < 1e-12
    for t in range(T):   # query t of the chunk == a decode step over prefix + first t+1 keys
        d = oatt.decode(q[t][None], [(pk[None], pv[None]), (ck[None, :, :t + 1], cv[None, :, :t + 1])])[0]
        assert np.abs(d - got[t]).max() < 1e-12


def test_block_sliding_equals_full_causal_within_2w():
    rng = np.random.default_rng(7)
    L, H, G, D, W = 30, 4, 2, 16, 16
    q, k, v = rng.standard_normal((L, H, D)), rng.standard_normal((L, G, D)), rng.standard_normal((L, G, D))
    got = oatt.block_sliding(q, k, v, k, W=W, S=0, theta=1e6)
    mask = torch.from_numpy(np.tril(np.ones((L, L), dtype=bool)))
    ref = _sdpa(torch.from_numpy(q.transpose(1, 0, 2))[None], torch.from_numpy(np.repeat(k, H // G, 1).transpose(1, 0, 2))[None],
                torch.from_numpy(np.repeat(v, H // G, 1).transpose(1, 0, 2))[None], mask)[0].numpy().transpose(1, 0, 2)
    assert np.abs(got - ref).max() < 1e-12


def test_block_sliding_chunks_with_sinks():
    rng = np.random.default_rng(8)
    L, H, G, D, W, S, theta = 53, 4, 2, 16, 12, 5, 1e6
    q, k, v = rng.standard_normal((L, H, D)), rng.standard_normal((L, G, D)), rng.standard_normal((L, G, D))
    kraw = rng.standard_normal((L, G, D))
    got = oatt.block_sliding(q, k, v, kraw, W=W, S=S, theta=theta)
    for i in range((L + W - 1) // W):
        r0, r1 = i * W, min(L, (i + 1) * W)
        lo = max(0, (i - 1) * W)
        prefix = []
        if i >= 2:
            c, s_ = orope.table_torch((i - 1) * W - S + np.arange(S), D, theta)
            ks = orope.rotate(kraw[:S].transpose(1, 0, 2), c, s_)
            prefix.append((ks, v[:S].transpose(1, 0, 2)))
        if i >= 1:
            prefix.append((k[lo:r0].transpose(1, 0, 2), v[lo:r0].transpose(1, 0, 2)))
        want = oatt.chunk(q[r0:r1], prefix, k[r0:r1].transpose(1, 0, 2), v[r0:r1].transpose(1, 0, 2))
        assert np.abs(got[r0:r1] - want).max() < 1e-12, i


@pytest.mark.parametrize("table", [orope.table_c, orope.table_torch])
def test_rope_identities(table):
    rng = np.random.default_rng(9)
    D, theta = 128, 1e6
    z = rng.standard_normal((5, D))
    c0, s0 = table([0], D, theta)
    assert np.array_equal(orope.rotate(z, c0, s0), z)
    c, s = table([777], D, theta)
    r = orope.rotate(z, c, s)
    assert np.allclose(np.linalg.norm(r, axis=-1), np.linalg.norm(z, axis=-1), rtol=1e-6)
    ca, sa = table([300], D, theta)
    cb, sb = table([-200], D, theta)
    cab, sab = table([100], D, theta)
    assert np.abs(orope.rotate(orope.rotate(z, ca, sa), cb, sb) - orope.rotate(z, cab, sab)).max() < 1e-4
    qv, kv = rng.standard_normal(D), rng.standard_normal(D)
    dots = []
    for p in (0, 50, 1000):
        cq, sq = table([p + 37], D, theta)
        ck, sk = table([p], D, theta)
        dots.append(orope.rotate(qv[None], cq, sq)[0] @ orope.rotate(kv[None], ck, sk)[0])
    # double-precision angles keep q.k translation invariant to fp32 rounding; the fp32 angles of
    # the Python reference drift by ~1e-4 rad near position 1000 (the gap between the two references)
    tol = 1e-5 if table is orope.table_c else 1e-3
    assert np.allclose(dots, dots[0], rtol=0, atol=tol)


def test_rope_conventions_agree_at_small_positions():
    D, theta = 128, 1e6
    pos = np.arange(0, 64)
    cc, sc = orope.table_c(pos, D, theta)
    ct, st = orope.table_torch(pos, D, theta)
    assert np.abs(cc - ct).max() < 1e-5 and np.abs(sc - st).max() < 1e-5


def _block_cfg():
    from tests import modelgen
    cfg = modelgen.tiny_cfg(seg_budget=0, window=16)
    return cfg, modelgen.build(cfg, "q8_0", seed=6)[2]


@pytest.mark.parametrize("seed", [0, 1])
def test_block_forward_equals_stream_with_sinks(seed):
    """The reference's own identity (tests/test_vault_v3.py:52-75): the parallel block form of a batch
    row (sinks re-rotated to (i-1)W - S + j, absolute positions) equals that row's token stream (sinks
    pinned, re-based ring positions, re-rotation at every chunk boundary) beyond 2W tokens.  This pins
    the sink-position rule of ``block_sliding`` through an independent path."""
    from oracle.model import OracleModel
    from tests import modelgen
    cfg, deq = _block_cfg()
    om = OracleModel(cfg, deq)
    ids = modelgen.ids_stream(cfg, 75, seed=20 + seed)            # 4.7 chunks: sinks from chunk 2 on
    blk = om.forward_block(ids)
    st = om.new_state(seg_budget=0)
    om.set_pinned(st, cfg.n_sink)
    stream = om.stream(ids, st)
    assert np.abs(blk - stream).max() < 1e-4 * max(1.0, np.abs(stream).max())
    # full causal equals block sliding within 2W tokens (tests/test_vault_v3.py:175-181)
    short = ids[:2 * cfg.window]
    assert np.abs(om.forward_block(short, mode="full") - om.forward_block(short)).max() == 0.0


@pytest.mark.parametrize("shift", [-1, 1, "chunk"])
def test_block_forward_identity_catches_wrong_sink_positions(shift):
    """Planted mistakes in the sink rule (one position off either way, or the sinks placed before the
    current chunk instead of the previous one) break the identity by far more than its bar."""
    from oracle import attention as oatt
    from oracle.model import OracleModel
    from tests import modelgen
    cfg, deq = _block_cfg()
    om = OracleModel(cfg, deq)
    ids = modelgen.ids_stream(cfg, 75, seed=20)
    if shift == "chunk":
        bad = lambda i, W, S: np.maximum(0, i * W - S + np.arange(S))
    else:
        bad = lambda i, W, S: np.maximum(0, (i - 1) * W - S + np.arange(S) + shift)
    st = om.new_state(seg_budget=0)
    om.set_pinned(st, cfg.n_sink)
    stream = om.stream(ids, st)
    wrong = om.forward_block(ids, sink_pos=bad)
    assert np.abs(wrong - stream).max() > 1e-3 * max(1.0, np.abs(stream).max())
    assert np.array_equal(oatt.sink_positions(3, 16, 4), [28, 29, 30, 31])
