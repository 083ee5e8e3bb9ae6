"""GPU parity of the decode-batch projection entry point (vgx_qkv_rope_batch): RMSNorm + q/k/v
projections as K-split partials, summed by the RoPE / ring-write launch.

Oracle chain per sequence, as for the one-token kernel: RMSNorm -> q/k/v GEMV + bias (oracle.linalg,
fp64 on the dequantized weights) -> rotate-half RoPE with the C-runtime table (oracle.rope); the ring /
sink writes must land at the slot of the step descriptor and nowhere else.  Bars: projections within
the fp32 accumulation bound of the fp64 oracle (rotation by an exact-norm 2x2 block at most doubles
it); bf16 state adds the rounding of the stored value.  The same step through the unfused path
(ops.qlinear, whose K-split reduce is a launch of its own, then ops.rope_qkv_write_step) must agree
to a few fp32 ulps.
"""
import numpy as np
import pytest
import torch

from oracle import codec, linalg, rope
from vault_amd import _lib as L
from vault_amd import ops, vlt3

pytestmark = pytest.mark.gpu

E_DTYPE, E_SHAPE, E_ARENA, E_LIMIT, E_ALIGN, E_ARG = -5, -7, -8, -10, -11, -31

CASES = [
    # (q dtype or None for one q|k|v weight, kv dtype, d_model, H, G, D, batch, state dtype, slot, table row, sink)
    (codec.Q4_0, codec.Q8_0, 1536, 12, 2, 128, 32, torch.float32, 672, 1696, -1),
    (codec.Q4_0, codec.Q8_0, 1536, 12, 2, 128, 64, torch.bfloat16, 1023, 2047, 7),
    (None, codec.Q8_0, 1536, 12, 2, 128, 17, torch.float32, 5, 5, 5),
    (None, codec.Q4_0, 256, 4, 2, 64, 8, torch.bfloat16, 3, 19, -1),
    (codec.Q8_0, codec.Q4_0, 512, 8, 1, 64, 9, torch.float32, 0, 16, 0),
]


def _fmt(dt):
    return {codec.Q8_0: "q8", codec.Q4_0: "q4", None: "one"}[dt]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{_fmt(c[0])}-{_fmt(c[1])}-d{c[2]}-B{c[6]}-{str(c[7])[6:]}")
def test_qkv_rope_batch_matches_oracle(dev, case):
    dq, dkv, d, H, G, D, B, sdt, slot, trow, sink = case
    rng = np.random.default_rng(d + H + B + slot)
    W, S = 1024, 512
    HD, GD = H * D, G * D
    kv_rows = 2 * GD if dq is not None else HD + 2 * GD
    raw_kv = vlt3.synthetic_blocks(dkv, kv_rows, d, rng)
    wkv = ops.QWeight.from_blocks(dkv, kv_rows, d, raw_kv, dev)
    Wkv = codec.decode(dkv, raw_kv, kv_rows, d).astype(np.float64)
    bkv = (rng.standard_normal(kv_rows) * 0.1).astype(np.float32)
    if dq is not None:
        raw_q = vlt3.synthetic_blocks(dq, HD, d, rng)
        wq = ops.QWeight.from_blocks(dq, HD, d, raw_q, dev)
        Wq = codec.decode(dq, raw_q, HD, d).astype(np.float64)
        bq = (rng.standard_normal(HD) * 0.1).astype(np.float32)
    else:
        wq, Wq, bq = None, Wkv[:HD], bkv[:HD]
        Wkv = Wkv[HD:]
    bkv_o = bkv if dq is not None else bkv[HD:]
    x = rng.standard_normal((B, d)).astype(np.float32) * 3.0
    lnw = (rng.random(d) * 0.4 + 0.8).astype(np.float32)
    neg = 2048
    cos, sin = rope.table_c(np.arange(-neg, 2 * W), D, 1e6)
    table = torch.from_numpy(np.concatenate([cos, sin], axis=1)).to(dev)
    stepv = torch.tensor([slot, trow, sink, slot + 1] + [0] * 12, dtype=torch.int32, device=dev)

    def ring(n):
        return torch.randn(B, G, n, D, device=dev).to(sdt)
    k_rot, k_raw, v_cur = ring(W), ring(W), ring(W)
    sk, sv = ring(S), ring(S)
    before = [t.clone() for t in (k_rot, k_raw, v_cur, sk, sv)]
    q_out = torch.full((B, H, D), float("nan"), device=dev)
    xd = torch.from_numpy(x).to(dev)
    lnw_d = torch.from_numpy(lnw).to(dev)
    bq_d = torch.from_numpy(bq).to(dev) if dq is not None else None
    bkv_d = torch.from_numpy(bkv).to(dev)
    ops.qkv_rope_batch(wq, bq_d, wkv, bkv_d, xd, (lnw_d, 1e-6), table, D, stepv, q_out, k_rot, k_raw, v_cur, sk, sv)
    torch.cuda.synchronize()

    u = linalg.rmsnorm(x.astype(np.float64), lnw.astype(np.float64), 1e-6)
    q = linalg.gemv(Wq, u, bq.astype(np.float64))
    kv = linalg.gemv(Wkv, u, bkv_o.astype(np.float64))
    k, v = kv[:, :GD], kv[:, GD:]
    c, s_ = cos[trow].astype(np.float64), sin[trow].astype(np.float64)
    swap = list(range(D // 2, D)) + list(range(D // 2))
    bnd_q = linalg.gemv_bound(Wq, u, dq if dq is not None else dkv).reshape(B, H, D)
    bnd_kv = linalg.gemv_bound(Wkv, u, dkv)
    bk = bnd_kv[:, :GD].reshape(B, G, D)
    bk = np.maximum(bk, bk[:, :, swap])
    bv = bnd_kv[:, GD:].reshape(B, G, D)
    tol_state = 1e-2 if sdt == torch.bfloat16 else 0.0

    def close(got, want, bnd, rel_state):
        got = got.double().cpu().numpy()
        lim = 2 * bnd + rel_state * np.abs(want) + 1e-7
        assert np.all(np.abs(got - want) <= lim), float(np.max(np.abs(got - want) - lim))

    for b in range(B):
        qr = rope.rotate(q[b].reshape(H, D), c, s_)
        kr = rope.rotate(k[b].reshape(G, D), c, s_)
        close(q_out[b], qr, np.maximum(bnd_q[b], bnd_q[b][:, swap]), 0.0)
        close(k_rot[b, :, slot], kr, bk[b], tol_state)
        close(k_raw[b, :, slot], k[b].reshape(G, D), bk[b], tol_state)
        close(v_cur[b, :, slot], v[b].reshape(G, D), bv[b], tol_state)
        if sink >= 0:
            close(sk[b, :, sink], k[b].reshape(G, D), bk[b], tol_state)
            close(sv[b, :, sink], v[b].reshape(G, D), bv[b], tol_state)
    for t, t0, row in ((k_rot, before[0], slot), (k_raw, before[1], slot), (v_cur, before[2], slot),
                       (sk, before[3], sink), (sv, before[4], sink)):
        keep = torch.ones(t.shape[2], dtype=torch.bool)
        if row >= 0:
            keep[row] = False
        assert torch.equal(t[:, :, keep.to(dev)], t0[:, :, keep.to(dev)])

    # the unfused path: separate projections (reduce launch of their own), then the RoPE / ring write
    if dq is not None:
        q2 = ops.qlinear(wq, xd, bias=bq_d, norm=(lnw_d, 1e-6)).view(B, H, D)
        kv2 = ops.qlinear(wkv, xd, bias=bkv_d, norm=(lnw_d, 1e-6))
        k2, v2 = kv2[:, :GD].view(B, G, D), kv2[:, GD:].view(B, G, D)
    else:
        qkv2 = ops.qlinear(wkv, xd, bias=bkv_d, norm=(lnw_d, 1e-6))
        q2 = qkv2[:, :HD].view(B, H, D)
        k2, v2 = qkv2[:, HD:HD + GD].view(B, G, D), qkv2[:, HD + GD:].view(B, G, D)
    rings2 = [t0.clone() for t0 in before]
    ops.rope_qkv_write_step(q2, k2, v2, table, D, stepv, *rings2)
    torch.cuda.synchronize()
    sc = float(q_out.abs().max())
    assert torch.allclose(q_out, q2, rtol=0, atol=4e-7 * sc)
    for got, want in zip((k_rot, k_raw, v_cur, sk, sv), rings2):
        assert torch.allclose(got.float(), want.float(), rtol=8e-3 if sdt == torch.bfloat16 else 0,
                              atol=4e-7 * float(want.float().abs().max()))


def test_qkv_rope_batch_rejects_bad_arguments(dev):
    lib = L.load()
    s = torch.cuda.current_stream().cuda_stream
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device=dev)
    p = buf.data_ptr()
    assert lib.vgx_qkv_rope_batch_workspace_bytes(8, 100, 4, 2, 64, 1) == E_SHAPE

    def call(B=8, d=256, kvw=L.Q8_0, wq=None, bq=None, x=p, ws_bytes=1 << 20, kvd=L.F32):
        return lib.vgx_qkv_rope_batch(L.Q8_0, wq, bq, kvw, p, None, d, 4, 2, 64, x, d, B, None, 0.0, p, 64, p, p,
                                      256, kvd, None, None, p, 0, 0, 0, None, None, 0, 0, 0, p, ws_bytes, s)
    assert call(B=65) == E_LIMIT            # beyond the small-batch kernel
    assert call(kvw=L.F32) == E_DTYPE
    assert call(kvd=L.Q8_0) == E_DTYPE
    assert call(d=100) == E_SHAPE
    assert call(bq=p) == E_ARG              # one q|k|v weight takes its bias in bkv
    assert call(x=p + 4) == E_ALIGN
    assert call(ws_bytes=256) == E_ARENA
