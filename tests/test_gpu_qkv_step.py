"""GPU parity of the one-token fused projection kernel (vgx_qkv_rope_step) and of the RoPE-pair weight
packing it reads, against the oracle.

The oracle chain is RMSNorm -> q/k/v GEMV + bias (oracle.linalg, fp64 on the dequantized weights) ->
rotate-half RoPE with the C-runtime table (oracle.rope); the ring / sink writes must land at the slot
of the step descriptor and nowhere else.  Bars: packing bit-exact; projections within the fp32
accumulation bound of the fp64 oracle; rotated values within that bound (rotation by an exact-norm
2x2 block does not enlarge it beyond 2x).
"""
import numpy as np
import pytest
import torch

from oracle import codec, linalg, rope
from vault_amd import _lib as L
from vault_amd import ops, vlt3

pytestmark = pytest.mark.gpu


def _raw(dt, rows, cols, rng):
    if dt == codec.F32:
        return (rng.standard_normal((rows, cols)).astype(np.float32) * 0.05).tobytes()
    return vlt3.synthetic_blocks(dt, rows, cols, rng)


def _perm(rows, D, n_rope):
    """Natural row of each packed row in the RoPE-pair order."""
    out = []
    for p in range(rows):
        if p < n_rope:
            h, w = divmod(p, D)
            j, k = divmod(w, 4)
            out.append(h * D + 2 * j + (k >> 1) + (k & 1) * (D // 2))
        else:
            out.append(p)
    return np.array(out)


@pytest.mark.parametrize("dt", [codec.Q8_0, codec.Q4_0, codec.F32])
@pytest.mark.parametrize("rows,D,n_rope", [(1536, 128, 1536), (512, 128, 256), (192, 64, 64)])
def test_pack_rope_is_a_row_permutation(dev, dt, rows, D, n_rope):
    rng = np.random.default_rng(rows + D)
    cols = 96
    raw = _raw(dt, rows, cols, rng)
    w = ops.QWeight.rope_from_blocks(dt, rows, cols, raw, D, n_rope, dev)
    got = w.dequant().cpu().numpy()
    want = codec.decode(dt, raw, rows, cols)[_perm(rows, D, n_rope)]
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_pack_rope_rejects_bad_shapes(dev):
    lib = L.load()
    dst = torch.empty(1 << 16, dtype=torch.uint8, device=dev)
    src = torch.zeros(1 << 16, dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    assert lib.vgx_qweight_pack_rope(L.Q8_0, src.data_ptr(), dst.data_ptr(), 256, 64, 6, 252, s) < 0
    assert lib.vgx_qweight_pack_rope(L.Q8_0, src.data_ptr(), dst.data_ptr(), 256, 64, 128, 384, s) < 0
    assert lib.vgx_qweight_pack_rope(L.Q8_0, src.data_ptr(), dst.data_ptr(), 256, 64, 128, 64, s) < 0


CASES = [
    # (q dtype, kv dtype, d_model, H, G, D, state dtype, slot, table row, sink slot)
    (codec.Q4_0, codec.Q8_0, 1536, 12, 2, 128, torch.float32, 672, 1696, -1),
    (codec.Q8_0, codec.Q8_0, 1536, 12, 2, 128, torch.float32, 5, 5, 5),
    (codec.Q4_0, codec.Q8_0, 1536, 12, 2, 128, torch.bfloat16, 1023, 2047, -1),
    (codec.Q4_0, codec.Q4_0, 256, 4, 2, 64, torch.float32, 3, 19, 3),
    (codec.F32, codec.F32, 128, 4, 1, 64, torch.float32, 0, 16, 0),
    (codec.Q8_0, codec.Q8_0, 2560, 16, 4, 128, torch.bfloat16, 17, 1041, 17),   # two passes of 64 blocks
]


@pytest.mark.parametrize("case", CASES)
def test_qkv_rope_step_matches_oracle(dev, case):
    dq, dkv, d, H, G, D, sdt, slot, trow, sink = case
    rng = np.random.default_rng(d + H + slot)
    W, S = 1024, 512
    raw_q = _raw(dq, H * D, d, rng)
    raw_kv = _raw(dkv, 2 * G * D, d, rng)
    wq = ops.QWeight.rope_from_blocks(dq, H * D, d, raw_q, D, H * D, dev)
    wkv = ops.QWeight.rope_from_blocks(dkv, 2 * G * D, d, raw_kv, D, G * D, dev)
    Wq = codec.decode(dq, raw_q, H * D, d).astype(np.float64)
    Wkv = codec.decode(dkv, raw_kv, 2 * G * D, d).astype(np.float64)
    x = rng.standard_normal(d).astype(np.float32) * 3.0
    lnw = (rng.random(d) * 0.4 + 0.8).astype(np.float32)
    bq = (rng.standard_normal(H * D) * 0.1).astype(np.float32)
    bkv = (rng.standard_normal(2 * G * D) * 0.1).astype(np.float32)
    # RoPE table rows of positions [-neg, 2W) as the model builds it
    neg = 2048
    cos, sin = rope.table_c(np.arange(-neg, 2 * W), D, 1e6)
    table = torch.from_numpy(np.concatenate([cos, sin], axis=1)).to(dev)
    stepv = torch.tensor([slot, trow, sink, slot + 1] + [0] * 12, dtype=torch.int32, device=dev)

    def ring(n):
        return torch.randn(1, G, n, D, device=dev).to(sdt)
    k_rot, k_raw, v_cur = ring(W), ring(W), ring(W)
    sk, sv = ring(S), ring(S)
    before = [t.clone() for t in (k_rot, k_raw, v_cur, sk, sv)]
    q_out = torch.empty(1, H, D, device=dev)
    xd = torch.from_numpy(x).to(dev).reshape(1, d)
    xc = torch.full((1, d), -7.0, device=dev)
    ops.qkv_rope_step(wq, torch.from_numpy(bq).to(dev), wkv, torch.from_numpy(bkv).to(dev), xd,
                      (torch.from_numpy(lnw).to(dev), 1e-6), table, D, stepv, q_out, k_rot, k_raw, v_cur, sk, sv,
                      x_copy=xc)
    torch.cuda.synchronize()

    u = linalg.rmsnorm(x.astype(np.float64)[None], lnw.astype(np.float64), 1e-6)[0]
    q = linalg.gemv(Wq, u[None], bq.astype(np.float64))[0]
    kv = linalg.gemv(Wkv, u[None], bkv.astype(np.float64))[0]
    k, v = kv[:G * D], kv[G * D:]
    c, s_ = cos[trow].astype(np.float64), sin[trow].astype(np.float64)
    qr = rope.rotate(q.reshape(H, D), c, s_)
    kr = rope.rotate(k.reshape(G, D), c, s_)
    bnd_q = linalg.gemv_bound(Wq, u[None], dq).reshape(H, D)
    bnd_kv = linalg.gemv_bound(Wkv, u[None], dkv).reshape(-1)
    tol_state = 1e-2 if sdt == torch.bfloat16 else 0.0   # bf16 state: rounding of the stored value

    def close(got, want, bnd, rel_state):
        got = got.double().cpu().numpy()
        lim = 2 * bnd + rel_state * np.abs(want) + 1e-7
        assert np.all(np.abs(got - want) <= lim), float(np.max(np.abs(got - want) - lim))

    close(q_out[0], qr, np.maximum(bnd_q, bnd_q[:, list(range(D // 2, D)) + list(range(D // 2))]), 0.0)
    bk = bnd_kv[:G * D].reshape(G, D)
    bk = np.maximum(bk, bk[:, list(range(D // 2, D)) + list(range(D // 2))])
    close(k_rot[0, :, slot], kr, bk, tol_state)
    close(k_raw[0, :, slot], k.reshape(G, D), bk, tol_state)
    close(v_cur[0, :, slot], v.reshape(G, D), bnd_kv[G * D:].reshape(G, D), tol_state)
    if sink >= 0:
        close(sk[0, :, sink], k.reshape(G, D), bk, tol_state)
        close(sv[0, :, sink], v.reshape(G, D), bnd_kv[G * D:].reshape(G, D), tol_state)
    # nothing else of the state changed
    for t, t0, row in ((k_rot, before[0], slot), (k_raw, before[1], slot), (v_cur, before[2], slot),
                       (sk, before[3], sink), (sv, before[4], sink)):
        keep = torch.ones(t.shape[2], dtype=torch.bool)
        if row >= 0:
            keep[row] = False
        assert torch.equal(t[:, :, keep.to(dev)], t0[:, :, keep.to(dev)])
    assert torch.equal(xc, xd)


def test_qkv_rope_step_rejects_bad_arguments(dev):
    lib = L.load()
    z = torch.zeros(1 << 22, dtype=torch.float32, device=dev)   # larger than any read the shapes imply
    p = z.data_ptr()
    s = torch.cuda.current_stream().cuda_stream

    def call(q_dtype=L.Q4_0, kv_w=L.Q8_0, d=1536, H=12, G=2, D=128, x=p, kv=L.F32, sink_v=p):
        return lib.vgx_qkv_rope_step(q_dtype, p, None, kv_w, p, None, d, H, G, D, x, p, 1e-6, None, p, D, p, p,
                                     kv, p, p, p, 128, 128, p, sink_v, 128, 128, s)
    assert call(q_dtype=L.Q8_0, kv_w=L.Q4_0) < 0          # unsupported dtype pair
    assert call(kv=L.Q8_0) < 0                             # state dtype
    assert call(d=1000) < 0                                # d_model % 32
    assert call(D=130) < 0                                 # D % 4
    assert call(H=12, G=5) < 0                             # H % G
    assert call(x=p + 4) < 0                               # alignment
    assert call(sink_v=None) < 0                           # sinks both or neither
