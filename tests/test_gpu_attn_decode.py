"""GPU parity of split-K decode attention and the row kernels against the float64 oracle.

Bars: attention max |d| <= 1e-5 with fp32 KV, <= 2e-3 with bf16 KV (oracle
fed the same bf16-rounded K/V); RoPE / RMSNorm within fp32 rounding; gather bit-exact.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import linalg, rope as orope
from vault_amd import ops

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-3}


def _spans(rng, B, G, D, lens, dtype, dev):
    out = []
    for n in lens:
        k = torch.from_numpy(rng.standard_normal((B, G, n, D)).astype(np.float32)).to(dtype)
        v = torch.from_numpy(rng.standard_normal((B, G, n, D)).astype(np.float32)).to(dtype)
        out.append((k.to(dev), v.to(dev)))
    return out


def _np(spans):
    return [(k.float().cpu().numpy(), v.float().cpu().numpy()) for k, v in spans]


@pytest.mark.parametrize("lens", [[64, 0, 1024, 1024], [1], [5, 0, 0, 17], [512, 1024, 1024, 1024]])
def test_decode_fp32_config1_shapes(dev, lens):
    rng = np.random.default_rng(sum(lens))
    B, H, G, D = 1, 12, 2, 128
    sp = _spans(rng, B, G, D, lens, torch.float32, dev)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    out = ops.attn_decode(torch.from_numpy(q).to(dev), sp).cpu().numpy()
    ref = oatt.decode(q, _np(sp))
    assert np.abs(out - ref).max() <= TOL[torch.float32]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_batched_config3(dev, dtype):
    """Batch 64, 512 sink + 1024 segment + 2048 window = 3584 keys, bias on the segment span."""
    rng = np.random.default_rng(3)
    B, H, G, D = 64, 12, 2, 128
    lens = [512, 1024, 1024, 1024]
    sp = _spans(rng, B, G, D, lens, dtype, dev)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    bias = (rng.standard_normal((H, 1024)) * 2.0).astype(np.float32)
    bias[:2] = 0.0
    bias[2, 100:110] = -1e30
    out = ops.attn_decode(torch.from_numpy(q).to(dev), sp, bias=torch.from_numpy(bias).to(dev),
                          bias_span=1).cpu().numpy()
    ref = oatt.decode(q, _np(sp), bias=bias, bias_span=1)
    assert np.abs(out - ref).max() <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 2, 16, 64])
def test_decode_split_tickets_reset_between_calls(dev, dtype, B):
    """Batch 64 (4 splits per (b, g)): the last workgroup of a pair merges its splits and puts the
    pair's ticket back to zero; batch 16 (16 splits) merges with the second launch; batch 1 and 2
    (56 splits of 64 keys per pair, one launch) merge in the pair's last workgroup.  Five calls on
    one workspace (and a graph replayed three times) give the same bits and match the oracle; the
    ticket words are zero afterwards."""
    rng = np.random.default_rng(B)
    H, G, D = 12, 2, 128
    lens = [512, 1024, 1024, 1024]
    sp = _spans(rng, B, G, D, lens, dtype, dev)
    q = torch.from_numpy(rng.standard_normal((B, H, D)).astype(np.float32)).to(dev)
    ws = ops.Workspace(dev)
    outs = [ops.attn_decode(q, sp, ws=ws).clone() for _ in range(5)]
    for o in outs[1:]:
        assert torch.equal(o, outs[0])
    ref = oatt.decode(q.cpu().numpy(), _np(sp))
    assert np.abs(outs[0].cpu().numpy() - ref).max() <= TOL[dtype]
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.attn_decode(q, sp, out=out, ws=ws)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.attn_decode(q, sp, out=out, ws=ws)
    for _ in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, outs[0])
    assert int(ws.buf[:B * G * 4].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B", [1, 2])
@pytest.mark.parametrize("m_live,c_live", [(700, 300), (1024, 1024), (0, 1), (5, 63)])
def test_decode_step_shape_bias_and_device_lengths(dev, dtype, B, m_live, c_live):
    """The decode step's spans at batch 1 and 2 (the one-launch kernel for few (batch, group) pairs):
    512 sinks | a segment bank of capacity 1024 with m_live slots counted on the device, with a bias per
    head on it (zero rows for the unbiased heads, -1e30 entries) | 1024 previous | the current window
    with c_live rows counted on the device.  Rows past the device counts hold NaN, which must not reach
    the output."""
    rng = np.random.default_rng(m_live * 3 + c_live + B)
    H, G, D = 12, 2, 128
    caps = [512, 1024, 1024, 1024]
    sp = _spans(rng, B, G, D, caps, dtype, dev)
    for i, n in ((1, m_live), (3, c_live)):
        sp[i][0][:, :, n:] = float("nan")
        sp[i][1][:, :, n:] = float("nan")
    m_dev = torch.tensor([m_live], dtype=torch.int32, device=dev)
    c_dev = torch.tensor([c_live], dtype=torch.int32, device=dev)
    spans = [sp[0], (sp[1][0], sp[1][1], m_dev), sp[2], (sp[3][0], sp[3][1], c_dev)]
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    bias = (rng.standard_normal((H, 1024)) * 2.0).astype(np.float32)
    bias[:2] = 0.0
    bias[2, 3:9] = -1e30
    out = ops.attn_decode(torch.from_numpy(q).to(dev), spans, bias=torch.from_numpy(bias).to(dev), bias_span=1)
    live = _np([sp[0], (sp[1][0][:, :, :m_live], sp[1][1][:, :, :m_live]), sp[2],
                (sp[3][0][:, :, :c_live], sp[3][1][:, :, :c_live])])
    ref = oatt.decode(q, live, bias=bias[:, :m_live], bias_span=1)
    assert np.abs(out.cpu().numpy() - ref).max() <= TOL[dtype]


@pytest.mark.parametrize("grp,D", [(1, 64), (2, 128), (4, 64), (6, 128), (8, 128)])
def test_decode_group_and_dim(dev, grp, D):
    rng = np.random.default_rng(grp * D)
    B, G = 3, 2
    H = G * grp
    sp = _spans(rng, B, G, D, [7, 33, 200, 99], torch.float32, dev)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    out = ops.attn_decode(torch.from_numpy(q).to(dev), sp).cpu().numpy()
    assert np.abs(out - oatt.decode(q, _np(sp))).max() <= 1e-5


def test_decode_special_cases(dev):
    rng = np.random.default_rng(7)
    B, H, G, D = 2, 12, 2, 128
    q = torch.from_numpy(rng.standard_normal((B, H, D)).astype(np.float32)).to(dev)
    # one key: output is its value row
    sp = _spans(rng, B, G, D, [1], torch.float32, dev)
    out = ops.attn_decode(q, sp)
    v = sp[0][1][:, :, 0]                        # [B, G, D]
    assert torch.allclose(out, v.repeat_interleave(6, dim=1), atol=1e-6, rtol=0)
    # identical keys: output is the mean of the values
    k = torch.randn(B, G, 1, D, device=dev).expand(B, G, 300, D).contiguous()
    vv = torch.randn(B, G, 300, D, device=dev)
    out = ops.attn_decode(q, [(k, vv)])
    assert torch.allclose(out, vv.mean(dim=2).repeat_interleave(6, dim=1), atol=2e-6, rtol=0)


def test_decode_strided_views(dev):
    """Spans taken as views of larger caches (batch and group strides != n*D)."""
    rng = np.random.default_rng(8)
    B, H, G, D, cap = 4, 12, 2, 128, 80
    kc = torch.from_numpy(rng.standard_normal((B, G, cap, D)).astype(np.float32)).to(dev)
    vc = torch.from_numpy(rng.standard_normal((B, G, cap, D)).astype(np.float32)).to(dev)
    sp = [(kc[:, :, :13], vc[:, :, :13]), (kc[:, :, 40:71], vc[:, :, 40:71])]
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    out = ops.attn_decode(torch.from_numpy(q).to(dev), sp).cpu().numpy()
    assert np.abs(out - oatt.decode(q, _np(sp))).max() <= 1e-5


def test_rmsnorm(dev):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((5, 1536)).astype(np.float32) * 3
    w = rng.uniform(0.8, 1.2, 1536).astype(np.float32)
    y = ops.rmsnorm(torch.from_numpy(x).to(dev), torch.from_numpy(w).to(dev), 1e-6).cpu().numpy()
    ref = linalg.rmsnorm(x, w, 1e-6)
    assert np.abs(y - ref).max() <= 2e-6 * np.abs(ref).max()


def _table(positions, D, theta=1e6):
    c, s = orope.table_c(positions, D, theta)
    return np.concatenate([c, s], axis=1).astype(np.float32)


@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16])
def test_rope_qkv_write_decode_and_prefill(dev, kv):
    rng = np.random.default_rng(10)
    H, G, D, W, S = 12, 2, 128, 16, 8
    # decode: 3 sequences at effective position 21, cache [B][G][W][D], slot c = 5
    B = 3
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    k = rng.standard_normal((B, G, D)).astype(np.float32)
    v = rng.standard_normal((B, G, D)).astype(np.float32)
    tab = torch.from_numpy(_table([21], D)).to(dev)
    kc = torch.zeros(B, G, W, D, dtype=kv, device=dev)
    kr = torch.zeros_like(kc)
    vc = torch.zeros_like(kc)
    sk = torch.zeros(B, G, S, D, dtype=kv, device=dev)
    sv = torch.zeros_like(sk)
    qt = torch.from_numpy(q).to(dev)
    c = 5
    ops.rope_qkv_write(qt, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev), tab, 0,
                       kc[:, :, c], kr[:, :, c], vc[:, :, c], kc.stride(0), kc.stride(1),
                       sk[:, :, c], sv[:, :, c], B, sk.stride(0), sk.stride(1))
    cs, sn = orope.table_c([21], D, 1e6)
    tol = 1e-6 if kv == torch.float32 else 8e-3
    assert np.abs(qt.cpu().numpy() - orope.rotate(q, cs, sn)).max() <= 1e-5
    assert np.abs(kc[:, :, c].float().cpu().numpy() - orope.rotate(k, cs, sn)).max() <= tol * 4
    assert np.abs(kr[:, :, c].float().cpu().numpy() - k).max() <= tol * 4
    assert np.abs(vc[:, :, c].float().cpu().numpy() - v).max() <= tol * 4
    assert np.abs(sk[:, :, c].float().cpu().numpy() - k).max() <= tol * 4
    assert float(kc[:, :, c + 1:].abs().max()) == 0.0
    # prefill: 10 tokens at positions 16..25 into slots 0..9 of one sequence, first 4 also sinks
    N = 10
    q = rng.standard_normal((N, H, D)).astype(np.float32)
    k = rng.standard_normal((N, G, D)).astype(np.float32)
    v = rng.standard_normal((N, G, D)).astype(np.float32)
    tab = torch.from_numpy(_table(np.arange(16, 26), D)).to(dev)
    kc = torch.zeros(G, W, D, dtype=kv, device=dev)
    kr, vc = torch.zeros_like(kc), torch.zeros_like(kc)
    sk = torch.zeros(G, S, D, dtype=kv, device=dev)
    sv = torch.zeros_like(sk)
    qt = torch.from_numpy(q).to(dev)
    ops.rope_qkv_write(qt, torch.from_numpy(k).to(dev), torch.from_numpy(v).to(dev), tab, D,
                       kc, kr, vc, D, kc.stride(0), sk, sv, 4, D, sk.stride(0))
    cs, sn = orope.table_c(np.arange(16, 26), D, 1e6)
    kt = np.transpose(k, (1, 0, 2))
    assert np.abs(qt.cpu().numpy() - np.transpose(orope.rotate(np.transpose(q, (1, 0, 2)), cs, sn), (1, 0, 2))).max() <= 1e-5
    assert np.abs(kc[:, :N].float().cpu().numpy() - orope.rotate(kt, cs, sn)).max() <= tol * 4
    assert np.abs(sk[:, :4].float().cpu().numpy() - kt[:, :4]).max() <= tol * 4
    assert float(sk[:, 4:].float().abs().max()) == 0.0


@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16])
def test_rope_rotate_rebase_and_prefix(dev, kv):
    rng = np.random.default_rng(11)
    L_, G, W, D = 3, 2, 32, 128
    x = torch.from_numpy(rng.standard_normal((L_, G, W, D)).astype(np.float32)).to(kv).to(dev)
    x0 = x.float().cpu().numpy()
    # re-base: every row by R_{-W}, in place, one table row (stride 0)
    tab = torch.from_numpy(_table([-W], D)).to(dev)
    v = x.view(L_ * G, W, D)
    ops.rope_rotate(v, v, tab, 0)
    cs, sn = orope.table_c([-W], D, 1e6)
    ref = orope.rotate(x0, cs, sn)
    tol = 2e-6 if kv == torch.float32 else 2e-2
    assert np.abs(x.float().cpu().numpy() - ref).max() <= tol
    # prefix: rows i at positions -7 + i into a separate buffer
    dst = torch.zeros_like(x)
    tab = torch.from_numpy(_table(np.arange(-7, -7 + W), D)).to(dev)
    ops.rope_rotate(x.view(L_ * G, W, D), dst.view(L_ * G, W, D), tab, D)
    cs, sn = orope.table_c(np.arange(-7, -7 + W), D, 1e6)
    ref = orope.rotate(x.float().cpu().numpy(), cs, sn)
    assert np.abs(dst.float().cpu().numpy() - ref).max() <= tol


def test_rope_relative_invariance(dev):
    """q.k after rotation depends only on the position difference (size-independent property)."""
    rng = np.random.default_rng(12)
    D = 128
    q = torch.from_numpy(rng.standard_normal((1, 1, 1, D)).astype(np.float32)).to(dev)
    k = torch.from_numpy(rng.standard_normal((1, 1, 1, D)).astype(np.float32)).to(dev)
    dots = []
    for p0 in (0, 1000, -1536):
        qa, ka = torch.empty_like(q), torch.empty_like(k)
        ops.rope_rotate(q.view(1, 1, D), qa.view(1, 1, D), torch.from_numpy(_table([p0 + 300], D)).to(dev), 0)
        ops.rope_rotate(k.view(1, 1, D), ka.view(1, 1, D), torch.from_numpy(_table([p0], D)).to(dev), 0)
        dots.append(float((qa * ka).sum()))
    assert max(dots) - min(dots) <= 1e-4 * max(1.0, abs(dots[0]))


@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16])
def test_gather_rows(dev, kv):
    src = torch.randn(4, 50, 128, device=dev).to(kv)
    dst = torch.full((4, 6, 128), 7.0, device=dev).to(kv)
    idx = torch.tensor([3, 0, 49, 3, 60, -1], dtype=torch.int32)
    ops.gather_rows(src, dst, idx)
    want = torch.zeros_like(dst)
    want[:, :4] = src[:, [3, 0, 49, 3]]
    assert torch.equal(dst, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_shared_workspace_across_batch_sizes(dev, dtype):
    """One workspace shared by calls of different (batch, group) counts: batch 1 at 3584 keys (more
    splits than one workgroup merges: a merge launch over partials) then batch 64 (ticket merge), then
    batch 1 again; each result equals the same call on a fresh workspace.  With the tickets placed
    right after a (B, G)-sized prefix, batch 1's partials landed where batch 64 reads its tickets."""
    rng = np.random.default_rng(11)
    H, G, D = 12, 2, 128
    lens = [512, 1024, 1024, 1024]
    lib = ops.L.load()
    shared = ops.Workspace(dev)
    shared.get(max(int(lib.vgx_attn_decode_workspace_bytes(B, H, G, D, sum(lens))) for B in (1, 16, 64)))
    buf = shared.buf
    for B in (1, 64, 1, 16, 64):
        sp = _spans(rng, B, G, D, lens, dtype, dev)
        q = torch.from_numpy(rng.standard_normal((B, H, D)).astype(np.float32)).to(dev)
        a = ops.attn_decode(q, sp, ws=shared)
        b = ops.attn_decode(q, sp, ws=ops.Workspace(dev))
        torch.cuda.synchronize()
        assert torch.equal(a, b), B
        assert shared.buf is buf, "the shared workspace was reallocated"
        assert int(shared.buf[:16384].view(torch.int32).abs().sum()) == 0, "tickets left non-zero"
