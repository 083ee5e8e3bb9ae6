"""GPU parity of the bf16 MFMA prefill attention (vgx_attn_prefill) and of the drop-in
block_sliding_attention (src/vault_v3_model.py:812-863) against the float64 oracle.

The oracle is fed the same bf16 k / v (and the same q: fp32 queries are used at fp32 accuracy, bf16
ones as given); the bar is the bf16 attention bound max |d| <= 2e-3, and 1e-5 for fp32 K / V (the
fp32 bar).  Re-rotated sinks of a bf16 call are rotated in fp32 and stored once in bf16, which the
oracle models (``sink_store``) so that the comparison measures the attention alone.  Shapes: ragged query counts
(not multiples of the 32-query tile), all four key runs (sinks | segment | prev | causal cur), every supported group size, more than
eight query blocks (split launches), and the full block-sliding prefill workload (L = 8192, W = 1024,
512 sinks) checked on sampled query rows.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import rope as orope
from oracle.model import bf16_round
from vault_amd import attention as vatt
from vault_amd import ops

pytestmark = pytest.mark.gpu
TOL = 2e-3
TOL32 = 1e-5


def _bf(x):
    return torch.as_tensor(x).to(torch.bfloat16)


def _f64(t):
    return t.double().cpu().numpy()


@pytest.mark.parametrize("qdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,lens", [(300, (40, 77, 200)), (33, (0, 0, 64)), (1, (5, 0, 0)), (1024, (512, 1024, 1024))])
def test_prefill_chunk_matches_oracle(dev, qdt, T, lens):
    rng = np.random.default_rng(T + sum(lens))
    H, G, D = 12, 2, 128
    runs = [(_bf(rng.standard_normal((G, n, D))).to(dev), _bf(rng.standard_normal((G, n, D))).to(dev))
            for n in lens if n > 0]
    kc = _bf(rng.standard_normal((G, T, D))).to(dev)
    vc = _bf(rng.standard_normal((G, T, D))).to(dev)
    q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev).to(qdt)
    out = torch.empty(T, H, D, device=dev)
    ops.attn_prefill([{"q": q, "out": out, "runs": runs + [(kc, vc)], "causal_base": 0}], H, G)
    qr = _f64(q)   # fp32 queries are used unrounded (fp16 hi + lo), bf16 ones as they are
    ref = oatt.chunk(qr, [(_f64(k), _f64(v)) for k, v in runs], _f64(kc), _f64(vc))
    assert np.abs(out.double().cpu().numpy() - ref).max() <= TOL


@pytest.mark.parametrize("H,G", [(4, 4), (4, 2), (8, 2), (16, 2)])
def test_prefill_group_sizes(dev, H, G):
    rng = np.random.default_rng(H * 10 + G)
    D, T, P = 128, 70, 90
    pk, pv = (_bf(rng.standard_normal((G, P, D))).to(dev) for _ in range(2))
    ck, cv = (_bf(rng.standard_normal((G, T, D))).to(dev) for _ in range(2))
    q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev)
    out = torch.empty(T, H, D, device=dev)
    ops.attn_prefill([{"q": q, "out": out, "runs": [(pk, pv), (ck, cv)], "causal_base": 0}], H, G)
    ref = oatt.chunk(_f64(q), [(_f64(pk), _f64(pv))], _f64(ck), _f64(cv))
    assert np.abs(out.double().cpu().numpy() - ref).max() <= TOL


def test_prefill_equals_valu_decode_kernel(dev):
    """Same chunk through the fp32 VALU split-K kernel (one query per entry, causal last span) and the
    MFMA kernel: equal within the bf16 bound (q is rounded to bf16 for both)."""
    rng = np.random.default_rng(9)
    H, G, D, T, P = 12, 2, 128, 200, 300
    pk, pv = (_bf(rng.standard_normal((1, G, P, D))).to(dev) for _ in range(2))
    ck, cv = (_bf(rng.standard_normal((1, G, T, D))).to(dev) for _ in range(2))
    q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev).to(torch.bfloat16).float()
    a = ops.attn_decode(q, [(pk, pv), (ck, cv)], causal_base=0)
    b = torch.empty(T, H, D, device=dev)
    ops.attn_prefill([{"q": q, "out": b, "runs": [(pk[0], pv[0]), (ck[0], cv[0])], "causal_base": 0}], H, G)
    assert (a - b).abs().max().item() <= TOL


@pytest.mark.parametrize("B,L,W,S", [(2, 1100, 256, 64), (1, 700, 256, 0), (1, 40, 16, 5)])
def test_block_sliding_matches_oracle(dev, B, L, W, S):
    rng = np.random.default_rng(L + W + S)
    H, G, D, theta = 12, 2, 128, 1e6
    q = _bf(rng.standard_normal((B, H, L, D))).float().to(dev)
    k = _bf(rng.standard_normal((B, G, L, D))).to(dev)
    v = _bf(rng.standard_normal((B, G, L, D))).to(dev)
    kr = _bf(rng.standard_normal((B, G, L, D))).to(dev)
    out = vatt.block_sliding_attention(q, k, v, W, k_raw=kr, n_sink=S, head_dim=D, rope_theta=theta)
    for b in range(B):
        ref = oatt.block_sliding(_f64(q[b]).transpose(1, 0, 2), _f64(k[b]).transpose(1, 0, 2),
                                 _f64(v[b]).transpose(1, 0, 2), _f64(kr[b]).transpose(1, 0, 2), W, S, theta,
                                 sink_store=bf16_round)
        got = out[b].double().cpu().numpy().transpose(1, 0, 2)
        assert np.abs(got - ref).max() <= TOL, b


@pytest.mark.parametrize("B,L,W,S", [(2, 1100, 256, 64), (1, 700, 256, 0), (1, 40, 16, 5)])
def test_block_sliding_fp32_inputs(dev, B, L, W, S):
    """fp32 q / k / v / k_raw that are not representable in bf16: the drop-in keeps them fp32 (three
    bf16 pieces per operand in the kernel, sinks rotated and stored in fp32) and meets the fp32 bar."""
    rng = np.random.default_rng(L + W + S + 1)
    H, G, D, theta = 12, 2, 128, 1e6
    f32 = lambda shape: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev)
    q, k, v, kr = f32((B, H, L, D)), f32((B, G, L, D)), f32((B, G, L, D)), f32((B, G, L, D))
    assert not torch.equal(k, k.to(torch.bfloat16).float())
    out = vatt.block_sliding_attention(q, k, v, W, k_raw=kr, n_sink=S, head_dim=D, rope_theta=theta)
    assert out.dtype == torch.float32
    for b in range(B):
        ref = oatt.block_sliding(_f64(q[b]).transpose(1, 0, 2), _f64(k[b]).transpose(1, 0, 2),
                                 _f64(v[b]).transpose(1, 0, 2), _f64(kr[b]).transpose(1, 0, 2), W, S, theta)
        got = out[b].double().cpu().numpy().transpose(1, 0, 2)
        assert np.abs(got - ref).max() <= TOL32, b


@pytest.mark.parametrize("B,L,W,S", [(2, 1100, 256, 64), (1, 40, 16, 5)])
def test_block_sliding_bf16_output_is_rounded_fp32(dev, B, L, W, S):
    """bf16 callers get the kernel's bf16 output: bit-exactly the fp32 result of the same call rounded
    to nearest even (no separate conversion pass)."""
    rng = np.random.default_rng(L + S + 7)
    H, G, D, theta = 12, 2, 128, 1e6
    q = _bf(rng.standard_normal((B, H, L, D))).to(dev)
    k = _bf(rng.standard_normal((B, G, L, D))).to(dev)
    v = _bf(rng.standard_normal((B, G, L, D))).to(dev)
    kr = _bf(rng.standard_normal((B, G, L, D))).to(dev)
    got = vatt.block_sliding_attention(q, k, v, W, k_raw=kr, n_sink=S, head_dim=D, rope_theta=theta)
    assert got.dtype == torch.bfloat16
    ref = vatt.block_sliding_attention(q.float(), k, v, W, k_raw=kr, n_sink=S, head_dim=D, rope_theta=theta)
    assert torch.equal(got, ref.to(torch.bfloat16))


def test_block_sliding_full_workload_sampled(dev):
    """L = 8192, W = 1024, 512 sinks, 12 q / 2 kv heads, D = 128: 48 sampled query rows (every chunk,
    first / last / random positions) against the oracle's per-query attention over exactly the keys the
    reference makes visible."""
    rng = np.random.default_rng(2024)
    B, H, G, D, L, W, S, theta = 1, 12, 2, 128, 8192, 1024, 512, 1e6
    q = _bf(rng.standard_normal((B, H, L, D), dtype=np.float32)).float().to(dev)
    k = _bf(rng.standard_normal((B, G, L, D), dtype=np.float32)).to(dev)
    v = _bf(rng.standard_normal((B, G, L, D), dtype=np.float32)).to(dev)
    kr = _bf(rng.standard_normal((B, G, L, D), dtype=np.float32)).to(dev)
    out = vatt.block_sliding_attention(q, k, v, W, k_raw=kr, n_sink=S, head_dim=D, rope_theta=theta)
    qn, kn, vn, krn, on = (_f64(t[0]) for t in (q, k, v, kr, out))
    rows = sorted(set([0, 1, W - 1, W, 2 * W, 2 * W + 1, L - 1] + rng.integers(0, L, 41).tolist()))
    for t in rows:
        i = t // W
        parts_k, parts_v = [], []
        if i >= 2:
            c, s_ = orope.table_torch((i - 1) * W - S + np.arange(S), D, theta)
            parts_k.append(bf16_round(orope.rotate(krn[:, :S], c, s_)))     # stored once in bf16
            parts_v.append(vn[:, :S])
        lo = max(0, (i - 1) * W)
        parts_k.append(kn[:, lo:t + 1])
        parts_v.append(vn[:, lo:t + 1])
        spans = [(pk[None], pv[None]) for pk, pv in zip(parts_k, parts_v)]
        ref = oatt.decode(qn[:, t][None], spans)[0]
        assert np.abs(on[:, t] - ref).max() <= TOL, t


@pytest.mark.parametrize("T,lens", [(300, (40, 77, 200)), (33, (0, 0, 64)), (1, (5, 0, 0)), (1024, (512, 1024, 1024))])
def test_prefill_fp32_kv_matches_oracle(dev, T, lens):
    """fp32 K / V (the fp32-state chunk prefill) on MFMA as three bf16 planes, fp32 queries and the
    probabilities as three bf16 pieces: 24 significant bits per operand, the six products of order
    <= 2 accumulated in fp32.  The fp32 bar, 1e-5."""
    rng = np.random.default_rng(T + sum(lens) + 7)
    H, G, D = 12, 2, 128
    f32 = lambda shape: torch.from_numpy(rng.standard_normal(shape).astype(np.float32)).to(dev)
    runs = [(f32((G, n, D)), f32((G, n, D))) for n in lens if n > 0]
    kc, vc = f32((G, T, D)), f32((G, T, D))
    q = f32((T, H, D))
    out = torch.empty(T, H, D, device=dev)
    ops.attn_prefill([{"q": q, "out": out, "runs": runs + [(kc, vc)], "causal_base": 0}], H, G)
    ref = oatt.chunk(_f64(q), [(_f64(k), _f64(v)) for k, v in runs], _f64(kc), _f64(vc))
    assert np.abs(out.double().cpu().numpy() - ref).max() <= TOL32


def test_prefill_fp32_kv_strided_state_views(dev):
    """fp32 runs as views of a [W]-row ring (row stride D, group stride W*D) with a causal last run."""
    rng = np.random.default_rng(77)
    H, G, D, W, T = 12, 2, 128, 256, 100
    ring_k = torch.from_numpy(rng.standard_normal((G, W, D)).astype(np.float32)).to(dev)
    ring_v = torch.from_numpy(rng.standard_normal((G, W, D)).astype(np.float32)).to(dev)
    prev_k = torch.from_numpy(rng.standard_normal((G, W, D)).astype(np.float32)).to(dev)
    prev_v = torch.from_numpy(rng.standard_normal((G, W, D)).astype(np.float32)).to(dev)
    q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev)
    out = torch.empty(T, H, D, device=dev)
    ops.attn_prefill([{"q": q, "out": out, "runs": [(prev_k, prev_v), (ring_k[:, :T], ring_v[:, :T])],
                       "causal_base": 0}], H, G)
    ref = oatt.chunk(_f64(q), [(_f64(prev_k), _f64(prev_v))], _f64(ring_k[:, :T]), _f64(ring_v[:, :T]))
    assert np.abs(out.double().cpu().numpy() - ref).max() <= TOL32


@pytest.mark.parametrize("kvdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,lens", [(300, (40, 77, 200)), (1024, (512, 1024, 1024)), (45, (0, 33, 64))])
def test_prefill_per_row_bias_on_segment_run(dev, kvdt, T, lens):
    """The chunk-level resonance bias: query t of head h adds bias[t, row(h), j] to its scores with the
    segment run's keys (rows: none / arch / sup by head class, 12 query / 2 KV heads), against the
    float64 oracle with the dense [T, H, n] bias; zero rows (positions where the mode is 0) and a bias
    run shorter than the bias rows are included."""
    rng = np.random.default_rng(T * 7 + sum(lens))
    H, G, D = 12, 2, 128
    cast = (lambda a: _bf(a)) if kvdt == torch.bfloat16 else (lambda a: torch.as_tensor(a, dtype=torch.float32))
    runs = [(cast(rng.standard_normal((G, n, D))).to(dev), cast(rng.standard_normal((G, n, D))).to(dev))
            for n in lens if n > 0]
    seg = 1 if lens[0] > 0 else 0                     # the segment run's index among the runs
    n_seg = lens[1]
    kc = cast(rng.standard_normal((G, T, D))).to(dev)
    vc = cast(rng.standard_normal((G, T, D))).to(dev)
    q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev)
    rows = [-1, -1, 0, 0, 1, 1] * 2
    bias = (rng.standard_normal((T, 2, n_seg + 7)) * 3).astype(np.float32)
    bias[rng.random(T) < 0.3] = 0.0
    out = torch.empty(T, H, D, device=dev)
    ops.attn_prefill([{"q": q, "out": out, "runs": runs + [(kc, vc)], "causal_base": 0,
                       "bias": torch.from_numpy(bias).to(dev), "bias_head_row": rows, "bias_run": seg}], H, G)
    dense = np.zeros((T, H, n_seg))
    for h, r in enumerate(rows):
        if r >= 0:
            dense[:, h] = bias[:, r, :n_seg]
    ref = oatt.chunk(_f64(q), [(_f64(k), _f64(v)) for k, v in runs], _f64(kc), _f64(vc), bias=dense, bias_span=seg)
    err = np.abs(out.double().cpu().numpy() - ref).max()
    assert err <= (TOL if kvdt == torch.bfloat16 else TOL32), err
    # the same bias on the wrong run is far outside the bar
    wrong = oatt.chunk(_f64(q), [(_f64(k), _f64(v)) for k, v in runs], _f64(kc), _f64(vc))
    assert np.abs(wrong - ref).max() > 100 * TOL


@pytest.mark.parametrize("kvdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("qdt", [torch.float32, torch.bfloat16])
def test_prefill_launch_shapes_agree(dev, kvdt, qdt):
    """A launch of many query tiles runs two waves of 16 queries per head and workgroup, a launch of
    few tiles one (the narrow shape, twice the workgroups); every query's arithmetic is the same in
    both.  Eight blocks in one launch (262 32-query tiles: the two-wave shape) against the same blocks
    launched one by one (narrow): equal bit for bit, biased blocks included, and two of the blocks
    against the float64 oracle."""
    rng = np.random.default_rng(31 if kvdt == torch.bfloat16 else 32)
    H, G, D = 12, 2, 128
    cast = (lambda a: _bf(a)) if kvdt == torch.bfloat16 else (lambda a: torch.as_tensor(a, dtype=torch.float32))
    sizes = [520, 611, 333, 700, 47, 600, 590, 655]
    blocks, refs = [], []
    for i, T in enumerate(sizes):
        lens = [int(rng.integers(1, 300)), int(rng.integers(1, 400))]
        runs = [(cast(rng.standard_normal((G, n, D))).to(dev), cast(rng.standard_normal((G, n, D))).to(dev))
                for n in lens]
        kc = cast(rng.standard_normal((G, T, D))).to(dev)
        vc = cast(rng.standard_normal((G, T, D))).to(dev)
        q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev).to(qdt)
        blk = {"q": q, "runs": runs + [(kc, vc)], "causal_base": 0}
        dense = None
        if i % 3 == 1:                                  # a resonance bias on the second run
            rows = [-1, 0, 1, 0, 1, -1] * 2
            bias = (rng.standard_normal((T, 2, lens[1])) * 3).astype(np.float32)
            blk.update(bias=torch.from_numpy(bias).to(dev), bias_head_row=rows, bias_run=1)
            dense = np.zeros((T, H, lens[1]))
            for h, r in enumerate(rows):
                if r >= 0:
                    dense[:, h] = bias[:, r]
        blocks.append(blk)
        refs.append(dense)
    wide = [dict(b, out=torch.empty(b["q"].shape[0], H, D, device=dev)) for b in blocks]
    ops.attn_prefill(wide, H, G)
    for b, w in zip(blocks, wide):
        narrow = dict(b, out=torch.empty_like(w["out"]))
        ops.attn_prefill([narrow], H, G)
        assert torch.equal(narrow["out"], w["out"])
    bar = TOL if kvdt == torch.bfloat16 else TOL32
    for i in (1, 4):
        b = blocks[i]
        (pk, pv), (sk, sv), (kc, vc) = b["runs"]
        ref = oatt.chunk(_f64(b["q"]), [(_f64(pk), _f64(pv)), (_f64(sk), _f64(sv))], _f64(kc), _f64(vc),
                         bias=refs[i], bias_span=1 if refs[i] is not None else -1)
        assert np.abs(wide[i]["out"].double().cpu().numpy() - ref).max() <= bar


@pytest.mark.parametrize("kvdt", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("T,lens", [(1024, (512, 1024, 1024)), (300, (40, 77, 200)), (33, (0, 0, 64)), (1, (5, 0, 0))])
def test_prefill_key_splits_match_oracle(dev, kvdt, T, lens):
    """With a workspace, a launch of few query tiles splits each tile's keys into 2-4 ranges and merges
    them (vgx_attn_prefill_ws): the float64 oracle's bar, fp32 and bf16 queries, a resonance bias on the
    segment run, and agreement with the unsplit call within the same bar; a workspace below
    vgx_attn_prefill_workspace_bytes is refused."""
    rng = np.random.default_rng(T * 3 + sum(lens) + (kvdt == torch.float32))
    H, G, D = 12, 2, 128
    cast = (lambda a: _bf(a)) if kvdt == torch.bfloat16 else (lambda a: torch.as_tensor(a, dtype=torch.float32))
    runs = [(cast(rng.standard_normal((G, n, D))).to(dev), cast(rng.standard_normal((G, n, D))).to(dev))
            for n in lens if n > 0]
    kc = cast(rng.standard_normal((G, T, D))).to(dev)
    vc = cast(rng.standard_normal((G, T, D))).to(dev)
    bar = TOL if kvdt == torch.bfloat16 else TOL32
    ws = ops.Workspace(dev)
    for qdt in (torch.float32, torch.bfloat16):
        q = torch.from_numpy(rng.standard_normal((T, H, D)).astype(np.float32)).to(dev).to(qdt)
        blk = {"q": q, "runs": runs + [(kc, vc)], "causal_base": 0}
        dense, seg = None, 0
        if len(runs) >= 2:
            seg, n_seg = 1, runs[1][0].shape[1]
            rows = [-1, 0, 1, 0, 1, -1] * 2
            bias = (rng.standard_normal((T, 2, n_seg)) * 3).astype(np.float32)
            blk.update(bias=torch.from_numpy(bias).to(dev), bias_head_row=rows, bias_run=1)
            dense = np.zeros((T, H, n_seg))
            for h, r in enumerate(rows):
                if r >= 0:
                    dense[:, h] = bias[:, r]
        split = dict(blk, out=torch.empty(T, H, D, device=dev))
        whole = dict(blk, out=torch.empty(T, H, D, device=dev))
        ops.attn_prefill([split], H, G, ws=ws)
        ops.attn_prefill([whole], H, G)
        ref = oatt.chunk(_f64(q), [(_f64(k), _f64(v)) for k, v in runs], _f64(kc), _f64(vc), bias=dense,
                         bias_span=seg if dense is not None else -1)
        got = split["out"].double().cpu().numpy()
        assert np.abs(got - ref).max() <= bar
        assert np.abs(got - whole["out"].double().cpu().numpy()).max() <= bar
    from vault_amd import _lib as L
    lib = L.load()
    need = int(lib.vgx_attn_prefill_workspace_bytes(H, G))
    assert need > 0
    arr = (L.AttnBlock * 1)()
    ra = (L.KVRun * 4)()
    ra[0] = L.KVRun(kc.data_ptr(), vc.data_ptr(), T, kc.stride(1), kc.stride(0))
    out = torch.empty(T, H, D, device=dev)
    q = torch.zeros(T, H, D, device=dev)
    arr[0] = L.AttnBlock(q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), out.stride(1), T, 0, 1, ra)
    small = torch.empty(need - 256, dtype=torch.uint8, device=dev)
    kd = L.BF16 if kvdt == torch.bfloat16 else L.F32
    assert lib.vgx_attn_prefill_ws(kd, L.F32, L.F32, arr, 1, H, G, D, 0.088, small.data_ptr(), small.numel(), None) == -8
