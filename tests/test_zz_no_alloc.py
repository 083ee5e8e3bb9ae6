"""The allocation-free decode attention entry point (vgx_attn_decode_noalloc) through the C ABI:
bit-identical to vgx_attn_decode with a caller workspace (same kernels) on consecutive calls of
decreasing size — batch 64 bf16 (MFMA path, ticket merge), batch 16 fp32 with a segment bias, batch 1
fp32 at 3584 keys (64 splits, merge launch over the partials) — and the size limit of its fixed
scratch rejected with VGX_E_LIMIT."""
import ctypes as C

import numpy as np
import pytest
import torch

from vault_amd import _lib as L
from vault_amd import ops

pytestmark = pytest.mark.gpu


def _spans(B, G, D, lens, dtype, dev, gen):
    out = []
    for n in lens:
        k = torch.randn(B, G, n, D, generator=gen).to(dtype).to(dev)
        v = torch.randn(B, G, n, D, generator=gen).to(dtype).to(dev)
        out.append((k, v))
    return out


def _call(lib, fn, kv_dt, q, spans, out, bias, bias_span, ws):
    B, H, D = q.shape
    G = spans[0][0].shape[1]
    arr = (L.KVSpan * 4)()
    for i, (k, v) in enumerate(spans):
        arr[i] = L.KVSpan(k.data_ptr(), v.data_ptr(), k.shape[2], k.stride(0), k.stride(1), None)
    args = [kv_dt, q.data_ptr(), q.stride(0), arr, len(spans), bias.data_ptr() if bias is not None else None,
            bias.stride(0) if bias is not None else 0, bias_span, -1, out.data_ptr(), B, H, G, D, float(D ** -0.5)]
    stream = torch.cuda.current_stream().cuda_stream
    if fn == "vgx_attn_decode":
        return getattr(lib, fn)(*args, ws.data_ptr(), ws.numel(), stream)
    return getattr(lib, fn)(*args, stream)


@pytest.mark.parametrize("order", ["noalloc_first", "workspace_first"])
def test_noalloc_matches_workspace_entry(dev, order):
    lib = L.load()
    gen = torch.Generator().manual_seed(3)
    H, G, D = 12, 2, 128
    cases = [(64, [512, 1024, 1024, 1024], torch.bfloat16, False),
             (16, [512, 1024, 1024, 1024], torch.float32, True),
             (1, [512, 1024, 1024, 1024], torch.float32, False),
             (1, [64, 0, 1024, 1024], torch.float32, False)]
    for B, lens, dt, with_bias in cases:
        spans = [s for s in _spans(B, G, D, lens, dt, dev, gen) if s[0].shape[2] > 0]
        q = torch.randn(B, H, D, generator=gen).to(dev)
        bias = (torch.randn(H, 1024, generator=gen) * 2).to(dev) if with_bias else None
        kv_dt = ops.KV_DTYPES[dt]
        need = int(lib.vgx_attn_decode_workspace_bytes(B, H, G, D, sum(lens)))
        ws = torch.zeros(max(need, 256), dtype=torch.uint8, device=dev)
        a = torch.full((B, H, D), float("nan"), device=dev)
        b = torch.full((B, H, D), float("nan"), device=dev)
        calls = [("vgx_attn_decode_noalloc", a), ("vgx_attn_decode", b)]
        if order == "workspace_first":
            calls.reverse()
        for fn, out in calls:
            assert _call(lib, fn, kv_dt, q, spans, out, bias, 1 if with_bias else -1, ws) == 0, fn
        torch.cuda.synchronize()
        assert torch.isfinite(a).all() and torch.equal(a, b), (B, lens, dt)


def test_noalloc_rejects_beyond_its_scratch(dev):
    lib = L.load()
    B, H, G, D, n = 8, 256, 32, 128, 3584
    assert lib.vgx_attn_decode_workspace_bytes(B, H, G, D, n) > (2 << 20)
    k = torch.zeros(B, G, n, D, dtype=torch.bfloat16, device=dev)
    q = torch.zeros(B, H, D, device=dev)
    out = torch.zeros(B, H, D, device=dev)
    rc = _call(lib, "vgx_attn_decode_noalloc", L.BF16, q, [(k, k)], out, None, -1, None)
    assert rc == -10   # VGX_E_LIMIT
