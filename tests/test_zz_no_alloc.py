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


def _graph_case(dev, gen):
    H, G, D, B = 12, 2, 128, 1
    spans = _spans(B, G, D, [512, 1024, 1024, 1024], torch.float32, dev, gen)
    q = torch.randn(B, H, D, generator=gen).to(dev)
    return q, spans


def test_noalloc_inside_graph_capture_replays_exactly(dev):
    """A captured noalloc call (after the device's set-up call outside capture) replayed three times,
    with eager work on the same data between the replays, equals vgx_attn_decode each time."""
    lib = L.load()
    gen = torch.Generator().manual_seed(11)
    q, spans = _graph_case(dev, gen)
    B, H, D = q.shape
    need = int(lib.vgx_attn_decode_workspace_bytes(B, H, 2, D, 3584))
    ws = torch.zeros(need, dtype=torch.uint8, device=dev)
    ref_out = torch.empty_like(q)
    out = torch.full_like(q, float("nan"))
    assert _call(lib, "vgx_attn_decode_noalloc", L.F32, q, spans, out, None, -1, None) == 0   # set-up, eager
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            rc = _call(lib, "vgx_attn_decode_noalloc", L.F32, q, spans, out, None, -1, None)
    assert rc == 0
    for i in range(3):
        q.copy_(torch.randn(q.shape, generator=gen).to(dev))
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert _call(lib, "vgx_attn_decode", L.F32, q, spans, ref_out, None, -1, ws) == 0
        torch.cuda.synchronize()
        assert torch.isfinite(out).all() and torch.equal(out, ref_out), i


_FRESH = r"""
import json, sys, torch
sys.path.insert(0, sys.argv[1])
from tests.test_zz_no_alloc import _call, _graph_case
from vault_amd import _lib as L
lib = L.load()
dev = torch.device("cuda:0")
q, spans = _graph_case(dev, torch.Generator().manual_seed(12))
out = torch.zeros_like(q)
g = torch.cuda.CUDAGraph()
s = torch.cuda.Stream()
with torch.cuda.stream(s):
    with torch.cuda.graph(g, stream=s):
        rc_capture = _call(lib, "vgx_attn_decode_noalloc", L.F32, q, spans, out, None, -1, None)
torch.cuda.synchronize()
rc_eager = _call(lib, "vgx_attn_decode_noalloc", L.F32, q, spans, out, None, -1, None)
torch.cuda.synchronize()
print(json.dumps({"capture": rc_capture, "eager": rc_eager, "finite": bool(torch.isfinite(out).all())}))
"""


def test_noalloc_first_call_inside_capture_is_refused():
    """In a fresh process the device's first noalloc call made inside a stream capture returns
    VGX_E_STATE (its set-up would launch a fill kernel that the capture records instead of running);
    the next call, outside capture, sets the device up and computes."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    print("fresh-process noalloc capture case", flush=True)
    r = subprocess.run([sys.executable, "-c", _FRESH, root], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res == {"capture": -33, "eager": 0, "finite": True}
