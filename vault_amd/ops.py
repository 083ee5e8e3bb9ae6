"""Torch-facing wrappers of libvault_amd entry points.

Torch provides device memory and the current HIP stream; every computation below is a call
into the HIP library (no torch fallback).  Tensors must live on a ROCm device.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Tuple

import numpy as np
import torch

from . import _lib as L

F32, F16, BF16, Q8_0, Q4_0 = L.F32, L.F16, L.BF16, L.Q8_0, L.Q4_0
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}
ELEM_BYTES = {F32: 4, F16: 2, BF16: 2}       # plain (unquantized) weight dtypes


def payload_bytes(dtype: int, rows: int, cols: int) -> int:
    """Bytes of a [rows x cols] tensor in its VLT3 layout (AoS blocks or row-major elements)."""
    if dtype in ELEM_BYTES:
        return rows * cols * ELEM_BYTES[dtype]
    return rows * (cols // 32) * BLOCK_BYTES[dtype]


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _need(t: torch.Tensor, dtype: torch.dtype, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")


class QWeight:
    """A [rows x cols] projection weight in the packed device layout (include/vault_amd.h).

    ``gateup`` tensors hold a gate and an up projection interleaved by row-quads; ``rows`` is then
    the number of output rows of the fused SwiGLU.
    """

    def __init__(self, dtype: int, rows: int, cols: int, packed: torch.Tensor, gateup: bool = False):
        self.dtype, self.rows, self.cols, self.packed, self.gateup = dtype, rows, cols, packed, gateup

    @property
    def device(self) -> torch.device:
        return self.packed.device

    @staticmethod
    def _upload(data, device) -> torch.Tensor:
        if isinstance(data, torch.Tensor):
            t = data.view(torch.uint8) if data.dtype != torch.uint8 else data
            return t.reshape(-1).to(device)
        arr = np.frombuffer(data, dtype=np.uint8) if isinstance(data, (bytes, bytearray, memoryview)) else \
            np.ascontiguousarray(data).view(np.uint8).reshape(-1)
        return torch.from_numpy(arr.copy()).to(device)

    @classmethod
    def from_blocks(cls, dtype: int, rows: int, cols: int, data, device) -> "QWeight":
        """``data``: VLT3 payload (AoS Q8_0/Q4_0 blocks, or row-major elements for F32 / BF16 / F16)."""
        lib = L.load()
        src = cls._upload(data, device)
        n = lib.vgx_qweight_packed_bytes(dtype, rows, cols)
        L.check(0 if n > 0 else int(n), "vgx_qweight_packed_bytes")
        dst = torch.empty(int(n), dtype=torch.uint8, device=device)
        L.check(lib.vgx_qweight_pack(dtype, src.data_ptr(), dst.data_ptr(), rows, cols, _stream(dst.device)),
                "vgx_qweight_pack")
        return cls(dtype, rows, cols, dst)

    @classmethod
    def gateup_from_blocks(cls, dtype: int, rows: int, cols: int, gate, up, device) -> "QWeight":
        lib = L.load()
        g = cls._upload(gate, device)
        u = cls._upload(up, device)
        n = lib.vgx_qweight_packed_bytes(dtype, 2 * rows, cols)
        L.check(0 if n > 0 else int(n), "vgx_qweight_packed_bytes")
        dst = torch.empty(int(n), dtype=torch.uint8, device=device)
        L.check(lib.vgx_qweight_pack_gateup(dtype, g.data_ptr(), u.data_ptr(), dst.data_ptr(), rows, cols,
                                            _stream(dst.device)), "vgx_qweight_pack_gateup")
        return cls(dtype, rows, cols, dst, gateup=True)

    @classmethod
    def rope_from_blocks(cls, dtype: int, rows: int, cols: int, data, head_dim: int, n_rope_rows: int,
                         device) -> "QWeight":
        """Packed with the RoPE-pair row order of vgx_qweight_pack_rope (for qkv_rope_step)."""
        lib = L.load()
        src = cls._upload(data, device)
        n = lib.vgx_qweight_packed_bytes(dtype, rows, cols)
        L.check(0 if n > 0 else int(n), "vgx_qweight_packed_bytes")
        dst = torch.empty(int(n), dtype=torch.uint8, device=device)
        L.check(lib.vgx_qweight_pack_rope(dtype, src.data_ptr(), dst.data_ptr(), rows, cols, head_dim, n_rope_rows,
                                          _stream(dst.device)), "vgx_qweight_pack_rope")
        return cls(dtype, rows, cols, dst)

    def unpack(self) -> torch.Tensor:
        """Packed -> AoS blocks (uint8 device tensor)."""
        if self.gateup:
            raise ValueError("unpack of a gate/up tensor is not supported")
        nbytes = payload_bytes(self.dtype, self.rows, self.cols)
        out = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        L.check(L.load().vgx_qweight_unpack(self.dtype, self.packed.data_ptr(), out.data_ptr(), self.rows, self.cols,
                                            _stream(self.device)), "vgx_qweight_unpack")
        return out

    def dequant(self) -> torch.Tensor:
        rows = 2 * self.rows if self.gateup else self.rows
        out = torch.empty(rows, self.cols, dtype=torch.float32, device=self.device)
        L.check(L.load().vgx_qweight_dequant(self.dtype, self.packed.data_ptr(), out.data_ptr(), rows, self.cols,
                                             _stream(self.device)), "vgx_qweight_dequant")
        return out

    @property
    def stream_bytes(self) -> int:
        """Bytes of weights one full pass reads (the algorithmic bytes of one GEMV)."""
        rows = 2 * self.rows if self.gateup else self.rows
        return payload_bytes(self.dtype, rows, self.cols)


def count_nonfinite(items, device) -> list:
    """Non-finite values per tensor, counted on the device: ``items`` is a list of (dtype, payload
    bytes, element count) in the VLT3 layouts; one host read for the whole list."""
    lib = L.load()
    counts = torch.zeros(max(1, len(items)), dtype=torch.int32, device=device)
    for i, (dt, data, n) in enumerate(items):
        # stream-ordered: the upload's memory is reused only after the scan that reads it
        src = QWeight._upload(data, device)
        L.check(lib.vgx_count_nonfinite(dt, src.data_ptr(), n, counts[i:].data_ptr(), _stream(torch.device(device))),
                "vgx_count_nonfinite")
    return counts[:len(items)].cpu().tolist()


GEMM_MIN_ROWS = 8   # activation rows from which Q8_0 / Q4_0 projections run on the MFMA GEMM
_GEMM_WS: dict = {}


def gemm_workspace(device) -> "Workspace":
    """Per-device workspace of the MFMA GEMM's activation splits and K-split partials (grow-only; a
    captured graph holds its address, so callers that capture size it first).  Its first 64 KiB are the
    GEMM's output-tile counters, zero-filled here and left at zero by every call."""
    key = str(torch.device(device))
    if key not in _GEMM_WS:
        _GEMM_WS[key] = Workspace(torch.device(device))
    return _GEMM_WS[key]


def _gemv(w: QWeight, x: torch.Tensor, out: Optional[torch.Tensor], epi: int, bias: Optional[torch.Tensor],
          norm: Optional[Tuple[torch.Tensor, float]]) -> torch.Tensor:
    _need(x, torch.float32, "x")
    x2 = x.reshape(-1, w.cols) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    if out is None:
        if epi == L.EPI_ACCUM:
            raise ValueError("accumulate needs out")
        out = torch.empty(B, w.rows, dtype=torch.float32, device=x.device)
    y2 = out.view(-1, w.rows)
    if y2.stride(-1) != 1:
        raise ValueError("out must have unit stride")
    if bias is not None:
        _need(bias, torch.float32, "bias")
    nw, eps = (None, 0.0) if norm is None else norm
    if nw is not None:
        _need(nw, torch.float32, "norm weight")
    if B >= GEMM_MIN_ROWS and w.dtype in ELEM_BYTES and nw is not None:
        # plain weights: the fp32 MFMA GEMM has no RMSNorm prologue; normalise first
        x2 = rmsnorm(x2, nw, eps)
        nw = None
    if B >= GEMM_MIN_ROWS and (w.dtype in (Q8_0, Q4_0) or w.dtype in ELEM_BYTES):
        lib = L.load()
        need = int(lib.vgx_qgemm_workspace_bytes(B, w.rows, w.cols, epi))
        ws = gemm_workspace(x.device).get(need)
        L.check(lib.vgx_qgemm(w.dtype, w.packed.data_ptr(), w.rows, w.cols, x2.data_ptr(), x2.stride(0), B, _ptr(nw),
                              float(eps), _ptr(bias), y2.data_ptr(), y2.stride(0), epi, ws.data_ptr(), ws.numel(),
                              _stream(x.device)), "vgx_qgemm")
        return out
    L.check(L.load().vgx_qlinear_ex(w.dtype, w.packed.data_ptr(), w.rows, w.cols, x2.data_ptr(), x2.stride(0), B,
                                    _ptr(nw), float(eps), _ptr(bias), y2.data_ptr(), y2.stride(0), epi,
                                    _stream(x.device)), "vgx_qlinear_ex")
    return out


def qlinear_indirect(w: QWeight, x: torch.Tensor, y_addr: torch.Tensor,
                     norm: Optional[Tuple[torch.Tensor, float]] = None) -> None:
    """y = u @ W^T into the [B, rows] fp32 buffer whose address the int64 device word ``y_addr`` holds
    when the launch runs (vgx_qlinear_indirect); GEMV batches (B < GEMM_MIN_ROWS) only."""
    _need(x, torch.float32, "x")
    if w.gateup:
        raise ValueError("qlinear_indirect takes a plain tensor")
    if y_addr.dtype != torch.int64 or y_addr.numel() != 1 or y_addr.device != x.device:
        raise ValueError("y_addr must be one int64 word on the activations' device")
    x2 = x.reshape(-1, w.cols) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    if B >= GEMM_MIN_ROWS:
        raise ValueError("qlinear_indirect runs the GEMV (batches below GEMM_MIN_ROWS)")
    nw, eps = (None, 0.0) if norm is None else norm
    if nw is not None:
        _need(nw, torch.float32, "norm weight")
    L.check(L.load().vgx_qlinear_indirect(w.dtype, w.packed.data_ptr(), w.rows, w.cols, x2.data_ptr(), x2.stride(0),
                                          B, _ptr(nw), float(eps), None, y_addr.data_ptr(), w.rows, L.EPI_STORE,
                                          _stream(x.device)), "vgx_qlinear_indirect")


def qlinear(w: QWeight, x: torch.Tensor, bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
            accumulate: bool = False, norm: Optional[Tuple[torch.Tensor, float]] = None) -> torch.Tensor:
    """y = u @ W^T (+ bias) with u = x, or u = RMSNorm(x) with norm = (weight, eps); with ``accumulate``
    the product is added into ``out``."""
    if w.gateup:
        raise ValueError("use qlinear_swiglu for gate/up tensors")
    return _gemv(w, x, out, L.EPI_ACCUM if accumulate else L.EPI_STORE, bias, norm)


def score_side(phase: int, feat: torch.Tensor, ema: torch.Tensor, first: bool, w1: QWeight, b1: torch.Tensor,
               ln_w: torch.Tensor, ln_b: torch.Tensor, eps: float, w2: torch.Tensor, b2: torch.Tensor, h: torch.Tensor,
               out: torch.Tensor, out_index: Optional[torch.Tensor] = None) -> "L.ScoreSide":
    """One half of seg_score_step as a job for qlinear_side (phase 1: fc1 into h; phase 2: the score and
    the EMA update).  The tensors must outlive the launches."""
    if w1.dtype != L.F32 or w1.cols != feat.numel():
        raise ValueError("the scorer job needs the F32 fc1 weight of the features' width")
    return L.ScoreSide(phase, feat.data_ptr(), feat.numel(), ema.data_ptr(), 1 if first else 0, w1.packed.data_ptr(),
                       w1.rows, b1.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(), float(eps), w2.data_ptr(),
                       b2.data_ptr(), h.data_ptr(), out.data_ptr(), _ptr(out_index))


def qlinear_side(w: QWeight, x: torch.Tensor, out: torch.Tensor, accumulate: bool, side: "L.ScoreSide") -> torch.Tensor:
    """qlinear on a few rows (below GEMM_MIN_ROWS) with a scorer job riding in the same launch when the
    GEMV leaves workgroups free for it (else launched after it)."""
    _need(x, torch.float32, "x")
    B = x.reshape(-1, w.cols).shape[0]
    if w.gateup or B >= GEMM_MIN_ROWS or x.stride(-1) != 1 or out.stride(-1) != 1:
        raise ValueError("qlinear_side takes a plain projection of a few contiguous rows")
    x2, y2 = x.reshape(B, w.cols), out.view(B, w.rows)
    L.check(L.load().vgx_qlinear_side(w.dtype, w.packed.data_ptr(), w.rows, w.cols, x2.data_ptr(), x2.stride(0), B,
                                      None, 0.0, None, y2.data_ptr(), y2.stride(0),
                                      L.EPI_ACCUM if accumulate else L.EPI_STORE, C.byref(side), _stream(x.device)),
            "vgx_qlinear_side")
    return out


def qlinear_swiglu(w: QWeight, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                   norm: Optional[Tuple[torch.Tensor, float]] = None) -> torch.Tensor:
    """h = silu(u @ Wg^T) * (u @ Wu^T), u = x or RMSNorm(x)."""
    if not w.gateup:
        raise ValueError("qlinear_swiglu needs a gate/up tensor")
    return _gemv(w, x, out, L.EPI_SWIGLU, None, norm)


def embed(w: QWeight, ids: torch.Tensor, pad_row: int = 0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ids64 = ids.reshape(-1).to(device=w.device, dtype=torch.int64)
    n = ids64.numel()
    if out is None:
        out = torch.empty(n, w.cols, dtype=torch.float32, device=w.device)
    o2 = out.view(n, w.cols)
    L.check(L.load().vgx_embed_rows(w.dtype, w.packed.data_ptr(), w.rows, w.cols, ids64.data_ptr(), n, pad_row,
                                    o2.data_ptr(), o2.stride(0), _stream(w.device)), "vgx_embed_rows")
    return out


# ------------------------------------------------------------------------------------------
# attention and row ops
# ------------------------------------------------------------------------------------------

KV_DTYPES = {torch.float32: L.F32, torch.bfloat16: L.BF16}


class Workspace:
    """Grow-only device scratch owned by the caller (the library never allocates)."""

    def __init__(self, device):
        self.device = device
        self.buf = torch.empty(0, dtype=torch.uint8, device=device)

    def get(self, nbytes: int) -> torch.Tensor:
        """At least ``nbytes`` bytes (256-byte aligned, zero-filled when first allocated)."""
        if self.buf.numel() < nbytes:
            self.buf = torch.zeros(max(nbytes, 2 * self.buf.numel()), dtype=torch.uint8, device=self.device)
        return self.buf


def attn_decode(q: torch.Tensor, spans, out: Optional[torch.Tensor] = None, bias: Optional[torch.Tensor] = None,
                bias_span: int = -1, scale: Optional[float] = None, ws: Optional[Workspace] = None,
                causal_base: int = -1) -> torch.Tensor:
    """q: [B, H, D] fp32 post-RoPE (heads and dims contiguous, any batch stride).  spans: list of
    (K, V) or (K, V, n_dev) with views shaped [B, G, n, D] (unit stride in D and n; any batch / group
    stride; batch stride 0 shares one span across entries) and n_dev an optional device int32 (one
    element) capping the span's length on the device.  bias: [H, n_bias] fp32 or None.  causal_base >= 0: the last
    span is causal (entry b sees causal_base + b + 1 keys).  Returns [B, H, D] fp32."""
    _need(q, torch.float32, "q")
    B, H, D = q.shape
    if q.stride(2) != 1 or q.stride(1) != D:
        q = q.contiguous()
    kv_dt = None
    arr = (L.KVSpan * 4)()
    n_tot = 0
    G = None
    for i, span in enumerate(spans):
        k, v = span[0], span[1]
        dyn = span[2] if len(span) > 2 else None
        if kv_dt is None:
            kv_dt = KV_DTYPES[k.dtype]
        if KV_DTYPES[k.dtype] != kv_dt or v.dtype != k.dtype:
            raise ValueError("mixed KV dtypes")
        if k.shape != v.shape or k.dim() != 4 or k.shape[3] != D or k.shape[0] not in (B, 1):
            raise ValueError(f"span {i} shape {tuple(k.shape)}")
        G = k.shape[1]
        if k.shape[2] == 0:
            arr[i] = L.KVSpan(None, None, 0, 0, 0)
            continue
        if k.stride(3) != 1 or k.stride(2) != D or v.stride(3) != 1 or v.stride(2) != D or \
                k.stride(0) != v.stride(0) or k.stride(1) != v.stride(1):
            raise ValueError(f"span {i} strides")
        G = k.shape[1]
        n = k.shape[2]
        bs = k.stride(0) if k.shape[0] == B and B > 1 else 0
        if dyn is not None and (dyn.dtype != torch.int32 or not dyn.is_cuda):
            raise ValueError("dynamic span length must be a device int32 tensor")
        arr[i] = L.KVSpan(k.data_ptr(), v.data_ptr(), n, bs, k.stride(1), _ptr(dyn))
        n_tot += n
    if out is None:
        out = torch.empty(B, H, D, dtype=torch.float32, device=q.device)
    lib = L.load()
    need = int(lib.vgx_attn_decode_workspace_bytes(B, H, G, D, n_tot))
    L.check(0 if need >= 0 else need, "vgx_attn_decode_workspace_bytes")
    ws = ws or Workspace(q.device)
    wbuf = ws.get(max(need, 1))
    if bias is not None:
        _need(bias, torch.float32, "bias")
        if bias.stride(1) != 1:
            raise ValueError("bias needs unit stride along keys")
        if not 0 <= bias_span < len(spans) or bias.shape[0] != H or bias.shape[1] < spans[bias_span][0].shape[2]:
            raise ValueError("bias must be [H, >= len(bias span)]")
    L.check(lib.vgx_attn_decode(kv_dt, q.data_ptr(), q.stride(0), arr, len(spans), _ptr(bias),
                                bias.stride(0) if bias is not None else 0, bias_span, causal_base, out.data_ptr(),
                                B, H, G, D,
                                float(scale if scale is not None else D ** -0.5), wbuf.data_ptr(), wbuf.numel(),
                                _stream(q.device)), "vgx_attn_decode")
    return out


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    _need(x, torch.float32, "x")
    d = x.shape[-1]
    x2 = x.reshape(-1, d)
    if out is None:
        out = torch.empty_like(x2)
    o2 = out.view(-1, d)
    L.check(L.load().vgx_rmsnorm(x2.data_ptr(), x2.stride(0), w.data_ptr(), o2.data_ptr(), o2.stride(0), x2.shape[0],
                                 d, float(eps), _stream(x.device)), "vgx_rmsnorm")
    return out.view(x.shape)


def rope_qkv_write(q: Optional[torch.Tensor], k: torch.Tensor, v: torch.Tensor, table: torch.Tensor,
                   table_rstride: int, k_rot: Optional[torch.Tensor], k_raw: Optional[torch.Tensor],
                   v_dst: torch.Tensor, dst_tstride: int, dst_gstride: int,
                   sink_k: Optional[torch.Tensor] = None, sink_v: Optional[torch.Tensor] = None, n_sink: int = 0,
                   sink_tstride: int = 0, sink_gstride: int = 0) -> None:
    """q [N,H,D] (rotated in place), k/v [N,G,D] fp32 (heads and dims contiguous, any token stride);
    destinations are the first rows to write (views into the KV cache), strides in elements."""
    N, G, D = k.shape
    H = 0 if q is None else q.shape[1]
    for t in (q, k, v):
        if t is not None and (t.stride(2) != 1 or t.stride(1) != D):
            raise ValueError("q/k/v need contiguous heads")
    kv_dt = KV_DTYPES[v_dst.dtype]
    L.check(L.load().vgx_rope_qkv_write(kv_dt, _ptr(q), q.stride(0) if q is not None else 0, k.data_ptr(), k.stride(0),
                                        v.data_ptr(), v.stride(0), N, H, G, D, table.data_ptr(),
                                        table_rstride, _ptr(k_rot), _ptr(k_raw), v_dst.data_ptr(), dst_tstride,
                                        dst_gstride, _ptr(sink_k), _ptr(sink_v), n_sink, sink_tstride, sink_gstride,
                                        _stream(k.device)), "vgx_rope_qkv_write")


def rope_rotate(src: torch.Tensor, dst: torch.Tensor, table: torch.Tensor, table_rstride: int) -> None:
    """src/dst: [O, n, D] views with contiguous rows (any outer stride); row i of every outer slice is
    rotated by table row i * table_rstride (fp32 [cos(D/2) | sin(D/2)])."""
    O, n, D = src.shape
    if dst.shape != src.shape or dst.dtype != src.dtype:
        raise ValueError("src/dst mismatch")
    for t in (src, dst):
        if t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError("rows must be contiguous")
    L.check(L.load().vgx_rope_rotate(KV_DTYPES[src.dtype], src.data_ptr(), dst.data_ptr(), O, src.stride(0),
                                     dst.stride(0), n, D, table.data_ptr(), table_rstride, _stream(src.device)),
            "vgx_rope_rotate")


def gather_rows(src: torch.Tensor, dst: torch.Tensor, idx: torch.Tensor) -> None:
    """src: [O, n_src, D], dst: [O, n_idx, D] (views, uniform outer stride); idx int32 [n_idx]."""
    O, n_src, D = src.shape
    assert dst.shape[0] == O and dst.shape[2] == D and idx.numel() == dst.shape[1]
    idx32 = idx.to(device=src.device, dtype=torch.int32).contiguous()
    L.check(L.load().vgx_gather_rows(KV_DTYPES[src.dtype], src.data_ptr(), dst.data_ptr(), idx32.data_ptr(),
                                     idx32.numel(), n_src, O, src.stride(0), dst.stride(0), D, _stream(src.device)),
            "vgx_gather_rows")


def ema_habituate(f: torch.Tensor, hab: torch.Tensor, ema: torch.Tensor, first: bool) -> None:
    T, fd = f.shape
    L.check(L.load().vgx_ema_habituate(f.data_ptr(), f.stride(0), hab.data_ptr(), hab.stride(0), ema.data_ptr(), T, fd,
                                       1 if first else 0, _stream(f.device)), "vgx_ema_habituate")


def layernorm(x: torch.Tensor, w: torch.Tensor, b: torch.Tensor, eps: float, out: torch.Tensor) -> torch.Tensor:
    n, d = x.shape
    L.check(L.load().vgx_layernorm(x.data_ptr(), x.stride(0), w.data_ptr(), b.data_ptr(), out.data_ptr(), out.stride(0),
                                   n, d, float(eps), _stream(x.device)), "vgx_layernorm")
    return out


def seg_score_step(feat: torch.Tensor, ema: torch.Tensor, first: bool, w1: "QWeight", b1: torch.Tensor,
                   ln_w: torch.Tensor, ln_b: torch.Tensor, eps: float, w2: torch.Tensor, b2: torch.Tensor,
                   out: torch.Tensor, out_index: Optional[torch.Tensor] = None) -> None:
    """The scorer of one decode token (two launches; the fc1 GEMV builds both LayerNormed rows itself):
    its score into out[0] (shifted by the device int32 ``out_index``) and the EMA state updated."""
    fd = feat.numel()
    if w1.dtype != L.F32 or w1.cols != fd:
        raise ValueError("seg_score_step needs the F32 fc1 weight of the features' width")
    h = torch.empty(2, w1.rows, dtype=torch.float32, device=feat.device)
    L.check(L.load().vgx_seg_score_step(feat.data_ptr(), fd, ema.data_ptr(), 1 if first else 0, w1.packed.data_ptr(),
                                        w1.rows, b1.data_ptr(), ln_w.data_ptr(), ln_b.data_ptr(), float(eps),
                                        w2.data_ptr(), b2.data_ptr(), h.data_ptr(), out.data_ptr(), _ptr(out_index),
                                        _stream(feat.device)), "vgx_seg_score_step")


def seg_score_tail(h: torch.Tensor, w2: torch.Tensor, b2: torch.Tensor, T: int, first: bool, out: torch.Tensor,
                   out_index: Optional[torch.Tensor] = None) -> None:
    """Scores of T tokens into out[0:T] (shifted by the device int32 ``out_index`` when given)."""
    L.check(L.load().vgx_seg_score_tail(h.data_ptr(), h.stride(0), w2.data_ptr(), b2.data_ptr(), h.shape[1], T,
                                        1 if first else 0, out.data_ptr(), _ptr(out_index), _stream(h.device)),
            "vgx_seg_score_tail")


def rope_qkv_write_step(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, table: torch.Tensor, table_rstride: int,
                        step: torch.Tensor, k_rot: Optional[torch.Tensor], k_raw: Optional[torch.Tensor],
                        v_dst: torch.Tensor, sink_k: Optional[torch.Tensor], sink_v: Optional[torch.Tensor]) -> None:
    """Decode-step RoPE + ring write for B sequences (one token each).  q [B,H,D], k/v [B,G,D] fp32;
    k_rot / k_raw / v_dst: ring tensors [B, G, W, D]; sink_k / sink_v: [B, G, S_cap, D]; slot, table
    row and sink slot come from the device descriptor ``step`` (int32, VGX_STEP_* words)."""
    B, G, D = k.shape
    H = q.shape[1]
    for t in (q, k, v):
        if t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError("q/k/v need contiguous heads")
    for t in (k_rot, k_raw, sink_k):
        if t is not None and t.stride(2) != D:
            raise ValueError("ring rows must be contiguous")
    kv_dt = KV_DTYPES[v_dst.dtype]
    sk_b, sk_g, sk_r = (sink_k.stride(0), sink_k.stride(1), sink_k.stride(2)) if sink_k is not None else (0, 0, 0)
    L.check(L.load().vgx_rope_qkv_write_step(
        kv_dt, q.data_ptr(), q.stride(0), k.data_ptr(), k.stride(0), v.data_ptr(), v.stride(0), B, H, G, D,
        table.data_ptr(), table_rstride, step.data_ptr(), _ptr(k_rot), _ptr(k_raw), v_dst.data_ptr(),
        v_dst.stride(0), v_dst.stride(1), v_dst.stride(2), _ptr(sink_k), _ptr(sink_v), sk_b, sk_g, sk_r,
        _stream(k.device)), "vgx_rope_qkv_write_step")


def qkv_rope_step(wq: QWeight, bq: Optional[torch.Tensor], wkv: QWeight, bkv: Optional[torch.Tensor],
                  x: torch.Tensor, norm: Optional[Tuple[torch.Tensor, float]], table: torch.Tensor,
                  table_rstride: int, step: torch.Tensor, q_out: torch.Tensor, k_rot: torch.Tensor,
                  k_raw: torch.Tensor, v_dst: torch.Tensor, sink_k: Optional[torch.Tensor],
                  sink_v: Optional[torch.Tensor], x_copy: Optional[torch.Tensor] = None) -> None:
    """One decode token: RMSNorm + q/k/v projections (RoPE-pair packed weights) + bias, RoPE, ring and
    sink writes in one launch.  x [1, d] fp32; q_out [1, H, D] fp32; k_rot / k_raw / v_dst ring
    tensors [1, G, W, D] and sink_k / sink_v [1, G, S_cap, D] of the state dtype; the slot, table row
    and sink slot come from ``step``."""
    G, D = k_rot.shape[1], k_rot.shape[3]
    H = q_out.shape[1]
    if x.shape[0] != 1 or not x.is_contiguous() or not q_out.is_contiguous():
        raise ValueError("qkv_rope_step takes one contiguous token")
    for t in (k_rot, k_raw, v_dst, sink_k, sink_v):
        if t is not None and t.stride(2) != D:
            raise ValueError("ring rows must be contiguous")
    if x_copy is not None and not x_copy.is_contiguous():
        raise ValueError("x_copy must be contiguous")
    nw, eps = (norm[0], float(norm[1])) if norm is not None else (None, 0.0)
    sk_g, sk_r = (sink_k.stride(1), sink_k.stride(2)) if sink_k is not None else (0, 0)
    L.check(L.load().vgx_qkv_rope_step(
        wq.dtype, wq.packed.data_ptr(), _ptr(bq), wkv.dtype, wkv.packed.data_ptr(), _ptr(bkv), x.shape[1], H, G, D,
        x.data_ptr(), _ptr(nw), eps, _ptr(x_copy), table.data_ptr(), table_rstride, step.data_ptr(),
        q_out.data_ptr(), KV_DTYPES[v_dst.dtype], k_rot.data_ptr(), k_raw.data_ptr(), v_dst.data_ptr(),
        v_dst.stride(1), v_dst.stride(2), _ptr(sink_k), _ptr(sink_v), sk_g, sk_r, _stream(x.device)),
        "vgx_qkv_rope_step")


def qkv_rope_batch(wq: Optional[QWeight], bq: Optional[torch.Tensor], wkv: QWeight, bkv: Optional[torch.Tensor],
                   x: torch.Tensor, norm: Optional[Tuple[torch.Tensor, float]], table: torch.Tensor,
                   table_rstride: int, step: torch.Tensor, q_out: torch.Tensor, k_rot: Optional[torch.Tensor],
                   k_raw: Optional[torch.Tensor], v_dst: torch.Tensor, sink_k: Optional[torch.Tensor],
                   sink_v: Optional[torch.Tensor]) -> None:
    """A decode batch of B <= 64 sequences (one token each): RMSNorm + q/k/v projections + bias, RoPE,
    ring and sink writes, with the projections' K-split sums taken by the RoPE launch.  wq [H*D, d] and
    wkv [2*G*D, d] (k then v rows), or wq None and wkv [(H+2*G)*D, d]; x [B, d] fp32; q_out [B, H, D]
    fp32; ring tensors [B, G, W, D] and sink tensors [B, G, S_cap, D] of the state dtype."""
    B, d = x.shape
    G, D = v_dst.shape[1], v_dst.shape[3]
    H = q_out.shape[1]
    if x.stride(1) != 1 or q_out.stride(2) != 1 or q_out.stride(1) != D:
        raise ValueError("x rows and q_out heads must be contiguous")
    for t in (k_rot, k_raw, v_dst, sink_k, sink_v):
        if t is not None and t.stride(2) != D:
            raise ValueError("ring rows must be contiguous")
    if k_rot is not None and k_rot.stride() != v_dst.stride():
        raise ValueError("k_rot and v_dst need equal strides")
    if k_raw is not None and k_raw.stride() != v_dst.stride():
        raise ValueError("k_raw and v_dst need equal strides")
    if sink_k is not None and sink_k.stride() != sink_v.stride():
        raise ValueError("sink_k and sink_v need equal strides")
    nw, eps = (norm[0], float(norm[1])) if norm is not None else (None, 0.0)
    lib = L.load()
    need = int(lib.vgx_qkv_rope_batch_workspace_bytes(B, d, H, G, D, 1 if wq is not None else 0))
    ws = gemm_workspace(x.device).get(need)
    sk_b, sk_g, sk_r = (sink_k.stride(0), sink_k.stride(1), sink_k.stride(2)) if sink_k is not None else (0, 0, 0)
    L.check(lib.vgx_qkv_rope_batch(
        wq.dtype if wq is not None else 0, wq.packed.data_ptr() if wq is not None else None, _ptr(bq), wkv.dtype,
        wkv.packed.data_ptr(), _ptr(bkv), d, H, G, D, x.data_ptr(), x.stride(0), B, _ptr(nw), eps,
        table.data_ptr(), table_rstride, step.data_ptr(), q_out.data_ptr(), q_out.stride(0), KV_DTYPES[v_dst.dtype],
        _ptr(k_rot), _ptr(k_raw), v_dst.data_ptr(), v_dst.stride(0), v_dst.stride(1), v_dst.stride(2),
        _ptr(sink_k), _ptr(sink_v), sk_b, sk_g, sk_r, ws.data_ptr(), ws.numel(), _stream(x.device)),
        "vgx_qkv_rope_batch")


_HEAD_ROWS: dict = {}


def _head_rows(rows: tuple, device) -> torch.Tensor:
    """Device int32 copy of a head -> bias-row map (made once per map and device)."""
    key = (rows, str(device))
    t = _HEAD_ROWS.get(key)
    if t is None:
        t = torch.tensor(rows, dtype=torch.int32, device=device)
        _HEAD_ROWS[key] = t
    return t


def attn_prefill(blocks, H: int, G: int, scale: Optional[float] = None, ws: Optional["Workspace"] = None) -> None:
    """MFMA prefill attention for up to 8 query blocks per launch (more are split).

    Each block is a dict: ``q`` [n_q, H, D] view (fp32 or bf16, any token / head stride, D contiguous),
    ``out`` [n_q, H, D] view, fp32 or bf16 (one dtype for all blocks), ``runs``: list of (K, V) views
    [G, n, D] (bf16, or fp32 entering the MFMAs as bf16 hi + lo; one dtype for all runs; D contiguous,
    any row and group stride), ``causal_base``: -1, or b >= 0 making the last run causal (query t sees
    its keys j <= b + t).  Optional ``bias`` fp32 [n_q, R, >= run length] with ``bias_head_row`` (H
    ints: the bias row of head h, < 0: none) and ``bias_run``: query t of head h adds
    bias[t, bias_head_row[h], j] to its score with key j of that run.  With ``ws`` (a Workspace) a launch
    of few query tiles splits its keys over more workgroups (vgx_attn_prefill_ws)."""
    lib = L.load()
    if not blocks:
        return
    D = blocks[0]["q"].shape[-1]
    qdt = blocks[0]["q"].dtype
    kvdt = blocks[0]["runs"][0][0].dtype
    odt = blocks[0]["out"].dtype
    if odt not in (torch.float32, torch.bfloat16):
        raise ValueError("out must be fp32 or bf16")
    if kvdt not in (torch.bfloat16, torch.float32):
        raise ValueError("key runs must be bf16 or fp32")
    scale = float(scale if scale is not None else D ** -0.5)
    for i0 in range(0, len(blocks), 8):
        part = blocks[i0:i0 + 8]
        arr = (L.AttnBlock * len(part))()
        keep = []
        for i, b in enumerate(part):
            q, out = b["q"], b["out"]
            if q.dtype != qdt or out.dtype != odt or q.stride(-1) != 1 or out.stride(-1) != 1:
                raise ValueError("q and out must each share one dtype, both D-contiguous")
            runs = b["runs"]
            if not 1 <= len(runs) <= 4:
                raise ValueError("1 to 4 key runs per block")
            ra = (L.KVRun * 4)()
            for j, (k, v) in enumerate(runs):
                if k.dtype != kvdt or v.dtype != kvdt or k.shape != v.shape:
                    raise ValueError("key runs must be K/V of one dtype and shape")
                if k.stride(-1) != 1 or v.stride(-1) != 1 or k.stride(0) != v.stride(0) or k.stride(1) != v.stride(1):
                    raise ValueError("K and V views need equal strides and contiguous rows")
                ra[j] = L.KVRun(k.data_ptr(), v.data_ptr(), k.shape[1], k.stride(1), k.stride(0))
                keep.append((k, v))
            arr[i] = L.AttnBlock(q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                                 q.shape[0], int(b.get("causal_base", -1)), len(runs), ra)
            if b.get("bias") is not None:
                bias, rows, run = b["bias"], tuple(int(r) for r in b["bias_head_row"]), int(b["bias_run"])
                _need(bias, torch.float32, "bias")
                if bias.dim() != 3 or bias.shape[0] < q.shape[0] or bias.stride(-1) != 1 or len(rows) != H:
                    raise ValueError("bias must be [n_q, head rows, keys] with unit key stride, bias_head_row H rows")
                if not 0 <= run < len(runs) or bias.shape[2] < runs[run][0].shape[1]:
                    raise ValueError("bias_run must name a run no longer than the bias rows")
                if max(rows) >= bias.shape[1]:
                    raise ValueError("bias_head_row names a row the bias does not have")
                rows_dev = _head_rows(rows, bias.device)
                arr[i].bias, arr[i].bias_head_row = bias.data_ptr(), rows_dev.data_ptr()
                arr[i].bias_ldq, arr[i].bias_rstride, arr[i].bias_run = bias.stride(0), bias.stride(1), run
                keep.append((bias, rows_dev))
        qd = L.BF16 if qdt == torch.bfloat16 else L.F32
        od = L.BF16 if odt == torch.bfloat16 else L.F32
        if ws is not None:
            need = int(lib.vgx_attn_prefill_workspace_bytes(H, G))
            L.check(0 if need > 0 else need, "vgx_attn_prefill_workspace_bytes")
            buf = ws.get(need)
            L.check(lib.vgx_attn_prefill_ws(KV_DTYPES[kvdt], qd, od, arr, len(part), H, G, D, scale, buf.data_ptr(),
                                            buf.numel(), _stream(part[0]["q"].device)), "vgx_attn_prefill_ws")
        else:
            L.check(lib.vgx_attn_prefill(KV_DTYPES[kvdt], qd, od, arr, len(part), H, G, D, scale,
                                         _stream(part[0]["q"].device)),
                    "vgx_attn_prefill")


# ------------------------------------------------------------------------------------------
# segment bank and token selection
# ------------------------------------------------------------------------------------------

def seg_step(ids: torch.Tensor, step: torch.Tensor, tok_cur: torch.Tensor, seg_cur: Optional[torch.Tensor],
             ctrl: Optional[torch.Tensor], tiers: Optional[torch.Tensor], seg_min: int, seg_max: int) -> None:
    """Ring and segmenter bookkeeping of one decode step (vgx_seg_step).  ids int64 [B] and step: device
    words; tok_cur int32 [B, W]; seg_cur int32 [W] and ctrl int32 [VGX_SEG_WORDS] for batch 1 with
    segment memory, else None; tiers uint8 [V] or None."""
    B, W = tok_cur.shape
    L.check(L.load().vgx_seg_step(ids.data_ptr(), B, step.data_ptr(), tok_cur.data_ptr(), tok_cur.stride(0),
                                  _ptr(seg_cur), _ptr(ctrl), _ptr(tiers), tiers.numel() if tiers is not None else 0,
                                  seg_min, seg_max, W, _stream(tok_cur.device)), "vgx_seg_step")


def step_begin(ring: int, n_slots: int, slot_bytes: int, counter: torch.Tensor, step: torch.Tensor, ids: torch.Tensor,
               out_ref: Optional[torch.Tensor], tok_cur: torch.Tensor, seg_cur: Optional[torch.Tensor],
               ctrl: Optional[torch.Tensor], tiers: Optional[torch.Tensor], seg_min: int, seg_max: int,
               bias: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
               embed: Optional[Tuple["QWeight", torch.Tensor]] = None) -> None:
    """The decode step's first launch (vgx_step_begin): the step words, ids and output address from
    slot (*counter mod n_slots) of the pinned host ring at address ``ring``, then vgx_seg_step's
    bookkeeping; with ``bias`` = (early, late) [H, cap] fp32 rows, the slot's bias rows; with ``embed`` =
    (table, out [B, cols] fp32), the embedding rows of the ids in the same launch (vgx_step_begin_embed,
    as embed with pad row 0)."""
    B, W = tok_cur.shape
    be, bl = bias if bias is not None else (None, None)
    H, ld, cap = (be.shape[0], be.stride(0), be.shape[1]) if be is not None else (0, 0, 0)
    args = (ring, n_slots, slot_bytes, counter.data_ptr(), step.data_ptr(), ids.data_ptr(), B, _ptr(out_ref),
            tok_cur.data_ptr(), tok_cur.stride(0), _ptr(seg_cur), _ptr(ctrl), _ptr(tiers),
            tiers.numel() if tiers is not None else 0, seg_min, seg_max, W, _ptr(be), _ptr(bl), H, ld, cap)
    if embed is None:
        L.check(L.load().vgx_step_begin(*args, _stream(tok_cur.device)), "vgx_step_begin")
        return
    w, out = embed
    _need(out, torch.float32, "embedding rows")
    if out.dim() != 2 or out.shape != (B, w.cols) or out.stride(1) != 1:
        raise ValueError("embedding rows must be [B, cols] with unit stride along cols")
    L.check(L.load().vgx_step_begin_embed(*args, w.dtype, w.packed.data_ptr(), w.rows, w.cols, out.data_ptr(),
                                          out.stride(0), _stream(tok_cur.device)), "vgx_step_begin_embed")


def seg_evict(sc_prev, seg_prev, tok_prev, mem_pos, mem_score, mem_tok, mem_seg, ctrl, ev: int, t0: int,
              budget: int, idx_old, idx_new) -> None:
    """The segment-bank merge at a chunk boundary (vgx_seg_evict), all on the device."""
    W = sc_prev.numel()
    L.check(L.load().vgx_seg_evict(sc_prev.data_ptr(), seg_prev.data_ptr(), tok_prev.data_ptr(), W, mem_pos.data_ptr(),
                                   mem_score.data_ptr(), mem_tok.data_ptr(), mem_seg.data_ptr(), ctrl.data_ptr(), ev,
                                   t0, budget, idx_old.data_ptr(), idx_new.data_ptr(), _stream(sc_prev.device)),
            "vgx_seg_evict")


def gather_rows_masked(src: torch.Tensor, dst: torch.Tensor, idx: torch.Tensor) -> None:
    """dst[:, j] = src[:, idx[j]] where idx[j] >= 0 (other rows untouched); [O, n, D] views."""
    O, n_src, D = src.shape
    assert dst.shape[0] == O and dst.shape[2] == D and idx.numel() == dst.shape[1] and idx.dtype == torch.int32
    L.check(L.load().vgx_gather_rows_masked(KV_DTYPES[src.dtype], src.data_ptr(), dst.data_ptr(), idx.data_ptr(),
                                            idx.numel(), n_src, O, src.stride(0), dst.stride(0), D,
                                            _stream(src.device)), "vgx_gather_rows_masked")


def rope_rotate_dyn(src: torch.Tensor, dst: torch.Tensor, table0: torch.Tensor, table_rstride: int,
                    dyn: torch.Tensor, row_base: int, limit_rows: bool) -> None:
    """Row i of every outer slice rotated by the table row of position (i + row_base - *dyn), table0
    being the row of position 0 (vgx_rope_rotate_dyn); rows i >= *dyn skipped with limit_rows."""
    O, n, D = src.shape
    for t in (src, dst):
        if t.stride(2) != 1 or t.stride(1) != D:
            raise ValueError("rows must be contiguous")
    L.check(L.load().vgx_rope_rotate_dyn(KV_DTYPES[src.dtype], src.data_ptr(), dst.data_ptr(), O, src.stride(0),
                                         dst.stride(0), n, D, table0.data_ptr(), table_rstride, dyn.data_ptr(),
                                         row_base, 1 if limit_rows else 0, _stream(src.device)), "vgx_rope_rotate_dyn")


def argmax(logits: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """[B, V] fp32 -> int64 [B] on the device (vgx_argmax; the first index on ties)."""
    _need(logits, torch.float32, "logits")
    B, V = logits.shape
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    out = torch.empty(B, dtype=torch.int64, device=logits.device) if out is None else out
    L.check(L.load().vgx_argmax(logits.data_ptr(), logits.stride(0), B, V, out.data_ptr(), _stream(logits.device)),
            "vgx_argmax")
    return out


def topk(logits: torch.Tensor, T: int, ws: Optional["Workspace"] = None):
    """[B, V] fp32 -> (int64 [B, T], fp32 [B, T]) on the device: the T (<= 256) largest logits of each
    row, value desc, index asc (vgx_topk; NaN never a candidate, short rows padded with -1 / -inf)."""
    _need(logits, torch.float32, "logits")
    B, V = logits.shape
    if logits.stride(1) != 1:
        raise ValueError("logits rows must be contiguous")
    lib = L.load()
    need = int(lib.vgx_topk_workspace_bytes(B, V, T))
    L.check(0 if need >= 0 else need, "vgx_topk_workspace_bytes")
    buf = (ws or Workspace(logits.device)).get(max(need, 1))
    idx = torch.empty(B, T, dtype=torch.int64, device=logits.device)
    val = torch.empty(B, T, dtype=torch.float32, device=logits.device)
    L.check(lib.vgx_topk(logits.data_ptr(), logits.stride(0), B, V, int(T), idx.data_ptr(), val.data_ptr(),
                         buf.data_ptr(), buf.numel(), _stream(logits.device)), "vgx_topk")
    return idx, val


def sample_topk(logits: torch.Tensor, k: int, temp: float, rng: torch.Tensor,
                out: Optional[torch.Tensor] = None, ws: Optional["Workspace"] = None) -> torch.Tensor:
    """Top-k sampling per row with the rows' xorshift64 states ``rng`` (uint64 as int64 [B], updated in
    place) -> int64 [B] on the device (vgx_sample_topk)."""
    _need(logits, torch.float32, "logits")
    B, V = logits.shape
    lib = L.load()
    out = torch.empty(B, dtype=torch.int64, device=logits.device) if out is None else out
    need = int(lib.vgx_sample_topk_workspace_bytes(B, V))
    buf = (ws or Workspace(logits.device)).get(need)
    L.check(lib.vgx_sample_topk(logits.data_ptr(), logits.stride(0), B, V, int(k), float(temp), rng.data_ptr(),
                                out.data_ptr(), buf.data_ptr(), buf.numel(), _stream(logits.device)), "vgx_sample_topk")
    return out
