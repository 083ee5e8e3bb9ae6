"""Torch-facing wrappers of libvault_amd entry points.

Torch provides device memory and the current HIP stream; every computation below is a call
into the HIP library (no torch fallback).  Tensors must live on a ROCm device.
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import _lib as L

F32, Q8_0, Q4_0 = L.F32, L.Q8_0, L.Q4_0
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}


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
        """``data``: VLT3 payload (AoS Q8_0/Q4_0 blocks, or row-major fp32 for F32)."""
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

    def unpack(self) -> torch.Tensor:
        """Packed -> AoS blocks (uint8 device tensor)."""
        if self.gateup:
            raise ValueError("unpack of a gate/up tensor is not supported")
        nbytes = self.rows * self.cols * 4 if self.dtype == F32 else self.rows * (self.cols // 32) * BLOCK_BYTES[self.dtype]
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
        if self.dtype == F32:
            return rows * self.cols * 4
        return rows * (self.cols // 32) * BLOCK_BYTES[self.dtype]


def qlinear(w: QWeight, x: torch.Tensor, bias: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
            accumulate: bool = False) -> torch.Tensor:
    """y = x @ W^T (+ bias); with ``accumulate`` the product is added into ``out``."""
    if w.gateup:
        raise ValueError("use qlinear_swiglu for gate/up tensors")
    _need(x, torch.float32, "x")
    x2 = x.reshape(-1, w.cols) if x.dim() != 2 else x
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    if out is None:
        if accumulate:
            raise ValueError("accumulate needs out")
        out = torch.empty(B, w.rows, dtype=torch.float32, device=x.device)
    y2 = out.view(-1, w.rows)
    if y2.stride(-1) != 1:
        raise ValueError("out must have unit stride")
    if bias is not None:
        _need(bias, torch.float32, "bias")
    L.check(L.load().vgx_qlinear(w.dtype, w.packed.data_ptr(), w.rows, w.cols, x2.data_ptr(), x2.stride(0), B,
                                 _ptr(bias), y2.data_ptr(), y2.stride(0), 1 if accumulate else 0,
                                 _stream(x.device)), "vgx_qlinear")
    return out


def qlinear_swiglu(w: QWeight, x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if not w.gateup:
        raise ValueError("qlinear_swiglu needs a gate/up tensor")
    _need(x, torch.float32, "x")
    x2 = x.reshape(-1, w.cols)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    B = x2.shape[0]
    if out is None:
        out = torch.empty(B, w.rows, dtype=torch.float32, device=x.device)
    h2 = out.view(-1, w.rows)
    L.check(L.load().vgx_qlinear_swiglu(w.dtype, w.packed.data_ptr(), w.rows, w.cols, x2.data_ptr(), x2.stride(0),
                                        B, h2.data_ptr(), h2.stride(0), _stream(x.device)), "vgx_qlinear_swiglu")
    return out


def embed(w: QWeight, ids: torch.Tensor, pad_row: int = 0, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    ids64 = ids.reshape(-1).to(device=w.device, dtype=torch.int64)
    n = ids64.numel()
    if out is None:
        out = torch.empty(n, w.cols, dtype=torch.float32, device=w.device)
    o2 = out.view(n, w.cols)
    L.check(L.load().vgx_embed_rows(w.dtype, w.packed.data_ptr(), w.rows, w.cols, ids64.data_ptr(), n, pad_row,
                                    o2.data_ptr(), o2.stride(0), _stream(w.device)), "vgx_embed_rows")
    return out
