"""Operator-level drop-ins for the attention functions of the reference model.

``block_sliding_attention`` keeps the signature, tensor layouts and semantics of
src/vault_v3_model.py:812-863: q (B, H, L, D) post-RoPE, k / v (B, G, L, D) post-RoPE / values, k_raw
(B, G, L, D) pre-RoPE keys for the sinks; a token of chunk i (W tokens each) attends to all of chunk
i-1, causally to chunk i, and for i >= 2 to the first n_sink tokens re-rotated to the virtual
positions (i-1)W - n_sink + j (clamped at 0; :805-809).  The attention runs in the MFMA prefill
kernel (vgx_attn_prefill) in the dtype of k / v, as the reference's SDPA runs in its input dtype:
bf16 K / V as they are, fp32 K / V as three bf16 pieces each (fp32-level results); other float
dtypes take the fp32 path.  The sink keys are re-rotated on the GPU (vgx_rope_rotate) in fp32 with
float32 angles, the reference's rope_cos_sin arithmetic (:777-782), and stored once in the K / V
dtype (the reference rotates bf16 keys in bf16 arithmetic, :790-794, which rounds three times).
"""
from __future__ import annotations

from typing import Optional

import numpy as np
import torch

from . import ops


def rope_table_fp32(positions: np.ndarray, head_dim: int, theta: float) -> np.ndarray:
    """[n, D] rows [cos(D/2) | sin(D/2)] with float32 inverse frequencies and float32 angles
    (src/vault_v3_model.py:777-782)."""
    exps = (np.arange(0, head_dim, 2, dtype=np.int64).astype(np.float32) / np.float32(head_dim)).astype(np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta), exps, dtype=np.float32)).astype(np.float32)
    ang = (np.asarray(positions, dtype=np.float32).reshape(-1, 1) * inv[None, :]).astype(np.float32)
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)


def rope_table_double(positions: np.ndarray, head_dim: int, theta: float) -> np.ndarray:
    """[n, D] rows [cos(D/2) | sin(D/2)] from double-precision angles of a float32 inverse frequency,
    rounded to float32 (the C runtime's arithmetic, runtime/vault3.c:840-849, 2126-2133)."""
    i = np.arange(head_dim // 2, dtype=np.float64)
    inv = (1.0 / np.exp(np.log(np.float64(np.float32(theta))) * (2.0 * i) / head_dim)).astype(np.float32)
    ang = np.asarray(positions, dtype=np.float64).reshape(-1, 1) * inv.astype(np.float64)[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)


_TABLES: dict = {}


def _sink_table(n: int, W: int, S: int, D: int, theta: float, device, angles: str) -> torch.Tensor:
    """Device RoPE rows of the re-rotated sink positions of chunks 2 .. n-1, built once per shape."""
    key = (n, W, S, D, float(theta), str(device), angles)
    t = _TABLES.get(key)
    if t is None:
        pos = np.concatenate([np.maximum(0, (i - 1) * W - S + np.arange(S)) for i in range(2, n)])
        fn = rope_table_double if angles == "double" else rope_table_fp32
        t = torch.from_numpy(fn(pos, D, theta)).to(device)
        if len(_TABLES) > 16:
            _TABLES.clear()
        _TABLES[key] = t
    return t


def _operand(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``t`` as ``dtype`` with unit stride along D and 16-byte aligned rows (a view when it already is)."""
    if t.dtype == dtype and t.stride(-1) == 1 and t.data_ptr() % 16 == 0 and \
            all(st * t.element_size() % 16 == 0 for st in t.stride()[:-1]):
        return t
    return t.to(dtype).contiguous()


def block_sliding_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int,
                            k_raw: Optional[torch.Tensor] = None, n_sink: int = 0, head_dim: int = 0,
                            rope_theta: float = 0.0, *, out: Optional[torch.Tensor] = None,
                            angles: str = "fp32") -> torch.Tensor:
    """Returns (B, H, L, D) in q's dtype (fp32 accumulation; operands as described above).

    Keywords beyond the reference signature: ``out``, a (B, H, L, D) fp32 or bf16 destination (any
    strides with unit stride along D), and ``angles``: "fp32" re-rotates the sinks with the
    reference's float32 angles, "double" with the C runtime's double-precision angles (for callers
    whose q / k were rotated that way).  Strided q / k / v views (unit stride along D) are read in
    place, without copies."""
    B, H, Lq, D = q.shape
    G = k.shape[1]
    W = int(window)
    if k.shape != (B, G, Lq, D) or v.shape != k.shape:
        raise ValueError("k / v must be (B, G, L, D) matching q")
    S = min(n_sink, Lq) if (k_raw is not None and n_sink > 0) else 0
    kvdt = torch.bfloat16 if k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16 else torch.float32
    kb = _operand(k, kvdt)
    vb = _operand(v, kvdt)
    if kb.stride() != vb.stride():
        kb, vb = kb.contiguous(), vb.contiguous()
    qq = _operand(q, q.dtype if q.dtype in (torch.float32, torch.bfloat16) else torch.float32)
    # bf16 callers get the kernel's bf16 output (fp32 result rounded to nearest even); others fp32
    odt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
    if out is None:
        out = torch.empty(B, H, Lq, D, dtype=odt, device=q.device)
    elif out.shape != q.shape or out.dtype not in (torch.float32, torch.bfloat16) or out.stride(-1) != 1:
        raise ValueError("out must be (B, H, L, D) fp32 or bf16 with unit stride along D")
    n = (Lq + W - 1) // W
    sinks = sink_v = None
    if S and n >= 3:
        # sink keys re-rotated for every chunk i >= 2 in one launch: the raw keys repeated per chunk,
        # [B*G][n-2][S][D], row (i - 2) * S + s rotated by table row (i - 2) * S + s
        tab = _sink_table(n, W, S, D, rope_theta or 1.0, q.device, angles)
        kr = k_raw[:, :, :S].to(kvdt).reshape(B * G, 1, S, D).expand(B * G, n - 2, S, D)
        kr = kr.contiguous().view(B * G, (n - 2) * S, D)
        sinks = torch.empty(B * G, (n - 2) * S, D, dtype=kvdt, device=q.device)
        ops.rope_rotate(kr, sinks, tab, D)
        sinks = sinks.view(B, G, n - 2, S, D)
        # values in the same layout (a K / V run shares one pair of strides)
        sink_v = vb[:, :, :S].reshape(B, G, 1, S, D).expand(B, G, n - 2, S, D).contiguous()
    blocks = []
    for b in range(B):
        for i in range(n):
            r0, r1 = i * W, min(Lq, (i + 1) * W)
            runs = []
            if i >= 2 and S:
                runs.append((sinks[b, :, i - 2], sink_v[b, :, i - 2]))
            if i >= 1:
                runs.append((kb[b, :, r0 - W:r0], vb[b, :, r0 - W:r0]))
            runs.append((kb[b, :, r0:r1], vb[b, :, r0:r1]))
            blocks.append({"q": qq[b, :, r0:r1].transpose(0, 1), "out": out[b, :, r0:r1].transpose(0, 1),
                           "runs": runs, "causal_base": 0})
    ops.attn_prefill(blocks, H, G)
    return out if out.dtype == q.dtype else out.to(q.dtype)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor, chunk: int = 1024) -> None:
    """Full causal attention (the reference's SDPA with is_causal, src/vault_v3_model.py:1057-1058)
    on the MFMA prefill kernel: q / out (B, H, L, D), k / v (B, G, L, D) views as in
    block_sliding_attention; queries in blocks of ``chunk``, each over the keys up to its last query
    (key tiles in a query tile's future skipped)."""
    B, H, Lq, D = q.shape
    G = k.shape[1]
    kvdt = torch.bfloat16 if k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16 else torch.float32
    kb, vb = _operand(k, kvdt), _operand(v, kvdt)
    if kb.stride() != vb.stride():
        kb, vb = kb.contiguous(), vb.contiguous()
    qq = _operand(q, q.dtype if q.dtype in (torch.float32, torch.bfloat16) else torch.float32)
    blocks = []
    for b in range(B):
        for r0 in range(0, Lq, chunk):
            r1 = min(Lq, r0 + chunk)
            blocks.append({"q": qq[b, :, r0:r1].transpose(0, 1), "out": out[b, :, r0:r1].transpose(0, 1),
                           "runs": [(kb[b, :, :r1], vb[b, :, :r1])], "causal_base": r0})
    ops.attn_prefill(blocks, H, G)
