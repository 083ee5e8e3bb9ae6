"""Operator-level drop-ins for the attention functions of the reference model.

``block_sliding_attention`` keeps the signature, tensor layouts and semantics of
src/vault_v3_model.py:812-863: q (B, H, L, D) post-RoPE, k / v (B, G, L, D) post-RoPE / values, k_raw
(B, G, L, D) pre-RoPE keys for the sinks; a token of chunk i (W tokens each) attends to all of chunk
i-1, causally to chunk i, and for i >= 2 to the first n_sink tokens re-rotated to the virtual
positions (i-1)W - n_sink + j (clamped at 0; :805-809).  The attention runs in the bf16 MFMA kernel
(vgx_attn_prefill); fp32 inputs are rounded to bf16 there (the reference's bf16 path).  The sink keys
are re-rotated on the GPU (vgx_rope_rotate) with float32 angles, the reference's rope_cos_sin
arithmetic (:777-782).
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


_TABLES: dict = {}


def _sink_table(n: int, W: int, S: int, D: int, theta: float, device) -> torch.Tensor:
    """Device RoPE rows of the re-rotated sink positions of chunks 2 .. n-1, built once per shape."""
    key = (n, W, S, D, float(theta), str(device))
    t = _TABLES.get(key)
    if t is None:
        pos = np.concatenate([np.maximum(0, (i - 1) * W - S + np.arange(S)) for i in range(2, n)])
        t = torch.from_numpy(rope_table_fp32(pos, D, theta)).to(device)
        if len(_TABLES) > 16:
            _TABLES.clear()
        _TABLES[key] = t
    return t


def block_sliding_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window: int,
                            k_raw: Optional[torch.Tensor] = None, n_sink: int = 0, head_dim: int = 0,
                            rope_theta: float = 0.0) -> torch.Tensor:
    """Returns (B, H, L, D) in q's dtype (computed in fp32 from bf16 operands)."""
    B, H, Lq, D = q.shape
    G = k.shape[1]
    W = int(window)
    if k.shape != (B, G, Lq, D) or v.shape != k.shape:
        raise ValueError("k / v must be (B, G, L, D) matching q")
    S = min(n_sink, Lq) if (k_raw is not None and n_sink > 0) else 0
    kb = k.to(torch.bfloat16).contiguous()
    vb = v.to(torch.bfloat16).contiguous()
    qq = q if q.dtype in (torch.float32, torch.bfloat16) else q.float()
    qq = qq.contiguous()
    # bf16 callers get the kernel's bf16 output (fp32 result rounded to nearest even); others fp32
    odt = torch.bfloat16 if q.dtype == torch.bfloat16 else torch.float32
    out = torch.empty(B, H, Lq, D, dtype=odt, device=q.device)
    n = (Lq + W - 1) // W
    sinks = sink_v = None
    if S and n >= 3:
        # sink keys re-rotated for every chunk i >= 2 in one launch: the raw keys repeated per chunk,
        # [B*G][n-2][S][D], row (i - 2) * S + s rotated by table row (i - 2) * S + s
        tab = _sink_table(n, W, S, D, rope_theta or 1.0, q.device)
        kr = k_raw[:, :, :S].to(torch.bfloat16).reshape(B * G, 1, S, D).expand(B * G, n - 2, S, D)
        kr = kr.contiguous().view(B * G, (n - 2) * S, D)
        sinks = torch.empty(B * G, (n - 2) * S, D, dtype=torch.bfloat16, device=q.device)
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
