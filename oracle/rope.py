"""RoPE tables and rotation (TEST INFRASTRUCTURE ONLY).

Rotate-half pairing (i, i + D/2), angle p * w_i with w_i = theta^(-2i/D)
(docs/VAULT_v3_SPEC.md:51-53; src/vault_v3_model.py:777-794; runtime/vault3.c:662-678):
    R_p(z)_i       = z_i cos - z_{i+D/2} sin
    R_p(z)_{i+D/2} = z_{i+D/2} cos + z_i sin

Two angle conventions exist in the reference:
* ``table_c``:     inv_freq in float32 from double exp/log, angle p * inv_freq evaluated in double,
                   cos/sin rounded to float32 (runtime/vault3.c:840-849, 2126-2133, 866-891).
* ``table_torch``: inv_freq and p * inv_freq in float32, then cos/sin of the float32 angle
                   (src/vault_v3_model.py:777-782).
"""
from __future__ import annotations

import numpy as np


def inv_freq_c(D: int, theta: float) -> np.ndarray:
    i = np.arange(D // 2, dtype=np.float64)
    return (1.0 / np.exp(np.log(np.float64(np.float32(theta))) * (2.0 * i) / D)).astype(np.float32)


def table_c(positions, D: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin: [n, D/2] float32 (double-precision angles)."""
    p = np.asarray(positions, dtype=np.float64).reshape(-1, 1)
    ang = p * inv_freq_c(D, theta).astype(np.float64)[None, :]
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def table_torch(positions, D: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos, sin: [n, D/2] float32 with float32 angles (the PyTorch model's arithmetic)."""
    exps = (np.arange(0, D, 2, dtype=np.int64).astype(np.float32) / np.float32(D)).astype(np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta), exps, dtype=np.float32)).astype(np.float32)
    ang = (np.asarray(positions, dtype=np.float32).reshape(-1, 1) * inv[None, :]).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


def rotate(z: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """z: [..., n, D]; cos/sin: [n, D/2] (or broadcastable).  Computed in float64."""
    z = np.asarray(z, dtype=np.float64)
    h = z.shape[-1] // 2
    a, b = z[..., :h], z[..., h:]
    c = np.asarray(cos, dtype=np.float64)
    s = np.asarray(sin, dtype=np.float64)
    return np.concatenate([a * c - b * s, b * c + a * s], axis=-1)
