"""fp64-accumulated GEMV / SwiGLU / RMSNorm (TEST INFRASTRUCTURE ONLY).

* ``gemv``: y = W x + b with W the dequantized fp32 weights, accumulated in float64
  (runtime/vault3.c:499-624 row_dot / matvec; src/vault_v3_model.py nn.Linear).
* ``gemv_bound``: a per-output bound on fp32 accumulation error, proportional to
  ``sum_j |w_j x_j|`` plus, for Q4_0, the magnitude of the nibble-offset term
  ``8 |d_b| sum_j |x_j|`` that an unsigned-nibble kernel accumulates and cancels.
* ``swiglu``: silu(g) * u with silu(t) = t / (1 + exp(-t)) (runtime/vault3.c:1949-1956,
  src/vault_v3_model.py:1149-1150).
* ``rmsnorm``: g * (x / sqrt(mean(x^2) + eps)) (runtime/vault3.c:656-660,
  src/vault_v3_model.py:764-774).
"""
from __future__ import annotations

import numpy as np

from .codec import QK, Q4_0


def gemv(w: np.ndarray, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    """w: [rows, cols] fp32 dequantized, x: [B, cols] -> [B, rows] float64."""
    y = np.asarray(x, dtype=np.float64) @ np.asarray(w, dtype=np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, dtype=np.float64)[None, :]
    return y


def gemv_bound(w: np.ndarray, x: np.ndarray, dtype: int, rel: float = 2e-6) -> np.ndarray:
    """Allowed |y_kernel - y_oracle| per output: rel * (|W| |x| + Q4 offset magnitude) + 1e-30."""
    aw = np.abs(np.asarray(w, dtype=np.float64))
    ax = np.abs(np.asarray(x, dtype=np.float64))
    mag = ax @ aw.T
    if dtype == Q4_0:
        rows, cols = w.shape
        nb = cols // QK
        # |d_b| per (row, block): max |w| over the block is at most 8 |d|, and >= |d| unless all zero;
        # use 16 * max|w| / 8 as a safe stand-in for the 8|d| sum|x| + sum n|x| terms.
        dmax = aw.reshape(rows, nb, QK).max(axis=2) / 8.0 * 16.0        # [rows, nb]
        xs = ax.reshape(ax.shape[0], nb, QK).sum(axis=2)                  # [B, nb]
        mag = mag + xs @ dmax.T
    return rel * mag * np.sqrt(max(1.0, w.shape[1] / 32.0)) + 1e-30


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, dtype=np.float64)


def rmsnorm(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return np.asarray(g, dtype=np.float64) * (x * inv)
