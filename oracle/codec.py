"""Q8_0 / Q4_0 block codec (and the BF16 / F16 element decode) restated in numpy (TEST INFRASTRUCTURE ONLY).

Block layouts (little endian), tools/vlt3.py:98-99 and docs/VAULT_v3_SPEC.md:141-142:

* Q8_0: 34 bytes per 32 weights: ``[d: fp16][q: int8 x 32]``, ``w[j] = f32(d) * q[j]``
  (tools/vlt3.py:114-116; runtime/vault3.c:536-563, 632-640).
* Q4_0: 18 bytes per 32 weights: ``[d: fp16][qs: u8 x 16]``; byte ``j`` holds weight ``j``
  in its low nibble and weight ``j + 16`` in its high nibble, value ``(n - 8) * f32(d)``
  (tools/vlt3.py:152-157; runtime/vault3.c:564-598, 641-650).  ``d`` may be negative.

The fp16 decode is written out bit by bit (not numpy's cast) so that it is pinned
independently against numpy's IEEE half conversion in the tests.
"""
from __future__ import annotations

import numpy as np

QK = 32
Q8_BYTES = 34
Q4_BYTES = 18

F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 8, 9


def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    """IEEE binary16 -> binary32, from the bit fields (runtime/vault3.c:49-66 semantics,
    except that non-finite values decode to inf/nan instead of the C table's 0)."""
    h = np.asarray(h, dtype=np.uint16).astype(np.uint32)
    s = (h >> 15) & 1
    e = (h >> 10) & 0x1F
    m = h & 0x3FF
    sign = np.where(s == 1, -1.0, 1.0)
    normal = sign * np.ldexp(1.0 + m / 1024.0, e.astype(np.int64) - 15)
    sub = sign * np.ldexp(m / 1024.0, -14)
    inf_nan = np.where(m == 0, sign * np.inf, np.nan)
    out = np.where(e == 0, sub, np.where(e == 31, inf_nan, normal))
    return out.astype(np.float32)


def q8_0_decode(raw: bytes | np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Q8_0 AoS blocks -> fp32 [rows, cols] (tools/vlt3.py:114-116)."""
    assert cols % QK == 0
    nb = cols // QK
    a = np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw.tobytes(), dtype=np.uint8)
    assert a.size == rows * nb * Q8_BYTES, (a.size, rows, cols)
    blk = a.reshape(rows, nb, Q8_BYTES)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint16) | (blk[..., 1].astype(np.uint16) << 8))
    q = blk[..., 2:].view(np.int8).astype(np.float32)
    return (q * d[..., None]).reshape(rows, cols)


def q4_0_decode(raw: bytes | np.ndarray, rows: int, cols: int) -> np.ndarray:
    """Q4_0 AoS blocks -> fp32 [rows, cols] (tools/vlt3.py:152-157)."""
    assert cols % QK == 0
    nb = cols // QK
    a = np.frombuffer(bytes(raw) if not isinstance(raw, np.ndarray) else raw.tobytes(), dtype=np.uint8)
    assert a.size == rows * nb * Q4_BYTES, (a.size, rows, cols)
    blk = a.reshape(rows, nb, Q4_BYTES)
    d = f16_bits_to_f32(blk[..., 0].astype(np.uint16) | (blk[..., 1].astype(np.uint16) << 8))
    qs = blk[..., 2:]
    lo = (qs & 0x0F).astype(np.int32) - 8
    hi = (qs >> 4).astype(np.int32) - 8
    q = np.concatenate([lo, hi], axis=-1).astype(np.float32)
    return (q * d[..., None]).reshape(rows, cols)


def decode(dtype: int, raw, rows: int, cols: int) -> np.ndarray:
    if dtype == Q8_0:
        return q8_0_decode(raw, rows, cols)
    if dtype == Q4_0:
        return q4_0_decode(raw, rows, cols)
    if dtype == F32:
        return np.frombuffer(bytes(raw), dtype="<f4").reshape(rows, cols).copy()
    if dtype == BF16:
        # the runtime widens by placing the 16 bits on top of a zero mantissa tail (runtime/vault3.c:517-525)
        h = np.frombuffer(bytes(raw), dtype="<u2").astype(np.uint32) << 16
        return h.view(np.float32).reshape(rows, cols).copy()
    if dtype == F16:
        return f16_bits_to_f32(np.frombuffer(bytes(raw), dtype="<u2")).reshape(rows, cols)
    raise ValueError(dtype)


def block_bytes(dtype: int) -> int:
    return {Q8_0: Q8_BYTES, Q4_0: Q4_BYTES}[dtype]


def nbytes(dtype: int, rows: int, cols: int) -> int:
    if dtype == F32:
        return 4 * rows * cols
    return rows * (cols // QK) * block_bytes(dtype)
