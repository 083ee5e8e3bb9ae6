"""Pins the oracle's Q8_0 / Q4_0 codec (CPU).

Pins: exhaustive fp16 decode vs numpy's IEEE conversion; hand-built known-answer blocks
(d = 1.0 with every int8 / nibble value, a negative-d Q4_0 block, subnormal and max fp16
scales); the quantizer round-trip error bound; and the block byte counts of every benchmark
shape.  The reference's own tests hold no committed vectors for this path, so these closed forms
are the pins (tools/vlt3.py:98-157; docs/VAULT_v3_SPEC.md:141-142).
"""
import struct

import numpy as np
import pytest

from oracle import codec
from vault_amd import vlt3


def test_f16_decode_exhaustive():
    bits = np.arange(65536, dtype=np.uint16)
    ours = codec.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    assert np.array_equal(ours[fin], ref[fin])
    assert np.array_equal(np.isnan(ours), np.isnan(ref))
    assert np.array_equal(np.isinf(ours), np.isinf(ref))


def _q8_block(d_bits: int, q: np.ndarray) -> bytes:
    return struct.pack("<H", d_bits) + q.astype(np.int8).tobytes()


def _q4_block(d_bits: int, nib: np.ndarray) -> bytes:
    nib = nib.astype(np.uint8)
    return struct.pack("<H", d_bits) + (nib[:16] | (nib[16:] << 4)).tobytes()


def test_q8_known_answers():
    vals = np.arange(-127, 128)
    pad = np.zeros(-len(vals) % 32, dtype=np.int64)
    q = np.concatenate([vals, pad]).reshape(-1, 32)
    raw = b"".join(_q8_block(0x3C00, row) for row in q)           # d = 1.0
    w = codec.q8_0_decode(raw, q.shape[0], 32)
    assert np.array_equal(w, q.astype(np.float32))
    # d = -2.0 (0xC000), max fp16 (0x7BFF = 65504), smallest subnormal (0x0001 = 2^-24)
    for bits, dval in ((0xC000, -2.0), (0x7BFF, 65504.0), (0x0001, 2.0 ** -24)):
        w = codec.q8_0_decode(_q8_block(bits, q[1]), 1, 32)
        assert np.array_equal(w[0], (q[1] * dval).astype(np.float32))


def test_q4_known_answers():
    nib = np.array(list(range(16)) + list(range(15, -1, -1)))
    w = codec.q4_0_decode(_q4_block(0x3C00, nib), 1, 32)[0]
    # byte j: low nibble -> weight j, high nibble -> weight j + 16
    assert np.array_equal(w, (nib - 8).astype(np.float32))
    # negative scale (clipped-MSE ratios are signed): d = -0.5
    w = codec.q4_0_decode(_q4_block(0xB800, nib), 1, 32)[0]
    assert np.array_equal(w, ((nib - 8) * -0.5).astype(np.float32))
    # a block stored as raw bytes 0x10 (low 0, high 1) decodes to -8 / -7
    raw = struct.pack("<H", 0x3C00) + bytes([0x10] * 16)
    w = codec.q4_0_decode(raw, 1, 32)[0]
    assert np.array_equal(w, np.array([-8.0] * 16 + [-7.0] * 16, dtype=np.float32))


def test_quantizer_roundtrip_bounds():
    rng = np.random.default_rng(0)
    w = rng.standard_normal((8, 256)).astype(np.float32) * 0.05
    dq8 = codec.q8_0_decode(vlt3.quantize_q8_0(w), 8, 256)
    d = np.abs(w.reshape(-1, 32)).max(axis=1) / 127.0
    # q is rounded against the fp32 scale, the stored scale is fp16: |err| <= d/2 + 127 |d16 - d|
    d16 = d.astype(np.float16).astype(np.float64)
    bound = d * 0.5 + 127.0 * np.abs(d16 - d)
    assert np.all(np.abs(dq8 - w).reshape(-1, 32) <= bound[:, None] * (1 + 1e-3) + 1e-9)
    dq4 = codec.q4_0_decode(vlt3.quantize_q4_0(w), 8, 256)
    # clipped-MSE Q4_0: per-block error never worse than the plain amax/8 scale choice
    err4 = np.square(dq4 - w).reshape(-1, 32).sum(axis=1)
    amax = w.reshape(-1, 32)[np.arange(64), np.abs(w.reshape(-1, 32)).argmax(axis=1)]
    dd = (amax / -8.0).astype(np.float16).astype(np.float32)
    n = np.clip(np.rint(w.reshape(-1, 32) / dd[:, None] + 8), 0, 15)
    base = np.square((n - 8) * dd[:, None] - w.reshape(-1, 32)).sum(axis=1)
    assert np.all(err4 <= base * (1 + 1e-6) + 1e-12)


@pytest.mark.parametrize("rows,cols,q8,q4", [
    (1536, 1536, 2506752, 1327104), (256, 1536, 417792, 221184), (8960, 1536, 14622720, 7741440),
    (1536, 8960, 14622720, 7741440), (151665, 1536, 247517280, 131038560)])
def test_benchmark_shape_bytes(rows, cols, q8, q4):
    assert codec.nbytes(codec.Q8_0, rows, cols) == q8
    assert codec.nbytes(codec.Q4_0, rows, cols) == q4


def test_synthetic_blocks_ranges():
    rng = np.random.default_rng(1)
    raw8 = np.frombuffer(vlt3.synthetic_blocks(codec.Q8_0, 4, 64, rng), dtype=np.uint8).reshape(-1, 34)
    q = raw8[:, 2:].view(np.int8)
    assert q.min() >= -127 and q.max() <= 127
    d = raw8[:, :2].copy().view(np.float16).astype(np.float32)
    assert np.all(d >= 0) and np.all(d < 0.02 * 8 / 127)


def test_bf16_f16_element_decode_known_answers():
    """BF16: the 16 bits on top of a zero mantissa tail (runtime/vault3.c:517-525); F16: IEEE half.
    Known answers, subnormals, and the writer's round-to-nearest-even BF16 encode against torch's cast."""
    import torch
    from vault_amd import vlt3
    bits = np.array([0x3F80, 0xC000, 0x0001, 0x8000, 0x7F7F, 0x3E4C], dtype="<u2")
    got = codec.decode(codec.BF16, bits.tobytes(), 1, 6)[0]
    want = np.array([1.0, -2.0, 2.0 ** -133, -0.0, 3.3895313892515355e38, 0.19921875], dtype=np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    h = np.array([0x3C00, 0xC000, 0x0001, 0x7BFF, 0x3555, 0x8400], dtype="<u2")
    got = codec.decode(codec.F16, h.tobytes(), 1, 6)[0]
    assert np.array_equal(got, h.view(np.float16).astype(np.float32))
    x = np.random.default_rng(0).standard_normal(4096).astype(np.float32) * 0.05
    enc = np.frombuffer(vlt3.quantize(vlt3.BF16, x), dtype="<u2")
    assert np.array_equal(enc, torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
