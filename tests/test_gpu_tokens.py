"""GPU drop-in loaded from VLT3 files with real token strings: the auto-pin state machine and the
byte-driven segment breaks against the reference C runtime (runtime/vault3.c v3_step, compiled into
oracle/_ref), through both the step stream and the chunk-recurrent prefill; and the device NaN / Inf
scan of the loader (runtime/vault3.c:215-271; tests/test_vlt3_runtime.py:176-196 cases 9-10).

Bars: n_pin and pin_locked exactly at every step, segment-memory slots exactly, logits rel < 1e-4
and 100% top-1 (tests/test_vlt3_runtime.py:90-94); non-finite counts exact."""
import os
import struct
import tempfile
import zlib

import numpy as np
import pytest
import torch

from oracle import ref
from tests import modelgen
from tests.test_oracle_tokens import PIN_CASES, pin_cfg, pin_stream
from vault_amd import ops, vlt3
from vault_amd.model import VAULTv3ForCausalLM
from vault_amd.weights import ModelWeights

pytestmark = pytest.mark.gpu
needs_ref = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")


def _load(image: bytes, dev, check_crc=True):
    with tempfile.TemporaryDirectory() as td:
        p = os.path.join(td, "m.vlt3")
        with open(p, "wb") as f:
            f.write(image)
        return ModelWeights.from_vlt3(p, dev, check_crc=check_crc)


@pytest.fixture(scope="module")
def pin_model(dev):
    cfg = pin_cfg(head_dim=128)
    vocab = modelgen.test_vocab(cfg)
    _, image, _ = modelgen.build(cfg, "q4_0", seed=4, vocab=vocab)
    w = _load(image, dev)
    assert w.tokens is not None and w.tokens.newline_id == modelgen.NEWLINE_ID
    return cfg, image, VAULTv3ForCausalLM(w)


def _rel(a, b):
    return float(np.abs(a - b).max() / np.abs(b).max())


@needs_ref
@pytest.mark.parametrize("case", list(PIN_CASES))
def test_auto_pin_stream_matches_reference_runtime(pin_model, case):
    cfg, image, m = pin_model
    rt = ref.RefRuntime(image, threads=2)
    st = m.new_state(1)
    ids = pin_stream(cfg, case)
    got, want = [], []
    for i, t in enumerate(ids):
        want.append(rt.step(t).astype(np.float64))
        got.append(m.step(torch.tensor([t]), st)[0].double().cpu().numpy())
        assert (rt.info()["n_pin"], rt.flags()["pin_locked"]) == (st.n_pin, st.pin_locked), (case, i)
    got, want = np.stack(got), np.stack(want)
    assert _rel(got, want) < 1e-4
    assert np.array_equal(got.argmax(-1), want.argmax(-1))
    assert np.array_equal(rt.mem_pos(), st.mem_pos.numpy())


@needs_ref
@pytest.mark.parametrize("case,split", [("system_nl", 3), ("system_nl", 9), ("system_nl", 40),
                                        ("system_no_nl", 8), ("past_limit", 17), ("past_limit", 50)])
def test_auto_pin_prefill_matches_reference_runtime(pin_model, case, split):
    """Chunk-recurrent prefill of a ChatML prompt (auto-pin decided on the prompt's first tokens),
    then the step stream: every logit row against the C runtime stepping the same ids."""
    cfg, image, m = pin_model
    rt = ref.RefRuntime(image, threads=2)
    ids = pin_stream(cfg, case, n_tail=60)
    want = np.stack([rt.step(t).astype(np.float64) for t in ids])
    last, st = m.prefill(torch.tensor([ids[:split]]))
    rows = [last[0].double().cpu().numpy()]
    for t in ids[split:]:
        rows.append(m.step(torch.tensor([t]), st)[0].double().cpu().numpy())
    got = np.stack(rows)
    assert _rel(got, want[split - 1:]) < 1e-4
    assert np.array_equal(got.argmax(-1), want[split - 1:].argmax(-1))
    assert st.n_pin == rt.info()["n_pin"] and st.pin_locked
    assert np.array_equal(rt.mem_pos(), st.mem_pos.numpy())


def _nan_cases(raw: bytes):
    """tests/test_vlt3_runtime.py:176-196: a quiet NaN in norm.weight with a valid tensor CRC, and an
    fp16 NaN block scale in the middle of embed_tokens (loaded without CRC checks)."""
    vf = vlt3.parse_vlt3(raw)
    dir_off = vf.header["tensor_dir_offset"]
    ents = {}
    for k in range(vf.header["n_tensors"]):
        eo = dir_off + k * 128
        tid, off, nb = struct.unpack_from("<I", raw, eo)[0], *struct.unpack_from("<QQ", raw, eo + 32)
        ents[tid] = (eo, off, nb)
    out = []
    b = bytearray(raw)
    eo, off, nb = ents[2]
    struct.pack_into("<I", b, off, 0x7FC00000)
    struct.pack_into("<I", b, eo + 48, zlib.crc32(bytes(b[off:off + nb])))
    out.append(("nan_norm_weight", b, True))
    b = bytearray(raw)
    eo, off, nb = ents[1]
    struct.pack_into("<H", b, off + (nb // 34) // 2 * 34, 0x7E00)
    out.append(("nan_q8_midblock_unverified", b, False))
    return out


def test_nonfinite_files_rejected(dev):
    cfg = modelgen.tiny_cfg()
    _, image, _ = modelgen.build(cfg, "q8_0", seed=2, vocab=modelgen.test_vocab(cfg))
    for name, data, verify in _nan_cases(image):
        with pytest.raises(vlt3.VLT3Error) as ei:
            _load(bytes(data), dev, check_crc=verify)
        assert ei.value.code == vlt3.E_NAN, name
        if ref.available():
            with pytest.raises(RuntimeError) as er:
                ref.RefRuntime(bytes(data), threads=1, verify=verify)
            assert er.value.code == vlt3.E_NAN, name
    _load(image, dev)


@pytest.mark.parametrize("dt", [vlt3.F32, vlt3.F16, vlt3.BF16, vlt3.Q8_0, vlt3.Q4_0])
def test_count_nonfinite_exact(dev, dt):
    """Planted Inf / NaN patterns at seeded positions: the device count equals the host count of
    all-ones exponent fields (F32 0x7F800000, F16 0x7C00, BF16 0x7F80; block scales at the head of
    34- / 18-byte blocks); quant bytes that look like NaN halves are not counted."""
    rng = np.random.default_rng(dt)
    n = 32 * 4097
    if dt == vlt3.F32:
        a = rng.standard_normal(n).astype(np.float32).view(np.uint32)
        pos = rng.choice(n, 37, replace=False)
        a[pos] = rng.choice([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001], 37)
        want, data = 37, a.tobytes()
    elif dt in (vlt3.F16, vlt3.BF16):
        a = rng.integers(0, 0x7C00 if dt == vlt3.F16 else 0x7F80, n).astype(np.uint16)
        pos = rng.choice(n, 21, replace=False)
        a[pos] |= np.uint16(0x7C00 if dt == vlt3.F16 else 0x7F80)
        want, data = 21, a.tobytes()
    else:
        bb = 34 if dt == vlt3.Q8_0 else 18
        blk = np.frombuffer(vlt3.synthetic_blocks(dt, 4097, 32, rng), dtype=np.uint8).reshape(-1, bb).copy()
        blk[:, 2:] = 0xFF                                   # quants that read as NaN halves: not scales
        pos = rng.choice(blk.shape[0], 13, replace=False)
        blk[pos, 0], blk[pos, 1] = 0x00, 0x7C               # +Inf scale
        want, data = 13, blk.tobytes()
    assert ops.count_nonfinite([(dt, data, n)], dev) == [want]
