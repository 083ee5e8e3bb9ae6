"""VLT3 loader: round trip of the writer, and rejection of the reference's corrupt-file cases
(tests/test_vlt3_runtime.py:141-218) with the same error class as the reference loader
(runtime/vault3.c:273-455, compiled into oracle/_ref).  The NaN / Inf cases run on the device
scan (tests/test_gpu_tokens.py)."""
import os
import struct
import tempfile
import zlib

import numpy as np
import pytest

from oracle import ref
from tests import modelgen
from vault_amd import vlt3
from vault_amd.config import VAULTv3Config
from vault_amd.tokens import TokenTable


@pytest.fixture(scope="module")
def image():
    cfg = modelgen.tiny_cfg(n_layers=8, seg_layers=(2, 4, 6))
    vocab = modelgen.test_vocab(cfg)
    tensors, img, _ = modelgen.build(cfg, "q4_0", seed=2, vocab=vocab)
    return cfg, tensors, img, vocab


def test_round_trip(image):
    cfg, tensors, img, vocab = image
    vf = vlt3.parse_vlt3(img)
    got = VAULTv3Config.from_vlt3_header(vf.header)
    for k in ("vocab_size", "d_model", "n_layers", "n_heads", "n_kv_heads", "head_dim", "d_ff", "window", "n_sink",
              "seg_budget", "seg_hidden", "seg_min", "seg_max", "seg_layers", "im_start_id", "im_end_id"):
        assert getattr(got, k) == getattr(cfg, k), k
    assert got.rms_eps == np.float32(cfg.rms_eps) and got.rope_theta == np.float32(cfg.rope_theta)
    assert set(vf.tensors) == set(tensors)
    for n, t in tensors.items():
        u = vf.tensors[n]
        assert (u.dtype, u.shape, u.data) == (t.dtype, t.shape, t.data), n
    assert isinstance(vf.tokens, TokenTable) and vf.tokens.tokens == vocab[0]
    assert vf.tokens.newline_id == modelgen.NEWLINE_ID
    with tempfile.TemporaryDirectory() as td:
        p = os.path.join(td, "m.vlt3")
        with open(p, "wb") as f:
            f.write(img)
        assert set(vlt3.read_vlt3(p).tensors) == set(tensors)


def _hdr_crc(b: bytearray) -> None:
    struct.pack_into("<I", b, 4092, zlib.crc32(bytes(b[:4092])))


def corrupt_cases(raw: bytes):
    """(name, bytes, verify_crc) of tests/test_vlt3_runtime.py:150-196 (cases 1-8 and 11); the
    reference expects every one rejected."""
    cases = []
    b = bytearray(raw); b[0:4] = b"BAD!"; cases.append(("bad_magic", b, True))
    b = bytearray(raw); b[80] ^= 0xFF; cases.append(("bad_hdr_crc", b, True))
    cases.append(("truncated", bytearray(raw[:-128]), True))
    b = bytearray(raw); struct.pack_into("<Q", b, 32, len(raw) + 4096); _hdr_crc(b)
    cases.append(("oob_dir_off", b, True))
    dir_off = struct.unpack_from("<Q", raw, 32)[0]
    t0_off = struct.unpack_from("<Q", raw, dir_off + 32)[0]
    b = bytearray(raw); struct.pack_into("<Q", b, dir_off + 32, t0_off + 8); cases.append(("unaligned_tensor", b, True))
    b = bytearray(raw); struct.pack_into("<Q", b, dir_off + 40, len(raw) * 2); cases.append(("oob_tensor_size", b, True))
    b = bytearray(raw); b[t0_off + 4] ^= 0x55; cases.append(("corrupt_tensor_crc", b, True))
    b = bytearray(raw)
    struct.pack_into("<I", b, 84, 65536)
    struct.pack_into("<I", b, 92, 65536)
    struct.pack_into("<I", b, 100, 65536)
    _hdr_crc(b)
    cases.append(("u32_hd_overflow", b, True))
    b = bytearray(raw); struct.pack_into("<I", b, 112, 3); _hdr_crc(b)
    cases.append(("nonzero_legacy_nbanks", b, False))
    return cases


def test_corrupt_files_rejected(image):
    _, _, img, _ = image
    for name, data, verify in corrupt_cases(img):
        with pytest.raises(vlt3.VLT3Error) as ei:
            vlt3.parse_vlt3(bytes(data), check_crc=verify)
        assert getattr(ei.value, "code", None) is not None, name


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built")
def test_corrupt_files_same_error_class_as_reference(image):
    _, _, img, _ = image
    for name, data, verify in corrupt_cases(img):
        with pytest.raises(vlt3.VLT3Error) as ei:
            vlt3.parse_vlt3(bytes(data), check_crc=verify)
        with pytest.raises(RuntimeError) as er:
            ref.RefRuntime(bytes(data), threads=1, verify=verify)
        assert ei.value.code == er.value.code, (name, ei.value.code, er.value.code)
    ref.RefRuntime(img, threads=1)       # the uncorrupted file loads in both


def test_bad_vtok_rejected(image):
    _, _, img, _ = image
    b = bytearray(img)
    tok_off = struct.unpack_from("<Q", b, 48)[0]
    b[tok_off:tok_off + 4] = b"XTOK"
    with pytest.raises(vlt3.VLT3Error) as ei:
        vlt3.parse_vlt3(bytes(b), check_crc=False)
    assert ei.value.code == vlt3.E_TOKENIZER
