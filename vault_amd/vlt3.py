"""VLT3 container and GGML-layout Q8_0 / Q4_0 block quantizers.

The byte layout is fixed by the format (docs/VAULT_v3_SPEC.md:105-149; tools/vlt3.py:22-99,
333-404, 453-545), so field order, offsets and block layouts here are necessarily the same;
the code is written from the spec.

* ``quantize_q8_0``: ``d = amax/127`` stored as fp16, ``q = clip(rint(w / d), -127, 127)``
  (tools/vlt3.py:102-111).
* ``quantize_q4_0``: clipped-MSE search over 8 signed scale ratios per 32-weight block,
  nibble ``n = clip(rint(w / d + 8), 0, 15)``; weight ``j`` in the low nibble of byte ``j``,
  weight ``j + 16`` in the high nibble (tools/vlt3.py:119-149).
* ``synthetic_q8_0_blocks`` / ``synthetic_q4_0_blocks``: blocks drawn directly in quantized
  form (int8 uniform[-127,127] / int4 uniform[-8,7], scales ``|N(0,0.02)|/127`` in fp16), the
  synthetic weight recipe of the 1.54B benchmark workloads.
* ``choose_dtype``: the hybrid Q4_0 policy (tools/vlt3.py:312-330): embeddings, every k/v
  projection and the q/o projections of layers {0, 1, L-2, L-1} stay Q8_0.
* ``write_vlt3`` / ``read_vlt3``: header (4096 B, CRC32 over bytes 0..4091), 128-byte
  directory entries, 64-byte aligned payloads, and a VTOK tokenizer blob.  ``minimal_vtok``
  emits a structurally valid VTOK with empty token strings (the offline configuration in which
  every segment-break tier is 0).
"""
from __future__ import annotations

import struct
import zlib
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

MAGIC = b"VLT3"
VERSION = 1
HEADER_SIZE = 4096
ENTRY_SIZE = 128
ALIGN = 64
ENDIAN_TAG = 0x01020304
QK = 32

F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 8, 9
BLOCK_BYTES = {Q8_0: 34, Q4_0: 18}

GLOBAL_IDS = {
    "embed_tokens.weight": 1,
    "norm.weight": 2,
    "seg_scorer.ln.weight": 4,
    "seg_scorer.ln.bias": 5,
    "seg_scorer.fc1.weight": 6,
    "seg_scorer.fc1.bias": 7,
    "seg_scorer.fc2.weight": 8,
    "seg_scorer.fc2.bias": 9,
}
GLOBAL_NAMES = {v: k for k, v in GLOBAL_IDS.items()}
LAYER_KINDS = (
    "input_layernorm.weight",
    "self_attn.q_proj.weight", "self_attn.q_proj.bias",
    "self_attn.k_proj.weight", "self_attn.k_proj.bias",
    "self_attn.v_proj.weight", "self_attn.v_proj.bias",
    "self_attn.o_proj.weight",
    "post_attention_layernorm.weight",
    "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
)
PROJ_KINDS = {
    "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
    "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight",
}


class VLT3Error(ValueError):
    pass


def tensor_id(name: str) -> int:
    if name in GLOBAL_IDS:
        return GLOBAL_IDS[name]
    if not name.startswith("layers."):
        raise VLT3Error(f"unknown tensor {name}")
    _, li, kind = name.split(".", 2)
    return ((int(li) + 1) << 8) | (LAYER_KINDS.index(kind) + 1)


def tensor_name(tid: int) -> str:
    if tid < 256:
        return GLOBAL_NAMES[tid]
    return f"layers.{(tid >> 8) - 1}.{LAYER_KINDS[(tid & 0xFF) - 1]}"


# ----------------------------------------------------------------------------------------
# quantizers
# ----------------------------------------------------------------------------------------

def _pack_blocks(d16: np.ndarray, payload: np.ndarray) -> np.ndarray:
    """d16: (nblk,) float16, payload: (nblk, P) uint8 -> (nblk, 2 + P) uint8."""
    n = d16.shape[0]
    out = np.empty((n, 2 + payload.shape[1]), dtype=np.uint8)
    out[:, :2] = d16.astype("<f2").view(np.uint8).reshape(n, 2)
    out[:, 2:] = payload
    return out


def quantize_q8_0(w: np.ndarray) -> bytes:
    x = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, QK)
    amax = np.max(np.abs(x), axis=1)
    d = amax / np.float32(127.0)
    safe = np.where(d > 0, d, np.float32(1.0))
    inv = np.where(d > 0, np.float32(1.0) / safe, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint(x * inv[:, None]), -127, 127).astype(np.int8)
    return _pack_blocks(d.astype(np.float16), q.view(np.uint8)).tobytes()


_Q4_RATIOS = np.array(
    [-1.0 / 8.0, -0.98 / 8.0, -0.96 / 8.0, -0.94 / 8.0, -0.92 / 8.0, -0.89 / 8.0, 1.0 / 7.5, 0.96 / 7.5],
    dtype=np.float32,
)


def quantize_q4_0(w: np.ndarray) -> bytes:
    x = np.ascontiguousarray(w, dtype=np.float32).reshape(-1, QK)
    nblk = x.shape[0]
    d_out = np.zeros(nblk, dtype=np.float16)
    n_out = np.full((nblk, QK), 8, dtype=np.uint8)
    step = 1 << 18
    for s0 in range(0, nblk, step):
        xb = x[s0:s0 + step]
        m = xb.shape[0]
        peak = xb[np.arange(m), np.argmax(np.abs(xb), axis=1)]
        best = np.full(m, np.inf, dtype=np.float32)
        nz = peak != 0.0
        for r in _Q4_RATIOS:
            d16 = (peak * r).astype(np.float16)
            d32 = d16.astype(np.float32)
            safe = np.where(d32 != 0.0, d32, np.float32(1.0))
            inv = np.where(d32 != 0.0, np.float32(1.0) / safe, np.float32(0.0)).astype(np.float32)
            n = np.clip(np.rint(xb * inv[:, None] + np.float32(8.0)), 0.0, 15.0).astype(np.uint8)
            err = np.square((n.astype(np.float32) - np.float32(8.0)) * d32[:, None] - xb).sum(axis=1)
            take = nz & (err < best)
            best[take] = err[take]
            d_out[s0:s0 + step][take] = d16[take]
            n_out[s0:s0 + step][take] = n[take]
    packed = n_out[:, :16] | (n_out[:, 16:] << 4)
    return _pack_blocks(d_out, packed).tobytes()


def quantize(dtype: int, w: np.ndarray) -> bytes:
    w = np.asarray(w, dtype=np.float32)
    if dtype == Q8_0:
        return quantize_q8_0(w)
    if dtype == Q4_0:
        return quantize_q4_0(w)
    if dtype == F32:
        return w.astype("<f4").tobytes()
    if dtype == F16:
        return w.astype("<f2").tobytes()
    if dtype == BF16:
        u = w.astype(np.float32).view(np.uint32)
        # round to nearest even, as torch's float -> bfloat16 cast
        r = ((u >> 16) & 1) + 0x7FFF
        return ((u + r) >> 16).astype("<u2").tobytes()
    raise VLT3Error(f"dtype {dtype}")


def synthetic_blocks(dtype: int, rows: int, cols: int, rng: np.random.Generator) -> bytes:
    """Quantized blocks drawn directly: int8 U[-127,127] / int4 U[-8,7] (nibble q+8) and
    fp16 scales |N(0, 0.02)| / 127."""
    if cols % QK:
        raise VLT3Error("cols must be a multiple of 32")
    nblk = rows * (cols // QK)
    d = (np.abs(rng.standard_normal(nblk, dtype=np.float32)) * np.float32(0.02 / 127.0)).astype(np.float16)
    if dtype == Q8_0:
        q = rng.integers(-127, 128, size=(nblk, QK), dtype=np.int8).view(np.uint8)
        return _pack_blocks(d, q).tobytes()
    if dtype == Q4_0:
        # 16 uniform bytes per block = 32 independent uniform nibbles (q + 8 in [0, 15])
        qs = np.frombuffer(rng.bytes(nblk * 16), dtype=np.uint8).reshape(nblk, 16)
        return _pack_blocks(d, qs).tobytes()
    raise VLT3Error(f"dtype {dtype}")


def nbytes_for(dtype: int, n: int) -> int:
    if dtype == F32:
        return 4 * n
    if dtype in (F16, BF16):
        return 2 * n
    if dtype in BLOCK_BYTES:
        if n % QK:
            raise VLT3Error("block dtype needs a multiple of 32 elements")
        return n // QK * BLOCK_BYTES[dtype]
    raise VLT3Error(f"dtype {dtype}")


def choose_dtype(name: str, fmt: str, n_layers: int = 0) -> int:
    """Hybrid policy (tools/vlt3.py:312-330)."""
    if fmt == "f32":
        return F32
    per_fmt = {"bf16": BF16, "q8_0": Q8_0, "q4_0": Q4_0}[fmt]
    if name == "embed_tokens.weight":
        return Q8_0 if fmt == "q4_0" else per_fmt
    if name.startswith("layers."):
        _, li_s, kind = name.split(".", 2)
        li = int(li_s)
    else:
        li, kind = -1, name
    if kind not in PROJ_KINDS:
        return F32
    if fmt == "q4_0":
        if kind in ("self_attn.k_proj.weight", "self_attn.v_proj.weight"):
            return Q8_0
        if n_layers >= 8 and li in (0, 1, n_layers - 2, n_layers - 1) and kind in (
                "self_attn.q_proj.weight", "self_attn.o_proj.weight"):
            return Q8_0
    return per_fmt


# ----------------------------------------------------------------------------------------
# container
# ----------------------------------------------------------------------------------------

# Header field layout: docs/VAULT_v3_SPEC.md:111-136 (offsets are part of the format).
_HDR = struct.Struct("<4sIIIQIIQQQQQQ8I10I3f5I2I64sI5I4I")
assert _HDR.size == 296
_ENTRY = struct.Struct("<III4IIQQI12x64s")
assert _ENTRY.size == ENTRY_SIZE


def minimal_vtok(n_vocab: int) -> bytes:
    """Structurally valid VTOK blob: every token string empty, no merges/specials/ranges,
    every raw byte mapped to token 0 (runtime/vault3.c:427-453 checks)."""
    head = 128
    o_tab = head
    o_pool = o_tab + 8 * n_vocab
    o_mer = o_pool
    o_spc = o_mer
    o_rng = o_spc
    o_byt = o_rng
    size = o_byt + 256 * 4
    blob = bytearray(size)
    struct.pack_into("<4sIIIIII6Q", blob, 0, b"VTOK", 1, n_vocab, 0, 0, 0, 0,
                     o_tab, o_pool, o_mer, o_spc, o_rng, o_byt)
    return bytes(blob)


@dataclass
class Tensor:
    name: str
    dtype: int
    shape: Tuple[int, ...]
    data: bytes


@dataclass
class VLT3:
    header: Dict
    tensors: Dict[str, Tensor] = field(default_factory=dict)


def write_vlt3(path: str, tensors: List[Tensor], cfg, fmt_tag: int, tok_blob: Optional[bytes] = None,
               special_ids: Optional[Dict[str, int]] = None, model_name: str = "VAULT-v3") -> int:
    """Write a VLT3 file from already-encoded tensors; returns the file size."""
    tensors = sorted(tensors, key=lambda t: tensor_id(t.name))
    tok_blob = tok_blob if tok_blob is not None else minimal_vtok(cfg.vocab_size)
    ids = dict(bos=0, eos=0, im_start=0, im_end=0, pad=0)
    if special_ids:
        ids.update(special_ids)
    dir_off = HEADER_SIZE
    dir_size = ENTRY_SIZE * len(tensors)
    tok_off = -(-(dir_off + dir_size) // ALIGN) * ALIGN
    data_off = -(-(tok_off + len(tok_blob)) // ALIGN) * ALIGN
    offs = []
    cur = data_off
    for t in tensors:
        cur = -(-cur // ALIGN) * ALIGN
        if len(t.data) != nbytes_for(t.dtype, int(np.prod(t.shape))):
            raise VLT3Error(f"{t.name}: payload size mismatch")
        offs.append(cur)
        cur += len(t.data)
    file_size = cur
    names = {t.name for t in tensors}
    seg_layers = list(getattr(cfg, "seg_layers", ()) or ())
    has_sc = bool(seg_layers) and "seg_scorer.ln.weight" in names
    nf = len(seg_layers) if has_sc else 0
    seg_layers4 = (seg_layers + [0, 0, 0, 0])[:4]
    flags = (1 if getattr(cfg, "tie_embeddings", True) else 0) | (4 if nf else 0) | 2
    hdr = _HDR.pack(
        MAGIC, VERSION, HEADER_SIZE, ENDIAN_TAG, file_size, ALIGN, len(tensors),
        dir_off, dir_size, tok_off, len(tok_blob), data_off, file_size - data_off,
        cfg.vocab_size, cfg.d_model, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.d_ff, cfg.window,
        *([0] * 10),
        float(cfg.rms_eps), float(cfg.rope_theta), 0.0,
        ids["bos"], ids["eos"], ids["im_start"], ids["im_end"], ids["pad"],
        fmt_tag, flags, model_name.encode()[:63],
        int(cfg.n_sink),
        int(cfg.seg_budget) if nf else 0, int(cfg.seg_hidden) if nf else 0,
        int(cfg.seg_min) if nf else 0, int(cfg.seg_max) if nf else 0, nf,
        *seg_layers4,
    ).ljust(HEADER_SIZE - 4, b"\0")
    hdr += struct.pack("<I", zlib.crc32(hdr))
    with open(path, "wb") as f:
        f.write(hdr)
        for t, off in zip(tensors, offs):
            dims = list(t.shape) + [1] * (4 - len(t.shape))
            f.write(_ENTRY.pack(tensor_id(t.name), t.dtype, len(t.shape), *dims, 0, off, len(t.data),
                                zlib.crc32(t.data), t.name.encode()[:63]))
        f.write(b"\0" * (tok_off - f.tell()))
        f.write(tok_blob)
        for t, off in zip(tensors, offs):
            f.write(b"\0" * (off - f.tell()))
            f.write(t.data)
        assert f.tell() == file_size
    return file_size


_HDR_NAMES = (
    ["magic", "version", "header_size", "endian_tag", "file_size", "alignment", "n_tensors",
     "tensor_dir_offset", "tensor_dir_size", "tokenizer_offset", "tokenizer_size", "data_offset", "data_size",
     "vocab_size", "d_model", "n_layers", "n_heads", "n_kv_heads", "head_dim", "d_ff", "window"]
    + [f"kenyon{i}" for i in range(10)]
    + ["rms_eps", "rope_theta", "reserved_eps", "bos_id", "eos_id", "im_start_id", "im_end_id", "pad_id",
       "weight_format", "flags", "model_name", "n_sink",
       "seg_budget", "seg_hidden", "seg_min", "seg_max", "seg_n_feat"]
    + [f"seg_layer{i}" for i in range(4)]
)


def read_vlt3(path: str, check_crc: bool = True) -> VLT3:
    """Parse and validate a VLT3 file (validation rules: docs/VAULT_v3_SPEC.md:111-136,
    tools/vlt3.py:453-545)."""
    with open(path, "rb") as f:
        buf = f.read()
    size = len(buf)
    if size < HEADER_SIZE:
        raise VLT3Error("file smaller than header")
    if zlib.crc32(buf[:HEADER_SIZE - 4]) != struct.unpack_from("<I", buf, HEADER_SIZE - 4)[0]:
        raise VLT3Error("header CRC mismatch")
    h = dict(zip(_HDR_NAMES, _HDR.unpack_from(buf, 0)))
    if h["magic"] != MAGIC or h["version"] != VERSION or h["header_size"] != HEADER_SIZE or h["endian_tag"] != ENDIAN_TAG:
        raise VLT3Error("bad magic/version/header size/endianness")
    if h["file_size"] != size or h["alignment"] != ALIGN:
        raise VLT3Error("file size or alignment mismatch")
    for off_k, size_k in (("tensor_dir_offset", "tensor_dir_size"), ("tokenizer_offset", "tokenizer_size"),
                          ("data_offset", "data_size")):
        o, n = h[off_k], h[size_k]
        if o < HEADER_SIZE or o > size or n > size - o:
            raise VLT3Error(f"{off_k} out of bounds")
    if h["tensor_dir_size"] != h["n_tensors"] * ENTRY_SIZE:
        raise VLT3Error("tensor directory size mismatch")
    if any(h[f"kenyon{i}"] for i in range(10)):
        raise VLT3Error("legacy bank fields must be zero")
    if h["n_heads"] % max(1, h["n_kv_heads"]) or h["n_heads"] * h["head_dim"] != h["d_model"]:
        raise VLT3Error("inconsistent head dimensions")
    if not (np.isfinite(h["rms_eps"]) and h["rms_eps"] > 0 and np.isfinite(h["rope_theta"]) and h["rope_theta"] > 1):
        raise VLT3Error("bad eps/theta")
    out = VLT3(header=h)
    prev_end = 0
    for k in range(h["n_tensors"]):
        e = _ENTRY.unpack_from(buf, h["tensor_dir_offset"] + k * ENTRY_SIZE)
        tid, dt, ndim, d0, d1, d2, d3, rsv, off, nb, crc, nm = e
        if rsv or not 1 <= ndim <= 4:
            raise VLT3Error(f"entry {k}: bad reserved/ndim")
        shape = tuple((d0, d1, d2, d3)[:ndim])
        n = int(np.prod(shape))
        if nb != nbytes_for(dt, n):
            raise VLT3Error(f"tensor {tid}: size mismatch")
        if off % ALIGN or off < h["data_offset"] or nb > h["data_offset"] + h["data_size"] - off or off < prev_end:
            raise VLT3Error(f"tensor {tid}: bad offset")
        prev_end = off + nb
        data = buf[off:off + nb]
        if check_crc and zlib.crc32(data) != crc:
            raise VLT3Error(f"tensor {tid}: CRC mismatch")
        name = tensor_name(tid)
        out.tensors[name] = Tensor(name, dt, shape, data)
    return out
