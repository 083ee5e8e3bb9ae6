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
  every segment-break tier is 0); ``vault_amd.tokens.build_vtok`` one with token strings.
  ``read_vlt3`` also parses the VTOK blob into a ``TokenTable`` and ``scan_finite`` applies the
  reference loader's NaN / Inf rejection (runtime/vault3.c:215-271) on the host.
"""
from __future__ import annotations

import struct
import zlib
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import numpy as np

from .tokens import TokenTable, VTOKError

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
    tokens: Optional[TokenTable] = None


def write_vlt3(path: str, tensors: List[Tensor], cfg, fmt_tag: int, tok_blob: Optional[bytes] = None,
               special_ids: Optional[Dict[str, int]] = None, model_name: str = "VAULT-v3") -> int:
    """Write a VLT3 file from already-encoded tensors; returns the file size."""
    tensors = sorted(tensors, key=lambda t: tensor_id(t.name))
    tok_blob = tok_blob if tok_blob is not None else minimal_vtok(cfg.vocab_size)
    # the ChatML ids the auto-pin rule reads come from the config unless given explicitly
    ids = dict(bos=0, eos=0, im_start=int(cfg.im_start_id), im_end=int(cfg.im_end_id), pad=0)
    if special_ids:
        ids.update(special_ids)
    if not all(0 <= v < cfg.vocab_size for v in ids.values()):
        raise VLT3Error("special token ids must be below vocab_size")
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


# Loader limits and error codes (runtime/vault3.h:26-48): a rejected file raises VLT3Error whose
# ``code`` is the reference loader's V3_E_* value for the same defect.
E_SIZE, E_MAGIC, E_CRC, E_BOUNDS, E_DTYPE, E_MISSING, E_SHAPE, E_TOKENIZER, E_LIMIT, E_NAN = \
    -1, -2, -3, -4, -5, -6, -7, -9, -10, -12
MAX_LAYERS, MAX_HEADS, MAX_HEAD_DIM, MAX_SINK, MAX_SEG_FEAT, MAX_SEG_HIDDEN, MAX_SEG_BUDGET = \
    64, 256, 256, 512, 4, 1024, 16384


def _fail(code: int, msg: str):
    e = VLT3Error(msg)
    e.code = code
    raise e


def read_vlt3(path: str, check_crc: bool = True) -> VLT3:
    """Parse and validate a VLT3 file; see ``parse_vlt3``."""
    with open(path, "rb") as f:
        buf = f.read()
    return parse_vlt3(buf, check_crc)


def parse_vlt3(buf: bytes, check_crc: bool = True) -> VLT3:
    """Validate a VLT3 image in the order of the reference loader (runtime/vault3.c:273-455):
    header magic / version / size / endianness, header CRC, file size, alignment, region bounds,
    legacy fields, hyper-parameter limits, directory entries (reserved word, ndim, dims, dtype size,
    block shape, alignment and bounds, ascending offsets, optional CRC), tensor ids (missing or
    duplicated), shapes and dtypes, then the VTOK blob.  Non-finite weights are rejected where the
    weights are uploaded (``ModelWeights.from_tensors`` scans them on the device)."""
    size = len(buf)
    if size < HEADER_SIZE:
        _fail(E_SIZE, "file smaller than header")
    if buf[:4] != MAGIC or struct.unpack_from("<III", buf, 4) != (VERSION, HEADER_SIZE, ENDIAN_TAG):
        _fail(E_MAGIC, "bad magic/version/header size/endianness")
    if zlib.crc32(buf[:HEADER_SIZE - 4]) != struct.unpack_from("<I", buf, HEADER_SIZE - 4)[0]:
        _fail(E_CRC, "header CRC mismatch")
    h = dict(zip(_HDR_NAMES, _HDR.unpack_from(buf, 0)))
    if h["file_size"] != size:
        _fail(E_SIZE, "file size mismatch")
    if h["alignment"] != ALIGN:
        _fail(E_MAGIC, "alignment mismatch")
    for off_k, size_k in (("tensor_dir_offset", "tensor_dir_size"), ("tokenizer_offset", "tokenizer_size"),
                          ("data_offset", "data_size")):
        o, n = h[off_k], h[size_k]
        if o < HEADER_SIZE or o > size or n > size - o:
            _fail(E_BOUNDS, f"{off_k} out of bounds")
    if h["n_tensors"] > 8192 or h["tensor_dir_size"] != h["n_tensors"] * ENTRY_SIZE:
        _fail(E_BOUNDS, "tensor directory size mismatch")
    if any(h[f"kenyon{i}"] for i in range(10)):
        _fail(E_LIMIT, "legacy bank fields must be zero")
    if not np.isfinite(h["reserved_eps"]):
        _fail(E_NAN, "non-finite reserved field")
    V, d, nl, H, G, D, F, W = (h[k] for k in ("vocab_size", "d_model", "n_layers", "n_heads", "n_kv_heads",
                                              "head_dim", "d_ff", "window"))
    if (V == 0 or V > 524288 or d == 0 or d > 16384 or nl == 0 or nl > MAX_LAYERS or H == 0 or H > MAX_HEADS
            or D == 0 or D > MAX_HEAD_DIM or D % 2 or G == 0 or G > H or H % G or F == 0 or F > 65536
            or W == 0 or W > 65536 or h["n_sink"] > MAX_SINK or h["n_sink"] > W):
        _fail(E_LIMIT, "hyper-parameter out of range")
    if H * D != d:
        _fail(E_SHAPE, "n_heads * head_dim != d_model")
    if not (np.isfinite(h["rope_theta"]) and np.isfinite(h["rms_eps"])):
        _fail(E_NAN, "non-finite eps / theta")
    if not (h["rope_theta"] > 1.0 and h["rms_eps"] > 0.0):
        _fail(E_LIMIT, "bad eps / theta")
    if any(h[k] >= V for k in ("bos_id", "eos_id", "im_start_id", "im_end_id", "pad_id")):
        _fail(E_LIMIT, "special token id beyond the vocabulary")
    nf = h["seg_n_feat"]
    if nf > MAX_SEG_FEAT:
        _fail(E_LIMIT, "too many scorer feature layers")
    if nf == 0:
        if h["seg_budget"] or h["seg_hidden"] or h["seg_min"] or h["seg_max"]:
            _fail(E_LIMIT, "segment fields set without a scorer")
    elif (h["seg_budget"] > MAX_SEG_BUDGET or h["seg_hidden"] == 0 or h["seg_hidden"] > MAX_SEG_HIDDEN
          or h["seg_min"] == 0 or h["seg_min"] > h["seg_max"] or h["seg_max"] > W
          or any(h[f"seg_layer{i}"] >= nl for i in range(nf))):
        _fail(E_LIMIT, "segment hyper-parameters out of range")
    out = VLT3(header=h)
    prev_end = 0
    d_end = h["data_offset"] + h["data_size"]
    for k in range(h["n_tensors"]):
        tid, dt, ndim, d0, d1, d2, d3, rsv, off, nb, crc, _ = \
            _ENTRY.unpack_from(buf, h["tensor_dir_offset"] + k * ENTRY_SIZE)
        if rsv:
            _fail(E_BOUNDS, f"entry {k}: reserved word set")
        if not 1 <= ndim <= 4:
            _fail(E_SHAPE, f"entry {k}: ndim {ndim}")
        shape = tuple((d0, d1, d2, d3)[:ndim])
        if any(x == 0 for x in shape):
            _fail(E_SHAPE, f"entry {k}: zero dimension")
        n = int(np.prod(shape, dtype=object))
        if dt not in (F32, F16, BF16, Q8_0, Q4_0):
            _fail(E_DTYPE, f"entry {k}: dtype {dt}")
        if dt in BLOCK_BYTES and shape[-1] % QK:
            _fail(E_SHAPE, f"entry {k}: block dtype needs rows of a multiple of 32")
        if nb != nbytes_for(dt, n):
            _fail(E_SHAPE, f"tensor {tid}: size mismatch")
        if off % ALIGN or off < h["data_offset"] or nb > d_end - off:
            _fail(E_BOUNDS, f"tensor {tid}: bad offset")
        if off < prev_end:
            _fail(E_BOUNDS, f"tensor {tid}: overlaps the previous tensor")
        prev_end = off + nb
        data = buf[off:off + nb]
        if check_crc and zlib.crc32(data) != crc:
            _fail(E_CRC, f"tensor {tid}: CRC mismatch")
        try:
            name = tensor_name(tid)
        except (KeyError, IndexError, VLT3Error):
            _fail(E_MISSING, f"unknown tensor id {tid}")
        if name.startswith("layers.") and int(name.split(".")[1]) >= nl:
            _fail(E_MISSING, f"tensor {tid}: layer beyond n_layers")
        if name in out.tensors:
            _fail(E_MISSING, f"tensor {tid}: duplicated")
        if name.startswith("seg_scorer.") and nf == 0:
            continue          # the reference ignores scorer tensors of a file without a scorer
        out.tensors[name] = Tensor(name, dt, shape, data)
    cfg_shapes = _expected_shapes(h)
    for name, shp in cfg_shapes.items():
        t = out.tensors.get(name)
        if t is None or t.shape != shp:
            _fail(E_SHAPE, f"{name}: missing or shape {None if t is None else t.shape} != {shp}")
        matmul = name.endswith("_proj.weight") or name in ("embed_tokens.weight", "seg_scorer.fc1.weight",
                                                           "seg_scorer.fc2.weight")
        if not matmul and t.dtype != F32:
            _fail(E_SHAPE, f"{name} must be F32")
    tb = buf[h["tokenizer_offset"]:h["tokenizer_offset"] + h["tokenizer_size"]]
    if len(tb) < 128:
        _fail(E_TOKENIZER, "VTOK blob too small")
    try:
        out.tokens = TokenTable.from_vtok(tb, V)
    except VTOKError as e:
        _fail(E_TOKENIZER, str(e))
    return out


def _expected_shapes(h: Dict) -> Dict[str, tuple]:
    """Tensor shapes the header implies (runtime/vault3.c:383-423)."""
    d, H, G, D, F = h["d_model"], h["n_heads"], h["n_kv_heads"], h["head_dim"], h["d_ff"]
    s = {"embed_tokens.weight": (h["vocab_size"], d), "norm.weight": (d,)}
    nf = h["seg_n_feat"]
    if nf:
        fd, hd = nf * d, h["seg_hidden"]
        s.update({"seg_scorer.ln.weight": (fd,), "seg_scorer.ln.bias": (fd,), "seg_scorer.fc1.weight": (hd, fd),
                  "seg_scorer.fc1.bias": (hd,), "seg_scorer.fc2.weight": (1, hd), "seg_scorer.fc2.bias": (1,)})
    for li in range(h["n_layers"]):
        p = f"layers.{li}."
        s.update({p + "input_layernorm.weight": (d,), p + "post_attention_layernorm.weight": (d,),
                  p + "self_attn.q_proj.weight": (H * D, d), p + "self_attn.k_proj.weight": (G * D, d),
                  p + "self_attn.v_proj.weight": (G * D, d), p + "self_attn.o_proj.weight": (d, H * D),
                  p + "mlp.gate_proj.weight": (F, d), p + "mlp.up_proj.weight": (F, d),
                  p + "mlp.down_proj.weight": (d, F), p + "self_attn.q_proj.bias": (H * D,),
                  p + "self_attn.k_proj.bias": (G * D,), p + "self_attn.v_proj.bias": (G * D,)})
    return s
