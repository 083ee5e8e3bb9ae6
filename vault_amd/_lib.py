"""ctypes binding of libvault_amd.so (the C ABI declared in include/vault_amd.h).

There is no fallback: if the library is missing or a symbol is absent, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libvault_amd.so")
HEADER = os.path.join(HERE, "..", "include", "vault_amd.h")

VGX_OK = 0
ERRORS = {
    -1: "VGX_E_SIZE", -5: "VGX_E_DTYPE", -7: "VGX_E_SHAPE", -8: "VGX_E_ARENA", -10: "VGX_E_LIMIT",
    -11: "VGX_E_ALIGN", -31: "VGX_E_ARG", -32: "VGX_E_HIP", -33: "VGX_E_STATE",
}

F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 8, 9
EPI_STORE, EPI_ACCUM, EPI_SWIGLU = 0, 1, 2
STEP_SLOT, STEP_TABLE_ROW, STEP_SINK_SLOT, STEP_N_CUR, STEP_WORDS = 0, 1, 2, 3, 4
SEG_MEM_CNT, SEG_ID_OFFSET, SEG_CUR_ID, SEG_LEN, SEG_WORDS = 0, 1, 2, 3, 4
SLOT_STEP, SLOT_FLAGS, SLOT_IDS_ADDR, SLOT_OUT_ADDR, SLOT_IDS = 0, 16, 24, 32, 64
SLOTF_DEVICE_IDS, SLOTF_BIAS = 1, 2

P = C.c_void_p
I32 = C.c_int
I64 = C.c_int64
U32 = C.c_uint32
U64 = C.c_uint64
F = C.c_float

# name -> (restype, argtypes)
_SIGS = {
    "vgx_abi_version": (I32, []),
    "vgx_qweight_packed_bytes": (I64, [I32, I64, I64]),
    "vgx_qweight_scale_offset": (I64, [I32, I64, I64]),
    "vgx_qweight_pack": (I32, [I32, P, P, I64, I64, P]),
    "vgx_qweight_pack_gateup": (I32, [I32, P, P, P, I64, I64, P]),
    "vgx_qweight_pack_rope": (I32, [I32, P, P, I64, I64, I64, I64, P]),
    "vgx_qweight_unpack": (I32, [I32, P, P, I64, I64, P]),
    "vgx_qweight_dequant": (I32, [I32, P, P, I64, I64, P]),
    "vgx_embed_rows": (I32, [I32, P, I64, I64, P, I64, I64, P, I64, P]),
    "vgx_count_nonfinite": (I32, [I32, P, I64, P, P]),
    "vgx_qlinear": (I32, [I32, P, I64, I64, P, I64, I64, P, P, I64, I32, P]),
    "vgx_qlinear_swiglu": (I32, [I32, P, I64, I64, P, I64, I64, P, I64, P]),
    "vgx_qlinear_ex": (I32, [I32, P, I64, I64, P, I64, I64, P, F, P, P, I64, I32, P]),
    "vgx_qlinear_indirect": (I32, [I32, P, I64, I64, P, I64, I64, P, F, P, P, I64, I32, P]),
    "vgx_qlinear_side": (I32, [I32, P, I64, I64, P, I64, I64, P, F, P, P, I64, I32, P, P]),
    "vgx_qgemm_workspace_bytes": (I64, [I64, I64, I64, I32]),
    "vgx_qgemm": (I32, [I32, P, I64, I64, P, I64, I64, P, F, P, P, I64, I32, P, I64, P]),
    "vgx_attn_decode_workspace_bytes": (I64, [I64, I64, I64, I64, I64]),
    "vgx_attn_decode": (I32, [I32, P, I64, P, I32, P, I64, I32, I64, P, I64, I64, I64, I64, F, P, I64, P]),
    "vgx_seg_step": (I32, [P, I64, P, P, I64, P, P, P, I64, I64, I64, I64, P]),
    "vgx_step_slot_bytes": (I64, [I64, I64, I64]),
    "vgx_step_slot_bias_off": (I64, [I64]),
    "vgx_host_alloc": (I32, [I64, C.POINTER(C.c_void_p)]),
    "vgx_host_free": (I32, [P]),
    "vgx_step_begin": (I32, [P, I64, I64, P, P, P, I64, P, P, I64, P, P, P, I64, I64, I64, I64, P, P, I64, I64, I64,
                             P]),
    "vgx_step_begin_embed": (I32, [P, I64, I64, P, P, P, I64, P, P, I64, P, P, P, I64, I64, I64, I64, P, P, I64, I64,
                                   I64, I32, P, I64, I64, P, I64, P]),
    "vgx_seg_evict": (I32, [P, P, P, I64, P, P, P, P, P, I64, I64, I64, P, P, P]),
    "vgx_gather_rows_masked": (I32, [I32, P, P, P, I64, I64, I64, I64, I64, I64, P]),
    "vgx_rope_rotate_dyn": (I32, [I32, P, P, I64, I64, I64, I64, I64, P, I64, P, I64, I32, P]),
    "vgx_argmax": (I32, [P, I64, I64, I64, P, P]),
    "vgx_sample_topk_workspace_bytes": (I64, [I64, I64]),
    "vgx_sample_topk": (I32, [P, I64, I64, I64, I64, F, P, P, P, I64, P]),
    "vgx_topk_workspace_bytes": (I64, [I64, I64, I64]),
    "vgx_topk": (I32, [P, I64, I64, I64, I64, P, P, P, I64, P]),
    "vgx_tokens_create": (P, [P, P, U32]),
    "vgx_tokens_destroy": (None, [P]),
    "vgx_res_create": (P, [P, U32, U32, U32, U32, U32]),
    "vgx_res_destroy": (None, [P]),
    "vgx_res_rebuild": (I32, [P, P, P, U32]),
    "vgx_res_update": (I32, [P, P, P, U32, U64, U32, P, P, P]),
    "vgx_spoof_check": (I32, [P, P, P, U32, U32, U64, U32, U32]),
    "vgx_gov_create": (P, [P, U32, U32, U32]),
    "vgx_gov_destroy": (None, [P]),
    "vgx_gov_reset_stream": (None, [P]),
    "vgx_gov_add_rule": (I32, [P, P, C.c_size_t]),
    "vgx_gov_arm_system": (I32, [P, P, C.c_size_t]),
    "vgx_gov_active": (I32, [P]),
    "vgx_gov_screen": (I32, [P, P, P, U32, U32, U32, P, U32]),
    "vgx_gov_commit": (I32, [P, U32]),
    "vgx_attn_decode_noalloc": (I32, [I32, P, I64, P, I32, P, I64, I32, I64, P, I64, I64, I64, I64, F, P]),
    "vgx_attn_prefill": (I32, [I32, I32, I32, P, I32, I64, I64, I64, F, P]),
    "vgx_attn_prefill_workspace_bytes": (I64, [I64, I64]),
    "vgx_attn_prefill_ws": (I32, [I32, I32, I32, P, I32, I64, I64, I64, F, P, I64, P]),
    "vgx_rmsnorm": (I32, [P, I64, P, P, I64, I64, I64, F, P]),
    "vgx_rope_qkv_write": (I32, [I32, P, I64, P, I64, P, I64, I64, I64, I64, I64, P, I64, P, P, P, I64, I64, P, P, I64,
                                 I64, I64, P]),
    "vgx_rope_rotate": (I32, [I32, P, P, I64, I64, I64, I64, I64, P, I64, P]),
    "vgx_gather_rows": (I32, [I32, P, P, P, I64, I64, I64, I64, I64, I64, P]),
    "vgx_ema_habituate": (I32, [P, I64, P, I64, P, I64, I64, I32, P]),
    "vgx_layernorm": (I32, [P, I64, P, P, P, I64, I64, I64, F, P]),
    "vgx_seg_score_tail": (I32, [P, I64, P, P, I64, I64, I32, P, P, P]),
    "vgx_seg_score_step": (I32, [P, I64, P, I32, P, I64, P, P, P, F, P, P, P, P, P, P]),
    "vgx_rope_qkv_write_step": (I32, [I32, P, I64, P, I64, P, I64, I64, I64, I64, I64, P, I64, P, P, P, P, I64, I64,
                                      I64, P, P, I64, I64, I64, P]),
    "vgx_qkv_rope_step": (I32, [I32, P, P, I32, P, P, I64, I64, I64, I64, P, P, F, P, P, I64, P, P, I32, P, P, P, I64,
                                I64, P, P, I64, I64, P]),
    "vgx_qkv_rope_batch_workspace_bytes": (I64, [I64, I64, I64, I64, I64, I32]),
    "vgx_qkv_rope_batch": (I32, [I32, P, P, I32, P, P, I64, I64, I64, I64, P, I64, I64, P, F, P, I64, P, P, I64, I32,
                                 P, P, P, I64, I64, I64, P, P, I64, I64, I64, P, I64, P]),
}


class KVSpan(C.Structure):
    """vgx_kv_span (include/vault_amd.h)."""
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("len", C.c_int64),
                ("batch_stride", C.c_int64), ("group_stride", C.c_int64), ("dyn_len", C.c_void_p)]


class KVRun(C.Structure):
    """vgx_kv_run (include/vault_amd.h)."""
    _fields_ = [("k", C.c_void_p), ("v", C.c_void_p), ("len", C.c_int64), ("row_stride", C.c_int64),
                ("group_stride", C.c_int64)]


class AttnBlock(C.Structure):
    """vgx_attn_block (include/vault_amd.h)."""
    _fields_ = [("q", C.c_void_p), ("ldq", C.c_int64), ("q_hstride", C.c_int64), ("out", C.c_void_p),
                ("ldo", C.c_int64), ("o_hstride", C.c_int64), ("n_q", C.c_int64), ("causal_base", C.c_int64),
                ("n_runs", C.c_int), ("runs", KVRun * 4), ("bias", C.c_void_p), ("bias_head_row", C.c_void_p),
                ("bias_ldq", C.c_int64), ("bias_rstride", C.c_int64), ("bias_run", C.c_int)]


class ScoreSide(C.Structure):
    """vgx_score_side (include/vault_amd.h)."""
    _fields_ = [("phase", C.c_int), ("feat", C.c_void_p), ("fd", C.c_int64), ("ema", C.c_void_p), ("first", C.c_int),
                ("w1", C.c_void_p), ("hidden", C.c_int64), ("b1", C.c_void_p), ("ln_w", C.c_void_p),
                ("ln_b", C.c_void_p), ("eps", C.c_float), ("w2", C.c_void_p), ("b2", C.c_void_p), ("h", C.c_void_p),
                ("out", C.c_void_p), ("out_index", C.c_void_p)]


class VGXError(RuntimeError):
    pass


_lib = None


def declared_symbols() -> list:
    """Every vgx_* function declared in include/vault_amd.h."""
    with open(HEADER) as f:
        txt = f.read()
    return sorted(set(re.findall(r"\b(vgx_[a-z0-9_]+)\s*\(", txt)))


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise VGXError(f"{LIB_PATH} is not built; run `python -c 'import __graft_entry__ as g; g.build()'`")
    # torch first: its HIP runtime is then the one the library binds to, so device pointers and streams
    # from torch are valid in the library's calls (loading the library first can bring in a second runtime)
    import torch  # noqa: F401
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.vgx_abi_version() != 2:
        raise VGXError("ABI version mismatch")
    _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != VGX_OK:
        raise VGXError(f"{what} failed: {ERRORS.get(rc, rc)}")
