// Shared device helpers for the gfx950 kernels of libvault_amd.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/vault_amd.h"

#define VGX_DEV __device__ __forceinline__

namespace vgx {

constexpr int kWave = 64;
constexpr int QK = 32;

// DPP control words (GFX9 encoding).
constexpr int DPP_QUAD_1032 = 0xB1;   // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;   // quad_perm [2,3,0,1]
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_HALF_MIRROR = 0x141;

template <int CTRL>
VGX_DEV float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
VGX_DEV float row16_sum(float v) {
    v += dpp_f<DPP_QUAD_1032>(v);
    v += dpp_f<DPP_QUAD_2301>(v);
    v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_f<DPP_ROW_MIRROR>(v);
    return v;
}

VGX_DEV float row16_max(float v) {
    v = fmaxf(v, dpp_f<DPP_QUAD_1032>(v));
    v = fmaxf(v, dpp_f<DPP_QUAD_2301>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_HALF_MIRROR>(v));
    v = fmaxf(v, dpp_f<DPP_ROW_MIRROR>(v));
    return v;
}

VGX_DEV float wave_sum(float v) {
    v = row16_sum(v);
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    return v;
}

VGX_DEV float wave_max(float v) {
    v = row16_max(v);
    v = fmaxf(v, __shfl_xor(v, 16, kWave));
    v = fmaxf(v, __shfl_xor(v, 32, kWave));
    return v;
}

// Combine a value with the same value in lane l ^ 16 / l ^ 32 using the gfx950 VALU lane swaps
// (v_permlane16_swap / v_permlane32_swap) instead of an LDS permute.  With both operands equal to x,
// the two results of a swap hold, in every lane l, x[l] and x[l ^ 16] (resp. x[l ^ 32]).
VGX_DEV float xor16_max(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
VGX_DEV float xor32_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
VGX_DEV float xor16_sum(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
VGX_DEV float xor32_sum(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

VGX_DEV float half_bits_to_float(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

VGX_DEV float bf16_bits_to_float(uint32_t b) { return __uint_as_float((b & 0xFFFFu) << 16); }

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs): the gfx950 conversion instruction
// (v_cvt_pk_bf16_f32), one VALU operation instead of the four of the integer rounding sequence.
VGX_DEV uint32_t float_to_bf16_bits(float f) { return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)f); }

typedef __bf16 vgx_bf16x2_t __attribute__((ext_vector_type(2)));
typedef float vgx_f32x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two RNE bf16 in one word (low half = a), one v_cvt_pk_bf16_f32.
VGX_DEV uint32_t pack_bf16x2(float a, float b) {
    const vgx_f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, vgx_bf16x2_t));
}

// hi = bf16(a, b), lo = bf16(a - hi_a, b - hi_b): the hi + lo split of two floats (2^-17 relative).
VGX_DEV void split_bf16x2(float a, float b, uint32_t &hi, uint32_t &lo) {
    hi = pack_bf16x2(a, b);
    lo = pack_bf16x2(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// hi = bf16(a, b), mid = bf16(a - hi), lo = bf16(a - hi - mid): three pieces holding 24 significant
// bits, the whole fp32 mantissa (exact except where a piece falls below the bf16 normal range).
VGX_DEV void split3_bf16x2(float a, float b, uint32_t &hi, uint32_t &mid, uint32_t &lo) {
    hi = pack_bf16x2(a, b);
    const float ra = a - __uint_as_float(hi << 16), rb = b - __uint_as_float(hi & 0xFFFF0000u);
    mid = pack_bf16x2(ra, rb);
    lo = pack_bf16x2(ra - __uint_as_float(mid << 16), rb - __uint_as_float(mid & 0xFFFF0000u));
}

typedef _Float16 vgx_f16x2_t __attribute__((ext_vector_type(2)));

// Two floats -> two RNE fp16 in one word (low half = a).
VGX_DEV uint32_t pack_f16x2(float a, float b) {
    const vgx_f32x2_t v = {a, b};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, vgx_f16x2_t));
}

// hi = bf16(a, b) and lo16 = fp16(16 (a - hi_a), 16 (b - hi_b)); r = {the two elements of (hi + lo16 /
// 16) that sit in the low halves, those in the high halves} (what the pieces represent, in fp32).
VGX_DEV void split_bf16_f16x2(float a, float b, uint32_t &hi, uint32_t &lo16, float r[2]) {
    hi = pack_bf16x2(a, b);
    const float ha = __uint_as_float(hi << 16), hb = __uint_as_float(hi & 0xFFFF0000u);
    lo16 = pack_f16x2(16.0f * (a - ha), 16.0f * (b - hb));
    const auto l = __builtin_bit_cast(vgx_f16x2_t, lo16);
    r[0] = fmaf((float)l[0], 0.0625f, ha);
    r[1] = fmaf((float)l[1], 0.0625f, hb);
}

// The reference runtime's own exp / erf / GELU (runtime/vault3.c:104-129), step for step, so that
// results that select indices (the top-k draw, the segment scores that rank the bank) are the
// runtime's bit for bit.  The runtime is C compiled in a standard mode, which does not contract a * b
// + c into an FMA; contraction is switched off here for the same reason.  exp: range reduction by a
// two-piece ln 2, a degree-7 Taylor polynomial in Horner form, scaling by an exponent built in the
// bits (two steps below 2^-126, so subnormal results round as the runtime's do).  erf: Abramowitz &
// Stegun 7.1.26 (|error| <= 1.5e-7).
VGX_DEV float bits_f(uint32_t u) { return __uint_as_float(u); }

VGX_DEV float ref_expf(float x) {
#pragma clang fp contract(off)
    if (x > 88.72f) return bits_f(0x7F800000u);
    if (x < -103.9f) return 0.0f;
    const float kf = x * 1.44269504088896341f;
    const int k = (int)(kf + (kf >= 0.0f ? 0.5f : -0.5f));
    const float r = (x - (float)k * 0.693145751953125f) - (float)k * 1.428606765330187e-06f;
    const float p =
        1.0f + r * (1.0f + r * (0.5f + r * (1.6666667e-1f + r * (4.1666668e-2f + r * (8.3333338e-3f +
                                                                                     r * (1.3888889e-3f +
                                                                                          r * 1.9841270e-4f))))));
    if (k > 127) return p * bits_f(254u << 23) * 2.0f;
    if (k < -126) return p * bits_f((uint32_t)(k + 126 + 127) << 23) * bits_f(1u << 23);
    return p * bits_f((uint32_t)(k + 127) << 23);
}

VGX_DEV float ref_erff(float x) {
#pragma clang fp contract(off)
    const float z = x < 0.0f ? -x : x;
    if (z > 4.0f) return x < 0.0f ? -1.0f : 1.0f;
    const float t = 1.0f / (1.0f + 0.3275911f * z);
    const float p = (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                     0.254829592f) * t;
    const float y = 1.0f - p * ref_expf(-z * z);
    return x < 0.0f ? -y : y;
}

VGX_DEV float ref_geluf(float x) {
#pragma clang fp contract(off)
    return 0.5f * x * (1.0f + ref_erff(x * 0.70710678118654752f));
}

// Loads of data that a decode step or a prefill chunk reads once (weights, KV rows): the non-temporal
// cache policy (nt), which streams them past the caches' normal replacement.  kStreamAux is the same
// policy for buffer loads.  Measured on the 151665 x 1536 Q8_0 LM head GEMV: 43.7 -> 38.3 us.
constexpr int kStreamAux = 2;
typedef unsigned vgx_u32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned vgx_u32x2_t __attribute__((ext_vector_type(2)));
typedef float vgx_f32x4_t __attribute__((ext_vector_type(4)));

VGX_DEV uint4 ld_stream(const uint4 *p) {
    const vgx_u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const vgx_u32x4_t *>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
VGX_DEV uint2 ld_stream(const uint2 *p) {
    const vgx_u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const vgx_u32x2_t *>(p));
    return make_uint2(v[0], v[1]);
}
VGX_DEV float4 ld_stream(const float4 *p) {
    const vgx_f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const vgx_f32x4_t *>(p));
    return make_float4(v[0], v[1], v[2], v[3]);
}

// The scorer's EMA habituation of one feature (src/vault_v3_model.py:2299-2304): the habituated input
// f - 0.65 e and the state update 0.985 e + 0.015 f, each product rounded before the sum (no
// contraction, as the reference's float32 arithmetic), so every kernel that applies them agrees bit
// for bit.
VGX_DEV float hab_of(float f, float e) {
#pragma clang fp contract(off)
    return f - 0.65f * e;
}
VGX_DEV float ema_step(float e, float f) {
#pragma clang fp contract(off)
    return 0.985f * e + 0.015f * f;
}

// LDS DMA: buffer loads that write LDS directly (buffer_load ... lds), issued from inline assembly so that
// the compiler does not make every later LDS read wait for them (it treats any LDS read after a DMA it
// knows of as dependent on it); the kernel waits for them itself (s_waitcnt vmcnt, then a barrier).
// Extra outstanding loads only make the compiler's own vmcnt waits wait longer (loads return in order),
// never shorter.  M0 (the LDS base) is written here and cannot be declared clobbered (a reserved
// register): a kernel that uses these makes no other use of M0 (gfx950 LDS instructions do not read
// it), which its compiled code has to be checked for.
typedef int dma_rsrc_t __attribute__((ext_vector_type(4)));
constexpr uint32_t kDmaPast = 0x80000000u;      // a buffer offset past every operand: reads zero

// Buffer resource over `bytes` bytes at p (wave-uniform): offsets at or past the end read zeros.
VGX_DEV dma_rsrc_t dma_rsrc(const void *p, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)p;
    dma_rsrc_t r;
    r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xFFFFu));
    r.z = __builtin_amdgcn_readfirstlane((int)bytes);
    r.w = 0x00020000;
    return r;
}

// Lane l's 16 (4) bytes at byte offset voff of the buffer into LDS at lds + 16 l (4 l); lds is
// wave-uniform.
VGX_DEV void dma16(dma_rsrc_t rs, uint32_t voff, const void *lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m), "v"(voff), "s"(rs)
                 : "memory");
}
VGX_DEV void dma4(dma_rsrc_t rs, uint32_t voff, const void *lds) {
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)lds);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(m), "v"(voff), "s"(rs)
                 : "memory");
}

// One element of a KV-state tensor of dtype KV (VGX_F32, or VGX_BF16 rounded to nearest even).
template <int KV>
VGX_DEV void store_kv(void *base, int64_t idx, float v) {
    if constexpr (KV == VGX_F32) {
        static_cast<float *>(base)[idx] = v;
    } else {
        static_cast<uint16_t *>(base)[idx] = (uint16_t)float_to_bf16_bits(v);
    }
}

template <int KV>
VGX_DEV float load_kv(const void *base, int64_t idx) {
    if constexpr (KV == VGX_F32) return static_cast<const float *>(base)[idx];
    return bf16_bits_to_float(static_cast<const uint16_t *>(base)[idx]);
}

}  // namespace vgx

#define VGX_CHECK_LAUNCH()                                  \
    do {                                                    \
        if (hipGetLastError() != hipSuccess) return VGX_E_HIP; \
    } while (0)
