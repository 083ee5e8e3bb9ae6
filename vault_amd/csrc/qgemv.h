// HBM-streaming Q8_0 / Q4_0 / F32 / BF16 / F16 GEMV for gfx950 (batch 1..4 rows per pass) with fused
// RMSNorm prologue and bias / residual / SwiGLU epilogues.  Instantiated per weight dtype in
// qgemv_q8.hip, qgemv_q4.hip, qgemv_f32.hip, qgemv_bf16.hip and qgemv_f16.hip so they compile in
// parallel.
//
// Reference semantics: runtime/vault3.c:499-624 (row_dot, matvec), 656-660 (rmsnorm),
// 1942-1956 (mlp_gu_run); src/vault_v3_model.py:764-774, 1041-1047, 1139, 1145-1150, 2150-2151.
//
// Weights are in the packed row-quad layout (include/vault_amd.h): a 32-weight block of four
// consecutive rows is one contiguous 64-byte (Q4_0) / 128-byte (Q8_0) / 512-byte (F32) run, and the
// four fp16 scales of that block are one 8-byte word of the scale plane.  A lane processes whole
// blocks of one row-quad: one set of 128-bit loads brings 4 x 32 weights, the 32 activations of
// the block are read from LDS once and used for the four rows.
//
// One activation row (the decode step) runs gemv1_kernel, whose mapping is picked from the shape
// (below), for 1536-column weights of >= 8192 rows (gate/up, the LM head) the persistent
// gemv1_stream_kernel, for other rows (the down and o projections) gemv1_pieces_kernel; 2-4 rows per
// pass run qgemv_kernel in row mode (16 lanes per row-quad, four row-quads per wave, 4 waves
// per workgroup) for >= 2048 row-quads, else in split-K mode (a wave per row-quad).
// Each lane requests the weights of up to U blocks at once to keep enough bytes in flight for HBM.
//
// Arithmetic is fp32 throughout, as in the reference: per block s = sum_j q_j x_j, acc += d * s.
// Q4_0 nibbles n are converted unsigned (v_cvt_f32_ubyte*) and the -8 offset is applied once per
// block as acc += d * (sum_j n_j x_j - 8 * sum_j x_j), sum_j x_j summed by the lane from the same
// 32 staged activations.
// With the RMSNorm prologue the staged activations are lnw[c] * x[c]; sum x^2 is accumulated while
// staging and the dot products are scaled by inv_rms = 1 / sqrt(mean(x^2) + eps) before the
// epilogue (the GEMV is linear in its input).
#pragma once

#include "common.h"

namespace vgx {

enum { EPI_STORE = 0, EPI_ACCUM = 1, EPI_SWIGLU = 2 };
enum { MODE_ROWS = 0, MODE_SPLITK = 1 };

constexpr int kGemvMaxChunkFloats = 8192;  // activations staged in LDS per chunk (all batch rows)
constexpr int kGemvPad = 36;               // floats per staged 32-float block (4 floats of padding)

// Bytes of one row's 32-element block in the packed layout (quants only for Q8_0 / Q4_0, whose
// scales sit in the scale plane; the elements themselves for the plain dtypes F32 / BF16 / F16).
__host__ __device__ constexpr int gemv_quant_bytes(int dt) {
    return dt == VGX_Q8_0 ? 32 : dt == VGX_Q4_0 ? 16 : dt == VGX_F32 ? 128 : (dt == VGX_BF16 || dt == VGX_F16) ? 64 : 0;
}
__host__ __device__ constexpr bool gemv_plain(int dt) { return dt == VGX_F32 || dt == VGX_BF16 || dt == VGX_F16; }
__host__ __device__ constexpr bool gemv_half(int dt) { return dt == VGX_BF16 || dt == VGX_F16; }
__host__ __device__ constexpr bool gemv_quant(int dt) { return dt == VGX_Q8_0 || dt == VGX_Q4_0; }

// Dequantize one 32-weight block of packed row r into out[0..31].
template <int DT>
__device__ __forceinline__ void dequant_block(const uint8_t *__restrict__ w, int64_t nblk, int64_t soff, int64_t r,
                                              int64_t b, float *__restrict__ out) {
    constexpr int QB = gemv_quant_bytes(DT);
    const int64_t rq = r >> 2, rr = r & 3;
    const uint8_t *qs = w + ((rq * nblk + b) * 4 + rr) * QB;
    if constexpr (DT == VGX_F32) {
        const float *s = reinterpret_cast<const float *>(qs);
        for (int j = 0; j < QK; ++j) out[j] = s[j];
    } else if constexpr (DT == VGX_BF16) {
        const uint16_t *s = reinterpret_cast<const uint16_t *>(qs);
        for (int j = 0; j < QK; ++j) out[j] = bf16_bits_to_float(s[j]);
    } else if constexpr (DT == VGX_F16) {
        const uint16_t *s = reinterpret_cast<const uint16_t *>(qs);
        for (int j = 0; j < QK; ++j) out[j] = half_bits_to_float(s[j]);
    } else {
        const float d = half_bits_to_float(reinterpret_cast<const uint16_t *>(w + soff)[(rq * nblk + b) * 4 + rr]);
        if constexpr (DT == VGX_Q8_0) {
            for (int j = 0; j < QK; ++j) out[j] = d * (float)(int8_t)qs[j];
        } else {
            for (int j = 0; j < 16; ++j) {
                out[j] = (float)((int)(qs[j] & 0x0F) - 8) * d;
                out[j + 16] = (float)((int)(qs[j] >> 4) - 8) * d;
            }
        }
    }
}

struct ScoreSide;

struct GemvArgs {
    const uint8_t *w;
    int nblk;            // 32-weight blocks per row
    int64_t soff;        // byte offset of the scale plane
    int64_t n_rq;        // packed row-quads
    int64_t rows_out;    // output rows (SwiGLU: half the packed rows)
    const float *x;
    int64_t ldx;
    int64_t batch;
    const float *lnw;    // RMSNorm weight (nullptr: no prologue)
    float eps;
    const float *bias;   // may be nullptr
    float *y;
    int64_t ldy;
    int epi;
    const int64_t *y_ref;   // non-null: y is the address stored in this device word when the launch runs,
    int64_t y_off;          // plus this many floats
    // Segment-scorer prologue (F32 weights, two output rows): with sc_ema set, the activation rows are
    // LayerNorm(f) and LayerNorm(f - 0.65 e) of the token's features f = x (e = sc_ema, or f itself
    // when sc_first), LayerNorm weight lnw, bias sc_lnb, eps.
    const float *sc_ema;
    const float *sc_lnb;
    int sc_first;
    const ScoreSide *side;  // host side only: a scorer job launched with this GEMV (in its spare workgroups)
};

// The output address of a launch whose GemvArgs name it indirectly (a captured graph whose output
// buffer changes per replay); one uniform load per workgroup.
__device__ __forceinline__ void gemv_resolve_y(GemvArgs &a) {
    if (a.y_ref != nullptr) a.y = reinterpret_cast<float *>(*a.y_ref) + a.y_off;
}

__device__ __forceinline__ float gemv_cvt_u8(uint32_t w, int k) {
    switch (k) {  // each pattern maps onto one v_cvt_f32_ubyte{0..3}
        case 0: return (float)(w & 0xFFu);
        case 1: return (float)((w >> 8) & 0xFFu);
        case 2: return (float)((w >> 16) & 0xFFu);
        default: return (float)(w >> 24);
    }
}

__device__ __forceinline__ float gemv_cvt_s8(uint32_t w, int k) { return (float)(int)(int8_t)(w >> (8 * k)); }

// w & 0x0F0F0F0F, opaque to the optimiser: otherwise each later byte extract is folded back into a
// per-nibble v_bfe_u32, doubling the conversion cost.  With the mask opaque, every nibble converts
// with a single v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t gemv_nibble_mask(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
    return r;
}

// Weights of one 32-weight block of a row-quad, held in registers.
template <int DT>
struct BlockRegs;
template <>
struct BlockRegs<VGX_Q4_0> {
    uint4 q[4];
    uint2 s;
};
template <>
struct BlockRegs<VGX_Q8_0> {
    uint4 q[8];
    uint2 s;
};
template <>
struct BlockRegs<VGX_F32> {
    const float4 *p;  // F32 weights are read at use (512 bytes per block would not fit twice)
};
// BF16 / F16: the 4 x 64 bytes of a row-quad block (row r in q[4 r .. 4 r + 3]).
template <>
struct BlockRegs<VGX_BF16> {
    uint4 q[16];
};
template <>
struct BlockRegs<VGX_F16> {
    uint4 q[16];
};

template <int DT>
__device__ __forceinline__ void gemv_load(BlockRegs<DT> &r, const uint8_t *__restrict__ W, int64_t soff, int64_t rq,
                                          int nblk, int64_t gb) {
    constexpr int QB = gemv_quant_bytes(DT);
    const uint8_t *qp = W + (rq * nblk + gb) * 4 * QB;
    if constexpr (DT == VGX_F32) {
        r.p = reinterpret_cast<const float4 *>(qp);
    } else if constexpr (gemv_half(DT)) {
#pragma unroll
        for (int i = 0; i < 16; ++i) r.q[i] = ld_stream(reinterpret_cast<const uint4 *>(qp) + i);
    } else {
#pragma unroll
        for (int i = 0; i < 4 * QB / 16; ++i) r.q[i] = ld_stream(reinterpret_cast<const uint4 *>(qp) + i);
        r.s = ld_stream(reinterpret_cast<const uint2 *>(W + soff + (rq * nblk + gb) * 8));
    }
}

// acc[r][n] += row r of the block . x_n (staged block xb_n = xs + n * stride_n).
template <int DT, int NB>
__device__ __forceinline__ void gemv_block(const BlockRegs<DT> &br, const float *__restrict__ xb, int stride_n,
                                           float (&acc)[4][NB]) {
    if constexpr (DT == VGX_F32) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float wv[QK];
#pragma unroll
            for (int j4 = 0; j4 < 8; ++j4) {
                const float4 t = ld_stream(br.p + r * 8 + j4);
                wv[j4 * 4 + 0] = t.x; wv[j4 * 4 + 1] = t.y; wv[j4 * 4 + 2] = t.z; wv[j4 * 4 + 3] = t.w;
            }
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const float *xn = xb + n * stride_n;
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < QK; ++j) s = fmaf(wv[j], xn[j], s);
                acc[r][n] += s;
            }
        }
    } else if constexpr (gemv_half(DT)) {
        // BF16 / F16 elements widened exactly to fp32 (runtime/vault3.c:510-533), products in fp32
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float wv[QK];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint4 t = br.q[4 * r + i];
                const uint32_t w4[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    if constexpr (DT == VGX_BF16) {
                        wv[8 * i + 2 * k] = __uint_as_float(w4[k] << 16);
                        wv[8 * i + 2 * k + 1] = __uint_as_float(w4[k] & 0xFFFF0000u);
                    } else {
                        wv[8 * i + 2 * k] = half_bits_to_float(w4[k]);
                        wv[8 * i + 2 * k + 1] = half_bits_to_float(w4[k] >> 16);
                    }
                }
            }
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                const float *xn = xb + n * stride_n;
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < QK; ++j) s = fmaf(wv[j], xn[j], s);
                acc[r][n] += s;
            }
        }
    } else {
        const float d[4] = {half_bits_to_float(br.s.x), half_bits_to_float(br.s.x >> 16),
                            half_bits_to_float(br.s.y), half_bits_to_float(br.s.y >> 16)};
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const float *xn = xb + n * stride_n;
            float xv[QK];
#pragma unroll
            for (int j4 = 0; j4 < 8; ++j4) {
                const float4 t = *reinterpret_cast<const float4 *>(xn + j4 * 4);
                xv[j4 * 4 + 0] = t.x; xv[j4 * 4 + 1] = t.y; xv[j4 * 4 + 2] = t.z; xv[j4 * 4 + 3] = t.w;
            }
            if constexpr (DT == VGX_Q4_0) {
                float xs_sum = 0.0f;  // sum of the block's activations, for the -8 nibble offset
#pragma unroll
                for (int j = 0; j < QK; ++j) xs_sum += xv[j];
                const float s8 = 8.0f * xs_sum;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t wq[4] = {br.q[r].x, br.q[r].y, br.q[r].z, br.q[r].w};
                    float s = 0.0f;
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        const uint32_t lo = gemv_nibble_mask(wq[k]);
                        const uint32_t hi = gemv_nibble_mask(wq[k] >> 4);
#pragma unroll
                        for (int t = 0; t < 4; ++t) {
                            s = fmaf(gemv_cvt_u8(lo, t), xv[4 * k + t], s);
                            s = fmaf(gemv_cvt_u8(hi, t), xv[16 + 4 * k + t], s);
                        }
                    }
                    acc[r][n] = fmaf(d[r], s - s8, acc[r][n]);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint4 a = br.q[2 * r], b = br.q[2 * r + 1];
                    const uint32_t wq[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                    float s = 0.0f;
#pragma unroll
                    for (int k = 0; k < 8; ++k)
#pragma unroll
                        for (int t = 0; t < 4; ++t) s = fmaf(gemv_cvt_s8(wq[k], t), xv[4 * k + t], s);
                    acc[r][n] = fmaf(d[r], s, acc[r][n]);
                }
            }
        }
    }
}

template <int DT, int NB, int EPI, int MODE, int KW, bool NORM>
__global__ __launch_bounds__(64 * (MODE == MODE_ROWS ? 4 : 1) * KW) void qgemv_kernel(GemvArgs a, int cbk) {
    gemv_resolve_y(a);
    extern __shared__ float smem[];
    constexpr int LPR = MODE == MODE_ROWS ? 16 : 64;     // lanes per row-quad
    constexpr int RQW = 64 / LPR;                          // row-quads per wave
    constexpr int RW = MODE == MODE_ROWS ? 4 : 1;          // waves with distinct row-quads
    constexpr int WPG = RW * KW;                           // waves per workgroup
    constexpr int RQG = RQW * RW;                          // row-quads per workgroup
    constexpr int NT = 64 * WPG;
    float *xs = smem;                                      // [NB][cbk][kGemvPad]
    __shared__ float red[WPG][RQW][4][NB];
    __shared__ float rsum[WPG][NB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int rw = wave / KW, ks = wave - rw * KW;         // row-wave, K-split index
    const int li = lane % LPR, rqi = lane / LPR;
    const int64_t rq = (int64_t)blockIdx.x * RQG + rw * RQW + rqi;
    const bool act = rq < a.n_rq;
    const int nblk = a.nblk;
    const int cols = nblk * QK;
    const int first = ks * LPR + li;
    const int stride = LPR * KW;

    float acc[4][NB];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[r][n] = 0.0f;
    float ssq[NB];  // RMSNorm: this thread's part of sum x^2 over the staged activations
#pragma unroll
    for (int n = 0; n < NB; ++n) ssq[n] = 0.0f;

    // Each lane issues the loads of U blocks at once (all of its blocks for the model's shapes), the
    // first batch before the activations are staged, so a lane has up to U x 64 B (Q4_0) /
    // U x 128 B (Q8_0) of weights in flight.
    // With 3 or more K-split waves a lane has at most one or two blocks of the model's rows (8 waves
    // over the 280-block down projection): one block per batch, fewer registers.
    constexpr int U = (KW >= 3) ? 1 : DT == VGX_Q4_0 ? 4 : DT == VGX_Q8_0 ? 3 : 1;
    BlockRegs<DT> br[U];
    int cb = min(cbk, nblk);
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (act && first + u * stride < cb) gemv_load<DT>(br[u], a.w, a.soff, rq, nblk, first + u * stride);

    for (int c0 = 0; c0 < nblk; c0 += cbk) {
        cb = min(cbk, nblk - c0);
        if (c0) __syncthreads();
        const bool vec = ((reinterpret_cast<uintptr_t>(a.x) & 15) == 0) && (a.ldx % 4 == 0);
        if (vec) {
            // kStageLoads float4 loads per thread in flight: one round trip for the model's shapes
            // (1536 activations over 256 threads; 8960 over the 512 threads of the 8-wave split-K)
            // without holding more staging registers than that needs.
            constexpr int kStageLoads = KW >= 4 ? 6 : 4;
            const int n4 = NB * cb * 8;
            for (int i0 = tid; i0 < n4; i0 += kStageLoads * NT) {
                float4 v[kStageLoads], gw[kStageLoads];
#pragma unroll
                for (int u = 0; u < kStageLoads; ++u) {
                    const int i = i0 + u * NT;
                    if (i < n4) {
                        const int n = i / (cb * 8), rem = i - n * cb * 8;
                        const int64_t c = (int64_t)c0 * QK + rem * 4;
                        v[u] = *reinterpret_cast<const float4 *>(a.x + n * a.ldx + c);
                        if constexpr (NORM) gw[u] = *reinterpret_cast<const float4 *>(a.lnw + c);
                    }
                }
#pragma unroll
                for (int u = 0; u < kStageLoads; ++u) {
                    const int i = i0 + u * NT;
                    if (i < n4) {
                        const int n = i / (cb * 8), rem = i - n * cb * 8, blk = rem >> 3, j4 = rem & 7;
                        float4 t = v[u];
                        if constexpr (NORM) {
                            const float q2 = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, t.w * t.w)));
#pragma unroll
                            for (int nn = 0; nn < NB; ++nn)
                                if (nn == n) ssq[nn] += q2;  // static register index
                            t.x *= gw[u].x; t.y *= gw[u].y; t.z *= gw[u].z; t.w *= gw[u].w;
                        }
                        *reinterpret_cast<float4 *>(xs + (n * cbk + blk) * kGemvPad + j4 * 4) = t;
                    }
                }
            }
        } else {
            for (int i = tid; i < NB * cb * QK; i += NT) {
                const int n = i / (cb * QK), rem = i - n * cb * QK, blk = rem >> 5, j = rem & 31;
                const int64_t c = (int64_t)(c0 + blk) * QK + j;
                float v = a.x[n * a.ldx + c];
                if constexpr (NORM) {
#pragma unroll
                    for (int nn = 0; nn < NB; ++nn)
                        if (nn == n) ssq[nn] = fmaf(v, v, ssq[nn]);
                    v *= a.lnw[c];
                }
                xs[(n * cbk + blk) * kGemvPad + j] = v;
            }
        }
        __syncthreads();
        if (act) {
            for (int b = first; b < cb; b += U * stride) {
                if (b != first) {
#pragma unroll
                    for (int u = 0; u < U; ++u)
                        if (b + u * stride < cb) gemv_load<DT>(br[u], a.w, a.soff, rq, nblk, c0 + b + u * stride);
                }
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int bb = b + u * stride;
                    if (bb < cb) gemv_block<DT, NB>(br[u], xs + bb * kGemvPad, cbk * kGemvPad, acc);
                }
            }
            // first batch of the next chunk
            const int cn = min(cbk, nblk - c0 - cbk);
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (first + u * stride < cn) gemv_load<DT>(br[u], a.w, a.soff, rq, nblk, c0 + cbk + first + u * stride);
        }
    }

    // RMSNorm: the staged activations were lnw * x, so every dot product is scaled by 1/rms here
    // (W . (lnw * x * inv) = inv * W . (lnw * x)).
    if constexpr (NORM) {
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const float t = wave_sum(ssq[n]);
            if (lane == 0) rsum[wave][n] = t;
        }
        __syncthreads();
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            float tot = 0.0f;
#pragma unroll
            for (int w = 0; w < WPG; ++w) tot += rsum[w][n];
            const float inv = 1.0f / sqrtf(tot / (float)cols + a.eps);
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[r][n] *= inv;
        }
    }

    // Reduce over the lanes of the row-quad, then over the K-split waves of the workgroup.
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[r][n] = LPR == 16 ? row16_sum(acc[r][n]) : wave_sum(acc[r][n]);
    if constexpr (KW > 1) {
        if (li == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int n = 0; n < NB; ++n) red[wave][rqi][r][n] = acc[r][n];
        }
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int n = 0; n < NB; ++n) {
                float s = red[wave][rqi][r][n];
#pragma unroll
                for (int w = 1; w < KW; ++w) s += red[wave + w][rqi][r][n];
                acc[r][n] = s;
            }
    }
    if (!act || li != 0) return;
    if constexpr (EPI == EPI_SWIGLU) {
        const int64_t o0 = rq * 2;
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (o0 + k >= a.rows_out) continue;
                const float g = acc[k][n], u = acc[2 + k][n];
                a.y[n * a.ldy + o0 + k] = g / (1.0f + __expf(-g)) * u;
            }
    } else {
        const int64_t r0 = rq * 4;
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = r0 + r;
                if (row >= a.rows_out) continue;
                float v = acc[r][n];
                if (a.bias) v += a.bias[row];
                if constexpr (EPI == EPI_ACCUM) v += a.y[n * a.ldy + row];
                a.y[n * a.ldy + row] = v;
            }
    }
}

// One-row GEMV (the decode step): lean register budget, one pass over K.
//   LPR lanes per row-quad (64: a lane per block; 16: a DPP row per row-quad, U blocks per lane),
//   WPG waves with distinct row-quads, KW waves splitting K (reduced through LDS).
//   Activations: XD = read directly by each lane; otherwise staged in LDS (lnw * x, sum x^2
//   accumulated while staging) with SF = the staging loads requested before the weights, so the
//   barrier after staging does not wait for the weights and each wave multiplies as soon as its
//   own weights arrive.
// Measured on MI355X (gate/up 2 x 8960 x 1536 Q4_0): LPR 64 / 4 waves / SF 7.6 us against 9.4 us for
// the DPP-row mapping; other tall weights keep the DPP-row mapping (the 151665-row LM head: 48 vs
// 53 us, before gemv1_stream_kernel took that shape: 44.7 us Q8_0, 26.2 us Q4_0).
template <int DT, int EPI, bool NORM, int LPR, int WPG, int KW, int U, bool SF, bool XD>
__global__ __launch_bounds__(64 * WPG * KW) void gemv1_kernel(GemvArgs a) {
    gemv_resolve_y(a);
    static_assert(!XD || WPG == 1, "direct activations: one row-quad set per workgroup");
    constexpr int RQW = 64 / LPR;
    constexpr int NW = WPG * KW;
    constexpr int NT = 64 * NW;
    constexpr int CH = 4;                          // staging float4 loads per thread and round
    extern __shared__ float xs[];                  // [nblk][kGemvPad]
    __shared__ float red[NW][RQW][4];
    __shared__ float rsum[NW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int rw = wave / KW, ks = wave - rw * KW;
    const int li = lane % LPR, rqi = lane / LPR;
    const int64_t rq = (int64_t)blockIdx.x * (WPG * RQW) + rw * RQW + rqi;
    const bool act = rq < a.n_rq;
    const int nblk = a.nblk;
    const int first = ks * LPR + li;
    constexpr int stride = LPR * KW;

    BlockRegs<DT> br[U];
    auto load_first = [&]() {
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (act && first + u * stride < nblk) gemv_load<DT>(br[u], a.w, a.soff, rq, nblk, first + u * stride);
    };
    if constexpr (!SF) load_first();

    float acc[4][1] = {{0.0f}, {0.0f}, {0.0f}, {0.0f}};
    float ssq = 0.0f;
    if constexpr (!XD) {
        const int n4 = nblk * 8;
        auto stage_load = [&](int i0, float4 (&v)[CH], float4 (&gw)[CH]) {
#pragma unroll
            for (int u = 0; u < CH; ++u) {
                const int i = i0 + u * NT;
                if (i < n4) {
                    v[u] = reinterpret_cast<const float4 *>(a.x)[i];
                    if constexpr (NORM) gw[u] = reinterpret_cast<const float4 *>(a.lnw)[i];
                }
            }
        };
        auto stage_store = [&](int i0, const float4 (&v)[CH], const float4 (&gw)[CH]) {
#pragma unroll
            for (int u = 0; u < CH; ++u) {
                const int i = i0 + u * NT;
                if (i < n4) {
                    float4 t = v[u];
                    if constexpr (NORM) {
                        ssq += fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, t.w * t.w)));
                        t.x *= gw[u].x; t.y *= gw[u].y; t.z *= gw[u].z; t.w *= gw[u].w;
                    }
                    *reinterpret_cast<float4 *>(xs + (i >> 3) * kGemvPad + (i & 7) * 4) = t;
                }
            }
        };
        {
            // first round, then (SF) every thread's weight loads, whether or not it stages anything
            float4 v[CH], gw[CH];
            stage_load(tid, v, gw);
            if constexpr (SF) load_first();
            stage_store(tid, v, gw);
        }
        for (int i0 = tid + CH * NT; i0 < n4; i0 += CH * NT) {
            float4 v[CH], gw[CH];
            stage_load(i0, v, gw);
            stage_store(i0, v, gw);
        }
        __syncthreads();
    } else if constexpr (SF) {
        load_first();
    }
    if (act) {
        for (int b = first; b < nblk; b += U * stride) {
            if (b != first) {
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (b + u * stride < nblk) gemv_load<DT>(br[u], a.w, a.soff, rq, nblk, b + u * stride);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int bb = b + u * stride;
                if (bb >= nblk) continue;
                if constexpr (XD) {
                    const float4 *xp = reinterpret_cast<const float4 *>(a.x + (int64_t)bb * QK);
                    float4 xv[8], gv[8];
#pragma unroll
                    for (int j = 0; j < 8; ++j) xv[j] = xp[j];
                    if constexpr (NORM) {
#pragma unroll
                        for (int j = 0; j < 8; ++j) gv[j] = reinterpret_cast<const float4 *>(a.lnw + (int64_t)bb * QK)[j];
                    }
                    float xb[QK];
#pragma unroll
                    for (int j = 0; j < 8; ++j) {
                        float4 t = xv[j];
                        if constexpr (NORM) {
                            ssq += fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, t.w * t.w)));
                            t.x *= gv[j].x; t.y *= gv[j].y; t.z *= gv[j].z; t.w *= gv[j].w;
                        }
                        xb[4 * j] = t.x; xb[4 * j + 1] = t.y; xb[4 * j + 2] = t.z; xb[4 * j + 3] = t.w;
                    }
                    gemv_block<DT, 1>(br[u], xb, 0, acc);
                } else {
                    gemv_block<DT, 1>(br[u], xs + bb * kGemvPad, 0, acc);
                }
            }
        }
    }
    if constexpr (NORM) {
        // XD: every lane summed its own blocks; the K-split waves together cover the row once.
        const float t = wave_sum(ssq);
        if (lane == 0) rsum[wave] = t;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) tot += rsum[w];
        const float inv = 1.0f / sqrtf(tot / (float)(nblk * QK) + a.eps);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r][0] *= inv;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r][0] = LPR == 64 ? wave_sum(acc[r][0]) : row16_sum(acc[r][0]);
    if constexpr (KW > 1) {
        if (li == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][rqi][r] = acc[r][0];
        }
        __syncthreads();
        if (ks != 0) return;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float sum = red[wave][rqi][r];
#pragma unroll
            for (int w = 1; w < KW; ++w) sum += red[wave + w][rqi][r];
            acc[r][0] = sum;
        }
    }
    if (!act || li != 0) return;
    if constexpr (EPI == EPI_SWIGLU) {
        const int64_t o0 = rq * 2;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            if (o0 + k >= a.rows_out) continue;
            const float g = acc[k][0], u = acc[2 + k][0];
            a.y[o0 + k] = g / (1.0f + __expf(-g)) * u;
        }
    } else {
        const int64_t r0 = rq * 4;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = r0 + r;
            if (row >= a.rows_out) continue;
            float v = acc[r][0];
            if (a.bias) v += a.bias[row];
            if constexpr (EPI == EPI_ACCUM) v += a.y[row];
            a.y[row] = v;
        }
    }
}

// One-row GEMV over tall Q8_0 / Q4_0 weights of 48 blocks per row (1536 columns: the LM head).
// Persistent: every wave walks row-quads gw, gw + n_waves, ... and keeps RB of them in flight.
//   Loads: one 16-byte buffer load per lane covers 1 KB of a row-quad's contiguous run (the whole
//   instruction reads one 1 KB range, not 64 pieces of separate blocks), NL = 6 (Q8_0) / 3 (Q4_0)
//   loads per row-quad, plus one 2-byte scale load per 16-byte piece.  Q8_0: lane l holds half h =
//   l & 1 of row r = (l >> 1) & 3 of block 8 j + (l >> 3); Q4_0: row r = l & 3 of block 16 j + (l >> 2).
//   A lane therefore always meets the same 96 activations; they stay in registers after one pass
//   through LDS (RMSNorm weight applied, sum x^2 while staging).
//   Arithmetic per 16-byte piece, fp32: Q8_0 s = sum q x, Q4_0 s = sum n x - 8 sum x; acc += d * s;
//   the 16 lanes of a row are summed by DPP / lane swaps, the RMSNorm scale applied last (the
//   product is linear in x).
//   Every load and store is unconditional: the quants and the scales are two buffers whose bounds
//   end with the last row-quad, so fetches of row-quads past the end read zero without touching
//   memory, and their stores land past y's bound; the loop has no branch around memory operations
//   and the compiler waits for exactly the loads of the row-quad it uses.
//   Epilogues: store, or SwiGLU over gate/up row-quads (rows 0, 1 gate, rows 2, 3 up of the same two
//   output rows), the up value taken from the lanes of row r + 2.
constexpr int kStreamBlocks = 48;
constexpr int kStreamMinRq = 2048;
constexpr uint32_t kStreamPastEnd = 0x80000000u;

template <int DT>
struct StreamGeom {
    static constexpr int QB = gemv_quant_bytes(DT);
    static constexpr int RQB = kStreamBlocks * 4 * QB;   // bytes of one row-quad's quants
    static constexpr int NL = RQB / 1024;                // 16-byte loads per lane per row-quad
    static constexpr int XL = 96 / NL;                   // activations per lane per load
    // row-quads in flight per wave and workgroups: Q8_0 2 and 768 (3 waves per SIMD), Q4_0 3 and 512 (2 per
    // SIMD); measured against 3 / 512 and 4 / 512: LM head Q8_0 43.1 vs 43.6 us, Q4_0 25.6 vs 28.2 us, gate/up
    // 6.69 vs 6.93 us (Q4_0 4 / 768, 6 / 512 and 2 / 768 measured slower)
    static constexpr int RB = DT == VGX_Q8_0 ? 2 : 3;
    static constexpr int GROUPS = DT == VGX_Q8_0 ? 768 : 512;
};

template <int DT>
VGX_DEV int stream_block(int lane, int j) { return DT == VGX_Q8_0 ? 8 * j + (lane >> 3) : 16 * j + (lane >> 2); }

template <int DT, int EPI, bool NORM>
__global__ __launch_bounds__(256) void gemv1_stream_kernel(GemvArgs a) {
    gemv_resolve_y(a);
    using G = StreamGeom<DT>;
    constexpr int NL = G::NL, XL = G::XL, RB = G::RB;
    const int lane = threadIdx.x & 63;
    const int gw = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * 4 + (threadIdx.x >> 6)));
    const int nw = (int)gridDim.x * 4;
    const int n_rq = (int)a.n_rq;
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *)a.w, 0, n_rq * G::RQB, 0x00020000);
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.w + a.soff), 0, n_rq * (kStreamBlocks * 8), 0x00020000);
    // per-lane parts of the offsets: piece j of a row-quad, its scale
    uint32_t qoff[NL], sofs[NL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        qoff[j] = (uint32_t)(j * 1024 + lane * 16);
        sofs[j] = DT == VGX_Q8_0 ? (uint32_t)(64 * j + 2 * (lane >> 1)) : (uint32_t)(128 * j + 2 * lane);
    }
    uint4 wq[RB][NL];
    uint32_t wsc[RB][NL];
    // Row-quads past the end are fetched too, without a branch: their offsets stay below 2^32 (the
    // quants are under 2 GiB and a wave runs at most 2 RB row-quads past the end) and read zero.
    auto fetch = [&](int s, int rq) {
        const uint32_t qb = (uint32_t)rq * G::RQB;
        const uint32_t sb = (uint32_t)rq * (kStreamBlocks * 8);
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, qb + qoff[j], 0, kStreamAux);
            wq[s][j] = make_uint4(v[0], v[1], v[2], v[3]);
        }
#pragma unroll
        for (int j = 0; j < NL; ++j) wsc[s][j] = __builtin_amdgcn_raw_buffer_load_b16(srs, sb + sofs[j], 0, kStreamAux);
    };
    // lnw * x staged once per workgroup (the activation loads go first, so waiting for them does not
    // wait for the weights), then the weight ring, then this lane's 96 activations from LDS.
    __shared__ float xs[kStreamBlocks * QK];
    __shared__ float red[4];
    constexpr int N4 = kStreamBlocks * QK / 4;   // 384 float4
    const int tid = threadIdx.x;
    float4 xa[2], ga[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = tid + 256 * u;
        if (i < N4) {
            xa[u] = reinterpret_cast<const float4 *>(a.x)[i];
            if constexpr (NORM) ga[u] = reinterpret_cast<const float4 *>(a.lnw)[i];
        }
    }
    // the ring's first fill in the loop's own issue order (slot by slot), so one wait count per use
    // holds for the first round and the steady state alike
#pragma unroll
    for (int s = 0; s < RB; ++s) {
        fetch(s, gw + s * nw);
        __builtin_amdgcn_sched_barrier(0);
    }
    float ssq = 0.0f;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const int i = tid + 256 * u;
        if (i < N4) {
            float4 t = xa[u];
            if constexpr (NORM) {
                ssq += fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, t.w * t.w)));
                t.x *= ga[u].x; t.y *= ga[u].y; t.z *= ga[u].z; t.w *= ga[u].w;
            }
            reinterpret_cast<float4 *>(xs)[i] = t;
        }
    }
    if constexpr (NORM) {
        const float w = wave_sum(ssq);
        if (lane == 0) red[tid >> 6] = w;
    }
    __syncthreads();
    float xv[NL][XL];
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        const int c0 = stream_block<DT>(lane, j) * QK + (DT == VGX_Q8_0 ? (lane & 1) * 16 : 0);
#pragma unroll
        for (int t4 = 0; t4 < XL / 4; ++t4) {
            const float4 t = reinterpret_cast<const float4 *>(xs + c0)[t4];
            xv[j][4 * t4] = t.x; xv[j][4 * t4 + 1] = t.y; xv[j][4 * t4 + 2] = t.z; xv[j][4 * t4 + 3] = t.w;
        }
    }
    float off[NL];   // Q4_0: the -8 offset term of each piece, 8 sum x
#pragma unroll
    for (int j = 0; j < NL; ++j) {
        float s = 0.0f;
        if constexpr (DT == VGX_Q4_0) {
#pragma unroll
            for (int t = 0; t < XL; ++t) s += xv[j][t];
        }
        off[j] = 8.0f * s;
    }
    float inv = 1.0f;
    if constexpr (NORM) inv = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)(kStreamBlocks * QK) + a.eps);
    const __amdgpu_buffer_rsrc_t yrs = __builtin_amdgcn_make_buffer_rsrc((void *)a.y, 0, (int)(a.rows_out * 4), 0x00020000);
    const int r_out = DT == VGX_Q8_0 ? lane >> 1 : lane;                  // the storing lanes' row
    // one lane per row of the row-quad (SwiGLU: per gate row)
    const bool stores = (DT == VGX_Q8_0 ? (lane & 0x39) == 0 : lane < 4) && (EPI != EPI_SWIGLU || r_out < 2);
    constexpr int kOutPerRq = EPI == EPI_SWIGLU ? 2 : 4;

    // row-quad i of this wave: gw + i * nw, i < cnt; ring slot s holds i = s (mod RB)
    const int cnt = gw < n_rq ? (n_rq - gw + nw - 1) / nw : 0;
    auto dot = [&](int s) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NL; ++j) {
            const uint32_t q[4] = {wq[s][j].x, wq[s][j].y, wq[s][j].z, wq[s][j].w};
            float p = 0.0f;
            if constexpr (DT == VGX_Q8_0) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
#pragma unroll
                    for (int t = 0; t < 4; ++t) p = fmaf(gemv_cvt_s8(q[k], t), xv[j][4 * k + t], p);
            } else {
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const uint32_t lo = gemv_nibble_mask(q[k]);
                    const uint32_t hi = gemv_nibble_mask(q[k] >> 4);
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        p = fmaf(gemv_cvt_u8(lo, t), xv[j][4 * k + t], p);
                        p = fmaf(gemv_cvt_u8(hi, t), xv[j][16 + 4 * k + t], p);
                    }
                }
            }
            if constexpr (DT == VGX_Q4_0) p -= off[j];
            acc = fmaf(half_bits_to_float(wsc[s][j]), p, acc);
        }
        if constexpr (DT == VGX_Q8_0) {
            acc += dpp_f<DPP_QUAD_1032>(acc);     // lane ^ 1: the other half of the row
            acc += dpp_f<0x128>(acc);             // row_ror 8: lane ^ 8
        } else {
            acc += dpp_f<0x124>(acc);             // row_ror 4 and 8: the lanes of the same l & 3
            acc += dpp_f<0x128>(acc);
        }
        acc = xor32_sum(xor16_sum(acc)) * inv;
        if constexpr (EPI == EPI_SWIGLU) {
            const float u = __shfl_xor(acc, DT == VGX_Q8_0 ? 4 : 2, kWave);   // row r + 2: the up row
            acc = acc / (1.0f + __expf(-acc)) * u;
        }
        return acc;
    };
    auto store = [&](int i, float v) {
        const uint32_t yo = stores ? (uint32_t)((gw + i * nw) * kOutPerRq + r_out) * 4 : kStreamPastEnd;   // rows >= rows_out: dropped
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrs, yo, 0, 0);
    };
    // Whole ring rounds without a branch (the refills of the last round fetch the remainder and
    // row-quads past the end), then the remainder.
    const int full = cnt / RB * RB;
    for (int i = 0; i < full; i += RB) {
#pragma unroll
        for (int s = 0; s < RB; ++s) {
            const float v = dot(s);
            fetch(s, gw + (i + s + RB) * nw);
            store(i + s, v);
        }
    }
#pragma unroll
    for (int s = 0; s < RB - 1; ++s)
        if (full + s < cnt) store(full + s, dot(s));
}

// One lane's 16-byte piece of a row-quad run against activations staged in LDS as padded blocks
// (kGemvPad floats per block) with Q4_0 block sums x 8: Q4_0 row l & 3 of block blk (32 nibbles), Q8_0
// half l & 1 of row (l >> 1) & 3 of block blk (16 bytes); d * (sum q x [- 8 sum x]).
template <int DT>
__device__ __forceinline__ float gemv_piece_dot(uint4 w, uint32_t sc, const float *xs, const float *xsum, int blk,
                                               int lane) {
    const uint32_t q[4] = {w.x, w.y, w.z, w.w};
    float p = 0.0f;
    if constexpr (DT == VGX_Q4_0) {
        const float4 *xb = reinterpret_cast<const float4 *>(xs + blk * kGemvPad);
        float xv[QK];
#pragma unroll
        for (int j4 = 0; j4 < 8; ++j4) {
            const float4 t = xb[j4];
            xv[4 * j4] = t.x; xv[4 * j4 + 1] = t.y; xv[4 * j4 + 2] = t.z; xv[4 * j4 + 3] = t.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = gemv_nibble_mask(q[k]);
            const uint32_t hi = gemv_nibble_mask(q[k] >> 4);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                p = fmaf(gemv_cvt_u8(lo, t), xv[4 * k + t], p);
                p = fmaf(gemv_cvt_u8(hi, t), xv[16 + 4 * k + t], p);
            }
        }
        p -= xsum[blk];
    } else {
        const float4 *xb = reinterpret_cast<const float4 *>(xs + blk * kGemvPad + (lane & 1) * 16);
        float xv[16];
#pragma unroll
        for (int j4 = 0; j4 < 4; ++j4) {
            const float4 t = xb[j4];
            xv[4 * j4] = t.x; xv[4 * j4 + 1] = t.y; xv[4 * j4 + 2] = t.z; xv[4 * j4 + 3] = t.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int t = 0; t < 4; ++t) p = fmaf(gemv_cvt_s8(q[k], t), xv[4 * k + t], p);
    }
    return half_bits_to_float(sc) * p;
}

// One-row Q8_0 / Q4_0 GEMV over rows of up to MAXB blocks (the down projection, 1536 x 8960: 16 waves
// x 2 row-quads; the o-projection, 1536 x 1536: 4 waves x 1 row-quad): a workgroup of NW waves takes
// RQG row-quads; their runs are cut into 1 KB pieces (Q4_0 16 blocks, Q8_0 8 blocks x 4 rows, the last
// piece of a row-quad partial), and each wave takes every NW-th of the RQG x pieces, one 16-byte
// buffer load per lane and piece (gemv_piece_dot), all requested before the activations are needed.  The activations are staged once per workgroup in LDS, blocks padded to 36
// floats (the 16 blocks a piece reads at once would otherwise share one bank), with their per-block
// sums (the -8 offset term); the lanes of a row and then the waves are summed in a fixed order
// (deterministic).
constexpr int kPiecesMaxBlocks = 320;

template <int DT, int EPI, int NW, int RQG, int MAXB>
__device__ __forceinline__ void gemv1_pieces_body(GemvArgs a, int bid) {
    gemv_resolve_y(a);
    constexpr int QB = gemv_quant_bytes(DT);
    constexpr int BPP = 1024 / (4 * QB);              // blocks per 1 KB piece: 16 (Q4_0) / 8 (Q8_0)
    constexpr int MAXI = (RQG * ((MAXB + BPP - 1) / BPP) + NW - 1) / NW;   // pieces per wave
    extern __shared__ float4 xs4[];                   // [nblk][36] activations, then [nblk] block sums
    float *xs = reinterpret_cast<float *>(xs4);
    __shared__ float red[NW][RQG][4];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = a.nblk, cols = nblk * QK;
    const int npc = (nblk + BPP - 1) / BPP;           // pieces per row-quad
    const int64_t rq0 = (int64_t)bid * RQG;
    const int n_rq = (int)a.n_rq;
    float *xsum = xs + nblk * kGemvPad;
    const int row = DT == VGX_Q8_0 ? (lane >> 1) & 3 : lane & 3;   // the lane's row of the row-quad

    // activations first (their wait then covers no weights), 8 float4 = one block per 8 threads
    const int n4 = cols / 4;
    constexpr int NT = 64 * NW;
    constexpr int XR = (MAXB * 8 + NT - 1) / NT;
    float4 xv4[XR];
#pragma unroll
    for (int u = 0; u < XR; ++u) {
        const int i = tid + NT * u;
        xv4[u] = i < n4 ? reinterpret_cast<const float4 *>(a.x)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    }
    // weights: piece item i = wave + NW k of the workgroup's RQG x npc; past the end: offsets past the
    // buffers (no traffic, zero quants and scales)
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *)a.w, 0, (int)a.soff, 0x00020000);
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(a.w + a.soff), 0, (int)(a.n_rq * nblk * 8), 0x00020000);
    uint4 wq[MAXI];
    uint32_t wsc[MAXI];
    int blk_of[MAXI];
#pragma unroll
    for (int k = 0; k < MAXI; ++k) {
        const int it = wave + NW * k;
        const int rql = it / npc, pc = it - rql * npc;
        const int64_t rq = rq0 + rql;
        const int blk = BPP * pc + (DT == VGX_Q8_0 ? lane >> 3 : lane >> 2);
        const bool ok = it < RQG * npc && rq < n_rq && blk < nblk;
        blk_of[k] = min(blk, nblk - 1);
        const uint32_t qo = ok ? (uint32_t)((rq * nblk + blk) * 4 * QB + row * QB + (DT == VGX_Q8_0 ? (lane & 1) * 16 : 0))
                               : kStreamPastEnd;
        const uint32_t so = ok ? (uint32_t)((rq * nblk + blk) * 8 + row * 2) : kStreamPastEnd;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, qo, 0, kStreamAux);
        wq[k] = make_uint4(v[0], v[1], v[2], v[3]);
        wsc[k] = __builtin_amdgcn_raw_buffer_load_b16(srs, so, 0, kStreamAux);
    }
#pragma unroll
    for (int u = 0; u < XR; ++u) {
        const int i = tid + NT * u;
        const float4 t = xv4[u];
        if (i < n4) xs4[(i >> 3) * (kGemvPad / 4) + (i & 7)] = t;   // padded rows: no bank conflicts
        float s = (t.x + t.y) + (t.z + t.w);        // the block's 8 float4 are 8 consecutive threads
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        s += __shfl_xor(s, 4, kWave);
        if (i < n4 && (i & 7) == 0) xsum[i >> 3] = 8.0f * s;
    }
    __syncthreads();

    float acc[RQG];
#pragma unroll
    for (int r = 0; r < RQG; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXI; ++k) {
        const int it = wave + NW * k;
        if (it >= RQG * npc) break;                   // uniform: the wave's item count
        const float v = gemv_piece_dot<DT>(wq[k], wsc[k], xs, xsum, blk_of[k], lane);
        const int rql = it / npc;
#pragma unroll
        for (int r = 0; r < RQG; ++r)
            if (r == rql) acc[r] += v;
    }
#pragma unroll
    for (int r = 0; r < RQG; ++r) {
        float v = acc[r];
        if constexpr (DT == VGX_Q8_0) {
            v += dpp_f<DPP_QUAD_1032>(v);             // lane ^ 1: the other half of the row
            v += dpp_f<0x128>(v);                     // row_ror 8: lane ^ 8
        } else {
            v += dpp_f<0x124>(v);                     // row_ror 4 and 8: the lanes of the same l & 3
            v += dpp_f<0x128>(v);
        }
        v = xor32_sum(xor16_sum(v));
        if (DT == VGX_Q8_0 ? (lane & 0x39) == 0 : lane < 4) red[wave][r][row] = v;
    }
    __syncthreads();
    if (tid < 4 * RQG) {
        const int rql = tid >> 2, r = tid & 3;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][rql][r];
        const int64_t orow = (rq0 + rql) * 4 + r;
        if (orow < a.rows_out) {
            if (a.bias) v += a.bias[orow];
            if constexpr (EPI == EPI_ACCUM) v += a.y[orow];
            a.y[orow] = v;
        }
    }
}

template <int DT, int EPI, int NW, int RQG, int MAXB>
__global__ __launch_bounds__(64 * NW) void gemv1_pieces_kernel(GemvArgs a) {
    gemv1_pieces_body<DT, EPI, NW, RQG, MAXB>(a, blockIdx.x);
}

// One or two activation rows against F32 weights of up to 160 blocks per row (the segment scorer's fc1,
// 256 x 4608, on the token's features and their habituated copy): the weights are read once for both
// rows.  A workgroup of 16 waves per row-quad; the row-quad's run (512 bytes per block) is cut into 1 KB
// pieces, lane l holding floats 4 (l & 7) .. + 3 of row (l >> 3) & 3 of block 2 p + l / 32, one 16-byte
// buffer load per lane and piece, all requested before the activations (staged once in LDS) are read.
constexpr int kF32PiecesMaxBlocks = 160;
constexpr int kF32PiecesWaves = 16;
constexpr int kScLnF4 = 5;                    // float4 per thread of a scorer row (rows up to 5120 floats)

// The scorer prologue's two rows into LDS (xs4[n * n4 + c]): waves 0-3 build row 0 = LayerNorm(f),
// waves 4-7 row 1 = LayerNorm(f - 0.65 e), each with the arithmetic of layernorm_reg_kernel (256
// threads per row, float4 t + 256 u, wave sums added in wave order) and of ema_habituate_kernel at
// T = 1, so the rows are those of the separate launches bit for bit.  scorer_load requests the
// thread's features, EMA state and LayerNorm weight and bias (before the weights, so that the rows
// do not wait for them); scorer_rows builds the rows.
__device__ __forceinline__ void scorer_load(const GemvArgs &a, float4 (&f)[kScLnF4], float4 (&e)[kScLnF4],
                                            float4 (&g)[kScLnF4], float4 (&b)[kScLnF4]) {
    const int tid = threadIdx.x, n = tid >> 8, t = tid & 255;
    const int n4 = a.nblk * QK / 4;
    // unconditional buffer loads (offsets past the end read zeros): all of them in flight at once
    auto rs = [&](const float *p) { return __builtin_amdgcn_make_buffer_rsrc((void *)p, 0, n4 * 16, 0x00020000); };
    const __amdgpu_buffer_rsrc_t frs = rs(a.x), ers = rs(a.sc_ema), grs = rs(a.lnw), brs = rs(a.sc_lnb);
    auto ld = [&](__amdgpu_buffer_rsrc_t r, uint32_t o) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, o, 0, 0);
        return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
    };
    const bool own_e = n == 1 && !a.sc_first;
#pragma unroll
    for (int u = 0; u < kScLnF4; ++u) {
        const int i = t + u * 256;
        const uint32_t o = n < 2 && i < n4 ? (uint32_t)i * 16 : kStreamPastEnd;
        f[u] = ld(frs, o);
        e[u] = ld(ers, own_e ? o : kStreamPastEnd);
        g[u] = ld(grs, o);
        b[u] = ld(brs, o);
    }
}

__device__ __forceinline__ void scorer_rows(const GemvArgs &a, const float4 (&f)[kScLnF4], const float4 (&e)[kScLnF4],
                                            const float4 (&g)[kScLnF4], const float4 (&b)[kScLnF4], float4 *xs4,
                                            float (*red)[2][4]) {
    const int tid = threadIdx.x, n = tid >> 8, t = tid & 255, w = t >> 6;
    const int dim = a.nblk * QK, n4 = dim / 4;
    const bool own_e = !a.sc_first;
    float4 v[kScLnF4];
#pragma unroll
    for (int u = 0; u < kScLnF4; ++u) {
        v[u] = f[u];
        if (n == 1 && t + u * 256 < n4) {
            const float4 ev = own_e ? e[u] : f[u];
            v[u] = make_float4(hab_of(f[u].x, ev.x), hab_of(f[u].y, ev.y), hab_of(f[u].z, ev.z), hab_of(f[u].w, ev.w));
        }
    }
    if (n < 2) {
        float s = 0.0f;
#pragma unroll
        for (int u = 0; u < kScLnF4; ++u) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
        s = wave_sum(s);
        if ((tid & 63) == 0) red[n][0][w] = s;
    }
    __syncthreads();
    if (n < 2) {
        const float mean = (red[n][0][0] + red[n][0][1] + red[n][0][2] + red[n][0][3]) / (float)dim;
        float q = 0.0f;
#pragma unroll
        for (int u = 0; u < kScLnF4; ++u) {
            if (t + u * 256 < n4) {
                const float p = v[u].x - mean, c = v[u].y - mean, d = v[u].z - mean, r = v[u].w - mean;
                q = fmaf(p, p, fmaf(c, c, fmaf(d, d, fmaf(r, r, q))));
            }
        }
        q = wave_sum(q);
        if ((tid & 63) == 0) red[n][1][w] = q;
    }
    __syncthreads();
    if (n < 2) {
        const float mean = (red[n][0][0] + red[n][0][1] + red[n][0][2] + red[n][0][3]) / (float)dim;
        const float inv = 1.0f / sqrtf((red[n][1][0] + red[n][1][1] + red[n][1][2] + red[n][1][3]) / (float)dim + a.eps);
#pragma unroll
        for (int u = 0; u < kScLnF4; ++u) {
            const int i = t + u * 256;
            if (i < n4)
                xs4[n * n4 + i] = make_float4((v[u].x - mean) * inv * g[u].x + b[u].x, (v[u].y - mean) * inv * g[u].y + b[u].y,
                                              (v[u].z - mean) * inv * g[u].z + b[u].z, (v[u].w - mean) * inv * g[u].w + b[u].w);
        }
    }
}

template <int NB, int EPI, bool SCORER>
__device__ __forceinline__ void gemv_f32_pieces_body(GemvArgs a, int64_t rq) {
    static_assert(!SCORER || (NB == 2 && EPI == EPI_STORE), "the scorer prologue builds two rows");
    gemv_resolve_y(a);
    constexpr int NW = kF32PiecesWaves;
    constexpr int MAXI = (kF32PiecesMaxBlocks / 2 + NW - 1) / NW;   // pieces per wave
    __shared__ float4 xs4[NB * kF32PiecesMaxBlocks * 8];
    __shared__ float red[NW][4][NB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = a.nblk, n4 = nblk * 8;
    const int npc = (nblk + 1) / 2;                   // pieces per row-quad
    const int row = (lane >> 3) & 3;
    // activations (both rows, or the scorer prologue's inputs), then the weights
    constexpr int XR = SCORER ? 1 : (NB * kF32PiecesMaxBlocks * 8 + 64 * NW - 1) / (64 * NW);
    float4 xv[XR];
    constexpr int SF = SCORER ? kScLnF4 : 1;
    float4 sf[SF], se[SF], sg[SF], sb[SF];
    if constexpr (SCORER) {
        scorer_load(a, sf, se, sg, sb);
    } else {
#pragma unroll
        for (int u = 0; u < XR; ++u) {
            const int i = tid + 64 * NW * u, n = i / n4, c = i - n * n4;
            xv[u] = n < NB ? reinterpret_cast<const float4 *>(a.x + n * a.ldx)[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    const __amdgpu_buffer_rsrc_t wrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)a.w, 0, (int)(a.n_rq * nblk * 512), 0x00020000);
    float4 wv[MAXI];
    int blk_of[MAXI];
#pragma unroll
    for (int k = 0; k < MAXI; ++k) {
        const int pc = wave + NW * k;
        const int blk = 2 * pc + (lane >> 5);
        const bool ok = pc < npc && blk < nblk;
        blk_of[k] = min(blk, nblk - 1);
        const uint32_t o = ok ? (uint32_t)((rq * nblk + blk) * 512 + (lane & 31) * 16) : kStreamPastEnd;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, o, 0, kStreamAux);
        wv[k] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
    }
    if constexpr (SCORER) {
        __shared__ float sred[2][2][4];
        scorer_rows(a, sf, se, sg, sb, xs4, sred);
    } else {
#pragma unroll
        for (int u = 0; u < XR; ++u) {
            const int i = tid + 64 * NW * u;
            if (i < NB * n4) xs4[i] = xv[u];
        }
    }
    __syncthreads();
    float acc[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) acc[n] = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXI; ++k) {
        if (wave + NW * k >= npc) break;              // uniform: the wave's piece count
        const float4 w = wv[k];
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            const float4 x = xs4[n * n4 + blk_of[k] * 8 + (lane & 7)];
            acc[n] = fmaf(w.x, x.x, fmaf(w.y, x.y, fmaf(w.z, x.z, fmaf(w.w, x.w, acc[n]))));
        }
    }
#pragma unroll
    for (int n = 0; n < NB; ++n) {
        float v = acc[n];
        v += dpp_f<DPP_QUAD_1032>(v);                 // lanes of the same row: bits 0..2 and 5
        v += dpp_f<DPP_QUAD_2301>(v);
        v += dpp_f<DPP_ROW_HALF_MIRROR>(v);
        v = xor32_sum(v);
        if ((lane & 0x27) == 0) red[wave][row][n] = v;
    }
    __syncthreads();
    if (tid < 4 * NB) {
        const int r = tid >> (NB == 2 ? 1 : 0), n = NB == 2 ? tid & 1 : 0;
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][r][n];
        const int64_t orow = rq * 4 + r;
        if (orow < a.rows_out) {
            if (a.bias) v += a.bias[orow];
            if constexpr (EPI == EPI_ACCUM) v += a.y[n * a.ldy + orow];
            a.y[n * a.ldy + orow] = v;
        }
    }
}

template <int NB, int EPI, bool SCORER = false>
__global__ __launch_bounds__(64 * kF32PiecesWaves) void gemv_f32_pieces_kernel(GemvArgs a) {
    gemv_f32_pieces_body<NB, EPI, SCORER>(a, blockIdx.x);
}

// The decode token's segment scorer as two jobs of 1024-thread workgroups, each either launched on its
// own (score_side_kernel) or carried by the spare workgroups of a 16-wave GEMV launch (the down
// projection of a later layer leaves a quarter of the CUs idle at batch 1), so that neither adds a
// launch to the step.  Phase 1: the fc1 GEMV with the LayerNorm prologue, one workgroup per row-quad
// (gemv_f32_pieces_body).  Phase 2: the tail (score_tail_kernel's arithmetic at T = 1, first wave of
// workgroup 0) and the EMA update (ema_habituate_kernel's at T = 1), 1024 features per workgroup.
struct ScoreSide {
    int phase;                  // 1 or 2
    GemvArgs fc1;               // phase 1: x = the features, y = h
    const float *h;             // phase 2: the fc1 outputs, [2][hidden]
    int64_t hidden;
    const float *w2, *b2;
    int first;
    float *out;
    const int32_t *out_index;   // may be null: added to out
    const float *f;             // the features
    float *ema;
    int64_t fd;
};

inline int64_t score_side_blocks(const ScoreSide &s) { return s.phase == 1 ? s.fc1.n_rq : 1 + (s.fd + 1023) / 1024; }

__device__ __forceinline__ void score_tail_body(const ScoreSide &s, int bid) {
    if (bid == 0) {
        if (threadIdx.x >= 64) return;
        float *out = s.out + (s.out_index ? *s.out_index : 0);
        float r = 0.0f, a = 0.0f;
        for (int64_t i = threadIdx.x; i < s.hidden; i += 64) {
            const float x0 = s.h[i], x1 = s.h[s.hidden + i];
            r = fmaf(ref_geluf(x0), s.w2[i], r);
            a = fmaf(ref_geluf(x1), s.w2[i], a);
        }
        r = wave_sum(r) + s.b2[0];
        a = wave_sum(a) + s.b2[0];
        if (threadIdx.x == 0) out[0] = s.first ? r : r + 0.35f * fmaxf(0.0f, a - r);
        return;
    }
    const int64_t i = (int64_t)(bid - 1) * 1024 + threadIdx.x;
    if (i >= s.fd) return;
    const float fv = s.f[i];
    s.ema[i] = s.first ? fv : ema_step(s.ema[i], fv);
}

__device__ __forceinline__ void score_side_run(const ScoreSide &s, int bid) {
    if (s.phase == 1) gemv_f32_pieces_body<2, EPI_STORE, true>(s.fc1, bid);
    else score_tail_body(s, bid);
}

// Checks of a scorer job against what its kernels assume (phase 1: the prologue's row width and
// alignment, the F32 pieces layout; phase 2: pointers).
inline int score_side_check(const ScoreSide &s) {
    if (s.phase == 1) {
        const GemvArgs &a = s.fc1;
        if (!a.w || !a.x || !a.sc_ema || !a.lnw || !a.sc_lnb || !a.y) return VGX_E_ARG;
        if (a.batch != 2 || a.epi != EPI_STORE || a.nblk <= 0 || a.nblk > kF32PiecesMaxBlocks ||
            a.nblk * QK > 256 * 4 * kScLnF4 || a.n_rq <= 0 || a.n_rq * a.nblk * 512 >= ((int64_t)1 << 31))
            return VGX_E_LIMIT;
        if ((((uintptr_t)a.x | (uintptr_t)a.sc_ema | (uintptr_t)a.lnw | (uintptr_t)a.sc_lnb) & 15) != 0)
            return VGX_E_ALIGN;
        return VGX_OK;
    }
    if (s.phase == 2) return s.h && s.w2 && s.b2 && s.out && s.f && s.ema && s.hidden > 0 && s.fd > 0 ? VGX_OK : VGX_E_ARG;
    return VGX_E_ARG;
}

// A scorer job from its C description (include/vault_amd.h: vgx_score_side), checked.
inline int make_score_side(const vgx_score_side &c, ScoreSide &s) {
    if (c.phase != 1 && c.phase != 2) return VGX_E_ARG;
    if (c.fd <= 0 || c.hidden <= 0 || c.fd % QK || !(c.eps > 0.0f)) return VGX_E_SIZE;
    if (!c.feat || !c.ema || !c.w1 || !c.b1 || !c.ln_w || !c.ln_b || !c.w2 || !c.b2 || !c.h || !c.out) return VGX_E_ARG;
    s = ScoreSide{};
    s.phase = c.phase;
    GemvArgs &a = s.fc1;
    a.w = static_cast<const uint8_t *>(c.w1);
    a.nblk = (int)(c.fd / QK);
    a.n_rq = (c.hidden + 3) / 4;
    a.rows_out = c.hidden;
    a.x = c.feat;
    a.ldx = c.fd;
    a.batch = 2;
    a.lnw = c.ln_w;
    a.eps = c.eps;
    a.bias = c.b1;
    a.y = c.h;
    a.ldy = c.hidden;
    a.epi = EPI_STORE;
    a.sc_ema = c.ema;
    a.sc_lnb = c.ln_b;
    a.sc_first = c.first ? 1 : 0;
    s.h = c.h;
    s.hidden = c.hidden;
    s.w2 = c.w2;
    s.b2 = c.b2;
    s.first = c.first ? 1 : 0;
    s.out = c.out;
    s.out_index = c.out_index;
    s.f = c.feat;
    s.ema = c.ema;
    s.fd = c.fd;
    return score_side_check(s);
}

// Launches a scorer job on its own (score_side_kernel, defined once in qlinear.hip).
int vgx_detail_score_side(const ScoreSide &s, hipStream_t st);

// The 16-wave pieces GEMV with a scorer job in workgroups main_blocks.. of the same launch.
template <int DT, int EPI, int RQG, int MAXB>
__global__ __launch_bounds__(1024) void gemv1_pieces_side_kernel(GemvArgs a, ScoreSide s, int main_blocks) {
    if ((int)blockIdx.x < main_blocks) gemv1_pieces_body<DT, EPI, 16, RQG, MAXB>(a, blockIdx.x);
    else score_side_run(s, (int)blockIdx.x - main_blocks);
}

constexpr int kGemv1MaxBlocks = 448;   // LDS staging of one row: 448 * 36 * 4 B = 63 KB

// Returns whether a scorer job (a.side) went with the launch; otherwise the caller launches it.
template <int DT, int EPI, bool NORM>
bool gemv1_launch(const GemvArgs &a, hipStream_t st) {
    const size_t lds = (size_t)a.nblk * kGemvPad * sizeof(float);
#define VGX_GEMV1(LPR, WPG, KW, U, SF, XD)                                                              \
    hipLaunchKernelGGL((gemv1_kernel<DT, EPI, NORM, LPR, WPG, KW, U, SF, XD>),                           \
                       dim3((unsigned)((a.n_rq + WPG * (64 / LPR) - 1) / (WPG * (64 / LPR)))),              \
                       dim3(64 * WPG * KW), XD ? 0 : lds, st, a)
    const bool aligned = ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.lnw & 15) == 0;
    if constexpr ((EPI == EPI_STORE || EPI == EPI_SWIGLU) && gemv_quant(DT)) {
        if (a.nblk == kStreamBlocks && !a.bias && a.n_rq >= kStreamMinRq && a.soff < ((int64_t)1 << 31) && aligned) {
            const unsigned grid = (unsigned)std::min<int64_t>(StreamGeom<DT>::GROUPS, (a.n_rq + 3) / 4);
            hipLaunchKernelGGL((gemv1_stream_kernel<DT, EPI, NORM>), dim3(grid), dim3(256), 0, st, a);
            return false;
        }
    }
    if constexpr (gemv_quant(DT) && !NORM && (EPI == EPI_STORE || EPI == EPI_ACCUM)) {
        if (a.nblk >= 192 && a.nblk <= kPiecesMaxBlocks && a.soff < ((int64_t)1 << 31) && aligned) {
            // 16 waves x 2 row-quads: 5.5 us for 1536 x 8960 (8 x 2: 5.8, 8 x 1: 6.0, 16 x 1: 5.9, 16 x 4: 7.3,
            // 4 x 1: 6.8; the lane-per-block kernel: 6.6)
            constexpr int NW = 16, RQG = 2;
            const unsigned main = (unsigned)((a.n_rq + RQG - 1) / RQG);
            const size_t lds = (size_t)(a.nblk * kGemvPad + a.nblk) * sizeof(float);
            if (a.side != nullptr)
                hipLaunchKernelGGL((gemv1_pieces_side_kernel<DT, EPI, RQG, kPiecesMaxBlocks>),
                                   dim3(main + (unsigned)score_side_blocks(*a.side)), dim3(64 * NW), lds, st, a, *a.side,
                                   (int)main);
            else
                hipLaunchKernelGGL((gemv1_pieces_kernel<DT, EPI, NW, RQG, kPiecesMaxBlocks>), dim3(main), dim3(64 * NW),
                                   lds, st, a);
            return a.side != nullptr;
        }
    }
    if constexpr (gemv_quant(DT) && !NORM && (EPI == EPI_STORE || EPI == EPI_ACCUM)) {
        if (a.nblk == kStreamBlocks && a.n_rq < kStreamMinRq && a.soff < ((int64_t)1 << 31) && aligned) {
            // 1536-column rows (the o-projection, 1536 x 1536): a workgroup of 4 waves per row-quad, one 1 KB
            // piece per wave (3 of them busy): 3.2 us against 4.2 us for the lane-per-block kernel (2 x 2: 3.7,
            // 4 x 2: 3.6, 3 x 1: 3.2, 6 x 2: 3.4, 8 x 4: 3.6)
            hipLaunchKernelGGL((gemv1_pieces_kernel<DT, EPI, 4, 1, kStreamBlocks>), dim3((unsigned)a.n_rq), dim3(256),
                               (size_t)(a.nblk * kGemvPad + a.nblk) * sizeof(float), st, a);
            return false;
        }
    }
    constexpr int UT = gemv_half(DT) ? 1 : 3;                           // BF16 / F16 blocks are 64 registers
    if (a.n_rq >= 16384) VGX_GEMV1(16, 4, 1, UT, false, false);       // other tall weights: DPP row per row-quad
    else if (a.n_rq >= 2048) VGX_GEMV1(64, 4, 1, 1, true, false);     // lane per block (gate/up before the streaming kernel)
    else if (a.nblk >= 192) {
        if constexpr (gemv_half(DT)) VGX_GEMV1(64, 1, 8, 1, true, false);   // 64-register blocks: 512 threads
        else VGX_GEMV1(64, 2, 8, 1, true, false);                     // long rows (Q8_0, fused norm, or beyond the
                                                                      // pieces kernel): 2 row-quads x 8 waves over K
                                                                      // (6.6 us; one row-quad 6.9 us, direct
                                                                      // activations 7.0 us)
    }
    else if (a.nblk >= 96 && a.n_rq < 256) VGX_GEMV1(64, 1, 8, 1, true, false);   // few rows: more waves
    else if (a.nblk >= 96) VGX_GEMV1(64, 1, 2, 1, true, false);
    else if (aligned && !gemv_plain(DT)) VGX_GEMV1(64, 1, 1, 1, false, true);   // small: direct
    else VGX_GEMV1(64, 2, 1, 1, true, false);
#undef VGX_GEMV1
    return false;
}

// Launch the GEMV over all batch rows.  A single row (the decode step) runs gemv1_kernel; more rows
// run qgemv_kernel in passes of up to 4, in row mode (16 lanes per row-quad, 4 waves per workgroup)
// for >= 2048 row-quads, else in split-K mode (one wave per row-quad).
template <int DT>
int qgemv_launch_impl(GemvArgs a, hipStream_t st, bool &carried) {
    const bool rows_mode = a.n_rq >= 2048;
    const bool norm = a.lnw != nullptr;
    if constexpr (DT == VGX_F32) {
        if (a.batch <= 2 && !norm && a.epi != EPI_SWIGLU && a.nblk <= kF32PiecesMaxBlocks &&
            a.n_rq * a.nblk * 512 < ((int64_t)1 << 31) && ((uintptr_t)a.x & 15) == 0 && a.ldx % 4 == 0) {
#define VGX_F32P(NB, EPIV) hipLaunchKernelGGL((gemv_f32_pieces_kernel<NB, EPIV>), dim3((unsigned)a.n_rq), dim3(64 * kF32PiecesWaves), 0, st, a)
            if (a.batch == 2) { if (a.epi == EPI_ACCUM) VGX_F32P(2, EPI_ACCUM); else VGX_F32P(2, EPI_STORE); }
            else { if (a.epi == EPI_ACCUM) VGX_F32P(1, EPI_ACCUM); else VGX_F32P(1, EPI_STORE); }
#undef VGX_F32P
            return hipGetLastError() == hipSuccess ? VGX_OK : VGX_E_HIP;
        }
    }
    if (a.batch == 1 && a.nblk <= kGemv1MaxBlocks && ((uintptr_t)a.x & 15) == 0 && ((uintptr_t)a.lnw & 15) == 0) {
        if (a.epi == EPI_SWIGLU) carried = norm ? gemv1_launch<DT, EPI_SWIGLU, true>(a, st) : gemv1_launch<DT, EPI_SWIGLU, false>(a, st);
        else if (a.epi == EPI_ACCUM) carried = norm ? gemv1_launch<DT, EPI_ACCUM, true>(a, st) : gemv1_launch<DT, EPI_ACCUM, false>(a, st);
        else carried = norm ? gemv1_launch<DT, EPI_STORE, true>(a, st) : gemv1_launch<DT, EPI_STORE, false>(a, st);
        return hipGetLastError() == hipSuccess ? VGX_OK : VGX_E_HIP;
    }
    for (int64_t b0 = 0; b0 < a.batch; b0 += 4) {
        GemvArgs p = a;
        const int nb = (int)std::min<int64_t>(4, a.batch - b0);
        p.x = a.x + b0 * a.ldx;
        if (a.y_ref != nullptr) p.y_off = a.y_off + b0 * a.ldy;
        else p.y = a.y + b0 * a.ldy;
        const int cbk = std::min(a.nblk, kGemvMaxChunkFloats / (QK * nb));
        const size_t lds = (size_t)nb * cbk * kGemvPad * sizeof(float);
        const unsigned grid = rows_mode ? (unsigned)((a.n_rq + 15) / 16) : (unsigned)a.n_rq;
        const unsigned threads = rows_mode ? 256u : 64u;
#define VGX_GEMV_GO(NBV, EPIV, MODEV, KWV, NORMV)                                                      \
    hipLaunchKernelGGL((qgemv_kernel<DT, NBV, EPIV, MODEV, KWV, NORMV>), dim3(grid), dim3(threads), lds, st, p, cbk)
#define VGX_GEMV_K1(NBV, EPIV, NORMV)                                                                  \
    do {                                                                                               \
        if (rows_mode) VGX_GEMV_GO(NBV, EPIV, MODE_ROWS, 1, NORMV);                                    \
        else VGX_GEMV_GO(NBV, EPIV, MODE_SPLITK, 1, NORMV);                                            \
    } while (0)
#define VGX_GEMV_EPI(NBV, SEL)                                                                         \
    do {                                                                                               \
        if (a.epi == EPI_SWIGLU) { if (norm) SEL(NBV, EPI_SWIGLU, true); else SEL(NBV, EPI_SWIGLU, false); } \
        else if (a.epi == EPI_ACCUM) { if (norm) SEL(NBV, EPI_ACCUM, true); else SEL(NBV, EPI_ACCUM, false); } \
        else { if (norm) SEL(NBV, EPI_STORE, true); else SEL(NBV, EPI_STORE, false); } \
    } while (0)
        switch (nb) {
            case 1: VGX_GEMV_EPI(1, VGX_GEMV_K1); break;
            case 2: VGX_GEMV_EPI(2, VGX_GEMV_K1); break;
            case 3: VGX_GEMV_EPI(3, VGX_GEMV_K1); break;
            default: VGX_GEMV_EPI(4, VGX_GEMV_K1); break;
        }
#undef VGX_GEMV_EPI
#undef VGX_GEMV_K1
#undef VGX_GEMV_GO
        if (hipGetLastError() != hipSuccess) return VGX_E_HIP;
    }
    return VGX_OK;
}

// The GEMV, then a scorer job (a.side) that did not go with its launch.
template <int DT>
int qgemv_launch(GemvArgs a, hipStream_t st) {
    bool carried = false;
    const int rc = qgemv_launch_impl<DT>(a, st, carried);
    if (rc != VGX_OK || a.side == nullptr || carried) return rc;
    return vgx_detail_score_side(*a.side, st);
}

}  // namespace vgx

// One launcher per weight dtype (defined in qgemv_q8.hip / qgemv_q4.hip / qgemv_f32.hip /
// qgemv_bf16.hip / qgemv_f16.hip).
int vgx_detail_qgemv_q8(const vgx::GemvArgs &a, hipStream_t st);
int vgx_detail_qgemv_q4(const vgx::GemvArgs &a, hipStream_t st);
int vgx_detail_qgemv_f32(const vgx::GemvArgs &a, hipStream_t st);
int vgx_detail_qgemv_bf16(const vgx::GemvArgs &a, hipStream_t st);
int vgx_detail_qgemv_f16(const vgx::GemvArgs &a, hipStream_t st);
