// Q8_0 / Q4_0 / F32 weights on gfx950: packing, bit-exact dequant, embedding rows and the
// HBM-streaming GEMV (batch 1..4 per pass) with fused bias / residual / SwiGLU epilogues.
//
// Reference semantics: runtime/vault3.c:499-654 (row_dot, matvec, embed_row), 1942-1956
// (mlp_gu_run); tools/vlt3.py:98-157 (block layouts and dequantization).
//
// GEMV mapping.  A wave owns 4 row-quads (16 rows); each 16-lane DPP row of the wave owns one
// row-quad and walks its 32-weight blocks with stride 16 (lane l16 takes blocks l16, l16+16, ...).
// Per block a lane issues one contiguous 64-byte (Q4_0) / 128-byte (Q8_0) load covering the four
// rows, one 8-byte scale load, and reads the 32 activations of that block from LDS once for all
// four rows.  The 16 lanes of a row-quad read 16 consecutive blocks: 1 KiB (Q4_0) / 2 KiB (Q8_0)
// contiguous per wave-row per step.  Partial sums are reduced across the 16 lanes with DPP.
//
// Arithmetic is fp32 throughout, as in the reference: per block s = sum_j q_j x_j, acc += d * s.
// Q4_0 nibbles n are converted unsigned (v_cvt_f32_ubyte*) and the -8 offset is applied once per
// block as acc += d * (sum_j n_j x_j - 8 * sum_j x_j), with sum_j x_j staged in LDS per block.
#include "common.h"

using namespace vgx;

namespace {

constexpr int kMaxChunkFloats = 8192;  // activations staged in LDS per chunk (all batch rows)
constexpr int kPad = 36;               // floats per staged 32-float block (4 floats of padding)

__host__ __device__ constexpr int quant_bytes(int dt) {
    return dt == VGX_Q8_0 ? 32 : dt == VGX_Q4_0 ? 16 : dt == VGX_F32 ? 128 : 0;
}
__host__ __device__ constexpr int aos_bytes(int dt) { return dt == VGX_Q8_0 ? 34 : dt == VGX_Q4_0 ? 18 : 0; }

inline int64_t rows4(int64_t r) { return (r + 3) / 4 * 4; }

inline bool dtype_ok(int dt) { return dt == VGX_Q8_0 || dt == VGX_Q4_0 || dt == VGX_F32; }

int64_t scale_off(int dt, int64_t rows, int64_t cols) {
    const int64_t q = rows4(rows) * (cols / QK) * quant_bytes(dt);
    return (q + 255) / 256 * 256;
}

int64_t packed_bytes(int dt, int64_t rows, int64_t cols) {
    if (dt == VGX_F32) return rows4(rows) * cols * 4;
    return scale_off(dt, rows, cols) + rows4(rows) * (cols / QK) * 2;
}

// ------------------------------------------------------------------------------------------
// packing
// ------------------------------------------------------------------------------------------

// One thread per (packed row p, block b).  mode 0: packed row p <- source row p of `a`.
// mode 1 (gate/up): packed row-quad q holds a[2q], a[2q+1], b[2q], b[2q+1].
template <int DT>
__global__ void pack_kernel(const uint8_t *__restrict__ a, const uint8_t *__restrict__ bsrc,
                            uint8_t *__restrict__ dst, int64_t src_rows, int64_t nblk, int64_t soff,
                            int64_t total, int mode) {
    constexpr int QB = quant_bytes(DT);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t p = i / nblk, b = i - p * nblk;
    const int64_t rq = p >> 2, rr = p & 3;
    const uint8_t *src = a;
    int64_t r = p;
    if (mode == 1) {
        r = 2 * rq + (rr & 1);
        src = rr < 2 ? a : bsrc;
    }
    uint8_t *qd = dst + ((rq * nblk + b) * 4 + rr) * QB;
    const bool live = r < src_rows;
    if constexpr (DT == VGX_F32) {
        const float *s = reinterpret_cast<const float *>(src) + r * nblk * QK + b * QK;
        float *d = reinterpret_cast<float *>(qd);
        for (int j = 0; j < QK; ++j) d[j] = live ? s[j] : 0.0f;
    } else {
        uint16_t *sd = reinterpret_cast<uint16_t *>(dst + soff) + (rq * nblk + b) * 4 + rr;
        const uint8_t *s = src + (r * nblk + b) * aos_bytes(DT);
        *sd = live ? (uint16_t)(s[0] | (s[1] << 8)) : (uint16_t)0;
        for (int j = 0; j < QB; ++j) qd[j] = live ? s[2 + j] : (uint8_t)0;
    }
}

template <int DT>
__global__ void unpack_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int64_t rows,
                              int64_t nblk, int64_t soff) {
    constexpr int QB = quant_bytes(DT);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nblk) return;
    const int64_t r = i / nblk, b = i - r * nblk;
    const int64_t rq = r >> 2, rr = r & 3;
    const uint8_t *qs = src + ((rq * nblk + b) * 4 + rr) * QB;
    if constexpr (DT == VGX_F32) {
        float *d = reinterpret_cast<float *>(dst) + r * nblk * QK + b * QK;
        const float *s = reinterpret_cast<const float *>(qs);
        for (int j = 0; j < QK; ++j) d[j] = s[j];
    } else {
        const uint16_t sc = reinterpret_cast<const uint16_t *>(src + soff)[(rq * nblk + b) * 4 + rr];
        uint8_t *d = dst + (r * nblk + b) * aos_bytes(DT);
        d[0] = (uint8_t)(sc & 0xFF);
        d[1] = (uint8_t)(sc >> 8);
        for (int j = 0; j < QB; ++j) d[2 + j] = qs[j];
    }
}

// Dequantize one 32-weight block of packed row r into out[0..31].
template <int DT>
__device__ __forceinline__ void dequant_block(const uint8_t *__restrict__ w, int64_t nblk, int64_t soff, int64_t r,
                                              int64_t b, float *__restrict__ out) {
    constexpr int QB = quant_bytes(DT);
    const int64_t rq = r >> 2, rr = r & 3;
    const uint8_t *qs = w + ((rq * nblk + b) * 4 + rr) * QB;
    if constexpr (DT == VGX_F32) {
        const float *s = reinterpret_cast<const float *>(qs);
        for (int j = 0; j < QK; ++j) out[j] = s[j];
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

template <int DT>
__global__ void dequant_kernel(const uint8_t *__restrict__ w, float *__restrict__ out, int64_t rows, int64_t nblk,
                               int64_t soff) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nblk) return;
    const int64_t r = i / nblk, b = i - r * nblk;
    dequant_block<DT>(w, nblk, soff, r, b, out + r * nblk * QK + b * QK);
}

template <int DT>
__global__ void embed_kernel(const uint8_t *__restrict__ w, const int64_t *__restrict__ ids, float *__restrict__ out,
                             int64_t ldo, int64_t rows, int64_t nblk, int64_t soff, int64_t n_ids, int64_t pad_row) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_ids * nblk) return;
    const int64_t t = i / nblk, b = i - t * nblk;
    int64_t r = ids[t];
    if (r < 0 || r >= rows) r = pad_row;
    dequant_block<DT>(w, nblk, soff, r, b, out + t * ldo + b * QK);
}

// ------------------------------------------------------------------------------------------
// GEMV
// ------------------------------------------------------------------------------------------

enum { EPI_STORE = 0, EPI_ACCUM = 1, EPI_SWIGLU = 2 };

__device__ __forceinline__ float cvt_u8(uint32_t w, int k) {
    // Each pattern maps onto one v_cvt_f32_ubyte{0..3}.
    switch (k) {
        case 0: return (float)(w & 0xFFu);
        case 1: return (float)((w >> 8) & 0xFFu);
        case 2: return (float)((w >> 16) & 0xFFu);
        default: return (float)(w >> 24);
    }
}

__device__ __forceinline__ float cvt_s8(uint32_t w, int k) { return (float)(int)(int8_t)(w >> (8 * k)); }

// w & 0x0F0F0F0F, opaque to the optimiser: otherwise each later byte extract is folded back
// into a per-nibble v_bfe_u32, doubling the conversion cost.  With the mask opaque, every
// nibble converts with a single v_cvt_f32_ubyte{0..3}.
__device__ __forceinline__ uint32_t nibble_mask(uint32_t w) {
    uint32_t r;
    asm("v_and_b32 %0, 0x0f0f0f0f, %1" : "=v"(r) : "v"(w));
    return r;
}

template <int DT, int NB, int EPI>
__global__ __launch_bounds__(256) void qgemv_kernel(const uint8_t *__restrict__ W, int nblk, int64_t soff,
                                                     int64_t n_rq, const float *__restrict__ x, int64_t ldx,
                                                     const float *__restrict__ bias, float *__restrict__ y,
                                                     int64_t ldy, int64_t rows_out, int cbk, int vec_x) {
    extern __shared__ float smem[];
    float *xs = smem;                       // [NB][cbk][kPad]
    float *xsum = smem + NB * cbk * kPad;   // [NB][cbk]
    constexpr int QB = quant_bytes(DT);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int l16 = lane & 15;
    const int qtr = lane >> 4;
    const int waves = blockDim.x >> 6;
    const int64_t rq = ((int64_t)blockIdx.x * waves + wave) * 4 + qtr;
    const bool act = rq < n_rq;

    float acc[4][NB];
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[r][n] = 0.0f;

    for (int c0 = 0; c0 < nblk; c0 += cbk) {
        const int cb = min(cbk, nblk - c0);
        if (c0) __syncthreads();
        if (vec_x) {
            for (int i = threadIdx.x; i < NB * cb * 8; i += blockDim.x) {
                const int n = i / (cb * 8), rem = i - n * cb * 8, blk = rem >> 3, j4 = rem & 7;
                const float4 v = *reinterpret_cast<const float4 *>(x + n * ldx + (int64_t)(c0 + blk) * QK + j4 * 4);
                *reinterpret_cast<float4 *>(xs + (n * cbk + blk) * kPad + j4 * 4) = v;
            }
        } else {
            for (int i = threadIdx.x; i < NB * cb * QK; i += blockDim.x) {
                const int n = i / (cb * QK), rem = i - n * cb * QK, blk = rem >> 5, j = rem & 31;
                xs[(n * cbk + blk) * kPad + j] = x[n * ldx + (int64_t)(c0 + blk) * QK + j];
            }
        }
        __syncthreads();
        if constexpr (DT == VGX_Q4_0) {
            for (int i = threadIdx.x; i < NB * cb; i += blockDim.x) {
                const int n = i / cb, blk = i - n * cb;
                const float *p = xs + (n * cbk + blk) * kPad;
                float s = 0.0f;
#pragma unroll
                for (int j = 0; j < QK; ++j) s += p[j];
                xsum[n * cbk + blk] = s;
            }
            __syncthreads();
        }
        if (!act) continue;
        for (int b = l16; b < cb; b += 16) {
            const int64_t gb = c0 + b;
            const uint8_t *qp = W + (rq * nblk + gb) * 4 * QB;
            if constexpr (DT == VGX_Q4_0) {
                uint4 qv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) qv[r] = reinterpret_cast<const uint4 *>(qp)[r];
                const uint2 sv = *reinterpret_cast<const uint2 *>(W + soff + (rq * nblk + gb) * 8);
                const float d[4] = {half_bits_to_float(sv.x), half_bits_to_float(sv.x >> 16),
                                    half_bits_to_float(sv.y), half_bits_to_float(sv.y >> 16)};
#pragma unroll
                for (int n = 0; n < NB; ++n) {
                    const float *xb = xs + (n * cbk + b) * kPad;
                    float xv[QK];
#pragma unroll
                    for (int j4 = 0; j4 < 8; ++j4) {
                        const float4 t = *reinterpret_cast<const float4 *>(xb + j4 * 4);
                        xv[j4 * 4 + 0] = t.x; xv[j4 * 4 + 1] = t.y; xv[j4 * 4 + 2] = t.z; xv[j4 * 4 + 3] = t.w;
                    }
                    const float s8 = 8.0f * xsum[n * cbk + b];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t wq[4] = {qv[r].x, qv[r].y, qv[r].z, qv[r].w};
                        float s = 0.0f;
#pragma unroll
                        for (int k = 0; k < 4; ++k) {
                            const uint32_t lo = nibble_mask(wq[k]);
                            const uint32_t hi = nibble_mask(wq[k] >> 4);
#pragma unroll
                            for (int t = 0; t < 4; ++t) {
                                s = fmaf(cvt_u8(lo, t), xv[4 * k + t], s);
                                s = fmaf(cvt_u8(hi, t), xv[16 + 4 * k + t], s);
                            }
                        }
                        acc[r][n] = fmaf(d[r], s - s8, acc[r][n]);
                    }
                }
            } else if constexpr (DT == VGX_Q8_0) {
                uint4 qv[4][2];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    qv[r][0] = reinterpret_cast<const uint4 *>(qp)[2 * r];
                    qv[r][1] = reinterpret_cast<const uint4 *>(qp)[2 * r + 1];
                }
                const uint2 sv = *reinterpret_cast<const uint2 *>(W + soff + (rq * nblk + gb) * 8);
                const float d[4] = {half_bits_to_float(sv.x), half_bits_to_float(sv.x >> 16),
                                    half_bits_to_float(sv.y), half_bits_to_float(sv.y >> 16)};
#pragma unroll
                for (int n = 0; n < NB; ++n) {
                    const float *xb = xs + (n * cbk + b) * kPad;
                    float xv[QK];
#pragma unroll
                    for (int j4 = 0; j4 < 8; ++j4) {
                        const float4 t = *reinterpret_cast<const float4 *>(xb + j4 * 4);
                        xv[j4 * 4 + 0] = t.x; xv[j4 * 4 + 1] = t.y; xv[j4 * 4 + 2] = t.z; xv[j4 * 4 + 3] = t.w;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const uint32_t wq[8] = {qv[r][0].x, qv[r][0].y, qv[r][0].z, qv[r][0].w,
                                                qv[r][1].x, qv[r][1].y, qv[r][1].z, qv[r][1].w};
                        float s = 0.0f;
#pragma unroll
                        for (int k = 0; k < 8; ++k)
#pragma unroll
                            for (int t = 0; t < 4; ++t) s = fmaf(cvt_s8(wq[k], t), xv[4 * k + t], s);
                        acc[r][n] = fmaf(d[r], s, acc[r][n]);
                    }
                }
            } else {  // F32 weights
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    float wv[QK];
#pragma unroll
                    for (int j4 = 0; j4 < 8; ++j4) {
                        const float4 t = reinterpret_cast<const float4 *>(qp + r * QB)[j4];
                        wv[j4 * 4 + 0] = t.x; wv[j4 * 4 + 1] = t.y; wv[j4 * 4 + 2] = t.z; wv[j4 * 4 + 3] = t.w;
                    }
#pragma unroll
                    for (int n = 0; n < NB; ++n) {
                        const float *xb = xs + (n * cbk + b) * kPad;
                        float s = 0.0f;
#pragma unroll
                        for (int j = 0; j < QK; ++j) s = fmaf(wv[j], xb[j], s);
                        acc[r][n] += s;
                    }
                }
            }
        }
    }

#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[r][n] = row16_sum(acc[r][n]);

    if (!act || l16 != 0) return;
    if constexpr (EPI == EPI_SWIGLU) {
        const int64_t o0 = rq * 2;
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (o0 + k >= rows_out) continue;
                const float g = acc[k][n], u = acc[2 + k][n];
                y[n * ldy + o0 + k] = g / (1.0f + __expf(-g)) * u;
            }
    } else {
        const int64_t r0 = rq * 4;
#pragma unroll
        for (int n = 0; n < NB; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = r0 + r;
                if (row >= rows_out) continue;
                float v = acc[r][n];
                if (bias) v += bias[row];
                if constexpr (EPI == EPI_ACCUM) v += y[n * ldy + row];
                y[n * ldy + row] = v;
            }
    }
}

template <int DT, int EPI>
int launch_qgemv_dt(const void *w, int64_t rows_packed, int64_t rows_out, int64_t cols, const float *x,
                    int64_t ldx, int64_t batch, const float *bias, float *y, int64_t ldy, hipStream_t st) {
    const int nblk = (int)(cols / QK);
    const int64_t n_rq = rows4(rows_packed) / 4;
    const int64_t soff = DT == VGX_F32 ? 0 : scale_off(DT, rows_packed, cols);
    // Small matrices: one wave per workgroup spreads the few row-quads over more CUs.
    const int waves = n_rq >= 4096 ? 4 : 1;
    const int64_t grid = (n_rq + waves * 4 - 1) / (waves * 4);
    for (int64_t b0 = 0; b0 < batch; b0 += 4) {
        const int nb = (int)std::min<int64_t>(4, batch - b0);
        const int cbk = std::min(nblk, kMaxChunkFloats / (QK * nb));
        const size_t lds = (size_t)nb * cbk * (kPad + 1) * sizeof(float);
        const float *xb = x + b0 * ldx;
        float *yb = y + b0 * ldy;
        const int vec = ((reinterpret_cast<uintptr_t>(xb) & 15) == 0) && (ldx % 4 == 0);
#define VGX_QGEMV_CASE(NBV)                                                                               \
    case NBV:                                                                                             \
        hipLaunchKernelGGL((qgemv_kernel<DT, NBV, EPI>), dim3((unsigned)grid), dim3(64 * waves), lds, st,    \
                           static_cast<const uint8_t *>(w), nblk, soff, n_rq, xb, ldx, bias, yb, ldy, rows_out, \
                           cbk, vec);                                                                     \
        break;
        switch (nb) {
            VGX_QGEMV_CASE(1)
            VGX_QGEMV_CASE(2)
            VGX_QGEMV_CASE(3)
            VGX_QGEMV_CASE(4)
        }
#undef VGX_QGEMV_CASE
        VGX_CHECK_LAUNCH();
    }
    return VGX_OK;
}

template <int EPI>
int launch_qgemv(int dt, const void *w, int64_t rows_packed, int64_t rows_out, int64_t cols, const float *x,
                 int64_t ldx, int64_t batch, const float *bias, float *y, int64_t ldy, hipStream_t st) {
    switch (dt) {
        case VGX_Q4_0: return launch_qgemv_dt<VGX_Q4_0, EPI>(w, rows_packed, rows_out, cols, x, ldx, batch, bias, y, ldy, st);
        case VGX_Q8_0: return launch_qgemv_dt<VGX_Q8_0, EPI>(w, rows_packed, rows_out, cols, x, ldx, batch, bias, y, ldy, st);
        case VGX_F32: return launch_qgemv_dt<VGX_F32, EPI>(w, rows_packed, rows_out, cols, x, ldx, batch, bias, y, ldy, st);
    }
    return VGX_E_DTYPE;
}

inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

}  // namespace

extern "C" {

int vgx_abi_version(void) { return VGX_ABI_VERSION; }

int64_t vgx_qweight_packed_bytes(int dtype, int64_t rows, int64_t cols) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    return packed_bytes(dtype, rows, cols);
}

int64_t vgx_qweight_scale_offset(int dtype, int64_t rows, int64_t cols) {
    if (dtype != VGX_Q8_0 && dtype != VGX_Q4_0) return VGX_E_DTYPE;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    return scale_off(dtype, rows, cols);
}

static int pack_common(int dtype, const void *a, const void *b, void *dst, int64_t rows, int64_t cols, int mode,
                       void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!a || !dst || (mode == 1 && !b)) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    if (mode == 1 && (rows % 2)) return VGX_E_SHAPE;
    const int64_t prow = mode == 1 ? 2 * rows : rows;
    const int64_t nblk = cols / QK;
    const int64_t total = rows4(prow) * nblk;
    const int64_t soff = dtype == VGX_F32 ? 0 : scale_off(dtype, prow, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *pa = static_cast<const uint8_t *>(a);
    const auto *pb = static_cast<const uint8_t *>(b);
    auto *pd = static_cast<uint8_t *>(dst);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(pack_kernel<VGX_Q8_0>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode); break;
        case VGX_Q4_0: hipLaunchKernelGGL(pack_kernel<VGX_Q4_0>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode); break;
        case VGX_F32: hipLaunchKernelGGL(pack_kernel<VGX_F32>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_qweight_pack(int dtype, const void *src_blocks, void *dst_packed, int64_t rows, int64_t cols, void *stream) {
    return pack_common(dtype, src_blocks, nullptr, dst_packed, rows, cols, 0, stream);
}

int vgx_qweight_pack_gateup(int dtype, const void *gate_blocks, const void *up_blocks, void *dst_packed,
                            int64_t rows, int64_t cols, void *stream) {
    return pack_common(dtype, gate_blocks, up_blocks, dst_packed, rows, cols, 1, stream);
}

int vgx_qweight_unpack(int dtype, const void *packed, void *dst_blocks, int64_t rows, int64_t cols, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!packed || !dst_blocks) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    const int64_t nblk = cols / QK;
    const int64_t soff = dtype == VGX_F32 ? 0 : scale_off(dtype, rows, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *ps = static_cast<const uint8_t *>(packed);
    auto *pd = static_cast<uint8_t *>(dst_blocks);
    const unsigned g = grid_for(rows * nblk, 256);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(unpack_kernel<VGX_Q8_0>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
        case VGX_Q4_0: hipLaunchKernelGGL(unpack_kernel<VGX_Q4_0>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
        case VGX_F32: hipLaunchKernelGGL(unpack_kernel<VGX_F32>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_qweight_dequant(int dtype, const void *packed, float *out, int64_t rows, int64_t cols, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!packed || !out) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    const int64_t nblk = cols / QK;
    const int64_t soff = dtype == VGX_F32 ? 0 : scale_off(dtype, rows, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *pw = static_cast<const uint8_t *>(packed);
    const unsigned g = grid_for(rows * nblk, 256);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(dequant_kernel<VGX_Q8_0>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
        case VGX_Q4_0: hipLaunchKernelGGL(dequant_kernel<VGX_Q4_0>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
        case VGX_F32: hipLaunchKernelGGL(dequant_kernel<VGX_F32>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_embed_rows(int dtype, const void *packed, int64_t rows, int64_t cols, const int64_t *ids, int64_t n_ids,
                   int64_t pad_row, float *out, int64_t ldo, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!packed || !ids || !out) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || n_ids < 0 || ldo < cols || pad_row < 0 || pad_row >= rows) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    if (n_ids == 0) return VGX_OK;
    const int64_t nblk = cols / QK;
    const int64_t soff = dtype == VGX_F32 ? 0 : scale_off(dtype, rows, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *pw = static_cast<const uint8_t *>(packed);
    const unsigned g = grid_for(n_ids * nblk, 256);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(embed_kernel<VGX_Q8_0>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
        case VGX_Q4_0: hipLaunchKernelGGL(embed_kernel<VGX_Q4_0>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
        case VGX_F32: hipLaunchKernelGGL(embed_kernel<VGX_F32>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_qlinear(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                int64_t batch, const float *bias, float *y, int64_t ldy, int accumulate, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!w_packed || !x || !y) return VGX_E_ARG;
    if (accumulate != 0 && accumulate != 1) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || batch < 0 || ldx < cols || ldy < rows) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    if (cols / QK > (1 << 24)) return VGX_E_LIMIT;
    if (batch == 0) return VGX_OK;
    hipStream_t st = (hipStream_t)stream;
    if (accumulate) return launch_qgemv<EPI_ACCUM>(dtype, w_packed, rows, rows, cols, x, ldx, batch, bias, y, ldy, st);
    return launch_qgemv<EPI_STORE>(dtype, w_packed, rows, rows, cols, x, ldx, batch, bias, y, ldy, st);
}

int vgx_qlinear_swiglu(int dtype, const void *w_gateup_packed, int64_t rows, int64_t cols, const float *x,
                       int64_t ldx, int64_t batch, float *h, int64_t ldh, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!w_gateup_packed || !x || !h) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || batch < 0 || ldx < cols || ldh < rows) return VGX_E_SIZE;
    if (cols % QK || rows % 2) return VGX_E_SHAPE;
    if (batch == 0) return VGX_OK;
    return launch_qgemv<EPI_SWIGLU>(dtype, w_gateup_packed, 2 * rows, rows, cols, x, ldx, batch, nullptr, h, ldh,
                                    (hipStream_t)stream);
}

}  // extern "C"
