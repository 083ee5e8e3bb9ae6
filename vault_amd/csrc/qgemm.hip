// Q8_0 / Q4_0 block-dequant GEMM on bf16 MFMA for many activation rows (chunk prefill, batched
// decode): Y[b, r] = sum_c W[r, c] * u[b, c] (+ bias, residual or SwiGLU epilogue), u = x or
// RMSNorm(x).
//
// Reference semantics: the same projections as the GEMV (runtime/vault3.c:499-624, 1942-1956;
// src/vault_v3_model.py:1036-1047, 1145-1150, 2051, 2095-2096) applied to a [rows of tokens x cols]
// activation block.
//
// Exactness.  One v_mfma_f32_16x16x32_bf16 spans exactly one 32-weight quant block.  The weights
// enter the MFMA as unsigned integers, exact in bf16: Q8_0 as q + 128 (byte ^ 0x80), Q4_0 as the
// nibble n (16 + n in the tiled kernel).  The activations enter in pieces that a bf16 pair hi + lo
// (2^-18 relative residual) would leave at 2.4e-6 relative error per output, ten times the one-row
// GEMV's; so the decode-batch kernels take hi = bf16(u) and lo16 = fp16(16 (u - hi)) (19 significant
// bits, 2^-20 relative residual; lo16 overflows only past |u| = 2^21), lo16 multiplied by the same
// weights divided by 16 as exact fp16 values, the two products added into one accumulator (two MFMAs
// per block; three bf16 pieces would take three and, in the decode-batch kernel, registers that its
// occupancy target does not have: spills).  With S_b the per-block sum of the pieces, per block the
// fp32 MFMA result C (= sum_j w_j u_j as pieces) is corrected and scaled:
//   acc += d * (C - off * S_b),   off = 128 (Q8_0), 8 (Q4_0),
// which is the reference's sum_b d_b sum_j q_j x_j at fp32-level accuracy.  The tiled kernels take two
// fp16 pieces of the row scaled by a power of two 2^k (hi = fp16(2^k u), lo = fp16(2^k u - hi): about
// 22 significant bits, both pieces in fp16's normal range for any row), both multiplied by the signed
// weights as exact fp16 (no offset, so acc += d * C), and scale their outputs by 2^-k.  The decode-batch kernels
// place the weights by byte permutes instead (Q4_0 bf16 128 + n / fp16 1024 + n against pieces of 16 u;
// fp16 1024 + unsigned weight in qgemm_wide_kernel, whose pieces are both fp16 of a power-of-two-scaled
// row) with the matching offsets; their comments give the arithmetic.
//
// Mapping.  Large batches (prefill chunks) run qgemm_tile_dma_kernel (256 x 64 LDS tiles filled by
// LDS DMA; qgemm_tile_kernel, 128 x 128 tiles staged through registers, where a weight or activation
// block passes 2 GiB) after the split pre-pass; decode batches of up to 64 rows run the K-split kernels (qgemm_kslice_kernel,
// qgemm_split_kernel, qkv_split_kernel), qgemm_wide_kernel for tall unsplit weights, or
// qgemm_small_kernel, which converts its activations itself.  In every MFMA a lane of a 16-row tile
// owns one weight row (l % 16) for the A
// operand and one activation row (l % 16) for the B operand, both with the K slots 8 (l / 16) .. + 7
// of the block (weights 8 lg .. 8 lg + 7); the accumulator lane holds weight rows 4 (l / 16) .. + 3
// (one packed row-quad, whose four fp16 scales are one 8-byte word) of activation row l % 16.
#include "qgemv.h"

using namespace vgx;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// u = (norm ? lnw * x * inv_rms : x), scaled per row by a power of two 2^k that puts the largest |u|
// in [2^14, 2^15), split into two fp16 planes hi = fp16(2^k u) and lo = fp16(2^k u - hi): together
// about 22 significant bits of every element, with the scale keeping both pieces in fp16's normal
// range whatever the row's magnitude.  Also the row's 2^-k, which the GEMM multiplies into its outputs
// (exactly: a power of two).  k stays within [-100, 126],
// so 2^-k is a normal float; a row holding an infinity or a NaN is not scaled (k = 0), so that it
// reaches the outputs as it would unsplit.
// Inside every group of four, elements 1 and 2 trade places (stored order 0, 2, 1, 3): the K-slot
// order of the tiled kernel's weight fragments, whose Q4_0 nibble pairs come out of a word that way.
// One workgroup of 256 threads per activation row.
constexpr int kXsplitRegs = 20;   // float4 per thread kept in registers: rows of up to 20480 elements
__global__ __launch_bounds__(256) void xsplit_kernel(const float *__restrict__ x, int64_t ldx,
                                                      const float *__restrict__ lnw, float eps, int cols,
                                                      uint16_t *__restrict__ xh, uint16_t *__restrict__ xl,
                                                      float *__restrict__ xscale) {
    __shared__ float red[4], redm[4];
    const int64_t b = blockIdx.x;
    const float *xr = x + b * ldx;
    const int n4 = cols / 4;
    const float4 *x4 = reinterpret_cast<const float4 *>(xr);
    const float4 *g4 = reinterpret_cast<const float4 *>(lnw);
    const bool vec = ((uintptr_t)xr & 15) == 0 && (lnw == nullptr || ((uintptr_t)lnw & 15) == 0);
    auto load_x = [&](int i) {
        if (vec) return x4[i];
        return make_float4(xr[4 * i], xr[4 * i + 1], xr[4 * i + 2], xr[4 * i + 3]);
    };
    auto load_g = [&](int i) {
        if (vec) return g4[i];
        return make_float4(lnw[4 * i], lnw[4 * i + 1], lnw[4 * i + 2], lnw[4 * i + 3]);
    };
    // one pass over the row (kept in registers when it fits): the sum of squares and max |lnw x| (the
    // largest |u| is that max times 1 / rms, up to rounding, which the scale's headroom absorbs)
    const bool keep = n4 <= 256 * kXsplitRegs;
    float4 xv[kXsplitRegs];
    float ss = 0.0f, mx = 0.0f;
    bool finite = true;
    auto scan = [&](float4 v, int i) {
        ss = fmaf(v.x, v.x, ss); ss = fmaf(v.y, v.y, ss); ss = fmaf(v.z, v.z, ss); ss = fmaf(v.w, v.w, ss);
        if (lnw) {
            const float4 g = load_g(i);
            v.x *= g.x; v.y *= g.y; v.z *= g.z; v.w *= g.w;
        }
        finite = finite && __builtin_isfinite(v.x) && __builtin_isfinite(v.y) && __builtin_isfinite(v.z) &&
                 __builtin_isfinite(v.w);
        mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    };
    if (keep) {
#pragma unroll
        for (int j = 0; j < kXsplitRegs; ++j) {
            const int i = j * 256 + (int)threadIdx.x;
            if (i < n4) {
                xv[j] = load_x(i);
                scan(xv[j], i);
            }
        }
    } else {
        for (int i = threadIdx.x; i < n4; i += 256) scan(load_x(i), i);
    }
    ss = wave_sum(ss);
    mx = wave_max(finite ? mx : __builtin_inff());
    if ((threadIdx.x & 63) == 0) {
        red[threadIdx.x >> 6] = ss;
        redm[threadIdx.x >> 6] = mx;
    }
    __syncthreads();
    const float inv = lnw ? 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)cols + eps) : 1.0f;
    const float m = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3])) * inv;
    int k = 0;
    if (m < __builtin_inff()) {
        int e = 0;
        (void)frexpf(m, &e);                  // m = f 2^e, f in [0.5, 1) (e = 0 for m = 0)
        k = min(max(15 - e, -100), 126);
    }
    const float sc = __builtin_ldexpf(1.0f, k);
    if (threadIdx.x == 0) xscale[b] = __builtin_ldexpf(1.0f, -k);
    // a thread converts four consecutive elements (two 8-byte stores per plane)
    auto convert = [&](float4 v, int i) {
        if (lnw) {
            const float4 g = load_g(i);
            v.x = g.x * (v.x * inv); v.y = g.y * (v.y * inv); v.z = g.z * (v.z * inv); v.w = g.w * (v.w * inv);
        }
        v.x *= sc; v.y *= sc; v.z *= sc; v.w *= sc;
        // stored order 0, 2, 1, 3
        const uint32_t h02 = pack_f16x2(v.x, v.z), h13 = pack_f16x2(v.y, v.w);
        const auto hp = __builtin_bit_cast(vgx_f16x2_t, h02), hq = __builtin_bit_cast(vgx_f16x2_t, h13);
        const uint32_t l02 = pack_f16x2(v.x - (float)hp[0], v.z - (float)hp[1]);
        const uint32_t l13 = pack_f16x2(v.y - (float)hq[0], v.w - (float)hq[1]);
        *reinterpret_cast<uint2 *>(xh + b * cols + 4 * i) = make_uint2(h02, h13);
        *reinterpret_cast<uint2 *>(xl + b * cols + 4 * i) = make_uint2(l02, l13);
    };
    if (keep) {
#pragma unroll
        for (int j = 0; j < kXsplitRegs; ++j) {
            const int i = j * 256 + (int)threadIdx.x;
            if (i < n4) convert(xv[j], i);
        }
    } else {
        for (int i = threadIdx.x; i < n4; i += 256) convert(load_x(i), i);
    }
}

template <int DT>
__device__ __forceinline__ uint2 load_a(const uint8_t *__restrict__ W, int64_t rq, int nblk, int blk, int r4, int lg) {
    // Q8_0: bytes 8 lg .. + 7 of row r4 of the row-quad block; Q4_0: bytes 8 (lg & 1) .. + 7
    constexpr int QB = DT == VGX_Q8_0 ? 32 : 16;
    const uint8_t *p = W + ((rq * nblk + blk) * 4 + r4) * QB + (DT == VGX_Q8_0 ? 8 * lg : 8 * (lg & 1));
    return *reinterpret_cast<const uint2 *>(p);
}

// 8 quant values -> 8 unsigned integers as bf16 (exact): weights 8 lg .. 8 lg + 7 of the block, in
// natural K-slot order; fh (when requested) the same integers divided by 16 as fp16 (exact).
template <int DT, bool F16 = false>
__device__ __forceinline__ bf16x8_t a_frag(uint2 w, int lg, f16x8_t *fh = nullptr) {
    uint32_t u[2] = {w.x, w.y};
    if constexpr (DT == VGX_Q8_0) {
        u[0] ^= 0x80808080u;
        u[1] ^= 0x80808080u;
    } else {
        const int sh = (lg >> 1) * 4;   // low nibbles for weights 0..15, high nibbles for 16..31
        u[0] = (u[0] >> sh) & 0x0F0F0F0Fu;
        u[1] = (u[1] >> sh) & 0x0F0F0F0Fu;
    }
    uint32_t o[4], h[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float f0 = (float)(u[i] & 0xFFu), f1 = (float)((u[i] >> 8) & 0xFFu);
        const float f2 = (float)((u[i] >> 16) & 0xFFu), f3 = (float)(u[i] >> 24);
        // small integers: the bf16 is the top half of the fp32 bits, exactly
        o[2 * i] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f1) & 0xFFFF0000u);
        o[2 * i + 1] = (__float_as_uint(f2) >> 16) | (__float_as_uint(f3) & 0xFFFF0000u);
        if constexpr (F16) {
            h[2 * i] = pack_f16x2(f0 * 0.0625f, f1 * 0.0625f);
            h[2 * i + 1] = pack_f16x2(f2 * 0.0625f, f3 * 0.0625f);
        }
    }
    if constexpr (F16) *fh = __builtin_bit_cast(f16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
    return __builtin_bit_cast(bf16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
}

// ---------------------------------------------------------------------------------------------
// Large batches (prefill chunks, more than 64 activation rows): LDS tiles.  A workgroup of 4 waves
// owns 128 weight rows (32 row-quads) x 128 activation rows; wave (wm, wn) = (wave & 1, wave >> 1)
// computes weight rows 64 wm .. + 63 x activation rows 64 wn .. + 63 as 4 x 4 MFMA tiles.  Per quant
// block the workgroup stages the raw quants and scales of its 128 weight rows and the fp16 hi / lo
// activations and block sums of its 128 activation rows in LDS (double-buffered, one barrier per
// block; the next block's global loads are in flight while the current one is multiplied), so every
// weight fragment serves 4 activation tiles and every activation fragment 4 weight tiles from LDS
// instead of each wave streaming both from L2.  The offset correction enters as the MFMA's initial
// accumulator (-off * S_b per activation row), leaving one FMA per output and block for the scale.
constexpr int kTM = 128;                 // weight rows per workgroup tile
constexpr int kTN = 128;                 // activation rows per workgroup tile
constexpr int kBRow = QK + 8;            // fp16 per staged activation row (16 B of padding)

// Q8_0 weights 8 lg .. 8 lg + 7 of the block as the decode-batch split kernel's A fragments, in K-slot
// order 0, 2, 1, 3, 4, 6, 5, 7 (the activations are staged in the same order): q + 128 through the
// byte conversions as exact bf16, and the same integers divided by 16 as exact fp16 (the B operand lo16
// is fp16 and carries a factor 16).  Both products then add into one accumulator.
template <int DT>
__device__ __forceinline__ void tile_a_frags(uint2 w, int lg, bf16x8_t &fb, f16x8_t &fh) {
    static_assert(DT == VGX_Q8_0, "Q4_0 fragments come from q4_word_frags");
    (void)lg;
    uint32_t o[4], h[4];
    const uint32_t u[2] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float f0 = (float)(u[i] & 0xFFu), f1 = (float)((u[i] >> 8) & 0xFFu);
        const float f2 = (float)((u[i] >> 16) & 0xFFu), f3 = (float)(u[i] >> 24);
        o[2 * i] = (__float_as_uint(f0) >> 16) | (__float_as_uint(f2) & 0xFFFF0000u);
        o[2 * i + 1] = (__float_as_uint(f1) >> 16) | (__float_as_uint(f3) & 0xFFFF0000u);
        h[2 * i] = pack_f16x2(f0 * 0.0625f, f2 * 0.0625f);
        h[2 * i + 1] = pack_f16x2(f1 * 0.0625f, f3 * 0.0625f);
    }
    fb = __builtin_bit_cast(bf16x8_t, make_uint4(o[0], o[1], o[2], o[3]));
    fh = __builtin_bit_cast(f16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
}

// The tiled kernels' A fragment: weights 8 lg .. 8 lg + 7 of the block as exact fp16 signed integers
// (Q4_0 n - 8, Q8_0 q) in K-slot order 0, 2, 1, 3, 4, 6, 5, 7 (the split pre-pass stores the
// activations in the same order); both activation planes (fp16 hi and lo) multiply it, and the MFMA
// sums need no offset correction.  Q4_0: fp16(16 + n) = 0x4C00 | n << 6 (the nibble rotated to bits
// 6..9 and 22..25, one AND-OR per two weights), then one packed fp16 subtraction of 24 (exact);
// Q8_0: q + 128 through the byte conversions, packed to fp16, minus 128.
template <int DT>
__device__ __forceinline__ f16x8_t tile_a_f16(uint2 w, int lg) {
    uint32_t h[4];
    if constexpr (DT == VGX_Q4_0) {
        const bool hi = (lg >> 1) != 0;       // low nibbles for weights 0..15, high nibbles for 16..31
        // bytes 0 / 2 and bytes 1 / 3 by rotations of their own (a left turn of six would wrap byte 3's
        // nibble)
        const int rh02 = hi ? 30 : 26, rh13 = hi ? 6 : 2;
        // (r & mask) | base as one v_and_or_b32 (VOP3 takes no literal here: the mask in an SGPR, the
        // base in a VGPR); the compiler emits an AND and an OR with literals otherwise
        const uint32_t base = 0x4C004C00u;
        auto and_or = [&](uint32_t r) {
            uint32_t o;
            asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(o) : "v"(r), "s"(0x03C003C0u), "v"(base));
            return o;
        };
        h[0] = and_or(__builtin_amdgcn_alignbit(w.x, w.x, rh02));   // weights 0, 2
        h[1] = and_or(__builtin_amdgcn_alignbit(w.x, w.x, rh13));   // weights 1, 3
        h[2] = and_or(__builtin_amdgcn_alignbit(w.y, w.y, rh02));
        h[3] = and_or(__builtin_amdgcn_alignbit(w.y, w.y, rh13));
    } else {
        const uint32_t u[2] = {w.x ^ 0x80808080u, w.y ^ 0x80808080u};
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float f0 = (float)(u[i] & 0xFFu), f1 = (float)((u[i] >> 8) & 0xFFu);
            const float f2 = (float)((u[i] >> 16) & 0xFFu), f3 = (float)(u[i] >> 24);
            h[2 * i] = pack_f16x2(f0, f2);
            h[2 * i + 1] = pack_f16x2(f1, f3);
        }
    }
    constexpr _Float16 off = DT == VGX_Q4_0 ? (_Float16)-24.0f : (_Float16)-128.0f;
    f16x8_t f = __builtin_bit_cast(f16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
    return f + f16x8_t{off, off, off, off, off, off, off, off};
}

template <int DT, int EPI, bool SPLIT>
__global__ __launch_bounds__(256, 2) void qgemm_tile_kernel(const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq,
                                                          int nblk, int64_t rows_out,
                                                          const uint16_t *__restrict__ xh,
                                                          const uint16_t *__restrict__ xl,
                                                          const float *__restrict__ xscale, int64_t batch,
                                                          const float *__restrict__ bias, float *__restrict__ y,
                                                          int64_t ldy, float *__restrict__ part, int kper) {
    constexpr int QB = DT == VGX_Q8_0 ? 32 : 16;
    constexpr int APARTS = 4 * QB / 16;                  // 16-byte pieces of one row-quad block
    constexpr int AQ16 = kTM / 4 * APARTS;               // 16-byte pieces of the tile's block
    // Stage buffers (two blocks) and, after the K loop, the epilogue's half tile share one LDS area.
    constexpr int A_B = kTM * QB, SC_B = kTM / 4 * 8, BH_B = kTN * kBRow * 2;
    constexpr int STAGE_B = A_B + SC_B + 2 * BH_B;
    constexpr int kERow = 64 + 4;                          // floats per activation row of a half tile
    constexpr int EPI_B = kTN * kERow * 4;
    __shared__ __align__(16) uint8_t smem[2 * STAGE_B > EPI_B ? 2 * STAGE_B : EPI_B];
    auto aq = [&](int buf) { return smem + buf * STAGE_B; };                         // [row-quad][row][QB]
    auto asc = [&](int buf) { return reinterpret_cast<uint2 *>(smem + buf * STAGE_B + A_B); };
    auto bh = [&](int buf) { return reinterpret_cast<uint16_t *>(smem + buf * STAGE_B + A_B + SC_B); };
    auto bl = [&](int buf) { return reinterpret_cast<uint16_t *>(smem + buf * STAGE_B + A_B + SC_B + BH_B); };

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
    const int cols = nblk * QK;
    const int64_t rq0 = (int64_t)blockIdx.x * (kTM / 4);
    const int64_t b0 = (int64_t)blockIdx.y * kTN;
    const int blk_lo = SPLIT ? (int)blockIdx.z * kper : 0;
    const int blk_hi = SPLIT ? min(nblk, blk_lo + kper) : nblk;

    // global -> registers (one block), registers -> LDS buffer
    // one block's staging registers; two sets, so the loads of block k + 2 leave while block k is
    // multiplied and block k + 1 waits in the other set
    struct Regs {
        uint4 ra, h0, h1, l0, l1;
        uint2 rs;
    };
    auto fetch_b = [&](int idx, int blk, uint4 &h, uint4 &l) {
        const int row = idx >> 2, pc = idx & 3;
        const int64_t b = b0 + row;
        if (b < batch) {
            const int64_t o = b * cols + (int64_t)blk * QK + pc * 8;
            h = *reinterpret_cast<const uint4 *>(xh + o);
            l = *reinterpret_cast<const uint4 *>(xl + o);
        } else {
            h = l = make_uint4(0, 0, 0, 0);
        }
    };
    auto fetch = [&](Regs &r, int blk) {
        r.ra = make_uint4(0, 0, 0, 0);
        r.rs = make_uint2(0, 0);
        if (tid < AQ16) {
            const int64_t rq = rq0 + tid / APARTS;
            if (rq < n_rq) r.ra = *reinterpret_cast<const uint4 *>(W + (rq * nblk + blk) * 4 * QB + (tid % APARTS) * 16);
        }
        if (tid < kTM / 4) {
            const int64_t rq = rq0 + tid;
            if (rq < n_rq) r.rs = *reinterpret_cast<const uint2 *>(W + soff + (rq * nblk + blk) * 8);
        }
        fetch_b(tid, blk, r.h0, r.l0);
        fetch_b(tid + 256, blk, r.h1, r.l1);
    };
    auto stage = [&](const Regs &r, int buf) {
        if (tid < AQ16) *reinterpret_cast<uint4 *>(aq(buf) + tid * 16) = r.ra;
        if (tid < kTM / 4) asc(buf)[tid] = r.rs;
        *reinterpret_cast<uint4 *>(bh(buf) + (tid >> 2) * kBRow + (tid & 3) * 8) = r.h0;
        *reinterpret_cast<uint4 *>(bl(buf) + (tid >> 2) * kBRow + (tid & 3) * 8) = r.l0;
        *reinterpret_cast<uint4 *>(bh(buf) + ((tid + 256) >> 2) * kBRow + (tid & 3) * 8) = r.h1;
        *reinterpret_cast<uint4 *>(bl(buf) + ((tid + 256) >> 2) * kBRow + (tid & 3) * 8) = r.l1;
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[t][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) {
        f16x8_t af[4];
        vgx_f16x2_t d[4][2];     // fp16 scales, widened inside the FMAs (mixed-precision FMA)
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int rql = wm * 16 + 4 * t + (l16 >> 2);       // A operand: weight row 16 t + l16
            const uint2 w = *reinterpret_cast<const uint2 *>(aq(buf) + (rql * 4 + (l16 & 3)) * QB +
                                                              (DT == VGX_Q8_0 ? 8 * lg : 8 * (lg & 1)));
            af[t] = tile_a_f16<DT>(w, lg);
            const uint2 sc = asc(buf)[wm * 16 + 4 * t + lg];     // accumulator rows 16 t + 4 lg .. + 3
            d[t][0] = __builtin_bit_cast(vgx_f16x2_t, sc.x);
            d[t][1] = __builtin_bit_cast(vgx_f16x2_t, sc.y);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int row = wn * 64 + 16 * c + l16;
            const f16x8_t hf = *reinterpret_cast<const f16x8_t *>(bh(buf) + row * kBRow + 8 * lg);
            const f16x8_t lf = *reinterpret_cast<const f16x8_t *>(bl(buf) + row * kBRow + 8 * lg);
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                f32x4_t pr = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], hf, pr, 0, 0, 0);
                pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], lf, pr, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][c][i] = fmaf((float)d[t][i >> 1][i & 1], pr[i], acc[t][c][i]);
            }
        }
    };

    // Blocks k (LDS buffer k % 2), k + 1 (register set (k + 1) % 2), k + 2 (loads in flight).
    Regs ra, rb;
    if (blk_lo < blk_hi) {
        fetch(ra, blk_lo);
        if (blk_lo + 1 < blk_hi) fetch(rb, blk_lo + 1);
        stage(ra, 0);
    }
    __syncthreads();
    for (int blk = blk_lo; blk < blk_hi; blk += 2) {
        // even step: block blk in buffer 0, block blk + 1 in rb; ra is free
        if (blk + 2 < blk_hi) fetch(ra, blk + 2);
        compute(0);
        if (blk + 1 < blk_hi) stage(rb, 1);
        __syncthreads();
        if (blk + 1 >= blk_hi) break;
        // odd step: block blk + 1 in buffer 1, block blk + 2 in ra; rb is free
        if (blk + 3 < blk_hi) fetch(rb, blk + 3);
        compute(1);
        if (blk + 2 < blk_hi) stage(ra, 0);
        __syncthreads();
    }

    // Epilogue.  Split K: the raw sums, float4 per (tile, lane).  Otherwise the tile goes through LDS
    // in two halves of 64 weight rows (waves wm = 0, then wm = 1 write theirs), and all threads then
    // apply bias / residual / SwiGLU and store rows of y with consecutive threads on consecutive
    // outputs.
    if constexpr (SPLIT) {
        // the activation rows' 2^-k, through LDS (the stages are free)
        float *tsc = reinterpret_cast<float *>(smem);
        for (int i = tid; i < kTN; i += 256) tsc[i] = b0 + i < batch ? xscale[b0 + i] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t crq = rq0 + wm * 16 + 4 * t + lg;
            if (crq >= n_rq) continue;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t b = b0 + wn * 64 + 16 * c + l16;
                if (b >= batch) continue;
                const float sc = tsc[wn * 64 + 16 * c + l16];
                float4 v;
                v.x = acc[t][c][0] * sc; v.y = acc[t][c][1] * sc; v.z = acc[t][c][2] * sc; v.w = acc[t][c][3] * sc;
                *reinterpret_cast<float4 *>(part + ((int64_t)blockIdx.z * batch + b) * (n_rq * 4) + crq * 4) = v;
            }
        }
        return;
    }
    float *et = reinterpret_cast<float *>(smem);       // [activation row][64 weight rows + pad]
    // each activation row's 2^-k in the row's first pad float (the halves below write floats 0..63)
    for (int i = tid; i < kTN; i += 256) et[i * kERow + 64] = b0 + i < batch ? xscale[b0 + i] : 0.0f;
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        if (wm == half) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float4 v;
                    v.x = acc[t][c][0]; v.y = acc[t][c][1]; v.z = acc[t][c][2]; v.w = acc[t][c][3];
                    *reinterpret_cast<float4 *>(et + (wn * 64 + 16 * c + l16) * kERow + 16 * t + 4 * lg) = v;
                }
        }
        __syncthreads();
        const int64_t r0 = (rq0 + half * 16) * 4;           // first packed weight row of this half
        if constexpr (EPI == EPI_SWIGLU) {
            // packed row-quad q: rows (gate 2q, gate 2q + 1, up 2q, up 2q + 1) -> outputs 2q, 2q + 1
            for (int i = tid; i < kTN * 32; i += 256) {
                const int bl_ = i >> 5, o = i & 31;
                const int64_t b = b0 + bl_, oo = r0 / 2 + o;
                if (b >= batch || oo >= rows_out) continue;
                const float *er = et + bl_ * kERow + (o >> 1) * 4 + (o & 1);
                const float sc = et[bl_ * kERow + 64];
                const float g = er[0] * sc, u = er[2] * sc;
                y[b * ldy + oo] = g / (1.0f + __expf(-g)) * u;
            }
        } else {
            for (int i = tid; i < kTN * 64; i += 256) {
                const int bl_ = i >> 6, rr = i & 63;
                const int64_t b = b0 + bl_, row = r0 + rr;
                if (b >= batch || row >= rows_out) continue;
                float v = et[bl_ * kERow + rr] * et[bl_ * kERow + 64];
                if (bias) v += bias[row];
                if constexpr (EPI == EPI_ACCUM) v += y[b * ldy + row];
                y[b * ldy + row] = v;
            }
        }
        __syncthreads();
    }
}

// The tiled kernel with its stages filled by LDS DMA (dma16 / dma4: buffer loads that write LDS directly;
// the kernel makes no other use of M0, which its compiled code was checked for).  Two stages: the loads of block k + 1
// leave right after the barrier of block k and land in the other stage while block k is multiplied, and
// they need no staging registers, which leaves room for three workgroups per CU (at most 160 VGPRs,
// 25.5 KB of LDS for Q4_0, 33.5 KB for Q8_0) instead of two (256 VGPRs with the register double buffer
// of qgemm_tile_kernel).  Same arithmetic as qgemm_tile_kernel, bit for bit.  The activation rows of a
// stage are unpadded 64-byte rows whose 16-byte pieces are swizzled by (row >> 2) & 3, so the MFMA
// operand reads stay free of bank conflicts.  Measured on a 1024-token chunk with the 128 x 128 tiles
// (Q4_0 / Q8_0): gate/up 228.9 -> 193.5 / 251.4 -> 222.5 us against the register double buffer, down
// 143.0 -> 137.2 / 156.1 -> 144.1, q|k|v 49.2 -> 48.3 / 50.8 -> 49.5, o 43.6 -> 45.8 / 46.6 -> 44.9; with
// three stages at two workgroups per CU 209.7 us for the Q4_0 gate/up, with four 221.1.
// Its tile is TM weight rows x TN activation rows, each wave 64 x 64 (wave w: weight rows 64 (w % (TM /
// 64)), activation rows 64 (w / (TM / 64))).  256 x 64 (kTMDma x kTNDma) stages 12.75 KB per block of
// a Q4_0 tile instead of the 18.75 KB of 128 x 128 for the same outputs per workgroup: gate/up 195.2
// -> 182.5 us, down 128.1 -> 122.3, q|k|v 47.4 -> 46.0, o 42.9 -> 43.2 (with bf16 hi / fp16 lo16
// pieces and their offset corrections; the fp16 pieces and signed weights then gave 152.8-155.1 /
// 108.4-109.1 / 43.8-44.2 / 39.0-42.3 us).  Four waves per SIMD (128 VGPRs, a few bytes spilled)
// measured no better (gate/up 151.6-152.9 against 153.3-155.1 us).
constexpr int kTMDma = 256, kTNDma = 64;
template <int DT, int EPI, bool SPLIT, int TM, int TN>
__global__ __launch_bounds__(256, 3) void qgemm_tile_dma_kernel(const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq,
                                                              int nblk, int64_t rows_out,
                                                              const uint16_t *__restrict__ xh,
                                                              const uint16_t *__restrict__ xl,
                                                              const float *__restrict__ xscale, int64_t batch,
                                                              const float *__restrict__ bias, float *__restrict__ y,
                                                              int64_t ldy, float *__restrict__ part, int kper) {
    constexpr int QB = DT == VGX_Q8_0 ? 32 : 16;
    constexpr int APARTS = 4 * QB / 16;
    static_assert(TM / 64 * (TN / 64) == 4, "four waves of 64 x 64");
    constexpr int NA = TM / 4 * APARTS / 64;            // 16-byte weight pieces: wave-loads per block
    constexpr int NSC = TM / 128;                       // scale wave-loads per block
    constexpr int A_B = TM * QB, SC_B = TM / 4 * 8, BH_B = TN * QK * 2;
    constexpr int STAGE_B = A_B + SC_B + 2 * BH_B;
    constexpr int NS = 2;
    constexpr int NJ = NA + NSC + 2 * (BH_B / 1024);   // wave-loads per block
    constexpr int kERow = 64 + 4;
    constexpr int EPI_B = TN * kERow * 4;
    __shared__ __align__(16) uint8_t smem[NS * STAGE_B > EPI_B ? NS * STAGE_B : EPI_B];
    auto aq = [&](int buf) { return smem + buf * STAGE_B; };
    auto asc = [&](int buf) { return reinterpret_cast<uint2 *>(smem + buf * STAGE_B + A_B); };
    auto bh = [&](int buf) { return reinterpret_cast<uint16_t *>(smem + buf * STAGE_B + A_B + SC_B); };
    auto bl = [&](int buf) { return reinterpret_cast<uint16_t *>(smem + buf * STAGE_B + A_B + SC_B + BH_B); };

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lg = lane >> 4;
    const int wm = wave % (TM / 64), wn = wave / (TM / 64);
    const int cols = nblk * QK;
    // XCD-aware tile order: workgroups go to the 8 XCDs round robin (linear id mod 8); each XCD takes a
    // contiguous run of the activation-tile-major tile sequence, so that it reads few activation tiles
    // (kept in its L2) and streams the weights, instead of every XCD reading every activation tile.
    int tr = blockIdx.x, tt = blockIdx.y;
    {
        const int64_t G = gridDim.x, total = G * gridDim.y, id = blockIdx.x + G * blockIdx.y;
        if (total % 8 == 0) {
            const int64_t s = (id % 8) * (total / 8) + id / 8;
            tt = (int)(s / G);
            tr = (int)(s - (int64_t)tt * G);
        }
    }
    const int64_t rq0 = (int64_t)tr * (TM / 4);
    const int64_t b0 = (int64_t)tt * TN;
    const int blk_lo = SPLIT ? (int)blockIdx.z * kper : 0;
    const int blk_hi = SPLIT ? min(nblk, blk_lo + kper) : nblk;

    const dma_rsrc_t wrs = dma_rsrc(W, (uint32_t)(soff + n_rq * nblk * 8));
    const dma_rsrc_t hrs = dma_rsrc(xh, (uint32_t)(batch * cols * 2));
    const dma_rsrc_t lrs = dma_rsrc(xl, (uint32_t)(batch * cols * 2));
    // wave-load j of a block: weight pieces (j < NA), scales, hi rows, lo rows
    auto issue = [&](int blk, int buf) {
#pragma unroll
        for (int jj = 0; jj < (NJ + 3) / 4; ++jj) {
            const int j = jj * 4 + wave;
            if (j < NA) {
                const int pc = j * 64 + lane;
                const int64_t rq = rq0 + pc / APARTS;
                const uint32_t o = rq < n_rq ? (uint32_t)((rq * nblk + blk) * 4 * QB + (pc % APARTS) * 16) : kDmaPast;
                dma16(wrs, o, aq(buf) + j * 1024);
            } else if (j < NA + NSC) {
                const int64_t rq = rq0 + (j - NA) * 32 + lane / 2;
                const uint32_t o = rq < n_rq ? (uint32_t)(soff + (rq * nblk + blk) * 8 + (lane & 1) * 4) : kDmaPast;
                dma4(wrs, o, reinterpret_cast<const uint8_t *>(asc(buf)) + (j - NA) * 256);
            } else if (j < NJ) {
                const int jb = j - NA - NSC, pl = jb / (BH_B / 1024), jr = jb % (BH_B / 1024);
                const int row = 16 * jr + (lane >> 2), slot = lane & 3, piece = slot ^ ((row >> 2) & 3);
                const int64_t b = b0 + row;
                const uint32_t o = b < batch ? (uint32_t)((b * cols + (int64_t)blk * QK + piece * 8) * 2) : kDmaPast;
                dma16(pl ? lrs : hrs, o, reinterpret_cast<const uint8_t *>(pl ? bl(buf) : bh(buf)) + jr * 1024);
            }
        }
    };
    f32x4_t acc[4][4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[t][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) {
        f16x8_t af[4];
        vgx_f16x2_t d[4][2];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int rql = wm * 16 + 4 * t + (l16 >> 2);
            const uint2 w = *reinterpret_cast<const uint2 *>(aq(buf) + (rql * 4 + (l16 & 3)) * QB +
                                                              (DT == VGX_Q8_0 ? 8 * lg : 8 * (lg & 1)));
            af[t] = tile_a_f16<DT>(w, lg);
            const uint2 sc = asc(buf)[wm * 16 + 4 * t + lg];
            d[t][0] = __builtin_bit_cast(vgx_f16x2_t, sc.x);
            d[t][1] = __builtin_bit_cast(vgx_f16x2_t, sc.y);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int row = wn * 64 + 16 * c + l16;
            const int off = row * QK + 8 * (lg ^ ((row >> 2) & 3));
            const f16x8_t hf = *reinterpret_cast<const f16x8_t *>(bh(buf) + off);
            const f16x8_t lf = *reinterpret_cast<const f16x8_t *>(bl(buf) + off);
            // four independent accumulator chains, so that the MFMAs of one tile overlap the next's
            f32x4_t pr[4];
#pragma unroll
            for (int t = 0; t < 4; ++t)
                pr[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], hf, f32x4_t{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t) pr[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[t], lf, pr[t], 0, 0, 0);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][c][i] = fmaf((float)d[t][i >> 1][i & 1], pr[t][i], acc[t][c][i]);
        }
    };

    const int nb = blk_hi - blk_lo;
    if (nb > 0) issue(blk_lo, 0);
    for (int k = 0; k < nb; ++k) {
        // this wave's loads of block k have landed and its reads of block k - 1 are done; the barrier
        // extends both to the workgroup, so block k is complete and stage (k + 1) % 2 is free
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
        if (k + 1 < nb) issue(blk_lo + k + 1, (k + 1) % NS);
        compute(k % NS);
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");   // the stages are free for the epilogue

    if constexpr (SPLIT) {
        // the activation rows' 2^-k, through LDS (the stages are free)
        float *tsc = reinterpret_cast<float *>(smem);
        for (int i = tid; i < TN; i += 256) tsc[i] = b0 + i < batch ? xscale[b0 + i] : 0.0f;
        __syncthreads();
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const int64_t crq = rq0 + wm * 16 + 4 * t + lg;
            if (crq >= n_rq) continue;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int64_t b = b0 + wn * 64 + 16 * c + l16;
                if (b >= batch) continue;
                const float sc = tsc[wn * 64 + 16 * c + l16];
                float4 v;
                v.x = acc[t][c][0] * sc; v.y = acc[t][c][1] * sc; v.z = acc[t][c][2] * sc; v.w = acc[t][c][3] * sc;
                *reinterpret_cast<float4 *>(part + ((int64_t)blockIdx.z * batch + b) * (n_rq * 4) + crq * 4) = v;
            }
        }
        return;
    }
    float *et = reinterpret_cast<float *>(smem);
    // each activation row's 2^-k in the row's first pad float (the halves below write floats 0..63)
    for (int i = tid; i < TN; i += 256) et[i * kERow + 64] = b0 + i < batch ? xscale[b0 + i] : 0.0f;
#pragma unroll
    for (int half = 0; half < TM / 64; ++half) {
        if (wm == half) {
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float4 v;
                    v.x = acc[t][c][0]; v.y = acc[t][c][1]; v.z = acc[t][c][2]; v.w = acc[t][c][3];
                    *reinterpret_cast<float4 *>(et + (wn * 64 + 16 * c + l16) * kERow + 16 * t + 4 * lg) = v;
                }
        }
        __syncthreads();
        const int64_t r0 = (rq0 + half * 16) * 4;
        if constexpr (EPI == EPI_SWIGLU) {
            for (int i = tid; i < TN * 32; i += 256) {
                const int bl_ = i >> 5, o = i & 31;
                const int64_t b = b0 + bl_, oo = r0 / 2 + o;
                if (b >= batch || oo >= rows_out) continue;
                const float *er = et + bl_ * kERow + (o >> 1) * 4 + (o & 1);
                const float sc = et[bl_ * kERow + 64];
                const float g = er[0] * sc, u = er[2] * sc;
                y[b * ldy + oo] = g / (1.0f + __expf(-g)) * u;
            }
        } else {
            for (int i = tid; i < TN * 64; i += 256) {
                const int bl_ = i >> 6, rr = i & 63;
                const int64_t b = b0 + bl_, row = r0 + rr;
                if (b >= batch || row >= rows_out) continue;
                float v = et[bl_ * kERow + rr] * et[bl_ * kERow + 64];
                if (bias) v += bias[row];
                if constexpr (EPI == EPI_ACCUM) v += y[b * ldy + row];
                y[b * ldy + row] = v;
            }
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// F32 / BF16 / F16 weights (the segment scorer's fc1, F32 and BF16 model files) for many activation
// rows, 16-bit elements widened exactly to fp32 as they are fetched: fp32 MFMA
// (v_mfma_f32_16x16x4_f32), so products and sums stay fp32 as in the reference.  A workgroup of 4
// waves owns 64 weight rows x 64 activation rows (each wave 32 x 32 as 2 x 2 tiles); per 32-wide
// block of K the workgroup stages both 64 x 32 fp32 tiles in LDS (double-buffered, one barrier per
// block, next block's loads in flight during the current one's MFMAs).  Weights are read from the
// packed row-quad layout (a row-quad block is 4 rows x 32 floats, contiguous).
constexpr int kFT = 64;                   // rows of each operand per workgroup tile
constexpr int kFRow = QK + 1;             // floats per staged row (one float of padding)

template <int WDT, int EPI, bool VEC>
__global__ __launch_bounds__(256) void f32gemm_tile_kernel(const void *__restrict__ W, int64_t n_rq, int nblk,
                                                           int64_t rows_out, const float *__restrict__ x,
                                                           int64_t ldx, int64_t batch, const float *__restrict__ bias,
                                                           float *__restrict__ y, int64_t ldy) {
    __shared__ float as[2][kFT * kFRow];
    __shared__ float bs[2][kFT * kFRow];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int wm = wave & 1, wn = wave >> 1;
    const int64_t rq0 = (int64_t)blockIdx.x * (kFT / 4);
    const int64_t b0 = (int64_t)blockIdx.y * kFT;

    float4 ra[2], rb[2];
    auto fetch = [&](int blk) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i;
            // weights: row-quad idx / 32, row (idx / 8) % 4, float4 idx % 8 of the block
            const int64_t rq = rq0 + (idx >> 5);
            const int64_t e0 = ((rq * nblk + blk) * 4 + ((idx >> 3) & 3)) * QK + (idx & 7) * 4;
            if (rq >= n_rq) {
                ra[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            } else if constexpr (WDT == VGX_F32) {
                ra[i] = *reinterpret_cast<const float4 *>(static_cast<const float *>(W) + e0);
            } else {
                // BF16 / F16 elements widened exactly (runtime/vault3.c:510-533)
                const uint2 h = *reinterpret_cast<const uint2 *>(static_cast<const uint16_t *>(W) + e0);
                if constexpr (WDT == VGX_BF16)
                    ra[i] = make_float4(__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xFFFF0000u),
                                        __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xFFFF0000u));
                else
                    ra[i] = make_float4(half_bits_to_float(h.x), half_bits_to_float(h.x >> 16),
                                        half_bits_to_float(h.y), half_bits_to_float(h.y >> 16));
            }
            const int64_t b = b0 + (idx >> 3);
            if (b < batch) {
                const float *xp = x + b * ldx + (int64_t)blk * QK + (idx & 7) * 4;
                if constexpr (VEC) rb[i] = *reinterpret_cast<const float4 *>(xp);
                else rb[i] = make_float4(xp[0], xp[1], xp[2], xp[3]);
            } else {
                rb[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        }
    };
    auto stage = [&](int buf) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int idx = tid + 256 * i, row = idx >> 3, c = (idx & 7) * 4;
            float *pa = as[buf] + row * kFRow + c;
            pa[0] = ra[i].x; pa[1] = ra[i].y; pa[2] = ra[i].z; pa[3] = ra[i].w;
            float *pb = bs[buf] + row * kFRow + c;
            pb[0] = rb[i].x; pb[1] = rb[i].y; pb[2] = rb[i].z; pb[3] = rb[i].w;
        }
    };
    f32x4_t acc[2][2];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < 2; ++c) acc[t][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto compute = [&](int buf) {
#pragma unroll
        for (int kk = 0; kk < QK / 4; ++kk) {
            float a[2], b[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) a[t] = as[buf][(wm * 32 + 16 * t + l16) * kFRow + 4 * kk + lg];
#pragma unroll
            for (int c = 0; c < 2; ++c) b[c] = bs[buf][(wn * 32 + 16 * c + l16) * kFRow + 4 * kk + lg];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int c = 0; c < 2; ++c) acc[t][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[t], b[c], acc[t][c], 0, 0, 0);
        }
    };
    fetch(0);
    stage(0);
    __syncthreads();
    int cb = 0;
    for (int blk = 0; blk < nblk; ++blk) {
        const bool more = blk + 1 < nblk;
        if (more) fetch(blk + 1);
        compute(cb);
        if (more) stage(cb ^ 1);
        __syncthreads();
        cb ^= 1;
    }
    // lane holds weight rows 4 crq .. + 3 (one packed row-quad) of activation row b
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const int64_t crq = rq0 + wm * 8 + 4 * t + lg;
        if (crq >= n_rq) continue;
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int64_t b = b0 + wn * 32 + 16 * c + l16;
            if (b >= batch) continue;
            float *yr = y + b * ldy;
            if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int64_t o = crq * 2 + k;
                    if (o >= rows_out) continue;
                    const float g = acc[t][c][k], u = acc[t][c][2 + k];
                    yr[o] = g / (1.0f + __expf(-g)) * u;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t row = crq * 4 + i;
                    if (row >= rows_out) continue;
                    float v = acc[t][c][i];
                    if (bias) v += bias[row];
                    if constexpr (EPI == EPI_ACCUM) v += yr[row];
                    yr[row] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Decode batches (up to 64 activation rows): one launch without the split pre-pass.  Each workgroup
// converts the activations of its K range itself, 4 blocks at a time, into LDS (bf16 hi and fp16
// lo16, the per-block sums of the pieces), shared by its 4 waves; the chunks are double-buffered so the next
// chunk's activations and weights are requested before the current one is multiplied (requesting
// the weights a second chunk earlier measured no faster).  The fused
// RMSNorm stages lnw * x and scales the finished sums by 1 / rms of the activation row (sum x^2 is
// accumulated by fixed threads while staging, reduced in a fixed order: deterministic).  K-split
// partials carry the raw sums and, with the RMSNorm, the per-split sum x^2 of every row.
constexpr int kCK = 4;                       // blocks per staged chunk
constexpr int kSRow = kCK * QK + 8;          // bf16 per staged activation row (16 B of padding)

// Occupancy: K-split instances (the layer projections of a decode batch) are held to three waves per
// SIMD (168 registers, a few spilled: batch-32 decode 9.51K against 9.19K tokens/s); the unsplit ones
// (tall weights such as the LM head) to two (three measured 166 against 101 us for the batch-16 LM head).
template <int DT, int NC, int EPI, bool SPLIT, bool NORM>
__global__ __launch_bounds__(256, SPLIT ? 3 : 2) void qgemm_small_kernel(const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq,
                                                           int nblk, int64_t rows_out, const float *__restrict__ x,
                                                           int64_t ldx, const float *__restrict__ lnw, float eps,
                                                           int64_t batch, const float *__restrict__ bias,
                                                           float *__restrict__ y, int64_t ldy, float *__restrict__ part,
                                                           float *__restrict__ part_ssq, int kper) {
    constexpr float OFF = DT == VGX_Q8_0 ? 128.0f : 8.0f;
    constexpr int R = 16 * NC;                     // staged activation rows
    constexpr int F4 = R * kCK * 8 / 256;          // staged float4 per thread per chunk
    __shared__ __align__(16) uint16_t sh[2][R][kSRow];
    __shared__ __align__(16) uint16_t sl[2][R][kSRow];
    __shared__ float ssum[2][R][kCK];
    __shared__ float sinv[R];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4, r4 = l16 & 3;
    const int64_t rq_wave = ((int64_t)blockIdx.x * 4 + wave) * 8;
    const int64_t b0 = (int64_t)blockIdx.y * R;
    const int cols = nblk * QK;

    int64_t arq[2], crq[2];
    bool aok[2], cok[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        arq[t] = rq_wave + 4 * t + (l16 >> 2);
        aok[t] = arq[t] < n_rq;
        crq[t] = rq_wave + 4 * t + lg;
        cok[t] = crq[t] < n_rq;
    }
    const int blk_lo = SPLIT ? (int)blockIdx.z * kper : 0;
    const int blk_hi = SPLIT ? min(nblk, blk_lo + kper) : nblk;
    const int n_chunks = blk_hi > blk_lo ? (blk_hi - blk_lo + kCK - 1) / kCK : 0;

    // staging: thread t takes float4 f = t + 256 i of the chunk (row f / 32, block (f / 8) % 4, quad f % 8)
    float4 xr[F4], gr[F4];
    float ssq[F4];
#pragma unroll
    for (int i = 0; i < F4; ++i) ssq[i] = 0.0f;
    auto stage_load = [&](int c) {
        const int cb0 = blk_lo + c * kCK;
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + 256 * i, row = f >> 5, blk = cb0 + ((f >> 3) & 3), j4 = f & 7;
            const int64_t br = b0 + row;
            xr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            gr[i] = make_float4(1.f, 1.f, 1.f, 1.f);
            if (br < batch && blk < blk_hi) {
                xr[i] = *reinterpret_cast<const float4 *>(x + br * ldx + blk * QK + j4 * 4);
                if constexpr (NORM) gr[i] = *reinterpret_cast<const float4 *>(lnw + blk * QK + j4 * 4);
            }
        }
    };
    auto stage_store = [&](int buf) {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + 256 * i, row = f >> 5, bl = (f >> 3) & 3, j4 = f & 7;
            const float e[4] = {xr[i].x, xr[i].y, xr[i].z, xr[i].w};
            const float g[4] = {gr[i].x, gr[i].y, gr[i].z, gr[i].w};
            float u[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (NORM) ssq[i] = fmaf(e[k], e[k], ssq[i]);
                u[k] = NORM ? g[k] * e[k] : e[k];
            }
            uint2 hw, lw;
            float r01[2], r23[2];
            split_bf16_f16x2(u[0], u[1], hw.x, lw.x, r01);
            split_bf16_f16x2(u[2], u[3], hw.y, lw.y, r23);
            float sum = (r01[0] + r01[1]) + (r23[0] + r23[1]);   // the four elements as the pieces represent them
            *reinterpret_cast<uint2 *>(&sh[buf][row][bl * QK + j4 * 4]) = hw;
            *reinterpret_cast<uint2 *>(&sl[buf][row][bl * QK + j4 * 4]) = lw;
            // the 8 threads of one (row, block) are 8 consecutive lanes
            sum += __shfl_xor(sum, 1, kWave);
            sum += __shfl_xor(sum, 2, kWave);
            sum += __shfl_xor(sum, 4, kWave);
            if (j4 == 0) ssum[buf][row][bl] = sum;
        }
    };

    struct AReg {
        uint2 wa[2], sc[2];
    };
    AReg ra[kCK], rb[kCK];
    auto fetch_a = [&](AReg (&r)[kCK], int c) {
        const int cb0 = blk_lo + c * kCK;
#pragma unroll
        for (int u = 0; u < kCK; ++u) {
            const int blk = cb0 + u;
            const bool in = blk < blk_hi;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                r[u].wa[t] = (in && aok[t]) ? load_a<DT>(W, arq[t], nblk, blk, r4, lg) : make_uint2(0, 0);
                r[u].sc[t] = (in && cok[t]) ? *reinterpret_cast<const uint2 *>(W + soff + (crq[t] * nblk + blk) * 8)
                                            : make_uint2(0, 0);
            }
        }
    };

    f32x4_t acc[2][NC];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int c = 0; c < NC; ++c) acc[t][c] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

    auto compute = [&](const AReg (&r)[kCK], int buf) {
#pragma unroll
        for (int u = 0; u < kCK; ++u) {
            bf16x8_t af[2];
            f16x8_t ah[2];
            float d[2][4];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                af[t] = a_frag<DT, true>(r[u].wa[t], lg, &ah[t]);
                d[t][0] = half_bits_to_float(r[u].sc[t].x);
                d[t][1] = half_bits_to_float(r[u].sc[t].x >> 16);
                d[t][2] = half_bits_to_float(r[u].sc[t].y);
                d[t][3] = half_bits_to_float(r[u].sc[t].y >> 16);
            }
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                const int row = c * 16 + l16;
                const uint4 xh = *reinterpret_cast<const uint4 *>(&sh[buf][row][u * QK + 8 * lg]);
                const uint4 xl = *reinterpret_cast<const uint4 *>(&sl[buf][row][u * QK + 8 * lg]);
                const float corr = OFF * ssum[buf][row][u];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    f32x4_t pr = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                    pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[t], __builtin_bit_cast(bf16x8_t, xh), pr, 0, 0, 0);
                    pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah[t], __builtin_bit_cast(f16x8_t, xl), pr, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[t][c][i] = fmaf(d[t][i], pr[i] - corr, acc[t][c][i]);
                }
            }
        }
    };

    if (n_chunks > 0) {
        stage_load(0);
        fetch_a(ra, 0);
        stage_store(0);
    }
    __syncthreads();
    for (int c = 0; c < n_chunks; c += 2) {
        // chunk c from buffer 0 with ra; chunk c + 1 staged into buffer 1 meanwhile
        if (c + 1 < n_chunks) {
            stage_load(c + 1);
            fetch_a(rb, c + 1);
        }
        compute(ra, 0);
        if (c + 1 < n_chunks) stage_store(1);
        __syncthreads();
        if (c + 1 >= n_chunks) break;
        if (c + 2 < n_chunks) {
            stage_load(c + 2);
            fetch_a(ra, c + 2);
        }
        compute(rb, 1);
        if (c + 2 < n_chunks) stage_store(0);
        __syncthreads();
    }

    // RMSNorm: sum x^2 of activation row (tid / 32 + 8 i) over this K range, reduced over its 32 threads
    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const float t = xor16_sum(row16_sum(ssq[i]));
            if ((tid & 31) == 0) sinv[(tid >> 5) + 8 * i] = t;
        }
        __syncthreads();
        if constexpr (SPLIT) {
            if (blockIdx.x == 0 && tid < R && b0 + tid < batch)
                part_ssq[(int64_t)blockIdx.z * batch + b0 + tid] = sinv[tid];
        }
    }

    int64_t bb[NC];
    bool bok[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        bb[c] = b0 + 16 * c + l16;
        bok[c] = bb[c] < batch;
    }
    if constexpr (SPLIT) {
        const int64_t rows_p = n_rq * 4;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (!cok[t]) continue;
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                if (!bok[c]) continue;
                float4 v;
                v.x = acc[t][c][0]; v.y = acc[t][c][1]; v.z = acc[t][c][2]; v.w = acc[t][c][3];
                *reinterpret_cast<float4 *>(part + ((int64_t)blockIdx.z * batch + bb[c]) * rows_p + crq[t] * 4) = v;
            }
        }
        return;
    }
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        float inv = 1.0f;
        if constexpr (NORM) inv = 1.0f / sqrtf(sinv[c * 16 + l16] / (float)cols + eps);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            if (!cok[t] || !bok[c]) continue;
            float *yr = y + bb[c] * ldy;
            if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
                for (int k = 0; k < 2; ++k) {
                    const int64_t o = crq[t] * 2 + k;
                    if (o >= rows_out) continue;
                    const float g = acc[t][c][k] * inv, u = acc[t][c][2 + k] * inv;
                    yr[o] = g / (1.0f + __expf(-g)) * u;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t row = crq[t] * 4 + i;
                    if (row >= rows_out) continue;
                    float v = acc[t][c][i] * inv;
                    if (bias) v += bias[row];
                    if constexpr (EPI == EPI_ACCUM) v += yr[row];
                    yr[row] = v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------------------------
// Decode batches, K-split projections: qgemm_split_kernel.  A workgroup of 4 waves owns 128 weight
// rows (32 row-quads; wave w takes row-quads 8 w .. 8 w + 7 as two 16-row MFMA tiles) x 16 activation
// rows x one K range of at most kSplitMaxBlocks blocks, and writes the range's partial sums.
//  * Weights: every wave requests its whole K range at the start, as contiguous 16-byte loads (the
//    blocks of one row-quad are adjacent in the packed layout: for Q4_0 lane l loads bytes 16 (l % 16)
//    .. + 15 of the chunk's 256-byte run of row-quad 4 h + l / 16) and its scales as one dword per lane.
//    The fragment-shaped loads of qgemm_small_kernel (a lane's 4-8 bytes, four row-quads 3 KB apart per
//    instruction) measured twice as slow to stream.  Per 4-block chunk the wave passes the loaded words
//    through a wave-private LDS area into the MFMA layout: lane (row l % 16, K group l / 16) reads its
//    four blocks' words of one row as a single 16-byte (Q4_0) or two (Q8_0) LDS loads.
//  * The loads are unconditional buffer loads: rows past the weight and chunks past the range use
//    offsets past the buffer, which read as zero without a memory access, so the compiler's waits count
//    exactly the loads a chunk needs and its math starts when its own words have arrived.
//  * Activations: the whole K range of the 16 rows is staged once into LDS, as bf16 hi and fp16 lo in
//    the K-slot order of the weight fragments, with each block's offset correction (four copies, the
//    first MFMA's accumulator input); blocks past the range are staged as zeros (their weights, read
//    from the neighbouring blocks, then add 0).
//  * Q4_0 fragments: a lane's word holds bytes 4 lg .. 4 lg + 3 of its row's block, i.e. weights
//    4 lg + i (low nibbles) and 16 + 4 lg + i (high nibbles), K-slot order 4 lg + {0, 1, 2, 3},
//    16 + 4 lg + {0, 1, 2, 3}.  Each nibble n goes to the low bits of a 16-bit lane beside a constant
//    high byte with one byte permute per dword: bf16 0x4300 | n = 128 + n, fp16 0x6400 | n = 1024 + n.
//    The pieces are hi = bf16(16 x), lo = fp16(16 x - hi), so a block's products sum to
//    sum (n - 8)(hi + lo) + 136 sum hi + 1032 sum lo; the staged correction holds -(136 sum hi +
//    1032 sum lo) and the partials are scaled by 1/16 at the end.
//    Q8_0: the tiled kernel's fragments of bytes 8 lg .. 8 lg + 7 (order 0 2 1 3 4 6 5 7, offset 128
//    against the pieces bf16 hi and fp16 16 (x - hi)).
constexpr int kSplitMaxBlocks = 16;            // blocks per split (4 chunks)
constexpr int kSplitMaxChunks = kSplitMaxBlocks / kCK;
constexpr uint32_t kPastEnd = 0x80000000u;     // a buffer offset past every weight: reads zero

template <int DT>
struct SplitGeom {
    static constexpr int QB = DT == VGX_Q8_0 ? 32 : 16;             // bytes of one row's block
    static constexpr int NLD = DT == VGX_Q8_0 ? 4 : 2;              // 16-byte weight loads per lane and chunk
    static constexpr int ROW = 4 * QB + 16;                         // LDS bytes per weight row (4 blocks + pad)
    static constexpr int SCR = 48;                                  // LDS bytes per row-quad of scales
    static constexpr int WAVE = 32 * ROW + 8 * SCR;                 // LDS bytes per wave
};

// LDS of one workgroup: the staged activations of kSplitMaxChunks chunks, then 4 waves' areas.
constexpr int split_lds_bytes(int dt) {
    return kSplitMaxChunks * (2 * 16 * kSRow * 2 + 16 * kCK * 16) +
           4 * (dt == VGX_Q8_0 ? SplitGeom<VGX_Q8_0>::WAVE : SplitGeom<VGX_Q4_0>::WAVE);
}
static_assert(split_lds_bytes(VGX_Q8_0) <= 64 * 1024, "static LDS of qgemm_split_kernel");

// Q4_0 fragments of one lane's word (bytes 4 lg .. 4 lg + 3 of its row's block): bf16 128 + n and
// fp16 1024 + n, in the order of the nibbles' weights (low nibbles of bytes 0..3, then high nibbles).
// v_perm_b32 byte selectors: 0..3 pick bytes of the second operand (the nibbles), 4 and 5 the bytes
// 0x43 and 0x64 of the first.
__device__ __forceinline__ void q4_word_frags(uint32_t w, bf16x8_t &fb, f16x8_t &fh) {
    constexpr uint32_t C = 0x00006443u;
    const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
    fb = __builtin_bit_cast(bf16x8_t, make_uint4(__builtin_amdgcn_perm(C, lo, 0x04010400u),
                                                 __builtin_amdgcn_perm(C, lo, 0x04030402u),
                                                 __builtin_amdgcn_perm(C, hi, 0x04010400u),
                                                 __builtin_amdgcn_perm(C, hi, 0x04030402u)));
    fh = __builtin_bit_cast(f16x8_t, make_uint4(__builtin_amdgcn_perm(C, lo, 0x05010500u),
                                                __builtin_amdgcn_perm(C, lo, 0x05030502u),
                                                __builtin_amdgcn_perm(C, hi, 0x05010500u),
                                                __builtin_amdgcn_perm(C, hi, 0x05030502u)));
}

// ---------------------------------------------------------------------------------------------
// K splits summed without a second launch.  With FIN >= 0 a workgroup of qgemm_kslice_kernel (128
// weight rows x 16 activation rows x one K range) writes its partials and its rows' sum x^2 with agent-scope stores
// (written through to the device-coherent level), waits for them, and takes a ticket from its output
// tile's counter; the workgroup that draws the last ticket reads the tile's partials of every split
// with agent-scope loads, adds them in split order (the arithmetic of qgemm_reduce_kernel, so the
// results are the same bits), applies the epilogue FIN and resets the counter to zero for the next
// launch.  The counters live in a fixed region at the start of the workspace that stays zero between
// launches, so a captured graph needs no memset.
constexpr int kFinNone = -1;                    // FIN of a launch whose partials a reduce launch sums
constexpr int kQgemmTickets = 16384;            // tile counters at the start of the GEMM workspace
constexpr int64_t kQgemmTicketBytes = kQgemmTickets * 4;
constexpr int kFinLoads = 9;                    // splits the finishing workgroup requests at once

// One 16-byte agent-scope store (buffer store with sc1) at byte offset off of the partial buffer.
__device__ __forceinline__ void store4_agent(__amdgpu_buffer_rsrc_t rs, uint32_t off, float4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(
        (__attribute__((ext_vector_type(4))) uint32_t){__float_as_uint(v.x), __float_as_uint(v.y), __float_as_uint(v.z),
                                                     __float_as_uint(v.w)},
        rs, off, 0, 16);
}

// The tile's last workgroup: part [ks][batch][rows_p], pssq [ks][gridDim.x][batch] (or null);
// thread (row-quad tid % 32, activation rows tid / 32 and 8 + tid / 32) of tile (blockIdx.x, blockIdx.y).
template <int EPI, int RQT = 32>
__device__ __forceinline__ void ksplit_finish(const float *part, int ks, int64_t batch, int64_t n_rq, int64_t rows_out,
                                              const float *pssq, int cols, float eps, const float *bias, float *y,
                                              int64_t ldy, int *cnt, int *flag) {
    const int tid = threadIdx.x;
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's partial stores have completed
    __syncthreads();
    if (tid == 0) {
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *flag = old == ks - 1;
    }
    __syncthreads();
    if (!*flag) return;
    // thread: row-quad tid % RQT of the tile, activation rows tid / RQT + (256 / RQT) i
    constexpr int NI = RQT / 16, BS = 256 / RQT;
    const int64_t rows_p = n_rq * 4;
    const int64_t rq = (int64_t)blockIdx.x * RQT + (tid % RQT);
    const int64_t bA = (int64_t)blockIdx.y * 16 + tid / RQT;
    const int64_t gx = gridDim.x;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void *)part, 0, (int)(ks * batch * rows_p * 4), 0x00020000);
    float4 v[NI];
    float t[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        v[i] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        t[i] = 0.0f;
    }
    for (int s0 = 0; s0 < ks; s0 += kFinLoads) {
        float4 p[NI][kFinLoads];
        float q[NI][kFinLoads];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int64_t b = bA + BS * i;
#pragma unroll
            for (int u = 0; u < kFinLoads; ++u) {
                const int64_t sp = min(s0 + u, ks - 1);
                const uint32_t o = b < batch && rq < n_rq ? (uint32_t)(((sp * batch + b) * rows_p + rq * 4) * 4) : kPastEnd;
                const auto w = __builtin_amdgcn_raw_buffer_load_b128(prs, o, 0, 16);
                p[i][u] = make_float4(__uint_as_float(w[0]), __uint_as_float(w[1]), __uint_as_float(w[2]), __uint_as_float(w[3]));
                q[i][u] = pssq && b < batch ? __hip_atomic_load(pssq + (sp * gx + blockIdx.x) * batch + b, __ATOMIC_RELAXED,
                                                                __HIP_MEMORY_SCOPE_AGENT)
                                            : 0.0f;
            }
        }
#pragma unroll
        for (int i = 0; i < NI; ++i)
#pragma unroll
            for (int u = 0; u < kFinLoads; ++u)
                if (s0 + u < ks) {
                    v[i].x += p[i][u].x;
                    v[i].y += p[i][u].y;
                    v[i].z += p[i][u].z;
                    v[i].w += p[i][u].w;
                    t[i] += q[i][u];
                }
    }
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int64_t b = bA + BS * i;
        if (b >= batch || rq >= n_rq) continue;
        const float inv = pssq ? 1.0f / sqrtf(t[i] / (float)cols + eps) : 1.0f;
        float *yr = y + b * ldy;
        const float e[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
        if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int64_t o = 2 * rq + k;
                if (o >= rows_out) continue;
                const float g = e[k] * inv, u = e[2 + k] * inv;
                yr[o] = g / (1.0f + __expf(-g)) * u;
            }
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t row = 4 * rq + r;
                if (row >= rows_out) continue;
                float a = e[r] * inv;
                if (bias) a += bias[row];
                if constexpr (EPI == EPI_ACCUM) a += yr[row];
                yr[row] = a;
            }
        }
    }
    if (tid == 0) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The work of one qgemm_split_kernel workgroup: row tile bx of W (blockIdx.y: activation tile,
// blockIdx.z: split), with the workgroup's LDS areas passed in.
template <int DT, bool NORM>
__device__ __forceinline__ void split_tile(uint8_t *__restrict__ smem_dyn, float *__restrict__ sinv, int64_t bx,
                                           const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq, int nblk,
                                           int w_bytes, const float *__restrict__ x, int64_t ldx,
                                           const float *__restrict__ lnw, int64_t batch, float *__restrict__ part,
                                           float *__restrict__ part_ssq, int kper) {
    using G = SplitGeom<DT>;
    constexpr int QB = G::QB;
    constexpr int R = 16;                                     // activation rows
    constexpr int F4 = R * kCK * 8 / 256;                     // staged float4 per thread and chunk
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, lg = lane >> 4;
    const int64_t rq_wave = (bx * 4 + wave) * 8;
    const int64_t b0 = (int64_t)blockIdx.y * R;
    const int blk_lo = (int)blockIdx.z * kper;
    const int blk_hi = min(nblk, blk_lo + kper);
    const int n_chunks = (blk_hi - blk_lo + kCK - 1) / kCK;   // 1 .. kSplitMaxChunks
    const int cols = nblk * QK;
    // LDS: activations [chunk][plane hi, lo][row][kSRow] bf16 / fp16, negated offset corrections
    // [chunk][row][kCK] (four copies each), then the waves' areas
    constexpr int PL = R * kSRow * 2;
    uint16_t *xs = reinterpret_cast<uint16_t *>(smem_dyn);
    float4 *cneg = reinterpret_cast<float4 *>(smem_dyn + kSplitMaxChunks * 2 * PL);
    uint8_t *wl = smem_dyn + kSplitMaxChunks * (2 * PL + R * kCK * 16) + wave * G::WAVE;
    uint8_t *wsc = wl + 32 * G::ROW;

    // activations first (their wait then leaves the weight loads in flight)
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (int)(((batch - 1) * ldx + cols) * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t grs =
        __builtin_amdgcn_make_buffer_rsrc((void *)lnw, 0, NORM ? cols * 4 : 0, 0x00020000);
    float4 xr[kSplitMaxChunks][F4], gr[kSplitMaxChunks];
#pragma unroll
    for (int c = 0; c < kSplitMaxChunks; ++c) {
        const int bl = (tid >> 3) & 3, j4 = tid & 7;
        const uint32_t ko = (uint32_t)(((blk_lo + c * kCK + bl) * QK + j4 * 4) * 4);
        if constexpr (NORM) {
            const auto g = __builtin_amdgcn_raw_buffer_load_b128(grs, ko, 0, 0);
            gr[c] = make_float4(__uint_as_float(g[0]), __uint_as_float(g[1]), __uint_as_float(g[2]), __uint_as_float(g[3]));
        }
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int64_t br = b0 + ((tid + 256 * i) >> 5);
            const uint32_t o = br < batch ? (uint32_t)(br * ldx * 4) + ko : kPastEnd;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, o, 0, 0);
            xr[c][i] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
        }
    }

    // weights and scales of the whole range
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, w_bytes, 0x00020000);
    uint32_t wv[G::NLD], sv;
#pragma unroll
    for (int h = 0; h < G::NLD; ++h) {
        const int64_t rq = rq_wave + (DT == VGX_Q8_0 ? 2 * h + (lane >> 5) : 4 * h + (lane >> 4));
        wv[h] = rq < n_rq ? (uint32_t)(rq * nblk * 4 * QB) + (uint32_t)((lane & (DT == VGX_Q8_0 ? 31 : 15)) * 16)
                          : kPastEnd;
    }
    {
        const int64_t rq = rq_wave + (lane >> 3);
        sv = rq < n_rq ? (uint32_t)(soff + rq * nblk * 8) + (uint32_t)((lane & 7) * 4) : kPastEnd;
    }
    // scales of every chunk first, then the quants chunk by chunk (a chunk's wait then leaves the later
    // chunks' loads in flight)
    uint4 wr[kSplitMaxChunks][G::NLD];
    uint32_t sr[kSplitMaxChunks];
#pragma unroll
    for (int c = 0; c < kSplitMaxChunks; ++c)
        sr[c] = __builtin_amdgcn_raw_buffer_load_b32(wrs, sv, c < n_chunks ? (blk_lo + c * kCK) * 8 : 0x40000000, 0);
#pragma unroll
    for (int c = 0; c < kSplitMaxChunks; ++c) {
        const int so = c < n_chunks ? (blk_lo + c * kCK) * 4 * QB : 0x40000000;   // past the range: past the buffer
#pragma unroll
        for (int h = 0; h < G::NLD; ++h) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, wv[h], so, 0);
            wr[c][h] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }

    // stage the activations: bf16 hi, fp16 lo, offset corrections; sum x^2 for the RMSNorm
    float ssq[F4];
#pragma unroll
    for (int i = 0; i < F4; ++i) ssq[i] = 0.0f;
#pragma unroll
    for (int c = 0; c < kSplitMaxChunks; ++c) {
        if (c >= n_chunks) break;
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const int f = tid + 256 * i, row = f >> 5, bl = (f >> 3) & 3, j4 = f & 7;
            const bool in = blk_lo + c * kCK + bl < blk_hi;
            const float e[4] = {in ? xr[c][i].x : 0.0f, in ? xr[c][i].y : 0.0f, in ? xr[c][i].z : 0.0f,
                                in ? xr[c][i].w : 0.0f};
            float u[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if constexpr (NORM) {
                    ssq[i] = fmaf(e[k], e[k], ssq[i]);
                    const float g = k == 0 ? gr[c].x : k == 1 ? gr[c].y : k == 2 ? gr[c].z : gr[c].w;
                    u[k] = g * e[k];
                } else {
                    u[k] = e[k];
                }
            }
            uint2 hw, lw;
            float sum;
            if constexpr (DT == VGX_Q4_0) {
                // pieces of 16 x in natural order; correction 136 sum hi + 1032 sum lo
                hw.x = pack_bf16x2(16.0f * u[0], 16.0f * u[1]);
                hw.y = pack_bf16x2(16.0f * u[2], 16.0f * u[3]);
                const float h[4] = {__uint_as_float(hw.x << 16), __uint_as_float(hw.x & 0xFFFF0000u),
                                    __uint_as_float(hw.y << 16), __uint_as_float(hw.y & 0xFFFF0000u)};
                lw.x = pack_f16x2(fmaf(16.0f, u[0], -h[0]), fmaf(16.0f, u[1], -h[1]));
                lw.y = pack_f16x2(fmaf(16.0f, u[2], -h[2]), fmaf(16.0f, u[3], -h[3]));
                const auto l01 = __builtin_bit_cast(vgx_f16x2_t, lw.x), l23 = __builtin_bit_cast(vgx_f16x2_t, lw.y);
                const float sh = (h[0] + h[1]) + (h[2] + h[3]);
                const float sl = ((float)l01[0] + (float)l01[1]) + ((float)l23[0] + (float)l23[1]);
                sum = fmaf(1032.0f, sl, 136.0f * sh);
            } else {
                float r02[2], r13[2];
                split_bf16_f16x2(u[0], u[2], hw.x, lw.x, r02);     // stored order 0, 2, 1, 3
                split_bf16_f16x2(u[1], u[3], hw.y, lw.y, r13);
                sum = 128.0f * ((r02[0] + r13[0]) + (r02[1] + r13[1]));
            }
            const int pos = DT == VGX_Q4_0 ? 8 * (j4 & 3) + 4 * (j4 >> 2) : 4 * j4;
            *reinterpret_cast<uint2 *>(xs + ((c * 2) * R + row) * kSRow + bl * QK + pos) = hw;
            *reinterpret_cast<uint2 *>(xs + ((c * 2 + 1) * R + row) * kSRow + bl * QK + pos) = lw;
            sum += __shfl_xor(sum, 1, kWave);
            sum += __shfl_xor(sum, 2, kWave);
            sum += __shfl_xor(sum, 4, kWave);
            if (j4 == 0) cneg[(c * R + row) * kCK + bl] = make_float4(-sum, -sum, -sum, -sum);
        }
    }
    __syncthreads();

    f32x4_t acc[2];
    acc[0] = acc[1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < kSplitMaxChunks; ++c) {
        if (c >= n_chunks) break;
        // the chunk's words into the MFMA layout through the wave's LDS area
#pragma unroll
        for (int h = 0; h < G::NLD; ++h) {
            const uint4 v = wr[c][h];
            if constexpr (DT == VGX_Q4_0) {
                const int row = (4 * h + (lane >> 4)) * 4 + (lane & 3), u = (lane & 15) >> 2;
                uint8_t *p = wl + row * G::ROW + u * 4;
                *reinterpret_cast<uint32_t *>(p) = v.x;
                *reinterpret_cast<uint32_t *>(p + 16) = v.y;
                *reinterpret_cast<uint32_t *>(p + 32) = v.z;
                *reinterpret_cast<uint32_t *>(p + 48) = v.w;
            } else {
                const int row = (2 * h + (lane >> 5)) * 4 + ((lane >> 1) & 3), u = (lane & 31) >> 3;
                uint8_t *p = wl + row * G::ROW + (2 * (lane & 1)) * 32 + u * 8;
                *reinterpret_cast<uint2 *>(p) = make_uint2(v.x, v.y);
                *reinterpret_cast<uint2 *>(p + 32) = make_uint2(v.z, v.w);
            }
        }
        *reinterpret_cast<uint32_t *>(wsc + (lane >> 3) * G::SCR + (lane & 7) * 4) = sr[c];
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint8_t *rp = wl + (16 * t + l16) * G::ROW + lg * QB;
            const uint4 s0 = *reinterpret_cast<const uint4 *>(wsc + (4 * t + lg) * G::SCR);
            const uint4 s1 = *reinterpret_cast<const uint4 *>(wsc + (4 * t + lg) * G::SCR + 16);
            uint32_t wq4[4];
            uint2 wq8[4];
            if constexpr (DT == VGX_Q4_0) {
                const uint4 a = *reinterpret_cast<const uint4 *>(rp);
                wq4[0] = a.x; wq4[1] = a.y; wq4[2] = a.z; wq4[3] = a.w;
            } else {
                const uint4 a = *reinterpret_cast<const uint4 *>(rp), b = *reinterpret_cast<const uint4 *>(rp + 16);
                wq8[0] = make_uint2(a.x, a.y); wq8[1] = make_uint2(a.z, a.w);
                wq8[2] = make_uint2(b.x, b.y); wq8[3] = make_uint2(b.z, b.w);
            }
            const uint2 scu[4] = {make_uint2(s0.x, s0.y), make_uint2(s0.z, s0.w), make_uint2(s1.x, s1.y),
                                  make_uint2(s1.z, s1.w)};
#pragma unroll
            for (int u = 0; u < kCK; ++u) {
                bf16x8_t af;
                f16x8_t ah;
                if constexpr (DT == VGX_Q4_0) q4_word_frags(wq4[u], af, ah);
                else tile_a_frags<DT>(wq8[u], lg, af, ah);
                const float d[4] = {half_bits_to_float(scu[u].x), half_bits_to_float(scu[u].x >> 16),
                                    half_bits_to_float(scu[u].y), half_bits_to_float(scu[u].y >> 16)};
                const uint4 xh = *reinterpret_cast<const uint4 *>(xs + ((c * 2) * R + l16) * kSRow + u * QK + 8 * lg);
                const uint4 xl = *reinterpret_cast<const uint4 *>(xs + ((c * 2 + 1) * R + l16) * kSRow + u * QK + 8 * lg);
                const float4 cn = cneg[(c * R + l16) * kCK + u];
                f32x4_t pr = f32x4_t{cn.x, cn.y, cn.z, cn.w};
                pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, __builtin_bit_cast(bf16x8_t, xh), pr, 0, 0, 0);
                pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, __builtin_bit_cast(f16x8_t, xl), pr, 0, 0, 0);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(d[i], pr[i], acc[t][i]);
            }
        }
        // this chunk's LDS reads are done before the next chunk's writes (in order within the wave)
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    if constexpr (NORM) {
#pragma unroll
        for (int i = 0; i < F4; ++i) {
            const float t = xor16_sum(row16_sum(ssq[i]));
            if ((tid & 31) == 0) sinv[(tid >> 5) + 8 * i] = t;
        }
        __syncthreads();
        if (bx == 0 && tid < R && b0 + tid < batch)
            part_ssq[(int64_t)blockIdx.z * batch + b0 + tid] = sinv[tid];
    }
    const int64_t bb = b0 + l16;
    if (bb < batch) {
        const int64_t rows_p = n_rq * 4;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int64_t crq = rq_wave + 4 * t + lg;
            if (crq >= n_rq) continue;
            constexpr float S = DT == VGX_Q4_0 ? 0.0625f : 1.0f;   // Q4_0 pieces carry 16 x
            *reinterpret_cast<float4 *>(part + ((int64_t)blockIdx.z * batch + bb) * rows_p + crq * 4) =
                make_float4(S * acc[t][0], S * acc[t][1], S * acc[t][2], S * acc[t][3]);
        }
    }
}

template <int DT, bool NORM>
__global__ __launch_bounds__(256, DT == VGX_Q8_0 ? 2 : 3) void qgemm_split_kernel(const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq,
                                                             int nblk, int w_bytes, const float *__restrict__ x,
                                                             int64_t ldx, const float *__restrict__ lnw,
                                                             int64_t batch, float *__restrict__ part,
                                                             float *__restrict__ part_ssq, int kper) {
    __shared__ __align__(16) uint8_t smem_dyn[split_lds_bytes(DT)];
    __shared__ float sinv[16];
    split_tile<DT, NORM>(smem_dyn, sinv, blockIdx.x, W, soff, n_rq, nblk, w_bytes, x, ldx, lnw, batch, part, part_ssq,
                         kper);
}

// The q and k|v projections of a decode batch (same activations, same K splits) in one launch: row
// tiles 0 .. q.gx - 1 of the grid are q's, the rest k|v's, so the two weights' workgroups share the GPU
// instead of two launches each filling part of it.
struct SplitJob {
    const uint8_t *w;
    int64_t soff, n_rq;
    int w_bytes, gx, ks;
    float *part, *pssq;
};

template <int QDT, int KDT, bool NORM>
__global__ __launch_bounds__(256, QDT == VGX_Q8_0 || KDT == VGX_Q8_0 ? 2 : 3) void qkv_split_kernel(
    SplitJob jq, SplitJob jk, int nblk, const float *__restrict__ x, int64_t ldx, const float *__restrict__ lnw,
    int64_t batch, int kper) {
    constexpr int LB = split_lds_bytes(QDT) > split_lds_bytes(KDT) ? split_lds_bytes(QDT) : split_lds_bytes(KDT);
    __shared__ __align__(16) uint8_t smem_dyn[LB];
    __shared__ float sinv[16];
    if ((int)blockIdx.x < jq.gx) {
        if ((int)blockIdx.z < jq.ks)
            split_tile<QDT, NORM>(smem_dyn, sinv, blockIdx.x, jq.w, jq.soff, jq.n_rq, nblk, jq.w_bytes, x, ldx, lnw,
                                  batch, jq.part, jq.pssq, kper);
    } else if ((int)blockIdx.z < jk.ks) {
        split_tile<KDT, NORM>(smem_dyn, sinv, (int64_t)blockIdx.x - jq.gx, jk.w, jk.soff, jk.n_rq, nblk, jk.w_bytes, x,
                              ldx, lnw, batch, jk.part, jk.pssq, kper);
    }
}

// ---------------------------------------------------------------------------------------------
// Decode batches, K-split Q4_0 projections of 16-block splits: qgemm_kslice_kernel.  A workgroup owns
// the tile of qgemm_split_kernel (128 weight rows, or 64 for projections of few rows such as o and down
// (RQT = 16), x 16 activation rows x a K range of 16 blocks), but each of its 4 waves takes one 4-block
// slice of the range for all the tile's rows, so the activations never
// pass through LDS (against qgemm_split_kernel, gate/up of the 1.5B model at batch 32 measured 17.0 ->
// 15.1 us per launch, down 11.0 -> 9.5 us):
//  * Activations: lane (row l16, K group lg) loads its 8 values of each block of the slice (K slots
//    4 lg + {0..3} and 16 + 4 lg + {0..3}, the order of q4_word_frags) and keeps them in registers
//    as the MFMA B operands, bf16 hi = 16 x and fp16 lo = 16 x - hi (x times the RMSNorm weight);
//    the block's correction 136 sum hi + 1032 sum lo is summed over the four K groups with lane swaps.
//  * Weights: the slice of a row-quad is one contiguous 256-byte run (4 blocks x 4 rows x 16 bytes),
//    loaded as 16-byte pieces into a wave-private LDS area in the MFMA layout: row r, piece lg of its
//    4 blocks in slot lg ^ ((r >> 2) & 3), so that both the writes and the 16-byte reads of a tile are
//    free of bank conflicts.  The slice's scales (32 bytes per row-quad) go next to them.
//  * Per 16-row tile: per block, the bf16 and fp16 MFMAs from a zero accumulator, then the block's
//    scales into the tile's sums (one fma per output); the offset corrections of the four blocks enter
//    with one fp32 MFMA (scales of the tile's rows x -correction of the activation rows).
//  * The four slices' sums are added in slice order through LDS; the workgroup writes one partial per
//    output, scaled by 1/16, and the per-row sum x^2 of its range.
//  * Four waves per SIMD (at most 128 VGPRs): 1024 workgroup slots, so gate/up (840 workgroups) runs
//    in one round.
constexpr int kKsRow = 64;                         // LDS bytes per weight row of a slice
constexpr int kKsSlice = 128 * kKsRow + 32 * 32;   // per slice: 128 rows, then 32 row-quads of scales
constexpr int kKsLds = 4 * kKsSlice;
static_assert(kKsLds >= 4 * 8 * 64 * 16 + 4 * 16 * 4, "the LDS of qgemm_kslice_kernel holds the cross-slice sums");

template <bool NORM, int FIN, int RQT = 32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 4))) void qgemm_kslice_kernel(
    const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq, int nblk, int w_bytes, const float *__restrict__ x,
    int64_t ldx, const float *__restrict__ lnw, int64_t batch, float *__restrict__ part, float *__restrict__ part_ssq,
    int kper, int64_t rows_out, float eps, const float *__restrict__ bias, float *__restrict__ y, int64_t ldy,
    int *__restrict__ cnt) {
    __shared__ __align__(16) uint8_t smem[kKsLds];
    const int tid = threadIdx.x, lane = tid & 63, sl = tid >> 6;   // the wave's K slice
    const int l16 = lane & 15, lg = lane >> 4;
    constexpr int NT = RQT / 4;                        // 16-row MFMA tiles of the workgroup's rows
    static_assert(RQT == 32 || RQT == 16, "row tiles of 128 or 64 rows");
    const int64_t rq0 = (int64_t)blockIdx.x * RQT;
    const int64_t b0 = (int64_t)blockIdx.y * 16;
    const int blk_lo = (int)blockIdx.z * kper;
    const int blk_hi = min(nblk, blk_lo + kper);
    const int wb0 = blk_lo + 4 * sl;                   // first block of this wave's slice
    const int cols = nblk * QK;
    uint8_t *wl = smem + sl * kKsSlice;
    uint8_t *wsc = wl + 128 * kKsRow;

    // activations of the slice first, then the weights and scales
    const __amdgpu_buffer_rsrc_t xrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)x, 0, (int)(((batch - 1) * ldx + cols) * 4), 0x00020000);
    const __amdgpu_buffer_rsrc_t grs =
        __builtin_amdgcn_make_buffer_rsrc((void *)lnw, 0, NORM ? cols * 4 : 0, 0x00020000);
    const int64_t brow = b0 + l16;
    float4 xv[4][2], gv[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        const bool in = wb0 + u < blk_hi;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            const uint32_t ko = (uint32_t)(((wb0 + u) * QK + 16 * hf + 4 * lg) * 4);
            const uint32_t o = in && brow < batch ? (uint32_t)(brow * ldx * 4) + ko : kPastEnd;
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(xrs, o, 0, 0);
            xv[u][hf] = make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
            if constexpr (NORM) {
                const auto g = __builtin_amdgcn_raw_buffer_load_b128(grs, in ? ko : kPastEnd, 0, 0);
                gv[u][hf] = make_float4(__uint_as_float(g[0]), __uint_as_float(g[1]), __uint_as_float(g[2]), __uint_as_float(g[3]));
            }
        }
    }
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, w_bytes, 0x00020000);
    const bool live = wb0 < blk_hi;                    // wave-uniform: a slice past the range adds nothing
    uint4 wr[NT];
#pragma unroll
    for (int h = 0; h < NT; ++h) {
        const int64_t rq = rq0 + 4 * h + (lane >> 4);
        const uint32_t o = live && rq < n_rq ? (uint32_t)(rq * nblk * 64 + (int64_t)wb0 * 64) + (uint32_t)(l16 * 16)
                                             : kPastEnd;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, o, 0, 0);
        wr[h] = make_uint4(v[0], v[1], v[2], v[3]);
    }
    uint4 sr;
    {
        const int64_t rq = rq0 + (lane >> 1);
        const uint32_t o = live && (lane >> 1) < RQT && rq < n_rq
                               ? (uint32_t)(soff + rq * nblk * 8 + (int64_t)(wb0 + 2 * (lane & 1)) * 8)
                               : kPastEnd;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, o, 0, 0);
        sr = make_uint4(v[0], v[1], v[2], v[3]);
    }

    // B operands: hi = bf16(16 v), lo = fp16(16 v - hi), v = x (times the RMSNorm weight)
    uint4 bh[4], bl[4];
    float cb[4], ssq = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        float e[8] = {xv[u][0].x, xv[u][0].y, xv[u][0].z, xv[u][0].w, xv[u][1].x, xv[u][1].y, xv[u][1].z, xv[u][1].w};
        if constexpr (NORM) {
            const float g[8] = {gv[u][0].x, gv[u][0].y, gv[u][0].z, gv[u][0].w,
                                gv[u][1].x, gv[u][1].y, gv[u][1].z, gv[u][1].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                ssq = fmaf(e[i], e[i], ssq);
                e[i] *= g[i];
            }
        }
        uint32_t hw[4], lw[4];
        float sh = 0.0f, sm = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            hw[i] = pack_bf16x2(16.0f * e[2 * i], 16.0f * e[2 * i + 1]);
            const float h0 = __uint_as_float(hw[i] << 16), h1 = __uint_as_float(hw[i] & 0xFFFF0000u);
            lw[i] = pack_f16x2(fmaf(16.0f, e[2 * i], -h0), fmaf(16.0f, e[2 * i + 1], -h1));
            const auto l2 = __builtin_bit_cast(vgx_f16x2_t, lw[i]);
            sh += h0 + h1;
            sm += (float)l2[0] + (float)l2[1];
        }
        bh[u] = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        bl[u] = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        cb[u] = xor32_sum(xor16_sum(fmaf(1032.0f, sm, 136.0f * sh)));
    }
    // the correction MFMA's B operand: -correction of (activation row l16, block lg)
    const float cneg = -(lg == 0 ? cb[0] : lg == 1 ? cb[1] : lg == 2 ? cb[2] : cb[3]);

    // the slice's weights into the MFMA layout, its scales next to them
#pragma unroll
    for (int h = 0; h < NT; ++h) {
        const int r = 4 * (4 * h + (lane >> 4)) + (lane & 3), u = (lane >> 2) & 3;
        uint32_t *p = reinterpret_cast<uint32_t *>(wl + r * kKsRow) + u;
        const int sw = (r >> 2) & 3;
        p[(0 ^ sw) * 4] = wr[h].x;
        p[(1 ^ sw) * 4] = wr[h].y;
        p[(2 ^ sw) * 4] = wr[h].z;
        p[(3 ^ sw) * 4] = wr[h].w;
    }
    *reinterpret_cast<uint4 *>(wsc + (lane >> 1) * 32 + (lane & 1) * 16) = sr;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    f32x4_t acc[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int row = 16 * t + l16;
            const uint4 a = *reinterpret_cast<const uint4 *>(wl + row * kKsRow + ((lg ^ ((l16 >> 2) & 3)) * 16));
            const uint4 s0 = *reinterpret_cast<const uint4 *>(wsc + (4 * t + lg) * 32);
            const uint4 s1 = *reinterpret_cast<const uint4 *>(wsc + (4 * t + lg) * 32 + 16);
            const uint32_t da = *reinterpret_cast<const uint16_t *>(wsc + (4 * t + (l16 >> 2)) * 32 + lg * 8 + (l16 & 3) * 2);
            const uint32_t wq[4] = {a.x, a.y, a.z, a.w};
            const uint2 scu[4] = {make_uint2(s0.x, s0.y), make_uint2(s0.z, s0.w), make_uint2(s1.x, s1.y),
                                  make_uint2(s1.z, s1.w)};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                bf16x8_t af;
                f16x8_t ah;
                q4_word_frags(wq[u], af, ah);
                f32x4_t pr = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                pr = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, __builtin_bit_cast(bf16x8_t, bh[u]), pr, 0, 0, 0);
                pr = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, __builtin_bit_cast(f16x8_t, bl[u]), pr, 0, 0, 0);
                const float d[4] = {half_bits_to_float(scu[u].x), half_bits_to_float(scu[u].x >> 16),
                                    half_bits_to_float(scu[u].y), half_bits_to_float(scu[u].y >> 16)};
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(d[i], pr[i], acc[t][i]);
            }
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(half_bits_to_float(da), cneg, acc[t], 0, 0, 0);
        }
    }

    // the four slices' sums, added in slice order; the per-row sum x^2 of the range
    __syncthreads();
    float4 *red = reinterpret_cast<float4 *>(smem);
    float *rss = reinterpret_cast<float *>(smem + 4 * 8 * 64 * 16);
#pragma unroll
    for (int t = 0; t < NT; ++t) red[(sl * NT + t) * 64 + lane] = make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    if constexpr (NORM) {
        const float sq = xor32_sum(xor16_sum(ssq));
        if (lg == 0) rss[sl * 16 + l16] = sq;
    }
    __syncthreads();
    const int64_t rows_p = n_rq * 4;
    const int64_t bb = b0 + l16;
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc((void *)part, 0, FIN >= 0 ? (int)(gridDim.z * batch * rows_p * 4) : 0, 0x00020000);
#pragma unroll
    for (int j = 0; j < NT / 4; ++j) {
        const int t = (NT / 4) * sl + j;
        float4 v = red[t * 64 + lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) {
            const float4 o = red[(w * NT + t) * 64 + lane];
            v.x += o.x; v.y += o.y; v.z += o.z; v.w += o.w;
        }
        const int64_t crq = rq0 + 4 * t + lg;
        const float4 r = make_float4(0.0625f * v.x, 0.0625f * v.y, 0.0625f * v.z, 0.0625f * v.w);
        if (bb < batch && crq < n_rq) {
            const int64_t off = ((int64_t)blockIdx.z * batch + bb) * rows_p + crq * 4;
            if constexpr (FIN >= 0) store4_agent(prs, (uint32_t)(off * 4), r);
            else *reinterpret_cast<float4 *>(part + off) = r;
        }
    }
    if constexpr (NORM) {
        if (tid < 16 && b0 + tid < batch) {
            const float sq = ((rss[tid] + rss[16 + tid]) + rss[32 + tid]) + rss[48 + tid];
            if constexpr (FIN >= 0)
                __hip_atomic_store(part_ssq + ((int64_t)blockIdx.z * gridDim.x + blockIdx.x) * batch + b0 + tid, sq,
                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            else if (blockIdx.x == 0)
                part_ssq[(int64_t)blockIdx.z * batch + b0 + tid] = sq;
        }
    }
    if constexpr (FIN >= 0) {
        __shared__ int last;
        ksplit_finish<FIN, RQT>(part, (int)gridDim.z, batch, n_rq, rows_out, NORM ? part_ssq : nullptr, cols, eps, bias,
                                y, ldy, cnt + (int64_t)blockIdx.y * gridDim.x + blockIdx.x, &last);
    }
}

// Sum of the K-split partials + epilogue.  One thread per (activation row b, packed row-quad q): one
// 16-byte load per split brings the four sums of the quad (SwiGLU: gate rows 2q, 2q + 1 and up rows 2q,
// 2q + 1; otherwise output rows 4q .. 4q + 3).
// part_ssq (when not null): per-split sum x^2 of every activation row; the sums are then scaled by
// 1 / sqrt(mean(x^2) + eps) (the RMSNorm of the small-batch kernels).
// KM >= ks is a compile-time bound (equal to ks up to 18 splits): every split's load goes out at once
// (indexes clamped to the last split), then the sums run in split order, instead of one load round
// trip per split.
template <int EPI, int KM>
__global__ __launch_bounds__(256) void qgemm_reduce_kernel(const float *__restrict__ part, int ks, int64_t batch,
                                                            int64_t rows_p, int64_t rows_out,
                                                            const float *__restrict__ bias, float *__restrict__ y,
                                                            int64_t ldy, const float *__restrict__ part_ssq,
                                                            int cols, float eps) {
    const int64_t nq = rows_p >> 2;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= batch * nq) return;
    const int64_t b = i / nq, q = i - b * nq;
    float *yr = y + b * ldy;
    float inv = 1.0f;
    if (part_ssq) {
        float p[KM];
#pragma unroll
        for (int s = 0; s < KM; ++s) p[s] = part_ssq[(int64_t)min(s, ks - 1) * batch + b];
        float t = 0.0f;
#pragma unroll
        for (int s = 0; s < KM; ++s)
            if (s < ks) t += p[s];
        inv = 1.0f / sqrtf(t / (float)cols + eps);
    }
    float4 p[KM];
#pragma unroll
    for (int s = 0; s < KM; ++s)
        p[s] = *reinterpret_cast<const float4 *>(part + ((int64_t)min(s, ks - 1) * batch + b) * rows_p + q * 4);
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KM; ++s) {
        if (s < ks) {
            v[0] += p[s].x;
            v[1] += p[s].y;
            v[2] += p[s].z;
            v[3] += p[s].w;
        }
    }
    if constexpr (EPI == EPI_SWIGLU) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int64_t o = 2 * q + k;
            if (o >= rows_out) continue;
            const float g = v[k] * inv, u = v[2 + k] * inv;
            yr[o] = g / (1.0f + __expf(-g)) * u;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = 4 * q + r;
            if (row >= rows_out) continue;
            float t = v[r] * inv;
            if (bias) t += bias[row];
            if constexpr (EPI == EPI_ACCUM) t += yr[row];
            yr[row] = t;
        }
    }
}

// Reduce launch with the split bound of ks.
template <int EPI>
void reduce_launch(const float *part, int ks, int64_t batch, int64_t rows_p, int64_t rows_out, const float *bias,
                   float *y, int64_t ldy, const float *part_ssq, int cols, float eps, hipStream_t st) {
    const unsigned g = (unsigned)((batch * (rows_p / 4) + 255) / 256);
#define VGX_RED(KM) hipLaunchKernelGGL((qgemm_reduce_kernel<EPI, KM>), dim3(g), dim3(256), 0, st, part, ks, batch, \
                                       rows_p, rows_out, bias, y, ldy, part_ssq, cols, eps)
    switch (ks) {
        case 1: case 2: VGX_RED(2); break;
        case 3: VGX_RED(3); break;
        case 4: VGX_RED(4); break;
        case 5: VGX_RED(5); break;
        case 6: VGX_RED(6); break;
        case 7: VGX_RED(7); break;
        case 8: VGX_RED(8); break;
        case 9: VGX_RED(9); break;
        case 10: VGX_RED(10); break;
        case 11: VGX_RED(11); break;
        case 12: VGX_RED(12); break;
        case 13: VGX_RED(13); break;
        case 14: VGX_RED(14); break;
        case 15: VGX_RED(15); break;
        case 16: VGX_RED(16); break;
        case 17: VGX_RED(17); break;
        case 18: VGX_RED(18); break;
        default:
            if (ks <= 24) VGX_RED(24);
            else VGX_RED(32);
    }
#undef VGX_RED
}

// ---------------------------------------------------------------------------------------------
// Decode batches, tall projections without K splits (the LM head, 151665 x 1536 Q8_0): qgemm_wide_kernel.
// One persistent workgroup of 8 waves per CU holds the whole K of its 16 activation rows in LDS and
// streams its share of the weight rows past them, so the activations are converted once per workgroup
// and neither K-split partials nor a reduce launch exist:
//  * Activations: the RMSNorm (when given) is applied in the staging pass (each workgroup has whole
//    rows), then row b is scaled by 2^-e_b (e_b from its largest element, so that no value exceeds 2^14)
//    and stored as fp16 hi = fp16(v) and lo = fp16(v - hi) (22 significant bits), in the K-slot order of
//    the weight fragments, 16-byte groups swizzled by (row >> 2) & 3 against bank conflicts; with each
//    block's offset correction off * sum (hi + lo) (off = 1152 for Q8_0, 1032 for Q4_0).
//  * Weights: one fp16 fragment serves both products.  Q8_0: fp16(1024 + (q ^ 0x80)) = 0x6400 | byte,
//    the byte beside a constant 0x64 by one byte permute per two weights; Q4_0: fp16(1024 + n) from the
//    nibbles the same way.  A block's products then sum to sum q (hi + lo) + off sum (hi + lo).
//  * A wave takes 32 weight rows (two 16-row tiles, sharing each B operand read) over the whole K in
//    4-block chunks, the next three chunks' contiguous 16-byte weight loads in flight while it multiplies
//    the current one (through a wave-private LDS area into the MFMA layout, as qgemm_kslice_kernel); per
//    chunk and tile the scales enter with one fma per output and the offset corrections with one fp32
//    MFMA.  At the end of a tile pair the sums are scaled back by 2^e_b and stored.
//  * Grid: P row groups x the activation tiles; the workgroups of one row group sit on one XCD (ids
//    8 k + r for the same r), so the second activation tile reads the group's weights from that XCD's L2.
constexpr int kWideWaves = 12;                         // waves 0..7 also stage the activations
constexpr int kWideMaxCols = 1536;                      // staged K of 16 rows: 64 KiB per 1024 columns

template <int DT>
struct WideGeom {
    static constexpr int QB = DT == VGX_Q8_0 ? 32 : 16;         // bytes of one row's block
    static constexpr int NLD = DT == VGX_Q8_0 ? 4 : 2;          // 16-byte weight loads per lane and chunk
    static constexpr int ROW = DT == VGX_Q8_0 ? 128 : 64;       // LDS bytes per weight row of a chunk
    static constexpr int WAVE = 32 * ROW + 8 * 32;             // per wave: 32 rows, then 8 row-quads of scales
};

constexpr int wide_lds_bytes(int dt) {
    return kWideMaxCols / QK * (2 * 16 * 64 + 16 * 4) + 16 * 4 +
           kWideWaves * (dt == VGX_Q8_0 ? WideGeom<VGX_Q8_0>::WAVE : WideGeom<VGX_Q4_0>::WAVE);
}
static_assert(wide_lds_bytes(VGX_Q8_0) <= 160 * 1024, "LDS of qgemm_wide_kernel");

// One lane's fp16 fragment (1024 + unsigned weight) of one block: Q8_0 from its 8 bytes, Q4_0 from its word.
template <int DT>
__device__ __forceinline__ f16x8_t wide_frag(uint2 w) {
    constexpr uint32_t C = 0x00000064u;                 // byte 4 of the permute: 0x64
    uint32_t a, b;
    if constexpr (DT == VGX_Q8_0) {
        a = w.x ^ 0x80808080u;
        b = w.y ^ 0x80808080u;
    } else {
        a = w.x & 0x0F0F0F0Fu;                          // weights 4 lg + i (low nibbles)
        b = (w.x >> 4) & 0x0F0F0F0Fu;                   // weights 16 + 4 lg + i
    }
    return __builtin_bit_cast(f16x8_t, make_uint4(__builtin_amdgcn_perm(C, a, 0x04010400u),
                                                  __builtin_amdgcn_perm(C, a, 0x04030402u),
                                                  __builtin_amdgcn_perm(C, b, 0x04010400u),
                                                  __builtin_amdgcn_perm(C, b, 0x04030402u)));
}

template <int DT, bool NORM, int NCH>
__global__ __launch_bounds__(64 * kWideWaves, 1) void qgemm_wide_kernel(
    const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq, int nblk, int w_bytes, const float *__restrict__ x,
    int64_t ldx, const float *__restrict__ lnw, float eps, int64_t batch, float *__restrict__ y, int64_t ldy,
    int64_t rows_out, int n_groups) {
    using G = WideGeom<DT>;
    constexpr int QB = G::QB;
    constexpr float OFF = DT == VGX_Q8_0 ? 1152.0f : 1032.0f;
    __shared__ __align__(16) uint8_t smem[wide_lds_bytes(DT)];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l16 = lane & 15, lg = lane >> 4;
    const int cols = nblk * QK;
    // workgroup -> (row group, activation tile): ids 8 k + r with equal k / nbt share row group 8 k' + r
    const int nbt = (int)((batch + 15) / 16);
    const int id = blockIdx.x;
    const int grp = (id / (8 * nbt)) * 8 + (id & 7);
    const int bt = (id >> 3) % nbt;
    const int64_t b0 = (int64_t)bt * 16;
    uint8_t *xs = smem;                                              // [block][plane][row][64 B]
    float *corr = reinterpret_cast<float *>(smem + kWideMaxCols / QK * 2 * 16 * 64);   // [block][row]
    float *escale = corr + kWideMaxCols / QK * 16;                  // [row] 2^e_b
    uint8_t *wl = smem + kWideMaxCols / QK * (2 * 16 * 64 + 16 * 4) + 16 * 4 + wave * G::WAVE;
    uint8_t *wsc = wl + 32 * G::ROW;

    // ---- staging: thread (row tid / 32, float4 groups (tid % 32) + 32 i) of the first 8 waves
    if (tid < 16 * 32) {
        const int r = tid >> 5, j = tid & 31;
        const int64_t b = b0 + r;
        const int n4 = cols / 4;
        constexpr int MAXI = kWideMaxCols / 4 / 32;
        float4 v[MAXI];
        float ssq = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXI; ++i) {
            const int k4 = j + 32 * i;
            v[i] = k4 < n4 && b < batch ? *reinterpret_cast<const float4 *>(x + b * ldx + 4 * k4) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            ssq += v[i].x * v[i].x + v[i].y * v[i].y + v[i].z * v[i].z + v[i].w * v[i].w;
        }
        float inv = 1.0f;
        if constexpr (NORM) {
            const float t = xor16_sum(row16_sum(ssq));               // the 32 threads of the row
            inv = 1.0f / sqrtf(t / (float)cols + eps);
        }
        float mx = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXI; ++i) {
            const int k4 = j + 32 * i;
            if (NORM && k4 < n4) {
                const float4 g = *reinterpret_cast<const float4 *>(lnw + 4 * k4);
                v[i] = make_float4(g.x * (v[i].x * inv), g.y * (v[i].y * inv), g.z * (v[i].z * inv), g.w * (v[i].w * inv));
            }
            mx = fmaxf(mx, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
        }
        mx = xor16_max(row16_max(mx));
        int ex = 0;
        (void)frexpf(mx, &ex);                                       // mx < 2^ex
        const int e = ex > 14 ? ex - 14 : 0;
        const float sdown = ldexpf(1.0f, -e);
        if (j == 0) escale[r] = ldexpf(1.0f, e);
#pragma unroll
        for (int i = 0; i < MAXI; ++i) {
            const int k4 = j + 32 * i;
            if (k4 >= n4) break;
            const int kb = k4 >> 3, m = k4 & 7;
            const float e4[4] = {v[i].x * sdown, v[i].y * sdown, v[i].z * sdown, v[i].w * sdown};
            uint2 hw, lw;
            float hs = 0.0f;
            {
                const uint32_t h01 = pack_f16x2(e4[0], e4[1]), h23 = pack_f16x2(e4[2], e4[3]);
                const auto f01 = __builtin_bit_cast(vgx_f16x2_t, h01), f23 = __builtin_bit_cast(vgx_f16x2_t, h23);
                const float h[4] = {(float)f01[0], (float)f01[1], (float)f23[0], (float)f23[1]};
                const uint32_t l01 = pack_f16x2(e4[0] - h[0], e4[1] - h[1]), l23 = pack_f16x2(e4[2] - h[2], e4[3] - h[3]);
                const auto g01 = __builtin_bit_cast(vgx_f16x2_t, l01), g23 = __builtin_bit_cast(vgx_f16x2_t, l23);
                hs = ((h[0] + h[1]) + (h[2] + h[3])) + (((float)g01[0] + (float)g01[1]) + ((float)g23[0] + (float)g23[1]));
                hw = make_uint2(h01, h23);
                lw = make_uint2(l01, l23);
            }
            // K-slot position (halves) within the row's 32-slot block, then the swizzled 16-byte group
            const int pos = DT == VGX_Q8_0 ? 4 * m : 8 * (m & 3) + 4 * (m >> 2);
            const int grp16 = (pos >> 3) ^ ((r >> 2) & 3);
            uint8_t *row = xs + ((int64_t)kb * 2 * 16 + r) * 64;
            *reinterpret_cast<uint2 *>(row + grp16 * 16 + (pos & 7) * 2) = hw;
            *reinterpret_cast<uint2 *>(row + 16 * 64 + grp16 * 16 + (pos & 7) * 2) = lw;
            hs += __shfl_xor(hs, 1, kWave);
            hs += __shfl_xor(hs, 2, kWave);
            hs += __shfl_xor(hs, 4, kWave);
            if ((j & 7) == 0) corr[kb * 16 + r] = -OFF * hs;
        }
    }
    __syncthreads();

    // ---- streaming: wave w of row group grp takes 32-row pairs of tiles grp * per + w, + 8, ...
    const int64_t n_pairs = (n_rq + 7) / 8;                          // 8 row-quads per pair
    const int64_t per = (n_pairs + n_groups - 1) / n_groups;
    const int64_t p_lo = (int64_t)grp * per, p_hi = min(n_pairs, p_lo + per);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, w_bytes, 0x00020000);
    const int64_t my_first = p_lo + wave;
    const int my_n = my_first < p_hi ? (int)((p_hi - my_first + kWideWaves - 1) / kWideWaves) : 0;
    // a position in the wave's stream: its pair (0 .. my_n - 1) and chunk (0 .. NCH - 1)
    struct Pos {
        int pair, c;
    };
    // loads of chunk q.c of pair q.pair; past the wave's last pair: offsets past the buffer, no traffic.
    // The offsets are a wave-uniform base plus constant lane parts: row-quads past the weight (the
    // last pair) read the bytes after it inside the buffer, finite values whose rows are not stored.
    constexpr int PIECES = DT == VGX_Q8_0 ? 32 : 16;               // 16-byte pieces per row-quad chunk
    const uint32_t rq_bytes = (uint32_t)nblk * 4 * QB;              // one row-quad's quants
    const uint32_t lane_w = (uint32_t)(lane / PIECES) * rq_bytes + (uint32_t)(lane % PIECES) * 16;
    const int lane_blk = (lane >> 1) & 3;
    const uint32_t lane_s = (uint32_t)(lane >> 3) * (uint32_t)nblk * 8 + (uint32_t)lane_blk * 8 + (lane & 1) * 4;
    auto fetch = [&](const Pos &q, uint4 (&wv)[G::NLD + 1]) {
        const bool in = q.pair < my_n;
        const uint32_t pr = (uint32_t)(my_first + (int64_t)(in ? q.pair : 0) * kWideWaves);
        const int bk = q.c * kCK;
        const uint32_t base = pr * 8 * rq_bytes + (uint32_t)bk * 4 * QB;
#pragma unroll
        for (int h = 0; h < G::NLD; ++h) {
            const uint32_t o = in ? base + (uint32_t)(h * (64 / PIECES)) * rq_bytes + lane_w : kPastEnd;
            const auto t = __builtin_amdgcn_raw_buffer_load_b128(wrs, o, 0, 0);
            wv[h] = make_uint4(t[0], t[1], t[2], t[3]);
        }
        // scales: 8 row-quads x 4 blocks x 8 bytes, lane l: row-quad l / 8, block l % 8 / 2, half l % 2;
        // blocks past K (a partial last chunk) read zero, which zeroes their weights' products
        const uint32_t so = in && bk + lane_blk < nblk ? (uint32_t)soff + pr * 8 * (uint32_t)nblk * 8 + (uint32_t)bk * 8 + lane_s
                                                      : kPastEnd;
        wv[G::NLD].x = __builtin_amdgcn_raw_buffer_load_b32(wrs, so, 0, 0);
    };

    // outputs through buffer stores (rows past the weight or the batch: offsets past the buffer), so the
    // waits for the streamed weights count exactly
    const __amdgpu_buffer_rsrc_t yrs =
        __builtin_amdgcn_make_buffer_rsrc((void *)y, 0, (int)(((batch - 1) * ldy + rows_out) * 4), 0x00020000);
    f32x4_t acc[2];
    acc[0] = acc[1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    auto step = [&](const Pos &q, const uint4 (&wv)[G::NLD + 1]) {
        const int c = q.c;
        const int bk = c * kCK;
        // the chunk's words into the MFMA layout: row r (32 rows of the pair), block u, lane group lg
#pragma unroll
        for (int h = 0; h < G::NLD; ++h) {
            const uint4 v = wv[h];
            if constexpr (DT == VGX_Q8_0) {
                // lane: row-quad 2 h + lane / 32, 16-byte piece (lane % 32) = block u = piece / 8, row
                // r4 = piece / 2 % 4, half hf = piece % 2 (bytes 16 hf .. + 15 of the row's block)
                const int pc = lane & 31, u = pc >> 3, r4 = (pc >> 1) & 3, hf = pc & 1;
                const int row = (2 * h + (lane >> 5)) * 4 + r4;
                // row layout: [lg (0..3)][u][8 bytes], lg-groups of 32 bytes swizzled by (row >> 2) & 3
                uint8_t *p = wl + row * G::ROW;
                const int sw = (row >> 2) & 3;
                *reinterpret_cast<uint2 *>(p + ((2 * hf) ^ sw) * 32 + u * 8) = make_uint2(v.x, v.y);
                *reinterpret_cast<uint2 *>(p + ((2 * hf + 1) ^ sw) * 32 + u * 8) = make_uint2(v.z, v.w);
            } else {
                const int row = (4 * h + (lane >> 4)) * 4 + (lane & 3), u = (lane & 15) >> 2;
                uint32_t *p = reinterpret_cast<uint32_t *>(wl + row * G::ROW) + u;
                const int sw = (row >> 2) & 3;
                p[(0 ^ sw) * 4] = v.x;
                p[(1 ^ sw) * 4] = v.y;
                p[(2 ^ sw) * 4] = v.z;
                p[(3 ^ sw) * 4] = v.w;
            }
        }
        reinterpret_cast<uint32_t *>(wsc)[lane] = wv[G::NLD].x;      // [row-quad][block][4 halves]
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        const int xsw = (l16 >> 2) & 3;
        f32x4_t pr[2][4];
#pragma unroll
        for (int u = 0; u < kCK; ++u) {
            const int kb = min(bk + u, nblk - 1);                    // a block past K reads zero weights
            const uint8_t *xr = xs + ((int64_t)kb * 2 * 16 + l16) * 64 + (lg ^ xsw) * 16;
            const f16x8_t xh = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4 *>(xr));
            const f16x8_t xl = __builtin_bit_cast(f16x8_t, *reinterpret_cast<const uint4 *>(xr + 16 * 64));
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int row = 16 * t + l16;
                const int sw = (row >> 2) & 3;
                uint2 w;
                if constexpr (DT == VGX_Q8_0) w = *reinterpret_cast<const uint2 *>(wl + row * G::ROW + (lg ^ sw) * 32 + u * 8);
                else w = make_uint2(*reinterpret_cast<const uint32_t *>(wl + row * G::ROW + (lg ^ sw) * 16 + u * 4), 0u);
                const f16x8_t a = wide_frag<DT>(w);
                f32x4_t q = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                q = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xh, q, 0, 0, 0);
                q = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, xl, q, 0, 0, 0);
                pr[t][u] = q;
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            // scales of the tile's row-quads 4 t + lg for the chunk's blocks: wsc [rq][u] 4 halves
            const uint4 s0 = *reinterpret_cast<const uint4 *>(wsc + (4 * t + lg) * 32);
            const uint4 s1 = *reinterpret_cast<const uint4 *>(wsc + (4 * t + lg) * 32 + 16);
            const uint2 scu[4] = {make_uint2(s0.x, s0.y), make_uint2(s0.z, s0.w), make_uint2(s1.x, s1.y),
                                  make_uint2(s1.z, s1.w)};
#pragma unroll
            for (int u = 0; u < kCK; ++u) {
                const float d[4] = {half_bits_to_float(scu[u].x), half_bits_to_float(scu[u].x >> 16),
                                    half_bits_to_float(scu[u].y), half_bits_to_float(scu[u].y >> 16)};
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[t][i] = fmaf(d[i], pr[t][u][i], acc[t][i]);
            }
            // offset corrections of the chunk's blocks: scales (row l16 of the tile, block lg) x -corr
            const uint32_t da = *reinterpret_cast<const uint16_t *>(wsc + (4 * t + (l16 >> 2)) * 32 + lg * 8 + (l16 & 3) * 2);
            const int kb = bk + lg;
            const float cn = kb < nblk ? corr[kb * 16 + l16] : 0.0f;
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(half_bits_to_float(da), cn, acc[t], 0, 0, 0);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (c == NCH - 1) {
            // the pair's outputs: lane holds rows 4 lg .. + 3 of tile t for activation row l16
            const int64_t pr_idx = my_first + (int64_t)q.pair * kWideWaves;
            const int64_t b = b0 + l16;
            const float sc = escale[l16];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                const int64_t rq = pr_idx * 8 + 4 * t + lg;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int64_t row = rq * 4 + i;
                    const uint32_t o = b < batch && row < rows_out ? (uint32_t)((b * ldy + row) * 4) : kPastEnd;
                    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[t][i] * sc), yrs, o, 0, 0);
                }
                acc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
        }
    };

    // a ring of RB register buffers (RB divides NCH, so chunk c of every pair sits in buffer c % RB):
    // chunk n + RB - 1 of the stream is requested while chunk n is multiplied
    constexpr int RB = NCH % 4 == 0 ? 4 : NCH % 3 == 0 ? 3 : 2;
    uint4 wb[RB][G::NLD + 1];
#pragma unroll
    for (int c = 0; c < RB - 1; ++c) fetch(Pos{0, c}, wb[c]);
    for (int pi = 0; pi < my_n; ++pi) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            constexpr int D = RB - 1;
            const int cn = c + D;
            fetch(cn < NCH ? Pos{pi, cn} : Pos{pi + 1, cn - NCH}, wb[cn % RB]);
            step(Pos{pi, c}, wb[c % RB]);
        }
    }
}

inline int64_t rows4(int64_t r) { return (r + 3) / 4 * 4; }

int64_t gemm_scale_off(int dt, int64_t rows, int64_t cols) {
    const int64_t q = rows4(rows) * (cols / QK) * (dt == VGX_Q8_0 ? 32 : 16);
    return (q + 255) / 256 * 256;
}

inline int64_t split_plane_bytes(int64_t batch, int64_t cols) { return (batch * cols * 2 + 255) / 256 * 256; }
// the fp16 hi and lo planes, the per-row scales
inline int64_t split_bytes(int64_t batch, int64_t cols) {
    return 2 * split_plane_bytes(batch, cols) + (batch * 4 + 255) / 256 * 256;
}

constexpr int kMaxKSplit = 16;
// Splits a reduce launch (and qkv_split_rope_kernel) sums: the largest compile-time bound.
constexpr int kReduceMaxSplits = 32;
static_assert(kMaxKSplit <= kReduceMaxSplits, "split bound of qgemm_reduce_kernel and qkv_split_rope_kernel");
constexpr int kTargetWaves = 2048;

// K splits: enough waves to fill the GPU, at least 8 blocks per split.
int choose_ksplit(int64_t n_rq, int64_t batch, int nc, int nblk) {
    const int64_t waves = (n_rq + 7) / 8 * ((batch + 16 * nc - 1) / (16 * nc));
    int64_t ks = (kTargetWaves + waves - 1) / waves;
    ks = std::min<int64_t>(ks, std::min<int64_t>(kMaxKSplit, nblk / 8));
    return (int)std::max<int64_t>(1, ks);
}

// K splits of the tiled kernels, counted on the DMA kernel's tiles: about 512 workgroups, 768 for long
// rows (one round at three workgroups per CU), at least 8 blocks per split.  The 1536 x 8960 down
// projection of a 1024-token chunk (96 tiles): 8 splits 95.6-96.7 us, 16 (a target of 2048) 108.3-108.6,
// 5 99.4-100.1, 4 110.8-111.9, the split partials (fp32, written and read back by the reduce) being
// what the extra splits cost; over 512 tokens (48 tiles) 16 and 10 splits 64.6-66.1 us, 8 68.9.  For
// short rows a target of 768 measured no better (q|k|v and o of a 1024-token chunk 45.4 / 40.7 ->
// 47.7 / 44.0 us).
int tile_ksplit(int64_t n_rq, int64_t batch, int nblk) {
    const int64_t tiles = (n_rq + kTMDma / 4 - 1) / (kTMDma / 4) * ((batch + kTNDma - 1) / kTNDma);
    const int64_t target = nblk >= 128 ? 768 : 512;
    // as many splits as fit the target without exceeding it: 512 workgroups are one round at two per
    // CU, and a few more would run as a mostly idle second round (o-projection of a 1024-token chunk:
    // 96 tiles x 5 splits, 45.9 us, against 6 splits, 52-54 us)
    int64_t ks = target / tiles;
    ks = std::min<int64_t>(ks, std::min<int64_t>(kMaxKSplit, nblk / 8));
    return (int)std::max<int64_t>(1, ks);
}

inline int64_t part_bytes(int ks, int64_t batch, int64_t rows_p) {
    return ks > 1 ? ((int64_t)ks * batch * rows_p * 4 + 255) / 256 * 256 : 0;
}

constexpr int64_t kSmallMaxBatch = 64;

// Activation tiles per workgroup (16 rows each).  Two (32 rows, held to two waves per SIMD by the
// launch bounds) only for very tall weights with more than 16 activation rows: the LM head (151665 x
// 1536 Q8_0) at batch 32 / 64 measured 134 / 232 us against 169 / 303 us with 16-row workgroups, which
// read its 248 MB once per activation tile; for the layer projections 16-row tiles measured ahead
// (batch-32 decode 9.10K against 9.03K tokens/s).
inline int small_nc(int64_t batch, int64_t n_rq) { return batch > 16 && n_rq >= 16384 ? 2 : 1; }

// K splits of the decode-batch path: as choose_ksplit, with whole chunks per split.  When the GPU
// wants more than one split, a split holds at most kSplitMaxBlocks blocks (qgemm_split_kernel stages
// its whole range; more splits for long rows: the 1536 x 8960 down projection takes 18); one split
// (tall weights such as the LM head) keeps qgemm_small_kernel's chunk loop.
inline int small_ksplit(int64_t n_rq, int64_t batch, int nblk, int *kper) {
    const int ks0 = choose_ksplit(n_rq, batch, small_nc(batch, n_rq), nblk);
    int kp = (nblk + ks0 - 1) / ks0;
    kp = (kp + kCK - 1) / kCK * kCK;
    if (ks0 > 1 && kp > kSplitMaxBlocks && (nblk + kSplitMaxBlocks - 1) / kSplitMaxBlocks <= kReduceMaxSplits)
        kp = kSplitMaxBlocks;
    *kper = kp;
    return (nblk + kp - 1) / kp;
}

// Whether qgemm_wide_kernel takes a projection of a decode batch (without bias): one split (tall
// weights), K of 48 or 24 blocks (its compiled chunk counts), the store epilogue, byte offsets within the 31-bit buffer range, and enough row
// tiles for its 256 persistent workgroups to stream.
inline bool use_wide_kernel(int ks, int64_t n_rq, int64_t cols, int epilogue, int64_t w_bytes) {
    return ks == 1 && epilogue == VGX_EPI_STORE && (cols == 1536 || cols == 768) && n_rq >= 4096 &&
           w_bytes < ((int64_t)1 << 31);
}

// Whether qgemm_split_kernel takes a split projection: splits of at most kSplitMaxBlocks blocks and a
// weight (quants + scales) whose byte offsets fit the 31-bit buffer range.
inline bool use_split_kernel(int ks, int kper, int64_t w_bytes) {
    return ks > 1 && kper <= kSplitMaxBlocks && w_bytes < ((int64_t)1 << 30);
}

// qgemm_split_kernel over grid (row tiles, 16-row activation tiles, splits); writes part / pssq.
// The tile epilogue a fused launch applies (kFinNone: partials only, for a reduce launch).
struct SplitFin {
    int epi = kFinNone;
    int64_t rows_out = 0;
    float eps = 0.0f;
    const float *bias = nullptr;
    float *y = nullptr;
    int64_t ldy = 0;
    int *cnt = nullptr;
};

// qgemm_split_kernel / qgemm_kslice_kernel over grid (row tiles, 16-row activation tiles, splits);
// writes part / pssq, and with fin.epi >= 0 also sums the splits of each tile into y.
void split_kernel_launch(int dtype, const uint8_t *w, int64_t soff, int64_t n_rq, int nblk, const float *x,
                         int64_t ldx, const float *norm_w, int64_t batch, float *part, float *pssq, int ks, int kper,
                         const SplitFin &fin, hipStream_t st) {
    const dim3 grid((unsigned)((n_rq + 31) / 32), (unsigned)((batch + 15) / 16), (unsigned)ks);
    const int wb = (int)(soff + n_rq * nblk * 8);
#define VGX_SK(DT, NORM)                                                                                       \
    hipLaunchKernelGGL((qgemm_split_kernel<DT, NORM>), grid, dim3(256), 0, st, w, soff, n_rq, nblk, wb, x, ldx, \
                       norm_w, batch, part, pssq, kper)
#define VGX_KS(NORM, F)                                                                                         \
    hipLaunchKernelGGL((qgemm_kslice_kernel<NORM, F>), grid, dim3(256), 0, st, w, soff, n_rq, nblk, wb, x, ldx,    \
                       norm_w, batch, part, pssq, kper, fin.rows_out, fin.eps, fin.bias, fin.y, fin.ldy, fin.cnt)
#define VGX_KSN(F) do { if (norm_w) VGX_KS(true, F); else VGX_KS(false, F); } while (0)
    // K slices of 4 blocks: 16-block splits keep all four waves busy; shorter splits (the 1536-column
    // projections take 8 blocks) stay on qgemm_split_kernel
    if (dtype == VGX_Q8_0) { if (norm_w) VGX_SK(VGX_Q8_0, true); else VGX_SK(VGX_Q8_0, false); }
    else if (kper != kSplitMaxBlocks) { if (norm_w) VGX_SK(VGX_Q4_0, true); else VGX_SK(VGX_Q4_0, false); }
    else if (fin.epi == EPI_STORE) VGX_KSN(EPI_STORE);
    else if (fin.epi == EPI_ACCUM) VGX_KSN(EPI_ACCUM);
    else if (fin.epi == EPI_SWIGLU) VGX_KSN(EPI_SWIGLU);
    else VGX_KSN(kFinNone);
#undef VGX_KSN
#undef VGX_KS
#undef VGX_SK
}

// Whether a split launch sums its own splits: qgemm_kslice_kernel (the fused finish measured slower than
// the reduce launch behind qgemm_split_kernel's 8-block splits: o-projection at batch 32, 9.6 against 8.5
// us per call; gate/up 17.0 against 19.1 us), a tile counter for every output tile and partial byte
// offsets within the 31-bit buffer range.
inline bool use_fused_finish(int dtype, int kper, int64_t n_rq, int64_t batch, int ks) {
    const int64_t tiles = (n_rq + 31) / 32 * ((batch + 15) / 16);
    return dtype == VGX_Q4_0 && kper == kSplitMaxBlocks && tiles <= kQgemmTickets &&
           (int64_t)ks * batch * n_rq * 16 < ((int64_t)1 << 31);
}

// Workspace of the small-batch path: the tile counters, the K-split partials, then the per-split sum
// x^2 of every row (per row tile when the launch sums its own splits).
// Whether a Q4_0 projection of a decode batch with few output rows (the o and down projections, 1536
// rows) runs qgemm_kslice_kernel on 64-row tiles over 16-block splits, summing its own splits: twice the
// workgroups of the 128-row tiles, and no reduce launch for the o-projection (batch-32 decode: 13.98K
// tok/s with 128-row tiles, 14.14K with the o-projection on 64-row tiles, 14.67K with down too; gate/up
// on them too measured 14.51K).
inline bool use_short_kslice(int dtype, int nblk, int64_t n_rq, int64_t batch) {
    const int ks = (nblk + kSplitMaxBlocks - 1) / kSplitMaxBlocks;
    return dtype == VGX_Q4_0 && ks >= 2 && ks <= 18 && n_rq <= 1024 &&
           (n_rq + 15) / 16 * ((batch + 15) / 16) <= kQgemmTickets && (int64_t)ks * batch * n_rq * 16 < ((int64_t)1 << 31);
}

inline int64_t small_bytes(int64_t batch, int64_t n_rq, int nblk, int dtype = VGX_Q4_0) {
    if (use_short_kslice(dtype, nblk, n_rq, batch)) {
        const int ks = (nblk + kSplitMaxBlocks - 1) / kSplitMaxBlocks;
        return kQgemmTicketBytes + part_bytes(ks, batch, n_rq * 4) +
               ((int64_t)ks * ((n_rq + 15) / 16) * batch * 4 + 255) / 256 * 256;
    }
    int kper = 0;
    const int ks = small_ksplit(n_rq, batch, nblk, &kper);
    if (ks <= 1) return 0;
    return kQgemmTicketBytes + part_bytes(ks, batch, n_rq * 4) +
           ((int64_t)ks * ((n_rq + 31) / 32) * batch * 4 + 255) / 256 * 256;
}

// K-split partials of one projection of a decode batch: part [ks][batch][rows_p] and, with the
// RMSNorm, the per-split sum x^2 of every activation row pssq [ks][batch]; roff is the first row of
// the part this launch reads (q rows then k and v rows when one weight holds all three).
struct SplitSrc {
    const float *part;
    const float *pssq;
    const float *bias;
    int ks;
    int64_t rows_p;
    int64_t roff;
};

// Sum over the splits (k = 0, 1, ... in order), then the RMSNorm scale and the bias, as
// qgemm_reduce_kernel does.  KM >= ks is a compile-time bound: the loads of all splits go out at
// once (indexes clamped to the last split, so none is out of range) instead of one round trip per
// split of a loop with a run-time count.
template <int KM>
__device__ __forceinline__ float split_value(const SplitSrc &s, int64_t batch, int64_t t, int64_t r, float inv) {
    float p[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) p[k] = s.part[((int64_t)min(k, s.ks - 1) * batch + t) * s.rows_p + s.roff + r];
    float v = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < s.ks) v += p[k];
    v *= inv;
    if (s.bias) v += s.bias[s.roff + r];
    return v;
}

template <int KM>
__device__ __forceinline__ float split_inv(const SplitSrc &s, int64_t batch, int64_t t, int cols, float eps) {
    if (!s.pssq) return 1.0f;
    float p[KM];
#pragma unroll
    for (int k = 0; k < KM; ++k) p[k] = s.pssq[(int64_t)min(k, s.ks - 1) * batch + t];
    float u = 0.0f;
#pragma unroll
    for (int k = 0; k < KM; ++k)
        if (k < s.ks) u += p[k];
    return 1.0f / sqrtf(u / (float)cols + eps);
}

// q / k / v of a decode batch from the K-split partials of their projections, with RoPE and the
// ring / sink writes, in one launch.  grid (batch, H + G), threads over the D / 2 RoPE pairs.  The
// ring slot, RoPE table row and sink slot come from the device step descriptor.
template <int KV, int KM>
__global__ __launch_bounds__(256) void qkv_split_rope_kernel(SplitSrc sq, SplitSrc skv, int64_t batch, int cols,
                                                             float eps, int H, int G, int D,
                                                             const float *__restrict__ table, int64_t trs,
                                                             const int32_t *__restrict__ step, float *q_out,
                                                             int64_t ldq, void *k_rot, void *k_raw, void *v_dst,
                                                             int64_t dbs, int64_t dgs, int64_t drs, void *sk, void *sv,
                                                             int64_t sbs, int64_t sgs, int64_t srs) {
    const int64_t t = blockIdx.x;
    const int hd = blockIdx.y;
    const int h2 = D / 2;
    const int64_t slot = step[VGX_STEP_SLOT];
    const int64_t sink = step[VGX_STEP_SINK_SLOT];
    const float *cs = table + (int64_t)step[VGX_STEP_TABLE_ROW] * trs;
    if (hd < H) {
        const float inv = split_inv<KM>(sq, batch, t, cols, eps);
        float *qp = q_out + t * ldq + (int64_t)hd * D;
        for (int i = threadIdx.x; i < h2; i += blockDim.x) {
            const float c = cs[i], s = cs[h2 + i];
            const float a = split_value<KM>(sq, batch, t, (int64_t)hd * D + i, inv);
            const float b = split_value<KM>(sq, batch, t, (int64_t)hd * D + i + h2, inv);
            qp[i] = a * c - b * s;
            qp[i + h2] = b * c + a * s;
        }
        return;
    }
    const int g = hd - H;
    const float inv = split_inv<KM>(skv, batch, t, cols, eps);
    const int64_t kr = (int64_t)g * D, vr = (int64_t)(G + g) * D;
    const int64_t o = t * dbs + g * dgs + slot * drs;
    const int64_t so = t * sbs + g * sgs + sink * srs;
    for (int i = threadIdx.x; i < h2; i += blockDim.x) {
        const float c = cs[i], s = cs[h2 + i];
        const float a = split_value<KM>(skv, batch, t, kr + i, inv);
        const float b = split_value<KM>(skv, batch, t, kr + i + h2, inv);
        const float va = split_value<KM>(skv, batch, t, vr + i, inv);
        const float vb = split_value<KM>(skv, batch, t, vr + i + h2, inv);
        if (k_rot) {
            store_kv<KV>(k_rot, o + i, a * c - b * s);
            store_kv<KV>(k_rot, o + i + h2, b * c + a * s);
        }
        if (k_raw) {
            store_kv<KV>(k_raw, o + i, a);
            store_kv<KV>(k_raw, o + i + h2, b);
        }
        store_kv<KV>(v_dst, o + i, va);
        store_kv<KV>(v_dst, o + i + h2, vb);
        if (sink >= 0 && sk) {
            store_kv<KV>(sk, so + i, a);
            store_kv<KV>(sk, so + i + h2, b);
            store_kv<KV>(sv, so + i, va);
            store_kv<KV>(sv, so + i + h2, vb);
        }
    }
}

// Whether the q and k|v projections of a decode batch run as one qkv_split_kernel launch: both on
// qgemm_split_kernel's tiles (K splits of the same length, not qgemm_kslice_kernel's 16-block ones).
inline bool group_qkv(int q_dt, int64_t q_rows, int kv_dt, int64_t kv_rows, int64_t d_model, int64_t batch) {
    const int nblk = (int)(d_model / QK);
    int kq = 0, kk = 0;
    const int64_t nq = rows4(q_rows) / 4, nk = rows4(kv_rows) / 4;
    const int ksq = small_ksplit(nq, batch, nblk, &kq), ksk = small_ksplit(nk, batch, nblk, &kk);
    const auto fits = [&](int dt, int64_t n_rq, int ks, int kp) {
        return use_split_kernel(ks, kp, gemm_scale_off(dt, n_rq * 4, d_model) + n_rq * nblk * 8) &&
               !(dt == VGX_Q4_0 && kp == kSplitMaxBlocks);
    };
    return kq == kk && fits(q_dt, nq, ksq, kq) && fits(kv_dt, nk, ksk, kk);
}

// Workspace of one split projection (partials, then the per-split sum x^2), 256-byte multiples.
inline int64_t split_proj_bytes(int64_t batch, int64_t rows, int nblk) {
    const int64_t n_rq = rows4(rows) / 4;
    int kper = 0;
    const int ks = small_ksplit(n_rq, batch, nblk, &kper);
    return ((int64_t)ks * batch * n_rq * 16 + 255) / 256 * 256 + ((int64_t)ks * batch * 4 + 255) / 256 * 256;
}

// The small-batch kernel writing K-split partials (one split or more) into part / pssq; returns ks.
int split_proj_launch(int dtype, const void *wp, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                      int64_t batch, const float *norm_w, float eps, float *part, float *pssq, hipStream_t st) {
    const int nblk = (int)(cols / QK);
    const int64_t n_rq = rows4(rows) / 4;
    int kper = 0;
    const int ks = small_ksplit(n_rq, batch, nblk, &kper);
    const int64_t soff = gemm_scale_off(dtype, rows, cols);
    const auto *w = static_cast<const uint8_t *>(wp);
    if (use_split_kernel(ks, kper, soff + n_rq * nblk * 8)) {
        split_kernel_launch(dtype, w, soff, n_rq, nblk, x, ldx, norm_w, batch, part, pssq, ks, kper, SplitFin{}, st);
        return ks;
    }
    const int nc = small_nc(batch, n_rq);
    const dim3 grid((unsigned)((n_rq + 31) / 32), (unsigned)((batch + 16 * nc - 1) / (16 * nc)), (unsigned)ks);
#define VGX_SP(DT, NC, NORM)                                                                                      \
    hipLaunchKernelGGL((qgemm_small_kernel<DT, NC, EPI_STORE, true, NORM>), grid, dim3(256), 0, st, w, soff, n_rq, \
                       nblk, rows, x, ldx, norm_w, eps, batch, nullptr, nullptr, (int64_t)0, part, pssq, kper)
#define VGX_SP_N(DT, NC) do { if (norm_w) VGX_SP(DT, NC, true); else VGX_SP(DT, NC, false); } while (0)
    if (dtype == VGX_Q8_0) { if (nc == 1) VGX_SP_N(VGX_Q8_0, 1); else VGX_SP_N(VGX_Q8_0, 2); }
    else { if (nc == 1) VGX_SP_N(VGX_Q4_0, 1); else VGX_SP_N(VGX_Q4_0, 2); }
#undef VGX_SP_N
#undef VGX_SP
    return ks;
}

}  // namespace

extern "C" {

int64_t vgx_qgemm_workspace_bytes(int64_t batch, int64_t rows, int64_t cols, int epilogue) {
    if (batch <= 0 || rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    const int64_t rows_p = rows4(epilogue == VGX_EPI_SWIGLU ? 2 * rows : rows);
    const int ks = tile_ksplit(rows_p / 4, batch, (int)(cols / QK));
    const int64_t big = kQgemmTicketBytes + split_bytes(batch, cols) + part_bytes(ks, batch, rows_p);
    // the weight dtype is not an argument: the larger of the Q4_0 and Q8_0 layouts
    const int64_t sq4 = small_bytes(batch, rows_p / 4, (int)(cols / QK), VGX_Q4_0);
    const int64_t sq8 = small_bytes(batch, rows_p / 4, (int)(cols / QK), VGX_Q8_0);
    return batch <= kSmallMaxBatch ? std::max(big, std::max(sq4, sq8)) : big;
}

int vgx_qgemm(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx, int64_t batch,
              const float *norm_w, float eps, const float *bias, float *y, int64_t ldy, int epilogue, void *workspace,
              int64_t workspace_bytes, void *stream) {
    if (dtype != VGX_Q8_0 && dtype != VGX_Q4_0 && dtype != VGX_F32 && dtype != VGX_BF16 && dtype != VGX_F16)
        return VGX_E_DTYPE;
    if (!w_packed || !x || !y) return VGX_E_ARG;
    if (epilogue != VGX_EPI_STORE && epilogue != VGX_EPI_ACCUM && epilogue != VGX_EPI_SWIGLU) return VGX_E_ARG;
    if (epilogue == VGX_EPI_SWIGLU && bias) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || batch < 0 || ldx < cols || ldy < rows) return VGX_E_SIZE;
    if (cols % QK || (epilogue == VGX_EPI_SWIGLU && rows % 2)) return VGX_E_SHAPE;
    if (norm_w && !(eps > 0.0f)) return VGX_E_ARG;
    if (batch == 0) return VGX_OK;
    if (batch > 65535 * 32 || cols / QK > (1 << 24)) return VGX_E_LIMIT;
    const int64_t rows_packed = epilogue == VGX_EPI_SWIGLU ? 2 * rows : rows;
    const int nblk = (int)(cols / QK);
    const int64_t n_rq = rows4(rows_packed) / 4;
    if (dtype == VGX_F32 || dtype == VGX_BF16 || dtype == VGX_F16) {
        if (norm_w) return VGX_E_ARG;                 // plain weights: no fused RMSNorm on this path
        const void *wf = w_packed;
        const dim3 grid((unsigned)((n_rq + kFT / 4 - 1) / (kFT / 4)), (unsigned)((batch + kFT - 1) / kFT));
        const bool vec = ((uintptr_t)x & 15) == 0 && ldx % 4 == 0;
        hipStream_t sf = (hipStream_t)stream;
#define VGX_F32G(WDT, EPI, V) hipLaunchKernelGGL((f32gemm_tile_kernel<WDT, EPI, V>), grid, dim3(256), 0, sf, wf, n_rq, nblk, rows, x, ldx, batch, bias, y, ldy)
#define VGX_F32E(WDT, V)                                                    \
    do {                                                                    \
        if (epilogue == VGX_EPI_SWIGLU) VGX_F32G(WDT, EPI_SWIGLU, V);        \
        else if (epilogue == VGX_EPI_ACCUM) VGX_F32G(WDT, EPI_ACCUM, V);     \
        else VGX_F32G(WDT, EPI_STORE, V);                                   \
    } while (0)
#define VGX_F32W(WDT) do { if (vec) VGX_F32E(WDT, true); else VGX_F32E(WDT, false); } while (0)
        if (dtype == VGX_BF16) VGX_F32W(VGX_BF16);
        else if (dtype == VGX_F16) VGX_F32W(VGX_F16);
        else VGX_F32W(VGX_F32);
#undef VGX_F32W
#undef VGX_F32E
#undef VGX_F32G
        VGX_CHECK_LAUNCH();
        return VGX_OK;
    }
    const int64_t soff0 = gemm_scale_off(dtype, rows_packed, cols);
    hipStream_t st0 = (hipStream_t)stream;
    if (batch <= kSmallMaxBatch && ((uintptr_t)x & 15) == 0 && ldx % 4 == 0 && ((uintptr_t)norm_w & 15) == 0) {
        int kper = 0;
        const int ks = small_ksplit(n_rq, batch, nblk, &kper);
        const int64_t need = small_bytes(batch, n_rq, nblk, dtype);
        if (need > 0 && (!workspace || workspace_bytes < need)) return VGX_E_ARENA;
        if (need > 0 && (uintptr_t)workspace % 256) return VGX_E_ALIGN;
        auto *tickets = static_cast<int *>(workspace);
        auto *part = need > 0 ? reinterpret_cast<float *>(static_cast<char *>(workspace) + kQgemmTicketBytes) : nullptr;
        auto *pssq = need > 0 ? reinterpret_cast<float *>(static_cast<char *>(workspace) + kQgemmTicketBytes +
                                                          part_bytes(ks, batch, n_rq * 4))
                              : nullptr;
        const int nc = small_nc(batch, n_rq);
        const dim3 grid((unsigned)((n_rq + 31) / 32), (unsigned)((batch + 16 * nc - 1) / (16 * nc)), (unsigned)ks);
        const auto *w = static_cast<const uint8_t *>(w_packed);
        if (!bias && use_wide_kernel(ks, n_rq, cols, epilogue, soff0 + n_rq * nblk * 8)) {
            const int nbt = (int)((batch + 15) / 16);
            const int n_groups = 256 / nbt / 8 * 8;
            const int wb = (int)(soff0 + n_rq * nblk * 8);
#define VGX_WD(DT, NORM, NCH)                                                                                     \
    hipLaunchKernelGGL((qgemm_wide_kernel<DT, NORM, NCH>), dim3((unsigned)(n_groups * nbt)), dim3(64 * kWideWaves), 0, st0, \
                       w, soff0, n_rq, nblk, wb, x, ldx, norm_w, eps, batch, y, ldy, rows, n_groups)
#define VGX_WDN(NCH)                                                                                            \
    do {                                                                                                        \
        if (dtype == VGX_Q8_0) { if (norm_w) VGX_WD(VGX_Q8_0, true, NCH); else VGX_WD(VGX_Q8_0, false, NCH); }     \
        else { if (norm_w) VGX_WD(VGX_Q4_0, true, NCH); else VGX_WD(VGX_Q4_0, false, NCH); }                      \
    } while (0)
            if (nblk == 48) VGX_WDN(12); else VGX_WDN(6);
#undef VGX_WDN
#undef VGX_WD
            VGX_CHECK_LAUNCH();
            return VGX_OK;
        }
        if (!bias && use_short_kslice(dtype, nblk, n_rq, batch) && soff0 + n_rq * nblk * 8 < ((int64_t)1 << 30)) {
            // 64-row tiles, 16-block splits summed by the launch (partials, then per-tile sum x^2)
            const int ks16 = (nblk + kSplitMaxBlocks - 1) / kSplitMaxBlocks;
            auto *pssq16 = reinterpret_cast<float *>(static_cast<char *>(workspace) + kQgemmTicketBytes +
                                                     part_bytes(ks16, batch, n_rq * 4));
            const dim3 g16((unsigned)((n_rq + 15) / 16), (unsigned)((batch + 15) / 16), (unsigned)ks16);
            const int wb = (int)(soff0 + n_rq * nblk * 8);
#define VGX_KS16(NORM, F)                                                                                       \
    hipLaunchKernelGGL((qgemm_kslice_kernel<NORM, F, 16>), g16, dim3(256), 0, st0, w, soff0, n_rq, nblk, wb, x, ldx, \
                       norm_w, batch, part, pssq16, kSplitMaxBlocks, rows, eps, bias, y, ldy, tickets)
#define VGX_KS16N(F) do { if (norm_w) VGX_KS16(true, F); else VGX_KS16(false, F); } while (0)
            if (epilogue == VGX_EPI_SWIGLU) VGX_KS16N(EPI_SWIGLU);
            else if (epilogue == VGX_EPI_ACCUM) VGX_KS16N(EPI_ACCUM);
            else VGX_KS16N(EPI_STORE);
#undef VGX_KS16N
#undef VGX_KS16
            VGX_CHECK_LAUNCH();
            return VGX_OK;
        }
        const bool sk = use_split_kernel(ks, kper, soff0 + n_rq * nblk * 8);
        if (sk && use_fused_finish(dtype, kper, n_rq, batch, ks)) {
            // the split launch sums its own splits: no reduce launch
            SplitFin fin;
            fin.epi = epilogue == VGX_EPI_SWIGLU ? EPI_SWIGLU : epilogue == VGX_EPI_ACCUM ? EPI_ACCUM : EPI_STORE;
            fin.rows_out = rows;
            fin.eps = eps;
            fin.bias = bias;
            fin.y = y;
            fin.ldy = ldy;
            fin.cnt = tickets;
            split_kernel_launch(dtype, w, soff0, n_rq, nblk, x, ldx, norm_w, batch, part, pssq, ks, kper, fin, st0);
            VGX_CHECK_LAUNCH();
            return VGX_OK;
        }
        if (sk) split_kernel_launch(dtype, w, soff0, n_rq, nblk, x, ldx, norm_w, batch, part, pssq, ks, kper, SplitFin{}, st0);
#define VGX_SG(DT, NC, EPI, SP, NORM)                                                                         \
    hipLaunchKernelGGL((qgemm_small_kernel<DT, NC, EPI, SP, NORM>), grid, dim3(256), 0, st0, w, soff0, n_rq, nblk, \
                       rows, x, ldx, norm_w, eps, batch, bias, y, ldy, part, pssq, kper)
#define VGX_SG_N(DT, NC, EPI, SP) do { if (norm_w) VGX_SG(DT, NC, EPI, SP, true); else VGX_SG(DT, NC, EPI, SP, false); } while (0)
#define VGX_SG_E(DT, NC)                                                                                      \
    do {                                                                                                      \
        if (ks > 1) VGX_SG_N(DT, NC, EPI_STORE, true);                                                        \
        else if (epilogue == VGX_EPI_SWIGLU) VGX_SG_N(DT, NC, EPI_SWIGLU, false);                             \
        else if (epilogue == VGX_EPI_ACCUM) VGX_SG_N(DT, NC, EPI_ACCUM, false);                               \
        else VGX_SG_N(DT, NC, EPI_STORE, false);                                                              \
    } while (0)
        if (sk) {
        } else if (dtype == VGX_Q8_0) {
            if (nc == 1) VGX_SG_E(VGX_Q8_0, 1); else VGX_SG_E(VGX_Q8_0, 2);
        } else {
            if (nc == 1) VGX_SG_E(VGX_Q4_0, 1); else VGX_SG_E(VGX_Q4_0, 2);
        }
#undef VGX_SG_E
#undef VGX_SG_N
#undef VGX_SG
        VGX_CHECK_LAUNCH();
        if (ks > 1) {
            const float *ps = norm_w ? pssq : nullptr;
            if (epilogue == VGX_EPI_SWIGLU)
                reduce_launch<EPI_SWIGLU>(part, ks, batch, n_rq * 4, rows, bias, y, ldy, ps, (int)cols, eps, st0);
            else if (epilogue == VGX_EPI_ACCUM)
                reduce_launch<EPI_ACCUM>(part, ks, batch, n_rq * 4, rows, bias, y, ldy, ps, (int)cols, eps, st0);
            else
                reduce_launch<EPI_STORE>(part, ks, batch, n_rq * 4, rows, bias, y, ldy, ps, (int)cols, eps, st0);
            VGX_CHECK_LAUNCH();
        }
        return VGX_OK;
    }
    const int ks = tile_ksplit(n_rq, batch, nblk);
    if (!workspace || workspace_bytes < kQgemmTicketBytes + split_bytes(batch, cols) + part_bytes(ks, batch, n_rq * 4))
        return VGX_E_ARENA;
    if ((uintptr_t)workspace % 256) return VGX_E_ALIGN;
    const int64_t soff = gemm_scale_off(dtype, rows_packed, cols);
    const int64_t pb = split_plane_bytes(batch, cols);
    char *const wsb = static_cast<char *>(workspace) + kQgemmTicketBytes;   // past the tile counters
    auto *xh = reinterpret_cast<uint16_t *>(wsb);
    auto *xl = reinterpret_cast<uint16_t *>(wsb + pb);
    auto *xsc = reinterpret_cast<float *>(wsb + 2 * pb);
    hipStream_t st = (hipStream_t)stream;
    hipLaunchKernelGGL(xsplit_kernel, dim3((unsigned)batch), dim3(256), 0, st, x, ldx, norm_w, eps, (int)cols, xh, xl,
                       xsc);
    VGX_CHECK_LAUNCH();
    auto *part = reinterpret_cast<float *>(wsb + split_bytes(batch, cols));
    const int kper = (nblk + ks - 1) / ks;
    constexpr int DTM = kTMDma, DTN = kTNDma;
    const dim3 grid((unsigned)((n_rq + kTM / 4 - 1) / (kTM / 4)), (unsigned)((batch + kTN - 1) / kTN), (unsigned)ks);
    const dim3 dgrid((unsigned)((n_rq + DTM / 4 - 1) / (DTM / 4)), (unsigned)((batch + DTN - 1) / DTN), (unsigned)ks);
    const auto *w = static_cast<const uint8_t *>(w_packed);
    // the DMA kernel wherever its 32-bit buffer ranges reach: it measured ahead of the register-staged
    // kernel at every grid size (Q4_0, 80 / 160 / 256 / 512 tokens: q|k|v 36.6 -> 36.1 / 37.5 -> 26.9
    // / 39.9 -> 30.0 / 47.7 -> 37.0 us, gate/up 59.7 -> 42.4 / 79.0 -> 60.1 / 83.4 -> 75.1 / 101.6 ->
    // 101.1, down 61.5 -> 40.1 / 73.0 -> 49.4 / 78.9 -> 51.4 / 69.1 -> 68.9)
    const bool dma = soff + n_rq * nblk * 8 < ((int64_t)1 << 31) && batch * cols * 2 < ((int64_t)1 << 31);
#define VGX_GEMM_GO(DT, EPI, SP)                                                                              \
    do {                                                                                                      \
        if (dma)                                                                                              \
            hipLaunchKernelGGL((qgemm_tile_dma_kernel<DT, EPI, SP, DTM, DTN>), dgrid, dim3(256), 0, st, w, soff, n_rq, nblk, rows, \
                               xh, xl, xsc, batch, bias, y, ldy, part, kper);                                  \
        else                                                                                                  \
            hipLaunchKernelGGL((qgemm_tile_kernel<DT, EPI, SP>), grid, dim3(256), 0, st, w, soff, n_rq, nblk, rows, xh, \
                               xl, xsc, batch, bias, y, ldy, part, kper);                                     \
    } while (0)
#define VGX_GEMM_EPI(DT)                                                                                      \
    do {                                                                                                      \
        if (ks > 1) VGX_GEMM_GO(DT, EPI_STORE, true);                                                         \
        else if (epilogue == VGX_EPI_SWIGLU) VGX_GEMM_GO(DT, EPI_SWIGLU, false);                              \
        else if (epilogue == VGX_EPI_ACCUM) VGX_GEMM_GO(DT, EPI_ACCUM, false);                                \
        else VGX_GEMM_GO(DT, EPI_STORE, false);                                                               \
    } while (0)
    if (dtype == VGX_Q8_0) VGX_GEMM_EPI(VGX_Q8_0);
    else VGX_GEMM_EPI(VGX_Q4_0);
#undef VGX_GEMM_EPI
#undef VGX_GEMM_GO
    VGX_CHECK_LAUNCH();
    if (ks > 1) {
        if (epilogue == VGX_EPI_SWIGLU)
            reduce_launch<EPI_SWIGLU>(part, ks, batch, n_rq * 4, rows, bias, y, ldy, nullptr, (int)cols, 0.0f, st);
        else if (epilogue == VGX_EPI_ACCUM)
            reduce_launch<EPI_ACCUM>(part, ks, batch, n_rq * 4, rows, bias, y, ldy, nullptr, (int)cols, 0.0f, st);
        else
            reduce_launch<EPI_STORE>(part, ks, batch, n_rq * 4, rows, bias, y, ldy, nullptr, (int)cols, 0.0f, st);
        VGX_CHECK_LAUNCH();
    }
    return VGX_OK;
}

int64_t vgx_qkv_rope_batch_workspace_bytes(int64_t B, int64_t d_model, int64_t H, int64_t G, int64_t D,
                                           int separate_q) {
    if (B <= 0 || d_model <= 0 || H <= 0 || G <= 0 || D <= 0) return VGX_E_SIZE;
    if (d_model % QK) return VGX_E_SHAPE;
    const int nblk = (int)(d_model / QK);
    if (separate_q) return kQgemmTicketBytes + split_proj_bytes(B, H * D, nblk) + split_proj_bytes(B, 2 * G * D, nblk);
    return kQgemmTicketBytes + split_proj_bytes(B, (H + 2 * G) * D, nblk);
}

int vgx_qkv_rope_batch(int q_wdtype, const void *wq, const float *bq, int kv_wdtype, const void *wkv,
                       const float *bkv, int64_t d_model, int64_t H, int64_t G, int64_t D, const float *x, int64_t ldx,
                       int64_t B, const float *norm_w, float eps, const float *table, int64_t table_rstride,
                       const int32_t *step, float *q_out, int64_t ldq, int kv_dtype, void *k_rot, void *k_raw,
                       void *v_dst, int64_t dst_bstride, int64_t dst_gstride, int64_t dst_rstride, void *sink_k_raw,
                       void *sink_v, int64_t sink_bstride, int64_t sink_gstride, int64_t sink_rstride,
                       void *workspace, int64_t workspace_bytes, void *stream) {
    const bool sep = wq != nullptr;
    if (kv_wdtype != VGX_Q8_0 && kv_wdtype != VGX_Q4_0) return VGX_E_DTYPE;
    if (sep && q_wdtype != VGX_Q8_0 && q_wdtype != VGX_Q4_0) return VGX_E_DTYPE;
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!wkv || !x || !table || !step || !q_out || !v_dst || !workspace) return VGX_E_ARG;
    if (!sep && bq) return VGX_E_ARG;                  // one weight for q|k|v: its bias is bkv
    if ((sink_k_raw == nullptr) != (sink_v == nullptr)) return VGX_E_ARG;
    if (norm_w && !(eps > 0.0f)) return VGX_E_ARG;
    if (B <= 0 || H <= 0 || G <= 0 || D <= 0 || (D & 1) || d_model <= 0 || ldx < d_model || ldq < H * D)
        return VGX_E_SIZE;
    if (d_model % QK) return VGX_E_SHAPE;
    if (B > kSmallMaxBatch || H + G > 65535 || D / 2 > 4096) return VGX_E_LIMIT;
    if (((uintptr_t)x & 15) || ldx % 4 || ((uintptr_t)norm_w & 15)) return VGX_E_ALIGN;
    if ((uintptr_t)workspace % 256) return VGX_E_ALIGN;
    if (workspace_bytes < vgx_qkv_rope_batch_workspace_bytes(B, d_model, H, G, D, sep ? 1 : 0)) return VGX_E_ARENA;
    hipStream_t st = (hipStream_t)stream;
    const int nblk = (int)(d_model / QK);
    auto *base = static_cast<char *>(workspace) + kQgemmTicketBytes;   // the GEMM tile counters stay untouched
    auto carve = [&](int64_t rows, float *&part, float *&pssq) {
        const int64_t n_rq = rows4(rows) / 4;
        int kper = 0;
        const int ks = small_ksplit(n_rq, B, nblk, &kper);
        part = reinterpret_cast<float *>(base);
        base += ((int64_t)ks * B * n_rq * 16 + 255) / 256 * 256;
        pssq = reinterpret_cast<float *>(base);
        base += ((int64_t)ks * B * 4 + 255) / 256 * 256;
    };
    SplitSrc sq{}, skv{};
    float *part = nullptr, *pssq = nullptr;
    if (sep && group_qkv(q_wdtype, H * D, kv_wdtype, 2 * G * D, d_model, B)) {
        // q and k|v in one launch of qkv_split_kernel
        const int64_t n_rq_q = rows4(H * D) / 4, n_rq_k = rows4(2 * G * D) / 4;
        int kper = 0, kper_k = 0;
        SplitJob jq{}, jk{};
        jq.ks = small_ksplit(n_rq_q, B, nblk, &kper);
        jk.ks = small_ksplit(n_rq_k, B, nblk, &kper_k);
        jq.w = static_cast<const uint8_t *>(wq);
        jq.soff = gemm_scale_off(q_wdtype, H * D, d_model);
        jq.n_rq = n_rq_q;
        jq.w_bytes = (int)(jq.soff + n_rq_q * nblk * 8);
        jq.gx = (int)((n_rq_q + 31) / 32);
        carve(H * D, jq.part, jq.pssq);
        jk.w = static_cast<const uint8_t *>(wkv);
        jk.soff = gemm_scale_off(kv_wdtype, 2 * G * D, d_model);
        jk.n_rq = n_rq_k;
        jk.w_bytes = (int)(jk.soff + n_rq_k * nblk * 8);
        jk.gx = (int)((n_rq_k + 31) / 32);
        carve(2 * G * D, jk.part, jk.pssq);
        const dim3 g3((unsigned)(jq.gx + jk.gx), (unsigned)((B + 15) / 16), (unsigned)std::max(jq.ks, jk.ks));
#define VGX_QKS(QDT, KDT)                                                                                         \
    do {                                                                                                          \
        if (norm_w) hipLaunchKernelGGL((qkv_split_kernel<QDT, KDT, true>), g3, dim3(256), 0, st, jq, jk, nblk, x, ldx, \
                                       norm_w, B, kper);                                                         \
        else hipLaunchKernelGGL((qkv_split_kernel<QDT, KDT, false>), g3, dim3(256), 0, st, jq, jk, nblk, x, ldx,    \
                                norm_w, B, kper);                                                                \
    } while (0)
        if (q_wdtype == VGX_Q4_0) { if (kv_wdtype == VGX_Q4_0) VGX_QKS(VGX_Q4_0, VGX_Q4_0); else VGX_QKS(VGX_Q4_0, VGX_Q8_0); }
        else { if (kv_wdtype == VGX_Q4_0) VGX_QKS(VGX_Q8_0, VGX_Q4_0); else VGX_QKS(VGX_Q8_0, VGX_Q8_0); }
#undef VGX_QKS
        sq.ks = jq.ks; sq.part = jq.part; sq.pssq = norm_w ? jq.pssq : nullptr; sq.bias = bq; sq.rows_p = rows4(H * D);
        sq.roff = 0;
        skv.ks = jk.ks; skv.part = jk.part; skv.pssq = norm_w ? jk.pssq : nullptr; skv.bias = bkv;
        skv.rows_p = rows4(2 * G * D); skv.roff = 0;
    } else if (sep) {
        carve(H * D, part, pssq);
        sq.ks = split_proj_launch(q_wdtype, wq, H * D, d_model, x, ldx, B, norm_w, eps, part, pssq, st);
        sq.part = part; sq.pssq = norm_w ? pssq : nullptr; sq.bias = bq; sq.rows_p = rows4(H * D); sq.roff = 0;
        VGX_CHECK_LAUNCH();
        carve(2 * G * D, part, pssq);
        skv.ks = split_proj_launch(kv_wdtype, wkv, 2 * G * D, d_model, x, ldx, B, norm_w, eps, part, pssq, st);
        skv.part = part; skv.pssq = norm_w ? pssq : nullptr; skv.bias = bkv; skv.rows_p = rows4(2 * G * D);
        skv.roff = 0;
    } else {
        const int64_t rows = (H + 2 * G) * D;
        carve(rows, part, pssq);
        skv.ks = split_proj_launch(kv_wdtype, wkv, rows, d_model, x, ldx, B, norm_w, eps, part, pssq, st);
        skv.part = part; skv.pssq = norm_w ? pssq : nullptr; skv.bias = bkv; skv.rows_p = rows4(rows);
        sq = skv;
        skv.roff = H * D;
    }
    VGX_CHECK_LAUNCH();
    const dim3 grid((unsigned)B, (unsigned)(H + G));
    const int thr = (int)std::min<int64_t>(256, std::max<int64_t>(64, D / 2));
    const int km = std::max(sq.ks, skv.ks);
#define VGX_QSR(KV, KM)                                                                                         \
    hipLaunchKernelGGL((qkv_split_rope_kernel<KV, KM>), grid, dim3(thr), 0, st, sq, skv, B, (int)d_model, eps,   \
                       (int)H, (int)G, (int)D, table, table_rstride, step, q_out, ldq, k_rot, k_raw, v_dst,       \
                       dst_bstride, dst_gstride, dst_rstride, sink_k_raw, sink_v, sink_bstride, sink_gstride,     \
                       sink_rstride)
#define VGX_QSR_K(KV) do { if (km <= 4) VGX_QSR(KV, 4); else if (km <= 8) VGX_QSR(KV, 8); else if (km <= 16) VGX_QSR(KV, 16); else VGX_QSR(KV, 32); } while (0)
    if (kv_dtype == VGX_F32) VGX_QSR_K(VGX_F32); else VGX_QSR_K(VGX_BF16);
#undef VGX_QSR_K
#undef VGX_QSR
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // extern "C"
