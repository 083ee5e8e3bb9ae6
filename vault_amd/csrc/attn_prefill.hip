// Prefill attention on bf16 MFMA: blocks of queries over up to four key runs (sinks | segment
// memory | previous chunk | current chunk), the last run causal.
//
// Reference semantics: block_sliding_attention (src/vault_v3_model.py:812-863, sinks re-rotated per
// query chunk :805-809, 849-856) and the chunk-recurrent attention of _forward_chunk_recurrent
// (:2029-2037, 2064-2093).  A query block is one chunk; query t of the block sees every key of the
// first runs and keys j <= causal_base + t of the last run.  A block may carry a bias per (query,
// head row, key) on one run: the chunk-level resonance bias on the segment-memory run
// (_build_chunk_resonance_bias, :1718-1793, added to the scores at :2083-2090), whose rows are the
// per-position biases of the step rule, so a chunk with resonance active stays on this kernel.
//
// Mapping.  A workgroup = one (query block, kv group g, tile of 16 NQT QW queries) with QW waves per
// query head of the group (GRP QW waves), so every K/V tile staged in LDS serves all GRP heads and QW
// query tiles.  A wave holds its 16 NQT queries as NQT 16-query MFMA tiles and computes, per 32 keys,
// with v_mfma_f32_16x16x32_bf16:
//   S^T (keys x queries) = K Q^T       A = K rows from LDS, B = Q^T fragments kept in registers;
//                                      fp32 queries enter as a bf16 hi + lo pair (two MFMAs), so
//                                      the scores keep fp32-level accuracy;
//   O^T (dims x queries) += V^T P^T    A = V^T from LDS, B = P^T straight from the S^T accumulators
//                                      as a bf16 hi + lo pair (two MFMAs): 8-bit probabilities alone
//                                      exceed the bf16 attention bound when few keys carry the weight.
// Staging.  bf16 K / V at 4 or more heads per group are copied into LDS by LDS DMA (buffer loads that
// write LDS, no registers or VALU involved), double-buffered in 128-key tiles: the next tile's loads
// leave right after the barrier that publishes the current one.  Both tiles keep the rows as they are
// in memory (256 bytes per key), each 16-byte piece p of row r stored at slot p ^ (r & 15), so the
// 16-byte K reads of 16 rows and the transposed V reads stay free of bank conflicts; the V^T operand
// comes from ds_read_b64_tr_b16, which hands lane i of a 16-lane group element i % 4 of the 8-byte
// pieces that lanes i / 4 + 4 k address (k = 0..3): lane lq addresses key 4 lg + lq / 4, dims
// 16 dt + 4 (lq % 4) .. + 3, and receives dim 16 dt + lq of keys 4 lg .. 4 lg + 3.  Otherwise (fp32
// K / V, one or two heads per group) each tile is loaded into registers during the previous tile's
// math and stored into LDS, K as is (padded rows), V transposed.
// bf16 K and V stay bf16 end to end (no conversions in the staging loop): MFMA throughput is abundant
// here, VALU issue is what bounds the kernel.  fp32 K and V (an fp32 state read in place) are staged
// as three bf16 planes (hi, mid, lo: 24 significant bits, the whole fp32 mantissa), and the fp32
// queries and the probabilities are split the same way; each product keeps the six piece pairs of
// order <= 2 (hi x hi, hi x mid, mid x hi, hi x lo, lo x hi, mid x mid) and drops those below 2^-24
// of it, so scores and outputs carry fp32-level error (about 2^-22 relative) instead of the 2^-17 of
// a hi + lo split.  In both products a lane of the 16 x 16 output owns
// one query column, so the online-softmax state (running max, rescale of O) is lane-local; the max
// over a query's keys needs two cross-lane steps.  The K-dimension slots of A and B are assigned the
// same way in each product (lane group lg holds slots 8 lg .. 8 lg + 7 of both operands), which is
// all the matrix product needs.  Key tiles entirely in the causal future of the workgroup's queries
// are not loaded, a wave skips the 32-key chunks in the future of its own queries, and keys of
// partially masked chunks get -inf (fully visible chunks skip the mask).
// Scores are scaled by scale * log2(e) and use the hardware exp2 (v_exp_f32, 1 ulp; results below
// the normal range flush to zero, which no probability normalised by the running max can notice).
#include "common.h"

using namespace vgx;

namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kKT = 64;             // keys per LDS tile
constexpr int kKTDma = 128;         // keys per LDS tile of bf16 K / V staged by LDS DMA
constexpr int kD = 128;             // head dim (the kernel is specialised for 128)
constexpr int kKRow = kD + 8;       // LDS row of K, bf16 (16 bytes of padding)
constexpr int kMaxBlocks = 8;
constexpr float kNegBig = -1.0e30f;
constexpr float kLazyMax = 8.0f;    // log2 of the largest unnormalised probability

typedef short v4i16_t __attribute__((ext_vector_type(4)));
typedef short v8i16_t __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives 16-bit element i % 4 of the 8-byte
// pieces addressed by lanes i / 4 + 4 k of the group, k = 0..3 (element k of the result).
__device__ __forceinline__ v4i16_t lds_read_tr16(const uint8_t *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) v4i16_t *)(p));
}

template <typename T>
__device__ __forceinline__ T sel4(int i, T a0, T a1, T a2, T a3) {
    return i == 0 ? a0 : i == 1 ? a1 : i == 2 ? a2 : a3;
}

struct RunArgs {
    const void *k;     // bf16 or fp32 rows
    const void *v;
    int64_t len;
    int64_t rstride;   // elements between consecutive keys
    int64_t gstride;   // elements between kv groups
};

struct BlockArgs {
    const void *q;     // query t, head h at t * ldq + h * q_hstride elements (fp32 or bf16)
    int64_t ldq;
    int64_t q_hstride;
    void *out;         // query t, head h at t * ldo + h * o_hstride elements (fp32 or bf16)
    int64_t ldo;
    int64_t o_hstride;
    int64_t n_q;
    int64_t causal_base;
    int n_runs;
    int tile0;         // first workgroup index of this block
    RunArgs run[4];
    // optional bias on run bias_run: query t of head h adds bias[t * bias_ldq + head_row[h] * bias_rstride
    // + j] to its score with key j of that run (head_row[h] < 0: none)
    const float *bias;
    const int32_t *bias_head_row;
    int64_t bias_ldq;
    int64_t bias_rstride;
    int bias_run;
};

struct PrefillArgs {
    BlockArgs blk[kMaxBlocks];
    int n_blocks;
    int n_tiles;
    int H, G;
    float scale_log2;  // scale * log2(e)
    int q_bf16;
    int o_bf16;        // output rounded to bf16 (round to nearest even) instead of fp32
    int n_split;       // key ranges per query tile (> 1: partials into ws, then attn_prefill_merge_kernel)
    float *ws;         // n_tiles * n_split slots of prefill_slot_floats
};

// Floats of one (query tile, key range) partial: O (unnormalised, the MFMA lane layout) and per query
// the running max and sum.
__host__ __device__ constexpr int prefill_slot_floats(int waves, int nqt) { return waves * nqt * (8 * 256 + 32); }

template <int GRP, bool QSPLIT, int NQT, bool KF, int QW, bool DMA>
__global__ __launch_bounds__(64 * GRP * QW) void attn_prefill_kernel(PrefillArgs a) {
    constexpr int kQTile = 16 * NQT * QW;
    // keys per LDS tile (fp32 K / V: 32, staged as three bf16 planes)
    constexpr int KT = KF ? 32 : (DMA ? kKTDma : kKT);
    constexpr int VROW = KT + 8;                    // LDS row of V^T, bf16 (16 bytes of padding)
    constexpr int NP = KF ? 3 : 1;                  // bf16 planes per K / V operand
    constexpr int NQP = QSPLIT ? (KF ? 3 : 2) : 1;  // bf16 pieces per query
    constexpr int NPP = KF ? 3 : 2;                 // bf16 pieces per probability
    constexpr int ORD = KF ? 2 : 1;                 // products of pieces i x j kept when i + j <= ORD
    constexpr int ESZ = KF ? 4 : 2;                 // bytes per K / V element in memory
    static_assert(!DMA || !KF, "LDS DMA stages bf16 K / V as they are");
    __shared__ __align__(16) uint16_t ks[DMA ? 2 * 2 * KT * kD : NP * KT * kKRow];   // DMA: [stage][K, V][key][dim]
    __shared__ __align__(16) uint16_t vt[DMA ? 8 : NP * kD * VROW];

    // XCD-aware order: consecutive tiles (same block and group, neighbouring queries, same keys; the
    // key ranges of one tile next to each other) on the same XCD so that its L2 serves their K/V.
    const int n_work = a.n_tiles * a.n_split;
    int work = blockIdx.x;
    if ((n_work & 7) == 0) work = (blockIdx.x & 7) * (n_work >> 3) + (blockIdx.x >> 3);
    const int tile = work / a.n_split, part = work - tile * a.n_split;
    int bi = 0;
#pragma unroll
    for (int i = 1; i < kMaxBlocks; ++i)
        if (i < a.n_blocks && a.blk[i].tile0 <= tile) bi = i;
    const BlockArgs &B = a.blk[bi];
    const int local = tile - B.tile0;
    const int g = local % a.G;
    const int64_t t0 = (int64_t)(local / a.G) * kQTile;

    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lq = lane & 15, lg = lane >> 4;
    const int h = g * GRP + wave % GRP;
    const int64_t tw = t0 + (int64_t)(wave / GRP) * 16 * NQT;   // the wave's first query

    // Q^T fragments (bf16): query t0 + 16 qt + lq, dims 32 kc + 8 lg .. + 7; fp32 queries as NQP
    // pieces: hi = bf16(q), then bf16 of what is left (lo, or mid and lo).
    bf16x8_t qf[NQP][NQT][4];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int64_t t = tw + qt * 16 + lq;
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) {
            const int d0 = kc * 32 + lg * 8;
            uint32_t pw[NQP][4];
            if (t < B.n_q) {
                if constexpr (!QSPLIT) {
                    const uint4 w = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(B.q) + t * B.ldq + h * B.q_hstride + d0);
                    pw[0][0] = w.x; pw[0][1] = w.y; pw[0][2] = w.z; pw[0][3] = w.w;
                } else {
                    const float *qp = static_cast<const float *>(B.q) + t * B.ldq + h * B.q_hstride + d0;
                    const float4 x0 = reinterpret_cast<const float4 *>(qp)[0], x1 = reinterpret_cast<const float4 *>(qp)[1];
                    const float e[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        if constexpr (NQP == 3) split3_bf16x2(e[2 * i], e[2 * i + 1], pw[0][i], pw[1][i], pw[2][i]);
                        else split_bf16x2(e[2 * i], e[2 * i + 1], pw[0][i], pw[NQP - 1][i]);
                    }
                }
            } else {
#pragma unroll
                for (int pp = 0; pp < NQP; ++pp)
#pragma unroll
                    for (int i = 0; i < 4; ++i) pw[pp][i] = 0;
            }
#pragma unroll
            for (int pp = 0; pp < NQP; ++pp)
                qf[pp][qt][kc] = __builtin_bit_cast(bf16x8_t, make_uint4(pw[pp][0], pw[pp][1], pw[pp][2], pw[pp][3]));
        }
    }

    f32x4_t o[NQT][8];
    float m[NQT], lsum[NQT];
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        m[qt] = kNegBig;
        lsum[qt] = 0.0f;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[qt][dt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    }

    // The block's key runs, read from the kernel arguments once and held in registers: the tile loop
    // selects among them instead of reloading argument memory at a run-dependent offset.
    const int n_runs = B.n_runs;
    const int64_t cbase = B.causal_base;
    int64_t rlen[4];
    const char *rkp[4], *rvp[4];
    int rrs[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const RunArgs &R = B.run[i];
        int64_t n = i < n_runs ? R.len : 0;
        if (i == n_runs - 1 && cbase >= 0) n = min(n, cbase + t0 + kQTile);   // the rest is in every query's future
        rlen[i] = n;
        rkp[i] = static_cast<const char *>(R.k) + (int64_t)g * R.gstride * ESZ;
        rvp[i] = static_cast<const char *>(R.v) + (int64_t)g * R.gstride * ESZ;
        rrs[i] = (int)R.rstride * ESZ;             // bytes between consecutive keys
    }

    // Key tiles in order over the runs; the global loads of the next tile are issued before the
    // current tile is computed (register double buffer), then stored into LDS (K as is, V transposed).
    auto run_len = [&](int r) -> int64_t { return sel4(r, rlen[0], rlen[1], rlen[2], rlen[3]); };
    constexpr int NT = 64 * GRP * QW;
    constexpr int CPR = kD * ESZ / 16;             // 16-byte chunks per key row
    constexpr int KCH = KT * CPR;                  // K chunks per tile
    constexpr int VCH = KT / 2 * CPR;              // V chunks per tile, counted in row pairs
    constexpr int KIT = (KCH + NT - 1) / NT, VIT = (VCH + NT - 1) / NT;
    uint4 kreg[KIT], vreg[VIT][2];
    auto fetch = [&](int r, int64_t j0) {
        const int64_t n = run_len(r);
        const int rs = sel4(r, rrs[0], rrs[1], rrs[2], rrs[3]);
        const char *kb = sel4(r, rkp[0], rkp[1], rkp[2], rkp[3]) + j0 * rs;   // wave-uniform
        const char *vb = sel4(r, rvp[0], rvp[1], rvp[2], rvp[3]) + j0 * rs;
        const int lim = (int)min<int64_t>(n - j0, KT);                        // rows of this tile
#pragma unroll
        for (int i = 0; i < KIT; ++i) {
            const int c = tid + i * NT;
            const int row = c / CPR, cc = c % CPR;
            kreg[i] = (c < KCH && row < lim) ? *reinterpret_cast<const uint4 *>(kb + row * rs + cc * 16)
                                             : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < VIT; ++i) {
            const int c = tid + i * NT;
            const int rp = c % (KT / 2), cc = c / (KT / 2);    // consecutive lanes: consecutive row pairs
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int row = 2 * rp + h2;
                vreg[i][h2] = (c < VCH && row < lim) ? *reinterpret_cast<const uint4 *>(vb + row * rs + cc * 16)
                                                     : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto issue = [&](int r, int64_t j0, int buf) {
        const int64_t n = run_len(r);
        const int rs = sel4(r, rrs[0], rrs[1], rrs[2], rrs[3]);
        const char *kb = sel4(r, rkp[0], rkp[1], rkp[2], rkp[3]) + j0 * rs;
        const char *vb = sel4(r, rvp[0], rvp[1], rvp[2], rvp[3]) + j0 * rs;
        const int lim = (int)min<int64_t>(n - j0, KT);
        const dma_rsrc_t krs = dma_rsrc(kb, (uint32_t)(lim * rs)), vrs = dma_rsrc(vb, (uint32_t)(lim * rs));
        uint8_t *base = reinterpret_cast<uint8_t *>(ks) + buf * (2 * KT * kD * 2);
        const int sub = lane >> 4, slot = lane & 15;
        for (int i = wave; i < KT / 2; i += NT / 64) {     // KT / 4 loads of 4 rows for K, as many for V
            const bool isv = i >= KT / 4;
            const int rb = 4 * (isv ? i - KT / 4 : i), row = rb + sub;
            dma16(isv ? vrs : krs, (uint32_t)(row * rs + ((slot ^ (row & 15)) << 4)),
                  base + (isv ? KT * kD * 2 : 0) + rb * kD * 2);
        }
    };
    auto stage = [&]() {
#pragma unroll
        for (int i = 0; i < KIT; ++i) {
            const int c = tid + i * NT;
            if (c >= KCH) continue;
            if constexpr (!KF) {
                *reinterpret_cast<uint4 *>(ks + (c >> 4) * kKRow + (c & 15) * 8) = kreg[i];
            } else {
                // four fp32 of row c / 32 -> bf16 hi, mid and lo (planes 0, 1, 2)
                uint2 hw, mw, lw;
                split3_bf16x2(__uint_as_float(kreg[i].x), __uint_as_float(kreg[i].y), hw.x, mw.x, lw.x);
                split3_bf16x2(__uint_as_float(kreg[i].z), __uint_as_float(kreg[i].w), hw.y, mw.y, lw.y);
                uint16_t *kp = ks + (c / CPR) * kKRow + (c % CPR) * 4;
                *reinterpret_cast<uint2 *>(kp) = hw;
                *reinterpret_cast<uint2 *>(kp + KT * kKRow) = mw;
                *reinterpret_cast<uint2 *>(kp + 2 * KT * kKRow) = lw;
            }
        }
#pragma unroll
        for (int i = 0; i < VIT; ++i) {
            const int c = tid + i * NT;
            if (c >= VCH) continue;
            const int rp = c % (KT / 2), cc = c / (KT / 2);
            const uint32_t a0[4] = {vreg[i][0].x, vreg[i][0].y, vreg[i][0].z, vreg[i][0].w};
            const uint32_t a1[4] = {vreg[i][1].x, vreg[i][1].y, vreg[i][1].z, vreg[i][1].w};
            if constexpr (!KF) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // dims 8 cc + 2 e and + 1 of keys 2 rp, 2 rp + 1: one 4-byte word each
                    *reinterpret_cast<uint32_t *>(vt + (cc * 8 + 2 * e) * VROW + 2 * rp) =
                        (a0[e] & 0xFFFFu) | (a1[e] << 16);
                    *reinterpret_cast<uint32_t *>(vt + (cc * 8 + 2 * e + 1) * VROW + 2 * rp) =
                        (a0[e] >> 16) | (a1[e] & 0xFFFF0000u);
                }
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // dim 4 cc + e of keys 2 rp, 2 rp + 1: the hi, mid and lo words
                    uint32_t hw, mw, lw;
                    split3_bf16x2(__uint_as_float(a0[e]), __uint_as_float(a1[e]), hw, mw, lw);
                    *reinterpret_cast<uint32_t *>(vt + (cc * 4 + e) * VROW + 2 * rp) = hw;
                    *reinterpret_cast<uint32_t *>(vt + kD * VROW + (cc * 4 + e) * VROW + 2 * rp) = mw;
                    *reinterpret_cast<uint32_t *>(vt + 2 * kD * VROW + (cc * 4 + e) * VROW + 2 * rp) = lw;
                }
            }
        }
    };

    const float sl2 = a.scale_log2;
    // this wave's bias rows (query t at brow + t * bias_ldq), when its head is biased
    const float *brow = nullptr;
    if (B.bias != nullptr) {
        const int hr = B.bias_head_row[h];
        if (hr >= 0) brow = B.bias + (int64_t)hr * B.bias_rstride;
    }
    // this workgroup's key range: part of the tile sequence over the runs (all of it without splits)
    int n_kt = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) n_kt += rlen[i] > 0 ? (int)((rlen[i] + KT - 1) / KT) : 0;
    const int per = (n_kt + a.n_split - 1) / a.n_split;
    int skip = part * per;
    int todo = max(0, min(n_kt, skip + per) - skip);
    int r = 0;
    while (r < n_runs && run_len(r) <= 0) ++r;
    int64_t j0 = 0;
    while (skip > 0 && r < n_runs) {
        const int nt = (int)((run_len(r) + KT - 1) / KT);
        if (skip < nt) {
            j0 = (int64_t)skip * KT;
            skip = 0;
        } else {
            skip -= nt;
            do { ++r; } while (r < n_runs && run_len(r) <= 0);
        }
    }
    if (todo == 0) r = n_runs;
    int buf = 0;
    if constexpr (DMA) {
        if (r < n_runs) issue(r, j0, 0);
    } else {
        if (r < n_runs) fetch(r, j0);
    }
    while (r < n_runs) {
        const int64_t n = run_len(r);
        const bool causal = (r == n_runs - 1) && cbase >= 0;
        int rn = r;
        int64_t jn = j0 + KT;
        if (jn >= n) {
            jn = 0;
            do { ++rn; } while (rn < n_runs && run_len(rn) <= 0);
        }
        if (todo <= 1) rn = n_runs;             // the range ends with this tile
        if constexpr (DMA) {
            // this tile's loads landed (each wave waits for its own, the barrier for every wave's), and
            // every wave is done with the other stage: the next tile's loads go there
            asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (rn < n_runs) issue(rn, jn, buf ^ 1);
        } else {
            __syncthreads();
            stage();
            __syncthreads();
            if (rn < n_runs) fetch(rn, jn);
        }
        const uint8_t *kst = reinterpret_cast<const uint8_t *>(ks) + buf * (2 * KT * kD * 2);
        const uint8_t *vst = kst + KT * kD * 2;
        auto scores = [&](int c, f32x4_t (&sc)[NQT][2]) {
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) {
                sc[qt][0] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
                sc[qt][1] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
            }
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
#pragma unroll
                for (int pk = 0; pk < NP; ++pk) {        // K plane: hi (then, fp32 K, mid and lo)
                    bf16x8_t a0, a1;
                    if constexpr (DMA) {
                        // rows c + lq, c + 16 + lq: 16-byte piece kc * 4 + lg stored at slot piece ^ (row & 15)
                        const int so = ((kc * 4 + lg) ^ lq) << 4;
                        a0 = *reinterpret_cast<const bf16x8_t *>(kst + (c + lq) * (kD * 2) + so);
                        a1 = *reinterpret_cast<const bf16x8_t *>(kst + (c + 16 + lq) * (kD * 2) + so);
                    } else {
                        const uint16_t *kp = ks + pk * KT * kKRow;
                        a0 = *reinterpret_cast<const bf16x8_t *>(kp + (c + lq) * kKRow + kc * 32 + lg * 8);
                        a1 = *reinterpret_cast<const bf16x8_t *>(kp + (c + 16 + lq) * kKRow + kc * 32 + lg * 8);
                    }
#pragma unroll
                    for (int qp = 0; qp < NQP; ++qp) {
                        if (pk + qp > ORD) continue;      // below 2^-(8 (ORD + 1)) of the product
#pragma unroll
                        for (int qt = 0; qt < NQT; ++qt) {
                            sc[qt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, qf[qp][qt][kc], sc[qt][0], 0, 0, 0);
                            sc[qt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, qf[qp][qt][kc], sc[qt][1], 0, 0, 0);
                        }
                    }
                }
            }
        };
        auto finish = [&](int c, f32x4_t (&sc)[NQT][2]) {
            bf16x8_t pf[NPP][NQT];
            // 32-key chunk fully visible to all 32 queries: no per-score mask
            const bool full = j0 + c + 32 <= n && (!causal || j0 + c + 31 <= cbase + tw);
            // the biased run of a biased head: its bias (log2 units) is added to the chunk's scores
            const bool biased = brow != nullptr && r == B.bias_run;   // wave-uniform
            // key index relative to the causal limit of query t0 (fits in 32 bits)
            const int kbase = (int)(j0 + c - (causal ? cbase + tw : 0));
            const int klim = (int)(n - (j0 + c));
#pragma unroll
            for (int qt = 0; qt < NQT; ++qt) {
                float v[8];
                if (full) {
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) v[kt * 4 + i] = sc[qt][kt][i] * sl2;
                } else {
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int kk = kt * 16 + lg * 4 + i;       // key within the 32-key chunk
                            const bool vis = kk < klim && (!causal || kbase + kk <= qt * 16 + lq);
                            v[kt * 4 + i] = vis ? sc[qt][kt][i] * sl2 : -INFINITY;
                        }
                }
                if (biased) {
                    const float *bq = brow + min(tw + qt * 16 + lq, B.n_q - 1) * B.bias_ldq;
#pragma unroll
                    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int64_t key = j0 + c + kt * 16 + lg * 4 + i;
                            if (key < n) v[kt * 4 + i] += bq[key] * 1.4426950408889634f;   // -inf stays -inf
                        }
                }
                float mt = v[0];
#pragma unroll
                for (int i = 1; i < 8; ++i) mt = fmaxf(mt, v[i]);
                mt = xor32_max(xor16_max(mt));
                // The reference max m (log2 units) moves only when a score exceeds it by more than
                // kLazyMax: probabilities then stay below 2^kLazyMax, and O and the sum are rescaled
                // far less often than the running max changes.
                if (__ballot(mt > m[qt] + kLazyMax)) {
                    const float mn = fmaxf(m[qt], mt);
                    const float corr = __builtin_amdgcn_exp2f(m[qt] - mn);
                    m[qt] = mn;
                    lsum[qt] *= corr;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt) o[qt][dt] *= corr;
                }
                const float mn = m[qt];
                float ps = 0.0f, pv[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    pv[i] = __builtin_amdgcn_exp2f(v[i] - mn);
                    ps += pv[i];
                }
                uint32_t pw[NPP][4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    if constexpr (NPP == 3) split3_bf16x2(pv[2 * i], pv[2 * i + 1], pw[0][i], pw[1][i], pw[2][i]);
                    else split_bf16x2(pv[2 * i], pv[2 * i + 1], pw[0][i], pw[1][i]);
                }
#pragma unroll
                for (int pp = 0; pp < NPP; ++pp)
                    pf[pp][qt] = __builtin_bit_cast(bf16x8_t, make_uint4(pw[pp][0], pw[pp][1], pw[pp][2], pw[pp][3]));
                lsum[qt] += ps;
            }
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
#pragma unroll
                for (int pv_ = 0; pv_ < NP; ++pv_) {     // V plane: hi (then, fp32 V, mid and lo)
                    bf16x8_t va;
                    if constexpr (DMA) {
                        // transposed reads of the row-major tile: lane lq of group lg addresses key
                        // c + 4 lg + lq / 4, dims 16 dt + 4 (lq % 4) .. + 3, and receives dim 16 dt + lq of
                        // keys c + 4 lg .. + 3 (then of the same keys + 16)
                        const int row = c + lg * 4 + (lq >> 2);
                        const int off = row * (kD * 2) + (((dt * 2 + ((lq & 3) >> 1)) ^ (row & 15)) << 4) + ((lq & 1) << 3);
                        const v4i16_t lo = lds_read_tr16(vst + off), hi = lds_read_tr16(vst + off + 16 * (kD * 2));
                        typedef short v8i16_t __attribute__((ext_vector_type(8)));
                        const v8i16_t w = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
                        va = __builtin_bit_cast(bf16x8_t, w);
                    } else {
                        const uint16_t *vr = vt + pv_ * kD * VROW + (dt * 16 + lq) * VROW + c + lg * 4;
                        const uint2 lo = *reinterpret_cast<const uint2 *>(vr);
                        const uint2 hi = *reinterpret_cast<const uint2 *>(vr + 16);
                        va = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                    }
#pragma unroll
                    for (int pp = 0; pp < NPP; ++pp) {
                        if (pv_ + pp > ORD) continue;     // as for the scores
#pragma unroll
                        for (int qt = 0; qt < NQT; ++qt)
                            o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[pp][qt], o[qt][dt], 0, 0, 0);
                    }
                }
            }
        };
        for (int c = 0; c < KT && j0 + c < n; c += 32) {
            if (causal && j0 + c > cbase + tw + 16 * NQT - 1) break;   // wave-uniform: the wave's future
            f32x4_t sc[NQT][2];
            scores(c, sc);
            finish(c, sc);
        }
        r = rn;
        j0 = jn;
        buf ^= 1;
        --todo;
    }

    if (a.n_split > 1) {
        // the partial of this key range: O as accumulated, and per query the max and sum
        constexpr int NWV = GRP * QW;
        float *slot = a.ws + (int64_t)work * prefill_slot_floats(NWV, NQT);
        float *ml = slot + NWV * NQT * 8 * 256;
#pragma unroll
        for (int qt = 0; qt < NQT; ++qt) {
            const float L = xor32_sum(xor16_sum(lsum[qt]));
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                *reinterpret_cast<float4 *>(slot + (((wave * NQT + qt) * 8 + dt) * 64 + lane) * 4) =
                    make_float4(o[qt][dt][0], o[qt][dt][1], o[qt][dt][2], o[qt][dt][3]);
            if (lg == 0) *reinterpret_cast<float2 *>(ml + ((wave * NQT + qt) * 16 + lq) * 2) = make_float2(m[qt], L);
        }
        return;
    }

#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const float L = xor32_sum(xor16_sum(lsum[qt]));
        const float inv = 1.0f / L;
        const int64_t t = tw + qt * 16 + lq;
        if (t >= B.n_q) continue;
        const int64_t oo = t * B.ldo + (int64_t)h * B.o_hstride;
        if (a.o_bf16) {
            uint16_t *op = static_cast<uint16_t *>(B.out) + oo;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
                *reinterpret_cast<uint2 *>(op + dt * 16 + lg * 4) =
                    make_uint2(pack_bf16x2(o[qt][dt][0] * inv, o[qt][dt][1] * inv),
                               pack_bf16x2(o[qt][dt][2] * inv, o[qt][dt][3] * inv));
        } else {
            float *op = static_cast<float *>(B.out) + oo;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) {
                float4 w;
                w.x = o[qt][dt][0] * inv; w.y = o[qt][dt][1] * inv; w.z = o[qt][dt][2] * inv; w.w = o[qt][dt][3] * inv;
                *reinterpret_cast<float4 *>(op + dt * 16 + lg * 4) = w;
            }
        }
    }
}

// The key ranges of each query tile combined: weights 2^(m_p - max m), O = sum w_p O_p / sum w_p L_p,
// written as the unsplit kernel writes its output.  One workgroup per query tile, the lanes of the
// attention kernel's layout.
template <int GRP, int NQT, int QW>
__global__ __launch_bounds__(64 * GRP * QW) void attn_prefill_merge_kernel(PrefillArgs a) {
    constexpr int kQTile = 16 * NQT * QW, NWV = GRP * QW;
    const int tile = blockIdx.x;
    int bi = 0;
#pragma unroll
    for (int i = 1; i < kMaxBlocks; ++i)
        if (i < a.n_blocks && a.blk[i].tile0 <= tile) bi = i;
    const BlockArgs &B = a.blk[bi];
    const int local = tile - B.tile0;
    const int g = local % a.G;
    const int64_t t0 = (int64_t)(local / a.G) * kQTile;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lq = lane & 15, lg = lane >> 4;
    const int h = g * GRP + wave % GRP;
    const int64_t tw = t0 + (int64_t)(wave / GRP) * 16 * NQT;
    const int ns = a.n_split;
    const float *slot0 = a.ws + (int64_t)tile * ns * prefill_slot_floats(NWV, NQT);
#pragma unroll
    for (int qt = 0; qt < NQT; ++qt) {
        const int64_t t = tw + qt * 16 + lq;
        float mp[4], lp[4], M = kNegBig;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            mp[p] = kNegBig;
            lp[p] = 0.0f;
            if (p < ns) {
                const float2 v = *reinterpret_cast<const float2 *>(slot0 + (int64_t)p * prefill_slot_floats(NWV, NQT) +
                                                                   NWV * NQT * 8 * 256 + ((wave * NQT + qt) * 16 + lq) * 2);
                mp[p] = v.x;
                lp[p] = v.y;
                M = fmaxf(M, v.x);
            }
        }
        float w[4], L = 0.0f;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            w[p] = p < ns ? __builtin_amdgcn_exp2f(mp[p] - M) : 0.0f;
            L += w[p] * lp[p];
        }
        const float inv = 1.0f / L;
        if (t >= B.n_q) continue;
        const int64_t oo = t * B.ldo + (int64_t)h * B.o_hstride;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                if (p >= ns) continue;
                const float4 x = *reinterpret_cast<const float4 *>(slot0 + (int64_t)p * prefill_slot_floats(NWV, NQT) +
                                                                   (((wave * NQT + qt) * 8 + dt) * 64 + lane) * 4);
                v.x = fmaf(w[p], x.x, v.x); v.y = fmaf(w[p], x.y, v.y); v.z = fmaf(w[p], x.z, v.z); v.w = fmaf(w[p], x.w, v.w);
            }
            if (a.o_bf16) {
                uint16_t *op = static_cast<uint16_t *>(B.out) + oo;
                *reinterpret_cast<uint2 *>(op + dt * 16 + lg * 4) =
                    make_uint2(pack_bf16x2(v.x * inv, v.y * inv), pack_bf16x2(v.z * inv, v.w * inv));
            } else {
                float *op = static_cast<float *>(B.out) + oo;
                *reinterpret_cast<float4 *>(op + dt * 16 + lg * 4) = make_float4(v.x * inv, v.y * inv, v.z * inv, v.w * inv);
            }
        }
    }
}

// Launch shape per K / V dtype and heads per group: NQT 16-query tiles per wave, QW waves per head, LDS
// DMA staging.  At 4 and 6 heads per group a workgroup of 2 GRP waves of 16 queries (at most 168
// registers, three waves per SIMD: one workgroup of 12 waves per CU at 6 heads) keeps more waves in
// flight than GRP waves of 32 queries (226-256 registers, two per SIMD, 6 waves per CU), for the same
// K / V tile per 32 queries.  Measured at L = 8192 (12 query / 2 KV heads, drop-in call): bf16 K / V
// 333 -> 295 us with 2 x 6 waves of 16 queries, -> 264 us with the tiles staged by LDS DMA (64 keys),
// -> 247 us with 128-key tiles; fp32 K / V 1082 -> 749 us with 2 x 6 waves.  Eight heads per group
// keep 8 waves of 32 queries (16 waves would need <= 128 registers and spill), one and two the
// register-staged 32-query waves.  A launch of fewer 2-wave-per-head workgroups than CUs (a 2048-query
// chunk of the chunk-recurrent prefill at 2 KV heads: 128) runs one wave per head instead (narrow):
// twice the workgroups over the CUs.
constexpr int kPrefillNarrowBelow = 256;
constexpr int prefill_nqt(int grp, bool kf) { return kf || grp == 4 || grp == 6 ? 1 : 2; }
constexpr int prefill_qw(int grp, bool kf, bool narrow) {
    return !narrow && (grp == 4 || grp == 6 || (kf && grp == 2)) ? 2 : 1;
}
constexpr bool prefill_dma(int grp, bool kf) { return !kf && grp >= 4; }

// Key-range splits: with a workspace, a launch of fewer than kPrefillNarrowBelow workgroups (a
// 1024-query chunk of the chunk-recurrent prefill at 2 KV heads: 128) splits each tile's keys into up to
// four ranges, so that the launch fills the CUs; attn_prefill_merge_kernel then combines them.
constexpr int kPrefillMaxSplit = 4;
// Workspace bound: at most kPrefillNarrowBelow (tile, range) slots, each of at most 2 GRP waves x 2
// 16-query tiles.
inline int64_t prefill_ws_bytes(int grp) {
    return (int64_t)kPrefillNarrowBelow * prefill_slot_floats(2 * grp, 2) * 4;
}

int attn_prefill_impl(int kv_dtype, int q_dtype, int out_dtype, const vgx_attn_block *blocks, int n_blocks, int64_t H,
                      int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes, void *stream) {
    if (kv_dtype != VGX_BF16 && kv_dtype != VGX_F32) return VGX_E_DTYPE;
    if (out_dtype != VGX_F32 && out_dtype != VGX_BF16) return VGX_E_DTYPE;
    const int oel = out_dtype == VGX_BF16 ? 2 : 4;
    const int esz = kv_dtype == VGX_F32 ? 4 : 2;
    if (q_dtype != VGX_F32 && q_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!blocks) return VGX_E_ARG;
    if (n_blocks < 0 || n_blocks > kMaxBlocks) return VGX_E_LIMIT;
    if (H <= 0 || G <= 0 || H % G) return VGX_E_SIZE;
    if (D != kD) return VGX_E_LIMIT;
    const int grp = (int)(H / G);
    if (grp != 1 && grp != 2 && grp != 4 && grp != 6 && grp != 8) return VGX_E_LIMIT;
    const bool kf = kv_dtype == VGX_F32;
    int64_t wide_tiles = 0;
    for (int i = 0; i < n_blocks; ++i)
        if (blocks[i].n_q > 0) wide_tiles += (blocks[i].n_q + 31) / 32 * G;
    const bool narrow = prefill_qw(grp, kf, false) > 1 && wide_tiles < kPrefillNarrowBelow;
    const int qtile = 16 * prefill_nqt(grp, kf) * prefill_qw(grp, kf, narrow);   // queries per workgroup
    PrefillArgs a{};
    a.H = (int)H;
    a.G = (int)G;
    a.scale_log2 = scale * 1.4426950408889634f;
    a.q_bf16 = q_dtype == VGX_BF16;
    a.o_bf16 = out_dtype == VGX_BF16;
    int64_t tiles = 0;
    int nb = 0;
    for (int i = 0; i < n_blocks; ++i) {
        const vgx_attn_block &b = blocks[i];
        if (b.n_q < 0 || b.n_runs < 1 || b.n_runs > 4) return VGX_E_SIZE;
        if (b.n_q == 0) continue;
        if (!b.q || !b.out) return VGX_E_ARG;
        const int qel = q_dtype == VGX_BF16 ? 2 : 4;
        if (b.q_hstride < D || b.o_hstride < D || b.ldq < 0 || b.ldo < 0) return VGX_E_SIZE;
        if (((uintptr_t)b.q % 16) || ((uintptr_t)b.out % 16) || (b.ldq * qel) % 16 || (b.q_hstride * qel) % 16 ||
            (b.ldo * oel) % 16 || (b.o_hstride * oel) % 16)
            return VGX_E_ALIGN;
        BlockArgs &B = a.blk[nb];
        B.q = b.q;
        B.ldq = b.ldq;
        B.q_hstride = b.q_hstride;
        B.out = b.out;
        B.ldo = b.ldo;
        B.o_hstride = b.o_hstride;
        B.n_q = b.n_q;
        B.causal_base = b.causal_base;
        B.n_runs = b.n_runs;
        B.tile0 = (int)tiles;
        if (b.bias) {
            if (!b.bias_head_row || b.bias_run < 0 || b.bias_run >= b.n_runs) return VGX_E_ARG;
            if (b.bias_ldq < 0 || b.bias_rstride < 0) return VGX_E_SIZE;
            B.bias = b.bias;
            B.bias_head_row = b.bias_head_row;
            B.bias_ldq = b.bias_ldq;
            B.bias_rstride = b.bias_rstride;
            B.bias_run = b.bias_run;
        }
        int64_t n_keys = 0;
        for (int r = 0; r < b.n_runs; ++r) {
            const vgx_kv_run &R = b.runs[r];
            if (R.len < 0) return VGX_E_SIZE;
            if (R.len > 0 && (!R.k || !R.v)) return VGX_E_ARG;
            if (R.len > 0 && (((uintptr_t)R.k | (uintptr_t)R.v) % 16 || (R.row_stride * esz) % 16 ||
                              (R.group_stride * esz) % 16))
                return VGX_E_ALIGN;
            if (R.row_stride < D || R.row_stride >= (1 << 24)) return VGX_E_SIZE;   // tile offsets are 32-bit
            B.run[r].k = R.k;
            B.run[r].v = R.v;
            B.run[r].len = R.len;
            B.run[r].rstride = R.row_stride;
            B.run[r].gstride = R.group_stride;
            n_keys += R.len;
        }
        if (b.causal_base >= 0 && b.causal_base + 1 > b.runs[b.n_runs - 1].len) return VGX_E_SIZE;
        if (n_keys == 0) return VGX_E_SIZE;
        tiles += (b.n_q + qtile - 1) / qtile * G;
        ++nb;
    }
    if (nb == 0) return VGX_OK;
    if (tiles > 0x7FFFFFFF) return VGX_E_LIMIT;
    a.n_blocks = nb;
    a.n_tiles = (int)tiles;
    a.n_split = 1;
    if (workspace != nullptr && tiles < kPrefillNarrowBelow) {
        if (workspace_bytes < prefill_ws_bytes(grp)) return VGX_E_ARENA;
        if ((uintptr_t)workspace % 16) return VGX_E_ALIGN;
        a.n_split = (int)std::min<int64_t>(kPrefillMaxSplit, kPrefillNarrowBelow / tiles);
        a.ws = static_cast<float *>(workspace);
    }
    hipStream_t st = (hipStream_t)stream;
    const dim3 grid((unsigned)(tiles * a.n_split));
#define VGX_PREFILL_SHAPE(G_, S_, KF_, N_)                                                                   \
    do {                                                                                                     \
        hipLaunchKernelGGL((attn_prefill_kernel<G_, S_, prefill_nqt(G_, KF_), KF_, prefill_qw(G_, KF_, N_),    \
                                                prefill_dma(G_, KF_)>),                                        \
                           grid, dim3(64 * G_ * prefill_qw(G_, KF_, N_)), 0, st, a);                           \
        if (a.n_split > 1)                                                                                   \
            hipLaunchKernelGGL((attn_prefill_merge_kernel<G_, prefill_nqt(G_, KF_), prefill_qw(G_, KF_, N_)>),  \
                               dim3((unsigned)tiles), dim3(64 * G_ * prefill_qw(G_, KF_, N_)), 0, st, a);      \
    } while (0)
#define VGX_PREFILL_GO(G_, S_)                                                                               \
    do {                                                                                                     \
        if (kf) {                                                                                            \
            if (narrow) VGX_PREFILL_SHAPE(G_, S_, true, true); else VGX_PREFILL_SHAPE(G_, S_, true, false);  \
        } else {                                                                                             \
            if (narrow) VGX_PREFILL_SHAPE(G_, S_, false, true); else VGX_PREFILL_SHAPE(G_, S_, false, false);\
        }                                                                                                    \
    } while (0)
#define VGX_PREFILL_GRP(S_)                      \
    switch (grp) {                               \
        case 1: VGX_PREFILL_GO(1, S_); break;    \
        case 2: VGX_PREFILL_GO(2, S_); break;    \
        case 4: VGX_PREFILL_GO(4, S_); break;    \
        case 6: VGX_PREFILL_GO(6, S_); break;    \
        case 8: VGX_PREFILL_GO(8, S_); break;    \
    }
    if (a.q_bf16) {
        VGX_PREFILL_GRP(false)
    } else {
        VGX_PREFILL_GRP(true)
    }
#undef VGX_PREFILL_GRP
#undef VGX_PREFILL_GO
#undef VGX_PREFILL_SHAPE
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // namespace

extern "C" {

int vgx_attn_prefill(int kv_dtype, int q_dtype, int out_dtype, const vgx_attn_block *blocks, int n_blocks, int64_t H,
                     int64_t G, int64_t D, float scale, void *stream) {
    return attn_prefill_impl(kv_dtype, q_dtype, out_dtype, blocks, n_blocks, H, G, D, scale, nullptr, 0, stream);
}

int64_t vgx_attn_prefill_workspace_bytes(int64_t H, int64_t G) {
    if (H <= 0 || G <= 0 || H % G) return VGX_E_SIZE;
    if (H / G > 8) return VGX_E_LIMIT;
    return prefill_ws_bytes((int)(H / G));
}

int vgx_attn_prefill_ws(int kv_dtype, int q_dtype, int out_dtype, const vgx_attn_block *blocks, int n_blocks, int64_t H,
                        int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes, void *stream) {
    if (!workspace) return VGX_E_ARG;
    return attn_prefill_impl(kv_dtype, q_dtype, out_dtype, blocks, n_blocks, H, G, D, scale, workspace, workspace_bytes,
                             stream);
}

}  // extern "C"
