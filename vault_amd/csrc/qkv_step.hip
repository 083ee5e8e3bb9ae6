// Decode step (one token): RMSNorm + q / k / v projections with the RoPE rotation and the KV ring
// and sink writes done in the projection's epilogue, in one launch.
//
// Reference semantics: src/vault_v3_model.py:2289-2290 (input_layernorm), 1041-1047 (q/k/v
// projections with bias), 777-794 (rotate-half RoPE), 1079-1094 (ring write of the rotated key, the
// raw key and the value, sink copy while pos < S_cap); runtime/vault3.c:2152-2179.
//
// Weights are packed for this kernel with vgx_qweight_pack_rope: inside every head the rows of a
// packed row-quad are (2j, 2j + D/2, 2j + 1, 2j + 1 + D/2), the two rotation pairs 2j and 2j + 1,
// so the rotation needs no exchange between lanes.  v rows keep their natural order.  q and k|v are
// two tensors that may have different block dtypes (hybrid Q4_0 q with Q8_0 k|v); workgroups
// [0, H D / 4) take q row-quads, the rest k|v, each with the code of its dtype.
//
// Mapping (rows of up to 64 Q8_0 / Q4_0 blocks: qkv_rope_step_pieces_kernel, below; otherwise
// qkv_rope_step_kernel): one wave per row-quad, lane i takes blocks i, i + 64, ... of the row-quad,
// loading its activation block and RMSNorm weights directly (the same 12 KB for every wave: L1 / L2
// hits); sum x^2 of the wave's blocks is the full sum.  The
// position-dependent values (ring slot, RoPE table row, sink slot) come from the device step
// descriptor, so a captured graph replays at every position of a chunk.
#include "qgemv.h"

using namespace vgx;

namespace {

struct QkvStepArgs {
    const uint8_t *wq;
    int64_t soff_q;
    const float *bq;
    const uint8_t *wkv;
    int64_t soff_kv;
    const float *bkv;
    int nblk;
    int H, G, D;
    const float *x;
    const float *lnw;
    float eps;
    float *x_copy;
    const float *table;
    int64_t trs;
    const int32_t *step;
    float *q_out;
    void *k_rot, *k_raw, *v_dst;
    int64_t dgs, drs;
    void *sk, *sv;
    int64_t sgs, srs;
};

template <int KV>
__device__ __forceinline__ void put(void *base, int64_t idx, float v) {
    if constexpr (KV == VGX_F32) static_cast<float *>(base)[idx] = v;
    else static_cast<uint16_t *>(base)[idx] = (uint16_t)float_to_bf16_bits(v);
}

// acc[r] = W[4 rq + r] . (lnw * x) over the blocks of this lane (not yet reduced over lanes);
// ssq = sum of x^2 over the same blocks.
template <int DT>
__device__ __forceinline__ void rq_dot(const uint8_t *__restrict__ W, int64_t soff, int64_t rq, int nblk,
                                       const float *__restrict__ x, const float *__restrict__ lnw,
                                       float *__restrict__ x_copy, float (&acc)[4][1], float &ssq) {
    const int lane = threadIdx.x & 63;
    for (int b = lane; b < nblk; b += 64) {
        BlockRegs<DT> br;
        gemv_load<DT>(br, W, soff, rq, nblk, b);
        const float4 *xp = reinterpret_cast<const float4 *>(x + b * QK);
        float4 xv[8], gv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) xv[j] = xp[j];
        if (lnw) {
            const float4 *gp = reinterpret_cast<const float4 *>(lnw + b * QK);
#pragma unroll
            for (int j = 0; j < 8; ++j) gv[j] = gp[j];
        }
        if (x_copy) {
#pragma unroll
            for (int j = 0; j < 8; ++j) reinterpret_cast<float4 *>(x_copy + b * QK)[j] = xv[j];
        }
        float xb[QK];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float4 t = xv[j];
            ssq += fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, t.w * t.w)));
            if (lnw) {
                t.x *= gv[j].x; t.y *= gv[j].y; t.z *= gv[j].z; t.w *= gv[j].w;
            }
            xb[4 * j] = t.x; xb[4 * j + 1] = t.y; xb[4 * j + 2] = t.z; xb[4 * j + 3] = t.w;
        }
        gemv_block<DT, 1>(br, xb, 0, acc);
    }
}

// Bias, RoPE and the ring / sink writes of row-quad wg (q row-quads first, then k, then v) from the
// four finished dot products acc[0..3] (rows 4 wg .. + 3, RMSNorm scale applied), held by every lane
// of the calling wave.
template <int KV>
__device__ __forceinline__ void qkv_epilogue(const QkvStepArgs &a, int64_t wg, int lane, const float (&acc)[4][1]) {
    const int D = a.D, h2 = D / 2, qpd = D / 4;
    const int64_t nq = (int64_t)a.H * qpd, nk = (int64_t)a.G * qpd;
    const int64_t slot = a.step[VGX_STEP_SLOT];
    const int64_t sink = a.step[VGX_STEP_SINK_SLOT];
    const float *cs = a.table + (int64_t)a.step[VGX_STEP_TABLE_ROW] * a.trs;
    if (wg < nq + nk) {
        // rotation pairs: lane 0 takes pair 2j (rows 0, 1 of the quad), lane 1 pair 2j + 1 (rows 2, 3)
        if (lane >= 2) return;
        const bool isq = wg < nq;
        const int64_t rq = isq ? wg : wg - nq;
        const int hd = (int)(rq / qpd), j = (int)(rq - (int64_t)hd * qpd);
        const int p = 2 * j + lane;
        const float *bias = isq ? a.bq : a.bkv;
        float x0 = lane ? acc[2][0] : acc[0][0];
        float x1 = lane ? acc[3][0] : acc[1][0];
        if (bias) {
            x0 += bias[(int64_t)hd * D + p];
            x1 += bias[(int64_t)hd * D + p + h2];
        }
        const float c = cs[p], s = cs[h2 + p];
        const float r0 = x0 * c - x1 * s, r1 = x1 * c + x0 * s;
        if (isq) {
            a.q_out[(int64_t)hd * D + p] = r0;
            a.q_out[(int64_t)hd * D + p + h2] = r1;
            return;
        }
        const int64_t o = hd * a.dgs + slot * a.drs;
        put<KV>(a.k_rot, o + p, r0);
        put<KV>(a.k_rot, o + p + h2, r1);
        put<KV>(a.k_raw, o + p, x0);
        put<KV>(a.k_raw, o + p + h2, x1);
        if (sink >= 0 && a.sk) {
            const int64_t so = hd * a.sgs + sink * a.srs;
            put<KV>(a.sk, so + p, x0);
            put<KV>(a.sk, so + p + h2, x1);
        }
        return;
    }
    // v rows in natural order: lane r < 4 writes row 4 rq + r
    if (lane >= 4) return;
    const int64_t row = (wg - nq - nk) * 4 + lane;
    const int g = (int)(row / D), i = (int)(row - (int64_t)g * D);
    float v = lane == 0 ? acc[0][0] : lane == 1 ? acc[1][0] : lane == 2 ? acc[2][0] : acc[3][0];
    if (a.bkv) v += a.bkv[(int64_t)a.G * D + row];
    put<KV>(a.v_dst, g * a.dgs + slot * a.drs + i, v);
    if (sink >= 0 && a.sv) put<KV>(a.sv, g * a.sgs + sink * a.srs + i, v);
}

template <int DTQ, int DTKV, int KV>
__global__ __launch_bounds__(64) void qkv_rope_step_kernel(QkvStepArgs a) {
    const int qpd = a.D / 4;                              // row-quads per head
    const int64_t nq = (int64_t)a.H * qpd;
    const int64_t wg = blockIdx.x;
    const int lane = threadIdx.x;
    float acc[4][1] = {{0.0f}, {0.0f}, {0.0f}, {0.0f}};
    float ssq = 0.0f;
    float *xc = wg == 0 ? a.x_copy : nullptr;
    if (wg < nq) rq_dot<DTQ>(a.wq, a.soff_q, wg, a.nblk, a.x, a.lnw, xc, acc, ssq);
    else rq_dot<DTKV>(a.wkv, a.soff_kv, wg - nq, a.nblk, a.x, a.lnw, xc, acc, ssq);
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r][0] = wave_sum(acc[r][0]);
    if (a.lnw) {
        const float inv = 1.0f / sqrtf(wave_sum(ssq) / (float)(a.nblk * QK) + a.eps);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r][0] *= inv;
    }
    qkv_epilogue<KV>(a, wg, lane, acc);
}

// Q8_0 / Q4_0 weights of rows up to 64 blocks (d_model <= 2048): a workgroup of NW waves per row-quad.
// The row-quad's run is cut into 1 KB pieces (Q4_0: 16 blocks x 4 rows, lane l row l & 3 of block
// 16 p + l / 4; Q8_0: 8 blocks x 4 rows, lane l half l & 1 of row (l >> 1) & 3 of block 8 p + l / 8),
// one 16-byte buffer load per lane and piece, wave w taking pieces w, w + NW, ...; every load instruction
// reads one contiguous 1 KB range.  The workgroup stages lnw * x once in LDS (blocks padded to 36
// floats against bank conflicts, Q4_0 block sums for the -8 offset) with sum x^2 for the RMSNorm
// scale; the lanes of a row and then the waves are summed in a fixed order, and wave 0 runs the
// epilogue.
constexpr int kQkvPiecesMaxBlocks = 64;

// the row-quad's dot products, summed over the workgroup: every lane of wave 0 gets rows 0..3
template <int DT, int NW>
__device__ __forceinline__ void qkv_pieces_rq(const uint8_t *__restrict__ W, int64_t soff, int64_t n_rq, int64_t rq,
                                              int nblk, const float *xs, const float *xsum, float (*red)[4],
                                              int wave, int lane) {
    constexpr int QB = DT == VGX_Q8_0 ? 32 : 16;
    constexpr int BPP = 1024 / (4 * QB);               // blocks per piece
    constexpr int MAXI = (kQkvPiecesMaxBlocks / BPP + NW - 1) / NW;   // pieces per wave
    const int npc = (nblk + BPP - 1) / BPP;
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc((void *)W, 0, (int)soff, 0x00020000);
    const __amdgpu_buffer_rsrc_t srs =
        __builtin_amdgcn_make_buffer_rsrc((void *)(W + soff), 0, (int)(n_rq * nblk * 8), 0x00020000);
    const int row = DT == VGX_Q8_0 ? (lane >> 1) & 3 : lane & 3;
    uint4 wq[MAXI];
    uint32_t wsc[MAXI];
    int blk_of[MAXI];
#pragma unroll
    for (int k = 0; k < MAXI; ++k) {
        const int pc = wave + NW * k;
        const int blk = BPP * pc + (DT == VGX_Q8_0 ? lane >> 3 : lane >> 2);
        const bool ok = pc < npc && blk < nblk;
        blk_of[k] = min(blk, nblk - 1);
        const uint32_t qo = ok ? (uint32_t)((rq * nblk + blk) * 4 * QB + row * QB + (DT == VGX_Q8_0 ? (lane & 1) * 16 : 0))
                               : kStreamPastEnd;
        const uint32_t so = ok ? (uint32_t)((rq * nblk + blk) * 8 + row * 2) : kStreamPastEnd;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(wrs, qo, 0, kStreamAux);
        wq[k] = make_uint4(v[0], v[1], v[2], v[3]);
        wsc[k] = __builtin_amdgcn_raw_buffer_load_b16(srs, so, 0, kStreamAux);
    }
    __syncthreads();                                   // the activations are staged
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < MAXI; ++k)
        if (wave + NW * k < npc) acc += gemv_piece_dot<DT>(wq[k], wsc[k], xs, xsum, blk_of[k], lane);
    if constexpr (DT == VGX_Q8_0) {
        acc += dpp_f<DPP_QUAD_1032>(acc);             // lane ^ 1: the other half of the row
        acc += dpp_f<0x128>(acc);                     // row_ror 8: lane ^ 8
    } else {
        acc += dpp_f<0x124>(acc);                     // row_ror 4 and 8: the lanes of the same l & 3
        acc += dpp_f<0x128>(acc);
    }
    acc = xor32_sum(xor16_sum(acc));
    if (DT == VGX_Q8_0 ? (lane & 0x39) == 0 : lane < 4) red[wave][row] = acc;
    __syncthreads();
}

template <int DTQ, int DTKV, int KV, int NW>
__global__ __launch_bounds__(64 * NW) void qkv_rope_step_pieces_kernel(QkvStepArgs a) {
    constexpr int NT = 64 * NW;
    constexpr int XR = (kQkvPiecesMaxBlocks * 8 + NT - 1) / NT;   // staging rounds of one float4 per thread
    __shared__ __align__(16) float xs[kQkvPiecesMaxBlocks * kGemvPad];
    __shared__ float xsum[kQkvPiecesMaxBlocks];
    __shared__ float red[NW][4];
    __shared__ float rss[NW];
    const int qpd = a.D / 4;
    const int64_t nq = (int64_t)a.H * qpd;
    const int64_t wg = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nblk = a.nblk, n4 = nblk * 8;
    // lnw * x staged (XR float4 per thread cover 64 blocks), sum x^2, Q4_0 block sums
    float4 xv[XR], gv[XR];
#pragma unroll
    for (int u = 0; u < XR; ++u) {
        const int i = tid + NT * u;
        xv[u] = i < n4 ? reinterpret_cast<const float4 *>(a.x)[i] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        gv[u] = a.lnw && i < n4 ? reinterpret_cast<const float4 *>(a.lnw)[i] : make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    }
    float ssq = 0.0f;
#pragma unroll
    for (int u = 0; u < XR; ++u) {
        const int i = tid + NT * u;
        float4 t = xv[u];
        if (i < n4 && wg == 0 && a.x_copy) reinterpret_cast<float4 *>(a.x_copy)[i] = t;
        ssq += fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, t.w * t.w)));
        t.x *= gv[u].x; t.y *= gv[u].y; t.z *= gv[u].z; t.w *= gv[u].w;
        if (i < n4) reinterpret_cast<float4 *>(xs)[(i >> 3) * (kGemvPad / 4) + (i & 7)] = t;
        float s = (t.x + t.y) + (t.z + t.w);          // the block's 8 float4 are 8 consecutive threads
        s += __shfl_xor(s, 1, kWave);
        s += __shfl_xor(s, 2, kWave);
        s += __shfl_xor(s, 4, kWave);
        if (i < n4 && (i & 7) == 0) xsum[i >> 3] = 8.0f * s;
    }
    ssq = wave_sum(ssq);
    if (lane == 0) rss[wave] = ssq;
    if (wg < nq) qkv_pieces_rq<DTQ, NW>(a.wq, a.soff_q, nq, wg, nblk, xs, xsum, red, wave, lane);
    else qkv_pieces_rq<DTKV, NW>(a.wkv, a.soff_kv, (int64_t)2 * a.G * qpd, wg - nq, nblk, xs, xsum, red, wave, lane);
    if (wave != 0) return;
    float acc[4][1];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        float v = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) v += red[w][r];
        acc[r][0] = v;
    }
    if (a.lnw) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < NW; ++w) t += rss[w];
        const float inv = 1.0f / sqrtf(t / (float)(nblk * QK) + a.eps);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r][0] *= inv;
    }
    qkv_epilogue<KV>(a, wg, lane, acc);
}

template <int DTQ, int DTKV>
void launch(int kv, const QkvStepArgs &a, unsigned grid, hipStream_t st) {
    if constexpr (gemv_quant(DTQ) && gemv_quant(DTKV)) {
        if (a.nblk <= kQkvPiecesMaxBlocks && a.soff_q < ((int64_t)1 << 31) && a.soff_kv < ((int64_t)1 << 31)) {
            // 8 waves per row-quad (the staging spread over 512 threads; pieces w and w + 8): decode step 1002
            // against 996 tok/s with 4 waves (2: 982, 3: 990, 6: 997)
            constexpr int NW = 8;
            if (kv == VGX_F32) hipLaunchKernelGGL((qkv_rope_step_pieces_kernel<DTQ, DTKV, VGX_F32, NW>), dim3(grid), dim3(64 * NW), 0, st, a);
            else hipLaunchKernelGGL((qkv_rope_step_pieces_kernel<DTQ, DTKV, VGX_BF16, NW>), dim3(grid), dim3(64 * NW), 0, st, a);
            return;
        }
    }
    if (kv == VGX_F32) hipLaunchKernelGGL((qkv_rope_step_kernel<DTQ, DTKV, VGX_F32>), dim3(grid), dim3(64), 0, st, a);
    else hipLaunchKernelGGL((qkv_rope_step_kernel<DTQ, DTKV, VGX_BF16>), dim3(grid), dim3(64), 0, st, a);
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

extern "C" {

int vgx_qkv_rope_step(int q_dtype, const void *wq, const float *bq, int kv_wdtype, const void *wkv, const float *bkv,
                      int64_t d_model, int64_t H, int64_t G, int64_t D, const float *x, const float *norm_w, float eps,
                      float *x_copy, const float *table, int64_t table_rstride, const int32_t *step, float *q_out,
                      int kv_dtype, void *k_rot, void *k_raw, void *v_dst, int64_t dst_gstride, int64_t dst_rstride,
                      void *sink_k_raw, void *sink_v, int64_t sink_gstride, int64_t sink_rstride, void *stream) {
    const bool pair_ok = (q_dtype == VGX_Q4_0 && kv_wdtype == VGX_Q8_0) ||
                         (q_dtype == kv_wdtype && (gemv_quant(q_dtype) || gemv_plain(q_dtype)));
    if (!pair_ok || (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16)) return VGX_E_DTYPE;
    if (!wq || !wkv || !x || !table || !step || !q_out || !k_rot || !k_raw || !v_dst) return VGX_E_ARG;
    if ((sink_k_raw == nullptr) != (sink_v == nullptr)) return VGX_E_ARG;
    if (d_model <= 0 || H <= 0 || G <= 0 || D <= 0 || H % G) return VGX_E_SIZE;
    if (d_model % QK || D % 4) return VGX_E_SHAPE;
    if (norm_w && !(eps > 0.0f)) return VGX_E_ARG;
    if (!aligned16(x) || (norm_w && !aligned16(norm_w)) || (x_copy && !aligned16(x_copy))) return VGX_E_ALIGN;
    if (d_model / QK > (1 << 24) || (H + 2 * G) * D / 4 > 0x7FFFFFFF) return VGX_E_LIMIT;
    QkvStepArgs a{};
    a.wq = static_cast<const uint8_t *>(wq);
    a.wkv = static_cast<const uint8_t *>(wkv);
    a.soff_q = gemv_plain(q_dtype) ? 0 : vgx_qweight_scale_offset(q_dtype, H * D, d_model);
    a.soff_kv = gemv_plain(kv_wdtype) ? 0 : vgx_qweight_scale_offset(kv_wdtype, 2 * G * D, d_model);
    a.bq = bq;
    a.bkv = bkv;
    a.nblk = (int)(d_model / QK);
    a.H = (int)H;
    a.G = (int)G;
    a.D = (int)D;
    a.x = x;
    a.lnw = norm_w;
    a.eps = eps;
    a.x_copy = x_copy;
    a.table = table;
    a.trs = table_rstride;
    a.step = step;
    a.q_out = q_out;
    a.k_rot = k_rot;
    a.k_raw = k_raw;
    a.v_dst = v_dst;
    a.dgs = dst_gstride;
    a.drs = dst_rstride;
    a.sk = sink_k_raw;
    a.sv = sink_v;
    a.sgs = sink_gstride;
    a.srs = sink_rstride;
    const unsigned grid = (unsigned)((H + 2 * G) * D / 4);
    hipStream_t st = (hipStream_t)stream;
    if (q_dtype == VGX_Q4_0 && kv_wdtype == VGX_Q8_0) launch<VGX_Q4_0, VGX_Q8_0>(kv_dtype, a, grid, st);
    else if (q_dtype == VGX_Q8_0) launch<VGX_Q8_0, VGX_Q8_0>(kv_dtype, a, grid, st);
    else if (q_dtype == VGX_Q4_0) launch<VGX_Q4_0, VGX_Q4_0>(kv_dtype, a, grid, st);
    else if (q_dtype == VGX_BF16) launch<VGX_BF16, VGX_BF16>(kv_dtype, a, grid, st);
    else if (q_dtype == VGX_F16) launch<VGX_F16, VGX_F16>(kv_dtype, a, grid, st);
    else launch<VGX_F32, VGX_F32>(kv_dtype, a, grid, st);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // extern "C"
