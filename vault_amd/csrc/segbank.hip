// Segment-memory bookkeeping on the device, so that a decode step and a chunk boundary need no host
// round trip: the token / segment-id ring, the segmenter's running state, and the top-B merge of the
// evicted chunk's candidates into the segment bank.
//
// Reference semantics: the step's segmentation (runtime/vault3.c:2107-2124; src/vault_v3_model.py:
// 2256-2268), the eviction merge update_segment_bank (runtime/vault3.c:1833-1915, quarantine
// :2079-2088; src/vault_v3_model.py:1858-1921, merge_segment_bank_indices :918-949).
//
// Control words (int32, VGX_SEG_*): the bank's entry count, the running segment-id offset, the
// current chunk's segment id and length.  The bank arrays: positions (int64), scores (fp32), tokens
// and global segment ids (int32), in chronological order.
#include "common.h"

using namespace vgx;

namespace {

constexpr int kEvictThreads = 1024;
constexpr int kEvictMaxItems = 4096;     // bank capacity + W candidates held in LDS

// One decode step: ring slot c = step[SLOT] of every sequence gets its token; with seg_cur, the
// single sequence's segment id and the segmenter's break rule.
__global__ void seg_step_kernel(const int64_t *__restrict__ ids, int B, const int32_t *__restrict__ step,
                                int32_t *__restrict__ tok_cur, int64_t ldt, int32_t *__restrict__ seg_cur,
                                int32_t *__restrict__ ctrl, const uint8_t *__restrict__ tiers, int64_t vocab,
                                int seg_min, int seg_max, int W) {
    const int c = step[VGX_STEP_SLOT];
    const int b = threadIdx.x + blockIdx.x * blockDim.x;
    if (b < B) tok_cur[b * ldt + c] = (int32_t)ids[b];
    if (seg_cur != nullptr && b == 0) {
        const int64_t id = ids[0];
        const int tr = (tiers != nullptr && id >= 0 && id < vocab) ? (int)tiers[id] : 0;
        const int t2 = max(seg_min, (seg_max * 2) / 3);
        const int t3 = max(seg_min, seg_max > 8 ? seg_max - 8 : seg_min);
        const int cur = ctrl[VGX_SEG_CUR_ID];
        const int len = ctrl[VGX_SEG_LEN] + 1;
        seg_cur[c] = cur;
        const bool brk = (tr == 1 && len >= seg_min) || (tr == 2 && len >= t2) || (tr == 3 && len >= t3);
        if (c == W - 1 || brk || len >= seg_max) {
            ctrl[VGX_SEG_CUR_ID] = cur + 1;
            ctrl[VGX_SEG_LEN] = 0;
        } else {
            ctrl[VGX_SEG_LEN] = len;
        }
    }
}

__device__ __forceinline__ int f2ord(float f) {      // order-preserving float -> int
    const int i = __float_as_int(f);
    return i >= 0 ? i : i ^ 0x7FFFFFFF;
}
__device__ __forceinline__ float ord2f(int i) { return __int_as_float(i >= 0 ? i : i ^ 0x7FFFFFFF); }

// Exclusive prefix count of `flag` over the block (1024 threads, one value each); returns the
// thread's offset, *total receives the sum.
__device__ int block_scan(int flag, int *sbuf, int *total) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint64_t m = __ballot(flag != 0);
    const int before = __popcll(m & ((1ull << lane) - 1ull));
    if (lane == 0) sbuf[wave] = __popcll(m);
    __syncthreads();
    if (tid == 0) {
        int s = 0;
        for (int w = 0; w < kEvictThreads / 64; ++w) {
            const int v = sbuf[w];
            sbuf[w] = s;
            s += v;
        }
        sbuf[kEvictThreads / 64] = s;
    }
    __syncthreads();
    const int off = sbuf[wave] + before;
    *total = sbuf[kEvictThreads / 64];
    __syncthreads();
    return off;
}

// The eviction merge at a chunk boundary, one workgroup.  Candidates are the tokens t >= t0 of the
// evicted chunk whose segment survives quarantine; every candidate carries its segment's maximum
// score minus 1e-6 (global segment id mod 16384).  Bank entries and candidates (positions ascending)
// compete on (score desc, position asc) for `budget` slots; the winners are written back in
// chronological order, with for every slot j the source row of its keys / values: idx_old[j] = bank
// slot (idx_new[j] = -1), or idx_new[j] = row of the evicted chunk (idx_old[j] = -1); slots past the
// new count get -1 in both.
__global__ __launch_bounds__(kEvictThreads) void seg_evict_kernel(
    float *__restrict__ sc_prev, const int32_t *__restrict__ seg_prev, const int32_t *__restrict__ tok_prev, int W,
    int64_t *__restrict__ mem_pos, float *__restrict__ mem_score, int32_t *__restrict__ mem_tok,
    int32_t *__restrict__ mem_seg, int32_t *__restrict__ ctrl, int64_t ev, int t0, int budget,
    int32_t *__restrict__ idx_old, int32_t *__restrict__ idx_new) {
    __shared__ float s_score[kEvictMaxItems];
    __shared__ int64_t s_pos[kEvictMaxItems];
    __shared__ int32_t s_tok[kEvictMaxItems];
    __shared__ int32_t s_seg[kEvictMaxItems];
    __shared__ int32_t s_src[kEvictMaxItems];     // evicted-chunk row of a candidate
    __shared__ int s_mx[kEvictMaxItems];          // per local segment: max score (ordered int), bad flag
    __shared__ int sbuf[kEvictThreads / 64 + 1];
    __shared__ int s_any_bad, s_nloc;
    const int tid = threadIdx.x;
    const int M = ctrl[VGX_SEG_MEM_CNT];
    const int off = ctrl[VGX_SEG_ID_OFFSET];
    if (tid == 0) {
        s_any_bad = 0;
        s_nloc = 0;
    }
    for (int i = tid; i < W; i += kEvictThreads) s_mx[i] = 0;
    __syncthreads();
    // quarantine: a token scored <= -1e29 marks its whole segment, whose scores become -1e30
    for (int t = tid; t < W; t += kEvictThreads) {
        atomicMax(&s_nloc, seg_prev[t] + 1);
        if (sc_prev[t] <= -1.0e29f) {
            s_any_bad = 1;
            s_mx[seg_prev[t]] = 1;
        }
    }
    __syncthreads();
    if (s_any_bad) {
        for (int t = tid; t < W; t += kEvictThreads)
            if (s_mx[seg_prev[t]]) sc_prev[t] = -1.0e30f;
    }
    __syncthreads();
    for (int i = tid; i < W; i += kEvictThreads) s_mx[i] = f2ord(-3.4e38f);
    __syncthreads();
    for (int t = tid; t < W; t += kEvictThreads) atomicMax(&s_mx[seg_prev[t]], f2ord(sc_prev[t]));
    __syncthreads();
    const int n_loc = s_nloc;
    // the bank, then the candidates in t order
    for (int i = tid; i < M; i += kEvictThreads) {
        s_score[i] = mem_score[i];
        s_pos[i] = mem_pos[i];
        s_tok[i] = mem_tok[i];
        s_seg[i] = mem_seg[i];
        s_src[i] = -1;
    }
    int n_cand = 0;
    for (int t0c = 0; t0c < W; t0c += kEvictThreads) {
        const int t = t0c + tid;
        float smx = 0.0f;
        int ok = 0;
        if (t < W && t >= t0) {
            smx = ord2f(s_mx[seg_prev[t]]);
            ok = smx > -1.0e29f;
        }
        int total;
        const int o = block_scan(ok, sbuf, &total);
        if (ok) {
            const int full = seg_prev[t] + off;
            const int i = M + n_cand + o;
            // two roundings, as the references compute it (no fused multiply-add: the order of
            // near-equal candidates depends on the last bit)
            s_score[i] = __fsub_rn(smx, __fmul_rn(1.0e-6f, (float)(full & 16383)));
            s_pos[i] = ev * (int64_t)W + t;
            s_tok[i] = tok_prev[t];
            s_seg[i] = full;
            s_src[i] = t;
        }
        n_cand += total;
    }
    __syncthreads();
    const int tot = M + n_cand;
    const bool merge = t0 < W;
    // winners: rank by (score desc, index asc) below the budget (all of them when they fit)
    const int n_items = merge ? tot : M;
    int K = 0;
    for (int i0 = 0; i0 < kEvictMaxItems; i0 += kEvictThreads) {
        const int i = i0 + tid;
        int win = 0;
        if (i < n_items) {
            if (!merge || tot <= budget) {
                win = 1;
            } else {
                const float s = s_score[i];
                int rank = 0;
                for (int j = 0; j < tot; ++j) {
                    const float sj = s_score[j];
                    rank += (sj > s) || (sj == s && j < i);
                }
                win = rank < budget;
            }
        }
        int total;
        const int slot = K + block_scan(win, sbuf, &total);
        if (win) {
            mem_pos[slot] = s_pos[i];
            mem_score[slot] = s_score[i];
            mem_tok[slot] = s_tok[i];
            mem_seg[slot] = s_seg[i];
            idx_old[slot] = i < M ? i : -1;
            idx_new[slot] = i < M ? -1 : s_src[i];
        }
        K += total;
    }
    for (int j = K + tid; j < budget; j += kEvictThreads) {
        idx_old[j] = -1;
        idx_new[j] = -1;
    }
    if (tid == 0) {
        ctrl[VGX_SEG_MEM_CNT] = K;
        ctrl[VGX_SEG_ID_OFFSET] = off + n_loc;
    }
}

// Row gather that leaves rows with a negative index untouched.
template <typename T>
__global__ void gather_masked_kernel(const T *__restrict__ src, T *__restrict__ dst, const int32_t *__restrict__ idx,
                                     int64_t src_rows, int64_t n_outer, int64_t sos, int64_t dos, int D) {
    const int64_t j = blockIdx.x;
    const int64_t sr = idx[j];
    if (sr < 0 || sr >= src_rows) return;
    for (int64_t o = blockIdx.y; o < n_outer; o += gridDim.y) {
        const T *s = src + o * sos + sr * D;
        T *d = dst + o * dos + j * D;
        for (int e = threadIdx.x; e < D; e += blockDim.x) d[e] = s[e];
    }
}

// Rotation of rows whose table row depends on a device count m = *dyn: row i uses table row
// (i + row_base - m); with limit, only rows i < m are rotated.
template <int KV>
__global__ void rope_rotate_dyn_kernel(const void *src, void *dst, int64_t n_outer, int64_t sos, int64_t dos, int D,
                                       const float *__restrict__ table, int64_t trs, const int32_t *__restrict__ dyn,
                                       int64_t row_base, int limit) {
    const int64_t i = blockIdx.x;
    const int64_t m = *dyn;
    if (limit && i >= m) return;
    const int h2 = D / 2;
    const float *cs = table + (i + row_base - m) * trs;
    for (int64_t o = blockIdx.y; o < n_outer; o += gridDim.y) {
        const int64_t so = o * sos + i * D, dof = o * dos + i * D;
        for (int p = threadIdx.x; p < h2; p += blockDim.x) {
            const float c = cs[p], s = cs[h2 + p];
            const float a = load_kv<KV>(src, so + p), b = load_kv<KV>(src, so + p + h2);
            store_kv<KV>(dst, dof + p, a * c - b * s);
            store_kv<KV>(dst, dof + p + h2, b * c + a * s);
        }
    }
}

}  // namespace

extern "C" {

int vgx_seg_step(const int64_t *ids, int64_t B, const int32_t *step, int32_t *tok_cur, int64_t tok_ld,
                 int32_t *seg_cur, int32_t *ctrl, const uint8_t *tiers, int64_t vocab, int64_t seg_min,
                 int64_t seg_max, int64_t window, void *stream) {
    if (!ids || !step || !tok_cur) return VGX_E_ARG;
    if (seg_cur && !ctrl) return VGX_E_ARG;
    if (B <= 0 || window <= 0 || tok_ld < window || (seg_cur && (seg_min <= 0 || seg_max < seg_min))) return VGX_E_SIZE;
    if (B > 65535 || window > 0x7FFFFFFF) return VGX_E_LIMIT;
    const int thr = B < 256 ? (int)((B + 63) / 64 * 64) : 256;
    hipLaunchKernelGGL(seg_step_kernel, dim3((unsigned)((B + thr - 1) / thr)), dim3(thr), 0, (hipStream_t)stream, ids,
                       (int)B, step, tok_cur, tok_ld, seg_cur, ctrl, tiers, vocab, (int)seg_min, (int)seg_max,
                       (int)window);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_seg_evict(float *sc_prev, const int32_t *seg_prev, const int32_t *tok_prev, int64_t window, int64_t *mem_pos,
                  float *mem_score, int32_t *mem_tok, int32_t *mem_seg, int32_t *ctrl, int64_t ev_chunk,
                  int64_t t0, int64_t budget, int32_t *idx_old, int32_t *idx_new, void *stream) {
    if (!sc_prev || !seg_prev || !tok_prev || !mem_pos || !mem_score || !mem_tok || !mem_seg || !ctrl || !idx_old ||
        !idx_new)
        return VGX_E_ARG;
    if (window <= 0 || budget <= 0 || t0 < 0 || ev_chunk < 0) return VGX_E_SIZE;
    if (window + budget > kEvictMaxItems) return VGX_E_LIMIT;
    hipLaunchKernelGGL(seg_evict_kernel, dim3(1), dim3(kEvictThreads), 0, (hipStream_t)stream, sc_prev, seg_prev,
                       tok_prev, (int)window, mem_pos, mem_score, mem_tok, mem_seg, ctrl, ev_chunk,
                       (int)std::min<int64_t>(t0, window), (int)budget, idx_old, idx_new);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_gather_rows_masked(int dtype, const void *src, void *dst, const int32_t *idx, int64_t n_idx, int64_t src_rows,
                           int64_t n_outer, int64_t src_ostride, int64_t dst_ostride, int64_t D, void *stream) {
    if (dtype != VGX_F32 && dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!src || !dst || !idx) return VGX_E_ARG;
    if (n_idx < 0 || n_outer < 0 || D <= 0 || src_rows < 0) return VGX_E_SIZE;
    if (n_idx == 0 || n_outer == 0) return VGX_OK;
    if (n_idx > 0x7FFFFFFF) return VGX_E_LIMIT;
    dim3 grid((unsigned)n_idx, (unsigned)std::min<int64_t>(n_outer, 1024));
    const int thr = (int)std::min<int64_t>(256, std::max<int64_t>(32, D));
    hipStream_t st = (hipStream_t)stream;
    if (dtype == VGX_F32)
        hipLaunchKernelGGL(gather_masked_kernel<float>, grid, dim3(thr), 0, st, static_cast<const float *>(src),
                           static_cast<float *>(dst), idx, src_rows, n_outer, src_ostride, dst_ostride, (int)D);
    else
        hipLaunchKernelGGL(gather_masked_kernel<uint16_t>, grid, dim3(thr), 0, st, static_cast<const uint16_t *>(src),
                           static_cast<uint16_t *>(dst), idx, src_rows, n_outer, src_ostride, dst_ostride, (int)D);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_rope_rotate_dyn(int kv_dtype, const void *src, void *dst, int64_t n_outer, int64_t src_ostride,
                        int64_t dst_ostride, int64_t n_rows, int64_t D, const float *table, int64_t table_rstride,
                        const int32_t *dyn, int64_t row_base, int limit_rows, void *stream) {
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!src || !dst || !table || !dyn) return VGX_E_ARG;
    if (n_outer < 0 || n_rows < 0 || D <= 0 || (D & 1)) return VGX_E_SIZE;
    if (n_outer == 0 || n_rows == 0) return VGX_OK;
    if (n_rows > 0x7FFFFFFF) return VGX_E_LIMIT;
    dim3 grid((unsigned)n_rows, (unsigned)std::min<int64_t>(n_outer, 1024));
    const int thr = (int)std::min<int64_t>(256, std::max<int64_t>(32, D / 2));
    hipStream_t st = (hipStream_t)stream;
    if (kv_dtype == VGX_F32)
        hipLaunchKernelGGL(rope_rotate_dyn_kernel<VGX_F32>, grid, dim3(thr), 0, st, src, dst, n_outer, src_ostride,
                           dst_ostride, (int)D, table, table_rstride, dyn, row_base, limit_rows);
    else
        hipLaunchKernelGGL(rope_rotate_dyn_kernel<VGX_BF16>, grid, dim3(thr), 0, st, src, dst, n_outer, src_ostride,
                           dst_ostride, (int)D, table, table_rstride, dyn, row_base, limit_rows);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // extern "C"
