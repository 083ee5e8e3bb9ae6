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
#include <string.h>

#include "qgemv.h"

using namespace vgx;

namespace {

constexpr int kEvictThreads = 1024;
constexpr int kEvictMaxItems = 4096;     // bank capacity + W candidates held in LDS

// The segmenter's step for the single sequence's token id at ring slot c: its segment id, then the
// break rule by the token's tier.
// cur / len0: the segmenter's words (ctrl[VGX_SEG_CUR_ID], ctrl[VGX_SEG_LEN]) as read before the call.
__device__ void segment_token(int64_t id, int c, int32_t *__restrict__ seg_cur, int32_t *__restrict__ ctrl, int cur,
                              int len0, const uint8_t *__restrict__ tiers, int64_t vocab, int seg_min, int seg_max,
                              int W) {
    const int tr = (tiers != nullptr && id >= 0 && id < vocab) ? (int)tiers[id] : 0;
    const int t2 = max(seg_min, (seg_max * 2) / 3);
    const int t3 = max(seg_min, seg_max > 8 ? seg_max - 8 : seg_min);
    const int len = len0 + 1;
    seg_cur[c] = cur;
    const bool brk = (tr == 1 && len >= seg_min) || (tr == 2 && len >= t2) || (tr == 3 && len >= t3);
    if (c == W - 1 || brk || len >= seg_max) {
        ctrl[VGX_SEG_CUR_ID] = cur + 1;
        ctrl[VGX_SEG_LEN] = 0;
    } else {
        ctrl[VGX_SEG_LEN] = len;
    }
}

// One decode step: ring slot c = step[SLOT] of every sequence gets its token; with seg_cur, the
// single sequence's segment id and the segmenter's break rule.
__global__ void seg_step_kernel(const int64_t *__restrict__ ids, int B, const int32_t *__restrict__ step,
                                int32_t *__restrict__ tok_cur, int64_t ldt, int32_t *__restrict__ seg_cur,
                                int32_t *__restrict__ ctrl, const uint8_t *__restrict__ tiers, int64_t vocab,
                                int seg_min, int seg_max, int W) {
    const int c = step[VGX_STEP_SLOT];
    const int b = threadIdx.x + blockIdx.x * blockDim.x;
    if (b < B) tok_cur[b * ldt + c] = (int32_t)ids[b];
    if (seg_cur != nullptr && b == 0)
        segment_token(ids[0], c, seg_cur, ctrl, ctrl[VGX_SEG_CUR_ID], ctrl[VGX_SEG_LEN], tiers, vocab, seg_min, seg_max, W);
}

// Loads of the pinned host ring at system scope: they reach the host's latest writes through no
// stale cache line, whatever the ring's earlier use of the same slot left in the device caches.
template <typename T>
__device__ __forceinline__ T sys_load(const void *p) {
    return __hip_atomic_load(static_cast<T *>(const_cast<void *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

constexpr int kBeginThreads = 256;
constexpr int kBeginSpecSlots = 16;        // rings of up to this many slots: every slot's words read at once
constexpr int kBeginBiasUnroll = 4;        // bias entries per thread whose host loads are in flight together

struct StepBeginArgs {
    const uint8_t *ring;
    int64_t n_slots, slot_bytes, bias_off;
    int32_t *counter, *step;
    int64_t *ids;
    int B;
    int64_t *out_ref;
    int32_t *tok_cur;
    int64_t ldt;
    int32_t *seg_cur, *ctrl;
    const uint8_t *tiers;
    int64_t vocab;
    int seg_min, seg_max, W;
    float *bias_early, *bias_late;
    int H;
    int64_t bias_ld;
    int bias_cap;
    // the embedding rows of the step's ids (vgx_step_begin_embed), or emb == nullptr
    const uint8_t *emb;
    int emb_dt;
    int64_t emb_rows, emb_nblk, emb_soff, emb_ldo;
    float *emb_out;
};

// One workgroup.  Every host load of the slot (header, host ids, bias row indices and vectors) is
// issued before any is used, so the step pays one host round trip; device ids are one more (device)
// load.  The counter advances after every thread has read it.
__global__ __launch_bounds__(kBeginThreads) void step_begin_kernel(StepBeginArgs a) {
    // The counter, the words and ids of every slot (rings of up to kBeginSpecSlots slots with
    // B * n_slots <= kBeginThreads ids) and the segmenter's words are requested together: one host
    // round trip, then the counter picks the slot.  Larger rings read the picked slot afterwards.
    __shared__ int64_t s_hdr[kBeginSpecSlots][4];
    __shared__ int64_t s_id[kBeginThreads];
    __shared__ int32_t s_flags[kBeginSpecSlots];
    __shared__ int s_k;
    const int tid = threadIdx.x;
    const bool spec = a.n_slots <= kBeginSpecSlots;
    const bool spec_ids = spec && a.B * a.n_slots <= kBeginThreads;
    if (tid == 0) s_k = *a.counter;
    int seg_cur_id = 0, seg_len = 0;
    if (tid == 0 && a.seg_cur != nullptr) {
        seg_cur_id = a.ctrl[VGX_SEG_CUR_ID];
        seg_len = a.ctrl[VGX_SEG_LEN];
    }
    if (spec && tid < a.n_slots) {
        const uint8_t *sl = a.ring + (int64_t)tid * a.slot_bytes;
        s_hdr[tid][0] = sys_load<int64_t>(sl + VGX_SLOT_STEP);
        s_hdr[tid][1] = sys_load<int64_t>(sl + VGX_SLOT_STEP + 8);
        s_hdr[tid][2] = sys_load<int64_t>(sl + VGX_SLOT_IDS_ADDR);
        s_hdr[tid][3] = sys_load<int64_t>(sl + VGX_SLOT_OUT_ADDR);
        s_flags[tid] = sys_load<int32_t>(sl + VGX_SLOT_FLAGS);
    }
    if (spec_ids && tid < a.B * a.n_slots)
        s_id[tid] = sys_load<int64_t>(a.ring + (int64_t)(tid / a.B) * a.slot_bytes + VGX_SLOT_IDS + 8 * (tid % a.B));
    __syncthreads();
    const uint32_t k = (uint32_t)s_k % (uint32_t)a.n_slots;   // in range whatever the word holds
    const uint8_t *slot = a.ring + (int64_t)k * a.slot_bytes;
    int64_t h0, h1, ids_addr, out_addr;
    int32_t flags;
    if (spec) {
        h0 = s_hdr[k][0];
        h1 = s_hdr[k][1];
        ids_addr = s_hdr[k][2];
        out_addr = s_hdr[k][3];
        flags = s_flags[k];
    } else {
        h0 = sys_load<int64_t>(slot + VGX_SLOT_STEP);
        h1 = sys_load<int64_t>(slot + VGX_SLOT_STEP + 8);
        flags = sys_load<int32_t>(slot + VGX_SLOT_FLAGS);
        ids_addr = sys_load<int64_t>(slot + VGX_SLOT_IDS_ADDR);
        out_addr = sys_load<int64_t>(slot + VGX_SLOT_OUT_ADDR);
    }
    int64_t hid = 0;
    if (tid < a.B) hid = spec_ids ? s_id[(int)k * a.B + tid] : sys_load<int64_t>(slot + VGX_SLOT_IDS + 8 * tid);
    const bool bias = a.bias_early != nullptr;
    int8_t rows[2] = {-1, -1};
    if (bias && tid < a.H) {
        rows[0] = sys_load<int8_t>(slot + a.bias_off + tid);
        rows[1] = sys_load<int8_t>(slot + a.bias_off + a.H + tid);
    }
    const int32_t w[VGX_STEP_WORDS] = {(int32_t)h0, (int32_t)(h0 >> 32), (int32_t)h1, (int32_t)(h1 >> 32)};
    if (tid < VGX_STEP_WORDS) a.step[tid] = w[tid];
    if (tid == 0 && a.out_ref != nullptr) *a.out_ref = out_addr;
    const int c = w[VGX_STEP_SLOT];
    const int64_t *dev_ids = reinterpret_cast<const int64_t *>(ids_addr);
    const bool on_dev = (flags & VGX_SLOTF_DEVICE_IDS) != 0;
    for (int b = tid; b < a.B && (uint32_t)c < (uint32_t)a.W; b += kBeginThreads) {   // a slot outside the ring: no write
        const int64_t id = on_dev ? dev_ids[b] : (b == tid ? hid : sys_load<int64_t>(slot + VGX_SLOT_IDS + 8 * b));
        a.ids[b] = id;
        a.tok_cur[b * a.ldt + c] = (int32_t)id;
        if (a.seg_cur != nullptr && b == 0)
            segment_token(id, c, a.seg_cur, a.ctrl, seg_cur_id, seg_len, a.tiers, a.vocab, a.seg_min, a.seg_max, a.W);
    }
    if (bias && (flags & VGX_SLOTF_BIAS)) {
        __shared__ int8_t s_rows[2][256];
        if (tid < a.H) {
            s_rows[0][tid] = rows[0];
            s_rows[1][tid] = rows[1];
        }
        __syncthreads();
        const float *v = reinterpret_cast<const float *>(slot + a.bias_off + ((2 * a.H + 15) / 16) * 16);
        // entries m0 + t, m0 + t + 256, ... of the three vectors: all their host loads in flight at once
        for (int m0 = 0; m0 < a.bias_cap; m0 += kBeginThreads * kBeginBiasUnroll) {
            float vec[kBeginBiasUnroll][3];
#pragma unroll
            for (int u = 0; u < kBeginBiasUnroll; ++u) {
                const int m = m0 + tid + u * kBeginThreads;
#pragma unroll
                for (int r = 0; r < 3; ++r) vec[u][r] = m < a.bias_cap ? sys_load<float>(v + r * a.bias_cap + m) : 0.0f;
            }
            for (int h = 0; h < a.H; ++h) {
                const int re = s_rows[0][h], rl = s_rows[1][h];
#pragma unroll
                for (int u = 0; u < kBeginBiasUnroll; ++u) {
                    const int m = m0 + tid + u * kBeginThreads;
                    if (m < a.bias_cap) {
                        float e = 0.0f, l = 0.0f;
#pragma unroll
                        for (int r = 0; r < 3; ++r) {
                            e = re == r ? vec[u][r] : e;
                            l = rl == r ? vec[u][r] : l;
                        }
                        a.bias_early[h * a.bias_ld + m] = e;
                        a.bias_late[h * a.bias_ld + m] = l;
                    }
                }
            }
        }
    }
    __syncthreads();
    if (tid == 0) *a.counter = (int32_t)((k + 1) % (uint32_t)a.n_slots);
    if (a.emb != nullptr) {
        // the embedding rows of the ids just written (visible to the workgroup after the barrier), one
        // thread per 32-element block, as vgx_embed_rows with pad row 0
        for (int t = tid; t < a.B * a.emb_nblk; t += kBeginThreads) {
            const int b = (int)(t / a.emb_nblk);
            const int64_t blk = t - (int64_t)b * a.emb_nblk;
            int64_t r = a.ids[b];
            if (r < 0 || r >= a.emb_rows) r = 0;
            float *o = a.emb_out + b * a.emb_ldo + blk * QK;
            switch (a.emb_dt) {
                case VGX_Q8_0: dequant_block<VGX_Q8_0>(a.emb, a.emb_nblk, a.emb_soff, r, blk, o); break;
                case VGX_Q4_0: dequant_block<VGX_Q4_0>(a.emb, a.emb_nblk, a.emb_soff, r, blk, o); break;
                case VGX_F32: dequant_block<VGX_F32>(a.emb, a.emb_nblk, a.emb_soff, r, blk, o); break;
                case VGX_BF16: dequant_block<VGX_BF16>(a.emb, a.emb_nblk, a.emb_soff, r, blk, o); break;
                default: dequant_block<VGX_F16>(a.emb, a.emb_nblk, a.emb_soff, r, blk, o); break;
            }
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
    __shared__ int s_mx[kEvictMaxItems];          // per local segment: max score (ordered int), bad flag;
                                                  // then the winner flags
    __shared__ uint64_t s_key[kEvictMaxItems];    // (score desc, index asc) sort keys
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
    // winners: the first `budget` items in (score desc, index asc) order (all of them when they fit):
    // a bitonic sort of 64-bit keys in LDS, the score's order-preserving bits inverted above the index
    // (-0 counts as +0, NaN scores sort last), then a flag per winning item
    const int n_items = merge ? tot : M;
    const bool rank = merge && tot > budget;
    if (rank) {
        int np = 1;
        while (np < tot) np <<= 1;
        for (int i = tid; i < np; i += kEvictThreads) {
            uint64_t key = ~0ull;
            if (i < tot) {
                const float f = s_score[i] + 0.0f;
                const uint32_t hi = f != f ? 0xFFFFFFFFu : (uint32_t)((int64_t)0x7FFFFFFF - (int64_t)f2ord(f));
                key = ((uint64_t)hi << 32) | (uint32_t)i;
            }
            s_key[i] = key;
        }
        __syncthreads();
        for (int k = 2; k <= np; k <<= 1) {
            for (int j = k >> 1; j > 0; j >>= 1) {
                for (int i = tid; i < np; i += kEvictThreads) {
                    const int l = i ^ j;
                    if (l > i) {
                        const uint64_t a = s_key[i], b = s_key[l];
                        if (((i & k) == 0) == (a > b)) {
                            s_key[i] = b;
                            s_key[l] = a;
                        }
                    }
                }
                __syncthreads();
            }
        }
        for (int i = tid; i < tot; i += kEvictThreads) s_mx[i] = 0;
        __syncthreads();
        for (int p = tid; p < budget; p += kEvictThreads) s_mx[(int)(s_key[p] & 0xFFFFFFFFu)] = 1;
        __syncthreads();
    }
    int K = 0;
    for (int i0 = 0; i0 < kEvictMaxItems; i0 += kEvictThreads) {
        const int i = i0 + tid;
        int win = 0;
        if (i < n_items) win = rank ? s_mx[i] : 1;
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

int64_t vgx_step_slot_bias_off(int64_t B) { return B < 0 ? -1 : VGX_SLOT_IDS + (8 * B + 15) / 16 * 16; }

int64_t vgx_step_slot_bytes(int64_t B, int64_t n_heads, int64_t bias_cap) {
    if (B < 0 || n_heads < 0 || bias_cap < 0) return -1;
    int64_t n = vgx_step_slot_bias_off(B);
    if (bias_cap > 0) n += (2 * n_heads + 15) / 16 * 16 + 3 * 4 * bias_cap;
    return (n + 255) / 256 * 256;
}

int vgx_host_alloc(int64_t bytes, void **ptr) {
    if (!ptr) return VGX_E_ARG;
    *ptr = nullptr;
    if (bytes <= 0) return VGX_E_SIZE;
    void *p = nullptr;
    if (hipHostMalloc(&p, (size_t)bytes, hipHostMallocCoherent | hipHostMallocMapped) != hipSuccess) return VGX_E_HIP;
    void *d = nullptr;
    if (hipHostGetDevicePointer(&d, p, 0) != hipSuccess || d != p) {   // the device must see the same address
        (void)hipHostFree(p);
        return VGX_E_HIP;
    }
    memset(p, 0, (size_t)bytes);
    *ptr = p;
    return VGX_OK;
}

int vgx_host_free(void *ptr) {
    if (!ptr) return VGX_OK;
    return hipHostFree(ptr) == hipSuccess ? VGX_OK : VGX_E_HIP;
}

int vgx_step_begin_embed(const void *ring, int64_t n_slots, int64_t slot_bytes, int32_t *counter, int32_t *step,
                         int64_t *ids, int64_t B, int64_t *out_ref, int32_t *tok_cur, int64_t tok_ld, int32_t *seg_cur,
                         int32_t *ctrl, const uint8_t *tiers, int64_t vocab, int64_t seg_min, int64_t seg_max,
                         int64_t window, float *bias_early, float *bias_late, int64_t n_heads, int64_t bias_ld,
                         int64_t bias_cap, int emb_dtype, const void *emb_packed, int64_t emb_rows, int64_t emb_cols,
                         float *emb_out, int64_t emb_ldo, void *stream) {
    if (emb_packed != nullptr) {
        if (emb_dtype != VGX_Q8_0 && emb_dtype != VGX_Q4_0 && emb_dtype != VGX_F32 && emb_dtype != VGX_BF16 &&
            emb_dtype != VGX_F16)
            return VGX_E_DTYPE;
        if (!emb_out) return VGX_E_ARG;
        if (emb_rows <= 0 || emb_cols <= 0 || emb_ldo < emb_cols) return VGX_E_SIZE;
        if (emb_cols % QK) return VGX_E_SHAPE;
    }
    if (!ring || !counter || !step || !ids || !tok_cur) return VGX_E_ARG;
    if (seg_cur && !ctrl) return VGX_E_ARG;
    if ((bias_early == nullptr) != (bias_late == nullptr)) return VGX_E_ARG;
    if (reinterpret_cast<uintptr_t>(ring) % 256 || reinterpret_cast<uintptr_t>(out_ref) % 8 ||
        reinterpret_cast<uintptr_t>(ids) % 8)
        return VGX_E_ALIGN;
    if (B <= 0 || n_slots <= 0 || window <= 0 || tok_ld < window ||
        (seg_cur && (seg_min <= 0 || seg_max < seg_min)))
        return VGX_E_SIZE;
    if (bias_early && (n_heads <= 0 || bias_cap <= 0 || bias_ld < bias_cap)) return VGX_E_SIZE;
    if (B > kBeginThreads * 64 || window > 0x7FFFFFFF || n_slots > (1 << 20) ||
        (bias_early && (n_heads > 256 || bias_cap > (1 << 24))))
        return VGX_E_LIMIT;
    if (slot_bytes % 256 || slot_bytes < vgx_step_slot_bytes(B, bias_early ? n_heads : 0, bias_early ? bias_cap : 0))
        return VGX_E_SIZE;
    StepBeginArgs a{};
    a.ring = static_cast<const uint8_t *>(ring);
    a.n_slots = n_slots;
    a.slot_bytes = slot_bytes;
    a.bias_off = vgx_step_slot_bias_off(B);
    a.counter = counter;
    a.step = step;
    a.ids = ids;
    a.B = (int)B;
    a.out_ref = out_ref;
    a.tok_cur = tok_cur;
    a.ldt = tok_ld;
    a.seg_cur = seg_cur;
    a.ctrl = ctrl;
    a.tiers = tiers;
    a.vocab = vocab;
    a.seg_min = (int)seg_min;
    a.seg_max = (int)seg_max;
    a.W = (int)window;
    a.bias_early = bias_early;
    a.bias_late = bias_late;
    a.H = (int)n_heads;
    a.bias_ld = bias_ld;
    a.bias_cap = (int)bias_cap;
    if (emb_packed != nullptr) {
        a.emb = static_cast<const uint8_t *>(emb_packed);
        a.emb_dt = emb_dtype;
        a.emb_rows = emb_rows;
        a.emb_nblk = emb_cols / QK;
        a.emb_soff = gemv_plain(emb_dtype) ? 0 : vgx_qweight_scale_offset(emb_dtype, emb_rows, emb_cols);
        a.emb_out = emb_out;
        a.emb_ldo = emb_ldo;
    }
    hipLaunchKernelGGL(step_begin_kernel, dim3(1), dim3(kBeginThreads), 0, (hipStream_t)stream, a);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_step_begin(const void *ring, int64_t n_slots, int64_t slot_bytes, int32_t *counter, int32_t *step, int64_t *ids,
                   int64_t B, int64_t *out_ref, int32_t *tok_cur, int64_t tok_ld, int32_t *seg_cur, int32_t *ctrl,
                   const uint8_t *tiers, int64_t vocab, int64_t seg_min, int64_t seg_max, int64_t window,
                   float *bias_early, float *bias_late, int64_t n_heads, int64_t bias_ld, int64_t bias_cap,
                   void *stream) {
    return vgx_step_begin_embed(ring, n_slots, slot_bytes, counter, step, ids, B, out_ref, tok_cur, tok_ld, seg_cur,
                                ctrl, tiers, vocab, seg_min, seg_max, window, bias_early, bias_late, n_heads, bias_ld,
                                bias_cap, 0, nullptr, 0, 0, nullptr, 0, stream);
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
