// Next-token selection on the device: argmax and top-k sampling over the logits rows, so that a decode
// loop can feed one step's choice to the next step without reading the logits on the host.
//
// Reference semantics: v3_argmax and v3_sample_topk (runtime/vault3.c:3198-3230); the candidate
// weights use the runtime's own exp arithmetic (ref_expf), so draws select the runtime's index.
//
// Ordering.  A logit l at index i gets the 64-bit key (ord(l) << 32) | (2^32 - 1 - i), ord the
// order-preserving map of the fp32 bits, so that larger keys are larger logits and, among equal
// logits, smaller indices: the order in which the reference's strict comparisons keep candidates.
// NaN logits get key 0 and are never chosen while any other value exists.
#include "common.h"

using namespace vgx;

namespace {

constexpr int kThreads = 1024;
constexpr int kChunk = 4096;         // keys sorted per workgroup in the first top-k pass
constexpr int kMaxK = 64;

__device__ __forceinline__ uint64_t key_of(float v, int64_t i) {
    if (v != v) return 0ull;
    const uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);   // -0 ranks as +0 (they compare equal)
    const uint32_t o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)i);
}
__device__ __forceinline__ int64_t index_of(uint64_t key) { return (int64_t)(0xFFFFFFFFu - (uint32_t)key); }
__device__ __forceinline__ float value_of(uint64_t key) {
    const uint32_t o = (uint32_t)(key >> 32);
    return __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t k) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const uint64_t o = ((uint64_t)__shfl_xor((unsigned)(k >> 32), off, kWave) << 32) |
                           (uint64_t)(unsigned)__shfl_xor((unsigned)k, off, kWave);
        k = o > k ? o : k;
    }
    return k;
}

// One workgroup per row: the largest key.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float *__restrict__ x, int64_t ld, int64_t V,
                                                          int64_t *__restrict__ out) {
    __shared__ uint64_t red[kThreads / 64];
    const int64_t b = blockIdx.x;
    const float *r = x + b * ld;
    uint64_t best = 0;
    for (int64_t i = threadIdx.x; i < V; i += kThreads) {
        const uint64_t k = key_of(r[i], i);
        best = k > best ? k : best;
    }
    best = wave_max_u64(best);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint64_t m = 0;
        for (int w = 0; w < kThreads / 64; ++w) m = red[w] > m ? red[w] : m;
        // every logit NaN: the reference keeps index 0
        out[b] = m == 0 ? 0 : index_of(m);
    }
}

// Bitonic sort of n (a power of two, <= kChunk) keys in LDS, descending.
__device__ void sort_desc(uint64_t *s, int n) {
    for (int size = 2; size <= n; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = threadIdx.x; i < n / 2; i += kThreads) {
                const int lo = 2 * i - (i & (stride - 1));
                const int hi = lo + stride;
                const bool desc = ((lo & size) == 0);
                const uint64_t a = s[lo], c = s[hi];
                if ((a < c) == desc) {
                    s[lo] = c;
                    s[hi] = a;
                }
            }
            __syncthreads();
        }
    }
}

// Pass 1: workgroup (chunk, row) sorts its kChunk keys and keeps the k largest.
__global__ __launch_bounds__(kThreads) void topk_chunk_kernel(const float *__restrict__ x, int64_t ld, int64_t V, int k,
                                                              int n_chunks, uint64_t *__restrict__ cand) {
    __shared__ uint64_t s[kChunk];
    const int64_t b = blockIdx.y;
    const int64_t base = (int64_t)blockIdx.x * kChunk;
    const float *r = x + b * ld;
    for (int i = threadIdx.x; i < kChunk; i += kThreads) {
        const int64_t g = base + i;
        s[i] = g < V ? key_of(r[g], g) : 0ull;
    }
    __syncthreads();
    sort_desc(s, kChunk);
    uint64_t *o = cand + (b * n_chunks + blockIdx.x) * kMaxK;
    for (int i = threadIdx.x; i < kMaxK; i += kThreads) o[i] = i < k ? s[i] : 0ull;
}

// Pass 2: one workgroup per row merges the chunks' candidates, then draws (one thread).
__global__ __launch_bounds__(kThreads) void topk_draw_kernel(const uint64_t *__restrict__ cand, int n_chunks, int k,
                                                             float temp, uint64_t *__restrict__ rng,
                                                             int64_t *__restrict__ out) {
    __shared__ uint64_t s[kChunk];
    const int64_t b = blockIdx.x;
    const int n = n_chunks * kMaxK;
    int p2 = 1;
    while (p2 < n) p2 <<= 1;
    for (int i = threadIdx.x; i < p2; i += kThreads) s[i] = i < n ? cand[b * n + i] : 0ull;
    __syncthreads();
    sort_desc(s, p2);
    if (threadIdx.x != 0) return;
    int cnt = 0;
    while (cnt < k && s[cnt] != 0ull) ++cnt;
    if (cnt == 0) {
        out[b] = 0;
        return;
    }
    const float top = value_of(s[0]);
    float p[kMaxK], sum = 0.0f;
    for (int j = 0; j < cnt; ++j) {
        p[j] = ref_expf((value_of(s[j]) - top) / temp);
        sum += p[j];
    }
    uint64_t xs = rng[b] ? rng[b] : 0x9E3779B97F4A7C15ull;
    xs ^= xs << 13;
    xs ^= xs >> 7;
    xs ^= xs << 17;
    rng[b] = xs;
    float rr = (float)((xs >> 40) & 0xFFFFFFull) / 16777216.0f * sum;
    int64_t pick = index_of(s[cnt - 1]);
    for (int j = 0; j < cnt; ++j) {
        rr -= p[j];
        if (rr <= 0.0f) {
            pick = index_of(s[j]);
            break;
        }
    }
    out[b] = pick;
}

int64_t chunks_of(int64_t V) { return (V + kChunk - 1) / kChunk; }

// Top-T selection: rounds of workgroups that each sort kChunk keys and keep their kKeep largest, the
// first round over the logits, later rounds over the previous round's survivors, until one chunk
// holds them all; that last workgroup writes the indices and values.  Ties keep the smaller index
// first (the key order), so the result is exactly the first T of the row sorted by value desc, index
// asc.  The survivors of a chunk include the row's top T whenever they fall in it (T <= kKeep).
constexpr int kKeep = 256;

template <bool LOGITS>
__global__ __launch_bounds__(kThreads) void select_kernel(const float *__restrict__ x, int64_t ld, int64_t V,
                                                          const uint64_t *__restrict__ in, int64_t n_in,
                                                          uint64_t *__restrict__ out, int64_t n_out_per_row, int T,
                                                          int64_t *__restrict__ idx, float *__restrict__ val) {
    __shared__ uint64_t s[kChunk];
    const int64_t b = blockIdx.y;
    const int64_t base = (int64_t)blockIdx.x * kChunk;
    for (int i = threadIdx.x; i < kChunk; i += kThreads) {
        const int64_t g = base + i;
        if constexpr (LOGITS) s[i] = g < V ? key_of(x[b * ld + g], g) : 0ull;
        else s[i] = g < n_in ? in[b * n_in + g] : 0ull;
    }
    __syncthreads();
    sort_desc(s, kChunk);
    if (idx != nullptr) {
        // the last round: one chunk per row
        for (int i = threadIdx.x; i < T; i += kThreads) {
            const uint64_t k = s[i];
            idx[b * T + i] = k == 0ull ? -1 : index_of(k);
            val[b * T + i] = k == 0ull ? -INFINITY : value_of(k);
        }
        return;
    }
    uint64_t *o = out + b * n_out_per_row + (int64_t)blockIdx.x * kKeep;
    for (int i = threadIdx.x; i < kKeep; i += kThreads) o[i] = s[i];
}

// Keys left per row after each round, and the workspace (two ping-pong survivor buffers).
int64_t select_ws_bytes(int64_t B, int64_t V) {
    const int64_t n1 = chunks_of(V) * kKeep;
    const int64_t n2 = chunks_of(n1) * kKeep;
    return V <= kChunk ? 0 : B * (n1 + (n1 > kChunk ? n2 : 0)) * 8;
}

}  // namespace

extern "C" {

int vgx_argmax(const float *logits, int64_t ld, int64_t B, int64_t V, int64_t *out, void *stream) {
    if (!logits || !out) return VGX_E_ARG;
    if (B <= 0 || V <= 0 || ld < V) return VGX_E_SIZE;
    if (B > 0x7FFFFFFF || V > 0xFFFFFFFFll) return VGX_E_LIMIT;
    hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)B), dim3(kThreads), 0, (hipStream_t)stream, logits, ld, V, out);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int64_t vgx_sample_topk_workspace_bytes(int64_t B, int64_t V) {
    if (B <= 0 || V <= 0) return VGX_E_SIZE;
    return B * chunks_of(V) * kMaxK * 8;
}

int vgx_sample_topk(const float *logits, int64_t ld, int64_t B, int64_t V, int64_t k, float temp, uint64_t *rng,
                    int64_t *out, void *workspace, int64_t workspace_bytes, void *stream) {
    if (!(temp > 0.0f) || k <= 1) return vgx_argmax(logits, ld, B, V, out, stream);
    if (!logits || !out || !rng) return VGX_E_ARG;
    if (B <= 0 || V <= 0 || ld < V) return VGX_E_SIZE;
    if (k > kMaxK) k = kMaxK;
    const int64_t nc = chunks_of(V);
    if (nc * kMaxK > kChunk) return VGX_E_LIMIT;     // V up to 262144
    if (B > 65535) return VGX_E_LIMIT;
    if (!workspace || workspace_bytes < vgx_sample_topk_workspace_bytes(B, V)) return VGX_E_ARENA;
    hipStream_t st = (hipStream_t)stream;
    auto *cand = static_cast<uint64_t *>(workspace);
    hipLaunchKernelGGL(topk_chunk_kernel, dim3((unsigned)nc, (unsigned)B), dim3(kThreads), 0, st, logits, ld, V, (int)k,
                       (int)nc, cand);
    VGX_CHECK_LAUNCH();
    hipLaunchKernelGGL(topk_draw_kernel, dim3((unsigned)B), dim3(kThreads), 0, st, cand, (int)nc, (int)k, temp, rng, out);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int64_t vgx_topk_workspace_bytes(int64_t B, int64_t V, int64_t T) {
    if (B <= 0 || V <= 0 || T <= 0 || T > kKeep) return VGX_E_SIZE;
    return select_ws_bytes(B, V);
}

int vgx_topk(const float *logits, int64_t ld, int64_t B, int64_t V, int64_t T, int64_t *idx, float *val,
             void *workspace, int64_t workspace_bytes, void *stream) {
    if (!logits || !idx || !val) return VGX_E_ARG;
    if (B <= 0 || V <= 0 || T <= 0 || ld < V) return VGX_E_SIZE;
    if (T > kKeep || B > 65535 || V > 0xFFFFFFFFll) return VGX_E_LIMIT;
    // rows of at most two rounds of survivors: V up to 16 x 16 chunks of 4096 keys
    if (chunks_of(chunks_of(V) * kKeep) * kKeep > kChunk) return VGX_E_LIMIT;
    const int64_t need = select_ws_bytes(B, V);
    if (need > 0 && (!workspace || workspace_bytes < need)) return VGX_E_ARENA;
    hipStream_t st = (hipStream_t)stream;
    if (V <= kChunk) {
        hipLaunchKernelGGL(select_kernel<true>, dim3(1, (unsigned)B), dim3(kThreads), 0, st, logits, ld, V,
                           (const uint64_t *)nullptr, (int64_t)0, (uint64_t *)nullptr, (int64_t)0, (int)T, idx, val);
        VGX_CHECK_LAUNCH();
        return VGX_OK;
    }
    auto *s1 = static_cast<uint64_t *>(workspace);
    const int64_t n1 = chunks_of(V) * kKeep;
    hipLaunchKernelGGL(select_kernel<true>, dim3((unsigned)chunks_of(V), (unsigned)B), dim3(kThreads), 0, st, logits,
                       ld, V, (const uint64_t *)nullptr, (int64_t)0, s1, n1, (int)T, (int64_t *)nullptr,
                       (float *)nullptr);
    VGX_CHECK_LAUNCH();
    const uint64_t *last = s1;
    int64_t n_last = n1;
    if (n1 > kChunk) {
        uint64_t *s2 = s1 + B * n1;
        const int64_t n2 = chunks_of(n1) * kKeep;
        hipLaunchKernelGGL(select_kernel<false>, dim3((unsigned)chunks_of(n1), (unsigned)B), dim3(kThreads), 0, st,
                           (const float *)nullptr, (int64_t)0, (int64_t)0, s1, n1, s2, n2, (int)T, (int64_t *)nullptr,
                           (float *)nullptr);
        VGX_CHECK_LAUNCH();
        last = s2;
        n_last = n2;
    }
    hipLaunchKernelGGL(select_kernel<false>, dim3(1, (unsigned)B), dim3(kThreads), 0, st, (const float *)nullptr,
                       (int64_t)0, (int64_t)0, last, n_last, (uint64_t *)nullptr, (int64_t)0, (int)T, idx, val);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // extern "C"
