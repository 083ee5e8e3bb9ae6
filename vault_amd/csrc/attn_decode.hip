// Split-K GQA decode attention over up to four key spans (sink | segment memory | prev | cur).
//
// Reference semantics: src/vault_v3_model.py:1098-1136 (concat spans, _expand_kv, optional fp32
// bias on the segment span, softmax, P V) and runtime/vault3.c:1958-2032 (attn_run).
//
// Mapping.  One workgroup = kWaves waves = one (batch b, kv group g, key split).  Every wave holds
// the GRP query heads of group g, so each K/V row is fetched once for all GRP heads (the reference
// re-reads K/V per head).  The split's keys are dealt to the waves in 16-key tiles; inside a wave
// the 4 DPP rows (16 lanes each) take 4 keys of the tile each, one key row spread over the 16 lanes
// of a DPP row (D/16 contiguous elements per lane: one 128-bit load for bf16 D=128, two for fp32),
// so one load instruction fetches four whole key rows.  q.k partials are reduced over the 16 lanes
// with DPP; every DPP row keeps its own online-softmax state (m, l, acc).  The states are merged
// across DPP rows with lane shuffles and across the waves of the workgroup through LDS; with more
// than one split, each split writes (m, l, acc) partials to the workspace and attn_merge_kernel
// combines them (a second launch: merging inside the first kernel would need a device-scope
// release fence per workgroup, an L2 write-back that measured 2x slower at batch 64).
#include "common.h"

using namespace vgx;

namespace {

constexpr int kKB = 4;       // keys per DPP row per 16-key tile
constexpr int kWaves = 4;    // waves per workgroup
constexpr int kMinKeysPerWave = 16;
constexpr int kTargetWaves = 2048;
constexpr int kMaxSplits = 64;
constexpr float kNegBig = -1.0e30f;

struct SpanArgs {
    const void *k[4];
    const void *v[4];
    int64_t len[4];
    int64_t bstride[4];
    int64_t gstride[4];
    const int32_t *dyn_len[4];
    int n;
};

template <int KV, int DPL>
__device__ __forceinline__ void load_chunk(const void *base, int64_t elem_off, float (&out)[DPL]) {
    if constexpr (KV == VGX_F32) {
        const float *p = static_cast<const float *>(base) + elem_off;
        if constexpr (DPL % 4 == 0) {
#pragma unroll
            for (int i = 0; i < DPL / 4; ++i) {
                const float4 t = reinterpret_cast<const float4 *>(p)[i];
                out[4 * i] = t.x; out[4 * i + 1] = t.y; out[4 * i + 2] = t.z; out[4 * i + 3] = t.w;
            }
        } else {
#pragma unroll
            for (int i = 0; i < DPL; ++i) out[i] = p[i];
        }
    } else {
        const uint16_t *p = static_cast<const uint16_t *>(base) + elem_off;
        if constexpr (DPL == 8) {
            const uint4 t = *reinterpret_cast<const uint4 *>(p);
            const uint32_t w[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                out[2 * i] = __uint_as_float(w[i] << 16);
                out[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
            }
        } else if constexpr (DPL == 4) {
            const uint2 t = *reinterpret_cast<const uint2 *>(p);
            out[0] = __uint_as_float(t.x << 16); out[1] = __uint_as_float(t.x & 0xFFFF0000u);
            out[2] = __uint_as_float(t.y << 16); out[3] = __uint_as_float(t.y & 0xFFFF0000u);
        } else {
#pragma unroll
            for (int i = 0; i < DPL; ++i) out[i] = __uint_as_float((uint32_t)p[i] << 16);
        }
    }
}

// Workspace layout: partials per (b, g, split, head): D accumulators, then m, l.

template <int KV, int GRP, int DPL>
__global__ __launch_bounds__(64 * kWaves) void attn_decode_kernel(
    const float *__restrict__ q, int64_t ldq, SpanArgs sp, const float *__restrict__ bias, int64_t bias_hstride,
    int bias_span, float *__restrict__ out, float *__restrict__ part, int H, int G,
    float scale, int64_t n_tot, int64_t kps, int n_splits, int64_t causal_base) {
    constexpr int D = DPL * 16;
    constexpr int SLOT = D + 2;
    __shared__ float red[kWaves][GRP][SLOT];

    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l16 = lane & 15, row = lane >> 4;

    float qr[GRP][DPL];
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        const float *qp = q + (int64_t)b * ldq + ((int64_t)g * GRP + hh) * D + l16 * DPL;
#pragma unroll
        for (int d = 0; d < DPL; ++d) qr[hh][d] = qp[d] * scale;
    }
    float m[GRP], l[GRP], acc[GRP][DPL];
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        m[hh] = kNegBig;
        l[hh] = 0.0f;
#pragma unroll
        for (int d = 0; d < DPL; ++d) acc[hh][d] = 0.0f;
    }

    const int64_t k0 = (int64_t)split * kps;
    const int64_t k1 = min(n_tot, k0 + kps);
    int64_t base = 0;
    for (int s = 0; s < sp.n; ++s) {
        const int64_t len = sp.len[s];
        const int64_t lo = max(k0, base) - base;
        int64_t hi = min(k1, base + len) - base;
        if (sp.dyn_len[s] != nullptr) hi = min(hi, (int64_t)*sp.dyn_len[s]);  // device-side length
        // Causal last span: batch entry b sees its first causal_base + b + 1 keys.
        if (causal_base >= 0 && s == sp.n - 1) hi = min(hi, causal_base + (int64_t)b + 1);
        base += len;
        if (lo >= hi) continue;
        const int64_t off = (int64_t)b * sp.bstride[s] + (int64_t)g * sp.gstride[s] + l16 * DPL;
        const void *kb = sp.k[s];
        const void *vb = sp.v[s];
        const float *bb = (bias != nullptr && s == bias_span) ? bias + (int64_t)g * GRP * bias_hstride : nullptr;
        for (int64_t t0 = lo + wave * 4 * kKB; t0 < hi; t0 += kWaves * 4 * kKB) {
            float kf[kKB][DPL], vf[kKB][DPL];
            bool valid[kKB];
#pragma unroll
            for (int j = 0; j < kKB; ++j) {
                const int64_t key = t0 + row * kKB + j;
                valid[j] = key < hi;
                if (valid[j]) {
                    load_chunk<KV, DPL>(kb, off + key * D, kf[j]);
                    load_chunk<KV, DPL>(vb, off + key * D, vf[j]);
                } else {
#pragma unroll
                    for (int d = 0; d < DPL; ++d) { kf[j][d] = 0.0f; vf[j][d] = 0.0f; }
                }
            }
            float sc[GRP][kKB];
#pragma unroll
            for (int j = 0; j < kKB; ++j)
#pragma unroll
                for (int hh = 0; hh < GRP; ++hh) {
                    float p = 0.0f;
#pragma unroll
                    for (int d = 0; d < DPL; ++d) p = fmaf(qr[hh][d], kf[j][d], p);
                    sc[hh][j] = row16_sum(p);
                }
#pragma unroll
            for (int j = 0; j < kKB; ++j) {
                const int64_t key = t0 + row * kKB + j;
#pragma unroll
                for (int hh = 0; hh < GRP; ++hh) {
                    float v = sc[hh][j];
                    if (bb != nullptr && valid[j]) v += bb[hh * bias_hstride + key];
                    sc[hh][j] = valid[j] ? v : -INFINITY;
                }
            }
#pragma unroll
            for (int hh = 0; hh < GRP; ++hh) {
                float mb = sc[hh][0];
#pragma unroll
                for (int j = 1; j < kKB; ++j) mb = fmaxf(mb, sc[hh][j]);
                const float mn = fmaxf(m[hh], mb);
                const float corr = __expf(m[hh] - mn);
                m[hh] = mn;
                float ls = l[hh] * corr;
#pragma unroll
                for (int j = 0; j < kKB; ++j) {
                    const float p = __expf(sc[hh][j] - mn);
                    sc[hh][j] = p;
                    ls += p;
                }
                l[hh] = ls;
#pragma unroll
                for (int d = 0; d < DPL; ++d) {
                    float a = acc[hh][d] * corr;
#pragma unroll
                    for (int j = 0; j < kKB; ++j) a = fmaf(sc[hh][j], vf[j][d], a);
                    acc[hh][d] = a;
                }
            }
        }
    }

    // Merge the online-softmax states of the four DPP rows of the wave.
#pragma unroll
    for (int sh = 16; sh <= 32; sh <<= 1) {
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
            const float mo = __shfl_xor(m[hh], sh, kWave);
            const float lo = __shfl_xor(l[hh], sh, kWave);
            const float mn = fmaxf(m[hh], mo);
            const float c1 = __expf(m[hh] - mn), c2 = __expf(mo - mn);
            l[hh] = l[hh] * c1 + lo * c2;
#pragma unroll
            for (int d = 0; d < DPL; ++d) {
                const float ao = __shfl_xor(acc[hh][d], sh, kWave);
                acc[hh][d] = acc[hh][d] * c1 + ao * c2;
            }
            m[hh] = mn;
        }
    }
    if (row == 0) {
#pragma unroll
        for (int hh = 0; hh < GRP; ++hh) {
#pragma unroll
            for (int d = 0; d < DPL; ++d) red[wave][hh][l16 * DPL + d] = acc[hh][d];
            if (l16 == 0) {
                red[wave][hh][D] = m[hh];
                red[wave][hh][D + 1] = l[hh];
            }
        }
    }
    __syncthreads();

    // Merge the waves: thread t owns (head t / D, dim t % D).
    const int64_t pair = (int64_t)b * G + g;
    for (int t = threadIdx.x; t < GRP * D; t += 64 * kWaves) {
        const int hh = t / D, d = t - hh * D;
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, red[w][hh][D]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float c = __expf(red[w][hh][D] - M);
            L = fmaf(c, red[w][hh][D + 1], L);
            A = fmaf(c, red[w][hh][d], A);
        }
        if (n_splits == 1) {
            out[((int64_t)b * H + (int64_t)g * GRP + hh) * D + d] = A / L;
        } else {
            float *pp = part + ((pair * n_splits + split) * GRP + hh) * SLOT;
            pp[d] = A;
            if (d == 0) {
                pp[D] = M;
                pp[D + 1] = L;
            }
        }
    }
}

// One workgroup of D threads per (b, h): out = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s.
// Every load is issued before the one barrier: thread d requests acc_s[d] of all n_splits splits, and
// the first wave also (m_s, l_s) of split s = lane; that wave turns them into the split weights in
// LDS.  One round trip to the partials instead of one per dependent step.
__global__ __launch_bounds__(128) void attn_merge_kernel(const float *__restrict__ part, float *__restrict__ out,
                                                         int H, int G, int D, int n_splits) {
    __shared__ float wgt[kMaxSplits];
    __shared__ float inv_l;
    const int bh = blockIdx.x;
    const int b = bh / H, h = bh - b * H;
    const int grp = H / G, g = h / grp, hh = h - g * grp;
    const int64_t stride = (int64_t)grp * (D + 2);
    const float *p0 = part + (((int64_t)b * G + g) * n_splits * grp + hh) * (D + 2);
    const int d = threadIdx.x;
    float v[kMaxSplits];
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s) v[s] = s < n_splits ? p0[s * stride + d] : 0.0f;
    if (threadIdx.x < 64) {
        const int s = threadIdx.x;
        const float ms = s < n_splits ? p0[s * stride + D] : kNegBig;
        const float ls = s < n_splits ? p0[s * stride + D + 1] : 0.0f;
        const float M = wave_max(ms);
        const float w = s < n_splits ? __expf(ms - M) : 0.0f;
        const float L = wave_sum(w * ls);
        wgt[s] = w;
        if (s == 0) inv_l = 1.0f / L;
    }
    __syncthreads();
    float a = 0.0f;
#pragma unroll
    for (int s = 0; s < kMaxSplits; ++s)
        if (s < n_splits) a = fmaf(wgt[s], v[s], a);
    out[((int64_t)b * H + h) * D + d] = a * inv_l;
}

int choose_splits(int64_t B, int64_t G, int64_t n_tot, int64_t *kps) {
    // About kTargetWaves waves in flight, at least kMinKeysPerWave keys per wave, at most kMaxSplits.
    const int64_t pairs = B * G;
    int64_t want = (kTargetWaves / kWaves + pairs - 1) / pairs;
    const int64_t cap = (n_tot + kWaves * kMinKeysPerWave - 1) / (kWaves * kMinKeysPerWave);
    want = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(want, cap), kMaxSplits));
    int64_t k = (n_tot + want - 1) / want;
    k = (k + 15) / 16 * 16;
    *kps = k;
    return (int)((n_tot + k - 1) / k);
}

int64_t partial_bytes(int64_t B, int64_t H, int64_t D, int ns) {
    return B * H * (int64_t)ns * (D + 2) * (int64_t)sizeof(float);
}

template <int KV, int GRP, int DPL>
void launch_decode(dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp, const float *bias,
                   int64_t bhs, int bspan, float *out, float *part, int H, int G, float scale, int64_t n_tot,
                   int64_t kps, int ns, int64_t cb) {
    hipLaunchKernelGGL((attn_decode_kernel<KV, GRP, DPL>), grid, dim3(64 * kWaves), 0, st, q, ldq, sp, bias, bhs,
                       bspan, out, part, H, G, scale, n_tot, kps, ns, cb);
}

template <int KV, int GRP>
bool dispatch_dpl(int D, dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp,
                  const float *bias, int64_t bhs, int bspan, float *out, float *part, int H, int G,
                  float scale, int64_t n_tot, int64_t kps, int ns, int64_t cb) {
    switch (D) {
        case 64: launch_decode<KV, GRP, 4>(grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb); return true;
        case 128: launch_decode<KV, GRP, 8>(grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb); return true;
    }
    return false;
}

template <int KV>
bool dispatch_grp(int grp, int D, dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp,
                  const float *bias, int64_t bhs, int bspan, float *out, float *part, int H, int G,
                  float scale, int64_t n_tot, int64_t kps, int ns, int64_t cb) {
    switch (grp) {
        case 1: return dispatch_dpl<KV, 1>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb);
        case 2: return dispatch_dpl<KV, 2>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb);
        case 4: return dispatch_dpl<KV, 4>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb);
        case 6: return dispatch_dpl<KV, 6>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb);
        case 8: return dispatch_dpl<KV, 8>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, part, H, G, scale, n_tot, kps, ns, cb);
    }
    return false;
}

}  // namespace

extern "C" {

int64_t vgx_attn_decode_workspace_bytes(int64_t B, int64_t H, int64_t G, int64_t D, int64_t n_keys) {
    if (B <= 0 || H <= 0 || G <= 0 || D <= 0 || n_keys <= 0 || H % G) return VGX_E_SIZE;
    int64_t kps = 0;
    const int ns = choose_splits(B, G, n_keys, &kps);
    if (ns <= 1) return 0;
    return partial_bytes(B, H, D, ns);
}

int vgx_attn_decode(int kv_dtype, const float *q, int64_t ldq, const vgx_kv_span *spans, int n_spans,
                    const float *bias, int64_t bias_hstride, int bias_span, int64_t causal_base, float *out, int64_t B,
                    int64_t H, int64_t G, int64_t D, float scale, void *workspace, int64_t workspace_bytes,
                    void *stream) {
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!q || !spans || !out) return VGX_E_ARG;
    if (n_spans < 1 || n_spans > 4) return VGX_E_LIMIT;
    if (B <= 0 || H <= 0 || G <= 0 || H % G) return VGX_E_SIZE;
    if (D != 64 && D != 128) return VGX_E_LIMIT;
    if (B > 65535 || G > 65535) return VGX_E_LIMIT;
    if (bias && (bias_span < 0 || bias_span >= n_spans)) return VGX_E_ARG;
    if (ldq < H * D) return VGX_E_SIZE;
    SpanArgs sp{};
    sp.n = n_spans;
    int64_t n_tot = 0;
    const int elem = kv_dtype == VGX_F32 ? 4 : 2;
    for (int s = 0; s < n_spans; ++s) {
        if (spans[s].len < 0) return VGX_E_SIZE;
        if (spans[s].len > 0 && (!spans[s].k || !spans[s].v)) return VGX_E_ARG;
        if (spans[s].len > 0 && (((uintptr_t)spans[s].k | (uintptr_t)spans[s].v) % 16)) return VGX_E_ALIGN;
        if (spans[s].len > 0 && ((spans[s].batch_stride * elem) % 16 || (spans[s].group_stride * elem) % 16)) return VGX_E_ALIGN;
        sp.k[s] = spans[s].k;
        sp.v[s] = spans[s].v;
        sp.len[s] = spans[s].len;
        sp.bstride[s] = spans[s].batch_stride;
        sp.gstride[s] = spans[s].group_stride;
        sp.dyn_len[s] = spans[s].dyn_len;
        n_tot += spans[s].len;
    }
    if (n_tot <= 0) return VGX_E_SIZE;
    int64_t kps = 0;
    const int ns = choose_splits(B, G, n_tot, &kps);
    float *part = nullptr;
    if (ns > 1) {
        if (!workspace || workspace_bytes < partial_bytes(B, H, D, ns)) return VGX_E_ARENA;
        if ((uintptr_t)workspace % 16) return VGX_E_ALIGN;
        part = static_cast<float *>(workspace);
    }
    const int grp = (int)(H / G);
    hipStream_t st = (hipStream_t)stream;
    dim3 grid((unsigned)ns, (unsigned)G, (unsigned)B);
    bool ok = kv_dtype == VGX_F32
                  ? dispatch_grp<VGX_F32>(grp, (int)D, grid, st, q, ldq, sp, bias, bias_hstride, bias_span, out,
                                          part, (int)H, (int)G, scale, n_tot, kps, ns, causal_base)
                  : dispatch_grp<VGX_BF16>(grp, (int)D, grid, st, q, ldq, sp, bias, bias_hstride, bias_span, out,
                                           part, (int)H, (int)G, scale, n_tot, kps, ns, causal_base);
    if (!ok) return VGX_E_LIMIT;
    VGX_CHECK_LAUNCH();
    if (ns > 1) {
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(B * H)), dim3((unsigned)D), 0, st, part, out, (int)H,
                           (int)G, (int)D, ns);
        VGX_CHECK_LAUNCH();
    }
    return VGX_OK;
}

}  // extern "C"
