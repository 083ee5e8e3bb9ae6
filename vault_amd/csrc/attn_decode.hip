// Split-K GQA decode attention over up to four key spans (sink | segment memory | prev | cur).
//
// Reference semantics: src/vault_v3_model.py:1098-1136 (concat spans, _expand_kv, optional fp32
// bias on the segment span, softmax, P V) and runtime/vault3.c:1958-2032 (attn_run).
//
// Mapping.  One workgroup = one wave = one (batch b, kv group g, key split).  The wave holds the
// GRP query heads of group g, so every K/V row is fetched once for all GRP heads (the reference
// re-reads K/V per head).  The 4 DPP rows (16 lanes each) of the wave each stream their own keys:
// a DPP row holds one key row spread over its 16 lanes (D/16 contiguous elements per lane, one
// 128-bit load for bf16 D=128, two for fp32), so one load instruction fetches four whole key rows.
// q.k partials are reduced across the 16 lanes with DPP; each DPP row keeps its own online-softmax
// state (m, l, acc), merged across rows with cross-lane shuffles at the end.  Splits write
// (m, l, acc) partials that attn_merge_kernel combines; a single split writes the output directly.
#include "common.h"

using namespace vgx;

namespace {

constexpr int kKB = 4;   // keys per DPP row per tile (16 keys per wave tile)
constexpr float kNegBig = -1.0e30f;

struct SpanArgs {
    const void *k[4];
    const void *v[4];
    int64_t len[4];
    int64_t bstride[4];
    int64_t gstride[4];
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

template <int KV, int GRP, int DPL>
__global__ __launch_bounds__(64) void attn_decode_kernel(const float *__restrict__ q, int64_t ldq, SpanArgs sp,
                                                          const float *__restrict__ bias, int64_t bias_hstride,
                                                          int bias_span, float *__restrict__ out,
                                                          float *__restrict__ ws, int H, int G, float scale,
                                                          int64_t n_tot, int64_t kps, int n_splits,
                                                          int64_t causal_base) {
    constexpr int D = DPL * 16;
    const int split = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
    const int lane = threadIdx.x, l16 = lane & 15, row = lane >> 4;

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
        int64_t len = sp.len[s];
        const int64_t lo = max(k0, base) - base;
        int64_t hi = min(k1, base + len) - base;
        // Causal last span: batch entry b sees its first causal_base + b + 1 keys.
        if (causal_base >= 0 && s == sp.n - 1) hi = min(hi, causal_base + (int64_t)b + 1);
        base += len;
        if (lo >= hi) continue;
        const int64_t off = (int64_t)b * sp.bstride[s] + (int64_t)g * sp.gstride[s] + l16 * DPL;
        const void *kb = sp.k[s];
        const void *vb = sp.v[s];
        const float *bb = (bias != nullptr && s == bias_span) ? bias + (int64_t)g * GRP * bias_hstride : nullptr;
        for (int64_t t0 = lo; t0 < hi; t0 += 4 * kKB) {
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

    // Merge the online-softmax states of the four DPP rows.
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
    if (row != 0) return;
#pragma unroll
    for (int hh = 0; hh < GRP; ++hh) {
        if (n_splits == 1) {
            float *op = out + ((int64_t)b * H + (int64_t)g * GRP + hh) * D + l16 * DPL;
            const float inv = 1.0f / l[hh];
#pragma unroll
            for (int d = 0; d < DPL; ++d) op[d] = acc[hh][d] * inv;
        } else {
            float *wp = ws + ((((int64_t)b * G + g) * n_splits + split) * GRP + hh) * (D + 2);
#pragma unroll
            for (int d = 0; d < DPL; ++d) wp[l16 * DPL + d] = acc[hh][d];
            if (l16 == 0) {
                wp[D] = m[hh];
                wp[D + 1] = l[hh];
            }
        }
    }
}

// One workgroup per (b, h): out = sum_s e^{m_s - M} acc_s / sum_s e^{m_s - M} l_s.
__global__ __launch_bounds__(128) void attn_merge_kernel(const float *__restrict__ ws, float *__restrict__ out,
                                                          int H, int G, int D, int n_splits) {
    const int bh = blockIdx.x;
    const int b = bh / H, h = bh - b * H;
    const int grp = H / G, g = h / grp, hh = h - g * grp;
    const int64_t stride = (int64_t)grp * (D + 2);
    const float *w0 = ws + (((int64_t)b * G + g) * n_splits * grp + hh) * (D + 2);
    float M = kNegBig;
    for (int s = 0; s < n_splits; ++s) M = fmaxf(M, w0[s * stride + D]);
    float L = 0.0f;
    for (int s = 0; s < n_splits; ++s) L += __expf(w0[s * stride + D] - M) * w0[s * stride + D + 1];
    const float inv = 1.0f / L;
    for (int d = threadIdx.x; d < D; d += blockDim.x) {
        float a = 0.0f;
        for (int s = 0; s < n_splits; ++s) a = fmaf(__expf(w0[s * stride + D] - M), w0[s * stride + d], a);
        out[((int64_t)b * H + h) * D + d] = a * inv;
    }
}

int choose_splits(int64_t B, int64_t G, int64_t n_tot, int64_t *kps) {
    // Aim for ~2048 waves in flight, at least 16 keys and at most 1024 keys per split.
    const int64_t pairs = B * G;
    int64_t want = (2048 + pairs - 1) / pairs;
    int64_t k = (n_tot + want - 1) / want;
    k = (k + 15) / 16 * 16;
    k = std::max<int64_t>(64, std::min<int64_t>(1024, k));
    if (n_tot <= 64) k = (n_tot + 15) / 16 * 16;
    *kps = k;
    return (int)((n_tot + k - 1) / k);
}

template <int KV, int GRP, int DPL>
void launch_decode(dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp, const float *bias,
                   int64_t bhs, int bspan, float *out, float *ws, int H, int G, float scale, int64_t n_tot, int64_t kps,
                   int ns, int64_t cb) {
    hipLaunchKernelGGL((attn_decode_kernel<KV, GRP, DPL>), grid, dim3(64), 0, st, q, ldq, sp, bias, bhs, bspan, out,
                       ws, H, G, scale, n_tot, kps, ns, cb);
}

template <int KV, int GRP>
bool dispatch_dpl(int D, dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp,
                  const float *bias, int64_t bhs, int bspan, float *out, float *ws, int H, int G, float scale,
                  int64_t n_tot, int64_t kps, int ns, int64_t cb) {
    switch (D) {
        case 64: launch_decode<KV, GRP, 4>(grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb); return true;
        case 128: launch_decode<KV, GRP, 8>(grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb); return true;
    }
    return false;
}

template <int KV>
bool dispatch_grp(int grp, int D, dim3 grid, hipStream_t st, const float *q, int64_t ldq, const SpanArgs &sp,
                  const float *bias, int64_t bhs, int bspan, float *out, float *ws, int H, int G, float scale,
                  int64_t n_tot, int64_t kps, int ns, int64_t cb) {
    switch (grp) {
        case 1: return dispatch_dpl<KV, 1>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb);
        case 2: return dispatch_dpl<KV, 2>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb);
        case 4: return dispatch_dpl<KV, 4>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb);
        case 6: return dispatch_dpl<KV, 6>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb);
        case 8: return dispatch_dpl<KV, 8>(D, grid, st, q, ldq, sp, bias, bhs, bspan, out, ws, H, G, scale, n_tot, kps, ns, cb);
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
    return B * H * (int64_t)ns * (D + 2) * (int64_t)sizeof(float);
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
        n_tot += spans[s].len;
    }
    if (n_tot <= 0) return VGX_E_SIZE;
    int64_t kps = 0;
    const int ns = choose_splits(B, G, n_tot, &kps);
    if (ns > 1) {
        const int64_t need = B * H * (int64_t)ns * (D + 2) * (int64_t)sizeof(float);
        if (!workspace || workspace_bytes < need) return VGX_E_ARENA;
    }
    if (ns > 65535) return VGX_E_LIMIT;
    const int grp = (int)(H / G);
    hipStream_t st = (hipStream_t)stream;
    dim3 grid((unsigned)ns, (unsigned)G, (unsigned)B);
    float *ws = static_cast<float *>(workspace);
    bool ok = kv_dtype == VGX_F32
                  ? dispatch_grp<VGX_F32>(grp, (int)D, grid, st, q, ldq, sp, bias, bias_hstride, bias_span, out, ws,
                                          (int)H, (int)G, scale, n_tot, kps, ns, causal_base)
                  : dispatch_grp<VGX_BF16>(grp, (int)D, grid, st, q, ldq, sp, bias, bias_hstride, bias_span, out, ws,
                                           (int)H, (int)G, scale, n_tot, kps, ns, causal_base);
    if (!ok) return VGX_E_LIMIT;
    VGX_CHECK_LAUNCH();
    if (ns > 1) {
        hipLaunchKernelGGL(attn_merge_kernel, dim3((unsigned)(B * H)), dim3(64), 0, st, ws, out, (int)H, (int)G, (int)D, ns);
        VGX_CHECK_LAUNCH();
    }
    return VGX_OK;
}

}  // extern "C"
