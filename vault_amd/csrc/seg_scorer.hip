// Segment-memory scorer on the device: causal EMA habituation of the scorer features, LayerNorm,
// and the GELU . fc2 tail with the habituated-score combine.
//
// Reference semantics: src/vault_v3_model.py:870-883 (SegmentScorer: LayerNorm eps 1e-5 ->
// Linear -> GELU -> Linear), :1224-1247 (_score_chunk_habituated) and :2294-2305 (step);
// runtime/vault3.c:961-977, 2201-2216.  The GELU is the C runtime's (v3_geluf, A&S 7.1.26 erf,
// runtime/vault3.c:118-129, 974: ref_geluf), bit for bit; the Python model's exact erf is within
// 1.5e-7 of it.  Per token t with features f_t and EMA state e:
//   hab_in_t = f_t - 0.65 e_{t-1};  e_t = 0.985 e_{t-1} + 0.015 f_t   (e_0 = f_0 on the first token)
//   score_t  = raw_t + 0.35 max(0, hab_t - raw_t)                     (score_0 = raw_0 on the first)
// The fc1 GEMV between LayerNorm and the tail runs through vgx_qlinear (F32 weights).
#include "qgemv.h"

using namespace vgx;

namespace {

// One thread per feature; scans the T tokens in order.
__global__ void ema_habituate_kernel(const float *__restrict__ f, int64_t ldf, float *__restrict__ hab,
                                     int64_t ldh, float *__restrict__ ema, int64_t T, int64_t fd, int first) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= fd) return;
    float e = first ? f[i] : ema[i];
    // The features do not depend on the recurrence: load kU of them at once, then run the sequential
    // update over them (one load round trip per kU steps instead of per step; same arithmetic in the
    // same order).
    constexpr int kU = 32;
    int64_t t = 0;
    for (; t + kU <= T; t += kU) {
        float fv[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) fv[u] = f[(t + u) * ldf + i];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            hab[(t + u) * ldh + i] = hab_of(fv[u], e);
            if (!(first && t + u == 0)) e = ema_step(e, fv[u]);
        }
    }
    for (; t < T; ++t) {
        const float ft = f[t * ldf + i];
        hab[t * ldh + i] = hab_of(ft, e);
        if (!(first && t == 0)) e = ema_step(e, ft);
    }
    ema[i] = e;
}

__global__ __launch_bounds__(256) void layernorm_kernel(const float *__restrict__ x, int64_t ldx,
                                                         const float *__restrict__ w, const float *__restrict__ b,
                                                         float *__restrict__ y, int64_t ldy, int64_t dim, float eps) {
    __shared__ float red[4];
    __shared__ float stat[2];
    const float *xr = x + (int64_t)blockIdx.x * ldx;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) s += xr[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) stat[0] = (red[0] + red[1] + red[2] + red[3]) / (float)dim;
    __syncthreads();
    const float mean = stat[0];
    float v = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) {
        const float d = xr[i] - mean;
        v = fmaf(d, d, v);
    }
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) stat[1] = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / (float)dim + eps);
    __syncthreads();
    const float inv = stat[1];
    float *yr = y + (int64_t)blockIdx.x * ldy;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = (xr[i] - mean) * inv * w[i] + b[i];
}

// Rows of up to 256 x 4 x kLnMaxF4 floats held in registers: every load of the row is issued at once
// (the loop form above waits for each pass over the row in turn).  One workgroup per row.
constexpr int kLnMaxF4 = 8;

__global__ __launch_bounds__(256) void layernorm_reg_kernel(const float *__restrict__ x, int64_t ldx,
                                                             const float *__restrict__ w,
                                                             const float *__restrict__ b, float *__restrict__ y,
                                                             int64_t ldy, int dim, float eps) {
    __shared__ float red[2][4];
    const float4 *xr = reinterpret_cast<const float4 *>(x + (int64_t)blockIdx.x * ldx);
    const int n4 = dim / 4;
    float4 v[kLnMaxF4];
    float s = 0.0f;
#pragma unroll
    for (int u = 0; u < kLnMaxF4; ++u) {
        const int i = threadIdx.x + u * 256;
        v[u] = i < n4 ? xr[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < kLnMaxF4; ++u) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[0][threadIdx.x >> 6] = s;
    __syncthreads();
    const float mean = (red[0][0] + red[0][1] + red[0][2] + red[0][3]) / (float)dim;
    float q = 0.0f;
#pragma unroll
    for (int u = 0; u < kLnMaxF4; ++u) {
        if (threadIdx.x + u * 256 < n4) {
            const float a = v[u].x - mean, c = v[u].y - mean, d = v[u].z - mean, e = v[u].w - mean;
            q = fmaf(a, a, fmaf(c, c, fmaf(d, d, fmaf(e, e, q))));
        }
    }
    q = wave_sum(q);
    if ((threadIdx.x & 63) == 0) red[1][threadIdx.x >> 6] = q;
    __syncthreads();
    const float inv = 1.0f / sqrtf((red[1][0] + red[1][1] + red[1][2] + red[1][3]) / (float)dim + eps);
    float4 *yr = reinterpret_cast<float4 *>(y + (int64_t)blockIdx.x * ldy);
    const float4 *w4 = reinterpret_cast<const float4 *>(w), *b4 = reinterpret_cast<const float4 *>(b);
#pragma unroll
    for (int u = 0; u < kLnMaxF4; ++u) {
        const int i = threadIdx.x + u * 256;
        if (i < n4) {
            const float4 g = w4[i], o = b4[i];
            yr[i] = make_float4((v[u].x - mean) * inv * g.x + o.x, (v[u].y - mean) * inv * g.y + o.y,
                                (v[u].z - mean) * inv * g.z + o.z, (v[u].w - mean) * inv * g.w + o.w);
        }
    }
}

// One wave per token t: raw = gelu(h[t]) . w2 + b2, hab = gelu(h[T + t]) . w2 + b2.
__global__ __launch_bounds__(64) void score_tail_kernel(const float *__restrict__ h, int64_t ldh,
                                                         const float *__restrict__ w2, const float *__restrict__ b2,
                                                         int64_t hidden, int64_t T, int first,
                                                         float *__restrict__ out,
                                                         const int32_t *__restrict__ out_index) {
    const int64_t t = blockIdx.x;
    if (out_index) out += *out_index;
    float r = 0.0f, a = 0.0f;
    for (int64_t i = threadIdx.x; i < hidden; i += 64) {
        const float x0 = h[t * ldh + i], x1 = h[(T + t) * ldh + i];
        r = fmaf(ref_geluf(x0), w2[i], r);
        a = fmaf(ref_geluf(x1), w2[i], a);
    }
    r = wave_sum(r) + b2[0];
    a = wave_sum(a) + b2[0];
    if (threadIdx.x == 0) out[t] = (first && t == 0) ? r : r + 0.35f * fmaxf(0.0f, a - r);
}

}  // namespace

extern "C" {

int vgx_ema_habituate(const float *f, int64_t ldf, float *hab, int64_t ldh, float *ema, int64_t T, int64_t fd,
                      int first, void *stream) {
    if (!f || !hab || !ema) return VGX_E_ARG;
    if (T < 0 || fd <= 0 || ldf < fd || ldh < fd) return VGX_E_SIZE;
    if (T == 0) return VGX_OK;
    hipLaunchKernelGGL(ema_habituate_kernel, dim3((unsigned)((fd + 255) / 256)), dim3(256), 0, (hipStream_t)stream, f,
                       ldf, hab, ldh, ema, T, fd, first ? 1 : 0);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_layernorm(const float *x, int64_t ldx, const float *w, const float *b, float *y, int64_t ldy, int64_t n_rows,
                  int64_t dim, float eps, void *stream) {
    if (!x || !w || !b || !y) return VGX_E_ARG;
    if (n_rows < 0 || dim <= 0 || ldx < dim || ldy < dim || !(eps > 0.0f)) return VGX_E_SIZE;
    if (n_rows == 0) return VGX_OK;
    if (n_rows > 0x7FFFFFFF) return VGX_E_LIMIT;
    const bool reg = dim % 4 == 0 && dim <= 256 * 4 * kLnMaxF4 && ldx % 4 == 0 && ldy % 4 == 0 &&
                     (((uintptr_t)x | (uintptr_t)y | (uintptr_t)w | (uintptr_t)b) & 15) == 0;
    if (reg)
        hipLaunchKernelGGL(layernorm_reg_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, x, ldx, w,
                           b, y, ldy, (int)dim, eps);
    else
        hipLaunchKernelGGL(layernorm_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, x, ldx, w, b,
                           y, ldy, dim, eps);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_seg_score_step(const float *feat, int64_t fd, float *ema, int first, const void *w1, int64_t hidden,
                       const float *b1, const float *ln_w, const float *ln_b, float eps, const float *w2,
                       const float *b2, float *h, float *out, const int32_t *out_index, void *stream) {
    const vgx_score_side c{1, feat, fd, ema, first, w1, hidden, b1, ln_w, ln_b, eps, w2, b2, h, out, out_index};
    ScoreSide s1, s2;
    int rc = make_score_side(c, s1);
    if (rc != VGX_OK) return rc;
    vgx_score_side c2 = c;
    c2.phase = 2;
    rc = make_score_side(c2, s2);
    if (rc != VGX_OK) return rc;
    hipStream_t st = (hipStream_t)stream;
    rc = vgx_detail_score_side(s1, st);
    return rc != VGX_OK ? rc : vgx_detail_score_side(s2, st);
}

int vgx_seg_score_tail(const float *h, int64_t ldh, const float *w2, const float *b2, int64_t hidden, int64_t T,
                       int first, float *out, const int32_t *out_index, void *stream) {
    if (!h || !w2 || !b2 || !out) return VGX_E_ARG;
    if (T < 0 || hidden <= 0 || ldh < hidden) return VGX_E_SIZE;
    if (T == 0) return VGX_OK;
    if (T > 0x7FFFFFFF) return VGX_E_LIMIT;
    hipLaunchKernelGGL(score_tail_kernel, dim3((unsigned)T), dim3(64), 0, (hipStream_t)stream, h, ldh, w2, b2, hidden,
                       T, first ? 1 : 0, out, out_index);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // extern "C"
