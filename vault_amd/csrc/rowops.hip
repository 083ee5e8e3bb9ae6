// Row-wise kernels of the decode/prefill step: RMSNorm, RoPE + KV-cache write, row rotation
// (chunk-boundary re-base and prefix re-rotation) and row gather (segment-bank compaction).
//
// Reference semantics: src/vault_v3_model.py:764-794, 1079-1094, 1842-1856, 1914-1927;
// runtime/vault3.c:656-678, 859-896, 1892-1913, 1930-1940, 2162-2179.
#include "common.h"

using namespace vgx;

namespace {

__global__ __launch_bounds__(256) void rmsnorm_kernel(const float *__restrict__ x, int64_t ldx,
                                                       const float *__restrict__ w, float *__restrict__ y,
                                                       int64_t ldy, int64_t dim, float eps) {
    __shared__ float red[4];
    const int64_t r = blockIdx.x;
    const float *xr = x + r * ldx;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) s = fmaf(xr[i], xr[i], s);
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.0f;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) tot += red[i];
    const float inv = 1.0f / sqrtf(tot / (float)dim + eps);
    float *yr = y + r * ldy;
    for (int64_t i = threadIdx.x; i < dim; i += blockDim.x) yr[i] = w[i] * (xr[i] * inv);
}

// grid.x = N tokens, grid.y = H + G heads; threads over D/2 rotation pairs.
template <int KV>
__global__ void rope_qkv_write_kernel(float *__restrict__ q, int64_t ldq, const float *__restrict__ k, int64_t ldk,
                                      const float *__restrict__ v, int64_t ldv, int H, int G, int D,
                                      const float *__restrict__ table, int64_t trs,
                                      void *k_rot, void *k_raw, void *v_dst, int64_t dts, int64_t dgs, void *sk,
                                      void *sv, int64_t n_sink, int64_t sts, int64_t sgs) {
    const int64_t t = blockIdx.x;
    const int hd = blockIdx.y;
    const int h2 = D / 2;
    const float *cs = table + t * trs;
    for (int i = threadIdx.x; i < h2; i += blockDim.x) {
        const float c = cs[i], s = cs[h2 + i];
        if (hd < H) {
            float *qp = q + t * ldq + (int64_t)hd * D;
            const float a = qp[i], b = qp[i + h2];
            qp[i] = a * c - b * s;
            qp[i + h2] = b * c + a * s;
        } else {
            const int g = hd - H;
            const float *kp = k + t * ldk + (int64_t)g * D;
            const float *vp = v + t * ldv + (int64_t)g * D;
            const float a = kp[i], b = kp[i + h2];
            const int64_t o = t * dts + g * dgs;
            if (k_rot) {
                store_kv<KV>(k_rot, o + i, a * c - b * s);
                store_kv<KV>(k_rot, o + i + h2, b * c + a * s);
            }
            if (k_raw) {
                store_kv<KV>(k_raw, o + i, a);
                store_kv<KV>(k_raw, o + i + h2, b);
            }
            store_kv<KV>(v_dst, o + i, vp[i]);
            store_kv<KV>(v_dst, o + i + h2, vp[i + h2]);
            if (t < n_sink) {
                const int64_t so = t * sts + g * sgs;
                store_kv<KV>(sk, so + i, a);
                store_kv<KV>(sk, so + i + h2, b);
                store_kv<KV>(sv, so + i, vp[i]);
                store_kv<KV>(sv, so + i + h2, vp[i + h2]);
            }
        }
    }
}

// Decode-step variant: grid.x = B sequences (one token each), grid.y = H + G heads.  The ring slot,
// RoPE table row and sink slot come from the device step descriptor, so a captured graph replays
// at every position of a chunk.
template <int KV>
__global__ void rope_qkv_write_step_kernel(float *__restrict__ q, int64_t ldq, const float *__restrict__ k, int64_t ldk,
                                           const float *__restrict__ v, int64_t ldv, int H, int G, int D,
                                           const float *__restrict__ table, int64_t trs,
                                           const int32_t *__restrict__ step, void *k_rot, void *k_raw, void *v_dst,
                                           int64_t dbs, int64_t dgs, int64_t drs, void *sk, void *sv, int64_t sbs,
                                           int64_t sgs, int64_t srs) {
    const int64_t t = blockIdx.x;
    const int hd = blockIdx.y;
    const int h2 = D / 2;
    const int64_t slot = step[VGX_STEP_SLOT];
    const int64_t sink = step[VGX_STEP_SINK_SLOT];
    const float *cs = table + (int64_t)step[VGX_STEP_TABLE_ROW] * trs;
    for (int i = threadIdx.x; i < h2; i += blockDim.x) {
        const float c = cs[i], s = cs[h2 + i];
        if (hd < H) {
            float *qp = q + t * ldq + (int64_t)hd * D;
            const float a = qp[i], b = qp[i + h2];
            qp[i] = a * c - b * s;
            qp[i + h2] = b * c + a * s;
        } else {
            const int g = hd - H;
            const float *kp = k + t * ldk + (int64_t)g * D;
            const float *vp = v + t * ldv + (int64_t)g * D;
            const float a = kp[i], b = kp[i + h2];
            const int64_t o = t * dbs + g * dgs + slot * drs;
            if (k_rot) {
                store_kv<KV>(k_rot, o + i, a * c - b * s);
                store_kv<KV>(k_rot, o + i + h2, b * c + a * s);
            }
            if (k_raw) {
                store_kv<KV>(k_raw, o + i, a);
                store_kv<KV>(k_raw, o + i + h2, b);
            }
            store_kv<KV>(v_dst, o + i, vp[i]);
            store_kv<KV>(v_dst, o + i + h2, vp[i + h2]);
            if (sink >= 0 && sk) {
                const int64_t so = t * sbs + g * sgs + sink * srs;
                store_kv<KV>(sk, so + i, a);
                store_kv<KV>(sk, so + i + h2, b);
                store_kv<KV>(sv, so + i, vp[i]);
                store_kv<KV>(sv, so + i + h2, vp[i + h2]);
            }
        }
    }
}

// grid.x = n_rows, grid.y = n_outer (chunked); threads over D/2 pairs.
template <int KV>
__global__ void rope_rotate_kernel(const void *src, void *dst, int64_t n_outer, int64_t sos, int64_t dos, int D,
                                   const float *__restrict__ table, int64_t trs) {
    const int64_t i = blockIdx.x;
    const int h2 = D / 2;
    const float *cs = table + i * trs;
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

template <typename T>
__global__ void gather_rows_kernel(const T *__restrict__ src, T *__restrict__ dst, const int32_t *__restrict__ idx,
                                   int64_t n_idx, int64_t src_rows, int64_t n_outer, int64_t sos, int64_t dos, int D) {
    const int64_t j = blockIdx.x;
    const int64_t sr = idx[j];
    const bool ok = sr >= 0 && sr < src_rows;
    for (int64_t o = blockIdx.y; o < n_outer; o += gridDim.y) {
        T *d = dst + o * dos + j * D;
        if (ok) {
            const T *s = src + o * sos + sr * D;
            for (int e = threadIdx.x; e < D; e += blockDim.x) d[e] = s[e];
        } else {
            for (int e = threadIdx.x; e < D; e += blockDim.x) d[e] = T(0);
        }
    }
}

}  // namespace

extern "C" {

int vgx_rmsnorm(const float *x, int64_t ldx, const float *w, float *y, int64_t ldy, int64_t n_rows, int64_t dim,
                float eps, void *stream) {
    if (!x || !w || !y) return VGX_E_ARG;
    if (n_rows < 0 || dim <= 0 || ldx < dim || ldy < dim || !(eps > 0.0f)) return VGX_E_SIZE;
    if (n_rows == 0) return VGX_OK;
    if (n_rows > 0x7FFFFFFF) return VGX_E_LIMIT;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream, x, ldx, w, y, ldy,
                       dim, eps);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_rope_qkv_write(int kv_dtype, float *q, int64_t ldq, const float *k, int64_t ldk, const float *v, int64_t ldv,
                       int64_t N, int64_t H, int64_t G, int64_t D, const float *table, int64_t table_rstride,
                       void *k_rot, void *k_raw, void *v_dst,
                       int64_t dst_tstride, int64_t dst_gstride, void *sink_k_raw, void *sink_v, int64_t n_sink,
                       int64_t sink_tstride, int64_t sink_gstride, void *stream) {
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!k || !v || !table || !v_dst) return VGX_E_ARG;
    if (H > 0 && !q) return VGX_E_ARG;
    if (n_sink > 0 && (!sink_k_raw || !sink_v)) return VGX_E_ARG;
    if (N < 0 || H < 0 || G <= 0 || D <= 0 || (D & 1) || n_sink < 0 || n_sink > N) return VGX_E_SIZE;
    if ((H > 0 && ldq < H * D) || ldk < G * D || ldv < G * D) return VGX_E_SIZE;
    if (N == 0) return VGX_OK;
    if (N > 0x7FFFFFFF || H + G > 65535) return VGX_E_LIMIT;
    dim3 grid((unsigned)N, (unsigned)(H + G));
    const int thr = (int)std::min<int64_t>(256, std::max<int64_t>(32, D / 2));
    hipStream_t st = (hipStream_t)stream;
    if (kv_dtype == VGX_F32)
        hipLaunchKernelGGL(rope_qkv_write_kernel<VGX_F32>, grid, dim3(thr), 0, st, q, ldq, k, ldk, v, ldv, (int)H, (int)G, (int)D,
                           table, table_rstride, k_rot, k_raw, v_dst, dst_tstride, dst_gstride, sink_k_raw, sink_v,
                           n_sink, sink_tstride, sink_gstride);
    else
        hipLaunchKernelGGL(rope_qkv_write_kernel<VGX_BF16>, grid, dim3(thr), 0, st, q, ldq, k, ldk, v, ldv, (int)H, (int)G, (int)D,
                           table, table_rstride, k_rot, k_raw, v_dst, dst_tstride, dst_gstride, sink_k_raw, sink_v,
                           n_sink, sink_tstride, sink_gstride);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_rope_qkv_write_step(int kv_dtype, float *q, int64_t ldq, const float *k, int64_t ldk, const float *v,
                            int64_t ldv, int64_t B, int64_t H, int64_t G, int64_t D, const float *table,
                            int64_t table_rstride, const int32_t *step, void *k_rot, void *k_raw, void *v_dst,
                            int64_t dst_bstride, int64_t dst_gstride, int64_t dst_rstride, void *sink_k_raw,
                            void *sink_v, int64_t sink_bstride, int64_t sink_gstride, int64_t sink_rstride,
                            void *stream) {
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!k || !v || !table || !v_dst || !step) return VGX_E_ARG;
    if (H > 0 && !q) return VGX_E_ARG;
    if ((sink_k_raw == nullptr) != (sink_v == nullptr)) return VGX_E_ARG;
    if (B < 0 || H < 0 || G <= 0 || D <= 0 || (D & 1)) return VGX_E_SIZE;
    if ((H > 0 && ldq < H * D) || ldk < G * D || ldv < G * D) return VGX_E_SIZE;
    if (B == 0) return VGX_OK;
    if (B > 0x7FFFFFFF || H + G > 65535) return VGX_E_LIMIT;
    dim3 grid((unsigned)B, (unsigned)(H + G));
    const int thr = (int)std::min<int64_t>(256, std::max<int64_t>(32, D / 2));
    hipStream_t st = (hipStream_t)stream;
    if (kv_dtype == VGX_F32)
        hipLaunchKernelGGL(rope_qkv_write_step_kernel<VGX_F32>, grid, dim3(thr), 0, st, q, ldq, k, ldk, v, ldv, (int)H,
                           (int)G, (int)D, table, table_rstride, step, k_rot, k_raw, v_dst, dst_bstride, dst_gstride,
                           dst_rstride, sink_k_raw, sink_v, sink_bstride, sink_gstride, sink_rstride);
    else
        hipLaunchKernelGGL(rope_qkv_write_step_kernel<VGX_BF16>, grid, dim3(thr), 0, st, q, ldq, k, ldk, v, ldv, (int)H,
                           (int)G, (int)D, table, table_rstride, step, k_rot, k_raw, v_dst, dst_bstride, dst_gstride,
                           dst_rstride, sink_k_raw, sink_v, sink_bstride, sink_gstride, sink_rstride);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_rope_rotate(int kv_dtype, const void *src, void *dst, int64_t n_outer, int64_t src_ostride,
                    int64_t dst_ostride, int64_t n_rows, int64_t D, const float *table, int64_t table_rstride,
                    void *stream) {
    if (kv_dtype != VGX_F32 && kv_dtype != VGX_BF16) return VGX_E_DTYPE;
    if (!src || !dst || !table) return VGX_E_ARG;
    if (n_outer < 0 || n_rows < 0 || D <= 0 || (D & 1)) return VGX_E_SIZE;
    if (n_outer == 0 || n_rows == 0) return VGX_OK;
    if (n_rows > 0x7FFFFFFF) return VGX_E_LIMIT;
    dim3 grid((unsigned)n_rows, (unsigned)std::min<int64_t>(n_outer, 1024));
    const int thr = (int)std::min<int64_t>(256, std::max<int64_t>(32, D / 2));
    hipStream_t st = (hipStream_t)stream;
    if (kv_dtype == VGX_F32)
        hipLaunchKernelGGL(rope_rotate_kernel<VGX_F32>, grid, dim3(thr), 0, st, src, dst, n_outer, src_ostride,
                           dst_ostride, (int)D, table, table_rstride);
    else
        hipLaunchKernelGGL(rope_rotate_kernel<VGX_BF16>, grid, dim3(thr), 0, st, src, dst, n_outer, src_ostride,
                           dst_ostride, (int)D, table, table_rstride);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_gather_rows(int dtype, const void *src, void *dst, const int32_t *idx, int64_t n_idx, int64_t src_rows,
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
        hipLaunchKernelGGL(gather_rows_kernel<float>, grid, dim3(thr), 0, st, static_cast<const float *>(src),
                           static_cast<float *>(dst), idx, n_idx, src_rows, n_outer, src_ostride, dst_ostride, (int)D);
    else
        hipLaunchKernelGGL(gather_rows_kernel<uint16_t>, grid, dim3(thr), 0, st, static_cast<const uint16_t *>(src),
                           static_cast<uint16_t *>(dst), idx, n_idx, src_rows, n_outer, src_ostride, dst_ostride, (int)D);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // extern "C"
