// Q8_0 / Q4_0 / F32 / BF16 / F16 weights on gfx950: packing into the row-quad layout, bit-exact
// dequant, embedding rows, and the C entry points of the GEMV (kernels in qgemv.h).
//
// Reference semantics: runtime/vault3.c:499-654 (row_dot with its F32 / BF16 / F16 / Q8_0 / Q4_0
// cases, matvec, embed_row), 1942-1956 (mlp_gu_run); tools/vlt3.py:98-157 (block layouts and
// dequantization), 312-342 (BF16 tensors of the "bf16" format and of rows that are not whole blocks).
#include "qgemv.h"

using namespace vgx;

namespace {

__host__ __device__ constexpr int quant_bytes(int dt) { return gemv_quant_bytes(dt); }
__host__ __device__ constexpr int aos_bytes(int dt) { return dt == VGX_Q8_0 ? 34 : dt == VGX_Q4_0 ? 18 : 0; }

inline int64_t rows4(int64_t r) { return (r + 3) / 4 * 4; }

inline bool dtype_ok(int dt) {
    return dt == VGX_Q8_0 || dt == VGX_Q4_0 || dt == VGX_F32 || dt == VGX_BF16 || dt == VGX_F16;
}

int64_t scale_off(int dt, int64_t rows, int64_t cols) {
    const int64_t q = rows4(rows) * (cols / QK) * quant_bytes(dt);
    return (q + 255) / 256 * 256;
}

int64_t packed_bytes(int dt, int64_t rows, int64_t cols) {
    if (gemv_plain(dt)) return rows4(rows) * (cols / QK) * quant_bytes(dt);
    return scale_off(dt, rows, cols) + rows4(rows) * (cols / QK) * 2;
}

// ------------------------------------------------------------------------------------------
// packing
// ------------------------------------------------------------------------------------------

// One thread per (packed row p, block b).  mode 0: packed row p <- source row p of `a`.
// mode 1 (gate/up): packed row-quad q holds a[2q], a[2q+1], b[2q], b[2q+1].
// mode 2 (RoPE pairs): for p < n_rope, inside each head of hd rows, row-quad j holds rows
// 2j, 2j + hd/2, 2j + 1, 2j + 1 + hd/2 (the rotation pairs 2j and 2j + 1); rows >= n_rope stay.
template <int DT>
__global__ void pack_kernel(const uint8_t *__restrict__ a, const uint8_t *__restrict__ bsrc,
                            uint8_t *__restrict__ dst, int64_t src_rows, int64_t nblk, int64_t soff,
                            int64_t total, int mode, int hd, int64_t n_rope) {
    constexpr int QB = quant_bytes(DT);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    const int64_t p = i / nblk, b = i - p * nblk;
    const int64_t rq = p >> 2, rr = p & 3;
    const uint8_t *src = a;
    int64_t r = p;
    if (mode == 1) {
        r = 2 * rq + (rr & 1);
        src = rr < 2 ? a : bsrc;
    } else if (mode == 2 && p < n_rope) {
        const int64_t h = p / hd, w = p - h * hd, j = w >> 2, k = w & 3;
        r = h * hd + 2 * j + (k >> 1) + (k & 1) * (hd / 2);
    }
    uint8_t *qd = dst + ((rq * nblk + b) * 4 + rr) * QB;
    const bool live = r < src_rows;
    if constexpr (gemv_plain(DT)) {
        // row-major elements: the block's QB bytes as 32-bit words
        const uint32_t *s = reinterpret_cast<const uint32_t *>(src + (r * nblk + b) * QB);
        uint32_t *d = reinterpret_cast<uint32_t *>(qd);
        for (int j = 0; j < QB / 4; ++j) d[j] = live ? s[j] : 0u;
    } else {
        uint16_t *sd = reinterpret_cast<uint16_t *>(dst + soff) + (rq * nblk + b) * 4 + rr;
        const uint8_t *s = src + (r * nblk + b) * aos_bytes(DT);
        *sd = live ? (uint16_t)(s[0] | (s[1] << 8)) : (uint16_t)0;
        for (int j = 0; j < QB; ++j) qd[j] = live ? s[2 + j] : (uint8_t)0;
    }
}

template <int DT>
__global__ void unpack_kernel(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst, int64_t rows,
                              int64_t nblk, int64_t soff) {
    constexpr int QB = quant_bytes(DT);
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nblk) return;
    const int64_t r = i / nblk, b = i - r * nblk;
    const int64_t rq = r >> 2, rr = r & 3;
    const uint8_t *qs = src + ((rq * nblk + b) * 4 + rr) * QB;
    if constexpr (gemv_plain(DT)) {
        uint32_t *d = reinterpret_cast<uint32_t *>(dst + (r * nblk + b) * QB);
        const uint32_t *s = reinterpret_cast<const uint32_t *>(qs);
        for (int j = 0; j < QB / 4; ++j) d[j] = s[j];
    } else {
        const uint16_t sc = reinterpret_cast<const uint16_t *>(src + soff)[(rq * nblk + b) * 4 + rr];
        uint8_t *d = dst + (r * nblk + b) * aos_bytes(DT);
        d[0] = (uint8_t)(sc & 0xFF);
        d[1] = (uint8_t)(sc >> 8);
        for (int j = 0; j < QB; ++j) d[2 + j] = qs[j];
    }
}

template <int DT>
__global__ void dequant_kernel(const uint8_t *__restrict__ w, float *__restrict__ out, int64_t rows, int64_t nblk,
                               int64_t soff) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows * nblk) return;
    const int64_t r = i / nblk, b = i - r * nblk;
    dequant_block<DT>(w, nblk, soff, r, b, out + r * nblk * QK + b * QK);
}

template <int DT>
__global__ void embed_kernel(const uint8_t *__restrict__ w, const int64_t *__restrict__ ids, float *__restrict__ out,
                             int64_t ldo, int64_t rows, int64_t nblk, int64_t soff, int64_t n_ids, int64_t pad_row) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_ids * nblk) return;
    const int64_t t = i / nblk, b = i - t * nblk;
    int64_t r = ids[t];
    if (r < 0 || r >= rows) r = pad_row;
    dequant_block<DT>(w, nblk, soff, r, b, out + t * ldo + b * QK);
}

inline unsigned grid_for(int64_t n, int threads) { return (unsigned)((n + threads - 1) / threads); }

__global__ __launch_bounds__(1024) void score_side_kernel(ScoreSide s) { score_side_run(s, (int)blockIdx.x); }

}  // namespace

int vgx::vgx_detail_score_side(const ScoreSide &s, hipStream_t st) {
    hipLaunchKernelGGL(score_side_kernel, dim3((unsigned)score_side_blocks(s)), dim3(1024), 0, st, s);
    return hipGetLastError() == hipSuccess ? VGX_OK : VGX_E_HIP;
}

extern "C" {

int vgx_abi_version(void) { return VGX_ABI_VERSION; }

int64_t vgx_qweight_packed_bytes(int dtype, int64_t rows, int64_t cols) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    return packed_bytes(dtype, rows, cols);
}

int64_t vgx_qweight_scale_offset(int dtype, int64_t rows, int64_t cols) {
    if (dtype != VGX_Q8_0 && dtype != VGX_Q4_0) return VGX_E_DTYPE;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    return scale_off(dtype, rows, cols);
}

static int pack_common(int dtype, const void *a, const void *b, void *dst, int64_t rows, int64_t cols, int mode,
                       void *stream, int hd = 0, int64_t n_rope = 0) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!a || !dst || (mode == 1 && !b)) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    if (mode == 1 && (rows % 2)) return VGX_E_SHAPE;
    const int64_t prow = mode == 1 ? 2 * rows : rows;
    const int64_t nblk = cols / QK;
    const int64_t total = rows4(prow) * nblk;
    const int64_t soff = gemv_plain(dtype) ? 0 : scale_off(dtype, prow, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *pa = static_cast<const uint8_t *>(a);
    const auto *pb = static_cast<const uint8_t *>(b);
    auto *pd = static_cast<uint8_t *>(dst);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(pack_kernel<VGX_Q8_0>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode, hd, n_rope); break;
        case VGX_Q4_0: hipLaunchKernelGGL(pack_kernel<VGX_Q4_0>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode, hd, n_rope); break;
        case VGX_F32: hipLaunchKernelGGL(pack_kernel<VGX_F32>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode, hd, n_rope); break;
        case VGX_BF16: hipLaunchKernelGGL(pack_kernel<VGX_BF16>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode, hd, n_rope); break;
        case VGX_F16: hipLaunchKernelGGL(pack_kernel<VGX_F16>, grid_for(total, 256), 256, 0, st, pa, pb, pd, rows, nblk, soff, total, mode, hd, n_rope); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_qweight_pack(int dtype, const void *src_blocks, void *dst_packed, int64_t rows, int64_t cols, void *stream) {
    return pack_common(dtype, src_blocks, nullptr, dst_packed, rows, cols, 0, stream);
}

int vgx_qweight_pack_gateup(int dtype, const void *gate_blocks, const void *up_blocks, void *dst_packed,
                            int64_t rows, int64_t cols, void *stream) {
    return pack_common(dtype, gate_blocks, up_blocks, dst_packed, rows, cols, 1, stream);
}

int vgx_qweight_pack_rope(int dtype, const void *src_blocks, void *dst_packed, int64_t rows, int64_t cols,
                          int64_t head_dim, int64_t n_rope_rows, void *stream) {
    if (head_dim <= 0 || head_dim % 4 || n_rope_rows < 0 || n_rope_rows > rows || n_rope_rows % head_dim)
        return VGX_E_SHAPE;
    if (head_dim > 0x7FFFFFFF) return VGX_E_LIMIT;
    return pack_common(dtype, src_blocks, nullptr, dst_packed, rows, cols, 2, stream, (int)head_dim, n_rope_rows);
}

int vgx_qweight_unpack(int dtype, const void *packed, void *dst_blocks, int64_t rows, int64_t cols, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!packed || !dst_blocks) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    const int64_t nblk = cols / QK;
    const int64_t soff = gemv_plain(dtype) ? 0 : scale_off(dtype, rows, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *ps = static_cast<const uint8_t *>(packed);
    auto *pd = static_cast<uint8_t *>(dst_blocks);
    const unsigned g = grid_for(rows * nblk, 256);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(unpack_kernel<VGX_Q8_0>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
        case VGX_Q4_0: hipLaunchKernelGGL(unpack_kernel<VGX_Q4_0>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
        case VGX_F32: hipLaunchKernelGGL(unpack_kernel<VGX_F32>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
        case VGX_BF16: hipLaunchKernelGGL(unpack_kernel<VGX_BF16>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
        case VGX_F16: hipLaunchKernelGGL(unpack_kernel<VGX_F16>, g, 256, 0, st, ps, pd, rows, nblk, soff); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_qweight_dequant(int dtype, const void *packed, float *out, int64_t rows, int64_t cols, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!packed || !out) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    const int64_t nblk = cols / QK;
    const int64_t soff = gemv_plain(dtype) ? 0 : scale_off(dtype, rows, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *pw = static_cast<const uint8_t *>(packed);
    const unsigned g = grid_for(rows * nblk, 256);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(dequant_kernel<VGX_Q8_0>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
        case VGX_Q4_0: hipLaunchKernelGGL(dequant_kernel<VGX_Q4_0>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
        case VGX_F32: hipLaunchKernelGGL(dequant_kernel<VGX_F32>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
        case VGX_BF16: hipLaunchKernelGGL(dequant_kernel<VGX_BF16>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
        case VGX_F16: hipLaunchKernelGGL(dequant_kernel<VGX_F16>, g, 256, 0, st, pw, out, rows, nblk, soff); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

int vgx_embed_rows(int dtype, const void *packed, int64_t rows, int64_t cols, const int64_t *ids, int64_t n_ids,
                   int64_t pad_row, float *out, int64_t ldo, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!packed || !ids || !out) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || n_ids < 0 || ldo < cols || pad_row < 0 || pad_row >= rows) return VGX_E_SIZE;
    if (cols % QK) return VGX_E_SHAPE;
    if (n_ids == 0) return VGX_OK;
    const int64_t nblk = cols / QK;
    const int64_t soff = gemv_plain(dtype) ? 0 : scale_off(dtype, rows, cols);
    hipStream_t st = (hipStream_t)stream;
    const auto *pw = static_cast<const uint8_t *>(packed);
    const unsigned g = grid_for(n_ids * nblk, 256);
    switch (dtype) {
        case VGX_Q8_0: hipLaunchKernelGGL(embed_kernel<VGX_Q8_0>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
        case VGX_Q4_0: hipLaunchKernelGGL(embed_kernel<VGX_Q4_0>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
        case VGX_F32: hipLaunchKernelGGL(embed_kernel<VGX_F32>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
        case VGX_BF16: hipLaunchKernelGGL(embed_kernel<VGX_BF16>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
        case VGX_F16: hipLaunchKernelGGL(embed_kernel<VGX_F16>, g, 256, 0, st, pw, ids, out, ldo, rows, nblk, soff, n_ids, pad_row); break;
    }
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

static int qgemv_dispatch(int dtype, const void *w, int64_t rows_packed, int64_t rows_out, int64_t cols,
                          const float *x, int64_t ldx, int64_t batch, const float *lnw, float eps, const float *bias,
                          float *y, int64_t ldy, int epi, void *stream, const int64_t *y_ref = nullptr,
                          const ScoreSide *side = nullptr) {
    GemvArgs a{};
    a.side = side;
    a.w = static_cast<const uint8_t *>(w);
    a.nblk = (int)(cols / QK);
    a.soff = gemv_plain(dtype) ? 0 : scale_off(dtype, rows_packed, cols);
    a.n_rq = rows4(rows_packed) / 4;
    a.rows_out = rows_out;
    a.x = x;
    a.ldx = ldx;
    a.batch = batch;
    a.lnw = lnw;
    a.eps = eps;
    a.bias = bias;
    a.y = y;
    a.ldy = ldy;
    a.epi = epi;
    a.y_ref = y_ref;
    hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case VGX_Q8_0: return vgx_detail_qgemv_q8(a, st);
        case VGX_Q4_0: return vgx_detail_qgemv_q4(a, st);
        case VGX_F32: return vgx_detail_qgemv_f32(a, st);
        case VGX_BF16: return vgx_detail_qgemv_bf16(a, st);
        case VGX_F16: return vgx_detail_qgemv_f16(a, st);
    }
    return VGX_E_DTYPE;
}

int vgx_qlinear_ex(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                   int64_t batch, const float *norm_w, float eps, const float *bias, float *y, int64_t ldy,
                   int epilogue, void *stream) {
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!w_packed || !x || !y) return VGX_E_ARG;
    if (epilogue != VGX_EPI_STORE && epilogue != VGX_EPI_ACCUM && epilogue != VGX_EPI_SWIGLU) return VGX_E_ARG;
    if (epilogue == VGX_EPI_SWIGLU && bias) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || batch < 0 || ldx < cols || ldy < rows) return VGX_E_SIZE;
    if (cols % QK || (epilogue == VGX_EPI_SWIGLU && rows % 2)) return VGX_E_SHAPE;
    if (cols / QK > (1 << 24)) return VGX_E_LIMIT;
    if (norm_w && !(eps > 0.0f)) return VGX_E_ARG;
    if (batch == 0) return VGX_OK;
    const int64_t rows_packed = epilogue == VGX_EPI_SWIGLU ? 2 * rows : rows;
    return qgemv_dispatch(dtype, w_packed, rows_packed, rows, cols, x, ldx, batch, norm_w, eps, bias, y, ldy,
                          epilogue, stream);
}

int vgx_qlinear_side(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                     int64_t batch, const float *norm_w, float eps, const float *bias, float *y, int64_t ldy,
                     int epilogue, const vgx_score_side *side, void *stream) {
    if (!side)
        return vgx_qlinear_ex(dtype, w_packed, rows, cols, x, ldx, batch, norm_w, eps, bias, y, ldy, epilogue, stream);
    ScoreSide sj;
    const int rc = make_score_side(*side, sj);
    if (rc != VGX_OK) return rc;
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!w_packed || !x || !y) return VGX_E_ARG;
    if (epilogue != VGX_EPI_STORE && epilogue != VGX_EPI_ACCUM && epilogue != VGX_EPI_SWIGLU) return VGX_E_ARG;
    if (epilogue == VGX_EPI_SWIGLU && bias) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || batch < 0 || ldx < cols || ldy < rows) return VGX_E_SIZE;
    if (cols % QK || (epilogue == VGX_EPI_SWIGLU && rows % 2)) return VGX_E_SHAPE;
    if (cols / QK > (1 << 24)) return VGX_E_LIMIT;
    if (norm_w && !(eps > 0.0f)) return VGX_E_ARG;
    if (batch == 0) return vgx_detail_score_side(sj, (hipStream_t)stream);
    const int64_t rows_packed = epilogue == VGX_EPI_SWIGLU ? 2 * rows : rows;
    return qgemv_dispatch(dtype, w_packed, rows_packed, rows, cols, x, ldx, batch, norm_w, eps, bias, y, ldy, epilogue,
                          stream, nullptr, &sj);
}

int vgx_qlinear_indirect(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                         int64_t batch, const float *norm_w, float eps, const float *bias, const int64_t *y_addr,
                         int64_t ldy, int epilogue, void *stream) {
    if (!y_addr) return VGX_E_ARG;
    if (reinterpret_cast<uintptr_t>(y_addr) % 8) return VGX_E_ALIGN;
    if (!dtype_ok(dtype)) return VGX_E_DTYPE;
    if (!w_packed || !x) return VGX_E_ARG;
    if (epilogue != VGX_EPI_STORE && epilogue != VGX_EPI_ACCUM && epilogue != VGX_EPI_SWIGLU) return VGX_E_ARG;
    if (epilogue == VGX_EPI_SWIGLU && bias) return VGX_E_ARG;
    if (rows <= 0 || cols <= 0 || batch < 0 || ldx < cols || ldy < rows) return VGX_E_SIZE;
    if (cols % QK || (epilogue == VGX_EPI_SWIGLU && rows % 2)) return VGX_E_SHAPE;
    if (cols / QK > (1 << 24)) return VGX_E_LIMIT;
    if (norm_w && !(eps > 0.0f)) return VGX_E_ARG;
    if (batch == 0) return VGX_OK;
    const int64_t rows_packed = epilogue == VGX_EPI_SWIGLU ? 2 * rows : rows;
    // the launch geometry never depends on y: a placeholder address stands in until the kernel reads *y_addr
    return qgemv_dispatch(dtype, w_packed, rows_packed, rows, cols, x, ldx, batch, norm_w, eps, bias, nullptr, ldy,
                          epilogue, stream, y_addr);
}

int vgx_qlinear(int dtype, const void *w_packed, int64_t rows, int64_t cols, const float *x, int64_t ldx,
                int64_t batch, const float *bias, float *y, int64_t ldy, int accumulate, void *stream) {
    if (accumulate != 0 && accumulate != 1) return VGX_E_ARG;
    return vgx_qlinear_ex(dtype, w_packed, rows, cols, x, ldx, batch, nullptr, 0.0f, bias, y, ldy,
                          accumulate ? VGX_EPI_ACCUM : VGX_EPI_STORE, stream);
}

int vgx_qlinear_swiglu(int dtype, const void *w_gateup_packed, int64_t rows, int64_t cols, const float *x,
                       int64_t ldx, int64_t batch, float *h, int64_t ldh, void *stream) {
    return vgx_qlinear_ex(dtype, w_gateup_packed, rows, cols, x, ldx, batch, nullptr, 0.0f, nullptr, h, ldh,
                          VGX_EPI_SWIGLU, stream);
}

}  // extern "C"
