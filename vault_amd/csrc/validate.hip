// Load-time validation on the device: count the non-finite values of an uploaded VLT3 payload.
//
// Reference semantics: check_tensor_finite (runtime/vault3.c:215-271) rejects a tensor when any F32
// / F16 / BF16 element, or any Q8_0 / Q4_0 block scale (the fp16 word at the head of each 34- or
// 18-byte block), has its exponent field all ones (Inf or NaN).  The quants themselves are integers
// and always finite.
#include "common.h"

using namespace vgx;

namespace {

// One element (or one block scale) per thread, grid-stride.
template <int DT>
__global__ void nonfinite_kernel(const uint8_t *__restrict__ p, int64_t n_items, uint32_t *__restrict__ count) {
    uint32_t bad = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_items;
         i += (int64_t)gridDim.x * blockDim.x) {
        if constexpr (DT == VGX_F32) {
            const uint32_t u = reinterpret_cast<const uint32_t *>(p)[i];
            bad += (u & 0x7F800000u) == 0x7F800000u;
        } else if constexpr (DT == VGX_F16) {
            const uint32_t u = reinterpret_cast<const uint16_t *>(p)[i];
            bad += (u & 0x7C00u) == 0x7C00u;
        } else if constexpr (DT == VGX_BF16) {
            const uint32_t u = reinterpret_cast<const uint16_t *>(p)[i];
            bad += (u & 0x7F80u) == 0x7F80u;
        } else {
            constexpr int64_t stride = DT == VGX_Q8_0 ? 34 : 18;
            const uint32_t u = (uint32_t)p[i * stride] | ((uint32_t)p[i * stride + 1] << 8);
            bad += (u & 0x7C00u) == 0x7C00u;
        }
    }
    // only lanes that found a non-finite value touch the counter (none for a valid file)
    if (bad) atomicAdd(count, bad);
}

template <int DT>
int launch(const void *data, int64_t n_items, uint32_t *count, hipStream_t s) {
    if (n_items == 0) return VGX_OK;
    const int64_t want = (n_items + 255) / 256;
    const unsigned grid = (unsigned)(want < 4096 ? want : 4096);
    nonfinite_kernel<DT><<<grid, 256, 0, s>>>(static_cast<const uint8_t *>(data), n_items, count);
    VGX_CHECK_LAUNCH();
    return VGX_OK;
}

}  // namespace

extern "C" int vgx_count_nonfinite(int dtype, const void *data, int64_t n_elems, uint32_t *count, void *stream) {
    if (!count || n_elems < 0 || (n_elems > 0 && !data)) return VGX_E_ARG;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (dtype) {
    case VGX_F32: return launch<VGX_F32>(data, n_elems, count, s);
    case VGX_F16: return launch<VGX_F16>(data, n_elems, count, s);
    case VGX_BF16: return launch<VGX_BF16>(data, n_elems, count, s);
    case VGX_Q8_0:
        if (n_elems % QK) return VGX_E_SHAPE;
        return launch<VGX_Q8_0>(data, n_elems / QK, count, s);
    case VGX_Q4_0:
        if (n_elems % QK) return VGX_E_SHAPE;
        return launch<VGX_Q4_0>(data, n_elems / QK, count, s);
    default: return VGX_E_DTYPE;
    }
}
