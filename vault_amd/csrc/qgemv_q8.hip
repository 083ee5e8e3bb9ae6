// Q8_0 instantiation of the GEMV kernels (qgemv.h).
#include "qgemv.h"

int vgx_detail_qgemv_q8(const vgx::GemvArgs &a, hipStream_t st) { return vgx::qgemv_launch<VGX_Q8_0>(a, st); }
