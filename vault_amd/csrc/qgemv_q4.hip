// Q4_0 instantiation of the GEMV kernels (qgemv.h).
#include "qgemv.h"

int vgx_detail_qgemv_q4(const vgx::GemvArgs &a, hipStream_t st) { return vgx::qgemv_launch<VGX_Q4_0>(a, st); }
