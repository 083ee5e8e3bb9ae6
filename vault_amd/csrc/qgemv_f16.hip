// F16 instantiation of the GEMV kernels (qgemv.h).
#include "qgemv.h"

int vgx_detail_qgemv_f16(const vgx::GemvArgs &a, hipStream_t st) { return vgx::qgemv_launch<VGX_F16>(a, st); }
