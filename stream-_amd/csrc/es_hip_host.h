// Shared by the library's host files: error reporting into es_hip_last_error() and the gfx950 device check
// (defined in es_hip_quant.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace esq {
int host_fail(int code, const char *msg);              // records msg, returns code
int host_hip_fail(hipError_t e, const char *what);     // ES_HIP_ENOMEM or ES_HIP_ERUNTIME with HIP's message
int host_need_device();                                // ES_HIP_OK, or ES_HIP_ENODEV with the reason recorded
}  // namespace esq
