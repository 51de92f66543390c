// Library-level entry points: version and error strings.
#include "common.h"

#include <rocblas/rocblas.h>

// Codes from 100000 up are rocBLAS statuses (qlora_gemm*), below are hipError_t values.
QLORA_API const char* qlora_error_string(int code) {
  if (code >= 100000) return rocblas_status_to_string((rocblas_status)(code - 100000));
  return hipGetErrorString((hipError_t)code);
}

QLORA_API int qlora_abi_version() { return 1; }
