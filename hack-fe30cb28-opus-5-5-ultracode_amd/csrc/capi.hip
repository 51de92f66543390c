// Library-level entry points: version and error strings.
#include "common.h"

#include <rocblas/rocblas.h>

// Codes from 300000 up are the library's own (QLORA_ERR_*), from 200000 up hipBLASLt statuses (qlora_gemmlt*), from 100000 up rocBLAS statuses
// (qlora_gemm*), below are hipError_t values.
QLORA_API const char* qlora_error_string(int code) {
  if (code == QLORA_ERR_SCRATCH_TOO_SMALL)
    return "qlora: the problem needs more scratch than the allocation-free entry point's static "
           "buffer holds; call the entry point that takes a workspace";
  if (code >= 300000) return "qlora: error";
  if (code >= 200000) {
    switch (code - 200000) {
      case 1: return "hipBLASLt: not initialized";
      case 2: return "hipBLASLt: allocation failed";
      case 3: return "hipBLASLt: invalid value";
      case 4: return "hipBLASLt: mapping error";
      case 5: return "hipBLASLt: execution failed";
      case 6: return "hipBLASLt: internal error";
      case 7: return "hipBLASLt: not supported";
      case 8: return "hipBLASLt: architecture mismatch";
      default: return "hipBLASLt: error";
    }
  }
  if (code >= 100000) return rocblas_status_to_string((rocblas_status)(code - 100000));
  return hipGetErrorString((hipError_t)code);
}

QLORA_API int qlora_abi_version() { return 1; }
