// Library-level entry points: version and error strings.
#include "common.h"

// Codes from 300000 up are the library's own (QLORA_ERR_*); below are hipError_t values.
QLORA_API const char* qlora_error_string(int code) {
  if (code == QLORA_ERR_SCRATCH_TOO_SMALL)
    return "qlora: the problem needs more scratch than the allocation-free entry point's static "
           "buffer holds; call the entry point that takes a workspace";
  if (code >= 300000) return "qlora: error";
  return hipGetErrorString((hipError_t)code);
}

QLORA_API int qlora_abi_version() { return 1; }
