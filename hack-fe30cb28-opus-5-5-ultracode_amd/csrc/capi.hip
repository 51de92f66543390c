// Library-level entry points: version and error strings.
#include "common.h"

QLORA_API const char* qlora_error_string(int code) {
  return hipGetErrorString((hipError_t)code);
}

QLORA_API int qlora_abi_version() { return 1; }
