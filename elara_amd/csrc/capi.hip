// Library-wide C-ABI helpers: version and error text.
#include "elr_common.h"

extern "C" int elr_version(void) { return 100; }  // 0.1.0

extern "C" const char* elr_error_string(int code) {
  switch (code) {
    case ELR_OK:
      return "ok";
    case ELR_EINVAL:
      return "invalid argument (null pointer, negative size or inconsistent shape)";
    case ELR_EUNSUPPORTED:
      return "argument outside this build's limits";
    case ELR_ECAPACITY:
      return "caller-provided scratch or output buffer too small";
    default:
      return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}
