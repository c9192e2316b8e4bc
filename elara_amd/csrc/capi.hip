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

// Device-visible address of pinned host memory (hipHostMalloc'd, e.g. torch's pin_memory tensors): the capacity
// tier keeps the MAT and log arenas there and the kernels read and write them over the host link.  Fails (with the
// HIP error) for memory that is not pinned and mapped, so no kernel is ever handed an address it cannot reach.
extern "C" int elr_host_device_ptr(const void* host, void** dev) {
  if (!host || !dev) return ELR_EINVAL;
  *dev = nullptr;
  void* d = nullptr;
  const hipError_t e = hipHostGetDevicePointer(&d, const_cast<void*>(host), 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return (int)e;
  }
  *dev = d;
  return ELR_OK;
}
