// Library-wide C entry points: error strings and version.
#include "common.hpp"

extern "C" const char* musc_strerror(int code) {
  switch (code) {
    case MUSC_OK: return "success";
    case MUSC_ERR_INVALID_ARG: return "musc: invalid argument (shape, rank window, pointer or alignment)";
    case MUSC_ERR_WORKSPACE: return "musc: workspace is missing or smaller than required";
    case MUSC_ERR_UNSUPPORTED: return "musc: shape outside the implemented range";
    case MUSC_ERR_SCRATCH_LIMIT:
      return "musc: the problem's workspace exceeds the no-allocation scratch (MUSC_NOALLOC_SCRATCH_BYTES = 256 MiB); "
             "use the entry point that takes a workspace";
    default: break;
  }
  if (code > 0 && code < 1000) return hipGetErrorString(static_cast<hipError_t>(code));
  return "musc: unknown error code";
}

extern "C" int musc_version(void) { return 100; }

#ifndef MUSC_TARGET_ARCH
#error "build with -DMUSC_TARGET_ARCH=\"<offload arch>\" (musc_hip/build.py passes it)"
#endif
extern "C" const char* musc_target_arch(void) { return MUSC_TARGET_ARCH; }
