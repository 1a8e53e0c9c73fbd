// Library-level C entry points: ABI version and status strings.
#include "dash_common.h"

extern "C" int dash_abi_version(void) { return 1; }

extern "C" const char* dash_status_string(int status) {
  switch (status) {
    case dash::kOk: return "ok";
    case dash::kErrUnsupported: return "unsupported shape or parameter";
    case dash::kErrInvalid: return "invalid argument";
    case dash::kErrWorkspace: return "workspace too small";
    case dash::kErrScratch:
      return "sizes exceed the fixed 64 MiB scratch of the allocation-free entry point";
    default: break;
  }
  if (status > 0) return hipGetErrorString((hipError_t)status);
  return "unknown status";
}
