// Library-level C entry points: version and status text.
#include "wgkv_common.h"

extern "C" int wgkv_version(void) { return 1; }

extern "C" const char* wgkv_status_string(int status) {
  switch (status) {
    case WGKV_OK: return "ok";
    case WGKV_ERR_ARG: return "invalid argument";
    case WGKV_ERR_UNSUPPORTED: return "unsupported shape or layout";
    case WGKV_ERR_CAPACITY: return "cache capacity exceeded";
    case WGKV_ERR_WORKSPACE: return "workspace missing or too small";
    case WGKV_ERR_HIP: return "HIP runtime error";
    default: return "unknown status";
  }
}
