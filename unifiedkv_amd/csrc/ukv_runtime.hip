// Library-wide entry points of libukv.so: version and status text.
#include "../../include/ukv.h"

extern "C" int ukv_version(void) { return (0 << 16) | (1 << 8) | 0; }

extern "C" const char* ukv_status_string(int status) {
  switch (status) {
    case UKV_OK: return "ok";
    case UKV_ERR_INVALID_ARGUMENT: return "invalid_argument";
    case UKV_ERR_EMPTY: return "empty";
    case UKV_ERR_GQA: return "gqa";
    case UKV_ERR_HEAD_DIM: return "head_dim";
    case UKV_ERR_DTYPE: return "dtype";
    case UKV_ERR_WORKSPACE: return "workspace";
    case UKV_ERR_LAUNCH: return "launch";
    case UKV_ERR_NO_DEVICE: return "no_device";
    default: return "unknown";
  }
}
