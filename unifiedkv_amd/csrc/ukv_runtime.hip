// Library-wide entry points of libukv.so: version, status text, and the strided
// host <-> device copy used by the pinned page arena.
#include <hip/hip_runtime.h>

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

extern "C" int ukv_copy_2d(void* dst, size_t dst_pitch, const void* src, size_t src_pitch, size_t width,
                           size_t height, ukv_stream_t stream) {
  if (width == 0 || height == 0) return UKV_OK;
  if (!dst || !src || dst_pitch < width || src_pitch < width) return UKV_ERR_INVALID_ARGUMENT;
  const hipError_t e = hipMemcpy2DAsync(dst, dst_pitch, src, src_pitch, width, height, hipMemcpyDefault,
                                        reinterpret_cast<hipStream_t>(stream));
  return e == hipSuccess ? UKV_OK : UKV_ERR_LAUNCH;
}
