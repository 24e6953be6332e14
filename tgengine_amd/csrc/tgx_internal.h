// Internal helpers shared by the libtgx translation units (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include "tgx.h"

namespace tgx {

constexpr int kWave = 64;

// thread-local message of the last failure (returned by tgx_last_error)
void set_error(const char* fmt, ...);

inline int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  set_error("%s", buf);
  return code;
}

inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TGX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return TGX_OK;
}

inline int feat_elem_bytes(int dtype) { return dtype == TGX_F32 ? 4 : (dtype == TGX_BF16 ? 2 : 0); }

// 16-byte aligned?
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace tgx
