// Host-side helpers shared by the C-ABI translation units: argument checks
// that record a message and return LFM25_EINVAL, and launch checks that map
// HIP runtime failures to LFM25_EDEVICE.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "lfm25_hip.h"  // include/ (on the compiler include path)

namespace lfm25 {

int set_error(int code, const char* fmt, ...);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(LFM25_EDEVICE, "%s: %s", what, hipGetErrorString(e));
  return LFM25_OK;
}

}  // namespace lfm25

#define LFM25_REQUIRE(cond, ...)                                   \
  do {                                                             \
    if (!(cond)) return ::lfm25::set_error(LFM25_EINVAL, __VA_ARGS__); \
  } while (0)
