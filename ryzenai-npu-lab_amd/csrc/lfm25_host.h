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

// The persistent batched decode (lfm25_decode.hip) behind lfm25_batch_decode:
// the bytes it keeps in the batch workspace after the batched pass's, and
// the call itself, which returns kBatchNotPersistent when it does not serve
// the call (batch size, positions, device or LFM25_BATCH_PERSISTENT=0), so
// the batched pass runs it instead. With `prefix` it may serve only the
// call's first steps (16 sequences: those below 256 positions); *done is the
// number of steps it ran.
constexpr int kBatchNotPersistent = -1;
size_t batch_persistent_bytes();
int batch_decode_persistent(const lfm25_batch* b, void* region, int32_t* status, const int32_t* tokens_in,
                            const int32_t* positions, int32_t n_steps, int32_t* tokens_out, uint16_t* hidden_out,
                            hipStream_t s, bool prefix, int32_t* done);

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
