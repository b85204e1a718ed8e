// Shared helpers for the tt-atom MI355X (gfx950) kernels: status codes, the thread-local error
// message behind tta_last_error(), launch checks and small device utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdarg.h>

namespace tta {

// Thread-local last-error text; every extern "C" entry point returns 0 on success and a
// non-zero status after writing a message here.
void set_error(const char* fmt, ...);

enum Status : int {
  kOk = 0,
  kBadArgument = 1,
  kLaunchFailed = 2,
  kUnsupported = 3,
};

}  // namespace tta

#define TTA_CHECK_ARG(cond, ...)                 \
  do {                                           \
    if (!(cond)) {                               \
      tta::set_error(__VA_ARGS__);               \
      return tta::kBadArgument;                  \
    }                                            \
  } while (0)

#define TTA_CHECK_LAUNCH(name)                                                   \
  do {                                                                           \
    hipError_t _e = hipGetLastError();                                           \
    if (_e != hipSuccess) {                                                      \
      tta::set_error("%s: launch failed: %s", name, hipGetErrorString(_e));      \
      return tta::kLaunchFailed;                                                 \
    }                                                                            \
  } while (0)

// ---------------------------------------------------------------------------- device helpers
__device__ __forceinline__ float tta_sigmoid(float x) { return 1.0f / (1.0f + __expf(-x)); }

// SiLU with an accurate exp: the parity tolerance of the force path is tight, so the
// transcendental functions use the full-precision library versions (expf, not __expf).
__device__ __forceinline__ float tta_sigmoid_acc(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float tta_silu(float x) { return x * tta_sigmoid_acc(x); }
// d silu / dx = s (1 + x (1 - s))
__device__ __forceinline__ float tta_silu_grad(float x) {
  float s = tta_sigmoid_acc(x);
  return s * (1.0f + x * (1.0f - s));
}

// Butterfly sum over `width` consecutive lanes (width a power of two <= 64).
__device__ __forceinline__ float tta_group_sum(float v, int width) {
  for (int o = width >> 1; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

static inline unsigned tta_blocks(int64_t n, int per) {
  return (unsigned)((n + per - 1) / per);
}
