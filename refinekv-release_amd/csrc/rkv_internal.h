// Host-side helpers shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

namespace rkv {

// Error codes returned by every entry point (0 = success).
enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kUnsupported = 2,
  kLaunchFailed = 3,
  kWorkspaceTooSmall = 4,
};

int set_error(int code, const char* fmt, ...);
void clear_error();

// Head dimensions with compiled kernels: 32..256 in steps of 32, as the
// reference's accelerated backend accepts (src/refinekv/attention.py:29-33).
inline bool supported_dim(int64_t d) { return d >= 32 && d <= 256 && d % 32 == 0; }
inline bool supported_block(int64_t b) { return b == 16 || b == 32 || b == 64; }

#define RKV_DISPATCH_DIM(dim, D, ...)                        \
  switch (dim) {                                             \
    case 32: { constexpr int D = 32; __VA_ARGS__; break; }   \
    case 64: { constexpr int D = 64; __VA_ARGS__; break; }   \
    case 96: { constexpr int D = 96; __VA_ARGS__; break; }   \
    case 128: { constexpr int D = 128; __VA_ARGS__; break; } \
    case 160: { constexpr int D = 160; __VA_ARGS__; break; } \
    case 192: { constexpr int D = 192; __VA_ARGS__; break; } \
    case 224: { constexpr int D = 224; __VA_ARGS__; break; } \
    case 256: { constexpr int D = 256; __VA_ARGS__; break; } \
    default: break;                                          \
  }

inline int check_launch(const char* what) {
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return set_error(kLaunchFailed, "%s: %s", what, hipGetErrorString(err));
  return kOk;
}

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }

}  // namespace rkv
