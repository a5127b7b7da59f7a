// C-ABI plumbing: error reporting, version, and a device probe of the scalar
// math used by the kernels (for bitwise tests against the CPU oracle).
#include <cstring>

#include "rkv_common.h"
#include "rkv_internal.h"

namespace rkv {

namespace {
thread_local char g_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

namespace {

__global__ void math_probe_kernel(int fn, const float* __restrict__ x, float* __restrict__ y,
                                  int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  float r;
  switch (fn) {
    case 0: r = expf_(v); break;
    case 1: r = logf_(v); break;
    case 2: r = round_bf16(v); break;
    case 3: r = sqrtf(v); break;
    case 4: r = exp_hw(v); break;
    default: r = log_hw(v); break;
  }
  y[i] = r;
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" const char* rkv_last_error(void) { return g_error; }

extern "C" int rkv_version(void) { return 2; }

// Applies a device scalar function elementwise: fn 0 = exp (expf_), 1 = log
// (logf_), 2 = bfloat16 round trip, 3 = sqrt, 4 = exp_hw, 5 = log_hw.  x and
// y are device arrays of n floats.
extern "C" int rkv_math_probe(int fn, const float* x, float* y, int64_t n, hipStream_t stream) {
  clear_error();
  if (!x || !y || n < 0 || fn < 0 || fn > 5)
    return set_error(kInvalidArgument, "rkv_math_probe: bad arguments");
  if (n == 0) return kOk;
  const int64_t blocks = (n + 255) / 256;
  math_probe_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(fn, x, y, n);
  return check_launch("math_probe_kernel");
}
