// Scalar fp32 arithmetic shared by every RefineKV kernel.
//
// Every function here uses only IEEE-754 basic operations (add, sub, mul,
// div, sqrt: each correctly rounded on gfx950 with this project's flags) and
// explicit fmaf.  The files are compiled with -ffp-contract=off, so no other
// fused operation appears.  The result of each function is therefore a fixed
// function of its inputs, independent of the device it runs on; a CPU
// restatement written with the same steps reproduces it bit for bit.
//
// exp/log follow textbook methods (named at each function) with Taylor
// coefficients; they are accurate to about 1 ulp, which is what the
// reference's fp32 torch ops provide (src/refinekv/reference.py:14-34).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define RKV_HD __host__ __device__ __forceinline__
#else
#include <math.h>
#include <string.h>
#define RKV_HD static inline
#endif

namespace rkv {

RKV_HD uint32_t f32_bits(float x) {
  uint32_t u;
  __builtin_memcpy(&u, &x, 4);
  return u;
}

RKV_HD float bits_f32(uint32_t u) {
  float x;
  __builtin_memcpy(&x, &u, 4);
  return x;
}

RKV_HD bool is_nan(float x) { return !(x == x); }

RKV_HD bool is_finite(float x) { return (f32_bits(x) & 0x7F800000u) != 0x7F800000u; }

// Round an fp32 value to bfloat16 (round to nearest, ties to even).  NaN maps
// to the canonical quiet NaN 0x7FC0, as torch's float->bfloat16 cast does
// (c10/util/BFloat16.h round_to_nearest_even).
RKV_HD uint16_t bf16_rne(float x) {
  if (is_nan(x)) return (uint16_t)0x7FC0u;
  uint32_t u = f32_bits(x);
  uint32_t bias = 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)((u + bias) >> 16);
}

RKV_HD float bf16_to_f32(uint16_t h) { return bits_f32((uint32_t)h << 16); }

// bfloat16 round trip: the fp32 value of bf16(x).
RKV_HD float round_bf16(float x) { return bf16_to_f32(bf16_rne(x)); }

// fp16 -> fp32, exact (used when the KV cache is half precision).
RKV_HD float f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  if (exp == 0x1Fu) return bits_f32(sign | 0x7F800000u | (man << 13));
  if (exp == 0) {
    if (man == 0) return bits_f32(sign);
    // subnormal half: value = man * 2^-24, exact in fp32
    float v = (float)man * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

// max/min that propagate NaN like torch.amax/amin/maximum.
RKV_HD float nanmax(float a, float b) { return (a > b || is_nan(a)) ? a : b; }
RKV_HD float nanmin(float a, float b) { return (a < b || is_nan(a)) ? a : b; }

// torch.clamp_min / clamp(max=) keep NaN.
RKV_HD float clamp_min(float x, float lo) { return x < lo ? lo : x; }
RKV_HD float clamp_max(float x, float hi) { return x > hi ? hi : x; }

// 2^k * p for |k| in the range exp() produces, with a single rounding.
RKV_HD float scale_pow2(float p, int k) {
  if (k > 127) {
    p = p * bits_f32(0x7F000000u);  // 2^127
    k -= 127;
  } else if (k < -126) {
    p = p * bits_f32((uint32_t)(k + 64 + 127) << 23);  // exact: stays normal
    return p * bits_f32((uint32_t)(-64 + 127) << 23);  // one rounding
  }
  return p * bits_f32((uint32_t)(k + 127) << 23);
}

// exp(x): Cody & Waite argument reduction x = k*ln2 + r (two-part ln2, with
// fma so k*ln2_hi is exact), then the degree-7 Taylor polynomial of e^r on
// |r| <= ln2/2 (truncation 5e-9 relative), then an exact scale by 2^k.
// exp(0) == 1 exactly; exp(-inf) == 0; exp(+inf) == +inf.
//
// The device build takes the main path in every lane (on an argument
// clamped to [-104, 88.8], which leaves every input of the main path
// unchanged) and selects the special cases after, so no lane branches; the
// results equal the host build's early returns bit for bit.
RKV_HD float expf_(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float xs = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 88.8f);
#else
  if (is_nan(x)) return x + x;
  if (x > 88.8f) return bits_f32(0x7F800000u);
  if (x < -104.0f) return 0.0f;
  const float xs = x;
#endif
  float k = __builtin_rintf(xs * 1.44269504088896341f);
  float r = __builtin_fmaf(k, -0.693145751953125f, xs);
  r = __builtin_fmaf(k, -1.42860682030941723e-06f, r);
  float p = 1.98412698412698413e-04f;         // 1/7!
  p = __builtin_fmaf(p, r, 1.38888888888888889e-03f);  // 1/6!
  p = __builtin_fmaf(p, r, 8.33333333333333333e-03f);  // 1/5!
  p = __builtin_fmaf(p, r, 4.16666666666666667e-02f);  // 1/4!
  p = __builtin_fmaf(p, r, 1.66666666666666667e-01f);  // 1/3!
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
#if defined(__HIP_DEVICE_COMPILE__)
  // v_ldexp_f32 rounds once, exactly as scale_pow2's exact-then-rounded
  // multiplies do.  The clamped ends need no select of their own: at
  // xs = 88.8 (k = 128, p > 1) the scale overflows to +inf, and at
  // xs = -104 (k = -150, p < 0.98) it rounds to +0, the host's results for
  // x > 88.8 and x < -104.  Only NaN (clamped to -104 by fmaxf) is selected.
  const float y = __builtin_amdgcn_ldexpf(p, (int)k);
  return is_nan(x) ? x + x : y;
#else
  return scale_pow2(p, (int)k);
#endif
}

// log(x): the reduction of fdlibm's e_log.c (Sun Microsystems, 1993):
// x = 2^e * m with m in [sqrt(2)/2, sqrt(2)), f = m - 1, s = f / (2 + f),
// log(1 + f) = f - (hfsq - s*(hfsq + R(s^2))) with hfsq = f^2/2 and R the
// Taylor series of 2*atanh(s)/s - 2 - ... truncated after s^8 (2/3, 2/5,
// 2/7, 2/9).  log(1) == +0 exactly; log(0) == -inf; log(x<0) == NaN.
//
// The device build runs the main path in every lane and, when any lane of
// the wave holds a special input (NaN, <= 0, +inf), selects the special
// results after.  It splits x with v_frexp_mant / v_frexp_exp (x = mant 2^ef,
// mant in [0.5, 1), subnormals included): m = 2 mant and e = ef - 1 are the
// host's m in [1, 2) and e, and its halving step (m > sqrt 2) is mant >
// sqrt(2) / 2 (the same float constant halved, exactly), keeping m = mant and
// e = ef.
RKV_HD float logf_(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  const float mant = __builtin_amdgcn_frexp_mantf(x);
  const int ef = __builtin_amdgcn_frexp_expf(x);
  const bool hi = mant > 0.5f * 1.41421356237309505f;
  const float m = hi ? mant : mant + mant;
  const int e = hi ? ef : ef - 1;
#else
  if (is_nan(x)) return x + x;
  if (x < 0.0f) return bits_f32(0x7FC00000u);
  if (x == 0.0f) return bits_f32(0xFF800000u);
  if (x == bits_f32(0x7F800000u)) return x;
  uint32_t u = f32_bits(x);
  int e = 0;
  if (u < 0x00800000u) {  // subnormal
    x = x * 8388608.0f;
    u = f32_bits(x);
    e = -23;
  }
  e += (int)(u >> 23) - 127;
  float m = bits_f32((u & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421356237309505f) {
    m = m * 0.5f;
    e += 1;
  }
#endif
  float f = m - 1.0f;
  float s = f / (2.0f + f);
  float s2 = s * s;
  float R = 0.222222222222222222f;              // 2/9
  R = __builtin_fmaf(R, s2, 0.285714285714285714f);  // 2/7
  R = __builtin_fmaf(R, s2, 0.4f);                   // 2/5
  R = __builtin_fmaf(R, s2, 0.666666666666666667f);  // 2/3
  R = R * s2;
  float hfsq = 0.5f * f * f;
  float dk = (float)e;
  const float y = dk * 0.693145751953125f -
                  ((hfsq - (s * (hfsq + R) + dk * 1.42860682030941723e-06f)) - f);
#if defined(__HIP_DEVICE_COMPILE__)
  // the host build's early returns, lowest priority first
  float r = y;
  if (__builtin_amdgcn_ballot_w64(!(x > 0.0f) || x == bits_f32(0x7F800000u)) != 0) {
    r = x == bits_f32(0x7F800000u) ? x : r;
    r = x == 0.0f ? bits_f32(0xFF800000u) : r;
    r = x < 0.0f ? bits_f32(0x7FC00000u) : r;
    r = is_nan(x) ? x + x : r;
  }
  return r;
#else
  return y;
#endif
}

}  // namespace rkv
