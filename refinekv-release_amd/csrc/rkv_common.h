// Device-side building blocks shared by the RefineKV kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rkv_math.h"

namespace rkv {

constexpr int kWave = 64;
constexpr int kTile = 64;             // blocks per log-sum-exp tile (one per lane)
constexpr int kMaxGroup = 16;         // query heads per KV head
constexpr float kDeltaMax = 10.0f;    // reference.py:20 switch between risk branches
constexpr float kInflate = 1.00390625f;  // 1 + 2^-8 (reference.py:16, summary.py:96)
constexpr float kLn2 = 0.693147182464599609375f;  // fp32(math.log(2))
constexpr float kLog2e = 1.44269504088896341f;    // fp32(1 / math.log(2))
constexpr float kNegInf = -__builtin_inff();
constexpr float kPosInf = __builtin_inff();

// e^x and log x on the hardware's transcendental unit: v_exp_f32 (2^x) and
// v_log_f32 (log2 x), about an ulp each, scaled by fp32 log2(e) and ln(2).
// Against exact e^x the rounding of x log2(e) adds about |x| 2^-24
// relative; log x is off by a few 2^-24 absolute plus an ulp.  Special
// values as expf_ / logf_: e^-inf = 0, e^+inf = +inf, log 0 = -inf, log of a
// negative = NaN, NaN in, NaN out.
__device__ __forceinline__ float exp_hw(float x) { return __builtin_amdgcn_exp2f(x * kLog2e); }
__device__ __forceinline__ float log_hw(float x) { return __builtin_amdgcn_logf(x) * kLn2; }

// Reduction codes of runtime.py:23.
enum Reduction { kMean = 0, kMax = 1, kAny = 2 };

// threadIdx.x as a value the compiler cannot hoist out of an enclosing loop:
// in a persistent kernel each work item recomputes its per-thread index math
// instead of keeping every item kind's hoisted copies live across the loop.
__device__ __forceinline__ int item_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

__device__ __forceinline__ float shfl_xor(float v, int mask) { return __shfl_xor(v, mask, kWave); }
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, kWave); }

// Sum over the 16 lanes of a lane group, xor butterfly with distances 8,4,2,1.
// Every lane of the group ends with the same value (fp32 add commutes).
__device__ __forceinline__ float group16_sum(float v) {
  v = v + shfl_xor(v, 8);
  v = v + shfl_xor(v, 4);
  v = v + shfl_xor(v, 2);
  v = v + shfl_xor(v, 1);
  return v;
}

// Sum over the wave, xor butterfly with distances 32..1.
__device__ __forceinline__ float wave_sum(float v) {
  v = v + shfl_xor(v, 32);
  v = v + shfl_xor(v, 16);
  v = v + shfl_xor(v, 8);
  v = v + shfl_xor(v, 4);
  v = v + shfl_xor(v, 2);
  v = v + shfl_xor(v, 1);
  return v;
}

__device__ __forceinline__ float wave_nanmax(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = nanmax(v, shfl_xor(v, o));
  return v;
}

__device__ __forceinline__ float wave_nanmin(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = nanmin(v, shfl_xor(v, o));
  return v;
}

// DPP row_shr:N -- lane i of each 16-lane row reads lane i-N of the same row
// (lanes i < N read 0).  A register move fused into the consuming VALU op.
template <int N>
__device__ __forceinline__ float row_shr(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x110 + N, 0xF, 0xF, false));
}

// Sum of each 16-lane row in the xor-butterfly tree (distances 8, 4, 2, 1:
// P[j] <- P[j] + P[j^o]).  Lane 15 of the row computes exactly the tree the
// butterfly leaves in lane 0 (operands commuted, which fp32 add ignores);
// other lanes hold partial sums.
__device__ __forceinline__ float row16_sum_last(float v) {
  v = v + row_shr<8>(v);
  v = v + row_shr<4>(v);
  v = v + row_shr<2>(v);
  v = v + row_shr<1>(v);
  return v;
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Cross-row butterfly steps without LDS (gfx950 v_permlane32_swap /
// v_permlane16_swap, which exchange lanes 32-63 of the first register with
// lanes 0-31 of the second, or the odd 16-lane rows of the first with the
// even rows of the second).  Swapping a value with a copy of itself leaves
// {x_l, x_(l^32)} (or {x_l, x_(l^16)}) in the two registers of every lane l,
// so op(a, b) is the xor-butterfly step in every lane (for a commutative op,
// bit-identical in both lanes of each pair).  Inline asm: both registers are
// results of the swap (the compiler builtin returns the first one twice).
// The s_nop covers the VALU-write -> permlane-read hazard.
__device__ __forceinline__ void xor32_pair(float v, float& a, float& b) {
  a = v;
  b = v;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

__device__ __forceinline__ void xor16_pair(float v, float& a, float& b) {
  a = v;
  b = v;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}

// DPP row_ror:N -- lane i of each 16-lane row reads lane (i + N) mod 16.
template <int N>
__device__ __forceinline__ float row_ror(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x120 + N, 0xF, 0xF, false));
}

// Sum of each 16-lane row in the xor-butterfly tree (distances 8, 4, 2, 1),
// in every lane of the row: rotating a vector of period 2k by k pairs lane i
// with lane i^k.
__device__ __forceinline__ float row16_sum_all(float v) {
  v = v + row_ror<8>(v);
  v = v + row_ror<4>(v);
  v = v + row_ror<2>(v);
  v = v + row_ror<1>(v);
  return v;
}

// Wave-wide sum in the 64-lane xor-butterfly tree (distances 32..1),
// returned uniformly.  Bit-identical to the plain butterfly.
__device__ __forceinline__ float wave_sum_u(float v) {
  float a, b;
  xor32_pair(v, a, b);
  v = a + b;
  xor16_pair(v, a, b);
  v = a + b;
  return readlane(row16_sum_last(v), 15);
}

// NaN-propagating wave max, returned uniformly, with the NaN-propagating
// maximum (v_maximum3_f32, one instruction per step).  A maximum is exact,
// so the tree's shape does not matter; it differs from nanmax's only in the
// zero a +0/-0 tie returns (and in a NaN's payload).  Every caller uses the
// result m as a shift, exp(x - m), added back after a log, log(s) + m:
// x - (+0) and x - (-0) differ only for x = ±0, where exp gives 1 either way,
// and log(s) + (±0) are equal for every s (logf_ never returns -0), so no
// output depends on the tie.
__device__ __forceinline__ float wave_nanmax_u(float v) {
  float a, b;
  xor32_pair(v, a, b);
  v = __builtin_elementwise_maximum(a, b);
  xor16_pair(v, a, b);
  v = __builtin_elementwise_maximum(a, b);
  v = __builtin_elementwise_maximum(v, row_shr<8>(v));
  v = __builtin_elementwise_maximum(v, row_shr<4>(v));
  v = __builtin_elementwise_maximum(v, row_shr<2>(v));
  v = __builtin_elementwise_maximum(v, row_shr<1>(v));
  return readlane(v, 15);
}

// Broadcast lane 15 of each 16-lane row to the whole row.
__device__ __forceinline__ float row_bcast_last(float v) {
  const int lane = threadIdx.x % kWave;
  return __shfl(v, (lane & ~15) | 15, kWave);
}

__device__ __forceinline__ float finite_or_zero(float m) { return is_finite(m) || is_nan(m) ? m : 0.0f; }

// 16-byte aligned bf16 vector loads.
template <int N>
struct Bf16Vec {
  uint16_t v[N];
};

template <int N>
__device__ __forceinline__ void load_bf16(const uint16_t* __restrict__ p, float (&out)[N]) {
  static_assert(N % 2 == 0, "even element count");
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 8) {
      uint4 u = *reinterpret_cast<const uint4*>(p + i);
      uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        out[i + 2 * j] = bits_f32(w[j] << 16);
        out[i + 2 * j + 1] = bits_f32(w[j] & 0xFFFF0000u);
      }
    }
  } else if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      uint2 u = *reinterpret_cast<const uint2*>(p + i);
      out[i] = bits_f32(u.x << 16);
      out[i + 1] = bits_f32(u.x & 0xFFFF0000u);
      out[i + 2] = bits_f32(u.y << 16);
      out[i + 3] = bits_f32(u.y & 0xFFFF0000u);
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      uint32_t u = *reinterpret_cast<const uint32_t*>(p + i);
      out[i] = bits_f32(u << 16);
      out[i + 1] = bits_f32(u & 0xFFFF0000u);
    }
  }
}

// Raw 16-bit payload of N bf16 values, loaded with the widest aligned vector
// loads and unpacked later: keeping the load and the conversion apart lets
// every load of a batch be in flight before the first wait.
template <int N>
struct RawBf16 {
  static_assert(N % 2 == 0, "even element count");
  uint32_t w[N / 2];
};

template <int N>
__device__ __forceinline__ RawBf16<N> load_raw(const uint16_t* __restrict__ p) {
  RawBf16<N> r;
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int i = 0; i < N / 8; ++i) {
      const uint4 u = *reinterpret_cast<const uint4*>(p + 8 * i);
      r.w[4 * i] = u.x;
      r.w[4 * i + 1] = u.y;
      r.w[4 * i + 2] = u.z;
      r.w[4 * i + 3] = u.w;
    }
  } else if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N / 4; ++i) {
      const uint2 u = *reinterpret_cast<const uint2*>(p + 4 * i);
      r.w[2 * i] = u.x;
      r.w[2 * i + 1] = u.y;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N / 2; ++i) r.w[i] = *reinterpret_cast<const uint32_t*>(p + 2 * i);
  }
  return r;
}

template <int N>
__device__ __forceinline__ void unpack(const RawBf16<N>& r, float (&out)[N]) {
#pragma unroll
  for (int j = 0; j < N / 2; ++j) {
    out[2 * j] = bits_f32(r.w[j] << 16);
    out[2 * j + 1] = bits_f32(r.w[j] & 0xFFFF0000u);
  }
}

// Data handed from one workgroup to another inside a launch.  The two may
// run on different XCDs, each with its own L2, so a plain store can sit in
// the writer's L2 while the reader's L2 holds a stale line.  These accesses
// carry the sc1 cache-policy bit: stores write through to the device's point
// of coherence and loads read from it.  A writer makes its stores visible by
// waiting for them (s_waitcnt) before it bumps a counter; a reader that has
// seen the counter reach its target then loads with these accesses.  No L2
// write-back or invalidate is needed (an agent-scope fence costs both).
// Offsets are bytes from `base`; accesses past `bytes` read 0 and are dropped.
constexpr int kCoherentPolicy = 16;  // sc1

struct Coherent {
  __amdgpu_buffer_rsrc_t r;
  __device__ Coherent(const void* base, uint32_t bytes)
      : r(__builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                            0x00020000)) {}
  __device__ float4 load4(uint32_t off) const {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kCoherentPolicy);
    return make_float4(bits_f32(v[0]), bits_f32(v[1]), bits_f32(v[2]), bits_f32(v[3]));
  }
  __device__ float2 load2(uint32_t off) const {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kCoherentPolicy);
    return make_float2(bits_f32(v[0]), bits_f32(v[1]));
  }
  __device__ uint32_t load_u32(uint32_t off) const {
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kCoherentPolicy);
  }
  __device__ void store4(uint32_t off, float4 x) const {
    typedef unsigned int U4 __attribute__((ext_vector_type(4)));
    const U4 v = {f32_bits(x.x), f32_bits(x.y), f32_bits(x.z), f32_bits(x.w)};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, (int)off, 0, kCoherentPolicy);
  }
  __device__ void store2(uint32_t off, float2 x) const {
    typedef unsigned int U2 __attribute__((ext_vector_type(2)));
    const U2 v = {f32_bits(x.x), f32_bits(x.y)};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, kCoherentPolicy);
  }
  __device__ void store_u32(uint32_t off, uint32_t x) const {
    __builtin_amdgcn_raw_buffer_store_b32(x, r, (int)off, 0, kCoherentPolicy);
  }
  __device__ void store_u8(uint32_t off, uint8_t x) const {
    __builtin_amdgcn_raw_buffer_store_b8(x, r, (int)off, 0, kCoherentPolicy);
  }
  __device__ uint64_t load_u64(uint32_t off) const {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kCoherentPolicy);
    return (uint64_t)v[0] | ((uint64_t)v[1] << 32);
  }
  __device__ void store_u64(uint32_t off, uint64_t x) const {
    typedef unsigned int U2 __attribute__((ext_vector_type(2)));
    const U2 v = {(uint32_t)x, (uint32_t)(x >> 32)};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, (int)off, 0, kCoherentPolicy);
  }
};

// Waits until every earlier memory access of this wave has completed (a
// writer's coherent stores before it signals a counter).
__device__ __forceinline__ void wait_memory() { __builtin_amdgcn_s_waitcnt(0); }

// Polls a device-scope counter until it reaches `target`; after `limit`
// polls it gives up, sets bit 0 of *error and returns false (so a launch
// whose hand-off never completes still ends, with its error recorded).
template <typename U>
__device__ __forceinline__ bool wait_counter(const U* counter, U target, uint32_t limit,
                                             uint32_t* error) {
  uint32_t n = 0;
  while (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
    if (++n >= limit) {
      __hip_atomic_fetch_or(error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return false;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return true;
}

// Position of the k-th (0-based) set bit of m; m must have more than k bits.
__device__ __forceinline__ int nth_set_bit(uint64_t m, int k) {
  int pos = 0;
#pragma unroll
  for (int w = 32; w >= 1; w >>= 1) {
    const uint64_t low = m & ((1ull << w) - 1ull);
    int c = __popcll(low);
    if (k >= c) {
      k -= c;
      m >>= w;
      pos += w;
    }
  }
  return pos;
}

}  // namespace rkv
