// Prefill summarizer: per-block counts, bf16 mean K/V, centred diagonal
// ellipsoid and value norms (src/refinekv/summary.py:46-113).
//
// One wave per (KV head, block).  Pass 1 streams the block's tokens once with
// coalesced row loads (each lane owns 2 or 4 adjacent columns) and keeps the
// column sums, min and max in registers.  Pass 2 re-reads the block (an
// L1/L2 hit) with each 8-lane group owning one token, so the per-token
// head_dim sums are lane-local.  Summation orders (fixed, shared with the CPU
// oracle and equal to torch's CPU kernels the reference runs):
//   column sums   16-token chunks summed left to right from +0, chunk sums
//                 added left to right from +0;
//   radius sum    8-wide lanes, four accumulators over vectors m = 4r + k,
//                 ((A0 + A1) + A2) + A3 per lane, lanes added left to right;
//   value norm    8-wide lanes, fma accumulation over vectors, lanes added
//                 left to right.
#include "rkv_common.h"
#include "rkv_internal.h"

namespace rkv {
namespace {

struct InBf16 {
  using T = uint16_t;
  static __device__ __forceinline__ float cvt(uint16_t h) { return bf16_to_f32(h); }
};
struct InF16 {
  using T = uint16_t;
  static __device__ __forceinline__ float cvt(uint16_t h) { return f16_to_f32(h); }
};
struct InF32 {
  using T = float;
  static __device__ __forceinline__ float cvt(float x) { return x; }
};

// Raw payload of N adjacent elements of the cache dtype, loaded with one
// vector load and converted later (so a batch of loads is in flight at once).
template <class In, int N>
struct RawCols {
  static constexpr int W = N * (int)sizeof(typename In::T) / 4;
  uint32_t w[W];
};

template <class In, int N>
__device__ __forceinline__ RawCols<In, N> load_cols(const typename In::T* __restrict__ p) {
  RawCols<In, N> r;
  constexpr int W = RawCols<In, N>::W;
  if constexpr (W == 1) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(p);
  } else if constexpr (W == 2) {
    const uint2 u = *reinterpret_cast<const uint2*>(p);
    r.w[0] = u.x;
    r.w[1] = u.y;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    r.w[0] = u.x;
    r.w[1] = u.y;
    r.w[2] = u.z;
    r.w[3] = u.w;
  }
  return r;
}

template <class In, int N>
__device__ __forceinline__ void store_cols(typename In::T* __restrict__ p, const RawCols<In, N>& r) {
  constexpr int W = RawCols<In, N>::W;
  if constexpr (W == 1) {
    *reinterpret_cast<uint32_t*>(p) = r.w[0];
  } else if constexpr (W == 2) {
    *reinterpret_cast<uint2*>(p) = make_uint2(r.w[0], r.w[1]);
  } else {
    *reinterpret_cast<uint4*>(p) = make_uint4(r.w[0], r.w[1], r.w[2], r.w[3]);
  }
}

template <class In, int N>
__device__ __forceinline__ void cols_f32(const RawCols<In, N>& r, float (&x)[N]) {
  if constexpr (sizeof(typename In::T) == 2) {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      x[2 * j] = In::cvt((uint16_t)(r.w[j] & 0xFFFFu));
      x[2 * j + 1] = In::cvt((uint16_t)(r.w[j] >> 16));
    }
  } else {
#pragma unroll
    for (int j = 0; j < N; ++j) x[j] = bits_f32(r.w[j]);
  }
}

template <class In>
__device__ __forceinline__ float elem_f32(const typename In::T* __restrict__ p) {
  if constexpr (sizeof(typename In::T) == 2) {
    return In::cvt(*reinterpret_cast<const uint16_t*>(p));
  } else {
    return *p;
  }
}

constexpr int kSummaryWaves = 4;
constexpr int kTokBatch = 8;  // tokens per batch of pass-1 row loads

// Where the keys and values also go when the summary is built while the
// prompt is written to the cache (kStore): the same element strides as the
// sources' meaning (head, token), head_dim dense.
template <class In>
struct CacheOut {
  typename In::T* keys;
  int64_t k_hs, k_ts;
  typename In::T* values;
  int64_t v_hs, v_ts;
};

template <int D, class In, bool kStore>
__global__ __launch_bounds__(kWave * kSummaryWaves) void summary_kernel(
    const typename In::T* __restrict__ keys, int64_t k_hs, int64_t k_ts,
    const typename In::T* __restrict__ values, int64_t v_hs, int64_t v_ts, int64_t length,
    int block, int64_t n_blocks, int64_t* __restrict__ counts, uint16_t* __restrict__ key_mean,
    uint16_t* __restrict__ value_mean, uint16_t* __restrict__ ellipsoid,
    float* __restrict__ value_norm, CacheOut<In> out) {
  constexpr int CPL = D <= 128 ? 2 : 4;  // columns per lane in pass 1
  constexpr int LANES1 = D / CPL;
  __shared__ float s_mk[kSummaryWaves][D];
  __shared__ float s_rs[kSummaryWaves][D];

  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t h = blockIdx.y;
  const int64_t b = (int64_t)blockIdx.x * kSummaryWaves + wave;
  const bool valid = b < n_blocks;
  const int64_t bb = valid ? b : n_blocks - 1;  // in-bounds block for addresses
  const int64_t cnt = !valid ? 0 : (b == n_blocks - 1 ? length - (n_blocks - 1) * block : block);

  // ---- pass 1: column sums (TOKSUM order), min, max -------------------
  const bool on1 = valid && lane < LANES1;
  const int col = lane < LANES1 ? lane * CPL : 0;
  const typename In::T* kb = keys + h * k_hs + (bb * block) * k_ts + col;
  const typename In::T* vb = values + h * v_hs + (bb * block) * v_ts + col;
  float ksum[CPL], vsum[CPL], kmax[CPL], kmin[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    ksum[j] = 0.0f;
    vsum[j] = 0.0f;
    kmax[j] = kNegInf;
    kmin[j] = kPosInf;
  }
  for (int c0 = 0; c0 < block; c0 += 16) {
    float ak[CPL], av[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) ak[j] = av[j] = 0.0f;
#pragma unroll
    for (int i0 = 0; i0 < 16; i0 += kTokBatch) {
      RawCols<In, CPL> rk[kTokBatch], rv[kTokBatch];
#pragma unroll
      for (int i = 0; i < kTokBatch; ++i) {
        const int t = c0 + i0 + i;
        const int tt = t < cnt ? t : 0;  // rows past the block end read its first row
        rk[i] = load_cols<In, CPL>(kb + tt * k_ts);
        rv[i] = load_cols<In, CPL>(vb + tt * v_ts);
      }
#pragma unroll
      for (int i = 0; i < kTokBatch; ++i) {
        const int t = c0 + i0 + i;
        const bool live = on1 && t < cnt;
        if constexpr (kStore) {
          if (live) {
            store_cols<In, CPL>(out.keys + h * out.k_hs + (bb * block + t) * out.k_ts + col, rk[i]);
            store_cols<In, CPL>(out.values + h * out.v_hs + (bb * block + t) * out.v_ts + col,
                                rv[i]);
          }
        }
        float xk[CPL], xv[CPL];
        cols_f32<In, CPL>(rk[i], xk);
        cols_f32<In, CPL>(rv[i], xv);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          // Padded tokens add +0, as the reference's zero-padded pages do.
          ak[j] = ak[j] + (live ? xk[j] : 0.0f);
          av[j] = av[j] + (live ? xv[j] : 0.0f);
          if (live) {
            kmax[j] = nanmax(kmax[j], xk[j]);
            kmin[j] = nanmin(kmin[j], xk[j]);
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      ksum[j] = ksum[j] + ak[j];
      vsum[j] = vsum[j] + av[j];
    }
  }
  float w2[CPL];
  if (on1) {
    const float fc = (float)cnt;
    const int64_t o = (h * n_blocks + b) * D + col;
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint16_t mkb = bf16_rne(ksum[j] / fc);
      key_mean[o + j] = mkb;
      value_mean[o + j] = bf16_rne(vsum[j] / fc);
      const float mk = bf16_to_f32(mkb);
      const float width = nanmax(kmax[j] - mk, mk - kmin[j]);
      const float cw = clamp_min(width, 1e-6f);
      w2[j] = round_bf16(cw * cw);
      s_mk[wave][col + j] = mk;
      s_rs[wave][col + j] = 1.0f / sqrtf(w2[j]);
    }
  }
  __syncthreads();

  // ---- pass 2: per-token radius (RADSUM) and value norm (NORMSUM) ------
  const int l8 = lane & 7;
  const int g8 = lane >> 3;
  const int base = lane & ~7;
  float r2max = kNegInf, vnmax = kNegInf;
  for (int t0 = 0; t0 < cnt; t0 += 8) {
    const int t = t0 + g8;
    const bool on = t < cnt;
    const int tt = on ? t : 0;
    const typename In::T* kr = keys + h * k_hs + (bb * block + tt) * k_ts;
    const typename In::T* vr = values + h * v_hs + (bb * block + tt) * v_ts;
    float kx[D / 8], vx[D / 8];
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
      kx[m] = elem_f32<In>(kr + 8 * m + l8);
      vx[m] = elem_f32<In>(vr + 8 * m + l8);
    }
    float A0 = 0.0f, A1 = 0.0f, A2 = 0.0f, A3 = 0.0f, an = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
      const int e = 8 * m + l8;
      const float c = (kx[m] - s_mk[wave][e]) * s_rs[wave][e];
      const float c2 = c * c;
      if ((m & 3) == 0) A0 = A0 + c2;
      if ((m & 3) == 1) A1 = A1 + c2;
      if ((m & 3) == 2) A2 = A2 + c2;
      if ((m & 3) == 3) A3 = A3 + c2;
      an = __builtin_fmaf(vx[m], vx[m], an);
    }
    const float P = ((A0 + A1) + A2) + A3;
    float tot = 0.0f;
    float vt = shfl(an, base);
#pragma unroll
    for (int j = 0; j < 8; ++j) tot = tot + shfl(P, base + j);
#pragma unroll
    for (int j = 1; j < 8; ++j) vt = vt + shfl(an, base + j);
    if (on) {
      r2max = nanmax(r2max, tot);
      vnmax = nanmax(vnmax, sqrtf(vt));
    }
  }
  r2max = wave_nanmax(r2max);
  vnmax = wave_nanmax(vnmax);
  if (on1) {
    float r2 = clamp_min(r2max, 0.0f);
    r2 = sqrtf(r2);
    r2 = r2 * r2;
    const int64_t o = (h * n_blocks + b) * D + col;
#pragma unroll
    for (int j = 0; j < CPL; ++j) ellipsoid[o + j] = bf16_rne((r2 * w2[j]) * kInflate);
  }
  if (valid && lane == 0) {
    value_norm[h * n_blocks + b] = vnmax;
    if (h == 0) counts[b] = cnt;
  }
}

// max_value_norm[h] = max over blocks (summary.py:148).
__global__ __launch_bounds__(256) void max_norm_kernel(const float* __restrict__ value_norm,
                                                       int64_t n_blocks,
                                                       float* __restrict__ max_value_norm) {
  __shared__ float part[4];
  const int64_t h = blockIdx.x;
  float m = kNegInf;
  for (int64_t b = threadIdx.x; b < n_blocks; b += blockDim.x) m = nanmax(m, value_norm[h * n_blocks + b]);
  m = wave_nanmax(m);
  if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = part[0];
    for (int w = 1; w < (int)(blockDim.x / kWave); ++w) r = nanmax(r, part[w]);
    max_value_norm[h] = r;
  }
}

template <class In>
int launch_summary(const void* keys, int64_t k_hs, int64_t k_ts, const void* values, int64_t v_hs,
                   int64_t v_ts, int64_t heads, int64_t length, int64_t dim, int64_t block,
                   int64_t* counts, void* key_mean, void* value_mean, void* ellipsoid,
                   float* value_norm, float* max_value_norm, const CacheOut<In>& out,
                   hipStream_t stream) {
  const int64_t n_blocks = (length + block - 1) / block;
  dim3 grid((unsigned)((n_blocks + kSummaryWaves - 1) / kSummaryWaves), (unsigned)heads);
  dim3 threads(kWave * kSummaryWaves);
  const auto* k = static_cast<const typename In::T*>(keys);
  const auto* v = static_cast<const typename In::T*>(values);
  auto* km = static_cast<uint16_t*>(key_mean);
  auto* vm = static_cast<uint16_t*>(value_mean);
  auto* el = static_cast<uint16_t*>(ellipsoid);
  if (out.keys) {
    RKV_DISPATCH_DIM(dim, D,
                     summary_kernel<D, In, true><<<grid, threads, 0, stream>>>(
                         k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, counts, km,
                         vm, el, value_norm, out));
  } else {
    RKV_DISPATCH_DIM(dim, D,
                     summary_kernel<D, In, false><<<grid, threads, 0, stream>>>(
                         k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, counts, km,
                         vm, el, value_norm, out));
  }
  int rc = check_launch("summary_kernel");
  if (rc) return rc;
  max_norm_kernel<<<dim3((unsigned)heads), dim3(256), 0, stream>>>(value_norm, n_blocks,
                                                                    max_value_norm);
  return check_launch("max_norm_kernel");
}

}  // namespace
}  // namespace rkv

using namespace rkv;

namespace {

int summary_impl(const char* who, const void* keys, int64_t k_head_stride,
                 int64_t k_token_stride, const void* values, int64_t v_head_stride,
                 int64_t v_token_stride, int dtype, int64_t heads, int64_t length, int64_t dim,
                 int64_t block_size, void* cache_keys, int64_t ck_head_stride,
                 int64_t ck_token_stride, void* cache_values, int64_t cv_head_stride,
                 int64_t cv_token_stride, int64_t* counts, void* key_mean, void* value_mean,
                 void* ellipsoid, float* value_norm, float* max_value_norm, hipStream_t stream) {
  if (!keys || !values || !counts || !key_mean || !value_mean || !ellipsoid || !value_norm ||
      !max_value_norm)
    return set_error(kInvalidArgument, "%s: null pointer argument", who);
  if (heads <= 0 || length <= 0 || heads > 65535)
    return set_error(kInvalidArgument, "%s: heads=%lld length=%lld out of range", who,
                     (long long)heads, (long long)length);
  if (!supported_dim(dim))
    return set_error(kUnsupported, "%s: head_dim %lld not in 32..256 step 32", who,
                     (long long)dim);
  if (!supported_block(block_size))
    return set_error(kInvalidArgument, "%s: block_size must be 16, 32 or 64", who);
  if (dtype < 0 || dtype > 2) return set_error(kUnsupported, "%s: dtype code %d", who, dtype);
  const int64_t elem = dtype == 2 ? 4 : 2;
  const int64_t cpl = dim <= 128 ? 2 : 4;
  // Pass-1 row loads (and the cache stores) move CPL adjacent elements; they
  // need that alignment.
  const uintptr_t need = (uintptr_t)(elem * cpl);
  if (!aligned(keys, need) || !aligned(values, need) || (k_head_stride * elem) % need ||
      (k_token_stride * elem) % need || (v_head_stride * elem) % need ||
      (v_token_stride * elem) % need)
    return set_error(kInvalidArgument, "%s: K/V rows must be %d-byte aligned", who, (int)need);
  if (k_token_stride < dim || v_token_stride < dim)
    return set_error(kInvalidArgument, "%s: token stride smaller than head_dim", who);
  const bool store = cache_keys != nullptr || cache_values != nullptr;
  if (store) {
    if (!cache_keys || !cache_values)
      return set_error(kInvalidArgument, "%s: null cache pointer", who);
    if (!aligned(cache_keys, need) || !aligned(cache_values, need) ||
        (ck_head_stride * elem) % need || (ck_token_stride * elem) % need ||
        (cv_head_stride * elem) % need || (cv_token_stride * elem) % need)
      return set_error(kInvalidArgument, "%s: cache rows must be %d-byte aligned", who,
                       (int)need);
    if (ck_token_stride < dim || cv_token_stride < dim)
      return set_error(kInvalidArgument, "%s: cache token stride smaller than head_dim", who);
  }
  const int64_t n_blocks = (length + block_size - 1) / block_size;
  if ((n_blocks + kSummaryWaves - 1) / kSummaryWaves > 0x7FFFFFFF)
    return set_error(kInvalidArgument, "%s: too many blocks", who);
  switch (dtype) {
    case 0: {
      const CacheOut<InBf16> out{static_cast<uint16_t*>(cache_keys), ck_head_stride,
                                 ck_token_stride, static_cast<uint16_t*>(cache_values),
                                 cv_head_stride, cv_token_stride};
      return launch_summary<InBf16>(keys, k_head_stride, k_token_stride, values, v_head_stride,
                                    v_token_stride, heads, length, dim, block_size, counts,
                                    key_mean, value_mean, ellipsoid, value_norm, max_value_norm,
                                    out, stream);
    }
    case 1: {
      const CacheOut<InF16> out{static_cast<uint16_t*>(cache_keys), ck_head_stride,
                                ck_token_stride, static_cast<uint16_t*>(cache_values),
                                cv_head_stride, cv_token_stride};
      return launch_summary<InF16>(keys, k_head_stride, k_token_stride, values, v_head_stride,
                                   v_token_stride, heads, length, dim, block_size, counts,
                                   key_mean, value_mean, ellipsoid, value_norm, max_value_norm,
                                   out, stream);
    }
    default: {
      const CacheOut<InF32> out{static_cast<float*>(cache_keys), ck_head_stride, ck_token_stride,
                                static_cast<float*>(cache_values), cv_head_stride,
                                cv_token_stride};
      return launch_summary<InF32>(keys, k_head_stride, k_token_stride, values, v_head_stride,
                                   v_token_stride, heads, length, dim, block_size, counts,
                                   key_mean, value_mean, ellipsoid, value_norm, max_value_norm,
                                   out, stream);
    }
  }
}

}  // namespace

extern "C" int rkv_summary(const void* keys, int64_t k_head_stride, int64_t k_token_stride,
                           const void* values, int64_t v_head_stride, int64_t v_token_stride,
                           int dtype, int64_t heads, int64_t length, int64_t dim,
                           int64_t block_size, int64_t* counts, void* key_mean, void* value_mean,
                           void* ellipsoid, float* value_norm, float* max_value_norm,
                           hipStream_t stream) {
  clear_error();
  return summary_impl("rkv_summary", keys, k_head_stride, k_token_stride, values, v_head_stride,
                      v_token_stride, dtype, heads, length, dim, block_size, nullptr, 0, 0,
                      nullptr, 0, 0, counts, key_mean, value_mean, ellipsoid, value_norm,
                      max_value_norm, stream);
}

extern "C" int rkv_summary_store(const void* keys, int64_t k_head_stride,
                                 int64_t k_token_stride, const void* values,
                                 int64_t v_head_stride, int64_t v_token_stride, int dtype,
                                 int64_t heads, int64_t length, int64_t dim, int64_t block_size,
                                 void* cache_keys, int64_t ck_head_stride,
                                 int64_t ck_token_stride, void* cache_values,
                                 int64_t cv_head_stride, int64_t cv_token_stride,
                                 int64_t* counts, void* key_mean, void* value_mean,
                                 void* ellipsoid, float* value_norm, float* max_value_norm,
                                 hipStream_t stream) {
  clear_error();
  if (!cache_keys || !cache_values)
    return set_error(kInvalidArgument, "rkv_summary_store: null cache pointer");
  return summary_impl("rkv_summary_store", keys, k_head_stride, k_token_stride, values,
                      v_head_stride, v_token_stride, dtype, heads, length, dim, block_size,
                      cache_keys, ck_head_stride, ck_token_stride, cache_values, cv_head_stride,
                      cv_token_stride, counts, key_mean, value_mean, ellipsoid, value_norm,
                      max_value_norm, stream);
}
