// Prefill summarizer: per-block counts, bf16 mean K/V, centred diagonal
// ellipsoid and value norms (src/refinekv/summary.py:46-113).
//
// One wave per (KV head, block).  Pass 1 streams the block's tokens once with
// coalesced row loads (each lane owns 2 or 4 adjacent columns) and keeps the
// column sums, min and max in registers.  Pass 2 re-reads the block (an L2
// hit: HBM sees each row once) with each 8-lane group owning one token, so the
// per-token head_dim sums are lane-local.  Every row access is a buffer load
// from a per-block buffer view (scalar base and token offset, one lane offset,
// immediate column offsets: no per-load address arithmetic), the block index
// is wave-uniform, and the min/max use the NaN-propagating v_maximum3 /
// v_minimum3 forms, which keeps the vector ALU well below the memory time.  Summation orders (fixed, shared with the CPU
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
  // v_cvt_f32_f16: exact for every finite and infinite half (as f16_to_f32);
  // a signalling NaN comes out quiet
  static __device__ __forceinline__ float cvt(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
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

// Buffer view of one block's rows: a scalar base and 32-bit byte offsets.
// Reads at or past `bytes` return 0 and writes there are dropped.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_view(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes, 0x00020000);
}

template <class In, int N>
__device__ __forceinline__ RawCols<In, N> buf_cols(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  RawCols<In, N> c;
  constexpr int W = RawCols<In, N>::W;
  if constexpr (W == 1) {
    c.w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0);
  } else if constexpr (W == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, 0);
    c.w[0] = v[0];
    c.w[1] = v[1];
  } else {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    c.w[0] = v[0];
    c.w[1] = v[1];
    c.w[2] = v[2];
    c.w[3] = v[3];
  }
  return c;
}

template <class In, int N>
__device__ __forceinline__ void buf_store_cols(__amdgpu_buffer_rsrc_t r, int voff, int soff,
                                               const RawCols<In, N>& c) {
  constexpr int W = RawCols<In, N>::W;
  typedef unsigned int U2 __attribute__((ext_vector_type(2)));
  typedef unsigned int U4 __attribute__((ext_vector_type(4)));
  if constexpr (W == 1) {
    __builtin_amdgcn_raw_buffer_store_b32(c.w[0], r, voff, soff, 0);
  } else if constexpr (W == 2) {
    const U2 v = {c.w[0], c.w[1]};
    __builtin_amdgcn_raw_buffer_store_b64(v, r, voff, soff, 0);
  } else {
    const U4 v = {c.w[0], c.w[1], c.w[2], c.w[3]};
    __builtin_amdgcn_raw_buffer_store_b128(v, r, voff, soff, 0);
  }
}

template <class In>
__device__ __forceinline__ float buf_elem(__amdgpu_buffer_rsrc_t r, int voff) {
  if constexpr (sizeof(typename In::T) == 2) {
    return In::cvt(__builtin_amdgcn_raw_buffer_load_b16(r, voff, 0, 0));
  } else {
    return bits_f32(__builtin_amdgcn_raw_buffer_load_b32(r, voff, 0, 0));
  }
}

// NaN-propagating max/min (v_maximum3_f32 / v_minimum3_f32).  They differ
// from nanmax/nanmin only in which zero a +0/-0 tie returns, which no output
// depends on: a zero extreme enters only |extreme - mean|, clamped to 1e-6.
__device__ __forceinline__ float max3_nan(float a, float b, float c) {
  return __builtin_elementwise_maximum(a, __builtin_elementwise_maximum(b, c));
}
__device__ __forceinline__ float min3_nan(float a, float b, float c) {
  return __builtin_elementwise_minimum(a, __builtin_elementwise_minimum(b, c));
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

// Byte strides of a block's rows fit 31 bits (checked on the host).
template <int D, class In, bool kStore>
__global__ __launch_bounds__(kWave * kSummaryWaves) void summary_kernel(
    const typename In::T* __restrict__ keys, int64_t k_hs, int64_t k_ts,
    const typename In::T* __restrict__ values, int64_t v_hs, int64_t v_ts, int64_t length,
    int block, int64_t n_blocks, int64_t* __restrict__ counts, uint16_t* __restrict__ key_mean,
    uint16_t* __restrict__ value_mean, uint16_t* __restrict__ ellipsoid,
    float* __restrict__ value_norm, CacheOut<In> out) {
  constexpr int E = (int)sizeof(typename In::T);
  constexpr int CPL = D <= 128 ? 2 : 4;  // columns per lane in pass 1
  constexpr int LANES1 = D / CPL;
  __shared__ float s_mk[kSummaryWaves][D];
  __shared__ float s_rs[kSummaryWaves][D];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int lane = threadIdx.x % kWave;
  const int64_t h = blockIdx.y;
  const int64_t b = (int64_t)blockIdx.x * kSummaryWaves + wave;
  const bool valid = b < n_blocks;
  const int64_t bb = valid ? b : n_blocks - 1;  // in-bounds block for addresses
  // (64-bit compares run on the vector ALU: readfirstlane keeps the counts
  // and buffer views in scalar registers)
  const int cnt = __builtin_amdgcn_readfirstlane(
      !valid ? 0 : (int)(b == n_blocks - 1 ? length - (n_blocks - 1) * block : block));
  // the block's rows; a wave past the last block reads nothing (zeros)
  const int kts = (int)k_ts * E, vts = (int)v_ts * E;
  auto extent = [&](int ts) { return __builtin_amdgcn_readfirstlane(cnt ? (cnt - 1) * ts + D * E : 0); };
  const auto kr = rows_view(keys + h * k_hs + bb * block * k_ts, extent(kts));
  const auto vr = rows_view(values + h * v_hs + bb * block * v_ts, extent(vts));

  // ---- pass 1: column sums (TOKSUM order), min, max -------------------
  const bool on1 = valid && lane < LANES1;
  const int col = lane < LANES1 ? lane * CPL : 0;
  float ksum[CPL], vsum[CPL], kmax[CPL], kmin[CPL];
#pragma unroll
  for (int j = 0; j < CPL; ++j) {
    ksum[j] = 0.0f;
    vsum[j] = 0.0f;
    kmax[j] = kNegInf;
    kmin[j] = kPosInf;
  }
  // the cache rows of this block (kStore): live tokens, lanes on1
  const int cks = kStore ? (int)out.k_ts * E : 0, cvs = kStore ? (int)out.v_ts * E : 0;
  const auto ckr =
      kStore ? rows_view(out.keys + h * out.k_hs + bb * block * out.k_ts, extent(cks)) : kr;
  const auto cvr =
      kStore ? rows_view(out.values + h * out.v_hs + bb * block * out.v_ts, extent(cvs)) : vr;
  // token t's columns added to the chunk sums (t < cnt, wave-uniform)
  auto take = [&](int t, const RawCols<In, CPL>& rk, const RawCols<In, CPL>& rv,
                  float (&ak)[CPL], float (&av)[CPL], float (&xk)[CPL]) {
    if constexpr (kStore) {
      if (on1) {
        buf_store_cols<In, CPL>(ckr, col * E, t * cks, rk);
        buf_store_cols<In, CPL>(cvr, col * E, t * cvs, rv);
      }
    }
    float xv[CPL];
    cols_f32<In, CPL>(rk, xk);
    cols_f32<In, CPL>(rv, xv);
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      ak[j] = ak[j] + xk[j];
      av[j] = av[j] + xv[j];
    }
  };
  for (int c0 = 0; c0 < block; c0 += 16) {
    float ak[CPL], av[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) ak[j] = av[j] = 0.0f;
    if (cnt - c0 >= 16) {
#pragma unroll
      for (int i0 = 0; i0 < 16; i0 += kTokBatch) {
        RawCols<In, CPL> rk[kTokBatch], rv[kTokBatch];
#pragma unroll
        for (int i = 0; i < kTokBatch; ++i) {
          rk[i] = buf_cols<In, CPL>(kr, col * E, (c0 + i0 + i) * kts);
          rv[i] = buf_cols<In, CPL>(vr, col * E, (c0 + i0 + i) * vts);
        }
#pragma unroll
        for (int i = 0; i < kTokBatch; i += 2) {
          float x0[CPL], x1[CPL];
          take(c0 + i0 + i, rk[i], rv[i], ak, av, x0);
          take(c0 + i0 + i + 1, rk[i + 1], rv[i + 1], ak, av, x1);
#pragma unroll
          for (int j = 0; j < CPL; ++j) {
            kmax[j] = max3_nan(kmax[j], x0[j], x1[j]);
            kmin[j] = min3_nan(kmin[j], x0[j], x1[j]);
          }
        }
      }
    } else {
      for (int t = c0; t < cnt; ++t) {
        float x[CPL];
        take(t, buf_cols<In, CPL>(kr, col * E, t * kts), buf_cols<In, CPL>(vr, col * E, t * vts),
             ak, av, x);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          kmax[j] = max3_nan(kmax[j], x[j], x[j]);
          kmin[j] = min3_nan(kmin[j], x[j], x[j]);
        }
      }
      // the chunk's padded tokens each add +0, as the reference's zero-padded
      // pages do (repeated +0 adds equal one)
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        ak[j] = ak[j] + 0.0f;
        av[j] = av[j] + 0.0f;
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
  float r2max = kNegInf, vnmax = kNegInf;
  for (int t0 = 0; t0 < cnt; t0 += 8) {
    const int t = t0 + g8;
    const bool on = t < cnt;
    const int tt = on ? t : 0;
    const int ko = tt * kts + l8 * E, vo = tt * vts + l8 * E;
    float kx[D / 8], vx[D / 8];
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
      kx[m] = buf_elem<In>(kr, ko + 8 * m * E);
      vx[m] = buf_elem<In>(vr, vo + 8 * m * E);
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
    // the group's lanes added left to right: a DPP scan whose last lane
    // (l8 == 7) holds ((P0 + P1) + P2) + ... + P7
    float tot = P, vt = an;
#pragma unroll
    for (int j = 1; j < 8; ++j) {
      tot = row_shr<1>(tot) + P;
      vt = row_shr<1>(vt) + an;
    }
    const bool last = on && l8 == 7;
    r2max = nanmax(r2max, last ? tot : kNegInf);
    vnmax = nanmax(vnmax, last ? sqrtf(vt) : kNegInf);
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
  // one block's rows are addressed with 31-bit byte offsets
  const int64_t row_limit = (int64_t{1} << 31) / (block_size * elem);
  if (k_token_stride >= row_limit || v_token_stride >= row_limit ||
      (store && (ck_token_stride >= row_limit || cv_token_stride >= row_limit)))
    return set_error(kUnsupported, "%s: token stride above %lld elements", who,
                     (long long)(row_limit - 1));
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
