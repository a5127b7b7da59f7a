// Prefill summarizer: per-block counts, bf16 mean K/V, centred diagonal
// ellipsoid and value norms (src/refinekv/summary.py:46-113).
//
// One wave per (KV head, block).  Pass 1 reads the block's rows with each lane
// owning 2 or 4 adjacent columns and keeps the column sums, min and max in
// registers.  Pass 2 reads the rows again with each 8-lane group owning one
// token, so the per-token head_dim sums are lane-local.  Where a block's K
// and V fit 64 KiB (kStage), the wave first moves the whole block from HBM
// into LDS with 16-byte buffer-to-LDS loads (all of it in flight at once) and
// both passes read LDS: HBM sees each row once.  Blocks of 32 and 64 tokens
// go to a workgroup of block / 16 waves instead, each staging one 16-token
// chunk, whose chunk sums wave 0 adds in order (the same sums); blocks that
// fit neither stream pass 1 from global memory and re-read the rows there in
// pass 2.  Row accesses go
// through per-block buffer views (scalar base and token offset, one lane
// offset, immediate column offsets: no per-load address arithmetic; rows past
// the block's end read 0), the block index is wave-uniform, and the min/max
// use the NaN-propagating v_maximum3 / v_minimum3 forms.  Summation orders (fixed, shared with the CPU
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

// 16 bytes per lane from a buffer view straight into LDS: lane i's bytes land
// at lds_base + 16 i (lds_base wave-uniform).
__device__ __forceinline__ void load_to_lds16(__amdgpu_buffer_rsrc_t r, uint4* lds_base, int voff) {
  typedef __attribute__((address_space(3))) void LdsVoid;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (LdsVoid*)lds_base, 16, voff, 0, 0, 0);
}

template <class In>
__device__ __forceinline__ float lds_elem(const typename In::T* p) {
  if constexpr (sizeof(typename In::T) == 2) {
    return In::cvt(*reinterpret_cast<const uint16_t*>(p));
  } else {
    return *p;
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
constexpr int64_t kStageWaveMax = 64 * 1024;   // LDS of one staged block, at most
constexpr int64_t kStageGroupMax = 32 * 1024;  // LDS of a staged workgroup, aimed at
// One wave stages a block while it holds at most 4096 elements per tensor
// (larger blocks in one wave leave too few waves per CU for their longer
// passes); blocks of 32 or more tokens are split into 16-token chunks over a
// workgroup's waves (summary_split_kernel) whenever that fits.
constexpr int64_t kStageElemsMax = 4096;

// A staged block in LDS (per wave): its K rows, then its V rows, as 16-byte
// chunks, then D key means and D inverse widths (fp32).  Chunk c of token t
// sits at slot c ^ swizzle(t) of the row so that the 8 tokens of one pass-2
// read start on different banks: pass 2 reads 8 consecutive elements of a
// row, G chunks (one for 2-byte types, two for fp32); the swizzle stays
// inside aligned groups of SW * G chunks, SW the largest power of two (at
// most 8) dividing NC / G (4 for head_dim 32, 96, 160 and 224).
template <class In, int D>
struct Staging {
  static constexpr int E = (int)sizeof(typename In::T);
  static constexpr int NC = D * E / 16;  // chunks per row
  static constexpr int EPC = 16 / E;     // elements per chunk
  static constexpr int G = 8 * E / 16;
  static constexpr int LOW = (NC / G) & -(NC / G);
  static constexpr int SW = LOW < 8 ? LOW : 8;
  static __device__ __forceinline__ int slot(int c, int t) { return c ^ ((t & (SW - 1)) * G); }
};

// LDS bytes of one wave's block (kStage) or of its means and widths alone.
__host__ __device__ constexpr int64_t summary_wave_lds(bool stage, int64_t dim, int64_t elem,
                                                       int64_t block) {
  return (stage ? 2 * block * dim * elem : 0) + 2 * dim * 4;
}

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
// blockDim.x / 64 waves (1, 2 or 4), one block each, and summary_wave_lds
// bytes of dynamic LDS per wave.  kStage needs 16-byte aligned rows.
// Pass 1 (column sums in TOKSUM order, min, max -> means, widths) and pass 2
// (per-token radius and value norm -> ellipsoid, value_norm) of block b of
// head h, whose rows are kr / vr (byte strides kts / vts) or, with kStage,
// staged in LDS at kst / vst; s_mk / s_rs: D floats each of LDS.  One wave;
// its workgroup holds whole waves only (the __syncthreads between the passes
// orders the LDS writes of the means before their reads).
// A block summarized by several waves of one workgroup (kSplit): wave w
// holds the block's 16-token chunk w (its own cnt and block are that chunk's
// live tokens and 16), and the chunks' sums meet in LDS.
struct SplitPart {
  int wave, waves;  // this wave's chunk, the block's chunks
  int cnt;          // the block's tokens
  float* part;      // LDS: waves x 4 x D floats (chunk sums, max, min), then waves x 2
};

template <int D, class In, bool kStore, bool kStage, bool kSplit = false>
__device__ __forceinline__ void summary_passes(
    int64_t h, int64_t b, int64_t row0, bool valid, int cnt, int block, int64_t n_blocks,
    __amdgpu_buffer_rsrc_t kr, __amdgpu_buffer_rsrc_t vr, int kts, int vts, const uint4* kst,
    const uint4* vst, float* s_mk, float* s_rs, int64_t* __restrict__ counts,
    uint16_t* __restrict__ key_mean, uint16_t* __restrict__ value_mean,
    uint16_t* __restrict__ ellipsoid, float* __restrict__ value_norm, const CacheOut<In>& out,
    const SplitPart& sp = SplitPart{0, 1, 0, nullptr}) {
  using T = typename In::T;
  using St = Staging<In, D>;
  constexpr int E = (int)sizeof(T);
  constexpr int CPL = D <= 128 ? 2 : 4;  // columns per lane in pass 1
  constexpr int LANES1 = D / CPL;
  const int lane = threadIdx.x % kWave;
  auto extent = [&](int ts) { return __builtin_amdgcn_readfirstlane(cnt ? (cnt - 1) * ts + D * E : 0); };
  // ---- pass 1: column sums (TOKSUM order), min, max -------------------
  const bool on1 = valid && lane < LANES1;
  const int col = lane < LANES1 ? lane * CPL : 0;
  // this lane's columns in a staged row: chunk c1, 4-byte word w1 within it
  const int c1 = col / St::EPC, w1 = (col % St::EPC) * E / 4;
  // a staged row's words at w (this lane's columns)
  auto lds_cols = [&](const uint32_t* w) {
    RawCols<In, CPL> x;
    constexpr int W = RawCols<In, CPL>::W;
    if constexpr (W == 1) {
      x.w[0] = w[0];
    } else if constexpr (W == 2) {
      const uint2 u = *reinterpret_cast<const uint2*>(w);
      x.w[0] = u.x;
      x.w[1] = u.y;
    } else {
      const uint4 u = *reinterpret_cast<const uint4*>(w);
      x.w[0] = u.x;
      x.w[1] = u.y;
      x.w[2] = u.z;
      x.w[3] = u.w;
    }
    return x;
  };
  // Token t's swizzle depends on t mod SW alone, so this lane's staged words
  // for each residue sit at fixed addresses kw1[s] / vw1[s] plus the row
  // offset t NC 16, a constant of the unrolled full-chunk loop below (the
  // reads' immediate offset): no per-read address arithmetic.
  // (head_dim 64 .. 128: above it the tables' registers cost the stream form
  // its second wave per SIMD; below it a staged block's 128 tokens are too
  // many to unroll)
  constexpr bool kFixed = kStage && D >= 64 && D <= 128;
  constexpr int kMaxBlock = kFixed ? (int)(kStageElemsMax / D) / 16 * 16 : 16;
  const char* kw1[St::SW];
  const char* vw1[St::SW];
#pragma unroll
  for (int sr = 0; sr < St::SW; ++sr) {
    const int o = St::slot(c1, sr) * 16 + w1 * 4;
    kw1[sr] = reinterpret_cast<const char*>(kst) + o;
    vw1[sr] = reinterpret_cast<const char*>(vst) + o;
  }
  auto row_cols = [&](const __amdgpu_buffer_rsrc_t& r, const uint4* st, int t, int ts) {
    if constexpr (kStage) {
      const uint32_t* w = reinterpret_cast<const uint32_t*>(st + t * St::NC + St::slot(c1, t)) + w1;
      RawCols<In, CPL> x;
      constexpr int W = RawCols<In, CPL>::W;
      if constexpr (W == 1) {
        x.w[0] = w[0];
      } else if constexpr (W == 2) {
        const uint2 u = *reinterpret_cast<const uint2*>(w);
        x.w[0] = u.x;
        x.w[1] = u.y;
      } else {
        const uint4 u = *reinterpret_cast<const uint4*>(w);
        x.w[0] = u.x;
        x.w[1] = u.y;
        x.w[2] = u.z;
        x.w[3] = u.w;
      }
      return x;
    } else {
      return buf_cols<In, CPL>(r, col * E, t * ts);
    }
  };
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
      kStore ? rows_view(out.keys + h * out.k_hs + row0 * out.k_ts, extent(cks)) : kr;
  const auto cvr =
      kStore ? rows_view(out.values + h * out.v_hs + row0 * out.v_ts, extent(cvs)) : vr;
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
  // the 16-token chunk at c0 (a multiple of 16)
  auto chunk = [&](int c0) {
    float ak[CPL], av[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) ak[j] = av[j] = 0.0f;
    if (cnt - c0 >= 16) {
#pragma unroll
      for (int i0 = 0; i0 < 16; i0 += kTokBatch) {
        RawCols<In, CPL> rk[kTokBatch], rv[kTokBatch];
#pragma unroll
        for (int i = 0; i < kTokBatch; ++i) {
          const int t = c0 + i0 + i;  // t mod SW == (i0 + i) mod SW
          if constexpr (kFixed) {
            const int row = t * St::NC * 16;
            rk[i] = lds_cols(reinterpret_cast<const uint32_t*>(kw1[(i0 + i) % St::SW] + row));
            rv[i] = lds_cols(reinterpret_cast<const uint32_t*>(vw1[(i0 + i) % St::SW] + row));
          } else {
            rk[i] = row_cols(kr, kst, t, kts);
            rv[i] = row_cols(vr, vst, t, vts);
          }
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
        take(t, row_cols(kr, kst, t, kts), row_cols(vr, vst, t, vts), ak, av, x);
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
  };
  if constexpr (kFixed) {
    // (a staged block holds at most kMaxBlock tokens)
#pragma unroll
    for (int c0 = 0; c0 < kMaxBlock; c0 += 16) {
      if (c0 >= block) break;
      chunk(c0);
    }
  } else {
    for (int c0 = 0; c0 < block; c0 += 16) chunk(c0);
  }
  if constexpr (kSplit) {
    // the chunk's sums, max and min out; wave 0 adds the chunks' sums left
    // to right from +0 (each is its chunk summed from +0, and a running sum
    // from +0 is never -0, so this is the one-wave TOKSUM order exactly)
    float* q = sp.part + sp.wave * 4 * D;
    if (on1) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        q[col + j] = ksum[j];
        q[D + col + j] = vsum[j];
        q[2 * D + col + j] = kmax[j];
        q[3 * D + col + j] = kmin[j];
      }
    }
    __syncthreads();
    if (sp.wave == 0) {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        ksum[j] = 0.0f;
        vsum[j] = 0.0f;
      }
      for (int w = 0; w < sp.waves; ++w) {
        const float* r = sp.part + w * 4 * D;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
          ksum[j] = ksum[j] + r[col + j];
          vsum[j] = vsum[j] + r[D + col + j];
          kmax[j] = max3_nan(kmax[j], r[2 * D + col + j], r[2 * D + col + j]);
          kmin[j] = min3_nan(kmin[j], r[3 * D + col + j], r[3 * D + col + j]);
        }
      }
    }
  }
  // the block's token count (the whole block's in split mode)
  const int bcnt = kSplit ? sp.cnt : cnt;
  float w2[CPL];
  if (on1 && (!kSplit || sp.wave == 0)) {
    const float fc = (float)bcnt;
    const int64_t o = (h * n_blocks + b) * D + col;
    // x / 2^k and x * 2^-k are the same correctly rounded value of x 2^-k,
    // so a power-of-two count (every full block) takes a multiply
    float km[CPL], vm[CPL];
    if ((bcnt & (bcnt - 1)) == 0) {
      const float inv = 1.0f / fc;
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        km[j] = ksum[j] * inv;
        vm[j] = vsum[j] * inv;
      }
    } else {
#pragma unroll
      for (int j = 0; j < CPL; ++j) {
        km[j] = ksum[j] / fc;
        vm[j] = vsum[j] / fc;
      }
    }
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
      const uint16_t mkb = bf16_rne(km[j]);
      key_mean[o + j] = mkb;
      value_mean[o + j] = bf16_rne(vm[j]);
      const float mk = bf16_to_f32(mkb);
      const float width = nanmax(kmax[j] - mk, mk - kmin[j]);
      const float cw = clamp_min(width, 1e-6f);
      w2[j] = round_bf16(cw * cw);
      s_mk[col + j] = mk;
      s_rs[col + j] = 1.0f / sqrtf(w2[j]);
    }
  }
  __syncthreads();

  // ---- pass 2: per-token radius (RADSUM) and value norm (NORMSUM) ------
  const int l8 = lane & 7;
  const int g8 = lane >> 3;
  // vnmax: the largest squared token norm; its square root is taken once,
  // after the block (a correctly rounded sqrt is monotone, so the root of the
  // maximum is the maximum of the roots; a NaN propagates either way)
  float r2max = kNegInf, vnmax = kNegInf;
  // the 8 tokens t0 + g8 (t0 a multiple of 8): this lane's elements 8 m + l8
  auto group = [&](const float (&kx)[D / 8], const float (&vx)[D / 8], bool on) {
    float A0 = 0.0f, A1 = 0.0f, A2 = 0.0f, A3 = 0.0f, an = 0.0f;
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
      const int e = 8 * m + l8;
      const float c = (kx[m] - s_mk[e]) * s_rs[e];
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
    vnmax = nanmax(vnmax, last ? vt : kNegInf);
  };
  if constexpr (kFixed) {
    // element 8 m + l8 of token t0 + g8 sits at ka2[m] / va2[m] plus the row
    // offset t0 NC 16 (t0 + g8 has the residue g8 mod SW): rows past cnt in
    // the group read the block's zero-filled tail (t0 + 7 < block), masked
    const char* ka2[D / 8];
    const char* va2[D / 8];
#pragma unroll
    for (int m = 0; m < D / 8; ++m) {
      const int e = 8 * m + l8;
      const int o = (g8 * St::NC + St::slot(e / St::EPC, g8)) * 16 + (e % St::EPC) * E;
      ka2[m] = reinterpret_cast<const char*>(kst) + o;
      va2[m] = reinterpret_cast<const char*>(vst) + o;
    }
#pragma unroll
    for (int t0 = 0; t0 < kMaxBlock; t0 += 8) {
      if (t0 >= cnt) break;
      const int row = t0 * St::NC * 16;
      float kx[D / 8], vx[D / 8];
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {
        kx[m] = lds_elem<In>(reinterpret_cast<const T*>(ka2[m] + row));
        vx[m] = lds_elem<In>(reinterpret_cast<const T*>(va2[m] + row));
      }
      group(kx, vx, t0 + g8 < cnt);
    }
  } else {
    for (int t0 = 0; t0 < cnt; t0 += 8) {
      const int t = t0 + g8;
      const bool on = t < cnt;
      const int tt = on ? t : 0;
      const int ko = tt * kts + l8 * E, vo = tt * vts + l8 * E;
      float kx[D / 8], vx[D / 8];
#pragma unroll
      for (int m = 0; m < D / 8; ++m) {
        if constexpr (kStage) {
          const int e = 8 * m + l8;
          const int o = tt * St::NC + St::slot(e / St::EPC, tt);
          kx[m] = lds_elem<In>(reinterpret_cast<const T*>(kst + o) + e % St::EPC);
          vx[m] = lds_elem<In>(reinterpret_cast<const T*>(vst + o) + e % St::EPC);
        } else {
          kx[m] = buf_elem<In>(kr, ko + 8 * m * E);
          vx[m] = buf_elem<In>(vr, vo + 8 * m * E);
        }
      }
      group(kx, vx, on);
    }
  }
  r2max = wave_nanmax(r2max);
  vnmax = wave_nanmax(vnmax);
  if constexpr (kSplit) {
    // the chunks' maxima meet in wave 0, which writes the block's outputs
    float* q = sp.part + sp.waves * 4 * D;
    if (lane == 0) {
      q[2 * sp.wave] = r2max;
      q[2 * sp.wave + 1] = vnmax;
    }
    __syncthreads();
    if (sp.wave != 0) return;
    for (int w = 0; w < sp.waves; ++w) {
      r2max = nanmax(r2max, q[2 * w]);
      vnmax = nanmax(vnmax, q[2 * w + 1]);
    }
  }
  vnmax = sqrtf(vnmax);
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
    if (h == 0) counts[b] = bcnt;
  }
}

template <int D, class In, bool kStore, bool kStage>
__global__ __launch_bounds__(kWave * kSummaryWaves) void summary_kernel(
    const typename In::T* __restrict__ keys, int64_t k_hs, int64_t k_ts,
    const typename In::T* __restrict__ values, int64_t v_hs, int64_t v_ts, int64_t length,
    int block, int64_t n_blocks, int64_t* __restrict__ counts, uint16_t* __restrict__ key_mean,
    uint16_t* __restrict__ value_mean, uint16_t* __restrict__ ellipsoid,
    float* __restrict__ value_norm, CacheOut<In> out) {
  using T = typename In::T;
  using St = Staging<In, D>;
  constexpr int E = (int)sizeof(T);
  extern __shared__ uint4 s_dyn[];

  const int waves = blockDim.x / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform
  const int lane = threadIdx.x % kWave;
  const int64_t h = blockIdx.y;
  const int64_t b = (int64_t)blockIdx.x * waves + wave;
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
  const int chunks = kStage ? block * St::NC : 0;  // per tensor, a multiple of 64
  uint4* kst = s_dyn + wave * (2 * chunks + D / 2);
  uint4* vst = kst + chunks;
  float* s_mk = reinterpret_cast<float*>(vst + chunks);
  float* s_rs = s_mk + D;
  if constexpr (kStage) {
    // the whole block in flight: LDS chunk p (token p / NC, slot p % NC)
    // takes chunk slot(p % NC, t) of that token's row
    for (int p0 = 0; p0 < chunks; p0 += kWave) {
      const int p = p0 + lane, t = p / St::NC;
      const int off = St::slot(p % St::NC, t) * 16;
      load_to_lds16(kr, kst + p0, t * kts + off);
      load_to_lds16(vr, vst + p0, t * vts + off);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  }

  summary_passes<D, In, kStore, kStage>(h, b, bb * block, valid, cnt, block, n_blocks, kr, vr,
                                        kts, vts, kst, vst, s_mk, s_rs, counts, key_mean,
                                        value_mean, ellipsoid, value_norm, out);
}

// Blocks of 32 or 64 tokens: one workgroup of block / 16 waves per block
// (what fits 64 KiB of LDS, with 16 tokens x head_dim <= 4096); wave w moves
// the block's 16-token chunk w into LDS (all its loads in flight at once) and
// runs both passes on it, and wave 0 combines the chunks (summary_passes,
// kSplit), so HBM sees each row once.  LDS: the waves' chunks (K then V, the
// staged layout), then D key means, D inverse widths and the chunks'
// partials.
template <int D, class In, bool kStore>
__global__ __launch_bounds__(kWave * 4) void summary_split_kernel(
    const typename In::T* __restrict__ keys, int64_t k_hs, int64_t k_ts,
    const typename In::T* __restrict__ values, int64_t v_hs, int64_t v_ts, int64_t length,
    int block, int64_t n_blocks, int64_t* __restrict__ counts, uint16_t* __restrict__ key_mean,
    uint16_t* __restrict__ value_mean, uint16_t* __restrict__ ellipsoid,
    float* __restrict__ value_norm, CacheOut<In> out) {
  using St = Staging<In, D>;
  constexpr int E = (int)sizeof(typename In::T);
  constexpr int chunks = 16 * St::NC;  // 16-byte chunks per tensor and wave, a multiple of 64
  extern __shared__ uint4 s_dyn[];
  const int waves = blockDim.x / kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int lane = threadIdx.x % kWave;
  const int64_t h = blockIdx.y, b = blockIdx.x;
  const int cnt_all = __builtin_amdgcn_readfirstlane(
      (int)(b == n_blocks - 1 ? length - (n_blocks - 1) * block : block));
  const int rest = cnt_all - 16 * wave;
  const int cnt = __builtin_amdgcn_readfirstlane(rest < 0 ? 0 : rest > 16 ? 16 : rest);
  const int64_t row0 = b * block + 16 * wave;
  const int kts = (int)k_ts * E, vts = (int)v_ts * E;
  auto extent = [&](int ts) { return __builtin_amdgcn_readfirstlane(cnt ? (cnt - 1) * ts + D * E : 0); };
  // the chunk's rows; rows past its live tokens read 0
  const auto kr = rows_view(keys + h * k_hs + row0 * k_ts, extent(kts));
  const auto vr = rows_view(values + h * v_hs + row0 * v_ts, extent(vts));
  uint4* kst = s_dyn + wave * 2 * chunks;
  uint4* vst = kst + chunks;
  float* s_mk = reinterpret_cast<float*>(s_dyn + waves * 2 * chunks);
  float* s_rs = s_mk + D;
  for (int p0 = 0; p0 < chunks; p0 += kWave) {
    const int p = p0 + lane, t = p / St::NC;
    const int off = St::slot(p % St::NC, t) * 16;
    load_to_lds16(kr, kst + p0, t * kts + off);
    load_to_lds16(vr, vst + p0, t * vts + off);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  summary_passes<D, In, kStore, true, true>(h, b, row0, true, cnt, 16, n_blocks, kr, vr, kts, vts,
                                            kst, vst, s_mk, s_rs, counts, key_mean, value_mean,
                                            ellipsoid, value_norm, out,
                                            SplitPart{wave, waves, cnt_all, s_rs + D});
}

// LDS bytes of a split block's workgroup (summary_split_kernel).
constexpr int64_t summary_split_lds(int64_t dim, int64_t elem, int64_t block) {
  return (block / 16) * (2 * 16 * dim * elem + 4 * dim * 4 + 2 * 4) + 2 * dim * 4;
}

// The staged summary as a stream (2-byte K/V, head_dim >= 192): one-wave
// workgroups, each going through the (head, block) pairs f = w, w + nw, ...
// (w its index, nw the grid).  The next block's rows are loaded into registers (16 bytes per
// lane per load, at most 8 per tensor) while the current block's passes read
// LDS, then written into the staged layout: the wave keeps a block's loads
// in flight all the time, where a wave per block waits for its loads, then
// computes with none in flight.  The passes are summary_kernel's.
constexpr int kStreamChunks = 8;  // 16-byte chunks per lane per tensor, at most

template <int D, class In, bool kStore>
__global__ __launch_bounds__(kWave) void summary_stream_kernel(
    const typename In::T* __restrict__ keys, int64_t k_hs, int64_t k_ts,
    const typename In::T* __restrict__ values, int64_t v_hs, int64_t v_ts, int64_t length,
    int block, int64_t n_blocks, int64_t heads, int64_t* __restrict__ counts,
    uint16_t* __restrict__ key_mean, uint16_t* __restrict__ value_mean,
    uint16_t* __restrict__ ellipsoid, float* __restrict__ value_norm, CacheOut<In> out) {
  using St = Staging<In, D>;
  constexpr int E = (int)sizeof(typename In::T);
  static_assert(E == 2, "the stream holds 2-byte elements");
  typedef unsigned int U4 __attribute__((ext_vector_type(4)));
  extern __shared__ uint4 s_dyn[];
  const int lane = threadIdx.x;
  const int64_t total = heads * n_blocks;
  const int64_t nw = gridDim.x;
  const int chunks = block * St::NC;  // per tensor: 64 .. 64 kStreamChunks
  const int per_lane = chunks / kWave;
  uint4* kst = s_dyn;
  uint4* vst = kst + chunks;
  float* s_mk = reinterpret_cast<float*>(vst + chunks);
  float* s_rs = s_mk + D;
  const int kts = (int)k_ts * E, vts = (int)v_ts * E;

  struct Views {
    int64_t h, b;
    int cnt;
    __amdgpu_buffer_rsrc_t kr, vr;
  };
  // (head, block) pair f: its token count and row views, wave-uniform
  auto views = [&](int64_t f) {
    Views v;
    v.h = f / n_blocks;
    v.b = f - v.h * n_blocks;
    v.cnt = __builtin_amdgcn_readfirstlane(
        (int)(v.b == n_blocks - 1 ? length - (n_blocks - 1) * block : block));
    const int ek = __builtin_amdgcn_readfirstlane((v.cnt - 1) * kts + D * E);
    const int ev = __builtin_amdgcn_readfirstlane((v.cnt - 1) * vts + D * E);
    v.kr = rows_view(keys + v.h * k_hs + v.b * block * k_ts, ek);
    v.vr = rows_view(values + v.h * v_hs + v.b * block * v_ts, ev);
    return v;
  };
  U4 rk[kStreamChunks], rv[kStreamChunks];
  // chunk p = 64 i + lane of the staged layout: token p / NC, slot p % NC
  // takes chunk slot(p % NC, t) of that token's row
  auto issue = [&](const Views& v) {
#pragma unroll
    for (int i = 0; i < kStreamChunks; ++i) {
      if (i < per_lane) {
        const int p = kWave * i + lane, t = p / St::NC;
        const int off = St::slot(p % St::NC, t) * 16;
        rk[i] = __builtin_amdgcn_raw_buffer_load_b128(v.kr, t * kts + off, 0, 0);
        rv[i] = __builtin_amdgcn_raw_buffer_load_b128(v.vr, t * vts + off, 0, 0);
      }
    }
  };
  int64_t f = blockIdx.x;
  if (f >= total) return;
  issue(views(f));
  for (;;) {
    // the block's rows from registers into the staged layout
#pragma unroll
    for (int i = 0; i < kStreamChunks; ++i) {
      if (i < per_lane) {
        kst[kWave * i + lane] = __builtin_bit_cast(uint4, rk[i]);
        vst[kWave * i + lane] = __builtin_bit_cast(uint4, rv[i]);
      }
    }
    __syncthreads();
    // the next block's loads fly while this one is summarized
    const int64_t fn = f + nw;
    if (fn < total) issue(views(fn));
    const Views cur = views(f);
    summary_passes<D, In, kStore, true>(cur.h, cur.b, cur.b * block, true, cur.cnt, block, n_blocks,
                                        cur.kr, cur.vr, kts, vts, kst, vst, s_mk, s_rs, counts,
                                        key_mean, value_mean, ellipsoid, value_norm, out);
    __syncthreads();
    if (fn >= total) break;
    f = fn;
  }
}

// max_value_norm[h] = max over blocks (summary.py:148).
__global__ __launch_bounds__(256) void max_norm_kernel(const float* __restrict__ value_norm,
                                                       int64_t n_blocks,
                                                       float* __restrict__ max_value_norm) {
  __shared__ float part[4];
  const int64_t h = blockIdx.x;
  const float* vn = value_norm + h * n_blocks;
  float m = kNegInf;
  // blocks tid, tid + 256, ... in that order, sixteen loads in flight at a
  // time (one batch for 4096 blocks)
  constexpr int kBatch = 16;
  for (int64_t b0 = threadIdx.x; b0 < n_blocks; b0 += (int64_t)blockDim.x * kBatch) {
    float x[kBatch];
#pragma unroll
    for (int k = 0; k < kBatch; ++k) {
      const int64_t b = b0 + (int64_t)k * blockDim.x;
      x[k] = b < n_blocks ? vn[b] : kNegInf;
    }
#pragma unroll
    for (int k = 0; k < kBatch; ++k) m = nanmax(m, x[k]);
  }
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
  const int64_t elem = (int64_t)sizeof(typename In::T);
  auto rows16 = [&](const void* p, int64_t hs, int64_t ts) {
    return reinterpret_cast<uintptr_t>(p) % 16 == 0 && (hs * elem) % 16 == 0 &&
           (ts * elem) % 16 == 0;
  };
  const bool stage = block * dim <= kStageElemsMax &&
                     summary_wave_lds(true, dim, elem, block) <= kStageWaveMax &&
                     rows16(keys, k_hs, k_ts) && rows16(values, v_hs, v_ts);
  const int64_t per_wave = summary_wave_lds(stage, dim, elem, block);
  // (head_dim >= 192: 161 -> 142 us at 65536 tokens, d 256, B 16; at d 128 the
  // passes' vector work bounds the kernel and the stream is no faster, at B 16
  // slower)
  if constexpr (sizeof(typename In::T) == 2) {
  if (stage && dim >= 192 && block * dim * elem / 16 <= kWave * kStreamChunks) {
    // the stream: one-wave workgroups, as many as the device holds at once
    int64_t resident = 0;
    int dev = -1, cus = 0, per_cu = 0;
    RKV_DISPATCH_DIM(dim, D, {
      if (hipGetDevice(&dev) == hipSuccess &&
          hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) ==
              hipSuccess &&
          hipOccupancyMaxActiveBlocksPerMultiprocessor(
              &per_cu, out.keys ? summary_stream_kernel<D, In, true>
                                : summary_stream_kernel<D, In, false>,
              kWave, (size_t)per_wave) == hipSuccess)
        resident = (int64_t)cus * per_cu;
    });
    const int64_t total = heads * n_blocks;
    const int64_t grid = resident > 0 ? (resident < total ? resident : total) : total;
    const auto* k = static_cast<const typename In::T*>(keys);
    const auto* v = static_cast<const typename In::T*>(values);
    RKV_DISPATCH_DIM(dim, D, {
      if (out.keys)
        summary_stream_kernel<D, In, true><<<dim3((unsigned)grid), dim3(kWave), per_wave,
                                              stream>>>(
            k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, heads, counts,
            static_cast<uint16_t*>(key_mean), static_cast<uint16_t*>(value_mean),
            static_cast<uint16_t*>(ellipsoid), value_norm, out);
      else
        summary_stream_kernel<D, In, false><<<dim3((unsigned)grid), dim3(kWave), per_wave,
                                               stream>>>(
            k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, heads, counts,
            static_cast<uint16_t*>(key_mean), static_cast<uint16_t*>(value_mean),
            static_cast<uint16_t*>(ellipsoid), value_norm, out);
    });
    int rc = check_launch("summary_stream_kernel");
    if (rc) return rc;
    max_norm_kernel<<<dim3((unsigned)heads), dim3(256), 0, stream>>>(value_norm, n_blocks,
                                                                      max_value_norm);
    return check_launch("max_norm_kernel");
  }
  }
  const auto* k = static_cast<const typename In::T*>(keys);
  const auto* v = static_cast<const typename In::T*>(values);
  auto* km = static_cast<uint16_t*>(key_mean);
  auto* vm = static_cast<uint16_t*>(value_mean);
  auto* el = static_cast<uint16_t*>(ellipsoid);
  // blocks of 32 and 64 tokens: a workgroup of block / 16 waves, a 16-token
  // chunk each (8 heads of 131072 tokens: d 128, B 64 160 -> 127 us, the
  // two-pass form's re-read of pass 2 gone; d 128, B 32 118-122 -> 116 us,
  // d 64, B 64 72 -> 66, d 96, B 32 97 -> 93: half the LDS per wave, twice
  // the waves per CU); 16-token blocks keep one wave each
  const int64_t split_lds = summary_split_lds(dim, elem, block);
  if (block >= 32 && 16 * dim <= kStageElemsMax && split_lds <= kStageWaveMax &&
      rows16(keys, k_hs, k_ts) && rows16(values, v_hs, v_ts)) {
    const dim3 sgrid((unsigned)n_blocks, (unsigned)heads);
    const dim3 sthreads((unsigned)(kWave * (block / 16)));
    RKV_DISPATCH_DIM(dim, D, {
      if (out.keys)
        summary_split_kernel<D, In, true><<<sgrid, sthreads, (size_t)split_lds, stream>>>(
            k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, counts, km, vm, el,
            value_norm, out);
      else
        summary_split_kernel<D, In, false><<<sgrid, sthreads, (size_t)split_lds, stream>>>(
            k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, counts, km, vm, el,
            value_norm, out);
    });
    int rc = check_launch("summary_split_kernel");
    if (rc) return rc;
    max_norm_kernel<<<dim3((unsigned)heads), dim3(256), 0, stream>>>(value_norm, n_blocks,
                                                                      max_value_norm);
    return check_launch("max_norm_kernel");
  }
  int waves = kSummaryWaves;
  while (stage && waves > 1 && waves * per_wave > kStageGroupMax) waves /= 2;
  dim3 grid((unsigned)((n_blocks + waves - 1) / waves), (unsigned)heads);
  dim3 threads(kWave * waves);
  const size_t lds = (size_t)(waves * per_wave);
#define RKV_SUMMARY_LAUNCH(STORE, STAGE)                                                   \
  RKV_DISPATCH_DIM(dim, D,                                                                 \
                   summary_kernel<D, In, STORE, STAGE><<<grid, threads, lds, stream>>>(    \
                       k, k_hs, k_ts, v, v_hs, v_ts, length, (int)block, n_blocks, counts, \
                       km, vm, el, value_norm, out))
  if (out.keys && stage) {
    RKV_SUMMARY_LAUNCH(true, true);
  } else if (out.keys) {
    RKV_SUMMARY_LAUNCH(true, false);
  } else if (stage) {
    RKV_SUMMARY_LAUNCH(false, true);
  } else {
    RKV_SUMMARY_LAUNCH(false, false);
  }
#undef RKV_SUMMARY_LAUNCH
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
  if (n_blocks > 0x7FFFFFFF)
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
