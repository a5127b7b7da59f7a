// Decode-step selection and mixed attention (src/refinekv/reference.py:10-73,
// the semantics the reference's Triton kernels in src/refinekv/kernels/ also
// follow).  No host sync, no allocation: the caller passes a workspace.
//
// Per KV head h the step has three phases:
//
//   score  (h, tile)   one 64-block tile: streams the tile's key means,
//                      ellipsoids and value means once; s = q.k_mean and the
//                      ellipsoid projection for every query row, z = s + ln n,
//                      delta, the tile's log-sum-exp partials of z and
//                      z + log cosh delta, and the representative accumulator
//                      sum_b exp(z_b - m_tile) v_mean_b over all its blocks
//                      (the z partial is that attention's (m, l)).
//   attend (h, tile)   after every score item of h: log Z / log C of each row
//                      from the tile partials, the risk, the GQA reduction,
//                      the non-finite fail-safes and the anchor union; the
//                      mask and the access counter; the tile's
//                      representative partial without its expanded blocks
//                      (l over the unexpanded blocks, acc minus the expanded
//                      blocks' terms: rounding error below fp32 eps times the
//                      tile's representative mass); then, from that partial,
//                      exact attention over the tile's expanded blocks token
//                      by token (64-row chunks, one shared max per chunk).
//                      One (m, l, acc) partial per query row and tile.
//   suffix (h)         exact attention over the generated tokens (a device
//                      length clamps them), independent of the decisions.
//   merge  (h, g, cols) the tiles' and the suffix's partials of row g ->
//                      bf16 output columns.
//
// Two ways to run them.  The split pipeline (default) launches three kernels:
// score; attend with the suffix as one more column of its grid; merge.  The
// persistent kernel (rkv_set_decode_pipeline) runs all phases in one launch:
// each XCD has a work queue that takes whole heads, so a head's items hand
// data to each other through that XCD's L2 (see decode_kernel).
//
// Scores, radii and log-sum-exp follow fixed fp32 orders shared with the CPU
// oracle (oracle/rkv_oracle.c), so masks and selection statistics are
// reproducible bit for bit; every summation order is fixed, so outputs are
// deterministic run to run.
#include "rkv_common.h"
#include "rkv_internal.h"

namespace rkv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr float kLog2e = 1.44269504088896341f;
constexpr int64_t kMaxHeads = 1024;    // KV heads in the persistent kernel (control block)
constexpr int64_t kMaxFusedDim = 128;    // widest head_dim the persistent kernel runs
constexpr size_t kMaxFusedLds = 64 * 1024;  // its LDS per workgroup (static + dynamic)
constexpr size_t kMaxFusedPrivate = 64;     // its private bytes per lane (no spill traffic)
// Control block of the persistent kernel (uint32 words; see decode_kernel).
constexpr int kMaxQueues = 16;               // one work queue per XCD (XCC_ID is 4 bits)
constexpr int64_t kCtlHeadTicket = 0, kCtlExits = 1, kCtlError = 2, kCtlEpoch = 3;
constexpr int64_t kCtlQueues = 16;           // per queue: -, -, ticket, -
constexpr int64_t kCtlSlots = kCtlQueues + 4 * kMaxQueues;  // per queue: kMaxHeads u64 slots
constexpr int64_t kCtlCounters = kCtlSlots + 2 * kMaxQueues * kMaxHeads;  // 2 x kMaxHeads
constexpr int64_t kControlWords = kCtlCounters + 2 * kMaxHeads;
constexpr uint32_t kSpinLimit = 1u << 20;  // polls before a dependency wait gives up (~1 s)

// Optional profiling events (rkv_set_profile_events): events[0] is recorded
// before the first kernel of a call and events[k] after its k-th kernel.
thread_local hipEvent_t* g_events = nullptr;

inline void mark(int i, hipStream_t stream) {
  if (g_events) (void)hipEventRecord(g_events[i], stream);
}

// Decode pipeline choice (rkv_set_decode_pipeline): 0 automatic (the split
// pipeline), 1 the persistent kernel, 2 the split pipeline, 3 the persistent
// kernel where it runs, else the split pipeline.
thread_local int g_pipeline = 0;

// ---------------------------------------------------------------------------
// Workspace layout.  The control block comes first and has a fixed size, so
// its words are at the same place for every shape that shares a workspace.
// ---------------------------------------------------------------------------
struct Layout {
  int64_t n_tiles, rows_per_block, row_blocks;
  // Padded row strides: every head's slice of an intermediate array covers
  // whole 256-byte lines, so no cache line holds two heads' data.
  int64_t z_stride, tile_stride, part_stride;
  int64_t control, z, delta, lse, tilebits, rep_acc, part_m, part_l, part_acc, total;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Rows of the GQA group one attention pass carries in registers: the next
// power of two >= group (at least 4), capped so that rows * head_dim / 16
// (per-lane accumulators) stays <= 64.
inline int64_t rows_per_block(int64_t group, int64_t dim) {
  const int64_t ch = dim / 16;
  const int64_t cap = 64 / ch;
  int64_t p = 16;
  while (p > cap) p >>= 1;
  int64_t want = 4;
  while (want < group && want < 16) want <<= 1;
  return want < p ? want : p;
}

Layout make_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks) {
  Layout L{};
  L.n_tiles = (n_blocks + kTile - 1) / kTile;
  L.rows_per_block = rows_per_block(group, dim);
  L.row_blocks = (group + L.rows_per_block - 1) / L.rows_per_block;
  auto round64 = [](int64_t x) { return (x + 63) / 64 * 64; };
  L.z_stride = L.n_tiles * kTile;
  L.tile_stride = round64(L.n_tiles);
  L.part_stride = round64(L.n_tiles + 1);  // one partial per tile + the suffix's
  const int64_t rows = heads * group;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off = align256(off + bytes);
    return at;
  };
  L.control = take(kControlWords * 4);
  L.z = take(rows * L.z_stride * 4);
  L.delta = take(rows * L.z_stride * 4);
  L.lse = take(rows * L.tile_stride * 4 * 4);
  L.tilebits = take(heads * L.tile_stride * 8);
  L.rep_acc = take(rows * L.tile_stride * dim * 4);
  L.part_m = take(rows * L.part_stride * 4);
  L.part_l = take(rows * L.part_stride * 4);
  L.part_acc = take(rows * L.part_stride * dim * 4);
  L.total = off;
  return L;
}

template <typename T>
T* at(void* ws, int64_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

// ---------------------------------------------------------------------------
// Shared scalar math (reference.py:16-34), identical to the CPU oracle.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float log_cosh(float delta) {
  const float c = clamp_max(delta, kDeltaMax);
  if (delta <= kDeltaMax) return logf_((expf_(c) + expf_(-c)) * 0.5f);
  return delta + logf_((1.0f + expf_(-2.0f * delta)) * 0.5f);
}

__device__ __forceinline__ float risk_of(float z, float delta, float log_z, float log_c,
                                         float vmax, float vnorm) {
  const float clipped = clamp_max(delta, kDeltaMax);
  const float t = expf_(clipped);
  const float exp_neg = expf_(-delta);
  float mass, th;
  if (delta <= kDeltaMax) {
    const float direct = (2.0f * vmax) * expf_(z - log_c);
    mass = direct * ((0.5f * (t + 1.0f / t)) - 1.0f);
    th = (t - 1.0f) / (t + 1.0f);
  } else {
    const float lcm1 = (delta + 2.0f * logf_(clamp_min(1.0f - exp_neg, 1e-30f))) - kLn2;
    mass = (2.0f * vmax) * expf_((z - log_c) + lcm1);
    th = (1.0f - exp_neg) / (1.0f + exp_neg);
  }
  const float value = ((2.0f * vnorm) * expf_(z - log_z)) * th;
  return mass + value;
}

__host__ __device__ __forceinline__ float inf_to_zero(float m) {
  return (m == kPosInf || m == kNegInf) ? 0.0f : m;
}

__device__ __forceinline__ int64_t block_count(int64_t b, int64_t n, int64_t block,
                                               int64_t length) {
  return b == n - 1 ? length - (n - 1) * block : block;
}

// Block-wide exclusive scan of one value per thread (integers: exact).
__device__ __forceinline__ uint32_t block_exclusive_scan(uint32_t v, uint32_t* wave_tot,
                                                         uint32_t& total) {
  const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
  uint32_t inc = v;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const uint32_t n = __shfl_up(inc, o, kWave);
    if (lane >= o) inc += n;
  }
  if (lane == kWave - 1) wave_tot[wave] = inc;
  __syncthreads();
  uint32_t before = 0;
  total = 0;
  for (int w = 0; w < kWaves; ++w) {
    if (w < wave) before += wave_tot[w];
    total += wave_tot[w];
  }
  __syncthreads();
  return before + inc - v;
}

// ---------------------------------------------------------------------------
// Phase 1: scores (+ representative accumulators) of one (head, tile)
// ---------------------------------------------------------------------------
struct ScoreArgs {
  const uint16_t* query;       // (H, G, D) bf16
  const uint16_t* key_mean;    // (H, N, D) bf16
  const uint16_t* ellipsoid;   // (H, N, D) bf16
  const uint16_t* value_mean;  // (H, N, D) bf16 (representatives only)
  float* z;                    // (H, G, N)
  float* delta;                // (H, G, N)
  float* lse;                  // (H, G, tiles, 4): zm, zl, cm, cl
  float* rep_acc;              // (H, G, tiles, D)
  int64_t n_blocks, n_tiles, block, length;
  int64_t z_stride;            // row stride of z / delta (blocks padded to whole tiles)
  int64_t tile_stride;         // row stride of the per-tile arrays (tiles padded to 64)
  int group;
  float scale;
};

inline size_t score_smem(int64_t group, int64_t dim, bool reps) {
  return sizeof(float) * (2 * group * dim + 5 * group * kTile) +
         (reps ? sizeof(uint16_t) * kTile * dim : 0);
}

template <int D, bool REPS>
__device__ __forceinline__ void score_tile(const ScoreArgs& a, int64_t h, int64_t tile,
                                          unsigned char* dyn) {
  constexpr int CH = D / 16;
  float* smem = reinterpret_cast<float*>(dyn);
  const int G = a.group;
  float* qs = smem;                 // [G][D] bf16(q)
  float* q2s = qs + G * D;          // [G][D] bf16(q^2)
  float* sdot = q2s + G * D;        // [G][64]
  float* pdot = sdot + G * kTile;   // [G][64]
  float* zbuf = pdot + G * kTile;   // [G][64]
  float* zcbuf = zbuf + G * kTile;  // [G][64]
  float* pbuf = zcbuf + G * kTile;  // [G][64] exp(z - m_tile)
  uint32_t* vsm = reinterpret_cast<uint32_t*>(pbuf + G * kTile);  // [64][D/2] value means

  const int tid = item_tid(), wave = tid / kWave, lane = tid % kWave;
  const int grp = lane / 16, c = lane % 16;
  const int64_t N = a.n_blocks;

  // Issue every load of the tile before the first wait.  Blocks past the end
  // read block N-1 (their scores are discarded, their weights are 0).
  RawBf16<CH> kraw[4], eraw[4], vraw[REPS ? 4 : 1];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    int64_t b = tile * kTile + wave * 16 + it * 4 + grp;
    b = b < N ? b : N - 1;
    const int64_t o = (h * N + b) * D + c * CH;
    kraw[it] = load_raw<CH>(a.key_mean + o);
    eraw[it] = load_raw<CH>(a.ellipsoid + o);
    if constexpr (REPS) vraw[it] = load_raw<CH>(a.value_mean + o);
  }
  const uint32_t* q32 = reinterpret_cast<const uint32_t*>(a.query + h * G * D);
  for (int i = tid; i < G * D / 2; i += kThreads) {
    const uint32_t u = q32[i];
    const float q0 = bits_f32(u << 16), q1 = bits_f32(u & 0xFFFF0000u);
    qs[2 * i] = q0;
    qs[2 * i + 1] = q1;
    q2s[2 * i] = round_bf16(q0 * q0);
    q2s[2 * i + 1] = round_bf16(q1 * q1);
  }
  // ln(count): every block holds block_size tokens except the last.
  const float ln_full = logf_((float)a.block);
  const float ln_last = logf_((float)(a.length - (N - 1) * a.block));
  __syncthreads();

  float km[4][CH], el[4][CH];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    unpack(kraw[it], km[it]);
    unpack(eraw[it], el[it]);
    if constexpr (REPS) {
      // stage the value means in LDS for the per-row representative sums
      const int bl = wave * 16 + it * 4 + grp;
#pragma unroll
      for (int j = 0; j < CH / 2; ++j) vsm[bl * (D / 2) + c * (CH / 2) + j] = vraw[it].w[j];
    }
  }

  for (int g = 0; g < G; ++g) {
    float qv[CH], q2v[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      qv[i] = qs[g * D + c * CH + i];
      q2v[i] = q2s[g * D + c * CH + i];
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      // DSUM: this lane's CH consecutive elements left to right, then the
      // 16-lane butterfly (complete in lane 15 of the row).
      float s = qv[0] * km[it][0];
      float p = q2v[0] * el[it][0];
#pragma unroll
      for (int i = 1; i < CH; ++i) {
        s = s + qv[i] * km[it][i];
        p = p + q2v[i] * el[it][i];
      }
      s = row16_sum_last(s);
      p = row16_sum_last(p);
      if (c == 15) {
        const int bl = wave * 16 + it * 4 + grp;
        sdot[g * kTile + bl] = s;
        pdot[g * kTile + bl] = p;
      }
    }
  }
  __syncthreads();

  for (int idx = tid; idx < G * kTile; idx += kThreads) {
    const int g = idx / kTile, bl = idx % kTile;
    const int64_t b = tile * kTile + bl;
    float z = kNegInf, zc = kNegInf;
    if (b < N) {
      const float s = sdot[idx] * a.scale;
      const float dl = (sqrtf(clamp_min(pdot[idx], 0.0f)) * a.scale) * kInflate;
      z = s + (b == N - 1 ? ln_last : ln_full);
      zc = z + log_cosh(dl);
      const int64_t o = (h * G + g) * a.z_stride + b;
      a.z[o] = z;
      a.delta[o] = dl;
    }
    zbuf[idx] = z;
    zcbuf[idx] = zc;
  }
  __syncthreads();

  for (int g = wave; g < G; g += kWaves) {
    const float x = zbuf[g * kTile + lane];
    const float zm = wave_nanmax_u(x);
    const float e = expf_(x - inf_to_zero(zm));
    const float zl = wave_sum_u(e);
    const float xc = zcbuf[g * kTile + lane];
    const float cm = wave_nanmax_u(xc);
    const float cl = wave_sum_u(expf_(xc - inf_to_zero(cm)));
    if (lane == 0) {
      *reinterpret_cast<float4*>(a.lse + ((h * G + g) * a.tile_stride + tile) * 4) =
          make_float4(zm, zl, cm, cl);
    }
    if constexpr (REPS) {
      // Representative accumulator of row g: sum_b e_b v_b over the tile.
      // Lane group grp takes blocks grp, grp+4, ...; the four partial sums
      // are then added by two cross-row permutes.
      pbuf[g * kTile + lane] = e;
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      float acc[CH];
#pragma unroll
      for (int k = 0; k < kTile / 4; ++k) {
        const int bl = grp + 4 * k;
        const float w = pbuf[g * kTile + bl];
        RawBf16<CH> r;
#pragma unroll
        for (int j = 0; j < CH / 2; ++j) r.w[j] = vsm[bl * (D / 2) + c * (CH / 2) + j];
        float v[CH];
        unpack(r, v);
#pragma unroll
        for (int i = 0; i < CH; ++i) acc[i] = k == 0 ? w * v[i] : acc[i] + w * v[i];
      }
#pragma unroll
      for (int i = 0; i < CH; ++i) {
        acc[i] = acc[i] + shfl_xor(acc[i], 16);
        acc[i] = acc[i] + shfl_xor(acc[i], 32);
      }
      if (grp == 0) {
        float* o = a.rep_acc + ((h * G + g) * a.tile_stride + tile) * D + c * CH;
#pragma unroll
        for (int i = 0; i < CH; ++i) o[i] = acc[i];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Phase 2: decisions (+ representative corrections) of one (head, tile)
// ---------------------------------------------------------------------------
struct DecideArgs {
  const float* z;
  const float* delta;
  const float* lse;
  const float* value_norm;      // (H, N)
  const float* max_value_norm;  // (H)
  const uint16_t* value_mean;   // (H, N, D) (representatives only)
  const uint8_t* anchor;        // (H, N) or null
  uint8_t* mask;                // (H, N)
  uint64_t* tilebits;           // (H, tiles)
  float* risk_out;              // (H, G, N) or null
  float* stats_out;             // (H, G, 2) or null: log Z, log C
  unsigned long long* accessed; // or null
  const float* rep_acc;         // (H, G, tiles, D) from the score pass (decode only)
  int64_t n_blocks, n_tiles, block, length;
  int64_t z_stride, tile_stride;  // padded row strides (see ScoreArgs)
  int group, reduction, dim;
  float eps;
};

constexpr int kLseRegs = 4;  // tile partials per lane held in registers (tiles <= 256)

// Merge the tile partials (m, l) of one row in the fixed order: max first,
// then 64 lane accumulators (tile t -> lane t % 64, left to right) and a
// butterfly.  m[k], l[k] hold tile lane + 64 k (k < kLseRegs), preloaded.
__device__ __forceinline__ float merge_lse(const float (&m)[kLseRegs], const float (&l)[kLseRegs],
                                           const float* part, int which, int64_t n_tiles,
                                           int lane) {
  // (register part unrolled, then the rest from memory: same order as one
  // loop over t, without indexing the register arrays at run time)
  constexpr int64_t kRegTiles = (int64_t)kLseRegs * kWave;
  float mx = kNegInf;
#pragma unroll
  for (int k = 0; k < kLseRegs; ++k)
    if (lane + (int64_t)k * kWave < n_tiles) mx = nanmax(mx, m[k]);
  for (int64_t t = lane + kRegTiles; t < n_tiles; t += kWave)
    mx = nanmax(mx, part[t * 4 + 2 * which]);
  mx = wave_nanmax_u(mx);
  const float ms = inf_to_zero(mx);
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < kLseRegs; ++k) {
    if (lane + (int64_t)k * kWave < n_tiles) {
      const float term = l[k] * expf_(m[k] - ms);
      acc = k == 0 ? term : acc + term;
    }
  }
  for (int64_t t = lane + kRegTiles; t < n_tiles; t += kWave)
    acc = acc + part[t * 4 + 2 * which + 1] * expf_(part[t * 4 + 2 * which] - ms);
  return logf_(wave_sum_u(acc)) + ms;
}

constexpr int kRiskPerThread = kMaxGroup * kTile / kThreads;  // (row, block) pairs per thread

// The tile's representative partial after its expanded blocks are removed,
// left in LDS for the attention that follows in the same workgroup.
struct RepShared {
  float* acc;      // [G][D]
  float* l;        // [G] (0: no live representative)
  float* m;        // [G] the partial's max, inf_to_zero(tile max of z)
  uint64_t* bits;  // the tile's expanded-block ballot
};

__device__ __forceinline__ void decide_tile(const DecideArgs& a, int64_t h, int64_t tile,
                                            const RepShared* rep) {
  __shared__ float gstat[kMaxGroup][2];
  __shared__ float risk_s[kMaxGroup][kTile];
  __shared__ float psel[kMaxGroup][kTile];
  __shared__ uint64_t sel_bits;
  const int tid = item_tid(), wave = tid / kWave, lane = tid % kWave;
  const int G = a.group;
  const int64_t N = a.n_blocks, T = a.n_tiles;
  const int64_t nvalid = N - tile * kTile >= kTile ? kTile : N - tile * kTile;

  // ---- every load this tile needs before any wait ---------------------
  float pz_m[kMaxGroup / kWaves][kLseRegs], pz_l[kMaxGroup / kWaves][kLseRegs];
  float pc_m[kMaxGroup / kWaves][kLseRegs], pc_l[kMaxGroup / kWaves][kLseRegs];
#pragma unroll
  for (int gi = 0; gi < kMaxGroup / kWaves; ++gi) {
    const int g = wave + gi * kWaves;
#pragma unroll
    for (int k = 0; k < kLseRegs; ++k) {
      const int64_t t = lane + (int64_t)k * kWave;
      if (g < G && t < T) {
        const float4 v =
            *reinterpret_cast<const float4*>(a.lse + ((h * G + g) * a.tile_stride + t) * 4);
        pz_m[gi][k] = v.x;
        pz_l[gi][k] = v.y;
        pc_m[gi][k] = v.z;
        pc_l[gi][k] = v.w;
      } else {
        pz_m[gi][k] = pc_m[gi][k] = kNegInf;
        pz_l[gi][k] = pc_l[gi][k] = 0.0f;
      }
    }
  }
  float rz[kRiskPerThread], rd[kRiskPerThread], rv[kRiskPerThread];
#pragma unroll
  for (int k = 0; k < kRiskPerThread; ++k) {
    const int idx = tid + k * kThreads;
    const int g = idx / kTile, bl = idx % kTile;
    if (g < G && bl < nvalid) {
      const int64_t b = tile * kTile + bl;
      const int64_t o = (h * G + g) * a.z_stride + b;
      rz[k] = a.z[o];
      rd[k] = a.delta[o];
      rv[k] = a.value_norm[h * N + b];
    } else {
      rz[k] = rd[k] = rv[k] = 0.0f;
    }
  }
  const bool anchored =
      wave == 0 && a.anchor && lane < nvalid && a.anchor[h * N + tile * kTile + lane] != 0;
  const float vmax = a.max_value_norm[h];
  // Representative partial of this tile: the z max (m of the partial) for
  // the rows this wave corrects, and the accumulator slice of this thread.
  float tile_m[kMaxGroup / kWaves];
#pragma unroll
  for (int gi = 0; gi < kMaxGroup / kWaves; ++gi) {
    const int g = wave + gi * kWaves;
    tile_m[gi] = (rep && g < G) ? a.lse[((h * G + g) * a.tile_stride + tile) * 4] : 0.0f;
  }
  constexpr int kAccPerThread = kMaxGroup * 256 / kThreads;  // G * D <= 16 * 256
  float racc[kAccPerThread];
  const int GD = G * a.dim;
#pragma unroll
  for (int k = 0; k < kAccPerThread; ++k) {
    const int idx = tid + k * kThreads;
    racc[k] = 0.0f;
    if (rep && idx < GD) {
      const int g = idx / a.dim, d = idx % a.dim;
      racc[k] = a.rep_acc[((h * G + g) * a.tile_stride + tile) * a.dim + d];
    }
  }

  // ---- global log Z / log C of each row --------------------------------
#pragma unroll
  for (int gi = 0; gi < kMaxGroup / kWaves; ++gi) {
    const int g = wave + gi * kWaves;
    if (g >= G) break;
    const float* part = a.lse + (h * G + g) * a.tile_stride * 4;
    const float lz = merge_lse(pz_m[gi], pz_l[gi], part, 0, T, lane);  // log Z
    const float lc = merge_lse(pc_m[gi], pc_l[gi], part, 1, T, lane);
    if (lane == 0) {
      gstat[g][0] = lz;
      gstat[g][1] = lc;
      if (a.stats_out && tile == 0) {
        a.stats_out[(h * G + g) * 2] = lz;
        a.stats_out[(h * G + g) * 2 + 1] = lc;
      }
    }
  }
  __syncthreads();

#pragma unroll
  for (int k = 0; k < kRiskPerThread; ++k) {
    const int idx = tid + k * kThreads;
    const int g = idx / kTile, bl = idx % kTile;
    if (g >= G) break;
    float r = 0.0f;
    if (bl < nvalid) {
      r = risk_of(rz[k], rd[k], gstat[g][0], gstat[g][1], vmax, rv[k]);
      if (a.risk_out) a.risk_out[(h * G + g) * N + tile * kTile + bl] = r;
    }
    risk_s[g][bl] = r;
  }
  __syncthreads();

  if (wave == 0) {
    const int64_t b = tile * kTile + lane;
    const bool valid = lane < nvalid;
    bool bad_global = false;
    for (int g = 0; g < G; ++g) bad_global |= !is_finite(gstat[g][0]) || !is_finite(gstat[g][1]);
    bool sel = false, bad_local = false;
    float acc = 0.0f, mx = 0.0f;
    for (int g = 0; g < G; ++g) {
      const float r = risk_s[g][lane];
      bad_local |= !is_finite(r);
      if (g == 0) {
        acc = r;
        mx = r;
      } else {
        acc = acc + r;
        mx = nanmax(mx, r);
      }
      if (a.reduction == kAny) sel |= r > a.eps;
    }
    if (a.reduction == kMean) sel = (acc / (float)G) > a.eps;
    if (a.reduction == kMax) sel = mx > a.eps;
    sel = (sel || bad_global || bad_local || anchored) && valid;
    if (valid) a.mask[h * N + b] = sel ? 1 : 0;
    const uint64_t bits = __ballot(sel);
    if (lane == 0) {
      a.tilebits[h * a.tile_stride + tile] = bits;
      sel_bits = bits;
    }
    if (a.accessed) {
      unsigned long long term =
          valid ? (sel ? (unsigned long long)block_count(b, N, a.block, a.length) : 1ull) : 0ull;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) term += __shfl_xor(term, o, kWave);
      if (lane == 0) atomicAdd(a.accessed, term);
    }
  }
  if (!rep) return;
  __syncthreads();

  // ---- representatives of this tile: drop the expanded blocks ----------
  // (thread tid's prefetched z/delta pair k is row wave + 4k, block lane)
  const uint64_t bits = sel_bits;
  const int nsel = __popcll(bits);
  if (tid == 0) *rep->bits = bits;
#pragma unroll
  for (int gi = 0; gi < kMaxGroup / kWaves; ++gi) {
    const int g = wave + gi * kWaves;
    if (g >= G) break;
    const bool valid = lane < nvalid;
    const bool expanded = (bits >> lane) & 1ull;
    const float mt = inf_to_zero(tile_m[gi]);
    const float e = valid ? expf_(rz[gi] - mt) : 0.0f;
    const float l = wave_sum_u(expanded ? 0.0f : e);
    psel[g][lane] = expanded ? e : 0.0f;
    if (lane == 0) {
      rep->l[g] = nsel == nvalid ? 0.0f : l;
      rep->m[g] = mt;
    }
  }
  __syncthreads();
  const int D = a.dim;
  const bool correct = nsel > 0 && nsel < nvalid;
#pragma unroll
  for (int k = 0; k < kAccPerThread; ++k) {
    const int idx = tid + k * kThreads;
    if (idx >= GD) break;
    const int g = idx / D, d = idx % D;
    float acc = racc[k];
    uint64_t m = correct ? bits : 0ull;
    while (m) {
      // up to 8 expanded blocks at a time: their loads in flight together
      constexpr int kBatch = 8;
      int js[kBatch];
      uint16_t raw[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        js[u] = m ? __builtin_ctzll(m) : -1;
        if (m) m &= m - 1;
        const int jj = js[u] < 0 ? 0 : js[u];
        raw[u] = a.value_mean[(h * N + tile * kTile + jj) * D + d];
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
        if (js[u] >= 0) acc = acc - psel[g][js[u]] * bf16_to_f32(raw[u]);
    }
    rep->acc[idx] = acc;
  }
}

template <int D, bool REPS>
__global__ __launch_bounds__(kThreads) void score_kernel(ScoreArgs a) {
  extern __shared__ unsigned char score_dyn[];
  score_tile<D, REPS>(a, blockIdx.y, blockIdx.x, score_dyn);
}

__global__ __launch_bounds__(kThreads) void decide_kernel(DecideArgs a) {
  decide_tile(a, blockIdx.y, blockIdx.x, nullptr);
}

// ---------------------------------------------------------------------------
// Phase 3: exact attention over a tile's expanded blocks, and over the suffix
// ---------------------------------------------------------------------------
// After deciding a tile, the same workgroup attends to the tile's expanded
// blocks token by token, starting from the tile's representative partial, and
// writes one (m, l, acc) partial per query row: slot `tile` of the row.  The
// generated suffix is one more item per head (slot n_tiles), independent of
// the decisions.  The merge then combines n_tiles + 1 partials per row.
struct AttendArgs {
  DecideArgs decide;
  const uint16_t* query;       // (H, G, D) bf16
  const uint16_t* key_pages;   // head h at key_pages + h * kp_hs; rows (N*B, D)
  const uint16_t* value_pages;
  const uint16_t* key_suffix;  // token t of head h at h * ks_hs + t * ks_ts
  const uint16_t* value_suffix;
  const int32_t* suffix_len_dev;  // or null
  float* part_m;               // (H, G, part_stride)
  float* part_l;
  float* part_acc;             // (H, G, part_stride, D)
  int64_t kp_hs, vp_hs, ks_hs, ks_ts, vs_hs, vs_ts;
  int64_t suffix_cap, part_stride;
  int row_blocks;
  float scale;
};

constexpr int kRowBatch = 4;                  // rows per lane group per chunk
constexpr int kChunkRows = 16 * kRowBatch;    // rows per chunk (one per lane of a wave)

// Exact logits of one K row for this lane's query slice (DSUM order, natural
// units), complete in lane 15 of the 16-lane group.
template <int D, int GBM>
__device__ __forceinline__ void row_logits(const float (&q)[GBM][D / 16], const float (&k)[D / 16],
                                           float (&x)[GBM]) {
  constexpr int CH = D / 16;
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    float s = q[g][0] * k[0];
#pragma unroll
    for (int i = 1; i < CH; ++i) s = s + q[g][i] * k[i];
    x[g] = row16_sum_last(s);
  }
}

// CH consecutive floats (CH even; 16-byte aligned when CH % 4 == 0, else 8).
template <int CH>
__device__ __forceinline__ void load_f32(const float* p, float (&out)[CH]) {
  if constexpr (CH % 4 == 0) {
#pragma unroll
    for (int j = 0; j < CH / 4; ++j) {
      const float4 v = reinterpret_cast<const float4*>(p)[j];
      out[4 * j] = v.x;
      out[4 * j + 1] = v.y;
      out[4 * j + 2] = v.z;
      out[4 * j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < CH / 2; ++j) {
      const float2 v = reinterpret_cast<const float2*>(p)[j];
      out[2 * j] = v.x;
      out[2 * j + 1] = v.y;
    }
  }
}

template <int GBM>
struct AttendShared {
  float xlog[GBM][kChunkRows];
  float cmax[GBM], csum[GBM];
};

// Folds n_rows K/V rows into the state, 64 rows per chunk: pass 1 loads the
// chunk's K and V and writes its logits, pass 2 weighs the V rows with one
// shared max per chunk.  row(v, kp, vp) points kp / vp at row v and returns
// false for a masked row (kp / vp must then stay valid addresses).
// The online-softmax state of GBM query rows is (m, l), uniform over the
// workgroup, and acc, per 16-lane group (this lane's D/16 columns; the groups
// are summed at the end).
template <int D, int GBM, typename RowFn>
__device__ __forceinline__ void attend_rows(const float (&q)[GBM][D / 16], float (&m_run)[GBM],
                                            float (&l_run)[GBM], float (&acc)[GBM][D / 16],
                                            int64_t n_rows, int gn, float scale, RowFn row,
                                            const uint16_t* kdef, const uint16_t* vdef,
                                            AttendShared<GBM>& sh) {
  constexpr int CH = D / 16;
  // Double-buffer the K/V rows (the next chunk's loads in flight while this
  // chunk is computed) when the registers allow it.
  constexpr bool kPrefetch = GBM * CH <= 32;
  const int tid = item_tid(), lg = tid >> 4, c = tid & 15, wave = tid / kWave;
  const int lane = tid % kWave;
  auto issue = [&](int64_t c0, RawBf16<CH> (&kr)[kRowBatch], RawBf16<CH> (&vr)[kRowBatch]) {
    uint32_t okm = 0;
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int64_t v = c0 + lg + 16 * u;
      const uint16_t* kp = kdef;
      const uint16_t* vp = vdef;
      if (v < n_rows && row(v, kp, vp)) okm |= 1u << u;
      kr[u] = load_raw<CH>(kp + c * CH);
      vr[u] = load_raw<CH>(vp + c * CH);
    }
    return okm;
  };
  auto consume = [&](const RawBf16<CH> (&kr)[kRowBatch], const RawBf16<CH> (&vr)[kRowBatch],
                     uint32_t okm) {
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      float kv[CH], x[GBM];
      unpack(kr[u], kv);
      row_logits<D, GBM>(q, kv, x);
      if (c == 15) {
#pragma unroll
        for (int g = 0; g < GBM; ++g)
          sh.xlog[g][lg + 16 * u] = ((okm >> u) & 1u) ? x[g] * scale : kNegInf;
      }
    }
    __syncthreads();
    // chunk max and sum per query row, one wave per row
    for (int g = wave; g < gn; g += kWaves) {
      const float x = sh.xlog[g][lane];
      const float cm = wave_nanmax_u(x);
      const float ms = cm == kNegInf ? 0.0f : cm;
      const float sum = wave_sum_u(__builtin_amdgcn_exp2f((x - ms) * kLog2e));
      if (lane == 0) {
        sh.cmax[g] = cm;
        sh.csum[g] = sum;
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g >= gn) break;
      const float cm = sh.cmax[g];
      const float mn = fmaxf(m_run[g], cm);
      if (mn == kNegInf) continue;
      const float sa = __builtin_amdgcn_exp2f((m_run[g] - mn) * kLog2e);
      const float sb = __builtin_amdgcn_exp2f((cm - mn) * kLog2e);
      l_run[g] = l_run[g] * sa + sh.csum[g] * sb;
#pragma unroll
      for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] * sa;
      m_run[g] = mn;
    }
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      float v[CH];
      unpack(vr[u], v);
#pragma unroll
      for (int g = 0; g < GBM; ++g) {
        if (g >= gn) break;
        const float ms = m_run[g] == kNegInf ? 0.0f : m_run[g];
        const float p = __builtin_amdgcn_exp2f((sh.xlog[g][lg + 16 * u] - ms) * kLog2e);
#pragma unroll
        for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] + p * v[i];
      }
    }
    __syncthreads();  // this chunk's logits are consumed
  };
  if (n_rows <= 0) return;
  if constexpr (kPrefetch) {
    RawBf16<CH> ka[kRowBatch], va[kRowBatch], kb[kRowBatch], vb[kRowBatch];
    uint32_t oka = issue(0, ka, va), okb = 0;
    for (int64_t c0 = 0;;) {
      if (c0 + kChunkRows < n_rows) okb = issue(c0 + kChunkRows, kb, vb);
      consume(ka, va, oka);
      c0 += kChunkRows;
      if (c0 >= n_rows) break;
      if (c0 + kChunkRows < n_rows) oka = issue(c0 + kChunkRows, ka, va);
      consume(kb, vb, okb);
      c0 += kChunkRows;
      if (c0 >= n_rows) break;
    }
  } else {
    for (int64_t c0 = 0; c0 < n_rows; c0 += kChunkRows) {
      RawBf16<CH> kr[kRowBatch], vr[kRowBatch];
      const uint32_t okm = issue(c0, kr, vr);
      consume(kr, vr, okm);
    }
  }
}

// Sums the 16 lane groups (one shared max: plain adds) and writes rows
// row0 .. row0+gn-1 of the partial arrays at `slot`.
template <int D, int GBM>
__device__ __forceinline__ void write_partial(const float (&m_run)[GBM], const float (&l_run)[GBM],
                                              float (&acc)[GBM][D / 16], int gn,
                                              const AttendArgs& a, int64_t row0, int64_t slot,
                                              float (&xacc)[kWaves][GBM][D]) {
  constexpr int CH = D / 16;
  const int tid = item_tid(), c = tid & 15, wave = tid / kWave, grp = (tid % kWave) >> 4;
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      acc[g][i] = acc[g][i] + shfl_xor(acc[g][i], 16);
      acc[g][i] = acc[g][i] + shfl_xor(acc[g][i], 32);
    }
  }
  __syncthreads();
  if (grp == 0) {
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g >= gn) break;
#pragma unroll
      for (int i = 0; i < CH; ++i) xacc[wave][g][c * CH + i] = acc[g][i];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < gn * D; idx += kThreads) {
    const int g = idx / D, d = idx % D;
    const int64_t at = (row0 + g) * a.part_stride + slot;
    a.part_acc[at * D + d] = ((xacc[0][g][d] + xacc[1][g][d]) + xacc[2][g][d]) + xacc[3][g][d];
    if (d == 0) {
      a.part_m[at] = m_run[g];
      a.part_l[at] = l_run[g];
    }
  }
}

template <int D, int GBM>
__device__ __forceinline__ void load_query(const AttendArgs& a, int64_t h, int g0, int gn,
                                           float (&q)[GBM][D / 16]) {
  constexpr int CH = D / 16;
  const int c = item_tid() & 15;
  const int G = a.decide.group;
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    const int gg = g < gn ? g : 0;
    RawBf16<CH> r = load_raw<CH>(a.query + ((h * G + g0 + gg) * D + c * CH));
    unpack(r, q[g]);
  }
}

// Decide tile `tile` of head h (RepShared in `dyn`), then attend to its
// expanded blocks from its representative partial.
template <int D, int GBM>
__device__ __forceinline__ void decide_attend_tile(const AttendArgs& a, int64_t h, int64_t tile,
                                                   unsigned char* dyn) {
  constexpr int CH = D / 16;
  __shared__ AttendShared<GBM> sh;
  __shared__ float xacc[kWaves][GBM][D];
  __shared__ int32_t blocks[kTile];
  __shared__ uint64_t tile_bits;
  const DecideArgs& da = a.decide;
  const int G = da.group;
  float* rep_acc = reinterpret_cast<float*>(dyn);
  RepShared rep{rep_acc, rep_acc + G * D, rep_acc + G * D + G, &tile_bits};
  decide_tile(da, h, tile, &rep);
  __syncthreads();

  const int tid = item_tid(), lg = tid >> 4, c = tid & 15;
  const uint64_t bits = tile_bits;
  const int nsel = __popcll(bits);
  if (tid < nsel) blocks[tid] = (int32_t)(tile * kTile + nth_set_bit(bits, tid));
  __syncthreads();
  const int64_t N = da.n_blocks, B = da.block, L = da.length;
  const uint16_t* kbase = a.key_pages + h * a.kp_hs;
  const uint16_t* vbase = a.value_pages + h * a.vp_hs;
  const int32_t* blk = blocks;
  auto row = [=](int64_t v, const uint16_t*& kp, const uint16_t*& vp) {
    const int64_t j = v / B, t = v - j * B;
    const int64_t b = blk[j];
    if (t >= block_count(b, N, B, L)) return false;
    kp = kbase + (b * B + t) * D;
    vp = vbase + (b * B + t) * D;
    return true;
  };
  for (int rb = 0; rb < a.row_blocks; ++rb) {
    const int g0 = rb * GBM, gn = min(GBM, G - g0);
    float q[GBM][CH];
    load_query<D, GBM>(a, h, g0, gn, q);
    float m_run[GBM], l_run[GBM], acc[GBM][CH];
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      const int gg = g < gn ? g0 + g : 0;
      const bool live = g < gn && rep.l[gg] > 0.0f;
      m_run[g] = live ? rep.m[gg] : kNegInf;
      l_run[g] = live ? rep.l[gg] : 0.0f;
#pragma unroll
      for (int i = 0; i < CH; ++i)
        acc[g][i] = (live && lg == 0) ? rep.acc[gg * D + c * CH + i] : 0.0f;
    }
    attend_rows<D, GBM>(q, m_run, l_run, acc, (int64_t)nsel * B, gn, a.scale, row, kbase, vbase,
                        sh);
    write_partial<D, GBM>(m_run, l_run, acc, gn, a, h * G + g0, tile, xacc);
  }
}

// Attention of head h's query rows over the generated suffix (slot n_tiles).
template <int D, int GBM>
__device__ __forceinline__ void suffix_item(const AttendArgs& a, int64_t h) {
  constexpr int CH = D / 16;
  __shared__ AttendShared<GBM> sh;
  __shared__ float xacc[kWaves][GBM][D];
  const int G = a.decide.group;
  int64_t S = a.suffix_cap;
  if (a.suffix_len_dev) {
    const int64_t s = *a.suffix_len_dev;
    S = s < 0 ? 0 : (s > a.suffix_cap ? a.suffix_cap : s);
  }
  const uint16_t* kbase = a.key_pages + h * a.kp_hs;  // valid rows for masked lanes
  const uint16_t* vbase = a.value_pages + h * a.vp_hs;
  const uint16_t* ks = a.key_suffix + h * a.ks_hs;
  const uint16_t* vs = a.value_suffix + h * a.vs_hs;
  const int64_t kts = a.ks_ts, vts = a.vs_ts;
  auto row = [=](int64_t v, const uint16_t*& kp, const uint16_t*& vp) {
    kp = ks + v * kts;
    vp = vs + v * vts;
    return true;
  };
  for (int rb = 0; rb < a.row_blocks; ++rb) {
    const int g0 = rb * GBM, gn = min(GBM, G - g0);
    float q[GBM][CH];
    load_query<D, GBM>(a, h, g0, gn, q);
    float m_run[GBM], l_run[GBM], acc[GBM][CH];
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      m_run[g] = kNegInf;
      l_run[g] = 0.0f;
#pragma unroll
      for (int i = 0; i < CH; ++i) acc[g][i] = 0.0f;
    }
    attend_rows<D, GBM>(q, m_run, l_run, acc, S, gn, a.scale, row, kbase, vbase, sh);
    write_partial<D, GBM>(m_run, l_run, acc, gn, a, h * G + g0, a.decide.n_tiles, xacc);
  }
}

inline size_t attend_smem(int64_t group, int64_t dim) {
  return sizeof(float) * (group * dim + 2 * group);
}

// Split pipeline, kernel 2: grid (tiles + 1, H); the last column is the suffix.
template <int D, int GBM>
__global__ __launch_bounds__(kThreads) void attend_kernel(AttendArgs a) {
  extern __shared__ unsigned char attend_dyn[];
  if ((int64_t)blockIdx.x == a.decide.n_tiles)
    suffix_item<D, GBM>(a, blockIdx.y);
  else
    decide_attend_tile<D, GBM>(a, blockIdx.y, blockIdx.x, attend_dyn);
}

// ---------------------------------------------------------------------------
// Phase 4: merge a row's partials -> bf16 output columns
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float* part_m;    // (H, G, part_stride)
  const float* part_l;
  const float* part_acc;  // (H, G, part_stride, D)
  uint16_t* out;          // (H*G, D)
  int64_t part_stride;    // row stride of the partials
  int group, parts, dim;  // parts = n_tiles + 1
};

constexpr int kMergeD = 32;                   // output columns per item
constexpr int kMergeK = kThreads / kMergeD;   // partial stripes
constexpr int kMergeBatch = 8;                // partials per stripe per batch

__device__ __forceinline__ void merge_item(const MergeArgs& a, int64_t h, int g, int dc) {
  __shared__ float red[kWaves];
  __shared__ float num_s[kMergeK][kMergeD];
  __shared__ float den_s[kMergeK];
  const int P = a.parts, D = a.dim;
  const int64_t r = h * a.group + g;
  const int tid = item_tid(), lane = tid % kWave, wave = tid / kWave;

  float mx = kNegInf;
  for (int i = tid; i < P; i += kThreads) {
    const float l = a.part_l[r * a.part_stride + i];
    const float m = a.part_m[r * a.part_stride + i];
    if (l > 0.0f) mx = fmaxf(mx, m);
  }
  mx = wave_nanmax_u(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float Ms = M == kNegInf ? 0.0f : M;

  const int dl = tid % kMergeD, kk = tid / kMergeD;
  const int d = dc * kMergeD + dl;
  const int dd = d < D ? d : 0;
  float num = 0.0f, den = 0.0f;
  for (int i0 = kk; i0 < P; i0 += kMergeK * kMergeBatch) {
    float mv[kMergeBatch], lv[kMergeBatch], av[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int i = i0 + u * kMergeK;
      const int ii = i < P ? i : 0;
      mv[u] = a.part_m[r * a.part_stride + ii];
      lv[u] = a.part_l[r * a.part_stride + ii];
      av[u] = a.part_acc[(r * a.part_stride + ii) * D + dd];
    }
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      if (i0 + u * kMergeK < P && lv[u] > 0.0f) {
        const float e = __builtin_amdgcn_exp2f((mv[u] - Ms) * kLog2e);
        den = den + lv[u] * e;
        num = num + av[u] * e;
      }
    }
  }
  num_s[kk][dl] = num;
  if (dl == 0) den_s[kk] = den;
  __syncthreads();
  if (tid < kMergeD && d < D) {
    float n = num_s[0][tid], den_all = den_s[0];
    for (int j = 1; j < kMergeK; ++j) {
      n = n + num_s[j][tid];
      den_all = den_all + den_s[j];
    }
    a.out[r * D + d] = bf16_rne(n / fmaxf(den_all, 1e-30f));
  }
}

// Split pipeline, kernel 3: grid (H * G, ceil(D / 32)).
__global__ __launch_bounds__(kThreads) void merge_kernel(MergeArgs a) {
  merge_item(a, blockIdx.x / a.group, blockIdx.x % a.group, blockIdx.y);
}

// ---------------------------------------------------------------------------
// The persistent decode kernel
// ---------------------------------------------------------------------------
struct DecodeArgs {
  ScoreArgs score;
  AttendArgs attend;
  MergeArgs merge;
  uint32_t* control;  // kControlWords words, zero when the workspace is new
  int heads, merge_cols;
};

// This workgroup's XCD (HW_REG_XCC_ID bits [3:0]).
__device__ __forceinline__ uint32_t xcc_id() {
  return __builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & (kMaxQueues - 1);
}

__device__ __forceinline__ uint32_t load_dev(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Thread 0: polls until *p >= target (bounded: on timeout it sets the sticky
// error word and returns).
__device__ __forceinline__ void poll_at_least(const uint32_t* p, uint32_t target, uint32_t* err) {
  for (uint32_t spins = 0; load_dev(p) < target; ++spins) {
    if (spins > kSpinLimit) {
      __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(2);
  }
}

// Waits until a head's completion counter reaches target.  The counted items
// ran on this XCD, whose L2 holds what they wrote, and this workgroup has not
// read those lines before: no cache maintenance is needed.
__device__ __forceinline__ void wait_count(const uint32_t* cnt, uint32_t target, uint32_t* err) {
  if (threadIdx.x == 0) poll_at_least(cnt, target, err);
  __syncthreads();
}

// Every thread waits until its stores have reached the XCD's L2, then thread
// 0 counts the item done.
__device__ __forceinline__ void signal_done(uint32_t* cnt) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The kernel's arguments re-read from the kernarg segment for each item:
// the item kinds' fields are not kept live (in SGPRs) across the item loop.
typedef __attribute__((address_space(4))) const DecodeArgs KernelArgs;
__device__ __forceinline__ const DecodeArgs* item_args() {
  KernelArgs* p = (KernelArgs*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return (const DecodeArgs*)p;
}

// Two workgroups per CU (<= 256 registers per lane): every phase fits in
// registers without spilling.
//
// Work distribution.  Every XCD has its own queue; its workgroups draw queue
// tickets, and a queue takes whole KV heads from a device-wide head counter,
// so all items of a head run on one XCD and hand data to each other through
// that XCD's L2.  A head is K consecutive tickets of its queue (its suffix
// item, its score items, its decide+attend items, its merge items, in that
// order); the workgroup that draws the first ticket of a head's slot claims
// the head and publishes it in the slot (tagged with the launch's epoch, so
// slots need no reset).  An item waits only for items with smaller tickets of
// its own queue (the slot's first ticket, or its head's earlier phase), so the
// smallest unfinished ticket of every queue is held by a running workgroup:
// the grid drains whatever the residency.  The last workgroup out resets the
// tickets and counters and advances the epoch.
template <int D, int GBM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(DecodeArgs a) {
  extern __shared__ unsigned char decode_dyn[];
  __shared__ uint32_t s_ticket, s_head, s_tag, s_last;
  uint32_t* ctl = a.control;
  uint32_t* err = ctl + kCtlError;
  uint32_t* score_done = ctl + kCtlCounters;
  uint32_t* attend_done = score_done + kMaxHeads;
  const uint32_t q = xcc_id();
  uint32_t* queue = ctl + kCtlQueues + 4 * q;  // [0] claim, [1] ready, [2] ticket
  uint64_t* slots = reinterpret_cast<uint64_t*>(ctl + kCtlSlots) + (int64_t)q * kMaxHeads;
  const uint32_t T = (uint32_t)a.score.n_tiles;
  const uint32_t merge_per_head = (uint32_t)a.merge.group * (uint32_t)a.merge_cols;
  // per head: the suffix item (no dependency: first, so it overlaps the
  // scores), T score items, T decide+attend items, the merge items
  const uint32_t e_suffix = 1, e_score = 1 + T, e_attend = 1 + 2 * T;
  const uint32_t K = e_attend + merge_per_head;  // tickets per head
  const int tid = threadIdx.x;

  if (tid == 0) {
    // this launch's slot tag, and a first ticket (queue tickets start at 0:
    // the previous launch's last workgroup reset them)
    s_tag = load_dev(ctl + kCtlEpoch) + 1;
    s_ticket = __hip_atomic_fetch_add(queue + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const uint32_t tag = s_tag;
  uint32_t ticket = s_ticket;
  for (;;) {
    const uint32_t slot = ticket / K, i = ticket % K;
    if (tid == 0) {
      uint32_t h = 0xFFFFFFFFu;
      if (slot < (uint32_t)kMaxHeads) {
        uint64_t* entry = slots + slot;
        if (i == 0) {
          // claim the next head for this queue (or none left) and publish it
          h = __hip_atomic_fetch_add(ctl + kCtlHeadTicket, 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
          if (h < (uint32_t)a.heads) {
            __hip_atomic_store(score_done + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(attend_done + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_s_waitcnt(0);
          } else {
            h = 0xFFFFFFFFu;
          }
          __hip_atomic_store(entry, ((uint64_t)tag << 32) | h, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
        } else {
          uint64_t v = 0;
          for (uint32_t spins = 0;; ++spins) {
            v = __hip_atomic_load(entry, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((uint32_t)(v >> 32) == tag) break;
            if (spins > kSpinLimit) {
              __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
              v = 0xFFFFFFFFull;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
          }
          h = (uint32_t)v;
        }
      }
      s_head = h;
    }
    __syncthreads();
    const uint32_t h = s_head;
    if (h >= (uint32_t)a.heads) break;
    // claim the next ticket now; it is larger than this one
    uint32_t next = 0;
    if (tid == 0)
      next = __hip_atomic_fetch_add(queue + 2, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (i < e_suffix) {
      const AttendArgs aa = item_args()->attend;
      suffix_item<D, GBM>(aa, h);
      signal_done(attend_done + h);
    } else if (i < e_score) {
      const ScoreArgs sa = item_args()->score;
      score_tile<D, true>(sa, h, i - e_suffix, decode_dyn);
      signal_done(score_done + h);
    } else if (i < e_attend) {
      wait_count(score_done + h, T, err);
      const AttendArgs aa = item_args()->attend;
      decide_attend_tile<D, GBM>(aa, h, i - e_score, decode_dyn);
      signal_done(attend_done + h);
    } else {
      const uint32_t r = i - e_attend;
      wait_count(attend_done + h, T + 1, err);
      const MergeArgs ma = item_args()->merge;
      merge_item(ma, h, (int)(r / a.merge_cols), (int)(r % a.merge_cols));
    }
    __syncthreads();
    if (tid == 0) s_ticket = next;
    __syncthreads();
    ticket = s_ticket;
  }

  // The last workgroup out resets the head ticket, the exit count and every
  // queue's ticket, and advances the epoch (every other workgroup has made its
  // last access to them; slots stay, tagged with the old epoch).
  if (tid == 0) {
    const uint32_t out =
        __hip_atomic_fetch_add(ctl + kCtlExits, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = out == gridDim.x - 1 ? 1u : 0u;
  }
  __syncthreads();
  if (s_last) {
    if (tid < kMaxQueues)
      __hip_atomic_store(ctl + kCtlQueues + 4 * tid + 2, 0u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
      __hip_atomic_store(ctl + kCtlHeadTicket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_store(ctl + kCtlExits, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __hip_atomic_fetch_add(ctl + kCtlEpoch, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
struct SelectParams {
  const void* query;
  const void* key_mean;
  const void* ellipsoid;
  const void* value_mean;  // non-null: also build representative partials
  const float* value_norm;
  const float* max_value_norm;
  int64_t heads, group, dim, n_blocks, block, length;
  float eps;
  int reduction;
  const uint8_t* anchor;
  uint8_t* mask;
  float* risk_out;
  float* stats_out;
  unsigned long long* accessed;
  void* ws;
  size_t ws_bytes;
  hipStream_t stream;
};

int validate_select(const SelectParams& p, const char* who, Layout& L) {
  if (!p.query || !p.key_mean || !p.ellipsoid || !p.value_norm || !p.max_value_norm || !p.mask)
    return set_error(kInvalidArgument, "%s: null pointer argument", who);
  if (p.heads <= 0 || p.heads > 65535 || p.group <= 0 || p.n_blocks <= 0 || p.length <= 0)
    return set_error(kInvalidArgument, "%s: empty or oversized shape", who);
  if (p.group > kMaxGroup)
    return set_error(kUnsupported, "%s: GQA group %lld exceeds %d", who, (long long)p.group,
                     kMaxGroup);
  if (!supported_dim(p.dim))
    return set_error(kUnsupported, "%s: head_dim %lld not in 32..256 step 32", who,
                     (long long)p.dim);
  if (!supported_block(p.block))
    return set_error(kInvalidArgument, "%s: block_size must be 16, 32 or 64", who);
  if ((p.length + p.block - 1) / p.block != p.n_blocks)
    return set_error(kInvalidArgument, "%s: n_blocks != ceil(prompt_length / block_size)", who);
  if (p.reduction < 0 || p.reduction > 2)
    return set_error(kInvalidArgument, "%s: reduction code %d", who, p.reduction);
  if (!aligned(p.query, 16) || !aligned(p.key_mean, 16) || !aligned(p.ellipsoid, 16) ||
      (p.value_mean && !aligned(p.value_mean, 16)))
    return set_error(kInvalidArgument, "%s: query/summary must be 16-byte aligned", who);
  L = make_layout(p.heads, p.group, p.dim, p.n_blocks);
  if (!p.ws || p.ws_bytes < (size_t)L.total || !aligned(p.ws, 256))
    return set_error(kWorkspaceTooSmall, "%s: workspace needs %lld bytes, 256-byte aligned", who,
                     (long long)L.total);
  if (L.n_tiles > 0x7FFFFFFF) return set_error(kInvalidArgument, "%s: too many blocks", who);
  if (score_smem(p.group, p.dim, true) > 64 * 1024)
    return set_error(kUnsupported, "%s: group x head_dim too large", who);
  return kOk;
}

ScoreArgs score_args(const SelectParams& p, const Layout& L) {
  ScoreArgs sa;
  sa.query = static_cast<const uint16_t*>(p.query);
  sa.key_mean = static_cast<const uint16_t*>(p.key_mean);
  sa.ellipsoid = static_cast<const uint16_t*>(p.ellipsoid);
  sa.value_mean = static_cast<const uint16_t*>(p.value_mean);
  sa.z = at<float>(p.ws, L.z);
  sa.delta = at<float>(p.ws, L.delta);
  sa.lse = at<float>(p.ws, L.lse);
  sa.rep_acc = at<float>(p.ws, L.rep_acc);
  sa.n_blocks = p.n_blocks;
  sa.n_tiles = L.n_tiles;
  sa.z_stride = L.z_stride;
  sa.tile_stride = L.tile_stride;
  sa.block = p.block;
  sa.length = p.length;
  sa.group = (int)p.group;
  sa.scale = (float)pow((double)p.dim, -0.5);
  return sa;
}

DecideArgs decide_args(const SelectParams& p, const Layout& L) {
  DecideArgs da;
  da.z = at<float>(p.ws, L.z);
  da.delta = at<float>(p.ws, L.delta);
  da.lse = at<float>(p.ws, L.lse);
  da.value_norm = p.value_norm;
  da.max_value_norm = p.max_value_norm;
  da.value_mean = static_cast<const uint16_t*>(p.value_mean);
  da.anchor = p.anchor;
  da.mask = p.mask;
  da.tilebits = at<uint64_t>(p.ws, L.tilebits);
  da.risk_out = p.risk_out;
  da.stats_out = p.stats_out;
  da.accessed = p.accessed;
  da.rep_acc = at<float>(p.ws, L.rep_acc);
  da.n_blocks = p.n_blocks;
  da.n_tiles = L.n_tiles;
  da.z_stride = L.z_stride;
  da.tile_stride = L.tile_stride;
  da.block = p.block;
  da.length = p.length;
  da.group = (int)p.group;
  da.reduction = p.reduction;
  da.dim = (int)p.dim;
  da.eps = p.eps;
  return da;
}

// Selection only (rkv_select): score and decide as two kernels.
int launch_select(const SelectParams& p, const Layout& L) {
  const ScoreArgs sa = score_args(p, L);
  const DecideArgs da = decide_args(p, L);
  const size_t smem = score_smem(p.group, p.dim, false);
  dim3 grid((unsigned)L.n_tiles, (unsigned)p.heads);
  mark(0, p.stream);
  RKV_DISPATCH_DIM(p.dim, D,
                   score_kernel<D, false><<<grid, dim3(kThreads), smem, p.stream>>>(sa));
  int rc = check_launch("score_kernel");
  if (rc) return rc;
  mark(1, p.stream);
  decide_kernel<<<grid, dim3(kThreads), 0, p.stream>>>(da);
  rc = check_launch("decide_kernel");
  mark(2, p.stream);
  return rc;
}

// Grid of the persistent kernel: as many workgroups as the device holds at
// once (more would only wait for a slot), never more than there are items.
struct GridCache {
  const void* fn;
  int device;
  size_t dyn;
  int per_cu, cus;
  size_t static_lds, private_bytes;
};

constexpr int kNotEligible = -1;  // internal: use the split pipeline

// Launches the persistent kernel, or returns kNotEligible when this build of
// it does not meet the persistent kernel's resource rules (LDS per
// workgroup, no private memory traffic): its workgroups wait on each other,
// so each must run with everything it needs from its first instruction.
template <int D, int GBM>
int launch_decode(const DecodeArgs& da, size_t dyn, uint32_t items, hipStream_t stream) {
  const void* fn = reinterpret_cast<const void*>(&decode_kernel<D, GBM>);
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess)
    return set_error(kLaunchFailed, "rkv_decode: no current device");
  thread_local GridCache cache[16] = {};
  thread_local int cache_next = 0;
  GridCache* hit = nullptr;
  for (GridCache& e : cache)
    if (e.fn == fn && e.device == device && e.dyn == dyn) hit = &e;
  if (!hit) {
    GridCache e{fn, device, dyn, 0, 0, 0, 0};
    hipFuncAttributes attr;
    if (hipFuncGetAttributes(&attr, fn) != hipSuccess ||
        hipDeviceGetAttribute(&e.cus, hipDeviceAttributeMultiprocessorCount, device) !=
            hipSuccess)
      return set_error(kLaunchFailed, "rkv_decode: cannot query the device");
    e.static_lds = attr.sharedSizeBytes;
    e.private_bytes = attr.localSizeBytes;
    if (e.static_lds + dyn <= kMaxFusedLds &&
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&e.per_cu, decode_kernel<D, GBM>, kThreads,
                                                     dyn) != hipSuccess)
      return set_error(kLaunchFailed, "rkv_decode: occupancy query failed");
    hit = &cache[cache_next];
    cache_next = (cache_next + 1) % 16;
    *hit = e;
  }
  if (hit->static_lds + dyn > kMaxFusedLds || hit->private_bytes > kMaxFusedPrivate ||
      hit->per_cu < 1)
    return kNotEligible;
  const int64_t slots = (int64_t)hit->per_cu * hit->cus;
  const unsigned grid = (unsigned)(slots < (int64_t)items ? slots : (int64_t)items);
  decode_kernel<D, GBM><<<dim3(grid), dim3(kThreads), dyn, stream>>>(da);
  return check_launch("decode_kernel");
}

template <int D>
int launch_decode_rows(const DecodeArgs& da, int64_t rows_per_block, size_t dyn, uint32_t items,
                       hipStream_t stream) {
  if constexpr (D > kMaxFusedDim) {
    return kNotEligible;
  } else {
    constexpr int CH = D / 16;
    constexpr int CAP = (64 / CH) >= 16 ? 16 : ((64 / CH) >= 8 ? 8 : 4);
    switch (rows_per_block) {
      case 4:
        return launch_decode<D, 4>(da, dyn, items, stream);
      case 8:
        if constexpr (CAP >= 8) return launch_decode<D, 8>(da, dyn, items, stream);
        break;
      default:
        if constexpr (CAP >= 16) return launch_decode<D, 16>(da, dyn, items, stream);
        break;
    }
    return kNotEligible;
  }
}

struct DecodeBuffers {
  const void* key_pages;
  int64_t kp_hs;
  const void* value_pages;
  int64_t vp_hs;
  const void* key_suffix;
  int64_t ks_hs, ks_ts;
  const void* value_suffix;
  int64_t vs_hs, vs_ts;
  int64_t suffix_cap;
  const int32_t* suffix_len;
  void* output;
};

AttendArgs attend_args(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  AttendArgs aa;
  aa.decide = decide_args(p, L);
  aa.query = static_cast<const uint16_t*>(p.query);
  aa.key_pages = static_cast<const uint16_t*>(b.key_pages);
  aa.value_pages = static_cast<const uint16_t*>(b.value_pages);
  aa.key_suffix = static_cast<const uint16_t*>(b.key_suffix);
  aa.value_suffix = static_cast<const uint16_t*>(b.value_suffix);
  aa.suffix_len_dev = b.suffix_len;
  aa.part_m = at<float>(p.ws, L.part_m);
  aa.part_l = at<float>(p.ws, L.part_l);
  aa.part_acc = at<float>(p.ws, L.part_acc);
  aa.kp_hs = b.kp_hs;
  aa.vp_hs = b.vp_hs;
  aa.ks_hs = b.ks_hs;
  aa.ks_ts = b.ks_ts;
  aa.vs_hs = b.vs_hs;
  aa.vs_ts = b.vs_ts;
  aa.suffix_cap = b.suffix_cap;
  aa.part_stride = L.part_stride;
  aa.row_blocks = (int)L.row_blocks;
  aa.scale = (float)pow((double)p.dim, -0.5);
  return aa;
}

MergeArgs merge_args(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  MergeArgs ma;
  ma.part_m = at<float>(p.ws, L.part_m);
  ma.part_l = at<float>(p.ws, L.part_l);
  ma.part_acc = at<float>(p.ws, L.part_acc);
  ma.out = static_cast<uint16_t*>(b.output);
  ma.part_stride = L.part_stride;
  ma.group = (int)p.group;
  ma.parts = (int)(L.n_tiles + 1);
  ma.dim = (int)p.dim;
  return ma;
}

// The split pipeline: score kernel, then decide+attend (and the suffix), then
// merge.
int launch_split(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  const ScoreArgs sa = score_args(p, L);
  const AttendArgs aa = attend_args(p, L, b);
  const MergeArgs ma = merge_args(p, L, b);
  const dim3 score_grid((unsigned)L.n_tiles, (unsigned)p.heads);
  const dim3 attend_grid((unsigned)(L.n_tiles + 1), (unsigned)p.heads);
  const size_t attend_lds = attend_smem(p.group, p.dim);
  mark(0, p.stream);
  RKV_DISPATCH_DIM(p.dim, D,
                   score_kernel<D, true><<<score_grid, dim3(kThreads),
                                           score_smem(p.group, p.dim, true), p.stream>>>(sa));
  int rc = check_launch("score_kernel");
  if (rc) return rc;
  mark(1, p.stream);
  rc = kUnsupported;
  RKV_DISPATCH_DIM(p.dim, D, {
    constexpr int CH = D / 16;
    constexpr int CAP = (64 / CH) >= 16 ? 16 : ((64 / CH) >= 8 ? 8 : 4);
    switch (L.rows_per_block) {
      case 4:
        attend_kernel<D, 4><<<attend_grid, dim3(kThreads), attend_lds, p.stream>>>(aa);
        rc = check_launch("attend_kernel");
        break;
      case 8:
        if constexpr (CAP >= 8) {
          attend_kernel<D, 8><<<attend_grid, dim3(kThreads), attend_lds, p.stream>>>(aa);
          rc = check_launch("attend_kernel");
        }
        break;
      default:
        if constexpr (CAP >= 16) {
          attend_kernel<D, 16><<<attend_grid, dim3(kThreads), attend_lds, p.stream>>>(aa);
          rc = check_launch("attend_kernel");
        }
        break;
    }
  });
  if (rc) return rc;
  mark(2, p.stream);
  merge_kernel<<<dim3((unsigned)(p.heads * p.group), (unsigned)((p.dim + kMergeD - 1) / kMergeD)),
                 dim3(kThreads), 0, p.stream>>>(ma);
  rc = check_launch("merge_kernel");
  mark(3, p.stream);
  return rc;
}

// The persistent kernel, or kNotEligible.
int launch_fused(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  if (p.dim > kMaxFusedDim || p.heads > kMaxHeads) return kNotEligible;
  DecodeArgs da;
  da.score = score_args(p, L);
  da.attend = attend_args(p, L, b);
  da.merge = merge_args(p, L, b);
  da.control = at<uint32_t>(p.ws, L.control);
  da.heads = (int)p.heads;
  da.merge_cols = (int)((p.dim + kMergeD - 1) / kMergeD);
  const uint32_t items =
      (uint32_t)(p.heads * (2 * L.n_tiles + 1 + p.group * da.merge_cols));
  const int64_t dyn_score = (int64_t)score_smem(p.group, p.dim, true);
  const int64_t dyn_attend = (int64_t)attend_smem(p.group, p.dim);
  const size_t dyn = (size_t)(dyn_score > dyn_attend ? dyn_score : dyn_attend);
  int rc = kNotEligible;
  RKV_DISPATCH_DIM(p.dim, D, rc = launch_decode_rows<D>(da, L.rows_per_block, dyn, items, p.stream));
  return rc;
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" size_t rkv_workspace_bytes(int64_t heads, int64_t group, int64_t dim,
                                      int64_t n_blocks) {
  if (heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0) return 0;
  return (size_t)make_layout(heads, group, dim, n_blocks).total;
}

// Byte offsets of the workspace regions, for tests: control, z, delta, lse,
// tilebits, rep_acc, part_m, part_l, part_acc, total, then n_tiles, the row
// stride of z / delta, of the per-tile arrays and of the partials.
extern "C" int rkv_workspace_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                                    int64_t* out14) {
  clear_error();
  if (!out14 || heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_workspace_layout: bad arguments");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  const int64_t v[14] = {L.control, L.z,        L.delta,    L.lse,         L.tilebits,
                         L.rep_acc, L.part_m,   L.part_l,   L.part_acc,    L.total,
                         L.n_tiles, L.z_stride, L.tile_stride, L.part_stride};
  for (int i = 0; i < 14; ++i) out14[i] = v[i];
  return kOk;
}

extern "C" int rkv_select(const void* query, const void* key_mean, const void* ellipsoid,
                          const float* value_norm, const float* max_value_norm, int64_t heads,
                          int64_t group, int64_t dim, int64_t n_blocks, int64_t block_size,
                          int64_t prompt_length, float eps, int reduction,
                          const uint8_t* anchor_mask, uint8_t* mask_out, float* risk_out,
                          float* stats_out, unsigned long long* accessed_blocks, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
  clear_error();
  SelectParams p{query, key_mean, ellipsoid, nullptr, value_norm, max_value_norm, heads, group,
                 dim, n_blocks, block_size, prompt_length, eps, reduction, anchor_mask, mask_out,
                 risk_out, stats_out, accessed_blocks, workspace, workspace_bytes, stream};
  Layout L;
  int rc = validate_select(p, "rkv_select", L);
  if (rc) return rc;
  return launch_select(p, L);
}

extern "C" int rkv_decode(const void* query, const void* key_mean, const void* ellipsoid,
                          const void* value_mean, const float* value_norm,
                          const float* max_value_norm, const void* key_pages,
                          int64_t key_page_head_stride, const void* value_pages,
                          int64_t value_page_head_stride, const void* key_suffix,
                          int64_t key_suffix_head_stride, int64_t key_suffix_token_stride,
                          const void* value_suffix, int64_t value_suffix_head_stride,
                          int64_t value_suffix_token_stride, int64_t suffix_capacity,
                          const int32_t* suffix_length, int64_t heads, int64_t group,
                          int64_t dim, int64_t n_blocks, int64_t block_size,
                          int64_t prompt_length, float eps, int reduction,
                          const uint8_t* anchor_mask, uint8_t* mask_out, void* output,
                          unsigned long long* accessed_blocks, void* workspace,
                          size_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (!value_mean) return set_error(kInvalidArgument, "rkv_decode: null value_mean");
  SelectParams p{query, key_mean, ellipsoid, value_mean, value_norm, max_value_norm, heads,
                 group, dim, n_blocks, block_size, prompt_length, eps, reduction, anchor_mask,
                 mask_out, nullptr, nullptr, accessed_blocks, workspace, workspace_bytes, stream};
  Layout L;
  int rc = validate_select(p, "rkv_decode", L);
  if (rc) return rc;
  if (!key_pages || !value_pages || !output)
    return set_error(kInvalidArgument, "rkv_decode: null pointer argument");
  if (suffix_capacity < 0)
    return set_error(kInvalidArgument, "rkv_decode: negative suffix capacity");
  if (suffix_capacity > 0 && (!key_suffix || !value_suffix))
    return set_error(kInvalidArgument, "rkv_decode: null suffix with nonzero capacity");
  const int64_t es = 2;
  const int64_t ch_bytes = dim / 16 * es;
  const uintptr_t need = ch_bytes % 16 == 0 ? 16 : (ch_bytes % 8 == 0 ? 8 : 4);
  if (!aligned(key_pages, need) || !aligned(value_pages, need) ||
      (key_page_head_stride * es) % need || (value_page_head_stride * es) % need)
    return set_error(kInvalidArgument, "rkv_decode: pages must be %d-byte aligned", (int)need);
  if (suffix_capacity > 0 &&
      (!aligned(key_suffix, need) || !aligned(value_suffix, need) ||
       (key_suffix_head_stride * es) % need || (key_suffix_token_stride * es) % need ||
       (value_suffix_head_stride * es) % need || (value_suffix_token_stride * es) % need))
    return set_error(kInvalidArgument, "rkv_decode: suffix rows must be %d-byte aligned",
                     (int)need);
  if (!aligned(output, 4)) return set_error(kInvalidArgument, "rkv_decode: output alignment");

  const DecodeBuffers b{key_pages,     key_page_head_stride,   value_pages,
                        value_page_head_stride,  key_suffix,   key_suffix_head_stride,
                        key_suffix_token_stride, value_suffix, value_suffix_head_stride,
                        value_suffix_token_stride, suffix_capacity, suffix_length, output};
  if (g_pipeline == 1 || g_pipeline == 3) {
    mark(0, stream);
    rc = launch_fused(p, L, b);
    if (rc != kNotEligible) {
      if (rc == kOk) mark(1, stream);
      return rc;
    }
    if (g_pipeline == 1)
      return set_error(kUnsupported, "rkv_decode: the persistent kernel does not run this shape");
  }
  return launch_split(p, L, b);
}

// Profiling hook: when events is non-null, the following rkv_select /
// rkv_decode calls on this thread record events[0] before their first kernel
// and events[k] after their k-th (rkv_select: score, decide; rkv_decode: the
// persistent kernel, or score, decide, pages, merge on the split pipeline).
// Pass NULL to stop.
extern "C" int rkv_set_profile_events(void* events) {
  g_events = static_cast<hipEvent_t*>(events);
  return kOk;
}

// Test and benchmark hook: 0 automatic (the split pipeline), 1 persistent
// kernel (RKV_UNSUPPORTED where it cannot run), 2 split pipeline, 3 the
// persistent kernel where it runs, else the split pipeline.  Per thread.
extern "C" int rkv_set_decode_pipeline(int mode) {
  clear_error();
  if (mode < 0 || mode > 3) return set_error(kInvalidArgument, "rkv_set_decode_pipeline: mode");
  g_pipeline = mode;
  return kOk;
}
