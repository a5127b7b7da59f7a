// Decode-step selection and mixed attention (src/refinekv/reference.py:10-73,
// the semantics the reference's Triton kernels in src/refinekv/kernels/ also
// follow).  No host sync, no allocation: the caller passes a workspace.
//
// rkv_decode runs ONE persistent kernel per step.  Its workgroups take work
// items from a ticket counter in the order below; an item waits only for
// items with smaller tickets (per-head completion counters), so the earliest
// unfinished item always belongs to a running workgroup and the grid drains
// whatever the residency.  Per KV head h:
//
//   score  (h, tile)   one 64-block tile: streams the tile's key means,
//                      ellipsoids and value means once; s = q.k_mean and the
//                      ellipsoid projection for every query row, z = s + ln n,
//                      delta, the tile's log-sum-exp partials of z and
//                      z + log cosh delta, and the representative accumulator
//                      sum_b exp(z_b - m_tile) v_mean_b over all its blocks
//                      (the z partial is that attention's (m, l)).
//   decide (h, tile)   after every score item of h: log Z / log C of each
//                      row from the tile partials, the risk, the GQA
//                      reduction, the non-finite fail-safes and the anchor
//                      union; the mask, a 64-bit ballot per tile and the
//                      access counter; then the tile's representative
//                      partial without its expanded blocks (l recomputed over
//                      the unexpanded blocks, acc minus the expanded blocks'
//                      terms: rounding error below fp32 eps times the tile's
//                      representative mass).
//   pages  (h, rows, k) after every decide item of h: the head's expanded
//                      pages and suffix tokens split into equal-cost ranges (a
//                      page costs 2 * block_size, a suffix token 2); item k
//                      also absorbs the representative partials of a 1/P
//                      share of the head's tiles.  Exact softmax over 64-row
//                      chunks with one shared max per chunk.
//   merge  (h, g, cols) after every page item of h: the P partials of row g
//                      -> bf16 output columns.
//
// The last workgroup to leave returns the counters to zero, so a workspace
// that was zero-filled once stays ready for the next call.  It runs on
// request (rkv_set_decode_pipeline) where its resource rules hold (head_dim
// <= 128, LDS per workgroup <= 64 KiB, no private-memory traffic): on a
// multi-XCD device every cross-workgroup hand-off pays a device-scope L2
// write-back and a same-address ticket atomic, which makes it slower than
// kernel boundaries for this workload today.
//
// The default is the split pipeline: the score and decide phases as two
// kernels, then a page kernel over global equal-cost ranges of every head's
// expanded pages and a merge kernel.  rkv_select runs the score and decide
// kernels only.
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
constexpr int64_t kMaxTiles = 2048;    // tiles per head in the decode kernel (LDS page index)
constexpr int64_t kMaxHeads = 1024;    // KV heads in the persistent kernel (control block)
constexpr int64_t kMaxPageItems = 64;  // page items per (head, row block)
constexpr int64_t kMaxHeadTiles = 8192;  // split page kernel: heads * tiles in LDS
constexpr int64_t kMaxFusedDim = 128;    // widest head_dim the persistent kernel runs
constexpr size_t kMaxFusedLds = 64 * 1024;  // its LDS per workgroup (static + dynamic)
constexpr size_t kMaxFusedPrivate = 64;     // its private bytes per lane (no spill traffic)
// Control block of the persistent kernel (uint32 words; see decode_kernel).
constexpr int kMaxQueues = 16;               // one work queue per XCD (XCC_ID is 4 bits)
constexpr int64_t kCtlHeadTicket = 0, kCtlExits = 1, kCtlError = 2, kCtlEpoch = 3;
constexpr int64_t kCtlQueues = 16;           // per queue: claim, ready, ticket, -
constexpr int64_t kCtlSlots = kCtlQueues + 4 * kMaxQueues;  // per queue: kMaxHeads u64 slots
constexpr int64_t kCtlCounters = kCtlSlots + 2 * kMaxQueues * kMaxHeads;  // 3 x kMaxHeads
constexpr int64_t kControlWords = kCtlCounters + 3 * kMaxHeads;
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
  int64_t n_tiles, page_items, workers, rows_per_block, row_blocks;
  // Padded row strides: every head's slice of an intermediate array covers
  // whole 256-byte lines, so no cache line holds two heads' data.
  int64_t z_stride, tile_stride, part_stride;
  int64_t control, z, delta, lse, tilebits, rep_l, rep_acc, header, page_m, page_l, page_acc,
      total;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

// Rows of the GQA group one page item carries in registers: the next power
// of two >= group (at least 4), capped so that rows * head_dim / 16
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

// Split pipeline: one page worker per 64 (head, block) pairs, 1..512.
inline int64_t workers_for(int64_t heads, int64_t n_blocks) {
  int64_t w = (heads * n_blocks + 63) / 64;
  if (w < 1) w = 1;
  if (w > 512) w = 512;
  return w;
}

// Page items per (head, row block): about 512 in all, at most one per tile
// and at most kMaxPageItems.
inline int64_t page_items_for(int64_t heads, int64_t row_blocks, int64_t n_tiles) {
  int64_t p = (512 + heads * row_blocks - 1) / (heads * row_blocks);
  if (p > n_tiles) p = n_tiles;
  if (p > kMaxPageItems) p = kMaxPageItems;
  return p < 1 ? 1 : p;
}

Layout make_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks) {
  Layout L{};
  L.n_tiles = (n_blocks + kTile - 1) / kTile;
  L.rows_per_block = rows_per_block(group, dim);
  L.row_blocks = (group + L.rows_per_block - 1) / L.rows_per_block;
  L.page_items = page_items_for(heads, L.row_blocks, L.n_tiles);
  L.workers = workers_for(heads, n_blocks);
  const int64_t rows = heads * group;
  // page partials: (rows, page_items) for the persistent kernel, (rows,
  // workers) for the split pipeline
  auto round64 = [](int64_t x) { return (x + 63) / 64 * 64; };
  L.z_stride = L.n_tiles * kTile;
  L.tile_stride = round64(L.n_tiles);
  L.part_stride = round64(L.page_items);
  const int64_t slots = L.part_stride > L.workers ? L.part_stride : L.workers;
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
  L.rep_l = take(rows * L.tile_stride * 4);
  L.rep_acc = take(rows * L.tile_stride * dim * 4);
  L.header = take((heads + 1) * 8);
  L.page_m = take(rows * slots * 4);
  L.page_l = take(rows * slots * 4);
  L.page_acc = take(rows * slots * dim * 4);
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
  float* rep_l;                 // (H, G, tiles) or null (select only)
  float* rep_acc;               // (H, G, tiles, D)
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

__device__ __forceinline__ void decide_tile(const DecideArgs& a, int64_t h, int64_t tile) {
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
    tile_m[gi] = (a.rep_l && g < G) ? a.lse[((h * G + g) * a.tile_stride + tile) * 4] : 0.0f;
  }
  constexpr int kAccPerThread = kMaxGroup * 256 / kThreads;  // G * D <= 16 * 256
  float racc[kAccPerThread];
  const int GD = G * a.dim;
#pragma unroll
  for (int k = 0; k < kAccPerThread; ++k) {
    const int idx = tid + k * kThreads;
    racc[k] = 0.0f;
    if (a.rep_l && idx < GD) {
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
  if (!a.rep_l) return;
  __syncthreads();

  // ---- representatives of this tile: drop the expanded blocks ----------
  // (thread tid's prefetched z/delta pair k is row wave + 4k, block lane)
  const uint64_t bits = sel_bits;
  const int nsel = __popcll(bits);
#pragma unroll
  for (int gi = 0; gi < kMaxGroup / kWaves; ++gi) {
    const int g = wave + gi * kWaves;
    if (g >= G) break;
    const bool valid = lane < nvalid;
    const bool expanded = (bits >> lane) & 1ull;
    const float e = valid ? expf_(rz[gi] - inf_to_zero(tile_m[gi])) : 0.0f;
    const float l = wave_sum_u(expanded ? 0.0f : e);
    psel[g][lane] = expanded ? e : 0.0f;
    if (lane == 0) a.rep_l[(h * G + g) * a.tile_stride + tile] = nsel == nvalid ? 0.0f : l;
  }
  if (nsel == 0 || nsel == nvalid) return;
  __syncthreads();
  const int D = a.dim;
#pragma unroll
  for (int k = 0; k < kAccPerThread; ++k) {
    const int idx = tid + k * kThreads;
    if (idx >= GD) break;
    const int g = idx / D, d = idx % D;
    float acc = racc[k];
    uint64_t m = bits;
    while (m) {
      const int j = __builtin_ctzll(m);
      m &= m - 1;
      const float v = bf16_to_f32(a.value_mean[(h * N + tile * kTile + j) * D + d]);
      acc = acc - psel[g][j] * v;
    }
    a.rep_acc[((h * G + g) * a.tile_stride + tile) * D + d] = acc;
  }
}

template <int D, bool REPS>
__global__ __launch_bounds__(kThreads) void score_kernel(ScoreArgs a) {
  extern __shared__ unsigned char score_dyn[];
  score_tile<D, REPS>(a, blockIdx.y, blockIdx.x, score_dyn);
}

__global__ __launch_bounds__(kThreads) void decide_kernel(DecideArgs a) {
  decide_tile(a, blockIdx.y, blockIdx.x);
}

// ---------------------------------------------------------------------------
// Phase 3: expanded pages, suffix tokens and representative partials
// ---------------------------------------------------------------------------
struct PageArgs {
  const uint16_t* query;       // (H, G, D) bf16
  const uint16_t* key_pages;   // head h at key_pages + h * kp_hs; rows (N*B, D)
  const uint16_t* value_pages;
  const uint16_t* key_suffix;  // token t of head h at h * ks_hs + t * ks_ts
  const uint16_t* value_suffix;
  const uint64_t* tilebits;    // (H, tiles)
  const int32_t* suffix_len_dev;  // or null
  const float* lse;            // (H, G, tiles, 4): representative m = inf_to_zero(zm)
  const float* rep_l;          // (H, G, tiles)
  const float* rep_acc;        // (H, G, tiles, D)
  float* page_m;               // (H, G, P)
  float* page_l;
  float* page_acc;             // (H, G, P, D)
  int64_t kp_hs, vp_hs, ks_hs, ks_ts, vs_hs, vs_ts;
  int64_t suffix_cap, n_blocks, n_tiles, block, length;
  int64_t tile_stride;         // row stride of the per-tile arrays
  int64_t part_stride;         // row stride of the page partials (items padded to 64)
  int group, page_items;
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

// LDS of a page item: the head's tile ballots, their prefix and a page list.
inline int64_t page_smem(int64_t n_tiles) {
  return align256(n_tiles * 8) + align256((n_tiles + 1) * 4) + 8 * 8;
}

template <int D, int GBM>
__device__ __forceinline__ void page_item(const PageArgs& a, int64_t h, int rb, int k,
                                          unsigned char* dyn) {
  constexpr int CH = D / 16;
  const int64_t T = a.n_tiles;
  uint64_t* bits_s = reinterpret_cast<uint64_t*>(dyn);                    // [T]
  uint32_t* pre = reinterpret_cast<uint32_t*>(dyn + align256(T * 8));     // [T + 1]
  int64_t* list = reinterpret_cast<int64_t*>(dyn + align256(T * 8) + align256((T + 1) * 4));
  __shared__ uint32_t wave_tot[kWaves];
  __shared__ float xlog[GBM][kChunkRows];
  __shared__ float cmax[GBM], csum[GBM];
  __shared__ float xacc[kWaves][GBM][D];

  const int G = a.group, P = a.page_items;
  const int g0 = rb * GBM;
  const int gn = min(GBM, G - g0);
  const int tid = item_tid(), lg = tid >> 4, c = tid & 15, wave = tid / kWave;
  const int lane = tid % kWave, grp = lane >> 4;
  const int64_t N = a.n_blocks, B = a.block;

  // ---- the head's expanded pages: ballots and their prefix --------------
  const int64_t per = (T + kThreads - 1) / kThreads;
  const int64_t t_begin = min((int64_t)tid * per, T), t_end = min(t_begin + per, T);
  uint32_t mine = 0;
  for (int64_t t = t_begin; t < t_end; ++t) {
    const uint64_t b = a.tilebits[h * a.tile_stride + t];
    bits_s[t] = b;
    mine += (uint32_t)__popcll(b);
  }
  uint32_t n_h;
  uint32_t run = block_exclusive_scan(mine, wave_tot, n_h);
  for (int64_t t = t_begin; t < t_end; ++t) {
    pre[t] = run;
    run += (uint32_t)__popcll(bits_s[t]);
  }
  if (tid == 0) pre[T] = n_h;

  // ---- this item's equal-cost range of pages and suffix tokens ----------
  int64_t S = a.suffix_cap;
  if (a.suffix_len_dev) {
    const int64_t s = *a.suffix_len_dev;
    S = s < 0 ? 0 : (s > a.suffix_cap ? a.suffix_cap : s);
  }
  const int64_t pc = 2 * B;  // cost of one page; a suffix token costs 2
  const int64_t C = pc * (int64_t)n_h + 2 * S;
  const int64_t lo = C * k / P, hi = C * (k + 1) / P;
  auto clampi = [](int64_t x, int64_t l, int64_t u) { return x < l ? l : (x > u ? u : x); };
  auto ceil_div = [](int64_t x, int64_t d) { return x <= 0 ? 0 : (x + d - 1) / d; };
  const int64_t p0 = clampi(ceil_div(lo, pc), 0, n_h), p1 = clampi(ceil_div(hi, pc), 0, n_h);
  const int64_t s0 = clampi(ceil_div(lo - pc * n_h, 2), 0, S);
  const int64_t s1 = clampi(ceil_div(hi - pc * n_h, 2), 0, S);
  const int64_t n_prow = (p1 - p0) * B, n_rows = n_prow + (s1 - s0);

  float q[GBM][CH];
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    const int gg = g < gn ? g : 0;
    RawBf16<CH> r = load_raw<CH>(a.query + ((h * G + g0 + gg) * D + c * CH));
    unpack(r, q[g]);
  }

  // ---- start from the representative partials of tiles [r0, r1) ---------
  // (m, l, acc) of each live tile, rescaled to their common max; lane group 0
  // holds the accumulator, the other groups start at zero.
  const int64_t r0 = T * k / P, r1 = T * (k + 1) / P;
  float m_run[GBM], l_run[GBM], acc[GBM][CH];
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    m_run[g] = kNegInf;
    l_run[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < CH; ++i) acc[g][i] = 0.0f;
    if (g >= gn) continue;
    const int64_t row = h * G + g0 + g;
    float mr = kNegInf;
    for (int64_t t = r0; t < r1; ++t) {
      const float lt = a.rep_l[row * a.tile_stride + t];
      const float mt = inf_to_zero(a.lse[(row * a.tile_stride + t) * 4]);
      if (lt > 0.0f) mr = fmaxf(mr, mt);
    }
    if (mr == kNegInf) continue;
    float l = 0.0f;
    for (int64_t t = r0; t < r1; ++t) {
      const float lt = a.rep_l[row * a.tile_stride + t];
      const float mt = inf_to_zero(a.lse[(row * a.tile_stride + t) * 4]);
      float at[CH];
      load_f32<CH>(a.rep_acc + (row * a.tile_stride + t) * D + c * CH, at);
      if (lt > 0.0f) {
        const float e = __builtin_amdgcn_exp2f((mt - mr) * kLog2e);
        l = l + lt * e;
        if (lg == 0) {
#pragma unroll
          for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] + at[i] * e;
        }
      }
    }
    m_run[g] = mr;
    l_run[g] = l;
  }

  // Rows in chunks of 64: pass 1 loads K/V and writes the chunk's logits,
  // pass 2 weighs the V rows with one shared max (no per-row rescaling).
  for (int64_t c0 = 0; c0 < n_rows; c0 += kChunkRows) {
    // pages touched by this chunk -> block indices (block_size divides 64)
    const int64_t j_first = c0 < n_prow ? p0 + c0 / B : p1;
    const int64_t j_last = min(c0 + kChunkRows, n_prow) - 1;
    const int64_t n_pages = c0 < n_prow ? p0 + j_last / B - j_first + 1 : 0;
    __syncthreads();
    if (tid < n_pages) {
      const int64_t j = j_first + tid;
      int64_t lo_t = 0, hi_t = T - 1;
      while (lo_t < hi_t) {
        const int64_t mid = (lo_t + hi_t + 1) >> 1;
        if ((int64_t)pre[mid] <= j) lo_t = mid; else hi_t = mid - 1;
      }
      list[tid] = lo_t * kTile + nth_set_bit(bits_s[lo_t], (int)(j - pre[lo_t]));
    }
    __syncthreads();
    RawBf16<CH> kr[kRowBatch], vr[kRowBatch];
    bool ok[kRowBatch];
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      const int64_t v = c0 + lg + 16 * u;
      const uint16_t* kp = a.key_pages + h * a.kp_hs;  // a valid row for idle lanes
      const uint16_t* vp = a.value_pages + h * a.vp_hs;
      ok[u] = false;
      if (v < n_prow) {
        const int64_t jj = v / B, t = v - jj * B;
        const int64_t b = list[p0 + jj - j_first];
        if (t < block_count(b, N, B, a.length)) {
          ok[u] = true;
          kp += (b * B + t) * D;
          vp += (b * B + t) * D;
        }
      } else if (v < n_rows) {
        const int64_t kk = s0 + (v - n_prow);
        ok[u] = true;
        kp = a.key_suffix + h * a.ks_hs + kk * a.ks_ts;
        vp = a.value_suffix + h * a.vs_hs + kk * a.vs_ts;
      }
      kr[u] = load_raw<CH>(kp + c * CH);
      vr[u] = load_raw<CH>(vp + c * CH);
    }
#pragma unroll
    for (int u = 0; u < kRowBatch; ++u) {
      float kv[CH], x[GBM];
      unpack(kr[u], kv);
      row_logits<D, GBM>(q, kv, x);
      if (c == 15) {
#pragma unroll
        for (int g = 0; g < GBM; ++g) xlog[g][lg + 16 * u] = ok[u] ? x[g] * a.scale : kNegInf;
      }
    }
    __syncthreads();
    // chunk max and sum per query row, one wave per row
    for (int g = wave; g < gn; g += kWaves) {
      const float x = xlog[g][lane];
      const float cm = wave_nanmax_u(x);
      const float ms = cm == kNegInf ? 0.0f : cm;
      const float sum = wave_sum_u(__builtin_amdgcn_exp2f((x - ms) * kLog2e));
      if (lane == 0) {
        cmax[g] = cm;
        csum[g] = sum;
      }
    }
    __syncthreads();
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g >= gn) break;
      const float cm = cmax[g];
      const float mn = fmaxf(m_run[g], cm);
      if (mn == kNegInf) continue;
      const float sa = __builtin_amdgcn_exp2f((m_run[g] - mn) * kLog2e);
      const float sb = __builtin_amdgcn_exp2f((cm - mn) * kLog2e);
      l_run[g] = l_run[g] * sa + csum[g] * sb;
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
        const float p = __builtin_amdgcn_exp2f((xlog[g][lg + 16 * u] - ms) * kLog2e);
#pragma unroll
        for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] + p * v[i];
      }
    }
  }

  // sum the 16 lane groups (one shared max: plain adds) and write
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
    const int64_t slot = (h * G + g0 + g) * a.part_stride + k;
    const float sum = ((xacc[0][g][d] + xacc[1][g][d]) + xacc[2][g][d]) + xacc[3][g][d];
    a.page_acc[slot * D + d] = sum;
    if (d == 0) {
      a.page_m[slot] = m_run[g];
      a.page_l[slot] = l_run[g];
    }
  }
}

// ---------------------------------------------------------------------------
// Phase 4: merge a row's page-item partials -> bf16 output columns
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float* page_m;    // (H, G, P)
  const float* page_l;
  const float* page_acc;  // (H, G, P, D)
  uint16_t* out;          // (H*G, D)
  int64_t part_stride;    // row stride of the page partials
  int group, page_items, dim;
};

constexpr int kMergeD = 32;                   // output columns per item
constexpr int kMergeK = kThreads / kMergeD;   // partial stripes
constexpr int kMergeBatch = 8;                // partials per stripe per batch

__device__ __forceinline__ void merge_item(const MergeArgs& a, int64_t h, int g, int dc) {
  __shared__ float red[kWaves];
  __shared__ float num_s[kMergeK][kMergeD];
  __shared__ float den_s[kMergeK];
  const int P = a.page_items, D = a.dim;
  const int64_t r = h * a.group + g;
  const int tid = item_tid(), lane = tid % kWave, wave = tid / kWave;

  float mx = kNegInf;
  for (int i = tid; i < P; i += kThreads) {
    const float l = a.page_l[r * a.part_stride + i];
    const float m = a.page_m[r * a.part_stride + i];
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
      mv[u] = a.page_m[r * a.part_stride + ii];
      lv[u] = a.page_l[r * a.part_stride + ii];
      av[u] = a.page_acc[(r * a.part_stride + ii) * D + dd];
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

// ---------------------------------------------------------------------------
// Split pipeline, kernel 3: expanded pages and suffix tokens
// ---------------------------------------------------------------------------
struct SplitPageArgs {
  const uint16_t* query;       // (H, G, D) bf16
  const uint16_t* key_pages;   // head h at key_pages + h * kp_hs; rows (N*B, D)
  const uint16_t* value_pages;
  const uint16_t* key_suffix;  // token t of head h at h * ks_hs + t * ks_ts
  const uint16_t* value_suffix;
  const uint64_t* tilebits;    // (H, tiles)
  const int32_t* suffix_len_dev;  // or null
  int64_t* header;             // (H + 1): cost start of each head's work, [H] = total
  float* page_m;               // (H*G, W), written only by workers touching the head
  float* page_l;
  float* page_acc;             // (H*G, W, D)
  int64_t kp_hs, vp_hs, ks_hs, ks_ts, vs_hs, vs_ts;
  int64_t suffix_cap, n_blocks, n_tiles, block, length;
  int64_t tile_stride;         // head stride of tilebits (tiles padded to 64)
  int heads, group, workers, rows_per_block;
  float scale;
};

// Ballot of dense (head, tile) index ht (ht = h * tiles + t).
__device__ __forceinline__ uint64_t head_tile_bits(const SplitPageArgs& a, int64_t ht) {
  const int64_t h = ht / a.n_tiles;
  return a.tilebits[h * a.tile_stride + (ht - h * a.n_tiles)];
}

inline size_t split_page_smem(int64_t heads, int64_t n_tiles) {
  return (size_t)(align256((heads * n_tiles + 1) * 4) + align256((heads + 1) * 8) +
                  sizeof(int64_t) * 8);
}

template <int D, int GBM>
__global__ __launch_bounds__(kThreads) void split_page_kernel(SplitPageArgs a) {
  constexpr int CH = D / 16;
  extern __shared__ unsigned char smem_raw[];
  const int64_t T = a.n_tiles, H = a.heads, HT = H * T;
  uint32_t* pre = reinterpret_cast<uint32_t*>(smem_raw);  // [HT + 1] page prefix, head-major
  int64_t* hs = reinterpret_cast<int64_t*>(smem_raw + align256((HT + 1) * 4));  // [H + 1]
  int64_t* list = hs + align256((H + 1) * 8) / 8;                               // [8]
  __shared__ uint32_t wave_tot[kWaves];
  __shared__ float xlog[GBM][kChunkRows];
  __shared__ float cmax[GBM], csum[GBM];
  __shared__ float xacc[kWaves][GBM][D];

  const int w = blockIdx.x;
  const int g0 = blockIdx.y * a.rows_per_block;
  const int gn = min(a.rows_per_block, a.group - g0);
  const int G = a.group;
  const int tid = item_tid(), lg = tid >> 4, c = tid & 15, wave = tid / kWave;
  const int lane = tid % kWave, grp = lane >> 4;
  const int64_t N = a.n_blocks, B = a.block;

  // ---- expanded-page prefix over every (head, tile) ----------------------
  const int64_t per = (HT + kThreads - 1) / kThreads;
  const int64_t t_begin = min((int64_t)tid * per, HT), t_end = min(t_begin + per, HT);
  uint32_t mine = 0;
  for (int64_t t = t_begin; t < t_end; ++t) mine += (uint32_t)__popcll(head_tile_bits(a, t));
  uint32_t total;
  uint32_t run = block_exclusive_scan(mine, wave_tot, total);
  for (int64_t t = t_begin; t < t_end; ++t) {
    pre[t] = run;
    run += (uint32_t)__popcll(head_tile_bits(a, t));
  }
  if (tid == 0) pre[HT] = total;
  __syncthreads();

  int64_t S = a.suffix_cap;
  if (a.suffix_len_dev) {
    const int64_t s = *a.suffix_len_dev;
    S = s < 0 ? 0 : (s > a.suffix_cap ? a.suffix_cap : s);
  }
  const int64_t pc = 2 * B;  // cost of one page; a suffix token costs 2
  for (int64_t h = tid; h <= H; h += kThreads) hs[h] = pc * (int64_t)pre[h * T] + 2 * S * h;
  __syncthreads();
  const int64_t C = hs[H];
  if (w == 0 && blockIdx.y == 0)
    for (int64_t h = tid; h <= H; h += kThreads) a.header[h] = hs[h];
  const int64_t lo = C * w / a.workers, hi = C * (w + 1) / a.workers;
  auto clampi = [](int64_t x, int64_t l, int64_t u) { return x < l ? l : (x > u ? u : x); };
  auto ceil_div = [](int64_t x, int64_t d) { return x <= 0 ? 0 : (x + d - 1) / d; };

  // first head whose range may hold lo: the largest h with hs[h] <= lo
  int64_t hb = 0, ht = H - 1;
  while (hb < ht) {
    const int64_t mid = (hb + ht + 1) >> 1;
    if (hs[mid] <= lo) hb = mid; else ht = mid - 1;
  }
  for (int64_t h = hb; h < H && hs[h] < hi; ++h) {
    const int64_t hs_h = hs[h], he_h = hs[h + 1];
    if (!(lo < he_h && hi > hs_h)) continue;
    const int64_t first = pre[h * T];
    const int64_t n_h = (int64_t)pre[(h + 1) * T] - first;
    const int64_t lo_h = lo - hs_h, hi_h = hi - hs_h;
    const int64_t p0 = clampi(ceil_div(lo_h, pc), 0, n_h), p1 = clampi(ceil_div(hi_h, pc), 0, n_h);
    const int64_t s0 = clampi(ceil_div(lo_h - pc * n_h, 2), 0, S);
    const int64_t s1 = clampi(ceil_div(hi_h - pc * n_h, 2), 0, S);
    const int64_t n_prow = (p1 - p0) * B, n_rows = n_prow + (s1 - s0);

    float q[GBM][CH];
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      const int gg = g < gn ? g : 0;
      RawBf16<CH> r = load_raw<CH>(a.query + ((h * G + g0 + gg) * D + c * CH));
      unpack(r, q[g]);
    }
    float m_run[GBM], l_run[GBM], acc[GBM][CH];
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      m_run[g] = kNegInf;
      l_run[g] = 0.0f;
#pragma unroll
      for (int i = 0; i < CH; ++i) acc[g][i] = 0.0f;
    }

    // Rows in chunks of 64: pass 1 loads K/V and writes the chunk's logits,
    // pass 2 weighs the V rows with one shared max (no per-row rescaling).
    for (int64_t c0 = 0; c0 < n_rows; c0 += kChunkRows) {
      // pages touched by this chunk -> block indices
      const int64_t j_first = c0 < n_prow ? p0 + c0 / B : p1;
      const int64_t j_last = min(c0 + kChunkRows, n_prow) - 1;
      const int64_t n_pages = c0 < n_prow ? p0 + j_last / B - j_first + 1 : 0;
      __syncthreads();
      if (tid < n_pages) {
        const int64_t j = first + j_first + tid;
        int64_t lo_t = h * T, hi_t = h * T + T - 1;
        while (lo_t < hi_t) {
          const int64_t mid = (lo_t + hi_t + 1) >> 1;
          if ((int64_t)pre[mid] <= j) lo_t = mid; else hi_t = mid - 1;
        }
        list[tid] = (lo_t - h * T) * kTile +
                    nth_set_bit(head_tile_bits(a, lo_t), (int)(j - pre[lo_t]));
      }
      __syncthreads();
      RawBf16<CH> kr[kRowBatch], vr[kRowBatch];
      bool ok[kRowBatch];
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        const int64_t v = c0 + lg + 16 * u;
        const uint16_t* kp = a.key_pages + h * a.kp_hs;  // a valid row for idle lanes
        const uint16_t* vp = a.value_pages + h * a.vp_hs;
        ok[u] = false;
        if (v < n_prow) {
          const int64_t jj = v / B, t = v - jj * B;
          const int64_t b = list[p0 + jj - j_first];
          if (t < block_count(b, N, B, a.length)) {
            ok[u] = true;
            kp += (b * B + t) * D;
            vp += (b * B + t) * D;
          }
        } else if (v < n_rows) {
          const int64_t k = s0 + (v - n_prow);
          ok[u] = true;
          kp = a.key_suffix + h * a.ks_hs + k * a.ks_ts;
          vp = a.value_suffix + h * a.vs_hs + k * a.vs_ts;
        }
        kr[u] = load_raw<CH>(kp + c * CH);
        vr[u] = load_raw<CH>(vp + c * CH);
      }
#pragma unroll
      for (int u = 0; u < kRowBatch; ++u) {
        float kv[CH], x[GBM];
        unpack(kr[u], kv);
        row_logits<D, GBM>(q, kv, x);
        if (c == 15) {
#pragma unroll
          for (int g = 0; g < GBM; ++g) xlog[g][lg + 16 * u] = ok[u] ? x[g] * a.scale : kNegInf;
        }
      }
      __syncthreads();
      // chunk max and sum per query row, one wave per row
      for (int g = wave; g < gn; g += kWaves) {
        const float x = xlog[g][lane];
        const float cm = wave_nanmax_u(x);
        const float ms = cm == kNegInf ? 0.0f : cm;
        const float sum = wave_sum_u(__builtin_amdgcn_exp2f((x - ms) * kLog2e));
        if (lane == 0) {
          cmax[g] = cm;
          csum[g] = sum;
        }
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < GBM; ++g) {
        if (g >= gn) break;
        const float cm = cmax[g];
        const float mn = fmaxf(m_run[g], cm);
        if (mn == kNegInf) continue;
        const float sa = __builtin_amdgcn_exp2f((m_run[g] - mn) * kLog2e);
        const float sb = __builtin_amdgcn_exp2f((cm - mn) * kLog2e);
        l_run[g] = l_run[g] * sa + csum[g] * sb;
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
          const float p = __builtin_amdgcn_exp2f((xlog[g][lg + 16 * u] - ms) * kLog2e);
#pragma unroll
          for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] + p * v[i];
        }
      }
    }

    // sum the 16 lane groups (one shared max: plain adds) and write
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
      const int64_t slot = (h * G + g0 + g) * a.workers + w;
      const float sum = ((xacc[0][g][d] + xacc[1][g][d]) + xacc[2][g][d]) + xacc[3][g][d];
      a.page_acc[slot * D + d] = sum;
      if (d == 0) {
        a.page_m[slot] = m_run[g];
        a.page_l[slot] = l_run[g];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Split pipeline, kernel 4: merge representative and page partials -> bf16 output
// ---------------------------------------------------------------------------
struct SplitMergeArgs {
  const float* lse;       // rep m = inf_to_zero(zm)
  const float* rep_l;
  const float* rep_acc;
  const int64_t* header;  // page-work cost starts per head (page kernel)
  const float* page_m;
  const float* page_l;
  const float* page_acc;
  uint16_t* out;          // (H*G, D)
  int64_t n_tiles;
  int64_t tile_stride;    // row stride of the per-tile arrays
  int heads, group, workers, dim;
};


inline size_t split_merge_smem(int64_t n_tiles, int64_t workers) {
  const int64_t P = n_tiles + workers;
  return sizeof(float) * 2 * P + sizeof(int) * P;
}

__global__ __launch_bounds__(kThreads) void split_merge_kernel(SplitMergeArgs a) {
  extern __shared__ unsigned char smem_raw[];
  const int64_t T = a.n_tiles, W = a.workers;
  float* pm = reinterpret_cast<float*>(smem_raw);  // [P] partial max (natural log)
  float* pl = pm + (T + W);                         // [P] partial l (0 if dead)
  int* live = reinterpret_cast<int*>(pl + (T + W)); // [P] live partial indices, in order
  __shared__ uint32_t wave_tot[kWaves];
  __shared__ float red[kWaves];
  __shared__ float num_s[kMergeK][kMergeD];
  __shared__ float den_s[kMergeK];
  const int64_t r = blockIdx.x;
  const int64_t h = r / a.group;
  const int d0 = blockIdx.y * kMergeD;
  const int tid = item_tid(), lane = tid % kWave, wave = tid / kWave;
  const int D = a.dim;

  // workers whose cost range meets head h's (the page kernel's own test):
  // w_first = ceil(W (hs+1) / C) - 1, w_last = ceil(W he / C) - 1
  const int64_t hs = a.header[h], he = a.header[h + 1], C = a.header[a.heads];
  int64_t w_first = 0, w_last = -1;
  if (C > 0 && he > hs) {
    w_first = (W * (hs + 1) + C - 1) / C - 1;
    w_last = (W * he + C - 1) / C - 1;
    if (w_first < 0) w_first = 0;
    if (w_last > W - 1) w_last = W - 1;
  }
  const int64_t P = T + (w_last - w_first + 1);

  float mx = kNegInf;
  for (int64_t i = tid; i < P; i += kThreads) {
    float m, l;
    if (i < T) {
      m = inf_to_zero(a.lse[(r * a.tile_stride + i) * 4]);
      l = a.rep_l[r * a.tile_stride + i];
    } else {
      const int64_t w = w_first + (i - T);
      m = a.page_m[r * W + w];
      l = a.page_l[r * W + w];
    }
    const bool alive = l > 0.0f;
    pm[i] = m;
    pl[i] = alive ? l : 0.0f;
    if (alive) mx = fmaxf(mx, m);
  }
  mx = wave_nanmax_u(mx);
  if (lane == 0) red[wave] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float Ms = M == kNegInf ? 0.0f : M;

  // live list in index order (chunked block scans)
  int64_t n_live = 0;
  for (int64_t base = 0; base < P; base += kThreads) {
    const int64_t i = base + tid;
    const bool alive = i < P && pl[i] > 0.0f;
    uint32_t tot;
    const uint32_t pos = block_exclusive_scan(alive ? 1u : 0u, wave_tot, tot);
    if (alive) live[n_live + pos] = (int)i;
    n_live += tot;
  }
  __syncthreads();

  const int dl = tid % kMergeD, k = tid / kMergeD;
  const int d = d0 + dl;
  const int dd = d < D ? d : 0;
  float num = 0.0f, den = 0.0f;
  constexpr int kBatch = 8;
  for (int64_t q0 = k; q0 < n_live; q0 += kMergeK * kBatch) {
    int idx[kBatch];
    float accv[kBatch];
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      const int64_t q = q0 + (int64_t)u * kMergeK;
      idx[u] = q < n_live ? live[q] : -1;
      const int64_t i = idx[u] < 0 ? 0 : idx[u];
      accv[u] = i < T ? a.rep_acc[(r * a.tile_stride + i) * D + dd]
                      : a.page_acc[(r * W + w_first + (i - T)) * D + dd];
    }
#pragma unroll
    for (int u = 0; u < kBatch; ++u) {
      if (idx[u] < 0) break;
      const float e = __builtin_amdgcn_exp2f((pm[idx[u]] - Ms) * kLog2e);
      den = den + pl[idx[u]] * e;
      num = num + accv[u] * e;
    }
  }
  num_s[k][dl] = num;
  if (dl == 0) den_s[k] = den;
  __syncthreads();
  if (tid < kMergeD && d < D) {
    float n = num_s[0][tid], den_all = den_s[0];
    for (int kk = 1; kk < kMergeK; ++kk) {
      n = n + num_s[kk][tid];
      den_all = den_all + den_s[kk];
    }
    a.out[r * D + d] = bf16_rne(n / fmaxf(den_all, 1e-30f));
  }
}


// ---------------------------------------------------------------------------
// The persistent decode kernel
// ---------------------------------------------------------------------------
struct DecodeArgs {
  ScoreArgs score;
  DecideArgs decide;
  PageArgs page;
  MergeArgs merge;
  uint32_t* control;  // kControlWords words, zero when the workspace is new
  int heads, row_blocks, merge_cols;
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
// that XCD's L2.  A head is K consecutive tickets of its queue (its score,
// decide, page and merge items, in that order); the workgroup that draws the
// first ticket of a head's slot claims the head and publishes it in the slot
// (epoch-tagged, so slots need no reset).  An item waits only for items with
// smaller tickets of its own queue (the slot's first ticket, or its head's
// earlier phases), so the smallest unfinished ticket of every queue is held
// by a running workgroup: the grid drains whatever the residency.  Queue
// state is reset by the queue's first workgroup of each launch (epoch), the
// device-wide counters by the last workgroup out.
template <int D, int GBM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void decode_kernel(DecodeArgs a) {
  extern __shared__ unsigned char decode_dyn[];
  __shared__ uint32_t s_ticket, s_head, s_tag, s_last;
  uint32_t* ctl = a.control;
  uint32_t* err = ctl + kCtlError;
  uint32_t* score_done = ctl + kCtlCounters;
  uint32_t* decide_done = score_done + kMaxHeads;
  uint32_t* page_done = decide_done + kMaxHeads;
  const uint32_t q = xcc_id();
  uint32_t* queue = ctl + kCtlQueues + 4 * q;  // [0] claim, [1] ready, [2] ticket
  uint64_t* slots = reinterpret_cast<uint64_t*>(ctl + kCtlSlots) + (int64_t)q * kMaxHeads;
  const uint32_t T = (uint32_t)a.score.n_tiles;
  const uint32_t P = (uint32_t)a.page.page_items;
  const uint32_t page_per_head = (uint32_t)a.row_blocks * P;
  const uint32_t merge_per_head = (uint32_t)a.merge.group * (uint32_t)a.merge_cols;
  const uint32_t e_score = T, e_decide = 2 * T, e_page = e_decide + page_per_head;
  const uint32_t K = e_page + merge_per_head;  // tickets per head
  const int tid = threadIdx.x;

  if (tid == 0) {
    // this launch's tag; the queue's first workgroup of the launch resets it
    const uint32_t tag = load_dev(ctl + kCtlEpoch) + 1;
    if (__hip_atomic_fetch_max(queue, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < tag) {
      __hip_atomic_store(queue + 2, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      __builtin_amdgcn_s_waitcnt(0);
      __hip_atomic_store(queue + 1, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
      poll_at_least(queue + 1, tag, err);
    }
    s_tag = tag;
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
            __hip_atomic_store(decide_done + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(page_done + h, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
    if (i < e_score) {
      const ScoreArgs sa = item_args()->score;
      score_tile<D, true>(sa, h, i, decode_dyn);
      signal_done(score_done + h);
    } else if (i < e_decide) {
      wait_count(score_done + h, T, err);
      const DecideArgs da = item_args()->decide;
      decide_tile(da, h, i - e_score);
      signal_done(decide_done + h);
    } else if (i < e_page) {
      const uint32_t r = i - e_decide;
      wait_count(decide_done + h, T, err);
      const PageArgs pa = item_args()->page;
      page_item<D, GBM>(pa, h, (int)(r / P), (int)(r % P), decode_dyn);
      signal_done(page_done + h);
    } else {
      const uint32_t r = i - e_page;
      wait_count(page_done + h, page_per_head, err);
      const MergeArgs ma = item_args()->merge;
      merge_item(ma, h, (int)(r / a.merge_cols), (int)(r % a.merge_cols));
    }
    __syncthreads();
    if (tid == 0) s_ticket = next;
    __syncthreads();
    ticket = s_ticket;
  }

  // The last workgroup out resets the device-wide counters and advances the
  // epoch (every other workgroup has made its last access to them).
  if (tid == 0) {
    const uint32_t out =
        __hip_atomic_fetch_add(ctl + kCtlExits, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (out == gridDim.x - 1) {
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
  const bool reps = p.value_mean != nullptr;
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
  da.rep_l = reps ? at<float>(p.ws, L.rep_l) : nullptr;
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

template <int D>
int launch_split_pages(const SplitPageArgs& pa, const Layout& L, hipStream_t stream) {
  const size_t smem = split_page_smem(pa.heads, L.n_tiles);
  dim3 grid((unsigned)L.workers, (unsigned)L.row_blocks);
  constexpr int CH = D / 16;
  constexpr int CAP = (64 / CH) >= 16 ? 16 : ((64 / CH) >= 8 ? 8 : 4);
  switch (L.rows_per_block) {
    case 4:
      split_page_kernel<D, 4><<<grid, dim3(kThreads), smem, stream>>>(pa);
      break;
    case 8:
      if constexpr (CAP >= 8) split_page_kernel<D, 8><<<grid, dim3(kThreads), smem, stream>>>(pa);
      break;
    default:
      if constexpr (CAP >= 16)
        split_page_kernel<D, 16><<<grid, dim3(kThreads), smem, stream>>>(pa);
      break;
  }
  return check_launch("split_page_kernel");
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

// The split pipeline: score and decide kernels, then the page kernel (global
// equal-cost ranges over every head's expanded pages) and the merge kernel.
int launch_split(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  const ScoreArgs sa = score_args(p, L);
  const DecideArgs da = decide_args(p, L);
  dim3 grid((unsigned)L.n_tiles, (unsigned)p.heads);
  mark(0, p.stream);
  RKV_DISPATCH_DIM(p.dim, D,
                   score_kernel<D, true><<<grid, dim3(kThreads), score_smem(p.group, p.dim, true),
                                           p.stream>>>(sa));
  int rc = check_launch("score_kernel");
  if (rc) return rc;
  mark(1, p.stream);
  decide_kernel<<<grid, dim3(kThreads), 0, p.stream>>>(da);
  rc = check_launch("decide_kernel");
  if (rc) return rc;
  mark(2, p.stream);

  SplitPageArgs pa;
  pa.query = static_cast<const uint16_t*>(p.query);
  pa.key_pages = static_cast<const uint16_t*>(b.key_pages);
  pa.value_pages = static_cast<const uint16_t*>(b.value_pages);
  pa.key_suffix = static_cast<const uint16_t*>(b.key_suffix);
  pa.value_suffix = static_cast<const uint16_t*>(b.value_suffix);
  pa.tilebits = at<uint64_t>(p.ws, L.tilebits);
  pa.suffix_len_dev = b.suffix_len;
  pa.header = at<int64_t>(p.ws, L.header);
  pa.page_m = at<float>(p.ws, L.page_m);
  pa.page_l = at<float>(p.ws, L.page_l);
  pa.page_acc = at<float>(p.ws, L.page_acc);
  pa.kp_hs = b.kp_hs;
  pa.vp_hs = b.vp_hs;
  pa.ks_hs = b.ks_hs;
  pa.ks_ts = b.ks_ts;
  pa.vs_hs = b.vs_hs;
  pa.vs_ts = b.vs_ts;
  pa.suffix_cap = b.suffix_cap;
  pa.n_blocks = p.n_blocks;
  pa.n_tiles = L.n_tiles;
  pa.tile_stride = L.tile_stride;
  pa.block = p.block;
  pa.length = p.length;
  pa.heads = (int)p.heads;
  pa.group = (int)p.group;
  pa.workers = (int)L.workers;
  pa.rows_per_block = (int)L.rows_per_block;
  pa.scale = (float)pow((double)p.dim, -0.5);
  rc = kOk;
  RKV_DISPATCH_DIM(p.dim, D, rc = launch_split_pages<D>(pa, L, p.stream));
  if (rc) return rc;
  mark(3, p.stream);

  SplitMergeArgs ma;
  ma.lse = at<float>(p.ws, L.lse);
  ma.rep_l = at<float>(p.ws, L.rep_l);
  ma.rep_acc = at<float>(p.ws, L.rep_acc);
  ma.header = pa.header;
  ma.page_m = pa.page_m;
  ma.page_l = pa.page_l;
  ma.page_acc = pa.page_acc;
  ma.out = static_cast<uint16_t*>(b.output);
  ma.n_tiles = L.n_tiles;
  ma.tile_stride = L.tile_stride;
  ma.heads = (int)p.heads;
  ma.group = (int)p.group;
  ma.workers = (int)L.workers;
  ma.dim = (int)p.dim;
  split_merge_kernel<<<dim3((unsigned)(p.heads * p.group), (unsigned)((p.dim + kMergeD - 1) / kMergeD)),
                       dim3(kThreads), split_merge_smem(L.n_tiles, L.workers), p.stream>>>(ma);
  rc = check_launch("split_merge_kernel");
  mark(4, p.stream);
  return rc;
}

// The persistent kernel, or kNotEligible.
int launch_fused(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  if (p.dim > kMaxFusedDim || p.heads > kMaxHeads || L.n_tiles > kMaxTiles) return kNotEligible;
  DecodeArgs da;
  da.score = score_args(p, L);
  da.decide = decide_args(p, L);
  PageArgs& pa = da.page;
  pa.query = static_cast<const uint16_t*>(p.query);
  pa.key_pages = static_cast<const uint16_t*>(b.key_pages);
  pa.value_pages = static_cast<const uint16_t*>(b.value_pages);
  pa.key_suffix = static_cast<const uint16_t*>(b.key_suffix);
  pa.value_suffix = static_cast<const uint16_t*>(b.value_suffix);
  pa.tilebits = at<uint64_t>(p.ws, L.tilebits);
  pa.suffix_len_dev = b.suffix_len;
  pa.lse = at<float>(p.ws, L.lse);
  pa.rep_l = at<float>(p.ws, L.rep_l);
  pa.rep_acc = at<float>(p.ws, L.rep_acc);
  pa.page_m = at<float>(p.ws, L.page_m);
  pa.page_l = at<float>(p.ws, L.page_l);
  pa.page_acc = at<float>(p.ws, L.page_acc);
  pa.kp_hs = b.kp_hs;
  pa.vp_hs = b.vp_hs;
  pa.ks_hs = b.ks_hs;
  pa.ks_ts = b.ks_ts;
  pa.vs_hs = b.vs_hs;
  pa.vs_ts = b.vs_ts;
  pa.suffix_cap = b.suffix_cap;
  pa.n_blocks = p.n_blocks;
  pa.n_tiles = L.n_tiles;
  pa.tile_stride = L.tile_stride;
  pa.part_stride = L.part_stride;
  pa.block = p.block;
  pa.length = p.length;
  pa.group = (int)p.group;
  pa.page_items = (int)L.page_items;
  pa.scale = (float)pow((double)p.dim, -0.5);
  MergeArgs& ma = da.merge;
  ma.page_m = pa.page_m;
  ma.page_l = pa.page_l;
  ma.page_acc = pa.page_acc;
  ma.out = static_cast<uint16_t*>(b.output);
  ma.part_stride = L.part_stride;
  ma.group = (int)p.group;
  ma.page_items = (int)L.page_items;
  ma.dim = (int)p.dim;
  da.control = at<uint32_t>(p.ws, L.control);
  da.heads = (int)p.heads;
  da.row_blocks = (int)L.row_blocks;
  da.merge_cols = (int)((p.dim + kMergeD - 1) / kMergeD);
  const uint32_t items = (uint32_t)(p.heads * (2 * L.n_tiles + L.row_blocks * L.page_items +
                                                p.group * da.merge_cols));
  const int64_t dyn_score = (int64_t)score_smem(p.group, p.dim, true);
  const int64_t dyn_page = page_smem(L.n_tiles);
  const size_t dyn = (size_t)(dyn_score > dyn_page ? dyn_score : dyn_page);
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
// tilebits, rep_l, rep_acc, header, page_m, page_l, page_acc, total, then
// n_tiles, the page items per head and row block (persistent kernel) and the
// page workers (split pipeline).
extern "C" int rkv_workspace_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                                    int64_t* out15) {
  clear_error();
  if (!out15 || heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_workspace_layout: bad arguments");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  const int64_t v[15] = {L.control, L.z,       L.delta,   L.lse,       L.tilebits,
                         L.rep_l,   L.rep_acc, L.header,  L.page_m,    L.page_l,
                         L.page_acc, L.total,  L.n_tiles, L.page_items, L.workers};
  for (int i = 0; i < 15; ++i) out15[i] = v[i];
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
  if (heads * L.n_tiles > kMaxHeadTiles)
    return set_error(kUnsupported, "rkv_decode: heads x tiles %lld exceeds %lld",
                     (long long)(heads * L.n_tiles), (long long)kMaxHeadTiles);
  if (split_merge_smem(L.n_tiles, L.workers) > 64 * 1024)
    return set_error(kUnsupported, "rkv_decode: too many partials");
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
