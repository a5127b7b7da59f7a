// Decode-step selection and mixed attention (src/refinekv/reference.py:10-73,
// the semantics the reference's Triton kernels in src/refinekv/kernels/ also
// follow).  Four kernels per step, all on the caller's stream, no host sync,
// no allocation (the caller passes a workspace):
//
//   score   grid (tiles, H): per 64-block tile, s = q.k_mean and the ellipsoid
//           projection for every query row; z = s + ln(count), delta, and the
//           tile's log-sum-exp partials of z and z + log cosh(delta).
//   decide  grid (tiles, H): merges the tile partials into log Z / log C,
//           evaluates the risk, the GQA reduction, non-finite fail-safes and
//           the anchor union; writes the mask, a 64-bit ballot per tile and
//           the access counter.
//   attend  grid (workers, H, row-blocks): split-K attention.  The head's work
//           (representatives of unexpanded blocks, pages of expanded blocks,
//           suffix tokens) is laid out as one list ordered by cost and cut
//           into equal-cost ranges, so clustered expansions do not serialize
//           on one workgroup.  Online-softmax state per 16-lane group.
//   merge   grid (rows): combines the workers' (m, l, acc) partials.
//
// Scores, radii and log-sum-exp follow the fixed fp32 orders documented in
// rkv_math.h / the oracle header, so masks are reproducible bit for bit.
#include "rkv_common.h"
#include "rkv_internal.h"

namespace rkv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Optional profiling events (rkv_set_profile_events): recorded on the launch
// stream before score and after score, decide, attend and merge.
thread_local hipEvent_t* g_events = nullptr;

inline void mark(int i, hipStream_t stream) {
  if (g_events) (void)hipEventRecord(g_events[i], stream);
}
constexpr float kLog2e = 1.44269504088896341f;

// ---------------------------------------------------------------------------
// Workspace layout
// ---------------------------------------------------------------------------
struct Layout {
  int64_t n_tiles, workers, row_blocks, rows_per_block;
  int64_t z, delta, lse, tilebits, attn_m, attn_l, attn_acc, total;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

inline int64_t rows_per_block(int64_t dim) {
  int64_t ch = dim / 16;
  int64_t r = 64 / ch;
  return r > kMaxGroup ? kMaxGroup : r;
}

inline int64_t workers_for(int64_t n_blocks) {
  int64_t w = (n_blocks + 63) / 64;
  if (w < 1) w = 1;
  if (w > 64) w = 64;
  return w;
}

Layout make_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks) {
  Layout L{};
  L.n_tiles = (n_blocks + kTile - 1) / kTile;
  L.workers = workers_for(n_blocks);
  L.rows_per_block = rows_per_block(dim);
  L.row_blocks = (group + L.rows_per_block - 1) / L.rows_per_block;
  const int64_t rows = heads * group;
  int64_t off = 0;
  L.z = off;
  off = align256(off + rows * n_blocks * 4);
  L.delta = off;
  off = align256(off + rows * n_blocks * 4);
  L.lse = off;
  off = align256(off + rows * L.n_tiles * 4 * 4);
  L.tilebits = off;
  off = align256(off + heads * L.n_tiles * 8);
  L.attn_m = off;
  off = align256(off + rows * L.workers * 4);
  L.attn_l = off;
  off = align256(off + rows * L.workers * 4);
  L.attn_acc = off;
  off = align256(off + rows * L.workers * dim * 4);
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

__device__ __forceinline__ float inf_to_zero(float m) {
  return (m == kPosInf || m == kNegInf) ? 0.0f : m;
}

// Log-sum-exp partial of one 64-block tile; x is lane j's value (-inf pads).
__device__ __forceinline__ void tile_lse(float x, float& m, float& l) {
  m = wave_nanmax(x);
  const float ms = inf_to_zero(m);
  l = wave_sum(expf_(x - ms));
}

// ---------------------------------------------------------------------------
// Kernel 1: scores
// ---------------------------------------------------------------------------
struct ScoreArgs {
  const uint16_t* query;      // (H, G, D) bf16
  const uint16_t* key_mean;   // (H, N, D) bf16
  const uint16_t* ellipsoid;  // (H, N, D) bf16
  float* z;                   // (H, G, N)
  float* delta;               // (H, G, N)
  float* lse;                 // (H, G, tiles, 4): zm, zl, cm, cl
  int64_t n_blocks, n_tiles, block, length;
  int group;
  float scale;
};

template <int D>
__global__ __launch_bounds__(kThreads) void score_kernel(ScoreArgs a) {
  constexpr int CH = D / 16;
  extern __shared__ float smem[];
  const int G = a.group;
  float* qs = smem;                 // [G][D] bf16(q)
  float* q2s = qs + G * D;          // [G][D] bf16(q^2)
  float* sdot = q2s + G * D;        // [G][64]
  float* pdot = sdot + G * kTile;   // [G][64]
  float* zbuf = pdot + G * kTile;   // [G][64]
  float* zcbuf = zbuf + G * kTile;  // [G][64]

  const int64_t h = blockIdx.y;
  const int64_t tile = blockIdx.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int grp = lane / 16, c = lane % 16;
  const int64_t N = a.n_blocks;

  for (int i = tid; i < G * D; i += kThreads) {
    const float q = bf16_to_f32(a.query[h * G * D + i]);
    qs[i] = q;
    q2s[i] = round_bf16(q * q);
  }

  float km[4][CH], el[4][CH];
#pragma unroll
  for (int it = 0; it < 4; ++it) {
    const int64_t b = tile * kTile + wave * 16 + it * 4 + grp;
    if (b < N) {
      load_bf16<CH>(a.key_mean + (h * N + b) * D + c * CH, km[it]);
      load_bf16<CH>(a.ellipsoid + (h * N + b) * D + c * CH, el[it]);
    } else {
#pragma unroll
      for (int i = 0; i < CH; ++i) km[it][i] = el[it][i] = 0.0f;
    }
  }
  __syncthreads();

  for (int g = 0; g < G; ++g) {
    float qv[CH], q2v[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      qv[i] = qs[g * D + c * CH + i];
      q2v[i] = q2s[g * D + c * CH + i];
    }
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      // DSUM: chunk of CH consecutive elements left to right, then butterfly.
      float s = qv[0] * km[it][0];
      float p = q2v[0] * el[it][0];
#pragma unroll
      for (int i = 1; i < CH; ++i) {
        s = s + qv[i] * km[it][i];
        p = p + q2v[i] * el[it][i];
      }
      s = group16_sum(s);
      p = group16_sum(p);
      if (c == 0) {
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
      const float cnt = (float)(b == N - 1 ? a.length - (N - 1) * a.block : a.block);
      z = s + logf_(cnt);
      zc = z + log_cosh(dl);
      const int64_t o = (h * G + g) * N + b;
      a.z[o] = z;
      a.delta[o] = dl;
    }
    zbuf[idx] = z;
    zcbuf[idx] = zc;
  }
  __syncthreads();

  for (int g = wave; g < G; g += kWaves) {
    float zm, zl, cm, cl;
    tile_lse(zbuf[g * kTile + lane], zm, zl);
    tile_lse(zcbuf[g * kTile + lane], cm, cl);
    if (lane == 0) {
      float* o = a.lse + ((h * G + g) * a.n_tiles + tile) * 4;
      o[0] = zm;
      o[1] = zl;
      o[2] = cm;
      o[3] = cl;
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 2: decisions
// ---------------------------------------------------------------------------
struct DecideArgs {
  const float* z;
  const float* delta;
  const float* lse;
  const float* value_norm;      // (H, N)
  const float* max_value_norm;  // (H)
  const uint8_t* anchor;        // (H, N) or null
  uint8_t* mask;                // (H, N)
  uint64_t* tilebits;           // (H, tiles)
  float* risk_out;              // (H, G, N) or null
  float* stats_out;             // (H, G, 2) or null: log Z, log C
  unsigned long long* accessed; // or null
  int64_t n_blocks, n_tiles, block, length;
  int group, reduction;
  float eps;
};

// Merge the tile partials of one row in the fixed order: max first, then
// 64 lane accumulators (tile t -> lane t % 64, left to right) and a butterfly.
__device__ __forceinline__ float merge_lse(const float* part, int64_t n_tiles, int which,
                                           int lane) {
  float m = kNegInf;
  for (int64_t t = lane; t < n_tiles; t += kWave) m = nanmax(m, part[t * 4 + 2 * which]);
  m = wave_nanmax(m);
  const float ms = inf_to_zero(m);
  float acc = 0.0f;
  bool first = true;
  for (int64_t t = lane; t < n_tiles; t += kWave) {
    const float term = part[t * 4 + 2 * which + 1] * expf_(part[t * 4 + 2 * which] - ms);
    acc = first ? term : acc + term;
    first = false;
  }
  const float L = wave_sum(acc);
  return logf_(L) + ms;
}

__global__ __launch_bounds__(kThreads) void decide_kernel(DecideArgs a) {
  __shared__ float gstat[kMaxGroup][2];
  __shared__ float risk_s[kMaxGroup][kTile];
  const int64_t h = blockIdx.y;
  const int64_t tile = blockIdx.x;
  const int tid = threadIdx.x, wave = tid / kWave, lane = tid % kWave;
  const int G = a.group;
  const int64_t N = a.n_blocks;

  for (int g = wave; g < G; g += kWaves) {
    const float* part = a.lse + (h * G + g) * a.n_tiles * 4;
    const float lz = merge_lse(part, a.n_tiles, 0, lane);
    const float lc = merge_lse(part, a.n_tiles, 1, lane);
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

  const float vmax = a.max_value_norm[h];
  for (int idx = tid; idx < G * kTile; idx += kThreads) {
    const int g = idx / kTile, bl = idx % kTile;
    const int64_t b = tile * kTile + bl;
    float r = 0.0f;
    if (b < N) {
      const int64_t o = (h * G + g) * N + b;
      r = risk_of(a.z[o], a.delta[o], gstat[g][0], gstat[g][1], vmax, a.value_norm[h * N + b]);
      if (a.risk_out) a.risk_out[o] = r;
    }
    risk_s[g][bl] = r;
  }
  __syncthreads();

  if (wave == 0) {
    const int64_t b = tile * kTile + lane;
    const bool valid = b < N;
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
    sel = sel || bad_global || bad_local;
    if (valid && a.anchor) sel = sel || a.anchor[h * N + b] != 0;
    sel = sel && valid;
    if (valid) a.mask[h * N + b] = sel ? 1 : 0;
    const uint64_t bits = __ballot(sel);
    if (lane == 0) a.tilebits[h * a.n_tiles + tile] = bits;
    if (a.accessed) {
      const int64_t cnt = b == N - 1 ? a.length - (N - 1) * a.block : a.block;
      unsigned long long term = valid ? (sel ? (unsigned long long)cnt : 1ull) : 0ull;
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) term += __shfl_xor(term, o, kWave);
      if (lane == 0) atomicAdd(a.accessed, term);
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 3: split-K mixed attention
// ---------------------------------------------------------------------------
struct AttendArgs {
  const uint16_t* query;       // (H, G, D) bf16
  const float* z;              // (H, G, N)
  const uint16_t* value_mean;  // (H, N, D)
  const uint16_t* key_pages;   // page h at key_pages + h * kp_hs; (N, B, D) rows
  const uint16_t* value_pages;
  const uint16_t* key_suffix;  // token t of head h at h * ks_hs + t * ks_ts
  const uint16_t* value_suffix;
  const uint64_t* tilebits;    // (H, tiles)
  const int32_t* suffix_len_dev;  // or null
  float* part_m;               // (H*G, W)
  float* part_l;
  float* part_acc;             // (H*G, W, D)
  int64_t kp_hs, vp_hs, ks_hs, ks_ts, vs_hs, vs_ts;
  int64_t suffix_cap, n_blocks, n_tiles, block, length;
  int group, workers, rows_per_block;
  float scale;
};

constexpr int kListCap = kThreads;  // block indices resolved per chunk

// Index -> block lookups over the per-tile ballots (prefix sums in LDS).
struct TileIndex {
  const uint32_t* selpre;    // [tiles + 1] exclusive prefix of expanded blocks
  const uint32_t* unselpre;  // [tiles + 1] exclusive prefix of unexpanded blocks
  const uint64_t* bits;      // [tiles]
  int64_t n_tiles, n_blocks;

  __device__ __forceinline__ int64_t find(const uint32_t* pre, int64_t i) const {
    int64_t lo = 0, hi = n_tiles - 1;
    while (lo < hi) {
      const int64_t mid = (lo + hi + 1) >> 1;
      if ((int64_t)pre[mid] <= i) lo = mid; else hi = mid - 1;
    }
    return lo;
  }
  __device__ __forceinline__ uint64_t valid_bits(int64_t t) const {
    const int64_t n = n_blocks - t * kTile;
    return n >= 64 ? ~0ull : ((1ull << n) - 1ull);
  }
  __device__ __forceinline__ int64_t selected(int64_t j) const {
    const int64_t t = find(selpre, j);
    return t * kTile + nth_set_bit(bits[t], (int)(j - selpre[t]));
  }
  __device__ __forceinline__ int64_t unselected(int64_t i) const {
    const int64_t t = find(unselpre, i);
    return t * kTile + nth_set_bit(~bits[t] & valid_bits(t), (int)(i - unselpre[t]));
  }
};

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

template <int D, int GBM>
struct SoftmaxState {
  static constexpr int CH = D / 16;
  float m[GBM], l[GBM], acc[GBM][CH];

  __device__ __forceinline__ void init() {
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      m[g] = kNegInf;
      l[g] = 0.0f;
#pragma unroll
      for (int i = 0; i < CH; ++i) acc[g][i] = 0.0f;
    }
  }
  // x: logits in log2 units (one per row); v: this lane's slice of the value row.
  __device__ __forceinline__ void update(const float (&x)[GBM], const float (&v)[CH], int gn) {
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g >= gn) break;
      const float mn = fmaxf(m[g], x[g]);
      if (mn == kNegInf) continue;
      const float alpha = __builtin_amdgcn_exp2f(m[g] - mn);
      const float p = __builtin_amdgcn_exp2f(x[g] - mn);
      l[g] = l[g] * alpha + p;
#pragma unroll
      for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] * alpha + p * v[i];
      m[g] = mn;
    }
  }
  // Merge another state (same lane slice) into this one.
  __device__ __forceinline__ void merge(const float* om, const float* ol, const float (*oacc)[CH],
                                        int gn) {
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g >= gn) break;
      const float mn = fmaxf(m[g], om[g]);
      if (mn == kNegInf) continue;
      const float a = __builtin_amdgcn_exp2f(m[g] - mn);
      const float b = __builtin_amdgcn_exp2f(om[g] - mn);
      l[g] = l[g] * a + ol[g] * b;
#pragma unroll
      for (int i = 0; i < CH; ++i) acc[g][i] = acc[g][i] * a + oacc[g][i] * b;
      m[g] = mn;
    }
  }
};

template <int D, int GBM>
__global__ __launch_bounds__(kThreads) void attend_kernel(AttendArgs a) {
  constexpr int CH = D / 16;
  extern __shared__ unsigned char smem_raw[];
  const int64_t T = a.n_tiles;
  uint32_t* selpre = reinterpret_cast<uint32_t*>(smem_raw);
  uint32_t* unselpre = selpre + (T + 1);
  uint64_t* bits = reinterpret_cast<uint64_t*>(smem_raw + align256((T + 1) * 8));
  int64_t* list = reinterpret_cast<int64_t*>(reinterpret_cast<unsigned char*>(bits) +
                                             align256(T * 8));
  __shared__ uint32_t wave_tot[kWaves];
  __shared__ float xm[kWaves][GBM], xl[kWaves][GBM];
  __shared__ float xacc[kWaves][GBM][D];

  const int64_t h = blockIdx.y;
  const int w = blockIdx.x;
  const int g0 = blockIdx.z * a.rows_per_block;
  const int gn = min(a.rows_per_block, a.group - g0);
  const int G = a.group;
  const int tid = threadIdx.x, lg = tid >> 4, c = tid & 15, wave = tid / kWave;
  const int64_t N = a.n_blocks;

  // ---- per-tile prefix sums of expanded / unexpanded blocks -------------
  const int64_t per = (T + kThreads - 1) / kThreads;
  const int64_t t_begin = min((int64_t)tid * per, T), t_end = min(t_begin + per, T);
  uint32_t my_sel = 0, my_valid = 0;
  for (int64_t t = t_begin; t < t_end; ++t) {
    const uint64_t b = a.tilebits[h * T + t];
    bits[t] = b;
    my_sel += (uint32_t)__popcll(b);
    const int64_t nv = N - t * kTile;
    my_valid += (uint32_t)(nv >= 64 ? 64 : nv);
  }
  uint32_t tot_sel, tot_valid;
  const uint32_t ex_sel = block_exclusive_scan(my_sel, wave_tot, tot_sel);
  const uint32_t ex_valid = block_exclusive_scan(my_valid, wave_tot, tot_valid);
  {
    uint32_t s = ex_sel, u = ex_valid - ex_sel;
    for (int64_t t = t_begin; t < t_end; ++t) {
      selpre[t] = s;
      unselpre[t] = u;
      const uint32_t ns = (uint32_t)__popcll(bits[t]);
      const int64_t nv = N - t * kTile;
      s += ns;
      u += (uint32_t)(nv >= 64 ? 64 : nv) - ns;
    }
    if (tid == 0) {
      selpre[T] = tot_sel;
      unselpre[T] = tot_valid - tot_sel;
    }
  }
  __syncthreads();
  const TileIndex index{selpre, unselpre, bits, T, N};

  // ---- this worker's equal-cost share of the head's work ---------------
  const int64_t n_sel = tot_sel, n_unsel = (int64_t)tot_valid - tot_sel;
  int64_t S = a.suffix_cap;
  if (a.suffix_len_dev) {
    const int64_t s = *a.suffix_len_dev;
    S = s < 0 ? 0 : (s > a.suffix_cap ? a.suffix_cap : s);
  }
  const int64_t page_cost = 2 * a.block;
  const int64_t C = n_unsel + page_cost * n_sel + 2 * S;
  const int64_t lo = C * w / a.workers, hi = C * (w + 1) / a.workers;
  auto clampi = [](int64_t x, int64_t lo_, int64_t hi_) { return x < lo_ ? lo_ : (x > hi_ ? hi_ : x); };
  auto ceil_div = [](int64_t x, int64_t d) { return x <= 0 ? 0 : (x + d - 1) / d; };
  const int64_t r0 = clampi(lo, 0, n_unsel), r1 = clampi(hi, 0, n_unsel);
  const int64_t p0 = clampi(ceil_div(lo - n_unsel, page_cost), 0, n_sel);
  const int64_t p1 = clampi(ceil_div(hi - n_unsel, page_cost), 0, n_sel);
  const int64_t sbase = n_unsel + page_cost * n_sel;
  const int64_t s0 = clampi(ceil_div(lo - sbase, 2), 0, S);
  const int64_t s1 = clampi(ceil_div(hi - sbase, 2), 0, S);

  // ---- query slice for this lane ---------------------------------------
  float q[GBM][CH];
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    if (g < gn) {
      load_bf16<CH>(a.query + ((h * G + g0 + g) * D + c * CH), q[g]);
    } else {
#pragma unroll
      for (int i = 0; i < CH; ++i) q[g][i] = 0.0f;
    }
  }
  const float qscale = a.scale * kLog2e;

  SoftmaxState<D, GBM> st;
  st.init();

  // ---- representatives: logit z, value k-mean row ----------------------
  for (int64_t base = r0; base < r1; base += kListCap) {
    const int64_t n = min((int64_t)kListCap, r1 - base);
    __syncthreads();
    if (tid < n) list[tid] = index.unselected(base + tid);
    __syncthreads();
    for (int64_t i = lg; i < n; i += 16) {
      const int64_t b = list[i];
      float x[GBM], v[CH];
#pragma unroll
      for (int g = 0; g < GBM; ++g)
        x[g] = g < gn ? a.z[(h * G + g0 + g) * N + b] * kLog2e : kNegInf;
      load_bf16<CH>(a.value_mean + (h * N + b) * D + c * CH, v);
      st.update(x, v, gn);
    }
  }

  // ---- expanded pages: exact tokens ------------------------------------
  for (int64_t base = p0; base < p1; base += kListCap) {
    const int64_t n = min((int64_t)kListCap, p1 - base);
    __syncthreads();
    if (tid < n) list[tid] = index.selected(base + tid);
    __syncthreads();
    const int64_t rows = n * a.block;
    for (int64_t r = lg; r < rows; r += 16) {
      const int64_t j = r / a.block, t = r - j * a.block;
      const int64_t b = list[j];
      const int64_t cnt = b == N - 1 ? a.length - (N - 1) * a.block : a.block;
      if (t >= cnt) continue;
      const int64_t row = b * a.block + t;
      float kv[CH], v[CH], x[GBM];
      load_bf16<CH>(a.key_pages + h * a.kp_hs + row * D + c * CH, kv);
      load_bf16<CH>(a.value_pages + h * a.vp_hs + row * D + c * CH, v);
#pragma unroll
      for (int g = 0; g < GBM; ++g) {
        float s = q[g][0] * kv[0];
#pragma unroll
        for (int i = 1; i < CH; ++i) s = s + q[g][i] * kv[i];
        s = group16_sum(s);
        x[g] = g < gn ? s * qscale : kNegInf;
      }
      st.update(x, v, gn);
    }
  }

  // ---- generated suffix tokens -----------------------------------------
  for (int64_t k = s0 + lg; k < s1; k += 16) {
    float kv[CH], v[CH], x[GBM];
    load_bf16<CH>(a.key_suffix + h * a.ks_hs + k * a.ks_ts + c * CH, kv);
    load_bf16<CH>(a.value_suffix + h * a.vs_hs + k * a.vs_ts + c * CH, v);
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      float s = q[g][0] * kv[0];
#pragma unroll
      for (int i = 1; i < CH; ++i) s = s + q[g][i] * kv[i];
      s = group16_sum(s);
      x[g] = g < gn ? s * qscale : kNegInf;
    }
    st.update(x, v, gn);
  }

  // ---- merge the 16 lane groups ----------------------------------------
#pragma unroll
  for (int o = 16; o <= 32; o <<= 1) {
    float om[GBM], ol[GBM], oacc[GBM][CH];
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      om[g] = shfl_xor(st.m[g], o);
      ol[g] = shfl_xor(st.l[g], o);
#pragma unroll
      for (int i = 0; i < CH; ++i) oacc[g][i] = shfl_xor(st.acc[g][i], o);
    }
    st.merge(om, ol, oacc, gn);
  }
  if ((tid & 63) < 16) {
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g < gn) {
        if (c == 0) {
          xm[wave][g] = st.m[g];
          xl[wave][g] = st.l[g];
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) xacc[wave][g][c * CH + i] = st.acc[g][i];
      }
    }
  }
  __syncthreads();
  if (tid < 16) {
    for (int ow = 1; ow < kWaves; ++ow) {
      float om[GBM], ol[GBM], oacc[GBM][CH];
#pragma unroll
      for (int g = 0; g < GBM; ++g) {
        om[g] = g < gn ? xm[ow][g] : kNegInf;
        ol[g] = g < gn ? xl[ow][g] : 0.0f;
#pragma unroll
        for (int i = 0; i < CH; ++i) oacc[g][i] = g < gn ? xacc[ow][g][c * CH + i] : 0.0f;
      }
      st.merge(om, ol, oacc, gn);
    }
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      if (g < gn) {
        const int64_t slot = (h * G + g0 + g) * a.workers + w;
        if (c == 0) {
          a.part_m[slot] = st.m[g];
          a.part_l[slot] = st.l[g];
        }
#pragma unroll
        for (int i = 0; i < CH; ++i) a.part_acc[slot * D + c * CH + i] = st.acc[g][i];
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Kernel 4: merge split-K partials -> bf16 output
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void merge_kernel(const float* __restrict__ part_m,
                                                    const float* __restrict__ part_l,
                                                    const float* __restrict__ part_acc,
                                                    uint16_t* __restrict__ out, int workers,
                                                    int dim) {
  const int64_t r = blockIdx.x;
  const int d = threadIdx.x;
  float M = kNegInf;
  for (int w = 0; w < workers; ++w) M = fmaxf(M, part_m[r * workers + w]);
  const float ms = M == kNegInf ? 0.0f : M;
  float den = 0.0f, num = 0.0f;
  for (int w = 0; w < workers; ++w) {
    const float l = part_l[r * workers + w];
    if (l > 0.0f) {
      const float e = __builtin_amdgcn_exp2f(part_m[r * workers + w] - ms);
      den = den + l * e;
      if (d < dim) num = num + part_acc[(r * workers + w) * dim + d] * e;
    }
  }
  if (d < dim) out[r * dim + d] = bf16_rne(num / fmaxf(den, 1e-30f));
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
struct SelectParams {
  const void* query;
  const void* key_mean;
  const void* ellipsoid;
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
  if (!aligned(p.query, 16) || !aligned(p.key_mean, 16) || !aligned(p.ellipsoid, 16))
    return set_error(kInvalidArgument, "%s: query/summary must be 16-byte aligned", who);
  L = make_layout(p.heads, p.group, p.dim, p.n_blocks);
  if (!p.ws || p.ws_bytes < (size_t)L.total || !aligned(p.ws, 256))
    return set_error(kWorkspaceTooSmall, "%s: workspace needs %lld bytes, 256-byte aligned", who,
                     (long long)L.total);
  if (L.n_tiles > 0x7FFFFFFF) return set_error(kInvalidArgument, "%s: too many blocks", who);
  return kOk;
}

int launch_select(const SelectParams& p, const Layout& L) {
  ScoreArgs sa;
  sa.query = static_cast<const uint16_t*>(p.query);
  sa.key_mean = static_cast<const uint16_t*>(p.key_mean);
  sa.ellipsoid = static_cast<const uint16_t*>(p.ellipsoid);
  sa.z = at<float>(p.ws, L.z);
  sa.delta = at<float>(p.ws, L.delta);
  sa.lse = at<float>(p.ws, L.lse);
  sa.n_blocks = p.n_blocks;
  sa.n_tiles = L.n_tiles;
  sa.block = p.block;
  sa.length = p.length;
  sa.group = (int)p.group;
  sa.scale = (float)pow((double)p.dim, -0.5);
  const size_t score_smem = sizeof(float) * (2 * p.group * p.dim + 4 * p.group * kTile);
  dim3 grid((unsigned)L.n_tiles, (unsigned)p.heads);
  mark(0, p.stream);
  RKV_DISPATCH_DIM(p.dim, D,
                   score_kernel<D><<<grid, dim3(kThreads), score_smem, p.stream>>>(sa));
  int rc = check_launch("score_kernel");
  if (rc) return rc;
  mark(1, p.stream);

  DecideArgs da;
  da.z = sa.z;
  da.delta = sa.delta;
  da.lse = sa.lse;
  da.value_norm = p.value_norm;
  da.max_value_norm = p.max_value_norm;
  da.anchor = p.anchor;
  da.mask = p.mask;
  da.tilebits = at<uint64_t>(p.ws, L.tilebits);
  da.risk_out = p.risk_out;
  da.stats_out = p.stats_out;
  da.accessed = p.accessed;
  da.n_blocks = p.n_blocks;
  da.n_tiles = L.n_tiles;
  da.block = p.block;
  da.length = p.length;
  da.group = (int)p.group;
  da.reduction = p.reduction;
  da.eps = p.eps;
  decide_kernel<<<grid, dim3(kThreads), 0, p.stream>>>(da);
  rc = check_launch("decide_kernel");
  mark(2, p.stream);
  return rc;
}

template <int D>
int launch_attend(const AttendArgs& aa, const Layout& L, int64_t heads, hipStream_t stream) {
  constexpr int GBM = (64 / (D / 16)) > kMaxGroup ? kMaxGroup : (64 / (D / 16));
  const size_t smem = align256((L.n_tiles + 1) * 8) + align256(L.n_tiles * 8) +
                      sizeof(int64_t) * kListCap;
  if (smem > 48 * 1024) return set_error(kUnsupported, "attend: %lld tiles exceed LDS",
                                         (long long)L.n_tiles);
  dim3 grid((unsigned)L.workers, (unsigned)heads, (unsigned)L.row_blocks);
  attend_kernel<D, GBM><<<grid, dim3(kThreads), smem, stream>>>(aa);
  return check_launch("attend_kernel");
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" size_t rkv_workspace_bytes(int64_t heads, int64_t group, int64_t dim,
                                      int64_t n_blocks) {
  if (heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0) return 0;
  return (size_t)make_layout(heads, group, dim, n_blocks).total;
}

// Byte offsets of the workspace regions, for tests: z, delta, lse, tilebits,
// attn_m, attn_l, attn_acc, total, n_tiles, workers.
extern "C" int rkv_workspace_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                                    int64_t* out10) {
  if (!out10 || heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_workspace_layout: bad arguments");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  const int64_t v[10] = {L.z, L.delta, L.lse, L.tilebits, L.attn_m,
                         L.attn_l, L.attn_acc, L.total, L.n_tiles, L.workers};
  for (int i = 0; i < 10; ++i) out10[i] = v[i];
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
  SelectParams p{query, key_mean, ellipsoid, value_norm, max_value_norm, heads, group, dim,
                 n_blocks, block_size, prompt_length, eps, reduction, anchor_mask, mask_out,
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
  SelectParams p{query, key_mean, ellipsoid, value_norm, max_value_norm, heads, group, dim,
                 n_blocks, block_size, prompt_length, eps, reduction, anchor_mask, mask_out,
                 nullptr, nullptr, accessed_blocks, workspace, workspace_bytes, stream};
  Layout L;
  int rc = validate_select(p, "rkv_decode", L);
  if (rc) return rc;
  if (!value_mean || !key_pages || !value_pages || !output)
    return set_error(kInvalidArgument, "rkv_decode: null pointer argument");
  if (suffix_capacity < 0)
    return set_error(kInvalidArgument, "rkv_decode: negative suffix capacity");
  if (suffix_capacity > 0 && (!key_suffix || !value_suffix))
    return set_error(kInvalidArgument, "rkv_decode: null suffix with nonzero capacity");
  const int64_t es = 2;
  const int64_t ch_bytes = dim / 16 * es;
  const uintptr_t need = ch_bytes % 16 == 0 ? 16 : (ch_bytes % 8 == 0 ? 8 : 4);
  if (!aligned(value_mean, 16) || !aligned(key_pages, need) || !aligned(value_pages, need) ||
      (key_page_head_stride * es) % need || (value_page_head_stride * es) % need)
    return set_error(kInvalidArgument, "rkv_decode: pages must be %d-byte aligned", (int)need);
  if (suffix_capacity > 0 &&
      (!aligned(key_suffix, need) || !aligned(value_suffix, need) ||
       (key_suffix_head_stride * es) % need || (key_suffix_token_stride * es) % need ||
       (value_suffix_head_stride * es) % need || (value_suffix_token_stride * es) % need))
    return set_error(kInvalidArgument, "rkv_decode: suffix rows must be %d-byte aligned",
                     (int)need);
  if (!aligned(output, 4)) return set_error(kInvalidArgument, "rkv_decode: output alignment");
  rc = launch_select(p, L);
  if (rc) return rc;

  AttendArgs aa;
  aa.query = static_cast<const uint16_t*>(query);
  aa.z = at<float>(workspace, L.z);
  aa.value_mean = static_cast<const uint16_t*>(value_mean);
  aa.key_pages = static_cast<const uint16_t*>(key_pages);
  aa.value_pages = static_cast<const uint16_t*>(value_pages);
  aa.key_suffix = static_cast<const uint16_t*>(key_suffix);
  aa.value_suffix = static_cast<const uint16_t*>(value_suffix);
  aa.tilebits = at<uint64_t>(workspace, L.tilebits);
  aa.suffix_len_dev = suffix_length;
  aa.part_m = at<float>(workspace, L.attn_m);
  aa.part_l = at<float>(workspace, L.attn_l);
  aa.part_acc = at<float>(workspace, L.attn_acc);
  aa.kp_hs = key_page_head_stride;
  aa.vp_hs = value_page_head_stride;
  aa.ks_hs = key_suffix_head_stride;
  aa.ks_ts = key_suffix_token_stride;
  aa.vs_hs = value_suffix_head_stride;
  aa.vs_ts = value_suffix_token_stride;
  aa.suffix_cap = suffix_capacity;
  aa.n_blocks = n_blocks;
  aa.n_tiles = L.n_tiles;
  aa.block = block_size;
  aa.length = prompt_length;
  aa.group = (int)group;
  aa.workers = (int)L.workers;
  aa.rows_per_block = (int)L.rows_per_block;
  aa.scale = (float)pow((double)dim, -0.5);
  rc = kOk;
  RKV_DISPATCH_DIM(dim, D, rc = launch_attend<D>(aa, L, heads, stream));
  if (rc) return rc;
  mark(3, stream);
  merge_kernel<<<dim3((unsigned)(heads * group)), dim3((unsigned)((dim + 63) / 64 * 64)), 0,
                 stream>>>(aa.part_m, aa.part_l, aa.part_acc, static_cast<uint16_t*>(output),
                           (int)L.workers, (int)dim);
  rc = check_launch("merge_kernel");
  mark(4, stream);
  return rc;
}

// Profiling hook: when events is non-null (an array of 5 hipEvent_t), the
// following rkv_select / rkv_decode calls on this thread record events[0]
// before the score kernel and events[1..4] after score, decide, attend and
// merge.  Pass NULL to stop.
extern "C" int rkv_set_profile_events(void* events) {
  g_events = static_cast<hipEvent_t*>(events);
  return kOk;
}
