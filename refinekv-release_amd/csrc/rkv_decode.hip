// Decode-step selection and mixed attention (src/refinekv/reference.py:10-73;
// the reference's Triton kernels in src/refinekv/kernels/ follow the same
// semantics).  No host sync, no allocation: the caller passes a workspace.
//
// A decode step runs as ONE launch where the shape allows it (step_kernel):
// workgroup (w, h) of the W per KV head h scores tile w mod T (64 blocks),
// publishes its log-sum-exp partials in tagged slots, reads the head's T
// tiles' slots, decides its blocks (risk, GQA reduction, anchors), folds its
// representatives, its slice of the suffix and the token rows of its own
// tile's expanded blocks (a copy of a tile, with more workgroups than
// tiles, an even slice of them), publishes an (m, l, acc) partial in tagged
// slots, and the head's last max(8, W / 4) workgroups by index (at most
// head_dim / 2) each merge a column slice of the partials into the bf16
// output.  Heads with more tiles
// than workgroups score up to 4 tiles per workgroup in the same launch.
// Other shapes run three kernels over the same workspace:
//
//   score  (tile, h)    one 64-block tile of head h: for every query row the
//                       selection dot products s = q.k_mean and
//                       p = q^2.ellipsoid (FMA chains over 8 or 16 lanes per
//                       block, then an xor butterfly), z = s*scale + ln n,
//                       delta, and the tile's log-sum-exp partials of z and
//                       of z + log cosh delta.
//   attend (tile, h)    log Z / log C of each row from the tile partials, the
//                       risk, the GQA reduction, the non-finite fail-safes and
//                       the anchor union -> mask and access count; then one
//                       online softmax per row over the tile's
//                       representatives, the tokens of its expanded blocks
//                       and a 1/T slice of the generated suffix -> one
//                       (m, l, acc) partial per row and tile.
//   merge  (row, cols)  the row's tile partials -> bf16 output columns, and
//                       the access counter.
//
// Token rows (representatives, expanded blocks, suffix) are attended on the
// matrix cores for head_dim <= 160 (QK^T and PV MFMAs, value rows staged in
// LDS), on the vector ALUs above.  The dense decode (dense_kernel + merge)
// attends every cached token with the same matrix-core engine.
//
// Selection statistics (z, delta, log Z, log C, risk) follow fixed fp32
// orders shared with the CPU oracle (oracle/rkv_oracle.c): z and delta equal
// the oracle's bit for bit; e^x and log x run on the hardware's
// transcendental unit (exp_hw / log_hw below), so log Z, log C and the risks
// are within a few ulp of the oracle's and a block's mask can differ from
// the oracle's only where a row's risk lies within that distance of eps.
// Every order is fixed, so masks and outputs are deterministic run to run.
#include <math.h>

#include <atomic>
#include <type_traits>
#include <utility>

#include "rkv_common.h"
#include "rkv_internal.h"

namespace rkv {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kLine = 8;  // u64 counters per 64-byte hand-off line
constexpr uint32_t kSpinLimit = 1u << 20;  // polls before a hand-off wait gives up (default)
constexpr int64_t kStepMaxTiles = 256;     // tiles per head the one-launch step takes
constexpr int kStepTiles = 4;              // tiles a workgroup of the one-launch step scores, at most

// Bytes of the one-launch step's hand-off counters: one line per KV head,
// one for the launch, then one launch counter per tile.
__host__ __device__ constexpr int64_t control_bytes(int64_t heads, int64_t tile_stride) {
  return (heads + 1) * kLine * 8 + heads * tile_stride * 8;
}

// Phase stamps of the one-launch step (the library built with
// RKV_PHASE_STAMPS only; bench.py --phases loads it): lane 0 of a wave notes
// the 100 MHz constant clock (s_memrealtime) in LDS at each phase boundary
// of its workgroup, and the workgroup copies its stamps to rkv_stamps
// (row h * 256 + workgroup) as it ends.  LDS stores leave the vector-memory
// counters alone, so the kernel's own waits are unchanged.  The product build
// compiles every stamp to nothing.
constexpr int kStamps = 42;
constexpr int kStampRowsPerHead = 256;
enum Stamp {
  kStEntry = 0, kStDots, kStStats, kStGather, kStDecided, kStRing, kStPagesWave0, kStCombine,
  kStPublished, kStMergeWait, kStMerged, kStSpec, kStEnd, kStMergeLoaded,
  kStMergeFolded, kStMergeStored, kStMergeCounted, kStChunk0, kStChunk1, kStChunk2,
  kStIssued2, kStFold0Start, kStRingStart, kStIssue2Addr,
  kStFoldStart0, kStFoldEnd0 = kStFoldStart0 + 6, kStIssueStart2 = kStFoldEnd0 + 6
};
#if defined(RKV_PHASE_STAMPS)
constexpr int kStampHeads = 64;
__device__ unsigned long long rkv_stamps[kStampHeads * kStampRowsPerHead][kStamps];
#define RKV_STAMP(stamps, i, cond)                                                   \
  do {                                                                               \
    if ((stamps) != nullptr && (cond)) (stamps)[i] = __builtin_amdgcn_s_memrealtime(); \
  } while (0)
#else
#define RKV_STAMP(stamps, i, cond) ((void)0)
#endif

// Optional profiling events (rkv_set_profile_events): events[0] is recorded
// before the first kernel of a call and events[k] after its k-th kernel.
thread_local hipEvent_t* g_events = nullptr;

inline void mark(int i, hipStream_t stream) {
  if (g_events) (void)hipEventRecord(g_events[i], stream);
}

// Query rows one attention pass carries in registers: the next power of two
// >= group (at least 4), capped so that rows * head_dim / 16 (per-lane
// accumulators) stays <= 64.
inline int64_t rows_per_pass(int64_t group, int64_t dim) {
  const int64_t cap = 64 / (dim / 16);
  int64_t p = 16;
  while (p > cap) p >>= 1;
  int64_t want = 4;
  while (want < group && want < 16) want <<= 1;
  return want < p ? want : p;
}

// ---------------------------------------------------------------------------
// Workspace layout.  Every per-row region starts on a 256-byte boundary and
// per-row strides cover whole tiles.
// ---------------------------------------------------------------------------
struct Layout {
  int64_t n_tiles, z_stride, tile_stride;
  int64_t step_workers;  // workgroups per head of the one-launch step
  int64_t step_tiles;    // tiles its workgroups score, at most (1: one each)
  int64_t control, zf, lse, lse_slots, part_ml, part_acc, counts, full, row_lse, total;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

Layout make_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks) {
  Layout L{};
  L.n_tiles = (n_blocks + kTile - 1) / kTile;
  L.z_stride = L.n_tiles * kTile;
  // The one-launch step runs max(n_tiles, min(S / heads, 256)) workgroups
  // per head: the n_tiles tiles and, with short prompts or few heads, copies
  // of them that also take a share of the head's suffix and expanded token
  // rows, so that the token work spreads over the GPU (S = 512, two
  // workgroups per CU on 256 CUs; 256 for the 16-row kernels, which take
  // more than 256 registers per lane).  The per-tile arrays have a slot per
  // workgroup.
  // With more tiles than that, four-row passes up to head_dim 128 keep
  // min(S / heads, 256) workgroups per head, each scoring up to kStepTiles
  // tiles (so 128K tokens at block 16 or 512K at block 32 stay one resident
  // launch); other shapes take one workgroup per tile.
  const int64_t pass_rows = rows_per_pass(group, dim);
  const int64_t slots = pass_rows == 16 ? 256 : 512;
  const int64_t want = slots / heads < kStepMaxTiles ? slots / heads : kStepMaxTiles;
  L.step_workers = L.n_tiles > want ? L.n_tiles : want;
  L.step_tiles = 1;
  if (L.n_tiles > want && want > 0 && pass_rows == 4 && dim <= 128 &&
      (L.n_tiles + want - 1) / want <= kStepTiles) {
    L.step_workers = want;
    L.step_tiles = (L.n_tiles + want - 1) / want;
  }
  const int64_t per_tile = L.step_workers > L.n_tiles ? L.step_workers : L.n_tiles;
  L.tile_stride = (per_tile + 63) / 64 * 64;
  const int64_t rows = heads * group;
  int64_t off = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = off;
    off = align256(off + bytes);
    return at;
  };
  L.control = take(control_bytes(heads, L.tile_stride));
  L.zf = take(rows * L.z_stride * 16);
  L.lse = take(rows * L.tile_stride * 4 * 4);
  L.lse_slots = take(rows * L.tile_stride * 2 * 16);
  // partials and access counts: the one-launch step's tagged 16-byte slots
  // (one per row for (m, l), one per row and column pair for acc, one per
  // workgroup for the count); the three kernels use the first half or
  // quarter of each region as plain (m, l) pairs, floats and u32 counts
  L.part_ml = take(rows * L.tile_stride * 16);
  L.part_acc = take(rows * L.tile_stride * dim * 8);
  L.counts = take(heads * L.tile_stride * 16);
  L.full = take(heads * L.tile_stride * 8);
  // per row log Z, log C merged once (three-kernel path, more than 64 tiles)
  L.row_lse = take(rows * 2 * 4);
  L.total = off;
  return L;
}

template <typename T>
T* at(void* ws, int64_t off) {
  return reinterpret_cast<T*>(static_cast<char*>(ws) + off);
}

// ---------------------------------------------------------------------------
// Selection math (reference.py:16-34): the oracle's operations in its order,
// with its exponentials and logarithms on the hardware's transcendental unit.
// ---------------------------------------------------------------------------
// e^x and log x of the selection statistics, decisions and LSE merges are
// exp_hw / log_hw (rkv_common.h): the hardware's transcendental unit in
// place of the oracle's expf_ / logf_, which the device runs bit for bit but
// at 3-4 times the instructions.  z and delta do not use them and stay
// bit-exact; log Z, log C and the risks are within a few ulp of the
// oracle's, and the masks equal its masks wherever no row's risk is within
// that distance of eps.
// The delta-only terms of a (row, block) pair, computed once by the score
// phase: log cosh delta (reference.py:19-22) and the two factors the risk
// (reference.py:24-34) multiplies in -- A = cosh(delta) - 1 written as
// 0.5 (t + 1/t) - 1 with t = e^delta (delta <= 10), or log(cosh(delta) - 1)
// in its large-delta form; th = tanh(delta / 2) in the matching form.
// Every lane computes the small-delta forms (on delta clamped to kDeltaMax);
// lanes with a larger delta (rare) take the large-delta forms behind a
// wave-uniform branch, so the common case is branch-free.  The terms come in
// two parts: log cosh delta, which the LSE partials need, and the risk's
// factors A and th, which only the decision needs (computed after the
// partials are out).  t = e^min(delta, kDeltaMax) passes between them.
__device__ __forceinline__ float delta_log_cosh(float delta, float& t) {
  const float c = clamp_max(delta, kDeltaMax);
  t = exp_hw(c);
  float log_cosh = log_hw((t + exp_hw(-c)) * 0.5f);
  const bool large = !(delta <= kDeltaMax);  // NaN takes the large form, as on the host
  if (__ballot(large) != 0) {
    const float d = large ? delta : 0.0f;
    const float lc = d + log_hw((1.0f + exp_hw(-2.0f * d)) * 0.5f);
    log_cosh = large ? lc : log_cosh;
  }
  return log_cosh;
}

__device__ __forceinline__ void delta_factors(float delta, float t, float& A, float& th) {
  A = (0.5f * (t + 1.0f / t)) - 1.0f;
  th = (t - 1.0f) / (t + 1.0f);
  const bool large = !(delta <= kDeltaMax);
  if (__ballot(large) != 0) {
    const float d = large ? delta : 0.0f;
    const float exp_neg = exp_hw(-d);
    const float la = (d + 2.0f * log_hw(clamp_min(1.0f - exp_neg, 1e-30f))) - kLn2;
    const float lt = (1.0f - exp_neg) / (1.0f + exp_neg);
    A = large ? la : A;
    th = large ? lt : th;
  }
}

// risk (reference.py:24-34) from z, delta and the delta terms: the same
// operations in the same order as computing everything here.
__device__ __forceinline__ float risk_from(float z, float delta, float A, float th, float log_z,
                                           float log_c, float vmax, float vnorm) {
  float mass;
  if (delta <= kDeltaMax) mass = ((2.0f * vmax) * exp_hw(z - log_c)) * A;
  else mass = (2.0f * vmax) * exp_hw((z - log_c) + A);
  const float value = ((2.0f * vnorm) * exp_hw(z - log_z)) * th;
  return mass + value;
}

__host__ __device__ __forceinline__ float inf_to_zero(float m) {
  return (m == kPosInf || m == kNegInf) ? 0.0f : m;
}

// Sum over each 8-lane group (lanes 0-7 and 8-15 of every 16-lane row) in
// the xor-butterfly tree (distances 4, 2, 1: P[j] <- P[j] + P[j^o]).  The
// group's last lane computes exactly the tree the butterfly leaves in its
// first lane (operands commuted, which fp32 add ignores); its dependency
// chain stays inside the group.
__device__ __forceinline__ float group8_sum_last(float v) {
  v = v + row_shr<4>(v);
  v = v + row_shr<2>(v);
  v = v + row_shr<1>(v);
  return v;
}

template <int L>
__device__ __forceinline__ float lanes_sum_last(float v) {
  if constexpr (L == 8) return group8_sum_last(v);
  else return row16_sum_last(v);
}

// The selection dot products of one block are split over kLanes lanes, each
// holding kCh consecutive elements: 8 lanes up to head_dim 128, else 16.
template <int D>
struct Dots {
  static constexpr int kLanes = D <= 128 ? 8 : 16;
  static constexpr int kCh = D / kLanes;
  static constexpr int kPerPass = kThreads / kLanes;  // blocks per pass of the workgroup
  static constexpr int kPasses = kTile / kPerPass;
};

// ---------------------------------------------------------------------------
// Kernel 1: scores of one (tile, head)
// ---------------------------------------------------------------------------
struct ScoreArgs {
  const uint16_t* query;      // (H, G, D) bf16
  const uint16_t* key_mean;   // (H, N, D) bf16
  const uint16_t* ellipsoid;  // (H, N, D) bf16
  float4* zf;                 // (H*G, z_stride): z, delta, A, th
  float* lse;                 // (H*G, tile_stride, 4): zm, zl, cm, cl
  int64_t n_blocks, block, length;
  int64_t z_stride, tile_stride;
  int group;
  int summary_heads;          // query head h reads the summaries of head h % summary_heads
  float scale;
  float ln_full, ln_last;     // logf_ of a full block's and of the last block's token count
};

// q and bf16(q^2) are staged once per workgroup in LDS as fp32, each row as
// kLanes slices of kCh values padded by 4 (so the slices the lanes of a block
// read start on distinct banks).  The workgroup's threads each stage one or
// more query word pairs, then a barrier.
constexpr int kQPad = 4;
constexpr int kQWords = 4;  // query words a thread loads ahead (G * D <= 2048 * 4)

// Floats of LDS that stage q and bf16(q^2) for `group` rows.
__host__ __device__ constexpr int64_t score_q_floats(int64_t group, int64_t dim) {
  return 2 * group * (dim + (dim <= 128 ? 8 : 16) * kQPad);
}

// The most score_q_floats needs for any group up to `group`.
__host__ __device__ constexpr int64_t score_q_floats_max(int64_t group, int64_t dim) {
  int64_t m = 0;
  for (int64_t g = 1; g <= group; ++g) m = score_q_floats(g, dim) > m ? score_q_floats(g, dim) : m;
  return m;
}

inline size_t score_smem(int64_t group, int64_t dim) {
  return sizeof(float) * (2 * group * kTile + score_q_floats(group, dim));
}

// N consecutive floats from LDS (16-byte loads when aligned, else 8-byte).
template <int N>
__device__ __forceinline__ void lds_read(const float* p, float (&out)[N]) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int j = 0; j < N / 4; ++j) {
      const float4 v = reinterpret_cast<const float4*>(p)[j];
      out[4 * j] = v.x;
      out[4 * j + 1] = v.y;
      out[4 * j + 2] = v.z;
      out[4 * j + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int j = 0; j < N / 2; ++j) {
      const float2 v = reinterpret_cast<const float2*>(p)[j];
      out[2 * j] = v.x;
      out[2 * j + 1] = v.y;
    }
  }
}

// The selection dot products of tile `tile` of head h for every query row:
// A tile's summary rows as loaded: this thread's key-mean and ellipsoid
// slices of its blocks (one per pass).
template <int D>
struct ScoreRaw {
  RawBf16<Dots<D>::kCh> k[Dots<D>::kPasses], e[Dots<D>::kPasses];
};

// The summary loads of tile `tile` of head h (blocks past the end read block
// N - 1; their results are discarded).
template <int D>
__device__ __forceinline__ void score_load(const ScoreArgs& a, int64_t h, int64_t tile,
                                           ScoreRaw<D>& raw) {
  using S = Dots<D>;
  constexpr int CH = S::kCh;
  const int64_t N = a.n_blocks;
  const int tid = threadIdx.x;
  const int c = tid % S::kLanes, sub = tid / S::kLanes;
  const int64_t hs = h % a.summary_heads;  // the summaries' head
#pragma unroll
  for (int ps = 0; ps < S::kPasses; ++ps) {
    int64_t b = tile * kTile + ps * S::kPerPass + sub;
    b = b < N ? b : N - 1;
    const int64_t o = (hs * N + b) * D + c * CH;
    raw.k[ps] = load_raw<CH>(a.key_mean + o);
    raw.e[ps] = load_raw<CH>(a.ellipsoid + o);
  }
}

// The dot products of a tile from its loaded rows and the staged q (see
// score_dots); ends with a barrier.  kLowReg (the score kernel, four
// workgroups per CU): one query row's slice of q at a time, read from LDS
// for each pass, instead of four rows' held across both passes -- the same
// dot products in the same order, in half the registers.
template <int D, int kMaxG = kMaxGroup, bool kLowReg = false>
__device__ __forceinline__ void score_from(const ScoreArgs& a, const ScoreRaw<D>& raw,
                                           float* sdot, float* pdot, const float* qstage) {
  using S = Dots<D>;
  constexpr int CH = S::kCh;
  const int G = a.group;
  const int tid = threadIdx.x;
  const int c = tid % S::kLanes, sub = tid / S::kLanes;
  constexpr int QW = CH + kQPad;          // padded slice
  constexpr int QS = S::kLanes * QW;      // padded row
  const float* qs = qstage;               // [G][QS] bf16(q)
  const float* q2s = qs + G * QS;         // [G][QS] bf16(q^2)
  if constexpr (kLowReg) {
#pragma unroll
    for (int ps = 0; ps < S::kPasses; ++ps) {
      float km[CH], el[CH];
      unpack(raw.k[ps], km);
      unpack(raw.e[ps], el);
      const int bl = ps * S::kPerPass + sub;
#pragma unroll 1
      for (int g = 0; g < G; ++g) {
        float qv[CH], q2v[CH];
        lds_read<CH>(qs + g * QS + c * QW, qv);
        lds_read<CH>(q2s + g * QS + c * QW, q2v);
        float s = qv[0] * km[0];
        float p = q2v[0] * el[0];
#pragma unroll
        for (int i = 1; i < CH; ++i) {
          s = __builtin_fmaf(qv[i], km[i], s);
          p = __builtin_fmaf(q2v[i], el[i], p);
        }
        s = lanes_sum_last<S::kLanes>(s);
        p = lanes_sum_last<S::kLanes>(p);
        if (c == S::kLanes - 1) {
          sdot[g * kTile + bl] = s;
          pdot[g * kTile + bl] = p;
        }
      }
    }
    __syncthreads();
    return;
  }

  // Rows g0 .. g0+3: a lambda so that the common case (G <= 4, one call)
  // waits for each pass's loads just before it, not for both passes first.
  auto four_rows = [&](int g0) {
    // this lane's slice of q and q^2 for rows g0 .. g0+3 (clamped)
    float qv[4][CH], q2v[4][CH];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int g = g0 + j < G ? g0 + j : G - 1;
      lds_read<CH>(qs + g * QS + c * QW, qv[j]);
      lds_read<CH>(q2s + g * QS + c * QW, q2v[j]);
    }
#pragma unroll
    for (int ps = 0; ps < S::kPasses; ++ps) {
      float km[CH], el[CH];
      unpack(raw.k[ps], km);
      unpack(raw.e[ps], el);
      float sv[4], pv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // DSUM: this lane's CH elements as an FMA chain from the first
        // product, then the butterfly over the block's lanes.
        float s = qv[j][0] * km[0];
        float p = q2v[j][0] * el[0];
#pragma unroll
        for (int i = 1; i < CH; ++i) {
          s = __builtin_fmaf(qv[j][i], km[i], s);
          p = __builtin_fmaf(q2v[j][i], el[i], p);
        }
        sv[j] = lanes_sum_last<S::kLanes>(s);
        pv[j] = lanes_sum_last<S::kLanes>(p);
      }
      if (c == S::kLanes - 1) {
        const int bl = ps * S::kPerPass + sub;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if (g0 + j < G) {
            sdot[(g0 + j) * kTile + bl] = sv[j];
            pdot[(g0 + j) * kTile + bl] = pv[j];
          }
        }
      }
    }
  };
  if (kMaxG <= 4 || G <= 4) {
    four_rows(0);
  } else {
    for (int g0 = 0; g0 < G; g0 += 4) four_rows(g0);
  }
  __syncthreads();
}

// sdot[g][b] = q_g . k_mean_b and pdot[g][b] = bf16(q_g^2) . ellipsoid_b
// (DSUM), b tile-relative; ends with a barrier.  qstage holds
// score_q_floats(G, D) floats of LDS (q and bf16(q^2), staged here; they
// stay for score_from of further tiles).  kMaxG bounds the group (the step
// kernel's rows per pass), so the four-row loop is compiled only where
// groups above four can reach it.
template <int D, int kMaxG = kMaxGroup, bool kLowReg = false>
__device__ __forceinline__ void score_dots(const ScoreArgs& a, int64_t h, int64_t tile,
                                           float* sdot, float* pdot, float* qstage) {
  using S = Dots<D>;
  constexpr int CH = S::kCh;
  const int G = a.group;
  const int tid = threadIdx.x;

  constexpr int QW = CH + kQPad;          // padded slice
  constexpr int QS = S::kLanes * QW;      // padded row
  float* qs = qstage;                     // [G][QS] bf16(q)
  float* q2s = qs + G * QS;               // [G][QS] bf16(q^2)
  const uint32_t* q32 = reinterpret_cast<const uint32_t*>(a.query + h * G * D);
  const int first = tid, step = kThreads;
  // The query words first (the staging below waits only for them: loads
  // complete in order), then every load of the tile.
  uint32_t qw[kQWords];
#pragma unroll
  for (int k = 0; k < kQWords; ++k) {
    const int i = first + k * step;
    qw[k] = q32[i < G * D / 2 ? i : 0];
  }
  ScoreRaw<D> raw;
  score_load<D>(a, h, tile, raw);
  // The query words are used here, after the summary loads are issued: a
  // query load sunk into the staging branch below would be issued after
  // them and wait for all of them.
#pragma unroll
  for (int k = 0; k < kQWords; ++k) asm volatile("" : "+v"(qw[k]));
  auto stage = [&](int i, uint32_t u) {
    const float q0 = bits_f32(u << 16), q1 = bits_f32(u & 0xFFFF0000u);
    const int g = 2 * i / D, e = 2 * i % D;  // element pair e, e + 1 of row g
    const int at = g * QS + (e / CH) * QW + e % CH;
    qs[at] = q0;
    qs[at + 1] = q1;
    q2s[at] = round_bf16(q0 * q0);
    q2s[at + 1] = round_bf16(q1 * q1);
  };
#pragma unroll
  for (int k = 0; k < kQWords; ++k) {
    const int i = first + k * step;
    if (i < G * D / 2) stage(i, qw[k]);
  }
  for (int i = first + kQWords * step; i < G * D / 2; i += step) stage(i, q32[i]);
  __syncthreads();
  score_from<D, kMaxG, kLowReg>(a, raw, sdot, pdot, qstage);
}

// z, delta, the risk's delta-only factors and the tile's LSE partials from
// the dot products: wave w owns rows w, w + 4, ...; lane = block of the
// tile.  put_z(g, valid, (z, delta, A, th)) is called by every lane (valid:
// the block exists); put_lse(g, (zm, zl, cm, cl)) by lane 0.
template <typename PutZ, typename PutLse>
__device__ __forceinline__ void score_stats(const ScoreArgs& a, int64_t tile, const float* sdot,
                                            const float* pdot, PutZ put_z, PutLse put_lse) {
  const int G = a.group;
  const int64_t N = a.n_blocks;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
  for (int g = wave; g < G; g += kWaves) {
    // Branch-free (lanes past the last block compute on its dot products and
    // take -inf): the z row's LSE chain interleaves with the delta terms.
    const int64_t b = tile * kTile + lane;
    const bool valid = b < N;
    const float s = sdot[g * kTile + lane] * a.scale;
    const float z = valid ? s + (b == N - 1 ? a.ln_last : a.ln_full) : kNegInf;
    const float zm = wave_nanmax_u(z);
    const float zl = wave_sum_u(exp_hw(z - inf_to_zero(zm)));
    const float dl = (sqrtf(clamp_min(pdot[g * kTile + lane], 0.0f)) * a.scale) * kInflate;
    float t = 1.0f;  // (set by delta_log_cosh on the lanes of existing blocks)
    const float zc = valid ? z + delta_log_cosh(dl, t) : kNegInf;
    const float cm = wave_nanmax_u(zc);
    const float cl = wave_sum_u(exp_hw(zc - inf_to_zero(cm)));
    if (lane == 0) put_lse(g, make_float4(zm, zl, cm, cl));
    float ra, rth;
    delta_factors(dl, t, ra, rth);
    put_z(g, valid, valid ? make_float4(z, dl, ra, rth) : make_float4(kNegInf, 0.0f, 0.0f, 0.0f));
  }
}

template <int D>
// (81 registers at head_dim 128 with score_from's low-register order: up to
// six workgroups per CU, which the 512-tile heads' 4096 workgroups need to
// overlap their loads with the dot products)
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void score_kernel(ScoreArgs a) {
  extern __shared__ float score_lds[];
  const int G = a.group;
  float* sdot = score_lds;          // [G][64]
  float* pdot = sdot + G * kTile;   // [G][64]
  const int64_t h = blockIdx.y, tile = blockIdx.x;
  const int lane = threadIdx.x % kWave;
  score_dots<D, kMaxGroup, true>(a, h, tile, sdot, pdot, pdot + G * kTile);
  score_stats(
      a, tile, sdot, pdot,
      [&](int g, bool valid, float4 zf) {
        if (valid) a.zf[(h * G + g) * a.z_stride + tile * kTile + lane] = zf;
      },
      [&](int g, float4 part) {
        *reinterpret_cast<float4*>(a.lse + ((h * G + g) * a.tile_stride + tile) * 4) = part;
      });
}

// ---------------------------------------------------------------------------
// Decisions of one (tile, head)
// ---------------------------------------------------------------------------
struct DecideArgs {
  const float4* zf;             // (H*G, z_stride): z, delta, A, th
  const float* lse;
  const float* value_norm;      // (H, N)
  const float* max_value_norm;  // (H)
  const uint8_t* anchor;        // (H, N) or null
  uint8_t* mask;                // (H, N)
  bool write_mask;              // false: mask only stands in for a null anchor
  float* risk_out;              // (H, G, N) or null
  float* stats_out;             // (H, G, 2) or null: log Z, log C
  const float* row_lse;         // (H, G, 2) log Z, log C merged once per row, or null
  int64_t n_blocks, n_tiles, block, length;
  int64_t z_stride, tile_stride;
  int group, reduction;
  float eps;
};

struct DecideShared {
  float risk[kMaxGroup][kTile];  // the mean reduction reads every row's risks
  uint64_t tile_bits[kStepTiles];  // several tiles per workgroup: each tile's expanded blocks
  uint64_t wsel[kWaves];         // per wave: OR over its rows of (risk > eps or not finite)
  uint32_t wbad[kWaves];         // per wave: a row's log Z or log C is not finite
  int32_t list[kWaves][kTile];   // per wave: the expanded blocks (tile-relative), ascending
};

// LSE of one row from the tile partials in the fixed order: the max first,
// then 64 lane accumulators (tile t -> lane t % 64, left to right) and the
// 64-wide butterfly.  (m0, l0) is this lane's partial of tile `lane`;
// part(t) gives tile t's (m, l) for tiles beyond the first 64.
template <typename Part>
__device__ __forceinline__ float merge_lse(float m0, float l0, Part part, int64_t n_tiles,
                                           int lane) {
  float mx = lane < n_tiles ? m0 : kNegInf;
  for (int64_t t = lane + kWave; t < n_tiles; t += kWave) mx = nanmax(mx, part(t).x);
  mx = wave_nanmax_u(mx);
  const float ms = inf_to_zero(mx);
  float acc = lane < n_tiles ? l0 * exp_hw(m0 - ms) : 0.0f;
  for (int64_t t = lane + kWave; t < n_tiles; t += kWave) {
    const float2 p = part(t);
    acc = acc + p.y * exp_hw(p.x - ms);
  }
  return log_hw(wave_sum_u(acc)) + ms;
}

// Decides tile `tile` of head h (select_blocks_reference plus the anchor
// union), from the loads decide_issue made: stores the mask (and risk /
// stats when asked) and returns the tile's expanded-block ballot, uniform
// over the workgroup; list (this wave's copy in sh) holds the expanded blocks
// in ascending order.  zsh, when not null, receives z of every (row, block)
// of the tile (-inf past the end).  count (thread 0) receives the tile's
// access count.  One barrier.  The next row's loads are issued before this
// row's arithmetic.
//
// After the fail-safes the max reduction selects exactly the blocks "any"
// selects: a NaN risk makes the max NaN (not > eps) but is non-finite, which
// selects the block anyway.  So both are the OR over rows of
// (risk > eps or risk not finite); mean sums the rows in order.
// The decision's inputs for this thread (block lane of the tile, this wave's
// first row), loaded before anything else is computed.  Every load is
// unconditional (clamped addresses and rows, a stand-in anchor pointer;
// results are selected only after all are issued), so no load waits for
// another at a branch join.
struct DecideLoads {
  float vnorm;
  uint8_t anc;
  float4 part, zf;
};

// kStats = false leaves part and zf to the caller (the one-launch step has
// them only after its hand-off).
// rh: the head index of the statistics rows (lse, zf) -- h except for the
// batched anchor selection, whose query q of head h has rows of head q H + h.
template <bool kStats = true>
__device__ __forceinline__ DecideLoads decide_issue(const DecideArgs& a, int64_t h,
                                                    int64_t tile, int64_t rh = -1) {
  if (rh < 0) rh = h;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
  const int G = a.group;
  const int64_t N = a.n_blocks, T = a.n_tiles;
  const int64_t b = tile * kTile + lane;
  const int64_t bc = b < N ? b : N - 1;
  const int tl = lane < T ? lane : 0;
  const int gl = wave < G ? wave : G - 1;
  const uint8_t* anc = a.anchor ? a.anchor : a.mask;
  DecideLoads d;
  d.vnorm = a.value_norm[h * N + bc];
  d.anc = anc[h * N + bc];
  if constexpr (kStats) {
    d.part = *reinterpret_cast<const float4*>(a.lse + ((rh * G + gl) * a.tile_stride + tl) * 4);
    d.zf = a.zf[(rh * G + gl) * a.z_stride + bc];
  }
  return d;
}

// Self-validating hand-off slots of the one-launch step: 16 bytes {a, b,
// tag, check} written with one coherent store, tag = the launch's epoch + 1
// (a zero-filled slot is never valid) and check = a ^ rotl(b, 13) ^ mix(tag),
// mix(tag) = tag * an odd constant (a bijection: two launches never share a
// mix).  A reader accepts a slot only when it carries this launch's tag and
// a matching check, so it needs no counter to know that the data has landed,
// and a stale or torn read is simply read again.  A torn read mixes words
// of this launch's store and of an earlier one: with this launch's tag and
// check, an older a or b (not both) fails unless it equals the new one;
// with an older check, the launches' mixes differ and the check fails
// unless the older words' differences cancel them exactly.  The mix is
// computed once per launch (the tag is uniform), the check in two
// operations per slot.
__host__ __device__ inline uint32_t tag_mix(uint32_t tag) { return tag * 0x9E3779B1u; }

__host__ __device__ inline uint32_t slot_check(uint32_t a, uint32_t b, uint32_t mix) {
  return a ^ ((b << 13) | (b >> 19)) ^ mix;
}

__device__ __forceinline__ float4 make_slot(uint32_t a, uint32_t b, uint32_t tag) {
  return make_float4(bits_f32(a), bits_f32(b), bits_f32(tag),
                     bits_f32(slot_check(a, b, tag_mix(tag))));
}

// mix = tag_mix(tag), tag this launch's (uniform)
__device__ __forceinline__ bool slot_ok(float4 s, uint32_t tag, uint32_t mix) {
  return f32_bits(s.z) == tag && f32_bits(s.w) == slot_check(f32_bits(s.x), f32_bits(s.y), mix);
}

constexpr int kChunks = (int)(kStepMaxTiles / kWave);  // tiles per lane, at most

// Where the one-launch step keeps what the separate kernels pass through
// the workspace: the tile's (z, delta, A, th) in LDS and the LSE partials in
// tagged slots (two per row and tile: (zm, zl) and (cm, cl)).
struct StepStats {
  const float4 (*zs)[kTile];  // [row][block of the tile]
  Coherent slots;             // (H*G, tile_stride, 2) tagged slots
  const uint32_t* tag;        // LDS: this launch's tag (what the workgroup publishes)
  const uint32_t* rtag;       // LDS: the tag its waits accept (the same, unless a test skews it)
  uint32_t* error;
  uint32_t spin;              // polls before a wait gives up
  unsigned long long* stamps;  // LDS phase stamps (RKV_PHASE_STAMPS build) or null
  uint32_t* gave_up;          // LDS: nonzero once a wait of this workgroup gave up
};

// A wait of the one-launch step gave up: the sticky error bit, and the
// workgroup's own flag, which makes its attention partial NaN (so the
// head's merged output is NaN and its mergers mark every block expanded).
// (lane 0 only; a rare path)
__device__ __forceinline__ void handoff_gave_up(const StepStats& ss) {
  __hip_atomic_fetch_or(ss.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (ss.gave_up != nullptr) *ss.gave_up = 1u;
}

// One row's LSE partials of the head's T tiles (lane t holds tiles t + 64 k)
// from the tagged slots, read until every slot carries this launch's tag
// (at most ss.spin rounds; then the wait is recorded as given up and the
// partials come back NaN, so log Z and log C are not finite and the
// decision's fail-safe expands every block).  With one tile per lane (T <=
// 64) the polls after the first keep two reads of the missing slots in
// flight: a poll that returns incomplete is reissued at once while the
// other is still out, so a slot that lands is seen sooner than with one
// round trip at a time.
struct RowLse {
  float zm[kChunks], zl[kChunks], cm[kChunks], cl[kChunks];
};

__device__ __forceinline__ RowLse gather_lse(const StepStats& ss, int64_t row, uint32_t T,
                                             int lane) {
  RowLse r;
  const uint32_t tag = __builtin_amdgcn_readfirstlane(*ss.rtag), mix = tag_mix(tag);
  // bit k: tile k * 64 + lane exists and its slots have not landed yet (a
  // poll reloads only those: the slots read past the caches)
  uint32_t need = 0;
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    r.zm[k] = r.cm[k] = kNegInf;
    r.zl[k] = r.cl[k] = 0.0f;
    if ((uint32_t)(k * kWave + lane) < T) need |= 1u << k;
  }
  if (T <= (uint32_t)kWave) {
    const uint32_t at = (uint32_t)((row + (uint32_t)lane) * 2) * 16u;
    bool miss = need != 0u;
    auto take = [&](float4 a, float4 b) {
      if (miss && slot_ok(a, tag, mix) && slot_ok(b, tag, mix)) {
        miss = false;
        r.zm[0] = a.x;
        r.zl[0] = a.y;
        r.cm[0] = b.x;
        r.cl[0] = b.y;
      }
    };
    float4 a0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b0 = a0, a1 = a0, b1 = a0;
    if (miss) {
      a0 = ss.slots.load4(at);
      b0 = ss.slots.load4(at + 16u);
    }
    take(a0, b0);
    if (__ballot(miss) == 0) return r;
    if (miss) {
      a0 = ss.slots.load4(at);
      b0 = ss.slots.load4(at + 16u);
    }
    __builtin_amdgcn_s_sleep(8);
    if (miss) {
      a1 = ss.slots.load4(at);
      b1 = ss.slots.load4(at + 16u);
    }
    for (uint32_t n = 3;; n += 2) {
      take(a0, b0);
      if (__ballot(miss) == 0) break;
      if (n >= ss.spin) {
        if (lane == 0) handoff_gave_up(ss);
        r.zm[0] = r.cm[0] = bits_f32(0x7FC00000u);
        break;
      }
      if (miss) {
        a0 = ss.slots.load4(at);
        b0 = ss.slots.load4(at + 16u);
      }
      take(a1, b1);
      if (__ballot(miss) == 0) break;
      if (miss) {
        a1 = ss.slots.load4(at);
        b1 = ss.slots.load4(at + 16u);
      }
    }
    return r;
  }
  for (uint32_t n = 0;; ++n) {
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
      if (k * kWave < (int)T && ((need >> k) & 1u)) {
        const uint32_t at = (uint32_t)((row + (uint32_t)(k * kWave + lane)) * 2);
        const float4 a = ss.slots.load4(at * 16);
        const float4 b = ss.slots.load4(at * 16 + 16);
        if (slot_ok(a, tag, mix) && slot_ok(b, tag, mix)) {
          need &= ~(1u << k);
          r.zm[k] = a.x;
          r.zl[k] = a.y;
          r.cm[k] = b.x;
          r.cl[k] = b.y;
        }
      }
    }
    if (__ballot(need != 0u) == 0) break;
    if (n + 1 >= ss.spin) {
      if (lane == 0) handoff_gave_up(ss);
      const float nan = bits_f32(0x7FC00000u);
#pragma unroll
      for (int k = 0; k < kChunks; ++k) r.zm[k] = r.cm[k] = nan;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
  return r;
}

// merge_lse over partials held per lane (tiles lane + 64 k; tiles past T
// hold m = -inf, l = 0): the same fixed order.
__device__ __forceinline__ float merge_lse_chunks(const float (&m)[kChunks],
                                                  const float (&l)[kChunks], uint32_t T,
                                                  int lane) {
  float mx = m[0];
#pragma unroll
  for (int k = 1; k < kChunks; ++k) mx = nanmax(mx, m[k]);
  mx = wave_nanmax_u(mx);
  const float ms = inf_to_zero(mx);
  float acc = (uint32_t)lane < T ? l[0] * exp_hw(m[0] - ms) : 0.0f;
#pragma unroll
  for (int k = 1; k < kChunks; ++k)
    if ((uint32_t)(k * kWave + lane) < T) acc = acc + l[k] * exp_hw(m[k] - ms);
  return log_hw(wave_sum_u(acc)) + ms;
}

// Both merges of one row (z and c): for T <= 64 (one tile per lane) a single
// branch-free block, so that the two independent chains interleave; the same
// operations as merge_lse_chunks, whose chunks past the first then hold
// m = -inf, l = 0 and change nothing.
__device__ __forceinline__ float2 merge_lse_pair(const RowLse& r, uint32_t T, int lane) {
  if (T > (uint32_t)kWave)
    return make_float2(merge_lse_chunks(r.zm, r.zl, T, lane),
                       merge_lse_chunks(r.cm, r.cl, T, lane));
  const float sz = inf_to_zero(wave_nanmax_u(r.zm[0]));
  const float sc = inf_to_zero(wave_nanmax_u(r.cm[0]));
  const bool live = (uint32_t)lane < T;
  const float az = live ? r.zl[0] * exp_hw(r.zm[0] - sz) : 0.0f;
  const float ac = live ? r.cl[0] * exp_hw(r.cm[0] - sc) : 0.0f;
  return make_float2(log_hw(wave_sum_u(az)) + sz, log_hw(wave_sum_u(ac)) + sc);
}

// Two rows' LSE partials (row1 only when has1) of a head with T <= 64
// tiles, polled together until every slot carries this launch's tag, so a
// wave that owns two rows waits one round trip, not two; each row as
// gather_lse returns it (at most ss.spin rounds, then recorded as given up
// with NaN partials).
__device__ __forceinline__ void gather_lse2(const StepStats& ss, int64_t row0, int64_t row1,
                                            bool has1, uint32_t T, int lane, RowLse& r0,
                                            RowLse& r1) {
  const uint32_t tag = __builtin_amdgcn_readfirstlane(*ss.rtag), mix = tag_mix(tag);
#pragma unroll
  for (int k = 0; k < kChunks; ++k) {
    r0.zm[k] = r0.cm[k] = r1.zm[k] = r1.cm[k] = kNegInf;
    r0.zl[k] = r0.cl[k] = r1.zl[k] = r1.cl[k] = 0.0f;
  }
  uint32_t miss = (uint32_t)lane < T ? (has1 ? 3u : 1u) : 0u;
  const uint32_t at0 = (uint32_t)((row0 + (uint32_t)lane) * 2) * 16u;
  const uint32_t at1 = (uint32_t)((row1 + (uint32_t)lane) * 2) * 16u;
  float4 a0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), b0 = a0, a1 = a0, b1 = a0;
#pragma unroll 1
  for (uint32_t n = 0;; ++n) {
    if (miss & 1u) {
      a0 = ss.slots.load4(at0);
      b0 = ss.slots.load4(at0 + 16u);
    }
    if (miss & 2u) {
      a1 = ss.slots.load4(at1);
      b1 = ss.slots.load4(at1 + 16u);
    }
    if ((miss & 1u) && slot_ok(a0, tag, mix) && slot_ok(b0, tag, mix)) {
      miss &= ~1u;
      r0.zm[0] = a0.x;
      r0.zl[0] = a0.y;
      r0.cm[0] = b0.x;
      r0.cl[0] = b0.y;
    }
    if ((miss & 2u) && slot_ok(a1, tag, mix) && slot_ok(b1, tag, mix)) {
      miss &= ~2u;
      r1.zm[0] = a1.x;
      r1.zl[0] = a1.y;
      r1.cm[0] = b1.x;
      r1.cl[0] = b1.y;
    }
    if (__ballot(miss != 0u) == 0) break;
    if (n + 1 >= ss.spin) {
      if (lane == 0) handoff_gave_up(ss);
      r0.zm[0] = r0.cm[0] = r1.zm[0] = r1.cm[0] = bits_f32(0x7FC00000u);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

// Access count of a tile with expanded blocks `bits` (transformers.py:590-594):
// the count of an expanded block, 1 for a representative; only the prompt's
// last block can be short.
__device__ __forceinline__ uint32_t tile_access_count(const DecideArgs& a, int64_t tile,
                                                      uint64_t bits) {
  const int64_t N = a.n_blocks, T = a.n_tiles;
  const int64_t nvalid = N - tile * kTile < kTile ? N - tile * kTile : kTile;
  const int64_t nsel = __popcll(bits);
  int64_t c = (nvalid - nsel) + nsel * a.block;
  if (tile == T - 1 && ((bits >> (N - 1 - tile * kTile)) & 1ull))
    c -= a.block - (a.length - (N - 1) * a.block);
  return (uint32_t)c;
}

// kMask = false leaves the mask store to the caller (the attention stores it
// after its loads are issued).
// kMaxG: the most query rows the caller's group can have (above four, a
// wave owns more than one row).
template <bool kFused = false, bool kMask = true, int kMaxG = kMaxGroup>
__device__ __forceinline__ uint64_t decide_finish(const DecideArgs& a, int64_t h, int64_t tile,
                                                  const DecideLoads& in, DecideShared& sh,
                                                  float (*zsh)[kTile], const int32_t*& list,
                                                  uint32_t& count,
                                                  const StepStats* ss = nullptr,
                                                  int64_t rh = -1) {
  if (rh < 0) rh = h;
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
  const int G = a.group;
  const int64_t N = a.n_blocks, T = a.n_tiles;
  const int64_t b = tile * kTile + lane;
  const bool valid = b < N;
  const bool owner = blockIdx.z == 0;  // row passes beyond the first repeat the decision
  const int64_t bc = valid ? b : N - 1;
  const int tl = lane < T ? lane : 0;
  const float vmax = a.max_value_norm[h];
  const float vnorm = valid ? in.vnorm : 0.0f;
  const bool anchored = valid && a.anchor != nullptr && in.anc != 0;

  // ---- log Z, log C of each row this wave owns, then its risks ----------
  uint64_t wsel = 0;
  bool wbad = false;
  auto row_tail = [&](int g, float lz, float lc, float4 zf) {
    if (a.stats_out && owner && tile == 0 && lane == 0) {
      a.stats_out[(rh * G + g) * 2] = lz;
      a.stats_out[(rh * G + g) * 2 + 1] = lc;
    }
    wbad |= !is_finite(lz) || !is_finite(lc);
    float r = 0.0f;
    if (valid) {
      r = risk_from(zf.x, zf.y, zf.z, zf.w, lz, lc, vmax, vnorm);
      if (a.risk_out && owner) a.risk_out[(rh * G + g) * N + b] = r;
    }
    wsel |= __ballot(valid && (r > a.eps || !is_finite(r)));
    sh.risk[g][lane] = r;
    if (zsh) zsh[g][lane] = valid ? zf.x : kNegInf;
  };
  if constexpr (kFused) {
    // every row from the head's tagged slots (read until all have landed);
    // a wave owning two rows (groups of 5 to 8, T <= 64) polls both at once
    bool two = false;
    if constexpr (kMaxG > kWaves) two = G > kWaves && G <= 2 * kWaves && T <= kWave;
    if (two) {
      const bool has1 = wave + kWaves < G;
      RowLse r0, r1;
      gather_lse2(*ss, (h * G + wave) * a.tile_stride, (h * G + wave + kWaves) * a.tile_stride,
                  has1, (uint32_t)T, lane, r0, r1);
      RKV_STAMP(ss->stamps, kStGather, wave == 0 && lane == 0);
      const float2 l0 = merge_lse_pair(r0, (uint32_t)T, lane);
      row_tail(wave, l0.x, l0.y, ss->zs[wave][lane]);
      if (has1) {
        const float2 l1 = merge_lse_pair(r1, (uint32_t)T, lane);
        row_tail(wave + kWaves, l1.x, l1.y, ss->zs[wave + kWaves][lane]);
      }
    }
#pragma unroll 1
    for (int g = wave; g < G && !two; g += kWaves) {
      const RowLse rl = gather_lse(*ss, (h * G + g) * a.tile_stride, (uint32_t)T, lane);
      RKV_STAMP(ss->stamps, kStGather, g == 0 && lane == 0);
      const float2 lzc = merge_lse_pair(rl, (uint32_t)T, lane);
      row_tail(g, lzc.x, lzc.y, ss->zs[g][lane]);
    }
  } else {
    auto row_stats = [&](int g, float4 part, float4 zf) {
      if (a.row_lse != nullptr) {
        // (merged once per row by lse_merge_kernel, in this same order)
        row_tail(g, a.row_lse[(rh * G + g) * 2], a.row_lse[(rh * G + g) * 2 + 1], zf);
        return;
      }
      const float* prow = a.lse + (rh * G + g) * a.tile_stride * 4;
      if (lane >= T) part = make_float4(kNegInf, 0.0f, kNegInf, 0.0f);
      auto pz = [&](int64_t t) { return make_float2(prow[t * 4], prow[t * 4 + 1]); };
      auto pc = [&](int64_t t) { return make_float2(prow[t * 4 + 2], prow[t * 4 + 3]); };
      row_tail(g, merge_lse(part.x, part.y, pz, T, lane), merge_lse(part.z, part.w, pc, T, lane),
               zf);
    };
    // the first row from the loads already made, further rows (groups above
    // four) with their own loads
    if (wave < G) row_stats(wave, in.part, in.zf);
#pragma unroll 1
    for (int g = wave + kWaves; g < G; g += kWaves) {
      const int64_t at = (rh * G + g) * a.tile_stride + tl;
      row_stats(g, *reinterpret_cast<const float4*>(a.lse + at * 4),
                a.zf[(rh * G + g) * a.z_stride + bc]);
    }
  }
  if (lane == 0) {
    sh.wsel[wave] = wsel;
    sh.wbad[wave] = wbad ? 1u : 0u;
  }
  __syncthreads();

  // ---- GQA reduction, fail-safes, anchors: every wave computes the same ---
  bool sel;
  if (a.reduction == kMean) {
    float acc = sh.risk[0][lane];
    bool bad_local = !is_finite(acc);
    for (int g = 1; g < G; ++g) {
      const float r = sh.risk[g][lane];
      acc = acc + r;
      bad_local |= !is_finite(r);
    }
    sel = (acc / (float)G) > a.eps || bad_local;
  } else {
    sel = (((sh.wsel[0] | sh.wsel[1]) | (sh.wsel[2] | sh.wsel[3])) >> lane) & 1ull;
  }
  const bool bad_global = (sh.wbad[0] | sh.wbad[1] | sh.wbad[2] | sh.wbad[3]) != 0;
  sel = (sel || bad_global || anchored) && valid;
  const uint64_t bits = __ballot(sel);
  if (sel) {
    const uint32_t below = __builtin_amdgcn_mbcnt_hi(
        (uint32_t)(bits >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bits, 0u));
    sh.list[wave][below] = lane;  // this wave's copy: its LDS writes precede its reads
  }
  list = sh.list[wave];
  if (wave == 0) {
    if (kMask && valid && owner && a.write_mask) a.mask[h * N + b] = sel ? 1 : 0;
    count = tile_access_count(a, tile, bits);
  }
  return bits;
}

// The tiles a one-launch step workgroup scores when its head has more tiles
// than workgroups (kTiles > 1, four-row passes: one row per wave): tiles
// wk + m W for m < n, each with this thread's decision inputs (block lane of
// the tile), this lane's (z, delta, A, th) of its wave's row, and the
// tile's z row in LDS (the logits of its representative chunk).
template <int kTiles, int GBM>
struct TileSet {
  uint32_t n;
  DecideLoads din[kTiles];
  float4 zown[kTiles];
  float (*z)[GBM][kTile];  // LDS: [m][row][block]
};

// The decisions of a workgroup's tiles (one-launch step, kTiles > 1): each
// wave's row's log Z / log C from the head's tagged slots once, then, tile
// by tile, decide_finish's risk, reduction, fail-safes, anchors, mask and
// access count (summed into count, thread 0).  bits[m]: tile m's expanded
// blocks, uniform over the workgroup (the caller stores the masks).
template <int kTiles, int GBM>
__device__ __forceinline__ void decide_tiles(const DecideArgs& a, int64_t h, uint32_t wk,
                                             uint32_t W, const TileSet<kTiles, GBM>& ts,
                                             DecideShared& sh, const StepStats& ss,
                                             uint64_t (&bits)[kTiles], uint32_t& count) {
  const int tid = threadIdx.x, lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform
  const int G = a.group;
  const int64_t N = a.n_blocks, T = a.n_tiles;
  const float vmax = a.max_value_norm[h];
  float lz = 0.0f, lc = 0.0f;
  bool bad = false;
  if (wave < G) {
    const RowLse rl = gather_lse(ss, (h * G + wave) * a.tile_stride, (uint32_t)T, lane);
    RKV_STAMP(ss.stamps, kStGather, wave == 0 && lane == 0);
    const float2 lzc = merge_lse_pair(rl, (uint32_t)T, lane);
    lz = lzc.x;
    lc = lzc.y;
    if (a.stats_out && wk == 0 && lane == 0) {
      a.stats_out[(h * G + wave) * 2] = lz;
      a.stats_out[(h * G + wave) * 2 + 1] = lc;
    }
    bad = !is_finite(lz) || !is_finite(lc);
  }
  count = 0;
#pragma unroll
  for (int m = 0; m < kTiles; ++m) {
    bits[m] = 0;
    if ((uint32_t)m >= ts.n) continue;
    const int64_t tile = wk + (int64_t)m * W;
    const int64_t b = tile * kTile + lane;
    const bool valid = b < N;
    const DecideLoads& in = ts.din[m];
    uint64_t wsel = 0;
    if (wave < G) {
      float r = 0.0f;
      if (valid) {
        const float4 zf = ts.zown[m];
        r = risk_from(zf.x, zf.y, zf.z, zf.w, lz, lc, vmax, in.vnorm);
        if (a.risk_out) a.risk_out[(h * G + wave) * N + b] = r;
      }
      wsel = __ballot(valid && (r > a.eps || !is_finite(r)));
      if (a.reduction == kMean) sh.risk[wave][lane] = r;
    }
    if (lane == 0) {
      sh.wsel[wave] = wsel;
      sh.wbad[wave] = bad ? 1u : 0u;
    }
    __syncthreads();
    bool sel;
    if (a.reduction == kMean) {
      float acc = sh.risk[0][lane];
      bool bad_local = !is_finite(acc);
      for (int g = 1; g < G; ++g) {
        const float r = sh.risk[g][lane];
        acc = acc + r;
        bad_local |= !is_finite(r);
      }
      sel = (acc / (float)G) > a.eps || bad_local;
    } else {
      sel = (((sh.wsel[0] | sh.wsel[1]) | (sh.wsel[2] | sh.wsel[3])) >> lane) & 1ull;
    }
    const bool bad_global = (sh.wbad[0] | sh.wbad[1] | sh.wbad[2] | sh.wbad[3]) != 0;
    const bool anchored = valid && a.anchor != nullptr && in.anc != 0;
    sel = (sel || bad_global || anchored) && valid;
    bits[m] = __ballot(sel);
    if (tid == 0) sh.tile_bits[m] = bits[m];
    if (wave == 0) count += tile_access_count(a, tile, bits[m]);
    __syncthreads();  // (sh is written again for the next tile)
  }
}

// rkv_select's second kernel: decisions only.
__global__ __launch_bounds__(kThreads) void decide_kernel(DecideArgs a,
                                                          unsigned long long* accessed) {
  __shared__ DecideShared sh;
  const int32_t* list;
  uint32_t count = 0;
  const DecideLoads in = decide_issue(a, blockIdx.y, blockIdx.x);
  decide_finish(a, blockIdx.y, blockIdx.x, in, sh, nullptr, list, count);
  if (accessed && threadIdx.x == 0) atomicAdd(accessed, (unsigned long long)count);
}

// log Z and log C of every row from its tiles' partials, once per row, in
// decide_finish's order (merge_lse over the lane partials), for heads of more
// than 64 tiles: each tile's decision then reads two floats instead of
// merging every tile's partials again.  Wave w of workgroup b takes row
// 4 b + w.
constexpr int kLseBatch = 8;  // partials per lane beyond its first loaded at once

__global__ __launch_bounds__(kThreads) void lse_merge_kernel(const float* lse, float* row_lse,
                                                             int64_t rows, int64_t n_tiles,
                                                             int64_t tile_stride) {
  const int lane = threadIdx.x % kWave;
  const int64_t r = (int64_t)blockIdx.x * kWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (r >= rows) return;
  const float* prow = lse + r * tile_stride * 4;
  const int tl = lane < n_tiles ? lane : 0;
  float4 part = *reinterpret_cast<const float4*>(prow + tl * 4);
  if (lane >= n_tiles) part = make_float4(kNegInf, 0.0f, kNegInf, 0.0f);
  float lz, lc;
  if (n_tiles <= kWave * (1 + kLseBatch)) {
    // every partial of this lane loaded at once (one round trip), then
    // merge_lse's operations in its order, the z and c chains side by side
    float4 pv[kLseBatch];
#pragma unroll
    for (int k = 0; k < kLseBatch; ++k) {
      const int64_t t = lane + (int64_t)kWave * (k + 1);
      pv[k] = t < n_tiles ? *reinterpret_cast<const float4*>(prow + t * 4)
                          : make_float4(kNegInf, 0.0f, kNegInf, 0.0f);
    }
    float mz = lane < n_tiles ? part.x : kNegInf, mc = lane < n_tiles ? part.z : kNegInf;
#pragma unroll
    for (int k = 0; k < kLseBatch; ++k) {
      if (lane + (int64_t)kWave * (k + 1) < n_tiles) {
        mz = nanmax(mz, pv[k].x);
        mc = nanmax(mc, pv[k].z);
      }
    }
    const float sz = inf_to_zero(wave_nanmax_u(mz)), sc = inf_to_zero(wave_nanmax_u(mc));
    float az = lane < n_tiles ? part.y * exp_hw(part.x - sz) : 0.0f;
    float ac = lane < n_tiles ? part.w * exp_hw(part.z - sc) : 0.0f;
#pragma unroll
    for (int k = 0; k < kLseBatch; ++k) {
      if (lane + (int64_t)kWave * (k + 1) < n_tiles) {
        az = az + pv[k].y * exp_hw(pv[k].x - sz);
        ac = ac + pv[k].w * exp_hw(pv[k].z - sc);
      }
    }
    lz = log_hw(wave_sum_u(az)) + sz;
    lc = log_hw(wave_sum_u(ac)) + sc;
  } else {
    auto pz = [&](int64_t t) { return make_float2(prow[t * 4], prow[t * 4 + 1]); };
    auto pc = [&](int64_t t) { return make_float2(prow[t * 4 + 2], prow[t * 4 + 3]); };
    lz = merge_lse(part.x, part.y, pz, n_tiles, lane);
    lc = merge_lse(part.z, part.w, pc, n_tiles, lane);
  }
  if (lane == 0) {
    row_lse[r * 2] = lz;
    row_lse[r * 2 + 1] = lc;
  }
}

// Batched anchor selection: the union over `anchors` queries of their
// decisions, for tile (blockIdx.x) of head h (blockIdx.y); query q's rows are
// those of head q H + h.  The OR of the tiles' ballots is stored once.
__global__ __launch_bounds__(kThreads) void anchor_decide_kernel(DecideArgs a, int anchors,
                                                                 int heads, uint8_t* mask_out) {
  __shared__ DecideShared sh;
  const int64_t h = blockIdx.y, tile = blockIdx.x;
  uint64_t any = 0;
  for (int q = 0; q < anchors; ++q) {
    const int64_t rh = (int64_t)q * heads + h;
    const DecideLoads in = decide_issue(a, h, tile, rh);
    const int32_t* list;
    uint32_t count = 0;
    any |= decide_finish(a, h, tile, in, sh, nullptr, list, count, nullptr, rh);
    __syncthreads();  // the next query reuses sh
  }
  const int lane = threadIdx.x % kWave;
  const int64_t b = tile * kTile + lane;
  if (threadIdx.x < kWave && b < a.n_blocks) mask_out[h * a.n_blocks + b] = (any >> lane) & 1u;
}

// ---------------------------------------------------------------------------
// Kernel 2: decisions + mixed attention of one (tile, head)
// ---------------------------------------------------------------------------
struct AttendArgs {
  DecideArgs decide;
  const uint16_t* query;        // (H, G, D) bf16
  const uint16_t* value_mean;   // (H, N, D) bf16
  const uint16_t* key_pages;    // head h at key_pages + h * kp_hs; rows (N*B, D)
  const uint16_t* value_pages;
  const uint16_t* key_suffix;   // token t of head h at h * ks_hs + t * ks_ts
  const uint16_t* value_suffix;
  const int32_t* suffix_len_dev;  // or null
  float2* part_ml;              // (H*G, tile_stride): m, l
  float* part_acc;              // (H*G, tile_stride, D)
  uint32_t* tile_counts;        // (H, tile_stride) or null
  int64_t kp_hs, vp_hs, ks_hs, ks_ts, vs_hs, vs_ts;
  int64_t suffix_cap;
  int log2_block;  // block_size is 16, 32 or 64
  int workers;     // workgroups per head (gridDim.x): n_tiles, or the step's step_workers
  float scale;
};

constexpr int kRowBatch = 2;  // token rows per lane group per batch

// Online-softmax state of GBM query rows held by one 16-lane group: m and l
// (uniform over the group) and acc, this lane's D/16 columns.
template <int D, int GBM>
struct GroupState {
  float m[GBM], l[GBM], acc[GBM][D / 16];
};

// Folds R rows (logits x[g][u], values v[u]) into the group's state with one
// rescale per row of the query.  Rows with x = -inf contribute nothing.
template <int D, int GBM, int R>
__device__ __forceinline__ void fold(GroupState<D, GBM>& st, const float (&x)[GBM][R],
                                     const float (&v)[R][D / 16], int gn) {
  constexpr int CH = D / 16;
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    if (g >= gn) break;
    float mx = x[g][0];
#pragma unroll
    for (int u = 1; u < R; ++u) mx = fmaxf(mx, x[g][u]);
    const float mn = fmaxf(st.m[g], mx);
    if (mn == kNegInf) continue;
    const float sc = __builtin_amdgcn_exp2f((st.m[g] - mn) * kLog2e);
    st.l[g] = st.l[g] * sc;
#pragma unroll
    for (int i = 0; i < CH; ++i) st.acc[g][i] = st.acc[g][i] * sc;
    st.m[g] = mn;
#pragma unroll
    for (int u = 0; u < R; ++u) {
      const float p = __builtin_amdgcn_exp2f((x[g][u] - mn) * kLog2e);
      st.l[g] = st.l[g] + p;
#pragma unroll
      for (int i = 0; i < CH; ++i) st.acc[g][i] = __builtin_fmaf(p, v[u][i], st.acc[g][i]);
    }
  }
}

// Logits of R token rows (K raw, this lane's slice) for GBM query rows, then
// the fold.  Row u is live when bit u of ok is set.  The dot products take
// the bf16 pairs as they are, with v_dot2_f32_bf16: this is the
// tolerance-checked attention, not the selection.
typedef __bf16 Bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(Bf16x2, a),
                                         __builtin_bit_cast(Bf16x2, b), c, false);
}

template <int D, int GBM, int R = kRowBatch>
__device__ __forceinline__ void fold_tokens(GroupState<D, GBM>& st,
                                            const RawBf16<D / 16> (&q)[GBM],
                                            const RawBf16<D / 16> (&kr)[R],
                                            const RawBf16<D / 16> (&vr)[R], uint32_t ok,
                                            float scale, int gn) {
  constexpr int CH = D / 16;
  float x[GBM][R], v[R][CH];
#pragma unroll
  for (int u = 0; u < R; ++u) {
    const bool live = (ok >> u) & 1u;
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      float s = dot2_bf16(q[g].w[0], kr[u].w[0], 0.0f);
#pragma unroll
      for (int i = 1; i < CH / 2; ++i) s = dot2_bf16(q[g].w[i], kr[u].w[i], s);
      s = row16_sum_all(s);
      x[g][u] = live ? s * scale : kNegInf;
    }
    unpack(vr[u], v[u]);
#pragma unroll
    for (int i = 0; i < CH; ++i) v[u][i] = live ? v[u][i] : 0.0f;
  }
  fold<D, GBM, R>(st, x, v, gn);
}

// ---------------------------------------------------------------------------
// Page rows on the matrix cores
// ---------------------------------------------------------------------------
// A wave attends 16-token chunks of page rows with MFMA.  QK^T:
// v_mfma_f32_16x16x32_bf16 with A = the chunk's key rows straight from
// memory (lane l: row l % 16, columns 8 (l / 16) + 32 s .. +7, 16 bytes) and
// B = the query rows (lane l: row g = l % 16, the same columns; zero past
// the pass's rows) gives S[t][g] in lane l for t = 4 (l / 16) + i, i = 0..3,
// g = l % 16.  The online softmax works on those values in place, and PV,
// v_mfma_f32_16x16x16_bf16, takes them unchanged as its A operand (lane l:
// P[g = l % 16][t = 4 (l / 16) + j]); its B operand (lane l: V[t = 4 (l /
// 16) + j][d0 + l % 16]) is one transposing LDS read (ds_read_b64_tr_b16:
// within each 16 lanes, lane p addresses 4 values of row p / 4 at column
// 4 (p % 4) and receives column p of the 4 rows) of the chunk's value rows,
// which buffer-to-LDS loads stage per wave.  The output O[g][d0 + n] sits in
// lane (g / 4) * 16 + n, register g % 4, one 4-register accumulator per 16
// columns.  Logits use the same bf16 products as the oracle's fp64 softmax;
// the sums' order is the matrix core's (tolerance-checked attention); P
// enters as the sum of two bf16 parts.
typedef __bf16 Bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 Bf16x2v __attribute__((ext_vector_type(2)));
typedef short I16x4 __attribute__((ext_vector_type(4)));
typedef float F32x4 __attribute__((ext_vector_type(4)));
typedef float F32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t U32x2 __attribute__((ext_vector_type(2)));

constexpr int kMmaStages = 3;     // value-chunk buffers per wave: two chunks in flight
constexpr int kMmaMaxDim = 160;   // head dims whose page rows run on the matrix cores

template <int D>
struct MmaShape {
  static constexpr int kSteps = D / 32;             // QK MFMAs per chunk (32 columns each)
  static constexpr int kBlocks = D / 16;            // PV MFMAs per chunk (16 columns each)
  static constexpr int kNC = D / 8;                 // 16-byte pieces per row
  static constexpr int kChunkBytes = 16 * D * 2;    // one chunk of value rows
  static constexpr int kLdsLoads = kChunkBytes / 1024;  // wave-wide 16-byte LDS loads per chunk
  static constexpr int kOps = kSteps + kLdsLoads;   // memory ops one chunk issues
};

// A wave's staged value chunks: row t of a chunk holds its 16-byte piece c at
// position (c + 2 t) mod kNC, so the 16 rows a transposing read touches at
// one column start on different banks.
template <int D>
struct MmaStage {
  alignas(16) char bytes[kMmaStages][MmaShape<D>::kChunkBytes];
};

// A wave's attention state after its page rows, for the combine.
template <int D, int GBM>
struct MmaOut {
  float acc[GBM][D];
  float ml[GBM][2];
};

template <int D>
struct MmaState {
  F32x4 o[MmaShape<D>::kBlocks];  // O[4 (l / 16) + i][16 b + l % 16] in o[b][i]
  float m;                        // running max of row l % 16
  float lsum;                     // this lane's share of row l % 16's denominator
};

__device__ __forceinline__ Bf16x8 load_b128(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(Bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0));
}

// A buffer view of `bytes` bytes at `base`; both must be wave-uniform (they
// are read from the first lane, so the view lives in scalar registers and the
// loads through it need no per-lane descriptor loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_view(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)a);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32));
  void* p = reinterpret_cast<void*>(((uint64_t)hi << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(p, (short)0,
                                           (int)__builtin_amdgcn_readfirstlane(bytes), 0x00020000);
}

// Waits until at most N vector-memory operations of this wave are pending
// (the buffer-to-LDS loads of a chunk are among them; the compiler does not
// track their LDS results).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Issues one chunk: the K operands of its 16 rows (lane l: row l % 16,
// columns 8 (l / 16) + 32 s .. +7) and its 16 value rows into the staged
// layout at dst.  krow(t) / vrow(t): byte offsets of row t in kres / vres.
template <int D, typename KRow, typename VRow>
__device__ __forceinline__ void mma_issue_rows(__amdgpu_buffer_rsrc_t kres,
                                               __amdgpu_buffer_rsrc_t vres, char* dst,
                                               Bf16x8 (&kop)[MmaShape<D>::kSteps], KRow krow,
                                               VRow vrow) {
  using S = MmaShape<D>;
  constexpr uint32_t NC = S::kNC;
  typedef __attribute__((address_space(3))) void LdsVoid;
  const uint32_t lane = threadIdx.x % kWave;
  const uint32_t k_off = krow(lane & 15u) + (lane >> 4) * 16u;
#pragma unroll
  for (int s = 0; s < S::kSteps; ++s) kop[s] = load_b128(kres, k_off + 64u * s);
#pragma unroll
  for (int u = 0; u < S::kLdsLoads; ++u) {
    // staged position p = 64 u + l: row p / NC, position p % NC holds piece
    // (position - 2 row) mod NC of that row
    const uint32_t p = 64u * u + lane, t = p / NC;
    const uint32_t piece = (p % NC + 32u * NC - 2u * t) % NC;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vres, (LdsVoid*)(dst + 1024 * u), 16,
                                             (int)(vrow(t) + piece * 16u), 0, 0, 0);
  }
}

// QK^T of a chunk: S[t = 4 (l / 16) + i][g = l % 16] in lane l, register i.
template <int D>
__device__ __forceinline__ F32x4 mma_qk(const Bf16x8 (&kop)[MmaShape<D>::kSteps],
                                        const Bf16x8 (&qop)[MmaShape<D>::kSteps]) {
  F32x4 s4 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int s = 0; s < MmaShape<D>::kSteps; ++s)
    s4 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop[s], qop[s], s4, 0, 0, 0);
  return s4;
}

// Folds a chunk into the wave's state: x[i] is the logit of row t = 4 (l /
// 16) + i for query row l % 16 (-inf for rows that do not count), src the
// chunk's staged value rows.  Online softmax in place, then PV with P as a
// sum of two bf16 parts (relative error ~2^-17, where bf16 alone leaves
// 2^-9) against the same value rows.
// N transposing 64-bit LDS reads (ds_read_b64_tr_b16) of the staged value
// rows at LDS byte addresses at[], issued by one asm statement that does not
// wait for them; lds_ready<N, b>(v[b]) then waits until read b has landed.
// The compiler does not see these reads, so it adds no wait for the
// buffer-to-LDS loads still in flight (it cannot tell that they fill other
// stages, and such a wait would drain the ring's two chunks ahead); the
// ring's own vmcnt wait before each chunk orders that chunk's LDS writes
// before these reads.  Each wait names its register as an operand, so no use
// of v[b] is placed before it.  LDS operations return in issue order, and
// any other LDS or scalar-memory operation counted by lgkmcnt only makes a
// count stricter, so lgkmcnt(N - 1 - b) always covers reads 0..b.
template <int N>
__device__ __forceinline__ void lds_read_tr(I16x4 (&v)[N], const uint32_t (&at)[N]) {
  static_assert(N == 2 || N == 4 || N == 6 || N == 8, "2-8 reads");
  if constexpr (N == 2) {
    asm volatile("ds_read_b64_tr_b16 %0, %2\n\tds_read_b64_tr_b16 %1, %3"
                 : "=&v"(v[0]), "=&v"(v[1])
                 : "v"(at[0]), "v"(at[1])
                 : "memory");
  } else if constexpr (N == 4) {
    asm volatile("ds_read_b64_tr_b16 %0, %4\n\tds_read_b64_tr_b16 %1, %5\n\t"
                 "ds_read_b64_tr_b16 %2, %6\n\tds_read_b64_tr_b16 %3, %7"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
                 : "v"(at[0]), "v"(at[1]), "v"(at[2]), "v"(at[3])
                 : "memory");
  } else if constexpr (N == 6) {
    asm volatile("ds_read_b64_tr_b16 %0, %6\n\tds_read_b64_tr_b16 %1, %7\n\t"
                 "ds_read_b64_tr_b16 %2, %8\n\tds_read_b64_tr_b16 %3, %9\n\t"
                 "ds_read_b64_tr_b16 %4, %10\n\tds_read_b64_tr_b16 %5, %11"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5])
                 : "v"(at[0]), "v"(at[1]), "v"(at[2]), "v"(at[3]), "v"(at[4]), "v"(at[5])
                 : "memory");
  } else {
    asm volatile("ds_read_b64_tr_b16 %0, %8\n\tds_read_b64_tr_b16 %1, %9\n\t"
                 "ds_read_b64_tr_b16 %2, %10\n\tds_read_b64_tr_b16 %3, %11\n\t"
                 "ds_read_b64_tr_b16 %4, %12\n\tds_read_b64_tr_b16 %5, %13\n\t"
                 "ds_read_b64_tr_b16 %6, %14\n\tds_read_b64_tr_b16 %7, %15"
                 : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
                   "=&v"(v[6]), "=&v"(v[7])
                 : "v"(at[0]), "v"(at[1]), "v"(at[2]), "v"(at[3]), "v"(at[4]), "v"(at[5]),
                   "v"(at[6]), "v"(at[7])
                 : "memory");
  }
}

template <int N, int B>
__device__ __forceinline__ void lds_ready(I16x4& v) {
  constexpr int k = N - 1 - B;
  static_assert(k >= 0 && k <= 7, "count");
  if constexpr (k == 0) asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(v));
  else if constexpr (k == 1) asm volatile("s_waitcnt lgkmcnt(1)" : "+v"(v));
  else if constexpr (k == 2) asm volatile("s_waitcnt lgkmcnt(2)" : "+v"(v));
  else if constexpr (k == 3) asm volatile("s_waitcnt lgkmcnt(3)" : "+v"(v));
  else if constexpr (k == 4) asm volatile("s_waitcnt lgkmcnt(4)" : "+v"(v));
  else if constexpr (k == 5) asm volatile("s_waitcnt lgkmcnt(5)" : "+v"(v));
  else if constexpr (k == 6) asm volatile("s_waitcnt lgkmcnt(6)" : "+v"(v));
  else asm volatile("s_waitcnt lgkmcnt(7)" : "+v"(v));
}

// o[b] += p x v[b] for each b, each product after its read has landed and
// (the scheduling barrier) before the next read's wait
template <int N, int... B>
__device__ __forceinline__ void mfma_as_ready(F32x4 (&o)[N], I16x4 p, I16x4 (&v)[N],
                                              std::integer_sequence<int, B...>) {
  ((lds_ready<N, B>(v[B]), o[B] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(p, v[B], o[B], 0, 0, 0),
    __builtin_amdgcn_sched_barrier(0)),
   ...);
}

template <int D, bool kAsmReads = true>
__device__ __forceinline__ void mma_fold(MmaState<D>& st, const float (&x)[4], const char* src) {
  using S = MmaShape<D>;
  constexpr uint32_t NC = S::kNC;
  const int lane = threadIdx.x % kWave;
  float mx = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
  float a, b2;
  xor16_pair(mx, a, b2);
  mx = fmaxf(a, b2);
  xor32_pair(mx, a, b2);
  mx = fmaxf(a, b2);
  const float mn = fmaxf(st.m, mx);
  const float ms = mn == kNegInf ? 0.0f : mn;
  const float alpha = __builtin_amdgcn_exp2f((st.m - ms) * kLog2e);
  float p[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) p[i] = __builtin_amdgcn_exp2f((x[i] - ms) * kLog2e);
  st.lsum = __builtin_fmaf(st.lsum, alpha, (p[0] + p[1]) + (p[2] + p[3]));
  st.m = mn;
  if (__ballot(alpha != 1.0f) != 0) {
    // O's rows in this lane: 4 (l / 16) + i; their factors from lanes 0..15
    float ar[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) ar[i] = __shfl(alpha, 4 * (lane >> 4) + i, kWave);
#pragma unroll
    for (int b = 0; b < S::kBlocks; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) st.o[b][i] *= ar[i];
  }
  // (whole bf16 pairs as 32-bit words: extracting single bf16 elements of
  // the converted pairs miscompiles to a duplicated half)
  auto pack = [](float x0, float x1) {
    const F32x2 v = {x0, x1};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, Bf16x2v));
  };
  const uint32_t h01 = pack(p[0], p[1]), h23 = pack(p[2], p[3]);
  const U32x2 hw = {h01, h23};
  const U32x2 lw = {pack(p[0] - bits_f32(h01 << 16), p[1] - bits_f32(h01 & 0xFFFF0000u)),
                    pack(p[2] - bits_f32(h23 << 16), p[3] - bits_f32(h23 & 0xFFFF0000u))};
  const I16x4 ph = __builtin_bit_cast(I16x4, hw), pl = __builtin_bit_cast(I16x4, lw);
  // transposing reads: row 4 (l / 16) + (l % 16) / 4, column 16 b + 4 (l % 4)
  const uint32_t t_row = 4u * (uint32_t)(lane >> 4) + (uint32_t)((lane & 15) >> 2);
  const uint32_t base = t_row * (uint32_t)(D * 2) + (uint32_t)(lane & 1) * 8u;
  const uint32_t rot = ((uint32_t)(lane >> 1) & 1u) + 2u * t_row;
  I16x4 vb[S::kBlocks];
  if constexpr (D <= 128 && kAsmReads) {
    const uint32_t lds = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const char*)src;
    uint32_t at[S::kBlocks];
#pragma unroll
    for (int b = 0; b < S::kBlocks; ++b) at[b] = lds + base + ((2u * b + rot) % NC) * 16u;
    lds_read_tr<S::kBlocks>(vb, at);
    mfma_as_ready(st.o, ph, vb, std::make_integer_sequence<int, S::kBlocks>{});
  } else {
    // (head_dim 160: the ten addresses and outputs live at once would spill.
    // The representative and suffix ring takes the compiler's reads too: it
    // is short, so the compiler's wait for every buffer-to-LDS load costs
    // little there, and it measured faster than the asm reads.  The
    // compiler's reads keep that wait.)
#pragma unroll
    for (int b = 0; b < S::kBlocks; ++b) {
      vb[b] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          (__attribute__((address_space(3))) I16x4*)(src + base + ((2u * b + rot) % NC) * 16u));
      st.o[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(ph, vb[b], st.o[b], 0, 0, 0);
    }
  }
#pragma unroll
  for (int b = 0; b < S::kBlocks; ++b)
    st.o[b] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pl, vb[b], st.o[b], 0, 0, 0);
}

// Runs `count` chunks of one wave through three stages, two chunks in
// flight: issue(j, sidx, kop) issues chunk j (exactly MmaShape<D>::kOps
// memory operations, or none for a chunk whose loads carry no K operands)
// into stage sidx, compute(j, sidx, kop) folds it.  Chunk j uses stage j % 3
// and registers kj % 3; the first `pre` chunks (at most 3) were issued by
// the caller before the ring.  The stage index is a constant in each
// unrolled slot.
template <int D, typename Issue, typename Compute>
__device__ __forceinline__ void mma_ring(uint32_t count, uint32_t pre,
                                         Bf16x8 (&k0)[MmaShape<D>::kSteps],
                                         Bf16x8 (&k1)[MmaShape<D>::kSteps],
                                         Bf16x8 (&k2)[MmaShape<D>::kSteps], Issue issue,
                                         Compute compute) {
  using S = MmaShape<D>;
  if (count == 0) return;
  if (pre < 1) issue(0u, 0, k0);
  if (count > 1 && pre < 2) issue(1u, 1, k1);
  // chunk j's loads landed: at most the chunks issued after it are pending
  // (loads complete in order)
  auto wait_for = [&](uint32_t j) {
    const uint32_t ahead = count - 1 - j;
    if (ahead >= 2) wait_vm<2 * S::kOps>();
    else if (ahead == 1) wait_vm<S::kOps>();
    else wait_vm<0>();
  };
#pragma unroll 1
  for (uint32_t j = 0; j < count; j += 3) {
    if (j + 2 < count && (j > 0 || pre < 3)) issue(j + 2, 2, k2);
    wait_for(j);
    compute(j, 0, k0);
    if (j + 1 >= count) break;
    if (j + 3 < count) issue(j + 3, 0, k0);
    wait_for(j + 1);
    compute(j + 1, 1, k1);
    if (j + 2 >= count) break;
    if (j + 4 < count) issue(j + 4, 1, k1);
    wait_for(j + 2);
    compute(j + 2, 2, k2);
  }
}

// The pass's query rows g0 .. g0 + 15 (zero past min(GBM, G - g0)) as QK B
// operands: lane l holds row g0 + l % 16, columns 32 s + 8 (l / 16) .. +7.
template <int D, int GBM>
__device__ __forceinline__ void mma_query(Bf16x8 (&qop)[MmaShape<D>::kSteps],
                                          const uint16_t* q_head, int g0, int G) {
  const int lane = threadIdx.x % kWave;
  const int g = lane & 15;
  const bool live = g < GBM && g0 + g < G;
  const uint16_t* row = q_head + (live ? g0 + g : 0) * D + 8 * (lane >> 4);
#pragma unroll
  for (int s = 0; s < MmaShape<D>::kSteps; ++s) {
    const uint4 u = *reinterpret_cast<const uint4*>(row + 32 * s);
    const uint4 z = live ? u : make_uint4(0u, 0u, 0u, 0u);
    qop[s] = __builtin_bit_cast(Bf16x8, z);
  }
}

// A wave's state into its MmaOut: (m, l) of rows g < GBM (l summed over the
// four lanes of each row) and O's rows g < GBM.
template <int D, int GBM>
__device__ __forceinline__ void mma_publish(const MmaState<D>& st, MmaOut<D, GBM>& out) {
  const int lane = threadIdx.x % kWave;
  float a, b;
  xor16_pair(st.lsum, a, b);
  float l = a + b;
  xor32_pair(l, a, b);
  l = a + b;
  if (lane < GBM) {
    out.ml[lane][0] = st.m;
    out.ml[lane][1] = l;
  }
  const int q = lane >> 4, n = lane & 15;
#pragma unroll
  for (int b2 = 0; b2 < MmaShape<D>::kBlocks; ++b2)
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (4 * q + i < GBM) out.acc[4 * q + i][16 * b2 + n] = st.o[b2][i];
}

// Lane-group states are combined through LDS in chunks of rows small enough
// that 16 groups' accumulators fit in 32 KiB.  A lane's D/16 columns sit in
// a slice padded by 4 floats, so the 16-byte stores of a group's lanes fall
// on distinct banks.  (Head dims above kMmaMaxDim.)
template <int D, int GBM>
struct LaneCombine {
  static constexpr int kRows = (512 / D) < GBM ? (512 / D) : GBM;
  static constexpr int kSlice = D / 16 + 4;
  float acc[16][kRows][16 * kSlice];
  float ml[16][kRows][2];
};

// The matrix-core path's LDS: each wave's staged value chunks, then each
// wave's state for the combine.
template <int D, int GBM>
struct MmaCombine {
  MmaStage<D> stage[kWaves];
  MmaOut<D, GBM> mma[kWaves];
};

// The four waves' published states -> one (m, l, acc) per query row j < gn,
// in a fixed order: put(j, d, (acc[d], acc[d + 1]), m, l) for each column
// pair d of each row (after a barrier that follows every wave's publish).
template <int D, int GBM, typename Put>
__device__ __forceinline__ void mma_combine(const MmaCombine<D, GBM>& cmb, int gn, Put put) {
  for (int idx = 2 * (int)threadIdx.x; idx < gn * D; idx += 2 * kThreads) {
    const int j = idx / D, d = idx % D;
    float M = kNegInf;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, cmb.mma[w].ml[j][0]);
    float a0 = 0.0f, a1 = 0.0f, l = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float mw = cmb.mma[w].ml[j][0];
      const float e = mw == kNegInf ? 0.0f : __builtin_amdgcn_exp2f((mw - M) * kLog2e);
      const float2 av = *reinterpret_cast<const float2*>(&cmb.mma[w].acc[j][d]);
      a0 = __builtin_fmaf(av.x, e, a0);
      a1 = __builtin_fmaf(av.y, e, a1);
      l = __builtin_fmaf(cmb.mma[w].ml[j][1], e, l);
    }
    put(j, d, make_float2(a0, a1), M, l);
  }
}

// ---------------------------------------------------------------------------
// One-launch step: hand-off counters and the merge of a head by its last tile
// ---------------------------------------------------------------------------
// Hand-offs between the tiles of a head.  Counters (u64 at the start of
// the workspace): a 64-byte line per head (unused); after the heads' lines,
// a line holding a sticky u32 error
// word (bit 0: a wait gave up after its poll limit; the static-scratch entry
// point keeps its own word) and, at [1], the launches' workgroup ticket
// count; then one launch counter per workgroup.  Nothing is reset: each
// launch adds one to every workgroup's counter, so a workgroup's own counter
// (old value) is the launch's epoch e, and e + 1 tags the slots it publishes
// (LSE partials, attention partials, access counts: readers poll the slots
// themselves).
// Each workgroup also leaves e + 2 in its flag of the `full` region when
// launch e expanded every block of its tile (read by launch e + 1, which
// then speculates).  This needs the workspace zero-filled once when created
// and used for one shape thereafter.
//
// Progress: a workgroup waits only for the workgroups of its own head, and
// only after publishing what they wait for from it.  When the whole grid fits
// on the device at once, every workgroup a wait depends on is running.  A
// grid of up to two device-fulls (blocks of 64 tokens) takes its (head,
// workgroup) from a ticket drawn when it starts instead of from blockIdx:
// tickets are handed out in start order, so every head whose tickets are all
// drawn is entirely running, and at most one head (the one holding the
// latest ticket) is partly running; its workgroups wait for peers that start
// as the fully drawn heads finish, whatever order the hardware dispatches
// workgroups in.  A wait that does not end within its poll limit records an
// error instead of hanging.

struct StepCtx {
  StepStats stats;
  Coherent ml, acc, counts;       // tagged slots: partial (m, l), partial acc, tile counts
  Coherent mask;                  // (H, N) expanded-block mask (write-through stores)
  uint16_t* out;                  // (H, G, D) bf16
  unsigned long long* accessed;   // or null
  unsigned long long* wsum;       // kWaves LDS words
  uint64_t* full;                 // this workgroup's flag: the launch whose tile fully expanded
  const uint32_t* spec;           // LDS: nonzero when the launch speculates (or null)
};

// Folds state (m2, d2, (n2a, n2b)) into (mx, den, (na, nb)) in one
// branch-free form: an empty state (m = -inf, d = 0) weighs 0, and from the
// empty initial state the first fold copies exactly (fma(d2, 1, 0 x 0) =
// d2), so the result is that of skipping empty states and copying the
// first.
__device__ __forceinline__ void merge_state2(float m2, float d2, float n2a, float n2b, float& mx,
                                             float& den, float& na, float& nb) {
  const float M = fmaxf(mx, m2);
  const float ms = M == kNegInf ? 0.0f : M;
  const float ea = __builtin_amdgcn_exp2f((mx - ms) * kLog2e);
  const float eb = __builtin_amdgcn_exp2f((m2 - ms) * kLog2e);
  den = __builtin_fmaf(d2, eb, den * ea);
  na = __builtin_fmaf(n2a, eb, na * ea);
  nb = __builtin_fmaf(n2b, eb, nb * ea);
  mx = M;
}

// The merge of a head's partials.  Every workgroup publishes its partial as
// tagged slots (the LSE slots' format and tag): per query row one slot
// (m, l) and one per column pair (acc[2p], acc[2p + 1]), and one slot with
// its access count.  The head's last K = mergers(W, D) workgroups by index each
// merge a column slice: slice m covers pairs [m P / K, (m + 1) P / K) of
// every row (P = D / 2).  A merger polls the slots it needs until every one
// carries this launch's tag, reloading only those still missing, so after
// the head's slowest workgroup publishes, one round trip brings in what is
// left.  Each (row, pair) unit is merged by S adjacent lanes (S a power of
// two <= 16, so a unit sits inside a 16-lane row; partials s, s + S, ... in
// order, in batches of kMergeHeld per lane), then a tree over the S lanes
// into the unit's last lane (DPP row shifts): a fixed order, so outputs
// repeat bit for bit.  Slice 0 also adds the head's access count.
constexpr int kMergers = 8;
constexpr int kMergeHeld = 8;  // partials a lane holds per batch

// Mergers of a head of W workgroups at head_dim D: W / 4, at least 8, at
// most W and D / 2 (every slice keeps at least one column pair, so slice 0,
// which also counts and marks a failed hand-off, always has units).  Slices
// shrink as the partials to fold per slice grow: each merger's poll reloads
// fewer slots per round (at 64 workgroups per head 16 mergers measured
// 0.6 us faster per layer-step than 8, and 32 slower again; at 128, 32
// beat 16 and 64).
__host__ __device__ __forceinline__ uint32_t mergers(uint32_t W, uint32_t D) {
  uint32_t k = W / 4u > (uint32_t)kMergers ? W / 4u : (uint32_t)kMergers;
  if (k > D / 2u) k = D / 2u;
  return W < k ? W : k;
}

// Byte offsets of a partial's slots: (row r of the head, workgroup t) at
// ml_slot(r, t) in the ml region and at acc_slot(r, t, p) in the acc region.
__host__ __device__ __forceinline__ uint32_t ml_slot(int64_t row_ts, uint32_t t) {
  return (uint32_t)((row_ts + t) * 16);
}
template <int D>
__device__ __forceinline__ uint32_t acc_slot(int64_t row_ts, uint32_t t, uint32_t p) {
  return (uint32_t)(((row_ts + t) * (D / 2) + p) * 16);
}

// If a wait of the head gave up (that workgroup's partial carries NaN, which
// the fold carries into every unit) or this merger's own poll does, the
// slice is written as NaN and slice 0 marks every block of the head
// expanded.
template <int D>
__device__ void merge_slice(const AttendArgs& a, const StepCtx& sx, int64_t h, int m, int K) {
  unsigned long long* const stamps = sx.stats.stamps;
  (void)stamps;
  const DecideArgs& da = a.decide;
  const int G = da.group, W = a.workers;  // the head's partials: one per workgroup
  const int64_t ts = da.tile_stride;
  const int tid = threadIdx.x;
  constexpr int P = D / 2;
  const int p0 = m * P / K, np = (m + 1) * P / K - p0;
  const int units = G * np;
  int S = 1;
  while (S * 2 * units <= kThreads && S < 16) S *= 2;
  const uint32_t tag = __builtin_amdgcn_readfirstlane(*sx.stats.rtag), mix = tag_mix(tag);
  bool gave_up = false, poisoned = false;
  auto give_up = [&]() {
    if (!gave_up)
      __hip_atomic_fetch_or(sx.stats.error, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    gave_up = true;
  };
  // slice 0 also sums the access counts of the min(n_tiles, W) workgroups
  // that decide distinct tiles (at most kStepMaxTiles <= kThreads), one per
  // thread
  const bool counting = sx.accessed && m == 0;
  const int n_counts = (int)da.n_tiles < W ? (int)da.n_tiles : W;
  uint32_t tile_count = 0;
  if (counting && tid < n_counts) {
    for (uint32_t n = 0;; ++n) {
      const float4 c = sx.counts.load4((uint32_t)((h * ts + tid) * 16));
      if (slot_ok(c, tag, mix)) {
        tile_count = f32_bits(c.x);
        break;
      }
      if (n + 1 >= sx.stats.spin) {
        give_up();
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  for (int u0 = 0; u0 < units; u0 += kThreads / S) {
    const int u = u0 + tid / S, sl = tid % S;
    const int uc = u < units ? u : units - 1;
    const int g = uc / np, pp = p0 + uc % np;
    const int64_t row = (h * G + g) * ts;
    float mx = kNegInf, den = 0.0f, na = 0.0f, nb = 0.0f;
    for (int t0 = sl; t0 < W; t0 += S * kMergeHeld) {
      float4 ml[kMergeHeld], av[kMergeHeld];
      uint32_t need = 0;  // bit k: partial t0 + S k exists and has not landed
#pragma unroll
      for (int k = 0; k < kMergeHeld; ++k) {
        ml[k] = make_float4(kNegInf, 0.0f, 0.0f, 0.0f);
        av[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (t0 + S * k < W) need |= 1u << k;
      }
      for (uint32_t n = 0;; ++n) {
#pragma unroll
        for (int k = 0; k < kMergeHeld; ++k) {
          if ((need >> k) & 1u) {
            const uint32_t t = (uint32_t)(t0 + S * k);
            ml[k] = sx.ml.load4(ml_slot(row, t));
            av[k] = sx.acc.load4(acc_slot<D>(row, t, (uint32_t)pp));
          }
        }
#pragma unroll
        for (int k = 0; k < kMergeHeld; ++k)
          if (((need >> k) & 1u) && slot_ok(ml[k], tag, mix) && slot_ok(av[k], tag, mix))
            need &= ~(1u << k);
        if (__ballot(need != 0u) == 0) break;
        if (n + 1 >= sx.stats.spin) {
          give_up();
          break;
        }
        __builtin_amdgcn_s_sleep(2);
      }
#pragma unroll
      for (int k = 0; k < kMergeHeld; ++k)
        if (t0 + S * k < W) merge_state2(ml[k].x, ml[k].y, av[k].x, av[k].y, mx, den, na, nb);
    }
    RKV_STAMP(stamps, kStMergeLoaded, tid == 0);
    auto fold_from = [&](auto shift) {
      merge_state2(shift(mx), shift(den), shift(na), shift(nb), mx, den, na, nb);
    };
    if (S > 8) fold_from([](float v) { return row_shr<8>(v); });
    if (S > 4) fold_from([](float v) { return row_shr<4>(v); });
    if (S > 2) fold_from([](float v) { return row_shr<2>(v); });
    if (S > 1) fold_from([](float v) { return row_shr<1>(v); });
    RKV_STAMP(stamps, kStMergeFolded, tid == 0);
    if (u0 == 0) poisoned = __syncthreads_or(gave_up || !(den == den)) != 0;
    if (sl == S - 1 && u < units) {
      const float dn = fmaxf(den, 1e-30f);
      // a hand-off of the head gave up: its output is NaN, not a plausible
      // wrong answer
      const uint32_t v = poisoned || gave_up
                             ? 0x7FC07FC0u
                             : (uint32_t)bf16_rne(na / dn) | ((uint32_t)bf16_rne(nb / dn) << 16);
      *reinterpret_cast<uint32_t*>(sx.out + (h * G + g) * D + 2 * pp) = v;
    }
  }
  RKV_STAMP(stamps, kStMergeStored, tid == 0);
  if (poisoned && m == 0 && da.write_mask) {
    // (the workgroups' own mask stores wrote through before their partials,
    // so these come last)
    const int64_t N = da.n_blocks;
    for (int64_t b = tid; b < N; b += kThreads) sx.mask.store_u8((uint32_t)(h * N + b), 1u);
  }
  // the step's access count: this head's tile counts, added once
  if (counting) {
    unsigned long long c = tile_count;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) c += __shfl_xor(c, o, kWave);
    if (tid % kWave == 0) sx.wsum[tid / kWave] = c;
    __syncthreads();
    if (tid == 0)
      atomicAdd(sx.accessed, ((sx.wsum[0] + sx.wsum[1]) + sx.wsum[2]) + sx.wsum[3]);
    RKV_STAMP(stamps, kStMergeCounted, tid == 0);
  }
}

// The attention of one (tile, head) on the vector ALUs (the three-kernel
// form's attend kernel above head_dim 160, where the matrix-core engine's
// staging does not fit): 16 lane groups, two workgroups per CU.
//
// Order of work: every load that does not depend on the decision is issued
// first (the decision's inputs, the value means, z and the tile max of this
// lane group's representatives, one suffix row per lane group); the full
// representative sum over the tile is folded while the decision's inputs
// are in flight; after the decision the expanded blocks' representative
// terms are taken out again and the expanded blocks' tokens and the suffix
// rows are attended.
template <int D, int GBM>
struct AttendLoads {
  DecideLoads din;
  uint32_t S;                            // suffix length
  RawBf16<D / 16> vraw[kTile / 16];      // value means of the lane group's blocks
  RawBf16<D / 16> qraw[GBM];             // the pass's query rows
  RawBf16<D / 16> ksr[1], vsr[1];        // the lane group's first suffix token
};

// Workgroup wk of head h (blockIdx.x and blockIdx.y).
template <int D, int GBM>
__device__ __forceinline__ AttendLoads<D, GBM> attend_issue(const AttendArgs& a, int64_t h,
                                                            uint32_t wk) {
  constexpr int CH = D / 16;
  constexpr int NB = kTile / 16;
  const DecideArgs& da = a.decide;
  // workgroup wk of the head's W scores tile wk % T (copies past the first T)
  const uint32_t tile = wk % (uint32_t)da.n_tiles;
  const int G = da.group;
  const uint32_t N = (uint32_t)da.n_blocks;
  const uint32_t W = (uint32_t)a.workers;  // the suffix is sliced over the workgroups
  const int tid = threadIdx.x;
  const int lg = tid >> 4, c = tid & 15;
  const int g0 = blockIdx.z * GBM;
  AttendLoads<D, GBM> ld;
  ld.din = decide_issue<true>(da, h, tile);
  // The suffix length does not change during a launch: a scalar load from
  // the constant address space, outside the vector loads' in-order count.
  uint32_t S = (uint32_t)a.suffix_cap;
  if (a.suffix_len_dev) {
    typedef __attribute__((address_space(4))) const int32_t ConstI32;
    const int32_t sl = *(ConstI32*)(uintptr_t)a.suffix_len_dev;
    S = sl < 0 ? 0u : ((uint32_t)sl > S ? S : (uint32_t)sl);
  }
  ld.S = S;
  // value means of this lane group's blocks lg + 16 i
  const uint16_t* vm = a.value_mean + (h * N) * D + c * CH;
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    uint32_t b = tile * kTile + lg + 16 * i;
    b = b < N ? b : N - 1;
    ld.vraw[i] = load_raw<CH>(vm + b * D);
  }
  const uint16_t* qh = a.query + (h * G) * D + c * CH;
#pragma unroll
  for (int g = 0; g < GBM; ++g)
    ld.qraw[g] = load_raw<CH>(qh + (g0 + g < G ? g0 + g : G - 1) * D);
  // This workgroup's slice of the suffix: tokens wk, wk + W, ... (< S); the
  // first 16 of them, one per lane group, are prefetched here.
  const uint32_t n_suffix = S > wk ? (S - wk + W - 1) / W : 0u;
  const uint32_t n_pre = n_suffix < 16u ? n_suffix : 16u;
  const uint16_t* kbase = a.key_pages + h * a.kp_hs;
  const uint16_t* vbase = a.value_pages + h * a.vp_hs;
  const bool has = (uint32_t)lg < n_pre;
  const uint64_t t = has ? wk + (uint32_t)lg * W : 0u;
  ld.ksr[0] = load_raw<CH>((has ? a.key_suffix + h * a.ks_hs + t * a.ks_ts : kbase) + c * CH);
  ld.vsr[0] = load_raw<CH>((has ? a.value_suffix + h * a.vs_hs + t * a.vs_ts : vbase) + c * CH);
  return ld;
}

template <int D, int GBM>
__device__ __forceinline__ void attend_tile(const AttendArgs& a, DecideShared& dsh,
                                            LaneCombine<D, GBM>& cmb,
                                            const AttendLoads<D, GBM>& ld, int64_t h,
                                            uint32_t wk) {
  constexpr int CH = D / 16;
  constexpr int R = kRowBatch;
  constexpr int NB = kTile / 16;  // representatives per lane group
  using Comb = LaneCombine<D, GBM>;
  const DecideArgs& da = a.decide;
  const int G = da.group;
  const uint32_t N = (uint32_t)da.n_blocks, T = (uint32_t)da.n_tiles;
  const uint32_t L = (uint32_t)da.length, lb = (uint32_t)a.log2_block, B = 1u << lb;
  const int tid = threadIdx.x;
  const int lg = tid >> 4, c = tid & 15;
  const int g0 = blockIdx.z * GBM, gn = min(GBM, G - g0);  // this pass's query rows
  // The launch's W workgroups per head: workgroup wk scores tile wk % T.
  // With short prompts the one-launch step runs copies of the T tiles (wk >=
  // T) so that the suffix and the head's expanded token rows spread over more
  // workgroups: a copy repeats its tile's scores and decision (publishing the
  // same slots, bit for bit) but adds no representatives of its own.
  const uint32_t W = (uint32_t)a.workers;
  const uint32_t tile = wk % T;
  const bool primary = wk < T;

  // ---- what attend_issue loaded; z and the row maxima from the statistics -
  const DecideLoads& din = ld.din;
  const uint32_t S = ld.S;
  const auto& vraw = ld.vraw;
  const auto& qraw = ld.qraw;
  const auto& ksr = ld.ksr;
  const auto& vsr = ld.vsr;
  float zr[GBM][NB], mt[GBM];
#pragma unroll
  for (int i = 0; i < NB; ++i) {
    uint32_t b = tile * kTile + lg + 16 * i;
    b = b < N ? b : N - 1;
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      const int gg = g0 + g < G ? g0 + g : G - 1;
      zr[g][i] = da.zf[(h * G + gg) * da.z_stride + b].x;
    }
  }
#pragma unroll
  for (int g = 0; g < GBM; ++g) {
    const int gg = g0 + g < G ? g0 + g : G - 1;
    mt[g] = da.lse[((h * G + gg) * da.tile_stride + tile) * 4];
  }
  const uint32_t n_suffix = S > wk ? (S - wk + W - 1) / W : 0u;
  const uint32_t n_pre = n_suffix < 16u ? n_suffix : 16u;
  const uint16_t* kbase = a.key_pages + h * a.kp_hs;
  const uint16_t* vbase = a.value_pages + h * a.vp_hs;
  const uint16_t* ks = a.key_suffix + h * a.ks_hs;
  const uint16_t* vs = a.value_suffix + h * a.vs_hs;
  const uint32_t kts = (uint32_t)a.ks_ts, vts = (uint32_t)a.vs_ts;

  // ---- every representative of this lane group, expanded or not ----------
  GroupState<D, GBM> st;
  float pw[GBM][NB];
  {
    float v[NB][CH];
#pragma unroll
    for (int i = 0; i < NB; ++i) unpack(vraw[i], v[i]);
#pragma unroll
    for (int g = 0; g < GBM; ++g) {
      const float m = inf_to_zero(mt[g]);
      st.m[g] = m;
      st.l[g] = 0.0f;
#pragma unroll
      for (int e = 0; e < CH; ++e) st.acc[g][e] = 0.0f;
#pragma unroll
      for (int i = 0; i < NB; ++i) {
        const bool valid = primary && tile * kTile + lg + 16 * i < N;
        pw[g][i] = valid ? __builtin_amdgcn_exp2f((zr[g][i] - m) * kLog2e) : 0.0f;
        st.l[g] = st.l[g] + pw[g][i];
#pragma unroll
        for (int e = 0; e < CH; ++e) st.acc[g][e] = __builtin_fmaf(pw[g][i], v[i][e], st.acc[g][e]);
      }
    }
  }
  // ---- the decision --------------------------------------------------------
  const int32_t* list;
  uint32_t count = 0;
  const uint64_t bits = decide_finish<false>(da, h, tile, din, dsh, nullptr, list, count);

  // take the expanded blocks' representatives out again
  if ((bits >> lg) & 0x0001000100010001ull) {
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      if ((bits >> (lg + 16 * i)) & 1ull) {
        float v[CH];
        unpack(vraw[i], v);
#pragma unroll
        for (int g = 0; g < GBM; ++g) {
          st.l[g] = st.l[g] - pw[g][i];
#pragma unroll
          for (int e = 0; e < CH; ++e) st.acc[g][e] = __builtin_fmaf(-pw[g][i], v[e], st.acc[g][e]);
        }
      }
    }
  }

  // ---- the prefetched suffix rows (after the subtraction, which assumes
  // the representatives' scale): lane groups lg < n_pre hold one; a wave
  // whose four lane groups hold none skips the fold, which would leave its
  // state unchanged (a masked row adds exp(-inf) = 0 times a zeroed value)
  if (4 * __builtin_amdgcn_readfirstlane(tid / kWave) < (int)n_pre)
    fold_tokens<D, GBM, 1>(st, qraw, ksr, vsr, (uint32_t)lg < n_pre ? 1u : 0u, a.scale, gn);

  // ---- token rows ---------------------------------------------------------
  // Runs n_rows rows through the online softmax, 16 R rows per batch, two
  // batches in flight; row(v, kp, vp) points kp / vp at row v (a valid row
  // when it is masked) and returns whether it is live.
  auto run_rows = [&](uint32_t n_rows, auto row) {
    if (n_rows == 0) return;
    auto issue = [&](uint32_t batch, RawBf16<CH> (&kr)[R], RawBf16<CH> (&vr)[R]) {
      uint32_t ok = 0;
#pragma unroll
      for (int u = 0; u < R; ++u) {
        const uint16_t *kp = kbase, *vp = vbase;
        const uint32_t v = batch * 16 * R + lg + 16 * u;
        if (v < n_rows && row(v, kp, vp)) ok |= 1u << u;
        kr[u] = load_raw<CH>(kp + c * CH);
        vr[u] = load_raw<CH>(vp + c * CH);
      }
      return ok;
    };
    // two batches in flight; no loads for batches past the last (their
    // loads would only hold up later waits)
    RawBf16<CH> ka[R], va[R], kb[R], vb[R];
    uint32_t oka = issue(0, ka, va);
    uint32_t okb = 0;
    if (16 * R < n_rows) okb = issue(1, kb, vb);
    // (a wave with no live row in a batch skips its fold: it would leave
    // the state unchanged)
#pragma unroll 1
    for (uint32_t k = 0; k * 16 * R < n_rows; k += 2) {
      if (__ballot(oka != 0)) fold_tokens<D, GBM>(st, qraw, ka, va, oka, a.scale, gn);
      if ((k + 2) * 16 * R < n_rows) oka = issue(k + 2, ka, va);
      if ((k + 1) * 16 * R >= n_rows) break;
      if (__ballot(okb != 0)) fold_tokens<D, GBM>(st, qraw, kb, vb, okb, a.scale, gn);
      if ((k + 3) * 16 * R < n_rows) okb = issue(k + 3, kb, vb);
    }
  };
  const uint32_t last = N - 1, last_count = L - last * B;
  // the row of token t of block bb of the head's pages
  auto page_row = [&](uint32_t bb, uint32_t t, const uint16_t*& kp, const uint16_t*& vp) {
    const uint32_t off = ((bb << lb) + t) * (uint32_t)D;
    kp = kbase + off;
    vp = vbase + off;
    return bb != last || t < last_count;
  };

  // ---- the rest of the suffix slice and this tile's expanded blocks
  const uint32_t n_rest = n_suffix - n_pre;
  const uint32_t own_rows = (uint32_t)__popcll(bits) * B;
  run_rows(n_rest + own_rows, [&](uint32_t v, const uint16_t*& kp, const uint16_t*& vp) {
    if (v < n_rest) {
      const uint64_t t = wk + (n_pre + v) * W;
      kp = ks + t * kts;
      vp = vs + t * vts;
      return true;
    }
    const uint32_t w = v - n_rest;
    return page_row(tile * kTile + (uint32_t)list[w >> lb], w & (B - 1), kp, vp);
  });


  // ---- the 16 lane groups -> one partial per query row, through LDS ------
  // (fully unrolled: the state arrays are indexed by constants only)
#pragma unroll
  for (int gc = 0; gc < GBM; gc += Comb::kRows) {
    if (gc > 0) __syncthreads();  // the previous chunk's reads are done
#pragma unroll
    for (int j = 0; j < Comb::kRows; ++j) {
      if (gc + j < gn) {
#pragma unroll
        for (int i = 0; i < CH; ++i) cmb.acc[lg][j][c * Comb::kSlice + i] = st.acc[gc + j][i];
        if (c == 0) {
          cmb.ml[lg][j][0] = st.m[gc + j];
          cmb.ml[lg][j][1] = st.l[gc + j];
        }
      }
    }
    __syncthreads();
    const int rows = gn - gc < Comb::kRows ? gn - gc : Comb::kRows;
    for (int idx = 2 * tid; idx < rows * D; idx += 2 * kThreads) {
      const int j = idx / D, d = idx % D;
      const int at_d = (d / CH) * Comb::kSlice + d % CH;  // CH is even: d, d+1 in one slice
      float M = kNegInf;
#pragma unroll
      for (int w = 0; w < 16; ++w) M = fmaxf(M, cmb.ml[w][j][0]);
      float a0 = 0.0f, a1 = 0.0f, l = 0.0f;
#pragma unroll
      for (int w = 0; w < 16; ++w) {
        const float mw = cmb.ml[w][j][0];
        const float e = mw == kNegInf ? 0.0f : __builtin_amdgcn_exp2f((mw - M) * kLog2e);
        const float2 av = *reinterpret_cast<const float2*>(&cmb.acc[w][j][at_d]);
        a0 = __builtin_fmaf(av.x, e, a0);
        a1 = __builtin_fmaf(av.y, e, a1);
        l = __builtin_fmaf(cmb.ml[w][j][1], e, l);
      }
      const int64_t at = (h * G + g0 + gc + j) * da.tile_stride + wk;
      *reinterpret_cast<float2*>(a.part_acc + at * D + d) = make_float2(a0, a1);
      if (d == 0) a.part_ml[at] = make_float2(M, l);
    }
  }
  if (a.tile_counts && tid == 0 && blockIdx.z == 0) a.tile_counts[h * da.tile_stride + wk] = count;
}

// ---------------------------------------------------------------------------
// The matrix-core attention of one (tile, head): representatives, suffix
// and expanded page rows as 16-row chunks on the MFMA engine
// ---------------------------------------------------------------------------
// What the matrix-core path loads before the statistics: the decision's
// inputs, the suffix length and the pass's query rows as QK operands.
template <int D>
struct MmaLoads {
  DecideLoads din;
  uint32_t S;
  Bf16x8 qop[MmaShape<D>::kSteps];
};

template <int D, int GBM, bool kFused>
__device__ __forceinline__ MmaLoads<D> mma_issue(const AttendArgs& a, int64_t h, uint32_t wk) {
  const DecideArgs& da = a.decide;
  const uint32_t tile = wk % (uint32_t)da.n_tiles;
  MmaLoads<D> ld;
  ld.din = decide_issue<!kFused>(da, h, tile);
  // the suffix length does not change during a launch: a scalar load
  uint32_t S = (uint32_t)a.suffix_cap;
  if (a.suffix_len_dev) {
    typedef __attribute__((address_space(4))) const int32_t ConstI32;
    const int32_t sl = *(ConstI32*)(uintptr_t)a.suffix_len_dev;
    S = sl < 0 ? 0u : ((uint32_t)sl > S ? S : (uint32_t)sl);
  }
  ld.S = S;
  mma_query<D, GBM>(ld.qop, a.query + (h * da.group) * D, (int)blockIdx.z * GBM, da.group);
  return ld;
}

// Wave w's representative chunk (the value means of blocks 16 w .. 16 w + 15
// of the tile, clamped to the last block) into dst (a stage): the first
// ones are issued before the decision, so they land during the wait for the
// head's LSE partials.
template <int D>
__device__ __forceinline__ void mma_stage_reps(const AttendArgs& a, int64_t h, uint32_t tile,
                                               char* dst) {
  using S = MmaShape<D>;
  constexpr uint32_t NC = S::kNC;
  typedef __attribute__((address_space(3))) void LdsVoid;
  const uint32_t N = (uint32_t)a.decide.n_blocks;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t first = tile * kTile + 16u * wave;
  if (first >= N) return;
  const uint32_t lane = threadIdx.x % kWave;
  const auto vres = buffer_view(a.value_mean + h * (int64_t)N * D, N * (uint32_t)(D * 2));
#pragma unroll
  for (int u = 0; u < S::kLdsLoads; ++u) {
    const uint32_t p = 64u * u + lane, t = p / NC;
    const uint32_t piece = (p % NC + 32u * NC - 2u * t) % NC;
    const uint32_t row = first + t < N ? first + t : N - 1;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(vres, (LdsVoid*)(dst + 1024 * u), 16,
                                             (int)(row * (uint32_t)(D * 2) + piece * 16u), 0,
                                             0, 0);
  }
}

// Decision, then attention of wave-sized chunks on the matrix cores, one ring
// of chunks per wave: its representative chunk (staged before the decision;
// logits z, expanded and missing blocks at -inf), its share of the suffix,
// then its share of the page rows of the expanded blocks of the workgroup's
// own tile (with several tiles per workgroup, of all of them; copies of a
// tile -- one-launch step with more workgroups than tiles -- each take an
// even slice of the tile's rows).  The first page rows' loads are issued as
// the ring starts, right after the decision, so they are in flight while the
// earlier chunks fold.  The four waves' states merge through LDS into the
// workgroup's partial, and (one-launch step) the head's last workgroups merge
// the partials.
template <int D, int GBM, bool kFused, int kTiles = 1>
__device__ __forceinline__ void attend_tile_mma(const AttendArgs& a, DecideShared& dsh,
                                                MmaCombine<D, GBM>& cmb, const StepCtx* sx,
                                                const MmaLoads<D>& ld, int64_t h, uint32_t wk,
                                                const TileSet<kTiles, GBM>* tset = nullptr) {
  constexpr bool kMulti = kTiles > 1;
  static_assert(!kMulti || (kFused && GBM == 4), "several tiles: one-launch step, 4-row passes");
  using S = MmaShape<D>;
  const DecideArgs& da = a.decide;
  const int G = da.group;
  const uint32_t N = (uint32_t)da.n_blocks, T = (uint32_t)da.n_tiles;
  const uint32_t L = (uint32_t)da.length, lb = (uint32_t)a.log2_block, B = 1u << lb;
  const int tid = threadIdx.x, lane = tid % kWave;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(tid / kWave);
  const int g0 = blockIdx.z * GBM, gn = min(GBM, G - g0);  // this pass's query rows
  const uint32_t W = (uint32_t)a.workers;
  const uint32_t tile = wk % T;
  const bool primary = wk < T;
  const uint32_t n_suffix = ld.S > wk ? (ld.S - wk + W - 1) / W : 0u;
  constexpr uint32_t kRowBytes = D * 2;
  // with more workgroups than tiles, workgroups wk, wk + T, ... decide the
  // same tile: this one is copy `copy` of `copies` and takes that slice of
  // the tile's expanded rows
  const uint32_t copies = kMulti ? 1u : (W - tile + T - 1u) / T;
  const uint32_t copy = kMulti ? 0u : wk / T;

  MmaStage<D>& stage = cmb.stage[wave];
  unsigned long long* stamps = nullptr;  // (phase stamps build)
  if constexpr (kFused) stamps = sx->stats.stamps;
  (void)stamps;

  // ---- representatives and suffix: loads issued before the decision -------
  // (the representative rows into stage 0; the wave's first suffix chunk
  // into the next stage and K registers), so that they land while it waits
  const bool has_reps = primary && tile * kTile + 16u * wave < N;
  // representative chunks (one per tile; chunk m < R is tile wk + m W's)
  const uint32_t R = kMulti ? tset->n : 1u;
  const uint32_t ns_chunks = (n_suffix + 15u) / 16u;
  const uint32_t ns_wave = ns_chunks > wave ? (ns_chunks - 1u - wave) / 4u + 1u : 0u;
  const uint32_t cap = (uint32_t)a.suffix_cap;
  const uint32_t kts = (uint32_t)a.ks_ts * 2u, vts = (uint32_t)a.vs_ts * 2u;  // bytes
  const auto kres_s = buffer_view(a.key_suffix + h * a.ks_hs, cap ? (cap - 1u) * kts + kRowBytes : 0u);
  const auto vres_s = buffer_view(a.value_suffix + h * a.vs_hs, cap ? (cap - 1u) * vts + kRowBytes : 0u);
  // Speculation (one-launch step, one tile per workgroup): when the previous
  // launch on this workspace expanded every block of the tile, the wave
  // issues its first three chunks (every stage of its ring) before the decision,
  // assuming every block expands again (so its ring has no representative
  // chunk: with every block expanded that chunk's logits are all -inf and its
  // fold would leave the state unchanged); if the decision agrees, the ring
  // goes on from them and the result is the normal order's bit for bit, else
  // the wave waits for them to land and runs the normal order.
  // (head_dim 160 does not speculate: its two rings below would need the
  // speculative order in both)
  const bool spec = kFused && D <= 128 && sx->spec != nullptr && *sx->spec != 0u;
  bool reps_on = has_reps && !spec;
#if defined(RKV_PHASE_STAMPS)
  if (stamps != nullptr && tid == 0) stamps[kStSpec] = spec ? 1u : 0u;
#endif
  Bf16x8 k0[S::kSteps], k1[S::kSteps], k2[S::kSteps];
  // The wave's ring: chunks m < Rr are the representative chunks (a no-op
  // without representatives: nothing issued, nothing folded; none while
  // speculating), chunk Rr <= j < n1 the wave's suffix chunk j - Rr, then its
  // page chunks of this workgroup's rows [pr0, pr1) -- chunk c = rows 16 c
  // .. 16 c + 15 (inside one block: B is a multiple of 16) goes to wave
  // (c - c0 + lead) mod 4, the waves with fewer suffix chunks first.
  uint32_t Rr = spec ? 0u : R;
  uint32_t pr0 = 0u, pr1 = 0u;
  const uint32_t lead = (wave + 4u - ns_chunks % 4u) % 4u;  // this wave's first page chunk
  auto rep_tile = [&](uint32_t m) { return kMulti ? wk + m * W : tile; };
  auto issue_suffix = [&](uint32_t j, int sidx, Bf16x8 (&kop)[S::kSteps]) {
    const uint32_t ci = wave + 4u * (j - Rr);
    // suffix row t of the chunk: token wk + (16 ci + t) W (rows past this
    // workgroup's slice repeat its last token and are masked)
    auto token = [&](uint32_t t) {
      const uint32_t r = 16u * ci + t;
      return wk + (r < n_suffix ? r : n_suffix - 1u) * W;
    };
    mma_issue_rows<D>(kres_s, vres_s, stage.bytes[sidx], kop,
                      [&](uint32_t t) { return token(t) * kts; },
                      [&](uint32_t t) { return token(t) * vts; });
  };
  // representative chunk m into dst.  With several tiles every chunk of the
  // ring issues the same loads (the ring's waits count them): the value
  // means through mma_issue_rows (an empty view past the last block) and
  // key operands from an empty view (zeros; a representative chunk has
  // none).  With one tile chunk 0 is issued before the ring and stages the
  // value means alone.
  auto issue_reps = [&](uint32_t m, char* dst, Bf16x8 (&kop)[S::kSteps]) {
    if constexpr (kMulti) {
      const uint32_t first = rep_tile(m) * kTile + 16u * wave;
      const auto vres =
          buffer_view(a.value_mean + h * (int64_t)N * D, first < N ? N * kRowBytes : 0u);
      mma_issue_rows<D>(buffer_view(a.value_mean, 0u), vres, dst, kop,
                        [](uint32_t) { return 0u; },
                        [&](uint32_t t) { return (first + t < N ? first + t : N - 1u) * kRowBytes; });
    } else {
      (void)kop;
      mma_stage_reps<D>(a, h, rep_tile(m), dst);
    }
  };

  // ---- page rows ------------------------------------------------------------
  // Expanded block ordinal e of the workgroup's tiles, in (tile, block)
  // order, gives B rows; row r is token r mod B of block block_of(r / B).
  // bits[m]: tile m's expanded blocks (wave-uniform, so the lookups below are
  // scalar arithmetic).
  uint64_t bits[kTiles] = {};
  // one tile: the decision's list of the tile's expanded blocks (this wave's
  // copy in LDS, ascending), or before the decision (speculating) every block
  const int32_t* plist = nullptr;
  auto block_of = [&](uint32_t e) -> uint32_t {
    if constexpr (!kMulti) return tile * kTile + (plist != nullptr ? (uint32_t)plist[e] : e);
    uint32_t t_sel = wk;
    uint64_t b_sel = bits[0];
    if constexpr (kMulti) {
      bool found = e < (uint32_t)__popcll(b_sel);
#pragma unroll
      for (int m = 1; m < kTiles; ++m) {
        if (!found) {
          e -= (uint32_t)__popcll(b_sel);
          t_sel = wk + (uint32_t)m * W;
          b_sel = bits[m];
          found = e < (uint32_t)__popcll(b_sel);
        }
      }
    }
    return t_sel * kTile + (uint32_t)nth_set_bit(b_sel, (int)e);
  };
  const uint16_t* kbase = a.key_pages + h * a.kp_hs;
  const uint16_t* vbase = a.value_pages + h * a.vp_hs;
  const uint32_t page_bytes = (N << lb) * kRowBytes;
  const auto kres = buffer_view(kbase, page_bytes), vres = buffer_view(vbase, page_bytes);
  const uint32_t last = N - 1, last_count = L - last * B;
  // the tile's blocks (the last tile may be short): what speculation assumes
  const uint32_t n_valid = N - tile * kTile < (uint32_t)kTile ? N - tile * kTile : (uint32_t)kTile;
  const uint64_t valid_bits = n_valid >= 64u ? ~0ull : (1ull << n_valid) - 1ull;
  // this workgroup's slice of the rows of `blocks` expanded blocks
  // (32-bit arithmetic: a workgroup's tiles hold at most 4 x 64 x 64 rows,
  // and copies come only with one tile, at most 256 per head)
  auto set_rows = [&](uint32_t blocks) {
    const uint32_t rows = blocks << lb;
    if (copies == 1u) {
      pr0 = 0u;
      pr1 = rows;
    } else {
      pr0 = copy * rows / copies;
      pr1 = (copy + 1u) * rows / copies;
    }
  };
  auto n1 = [&]() { return Rr + ns_wave; };
  auto n_chunks = [&]() {
    const uint32_t c0 = pr0 >> 4, c_end = (pr1 + 15u) >> 4;
    const uint32_t np = pr1 > pr0 && c0 + lead < c_end ? (c_end - c0 - lead - 1u) / 4u + 1u : 0u;
    return n1() + np;
  };
  auto chunk_of = [&](uint32_t j) { return (pr0 >> 4) + lead + 4u * (j - n1()); };
  auto issue_page = [&](uint32_t j, int sidx, Bf16x8 (&kop)[S::kSteps]) {
    const uint32_t c = chunk_of(j);
    const uint32_t row0 = (block_of((c << 4) >> lb) << lb) + ((c << 4) & (B - 1u));
    RKV_STAMP(stamps, kStIssue2Addr, tid == 0 && j == 2u);
    auto row = [&](uint32_t t) { return (row0 + t) * kRowBytes; };
    mma_issue_rows<D>(kres, vres, stage.bytes[sidx], kop, row, row);
  };
  auto issue = [&](uint32_t j, int sidx, Bf16x8 (&kop)[S::kSteps]) {
    RKV_STAMP(stamps, kStIssueStart2 + (j - 2u), tid == 0 && j >= 2u && j < 8u);
    if (j < Rr) issue_reps(j, stage.bytes[sidx], kop);
    else if (j < n1()) issue_suffix(j, sidx, kop);
    else issue_page(j, sidx, kop);
    RKV_STAMP(stamps, kStIssued2, tid == 0 && j == 2u);
  };
  // chunks 0 and 1 are issued before the decision (a representative chunk
  // without representatives issues nothing)
  auto pre_issue = [&]() {
    const uint32_t n = n_chunks();
    if (Rr == 0u || kMulti || reps_on) {
      if (n > 0) issue(0u, 0, k0);
    }
    if (n > 1 && (Rr == 0u || n1() > 1u)) issue(1u, 1, k1);
    if (spec && Rr == 0u && n > 2) issue(2u, 2, k2);  // (speculating: all three stages)
  };

  MmaState<D> st;
  st.m = kNegInf;
  st.lsum = 0.0f;
#pragma unroll
  for (int b = 0; b < S::kBlocks; ++b) st.o[b] = F32x4{0.0f, 0.0f, 0.0f, 0.0f};

  if (spec) {
    bits[0] = valid_bits;
    set_rows(n_valid);
  }
  pre_issue();

  // ---- the decision (one-launch step: from the head's tagged LSE slots) ----
  uint32_t count = 0;
  if constexpr (kMulti) {
    decide_tiles<kTiles, GBM>(da, h, wk, W, *tset, dsh, sx->stats, bits, count);
  } else {
    bits[0] = decide_finish<kFused, false, GBM>(da, h, tile, ld.din, dsh, nullptr, plist, count,
                                           kFused ? &sx->stats : nullptr);
  }
  RKV_STAMP(stamps, kStDecided, tid == 0);
  if (spec && bits[0] != valid_bits) {
    // the speculation missed: the chunks issued for it land, then the
    // normal order
    wait_vm<0>();
    Rr = R;
    reps_on = has_reps;
  }
  if (!spec || Rr != 0u) {
    uint32_t blocks = 0;
#pragma unroll
    for (int m = 0; m < kTiles; ++m) blocks += (uint32_t)__popcll(bits[m]);
    set_rows(blocks);
    if (spec) pre_issue();
  }

  // ---- the ring -------------------------------------------------------------
  // logits of chunk j: representative, suffix or page chunk
  auto rep_logits = [&](uint32_t j, float (&x)[4]) {
    // logit z of block rep_first + 4 (l / 16) + i for query row g
    const int g = lane & 15, gg = g < gn ? g : 0;
    const uint32_t rt = rep_tile(j);
    // (tile j's bits from LDS: a register array indexed by j would live in
    // scratch)
    const uint64_t rbits = kMulti ? dsh.tile_bits[j] : bits[0];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t tb = 16u * wave + 4u * (uint32_t)(lane >> 4) + i;  // in the tile
      const uint32_t b = rt * kTile + tb;
      const bool live = b < N && !((rbits >> tb) & 1ull);
      float z;
      if constexpr (kMulti) z = tset->z[j < kTiles ? j : 0][gg][tb];
      else if constexpr (kFused) z = sx->stats.zs[gg][tb].x;
      else z = da.zf[(h * G + g0 + gg) * da.z_stride + (b < N ? b : N - 1)].x;
      x[i] = live ? z : kNegInf;
    }
  };
  auto suffix_logits = [&](uint32_t j, const Bf16x8 (&kop)[S::kSteps], float (&x)[4]) {
    const uint32_t ci = wave + 4u * (j - Rr);
    const F32x4 s4 = mma_qk<D>(kop, ld.qop);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = 16u * ci + 4u * (uint32_t)(lane >> 4) + i;
      x[i] = r < n_suffix ? s4[i] * a.scale : kNegInf;
    }
  };
  auto page_logits = [&](uint32_t j, const Bf16x8 (&kop)[S::kSteps], float (&x)[4]) {
    const uint32_t c = chunk_of(j);
    const uint32_t bb = block_of((c << 4) >> lb);
    const F32x4 s4 = mma_qk<D>(kop, ld.qop);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t r = (c << 4) + 4u * (uint32_t)(lane >> 4) + i;
      const uint32_t tok = r & (B - 1u);
      const bool live = r >= pr0 && r < pr1 && (bb != last || tok < last_count);
      x[i] = live ? s4[i] * a.scale : kNegInf;
    }
  };
  // a representative chunk without representatives folds nothing
  auto reps_live = [&](uint32_t j) {
    return kMulti ? rep_tile(j) * kTile + 16u * wave < N : reps_on;
  };
  const uint32_t pre = !spec || Rr != 0u ? (n1() > 1u ? 2u : 1u)
                                         : (n_chunks() > 2u ? 3u : n_chunks() > 1u ? 2u : 1u);
  RKV_STAMP(stamps, kStRingStart, tid == 0);
  if constexpr (D <= 128) {
    // one ring: the first page rows' loads are issued as it starts
    mma_ring<D>(n_chunks(), pre, k0, k1, k2, issue,
                [&](uint32_t j, int sidx, const Bf16x8 (&kop)[S::kSteps]) {
                  float x[4];
                  RKV_STAMP(stamps, kStFold0Start, tid == 0 && j == 0u);
                  RKV_STAMP(stamps, kStFoldStart0 + j, tid == 0 && j < 6u);
                  if (j < Rr) {
                    if (!reps_live(j)) return;
                    rep_logits(j, x);
                  } else if (j < n1()) {
                    suffix_logits(j, kop, x);
                  } else {
                    page_logits(j, kop, x);
                  }
                  mma_fold<D>(st, x, stage.bytes[sidx]);
                  RKV_STAMP(stamps, kStChunk0 + (j < 3u ? j : 2u), tid == 0 && j < 3u);
                  RKV_STAMP(stamps, kStFoldEnd0 + j, tid == 0 && j < 6u);
                });
  } else {
    // (head_dim 160: one ring of every kind holds more registers than the
    // kernel has) the representative and suffix chunks, then the page rows
    // in a ring of their own
    const uint32_t first = n1();
    mma_ring<D>(first, pre, k0, k1, k2,
                [&](uint32_t j, int sidx, Bf16x8 (&kop)[S::kSteps]) {
                  if (j < Rr) issue_reps(j, stage.bytes[sidx], kop);
                  else issue_suffix(j, sidx, kop);
                },
                [&](uint32_t j, int sidx, const Bf16x8 (&kop)[S::kSteps]) {
                  float x[4];
                  if (j < Rr) {
                    if (!reps_live(j)) return;
                    rep_logits(j, x);
                  } else {
                    suffix_logits(j, kop, x);
                  }
                  mma_fold<D>(st, x, stage.bytes[sidx]);
                });
    mma_ring<D>(n_chunks() - first, 0u, k0, k1, k2,
                [&](uint32_t j, int sidx, Bf16x8 (&kop)[S::kSteps]) {
                  issue_page(first + j, sidx, kop);
                },
                [&](uint32_t j, int sidx, const Bf16x8 (&kop)[S::kSteps]) {
                  float x[4];
                  page_logits(first + j, kop, x);
                  mma_fold<D>(st, x, stage.bytes[sidx]);
                });
  }
  RKV_STAMP(stamps, kStRing, tid == 0);

  // the expanded-block mask, stored after the ring (a store issued ahead of
  // the ring's loads would hold its first waits), and for the next launch's
  // speculation whether every block of the tile expanded
  if (wave == 0 && blockIdx.z == 0 && da.write_mask) {
#pragma unroll
    for (int m = 0; m < kTiles; ++m) {
      const uint32_t b = rep_tile((uint32_t)m) * kTile + (uint32_t)lane;
      const uint8_t v = (uint8_t)((bits[m] >> lane) & 1ull);
      if ((uint32_t)m < R && b < N) {
        // (one-launch step: written through, so that a merger's later
        // all-expanded mask after a failed hand-off is the last write)
        if constexpr (kFused) sx->mask.store_u8((uint32_t)(h * (int64_t)N + b), v);
        else da.mask[h * (int64_t)N + b] = v;
      }
    }
  }
  if constexpr (kFused && !kMulti) {
    if (tid == 0 && sx->full != nullptr)
      __hip_atomic_store(sx->full, bits[0] == valid_bits ? (uint64_t)*sx->stats.tag + 1u : 0ull,
                         __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // ---- the four waves -> one partial per query row, through LDS ------------
  RKV_STAMP(stamps, kStPagesWave0, tid == 0);
  mma_publish<D, GBM>(st, cmb.mma[wave]);
  __syncthreads();
  RKV_STAMP(stamps, kStCombine, tid == 0);
  uint32_t tag = 0u;
  bool nan_partial = false;  // a wait of this workgroup gave up
  if constexpr (kFused) {
    tag = __builtin_amdgcn_readfirstlane(*sx->stats.tag);
    nan_partial = *sx->stats.gave_up != 0u;
  }
  mma_combine<D, GBM>(cmb, gn, [&](int j, int d, float2 acc, float M, float l) {
    if (nan_partial) l = bits_f32(0x7FC00000u);
    const int64_t at = (h * G + g0 + j) * da.tile_stride + wk;
    if constexpr (kFused) {
      // the partial as tagged slots (the mergers poll them)
      const int64_t row = (h * G + g0 + j) * da.tile_stride;
      sx->acc.store4(acc_slot<D>(row, wk, (uint32_t)d / 2u),
                     make_slot(f32_bits(acc.x), f32_bits(acc.y), tag));
      if (d == 0) sx->ml.store4(ml_slot(row, wk), make_slot(f32_bits(M), f32_bits(l), tag));
    } else {
      *reinterpret_cast<float2*>(a.part_acc + at * D + d) = acc;
      if (d == 0) a.part_ml[at] = make_float2(M, l);
    }
  });
  if (tid == 0 && blockIdx.z == 0) {
    // (a copy's count sits past the first T entries, which alone are summed)
    if constexpr (kFused) {
      if (sx->accessed)
        sx->counts.store4((uint32_t)((h * da.tile_stride + wk) * 16), make_slot(count, 0u, tag));
    } else if (a.tile_counts) {
      a.tile_counts[h * da.tile_stride + wk] = count;
    }
  }
  RKV_STAMP(stamps, kStPublished, tid == 0);
  if constexpr (kFused) {
    // the head's last K workgroups each merge a column slice
    const uint32_t K = mergers(W, (uint32_t)D);
    if (wk >= W - K) {
      RKV_STAMP(stamps, kStMergeWait, tid == 0);
      merge_slice<D>(a, *sx, h, (int)(wk - (W - K)), (int)K);
      RKV_STAMP(stamps, kStMerged, tid == 0);
    }
  }
}

template <int D, int GBM>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void attend_kernel(AttendArgs a) {
  __shared__ alignas(16) DecideShared dsh;
  if constexpr (D <= kMmaMaxDim) {
    __shared__ alignas(16) MmaCombine<D, GBM> cmb;
    const int64_t h = blockIdx.y;
    const uint32_t wk = blockIdx.x;
    const MmaLoads<D> ld = mma_issue<D, GBM, false>(a, h, wk);
    attend_tile_mma<D, GBM, false>(a, dsh, cmb, nullptr, ld, h, wk);
  } else {
    __shared__ alignas(16) LaneCombine<D, GBM> cmb;
    const AttendLoads<D, GBM> ld = attend_issue<D, GBM>(a, blockIdx.y, blockIdx.x);
    attend_tile<D, GBM>(a, dsh, cmb, ld, blockIdx.y, blockIdx.x);
  }
}

// ---------------------------------------------------------------------------
// Dense decode: every cached token of every head, no summary (the
// full-attention decode of dense layers and of the dense baseline,
// transformers.py:510-520's SDPA call)
// ---------------------------------------------------------------------------
struct DenseArgs {
  const uint16_t* query;           // (H, G, D) bf16
  const uint16_t* keys;            // token t of head h at keys + h * k_hs + t * k_ts
  const uint16_t* values;          // likewise with v_hs, v_ts
  int64_t k_hs, v_hs;              // elements
  uint32_t k_ts, v_ts;             // elements
  const int32_t* length_dev;       // tokens, read on the device (null: cap)
  uint32_t cap;                    // tokens the key/value views address
  int group, splits;
  float scale;
  float2* part_ml;                 // (H G, splits): m, l
  float* part_acc;                 // (H G, splits, D)
};

// Workgroup (split sp, head h, row pass z): the split's share of the head's
// 16-token chunks, C sp / splits .. C (sp + 1) / splits (C = ceil(L / 16)),
// chunk c0 + w + 4 j to wave w, through the same three-stage matrix-core ring
// as the decode's page rows; the four waves' states combine into one partial
// per query row, which merge_kernel folds with the other splits'.
// (two workgroups per CU up to head_dim 128 and 8 query rows; beyond, the
// ring's registers take a whole SIMD per wave, one workgroup per CU, rather
// than spill)
template <int D, int GBM>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(D <= 128 && GBM <= 8 ? 2 : 1)))
void dense_kernel(DenseArgs a) {
  using S = MmaShape<D>;
  constexpr uint32_t kRowBytes = D * 2;
  __shared__ alignas(16) MmaCombine<D, GBM> cmb;
  const int64_t h = blockIdx.y;
  const uint32_t sp = blockIdx.x, splits = (uint32_t)a.splits;
  const int G = a.group, g0 = blockIdx.z * GBM, gn = min(GBM, G - g0);
  const int lane = threadIdx.x % kWave;
  const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  uint32_t L = a.cap;
  if (a.length_dev) {
    // the length does not change during a launch: a scalar load
    typedef __attribute__((address_space(4))) const int32_t ConstI32;
    const int32_t n = *(ConstI32*)(uintptr_t)a.length_dev;
    L = n < 0 ? 0u : ((uint32_t)n > a.cap ? a.cap : (uint32_t)n);
  }
  const uint32_t C = (L + 15u) / 16u;
  const uint32_t c0 = (uint32_t)((uint64_t)C * sp / splits);
  const uint32_t c1 = (uint32_t)((uint64_t)C * (sp + 1u) / splits);
  const uint32_t n = c0 + wave < c1 ? (c1 - c0 - wave - 1u) / 4u + 1u : 0u;
  const uint32_t kts = a.k_ts * 2u, vts = a.v_ts * 2u;  // bytes
  const auto kres = buffer_view(a.keys + h * a.k_hs, a.cap ? (a.cap - 1u) * kts + kRowBytes : 0u);
  const auto vres = buffer_view(a.values + h * a.v_hs, a.cap ? (a.cap - 1u) * vts + kRowBytes : 0u);
  Bf16x8 qop[S::kSteps];
  mma_query<D, GBM>(qop, a.query + h * (int64_t)G * D, g0, G);
  MmaStage<D>& stage = cmb.stage[wave];
  MmaState<D> st;
  st.m = kNegInf;
  st.lsum = 0.0f;
#pragma unroll
  for (int b = 0; b < S::kBlocks; ++b) st.o[b] = F32x4{0.0f, 0.0f, 0.0f, 0.0f};
  Bf16x8 k0[S::kSteps], k1[S::kSteps], k2[S::kSteps];
  mma_ring<D>(
      n, 0u, k0, k1, k2,
      [&](uint32_t j, int sidx, Bf16x8 (&kop)[S::kSteps]) {
        const uint32_t c = c0 + wave + 4u * j;
        // rows past the last token repeat it and are masked
        auto token = [&](uint32_t t) { return 16u * c + t < L ? 16u * c + t : L - 1u; };
        mma_issue_rows<D>(kres, vres, stage.bytes[sidx], kop,
                          [&](uint32_t t) { return token(t) * kts; },
                          [&](uint32_t t) { return token(t) * vts; });
      },
      [&](uint32_t j, int sidx, const Bf16x8 (&kop)[S::kSteps]) {
        const uint32_t c = c0 + wave + 4u * j;
        const F32x4 s4 = mma_qk<D>(kop, qop);
        float x[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t r = 16u * c + 4u * (uint32_t)(lane >> 4) + i;
          x[i] = r < L ? s4[i] * a.scale : kNegInf;
        }
        mma_fold<D>(st, x, stage.bytes[sidx]);
      });
  mma_publish<D, GBM>(st, cmb.mma[wave]);
  __syncthreads();
  mma_combine<D, GBM>(cmb, gn, [&](int j, int d, float2 acc, float M, float l) {
    const int64_t at = (h * G + g0 + j) * (int64_t)splits + sp;
    *reinterpret_cast<float2*>(a.part_acc + at * D + d) = acc;
    if (d == 0) a.part_ml[at] = make_float2(M, l);
  });
}



// ---------------------------------------------------------------------------
// The one-launch step: score, decision, attention and merge of every tile
// ---------------------------------------------------------------------------
struct StepArgs {
  ScoreArgs score;
  AttendArgs attend;
  uint64_t* control;              // hand-off counters
  uint32_t* counts;               // (H, tile_stride) tile access counts
  uint16_t* out;                  // (H, G, D) bf16
  unsigned long long* accessed;   // or null
  float4* lse_slots;              // (H*G, tile_stride, 2) tagged LSE slots
  uint64_t* full;                 // (H, tile_stride): tag + 1 of the launch whose tile fully expanded
  uint32_t* error;                // the sticky status word (bit 0: a wait gave up)
  uint32_t slots_bytes, ml_bytes, acc_bytes, counts_bytes, mask_bytes;
  int heads;
  uint32_t spin;      // polls before a hand-off wait gives up
  uint32_t skew;      // 0 (a test hook's nonzero value makes every wait run out)
  uint32_t speculate; // 1: speculate where the previous launch expanded every block
};

// z of each (row, block) of a workgroup's tiles when it scores several
// (kTiles > 1): the logits of their representative chunks.
template <int kTiles, int GBM>
struct TileZ {
  float z[kTiles][GBM][kTile];
};
template <int GBM>
struct TileZ<1, GBM> {};

// Every region starts on a 16-byte boundary: the q staging and the combine
// buffer are read with 16-byte LDS accesses.
template <int D, int GBM, int kTiles = 1>
struct StepShared {
  alignas(16) float4 zs[GBM][kTile];  // z, delta, A, th of the tile's (row, block) pairs
  alignas(16) TileZ<kTiles, GBM> tz;  // several tiles: each tile's z rows
  alignas(16) unsigned long long wsum[kWaves];
  uint32_t tag, rtag;
  uint32_t ticket;
  uint32_t spec;
  uint32_t gave_up;  // a wait of this workgroup gave up
  alignas(16) DecideShared dec;
  alignas(16) union {
    struct {
      alignas(16) float sdot[GBM * kTile];
      alignas(16) float pdot[GBM * kTile];
      alignas(16) float q[score_q_floats_max(GBM, D)];
    } score;
    alignas(16) MmaCombine<D, GBM> cmb;
  } u;
#if defined(RKV_PHASE_STAMPS)
  unsigned long long stamps[kStamps];
#endif
};

// Workgroup (tile, h): the tile's scores (z, delta and the risk's delta
// factors stay in LDS; the LSE partials are published and the head's
// arrival counter bumped), then attend_tile's decision (after the head's
// tiles have all arrived), attention and, for the head's last tile, the
// merge.
// kTicketed: (head, workgroup) from a start-order ticket instead of blockIdx
// (grids larger than the device holds at once).
// kTiles > 1: heads with more tiles than workgroups (W < n_tiles, four-row
// passes): workgroup wk scores tiles wk, wk + W, ... (at most kTiles), one
// after another, and attend_tile_mma decides and attends all of them.
template <int D, int GBM, bool kTicketed, int kTiles = 1>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2)))
void step_kernel(StepArgs s) {
  static_assert(kTiles == 1 || (!kTicketed && GBM == 4), "several tiles: resident 4-row step");
  __shared__ StepShared<D, GBM, kTiles> sh;
  const ScoreArgs& sa = s.score;
  const int G = sa.group, tid = threadIdx.x, lane = tid % kWave;
  const uint32_t W = (uint32_t)s.attend.workers;
#if defined(RKV_PHASE_STAMPS)
  unsigned long long* const stamps = sh.stamps;
  if (tid < kStamps) stamps[tid] = 0ull;
#else
  unsigned long long* const stamps = nullptr;
#endif
  RKV_STAMP(stamps, kStEntry, tid == 0);
  // this launch's epoch, from the workgroup's own launch counter: its tag
  // marks the slots the launch publishes (read only after the score loads
  // are issued: a read right after the atomic would wait out its round trip)
  uint64_t epoch = 0;
  if (tid == 0)
    epoch = __hip_atomic_fetch_add(
        s.control + ((int64_t)s.heads + 1) * kLine + (int64_t)blockIdx.y * sa.tile_stride +
            blockIdx.x,
        1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // workgroup wk of head h scores tile wk % n_tiles (copies past the first
  // n_tiles with short prompts, see attend_tile): blockIdx, or with a grid
  // larger than the device holds at once, the ticket this workgroup draws as
  // it starts (launch e's tickets are e * grid + 0 .. grid - 1)
  int64_t h = blockIdx.y, wk = blockIdx.x;
  if constexpr (kTicketed) {
    if (tid == 0) {
      const uint64_t t = __hip_atomic_fetch_add(s.control + (int64_t)s.heads * kLine + 1, 1ull,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      sh.ticket = (uint32_t)(t - epoch * (uint64_t)(W * gridDim.y));
    }
    __syncthreads();
    const uint32_t t = __builtin_amdgcn_readfirstlane(sh.ticket);
    h = t / W;
    wk = t % W;
  }
  const int64_t tile = wk % (int64_t)s.attend.decide.n_tiles;
  const StepCtx sx{StepStats{sh.zs, Coherent(s.lse_slots, s.slots_bytes), &sh.tag, &sh.rtag,
                             s.error, s.spin, stamps, &sh.gave_up},
                   Coherent(s.attend.part_ml, s.ml_bytes),
                   Coherent(s.attend.part_acc, s.acc_bytes),
                   Coherent(s.counts, s.counts_bytes),
                   Coherent(s.attend.decide.mask, s.mask_bytes),
                   s.out,
                   s.accessed,
                   sh.wsum,
                   kTiles == 1 ? s.full + h * sa.tile_stride + wk : nullptr,
                   &sh.spec};
  // whether the previous launch on the workspace expanded every block of
  // this workgroup's tile (it left that launch's tag + 1 in its flag)
  // (a workgroup of several tiles does not speculate)
  uint64_t prev_full = 0;
  if (kTiles == 1 && tid == 0 && s.speculate)
    prev_full = __hip_atomic_load(s.full + h * sa.tile_stride + wk, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
  // (8-row passes: one query row's slice of q at a time, as the score kernel
  // does; holding four rows' across both passes spilled)
  score_dots<D, GBM, (GBM > 4)>(sa, h, tile, sh.u.score.sdot, sh.u.score.pdot, sh.u.score.q);
  RKV_STAMP(stamps, kStDots, tid == 0);
  // (the epoch is read before the loads below are issued: loads complete in
  // order, so a later read would wait for them too)
  if (tid == 0) {
    sh.gave_up = 0u;
    sh.tag = (uint32_t)epoch + 1u;
    sh.rtag = sh.tag + s.skew;
    sh.spec = s.speculate && prev_full == epoch + 1u ? 1u : 0u;
  }
  // the attention's loads that need no statistics land during them (with
  // several tiles after the last tile's statistics: the query operands
  // would stay live through the later tiles' scores)
  MmaLoads<D> ld;
  if constexpr (kTiles == 1) ld = mma_issue<D, GBM, true>(s.attend, h, (uint32_t)wk);
  __syncthreads();
  // a tile's LSE partials out as two tagged slots
  auto publish = [&](int64_t t, int g, float4 part) {
    const uint32_t at = (uint32_t)(((h * G + g) * sa.tile_stride + t) * 2 * 16);
    const uint32_t tag = __builtin_amdgcn_readfirstlane(sh.tag);
    sx.stats.slots.store4(at, make_slot(f32_bits(part.x), f32_bits(part.y), tag));
    sx.stats.slots.store4(at + 16, make_slot(f32_bits(part.z), f32_bits(part.w), tag));
  };
  if constexpr (kTiles == 1) {
    score_stats(
        sa, tile, sh.u.score.sdot, sh.u.score.pdot,
        [&](int g, bool, float4 zf) { sh.zs[g][lane] = zf; },
        [&](int g, float4 part) { publish(tile, g, part); });
    __syncthreads();
    RKV_STAMP(stamps, kStStats, tid == 0);
    // (the score arrays are dead: the representative rows and the first
    // suffix chunks stage over them and land while the decision waits for
    // the head's LSE partials)
    attend_tile_mma<D, GBM, true>(s.attend, sh.dec, sh.u.cmb, &sx, ld, h, (uint32_t)wk);
  } else {
    const uint32_t T = (uint32_t)s.attend.decide.n_tiles;
    const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
    TileSet<kTiles, GBM> tset;
    tset.n = (T - (uint32_t)wk + W - 1u) / W;
    tset.z = sh.tz.z;
#pragma unroll
    for (int m = 0; m < kTiles; ++m) tset.zown[m] = make_float4(kNegInf, 0.0f, 0.0f, 0.0f);
    // tile m + 1's summary loads are issued before tile m's statistics (and
    // land during them); its dot products follow the statistics (a barrier
    // first: the statistics read the score arrays), from q as staged for
    // tile 0
    ScoreRaw<D> next;
#pragma unroll
    for (int m = 0; m < kTiles; ++m) {
      if ((uint32_t)m >= tset.n) break;
      const int64_t t = wk + (int64_t)m * W;
      const bool more = (uint32_t)m + 1u < tset.n;
      if (more) score_load<D>(sa, h, t + W, next);
      score_stats(
          sa, t, sh.u.score.sdot, sh.u.score.pdot,
          [&](int g, bool, float4 zf) {
            sh.tz.z[m][g][lane] = zf.x;
            if (g == wave) tset.zown[m] = zf;
          },
          [&](int g, float4 part) { publish(t, g, part); });
      if (more) {
        __syncthreads();
        score_from<D, GBM>(sa, next, sh.u.score.sdot, sh.u.score.pdot, sh.u.score.q);
      }
    }
    ld = mma_issue<D, GBM, true>(s.attend, h, (uint32_t)wk);
    tset.din[0] = ld.din;
#pragma unroll
    for (int m = 1; m < kTiles; ++m)
      if ((uint32_t)m < tset.n) tset.din[m] = decide_issue<false>(s.attend.decide, h, wk + (int64_t)m * W);
    __syncthreads();
    RKV_STAMP(stamps, kStStats, tid == 0);
    attend_tile_mma<D, GBM, true, kTiles>(s.attend, sh.dec, sh.u.cmb, &sx, ld, h, (uint32_t)wk,
                                          &tset);
  }
#if defined(RKV_PHASE_STAMPS)
  RKV_STAMP(stamps, kStEnd, tid == 0);
  __syncthreads();
  if (tid < kStamps && h < kStampHeads && wk < kStampRowsPerHead)
    rkv_stamps[h * kStampRowsPerHead + wk][tid] = stamps[tid];
#endif
}

// ---------------------------------------------------------------------------
// Kernel 3: merge a row's tile partials -> bf16 output columns
// ---------------------------------------------------------------------------
struct MergeArgs {
  const float2* part_ml;  // (H*G, tile_stride): m, l
  const float* part_acc;  // (H*G, tile_stride, D)
  uint16_t* out;          // (H*G, D)
  const uint32_t* tile_counts;     // (H, tile_stride) or null
  unsigned long long* accessed;    // or null
  int64_t tile_stride;
  int parts, dim, heads;
};

// merge_kernel<MD, MB>: MD output columns per workgroup, kThreads / MD
// partial stripes, MB partials per lane per batch of loads.  Few partials
// (the dense decode's splits, a head of up to 128 tiles): 32 columns, 8
// stripes of batches of 8; many (more tiles): 8 columns, so that the
// workgroups fill the device and each stripe takes one or two batches of 16.
constexpr int kMergeFewParts = 128;

// Online merge of one partial into (mx, num, den); skips empty partials.
__device__ __forceinline__ void merge_one(float m, float l, float acc, float& mx, float& num,
                                          float& den) {
  if (!(l > 0.0f)) return;
  if (m > mx) {
    const float s = mx == kNegInf ? 0.0f : __builtin_amdgcn_exp2f((mx - m) * kLog2e);
    num = num * s + acc;
    den = den * s + l;
    mx = m;
  } else {
    const float e = __builtin_amdgcn_exp2f((m - mx) * kLog2e);
    num = __builtin_fmaf(acc, e, num);
    den = __builtin_fmaf(l, e, den);
  }
}

template <int kMergeD, int kMergeBatch>
__global__ __launch_bounds__(kThreads) void merge_kernel(MergeArgs a) {
  constexpr int kMergeK = kThreads / kMergeD;  // partial stripes
  __shared__ float sm[kMergeK], sd[kMergeK], sn[kMergeK][kMergeD];
  __shared__ unsigned long long wsum[kWaves];
  const int64_t r = blockIdx.x;
  const int P = a.parts, D = a.dim;
  const int tid = threadIdx.x, dl = tid % kMergeD, kk = tid / kMergeD;
  const int d = blockIdx.y * kMergeD + dl;
  const int dd = d < D ? d : 0;
  const float2* pml = a.part_ml + r * a.tile_stride;
  const float* pa = a.part_acc + r * a.tile_stride * D + dd;
  float mx = kNegInf, num = 0.0f, den = 0.0f;
  for (int i0 = kk; i0 < P; i0 += kMergeK * kMergeBatch) {
    float mv[kMergeBatch], lv[kMergeBatch], av[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) {
      const int i = i0 + u * kMergeK;
      const int ii = i < P ? i : 0;
      const float2 ml = pml[ii];
      mv[u] = ml.x;
      lv[u] = ml.y;
      av[u] = pa[(int64_t)ii * D];
      if (i >= P) lv[u] = 0.0f;
    }
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u) merge_one(mv[u], lv[u], av[u], mx, num, den);
  }
  sn[kk][dl] = num;
  if (dl == 0) {
    sm[kk] = mx;
    sd[kk] = den;
  }
  __syncthreads();
  if (tid < kMergeD && d < D) {
    float m2 = kNegInf, n2 = 0.0f, d2 = 0.0f;
    for (int j = 0; j < kMergeK; ++j) merge_one(sm[j], sd[j], sn[j][tid], m2, n2, d2);
    a.out[r * D + d] = bf16_rne(n2 / fmaxf(d2, 1e-30f));
  }
  // the step's access count: sum of the tile counts, added once
  if (a.accessed && blockIdx.x == 0 && blockIdx.y == 0) {
    // (the loads of a batch are issued together: one round trip per batch)
    unsigned long long s = 0;
    const int64_t n = (int64_t)a.heads * a.tile_stride;
    for (int64_t i0 = tid; i0 < n; i0 += kThreads * kMergeBatch) {
      uint32_t c[kMergeBatch];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const int64_t i = i0 + (int64_t)u * kThreads;
        c[u] = i < n ? a.tile_counts[i] : 0u;
      }
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) s += c[u];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s += __shfl_xor(s, o, kWave);
    if (tid % kWave == 0) wsum[tid / kWave] = s;
    __syncthreads();
    if (tid == 0) atomicAdd(a.accessed, ((wsum[0] + wsum[1]) + wsum[2]) + wsum[3]);
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
int launch_merge(const MergeArgs& ma, int64_t rows, int64_t dim, hipStream_t stream) {
  if (ma.parts <= kMergeFewParts)
    merge_kernel<32, 8><<<dim3((unsigned)rows, (unsigned)((dim + 31) / 32)), dim3(kThreads), 0,
                          stream>>>(ma);
  else
    merge_kernel<8, 16><<<dim3((unsigned)rows, (unsigned)((dim + 7) / 8)), dim3(kThreads), 0,
                          stream>>>(ma);
  return check_launch("merge_kernel");
}

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
  if (score_smem(p.group, p.dim) > 64 * 1024)
    return set_error(kUnsupported, "%s: group x head_dim too large", who);
  return kOk;
}

ScoreArgs score_args(const SelectParams& p, const Layout& L) {
  ScoreArgs sa;
  sa.query = static_cast<const uint16_t*>(p.query);
  sa.key_mean = static_cast<const uint16_t*>(p.key_mean);
  sa.ellipsoid = static_cast<const uint16_t*>(p.ellipsoid);
  sa.zf = at<float4>(p.ws, L.zf);
  sa.lse = at<float>(p.ws, L.lse);
  sa.n_blocks = p.n_blocks;
  sa.block = p.block;
  sa.length = p.length;
  sa.z_stride = L.z_stride;
  sa.tile_stride = L.tile_stride;
  sa.group = (int)p.group;
  sa.summary_heads = (int)p.heads;
  sa.scale = (float)pow((double)p.dim, -0.5);
  // (the oracle's logf_, on the host: z stays bit-exact)
  sa.ln_full = logf_((float)p.block);
  sa.ln_last = logf_((float)(p.length - (p.n_blocks - 1) * p.block));
  return sa;
}

DecideArgs decide_args(const SelectParams& p, const Layout& L) {
  DecideArgs da;
  da.zf = at<float4>(p.ws, L.zf);
  da.lse = at<float>(p.ws, L.lse);
  da.value_norm = p.value_norm;
  da.max_value_norm = p.max_value_norm;
  da.anchor = p.anchor;
  da.mask = p.mask;
  da.write_mask = true;
  da.risk_out = p.risk_out;
  da.stats_out = p.stats_out;
  da.row_lse = nullptr;
  da.n_blocks = p.n_blocks;
  da.n_tiles = L.n_tiles;
  da.block = p.block;
  da.length = p.length;
  da.z_stride = L.z_stride;
  da.tile_stride = L.tile_stride;
  da.group = (int)p.group;
  da.reduction = p.reduction;
  da.eps = p.eps;
  return da;
}

int launch_score(const SelectParams& p, const Layout& L, int64_t queries = 1) {
  const ScoreArgs sa = score_args(p, L);
  const dim3 grid((unsigned)L.n_tiles, (unsigned)(p.heads * queries));
  RKV_DISPATCH_DIM(p.dim, D,
                   score_kernel<D><<<grid, dim3(kThreads), score_smem(p.group, p.dim),
                                     p.stream>>>(sa));
  return check_launch("score_kernel");
}

// With more than 64 tiles per head the rows' log Z / log C are merged once
// (lse_merge_kernel) and every tile's decision reads them: da.row_lse.
int launch_lse_merge(const SelectParams& p, const Layout& L, int64_t queries, DecideArgs& da) {
  if (L.n_tiles <= kWave) return kOk;
  const int64_t rows = p.heads * queries * p.group;
  float* row_lse = at<float>(p.ws, L.row_lse);
  lse_merge_kernel<<<dim3((unsigned)((rows + kWaves - 1) / kWaves)), dim3(kThreads), 0,
                     p.stream>>>(at<float>(p.ws, L.lse), row_lse, rows, L.n_tiles, L.tile_stride);
  const int rc = check_launch("lse_merge_kernel");
  if (rc == kOk) da.row_lse = row_lse;
  return rc;
}

// Selection only (rkv_select): score and decide kernels.
int launch_select(const SelectParams& p, const Layout& L) {
  mark(0, p.stream);
  int rc = launch_score(p, L);
  if (rc) return rc;
  mark(1, p.stream);
  DecideArgs da = decide_args(p, L);
  if ((rc = launch_lse_merge(p, L, 1, da))) return rc;
  decide_kernel<<<dim3((unsigned)L.n_tiles, (unsigned)p.heads), dim3(kThreads), 0, p.stream>>>(
      da, p.accessed);
  rc = check_launch("decide_kernel");
  mark(2, p.stream);
  return rc;
}

// Batched anchor selection: score every (query, head, tile), then one
// workgroup per (tile, head) ORs the queries' decisions.  The layout is the
// one of heads * anchors heads.
int launch_select_anchors(const SelectParams& p, int64_t anchors) {
  const Layout L = make_layout(p.heads * anchors, p.group, p.dim, p.n_blocks);
  int rc = launch_score(p, L, anchors);
  if (rc) return rc;
  DecideArgs da = decide_args(p, L);
  da.write_mask = false;  // the mask only stands in for the (absent) anchor input
  if ((rc = launch_lse_merge(p, L, anchors, da))) return rc;
  anchor_decide_kernel<<<dim3((unsigned)L.n_tiles, (unsigned)p.heads), dim3(kThreads), 0,
                         p.stream>>>(da, (int)anchors, (int)p.heads, p.mask);
  return check_launch("anchor_decide_kernel");
}

struct DecodeBuffers {
  const void* value_mean;
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
  aa.value_mean = static_cast<const uint16_t*>(b.value_mean);
  aa.key_pages = static_cast<const uint16_t*>(b.key_pages);
  aa.value_pages = static_cast<const uint16_t*>(b.value_pages);
  // with no suffix the pages stand in (never read: no suffix rows)
  aa.key_suffix = static_cast<const uint16_t*>(b.suffix_cap ? b.key_suffix : b.key_pages);
  aa.value_suffix = static_cast<const uint16_t*>(b.suffix_cap ? b.value_suffix : b.value_pages);
  aa.suffix_len_dev = b.suffix_len;
  aa.part_ml = at<float2>(p.ws, L.part_ml);
  aa.part_acc = at<float>(p.ws, L.part_acc);
  aa.tile_counts = p.accessed ? at<uint32_t>(p.ws, L.counts) : nullptr;
  aa.kp_hs = b.kp_hs;
  aa.vp_hs = b.vp_hs;
  aa.ks_hs = b.ks_hs;
  aa.ks_ts = b.ks_ts;
  aa.vs_hs = b.vs_hs;
  aa.vs_ts = b.vs_ts;
  aa.suffix_cap = b.suffix_cap;
  aa.log2_block = p.block == 16 ? 4 : (p.block == 32 ? 5 : 6);
  aa.workers = (int)L.n_tiles;
  aa.scale = (float)pow((double)p.dim, -0.5);
  return aa;
}

MergeArgs merge_args(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  MergeArgs ma;
  ma.part_ml = at<float2>(p.ws, L.part_ml);
  ma.part_acc = at<float>(p.ws, L.part_acc);
  ma.out = static_cast<uint16_t*>(b.output);
  ma.tile_counts = at<uint32_t>(p.ws, L.counts);
  ma.accessed = p.accessed;
  ma.tile_stride = L.tile_stride;
  ma.parts = (int)L.n_tiles;
  ma.dim = (int)p.dim;
  ma.heads = (int)p.heads;
  return ma;
}

template <int D>
int launch_attend(const AttendArgs& aa, int64_t rows, dim3 grid, hipStream_t stream) {
  constexpr int CH = D / 16;
  constexpr int CAP = (64 / CH) >= 16 ? 16 : ((64 / CH) >= 8 ? 8 : 4);
  switch (rows) {
    case 4:
      attend_kernel<D, 4><<<grid, dim3(kThreads), 0, stream>>>(aa);
      return check_launch("attend_kernel");
    case 8:
      if constexpr (CAP >= 8) {
        attend_kernel<D, 8><<<grid, dim3(kThreads), 0, stream>>>(aa);
        return check_launch("attend_kernel");
      }
      break;
    default:
      if constexpr (CAP >= 16) {
        attend_kernel<D, 16><<<grid, dim3(kThreads), 0, stream>>>(aa);
        return check_launch("attend_kernel");
      }
      break;
  }
  return set_error(kUnsupported, "rkv_decode: no attention kernel for this group");
}

// The one-launch step is built for head_dim <= kStepMaxDim: at head_dim 160
// its one resident workgroup per two CUs spills registers (its ring of
// representative, suffix and page chunks, or both rings, hold more than the
// 256 a wave has at two waves per SIMD), so 160 and above take the three
// kernels.
constexpr int kStepMaxDim = 128;

template <int D, int GBM>
int launch_step_g(const StepArgs& sa, bool ticketed, bool multi, dim3 grid, hipStream_t stream) {
  if constexpr (GBM == 4 && D <= 128) {
    if (multi) {
      step_kernel<D, GBM, false, kStepTiles><<<grid, dim3(kThreads), 0, stream>>>(sa);
      return check_launch("step_kernel");
    }
  }
  if (multi) return set_error(kUnsupported, "rkv_decode: no several-tile step for this shape");
  if (ticketed) step_kernel<D, GBM, true><<<grid, dim3(kThreads), 0, stream>>>(sa);
  else step_kernel<D, GBM, false><<<grid, dim3(kThreads), 0, stream>>>(sa);
  return check_launch("step_kernel");
}

template <int D>
int launch_step_d(const StepArgs& sa, int64_t rows, bool ticketed, bool multi, dim3 grid,
                  hipStream_t stream) {
  constexpr int CH = D / 16;
  constexpr int CAP = (64 / CH) >= 16 ? 16 : ((64 / CH) >= 8 ? 8 : 4);
  if constexpr (D <= kStepMaxDim) {
    switch (rows) {
      case 4:
        return launch_step_g<D, 4>(sa, ticketed, multi, grid, stream);
      case 8:
        if constexpr (CAP >= 8) return launch_step_g<D, 8>(sa, ticketed, multi, grid, stream);
        break;
      default:
        if constexpr (CAP >= 16) return launch_step_g<D, 16>(sa, ticketed, multi, grid, stream);
        break;
    }
  }
  return set_error(kUnsupported, "rkv_decode: no step kernel for this group");
}

// Which path rkv_decode takes (rkv_set_decode_path, per thread): 0 = the
// one-launch step where the shape allows it, else three kernels; 1 = always
// the three kernels.
thread_local int g_decode_path = 0;

// Workgroups of step_kernel<D, GBM> the current device holds at once (its
// occupancy per CU times the CUs), 0 if unknown.
template <int D, int GBM, int kTiles = 1>
int64_t step_resident() {  // (the ticketed build's occupancy is the same: same resources)
  static std::atomic<int> of_dev[64];  // per device; 0 = not asked yet
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = of_dev[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, step_kernel<D, GBM, false, kTiles>,
                                                     kThreads, 0) !=
            hipSuccess)
      return 0;
    n = cus * per_cu;
    of_dev[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// The residency of the step kernel launch_step_d<D> takes for `rows` rows
// (multi: the several-tile build).
template <int D>
int64_t step_resident_d(int64_t rows, bool multi) {
  constexpr int CH = D / 16;
  constexpr int CAP = (64 / CH) >= 16 ? 16 : ((64 / CH) >= 8 ? 8 : 4);
  if constexpr (D <= kStepMaxDim) {
    if constexpr (D <= 128)
      if (rows == 4 && multi) return step_resident<D, 4, kStepTiles>();
    if (multi) return 0;
    if (rows == 4) return step_resident<D, 4>();
    if constexpr (CAP >= 8)
      if (rows == 8) return step_resident<D, 8>();
    if constexpr (CAP >= 16)
      if (rows == 16) return step_resident<D, 16>();
  }
  return 0;
}

// How rkv_decode runs a step.
enum StepMode { kSplit = 0, kResident = 1, kTicketed = 2 };

// The one-launch step needs every query row in one attention pass, at most
// kStepMaxTiles tiles per head, its coherent regions addressable with 31-bit
// byte offsets, an 8-byte aligned output (it stores 4 columns at a time) and
// every workgroup a wait depends on running: the whole grid resident at once
// (kResident), or, with blocks of 64 tokens (measured faster than the three
// kernels there), a grid of up to two device-fulls whose workgroups draw
// their (head, workgroup) from start-order tickets (kTicketed: a head's W
// workgroups must fit the device at once).
StepMode step_mode(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  const int64_t rows = rows_per_pass(p.group, p.dim);
  const int64_t hg = p.heads * p.group, ts = L.tile_stride;
  const int64_t limit = int64_t(1) << 31;
  if (!(p.dim <= kStepMaxDim && p.group <= rows && L.n_tiles <= kStepMaxTiles &&
        hg * ts * 32 < limit && hg * ts * p.dim * 8 < limit && p.heads * ts * 16 < limit &&
        p.heads * p.n_blocks < limit && aligned(b.output, 8)))
    return kSplit;
  int64_t resident = 0;
  const bool multi = L.step_tiles > 1;
  RKV_DISPATCH_DIM(p.dim, D, resident = step_resident_d<D>(rows, multi));
  const int64_t grid = p.heads * L.step_workers;
  if (grid <= resident) return kResident;
  if (!multi && p.block >= 64 && L.step_workers <= resident && grid <= 2 * resident)
    return kTicketed;
  return kSplit;
}

// The status word the step's waits report to: the workspace's own (null),
// or the static scratch's fixed word while rkv_decode_static runs.
thread_local uint32_t* g_error_word = nullptr;

// Test hooks (rkv_set_handoff_test, per thread): the step's poll limit per
// wait (0 = kSpinLimit) and a tag skew that makes every wait run out.
thread_local uint32_t g_spin_limit = 0;
thread_local uint32_t g_skew = 0;
// Test hook (rkv_set_speculation, per thread): 0 turns the step's
// speculation off, 1 (default) and 2 leave it on.  (A miss costs a
// workgroup at most three chunks' loads per wave, and only where the previous
// launch expanded all of its tile, so it needs no size threshold.)
thread_local uint32_t g_speculate = 1;

int launch_step(const SelectParams& p, const Layout& L, const DecodeBuffers& b, bool ticketed) {
  StepArgs s;
  s.score = score_args(p, L);
  s.attend = attend_args(p, L, b);
  s.attend.workers = (int)L.step_workers;
  s.control = at<uint64_t>(p.ws, L.control);
  s.counts = at<uint32_t>(p.ws, L.counts);
  s.attend.tile_counts = p.accessed ? s.counts : nullptr;
  s.out = static_cast<uint16_t*>(b.output);
  s.accessed = p.accessed;
  const int64_t hg = p.heads * p.group, ts = L.tile_stride;
  s.lse_slots = at<float4>(p.ws, L.lse_slots);
  s.slots_bytes = (uint32_t)(hg * ts * 32);
  s.ml_bytes = (uint32_t)(hg * ts * 16);
  s.acc_bytes = (uint32_t)(hg * ts * p.dim * 8);
  s.counts_bytes = (uint32_t)(p.heads * ts * 16);
  s.mask_bytes = (uint32_t)(p.heads * p.n_blocks);
  s.full = at<uint64_t>(p.ws, L.full);
  s.error = g_error_word != nullptr
                ? g_error_word
                : reinterpret_cast<uint32_t*>(s.control + (int64_t)p.heads * kLine);
  s.heads = (int)p.heads;
  s.spin = g_spin_limit ? g_spin_limit : kSpinLimit;
  s.skew = g_skew;
  s.speculate = g_speculate != 0 && L.step_tiles == 1 ? 1u : 0u;
  const int64_t rows = rows_per_pass(p.group, p.dim);
  mark(0, p.stream);
  int rc = kUnsupported;
  RKV_DISPATCH_DIM(p.dim, D,
                   rc = launch_step_d<D>(s, rows, ticketed, L.step_tiles > 1,
                                         dim3((unsigned)L.step_workers, (unsigned)p.heads),
                                         p.stream));
  mark(1, p.stream);
  return rc;
}

// One decode step: the one-launch step, or score, decide + attend, merge.
int launch_decode(const SelectParams& p, const Layout& L, const DecodeBuffers& b) {
  if (g_decode_path == 0) {
    const StepMode mode = step_mode(p, L, b);
    if (mode != kSplit) return launch_step(p, L, b, mode == kTicketed);
  }
  AttendArgs aa = attend_args(p, L, b);
  const MergeArgs ma = merge_args(p, L, b);
  const int64_t rows = rows_per_pass(p.group, p.dim);
  const dim3 tiles((unsigned)L.n_tiles, (unsigned)p.heads, (unsigned)((p.group + rows - 1) / rows));
  mark(0, p.stream);
  int rc = launch_score(p, L);
  if (rc) return rc;
  mark(1, p.stream);
  if ((rc = launch_lse_merge(p, L, 1, aa.decide))) return rc;
  rc = kUnsupported;
  RKV_DISPATCH_DIM(p.dim, D, rc = launch_attend<D>(aa, rows, tiles, p.stream));
  if (rc) return rc;
  mark(2, p.stream);
  rc = launch_merge(ma, p.heads * p.group, p.dim, p.stream);
  mark(3, p.stream);
  return rc;
}

// ---- dense decode -----------------------------------------------------------
// Workgroups of dense_kernel<D, GBM> the current device holds at once, 0 if
// unknown.
template <int D, int GBM>
int64_t dense_resident() {
  static std::atomic<int> of_dev[64];  // per device; 0 = not asked yet
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = of_dev[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    int cus = 0, per_cu = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, dense_kernel<D, GBM>, kThreads,
                                                     0) != hipSuccess)
      return 0;
    n = cus * per_cu;
    of_dev[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

constexpr int64_t kDenseMaxSplits = 1024;

// Query rows per workgroup (the matrix core's 16 columns hold up to 16) and
// the split of each head's tokens: enough workgroups to fill the device
// once, each wave with at least one 16-token chunk of the longest length.
struct DensePlan {
  int64_t rows = 0, passes = 0, splits = 0;
  size_t ml_off = 0, acc_off = 0, total = 0;
};

inline int64_t dense_rows(int64_t group) { return group <= 4 ? 4 : (group <= 8 ? 8 : 16); }

DensePlan dense_plan(int64_t heads, int64_t group, int64_t dim, int64_t cap) {
  DensePlan P;
  P.rows = dense_rows(group);
  P.passes = (group + P.rows - 1) / P.rows;
  int64_t resident = 0;
  RKV_DISPATCH_DIM(dim, D, {
    if constexpr (D <= kMmaMaxDim) {
      if (P.rows == 4) resident = dense_resident<D, 4>();
      else if (P.rows == 8) resident = dense_resident<D, 8>();
      else resident = dense_resident<D, 16>();
    }
  });
  if (resident <= 0) resident = 512;
  const int64_t chunks = (cap + 15) / 16;
  int64_t splits = resident / (heads * P.passes);
  const int64_t most = chunks / kWaves > 1 ? chunks / kWaves : 1;
  splits = splits < most ? splits : most;
  splits = splits < kDenseMaxSplits ? splits : kDenseMaxSplits;
  P.splits = splits > 1 ? splits : 1;
  auto up = [](size_t x) { return (x + 255) & ~(size_t)255; };
  const size_t parts = (size_t)(heads * group * P.splits);
  P.ml_off = 0;
  P.acc_off = up(parts * 8);
  P.total = P.acc_off + up(parts * (size_t)dim * 4);
  return P;
}

struct DenseParams {
  const void* query;
  const void* keys;
  const void* values;
  int64_t k_hs, k_ts, v_hs, v_ts;
  int64_t heads, group, dim, length;
  const int32_t* length_dev;
  void* workspace;
  size_t workspace_bytes;
  void* out;
  hipStream_t stream;
};

template <int D>
int launch_dense_d(const DenseArgs& da, int64_t rows, dim3 grid, hipStream_t stream) {
  if constexpr (D <= kMmaMaxDim) {
    if (rows == 4) dense_kernel<D, 4><<<grid, dim3(kThreads), 0, stream>>>(da);
    else if (rows == 8) dense_kernel<D, 8><<<grid, dim3(kThreads), 0, stream>>>(da);
    else dense_kernel<D, 16><<<grid, dim3(kThreads), 0, stream>>>(da);
    return check_launch("dense_kernel");
  }
  return set_error(kUnsupported, "rkv_dense_decode: head_dim %d above %d", D, kMmaMaxDim);
}

int validate_dense(const DenseParams& p, DensePlan& P) {
  const char* who = "rkv_dense_decode";
  if (!p.query || !p.keys || !p.values || !p.out)
    return set_error(kInvalidArgument, "%s: null pointer argument", who);
  if (p.heads <= 0 || p.group <= 0 || p.length <= 0 || p.heads > 65535)
    return set_error(kInvalidArgument, "%s: empty or oversized shape", who);
  if (p.group > 16) return set_error(kUnsupported, "%s: GQA group %lld exceeds 16", who,
                                     (long long)p.group);
  if (p.dim < 32 || p.dim > kMmaMaxDim || p.dim % 32)
    return set_error(kUnsupported, "%s: head_dim %lld not in 32..%d step 32", who,
                     (long long)p.dim, kMmaMaxDim);
  if (p.k_ts < p.dim || p.v_ts < p.dim || p.k_hs < 0 || p.v_hs < 0 || p.k_ts % 8 ||
      p.v_ts % 8 || p.k_hs % 8 || p.v_hs % 8)
    return set_error(kInvalidArgument,
                     "%s: token strides must be >= head_dim and strides multiples of 8", who);
  if (!aligned(p.query, 16) || !aligned(p.keys, 16) || !aligned(p.values, 16) ||
      !aligned(p.out, 16))
    return set_error(kInvalidArgument, "%s: query, keys, values and out must be 16-byte aligned",
                     who);
  // a head's keys (values) are addressed with 32-bit byte offsets
  const int64_t lim = (int64_t(1) << 32) - 1;
  if ((p.length - 1) * p.k_ts * 2 + p.dim * 2 > lim || (p.length - 1) * p.v_ts * 2 + p.dim * 2 > lim)
    return set_error(kUnsupported, "%s: a head's keys or values span more than 4 GiB", who);
  P = dense_plan(p.heads, p.group, p.dim, p.length);
  if (!p.workspace || p.workspace_bytes < P.total)
    return set_error(kWorkspaceTooSmall, "%s: workspace of %zu bytes, %zu needed", who,
                     p.workspace_bytes, P.total);
  if (!aligned(p.workspace, 16))
    return set_error(kInvalidArgument, "%s: workspace must be 16-byte aligned", who);
  return kOk;
}

int launch_dense(const DenseParams& p, const DensePlan& P) {
  char* ws = static_cast<char*>(p.workspace);
  DenseArgs da;
  da.query = static_cast<const uint16_t*>(p.query);
  da.keys = static_cast<const uint16_t*>(p.keys);
  da.values = static_cast<const uint16_t*>(p.values);
  da.k_hs = p.k_hs;
  da.v_hs = p.v_hs;
  da.k_ts = (uint32_t)p.k_ts;
  da.v_ts = (uint32_t)p.v_ts;
  da.length_dev = p.length_dev;
  da.cap = (uint32_t)p.length;
  da.group = (int)p.group;
  da.splits = (int)P.splits;
  da.scale = (float)pow((double)p.dim, -0.5);
  da.part_ml = reinterpret_cast<float2*>(ws + P.ml_off);
  da.part_acc = reinterpret_cast<float*>(ws + P.acc_off);
  const dim3 grid((unsigned)P.splits, (unsigned)p.heads, (unsigned)P.passes);
  int rc = kUnsupported;
  RKV_DISPATCH_DIM(p.dim, D, rc = launch_dense_d<D>(da, P.rows, grid, p.stream));
  if (rc) return rc;
  MergeArgs ma;
  ma.part_ml = da.part_ml;
  ma.part_acc = da.part_acc;
  ma.out = static_cast<uint16_t*>(p.out);
  ma.tile_counts = nullptr;
  ma.accessed = nullptr;
  ma.tile_stride = P.splits;
  ma.parts = (int)P.splits;
  ma.dim = (int)p.dim;
  ma.heads = (int)p.heads;
  return launch_merge(ma, p.heads * p.group, p.dim, p.stream);
}

}  // namespace
}  // namespace rkv

using namespace rkv;

extern "C" size_t rkv_workspace_bytes(int64_t heads, int64_t group, int64_t dim,
                                      int64_t n_blocks) {
  if (heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0) return 0;
  return (size_t)make_layout(heads, group, dim, n_blocks).total;
}

// Byte offsets of the workspace regions, for tests: control (hand-off
// counters), zf (z, delta, A, th per row and block), lse, lse_slots (the
// step's tagged LSE partials), part_ml, part_acc, counts, full (the step's
// per-workgroup speculation flags), total, then n_tiles, the row stride
// (blocks) of zf and of the per-tile arrays, and the step's workgroups per
// head.
extern "C" int rkv_workspace_layout(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                                    int64_t* out13) {
  clear_error();
  if (!out13 || heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_workspace_layout: bad arguments");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  const int64_t v[13] = {L.control,  L.zf,     L.lse,         L.lse_slots, L.part_ml,
                         L.part_acc, L.counts, L.full,        L.total,     L.n_tiles,
                         L.z_stride, L.tile_stride, L.step_workers};
  for (int i = 0; i < 13; ++i) out13[i] = v[i];
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

extern "C" int rkv_select_anchors(const void* queries, const void* key_mean,
                                  const void* ellipsoid, const float* value_norm,
                                  const float* max_value_norm, int64_t heads, int64_t group,
                                  int64_t dim, int64_t n_blocks, int64_t block_size,
                                  int64_t prompt_length, float eps, int reduction,
                                  int64_t anchors, uint8_t* mask_out, void* workspace,
                                  size_t workspace_bytes, hipStream_t stream) {
  clear_error();
  if (anchors <= 0 || anchors > 65535)
    return set_error(kInvalidArgument, "rkv_select_anchors: anchors must be in 1..65535");
  if (heads > 0 && heads * anchors > 65535)
    return set_error(kUnsupported, "rkv_select_anchors: heads x anchors exceeds 65535");
  SelectParams p{queries, key_mean, ellipsoid, value_norm, max_value_norm, heads, group, dim,
                 n_blocks, block_size, prompt_length, eps, reduction, nullptr, mask_out,
                 nullptr, nullptr, nullptr, workspace, workspace_bytes, stream};
  Layout L;
  int rc = validate_select(p, "rkv_select_anchors", L);
  if (rc) return rc;
  const Layout LA = make_layout(heads * anchors, group, dim, n_blocks);
  if (workspace_bytes < (size_t)LA.total)
    return set_error(kWorkspaceTooSmall,
                     "rkv_select_anchors: workspace needs %lld bytes (rkv_workspace_bytes of "
                     "heads x anchors heads)", (long long)LA.total);
  return launch_select_anchors(p, anchors);
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
  SelectParams p{query, key_mean, ellipsoid, value_norm, max_value_norm, heads, group, dim,
                 n_blocks, block_size, prompt_length, eps, reduction, anchor_mask, mask_out,
                 nullptr, nullptr, accessed_blocks, workspace, workspace_bytes, stream};
  Layout L;
  int rc = validate_select(p, "rkv_decode", L);
  if (rc) return rc;
  if (!key_pages || !value_pages || !output)
    return set_error(kInvalidArgument, "rkv_decode: null pointer argument");
  // the attention kernel addresses a head's pages with 32-bit element offsets
  if (n_blocks * block_size * dim >= (int64_t(1) << 31))
    return set_error(kUnsupported, "rkv_decode: more than 2^31 page elements per head");
  if (suffix_capacity < 0)
    return set_error(kInvalidArgument, "rkv_decode: negative suffix capacity");
  if (suffix_capacity > 0 && (!key_suffix || !value_suffix))
    return set_error(kInvalidArgument, "rkv_decode: null suffix with nonzero capacity");
  const int64_t es = 2;
  const int64_t ch_bytes = dim / 16 * es;
  const uintptr_t need = ch_bytes % 16 == 0 ? 16 : (ch_bytes % 8 == 0 ? 8 : 4);
  if (!aligned(value_mean, need))
    return set_error(kInvalidArgument, "rkv_decode: value_mean must be %d-byte aligned",
                     (int)need);
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

  const DecodeBuffers b{value_mean, key_pages, key_page_head_stride, value_pages,
                        value_page_head_stride, key_suffix, key_suffix_head_stride,
                        key_suffix_token_stride, value_suffix, value_suffix_head_stride,
                        value_suffix_token_stride, suffix_capacity, suffix_length, output};
  return launch_decode(p, L, b);
}

// Profiling hook: when events is non-null, the following rkv_select /
// rkv_decode calls on this thread record events[0] before their first kernel
// and events[k] after their k-th (rkv_select: score, decide; rkv_decode:
// step, or score, attend, merge).  Pass NULL to stop.
extern "C" int rkv_set_profile_events(void* events) {
  g_events = static_cast<hipEvent_t*>(events);
  return kOk;
}

// Test hook: 0 = rkv_decode uses the one-launch step where it fits (the
// default), 1 = always the three kernels.  Per thread.
extern "C" int rkv_set_decode_path(int path) {
  clear_error();
  if (path < 0 || path > 1) return set_error(kInvalidArgument, "rkv_set_decode_path: %d", path);
  g_decode_path = path;
  return kOk;
}

// Test hook: the one-launch step's poll limit per hand-off wait (0 = the
// default) and, with skew != 0, readers that accept no published slot, so
// that every wait runs out its limit, sets the error word and goes on (every
// kernel still ends).  Per thread.
extern "C" int rkv_set_handoff_test(uint32_t spin_limit, uint32_t skew) {
  clear_error();
  g_spin_limit = spin_limit;
  g_skew = skew;
  return kOk;
}

// Test hook: the one-launch step's speculation (issuing the first page rows
// of a workgroup's tile before the decision when the previous launch on the
// workspace expanded every block of it): 0 off, 1 (default) and 2 on.
// Results are the same bit for bit either way.  Per thread.
extern "C" int rkv_set_speculation(int mode) {
  clear_error();
  if (mode < 0 || mode > 2) return set_error(kInvalidArgument, "rkv_set_speculation: mode %d (0, 1 or 2)", mode);
  g_speculate = (uint32_t)mode;
  return kOk;
}

// Which path rkv_decode takes for a shape on the current device (with an
// aligned output): 0 = three kernels, 1 = one launch with the grid resident,
// 2 = one launch with start-order tickets, 3 = one resident launch whose
// workgroups score several tiles each.
extern "C" int rkv_decode_plan(int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                               int64_t block_size, int* mode_out) {
  clear_error();
  if (!mode_out || heads <= 0 || group <= 0 || n_blocks <= 0 || !supported_dim(dim) ||
      !supported_block(block_size) || group > kMaxGroup)
    return set_error(kInvalidArgument, "rkv_decode_plan: bad arguments");
  SelectParams p{};
  p.heads = heads;
  p.group = group;
  p.dim = dim;
  p.n_blocks = n_blocks;
  p.block = block_size;
  const Layout L = make_layout(heads, group, dim, n_blocks);
  DecodeBuffers b{};
  b.output = reinterpret_cast<void*>(uintptr_t(256));
  const StepMode mode = g_decode_path == 0 ? step_mode(p, L, b) : kSplit;
  *mode_out = mode == kResident && L.step_tiles > 1 ? 3 : (int)mode;
  return kOk;
}

namespace {
__global__ void clear_word_kernel(uint32_t* word) { *word = 0u; }
}  // namespace

// The hand-off status word of an rkv_decode workspace: bit 0 set when a wait
// of the one-launch step gave up (its output is then not to be trusted).
// Copies the word to the host and synchronizes `stream`; not for capture.
extern "C" int rkv_workspace_status(const void* workspace, size_t workspace_bytes,
                                    int64_t heads, int64_t group, int64_t dim, int64_t n_blocks,
                                    uint32_t* status, hipStream_t stream) {
  clear_error();
  if (!workspace || !status || heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_workspace_status: bad arguments");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  if (workspace_bytes < (size_t)L.total)
    return set_error(kWorkspaceTooSmall, "rkv_workspace_status: workspace smaller than its shape");
  const char* word = static_cast<const char*>(workspace) + L.control + heads * kLine * 8;
  uint32_t host = 0;
  if (hipMemcpyAsync(&host, word, sizeof(host), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return set_error(kLaunchFailed, "rkv_workspace_status: copy failed");
  *status = host;
  return kOk;
}

// Clears the status word (a one-thread kernel on `stream`, capturable).
extern "C" int rkv_workspace_clear_status(void* workspace, size_t workspace_bytes, int64_t heads,
                                          int64_t group, int64_t dim, int64_t n_blocks,
                                          hipStream_t stream) {
  clear_error();
  if (!workspace || heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_workspace_clear_status: bad arguments");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  if (workspace_bytes < (size_t)L.total)
    return set_error(kWorkspaceTooSmall,
                     "rkv_workspace_clear_status: workspace smaller than its shape");
  clear_word_kernel<<<1, 1, 0, stream>>>(
      reinterpret_cast<uint32_t*>(static_cast<char*>(workspace) + L.control + heads * kLine * 8));
  return check_launch("clear_word_kernel");
}

// ---------------------------------------------------------------------------
// rkv_decode_static: rkv_decode with the library's own device scratch
// ---------------------------------------------------------------------------
extern "C" const char* rkv_last_error(void);

namespace rkv {

// The scratch of rkv_decode_static: one array per GPU the library runs on,
// held until the process ends.  Host code never uses its name as an address:
// each device's copy is found with hipGetSymbolAddress.
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
static __device__ __align__(256) char scratch[kStaticScratchBytes];
// The static path's status word sits in the scratch's last 256 bytes, apart
// from any shape's workspace (whose layout is cleared on every call), so it
// keeps a failed wait's report until rkv_static_status clears it.
constexpr size_t kStaticWorkspaceBytes = kStaticScratchBytes - 256;

namespace {

constexpr int kMaxDevices = 64;
std::atomic<char*> g_scratch_ptr[kMaxDevices];

// This device's scratch address (looked up once per device, with it current).
int static_scratch(char** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return set_error(kLaunchFailed, "rkv_decode_static: no current device (or index >= %d)",
                     kMaxDevices);
  char* ptr = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    void* addr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || addr == nullptr)
      return set_error(kLaunchFailed, "rkv_decode_static: hipGetSymbolAddress: %s",
                       hipGetErrorString(err));
    ptr = static_cast<char*>(addr);
    g_scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return kOk;
}

// Zero-fills [begin, begin + bytes) (16-byte aligned, a multiple of 16).
__global__ void zero_fill_kernel(uint4* begin, int64_t n16) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16;
       i += (int64_t)gridDim.x * blockDim.x)
    begin[i] = make_uint4(0u, 0u, 0u, 0u);
}

int zero_region(char* base, int64_t off, int64_t bytes, hipStream_t stream) {
  const int64_t n16 = (bytes + 15) / 16;
  if (n16 == 0) return kOk;
  const int64_t blocks = (n16 + 255) / 256 < 1024 ? (n16 + 255) / 256 : 1024;
  zero_fill_kernel<<<dim3((unsigned)blocks), dim3(256), 0, stream>>>(
      reinterpret_cast<uint4*>(base + off), n16);
  return check_launch("zero_fill_kernel");
}

}  // namespace
}  // namespace rkv

// No counterpart in the reference: rkv_decode for callers that cannot
// allocate (HIP graph capture, serving loops, harnesses that forbid it).  The
// workspace is a file-scope device array of kStaticScratchBytes (64 MiB) per
// GPU; shapes whose rkv_workspace_bytes exceed it are rejected.  Each call
// first clears the array's hand-off counters and tagged slots (a fill kernel
// on `stream`), so calls of any shapes may follow each other; calls that
// overlap on one GPU (other streams, other threads) race on the array.
extern "C" int rkv_decode_static(const void* query, const void* key_mean, const void* ellipsoid,
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
                                 unsigned long long* accessed_blocks, hipStream_t stream) {
  clear_error();
  if (heads <= 0 || group <= 0 || dim <= 0 || n_blocks <= 0)
    return set_error(kInvalidArgument, "rkv_decode_static: empty shape");
  const Layout L = make_layout(heads, group, dim, n_blocks);
  if ((size_t)L.total > kStaticWorkspaceBytes)
    return set_error(kWorkspaceTooSmall,
                     "rkv_decode_static: this shape needs %lld bytes of workspace, more than the "
                     "static scratch's %lld; use rkv_decode with a caller workspace",
                     (long long)L.total, (long long)kStaticWorkspaceBytes);
  char* ws = nullptr;
  int rc = static_scratch(&ws);
  if (rc) return rc;
  // the one-launch step's counters and tagged slots start at zero (the
  // launch counters restart, so a slot left by an earlier call must not carry
  // a tag this call's launches use)
  if ((rc = zero_region(ws, L.control, control_bytes(heads, L.tile_stride), stream)) ||
      (rc = zero_region(ws, L.lse_slots, L.part_acc + heads * group * L.tile_stride * dim * 8 -
                                             L.lse_slots, stream)) ||
      (rc = zero_region(ws, L.counts, L.total - L.counts, stream)))
    return rc;
  g_error_word = reinterpret_cast<uint32_t*>(ws + kStaticWorkspaceBytes);
  rc = rkv_decode(query, key_mean, ellipsoid, value_mean, value_norm, max_value_norm, key_pages,
                  key_page_head_stride, value_pages, value_page_head_stride, key_suffix,
                  key_suffix_head_stride, key_suffix_token_stride, value_suffix,
                  value_suffix_head_stride, value_suffix_token_stride, suffix_capacity,
                  suffix_length, heads, group, dim, n_blocks, block_size, prompt_length, eps,
                  reduction, anchor_mask, mask_out, output, accessed_blocks, ws,
                  kStaticWorkspaceBytes, stream);
  g_error_word = nullptr;
  if (rc) {
    // rkv_decode's message names rkv_decode; say which entry point failed
    char message[512];
    snprintf(message, sizeof(message), "%s", rkv_last_error());
    return set_error(rc, "rkv_decode_static: %s", message);
  }
  return kOk;
}

// The static scratch's status word on the current device (bit 0: a wait of
// an rkv_decode_static call gave up since the word was last cleared; that
// call's output rows were written as NaN and its mask as all-expanded).
// Copies the word to the host and synchronizes `stream`; with clear != 0 it
// then zeroes the word (a one-thread kernel on `stream`).  Not for capture.
extern "C" int rkv_static_status(uint32_t* status, int clear, hipStream_t stream) {
  clear_error();
  if (!status) return set_error(kInvalidArgument, "rkv_static_status: null status");
  char* ws = nullptr;
  int rc = static_scratch(&ws);
  if (rc) return rc;
  uint32_t* word = reinterpret_cast<uint32_t*>(ws + kStaticWorkspaceBytes);
  uint32_t host = 0;
  if (hipMemcpyAsync(&host, word, sizeof(host), hipMemcpyDeviceToHost, stream) != hipSuccess ||
      hipStreamSynchronize(stream) != hipSuccess)
    return set_error(kLaunchFailed, "rkv_static_status: copy failed");
  *status = host;
  if (clear) {
    clear_word_kernel<<<1, 1, 0, stream>>>(word);
    return check_launch("clear_word_kernel");
  }
  return kOk;
}

// Dense decode of one token per query row over every cached token (no
// summary): out[h, g] = softmax(q[h, g] K_h^T / sqrt(D)) V_h over tokens
// 0 .. L - 1, L = *length_dev clamped to [0, length] when length_dev is
// given (graph replays), else length.
extern "C" int rkv_dense_plan(int64_t heads, int64_t group, int64_t dim, int64_t length,
                              int64_t* splits, size_t* workspace_bytes) {
  clear_error();
  if (heads <= 0 || group <= 0 || length <= 0 || dim <= 0)
    return set_error(kInvalidArgument, "rkv_dense_plan: empty shape");
  if (group > 16 || dim < 32 || dim > kMmaMaxDim || dim % 32)
    return set_error(kUnsupported, "rkv_dense_plan: group %lld / head_dim %lld not supported",
                     (long long)group, (long long)dim);
  const DensePlan P = dense_plan(heads, group, dim, length);
  if (splits) *splits = P.splits;
  if (workspace_bytes) *workspace_bytes = P.total;
  return kOk;
}

extern "C" int rkv_dense_decode(const void* query, const void* keys, int64_t key_head_stride,
                                int64_t key_token_stride, const void* values,
                                int64_t value_head_stride, int64_t value_token_stride,
                                int64_t heads, int64_t group, int64_t dim, int64_t length,
                                const int32_t* length_dev, void* output, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
  clear_error();
  const DenseParams p{query, keys, values, key_head_stride, key_token_stride,
                      value_head_stride, value_token_stride, heads, group, dim, length,
                      length_dev, workspace, workspace_bytes, output, stream};
  DensePlan P;
  const int rc = validate_dense(p, P);
  if (rc) return rc;
  return launch_dense(p, P);
}

#if defined(RKV_PHASE_STAMPS)
// The phase-stamps build only: copies the stamps of the last step launch on
// each (head, workgroup) row to host memory (bytes = 64 * 256 * kStamps * 8).
extern "C" int rkv_phase_stamps_read(void* host, size_t bytes) {
  if (!host || bytes < sizeof(rkv::rkv_stamps)) return 1;
  return hipMemcpyFromSymbol(host, HIP_SYMBOL(rkv::rkv_stamps), sizeof(rkv::rkv_stamps)) ==
                 hipSuccess ? 0 : 3;
}
#endif
