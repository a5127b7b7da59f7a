/*
 * RefineKV CPU oracle -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's torch path for the decode-time
 * attention hot path.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker or as the
 * timed CPU baseline; the product (refinekv-release_amd/) never calls it.
 *
 * Functions and the reference code they restate:
 *   orc_summary         src/refinekv/summary.py:35-113   (_pages, build_summary)
 *   orc_select_stats    src/refinekv/reference.py:10-34  (selection_statistics)
 *   orc_select          src/refinekv/reference.py:37-47  (select_blocks_reference)
 *   orc_sparse_attention src/refinekv/reference.py:50-73 (sparse_attention_reference)
 *   orc_dense_attention  src/refinekv/integrations/transformers.py:510-520 (dense
 *                        decode: SDPA over the visible cache)
 *   orc_expf / orc_logf  elementary functions used by all of the above
 *
 * fp32 evaluation order.  torch leaves the order of fp32 sums open; this
 * oracle fixes one order per reduction so that the HIP kernels, which use
 * the same orders, agree with it bit for bit:
 *   TOKSUM  sum over the tokens of a block (key/value means), per column:
 *           tokens in chunks of 16, each chunk summed left to right from +0,
 *           chunk sums added left to right from +0 (torch's CPU cascade sum
 *           over a non-innermost dimension, multi_row_sum with level step 16).
 *   RADSUM  sum over head_dim of squared centred coordinates (ellipsoid
 *           radius): 8-wide vectors V_m = x[8m .. 8m+7]; four vector
 *           accumulators A_k = V_k + V_{k+4} + V_{k+8} + ... (from +0);
 *           lane-wise P = ((A_0 + A_1) + A_2) + A_3; result = P[0] + ... +
 *           P[7] left to right from +0 (torch's CPU inner sum, row_sum with
 *           four-way ILP, as centered.sum(-1) runs it).
 *   NORMSUM squared value norm over head_dim: one 8-wide accumulator
 *           A[l] = fma(x[8m+l], x[8m+l], A[l]) over m (from +0), result
 *           ((A[0] + A[1]) + ...) + A[7]: torch's CPU vector_norm (its
 *           2-norm kernel runs 8-wide with fused multiply-adds).
 *   DSUM    head_dim dot products x.y in selection and attention (torch
 *           uses MKL there, whose order is not reproducible): W = 8 lanes for
 *           D <= 128, else 16; lane j takes the D/W consecutive elements
 *           j*D/W ..., starting from the rounded first product x0*y0 and
 *           adding the rest with fmaf left to right; then an xor butterfly
 *           over the W lanes with distances W/2, ..., 1
 *           (P[j] <- P[j] + P[j^o]); the result is P[0].
 *   LSE     log-sum-exp over blocks: tiles of 64 consecutive blocks; per tile
 *           m = max, l = butterfly sum (distances 32..1) of exp(x - m);
 *           tiles merged per row by 64 lane accumulators (tile t goes to
 *           lane t % 64, left to right) then the same 64-wide butterfly.
 *   GQA     mean over the group: left to right, then divided by G.
 * Elementwise steps follow the reference's operator order exactly; scalars
 * the reference writes as Python floats are rounded to fp32 first, as torch
 * does for wrapped scalars.  exp/log are orc_expf/orc_logf below.
 *
 * Parity pins (tests/test_oracle_*.py): torch golden vectors written by
 * tests/golden/make_golden.py from the reference's own torch path, libm
 * accuracy sweeps for orc_expf/orc_logf, fp64 closed forms and brute force
 * on tiny inputs, and the reference's own CPU tests restated.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_TILE 64
#define ORC_DELTA_MAX 10.0f
#define ORC_INFLATE 1.00390625f /* 1 + 2^-8 */

/* ------------------------------------------------------------------ */
/* scalar helpers                                                      */
/* ------------------------------------------------------------------ */

static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }
static inline int isnanf_(float x) { return !(x == x); }
static inline int finitef_(float x) { return (fbits(x) & 0x7F800000u) != 0x7F800000u; }

uint16_t orc_bf16(float x) {
  if (isnanf_(x)) return 0x7FC0u;
  uint32_t u = fbits(x);
  return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}
static inline float bf16f(uint16_t h) { return bitsf((uint32_t)h << 16); }
static inline float rbf16(float x) { return bf16f(orc_bf16(x)); }

static inline float nmax(float a, float b) { return (a > b || isnanf_(a)) ? a : b; }
static inline float nmin(float a, float b) { return (a < b || isnanf_(a)) ? a : b; }
static inline float cmin(float x, float lo) { return x < lo ? lo : x; }
static inline float cmax(float x, float hi) { return x > hi ? hi : x; }

static inline float pow2scale(float p, int k) {
  if (k > 127) {
    p = p * bitsf(0x7F000000u);
    k -= 127;
  } else if (k < -126) {
    p = p * bitsf((uint32_t)(k + 64 + 127) << 23);
    return p * bitsf((uint32_t)(-64 + 127) << 23);
  }
  return p * bitsf((uint32_t)(k + 127) << 23);
}

/* exp: Cody-Waite reduction with a two-part ln2 and fma, degree-7 Taylor
 * polynomial of e^r on |r| <= ln2/2, exact power-of-two scaling. */
float orc_expf(float x) {
  if (isnanf_(x)) return x + x;
  if (x > 88.8f) return bitsf(0x7F800000u);
  if (x < -104.0f) return 0.0f;
  float k = rintf(x * 1.44269504088896341f);
  float r = fmaf(k, -0.693145751953125f, x);
  r = fmaf(k, -1.42860682030941723e-06f, r);
  float p = 1.98412698412698413e-04f;
  p = fmaf(p, r, 1.38888888888888889e-03f);
  p = fmaf(p, r, 8.33333333333333333e-03f);
  p = fmaf(p, r, 4.16666666666666667e-02f);
  p = fmaf(p, r, 1.66666666666666667e-01f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return pow2scale(p, (int)k);
}

/* log: fdlibm e_log.c reduction (x = 2^e m, m in [sqrt2/2, sqrt2),
 * f = m-1, s = f/(2+f)), log(1+f) = f - (hfsq - s(hfsq + R(s^2))) with the
 * Taylor coefficients 2/3, 2/5, 2/7, 2/9 of 2 atanh(s). */
float orc_logf(float x) {
  if (isnanf_(x)) return x + x;
  if (x < 0.0f) return bitsf(0x7FC00000u);
  if (x == 0.0f) return bitsf(0xFF800000u);
  if (x == bitsf(0x7F800000u)) return x;
  uint32_t u = fbits(x);
  int e = 0;
  if (u < 0x00800000u) {
    x = x * 8388608.0f;
    u = fbits(x);
    e = -23;
  }
  e += (int)(u >> 23) - 127;
  float m = bitsf((u & 0x007FFFFFu) | 0x3F800000u);
  if (m > 1.41421356237309505f) {
    m = m * 0.5f;
    e += 1;
  }
  float f = m - 1.0f;
  float s = f / (2.0f + f);
  float s2 = s * s;
  float R = 0.222222222222222222f;
  R = fmaf(R, s2, 0.285714285714285714f);
  R = fmaf(R, s2, 0.4f);
  R = fmaf(R, s2, 0.666666666666666667f);
  R = R * s2;
  float hfsq = 0.5f * f * f;
  float dk = (float)e;
  return dk * 0.693145751953125f -
         ((hfsq - (s * (hfsq + R) + dk * 1.42860682030941723e-06f)) - f);
}

/* DSUM order of x.y over D elements, D a multiple of 16. */
static float dsum(const float *x, const float *y, int64_t D) {
  float P[16], Q[16];
  int W = D <= 128 ? 8 : 16;
  int64_t c = D / W;
  for (int j = 0; j < W; ++j) {
    float a = x[j * c] * y[j * c];
    for (int64_t i = 1; i < c; ++i) a = fmaf(x[j * c + i], y[j * c + i], a);
    P[j] = a;
  }
  for (int o = W / 2; o >= 1; o >>= 1) {
    for (int j = 0; j < W; ++j) Q[j] = P[j] + P[j ^ o];
    memcpy(P, Q, sizeof(P));
  }
  return P[0];
}

/* TOKSUM order over x[0..n-1] (n = block_size, padded tokens are +0). */
static float toksum(const float *x, int64_t n) {
  float total = 0.0f;
  for (int64_t c0 = 0; c0 < n; c0 += 16) {
    float a = 0.0f;
    for (int64_t i = c0; i < c0 + 16 && i < n; ++i) a = a + x[i];
    total = total + a;
  }
  return total;
}

/* RADSUM order over x[0..D-1], D a multiple of 32. */
static float radsum(const float *x, int64_t D) {
  int64_t rows = D / 32;
  float A[4][8];
  for (int k = 0; k < 4; ++k)
    for (int l = 0; l < 8; ++l) {
      A[k][l] = 0.0f;
      for (int64_t r = 0; r < rows; ++r) A[k][l] = A[k][l] + x[(4 * r + k) * 8 + l];
    }
  float total = 0.0f;
  for (int l = 0; l < 8; ++l) total = total + (((A[0][l] + A[1][l]) + A[2][l]) + A[3][l]);
  return total;
}

/* NORMSUM order: squared L2 norm of x[0..D-1]. */
static float normsum(const float *x, int64_t D) {
  float A[8];
  for (int l = 0; l < 8; ++l) {
    A[l] = 0.0f;
    for (int64_t v = 0; v < D / 8; ++v) A[l] = fmaf(x[v * 8 + l], x[v * 8 + l], A[l]);
  }
  float total = A[0];
  for (int l = 1; l < 8; ++l) total = total + A[l];
  return total;
}

static float butterfly64(float *v) {
  float w[64];
  for (int o = 32; o >= 1; o >>= 1) {
    for (int j = 0; j < 64; ++j) w[j] = v[j] + v[j ^ o];
    memcpy(v, w, sizeof(w));
  }
  return v[0];
}

static inline int64_t block_count(int64_t b, int64_t n_blocks, int64_t block, int64_t length) {
  return b == n_blocks - 1 ? length - (n_blocks - 1) * block : block;
}

/* ------------------------------------------------------------------ */
/* build_summary (summary.py:46-113)                                   */
/* ------------------------------------------------------------------ */

/* keys/values: (H, L, D) fp32 holding the exact values of the cache dtype.
 * Outputs: counts (N,), key_mean/value_mean/ellipsoid (H,N,D) bf16 bits,
 * value_norm (H,N), max_value_norm (H,). */
int orc_summary(const float *keys, const float *values, int64_t H, int64_t L, int64_t D,
                int64_t B, int64_t *counts, uint16_t *key_mean, uint16_t *value_mean,
                uint16_t *ellipsoid, float *value_norm, float *max_value_norm) {
  if (H <= 0 || L <= 0 || D <= 0 || D % 32 || (B != 16 && B != 32 && B != 64)) return 1;
  int64_t N = (L + B - 1) / B;
  float *colk = malloc(sizeof(float) * B), *colv = malloc(sizeof(float) * B);
  float *mk = malloc(sizeof(float) * D), *w2 = malloc(sizeof(float) * D);
  float *rs = malloc(sizeof(float) * D), *row = malloc(sizeof(float) * D);
  for (int64_t b = 0; b < N; ++b) counts[b] = block_count(b, N, B, L);
  for (int64_t h = 0; h < H; ++h) {
    float vmax_all = -INFINITY;
    for (int64_t b = 0; b < N; ++b) {
      int64_t cnt = counts[b];
      const float *K = keys + (h * L + b * B) * D;
      const float *V = values + (h * L + b * B) * D;
      int64_t o = (h * N + b) * D;
      for (int64_t d = 0; d < D; ++d) {
        float hi = -INFINITY, lo = INFINITY;
        for (int64_t t = 0; t < B; ++t) {
          colk[t] = t < cnt ? K[t * D + d] : 0.0f;
          colv[t] = t < cnt ? V[t * D + d] : 0.0f;
          if (t < cnt) {
            hi = nmax(hi, colk[t]);
            lo = nmin(lo, colk[t]);
          }
        }
        key_mean[o + d] = orc_bf16(toksum(colk, B) / (float)cnt);
        value_mean[o + d] = orc_bf16(toksum(colv, B) / (float)cnt);
        mk[d] = bf16f(key_mean[o + d]);
        float width = nmax(hi - mk[d], mk[d] - lo);
        float cw = cmin(width, 1e-6f);
        w2[d] = rbf16(cw * cw);
        rs[d] = 1.0f / sqrtf(w2[d]);
      }
      float r2 = -INFINITY, vn = -INFINITY;
      for (int64_t t = 0; t < cnt; ++t) {
        for (int64_t d = 0; d < D; ++d) {
          float c = (K[t * D + d] - mk[d]) * rs[d];
          row[d] = c * c;
        }
        r2 = nmax(r2, radsum(row, D));
        vn = nmax(vn, sqrtf(normsum(V + t * D, D)));
      }
      r2 = cmin(r2, 0.0f);
      r2 = sqrtf(r2);
      r2 = r2 * r2;
      for (int64_t d = 0; d < D; ++d) ellipsoid[o + d] = orc_bf16((r2 * w2[d]) * ORC_INFLATE);
      value_norm[h * N + b] = vn;
      vmax_all = nmax(vmax_all, vn);
    }
    max_value_norm[h] = vmax_all;
  }
  free(colk); free(colv); free(mk); free(w2); free(rs); free(row);
  return 0;
}

/* ------------------------------------------------------------------ */
/* selection_statistics (reference.py:10-34)                           */
/* ------------------------------------------------------------------ */

static float log_cosh(float delta) {
  float c = cmax(delta, ORC_DELTA_MAX);
  if (delta <= ORC_DELTA_MAX) return orc_logf((orc_expf(c) + orc_expf(-c)) * 0.5f);
  return delta + orc_logf((1.0f + orc_expf(-2.0f * delta)) * 0.5f);
}

static float risk_of(float z, float delta, float log_z, float log_c, float vmax, float vnorm) {
  const float ln2 = 0.693147182464599609375f; /* fp32(math.log(2)) */
  float clipped = cmax(delta, ORC_DELTA_MAX);
  float t = orc_expf(clipped);
  float exp_neg = orc_expf(-delta);
  float mass, th;
  if (delta <= ORC_DELTA_MAX) {
    float direct = (2.0f * vmax) * orc_expf(z - log_c);
    mass = direct * ((0.5f * (t + 1.0f / t)) - 1.0f);
    th = (t - 1.0f) / (t + 1.0f);
  } else {
    float lcm1 = (delta + 2.0f * orc_logf(cmin(1.0f - exp_neg, 1e-30f))) - ln2;
    mass = (2.0f * vmax) * orc_expf((z - log_c) + lcm1);
    th = (1.0f - exp_neg) / (1.0f + exp_neg);
  }
  float value = ((2.0f * vnorm) * orc_expf(z - log_z)) * th;
  return mass + value;
}

/* LSE of x[0..N-1] in the LSE order. */
static float lse(const float *x, int64_t N) {
  int64_t nt = (N + ORC_TILE - 1) / ORC_TILE;
  float *tm = malloc(sizeof(float) * nt), *tl = malloc(sizeof(float) * nt);
  float v[64];
  for (int64_t t = 0; t < nt; ++t) {
    float m = -INFINITY;
    for (int j = 0; j < 64; ++j) {
      int64_t b = t * ORC_TILE + j;
      if (b < N) m = nmax(m, x[b]);
    }
    float ms = (m == INFINITY || m == -INFINITY) ? 0.0f : m;
    for (int j = 0; j < 64; ++j) {
      int64_t b = t * ORC_TILE + j;
      v[j] = b < N ? orc_expf(x[b] - ms) : 0.0f;
    }
    tm[t] = m;
    tl[t] = butterfly64(v);
  }
  float M = -INFINITY;
  for (int64_t t = 0; t < nt; ++t) M = nmax(M, tm[t]);
  float Ms = (M == INFINITY || M == -INFINITY) ? 0.0f : M;
  for (int j = 0; j < 64; ++j) {
    float a = 0.0f;
    int first = 1;
    for (int64_t t = j; t < nt; t += 64) {
      float term = tl[t] * orc_expf(tm[t] - Ms);
      a = first ? term : a + term;
      first = 0;
    }
    v[j] = a;
  }
  float L = butterfly64(v);
  free(tm);
  free(tl);
  return orc_logf(L) + Ms;
}

/* q: (H, G, D) fp32 (any source dtype; rounded to bf16 here as the reference
 * does).  key_mean/ellipsoid: (H, N, D) bf16 bits.  Outputs (H, G, N):
 * z, delta, risk; (H, G): log_z, log_c.  Any output may be NULL except the
 * ones later steps need internally. */
int orc_select_stats(const float *q, const uint16_t *key_mean, const uint16_t *ellipsoid,
                     const float *value_norm, const float *max_value_norm, int64_t H,
                     int64_t G, int64_t D, int64_t N, int64_t B, int64_t L, float *z,
                     float *delta, float *risk, float *log_z, float *log_c) {
  if (H <= 0 || G <= 0 || N <= 0 || D % 16) return 1;
  float scale = (float)pow((double)D, -0.5);
  float *qt = malloc(sizeof(float) * D), *q2 = malloc(sizeof(float) * D);
  float *prod = malloc(sizeof(float) * D), *zc = malloc(sizeof(float) * N);
  for (int64_t h = 0; h < H; ++h) {
    for (int64_t g = 0; g < G; ++g) {
      int64_t r = h * G + g;
      for (int64_t d = 0; d < D; ++d) {
        qt[d] = rbf16(q[r * D + d]);
        q2[d] = rbf16(qt[d] * qt[d]);
      }
      float *zr = z + r * N, *dr = delta + r * N;
      for (int64_t b = 0; b < N; ++b) {
        const uint16_t *km = key_mean + (h * N + b) * D;
        const uint16_t *el = ellipsoid + (h * N + b) * D;
        for (int64_t d = 0; d < D; ++d) prod[d] = bf16f(km[d]);
        float s = dsum(qt, prod, D) * scale;
        for (int64_t d = 0; d < D; ++d) prod[d] = bf16f(el[d]);
        float p = dsum(q2, prod, D);
        float dl = (sqrtf(cmin(p, 0.0f)) * scale) * ORC_INFLATE;
        float cnt = (float)block_count(b, N, B, L);
        zr[b] = s + orc_logf(cnt);
        dr[b] = dl;
        zc[b] = zr[b] + log_cosh(dl);
      }
      float lz = lse(zr, N), lc = lse(zc, N);
      if (log_z) log_z[r] = lz;
      if (log_c) log_c[r] = lc;
      if (risk)
        for (int64_t b = 0; b < N; ++b)
          risk[r * N + b] = risk_of(zr[b], dr[b], lz, lc, max_value_norm[h], value_norm[h * N + b]);
    }
  }
  free(qt); free(q2); free(prod); free(zc);
  return 0;
}

/* ------------------------------------------------------------------ */
/* select_blocks_reference (reference.py:37-47) + anchor union         */
/* ------------------------------------------------------------------ */

/* reduction: 0 mean, 1 max, 2 any.  anchor (H,N) may be NULL.  mask (H,N)
 * gets 0/1.  z (H,G,N) and risk (H,G,N) are outputs (caller-allocated). */
int orc_select(const float *q, const uint16_t *key_mean, const uint16_t *ellipsoid,
               const float *value_norm, const float *max_value_norm, int64_t H, int64_t G,
               int64_t D, int64_t N, int64_t B, int64_t L, float eps, int reduction,
               const uint8_t *anchor, uint8_t *mask, float *z, float *risk) {
  float *delta = malloc(sizeof(float) * H * G * N);
  float *lz = malloc(sizeof(float) * H * G), *lc = malloc(sizeof(float) * H * G);
  int rc = orc_select_stats(q, key_mean, ellipsoid, value_norm, max_value_norm, H, G, D, N, B, L,
                            z, delta, risk, lz, lc);
  if (rc) goto done;
  for (int64_t h = 0; h < H; ++h) {
    int bad_global = 0;
    for (int64_t g = 0; g < G; ++g)
      bad_global |= !finitef_(lz[h * G + g]) || !finitef_(lc[h * G + g]);
    for (int64_t b = 0; b < N; ++b) {
      int sel = 0, bad_local = 0;
      float acc = 0.0f, mx = 0.0f;
      for (int64_t g = 0; g < G; ++g) {
        float c = risk[(h * G + g) * N + b];
        bad_local |= !finitef_(c);
        if (g == 0) {
          acc = c;
          mx = c;
        } else {
          acc = acc + c;
          mx = nmax(mx, c);
        }
        if (reduction == 2) sel |= c > eps;
      }
      if (reduction == 0) sel = (acc / (float)G) > eps;
      if (reduction == 1) sel = mx > eps;
      sel = sel || bad_global || bad_local || (anchor && anchor[h * N + b]);
      mask[h * N + b] = (uint8_t)sel;
    }
  }
done:
  free(delta); free(lz); free(lc);
  return rc;
}

/* ------------------------------------------------------------------ */
/* sparse_attention_reference (reference.py:50-73)                     */
/* ------------------------------------------------------------------ */

/* key_pages/value_pages: (H, N, B, D) bf16 bits (the reference rounds
 * exact K/V to bf16, reference.py:63-66).  suffix: (H, S, D) bf16 bits.
 * out: (H, G, D) fp32 before the final cast to the query dtype. */
int orc_sparse_attention(const float *q, const uint16_t *key_mean, const uint16_t *value_mean,
                         const uint16_t *ellipsoid, const float *value_norm,
                         const float *max_value_norm, const uint16_t *key_pages,
                         const uint16_t *value_pages, const uint16_t *key_suffix,
                         const uint16_t *value_suffix, int64_t S, int64_t H, int64_t G,
                         int64_t D, int64_t N, int64_t B, int64_t L, float eps, int reduction,
                         const uint8_t *anchor, uint8_t *mask, float *out) {
  float *z = malloc(sizeof(float) * H * G * N), *risk = malloc(sizeof(float) * H * G * N);
  int rc = orc_select(q, key_mean, ellipsoid, value_norm, max_value_norm, H, G, D, N, B, L, eps,
                      reduction, anchor, mask, z, risk);
  if (rc) {
    free(z); free(risk);
    return rc;
  }
  float scale = (float)pow((double)D, -0.5);
  int64_t cap = N * B + S;
  float *logit = malloc(sizeof(float) * cap);
  const uint16_t **vrow = malloc(sizeof(uint16_t *) * cap);
  float *qt = malloc(sizeof(float) * D), *prod = malloc(sizeof(float) * D);
  double *acc = malloc(sizeof(double) * D);
  for (int64_t h = 0; h < H; ++h) {
    for (int64_t g = 0; g < G; ++g) {
      int64_t r = h * G + g, n = 0;
      for (int64_t d = 0; d < D; ++d) qt[d] = rbf16(q[r * D + d]);
      /* representatives first, then exact tokens, as in the reference's cat */
      for (int64_t b = 0; b < N; ++b)
        if (!mask[h * N + b]) {
          logit[n] = z[r * N + b];
          vrow[n++] = value_mean + (h * N + b) * D;
        }
      for (int64_t b = 0; b < N; ++b) {
        if (!mask[h * N + b]) continue;
        int64_t cnt = block_count(b, N, B, L);
        for (int64_t t = 0; t < cnt; ++t) {
          const uint16_t *k = key_pages + ((h * N + b) * B + t) * D;
          for (int64_t d = 0; d < D; ++d) prod[d] = bf16f(k[d]);
          logit[n] = dsum(qt, prod, D) * scale;
          vrow[n++] = value_pages + ((h * N + b) * B + t) * D;
        }
      }
      for (int64_t t = 0; t < S; ++t) {
        const uint16_t *k = key_suffix + (h * S + t) * D;
        for (int64_t d = 0; d < D; ++d) prod[d] = bf16f(k[d]);
        logit[n] = dsum(qt, prod, D) * scale;
        vrow[n++] = value_suffix + (h * S + t) * D;
      }
      /* softmax(-1) @ values in fp32; sums accumulated in fp64 here so the
       * oracle's own rounding stays far below the tolerance it checks. */
      float m = -INFINITY;
      for (int64_t j = 0; j < n; ++j) m = nmax(m, logit[j]);
      double den = 0.0;
      for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
      for (int64_t j = 0; j < n; ++j) {
        double p = exp((double)logit[j] - (double)m);
        den += p;
        for (int64_t d = 0; d < D; ++d) acc[d] += p * (double)bf16f(vrow[j][d]);
      }
      for (int64_t d = 0; d < D; ++d) out[r * D + d] = (float)(acc[d] / den);
    }
  }
  free(z); free(risk); free(logit); free(vrow); free(qt); free(prod); free(acc);
  return 0;
}

/* Dense decode (the SDPA call of src/refinekv/integrations/transformers.py:
 * 510-520, softmax(q k^T * D^-0.5) v over the first L cached tokens): the
 * exact-token half of orc_sparse_attention with every token visible.
 * q: (H, G, D) fp32 (rounded to bf16 as the attention's query is);
 * keys/values: (H, L, D) bf16 bits; out: (H, G, D) fp32. */
int orc_dense_attention(const float *q, const uint16_t *keys, const uint16_t *values,
                        int64_t H, int64_t G, int64_t D, int64_t L, float *out) {
  if (H <= 0 || G <= 0 || D <= 0 || D % 16 || L <= 0) return 1;
  float scale = (float)pow((double)D, -0.5);
  float *logit = malloc(sizeof(float) * L);
  float *qt = malloc(sizeof(float) * D), *prod = malloc(sizeof(float) * D);
  double *acc = malloc(sizeof(double) * D);
  for (int64_t h = 0; h < H; ++h) {
    for (int64_t g = 0; g < G; ++g) {
      int64_t r = h * G + g;
      for (int64_t d = 0; d < D; ++d) qt[d] = rbf16(q[r * D + d]);
      float m = -INFINITY;
      for (int64_t t = 0; t < L; ++t) {
        const uint16_t *k = keys + (h * L + t) * D;
        for (int64_t d = 0; d < D; ++d) prod[d] = bf16f(k[d]);
        logit[t] = dsum(qt, prod, D) * scale;
        m = nmax(m, logit[t]);
      }
      double den = 0.0;
      for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
      for (int64_t t = 0; t < L; ++t) {
        double p = exp((double)logit[t] - (double)m);
        const uint16_t *v = values + (h * L + t) * D;
        den += p;
        for (int64_t d = 0; d < D; ++d) acc[d] += p * (double)bf16f(v[d]);
      }
      for (int64_t d = 0; d < D; ++d) out[r * D + d] = (float)(acc[d] / den);
    }
  }
  free(logit); free(qt); free(prod); free(acc);
  return 0;
}

/* Vector forms of the elementary functions, for the accuracy sweeps. */
void orc_expf_n(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}
void orc_logf_n(const float *x, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_logf(x[i]);
}
void orc_bf16_n(const float *x, uint16_t *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = orc_bf16(x[i]);
}

/* Elementwise risk (reference.py:26-34) for given statistics; for the
 * closed-form and known-answer checks. */
void orc_risk_n(const float *z, const float *delta, const float *log_z, const float *log_c,
                const float *vmax, const float *vnorm, float *out, int64_t n) {
  for (int64_t i = 0; i < n; ++i)
    out[i] = risk_of(z[i], delta[i], log_z[i], log_c[i], vmax[i], vnorm[i]);
}
