/*
 * mcke_oracle.c -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the CPU reference that the MCKE kernel layer is judged
 * against (tests/reference.hpp and include/mcke/kernels/softmax_online.hpp in the
 * reference tree).  Only the test suite, the smoke entry point and the benchmark's
 * cpu_baseline leg may load this library, and only as the checker.  Nothing in the
 * product library links or calls it.
 *
 * Every function names the reference lines it restates.  All references accumulate
 * in double and round once to float at the store, as the reference does.
 *
 * How each function is pinned (so that a plausible mistake fails a check):
 *   orc_mt64_*           C++ standard [rand.predef]: the 10000th output of a
 *                        default-seeded mt19937_64 is 9981545732273789042; and
 *                        bit-equality with std::mt19937_64 via oracle/_ref.
 *   orc_fill_random      bit-equality with the reference's fill_random (oracle/_ref)
 *                        and with the product library's independent generator.
 *   orc_fill_normal      no reference counterpart (the reference has no normal
 *                        generator).  Pinned by moments and a Box-Muller closed
 *                        form on the first pair; parity never depends on it since
 *                        CPU and GPU read the same host bytes.
 *   orc_bias_act         19 golden vectors (4 bias_act cases), hand KATs, the
 *                        erf-vs-tanh GELU gap, and bit-equality with oracle/_ref.
 *   orc_row_reduce       golden cases (sum/max/mean incl. an all-negative row),
 *                        hand KATs, brute force vs math.fsum, oracle/_ref.
 *   orc_row_softmax      golden approx case (a 90.0 logit), uniform row -> 1/n,
 *                        {1,2,3,1000}, ordering, row sums, oracle/_ref.
 *   orc_gemm             11 exact golden cases (quarter-multiple inputs, bit-exact),
 *                        2x2 and 2x3x2 hand KATs, alpha/beta, oracle/_ref.
 *   orc_compare          semantics tests (NaN/Inf flags, worst-mismatch index).
 *   orc_tol_gemm/...     closed forms at k=256 (~1e-5) and monotonicity, oracle/_ref.
 *   orc_spot_check_gemm  agreement with the full reference, fires on corruption,
 *                        bit-equality of the sample stream with oracle/_ref.
 *   orc_online_*         identity/associativity/commutativity properties and
 *                        equality with oracle/_ref's online_update/online_combine.
 *   orc_f32_to_bf16,     no reference counterpart (the reference reserves the 16-bit
 *   orc_bf16_to_f32      DType tags only).  Bit-equality with torch's CPU bfloat16
 *                        conversions on every 16-bit pattern and on 10^6 floats
 *                        with ties, overflow, subnormals, signed zeros and NaN,
 *                        plus hand values (1.0 -> 0x3F80, tie 1+2^-8 -> 0x3F80).
 *   orc_f32_to_f16,      no reference counterpart.  Bit-equality with numpy's
 *   orc_f16_to_f32       float16 conversions on every 16-bit pattern and the same
 *                        float set, plus hand values (65504, 65520 -> inf, 2^-24,
 *                        2^-25 -> 0).
 */
#include <float.h>
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

/* ------------------------------------------------------------------------- */
/* MT19937-64 (Matsumoto & Nishimura, ACM TOMACS 2000), the engine the         */
/* reference's fill_random and spot_check_gemm draw from (std::mt19937_64,     */
/* reference.hpp:101-109 and :405-407).  Written from the published            */
/* recurrence and parameters, not from any library source.                     */
/* ------------------------------------------------------------------------- */
#define MT_N 312
#define MT_M 156

typedef struct {
  uint64_t s[MT_N];
  int i;
} orc_mt64;

ORC_API void orc_mt64_seed(orc_mt64* g, uint64_t seed) {
  g->s[0] = seed;
  for (int i = 1; i < MT_N; ++i)
    g->s[i] = 6364136223846793005ULL * (g->s[i - 1] ^ (g->s[i - 1] >> 62)) + (uint64_t)i;
  g->i = MT_N;
}

static void mt64_twist(orc_mt64* g) {
  const uint64_t upper = 0xFFFFFFFF80000000ULL, lower = 0x7FFFFFFFULL;
  const uint64_t a = 0xB5026F5AA96619E9ULL;
  for (int k = 0; k < MT_N; ++k) {
    const uint64_t y = (g->s[k] & upper) | (g->s[(k + 1) % MT_N] & lower);
    uint64_t v = g->s[(k + MT_M) % MT_N] ^ (y >> 1);
    if (y & 1ULL) v ^= a;
    g->s[k] = v;
  }
  g->i = 0;
}

ORC_API uint64_t orc_mt64_next(orc_mt64* g) {
  if (g->i >= MT_N) mt64_twist(g);
  uint64_t x = g->s[g->i++];
  x ^= (x >> 29) & 0x5555555555555555ULL;
  x ^= (x << 17) & 0x71D67FFFEDA60000ULL;
  x ^= (x << 37) & 0xFFF7EEE000000000ULL;
  x ^= x >> 43;
  return x;
}

ORC_API size_t orc_mt64_sizeof(void) { return sizeof(orc_mt64); }

/* Convenience for tests: the n-th output (1-based) of an engine seeded with seed. */
ORC_API uint64_t orc_mt64_nth(uint64_t seed, uint64_t n) {
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  uint64_t v = 0;
  for (uint64_t i = 0; i < n; ++i) v = orc_mt64_next(&g);
  return v;
}

/* ------------------------------------------------------------------------- */
/* fill_random: reference.hpp:101-109.  The top 24 bits of each engine output  */
/* scaled to [0,1); then lo + u*(hi-lo) in double, where (hi - lo) is a float  */
/* subtraction because both operands are float in the reference; one rounding  */
/* to float at the store.                                                      */
/* ------------------------------------------------------------------------- */
ORC_API void orc_fill_random(float* p, size_t n, uint64_t seed, float lo, float hi) {
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  const float span = hi - lo;
  for (size_t i = 0; i < n; ++i) {
    const double u = (double)(orc_mt64_next(&g) >> 40) / (double)(1u << 24);
    p[i] = (float)((double)lo + u * (double)span);
  }
}

/* Normal N(mu, sigma^2) from the same engine (no reference counterpart; the
 * reference only has the uniform map).  Box-Muller on 53-bit uniforms:
 *   u1 = ((e1 >> 11) + 0.5) * 2^-53   in (0,1)      u2 = (e2 >> 11) * 2^-53
 *   r  = sqrt(-2 ln u1);  z0 = r cos(2 pi u2);  z1 = r sin(2 pi u2)
 * Elements 2j and 2j+1 take z0 and z1 of pair j.  Value = (float)(mu + sigma*z). */
ORC_API void orc_fill_normal(float* p, size_t n, uint64_t seed, float mu, float sigma) {
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  const double two_pi = 6.283185307179586476925286766559;
  const double inv53 = 1.0 / 9007199254740992.0; /* 2^-53 */
  for (size_t i = 0; i < n; i += 2) {
    const double u1 = ((double)(orc_mt64_next(&g) >> 11) + 0.5) * inv53;
    const double u2 = (double)(orc_mt64_next(&g) >> 11) * inv53;
    const double r = sqrt(-2.0 * log(u1));
    p[i] = (float)((double)mu + (double)sigma * (r * cos(two_pi * u2)));
    if (i + 1 < n) p[i + 1] = (float)((double)mu + (double)sigma * (r * sin(two_pi * u2)));
  }
}

/* ------------------------------------------------------------------------- */
/* Activations: reference.hpp:116-136.  Activation codes follow the reference  */
/* enum (kernels.hpp:65): 0 none, 1 relu, 2 gelu-erf, 3 gelu-tanh.             */
/* ------------------------------------------------------------------------- */
ORC_API double orc_gelu_erf(double x) {
  return 0.5 * x * (1.0 + erf(x * 0.70710678118654752440));
}

ORC_API double orc_gelu_tanh(double x) {
  const double k = 0.79788456080286535588; /* sqrt(2/pi) */
  return 0.5 * x * (1.0 + tanh(k * (x + 0.044715 * x * x * x)));
}

static double apply_act(double v, int act) {
  switch (act) {
    case 0: return v;
    case 1: return v > 0.0 ? v : 0.0;
    case 2: return orc_gelu_erf(v);
    case 3: return orc_gelu_tanh(v);
    default: return v;
  }
}

/* y[r][c] = act(x[r][c] + bias[c]); reference.hpp:143-151. */
ORC_API void orc_bias_act(const float* x, const float* bias, float* y, int64_t rows,
                          int64_t cols, int act) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c) {
      const double v = (double)x[r * cols + c] + (double)bias[c];
      y[r * cols + c] = (float)apply_act(v, act);
    }
}

/* out[r] = sum / max / mean of row r; reference.hpp:154-172.  Kind codes follow
 * ReduceKind (kernels.hpp:153): 0 sum, 1 max, 2 mean.  Max starts from -inf. */
ORC_API void orc_row_reduce(const float* x, float* out, int64_t rows, int64_t cols,
                            int kind) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    if (kind == 1) {
      double m = -INFINITY;
      for (int64_t c = 0; c < cols; ++c) {
        const double v = (double)row[c];
        m = (m < v) ? v : m; /* std::max(m, v) keeps m unless m < v */
      }
      out[r] = (float)m;
    } else {
      double s = 0.0;
      for (int64_t c = 0; c < cols; ++c) s += (double)row[c];
      if (kind == 2) s /= (double)cols;
      out[r] = (float)s;
    }
  }
}

/* Stable softmax per row: max, sum of exp(x - max), then exp(x - max) / sum;
 * reference.hpp:175-191. */
ORC_API void orc_row_softmax(const float* x, float* y, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = x + r * cols;
    float* o = y + r * cols;
    double m = -INFINITY;
    for (int64_t c = 0; c < cols; ++c) {
      const double v = (double)row[c];
      m = (m < v) ? v : m;
    }
    double s = 0.0;
    for (int64_t c = 0; c < cols; ++c) s += exp((double)row[c] - m);
    for (int64_t c = 0; c < cols; ++c) o[c] = (float)(exp((double)row[c] - m) / s);
  }
}

/* C = alpha * A[m,k] B[k,n] + beta * C, row-major, double accumulation in the
 * i-j-p loop order of reference.hpp:199-211.  C is read even when beta == 0
 * (0 * NaN would be NaN), exactly as the reference does. */
ORC_API void orc_gemm(const float* a, const float* b, float* c, int64_t m, int64_t n,
                      int64_t k, float alpha, float beta) {
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int64_t p = 0; p < k; ++p) acc += (double)a[i * k + p] * (double)b[p * n + j];
      const double prev = (double)c[i * n + j];
      c[i * n + j] = (float)((double)alpha * acc + (double)beta * prev);
    }
}

/* Rows [r0, r1) of orc_gemm only: the CPU-baseline slab for shapes whose full
 * reference takes minutes (same arithmetic, same order). */
ORC_API void orc_gemm_rows(const float* a, const float* b, float* c, int64_t m, int64_t n,
                           int64_t k, float alpha, float beta, int64_t r0, int64_t r1) {
  (void)m;
  for (int64_t i = r0; i < r1; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double acc = 0.0;
      for (int64_t p = 0; p < k; ++p) acc += (double)a[i * k + p] * (double)b[p * n + j];
      const double prev = (double)c[i * n + j];
      c[i * n + j] = (float)((double)alpha * acc + (double)beta * prev);
    }
}

/* ------------------------------------------------------------------------- */
/* compare(): reference.hpp:249-287.  |g - w| <= abs + rel*|w|, with NaN and a */
/* one-sided Inf counted as mismatches and flagged, and the worst FLAGGED      */
/* element (largest relative error among the failures) reported.               */
/* ------------------------------------------------------------------------- */
typedef struct {
  uint64_t n;
  uint64_t mismatches;
  double max_abs_err;
  double max_rel_err;
  uint64_t worst_index;
  double worst_got;
  double worst_want;
  int32_t any_nan;
  int32_t any_inf;
} orc_compare_result;

ORC_API void orc_compare(const float* got, const float* want, size_t n, double rel_tol,
                         double abs_tol, orc_compare_result* out) {
  orc_compare_result r;
  memset(&r, 0, sizeof r);
  r.n = n;
  double worst = -1.0;
  for (size_t i = 0; i < n; ++i) {
    const double g = (double)got[i], w = (double)want[i];
    if (isnan(g) || isnan(w)) {
      r.any_nan = 1;
      ++r.mismatches;
      continue;
    }
    if ((isinf(g) != 0) != (isinf(w) != 0)) {
      r.any_inf = 1;
      ++r.mismatches;
      continue;
    }
    const double ae = fabs(g - w);
    const double re = fabs(w) > 0.0 ? ae / fabs(w) : 0.0;
    if (ae > r.max_abs_err) r.max_abs_err = ae;
    if (re > r.max_rel_err) r.max_rel_err = re;
    if (ae > abs_tol + rel_tol * fabs(w)) {
      ++r.mismatches;
      if (re > worst) {
        worst = re;
        r.worst_index = i;
        r.worst_got = g;
        r.worst_want = w;
      }
    }
  }
  *out = r;
}

ORC_API size_t orc_compare_result_sizeof(void) { return sizeof(orc_compare_result); }

/* Named tolerances, reference.hpp:292-295 and :328-329. */
ORC_API double orc_tol_elementwise(void) { return 1e-6; }
ORC_API double orc_tol_reduce4096(void) { return 1e-5; }
ORC_API double orc_tol_softmax(void) { return 1e-5; }
ORC_API double orc_tol_gemm_k256(void) { return 1e-5; }
ORC_API double orc_abs_tol_gelu_cancellation(void) { return 1e-6; }
ORC_API double orc_abs_tol_reduce_sum4096(void) { return 5e-5; }

/* K-scaled GEMM tolerances, reference.hpp:344-374. */
ORC_API double orc_tol_gemm(int64_t k) {
  const double eps = 1.1920929e-7;
  return 4.0 * sqrt((double)(k < 1 ? 1 : k)) * eps;
}

ORC_API double orc_abs_tol_gemm(int64_t k, double amax) {
  const double eps = 1.1920929e-7;
  return 3.0 * (0.5 * (double)(k < 1 ? 1 : k) * eps * amax * amax / 3.0);
}

/* spot_check_gemm: reference.hpp:401-426.  `samples` output elements chosen by an
 * mt19937_64 stream (row = next() % m, then col = next() % n), recomputed in
 * double, judged against alpha*acc (beta assumed 0). */
typedef struct {
  uint64_t checked;
  uint64_t mismatches;
  double max_abs_err;
  double max_rel_err;
} orc_spot_result;

ORC_API void orc_spot_check_gemm(const float* a, const float* b, const float* got, int64_t m,
                                 int64_t n, int64_t k, float alpha, size_t samples,
                                 uint64_t seed, double rel_tol, double abs_tol,
                                 orc_spot_result* out) {
  orc_spot_result r;
  memset(&r, 0, sizeof r);
  if (m <= 0 || n <= 0 || k <= 0) {
    *out = r;
    return;
  }
  orc_mt64 g;
  orc_mt64_seed(&g, seed);
  for (size_t s = 0; s < samples; ++s) {
    const int64_t i = (int64_t)(orc_mt64_next(&g) % (uint64_t)m);
    const int64_t j = (int64_t)(orc_mt64_next(&g) % (uint64_t)n);
    double acc = 0.0;
    for (int64_t p = 0; p < k; ++p) acc += (double)a[i * k + p] * (double)b[p * n + j];
    const double want = (double)alpha * acc;
    const double gv = (double)got[i * n + j];
    ++r.checked;
    if (isnan(gv) || isinf(gv)) {
      ++r.mismatches;
      continue;
    }
    const double ae = fabs(gv - want);
    const double re = fabs(want) > 0.0 ? ae / fabs(want) : 0.0;
    if (ae > r.max_abs_err) r.max_abs_err = ae;
    if (re > r.max_rel_err) r.max_rel_err = re;
    if (ae > abs_tol + rel_tol * fabs(want)) ++r.mismatches;
  }
  *out = r;
}

/* ------------------------------------------------------------------------- */
/* Online softmax state, softmax_online.hpp:73-112, in float as the reference  */
/* evaluates it (fmaxf / expf).  Identity is (-FLT_MAX, 0); combine returns    */
/* the other operand when one side is empty.                                   */
/* ------------------------------------------------------------------------- */
ORC_API void orc_online_update(float m, float d, float x, float* out_m, float* out_d) {
  const float mn = fmaxf(m, x);
  *out_m = mn;
  *out_d = d * expf(m - mn) + expf(x - mn);
}

ORC_API void orc_online_combine(float am, float ad, float bm, float bd, float* out_m,
                                float* out_d) {
  if (bd == 0.0f) {
    *out_m = am;
    *out_d = ad;
    return;
  }
  if (ad == 0.0f) {
    *out_m = bm;
    *out_d = bd;
    return;
  }
  const float mm = fmaxf(am, bm);
  *out_m = mm;
  *out_d = ad * expf(am - mm) + bd * expf(bm - mm);
}

ORC_API float orc_online_identity_m(void) { return -FLT_MAX; }

/* ------------------------------------------------------------------------- */
/* 16-bit storage formats for the 16-bit-input GEMM.  The reference has no     */
/* conversion code (its DType reserves kF16 / kBF16, dtype.hpp:33-41, and      */
/* dtype_size gives 2 bytes for both, :43-52); these restate IEEE 754-2008      */
/* binary16 and the bfloat16 format (binary32 with the low 16 fraction bits    */
/* dropped), each with round-to-nearest-even on the narrowing conversion.      */
/* NaN stays NaN (quiet bit set, sign kept), overflow rounds to infinity.       */
/* ------------------------------------------------------------------------- */
static uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

static float bits_f32(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  /* Add half an ulp of the 16-bit result, plus one more when the kept part is
   * odd, so exact ties go to the even neighbour; a carry moves into the
   * exponent (and the largest finite values round to infinity). */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static uint16_t f32_to_f16_rne(float f) {
  const uint32_t u = f32_bits(f);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
  if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
  const int e = (int)(a >> 23) - 127;          /* unbiased exponent (-127 for zero/denormal) */
  const uint32_t frac = a & 0x7fffffu;
  if (e > 15) return (uint16_t)(sign | 0x7c00u);
  if (e >= -14) {
    /* Normal binary16: keep 10 of 23 fraction bits, round on the 13 dropped. */
    uint32_t h = ((uint32_t)(e + 15) << 10) | (frac >> 13);
    const uint32_t rest = frac & 0x1fffu;
    if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h += 1u;   /* may carry to 0x7c00 = inf */
    return (uint16_t)(sign | h);
  }
  /* Subnormal binary16: units of 2^-24.  The value is sig * 2^(e-23) with the
   * 24-bit significand sig, i.e. sig >> (-e-1) units; below 2^-25 it rounds to 0
   * (2^-25 itself is a tie that goes to the even 0). */
  if (e < -25) return sign;
  const uint32_t sig = frac | 0x800000u;
  const int s = -e - 1;                         /* 14 .. 24 */
  uint32_t q = sig >> s;
  const uint32_t rest = sig & ((1u << s) - 1u), half = 1u << (s - 1);
  if (rest > half || (rest == half && (q & 1u))) q += 1u;   /* 0x400 = smallest normal */
  return (uint16_t)(sign | q);
}

static float f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  if (e == 0x1fu) return bits_f32(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    const float v = ldexpf((float)m, -24);     /* exact: m < 2^10 */
    return sign ? -v : v;
  }
  return bits_f32(sign | ((e + 112u) << 23) | (m << 13));   /* rebias 15 -> 127 */
}

ORC_API void orc_f32_to_bf16(const float* x, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f32_to_bf16_rne(x[i]);
}

ORC_API void orc_bf16_to_f32(const uint16_t* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = bits_f32((uint32_t)x[i] << 16);
}

ORC_API void orc_f32_to_f16(const float* x, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f32_to_f16_rne(x[i]);
}

ORC_API void orc_f16_to_f32(const uint16_t* x, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = f16_to_f32(x[i]);
}
