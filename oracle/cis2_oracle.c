/* oracle/cis2_oracle.c — CPU restatement of the CIS-2 pinned-order fp32
 * forward pass.  TEST INFRASTRUCTURE ONLY (it produces the expected bits
 * for the tests; never shipped, never called by the product path).
 *
 * Build contract (oracle/Makefile): C11, -O2 -ffp-contract=off
 * -fno-fast-math -msse2 -mfpmath=sse -fexcess-precision=standard, no
 * -march=native (no FMA can be selected), FTZ|DAZ pinned on every thread
 * that does arithmetic.  Every multiply and add below is its own statement,
 * rounded to binary32 on its own.
 *
 * Reference citations are relative to the reference archive root.
 */
#define _GNU_SOURCE
#include "cis2_oracle.h"

#include <emmintrin.h>
#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ======================================================================
 * Bit helpers
 * ====================================================================== */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* ======================================================================
 * Pinned constants — numeric facts of the spec, given here by bit pattern.
 * code/cis2-fp/gpu/cis2_consts.inc:5-32 (bit patterns in its comments),
 * code/cis2-fp/src/math.rs:153-165,248,266-272,347-362.
 * ====================================================================== */
#define B_EXP_LOG2E 0x3fb8aa3bu
#define B_EXP_C1 0x3f318000u
#define B_EXP_C2 0xb95e8083u
static const uint32_t B_EXP_P[6] = {0x39506967u, 0x3ab743ceu, 0x3c088908u,
                                    0x3d2aa9c1u, 0x3e2aaaaau, 0x3f000000u};
#define B_SIN_C0 0xbe2aaaa3u
#define B_SIN_C1 0x3c08839eu
#define B_SIN_C2 0xb94ca1f9u
#define B_COS_C0 0x3d2aaaa5u
#define B_COS_C1 0xbab6061au
#define B_COS_C2 0x37ccf5ceu
#define B_LOG_SQRTHF 0x3f3504f3u
#define B_LOG_Q1 0xb95e8083u
#define B_LOG_Q2 0x3f318000u
static const uint32_t B_LOG_P[9] = {0x3d9021bbu, 0xbdebd1b8u, 0x3def251bu,
                                    0xbdfe5d4fu, 0x3e11e9bfu, 0xbe2aae50u,
                                    0x3e4cceadu, 0xbe7ffffcu, 0x3eaaaaaau};
#define B_PI_2_F64 0x3ff921fb54442d18ull

/* ======================================================================
 * FP environment — code/cis2-fp/src/denormal.rs:22-57 (MXCSR bits 15/6),
 * self-test code/cis2-fp/gpu/cis2_fpenv.h:90-107, spec
 * code/cis2-fp/docs/CIS2_SPEC_v0.3.md:102-157.
 * ====================================================================== */
static inline float opaque(float x) {
  __asm__ volatile("" : "+x"(x) : : "memory");
  return x;
}

/* Planted mistakes (orc_set_mutation): tests turn them on to show that a
 * fixture detects the mistake; 0 everywhere else. */
static _Atomic int g_mutation;
void orc_set_mutation(int m) { atomic_store(&g_mutation, m); }

int orc_fpenv_pin(void) {
  unsigned csr = _mm_getcsr();
  if (atomic_load(&g_mutation) & ORC_MUT_NO_FTZ) { /* planted: subnormals kept */
    _mm_setcsr(csr & ~((1u << 15) | (1u << 6)));
    return 0;
  }
  _mm_setcsr(csr | (1u << 15) | (1u << 6));
  csr = _mm_getcsr();
  if (!(csr & (1u << 15)) || !(csr & (1u << 6))) return -1;
  /* 2^-126 * 1e-10 must flush to +0.0 (FTZ on the output). */
  float p = opaque(u2f(0x00800000u)) * opaque(1.0e-10f);
  if (f2u(p) != 0u) return -2;
  /* smallest subnormal + 0.0 must be +0.0 (DAZ on the input). */
  float s = opaque(u2f(0x00000001u)) + opaque(0.0f);
  if (f2u(s) != 0u) return -3;
  return 0;
}

/* Clears FTZ|DAZ on the calling thread (the default IEEE environment), so a
 * test process can run code that needs subnormals after the oracle pinned
 * its thread; every oracle entry pins again on its next call. */
void orc_fpenv_release(void) {
  _mm_setcsr(_mm_getcsr() & ~((1u << 15) | (1u << 6)));
}

/* ======================================================================
 * Integer/rounding helpers without libm.
 * Saturating casts: Rust `as` semantics, code/cis2-fp/src/math.rs:167-225
 * (exp `k as i32`), :253-264 (`k as i64`); spec :553-917.
 * ====================================================================== */
static inline int32_t sat_f32_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}
static inline int64_t sat_f64_i64(double x) {
  if (x != x) return 0;
  if (x >= 9223372036854775808.0) return INT64_MAX;
  if (x <= -9223372036854775808.0) return INT64_MIN;
  return (int64_t)x;
}
/* f32 floor: values with |x| >= 2^23 (and inf/NaN) are already integral;
 * below that the truncating int conversion is exact. */
static inline float floor_f32(float x) {
  float ax = x < 0.0f ? -x : x;
  if (!(ax < 8388608.0f)) return x;
  float t = (float)(int32_t)x;
  if (x < t) t = t - 1.0f;
  return t;
}
/* f64 round half away from zero, sign of zero preserved (Rust f64::round). */
static inline double round_away_f64(double x) {
  double ax = x < 0.0 ? -x : x;
  if (!(ax < 4503599627370496.0)) return x; /* 2^52, inf, NaN */
  double t = (double)(int64_t)ax;
  if (ax - t >= 0.5) t = t + 1.0;
  uint64_t mag = d2u(t) & 0x7FFFFFFFFFFFFFFFull;
  return u2d(mag | (d2u(x) & 0x8000000000000000ull));
}

/* ======================================================================
 * Pinned transcendentals
 * ====================================================================== */

/* Correctly rounded sqrt: one SSE sqrtss (IEEE-754 requires correct
 * rounding).  code/cis2-fp/src/math.rs:133-135, gpu/cis2_math.h:162-178. */
float orc_sqrt(float x) { return _mm_cvtss_f32(_mm_sqrt_ss(_mm_set_ss(x))); }

/* rsqrt_cr = 1 / sqrt(x), both correctly rounded.
 * code/cis2-fp/src/math.rs:133-135; spec §6.1. */
float orc_rsqrt(float x) {
  float s = orc_sqrt(x);
  return 1.0f / s;
}

/* Exponent-field scaling; underflow gives +0 whatever the sign of x,
 * overflow gives a signed infinity.  code/cis2-fp/src/math.rs:206-225. */
static inline float ldexp_bits(float x, int32_t k) {
  if (x == 0.0f) return x;
  uint32_t b = f2u(x);
  int32_t e = (int32_t)((b >> 23) & 0xFFu) + k;
  if (e <= 0) return 0.0f;
  if (e >= 0xFF) return (b >> 31) ? u2f(0xFF800000u) : u2f(0x7F800000u);
  return u2f((b & 0x807FFFFFu) | ((uint32_t)e << 23));
}

/* exp: clamp at +-88, split reduction r = (x - k*C1) - k*C2 with
 * k = floor(x*log2e + 0.5), degree-5 Horner, then (p*r^2 + r) + 1, scaled
 * by 2^k on the exponent field.  code/cis2-fp/src/math.rs:167-204,
 * spec §6.2 (code/cis2-fp/docs/CIS2_SPEC_v0.3.md:553-760). */
float orc_exp(float x) {
  if (x != x) return u2f(0x7FC00000u);
  if (x > 88.0f) return u2f(0x7F800000u);
  if (x < -88.0f) return 0.0f;
  float t = x * u2f(B_EXP_LOG2E);
  float z0 = t + 0.5f;
  float k = floor_f32(z0);
  float kc1 = k * u2f(B_EXP_C1);
  float r0 = x - kc1;
  float kc2 = k * u2f(B_EXP_C2);
  float r = r0 - kc2;
  float r2 = r * r;
  float p = u2f(B_EXP_P[0]);
  for (int i = 1; i < 6; ++i) {
    float m = p * r;
    p = m + u2f(B_EXP_P[i]);
  }
  float pr2 = p * r2;
  float s = pr2 + r;
  float y = s + 1.0f;
  return ldexp_bits(y, sat_f32_i32(k));
}

/* Octant reduction in binary64: exact widening, correctly rounded divide,
 * ties-away round, multiply, subtract, one narrowing to binary32.
 * code/cis2-fp/src/math.rs:248-264, spec §6.3. */
static inline float reduce_half_pi(float x, int64_t *k_out) {
  const double pio2 = u2d(B_PI_2_F64);
  double xd = (double)x;
  double q = xd / pio2;
  double kd = round_away_f64(q);
  double kp = kd * pio2;
  double rd = xd - kp;
  *k_out = sat_f64_i64(kd);
  return (float)rd;
}
/* r + (((S2*r2 + S1)*r2 + S0) * (r2*r)), code/cis2-fp/src/math.rs:275-286 */
static inline float sin_kernel(float r) {
  float r2 = r * r;
  float a = u2f(B_SIN_C2);
  float m0 = a * r2;
  a = m0 + u2f(B_SIN_C1);
  float m1 = a * r2;
  a = m1 + u2f(B_SIN_C0);
  float r3 = r2 * r;
  float tail = a * r3;
  return r + tail;
}
/* (1 - 0.5*r2) + (((C2*r2 + C1)*r2 + C0) * (r2*r2)),
 * code/cis2-fp/src/math.rs:288-302 */
static inline float cos_kernel(float r) {
  float r2 = r * r;
  float a = u2f(B_COS_C2);
  float m0 = a * r2;
  a = m0 + u2f(B_COS_C1);
  float m1 = a * r2;
  a = m1 + u2f(B_COS_C0);
  float r4 = r2 * r2;
  float tail = a * r4;
  float h = 0.5f * r2;
  float lead = 1.0f - h;
  return lead + tail;
}
/* quadrant = ((k % 4) + 4) % 4 with truncating %, math.rs:304-308 */
static inline int quadrant_of(int64_t k) { return (int)(((k % 4) + 4) % 4); }

/* code/cis2-fp/src/math.rs:310-322 */
float orc_sin(float x) {
  int64_t k;
  float r = reduce_half_pi(x, &k);
  float s = sin_kernel(r), c = cos_kernel(r);
  switch (quadrant_of(k)) {
    case 0: return s;
    case 1: return c;
    case 2: return -s;
    default: return -c;
  }
}
/* code/cis2-fp/src/math.rs:324-334 */
float orc_cos(float x) {
  int64_t k;
  float r = reduce_half_pi(x, &k);
  float s = sin_kernel(r), c = cos_kernel(r);
  switch (quadrant_of(k)) {
    case 0: return c;
    case 1: return -s;
    case 2: return -c;
    default: return s;
  }
}

/* ln: bit-level frexp (mantissa in [0.5,1)), sqrt(1/2) fold, degree-9
 * Horner in m, then y = (p*m)*z + e*Q1 - 0.5*z, result (m + y) + e*Q2.
 * code/cis2-fp/src/math.rs:366-410, spec §6.5. */
float orc_ln(float x) {
  if (x != x || x < 0.0f) return u2f(0x7FC00000u);
  if (x == 0.0f) return u2f(0xFF800000u);
  uint32_t b = f2u(x);
  int32_t e = (int32_t)((b >> 23) & 0xFFu) - 126;
  float m = u2f((b & 0x807FFFFFu) | (126u << 23));
  if (m < u2f(B_LOG_SQRTHF)) {
    e = e - 1;
    float mm = m + m;
    m = mm - 1.0f;
  } else {
    m = m - 1.0f;
  }
  float z = m * m;
  float p = u2f(B_LOG_P[0]);
  for (int i = 1; i < 9; ++i) {
    float t = p * m;
    p = t + u2f(B_LOG_P[i]);
  }
  float y = p * m;
  y = y * z;
  float fe = (float)e;
  float q1 = fe * u2f(B_LOG_Q1);
  y = y + q1;
  float hz = 0.5f * z;
  y = y - hz;
  float res = m + y;
  float q2 = fe * u2f(B_LOG_Q2);
  return res + q2;
}

/* silu(x) = x / (1 + exp(-x)), a true divide.  code/cis2-fp/src/math.rs:414-419 */
float orc_silu(float x) {
  float nx = -x;
  float e = orc_exp(nx);
  float d = 1.0f + e;
  return x / d;
}

typedef float (*orc_unary)(float);
static orc_unary unary_of(int fn) {
  switch (fn) {
    case ORC_FN_EXP: return orc_exp;
    case ORC_FN_SIN: return orc_sin;
    case ORC_FN_COS: return orc_cos;
    case ORC_FN_LN: return orc_ln;
    case ORC_FN_SILU: return orc_silu;
    case ORC_FN_RSQRT: return orc_rsqrt;
    case ORC_FN_SQRT: return orc_sqrt;
    default: return NULL;
  }
}

void orc_math_map(int fn, const float *in, float *out, size_t n) {
  orc_unary f = unary_of(fn);
  orc_fpenv_pin();
  for (size_t i = 0; i < n; ++i) out[i] = f(in[i]);
}

void orc_div_map(const float *a, const float *b, float *out, size_t n) {
  orc_fpenv_pin();
  for (size_t i = 0; i < n; ++i) out[i] = a[i] / b[i];
}

uint64_t orc_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t orc_math_chunk_hash(int fn, uint32_t first, uint32_t count) {
  orc_unary f = unary_of(fn);
  orc_fpenv_pin();
  uint64_t h = 0;
  for (uint32_t j = 0; j < count; ++j) {
    uint32_t bits = first + j;
    uint32_t ob = f2u(f(u2f(bits)));
    h += orc_mix64((uint64_t)ob ^ ((uint64_t)bits * 0x9E3779B97F4A7C15ull));
  }
  return h;
}

/* ======================================================================
 * Reductions
 * ====================================================================== */

/* Strict left-to-right: acc = 0; acc = acc + (a_i*b_i).
 * code/cis2-fp/src/math.rs:40-48; spec §5.1 (CIS2_SPEC_v0.3.md:510-536). */
float orc_dot_seq(const float *a, const float *b, int n) {
  float acc = 0.0f;
  for (int i = 0; i < n; ++i) {
    float p = a[i] * b[i];
    acc = acc + p;
  }
  return acc;
}
/* code/cis2-fp/src/math.rs:52-58; spec §5.3 */
float orc_sum_seq(const float *a, int n) {
  float acc = 0.0f;
  for (int i = 0; i < n; ++i) acc = acc + a[i];
  return acc;
}

/* v0.4 candidate tree order: 32-leaf blocks (zero padded), five in-place
 * halving rounds leaf[i] = leaf[2i] + leaf[2i+1], block partials combined
 * left to right from 0.  code/cis2-fp/src/math.rs:60-125;
 * code/cis2-fp/docs/design/CIS2_V04_TREE_REDUCTION.md:35-98. */
static float tree_block(float leaf[32]) {
  for (int w = 32; w > 1; w >>= 1)
    for (int i = 0; i < w / 2; ++i) leaf[i] = leaf[2 * i] + leaf[2 * i + 1];
  return leaf[0];
}
float orc_dot_tree(const float *a, const float *b, int n) {
  float acc = 0.0f;
  for (int s = 0; s < n; s += 32) {
    float leaf[32];
    for (int i = 0; i < 32; ++i) leaf[i] = 0.0f;
    int len = n - s < 32 ? n - s : 32;
    for (int i = 0; i < len; ++i) leaf[i] = a[s + i] * b[s + i];
    float part = tree_block(leaf);
    acc = acc + part;
  }
  return acc;
}
float orc_sum_tree(const float *a, int n) {
  float acc = 0.0f;
  for (int s = 0; s < n; s += 32) {
    float leaf[32];
    for (int i = 0; i < 32; ++i) leaf[i] = 0.0f;
    int len = n - s < 32 ? n - s : 32;
    for (int i = 0; i < len; ++i) leaf[i] = a[s + i];
    float part = tree_block(leaf);
    acc = acc + part;
  }
  return acc;
}

/* Softmax: first-wins max scan (strict >), pinned exp of (v - max),
 * denominator by the pinned sum, then a true divide per element.
 * code/cis2-fp/src/math.rs:425-465; spec §9.3 (CIS2_SPEC_v0.3.md:1067-1077). */
void orc_softmax(float *v, int n, int mode) {
  if (n <= 0) return;
  float mx = v[0];
  for (int i = 1; i < n; ++i)
    if (v[i] > mx) mx = v[i];
  for (int i = 0; i < n; ++i) {
    float d = v[i] - mx;
    v[i] = orc_exp(d);
  }
  float den = mode ? orc_sum_tree(v, n) : orc_sum_seq(v, n);
  for (int i = 0; i < n; ++i) v[i] = v[i] / den;
}

/* Greedy argmax: scan from index 0 with strict >, first maximum wins.
 * code/cis2-fp/src/main.rs:1161-1169; spec §11.2 (CIS2_SPEC_v0.3.md:1131-1143). */
uint32_t orc_argmax(const float *v, int n) {
  int best = 0;
  float bv = v[0];
  if (atomic_load(&g_mutation) & ORC_MUT_ARGMAX_GE) { /* planted: last maximum wins */
    for (int i = 0; i < n; ++i)
      if (v[i] >= bv) { bv = v[i]; best = i; }
    return (uint32_t)best;
  }
  for (int i = 0; i < n; ++i)
    if (v[i] > bv) { bv = v[i]; best = i; }
  return (uint32_t)best;
}

/* ======================================================================
 * Worker pool (row-parallel work; each worker pins its own MXCSR)
 * ====================================================================== */
typedef void (*range_fn)(void *ctx, int lo, int hi);
typedef struct {
  pthread_mutex_t mu;
  pthread_cond_t go, done;
  int nthreads;
  pthread_t *tid;
  long gen;
  int pending;
  int quit;
  range_fn fn;
  void *ctx;
  int n;
} pool_t;

typedef struct { pool_t *p; int idx; } worker_arg;

static void chunk_bounds(int n, int parts, int idx, int *lo, int *hi) {
  int base = n / parts, rem = n % parts;
  *lo = idx * base + (idx < rem ? idx : rem);
  *hi = *lo + base + (idx < rem ? 1 : 0);
}

static void *worker_main(void *arg) {
  worker_arg *wa = (worker_arg *)arg;
  pool_t *p = wa->p;
  int idx = wa->idx;
  free(wa);
  orc_fpenv_pin();
  long seen = 0;
  for (;;) {
    pthread_mutex_lock(&p->mu);
    while (p->gen == seen && !p->quit) pthread_cond_wait(&p->go, &p->mu);
    if (p->quit) { pthread_mutex_unlock(&p->mu); return NULL; }
    seen = p->gen;
    range_fn fn = p->fn; void *ctx = p->ctx; int n = p->n;
    pthread_mutex_unlock(&p->mu);
    int lo, hi;
    chunk_bounds(n, p->nthreads, idx, &lo, &hi);
    orc_fpenv_pin(); /* per task: follows orc_set_mutation */
    if (lo < hi) fn(ctx, lo, hi);
    pthread_mutex_lock(&p->mu);
    if (--p->pending == 0) pthread_cond_signal(&p->done);
    pthread_mutex_unlock(&p->mu);
  }
}

static pool_t *pool_create(int nthreads) {
  if (nthreads <= 1) return NULL;
  pool_t *p = (pool_t *)calloc(1, sizeof(pool_t));
  pthread_mutex_init(&p->mu, NULL);
  pthread_cond_init(&p->go, NULL);
  pthread_cond_init(&p->done, NULL);
  p->nthreads = nthreads;
  p->tid = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
  for (int i = 1; i < nthreads; ++i) {
    worker_arg *wa = (worker_arg *)malloc(sizeof(worker_arg));
    wa->p = p; wa->idx = i;
    pthread_create(&p->tid[i], NULL, worker_main, wa);
  }
  return p;
}

static void pool_destroy(pool_t *p) {
  if (!p) return;
  pthread_mutex_lock(&p->mu);
  p->quit = 1;
  pthread_cond_broadcast(&p->go);
  pthread_mutex_unlock(&p->mu);
  for (int i = 1; i < p->nthreads; ++i) pthread_join(p->tid[i], NULL);
  free(p->tid);
  free(p);
}

/* Runs fn over [0,n) split into contiguous ranges; the caller's thread does
 * range 0.  Work below `grain` items runs on the caller only. */
static void pool_run(pool_t *p, int n, int grain, range_fn fn, void *ctx) {
  if (!p || n < grain) { if (n > 0) fn(ctx, 0, n); return; }
  pthread_mutex_lock(&p->mu);
  p->fn = fn; p->ctx = ctx; p->n = n;
  p->pending = p->nthreads - 1;
  p->gen++;
  pthread_cond_broadcast(&p->go);
  pthread_mutex_unlock(&p->mu);
  int lo, hi;
  chunk_bounds(n, p->nthreads, 0, &lo, &hi);
  if (lo < hi) fn(ctx, lo, hi);
  pthread_mutex_lock(&p->mu);
  while (p->pending > 0) pthread_cond_wait(&p->done, &p->mu);
  pthread_mutex_unlock(&p->mu);
}

/* ======================================================================
 * GEMV — every row is one strict chain (matvec -> dot_seq,
 * code/cis2-fp/src/main.rs:228-243).  Eight rows are carried at once, each
 * still summed strictly left to right: the order of the 4-row-interleaved
 * kernel (labs/rust-5/PREREG-from-ledger.md:54), which is memcmp-equal to
 * the single-row fold (labs/rust-5/reports/rust-5/RESULT.md:59).
 * ====================================================================== */
typedef struct { const float *W, *x; float *y; int K; int mode; } gemv_ctx;

static void gemv_rows(void *vctx, int lo, int hi) {
  gemv_ctx *c = (gemv_ctx *)vctx;
  const int K = c->K;
  int r = lo;
  if (c->mode == 0) {
    for (; r + 8 <= hi; r += 8) {
      const float *w0 = c->W + (size_t)r * K;
      float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
      float a4 = 0.0f, a5 = 0.0f, a6 = 0.0f, a7 = 0.0f;
      for (int k = 0; k < K; ++k) {
        float xk = c->x[k];
        float p0 = w0[k] * xk, p1 = w0[K + k] * xk;
        float p2 = w0[2 * (size_t)K + k] * xk, p3 = w0[3 * (size_t)K + k] * xk;
        float p4 = w0[4 * (size_t)K + k] * xk, p5 = w0[5 * (size_t)K + k] * xk;
        float p6 = w0[6 * (size_t)K + k] * xk, p7 = w0[7 * (size_t)K + k] * xk;
        a0 = a0 + p0; a1 = a1 + p1; a2 = a2 + p2; a3 = a3 + p3;
        a4 = a4 + p4; a5 = a5 + p5; a6 = a6 + p6; a7 = a7 + p7;
      }
      c->y[r] = a0; c->y[r + 1] = a1; c->y[r + 2] = a2; c->y[r + 3] = a3;
      c->y[r + 4] = a4; c->y[r + 5] = a5; c->y[r + 6] = a6; c->y[r + 7] = a7;
    }
    for (; r < hi; ++r) c->y[r] = orc_dot_seq(c->W + (size_t)r * K, c->x, K);
  } else {
    for (; r < hi; ++r) c->y[r] = orc_dot_tree(c->W + (size_t)r * K, c->x, K);
  }
}

void orc_gemv(const float *W, const float *x, float *y, int M, int K, int mode,
              int threads) {
  orc_fpenv_pin();
  gemv_ctx c = {W, x, y, K, mode};
  pool_t *p = pool_create(threads);
  pool_run(p, M, 64, gemv_rows, &c);
  pool_destroy(p);
}

/* ======================================================================
 * SHA-256 (FIPS 180-4), used for the witness and every digest.
 * ====================================================================== */
typedef struct { uint32_t h[8]; uint64_t bytes; uint8_t buf[64]; size_t fill; } sha_t;

static const uint32_t SHA_K[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u,
    0x923f82a4u, 0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u,
    0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u,
    0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u,
    0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u,
    0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
    0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au,
    0x5b9cca4fu, 0x682e6ff3u, 0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u,
    0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

static inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

static void sha_init(sha_t *s) {
  static const uint32_t iv[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                 0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  memcpy(s->h, iv, sizeof iv);
  s->bytes = 0;
  s->fill = 0;
}

static void sha_compress(uint32_t st[8], const uint8_t *blk) {
  uint32_t w[64];
  for (int i = 0; i < 16; ++i)
    w[i] = (uint32_t)blk[4 * i] << 24 | (uint32_t)blk[4 * i + 1] << 16 |
           (uint32_t)blk[4 * i + 2] << 8 | blk[4 * i + 3];
  for (int i = 16; i < 64; ++i) {
    uint32_t a = w[i - 15], b = w[i - 2];
    uint32_t s0 = rotr(a, 7) ^ rotr(a, 18) ^ (a >> 3);
    uint32_t s1 = rotr(b, 17) ^ rotr(b, 19) ^ (b >> 10);
    w[i] = w[i - 16] + s0 + w[i - 7] + s1;
  }
  uint32_t v[8];
  memcpy(v, st, sizeof v);
  for (int i = 0; i < 64; ++i) {
    uint32_t e = v[4], a = v[0];
    uint32_t t1 = v[7] + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) +
                  ((e & v[5]) ^ (~e & v[6])) + SHA_K[i] + w[i];
    uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) +
                  ((a & v[1]) ^ (a & v[2]) ^ (v[1] & v[2]));
    memmove(&v[1], &v[0], 7 * sizeof(uint32_t));
    v[4] += t1;
    v[0] = t1 + t2;
  }
  for (int i = 0; i < 8; ++i) st[i] += v[i];
}

static void sha_update(sha_t *s, const void *data, size_t n) {
  const uint8_t *p = (const uint8_t *)data;
  s->bytes += n;
  if (s->fill) {
    size_t take = 64 - s->fill < n ? 64 - s->fill : n;
    memcpy(s->buf + s->fill, p, take);
    s->fill += take; p += take; n -= take;
    if (s->fill == 64) { sha_compress(s->h, s->buf); s->fill = 0; }
  }
  while (n >= 64) { sha_compress(s->h, p); p += 64; n -= 64; }
  if (n) { memcpy(s->buf, p, n); s->fill = n; }
}

static void sha_u32le(sha_t *s, uint32_t v) {
  uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
  sha_update(s, b, 4);
}

static void sha_final(sha_t *s, uint8_t out[32]) {
  uint64_t bits = s->bytes * 8;
  uint8_t pad = 0x80;
  sha_update(s, &pad, 1);
  uint8_t z = 0;
  while (s->fill != 56) sha_update(s, &z, 1);
  uint8_t lb[8];
  for (int i = 0; i < 8; ++i) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
  sha_update(s, lb, 8);
  for (int i = 0; i < 8; ++i) {
    out[4 * i] = (uint8_t)(s->h[i] >> 24);
    out[4 * i + 1] = (uint8_t)(s->h[i] >> 16);
    out[4 * i + 2] = (uint8_t)(s->h[i] >> 8);
    out[4 * i + 3] = (uint8_t)s->h[i];
  }
}

void orc_sha256(const void *data, size_t n, uint8_t out[32]) {
  sha_t s;
  sha_init(&s);
  sha_update(&s, data, n);
  sha_final(&s, out);
}

/* sha256 over the little-endian bit patterns of n floats (the trace and
 * per-step logit digests; on x86 the in-memory bytes are exactly that). */
static void sha_floats(const float *v, size_t n, uint8_t out[32]) {
  orc_sha256(v, n * sizeof(float), out);
}

/* Table digest: LE bytes of the pinned constants in declared order
 * EXP_LOG2E, EXP_C1, EXP_C2, EXP_P0..5, PI_2 (8 bytes), SIN_C0..2,
 * COS_C0..2, LOG_SQRTHF, LOG_Q1, LOG_Q2, LOG_P0..8.
 * code/cis2-fp/src/math.rs:472-500; spec §6.6 (CIS2_SPEC_v0.3.md:856-878). */
void orc_table_digest(uint8_t out[32]) {
  sha_t s;
  sha_init(&s);
  sha_u32le(&s, B_EXP_LOG2E);
  sha_u32le(&s, B_EXP_C1);
  sha_u32le(&s, B_EXP_C2);
  for (int i = 0; i < 6; ++i) sha_u32le(&s, B_EXP_P[i]);
  uint64_t pb = B_PI_2_F64;
  sha_u32le(&s, (uint32_t)pb);
  sha_u32le(&s, (uint32_t)(pb >> 32));
  sha_u32le(&s, B_SIN_C0); sha_u32le(&s, B_SIN_C1); sha_u32le(&s, B_SIN_C2);
  sha_u32le(&s, B_COS_C0); sha_u32le(&s, B_COS_C1); sha_u32le(&s, B_COS_C2);
  sha_u32le(&s, B_LOG_SQRTHF); sha_u32le(&s, B_LOG_Q1); sha_u32le(&s, B_LOG_Q2);
  for (int i = 0; i < 9; ++i) sha_u32le(&s, B_LOG_P[i]);
  sha_final(&s, out);
}

/* inv_freq[i] = exp(-(((f32)(2i) / (f32)hd) * ln((f32)theta))), digest over
 * the LE value bytes.  code/cis2-fp/src/main.rs:849-869; spec §7.1-7.2
 * (CIS2_SPEC_v0.3.md:920-972). */
void orc_inv_freq(double rope_theta, int head_dim, float *out, uint8_t digest[32]) {
  orc_fpenv_pin();
  float lt = orc_ln((float)rope_theta);
  int half = head_dim / 2;
  sha_t s;
  sha_init(&s);
  for (int i = 0; i < half; ++i) {
    float frac = (float)(2 * i) / (float)head_dim;
    float a = frac * lt;
    float na = -a;
    out[i] = orc_exp(na);
    sha_u32le(&s, f2u(out[i]));
  }
  sha_final(&s, digest);
}

/* ======================================================================
 * Model
 * ====================================================================== */
typedef struct {
  float *ln1, *ln2, *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  float *bq, *bk, *bv, *qn, *kn; /* optional */
  float *kc, *vc;                /* KV cache [max_pos][kvd] */
} layer_t;

struct orc_model {
  orc_config c;
  int qd, kvd;
  float *embed, *lm_head, *final_norm;
  float *inv_freq;
  uint8_t table_dig[32], invf_dig[32];
  layer_t *L;
  pool_t *pool;
  /* scratch */
  float *h, *x, *q, *k, *v, *att, *o, *g, *u, *hid, *dn, *sc, *logits;
  char names[64][96]; /* tensor name buffer for orc_model_tensor */
};

static float *falloc(size_t n) {
  float *p = (float *)calloc(n ? n : 1, sizeof(float));
  if (!p) { fprintf(stderr, "oracle: out of memory (%zu floats)\n", n); abort(); }
  return p;
}

orc_model *orc_model_create(const orc_config *cfg) {
  orc_fpenv_pin();
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  m->c = *cfg;
  if (m->c.threads < 1) m->c.threads = 1;
  const orc_config *c = &m->c;
  m->qd = c->n_heads * c->head_dim;
  m->kvd = c->n_kv_heads * c->head_dim;
  m->inv_freq = falloc((size_t)c->head_dim / 2);
  orc_inv_freq(c->rope_theta, c->head_dim, m->inv_freq, m->invf_dig);
  orc_table_digest(m->table_dig);
  m->L = (layer_t *)calloc((size_t)c->n_layers, sizeof(layer_t));
  for (int l = 0; l < c->n_layers; ++l) {
    m->L[l].kc = falloc((size_t)c->max_pos * m->kvd);
    m->L[l].vc = falloc((size_t)c->max_pos * m->kvd);
  }
  int wide = c->hidden > m->qd ? c->hidden : m->qd;
  m->h = falloc((size_t)c->hidden);
  m->x = falloc((size_t)wide);
  m->q = falloc((size_t)m->qd);
  m->k = falloc((size_t)m->kvd);
  m->v = falloc((size_t)m->kvd);
  m->att = falloc((size_t)m->qd);
  m->o = falloc((size_t)c->hidden);
  m->g = falloc((size_t)c->inter);
  m->u = falloc((size_t)c->inter);
  m->hid = falloc((size_t)c->inter);
  m->dn = falloc((size_t)c->hidden);
  m->sc = falloc((size_t)c->n_heads * c->max_pos);
  m->logits = falloc((size_t)c->vocab);
  m->pool = pool_create(c->threads);
  return m;
}

void orc_model_destroy(orc_model *m) {
  if (!m) return;
  pool_destroy(m->pool);
  for (int l = 0; l < m->c.n_layers; ++l) {
    layer_t *L = &m->L[l];
    float *ps[] = {L->ln1, L->ln2, L->wq, L->wk, L->wv, L->wo, L->wg, L->wu, L->wd,
                   L->bq, L->bk, L->bv, L->qn, L->kn, L->kc, L->vc};
    for (size_t i = 0; i < sizeof ps / sizeof ps[0]; ++i) free(ps[i]);
  }
  free(m->L);
  free(m->embed); free(m->lm_head); free(m->final_norm); free(m->inv_freq);
  free(m->h); free(m->x); free(m->q); free(m->k); free(m->v); free(m->att);
  free(m->o); free(m->g); free(m->u); free(m->hid); free(m->dn); free(m->sc);
  free(m->logits);
  free(m);
}

void orc_model_digests(const orc_model *m, uint8_t table[32], uint8_t inv_freq[32]) {
  memcpy(table, m->table_dig, 32);
  memcpy(inv_freq, m->invf_dig, 32);
}

void orc_model_reset(orc_model *m) {
  for (int l = 0; l < m->c.n_layers; ++l) {
    memset(m->L[l].kc, 0, (size_t)m->c.max_pos * m->kvd * sizeof(float));
    memset(m->L[l].vc, 0, (size_t)m->c.max_pos * m->kvd * sizeof(float));
  }
}

/* Locate the slot and expected element count of a tensor name, following
 * the checkpoint naming the reference loader uses
 * (code/cis2-fp/gpu/cis2_host.cpp:133-158, Qwen3 q/k norms
 * labs/w1x-qwen3/scripts/qwen3-port.diff:139-141). */
static float **slot_of(orc_model *m, const char *name, size_t *want) {
  const orc_config *c = &m->c;
  size_t H = (size_t)c->hidden, I = (size_t)c->inter, V = (size_t)c->vocab;
  size_t QD = (size_t)m->qd, KV = (size_t)m->kvd, HD = (size_t)c->head_dim;
  if (!strcmp(name, "model.embed_tokens.weight")) { *want = V * H; return &m->embed; }
  if (!strcmp(name, "model.norm.weight")) { *want = H; return &m->final_norm; }
  if (!strcmp(name, "lm_head.weight")) { *want = V * H; return &m->lm_head; }
  int li = -1, off = 0;
  if (sscanf(name, "model.layers.%d.%n", &li, &off) != 1 || off == 0) return NULL;
  if (li < 0 || li >= c->n_layers) return NULL;
  layer_t *L = &m->L[li];
  const char *s = name + off;
  struct { const char *n; float **p; size_t w; } tab[] = {
      {"input_layernorm.weight", &L->ln1, H},
      {"post_attention_layernorm.weight", &L->ln2, H},
      {"self_attn.q_proj.weight", &L->wq, QD * H},
      {"self_attn.k_proj.weight", &L->wk, KV * H},
      {"self_attn.v_proj.weight", &L->wv, KV * H},
      {"self_attn.o_proj.weight", &L->wo, H * QD},
      {"mlp.gate_proj.weight", &L->wg, I * H},
      {"mlp.up_proj.weight", &L->wu, I * H},
      {"mlp.down_proj.weight", &L->wd, H * I},
      {"self_attn.q_proj.bias", &L->bq, QD},
      {"self_attn.k_proj.bias", &L->bk, KV},
      {"self_attn.v_proj.bias", &L->bv, KV},
      {"self_attn.q_norm.weight", &L->qn, HD},
      {"self_attn.k_norm.weight", &L->kn, HD},
  };
  for (size_t i = 0; i < sizeof tab / sizeof tab[0]; ++i)
    if (!strcmp(s, tab[i].n)) { *want = tab[i].w; return tab[i].p; }
  return NULL;
}

/* BF16 -> F32 is the exact bit shift (u16 << 16), a bit operation that is
 * not subject to FTZ.  code/cis2-fp/src/math.rs:33-35; spec §4. */
int orc_model_set_bf16(orc_model *m, const char *name, const uint16_t *bits, size_t n) {
  size_t want = 0;
  float **slot = slot_of(m, name, &want);
  if (!slot) return -1;
  if (n != want) return -2;
  free(*slot);
  float *d = falloc(n);
  uint32_t *du = (uint32_t *)d;
  for (size_t i = 0; i < n; ++i) du[i] = (uint32_t)bits[i] << 16;
  *slot = d;
  return 0;
}

const char *orc_model_tensor(const orc_model *m_in, int i, size_t *count) {
  orc_model *m = (orc_model *)m_in;
  const orc_config *c = &m->c;
  static const char *per_layer[] = {
      "input_layernorm.weight", "post_attention_layernorm.weight",
      "self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
      "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight",
      "mlp.down_proj.weight"};
  static __thread char buf[128];
  if (i == 0) { snprintf(buf, sizeof buf, "model.embed_tokens.weight"); }
  else if (i <= 9 * c->n_layers) {
    int li = (i - 1) / 9, j = (i - 1) % 9;
    snprintf(buf, sizeof buf, "model.layers.%d.%s", li, per_layer[j]);
  } else if (i == 9 * c->n_layers + 1) { snprintf(buf, sizeof buf, "model.norm.weight"); }
  else if (i == 9 * c->n_layers + 2 && !c->tied) { snprintf(buf, sizeof buf, "lm_head.weight"); }
  else return NULL;
  size_t want = 0;
  slot_of(m, buf, &want);
  if (count) *count = want;
  return buf;
}

/* ---- forward-pass building blocks -------------------------------------- */

/* RMSNorm: sq_i = x_i*x_i materialised, ss = pinned sum, mean = ss/(f32)n
 * (a divide), inv = rsqrt_cr(mean + eps), out_i = (x_i*inv)*w_i.
 * code/cis2-fp/src/main.rs:245-260; spec §8 (CIS2_SPEC_v0.3.md:1008-1035). */
static void rmsnorm(const float *x, const float *w, float eps, int n, int mode,
                    float *out) {
  float *sq = (float *)malloc((size_t)n * sizeof(float));
  for (int i = 0; i < n; ++i) sq[i] = x[i] * x[i];
  float ss = mode ? orc_sum_tree(sq, n) : orc_sum_seq(sq, n);
  free(sq);
  float mean = ss / (float)n;
  float arg = mean + eps;
  float inv = orc_rsqrt(arg);
  for (int i = 0; i < n; ++i) {
    float sx = x[i] * inv;
    out[i] = sx * w[i];
  }
}

typedef struct { const float *W, *x; float *y; int K; int mode; } mv_ctx;
static void mv_rows(void *vctx, int lo, int hi) {
  mv_ctx *c = (mv_ctx *)vctx;
  gemv_ctx g = {c->W, c->x, c->y, c->K, c->mode};
  gemv_rows(&g, lo, hi);
}
static void matvec(orc_model *m, const float *W, const float *x, int M, int K, float *y) {
  mv_ctx c = {W, x, y, K, m->c.reduction};
  pool_run(m->pool, M, 64, mv_rows, &c);
}

static void add_bias(float *x, const float *b, int n) {
  if (!b) return;
  for (int i = 0; i < n; ++i) x[i] = x[i] + b[i];
}

/* Rotate-half RoPE on one head: angle = (f32)pos * inv_freq[i];
 * o1 = x1*cos + (-x2)*sin, o2 = x2*cos + x1*sin.
 * code/cis2-fp/src/main.rs:285-307; spec §7.3-7.4 (CIS2_SPEC_v0.3.md:973-1007). */
static void rope_head(float *hv, int hd, int pos, const float *inv_freq) {
  int half = hd / 2;
  for (int i = 0; i < half; ++i) {
    float ang = (float)pos * inv_freq[i];
    float cv = orc_cos(ang), sv = orc_sin(ang);
    float x1 = hv[i], x2 = hv[i + half];
    float t1 = x1 * cv;
    float nx2 = -x2;
    float t2 = nx2 * sv;
    float t3 = x2 * cv;
    float t4 = x1 * sv;
    hv[i] = t1 + t2;
    hv[i + half] = t3 + t4;
  }
}

typedef struct { orc_model *m; const layer_t *L; int pos; float scale; } att_ctx;

/* Per query head: scores_j = dot(q_h, k_j) * scale, softmax, then
 * out_d = fold over j of (p_j * v_j[d]) — the V mix is always sequential.
 * code/cis2-fp/src/main.rs:429-467; spec §9 (CIS2_SPEC_v0.3.md:1036-1094);
 * GQA head map kv = qh / group (main.rs:205). */
static void att_heads(void *vctx, int lo, int hi) {
  att_ctx *a = (att_ctx *)vctx;
  orc_model *m = a->m;
  const orc_config *c = &m->c;
  int hd = c->head_dim, group = c->n_heads / c->n_kv_heads, len = a->pos + 1;
  for (int qh = lo; qh < hi; ++qh) {
    int kvh = qh / group;
    const float *qv = m->q + (size_t)qh * hd;
    float *s = m->sc + (size_t)qh * len;
    for (int j = 0; j < len; ++j) {
      const float *kj = a->L->kc + (size_t)j * m->kvd + (size_t)kvh * hd;
      float d = c->reduction ? orc_dot_tree(qv, kj, hd) : orc_dot_seq(qv, kj, hd);
      s[j] = d * a->scale;
    }
  }
}
static void att_softmax(void *vctx, int lo, int hi) {
  att_ctx *a = (att_ctx *)vctx;
  int len = a->pos + 1;
  for (int qh = lo; qh < hi; ++qh)
    orc_softmax(a->m->sc + (size_t)qh * len, len, a->m->c.reduction);
}
static void att_mix(void *vctx, int lo, int hi) {
  att_ctx *a = (att_ctx *)vctx;
  orc_model *m = a->m;
  const orc_config *c = &m->c;
  int hd = c->head_dim, group = c->n_heads / c->n_kv_heads, len = a->pos + 1;
  for (int idx = lo; idx < hi; ++idx) {
    int qh = idx / hd, d = idx % hd, kvh = qh / group;
    const float *s = m->sc + (size_t)qh * len;
    const float *vb = a->L->vc + (size_t)kvh * hd + d;
    float acc = 0.0f;
    for (int j = 0; j < len; ++j) {
      float p = s[j] * vb[(size_t)j * m->kvd];
      acc = acc + p;
    }
    m->att[idx] = acc;
  }
}

static void trace_emit(orc_trace_fn cb, void *user, int pos, int layer, const char *op,
                       const float *v, size_t n) {
  if (!cb) return;
  uint8_t d[32];
  sha_floats(v, n, d);
  cb(pos, layer, op, d, user);
}

/* One decode step, in the op order of code/cis2-fp/src/main.rs:355-529
 * (C++ mirror gpu/cis2_model.h:685-760, Qwen3 QK-norm
 * labs/w1x-qwen3/scripts/qwen3-port.diff:66-80). */
int orc_forward(orc_model *m, int pos, uint32_t token, float *logits,
                orc_trace_fn cb, void *user) {
  const orc_config *c = &m->c;
  if (pos < 0 || pos >= c->max_pos) return -3;
  if ((int)token >= c->vocab) return -4;
  if (!m->embed || !m->final_norm || (!c->tied && !m->lm_head)) return -5;
  orc_fpenv_pin();
  const int H = c->hidden, hd = c->head_dim, qd = m->qd, kvd = m->kvd;
  const int mode = c->reduction;
  const float scale = orc_rsqrt((float)hd);

  memcpy(m->h, m->embed + (size_t)token * H, (size_t)H * sizeof(float));
  trace_emit(cb, user, pos, -1, "embedding", m->h, H);

  for (int l = 0; l < c->n_layers; ++l) {
    layer_t *L = &m->L[l];
    if (!L->wq || !L->wd || !L->ln1) return -5;
    rmsnorm(m->h, L->ln1, c->eps, H, mode, m->x);
    trace_emit(cb, user, pos, l, "norm1", m->x, H);
    matvec(m, L->wq, m->x, qd, H, m->q);
    add_bias(m->q, L->bq, qd);
    trace_emit(cb, user, pos, l, "q", m->q, qd);
    matvec(m, L->wk, m->x, kvd, H, m->k);
    add_bias(m->k, L->bk, kvd);
    trace_emit(cb, user, pos, l, "k", m->k, kvd);
    matvec(m, L->wv, m->x, kvd, H, m->v);
    add_bias(m->v, L->bv, kvd);
    trace_emit(cb, user, pos, l, "v", m->v, kvd);
    if (L->qn) {
      for (int hh = 0; hh < c->n_heads; ++hh)
        rmsnorm(m->q + (size_t)hh * hd, L->qn, c->eps, hd, mode, m->q + (size_t)hh * hd);
      trace_emit(cb, user, pos, l, "q_norm", m->q, qd);
    }
    if (L->kn) {
      for (int hh = 0; hh < c->n_kv_heads; ++hh)
        rmsnorm(m->k + (size_t)hh * hd, L->kn, c->eps, hd, mode, m->k + (size_t)hh * hd);
      trace_emit(cb, user, pos, l, "k_norm", m->k, kvd);
    }
    for (int hh = 0; hh < c->n_heads; ++hh) rope_head(m->q + (size_t)hh * hd, hd, pos, m->inv_freq);
    trace_emit(cb, user, pos, l, "rope_q", m->q, qd);
    for (int hh = 0; hh < c->n_kv_heads; ++hh) rope_head(m->k + (size_t)hh * hd, hd, pos, m->inv_freq);
    trace_emit(cb, user, pos, l, "rope_k", m->k, kvd);
    /* cache holds rotated keys and raw values (main.rs:426-427) */
    memcpy(L->kc + (size_t)pos * kvd, m->k, (size_t)kvd * sizeof(float));
    memcpy(L->vc + (size_t)pos * kvd, m->v, (size_t)kvd * sizeof(float));

    att_ctx ac = {m, L, pos, scale};
    int len = pos + 1;
    pool_run(m->pool, c->n_heads, (len * hd < 4096) ? 1 << 30 : 2, att_heads, &ac);
    trace_emit(cb, user, pos, l, "scores", m->sc, (size_t)c->n_heads * len);
    pool_run(m->pool, c->n_heads, len < 512 ? 1 << 30 : 2, att_softmax, &ac);
    trace_emit(cb, user, pos, l, "softmax", m->sc, (size_t)c->n_heads * len);
    pool_run(m->pool, qd, len < 64 ? 1 << 30 : 64, att_mix, &ac);
    trace_emit(cb, user, pos, l, "attn_out", m->att, qd);

    matvec(m, L->wo, m->att, H, qd, m->o);
    trace_emit(cb, user, pos, l, "o_proj", m->o, H);
    for (int i = 0; i < H; ++i) m->h[i] = m->h[i] + m->o[i];
    trace_emit(cb, user, pos, l, "resid1", m->h, H);

    rmsnorm(m->h, L->ln2, c->eps, H, mode, m->x);
    trace_emit(cb, user, pos, l, "norm2", m->x, H);
    matvec(m, L->wg, m->x, c->inter, H, m->g);
    trace_emit(cb, user, pos, l, "gate", m->g, c->inter);
    matvec(m, L->wu, m->x, c->inter, H, m->u);
    trace_emit(cb, user, pos, l, "up", m->u, c->inter);
    /* hid = silu(gate) * up, main.rs:484-487 */
    for (int i = 0; i < c->inter; ++i) {
      float sg = orc_silu(m->g[i]);
      m->hid[i] = sg * m->u[i];
    }
    trace_emit(cb, user, pos, l, "silu_mul", m->hid, c->inter);
    matvec(m, L->wd, m->hid, H, c->inter, m->dn);
    trace_emit(cb, user, pos, l, "down", m->dn, H);
    for (int i = 0; i < H; ++i) m->h[i] = m->h[i] + m->dn[i];
    trace_emit(cb, user, pos, l, "resid2", m->h, H);
  }
  rmsnorm(m->h, m->final_norm, c->eps, H, mode, m->x);
  trace_emit(cb, user, pos, -1, "final_norm", m->x, H);
  const float *lm = c->tied ? m->embed : m->lm_head;
  matvec(m, lm, m->x, c->vocab, H, logits);
  trace_emit(cb, user, pos, -1, "logits", logits, c->vocab);
  return 0;
}

int orc_model_hidden(const orc_model *m, float *out) {
  if (!m || !out || !m->x) return -1;
  memcpy(out, m->x, sizeof(float) * (size_t)m->c.hidden);
  return 0;
}

/* Witness fold: raw 32-byte sha256 of weights, tokenizer, config, then the
 * table digest and inv_freq digest, the prompt ids (u32 LE), then per step
 * the already-computed logits (u32 LE bit patterns, vocab order) and the
 * argmax id.  Argmax digest = sha256(prompt ids ++ generated ids).
 * code/cis2-fp/src/main.rs:1084-1092,1159-1194,1214-1226;
 * code/cis2-fp/gpu/cis2_host.cpp:180-218; spec §12 (CIS2_SPEC_v0.3.md:1144-1249). */
int orc_decode(orc_model *m, const uint32_t *prompt, int n_prompt, int gen_toks,
               const uint8_t hdr[96], uint32_t *out_ids, uint8_t witness[32],
               uint8_t argmax_digest[32], uint8_t *step_digests,
               orc_trace_fn cb, void *user) {
  const orc_config *c = &m->c;
  if (n_prompt <= 0) return -6;
  if (n_prompt + gen_toks > c->max_pos) return -3;
  orc_model_reset(m);
  sha_t w;
  sha_init(&w);
  sha_update(&w, hdr, 96);
  sha_update(&w, m->table_dig, 32);
  sha_update(&w, m->invf_dig, 32);
  for (int i = 0; i < n_prompt; ++i) sha_u32le(&w, prompt[i]);
  float *lg = m->logits;
  for (int p = 0; p < n_prompt; ++p) {
    int rc = orc_forward(m, p, prompt[p], lg, cb, user);
    if (rc) return rc;
  }
  for (int i = 0; i < n_prompt; ++i) out_ids[i] = prompt[i];
  for (int s = 0; s < gen_toks; ++s) {
    uint32_t nid = orc_argmax(lg, c->vocab);
    sha_update(&w, lg, (size_t)c->vocab * sizeof(float));
    sha_u32le(&w, nid);
    if (step_digests) sha_floats(lg, (size_t)c->vocab, step_digests + 32 * (size_t)s);
    out_ids[n_prompt + s] = nid;
    int rc = orc_forward(m, n_prompt + s, nid, lg, cb, user);
    if (rc) return rc;
  }
  sha_final(&w, witness);
  sha_t a;
  sha_init(&a);
  for (int i = 0; i < n_prompt + gen_toks; ++i) sha_u32le(&a, out_ids[i]);
  sha_final(&a, argmax_digest);
  return 0;
}

/* ======================================================================
 * Seeded sampling, CIS-2 v0.4 draft section 14
 * (code/patches/cis2-spec__seeded-sampling.patch:57-196).
 * ====================================================================== */

static uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

/* MurmurHash3_x86_32: 4-byte little-endian blocks mixed into h, the tail,
 * the length, then the fmix32 finaliser (draft 14.2: the public-domain
 * reference function of that name). */
uint32_t orc_murmur3_32(const void *key, size_t len, uint32_t seed) {
  const uint8_t *d = (const uint8_t *)key;
  const uint32_t c1 = 0xcc9e2d51u, c2 = 0x1b873593u;
  uint32_t h = seed;
  const size_t nb = len / 4;
  for (size_t i = 0; i < nb; ++i) {
    uint32_t k = (uint32_t)d[4 * i] | ((uint32_t)d[4 * i + 1] << 8) |
                 ((uint32_t)d[4 * i + 2] << 16) | ((uint32_t)d[4 * i + 3] << 24);
    k *= c1;
    k = rotl32(k, 15);
    k *= c2;
    h ^= k;
    h = rotl32(h, 13);
    h = h * 5u + 0xe6546b64u;
  }
  const uint8_t *t = d + 4 * nb;
  uint32_t k = 0;
  switch (len & 3) {
    case 3: k ^= (uint32_t)t[2] << 16; /* fall through */
    case 2: k ^= (uint32_t)t[1] << 8;  /* fall through */
    case 1:
      k ^= t[0];
      k *= c1;
      k = rotl32(k, 15);
      k *= c2;
      h ^= k;
  }
  h ^= (uint32_t)len;
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  return h;
}

/* Draft 14.2: key = seed (u64 LE) || step (u32 LE) || index (u32 LE),
 * hash seed 0x43495332 ("CIS2"); m = (h >> 9) * 2 + 1 (odd, < 2^24),
 * u = f32(m) * 2^-24 (both exact); g = 0 - ln(0 - ln(u)) with the pinned
 * logarithm of section 6.5. */
void orc_sample_noise(uint64_t seed, uint32_t step, uint32_t index, uint32_t *h,
                      float *u, float *g) {
  uint8_t key[16];
  for (int i = 0; i < 8; ++i) key[i] = (uint8_t)(seed >> (8 * i));
  for (int i = 0; i < 4; ++i) key[8 + i] = (uint8_t)(step >> (8 * i));
  for (int i = 0; i < 4; ++i) key[12 + i] = (uint8_t)(index >> (8 * i));
  const uint32_t hv = orc_murmur3_32(key, 16, 0x43495332u);
  const uint32_t m = (hv >> 9) * 2u + 1u;
  const float two_m24 = 5.9604644775390625e-08f; /* 2^-24 */
  const float uv = (float)m * two_m24;
  const float inner = 0.0f - orc_ln(uv);
  const float gv = 0.0f - orc_ln(inner);
  if (h) *h = hv;
  if (u) *u = uv;
  if (g) *g = gv;
}

/* Draft 14.1: temperature finite and > 0; top_p in (0, 1]. */
int orc_sample_params_ok(float temperature, uint32_t top_k, float top_p) {
  (void)top_k;
  if (!(temperature > 0.0f) || temperature == INFINITY) return -1;
  if (!(top_p > 0.0f) || !(top_p <= 1.0f)) return -1;
  return 0;
}

/* rank order of 14.3 step 2: i precedes j iff s_i > s_j, or s_i == s_j and
 * i < j (so -0 and +0 tie and fall back to the index) */
static const float *g_rank_s;
static int rank_cmp(const void *a, const void *b) {
  const uint32_t i = *(const uint32_t *)a, j = *(const uint32_t *)b;
  const float si = g_rank_s[i], sj = g_rank_s[j];
  if (si > sj) return -1;
  if (si < sj) return 1;
  return i < j ? -1 : (i > j ? 1 : 0);
}

/* Draft 14.3-14.4.  s_i = l_i / T; rank order; top-k keeps ranks < k;
 * top-p over the kept ranks: m = s of rank 0, e_r = exp(s_r - m),
 * denom = sum_seq(e) in rank order, p_r = e_r / denom, running c_r =
 * c_{r-1} + p_r from 0; rank r is kept iff r == 0 or c_{r-1} < top_p.
 * z_i = s_i + g_i for kept i, -inf otherwise; the first index of the
 * maximum z (strict > scan from index 0, section 11.2) is drawn. */
uint32_t orc_sample(const float *logits, int V, uint64_t seed, uint32_t step,
                    float temperature, uint32_t top_k, float top_p, float *z,
                    uint32_t *nkeep) {
  if (V <= 0 || orc_sample_params_ok(temperature, top_k, top_p)) return UINT32_MAX;
  float *s = (float *)malloc((size_t)V * sizeof(float));
  uint32_t *ord = (uint32_t *)malloc((size_t)V * sizeof(uint32_t));
  float *zz = z ? z : (float *)malloc((size_t)V * sizeof(float));
  uint32_t res = UINT32_MAX;
  if (!s || !ord || !zz) goto done;
  for (int i = 0; i < V; ++i) {
    s[i] = logits[i] / temperature;
    if (s[i] != s[i]) goto done;
    ord[i] = (uint32_t)i;
  }
  g_rank_s = s;
  qsort(ord, (size_t)V, sizeof(uint32_t), rank_cmp);
  uint32_t K = (top_k > 0 && top_k < (uint32_t)V) ? top_k : (uint32_t)V;
  uint32_t keep = K;
  if (top_p < 1.0f) {
    float *e = (float *)malloc((size_t)K * sizeof(float));
    if (!e) goto done;
    const float m = s[ord[0]];
    for (uint32_t r = 0; r < K; ++r) e[r] = orc_exp(s[ord[r]] - m);
    float den = 0.0f;
    for (uint32_t r = 0; r < K; ++r) den = den + e[r];
    float c = 0.0f;
    for (uint32_t r = 0; r < K; ++r) {
      if (r > 0 && !(c < top_p)) {
        keep = r;
        break;
      }
      const float p = e[r] / den;
      c = c + p;
    }
    free(e);
  }
  for (int i = 0; i < V; ++i) zz[i] = -INFINITY;
  for (uint32_t r = 0; r < keep; ++r) {
    const uint32_t i = ord[r];
    float g;
    orc_sample_noise(seed, step, i, NULL, NULL, &g);
    zz[i] = s[i] + g;
  }
  res = orc_argmax(zz, V);
  if (nkeep) *nkeep = keep;
done:
  free(s);
  free(ord);
  if (!z) free(zz);
  return res;
}

/* Draft 14.5: greedy receipt with, after the prompt ids, "CIS2-SAMPLE-1"
 * (13 bytes), seed (u64 LE), temperature bits, top_k, top_p bits (u32
 * LE); per step the logits then the drawn id; the argmax digest is fed the
 * drawn ids. */
int orc_decode_sampled(orc_model *m, const uint32_t *prompt, int n_prompt, int gen_toks,
                       const uint8_t hdr[96], uint64_t seed, float temperature,
                       uint32_t top_k, float top_p, uint32_t *out_ids, uint8_t witness[32],
                       uint8_t argmax_digest[32], uint8_t *step_digests) {
  const orc_config *c = &m->c;
  if (n_prompt <= 0) return -6;
  if (n_prompt + gen_toks > c->max_pos) return -3;
  if (orc_sample_params_ok(temperature, top_k, top_p)) return -1;
  orc_model_reset(m);
  sha_t w;
  sha_init(&w);
  sha_update(&w, hdr, 96);
  sha_update(&w, m->table_dig, 32);
  sha_update(&w, m->invf_dig, 32);
  for (int i = 0; i < n_prompt; ++i) sha_u32le(&w, prompt[i]);
  sha_update(&w, "CIS2-SAMPLE-1", 13);
  sha_u32le(&w, (uint32_t)seed);
  sha_u32le(&w, (uint32_t)(seed >> 32));
  uint32_t tb, pb;
  memcpy(&tb, &temperature, 4);
  memcpy(&pb, &top_p, 4);
  sha_u32le(&w, tb);
  sha_u32le(&w, top_k);
  sha_u32le(&w, pb);
  float *lg = m->logits;
  for (int p = 0; p < n_prompt; ++p) {
    int rc = orc_forward(m, p, prompt[p], lg, NULL, NULL);
    if (rc) return rc;
  }
  for (int i = 0; i < n_prompt; ++i) out_ids[i] = prompt[i];
  for (int s = 0; s < gen_toks; ++s) {
    const uint32_t nid = orc_sample(lg, c->vocab, seed, (uint32_t)s, temperature, top_k, top_p,
                                    NULL, NULL);
    if (nid == UINT32_MAX) return -10;
    sha_update(&w, lg, (size_t)c->vocab * sizeof(float));
    sha_u32le(&w, nid);
    if (step_digests) sha_floats(lg, (size_t)c->vocab, step_digests + 32 * (size_t)s);
    out_ids[n_prompt + s] = nid;
    int rc = orc_forward(m, n_prompt + s, nid, lg, NULL, NULL);
    if (rc) return rc;
  }
  sha_final(&w, witness);
  sha_t a;
  sha_init(&a);
  for (int i = 0; i < n_prompt + gen_toks; ++i) sha_u32le(&a, out_ids[i]);
  sha_final(&a, argmax_digest);
  return 0;
}
