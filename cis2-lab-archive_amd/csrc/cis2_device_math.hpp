// cis2_device_math.hpp — CIS-2 v0.3b pinned arithmetic for gfx950.
//
// Every function here reproduces, bit for bit on all 2^32 binary32 inputs,
// the x86-64 SSE reference evaluated under MXCSR FTZ|DAZ with no FMA
// (code/cis2-fp/gpu/cis2_math.h, code/cis2-fp/src/math.rs):
//
//   * Build contract: hipcc -O3 -ffp-contract=off, f32 denormals flushed
//     (-fgpu-flush-denormals-to-zero), no fast math, packed-fp32 ops
//     disabled.  Each mul and add is its own statement and its own rounding.
//   * DAZ is made explicit: a subnormal input is replaced by the signed zero
//     before anything else, so comparisons and the f32->f64 widening in the
//     sin/cos reduction see what x86 DAZ shows them.
//   * Non-finite inputs return the exact bits x86 produces (its NaN
//     propagation keeps the first NaN operand's payload, quieted; an invalid
//     operation yields the negative "indefinite" NaN 0xFFC00000).  These
//     paths are pinned by the exhaustive fixture and never taken in decode.
//   * Divide and sqrt are the compiler's correctly rounded f32 sequences
//     (HIP's default -fhip-fp32-correctly-rounded-divide-sqrt); the f64
//     divide in the octant reduction is the correctly rounded f64 sequence.
//     No hardware approximate transcendental (v_exp/v_log/v_sin/v_cos,
//     v_rcp/v_rsq on their own) is used.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cis2 {

// Pinned constants by bit pattern (code/cis2-fp/gpu/cis2_consts.inc:5-32).
constexpr uint32_t kExpLog2e = 0x3fb8aa3bu;
constexpr uint32_t kExpC1 = 0x3f318000u;
constexpr uint32_t kExpC2 = 0xb95e8083u;
constexpr uint32_t kExpP0 = 0x39506967u, kExpP1 = 0x3ab743ceu, kExpP2 = 0x3c088908u,
                   kExpP3 = 0x3d2aa9c1u, kExpP4 = 0x3e2aaaaau, kExpP5 = 0x3f000000u;
constexpr uint32_t kSinC0 = 0xbe2aaaa3u, kSinC1 = 0x3c08839eu, kSinC2 = 0xb94ca1f9u;
constexpr uint32_t kCosC0 = 0x3d2aaaa5u, kCosC1 = 0xbab6061au, kCosC2 = 0x37ccf5ceu;
constexpr uint32_t kLogSqrtHf = 0x3f3504f3u, kLogQ1 = 0xb95e8083u, kLogQ2 = 0x3f318000u;
constexpr uint32_t kLogP0 = 0x3d9021bbu, kLogP1 = 0xbdebd1b8u, kLogP2 = 0x3def251bu,
                   kLogP3 = 0xbdfe5d4fu, kLogP4 = 0x3e11e9bfu, kLogP5 = 0xbe2aae50u,
                   kLogP6 = 0x3e4cceadu, kLogP7 = 0xbe7ffffcu, kLogP8 = 0x3eaaaaaau;
constexpr uint64_t kPio2F64 = 0x3ff921fb54442d18ull;
constexpr uint32_t kQNaN = 0x7FC00000u;       // the spec's NaN (Rust f32::NAN)
constexpr uint32_t kIndefinite = 0xFFC00000u; // x86 default NaN of an invalid op

__device__ __forceinline__ float fb(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t bf(float f) { return __float_as_uint(f); }
__device__ __forceinline__ bool is_nan_bits(uint32_t b) {
  return (b & 0x7F800000u) == 0x7F800000u && (b & 0x007FFFFFu) != 0u;
}
// DAZ: a subnormal operand reads as the zero of the same sign.
__device__ __forceinline__ float daz(float x) {
  uint32_t b = bf(x);
  return (b & 0x7F800000u) == 0u ? fb(b & 0x80000000u) : x;
}

// Rust `as` casts saturate (code/cis2-fp/src/math.rs:167-225, :253-264).
__device__ __forceinline__ int32_t sat_i32(float x) {
  if (x != x) return 0;
  if (x >= 2147483648.0f) return INT32_MAX;
  if (x <= -2147483648.0f) return INT32_MIN;
  return (int32_t)x;
}
__device__ __forceinline__ int64_t sat_i64(double x) {
  if (x != x) return 0;
  if (x >= 9223372036854775808.0) return INT64_MAX;
  if (x <= -9223372036854775808.0) return INT64_MIN;
  return (int64_t)x;
}
// floor for binary32 through the exact truncating conversion.
__device__ __forceinline__ float floor_f32(float x) {
  float ax = x < 0.0f ? -x : x;
  if (!(ax < 8388608.0f)) return x;
  float t = (float)(int32_t)x;
  if (x < t) t = t - 1.0f;
  return t;
}
// Round half away from zero with the sign of zero kept (Rust f64::round).
__device__ __forceinline__ double round_away(double x) {
  double ax = x < 0.0 ? -x : x;
  if (!(ax < 4503599627370496.0)) return x;
  double t = (double)(int64_t)ax;
  if (ax - t >= 0.5) t = t + 1.0;
  uint64_t mag = (uint64_t)__double_as_longlong(t) & 0x7FFFFFFFFFFFFFFFull;
  uint64_t sgn = (uint64_t)__double_as_longlong(x) & 0x8000000000000000ull;
  return __longlong_as_double((long long)(mag | sgn));
}

// The value-level compiler treats NaN bits as unspecified and may fold an
// explicit NaN return into the sqrt of a negative input; selecting on the
// integer bits after an opaque copy keeps the x86 pattern.
__device__ __forceinline__ uint32_t opaque_u32(uint32_t v) {
  __asm__ volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ float nan_fixup(float r, uint32_t in_bits) {
  uint32_t rb = opaque_u32(bf(r));
  if (is_nan_bits(in_bits)) rb = in_bits | 0x00400000u;  // quiet the input NaN
  else if ((in_bits >> 31) && (in_bits & 0x7FFFFFFFu)) rb = kIndefinite;  // sqrt(x<0)
  return fb(rb);
}
// Correctly rounded sqrt (IEEE), code/cis2-fp/src/math.rs:133-135.
__device__ __forceinline__ float sqrt_cr(float x) {
  x = daz(x);
  uint32_t b = bf(x);
  return nan_fixup(__builtin_sqrtf(x), b);
}
// rsqrt_cr(x) = 1 / sqrt(x), two correctly rounded operations.
__device__ __forceinline__ float rsqrt_cr(float x) {
  x = daz(x);
  uint32_t b = bf(x);
  float s = __builtin_sqrtf(x);
  return nan_fixup(1.0f / s, b);
}

// Exponent-field scaling (code/cis2-fp/src/math.rs:206-225): underflow is
// +0 for either sign, overflow a signed infinity.
// Written as selects (the same value as testing the cases in turn: zero,
// underflow, overflow, in range) so that a loop over it does not branch.
__device__ __forceinline__ float ldexp_bits(float y, int32_t k) {
  const uint32_t b = bf(y);
  const int32_t e = (int32_t)((b >> 23) & 0xFFu) + k;
  const float ov = (b >> 31) ? fb(0xFF800000u) : fb(0x7F800000u);
  const float in = fb((b & 0x807FFFFFu) | ((uint32_t)e << 23));
  const float r = e <= 0 ? 0.0f : (e >= 0xFF ? ov : in);
  return y == 0.0f ? y : r;
}

// exp (code/cis2-fp/src/math.rs:167-204; spec §6.2).  The main path runs
// on every lane, with 0 standing in for the special inputs (NaN, x > 88,
// x < -88) whose results are selected at the end: the same bits as
// returning early, without divergent branches in a loop over positions.
// On the main path |z0| < 128, where floor_f32 and sat_i32 reduce to the
// truncating conversion (and its correction) used here.
__device__ __forceinline__ float exp_pinned(float x) {
  x = daz(x);
  const bool nan = x != x, hi = x > 88.0f, lo = x < -88.0f;
  const float xr = (nan || hi || lo) ? 0.0f : x;
  float t = xr * fb(kExpLog2e);
  float z0 = t + 0.5f;
  const int32_t zi = (int32_t)z0;
  float k = (float)zi;
  if (z0 < k) k = k - 1.0f;
  float kc1 = k * fb(kExpC1);
  float r0 = xr - kc1;
  float kc2 = k * fb(kExpC2);
  float r = r0 - kc2;
  float r2 = r * r;
  float p = fb(kExpP0);
  float m;
  m = p * r; p = m + fb(kExpP1);
  m = p * r; p = m + fb(kExpP2);
  m = p * r; p = m + fb(kExpP3);
  m = p * r; p = m + fb(kExpP4);
  m = p * r; p = m + fb(kExpP5);
  float pr2 = p * r2;
  float s = pr2 + r;
  float y = s + 1.0f;
  float e = ldexp_bits(y, (int32_t)k);
  e = lo ? 0.0f : e;
  e = hi ? fb(0x7F800000u) : e;
  e = nan ? fb(kQNaN) : e;
  return e;
}

// Octant reduction in binary64 (code/cis2-fp/src/math.rs:248-264).
__device__ __forceinline__ float reduce_half_pi(float x, int64_t* k) {
  const double pio2 = __longlong_as_double((long long)kPio2F64);
  double xd = (double)x;
  double q = xd / pio2;
  double kd = round_away(q);
  double kp = kd * pio2;
  double rd = xd - kp;
  *k = sat_i64(kd);
  return (float)rd;
}
__device__ __forceinline__ float sin_kernel(float r) {
  float r2 = r * r;
  float a = fb(kSinC2);
  float m0 = a * r2;
  a = m0 + fb(kSinC1);
  float m1 = a * r2;
  a = m1 + fb(kSinC0);
  float r3 = r2 * r;
  float tail = a * r3;
  return r + tail;
}
__device__ __forceinline__ float cos_kernel(float r) {
  float r2 = r * r;
  float a = fb(kCosC2);
  float m0 = a * r2;
  a = m0 + fb(kCosC1);
  float m1 = a * r2;
  a = m1 + fb(kCosC0);
  float r4 = r2 * r2;
  float tail = a * r4;
  float h = 0.5f * r2;
  float lead = 1.0f - h;
  return lead + tail;
}
__device__ __forceinline__ int quadrant_of(int64_t k) { return (int)(((k % 4) + 4) % 4); }

// sin and cos (code/cis2-fp/src/math.rs:310-334; spec §6.3).
__device__ __forceinline__ void sincos_pinned(float x, float* s_out, float* c_out) {
  x = daz(x);
  uint32_t b = bf(x);
  if ((b & 0x7F800000u) == 0x7F800000u) {  // inf / NaN
    if (b & 0x007FFFFFu) { *s_out = *c_out = fb(b | 0x00400000u); return; }
    *s_out = (b >> 31) ? fb(kIndefinite) : fb(kQNaN);
    *c_out = fb(kIndefinite);
    return;
  }
  int64_t k;
  float r = reduce_half_pi(x, &k);
  float s = sin_kernel(r), c = cos_kernel(r);
  switch (quadrant_of(k)) {
    case 0: *s_out = s; *c_out = c; break;
    case 1: *s_out = c; *c_out = -s; break;
    case 2: *s_out = -s; *c_out = -c; break;
    default: *s_out = -c; *c_out = s; break;
  }
}
__device__ __forceinline__ float sin_pinned(float x) { float s, c; sincos_pinned(x, &s, &c); return s; }
__device__ __forceinline__ float cos_pinned(float x) { float s, c; sincos_pinned(x, &s, &c); return c; }

// ln (code/cis2-fp/src/math.rs:366-410; spec §6.5).
__device__ __forceinline__ float ln_pinned(float x) {
  x = daz(x);
  if (x != x || x < 0.0f) return fb(kQNaN);
  if (x == 0.0f) return fb(0xFF800000u);
  uint32_t b = bf(x);
  int32_t e = (int32_t)((b >> 23) & 0xFFu) - 126;
  float m = fb((b & 0x807FFFFFu) | (126u << 23));
  if (m < fb(kLogSqrtHf)) {
    e = e - 1;
    float mm = m + m;
    m = mm - 1.0f;
  } else {
    m = m - 1.0f;
  }
  float z = m * m;
  float p = fb(kLogP0);
  float t;
  t = p * m; p = t + fb(kLogP1);
  t = p * m; p = t + fb(kLogP2);
  t = p * m; p = t + fb(kLogP3);
  t = p * m; p = t + fb(kLogP4);
  t = p * m; p = t + fb(kLogP5);
  t = p * m; p = t + fb(kLogP6);
  t = p * m; p = t + fb(kLogP7);
  t = p * m; p = t + fb(kLogP8);
  float y = p * m;
  y = y * z;
  float fe = (float)e;
  float q1 = fe * fb(kLogQ1);
  y = y + q1;
  float hz = 0.5f * z;
  y = y - hz;
  float res = m + y;
  float q2 = fe * fb(kLogQ2);
  return res + q2;
}

// silu(x) = x / (1 + exp(-x)) (code/cis2-fp/src/math.rs:414-419).
__device__ __forceinline__ float silu_pinned(float x) {
  x = daz(x);
  uint32_t b = bf(x);
  if (is_nan_bits(b)) return fb(b | 0x00400000u);
  if (b == 0xFF800000u) return fb(kIndefinite);
  float nx = -x;
  float e = exp_pinned(nx);
  float d = 1.0f + e;
  return x / d;
}

// v0.4-candidate tree order for one 32-leaf block (code/cis2-fp/src/math.rs:
// 60-125): five in-place rounds leaf[i] = leaf[2i] + leaf[2i+1]; leaves past
// the data are +0.  The caller folds the block results left to right from 0.
__device__ __forceinline__ float tree32(float (&l)[32]) {
#pragma unroll
  for (int w = 32; w > 1; w >>= 1) {
#pragma unroll
    for (int i = 0; i < w / 2; ++i) l[i] = l[2 * i] + l[2 * i + 1];
  }
  return l[0];
}

// Cross-lane moves within a wave64 (DPP): row_shr:n inside 16-lane rows and
// the broadcasts of lane 15 / lane 31 into later rows; lanes without a
// source keep `old`.  A max (min) scan with shifts 1, 2, 4, 8 leaves each
// row's extreme in its lane 15, the two broadcasts carry them to lane 63.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t dpp_move(uint32_t old, uint32_t src) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)old, (int)src, CTRL, ROWMASK, 0xF, false);
}
template <int CTRL, int ROWMASK>
__device__ __forceinline__ float max_step(float x) {
  const uint32_t u = __float_as_uint(x);
  const float y = __uint_as_float(dpp_move<CTRL, ROWMASK>(u, u));
  return y > x ? y : x;
}
// Largest value over the wave (inputs NaN-free), in every lane.
__device__ __forceinline__ float wave_max(float x) {
  x = max_step<0x111, 0xF>(x);
  x = max_step<0x112, 0xF>(x);
  x = max_step<0x114, 0xF>(x);
  x = max_step<0x118, 0xF>(x);
  x = max_step<0x142, 0xA>(x);
  x = max_step<0x143, 0xC>(x);
  return __uint_as_float(__builtin_amdgcn_readlane(__float_as_uint(x), 63));
}

}  // namespace cis2
