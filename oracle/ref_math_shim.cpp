// oracle/ref_math_shim.cpp — exposes the reference's own pinned math
// (code/cis2-fp/gpu/cis2_math.h, compiled from where it lies in the archive)
// through a C ABI, so the repository's oracle can be compared against it
// exhaustively.  TEST INFRASTRUCTURE ONLY; built into oracle/_ref/ and
// never shipped.
#include "cis2_math.h"

#include <emmintrin.h>
#include <pthread.h>
#include <stdint.h>
#include <string.h>

namespace {
void pin_mxcsr() { _mm_setcsr(_mm_getcsr() | (1u << 15) | (1u << 6)); }

float apply(int fn, float x) {
  switch (fn) {
    case 0: return cis2_exp_pinned(x);
    case 1: return cis2_sin_pinned(x);
    case 2: return cis2_cos_pinned(x);
    case 3: return cis2_ln_pinned(x);
    case 4: return cis2_silu_pinned(x);
    case 5: return cis2_rsqrt_cr(x);
    default: return cis2_sqrt_f32(x);
  }
}

uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
}  // namespace

extern "C" {

void ref_math_map(int fn, const float *in, float *out, size_t n) {
  pin_mxcsr();
  for (size_t i = 0; i < n; ++i) out[i] = apply(fn, in[i]);
}

// Same order-free chunk hash as the oracle's orc_math_chunk_hash.
uint64_t ref_math_chunk_hash(int fn, uint32_t first, uint32_t count) {
  pin_mxcsr();
  uint64_t h = 0;
  for (uint32_t j = 0; j < count; ++j) {
    uint32_t bits = first + j;
    float x, y;
    memcpy(&x, &bits, 4);
    y = apply(fn, x);
    uint32_t ob;
    memcpy(&ob, &y, 4);
    h += mix64((uint64_t)ob ^ ((uint64_t)bits * 0x9E3779B97F4A7C15ull));
  }
  return h;
}

float ref_dot_seq(const float *a, const float *b, int n) {
  pin_mxcsr();
  return cis2_dot_seq(a, b, n);
}
float ref_dot_tree(const float *a, const float *b, int n) {
  pin_mxcsr();
  return cis2_tree_dot(a, b, n);
}
float ref_sum_tree(const float *a, int n) {
  pin_mxcsr();
  return cis2_tree_sum(a, n);
}
void ref_softmax(float *v, int n, int tree) {
  pin_mxcsr();
  if (tree) cis2_softmax_tree(v, n); else cis2_softmax_seq(v, n);
}
}
