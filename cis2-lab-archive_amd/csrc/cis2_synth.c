/* cis2_synth.c — deterministic synthetic weights and token ids (see
 * cis2_synth.h for the exact definition). */
#include "cis2_synth.h"

#include <math.h>
#include <string.h>

#define GAMMA 0x9E3779B97F4A7C15ull

uint64_t cis2_synth_mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static uint64_t stream_base(uint64_t seed, uint64_t ordinal) {
  return cis2_synth_mix64(seed ^ cis2_synth_mix64(ordinal + 0x632BE59BD9B4E019ull));
}

static double unit_scale(double sigma) {
  /* sd of the sum of four uniform 16-bit integers */
  double var = 4.0 * (65536.0 * 65536.0 - 1.0) / 12.0;
  return sigma / sqrt(var);
}

static inline double draw(uint64_t s0, uint64_t i, double scale) {
  uint64_t z = cis2_synth_mix64(s0 + (i + 1) * GAMMA);
  int64_t s = (int64_t)(z & 0xFFFFu) + (int64_t)((z >> 16) & 0xFFFFu) +
              (int64_t)((z >> 32) & 0xFFFFu) + (int64_t)(z >> 48);
  return (double)(s - 131070) * scale;
}

void cis2_synth_f32(uint64_t seed, uint64_t ordinal, double sigma, float *out, uint64_t n) {
  uint64_t s0 = stream_base(seed, ordinal);
  double scale = unit_scale(sigma);
  for (uint64_t i = 0; i < n; ++i) out[i] = (float)draw(s0, i, scale);
}

void cis2_synth_bf16(uint64_t seed, uint64_t ordinal, double sigma, uint16_t *out, uint64_t n) {
  uint64_t s0 = stream_base(seed, ordinal);
  double scale = unit_scale(sigma);
  for (uint64_t i = 0; i < n; ++i) {
    float f = (float)draw(s0, i, scale);
    uint32_t b;
    memcpy(&b, &f, 4);
    b = b + 0x7FFFu + ((b >> 16) & 1u); /* RNE to the upper 16 bits (finite inputs) */
    out[i] = (uint16_t)(b >> 16);
  }
}

void cis2_synth_uniform(uint64_t seed, uint64_t ordinal, uint32_t lo, uint32_t hi,
                        uint32_t *out, uint64_t n) {
  uint64_t s0 = stream_base(seed, ordinal);
  uint64_t span = (uint64_t)hi - lo + 1;
  for (uint64_t i = 0; i < n; ++i) {
    uint64_t z = cis2_synth_mix64(s0 + (i + 1) * GAMMA);
    out[i] = lo + (uint32_t)(((z >> 32) * span) >> 32);
  }
}
