/* cis2_synth.h — deterministic synthetic artifacts for the CIS-2 workloads.
 *
 * Real checkpoints cannot be fetched here, so every workload runs on seeded
 * random weights that any machine regenerates bit for bit:
 *   stream(seed, ordinal): splitmix64 outputs z_i = mix64(s0 + (i+1)*gamma)
 *     with s0 = mix64(seed ^ mix64(ordinal + 0x632BE59BD9B4E019)).
 *   weight i: S = sum of the four 16-bit fields of z_i (Irwin-Hall, n=4),
 *     v = (S - 131070) * (sigma / sqrt(4*(65536^2-1)/12))  in binary64,
 *     rounded once to binary32, then to BF16 by round-to-nearest-even on the
 *     bit pattern.  Every step is an IEEE-exact or correctly rounded
 *     operation, so the bits do not depend on the host.
 *   uniform integer in [lo, hi]: lo + ((z >> 32) * (hi - lo + 1)) >> 32.
 */
#ifndef CIS2_SYNTH_H
#define CIS2_SYNTH_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

uint64_t cis2_synth_mix64(uint64_t z);
/* n BF16 weights of tensor `ordinal` (N(0, sigma)-shaped). */
void cis2_synth_bf16(uint64_t seed, uint64_t ordinal, double sigma, uint16_t *out, uint64_t n);
/* n integers uniform in [lo, hi] from stream (seed, ordinal). */
void cis2_synth_uniform(uint64_t seed, uint64_t ordinal, uint32_t lo, uint32_t hi,
                        uint32_t *out, uint64_t n);
/* n float32 values N(0, sigma)-shaped (same transform, no BF16 rounding). */
void cis2_synth_f32(uint64_t seed, uint64_t ordinal, double sigma, float *out, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
