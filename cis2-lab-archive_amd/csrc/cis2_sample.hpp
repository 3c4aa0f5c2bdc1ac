// cis2_sample.hpp — launch interface of the seeded-sampling kernels
// (CIS-2 v0.4 draft section 14,
// code/patches/cis2-spec__seeded-sampling.patch:57-196).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cis2 {

struct SampleParams {
  uint64_t seed;
  float temperature;  // finite, > 0
  uint32_t top_k;     // 0 or >= V: disabled
  float top_p;        // (0, 1]; 1: disabled
};

// Device scratch of one sampler (sized for a vocabulary of V).
struct SampleBufs {
  uint32_t V = 0, Vp = 0;      // vocabulary, sort length (power of two >= V, >= tile)
  uint64_t* key = nullptr;     // [Vp] rank keys, sorted in place
  uint64_t* key2 = nullptr;    // [Vp] top-k candidates
  float* e = nullptr;          // [V] exp terms / probabilities in rank order
  uint64_t* cand = nullptr;    // [kSampleBlocks] per-workgroup (z, index) candidates
  uint32_t* nkeep = nullptr;   // [1] size of the kept set
};
constexpr uint32_t kSampleBlocks = 256;

// Sort length for a vocabulary of V entries.
uint32_t sample_sort_len(uint32_t V);

// Draws the next id from logits[V] at generation step `step` into *out on
// stream s (no host synchronisation).  A NaN among logits / temperature
// sets bit 0x100 of *err.  nkeep_host (optional) is not written here: read
// b.nkeep after the stream drains.
hipError_t launch_sample(const float* logits, uint32_t V, const SampleParams& p, uint32_t step,
                         const SampleBufs& b, uint32_t* out, uint32_t* err, hipStream_t s);

}  // namespace cis2
