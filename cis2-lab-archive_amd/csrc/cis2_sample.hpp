// cis2_sample.hpp — launch interface of the seeded-sampling kernels
// (CIS-2 v0.4 draft section 14,
// code/patches/cis2-spec__seeded-sampling.patch:57-196).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <mutex>

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
// sets bit 0x100 of *err.  nkeep_out (optional, device) receives the size
// of the kept set.
hipError_t launch_sample(const float* logits, uint32_t V, const SampleParams& p, uint32_t step,
                         const SampleBufs& b, uint32_t* out, uint32_t* err, hipStream_t s,
                         uint32_t* nkeep_out = nullptr);

// ---- Preallocated per-GPU scratch for the no-allocation draw ----------------
// Largest vocabulary the static scratch serves (Qwen3's 151,936 fits), and
// its size: two key arrays of the sort length, the f32 terms, the candidates
// and two flag words.
constexpr uint32_t kNoAllocMaxVocab = 262144;
constexpr size_t kNoAllocScratchBytes =
    (2 * (size_t)kNoAllocMaxVocab + kNoAllocMaxVocab / 2 + kSampleBlocks + 8) * 8;
// Resolves the current GPU's copy of the scratch array (once per device,
// with that device current).  Called at context creation.
hipError_t sample_scratch_init();
// The lock a draw holds from clearing the error flag until its results are
// back, so that draws from several host threads on one GPU take turns with
// the shared scratch (null for a device index out of range).
std::mutex* sample_scratch_lock(int dev);
// The sampler buffers and the error-flag word carved out of GPU dev's
// scratch for a vocabulary of V (<= kNoAllocMaxVocab).  No allocation.
hipError_t sample_scratch_bufs(int dev, uint32_t V, SampleBufs* b, uint32_t** err);
// p[0..n) = v on stream s (a kernel, not a memset node).
hipError_t launch_fill_u32(uint32_t* p, uint32_t n, uint32_t v, hipStream_t s);

}  // namespace cis2
