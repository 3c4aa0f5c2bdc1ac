// cis2_kernels.hpp — launch interface of the gfx950 kernels of the CIS-2
// forward pass.  Device buffers only; shapes are validated by the caller
// (cis2_runtime.hip) before any launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cis2 {

// GEMV weight layout in HBM ("row-block interleaved"): rows are grouped in
// blocks of R <= 64 (one row per lane of a wavefront); inside a block the
// matrix is stored k-group-major with 4 consecutive k per lane, so a
// wave-wide 16-byte load per lane reads R*16 contiguous bytes and a block is
// one contiguous R*K run (what a workgroup copies into its LDS):
//   W_blk[((b * (K/4) + g) * R + lane) * 4 + j] = W[b*R + lane][4*g + j]
// Rows past M in the last block are zero.  K must be a multiple of 4.
size_t blocked_floats(uint32_t M, uint32_t K, uint32_t R);

// Raises kernel fn's dynamic-LDS limit to at least `bytes` on the current
// device.  Each (device, kernel) is configured once per size: a process-wide
// table under a lock, so contexts on different devices or host threads each
// see their own device's setting.
hipError_t ensure_dynamic_lds(const void* fn, size_t bytes);
// Compute units of the current device (cached per device, thread-safe).
int device_cu_count();

// One output segment of a multi-segment GEMV launch.
struct GemvSeg {
  const float* W;      // blocked weights
  const float* x;      // input vector [K]
  const float* add;    // optional: y = add + W x (residual) or W x + add (bias)
  float* y;            // output [M]
  uint32_t M, K;
  uint32_t add_first;  // 1: y = add[i] + acc (residual); 0: y = acc + add[i] (bias)
  uint32_t R;          // rows per block of W's layout (1..64)
};

// Per-row GEMV over up to 4 segments in one launch: strict left-to-right
// products, or (tree) 32-product blocks by tree32 folded left to right.
// The RMSNorm sum and the attention scores / softmax denominator take the
// same `tree` switch; the V mix is sequential in both orders.
hipError_t launch_gemv(const GemvSeg* segs, int nseg, hipStream_t s, bool tree = false);
// Gate/up pair fused with hid = silu(gate) * up.
hipError_t launch_gate_up_silu(const float* Wg, const float* Wu, const float* x,
                               float* gate, float* up, float* hid, uint32_t I,
                               uint32_t H, uint32_t R, hipStream_t s, bool tree = false);
// Relayout a row-major [M,K] f32 matrix (device) into the blocked layout.
hipError_t launch_relayout(const float* src, float* dst, uint32_t M, uint32_t K, uint32_t R,
                           hipStream_t s);
// Exact BF16 -> F32 widening (bits << 16).
hipError_t launch_widen(const uint16_t* src, float* dst, uint64_t n, hipStream_t s);

// h = embed[tok] (tok read from device memory).
hipError_t launch_embed(const float* E, const uint32_t* tok, float* h, uint32_t H,
                        uint32_t vocab, uint32_t* err, hipStream_t s);
// out = RMSNorm(x) * w over n elements; `nvec` independent vectors of
// length n at stride n (the per-head QK-norm uses nvec = heads).
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, uint32_t n,
                          uint32_t nvec, float* out, hipStream_t s, bool tree = false);
// RoPE on q (nh heads) and k (nkv heads) in place from the per-position
// table, then store rotated k and raw v into the caches at pos.
// Caches: K and V both as [kvh][hd][max_pos] (one row per head dimension).
hipError_t launch_rope_store(float* q, float* k, const float* v, const float* rope_cs,
                             uint32_t pos, uint32_t nh, uint32_t nkv, uint32_t hd,
                             uint32_t max_pos, float* kc, float* vc, hipStream_t s);
// Attention per query head: scores (dot * scale), softmax, V mix.
// If scores_out/probs_out are non-null they receive [nh][pos+1].
hipError_t launch_attention(const float* q, const float* kc, const float* vc,
                            uint32_t pos, uint32_t nh, uint32_t nkv, uint32_t hd,
                            uint32_t max_pos, float scale, float* att_out,
                            float* scores_out, float* probs_out, hipStream_t s,
                            bool tree = false);
// Greedy argmax (strict >, first maximum wins) -> *tok_out.
hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t* tok_out,
                         hipStream_t s);
// inv_freq[i] and the per-position cos/sin table [max_pos][hd/2][2].
hipError_t launch_rope_table(float theta_f32, uint32_t hd, uint32_t max_pos,
                             float* inv_freq, float* rope_cs, hipStream_t s);
// Device FTZ/DAZ probes: out[0] = bits(2^-126 * 1e-10), out[1] = bits(denorm + 0).
hipError_t launch_fpenv_probe(uint32_t* out, hipStream_t s);
// Wait-counter capacity probes (verification): bad[0] = wrong registers after
// 128 vector loads and one vmcnt(0) wait, bad[1] = wrong words after 40 LDS
// reads and one lgkmcnt(0) wait (both 0 on hardware that holds issue at the
// counters' maxima).
hipError_t run_wait_probes(uint32_t bad[2]);
// Exhaustive-sweep helper: per-chunk order-free hash of fn over the input
// bit patterns [first, first + count).
hipError_t launch_math_hash(int fn, uint32_t first, uint32_t count,
                            unsigned long long* hash_out, hipStream_t s);
hipError_t launch_math_map(int fn, const float* in, float* out, uint64_t n,
                           hipStream_t s);
hipError_t launch_div_map(const float* a, const float* b, float* out, uint64_t n,
                          hipStream_t s);

}  // namespace cis2
