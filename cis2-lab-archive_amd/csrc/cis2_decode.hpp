// cis2_decode.hpp — the persistent per-token decode kernel (one launch per
// position: all layers, the LM head and the greedy argmax).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cis2 {

// Device-side weight pointers of one layer (blocked GEMV layout, see
// cis2_kernels.hpp; biases / QK-norm weights may be null).
struct LayerW {
  const float *ln1, *ln2, *wq, *wk, *wv, *wo, *wg, *wu, *wd;
  const float *bq, *bk, *bv, *qn, *kn;
};

// Rows per GEMV row block for a reduction length K: the block (R x K
// floats) of one task fits the 144 KiB LDS weight budget, and R <= cap.
// The persistent kernel uses cap 32 where its roles fit the device (two
// k-groups per product instruction); the per-op kernels use cap 64.
inline uint32_t rows_per_block(uint32_t K, uint32_t cap = 64) {
  uint32_t r = 36864u / K;
  return r > cap ? cap : (r < 1 ? 1 : r);
}

constexpr uint32_t kDefaultSpinCap = 1u << 24;

struct DecodeArgs {
  const LayerW* layers;  // device array [L]
  const float* embed;    // row-major [V][H]
  const float* lm;       // blocked [V][H], Rl rows per block
  const float* fnorm;    // [H]
  const float* rope_cs;  // [max_pos][hd/2][2]
  float* kc0;            // this sequence's caches: layer l at kc0 + l*cache_stride
  float* vc0;
  float* act;            // per-layer activations as 64-bit {f32 bits, epoch} words (zeroed at start)
  uint32_t* cnt;         // [0]: LM-head ticket (blocks completed, all launches)
  float* logits;         // [V]
  uint32_t* cand;        // [nl][2] (value bits, index) per LM block
  uint32_t* tok_in;      // token of this position
  uint32_t* tok_out;     // argmax written here (may alias tok_in)
  uint32_t* err;
  // Sleeps a phase wait may take before it raises error bit 2 and gives up
  // (kDefaultSpinCap, about 0.5 s; a test can set a tiny cap to make the
  // waits give up while every workgroup still exits normally).
  uint32_t spin_cap;
  // Optional per-task timestamps (s_memrealtime, 100 MHz), null when off:
  // [(l * 6 + phase) * 64 + task] * 4 words: wait start, wait end, done,
  // and a mid-point (after RMSNorm for QKV/GU, after the GEMV for O/D,
  // after the softmax for ATT, the argmax reduction for LM).
  uint64_t* tline;
  uint64_t cache_stride;
  uint32_t H, I, V, L, nh, nkv, hd, qd, kvd, max_pos;
  uint32_t Rq, Ro, Rg, Rd, Rl;
  uint32_t nq_q, nq_k, nq;  // QKV tasks: q blocks, k blocks, total (q + k + v)
  uint32_t no, ng, nd, nl;  // O, gate/up, down, LM-head task counts
  // Tasks of each workgroup, in the order it runs them within a layer:
  // wg_tasks[wg * kMaxTasks + i] = phase << 12 | task (kNoTask ends a list).
  const uint16_t* wg_tasks;
  uint32_t nwg;
  float eps, scale;
  uint32_t pos, epoch, lm_epoch, want_logits;
  uint32_t tree;  // 1: v0.4-candidate tree reduction order, 0: sequential
  // Split attention (contexts whose K/V rows do not fit one workgroup's
  // LDS): the ATT phase runs natt_s = nkv * att_chunks score tasks (all
  // query heads of one kv head over att_cpos positions, a multiple of 64 in
  // [256, 512], K columns staged in LDS) and natt_v = nh * att_dvc mix
  // tasks (8 output dims of one query head each, att_dvc = hd / 8, V tiles
  // of att_tp positions in a ring of att_nr); scores pass through scw,
  // tagged words [L][nh][max_pos] (zeroed at start).
  uint32_t att_split, att_chunks, natt_s, att_dvc, natt_v, att_tp, att_cpos, att_nr;
  uint64_t* scw;
  // floats of the largest set of weight blocks one workgroup without an
  // attention task keeps in LDS (one slot per task; 0: none kept)
  uint32_t wslot;
};

// Floats (4-byte units) of one layer's tagged activation storage.
size_t decode_act_floats(uint32_t H, uint32_t I, uint32_t qd, uint32_t kvd);
constexpr uint32_t kTimelineTasks = 512;
constexpr uint32_t kMaxTasks = 6;       // tasks per workgroup per layer
constexpr uint16_t kNoTask = 0xFFFF;
// Phases of a layer, in dependency order.
enum { kPhaseQKV = 0, kPhaseATT = 1, kPhaseO = 2, kPhaseGU = 3, kPhaseD = 4, kPhases = 5 };
// Dynamic LDS bytes the kernel needs for this configuration.
size_t decode_lds_bytes(const DecodeArgs& a);
// True when attention fits the configuration: every cached position in LDS,
// or tiles of at least 32 positions beside the scores.
bool decode_att_ok(const DecodeArgs& a);
// Fills the split-attention fields of a (split: on or off) from its shape
// and LDS plan.
void decode_att_plan(DecodeArgs& a, bool split);
// True when one workgroup cannot hold a head's K/V rows at max_pos.
bool decode_att_needs_split(const DecodeArgs& a);
hipError_t launch_decode(const DecodeArgs& a, hipStream_t s);
// *ok: every one of the a.nwg workgroups can be resident at once on the
// current device (ncu CUs) with the kernel's LDS and registers.
hipError_t decode_coresident(const DecodeArgs& a, uint32_t ncu, bool* ok);

// Standalone strict-order GEMV y = W x on the blocked layout with R rows per
// block (R = 16 or 32): one workgroup per block, block and x staged in LDS.
size_t gemv_blk_lds_bytes(uint32_t K, uint32_t R);
hipError_t launch_gemv_blk(const float* W, const float* x, float* y, uint32_t M, uint32_t K,
                           uint32_t R, hipStream_t s);
// n independent GEMVs in one launch: y_i = W_c x_i, W_c the replica
// c = (first + i) % copies at W + c * w_per (blocked layout), x_i = x + i*K,
// y_i = y + i*M.
hipError_t launch_gemv_many(const float* W, uint64_t w_per, uint32_t copies, uint32_t first,
                            uint32_t n, const float* x, float* y, uint32_t M, uint32_t K,
                            uint32_t R, hipStream_t s);

}  // namespace cis2
