// cis2_rows.hpp — the forward pass over a set of rows at once.  A row is one
// (sequence, position, token) triple; a layer runs every op for all rows
// before the next op, so a batch of sequences (one row each) and the
// teacher-forced prefill of one sequence (one row per position, causal
// through the KV cache) share one code path.  Every output is the same
// per-row computation as the single-row kernels, in the same order, so each
// row is bit-identical to its single-row run.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cis2 {

// Y[b][m] = X[b][:] . W[m][:] for b < n, m < M, one strict chain per output
// (or tree32 blocks when tree), with an epilogue:
//   kEpiNone:     Y = acc
//   kEpiBias:     Y = acc + add[m]             (q/k/v bias, main.rs:265-272)
//   kEpiResidual: Y = add[b * ldadd + m] + acc (h + o, h + down, main.rs:274-280)
// W is the blocked layout of cis2_kernels.hpp with R rows per block.
enum { kEpiNone = 0, kEpiBias = 1, kEpiResidual = 2 };
struct BgemmSeg {
  const float* W;
  uint32_t M, K, R;
  const float* X;  // row b at X + b * ldx
  uint32_t ldx;
  float* Y;        // row b at Y + b * ldy
  uint32_t ldy;
  const float* add;
  uint32_t ldadd, epi;
};
hipError_t launch_bgemm(const BgemmSeg& s, uint32_t n, bool tree, hipStream_t st);

// Options of a multi-matrix launch.
struct BgemmOpts {
  // RMSNorm weight (main.rs:245-260): each X row is normalised first,
  // inv = 1/sqrt(sum of squares / K + eps), x' = (x*inv)*w[k]
  const float* norm_w = nullptr;
  float eps = 0.0f;
  // second matrix of segs[0]'s shape and layout (one segment only):
  // Y = silu(X.W) * (X.W2), the gated MLP's hidden row (main.rs:484-487)
  const float* W2 = nullptr;
  bool tree = false;
};
// Up to three matrices over the same X rows (same K, R, X, ldx) in one
// launch, each with its own M, Y and epilogue.
hipError_t launch_bgemm_multi(const BgemmSeg* segs, uint32_t nseg, uint32_t n,
                              const BgemmOpts& o, hipStream_t st);

// Per-row device descriptors: seq[r], pos[r], tok[r].
struct RowsDesc {
  const uint32_t* seq;
  const uint32_t* pos;
  const uint32_t* tok;
  uint32_t n;
};

// h[r] = E[tok[r]] (token range checked on the device: err |= 1, row 0 used).
hipError_t launch_embed_rows(const float* E, RowsDesc rows, uint32_t H, uint32_t vocab,
                             float* h, uint32_t* err, hipStream_t st);
// RoPE of row r's q (nh heads) and k (nkv heads) at pos[r] in place, then
// the rotated k and the raw v into sequence seq[r]'s layer caches at pos[r].
// Caches of sequence s: K at kc + s * seq_stride, V at vc + s * seq_stride,
// both [kvh][hd][max_pos].
hipError_t launch_rope_store_rows(float* q, float* k, const float* v, const float* rope_cs,
                                  RowsDesc rows, uint32_t nh, uint32_t nkv, uint32_t hd,
                                  uint32_t max_pos, float* kc, float* vc, uint64_t seq_stride,
                                  hipStream_t st);
// Attention of every (row, query head) over positions 0..pos[r] of the
// row's sequence; out [n][nh*hd].  max_len: the largest pos[r] + 1.
hipError_t launch_attention_rows(const float* q, const float* kc, const float* vc,
                                 RowsDesc rows, uint32_t max_len, uint32_t nh, uint32_t nkv,
                                 uint32_t hd, uint32_t max_pos, uint64_t seq_stride, float scale,
                                 float* out, bool tree, hipStream_t st);
// Rows of distinct sequences (decode steps): launch_rope_store_rows and
// launch_attention_rows in one launch, with the same bits and the same cache
// writes, when the shape takes the one-workgroup-per-(row, KV head)
// attention (head_dim 64 or 128, rows x kv heads < 4 x CUs);
// hipErrorNotSupported otherwise, with nothing launched.  q, k and v are
// the rows' un-rotated projections (q and k are not rotated in place).
hipError_t launch_rope_attention_rows(const float* q, const float* k, const float* v,
                                      const float* rope_cs, RowsDesc rows, uint32_t max_len,
                                      uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_pos,
                                      float* kc, float* vc, uint64_t seq_stride, float scale,
                                      float* out, bool tree, hipStream_t st);
// Prefill attention in tiles: rows row0 .. row0+nr-1 (nr <= 16) are rows of
// sequence seq at positions p0 .. p0+nr-1; each tile's rows get the same
// bits as launch_attention_rows gives them (sequential order only), with
// each K and V element read once per tile and KV head.  Shapes: head_dim
// 64 with 1..4 query heads per KV head, head_dim 128 with 2 or 4.
// scratch: attention_tiles_scratch_floats(ntiles, nh, nkv, max_len) floats.
struct AttTile {
  uint32_t row0, nr, seq, p0;
};
constexpr uint32_t kAttTileRows = 16;
bool attention_tiles_supported(uint32_t nh, uint32_t nkv, uint32_t hd);
size_t attention_tiles_scratch_floats(uint32_t ntiles, uint32_t nh, uint32_t nkv,
                                      uint32_t max_len);
hipError_t launch_attention_tiles(const float* q, const float* kc, const float* vc,
                                  const AttTile* tiles, uint32_t ntiles, uint32_t max_len,
                                  uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_pos,
                                  uint64_t seq_stride, float scale, float* out, float* scratch,
                                  hipStream_t st);
// dst[i] = src[idx[i]] rows of `width` floats, i < n.
hipError_t launch_gather_rows(const float* src, const uint32_t* idx, uint32_t n, uint32_t width,
                              float* dst, hipStream_t st);
// pos[i] += 1 for i < n (the next decode step's positions, on the device).
hipError_t launch_advance_rows(uint32_t* pos, uint32_t n, hipStream_t st);
// Greedy argmax of each of n rows of v (stride `width`): strict >, first
// maximum wins, NaN at index 0 wins.
hipError_t launch_argmax_rows(const float* v, uint32_t n, uint32_t width, uint32_t* out,
                              hipStream_t st);

}  // namespace cis2
