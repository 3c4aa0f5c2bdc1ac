// cis2_rows.hip — gfx950 kernels of the row-batched forward pass (several
// sequences per step, or every position of one sequence).  Each output is
// computed by one lane in the order the single-row kernels use
// (code/cis2-fp/src/main.rs:355-529), so a row's results do not depend on
// which other rows share the launch (batch invariance).
#include "cis2_device_math.hpp"
#include "cis2_rows.hpp"
#include "cis2_kernels.hpp"

#include <algorithm>
#include <type_traits>
#include <cstdlib>

namespace cis2 {
namespace {

// 16-byte vector as a native vector type: local arrays of it stay in
// registers (the struct-based float4 keeps them in scratch memory).
typedef float v4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kT = 256;
// Query heads per attention workgroup at most (those of one KV head).
constexpr uint32_t kMaxHeadsPerWg = 4;
// Threads per attention workgroup.
constexpr uint32_t kAttT = 256;

#define AS_LDS __attribute__((address_space(3)))
#define AS_GLB __attribute__((address_space(1)))

// 16 bytes from global memory straight into LDS (global_load_lds_dwordx4).
// The LDS address is dst_wave + 16 * lane, with dst_wave uniform across the
// wave: lanes that take part fill consecutive slots.  The data is in LDS
// once vmcnt reaches 0, and visible to other waves after a barrier.
__device__ __forceinline__ void lds_load16(const v4* src, v4* dst_wave) {
  __builtin_amdgcn_global_load_lds((const AS_GLB void*)src, (AS_LDS void*)dst_wave, 16, 0, 0);
}
// s_waitcnt vmcnt(0) (expcnt, lgkmcnt fields at their maxima: no wait).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Lane k of this lane's 16-lane row (DPP row_newbcast:k).
template <uint32_t K>
__device__ __forceinline__ float bcast16(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + (int)K, 0xF, 0xF, false));
}
// LDS per batched-GEMM workgroup: two workgroups fit one CU; small grids
// may use one workgroup's worth of almost all of it.
constexpr uint32_t kBgemmLds = 78 * 1024;
constexpr uint32_t kBgemmLdsBig = 150 * 1024;

// ---------------------------------------------------------------------------
// Batched GEMM.  A workgroup owns one R-row block of W and TB = 256 / R batch
// rows: thread t computes output (row b0 + t / R, column blk * R + t % R).
// K runs in chunks of KC: the block's [KC/4][R] v4 slice (contiguous in
// the blocked layout) and the TB input rows' KC floats are staged in LDS,
// then each thread continues its own chain acc = acc + W[m][k] * X[b][k],
// k ascending (code/cis2-fp/src/main.rs:228-243, math.rs:40-48); in tree
// mode the chain adds one tree32 block result per 32 k (math.rs:60-125).
//
// One launch may cover up to three matrices that read the same X (q, k and
// v): the grid's x blocks run over the segments in turn.  DUAL computes two
// chains per thread over W and W2 (gate and up) and stores
// silu(gate) * up (main.rs:484-487).  NORM applies the RMSNorm of each X row
// first (main.rs:245-260): the row's squares are summed in one strict chain
// (or tree32 blocks) from 0 over the row as staged in LDS (a first pass over
// the chunks when the row spans several), inv = 1/sqrt(sum/K + eps), and
// each staged element becomes (x*inv)*w[k].
// ---------------------------------------------------------------------------
constexpr uint32_t kMaxSegs = 3;
struct BgemmArgs {
  BgemmSeg s[kMaxSegs];
  uint32_t blk0[kMaxSegs + 1];  // first x block of each segment; blk0[nseg] = grid.x
  uint32_t nseg, n, TB, KC, tree;
  const float* W2;  // DUAL
  const float* nw;  // NORM
  float eps;
};

// Sum of squares of q4 16-byte groups, continuing the strict chain acc (or
// adding one tree32 per 8 groups, the last block zero-padded), read from
// LDS or global memory.
__device__ __forceinline__ float sumsq_groups(const v4* x4, uint32_t q4, float acc, bool tree) {
  if (tree) {
    for (uint32_t q0 = 0; q0 < q4; q0 += 8) {
      float l[32];
#pragma unroll
      for (uint32_t i = 0; i < 8; ++i) {
        const v4 v = q0 + i < q4 ? x4[q0 + i] : v4{0.0f, 0.0f, 0.0f, 0.0f};
        l[4 * i] = v.x * v.x;
        l[4 * i + 1] = v.y * v.y;
        l[4 * i + 2] = v.z * v.z;
        l[4 * i + 3] = v.w * v.w;
      }
      acc = acc + tree32(l);
    }
  } else {
#pragma unroll 8
    for (uint32_t q = 0; q < q4; ++q) {
      const v4 v = x4[q];
      float sq;
      sq = v.x * v.x; acc = acc + sq;
      sq = v.y * v.y; acc = acc + sq;
      sq = v.z * v.z; acc = acc + sq;
      sq = v.w * v.w; acc = acc + sq;
    }
  }
  return acc;
}
// RMSNorm factor from a row's sum of squares over K elements.
__device__ __forceinline__ float inv_rms_of(float sumsq, uint32_t K, float eps) {
  const float mean = sumsq / (float)K;
  const float arg = mean + eps;
  return rsqrt_cr(arg);
}

template <bool DUAL, bool NORM, uint32_t CB>
__global__ __launch_bounds__(256) void k_bgemm(BgemmArgs a) {
  extern __shared__ v4 sm[];
  __shared__ float s_inv[kT];
  uint32_t si = 0;
  if (a.nseg > 1 && blockIdx.x >= a.blk0[1]) si = (a.nseg > 2 && blockIdx.x >= a.blk0[2]) ? 2 : 1;
  const BgemmSeg g = si == 0 ? a.s[0] : (si == 1 ? a.s[1] : a.s[2]);
  const uint32_t R = g.R, TB = a.TB, KC = a.KC, K = g.K, NB = TB * CB;  // NB batch rows staged
  const uint32_t blk = blockIdx.x - a.blk0[si], b0 = blockIdx.y * NB, t = threadIdx.x;
  const uint32_t r = t % R, bb = t / R;  // the thread's rows: b0 + bb + c * TB, c < CB
  const uint32_t wv = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const bool live = t < R * TB;
  const uint32_t qmax = KC / 4, xs4 = qmax + 1;  // padded X rows: no bank aliasing
  v4* Ws = sm;                                   // [q4][R] (DUAL: then W2's at Ws + qmax * R)
  v4* Xs = sm + (size_t)(DUAL ? 2 : 1) * qmax * R;
  v4* NWs = Xs + (size_t)NB * xs4;               // NORM: the chunk's norm weights
  const v4* Wg = reinterpret_cast<const v4*>(g.W + (size_t)blk * R * K);
  const v4* Wg2 = DUAL ? reinterpret_cast<const v4*>(a.W2 + (size_t)blk * R * K) : nullptr;
  float acc[CB], acc2[CB];
#pragma unroll
  for (uint32_t c = 0; c < CB; ++c) acc[c] = acc2[c] = 0.0f;
  // the chunk's X rows (and norm weights), every load in flight at once,
  // straight into LDS; each wave instruction fills 64 consecutive 16-byte
  // slots
  auto stage_x = [&](uint32_t g0, uint32_t q4, bool with_nw) {
    const uint32_t pieces = (q4 + 63) / 64, nx = NB * pieces;
    // workgroups start at different rows: the grid's requests for the
    // shared X rows spread over the cache channels
    const uint32_t rot = (blockIdx.x * 5) % nx;
    for (uint32_t j0 = wv; j0 < nx; j0 += kT / 64) {
      const uint32_t j = j0 + rot < nx ? j0 + rot : j0 + rot - nx;
      const uint32_t bx = j / pieces, q0 = (j - bx * pieces) * 64;
      const uint32_t row = std::min(b0 + bx, a.n - 1);
      const v4* xr = reinterpret_cast<const v4*>(g.X + (size_t)row * g.ldx) + g0 + q0;
      if (q0 + lane < q4) lds_load16(xr + lane, Xs + bx * xs4 + q0);
    }
    if (NORM && with_nw) {
      const v4* nw4p = reinterpret_cast<const v4*>(a.nw) + g0;
      for (uint32_t i0 = wv * 64; i0 < q4; i0 += kT)
        if (i0 + lane < q4) lds_load16(nw4p + i0 + lane, NWs + i0);
    }
  };
  // RMSNorm of the staged rows: one lane per batch row continues its
  // sum-of-squares chain over each chunk from LDS.  Rows longer than one
  // chunk take a first pass over their chunks before the GEMM's.
  float ssq = 0.0f;
  if (NORM && K > KC) {
    for (uint32_t k0 = 0; k0 < K; k0 += KC) {
      const uint32_t q4 = std::min(KC, K - k0) / 4;
      stage_x(k0 / 4, q4, false);
      wait_vm0();
      __syncthreads();
      if (t < NB) ssq = sumsq_groups(Xs + t * xs4, q4, ssq, a.tree);
      __syncthreads();
    }
    if (t < NB) s_inv[t] = inv_rms_of(ssq, K, a.eps);
  }
  for (uint32_t k0 = 0; k0 < K; k0 += KC) {
    const uint32_t q4 = std::min(KC, K - k0) / 4, g0 = k0 / 4;
    const uint32_t nw4 = q4 * R;
    for (uint32_t i0 = wv * 64; i0 < nw4; i0 += kT)
      if (i0 + lane < nw4) lds_load16(Wg + (size_t)g0 * R + i0 + lane, Ws + i0);
    if (DUAL) {
      for (uint32_t i0 = wv * 64; i0 < nw4; i0 += kT)
        if (i0 + lane < nw4) lds_load16(Wg2 + (size_t)g0 * R + i0 + lane, Ws + qmax * R + i0);
    }
    stage_x(g0, q4, true);
    wait_vm0();
    __syncthreads();
    if (NORM) {
      if (K <= KC) {
        if (t < NB) s_inv[t] = inv_rms_of(sumsq_groups(Xs + t * xs4, q4, 0.0f, a.tree), K, a.eps);
        __syncthreads();
      }
      for (uint32_t i = t; i < NB * q4; i += kT) {
        const uint32_t bx = i / q4, q = i - bx * q4;
        const float inv = s_inv[bx];
        const v4 x = Xs[bx * xs4 + q], w = NWs[q];
        v4 y;
        float sx;
        sx = x.x * inv; y.x = sx * w.x;
        sx = x.y * inv; y.y = sx * w.y;
        sx = x.z * inv; y.z = sx * w.z;
        sx = x.w * inv; y.w = sx * w.w;
        Xs[bx * xs4 + q] = y;
      }
      __syncthreads();
    }
    if (live) {
      const v4* wp = Ws + r;
      const v4* wp2 = Ws + qmax * R + r;
      const v4* xp[CB];
#pragma unroll
      for (uint32_t c = 0; c < CB; ++c) xp[c] = Xs + (bb + c * TB) * xs4;
      if (a.tree) {
        for (uint32_t q = 0; q < q4; q += 8) {
#pragma unroll
          for (uint32_t c = 0; c < CB; ++c) {
            float l[32], l2[32];
#pragma unroll
            for (uint32_t j = 0; j < 8; ++j) {
              v4 w = v4{0.0f, 0.0f, 0.0f, 0.0f}, x = w, w2 = w;
              if (q + j < q4) {
                w = wp[(size_t)(q + j) * R];
                x = xp[c][q + j];
                if (DUAL) w2 = wp2[(size_t)(q + j) * R];
              }
              l[4 * j] = w.x * x.x;
              l[4 * j + 1] = w.y * x.y;
              l[4 * j + 2] = w.z * x.z;
              l[4 * j + 3] = w.w * x.w;
              if (DUAL) {
                l2[4 * j] = w2.x * x.x;
                l2[4 * j + 1] = w2.y * x.y;
                l2[4 * j + 2] = w2.z * x.z;
                l2[4 * j + 3] = w2.w * x.w;
              }
            }
            acc[c] = acc[c] + tree32(l);
            if (DUAL) acc2[c] = acc2[c] + tree32(l2);
          }
        }
      } else {
        // software pipelined over two register sets: the reads of the next
        // 4 q go out before the current 4 q's products and chain steps
        // (reads past the end are clamped to the last q and unused); a W
        // group read serves the CB rows' chains
        constexpr uint32_t U = 4;
        v4 aw[U], ax[CB][U], aw2[U], bw[U], bx[CB][U], bw2[U];
        auto load = [&](v4 (&w)[U], v4 (&x)[CB][U], v4 (&w2)[U], uint32_t q0) {
#pragma unroll
          for (uint32_t u = 0; u < U; ++u) {
            const uint32_t qq = std::min(q0 + u, q4 - 1);
            w[u] = wp[(size_t)qq * R];
#pragma unroll
            for (uint32_t c = 0; c < CB; ++c) x[c][u] = xp[c][qq];
            if (DUAL) w2[u] = wp2[(size_t)qq * R];
          }
        };
        auto step = [&](const v4 (&w)[U], const v4 (&x)[CB][U], const v4 (&w2)[U]) {
#pragma unroll
          for (uint32_t c = 0; c < CB; ++c) {
            float p[4 * U], p2[4 * U];
#pragma unroll
            for (uint32_t u = 0; u < U; ++u) {
              p[4 * u] = w[u].x * x[c][u].x;
              p[4 * u + 1] = w[u].y * x[c][u].y;
              p[4 * u + 2] = w[u].z * x[c][u].z;
              p[4 * u + 3] = w[u].w * x[c][u].w;
              if (DUAL) {
                p2[4 * u] = w2[u].x * x[c][u].x;
                p2[4 * u + 1] = w2[u].y * x[c][u].y;
                p2[4 * u + 2] = w2[u].z * x[c][u].z;
                p2[4 * u + 3] = w2[u].w * x[c][u].w;
              }
            }
#pragma unroll
            for (uint32_t i = 0; i < 4 * U; ++i) {
              acc[c] = acc[c] + p[i];
              if (DUAL) acc2[c] = acc2[c] + p2[i];
            }
          }
        };
        uint32_t q = 0;
        if (q4 >= U) {
          load(aw, ax, aw2, 0);
          for (; q + 2 * U <= q4; q += 2 * U) {
            load(bw, bx, bw2, q + U);
            step(aw, ax, aw2);
            load(aw, ax, aw2, q + 2 * U);
            step(bw, bx, bw2);
          }
          if (q + U <= q4) {  // set a holds q .. q+U-1
            step(aw, ax, aw2);
            q += U;
          }
        }
        for (; q < q4; ++q) {
          const v4 w = wp[(size_t)q * R];
          const v4 w2 = DUAL ? wp2[(size_t)q * R] : w;
#pragma unroll
          for (uint32_t c = 0; c < CB; ++c) {
            const v4 x = xp[c][q];
            float pp;
            pp = w.x * x.x; acc[c] = acc[c] + pp;
            pp = w.y * x.y; acc[c] = acc[c] + pp;
            pp = w.z * x.z; acc[c] = acc[c] + pp;
            pp = w.w * x.w; acc[c] = acc[c] + pp;
            if (DUAL) {
              pp = w2.x * x.x; acc2[c] = acc2[c] + pp;
              pp = w2.y * x.y; acc2[c] = acc2[c] + pp;
              pp = w2.z * x.z; acc2[c] = acc2[c] + pp;
              pp = w2.w * x.w; acc2[c] = acc2[c] + pp;
            }
          }
        }
      }
    }
    __syncthreads();
  }
  const uint32_t m = blk * R + r;
#pragma unroll
  for (uint32_t c = 0; c < CB; ++c) {
    const uint32_t row = b0 + bb + c * TB;
    if (live && row < a.n && m < g.M) {
      float y = acc[c];
      if (DUAL) {
        const float sg = silu_pinned(acc[c]);
        y = sg * acc2[c];
      } else if (g.epi == kEpiBias) {
        y = acc[c] + g.add[m];
      } else if (g.epi == kEpiResidual) {
        y = g.add[(size_t)row * g.ldadd + m] + acc[c];
      }
      g.Y[(size_t)row * g.ldy + m] = y;
    }
  }
}

// ---------------------------------------------------------------------------
// Batched GEMM in tiles of 16 outputs x 16 batch rows (sequential order, W
// in blocks of R = 8 or 16 rows): a workgroup owns 16 consecutive outputs m
// (16 / R blocks of W) and 16 batch rows; lane l of wave w computes output
// (row 4w + l/16, column l%16) as one strict chain acc + W[m][k] * X[b][k],
// k ascending (code/cis2-fp/src/main.rs:228-243, math.rs:40-48), the bits
// of k_bgemm.  A 16-lane row of a wave shares one batch row: each lane
// reads 4 consecutive k of X per 16-byte LDS read (the row: 64 k), and a
// chain takes X[b][k] from lane (k/4) % 16 of its row by DPP broadcast
// (row_newbcast) inside the multiply; the chains' LDS reads are the W groups
// (a ring of D reads ahead) and one X read per 64 k, where k_bgemm's lanes
// read an X group per 4 k.  NORM: each 16-lane row computes its row's
// inverse RMS from the staged X (the squares' sum in one strict chain, the
// partial sums broadcast the same way), and the chain scales each X read,
// (x * inv) * w[k], before use.  Operands go through registers per K chunk:
// every load of the chunk in flight, then the LDS writes.
// LDS (16-byte groups): W blocks [16/R][q4max * R + 8] (the pad keeps the
// two blocks' reads in distinct banks), W2 the same (DUAL), norm weights
// [q4max], X [16][q4max + 1], then b16_slack(R) readable groups (the
// rings read up to 23 W groups, at stride R, and 31 X groups past a
// chunk's end; the values are never used).
// ---------------------------------------------------------------------------
inline uint32_t b16_slack(uint32_t R) { return 24 * R + 64; }

// Steps G .. 15 of a 16-group block starting at group q: ring slot G % D
// holds W group q + G (refilled with q + G + D), xq is this lane's X group
// q + (lane % 16); X[b][4(q + G) + j] is component j of lane G's xq.
template <bool DUAL, uint32_t D, uint32_t G = 0>
__device__ __forceinline__ void b16_block(float& acc, float& acc2, const v4& xq, v4 (&rw)[D],
                                          v4 (&rw2)[D], const v4* wp, const v4* wp2, uint32_t R,
                                          uint32_t q) {
  if constexpr (G < 16) {
    const v4 w = rw[G % D];
    const float x0 = bcast16<G>(xq.x), x1 = bcast16<G>(xq.y);
    const float x2 = bcast16<G>(xq.z), x3 = bcast16<G>(xq.w);
    float p;
    p = x0 * w.x; acc = acc + p;
    p = x1 * w.y; acc = acc + p;
    p = x2 * w.z; acc = acc + p;
    p = x3 * w.w; acc = acc + p;
    if (DUAL) {
      const v4 w2 = rw2[G % D];
      p = x0 * w2.x; acc2 = acc2 + p;
      p = x1 * w2.y; acc2 = acc2 + p;
      p = x2 * w2.z; acc2 = acc2 + p;
      p = x3 * w2.w; acc2 = acc2 + p;
    }
    rw[G % D] = wp[(size_t)(q + G + D) * R];
    if (DUAL) rw2[G % D] = wp2[(size_t)(q + G + D) * R];
    __builtin_amdgcn_sched_barrier(0);
    b16_block<DUAL, D, G + 1>(acc, acc2, xq, rw, rw2, wp, wp2, R, q);
  }
}
// The first nt (< 16) steps of b16_block.
template <bool DUAL, uint32_t D, uint32_t G = 0>
__device__ __forceinline__ void b16_tail(float& acc, float& acc2, const v4& xq, v4 (&rw)[D],
                                         v4 (&rw2)[D], const v4* wp, const v4* wp2, uint32_t R,
                                         uint32_t q, uint32_t nt) {
  if constexpr (G < 15) {
    if (G < nt) {
      const v4 w = rw[G % D];
      const float x0 = bcast16<G>(xq.x), x1 = bcast16<G>(xq.y);
      const float x2 = bcast16<G>(xq.z), x3 = bcast16<G>(xq.w);
      float p;
      p = x0 * w.x; acc = acc + p;
      p = x1 * w.y; acc = acc + p;
      p = x2 * w.z; acc = acc + p;
      p = x3 * w.w; acc = acc + p;
      if (DUAL) {
        const v4 w2 = rw2[G % D];
        p = x0 * w2.x; acc2 = acc2 + p;
        p = x1 * w2.y; acc2 = acc2 + p;
        p = x2 * w2.z; acc2 = acc2 + p;
        p = x3 * w2.w; acc2 = acc2 + p;
      }
      rw[G % D] = wp[(size_t)(q + G + D) * R];
      if (DUAL) rw2[G % D] = wp2[(size_t)(q + G + D) * R];
      __builtin_amdgcn_sched_barrier(0);
      b16_tail<DUAL, D, G + 1>(acc, acc2, xq, rw, rw2, wp, wp2, R, q, nt);
    }
  }
}
// Sum of squares of n groups x4[0 .. n-1] continuing acc, strict order:
// blocks of 8 groups, the next block's squares formed between this block's
// adds (x4 in LDS with 16 readable groups past n).
template <uint32_t U = 0>
__device__ __forceinline__ void sq_step(float& acc, float (&s)[8][4], const v4* x4, uint32_t gn) {
  if constexpr (U < 8) {
    const v4 v = x4[gn + U];
    acc = acc + s[U][0];
    s[U][0] = v.x * v.x;
    acc = acc + s[U][1];
    s[U][1] = v.y * v.y;
    acc = acc + s[U][2];
    s[U][2] = v.z * v.z;
    acc = acc + s[U][3];
    s[U][3] = v.w * v.w;
    sq_step<U + 1>(acc, s, x4, gn);
  }
}
__device__ __forceinline__ float sumsq_pipe(const v4* x4, uint32_t n, float acc) {
  float s[8][4];
#pragma unroll
  for (uint32_t u = 0; u < 8; ++u) {
    const v4 v = x4[u];
    s[u][0] = v.x * v.x;
    s[u][1] = v.y * v.y;
    s[u][2] = v.z * v.z;
    s[u][3] = v.w * v.w;
  }
  uint32_t g = 0;
  for (; g + 8 < n; g += 8) sq_step(acc, s, x4, g + 8);
#pragma unroll
  for (uint32_t u = 0; u < 8; ++u)
    if (g + u < n) {
      acc = acc + s[u][0];
      acc = acc + s[u][1];
      acc = acc + s[u][2];
      acc = acc + s[u][3];
    }
  return acc;
}

template <bool DUAL, bool NORM>
__global__ __launch_bounds__(256) void k_bgemm16(BgemmArgs a) {
  extern __shared__ v4 sm[];
  constexpr uint32_t D = 8;  // W groups read ahead (a divisor of 16: the ring slot of
                             // group q + G is G % D for every block start q)
  uint32_t si = 0;
  if (a.nseg > 1 && blockIdx.x >= a.blk0[1]) si = (a.nseg > 2 && blockIdx.x >= a.blk0[2]) ? 2 : 1;
  const BgemmSeg g = si == 0 ? a.s[0] : (si == 1 ? a.s[1] : a.s[2]);
  const uint32_t R = g.R, KC = a.KC, K = g.K, nblk = 16 / R;
  const uint32_t tile = blockIdx.x - a.blk0[si], b0 = blockIdx.y * 16, t = threadIdx.x;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const uint32_t c = lane & 15, bb = wv * 4 + (lane >> 4);  // output column, batch row
  const uint32_t qmax = KC / 4, xs4 = qmax + 1, BS = qmax * R + 8;
  v4* Ws = sm;                                   // [nblk][BS]
  v4* W2s = Ws + (size_t)nblk * BS;              // DUAL
  v4* NWs = W2s + (DUAL ? (size_t)nblk * BS : 0);  // NORM: the chunk's norm weights
  v4* Xs = NWs + (NORM ? qmax : 0);              // [16][xs4]
  const v4* Wg = reinterpret_cast<const v4*>(g.W + (size_t)tile * 16 * K);
  const v4* Wg2 = DUAL ? reinterpret_cast<const v4*>(a.W2 + (size_t)tile * 16 * K) : nullptr;
  // A chunk's operands (groups g0 .. g0+q4-1): per round, a thread loads up
  // to 8 W (and 8 W2) groups of the tile's blocks, the X groups of 4 rows
  // (wave w: rows 4w .. 4w+3, lanes over the groups) and one norm weight
  // group, all in flight, then writes them.
  auto stage = [&](uint32_t g0, uint32_t q4, bool with_w) {
    constexpr uint32_t WB = 8, XP = 4;
    const uint32_t nwb = q4 * R, nw = with_w ? nblk * nwb : 0, pieces = (q4 + 63) / 64;
    for (uint32_t rd = 0; rd == 0 || rd * 256 * WB < nw; ++rd) {
      v4 tw[WB], tw2[WB], tx[4][XP], tn;
#pragma unroll
      for (uint32_t u = 0; u < WB; ++u) {
        const uint32_t i = (rd * WB + u) * 256 + t;
        if (i < nw) {
          const uint32_t cb = i >= nwb ? 1 : 0, j = i - cb * nwb;
          tw[u] = Wg[(size_t)cb * R * K / 4 + (size_t)g0 * R + j];
          if (DUAL) tw2[u] = Wg2[(size_t)cb * R * K / 4 + (size_t)g0 * R + j];
        }
      }
      if (rd == 0) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const uint32_t bx = wv * 4 + j, row = std::min(b0 + bx, a.n - 1);
          const v4* xr = reinterpret_cast<const v4*>(g.X + (size_t)row * g.ldx) + g0;
#pragma unroll
          for (uint32_t pc = 0; pc < XP; ++pc) {
            const uint32_t q = pc * 64 + lane;
            if (pc < pieces && q < q4) tx[j][pc] = xr[q];
          }
        }
        if (NORM && with_w && t < q4) tn = reinterpret_cast<const v4*>(a.nw)[g0 + t];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (uint32_t u = 0; u < WB; ++u) {
        const uint32_t i = (rd * WB + u) * 256 + t;
        if (i < nw) {
          const uint32_t cb = i >= nwb ? 1 : 0, j = i - cb * nwb;
          Ws[cb * BS + j] = tw[u];
          if (DUAL) W2s[cb * BS + j] = tw2[u];
        }
      }
      if (rd == 0) {
#pragma unroll
        for (uint32_t j = 0; j < 4; ++j) {
          const uint32_t bx = wv * 4 + j;
#pragma unroll
          for (uint32_t pc = 0; pc < XP; ++pc) {
            const uint32_t q = pc * 64 + lane;
            if (pc < pieces && q < q4) Xs[bx * xs4 + q] = tx[j][pc];
          }
        }
        if (NORM && with_w && t < q4) NWs[t] = tn;
      }
    }
  };
  // RMSNorm: the 16 lanes of a batch row chain its squares (strict order)
  // over each staged chunk (16-byte reads, the same address across the
  // row's lanes); rows longer than one chunk take a first pass over their
  // chunks before the GEMM's.
  const v4* xrow = Xs + bb * xs4;
  const v4* xr = xrow + c;
  auto sumsq_chunk = [&](uint32_t q4, float acc0) { return sumsq_pipe(xrow, q4, acc0); };
  float inv = 0.0f;
  if (NORM && K > KC) {
    float ssq = 0.0f;
    for (uint32_t k0 = 0; k0 < K; k0 += KC) {
      const uint32_t q4 = std::min(KC, K - k0) / 4;
      stage(k0 / 4, q4, false);
      __syncthreads();
      ssq = sumsq_chunk(q4, ssq);
      __syncthreads();
    }
    inv = inv_rms_of(ssq, K, a.eps);
  }
  float acc = 0.0f, acc2 = 0.0f;
  const uint32_t cb = c / R, r = c - cb * R;
  const v4* wp = Ws + cb * BS + r;
  const v4* wp2 = W2s + cb * BS + r;
  for (uint32_t k0 = 0; k0 < K; k0 += KC) {
    const uint32_t q4 = std::min(KC, K - k0) / 4;
    stage(k0 / 4, q4, true);
    __syncthreads();
    if (NORM && K <= KC) inv = inv_rms_of(sumsq_chunk(q4, 0.0f), K, a.eps);
    // this lane's X group of a block, scaled for NORM
    auto xget = [&](uint32_t q) {
      v4 x = xr[q];
      if (NORM) {
        const v4 w = NWs[q + c];
        float sx;
        sx = x.x * inv; x.x = sx * w.x;
        sx = x.y * inv; x.y = sx * w.y;
        sx = x.z * inv; x.z = sx * w.z;
        sx = x.w * inv; x.w = sx * w.w;
      }
      return x;
    };
    v4 rw[D], rw2[D];
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      rw[u] = wp[(size_t)u * R];
      if (DUAL) rw2[u] = wp2[(size_t)u * R];
    }
    v4 xq = xget(0);
    uint32_t q = 0;
    for (; q + 16 <= q4; q += 16) {
      const v4 xn = xget(q + 16);  // the next block's X (past the end: unused)
      b16_block<DUAL, D>(acc, acc2, xq, rw, rw2, wp, wp2, R, q);
      xq = xn;
    }
    if (q < q4) b16_tail<DUAL, D>(acc, acc2, xq, rw, rw2, wp, wp2, R, q, q4 - q);
    __syncthreads();
  }
  const uint32_t m = tile * 16 + c, row = b0 + bb;
  if (row < a.n && m < g.M) {
    float y = acc;
    if (DUAL) {
      const float sg = silu_pinned(acc);
      y = sg * acc2;
    } else if (g.epi == kEpiBias) {
      y = acc + g.add[m];
    } else if (g.epi == kEpiResidual) {
      y = g.add[(size_t)row * g.ldadd + m] + acc;
    }
    g.Y[(size_t)row * g.ldy + m] = y;
  }
}

// (value, index) pick of a strict-> scan from index 0 (first maximum wins;
// a NaN wins only at index 0, handled by the caller).
struct Pick {
  float v;
  uint32_t i;  // UINT32_MAX: none
};
__device__ __forceinline__ Pick pick2(Pick a, Pick b) {
  if (b.i == UINT32_MAX) return a;
  if (a.i == UINT32_MAX) return b;
  if (b.v > a.v) return b;
  if (a.v > b.v) return a;
  return b.i < a.i ? b : a;
}
__device__ Pick pick_block(Pick x, Pick* scratch) {
  for (int off = 32; off > 0; off >>= 1) {
    Pick o;
    o.v = __shfl_xor(x.v, off, 64);
    o.i = __shfl_xor(x.i, off, 64);
    x = pick2(x, o);
  }
  const uint32_t wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wv] = x;
  __syncthreads();
  Pick r = scratch[0];
  for (uint32_t i = 1; i < nw; ++i) r = pick2(r, scratch[i]);
  __syncthreads();
  return r;
}

__global__ void k_embed_rows(const float* __restrict__ E, RowsDesc rows, uint32_t H,
                             uint32_t vocab, float* h, uint32_t* err) {
  const uint32_t r = blockIdx.x;
  uint32_t tok = rows.tok[r];
  if (tok >= vocab) {
    if (threadIdx.x == 0) atomicOr(err, 1u);
    tok = 0;
  }
  const float* src = E + (size_t)tok * H;
  for (uint32_t i = threadIdx.x; i < H; i += blockDim.x) h[(size_t)r * H + i] = src[i];
}

// RoPE rotate-half (main.rs:285-307): o1 = x1*c + (-x2)*s, o2 = x2*c + x1*s.
__global__ __launch_bounds__(256) void k_rope_store_rows(float* q, float* k, const float* v,
                                                         const float* __restrict__ cs,
                                                         RowsDesc rows, uint32_t nh,
                                                         uint32_t nkv, uint32_t hd,
                                                         uint32_t max_pos, float* kc, float* vc,
                                                         uint64_t seq_stride) {
  const uint32_t r = blockIdx.x, pos = rows.pos[r], half = hd / 2;
  const size_t sb = (size_t)rows.seq[r] * seq_stride;
  float* qr = q + (size_t)r * nh * hd;
  float* kr = k + (size_t)r * nkv * hd;
  const float* vr = v + (size_t)r * nkv * hd;
  const float* c = cs + (size_t)pos * half * 2;
  const uint32_t total = (nh + nkv) * half;
  for (uint32_t idx = threadIdx.x; idx < total; idx += blockDim.x) {
    const uint32_t head = idx / half, i = idx - head * half;
    float* hv = head < nh ? qr + (size_t)head * hd : kr + (size_t)(head - nh) * hd;
    const float cv = c[2 * i], sv = c[2 * i + 1];
    const float x1 = hv[i], x2 = hv[i + half];
    float t1 = x1 * cv;
    float nx2 = -x2;
    float t2 = nx2 * sv;
    float t3 = x2 * cv;
    float t4 = x1 * sv;
    const float o1 = t1 + t2, o2 = t3 + t4;
    hv[i] = o1;
    hv[i + half] = o2;
    if (head >= nh) {
      const size_t base = (size_t)(head - nh) * hd;
      kc[sb + (base + i) * max_pos + pos] = o1;
      kc[sb + (base + i + half) * max_pos + pos] = o2;
    }
  }
  for (uint32_t idx = threadIdx.x; idx < nkv * hd; idx += blockDim.x)
    vc[sb + (size_t)idx * max_pos + pos] = vr[idx];
}

// One workgroup per (row, HPW query heads that share one KV head): per head
// scores_j = dot(q, k_j) * scale (dot_seq, or dot_tree), softmax (first-wins
// max, pinned exp, strict or tree denominator, true divide), then
// out_d = fold_j (p_j * v_j[d]) in position order
// (code/cis2-fp/src/main.rs:429-467; math.rs:425-465).  The heads of a
// workgroup read each K and V element once: a column's K values are loaded
// once for all HPW score chains, and the V rows of the HPW * hd output
// chains come from the same addresses.
// LDS: q [HPW][hd4], scores [HPW][ls], tree partials [HPW][nbs], with
// hd4 = hd rounded up to 4 and ls = max_len rounded up to 4.
template <uint32_t HPW>
__global__ __launch_bounds__(kAttT) void k_attention_rows(const float* __restrict__ q,
                                                        const float* __restrict__ kc,
                                                        const float* __restrict__ vc,
                                                        RowsDesc rows, uint32_t nh, uint32_t nkv,
                                                        uint32_t hd, uint32_t max_pos,
                                                        uint64_t seq_stride, float scale,
                                                        float* out, uint32_t tree, uint32_t ls) {
  extern __shared__ v4 sh4[];  // 16-byte aligned: q and scores are read 16 bytes at a time
  float* sh = reinterpret_cast<float*>(sh4);
  __shared__ Pick red[kAttT / 64];
  __shared__ float s_den[HPW];
  const uint32_t r = blockIdx.x, qh0 = blockIdx.y * HPW;  // rows on x: up to 2^31 of them
  const uint32_t group = nh / nkv, kvh = qh0 / group, pos = rows.pos[r], len = pos + 1;
  const uint32_t hd4 = (hd + 3) & ~3u, nbs = (ls + 31) / 32, t = threadIdx.x;
  const size_t sb = (size_t)rows.seq[r] * seq_stride;
  float* sq = sh;
  float* ssb = sh + HPW * hd4;
  float* partb = ssb + HPW * ls;
  const float* qv = q + (size_t)r * nh * hd + (size_t)qh0 * hd;
  for (uint32_t i = t; i < HPW * hd; i += blockDim.x) {
    const uint32_t h = i / hd, d = i - h * hd;
    sq[h * hd4 + d] = qv[i];
  }
  __syncthreads();
  const float* kb = kc + sb + (size_t)kvh * hd * max_pos;
  for (uint32_t j = t; j < len; j += blockDim.x) {
    float acc[HPW];
#pragma unroll
    for (uint32_t h = 0; h < HPW; ++h) acc[h] = 0.0f;
    if (tree) {
      for (uint32_t d0 = 0; d0 < hd; d0 += 32) {
        float kv[32];
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) kv[i] = d0 + i < hd ? kb[(size_t)(d0 + i) * max_pos + j] : 0.0f;
#pragma unroll
        for (uint32_t h = 0; h < HPW; ++h) {
          float l[32];
#pragma unroll
          for (uint32_t i = 0; i < 32; ++i) l[i] = d0 + i < hd ? sq[h * hd4 + d0 + i] * kv[i] : 0.0f;
          acc[h] = acc[h] + tree32(l);
        }
      }
    } else {
      // the column's loads go out 64 at a time, then the heads' chain steps
      // over them, interleaved
      uint32_t d0 = 0;
      for (; d0 + 64 <= hd; d0 += 64) {
        float kv[64];
#pragma unroll
        for (uint32_t i = 0; i < 64; ++i) kv[i] = kb[(size_t)(d0 + i) * max_pos + j];
#pragma unroll
        for (uint32_t i = 0; i < 64; ++i) {
#pragma unroll
          for (uint32_t h = 0; h < HPW; ++h) {
            const float p = sq[h * hd4 + d0 + i] * kv[i];
            acc[h] = acc[h] + p;
          }
        }
      }
      for (; d0 < hd; ++d0) {
        const float kv = kb[(size_t)d0 * max_pos + j];
#pragma unroll
        for (uint32_t h = 0; h < HPW; ++h) {
          const float p = sq[h * hd4 + d0] * kv;
          acc[h] = acc[h] + p;
        }
      }
    }
#pragma unroll
    for (uint32_t h = 0; h < HPW; ++h) ssb[h * ls + j] = acc[h] * scale;
  }
  __syncthreads();
  // per head: first-wins maximum (NaN at 0 wins), then exp(s - max)
  for (uint32_t h = 0; h < HPW; ++h) {
    float* ss = ssb + h * ls;
    Pick best = {0.0f, UINT32_MAX};
    for (uint32_t j = t; j < len; j += blockDim.x) {
      const float v = ss[j];
      if (v == v) best = pick2(best, Pick{v, j});
    }
    best = pick_block(best, red);
    const float mx = (ss[0] != ss[0]) ? ss[0] : best.v;
    for (uint32_t j = t; j < len; j += blockDim.x) {
      const float dlt = ss[j] - mx;
      ss[j] = exp_pinned(dlt);
    }
  }
  __syncthreads();
  const uint32_t nb = (len + 31) / 32;
  if (tree) {
    for (uint32_t i = t; i < HPW * nb; i += blockDim.x) {
      const uint32_t h = i / nb, tb = i - h * nb;
      const float* ss = ssb + h * ls;
      float l[32];
#pragma unroll
      for (uint32_t k = 0; k < 32; ++k) l[k] = 32 * tb + k < len ? ss[32 * tb + k] : 0.0f;
      partb[h * nbs + tb] = tree32(l);
    }
    __syncthreads();
  }
  // denominators: wave w sums heads w, w + 4, ...; every lane of the wave
  // runs the same chain
  for (uint32_t h = t >> 6; h < HPW; h += blockDim.x >> 6) {
    float acc = 0.0f;
    if (tree) {
      for (uint32_t tb = 0; tb < nb; ++tb) acc = acc + partb[h * nbs + tb];
    } else {
      // 16-byte reads (every lane the same address), 8 of them per batch
      const float* ss = ssb + h * ls;
      const v4* s4p = reinterpret_cast<const v4*>(ss);
      uint32_t j = 0;
      for (; j + 32 <= len; j += 32) {
        v4 e[8];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) e[u] = s4p[j / 4 + u];
#pragma unroll
        for (uint32_t u = 0; u < 8; ++u) {
          acc = acc + e[u].x;
          acc = acc + e[u].y;
          acc = acc + e[u].z;
          acc = acc + e[u].w;
        }
      }
      for (; j < len; ++j) acc = acc + ss[j];
    }
    if ((t & 63) == 0) s_den[h] = acc;
  }
  __syncthreads();
  for (uint32_t i = t; i < HPW * len; i += blockDim.x) {
    const uint32_t h = i / len, j = i - h * len;
    const float pj = ssb[h * ls + j] / s_den[h];
    ssb[h * ls + j] = pj;
  }
  __syncthreads();
  const float* vb = vc + sb + (size_t)kvh * hd * max_pos;
  for (uint32_t i = t; i < HPW * hd; i += blockDim.x) {
    const uint32_t h = i / hd, d = i - h * hd;
    float* o = out + (size_t)r * nh * hd + (size_t)(qh0 + h) * hd;
    const float* ss = ssb + h * ls;
    // row d of V is contiguous: 16-byte loads, a batch of 64 positions in
    // flight while the previous batch's chain steps run
    const v4* vr4 = reinterpret_cast<const v4*>(vb + (size_t)d * max_pos);
    const v4* p4 = reinterpret_cast<const v4*>(ss);
    float acc = 0.0f;
    uint32_t j = 0;
    constexpr uint32_t VB = 16;
    v4 cur[VB], nxt[VB];
    const uint32_t full = len / (4 * VB);
    if (full > 0) {
#pragma unroll
      for (uint32_t u = 0; u < VB; ++u) cur[u] = vr4[u];
    }
    for (uint32_t bt = 0; bt < full; ++bt, j += 4 * VB) {
      if (bt + 1 < full) {
#pragma unroll
        for (uint32_t u = 0; u < VB; ++u) nxt[u] = vr4[(j + 4 * VB) / 4 + u];
      }
#pragma unroll
      for (uint32_t u = 0; u < VB; ++u) {
        const v4 pp = p4[j / 4 + u];
        float p;
        p = pp.x * cur[u].x; acc = acc + p;
        p = pp.y * cur[u].y; acc = acc + p;
        p = pp.z * cur[u].z; acc = acc + p;
        p = pp.w * cur[u].w; acc = acc + p;
      }
#pragma unroll
      for (uint32_t u = 0; u < VB; ++u) cur[u] = nxt[u];
    }
    const float* vr = vb + (size_t)d * max_pos;
    for (; j < len; ++j) {
      const float p = ss[j] * vr[j];
      acc = acc + p;
    }
    o[d] = acc;
  }
}

// Strict sums over LDS with a ring of 16-byte reads in flight; the caller
// keeps D groups of readable LDS after the last one, so the ring is refilled
// unconditionally at fixed offsets (the extra reads are never used) and the
// last partial round adds its groups under uniform tests.  n wave-uniform.
//   chain_lds_s:  acc + x[0] + x[1] + ... + x[n-1]
//   mix_lds_s:    acc + p[0]*v[0] + ... + p[n-1]*v[n-1]
// x, p and v 16-byte aligned.
template <uint32_t D>
__device__ __forceinline__ float chain_lds_s(const float* x, uint32_t n, float acc) {
  const v4* x4 = reinterpret_cast<const v4*>(x);
  const uint32_t ng = n / 4;
  v4 ring[D];
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) ring[u] = x4[u];
  uint32_t g = 0;
  for (; g + D <= ng; g += D) {
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      const v4 r = ring[u];
      acc = acc + r.x;
      acc = acc + r.y;
      acc = acc + r.z;
      acc = acc + r.w;
      ring[u] = x4[g + u + D];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (uint32_t u = 0; u + 1 < D; ++u) {
    if (g + u < ng) {
      const v4 r = ring[u];
      acc = acc + r.x;
      acc = acc + r.y;
      acc = acc + r.z;
      acc = acc + r.w;
    }
  }
  for (uint32_t j = 4 * ng; j < n; ++j) acc = acc + x[j];
  return acc;
}
template <uint32_t D>
__device__ __forceinline__ float mix_lds_s(const float* p, const float* v, uint32_t n, float acc) {
  const v4* p4 = reinterpret_cast<const v4*>(p);
  const v4* v4p = reinterpret_cast<const v4*>(v);
  const uint32_t ng = n / 4;
  v4 rp[D], rv[D];
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) {
    rp[u] = p4[u];
    rv[u] = v4p[u];
  }
  auto step = [&](const v4& a, const v4& b) {
    float pr;
    pr = a.x * b.x; acc = acc + pr;
    pr = a.y * b.y; acc = acc + pr;
    pr = a.z * b.z; acc = acc + pr;
    pr = a.w * b.w; acc = acc + pr;
  };
  uint32_t g = 0;
  for (; g + D <= ng; g += D) {
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      step(rp[u], rv[u]);
      rp[u] = p4[g + u + D];
      rv[u] = v4p[g + u + D];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (uint32_t u = 0; u + 1 < D; ++u)
    if (g + u < ng) step(rp[u], rv[u]);
  for (uint32_t j = 4 * ng; j < n; ++j) {
    const float pr = p[j] * v[j];
    acc = acc + pr;
  }
  return acc;
}
// The same strict sum from two register sets of 8 groups: the next set's
// reads go out before the current set's 32 adds (one wait per set); no read
// past the end.  Faster than the ring on chains of 100+ groups.
__device__ __forceinline__ float chain_lds_pp(const float* x, uint32_t n, float acc) {
  constexpr uint32_t U = 8;
  const v4* x4 = reinterpret_cast<const v4*>(x);
  const uint32_t ng = n / 4;
  auto add1 = [&](const v4 v) {
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  };
  uint32_t g = 0;
  if (ng >= U) {
    v4 a[U], b[U];
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) a[u] = x4[u];
    for (; g + 3 * U <= ng; g += 2 * U) {
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) b[u] = x4[g + U + u];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) add1(a[u]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) a[u] = x4[g + 2 * U + u];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (uint32_t u = 0; u < U; ++u) add1(b[u]);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
      if (g + U + u < ng) b[u] = x4[g + U + u];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) add1(a[u]);
    g += U;
#pragma unroll
    for (uint32_t u = 0; u < U; ++u)
      if (g + u < ng) add1(b[u]);
    g = g + U < ng ? g + U : ng;
  }
  for (; g < ng; ++g) add1(x4[g]);
  for (uint32_t j = 4 * ng; j < n; ++j) acc = acc + x[j];
  return acc;
}
// Readable floats the decode-rows attention keeps after its LDS regions.
constexpr uint32_t kKvSlack = 64;

// acc + p[0] + ... + p[n-1], strictly left to right (16-byte LDS reads,
// eight of them per batch).
__device__ __forceinline__ float chain_lds(const float* p, uint32_t n, float acc) {
  const v4* p4 = reinterpret_cast<const v4*>(p);
  uint32_t j = 0;
  for (; j + 32 <= n; j += 32) {
    v4 e[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) e[u] = p4[j / 4 + u];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u) {
      acc = acc + e[u].x;
      acc = acc + e[u].y;
      acc = acc + e[u].z;
      acc = acc + e[u].w;
    }
  }
  for (; j < n; ++j) acc = acc + p[j];
  return acc;
}

// ---------------------------------------------------------------------------
// Attention of decode rows (few rows, one per sequence): one workgroup of
// kKvT threads per (row, KV head) takes the HPW = nh / nkv query heads of
// that KV head, with the per-row kernel's arithmetic in the same order
// (scores d ascending, dot_seq or tree32 blocks, first-wins maximum, pinned
// exp, strict or tree denominator, true divide, V-mix j ascending;
// code/cis2-fp/src/main.rs:429-467, math.rs:425-465), so every output has
// the per-row kernel's bits.
//   scores:  a thread takes two adjacent positions per round (8-byte K
//            loads, 64 d per batch in flight), one chain per (position,
//            head);
//   V rows:  then copied into LDS with global_load_lds by every wave, in
//            chunks of C <= 256 positions over two buffers (row stride
//            C + 4 floats: lane d's 16-byte reads fall in distinct banks);
//            the softmax's barriers wait for LDS only, so the copies land
//            meanwhile; a buffer is refilled two chunks ahead while the
//            V-mix runs over the other;
//   softmax: the maximum with DPP, exp, the HPW denominators on HPW waves
//            at once (a ring of LDS reads), the divide;
//   V-mix:   HPW * HD / 64 waves, lane = d, each product formed with p_j
//            taken by DPP broadcast (row_newbcast) from a register holding
//            16 consecutive probabilities in every 16-lane row, the next 16
//            positions' reads in flight.
// LDS (floats): q [HPW][HD], scores [HPW][ls], tree partials [HPW][nbs]
// (rounded up to 4), V [2][HD][C + 4], kKvSlack readable floats (the read
// rings run up to 56 floats past a row's end).
// ---------------------------------------------------------------------------
constexpr uint32_t kKvT = 512;
typedef float v2 __attribute__((ext_vector_type(2)));
// RoPE inputs of the fused form: the rows' raw k and v ([n][nkv][hd]) and
// the cos/sin table ([max_pos][hd/2][2]).
struct KvFuse {
  const float* k;
  const float* v;
  const float* rope_cs;
  uint32_t nkv;
};

// s_waitcnt lgkmcnt(0), then s_barrier: LDS written before it is visible
// after it; global loads in flight stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);
  __builtin_amdgcn_s_barrier();
}
// acc + P_0 * v[0].x + P_1 * v[0].y + ... + P_15 * v[3].w in order (P_k:
// lane k of this lane's 16-lane row), each product rounded, then the add.
template <uint32_t K = 0>
__device__ __forceinline__ void mix16(float& acc, float P, const v4 (&v)[4]) {
  if constexpr (K < 16) {
    const v4 w = v[K / 4];
    const float x = K % 4 == 0 ? w.x : K % 4 == 1 ? w.y : K % 4 == 2 ? w.z : w.w;
    const float t = bcast16<K>(P) * x;
    acc = acc + t;
    mix16<K + 1>(acc, P, v);
  }
}
// The first rem (< 16) steps of mix16.
template <uint32_t K = 0>
__device__ __forceinline__ void mix16_part(float& acc, float P, const v4 (&v)[4], uint32_t rem) {
  if constexpr (K < 15) {
    if (K < rem) {
      const v4 w = v[K / 4];
      const float x = K % 4 == 0 ? w.x : K % 4 == 1 ? w.y : K % 4 == 2 ? w.z : w.w;
      const float t = bcast16<K>(P) * x;
      acc = acc + t;
      mix16_part<K + 1>(acc, P, v, rem);
    }
  }
}
// acc + p[0]*v[0] + ... + p[n-1]*v[n-1] in order; p and v in LDS, 16-byte
// aligned, 16 readable floats past n; two register sets, each block of 16
// positions read one block ahead.  n wave-uniform.
__device__ __forceinline__ float mix_dpp(const float* p, const float* v, uint32_t n, float acc) {
  const uint32_t k = threadIdx.x & 15, nb = n >> 4;
  const v4* v4p = reinterpret_cast<const v4*>(v);
  float PA = p[k], PB;
  v4 vA[4], vB[4];
#pragma unroll
  for (uint32_t u = 0; u < 4; ++u) vA[u] = v4p[u];
  uint32_t m = 0;
  for (; m + 2 <= nb; m += 2) {
    PB = p[16 * (m + 1) + k];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) vB[u] = v4p[4 * (m + 1) + u];
    mix16(acc, PA, vA);
    PA = p[16 * (m + 2) + k];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) vA[u] = v4p[4 * (m + 2) + u];
    mix16(acc, PB, vB);
  }
  if (m < nb) {  // one whole block left
    PB = p[16 * (m + 1) + k];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) vB[u] = v4p[4 * (m + 1) + u];
    mix16(acc, PA, vA);
    PA = PB;
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) vA[u] = vB[u];
  }
  mix16_part(acc, PA, vA, n - 16 * nb);
  return acc;
}

template <uint32_t HPW, uint32_t HD, bool FUSE>
__global__ __launch_bounds__(kKvT) void k_attention_kv(const float* __restrict__ q,
                                                     float* kc, float* vc, RowsDesc rows,
                                                     uint32_t nh, uint32_t max_pos,
                                                     uint64_t seq_stride, float scale,
                                                     float* out, uint32_t tree, uint32_t ls,
                                                     uint32_t C, KvFuse fz) {
  constexpr uint32_t NW = kKvT / 64, WPH = HD / 64, CW = HPW * WPH;
  static_assert(HD % 64 == 0 && CW <= NW, "chain waves");
  extern __shared__ v4 sh4[];
  float* sh = reinterpret_cast<float*>(sh4);
  __shared__ float s_red[NW][HPW];
  __shared__ float s_den[HPW];
  const uint32_t r = blockIdx.x, kvh = blockIdx.y, qh0 = kvh * HPW, t = threadIdx.x;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(t >> 6), lane = t & 63;
  const uint32_t pos = rows.pos[r], len = pos + 1, S = C + 4;
  // FUSE: position pos comes from this launch (its K and V from LDS), the
  // caches serve positions 0 .. pos-1
  const uint32_t lc = FUSE ? pos : len;
  const uint32_t nbs = (ls + 31) / 32, len4 = (lc + 3) & ~3u;
  const size_t sb = (size_t)rows.seq[r] * seq_stride;
  float* kb = kc + sb + (size_t)kvh * HD * max_pos;
  float* vb = vc + sb + (size_t)kvh * HD * max_pos;
  float* sq = sh;
  float* kself = sq + HPW * HD;  // FUSE: this position's rotated k and its v
  float* vself = kself + HD;
  float* ssb = vself + HD;
  float* partb = ssb + HPW * ls;
  float* VL = partb + ((HPW * nbs + 3) & ~3u);
  const uint32_t nch = (lc + C - 1) / C;
  // chunk ch of V row d into buffer ch % 2: one wave instruction (C <= 256
  // positions), lanes past the chunk or the row's end idle
  auto stage_row = [&](uint32_t ch, uint32_t d) {
    const uint32_t o = lane * 4, j = ch * C + o;
    if (o < C && j < len4)
      lds_load16(reinterpret_cast<const v4*>(vb + (size_t)d * max_pos + j),
                 reinterpret_cast<v4*>(VL + (size_t)(ch & 1) * HD * S + (size_t)d * S));
  };
  const float* qv = q + (size_t)r * nh * HD + (size_t)qh0 * HD;
  if constexpr (FUSE) {
    // RoPE at pos of the HPW query heads and of KV head kvh, in
    // k_rope_store_rows's order (o1 = x1*c + (-x2)*s, o2 = x2*c + x1*s); the
    // rotated k and the raw v also into the caches at pos
    constexpr uint32_t half = HD / 2;
    const float* cs = fz.rope_cs + (size_t)pos * half * 2;
    const float* kin = fz.k + (size_t)r * fz.nkv * HD + (size_t)kvh * HD;
    const float* vin = fz.v + (size_t)r * fz.nkv * HD + (size_t)kvh * HD;
    for (uint32_t i = t; i < (HPW + 1) * half; i += kKvT) {
      const uint32_t h = i / half, ii = i - h * half;
      const float* src = h < HPW ? qv + (size_t)h * HD : kin;
      const float cv = cs[2 * ii], sv = cs[2 * ii + 1];
      const float x1 = src[ii], x2 = src[ii + half];
      const float t1 = x1 * cv;
      const float nx2 = -x2;
      const float t2 = nx2 * sv;
      const float t3 = x2 * cv;
      const float t4 = x1 * sv;
      const float o1 = t1 + t2, o2 = t3 + t4;
      if (h < HPW) {
        sq[h * HD + ii] = o1;
        sq[h * HD + ii + half] = o2;
      } else {
        kself[ii] = o1;
        kself[ii + half] = o2;
        kb[(size_t)ii * max_pos + pos] = o1;
        kb[(size_t)(ii + half) * max_pos + pos] = o2;
      }
    }
    for (uint32_t d = t; d < HD; d += kKvT) {
      const float vv = vin[d];
      vself[d] = vv;
      vb[(size_t)d * max_pos + pos] = vv;
    }
  } else {
    for (uint32_t i = t; i < HPW * HD; i += kKvT) sq[i] = qv[i];
  }
  lds_barrier();
  // FUSE: position pos's scores from the rotated k in LDS, one lane per head
  if (FUSE && t < HPW) {
    float acc = 0.0f;
    if (tree) {
#pragma unroll
      for (uint32_t d0 = 0; d0 < HD; d0 += 32) {
        float l[32];
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) l[i] = sq[t * HD + d0 + i] * kself[d0 + i];
        acc = acc + tree32(l);
      }
    } else {
      for (uint32_t d = 0; d < HD; ++d) {
        const float pr = sq[t * HD + d] * kself[d];
        acc = acc + pr;
      }
    }
    ssb[t * ls + pos] = acc * scale;
  }
  // scores: thread t takes positions jp, jp + 1 (jp = 2 * (t + k * kKvT);
  // len4 <= max_pos, so a pair below len4 stays in the row; a pair's
  // second position past the cached ones is computed and dropped)
  for (uint32_t jp = 2 * t; jp < lc; jp += 2 * kKvT) {
    float acc[2][HPW];
#pragma unroll
    for (uint32_t p = 0; p < 2; ++p)
#pragma unroll
      for (uint32_t h = 0; h < HPW; ++h) acc[p][h] = 0.0f;
#pragma unroll
    for (uint32_t d0 = 0; d0 < HD; d0 += 64) {
      v2 kv[64];
#pragma unroll
      for (uint32_t i = 0; i < 64; ++i)
        kv[i] = *reinterpret_cast<const v2*>(kb + (size_t)(d0 + i) * max_pos + jp);
      if (tree) {
#pragma unroll
        for (uint32_t b0 = 0; b0 < 64; b0 += 32)
#pragma unroll
          for (uint32_t p = 0; p < 2; ++p)
#pragma unroll
            for (uint32_t h = 0; h < HPW; ++h) {
              float l[32];
#pragma unroll
              for (uint32_t i = 0; i < 32; ++i)
                l[i] = sq[h * HD + d0 + b0 + i] * (p ? kv[b0 + i].y : kv[b0 + i].x);
              acc[p][h] = acc[p][h] + tree32(l);
            }
      } else {
#pragma unroll
        for (uint32_t i = 0; i < 64; ++i)
#pragma unroll
          for (uint32_t h = 0; h < HPW; ++h) {
            const float qd = sq[h * HD + d0 + i];
            float pr;
            pr = qd * kv[i].x; acc[0][h] = acc[0][h] + pr;
            pr = qd * kv[i].y; acc[1][h] = acc[1][h] + pr;
          }
      }
    }
#pragma unroll
    for (uint32_t p = 0; p < 2; ++p)
      if (jp + p < lc)
#pragma unroll
        for (uint32_t h = 0; h < HPW; ++h) ssb[h * ls + jp + p] = acc[p][h] * scale;
  }
  // the V copies of chunks 0 and 1, spread over the waves
  for (uint32_t d = wv; d < HD; d += NW) {
    stage_row(0, d);
    if (nch > 1) stage_row(1, d);
  }
  lds_barrier();
  // maximum per head: the largest non-NaN score (its value does not depend
  // on which of equal scores is first: exp(s - (+0)) = exp(s - (-0))), a NaN
  // score at 0 wins
  {
    float m[HPW];
#pragma unroll
    for (uint32_t h = 0; h < HPW; ++h) m[h] = -__builtin_huge_valf();
    for (uint32_t j = t; j < len; j += kKvT)
#pragma unroll
      for (uint32_t h = 0; h < HPW; ++h) {
        const float v = ssb[h * ls + j];
        m[h] = v > m[h] ? v : m[h];
      }
#pragma unroll
    for (uint32_t h = 0; h < HPW; ++h) {
      m[h] = wave_max(m[h]);
      if (lane == 0) s_red[wv][h] = m[h];
    }
    lds_barrier();
#pragma unroll
    for (uint32_t h = 0; h < HPW; ++h) {
      float mx = s_red[0][h];
#pragma unroll
      for (uint32_t w = 1; w < NW; ++w) mx = s_red[w][h] > mx ? s_red[w][h] : mx;
      const float s0 = ssb[h * ls];
      m[h] = s0 != s0 ? s0 : mx;
    }
    for (uint32_t j = t; j < len; j += kKvT)
#pragma unroll
      for (uint32_t h = 0; h < HPW; ++h) {
        const float dlt = ssb[h * ls + j] - m[h];
        ssb[h * ls + j] = exp_pinned(dlt);
      }
  }
  lds_barrier();
  const uint32_t nb = (len + 31) / 32;
  if (tree) {
    for (uint32_t i = t; i < HPW * nb; i += kKvT) {
      const uint32_t h = i / nb, tb = i - h * nb;
      const float* ss = ssb + h * ls;
      float l[32];
#pragma unroll
      for (uint32_t k = 0; k < 32; ++k) l[k] = 32 * tb + k < len ? ss[32 * tb + k] : 0.0f;
      partb[h * nbs + tb] = tree32(l);
    }
    lds_barrier();
  }
  // denominators: wave h sums head h (every lane the same chain)
  if (wv < HPW) {
    const float acc = tree ? chain_lds_s<14>(partb + wv * nbs, nb, 0.0f)
                           : chain_lds_pp(ssb + wv * ls, len, 0.0f);
    if (lane == 0) s_den[wv] = acc;
  }
  lds_barrier();
#pragma unroll
  for (uint32_t h = 0; h < HPW; ++h) {
    const float den = s_den[h];
    for (uint32_t j = t; j < len; j += kKvT) {
      const float pj = ssb[h * ls + j] / den;
      ssb[h * ls + j] = pj;
    }
  }
  // V-mix over the staged chunks
  const uint32_t h = wv / WPH, d = (wv - h * WPH) * 64 + lane;
  const float* ps = ssb + (size_t)(wv < CW ? h : 0) * ls;
  float acc = 0.0f;
  for (uint32_t ch = 0; ch < nch; ++ch) {
    // chunk ch's copies (issued after the scores or two chunks back) have
    // landed and every wave is done with chunk ch - 1, whose buffer takes
    // chunk ch + 1 (copied by the waves without a chain)
    wait_vm0();
    __syncthreads();
    if (wv >= CW && ch > 0 && ch + 1 < nch)
      for (uint32_t dd = wv - CW; dd < HD; dd += NW - CW) stage_row(ch + 1, dd);
    if (wv < CW) {
      const uint32_t jc = ch * C;
      acc = mix_dpp(ps + jc, VL + (size_t)(ch & 1) * HD * S + (size_t)d * S,
                    std::min(C, lc - jc), acc);
    }
  }
  wait_vm0();  // no copy still in flight when the workgroup ends (lc = 0)
  if (FUSE && nch == 0) __syncthreads();  // the divide's p_pos, with no chunk loop
  if (FUSE && wv < CW) {
    const float pr = ps[pos] * vself[d];
    acc = acc + pr;
  }
  if (wv < CW) out[(size_t)r * nh * HD + (size_t)(qh0 + h) * HD + d] = acc;
}

// ---------------------------------------------------------------------------
// Attention of prefill rows in tiles.  A tile is up to kAttQT rows of one
// sequence at consecutive positions p0 .. p0+nr-1 (built on the host); a
// workgroup takes one tile and the HPW = nh/nkv query heads of one KV head,
// P = kAttQT * HPW (row, head) pairs (pair a = row i * HPW + head h), and
// reads each K and V element of the kv head once for all of them, where the
// per-row kernel reads them once per row.  Each pair's arithmetic is the
// per-row kernel's, in the same order (sequential reduction order only):
//   scores  s_j = dot_seq(q, k_j) * scale, d ascending: K tiles of TK
//           positions in LDS, a thread carries PB pairs x 4 positions; the
//           scores go to a global scratch row per pair, the first-wins
//           maximum (NaN at position 0 wins) is kept on the way;
//   softmax the denominator as one strict chain per pair: waves 1..3 copy
//           stages of TE scores into LDS one stage ahead and turn them into
//           exp(s - max) in place (written back for the V-mix) while lanes
//           a < P of wave 0 continue their chains;
//   V-mix   out_d = fold_j (p_j * v_j[d]), j ascending, p_j = e_j / den:
//           V tiles and e tiles of TK positions in LDS (the next pair copied
//           while the current one is used), a thread carries PB3 pairs x 4
//           dims.
// LDS (floats): q [P][HD+4], then the phase regions (K tiles 2 x [HD][TK];
// e stages 2 x [P][TE+4]; V tiles 2 x [HD][TK+4] + e tiles 2 x [P][TK+4]),
// plus the per-pair maximum and denominator.
// ---------------------------------------------------------------------------
constexpr uint32_t kAttQT = kAttTileRows;  // rows per attention tile
constexpr uint32_t kAttTE = 128; // positions per softmax stage

template <uint32_t HPW, uint32_t HD, uint32_t TK>
struct AttTileCfg {
  static constexpr uint32_t P = kAttQT * HPW;
  static constexpr uint32_t QS = HD + 4;                 // q row stride
  static constexpr uint32_t PB = P * TK / 1024;          // pairs per thread, scores
  static constexpr uint32_t PB3 = P * HD / 1024;         // pairs per thread, V-mix
  static constexpr uint32_t ES = kAttTE + 4;             // e stage row stride
  static constexpr uint32_t VS = TK + 4;                 // V / e tile row stride
  static constexpr size_t region1 = 2 * (size_t)HD * TK;
  static constexpr size_t region2 = 2 * (size_t)P * ES;
  static constexpr size_t region3 = 2 * (size_t)HD * VS + 2 * (size_t)P * VS;
  static constexpr size_t region = region1 > region2 ? (region1 > region3 ? region1 : region3)
                                                     : (region2 > region3 ? region2 : region3);
  static constexpr size_t floats = (size_t)P * QS + region + 2 * P;
  static_assert(P * TK % 1024 == 0 && P * HD % 1024 == 0, "thread blocking");
  static_assert(P <= 64, "one denominator lane per pair in wave 0");
};

// n positions of `rows` rows (row stride `gstride` floats in global memory,
// starting at src) into LDS rows of stride `lstride` at dst, 16 bytes per
// lane with global_load_lds_dwordx4, one wave instruction per 256 positions
// of a row; waves [w0, w0 + nw) issue the rows w0-relative round-robin.
__device__ __forceinline__ void copy_rows_lds(float* dst, uint32_t lstride, const float* src,
                                              size_t gstride, uint32_t rows, uint32_t n,
                                              uint32_t w0, uint32_t nw) {
  const uint32_t n4 = (n + 3) >> 2, lane = threadIdx.x & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (w < w0 || w >= w0 + nw) return;
  for (uint32_t r = w - w0; r < rows; r += nw)
    for (uint32_t q0 = 0; q0 < n4; q0 += 64)
      if (q0 + lane < n4)
        lds_load16(reinterpret_cast<const v4*>(src + r * gstride) + q0 + lane,
                   reinterpret_cast<v4*>(dst + (size_t)r * lstride) + q0);
}

template <uint32_t HPW, uint32_t HD, uint32_t TK>
__global__ __launch_bounds__(256) void k_attention_tiles(
    const float* __restrict__ q, const float* __restrict__ kc, const float* __restrict__ vc,
    const AttTile* __restrict__ tiles, uint32_t nh, uint32_t max_pos, uint64_t seq_stride,
    float scale, float* out, float* scratch, uint32_t ls) {
  using C = AttTileCfg<HPW, HD, TK>;
  constexpr uint32_t P = C::P, QS = C::QS, PB = C::PB, PB3 = C::PB3, ES = C::ES, VS = C::VS;
  extern __shared__ v4 sh4[];
  float* sh = reinterpret_cast<float*>(sh4);
  float* qs = sh;                                  // [P][QS]
  float* reg = qs + (size_t)P * QS;                // phase region
  float* smx = reg + C::region;                    // [P] maxima
  float* sden = smx + P;                           // [P] denominators
  const AttTile tl = tiles[blockIdx.x];
  const uint32_t g = blockIdx.y, qh0 = g * HPW, nkv = nh / HPW, kvh = g;
  const uint32_t t = threadIdx.x, wv = t >> 6, lane = t & 63;
  const uint32_t npair = tl.nr * HPW, len_max = tl.p0 + tl.nr;
  float* S = scratch + ((size_t)blockIdx.x * nkv + g) * P * ls;  // [P][ls] scores, then exps
  const size_t sb = (size_t)tl.seq * seq_stride + (size_t)kvh * HD * max_pos;
  const float* kb = kc + sb;
  const float* vb = vc + sb;
  auto pair_len = [=](uint32_t a) { return tl.p0 + a / HPW + 1; };
  // q of every pair (rows past nr: zero, never stored)
  for (uint32_t i = t; i < P * HD; i += 256) {
    const uint32_t a = i / HD, d = i - a * HD, ri = a / HPW, h = a - ri * HPW;
    qs[a * QS + d] = a < npair ? q[(size_t)(tl.row0 + ri) * nh * HD + (size_t)(qh0 + h) * HD + d]
                               : 0.0f;
  }
  // ---- scores ------------------------------------------------------------
  constexpr uint32_t TPR = TK / 4;  // threads per pair group (4 positions each)
  const uint32_t pg = t / TPR, jg = t - pg * TPR;
  Pick best[PB];
  bool nan0[PB];
#pragma unroll
  for (uint32_t u = 0; u < PB; ++u) {
    best[u] = Pick{0.0f, UINT32_MAX};
    nan0[u] = false;
  }
  const uint32_t nkt = (len_max + TK - 1) / TK;
  float* kt0 = reg;
  auto kt = [=](uint32_t i) { return kt0 + (size_t)(i & 1) * HD * TK; };
  auto copy_k = [=](uint32_t i) {
    const uint32_t j0 = i * TK, n = min(TK, len_max - j0);
    // rows of TK floats back to back: a wave instruction covers 64 / (TK/4) rows
    const uint32_t n4 = (n + 3) >> 2, rows_per = 64 / (TK / 4);
    float* dst = kt(i);
    for (uint32_t r0 = wv * rows_per; r0 < HD; r0 += 4 * rows_per) {
      const uint32_t r = r0 + lane / (TK / 4), qq = lane % (TK / 4);
      if (r < HD && qq < n4)
        lds_load16(reinterpret_cast<const v4*>(kb + (size_t)r * max_pos + j0) + qq,
                   reinterpret_cast<v4*>(dst + (size_t)r0 * TK));
    }
  };
  copy_k(0);
  for (uint32_t i = 0; i < nkt; ++i) {
    wait_vm0();
    __syncthreads();
    if (i + 1 < nkt) copy_k(i + 1);
    const float* k = kt(i);
    float acc[PB][4];
#pragma unroll
    for (uint32_t u = 0; u < PB; ++u)
#pragma unroll
      for (uint32_t v = 0; v < 4; ++v) acc[u][v] = 0.0f;
#pragma unroll 2
    for (uint32_t d4 = 0; d4 < HD; d4 += 4) {
      v4 qv[PB], kk[4];
#pragma unroll
      for (uint32_t u = 0; u < PB; ++u)
        qv[u] = *reinterpret_cast<const v4*>(qs + (size_t)(pg * PB + u) * QS + d4);
#pragma unroll
      for (uint32_t e = 0; e < 4; ++e)
        kk[e] = *reinterpret_cast<const v4*>(k + (size_t)(d4 + e) * TK + 4 * jg);
#pragma unroll
      for (uint32_t e = 0; e < 4; ++e)
#pragma unroll
        for (uint32_t u = 0; u < PB; ++u) {
          float p;
          p = qv[u][e] * kk[e].x; acc[u][0] = acc[u][0] + p;
          p = qv[u][e] * kk[e].y; acc[u][1] = acc[u][1] + p;
          p = qv[u][e] * kk[e].z; acc[u][2] = acc[u][2] + p;
          p = qv[u][e] * kk[e].w; acc[u][3] = acc[u][3] + p;
        }
    }
#pragma unroll
    for (uint32_t u = 0; u < PB; ++u) {
      const uint32_t a = pg * PB + u;
      if (a < npair) {
        const uint32_t len = pair_len(a);
#pragma unroll
        for (uint32_t v = 0; v < 4; ++v) {
          const uint32_t j = i * TK + 4 * jg + v;
          if (j < len) {
            const float s = acc[u][v] * scale;
            S[(size_t)a * ls + j] = s;
            if (s == s) best[u] = pick2(best[u], Pick{s, j});
            else if (j == 0) nan0[u] = true;
          }
        }
      }
    }
  }
  // maxima: the TPR threads of a pair group are consecutive lanes of one wave
#pragma unroll
  for (uint32_t u = 0; u < PB; ++u) {
    Pick b = best[u];
    uint32_t n0 = nan0[u] ? 1u : 0u;
    for (uint32_t off = TPR / 2; off > 0; off >>= 1) {
      Pick o;
      o.v = __shfl_xor(b.v, off, 64);
      o.i = __shfl_xor(b.i, off, 64);
      b = pick2(b, o);
      n0 |= __shfl_xor(n0, off, 64);
    }
    const uint32_t a = pg * PB + u;
    if (jg == 0 && a < P) smx[a] = n0 ? __builtin_nanf("") : b.v;
  }
  // ---- softmax denominators ---------------------------------------------
  // the scores reach global memory, and no stale copy stays in this CU's
  // cache, before they are read back (agent-scope fence: release + acquire)
  __threadfence();
  __syncthreads();
  // a NaN at position 0 wins with its own bits: re-read the score
  if (t < npair && smx[t] != smx[t]) smx[t] = S[(size_t)t * ls];
  const uint32_t nst = (len_max + kAttTE - 1) / kAttTE;
  float* es0 = reg;
  auto es = [=](uint32_t i) { return es0 + (size_t)(i & 1) * P * ES; };
  // waves 1..3: copy stage i of every pair's scores and exponentiate it in
  // place, each wave on the pair rows it copied
  auto load_stage = [=](uint32_t i) {
    const uint32_t j0 = i * kAttTE, n = min(kAttTE, len_max - j0);
    copy_rows_lds(es(i), ES, S + j0, ls, npair, n, 1, 3);
  };
  auto exp_stage = [=](uint32_t i) {
    const uint32_t j0 = i * kAttTE;
    float* st = es(i);
    for (uint32_t a = wv - 1; a < npair; a += 3) {
      const uint32_t len = pair_len(a);
      if (j0 >= len) continue;
      const uint32_t n = min(kAttTE, len - j0);
      const float mx = smx[a];
      for (uint32_t j = lane; j < n; j += 64) {
        const float dlt = st[(size_t)a * ES + j] - mx;
        const float e = exp_pinned(dlt);
        st[(size_t)a * ES + j] = e;
        S[(size_t)a * ls + j0 + j] = e;
      }
    }
  };
  __syncthreads();
  if (wv >= 1) {
    load_stage(0);
    wait_vm0();
    exp_stage(0);
  }
  __syncthreads();
  float den = 0.0f;
  for (uint32_t i = 0; i < nst; ++i) {
    // lanes a < npair of wave 0 chain stage i; waves 1..3 prepare stage i+1
    // in the other buffer (its stage i-1 was chained before this barrier)
    if (wv == 0) {
      if (lane < npair) {
        const uint32_t j0 = i * kAttTE, len = pair_len(lane);
        if (j0 < len) den = chain_lds(es(i) + (size_t)lane * ES, min(kAttTE, len - j0), den);
      }
    } else if (i + 1 < nst) {
      load_stage(i + 1);
      wait_vm0();
      exp_stage(i + 1);
    }
    __syncthreads();
  }
  if (wv == 0 && lane < npair) sden[lane] = den;
  // the exps written by waves 1..3 reach global memory before the V-mix
  // reads them back through the async copies
  __threadfence();
  __syncthreads();
  // ---- V-mix --------------------------------------------------------------
  const uint32_t dg = t % (HD / 4), pg3 = t / (HD / 4);
  float* vt0 = reg;                                // 2 x [HD][VS]
  float* et0 = reg + 2 * (size_t)HD * VS;          // 2 x [P][VS]
  auto vt = [=](uint32_t i) { return vt0 + (size_t)(i & 1) * HD * VS; };
  auto et = [=](uint32_t i) { return et0 + (size_t)(i & 1) * P * VS; };
  auto copy_ve = [=](uint32_t i) {
    const uint32_t j0 = i * TK, n = min(TK, len_max - j0);
    copy_rows_lds(vt(i), VS, vb + j0, max_pos, HD, n, 0, 4);
    copy_rows_lds(et(i), VS, S + j0, ls, npair, n, 0, 4);
  };
  float acc3[PB3][4];
#pragma unroll
  for (uint32_t u = 0; u < PB3; ++u)
#pragma unroll
    for (uint32_t v = 0; v < 4; ++v) acc3[u][v] = 0.0f;
  copy_ve(0);
  for (uint32_t i = 0; i < nkt; ++i) {
    wait_vm0();
    __syncthreads();
    // p_j = e_j / den in place (main.rs softmax: true divide)
    {
      const uint32_t j0 = i * TK;
      float* e = et(i);
      for (uint32_t x = t; x < npair * TK; x += 256) {
        const uint32_t a = x / TK, j = x - a * TK;
        if (j0 + j < pair_len(a)) {
          const float pj = e[(size_t)a * VS + j] / sden[a];
          e[(size_t)a * VS + j] = pj;
        }
      }
    }
    __syncthreads();
    if (i + 1 < nkt) copy_ve(i + 1);
    const float* v = vt(i);
    const float* e = et(i);
    const uint32_t j0 = i * TK, n = min(TK, len_max - j0);
    // positions of this tile each of the thread's pairs sees; the common
    // 4-aligned part reads each V group once for all the pairs
    uint32_t m[PB3], mall = n;
#pragma unroll
    for (uint32_t u = 0; u < PB3; ++u) {
      const uint32_t a = pg3 * PB3 + u;
      const uint32_t len = a < npair ? pair_len(a) : 0;
      m[u] = len > j0 ? min(n, len - j0) : 0;
      mall = min(mall, m[u]);
    }
    const uint32_t m4 = mall & ~3u;
#pragma unroll 2
    for (uint32_t j = 0; j < m4; j += 4) {
      v4 vv[4];
#pragma unroll
      for (uint32_t dd = 0; dd < 4; ++dd)
        vv[dd] = *reinterpret_cast<const v4*>(v + (size_t)(4 * dg + dd) * VS + j);
#pragma unroll
      for (uint32_t u = 0; u < PB3; ++u) {
        const v4 pp = *reinterpret_cast<const v4*>(e + (size_t)(pg3 * PB3 + u) * VS + j);
#pragma unroll
        for (uint32_t dd = 0; dd < 4; ++dd) {
          float p;
          p = pp.x * vv[dd].x; acc3[u][dd] = acc3[u][dd] + p;
          p = pp.y * vv[dd].y; acc3[u][dd] = acc3[u][dd] + p;
          p = pp.z * vv[dd].z; acc3[u][dd] = acc3[u][dd] + p;
          p = pp.w * vv[dd].w; acc3[u][dd] = acc3[u][dd] + p;
        }
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < PB3; ++u) {
      const float* pr = e + (size_t)(pg3 * PB3 + u) * VS;
      for (uint32_t j = m4; j < m[u]; ++j) {
#pragma unroll
        for (uint32_t dd = 0; dd < 4; ++dd) {
          const float p = pr[j] * v[(size_t)(4 * dg + dd) * VS + j];
          acc3[u][dd] = acc3[u][dd] + p;
        }
      }
    }
  }
#pragma unroll
  for (uint32_t u = 0; u < PB3; ++u) {
    const uint32_t a = pg3 * PB3 + u;
    if (a < npair) {
      const uint32_t ri = a / HPW, h = a - ri * HPW;
      float* o = out + (size_t)(tl.row0 + ri) * nh * HD + (size_t)(qh0 + h) * HD + 4 * dg;
#pragma unroll
      for (uint32_t dd = 0; dd < 4; ++dd) o[dd] = acc3[u][dd];
    }
  }
}

__global__ void k_gather_rows(const float* __restrict__ src, const uint32_t* __restrict__ idx,
                              uint32_t width, float* dst) {
  const uint32_t r = blockIdx.x;
  const float* s = src + (size_t)idx[r] * width;
  for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) dst[(size_t)r * width + i] = s[i];
}

__global__ void k_advance_rows(uint32_t* pos, uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) pos[i] = pos[i] + 1u;
}

__global__ __launch_bounds__(1024) void k_argmax_rows(const float* __restrict__ v,
                                                      uint32_t width, uint32_t* out) {
  __shared__ Pick red[16];
  const float* row = v + (size_t)blockIdx.x * width;
  Pick best = {0.0f, UINT32_MAX};
  for (uint32_t i = threadIdx.x; i < width; i += blockDim.x) {
    const float x = row[i];
    if (x == x) best = pick2(best, Pick{x, i});
  }
  best = pick_block(best, red);
  if (threadIdx.x == 0) {
    const float v0 = row[0];
    out[blockIdx.x] = (v0 != v0 || best.i == UINT32_MAX) ? 0u : best.i;
  }
}

}  // namespace

template <bool DUAL, bool NORM, uint32_t CB>
hipError_t launch_bgemm_t(const BgemmArgs& a, dim3 grid, size_t lds, hipStream_t st) {
  hipLaunchKernelGGL((k_bgemm<DUAL, NORM, CB>), grid, dim3(kT), lds, st, a);
  return hipGetLastError();
}

// The LDS limit of every k_bgemm and k_attention_kv variant, set at the
// first launch of any (a forward launches a GEMM before its first
// attention), so that no attribute call happens later, e.g. inside a graph
// capture.
hipError_t rows_configure() {
  const void* fns[20] = {reinterpret_cast<const void*>(&k_bgemm<false, false, 1>),
                         reinterpret_cast<const void*>(&k_bgemm16<false, false>),
                         reinterpret_cast<const void*>(&k_bgemm16<false, true>),
                         reinterpret_cast<const void*>(&k_bgemm16<true, false>),
                         reinterpret_cast<const void*>(&k_bgemm16<true, true>),
                         reinterpret_cast<const void*>(&k_bgemm<false, true, 1>),
                         reinterpret_cast<const void*>(&k_bgemm<true, false, 1>),
                         reinterpret_cast<const void*>(&k_bgemm<true, true, 1>),
                         reinterpret_cast<const void*>(&k_bgemm<false, false, 2>),
                         reinterpret_cast<const void*>(&k_bgemm<true, false, 2>),
                         reinterpret_cast<const void*>(&k_attention_kv<1, 64, false>),
                         reinterpret_cast<const void*>(&k_attention_kv<2, 64, false>),
                         reinterpret_cast<const void*>(&k_attention_kv<3, 64, false>),
                         reinterpret_cast<const void*>(&k_attention_kv<1, 128, false>),
                         reinterpret_cast<const void*>(&k_attention_kv<2, 128, false>),
                         reinterpret_cast<const void*>(&k_attention_kv<1, 64, true>),
                         reinterpret_cast<const void*>(&k_attention_kv<2, 64, true>),
                         reinterpret_cast<const void*>(&k_attention_kv<3, 64, true>),
                         reinterpret_cast<const void*>(&k_attention_kv<1, 128, true>),
                         reinterpret_cast<const void*>(&k_attention_kv<2, 128, true>)};
  for (const void* f : fns) {
    hipError_t e = ensure_dynamic_lds(f, kBgemmLdsBig);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// CIS2_BGEMM_CB=1 keeps one batch row per thread on every grid (for A/B
// timing of the two-row form; the results are the same bits either way).
static bool bgemm_cb_allowed() {
  static const bool allowed = [] {
    const char* e = std::getenv("CIS2_BGEMM_CB");
    return !(e && e[0] == '1' && e[1] == 0);
  }();
  return allowed;
}

// CIS2_BGEMM16=0 keeps every batched GEMM on k_bgemm (for A/B timing; the
// results are the same bits either way).
static bool bgemm16_allowed() {
  const char* e = std::getenv("CIS2_BGEMM16");
  return !(e && e[0] == '0' && e[1] == 0);
}

// k_bgemm16 for sequential-order GEMMs whose W blocks have 8 or 16 rows and
// whose segments are whole 16-output tiles.
static hipError_t launch_bgemm16(const BgemmSeg* segs, uint32_t nseg, uint32_t n,
                                 const BgemmOpts& o, int ncu, hipStream_t st) {
  const BgemmSeg& s0 = segs[0];
  BgemmArgs a = {};
  a.blk0[0] = 0;
  for (uint32_t i = 0; i < nseg; ++i) {
    a.s[i] = segs[i];
    a.blk0[i + 1] = a.blk0[i] + segs[i].M / 16;
  }
  for (uint32_t i = nseg; i < kMaxSegs; ++i) {
    a.s[i] = s0;
    a.blk0[i + 1] = a.blk0[nseg];
  }
  a.nseg = nseg;
  a.n = n;
  a.TB = 16;
  a.tree = 0;
  a.W2 = o.W2;
  a.nw = o.norm_w;
  a.eps = o.eps;
  const uint32_t S = o.W2 ? 2 : 1, NW = o.norm_w ? 1 : 0, nblk = 16 / s0.R;
  const uint64_t wgs = (uint64_t)a.blk0[nseg] * ((n + 15) / 16);
  const uint32_t budget = wgs <= (uint64_t)ncu ? kBgemmLdsBig : kBgemmLds;
  // LDS groups: S * nblk * (q * R + 8) + NW * q + 16 * (q + 1) + slack
  const uint32_t fixed = 8 * S * nblk + 16 + b16_slack(s0.R);
  const uint32_t q_fit = (budget / 16 - fixed) / (16 * S + NW + 16);
  uint32_t KC = std::min((q_fit * 4) & ~31u, 1024u);
  if (KC == 0) return hipErrorInvalidValue;
  const uint32_t K32 = (s0.K + 31) & ~31u;
  if (KC > K32) KC = K32;
  a.KC = KC;
  const size_t q = KC / 4;
  const size_t lds =
      ((size_t)S * nblk * (q * s0.R + 8) + NW * q + 16 * (q + 1) + b16_slack(s0.R)) * 16;
  const dim3 grid(a.blk0[nseg], (n + 15) / 16);
  if (o.W2)
    hipLaunchKernelGGL((o.norm_w ? k_bgemm16<true, true> : k_bgemm16<true, false>), grid,
                       dim3(kT), lds, st, a);
  else
    hipLaunchKernelGGL((o.norm_w ? k_bgemm16<false, true> : k_bgemm16<false, false>), grid,
                       dim3(kT), lds, st, a);
  return hipGetLastError();
}

hipError_t launch_bgemm_multi(const BgemmSeg* segs, uint32_t nseg, uint32_t n,
                              const BgemmOpts& o, hipStream_t st) {
  if (n == 0) return hipSuccess;
  if (nseg == 0 || nseg > kMaxSegs || (o.W2 && nseg != 1)) return hipErrorInvalidValue;
  {
    hipError_t e = rows_configure();
    if (e != hipSuccess) return e;
  }
  const BgemmSeg& s0 = segs[0];
  if (s0.K % 4 || s0.ldx % 4 || s0.R == 0 || s0.R > kT) return hipErrorInvalidValue;
  const int ncu = device_cu_count();
  {
    bool tiles = !o.tree && (s0.R == 8 || s0.R == 16) && bgemm16_allowed();
    for (uint32_t i = 0; i < nseg && tiles; ++i)
      tiles = segs[i].M % 16 == 0 && segs[i].R == s0.R && segs[i].K == s0.K &&
              segs[i].X == s0.X && segs[i].ldx == s0.ldx;
    if (tiles) return launch_bgemm16(segs, nseg, n, o, ncu, st);
  }
  BgemmArgs a = {};
  a.blk0[0] = 0;
  for (uint32_t i = 0; i < nseg; ++i) {
    const BgemmSeg& s = segs[i];
    if (s.M == 0 || s.K != s0.K || s.R != s0.R || s.X != s0.X || s.ldx != s0.ldx)
      return hipErrorInvalidValue;
    a.s[i] = s;
    a.blk0[i + 1] = a.blk0[i] + (s.M + s.R - 1) / s.R;
  }
  for (uint32_t i = nseg; i < kMaxSegs; ++i) {
    a.s[i] = s0;
    a.blk0[i + 1] = a.blk0[nseg];
  }
  a.nseg = nseg;
  a.n = n;
  a.TB = kT / s0.R;
  a.tree = o.tree ? 1u : 0u;
  a.W2 = o.W2;
  a.nw = o.norm_w;
  a.eps = o.eps;
  const uint32_t S = o.W2 ? 2 : 1;
  const uint64_t wgs = (uint64_t)a.blk0[nseg] * ((n + a.TB - 1) / a.TB);
  // grids of many workgroups per CU (prefill) give each thread two batch
  // rows, so that one W read from LDS feeds two chains
  const uint32_t CB = (!o.norm_w && !o.tree && wgs >= 8ull * ncu && bgemm_cb_allowed()) ? 2 : 1;
  const uint32_t NB = a.TB * CB;
  // a grid of at most one workgroup per CU may take most of a CU's LDS
  // (fewer K chunks, each a full round trip); larger grids keep two
  // workgroups per CU, so that up to two per CU all run at once
  const uint32_t budget = wgs <= (uint64_t)ncu ? kBgemmLdsBig : kBgemmLds;
  // largest chunk (a multiple of 32 k) whose W slices, X rows and norm
  // weights fit
  const uint32_t NW = o.norm_w ? 1 : 0;
  const uint32_t q_fit = (budget / 16 - NB) / (S * s0.R + NB + NW);
  uint32_t KC = (q_fit * 4) & ~31u;
  if (KC == 0) return hipErrorInvalidValue;
  const uint32_t K32 = (s0.K + 31) & ~31u;
  if (KC > K32) KC = K32;
  a.KC = KC;
  const size_t lds = ((size_t)(KC / 4) * (s0.R * S + NW) + (size_t)NB * (KC / 4 + 1)) * 16;
  const dim3 grid(a.blk0[nseg], (n + NB - 1) / NB);
  if (CB == 2) return o.W2 ? launch_bgemm_t<true, false, 2>(a, grid, lds, st)
                           : launch_bgemm_t<false, false, 2>(a, grid, lds, st);
  if (o.W2) return o.norm_w ? launch_bgemm_t<true, true, 1>(a, grid, lds, st)
                            : launch_bgemm_t<true, false, 1>(a, grid, lds, st);
  return o.norm_w ? launch_bgemm_t<false, true, 1>(a, grid, lds, st)
                  : launch_bgemm_t<false, false, 1>(a, grid, lds, st);
}

hipError_t launch_bgemm(const BgemmSeg& s, uint32_t n, bool tree, hipStream_t st) {
  BgemmOpts o;
  o.tree = tree;
  return launch_bgemm_multi(&s, 1, n, o, st);
}

hipError_t launch_embed_rows(const float* E, RowsDesc rows, uint32_t H, uint32_t vocab,
                             float* h, uint32_t* err, hipStream_t st) {
  if (rows.n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_embed_rows, dim3(rows.n), dim3(kT), 0, st, E, rows, H, vocab, h, err);
  return hipGetLastError();
}

hipError_t launch_rope_store_rows(float* q, float* k, const float* v, const float* rope_cs,
                                  RowsDesc rows, uint32_t nh, uint32_t nkv, uint32_t hd,
                                  uint32_t max_pos, float* kc, float* vc, uint64_t seq_stride,
                                  hipStream_t st) {
  if (rows.n == 0) return hipSuccess;
  if (hd % 2) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rope_store_rows, dim3(rows.n), dim3(kT), 0, st, q, k, v, rope_cs, rows,
                     nh, nkv, hd, max_pos, kc, vc, seq_stride);
  return hipGetLastError();
}

// CIS2_ATT_KV=0 keeps decode rows on the one-head-per-workgroup kernel;
// CIS2_ATT_KV=<n> caps the V chunk at n positions (rounded down to a
// multiple of 64), so that short rows run through the chunk ring too.  For
// A/B timing and tests: the results are the same bits either way.
static size_t kv_attention_cap() {
  const char* e = std::getenv("CIS2_ATT_KV");
  if (!e || !*e) return SIZE_MAX;
  return (size_t)std::strtoul(e, nullptr, 10) / 64 * 64;
}

// Decode rows (rows x kv heads < 4 x CUs), head_dim 64 or 128: one
// workgroup per (row, KV head) with the V rows staged in LDS, in chunks of C
// positions (two buffers: the longest row in one pass of each when they
// fit).  A grid of at most one workgroup per CU may take most of the LDS,
// larger ones half.  C = 0: another kernel.
struct KvPlan {
  size_t C = 0, shmem = 0;
  uint32_t group = 0, ls = 0;
};
static hipError_t kv_plan(uint32_t n, uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_len,
                          KvPlan* p) {
  *p = KvPlan{};
  if (nkv == 0 || nh % nkv) return hipErrorInvalidValue;
  const uint32_t group = nh / nkv;
  const int ncu = device_cu_count();
  const uint64_t wgs_kv = (uint64_t)n * nkv;
  // instances for groups of up to 3 heads at head_dim 64 and 2 at 128 (a
  // group of 4 at head_dim 64 needed more registers than a wave has and
  // spilled to scratch; such models take the per-row kernel)
  if (!(wgs_kv < 4 * (uint64_t)ncu && ((hd == 64 && group <= 3) || (hd == 128 && group <= 2))))
    return hipSuccess;
  hipError_t e = rows_configure();
  if (e != hipSuccess) return e;
  const size_t ls = ((size_t)max_len + 3) / 4 * 4, nbs = (ls + 31) / 32;
  const size_t fixed =
      (group * hd + 2 * hd + group * ls + ((group * nbs + 3) & ~(size_t)3)) * 4;
  const size_t budget = wgs_kv <= (uint64_t)ncu ? kBgemmLdsBig : kBgemmLds;
  const size_t c_need =
      std::min<size_t>((((size_t)max_len + 1) / 2 + 63) & ~(size_t)63, 256);
  size_t c_fit = 0;
  if (budget > fixed + kKvSlack * 4 + 8 * hd * 68)
    c_fit = ((budget - fixed - kKvSlack * 4) / (8 * hd) - 4) & ~(size_t)63;
  const size_t C = std::min(std::min(c_need, c_fit), kv_attention_cap());
  if (C < 64) return hipSuccess;
  p->C = C;
  p->shmem = fixed + 2 * hd * (C + 4) * 4 + kKvSlack * 4;
  p->group = group;
  p->ls = (uint32_t)ls;
  return hipSuccess;
}
static hipError_t launch_kv(const KvPlan& kp, bool fuse, const float* q, float* kc, float* vc,
                            RowsDesc rows, uint32_t nh, uint32_t hd, uint32_t max_pos,
                            uint64_t seq_stride, float scale, float* out, bool tree,
                            const KvFuse& fz, hipStream_t st) {
  const dim3 grid(rows.n, nh / kp.group);
  const uint32_t tr = tree ? 1u : 0u, c32 = (uint32_t)kp.C;
#define CIS2_ATT_KV(H, D)                                                                     \
  do {                                                                                        \
    if (fuse)                                                                                 \
      hipLaunchKernelGGL((k_attention_kv<H, D, true>), grid, dim3(kKvT), kp.shmem, st, q, kc, \
                         vc, rows, nh, max_pos, seq_stride, scale, out, tr, kp.ls, c32, fz);  \
    else                                                                                      \
      hipLaunchKernelGGL((k_attention_kv<H, D, false>), grid, dim3(kKvT), kp.shmem, st, q,    \
                         kc, vc, rows, nh, max_pos, seq_stride, scale, out, tr, kp.ls, c32,   \
                         fz);                                                                 \
  } while (0)
  if (hd == 64) {
    switch (kp.group) {
      case 1: CIS2_ATT_KV(1, 64); break;
      case 2: CIS2_ATT_KV(2, 64); break;
      default: CIS2_ATT_KV(3, 64);
    }
  } else {
    if (kp.group == 1) CIS2_ATT_KV(1, 128);
    else CIS2_ATT_KV(2, 128);
  }
#undef CIS2_ATT_KV
  return hipGetLastError();
}

hipError_t launch_rope_attention_rows(const float* q, const float* k, const float* v,
                                      const float* rope_cs, RowsDesc rows, uint32_t max_len,
                                      uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_pos,
                                      float* kc, float* vc, uint64_t seq_stride, float scale,
                                      float* out, bool tree, hipStream_t st) {
  if (rows.n == 0) return hipSuccess;
  if (max_len == 0 || max_len > max_pos || max_pos % 4 || hd % 2) return hipErrorInvalidValue;
  KvPlan kp;
  hipError_t e = kv_plan(rows.n, nh, nkv, hd, max_len, &kp);
  if (e != hipSuccess) return e;
  if (!kp.C) return hipErrorNotSupported;
  const KvFuse fz{k, v, rope_cs, nkv};
  return launch_kv(kp, true, q, kc, vc, rows, nh, hd, max_pos, seq_stride, scale, out, tree, fz,
                   st);
}

hipError_t launch_attention_rows(const float* q, const float* kc, const float* vc,
                                 RowsDesc rows, uint32_t max_len, uint32_t nh, uint32_t nkv,
                                 uint32_t hd, uint32_t max_pos, uint64_t seq_stride, float scale,
                                 float* out, bool tree, hipStream_t st) {
  if (rows.n == 0) return hipSuccess;
  if (nkv == 0 || nh % nkv || max_len == 0 || max_len > max_pos || max_pos % 4)
    return hipErrorInvalidValue;
  const uint32_t group = nh / nkv;
  const size_t hd4 = ((size_t)hd + 3) / 4 * 4, ls = ((size_t)max_len + 3) / 4 * 4;
  auto lds_of = [&](uint32_t hpw) { return hpw * (hd4 + ls + (ls + 31) / 32) * sizeof(float); };
  const int ncu = device_cu_count();
  const uint64_t wgs_kv = (uint64_t)rows.n * nkv;
  const uint32_t tr = tree ? 1u : 0u, ls32 = (uint32_t)ls;
  {
    KvPlan kp;
    hipError_t e = kv_plan(rows.n, nh, nkv, hd, max_len, &kp);
    if (e != hipSuccess) return e;
    if (kp.C) return launch_kv(kp, false, q, const_cast<float*>(kc), const_cast<float*>(vc),
                               rows, nh, hd, max_pos, seq_stride, scale, out, tree, KvFuse{}, st);
  }
  // Otherwise, few rows: one head per workgroup, for the most workgroups.
  // Many rows: the most heads of one KV head (a divisor of the group) whose
  // LDS fits, so K and V are read once per group.
  uint32_t hpw = 1;
  if (wgs_kv >= 4 * (uint64_t)ncu) {
    for (uint32_t h = std::min(group, kMaxHeadsPerWg); h > 1; --h)
      if (group % h == 0 && lds_of(h) <= 60 * 1024) {
        hpw = h;
        break;
      }
  }
  const size_t shmem = lds_of(hpw);
  if (shmem > 60 * 1024) return hipErrorInvalidValue;
  const dim3 grid(rows.n, nh / hpw);
  switch (hpw) {
    case 4:
      hipLaunchKernelGGL(k_attention_rows<4>, grid, dim3(kAttT), shmem, st, q, kc, vc, rows, nh,
                         nkv, hd, max_pos, seq_stride, scale, out, tr, ls32);
      break;
    case 3:
      hipLaunchKernelGGL(k_attention_rows<3>, grid, dim3(kAttT), shmem, st, q, kc, vc, rows, nh,
                         nkv, hd, max_pos, seq_stride, scale, out, tr, ls32);
      break;
    case 2:
      hipLaunchKernelGGL(k_attention_rows<2>, grid, dim3(kAttT), shmem, st, q, kc, vc, rows, nh,
                         nkv, hd, max_pos, seq_stride, scale, out, tr, ls32);
      break;
    default:
      hipLaunchKernelGGL(k_attention_rows<1>, grid, dim3(kAttT), shmem, st, q, kc, vc, rows, nh,
                         nkv, hd, max_pos, seq_stride, scale, out, tr, ls32);
  }
  return hipGetLastError();
}

hipError_t launch_gather_rows(const float* src, const uint32_t* idx, uint32_t n, uint32_t width,
                              float* dst, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_gather_rows, dim3(n), dim3(kT), 0, st, src, idx, width, dst);
  return hipGetLastError();
}

hipError_t launch_advance_rows(uint32_t* pos, uint32_t n, hipStream_t st) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_advance_rows, dim3((n + kT - 1) / kT), dim3(kT), 0, st, pos, n);
  return hipGetLastError();
}

hipError_t launch_argmax_rows(const float* v, uint32_t n, uint32_t width, uint32_t* out,
                              hipStream_t st) {
  if (n == 0) return hipSuccess;
  if (width == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_argmax_rows, dim3(n), dim3(1024), 0, st, v, width, out);
  return hipGetLastError();
}


template <uint32_t HPW, uint32_t HD, uint32_t TK>
static hipError_t launch_att_tiles_t(const float* q, const float* kc, const float* vc,
                                     const AttTile* tiles, uint32_t ntiles, uint32_t nh,
                                     uint32_t max_pos, uint64_t seq_stride, float scale, float* out,
                                     float* scratch, uint32_t ls, hipStream_t st) {
  using C = AttTileCfg<HPW, HD, TK>;
  const size_t lds = C::floats * sizeof(float);
  hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&k_attention_tiles<HPW, HD, TK>), lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_attention_tiles<HPW, HD, TK>), dim3(ntiles, nh / HPW), dim3(256), lds, st,
                     q, kc, vc, tiles, nh, max_pos, seq_stride, scale, out, scratch, ls);
  return hipGetLastError();
}

bool attention_tiles_supported(uint32_t nh, uint32_t nkv, uint32_t hd) {
  if (nkv == 0 || nh % nkv) return false;
  const uint32_t g = nh / nkv;
  if (hd == 64) return g >= 1 && g <= 4;
  if (hd == 128) return g == 2 || g == 4;
  return false;
}

size_t attention_tiles_scratch_floats(uint32_t ntiles, uint32_t nh, uint32_t nkv,
                                      uint32_t max_len) {
  const size_t ls = ((size_t)max_len + 3) / 4 * 4;
  return (size_t)ntiles * nkv * kAttQT * (nh / nkv) * ls;
}

hipError_t launch_attention_tiles(const float* q, const float* kc, const float* vc,
                                  const AttTile* tiles, uint32_t ntiles, uint32_t max_len,
                                  uint32_t nh, uint32_t nkv, uint32_t hd, uint32_t max_pos,
                                  uint64_t seq_stride, float scale, float* out, float* scratch,
                                  hipStream_t st) {
  if (ntiles == 0) return hipSuccess;
  if (!attention_tiles_supported(nh, nkv, hd) || max_len == 0 || max_len > max_pos ||
      max_pos % 4)
    return hipErrorInvalidValue;
  const uint32_t g = nh / nkv, ls = (max_len + 3) / 4 * 4;
  if (hd == 64) {
    switch (g) {
      case 1: return launch_att_tiles_t<1, 64, 64>(q, kc, vc, tiles, ntiles, nh, max_pos, seq_stride, scale, out, scratch, ls, st);
      case 2: return launch_att_tiles_t<2, 64, 64>(q, kc, vc, tiles, ntiles, nh, max_pos, seq_stride, scale, out, scratch, ls, st);
      case 3: return launch_att_tiles_t<3, 64, 64>(q, kc, vc, tiles, ntiles, nh, max_pos, seq_stride, scale, out, scratch, ls, st);
      default: return launch_att_tiles_t<4, 64, 64>(q, kc, vc, tiles, ntiles, nh, max_pos, seq_stride, scale, out, scratch, ls, st);
    }
  }
  if (g == 2) return launch_att_tiles_t<2, 128, 32>(q, kc, vc, tiles, ntiles, nh, max_pos, seq_stride, scale, out, scratch, ls, st);
  return launch_att_tiles_t<4, 128, 32>(q, kc, vc, tiles, ntiles, nh, max_pos, seq_stride, scale, out, scratch, ls, st);
}

}  // namespace cis2
