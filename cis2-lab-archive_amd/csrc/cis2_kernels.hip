// cis2_kernels.hip — gfx950 kernels for the CIS-2 pinned-order fp32 forward
// pass.  Every reduction on the decode path is evaluated in the order the
// reference pins (code/cis2-fp/docs/CIS2_SPEC_v0.3.md §5): one lane owns one
// output and folds its terms strictly left to right; order-free reductions
// (max, argmax with lowest-index ties) use wavefront trees.
#include "cis2_device_math.hpp"
#include "cis2_kernels.hpp"

#include <algorithm>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include <float.h>
#include <string.h>

namespace cis2 {

size_t blocked_floats(uint32_t M, uint32_t K, uint32_t R) {
  size_t blocks = (M + R - 1) / R;
  return blocks * R * (size_t)K;
}

// ---------------------------------------------------------------------------
// GEMV: y[o] = fold_k (W[o,k] * x[k]) from acc = 0, one lane per row.
// code/cis2-fp/src/main.rs:228-243 (matvec -> dot_seq, math.rs:40-48);
// the C++ port's one-thread-per-row kernel is gpu/cis2_model.h:527-532.
// ---------------------------------------------------------------------------
struct GemvArgs {
  GemvSeg seg[4];
  uint32_t blk_start[5];
  int nseg;
  uint32_t tree;
};

// Tree order (code/cis2-fp/src/math.rs:60-125): per 32-wide k block the
// products are reduced by tree32, the block results folded from 0.
__device__ __forceinline__ float gemv_tree(const float* __restrict__ Wb,
                                           const float* __restrict__ x, uint32_t K, uint32_t R,
                                           uint32_t lane) {
  const float4* __restrict__ wp =
      reinterpret_cast<const float4*>(Wb) + (lane < R ? lane : R - 1);
  const float4* __restrict__ xp = reinterpret_cast<const float4*>(x);
  const uint32_t KG = K >> 2;
  float acc = 0.0f;
  for (uint32_t g0 = 0; g0 < KG; g0 += 8) {
    float l[32];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      float4 w = make_float4(0.0f, 0.0f, 0.0f, 0.0f), xv = w;
      if (g0 + j < KG) {
        w = wp[(size_t)(g0 + j) * R];
        xv = xp[g0 + j];
      }
      l[4 * j] = w.x * xv.x;
      l[4 * j + 1] = w.y * xv.y;
      l[4 * j + 2] = w.z * xv.z;
      l[4 * j + 3] = w.w * xv.w;
    }
    acc = acc + tree32(l);
  }
  return acc;
}

__device__ __forceinline__ float gemv_chain(const float* __restrict__ Wb,
                                            const float* __restrict__ x, uint32_t K,
                                            uint32_t R, uint32_t lane) {
  const float4* __restrict__ wp =
      reinterpret_cast<const float4*>(Wb) + (lane < R ? lane : R - 1);
  const float4* __restrict__ xp = reinterpret_cast<const float4*>(x);
  const uint32_t KG = K >> 2;
  float acc = 0.0f;
#pragma unroll 8
  for (uint32_t g = 0; g < KG; ++g) {
    float4 w = wp[(size_t)g * R];
    float4 xv = xp[g];
    float p;
    p = w.x * xv.x; acc = acc + p;
    p = w.y * xv.y; acc = acc + p;
    p = w.z * xv.z; acc = acc + p;
    p = w.w * xv.w; acc = acc + p;
  }
  return acc;
}

__global__ __launch_bounds__(64) void k_gemv(GemvArgs a) {
  uint32_t b = blockIdx.x;
  int s = 0;
  while (s + 1 < a.nseg && b >= a.blk_start[s + 1]) ++s;
  const GemvSeg g = a.seg[s];
  b -= a.blk_start[s];
  const uint32_t lane = threadIdx.x;
  const float* Wb = g.W + (size_t)b * g.R * g.K;
  float acc = a.tree ? gemv_tree(Wb, g.x, g.K, g.R, lane) : gemv_chain(Wb, g.x, g.K, g.R, lane);
  uint32_t row = b * g.R + lane;
  if (lane < g.R && row < g.M) {
    float r = acc;
    if (g.add) r = g.add_first ? (g.add[row] + acc) : (acc + g.add[row]);
    g.y[row] = r;
  }
}

hipError_t launch_gemv(const GemvSeg* segs, int nseg, hipStream_t s, bool tree) {
  if (nseg < 1 || nseg > 4) return hipErrorInvalidValue;
  GemvArgs a;
  a.tree = tree ? 1u : 0u;
  uint32_t total = 0;
  for (int i = 0; i < nseg; ++i) {
    if (segs[i].K % 4 != 0 || segs[i].M == 0 || segs[i].R == 0 || segs[i].R > 64)
      return hipErrorInvalidValue;
    a.seg[i] = segs[i];
    a.blk_start[i] = total;
    total += (segs[i].M + segs[i].R - 1) / segs[i].R;
  }
  a.blk_start[nseg] = total;
  a.nseg = nseg;
  hipLaunchKernelGGL(k_gemv, dim3(total), dim3(64), 0, s, a);
  return hipGetLastError();
}

// Gate and up rows of the same block in two waves of one workgroup, then
// hid = silu(gate) * up (code/cis2-fp/src/main.rs:480-487).
__global__ __launch_bounds__(128) void k_gate_up_silu(const float* __restrict__ Wg,
                                                      const float* __restrict__ Wu,
                                                      const float* __restrict__ x,
                                                      float* gate, float* up, float* hid,
                                                      uint32_t I, uint32_t H, uint32_t R,
                                                      uint32_t tree) {
  __shared__ float sg[64];
  const uint32_t b = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float* Wb = (w ? Wu : Wg) + (size_t)b * R * H;
  float acc = tree ? gemv_tree(Wb, x, H, R, lane) : gemv_chain(Wb, x, H, R, lane);
  const uint32_t row = b * R + lane;
  if (w == 0) {
    sg[lane] = acc;
    if (lane < R && row < I) gate[row] = acc;
  }
  __syncthreads();
  if (w == 1 && lane < R && row < I) {
    up[row] = acc;
    float sgl = silu_pinned(sg[lane]);
    hid[row] = sgl * acc;
  }
}

hipError_t launch_gate_up_silu(const float* Wg, const float* Wu, const float* x,
                               float* gate, float* up, float* hid, uint32_t I,
                               uint32_t H, uint32_t R, hipStream_t s, bool tree) {
  if (H % 4 != 0 || R == 0 || R > 64) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_gate_up_silu, dim3((I + R - 1) / R), dim3(128), 0, s, Wg, Wu, x,
                     gate, up, hid, I, H, R, tree ? 1u : 0u);
  return hipGetLastError();
}

__global__ void k_relayout(const float* __restrict__ src, float* __restrict__ dst,
                           uint32_t M, uint32_t K, uint32_t R, size_t total) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const size_t KG = K / 4;
  for (; i < total; i += stride) {
    size_t j = i & 3, q = i >> 2;
    size_t lane = q % R, rest = q / R;
    size_t g = rest % KG, b = rest / KG;
    size_t row = b * R + lane;
    dst[i] = row < M ? src[row * K + 4 * g + j] : 0.0f;
  }
}

hipError_t launch_relayout(const float* src, float* dst, uint32_t M, uint32_t K, uint32_t R,
                           hipStream_t s) {
  if (K % 4 != 0 || R == 0 || R > 64) return hipErrorInvalidValue;
  size_t total = blocked_floats(M, K, R);
  hipLaunchKernelGGL(k_relayout, dim3(2048), dim3(256), 0, s, src, dst, M, K, R, total);
  return hipGetLastError();
}

// BF16 -> F32 by the exact bit shift (code/cis2-fp/src/math.rs:33-35).
__global__ void k_widen(const uint16_t* __restrict__ src, uint32_t* __restrict__ dst,
                        uint64_t n) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) dst[i] = (uint32_t)src[i] << 16;
}

hipError_t launch_widen(const uint16_t* src, float* dst, uint64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_widen, dim3(2048), dim3(256), 0, s, src,
                     reinterpret_cast<uint32_t*>(dst), n);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Embedding gather (code/cis2-fp/src/main.rs:374-377).
// ---------------------------------------------------------------------------
__global__ void k_embed(const float* __restrict__ E, const uint32_t* tokp, float* h,
                        uint32_t H, uint32_t vocab, uint32_t* err) {
  uint32_t tok = *tokp;
  if (tok >= vocab) {
    if (threadIdx.x == 0 && blockIdx.x == 0) atomicOr(err, 1u);
    tok = 0;
  }
  const float* row = E + (size_t)tok * H;
  for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x)
    h[i] = row[i];
}

hipError_t launch_embed(const float* E, const uint32_t* tok, float* h, uint32_t H,
                        uint32_t vocab, uint32_t* err, hipStream_t s) {
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, s, E, tok, h, H, vocab, err);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RMSNorm (code/cis2-fp/src/main.rs:245-260; spec §8): squares materialised,
// one strict chain from 0, mean by a true divide, inv = 1/sqrt(mean+eps),
// out = (x*inv)*w.  Wave 0 runs the chain with every lane holding the same
// value; the other work is lane-parallel.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, const float* __restrict__ w,
                                                 float eps, uint32_t n, float* out,
                                                 uint32_t tree) {
  extern __shared__ float sq[];
  __shared__ float s_inv;
  const float* xv = x + (size_t)blockIdx.x * n;
  float* ov = out + (size_t)blockIdx.x * n;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    float v = xv[i];
    sq[i] = v * v;
  }
  __syncthreads();
  const uint32_t nb = (n + 31) / 32;
  if (tree) {
    // block partials by tree32 (code/cis2-fp/src/math.rs:60-125), stored
    // after the squares; thread t owns block t
    for (uint32_t t = threadIdx.x; t < nb; t += blockDim.x) {
      float l[32];
#pragma unroll
      for (uint32_t i = 0; i < 32; ++i) l[i] = 32 * t + i < n ? sq[32 * t + i] : 0.0f;
      sq[n + t] = tree32(l);
    }
    __syncthreads();
  }
  if (threadIdx.x < 64) {
    float acc = 0.0f;
    if (tree) {
      for (uint32_t t = 0; t < nb; ++t) acc = acc + sq[n + t];
    } else {
      for (uint32_t i = 0; i < n; ++i) acc = acc + sq[i];
    }
    float mean = acc / (float)n;
    float arg = mean + eps;
    float inv = rsqrt_cr(arg);
    if (threadIdx.x == 0) s_inv = inv;
  }
  __syncthreads();
  const float inv = s_inv;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    float sx = xv[i] * inv;
    ov[i] = sx * w[i];
  }
}

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, uint32_t n,
                          uint32_t nvec, float* out, hipStream_t s, bool tree) {
  if (n == 0 || n > 8192) return hipErrorInvalidValue;  // LDS: squares, partials, scalars
  const size_t shmem = (n + (n + 31) / 32) * sizeof(float);
  hipLaunchKernelGGL(k_rmsnorm, dim3(nvec), dim3(256), shmem, s, x, w, eps, n, out,
                     tree ? 1u : 0u);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RoPE rotate-half + KV store (code/cis2-fp/src/main.rs:285-307,426-427;
// spec §7.3-7.4): o1 = x1*c + (-x2)*s, o2 = x2*c + x1*s.  The cache keeps
// rotated keys and raw values.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_rope_store(float* q, float* k, const float* v,
                                                    const float* __restrict__ cs, uint32_t pos,
                                                    uint32_t nh, uint32_t nkv, uint32_t hd,
                                                    uint32_t max_pos, float* kc, float* vc) {
  const uint32_t half = hd / 2;
  const float* c = cs + (size_t)pos * half * 2;
  const uint32_t total = (nh + nkv) * half;
  for (uint32_t idx = threadIdx.x; idx < total; idx += blockDim.x) {
    uint32_t head = idx / half, i = idx - head * half;
    float* hv = head < nh ? q + (size_t)head * hd : k + (size_t)(head - nh) * hd;
    float cv = c[2 * i], sv = c[2 * i + 1];
    float x1 = hv[i], x2 = hv[i + half];
    float t1 = x1 * cv;
    float nx2 = -x2;
    float t2 = nx2 * sv;
    float t3 = x2 * cv;
    float t4 = x1 * sv;
    float o1 = t1 + t2, o2 = t3 + t4;
    hv[i] = o1;
    hv[i + half] = o2;
    if (head >= nh) {
      size_t base = (size_t)(head - nh) * hd;
      kc[(base + i) * max_pos + pos] = o1;
      kc[(base + i + half) * max_pos + pos] = o2;
    }
  }
  for (uint32_t idx = threadIdx.x; idx < nkv * hd; idx += blockDim.x) {
    uint32_t kvh = idx / hd, d = idx - kvh * hd;
    vc[((size_t)kvh * hd + d) * max_pos + pos] = v[idx];
  }
}

hipError_t launch_rope_store(float* q, float* k, const float* v, const float* rope_cs,
                             uint32_t pos, uint32_t nh, uint32_t nkv, uint32_t hd,
                             uint32_t max_pos, float* kc, float* vc, hipStream_t s) {
  if (pos >= max_pos || hd % 2) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_rope_store, dim3(1), dim3(256), 0, s, q, k, v, rope_cs, pos, nh, nkv,
                     hd, max_pos, kc, vc);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// (value, index) argmax semantics of a strict-> scan from index 0 (first
// maximum wins): among non-NaN values the largest, ties (==, which includes
// +0 vs -0) to the lowest index; a NaN at index 0 wins outright and a NaN
// anywhere else never does.  Order-free, so a tree reduction is exact.
// ---------------------------------------------------------------------------
struct VI { float v; uint32_t i; };  // i == UINT32_MAX: no candidate
__device__ __forceinline__ VI vi_pick(VI a, VI b) {
  if (b.i == UINT32_MAX) return a;
  if (a.i == UINT32_MAX) return b;
  if (b.v > a.v) return b;
  if (a.v > b.v) return a;
  return b.i < a.i ? b : a;
}
__device__ __forceinline__ VI vi_wave_reduce(VI x) {
  for (int off = 32; off > 0; off >>= 1) {
    VI o;
    o.v = __shfl_xor(x.v, off, 64);
    o.i = __shfl_xor(x.i, off, 64);
    x = vi_pick(x, o);
  }
  return x;
}
// Block-wide reduction; every thread gets the result.  blockDim % 64 == 0.
__device__ VI vi_block_reduce(VI x, VI* scratch) {
  x = vi_wave_reduce(x);
  const uint32_t wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  if ((threadIdx.x & 63) == 0) scratch[wv] = x;
  __syncthreads();
  VI r = scratch[0];
  for (uint32_t i = 1; i < nw; ++i) r = vi_pick(r, scratch[i]);
  __syncthreads();
  return r;
}

// ---------------------------------------------------------------------------
// Attention, one workgroup per query head (code/cis2-fp/src/main.rs:429-467;
// spec §9): scores_j = dot_seq(q_h, k_j) * scale, softmax_seq (first-wins
// max, pinned exp, strict-chain denominator, true divide), then the V mix
// out_d = fold_j (p_j * v_j[d]).  GQA: kv head = qh / (nh / nkv).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_attention(const float* __restrict__ q,
                                                   const float* __restrict__ kc,
                                                   const float* __restrict__ vc, uint32_t pos,
                                                   uint32_t nh, uint32_t nkv, uint32_t hd,
                                                   uint32_t max_pos, float scale,
                                                   float* att_out, float* scores_out,
                                                   float* probs_out, uint32_t tree) {
  extern __shared__ float sh[];
  __shared__ VI red[4];
  __shared__ float s_den;
  const uint32_t qh = blockIdx.x, group = nh / nkv, kvh = qh / group, len = pos + 1;
  float* sq = sh;
  float* ss = sh + hd;
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) sq[d] = q[(size_t)qh * hd + d];
  __syncthreads();
  const float* kb = kc + (size_t)kvh * hd * max_pos;
  for (uint32_t j = threadIdx.x; j < len; j += blockDim.x) {
    float acc = 0.0f;
    if (tree) {  // dot_tree (code/cis2-fp/src/math.rs:60-125)
      for (uint32_t d0 = 0; d0 < hd; d0 += 32) {
        float l[32];
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i)
          l[i] = d0 + i < hd ? sq[d0 + i] * kb[(size_t)(d0 + i) * max_pos + j] : 0.0f;
        acc = acc + tree32(l);
      }
    } else {
      for (uint32_t d = 0; d < hd; ++d) {
        float p = sq[d] * kb[(size_t)d * max_pos + j];
        acc = acc + p;
      }
    }
    float sc = acc * scale;
    ss[j] = sc;
    if (scores_out) scores_out[(size_t)qh * len + j] = sc;
  }
  __syncthreads();
  VI best = {0.0f, UINT32_MAX};
  for (uint32_t j = threadIdx.x; j < len; j += blockDim.x) {
    float v = ss[j];
    if (v == v) best = vi_pick(best, VI{v, j});
  }
  best = vi_block_reduce(best, red);
  const float mx = (ss[0] != ss[0]) ? ss[0] : best.v;
  for (uint32_t j = threadIdx.x; j < len; j += blockDim.x) {
    float dlt = ss[j] - mx;
    ss[j] = exp_pinned(dlt);
  }
  __syncthreads();
  const uint32_t nb = (len + 31) / 32;
  float* part = ss + len;  // tree: block partials of the denominator
  if (tree) {  // softmax_tree's sum (code/cis2-fp/src/math.rs:448-465)
    for (uint32_t t = threadIdx.x; t < nb; t += blockDim.x) {
      float l[32];
#pragma unroll
      for (uint32_t i = 0; i < 32; ++i) l[i] = 32 * t + i < len ? ss[32 * t + i] : 0.0f;
      part[t] = tree32(l);
    }
    __syncthreads();
  }
  if (threadIdx.x < 64) {
    float acc = 0.0f;
    if (tree) {
      for (uint32_t t = 0; t < nb; ++t) acc = acc + part[t];
    } else {
      for (uint32_t j = 0; j < len; ++j) acc = acc + ss[j];
    }
    if (threadIdx.x == 0) s_den = acc;
  }
  __syncthreads();
  const float den = s_den;
  for (uint32_t j = threadIdx.x; j < len; j += blockDim.x) {
    float pj = ss[j] / den;
    ss[j] = pj;
    if (probs_out) probs_out[(size_t)qh * len + j] = pj;
  }
  __syncthreads();
  const float* vb = vc + (size_t)kvh * hd * max_pos;
  for (uint32_t d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.0f;
    for (uint32_t j = 0; j < len; ++j) {
      float p = ss[j] * vb[(size_t)d * max_pos + j];
      acc = acc + p;
    }
    att_out[(size_t)qh * hd + d] = acc;
  }
}

hipError_t launch_attention(const float* q, const float* kc, const float* vc,
                            uint32_t pos, uint32_t nh, uint32_t nkv, uint32_t hd,
                            uint32_t max_pos, float scale, float* att_out,
                            float* scores_out, float* probs_out, hipStream_t s, bool tree) {
  if (pos >= max_pos || nkv == 0 || nh % nkv) return hipErrorInvalidValue;
  // q, scores, and the denominator's block partials
  size_t shmem = (size_t)(hd + pos + 1 + (pos + 32) / 32) * sizeof(float);
  if (shmem > 60 * 1024) return hipErrorInvalidValue;  // leaves room for static LDS
  hipLaunchKernelGGL(k_attention, dim3(nh), dim3(256), shmem, s, q, kc, vc, pos, nh, nkv, hd,
                     max_pos, scale, att_out, scores_out, probs_out, tree ? 1u : 0u);
  return hipGetLastError();
}

// Greedy argmax (code/cis2-fp/src/main.rs:1161-1169; spec §11.2).
__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ v, uint32_t n,
                                                 uint32_t* out) {
  __shared__ VI red[16];
  VI best = {0.0f, UINT32_MAX};
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    float x = v[i];
    if (x == x) best = vi_pick(best, VI{x, i});
  }
  best = vi_block_reduce(best, red);
  if (threadIdx.x == 0) {
    float v0 = v[0];
    *out = (v0 != v0 || best.i == UINT32_MAX) ? 0u : best.i;
  }
}

hipError_t launch_argmax(const float* logits, uint32_t n, uint32_t* tok_out, hipStream_t s) {
  if (n == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, logits, n, tok_out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// inv_freq and the per-position rotation table
// (code/cis2-fp/src/main.rs:849-869, :285-307; spec §7): ln_theta =
// ln((f32)theta), inv_freq[i] = exp(-(((f32)(2i)/(f32)hd) * ln_theta)),
// angle = (f32)pos * inv_freq[i], table = (cos(angle), sin(angle)).
// ---------------------------------------------------------------------------
__global__ void k_inv_freq(float theta, uint32_t hd, float* inv_freq) {
  const uint32_t i = threadIdx.x;
  if (i >= hd / 2) return;
  float lt = ln_pinned(theta);
  float frac = (float)(2 * i) / (float)hd;
  float a = frac * lt;
  float na = -a;
  inv_freq[i] = exp_pinned(na);
}
__global__ void k_rope_table(const float* __restrict__ inv_freq, uint32_t half,
                             uint32_t max_pos, float* cs) {
  size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)half * max_pos) return;
  uint32_t pos = (uint32_t)(idx / half), i = (uint32_t)(idx % half);
  float ang = (float)pos * inv_freq[i];
  float sv, cv;
  sincos_pinned(ang, &sv, &cv);
  cs[2 * idx] = cv;
  cs[2 * idx + 1] = sv;
}

hipError_t launch_rope_table(float theta_f32, uint32_t hd, uint32_t max_pos, float* inv_freq,
                             float* rope_cs, hipStream_t s) {
  if (hd == 0 || hd % 2 || hd > 1024) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_inv_freq, dim3(1), dim3(512), 0, s, theta_f32, hd, inv_freq);
  size_t n = (size_t)(hd / 2) * max_pos;
  hipLaunchKernelGGL(k_rope_table, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     inv_freq, hd / 2, max_pos, rope_cs);
  return hipGetLastError();
}

// Device FP-environment probes (spec §1.3; code/cis2-fp/gpu/cis2_fpenv.h:90-107).
__global__ void k_fpenv_probe(const float* in, uint32_t* out) {
  float p = in[0] * in[1];
  float s = in[2] + in[3];
  out[0] = __float_as_uint(p);
  out[1] = __float_as_uint(s);
}

hipError_t launch_fpenv_probe(uint32_t* out, hipStream_t s) {
  // operands staged in device memory so nothing is folded at compile time
  const uint32_t in_bits[4] = {0x00800000u, 0x2edbe6ffu /* 1e-10f */, 0x00000001u, 0u};
  float host_in[4];
  memcpy(host_in, in_bits, sizeof host_in);
  float* din = nullptr;
  hipError_t e = hipMalloc(&din, sizeof host_in);
  if (e != hipSuccess) return e;
  e = hipMemcpyAsync(din, host_in, sizeof host_in, hipMemcpyHostToDevice, s);
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_fpenv_probe, dim3(1), dim3(1), 0, s, din, out);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  (void)hipFree(din);
  return e;
}

// ---------------------------------------------------------------------------
// Wait-counter capacity probes (verification only).  One wave issues N
// vector loads (global_load_dword) or N LDS reads (ds_read_b128) into N
// distinct registers with no wait in between (inline asm: the compiler adds
// none), then one s_waitcnt vmcnt(0) / lgkmcnt(0), then stores every
// register.  The counters' fields hold 63 and 15 operations; the decode
// kernel's score tasks keep 64 (head_dim 64) or 128 (head_dim 128) loads
// per thread in flight and rely on the hardware holding further issue at
// the field's maximum rather than losing count.  A wrong value here would
// mean a wait can return while more operations are in flight than the
// field holds.  N stays small enough that no destination register is
// spilled or moved before the wait (checked on the built code object).
// ---------------------------------------------------------------------------
typedef float pf4 __attribute__((ext_vector_type(4)));
constexpr int kProbeVm = 128, kProbeLds = 40;
// element of `in` that vector load I of lane l reads (16384 floats)
__host__ __device__ constexpr uint32_t probe_vm_index(int I, uint32_t lane) {
  return (uint32_t)(I / 8) * 1024u + lane + (uint32_t)(I % 8) * 64u;
}
template <int I, int N>
__device__ __forceinline__ void probe_vm_issue(float (&r)[N], const float* base) {
  if constexpr (I < N) {
    asm volatile("global_load_dword %0, %1, off offset:%2"
                 : "=&v"(r[I])
                 : "v"(base + (I / 8) * 1024), "i"((I % 8) * 256)
                 : "memory");
    probe_vm_issue<I + 1, N>(r, base);
  }
}
__global__ __launch_bounds__(64) void k_probe_vm(const float* in, float* out) {
  const uint32_t lane = threadIdx.x;
  float r[kProbeVm];
  probe_vm_issue<0, kProbeVm>(r, in + lane);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < kProbeVm; ++i) out[i * 64 + lane] = r[i];
}
template <int I, int N>
__device__ __forceinline__ void probe_lds_issue(pf4 (&r)[N], uint32_t addr) {
  if constexpr (I < N) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(r[I]) : "v"(addr), "i"(I * 1024)
                 : "memory");
    probe_lds_issue<I + 1, N>(r, addr);
  }
}
__global__ __launch_bounds__(64) void k_probe_lds(const pf4* in, pf4* out) {
  __shared__ pf4 lds[kProbeLds * 64];
  const uint32_t lane = threadIdx.x;
  for (uint32_t i = lane; i < kProbeLds * 64; i += 64) lds[i] = in[i];
  __syncthreads();
  pf4 r[kProbeLds];
  // LDS byte offset of slot `lane`; load I reads slot I * 64 + lane
  const uint32_t addr = (uint32_t)(size_t)((__attribute__((address_space(3))) pf4*)lds + lane);
  probe_lds_issue<0, kProbeLds>(r, addr);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
  for (int i = 0; i < kProbeLds; ++i) out[i * 64 + lane] = r[i];
}

hipError_t run_wait_probes(uint32_t bad[2]) {
  // input: 16384 floats (the vector probe's largest index, probe_vm_index(127, 63),
  // is 15871; the LDS probe reads the first kProbeLds * 64 16-byte slots);
  // output: the larger of the two probes' results (128 x 64 floats, 40 x 64 x 4)
  const size_t nvm = 16384, nlds = (size_t)kProbeLds * 64;
  const size_t nout = std::max((size_t)kProbeVm * 64, nlds * 4);
  static_assert(probe_vm_index(kProbeVm - 1, 63) < 16384, "vector probe input");
  static_assert(kProbeLds * 64 * 4 <= 16384, "LDS probe input");
  std::vector<float> hin(nvm);
  for (size_t i = 0; i < nvm; ++i) hin[i] = (float)i;
  float *din = nullptr, *dout = nullptr;
  hipError_t e = hipMalloc(&din, nvm * 4);
  if (e == hipSuccess) e = hipMalloc(&dout, nout * 4);
  if (e == hipSuccess) e = hipMemcpy(din, hin.data(), nvm * 4, hipMemcpyHostToDevice);
  std::vector<float> hout(nout);
  bad[0] = bad[1] = 0;
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_probe_vm, dim3(1), dim3(64), 0, 0, din, dout);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(hout.data(), dout, (size_t)kProbeVm * 64 * 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    for (int i = 0; i < kProbeVm; ++i)
      for (uint32_t l = 0; l < 64; ++l)
        if (hout[(size_t)i * 64 + l] != hin[probe_vm_index(i, l)]) ++bad[0];
  // LDS: f4 slot j holds (4j, 4j+1, 4j+2, 4j+3); the first nlds slots of hin
  if (e == hipSuccess) {
    hipLaunchKernelGGL(k_probe_lds, dim3(1), dim3(64), 0, 0, reinterpret_cast<const pf4*>(din),
                       reinterpret_cast<pf4*>(dout));
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(hout.data(), dout, nlds * 16, hipMemcpyDeviceToHost);
  if (e == hipSuccess)
    for (size_t j = 0; j < nlds * 4; ++j)
      if (hout[j] != hin[j]) ++bad[1];
  if (din) (void)hipFree(din);
  if (dout) (void)hipFree(dout);
  return e;
}

// ---------------------------------------------------------------------------
// Pinned-math sweep helpers (exhaustive parity tests).
// fn: 0 exp, 1 sin, 2 cos, 3 ln, 4 silu, 5 rsqrt, 6 sqrt.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float apply_fn(int fn, float x) {
  switch (fn) {
    case 0: return exp_pinned(x);
    case 1: return sin_pinned(x);
    case 2: return cos_pinned(x);
    case 3: return ln_pinned(x);
    case 4: return silu_pinned(x);
    case 5: return rsqrt_cr(x);
    default: return sqrt_cr(x);
  }
}
__device__ __forceinline__ unsigned long long mix64(unsigned long long z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Each block covers 65536 consecutive input bit patterns (one chunk of
// 2^24 holds 256 blocks) and adds its partial hash to hash_out[chunk].
__global__ __launch_bounds__(256) void k_math_hash(int fn, uint32_t first, uint32_t count,
                                                   unsigned long long* hash_out) {
  const uint32_t per_block = 65536;
  uint64_t base = (uint64_t)first + (uint64_t)blockIdx.x * per_block;
  unsigned long long h = 0;
  for (uint32_t j = threadIdx.x; j < per_block; j += blockDim.x) {
    uint64_t off = (uint64_t)blockIdx.x * per_block + j;
    if (off >= count) break;
    uint32_t bits = (uint32_t)(base + j);
    uint32_t ob = __float_as_uint(apply_fn(fn, __uint_as_float(bits)));
    h += mix64((unsigned long long)ob ^ ((unsigned long long)bits * 0x9E3779B97F4A7C15ull));
  }
  for (int off = 32; off > 0; off >>= 1) h += __shfl_xor(h, off, 64);
  __shared__ unsigned long long part[4];
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = h;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long t = part[0] + part[1] + part[2] + part[3];
    uint32_t chunk = (uint32_t)((base - first) >> 24);
    atomicAdd(&hash_out[chunk], t);
  }
}

hipError_t launch_math_hash(int fn, uint32_t first, uint32_t count,
                            unsigned long long* hash_out, hipStream_t s) {
  if ((first & 0xFFFFu) || (count & 0xFFFFu) || count == 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_math_hash, dim3(count / 65536), dim3(256), 0, s, fn, first, count,
                     hash_out);
  return hipGetLastError();
}

__global__ void k_math_map(int fn, const float* __restrict__ in, float* __restrict__ out,
                           uint64_t n) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = apply_fn(fn, in[i]);
}
hipError_t launch_math_map(int fn, const float* in, float* out, uint64_t n, hipStream_t s) {
  hipLaunchKernelGGL(k_math_map, dim3(1024), dim3(256), 0, s, fn, in, out, n);
  return hipGetLastError();
}
__global__ void k_div_map(const float* __restrict__ a, const float* __restrict__ b,
                          float* __restrict__ out, uint64_t n) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = a[i] / b[i];
}
hipError_t launch_div_map(const float* a, const float* b, float* out, uint64_t n,
                          hipStream_t s) {
  hipLaunchKernelGGL(k_div_map, dim3(1024), dim3(256), 0, s, a, b, out, n);
  return hipGetLastError();
}

int device_cu_count() {
  static std::mutex mu;
  static std::map<int, int> cus;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> g(mu);
  auto it = cus.find(dev);
  if (it != cus.end()) return it->second;
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
    n = 256;
  cus[dev] = n;
  return n;
}

hipError_t ensure_dynamic_lds(const void* fn, size_t bytes) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, size_t> done;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> g(mu);
  size_t& have = done[{dev, fn}];
  if (have >= bytes) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess) have = bytes;
  return e;
}

}  // namespace cis2
