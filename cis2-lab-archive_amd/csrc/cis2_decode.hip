// cis2_decode.hip — persistent per-token decode kernel for gfx950.
//
// One launch computes one position of one sequence: all layers, the LM head
// and the greedy argmax (code/cis2-fp/src/main.rs:355-529 and :1161-1169;
// C++ mirror code/cis2-fp/gpu/cis2_model.h:685-774).  Every workgroup owns
// one fixed task per layer phase, so the weights a task needs for the next
// layer are copied into its LDS while it waits, and phases hand over through
// per-layer counters instead of kernel boundaries:
//
//   QKV  row blocks of q/k/v (+ RMSNorm input_layernorm, recomputed per task)
//   ATT  one workgroup per query head: optional QK-norm, RoPE, KV store,
//        scores, softmax, V mix
//   O    row blocks of o_proj, + residual
//   GU   row blocks of gate and up (+ post_attention_layernorm per task),
//        hid = silu(gate) * up
//   D    row blocks of down_proj, + residual
//   LM   final norm, LM-head rows, per-block argmax candidates; the last
//        workgroup to finish reduces them to the next token id.
//
// Arithmetic order is exactly the per-op kernels' (cis2_kernels.hip): one
// lane owns an output and folds its terms left to right from 0.
//
// Cross-workgroup data within a launch is written and read with agent-scope
// (sc1) accesses; a counter is incremented only after the writer's stores
// completed (s_waitcnt vmcnt(0)) and a reader loads the data only after it
// saw the counter.  Counters grow monotonically: a launch with epoch e
// waits for e * (task count).  Every wait has a spin cap that raises an
// error flag instead of hanging.
#include "cis2_decode.hpp"
#include "cis2_device_math.hpp"

namespace cis2 {

namespace {

constexpr uint32_t kThreads = 256;
constexpr uint32_t kSpinCap = 1u << 24;  // ~0.5 s of s_sleep(1)

enum { C_QKV = 0, C_ATT = 1, C_O = 2, C_GU = 3, C_D = 4 };

struct Act {
  float *q, *k, *v, *att, *h1, *hid, *hout;
};

// Bytes of the LDS region that holds a task's weight block, or the
// attention task's scores and cached K/V (up to the LDS budget).
__host__ __device__ inline size_t decode_wregion_bytes(const DecodeArgs& a) {
  size_t q = (size_t)a.Rq * a.H, o = (size_t)a.Ro * a.qd, g = 2 * (size_t)a.Rg * a.H,
         d = (size_t)a.Rd * a.I;
  size_t m = q > o ? q : o;
  m = m > g ? m : g;
  m = m > d ? m : d;
  size_t att = (size_t)a.max_pos + 64 + 2 * (size_t)a.hd * (((size_t)a.max_pos + 3) & ~(size_t)3);
  const size_t cap = 38400;  // 150 KiB in floats: what LDS can give this region
  if (att > cap) att = m > (size_t)a.max_pos + 64 ? m : (size_t)a.max_pos + 64;
  m = m > att ? m : att;
  return ((m * 4 + 255) / 256) * 256;
}

__host__ __device__ inline size_t layer_stride(uint32_t H, uint32_t I, uint32_t qd,
                                               uint32_t kvd) {
  size_t s = 2 * (size_t)qd + 2 * (size_t)kvd + 2 * (size_t)H + I;
  return (s + 63) & ~(size_t)63;
}

__device__ __forceinline__ Act act_of(const DecodeArgs& a, uint32_t l) {
  float* b = a.act + (size_t)l * layer_stride(a.H, a.I, a.qd, a.kvd);
  Act r;
  r.q = b;
  r.k = r.q + a.qd;
  r.v = r.k + a.kvd;
  r.att = r.v + a.kvd;
  r.h1 = r.att + a.qd;
  r.hid = r.h1 + a.H;
  r.hout = r.hid + a.I;
  return r;
}

__device__ __forceinline__ float ld_ag(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t ld_ag(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ag(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ag(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void stamp(const DecodeArgs& a, uint32_t l, uint32_t ph, uint32_t t,
                                      uint32_t slot) {
  if (a.tline && threadIdx.x == 0 && t < kTimelineTasks)
    a.tline[(((size_t)l * 6 + ph) * kTimelineTasks + t) * 4 + slot] = __builtin_amdgcn_s_memrealtime();
}

__device__ void wait_ge(uint32_t* ctr, uint32_t target, uint32_t* err) {
  if (threadIdx.x == 0) {
    uint32_t spins = 0;
    while ((int32_t)(ld_ag(ctr) - target) < 0) {
      __builtin_amdgcn_s_sleep(1);
      if ((++spins & 255u) == 0 && ld_ag(err) != 0u) break;  // another task failed
      if (spins > kSpinCap) {
        atomicOr(err, 2u);
        break;
      }
    }
  }
  __syncthreads();
}

// All of this workgroup's stores are complete before the counter moves.
__device__ void signal_add(uint32_t* ctr, uint32_t n) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Copies n4 float4 from global memory into LDS with 12 loads in flight per
// thread.
__device__ void copy_block_to_lds(float4* dst, const float4* __restrict__ src, uint32_t n4) {
  uint32_t i = threadIdx.x;
  constexpr int B = 12;
  for (; i + (B - 1) * kThreads < n4; i += B * kThreads) {
    float4 t[B];
#pragma unroll
    for (int u = 0; u < B; ++u) t[u] = src[i + u * kThreads];
#pragma unroll
    for (int u = 0; u < B; ++u) dst[i + u * kThreads] = t[u];
  }
  for (; i < n4; i += kThreads) dst[i] = src[i];
}

// Strict left-to-right chain over K for row `lane` of an LDS block laid out
// [K/4][R][4]; x is the LDS input vector.  Lanes >= R read row R-1 (their
// result is discarded).
__device__ __forceinline__ float chain_lds(const float* W, uint32_t R, const float* x, uint32_t K,
                                           uint32_t lane) {
  const uint32_t ln = lane < R ? lane : R - 1;
  const float4* wp = reinterpret_cast<const float4*>(W) + ln;
  const float4* xp = reinterpret_cast<const float4*>(x);
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

// Same chain with the block streamed from global memory; `D` float4 loads
// are kept in flight per lane.
__device__ __forceinline__ float chain_global(const float* __restrict__ W, uint32_t R,
                                              const float* x, uint32_t K, uint32_t lane) {
  const uint32_t ln = lane < R ? lane : R - 1;
  const float4* __restrict__ wp = reinterpret_cast<const float4*>(W) + ln;
  const float4* xp = reinterpret_cast<const float4*>(x);
  const uint32_t KG = K >> 2;
  constexpr uint32_t D = 16;
  float4 buf[D];
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) buf[u] = u < KG ? wp[(size_t)u * R] : make_float4(0, 0, 0, 0);
  float acc = 0.0f;
  for (uint32_t g0 = 0; g0 < KG; g0 += D) {
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      const uint32_t g = g0 + u;
      if (g < KG) {
        float4 w = buf[u];
        if (g + D < KG) buf[u] = wp[(size_t)(g + D) * R];
        float4 xv = xp[g];
        float p;
        p = w.x * xv.x; acc = acc + p;
        p = w.y * xv.y; acc = acc + p;
        p = w.z * xv.z; acc = acc + p;
        p = w.w * xv.w; acc = acc + p;
      }
    }
  }
  return acc;
}

// RMSNorm of an LDS vector (code/cis2-fp/src/main.rs:245-260): squares
// into `tmp`, one strict chain in wave 0, mean by a true divide,
// inv = 1/sqrt(mean + eps), out = (x*inv)*w.  `out` may alias `tmp` (not x).
__device__ void rmsnorm_lds(const float* x, const float* __restrict__ w, float eps, uint32_t n,
                            float* tmp, float* out, float* s_inv) {
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
    float v = x[i];
    tmp[i] = v * v;
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const float4* p = reinterpret_cast<const float4*>(tmp);
    float acc = 0.0f;
#pragma unroll 8
    for (uint32_t i = 0; i < (n >> 2); ++i) {
      float4 v = p[i];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
    for (uint32_t i = n & ~3u; i < n; ++i) acc = acc + tmp[i];
    float mean = acc / (float)n;
    float arg = mean + eps;
    float inv = rsqrt_cr(arg);
    if (threadIdx.x == 0) *s_inv = inv;
  }
  __syncthreads();
  const float inv = *s_inv;
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) {
    float sx = x[i] * inv;
    out[i] = sx * w[i];
  }
  __syncthreads();
}

struct Cand {
  float v;
  uint32_t i;  // UINT32_MAX: none
};
__device__ __forceinline__ Cand cand_pick(Cand a, Cand b) {
  if (b.i == UINT32_MAX) return a;
  if (a.i == UINT32_MAX) return b;
  if (b.v > a.v) return b;
  if (a.v > b.v) return a;
  return b.i < a.i ? b : a;
}
__device__ __forceinline__ Cand cand_wave(Cand x) {
  for (int off = 32; off > 0; off >>= 1) {
    Cand o;
    o.v = __shfl_xor(x.v, off, 64);
    o.i = __shfl_xor(x.i, off, 64);
    x = cand_pick(x, o);
  }
  return x;
}

// LDS layout: [weights | vec region].  The vec region holds the task's
// input vector and scratch.
struct Lds {
  float* w;
  float* v;
};

__device__ const float* hin_of(const DecodeArgs& a, uint32_t l, uint32_t tok) {
  return l == 0 ? a.embed + (size_t)tok * a.H : act_of(a, l - 1).hout;
}

// Loads n floats of a layer input into LDS: the embedding row (weights, plain
// loads) for layer 0, otherwise the previous layer's output (agent scope).
__device__ void load_vec(float* dst, const float* src, uint32_t n, bool shared) {
  for (uint32_t i = threadIdx.x; i < n; i += kThreads) dst[i] = shared ? ld_ag(src + i) : src[i];
}

// ---------------------------------------------------------------------------
// Phase tasks
// ---------------------------------------------------------------------------

// QKV task t: which matrix and block.
__device__ void qkv_task_geom(const DecodeArgs& a, const LayerW& Lw, uint32_t t, const float** W,
                              const float** bias, uint32_t* M, uint32_t* blk, float** out,
                              const Act& ac) {
  if (t < a.nq_q) {
    *W = Lw.wq; *bias = Lw.bq; *M = a.qd; *blk = t; *out = ac.q;
  } else if (t < a.nq_q + a.nq_k) {
    *W = Lw.wk; *bias = Lw.bk; *M = a.kvd; *blk = t - a.nq_q; *out = ac.k;
  } else {
    *W = Lw.wv; *bias = Lw.bv; *M = a.kvd; *blk = t - a.nq_q - a.nq_k; *out = ac.v;
  }
}

__device__ void prefetch_qkv(const DecodeArgs& a, uint32_t l, uint32_t t, Lds& s) {
  const LayerW& Lw = a.layers[l];
  const float *W, *bias;
  uint32_t M, blk;
  float* out;
  qkv_task_geom(a, Lw, t, &W, &bias, &M, &blk, &out, act_of(a, l));
  const size_t blkf = (size_t)a.Rq * a.H;
  copy_block_to_lds(reinterpret_cast<float4*>(s.w),
                    reinterpret_cast<const float4*>(W + blk * blkf), (uint32_t)(blkf / 4));
}

__device__ void run_qkv(const DecodeArgs& a, uint32_t l, uint32_t t, Lds& s, uint32_t tok) {
  const LayerW& Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const float *W, *bias;
  uint32_t M, blk;
  float* out;
  qkv_task_geom(a, Lw, t, &W, &bias, &M, &blk, &out, ac);
  stamp(a, l, C_QKV, t, 0);
  if (l > 0) wait_ge(a.cnt + (size_t)(l - 1) * kCountersPerLayer + C_D, a.epoch * a.nd, a.err);
  stamp(a, l, C_QKV, t, 1);
  float* x = s.v;
  float* ln = s.v + a.H;
  float* s_inv = s.v + 2 * a.H;
  load_vec(x, hin_of(a, l, tok), a.H, l > 0);
  __syncthreads();
  rmsnorm_lds(x, Lw.ln1, a.eps, a.H, ln, ln, s_inv);
  if (threadIdx.x < 64) {
    float acc = chain_lds(s.w, a.Rq, ln, a.H, threadIdx.x);
    uint32_t row = blk * a.Rq + threadIdx.x;
    if (threadIdx.x < a.Rq && row < M) {
      float r = bias ? acc + bias[row] : acc;
      st_ag(out + row, r);
    }
  }
  signal_add(a.cnt + (size_t)l * kCountersPerLayer + C_QKV, 1);
  stamp(a, l, C_QKV, t, 2);
}

// LDS floats the attention task needs to hold `pos` cached positions of one
// kv head (K as [hd][pos4], V as [pos][hd]) plus the scores.
__host__ __device__ inline size_t att_lds_floats(uint32_t hd, uint32_t pos, uint32_t max_pos) {
  size_t pos4 = (pos + 3) & ~3u;
  return (size_t)max_pos + 64 + (size_t)hd * pos4 + (size_t)pos * hd;
}

// Copies the cached K/V of positions [0, pos) of one kv head into LDS
// (before the phase wait: those positions were written by earlier launches).
__device__ void prefetch_kv(const DecodeArgs& a, uint32_t l, uint32_t kvh, float* kl, float* vl) {
  const uint32_t hd = a.hd, pos = a.pos, pos4 = (pos + 3) & ~3u, mp4 = a.max_pos >> 2;
  const float4* kc = reinterpret_cast<const float4*>(a.kc0 + (size_t)l * a.cache_stride) +
                     (size_t)kvh * hd * mp4;
  const float4* vc = reinterpret_cast<const float4*>(a.vc0 + (size_t)l * a.cache_stride +
                                                     (size_t)kvh * a.max_pos * hd);
  const uint32_t kq = pos4 >> 2, nk = hd * kq, nv = (pos * hd) >> 2;
  float4* kl4 = reinterpret_cast<float4*>(kl);
  float4* vl4 = reinterpret_cast<float4*>(vl);
  constexpr int B = 8;
  uint32_t i = threadIdx.x;
  for (; i + (B - 1) * kThreads < nk; i += B * kThreads) {
    float4 t[B];
#pragma unroll
    for (int u = 0; u < B; ++u) {
      uint32_t e = i + u * kThreads, d = e / kq, q = e - d * kq;
      t[u] = kc[(size_t)d * mp4 + q];
    }
#pragma unroll
    for (int u = 0; u < B; ++u) kl4[i + u * kThreads] = t[u];
  }
  for (; i < nk; i += kThreads) {
    uint32_t d = i / kq, q = i - d * kq;
    kl4[i] = kc[(size_t)d * mp4 + q];
  }
  copy_block_to_lds(vl4, vc, nv);
}

// Attention for query head h (code/cis2-fp/src/main.rs:415-467).
__device__ void run_att(const DecodeArgs& a, uint32_t l, uint32_t h, Lds& s, size_t wfloats) {
  const LayerW& Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const uint32_t hd = a.hd, group = a.nh / a.nkv, kvh = h / group, len = a.pos + 1;
  const uint32_t pos4 = (a.pos + 3) & ~3u;
  float* qv = s.v;
  float* kv = qv + hd;
  float* vv = kv + hd;
  float* tmp = vv + hd;
  float* misc = tmp + hd;  // [0] inv, [1] den, [4..] reduction scratch
  float* ss = s.w;         // scores / probabilities, len floats
  float* kl = ss + a.max_pos + 64;
  float* vl = kl + (size_t)hd * pos4;
  const bool in_lds = att_lds_floats(hd, a.pos, a.max_pos) <= wfloats;
  stamp(a, l, C_ATT, h, 0);
  if (in_lds) prefetch_kv(a, l, kvh, kl, vl);
  wait_ge(a.cnt + (size_t)l * kCountersPerLayer + C_QKV, a.epoch * a.nq, a.err);
  stamp(a, l, C_ATT, h, 1);
  for (uint32_t d = threadIdx.x; d < hd; d += kThreads) {
    qv[d] = ld_ag(ac.q + (size_t)h * hd + d);
    kv[d] = ld_ag(ac.k + (size_t)kvh * hd + d);
    vv[d] = ld_ag(ac.v + (size_t)kvh * hd + d);
  }
  __syncthreads();
  // Qwen3 per-head QK-norm, after bias and before RoPE
  // (labs/w1x-qwen3/scripts/qwen3-port.diff:66-80).
  if (Lw.qn) rmsnorm_lds(qv, Lw.qn, a.eps, hd, tmp, qv, misc);
  if (Lw.kn) rmsnorm_lds(kv, Lw.kn, a.eps, hd, tmp, kv, misc);
  // RoPE rotate-half (main.rs:285-307): o1 = x1*c + (-x2)*s, o2 = x2*c + x1*s.
  const uint32_t half = hd / 2;
  const float* cs = a.rope_cs + (size_t)a.pos * half * 2;
  for (uint32_t idx = threadIdx.x; idx < 2 * half; idx += kThreads) {
    float* hv = idx < half ? qv : kv;
    uint32_t i = idx < half ? idx : idx - half;
    float c = cs[2 * i], sn = cs[2 * i + 1];
    float x1 = hv[i], x2 = hv[i + half];
    float t1 = x1 * c;
    float nx2 = -x2;
    float t2 = nx2 * sn;
    float t3 = x2 * c;
    float t4 = x1 * sn;
    hv[i] = t1 + t2;
    hv[i + half] = t3 + t4;
  }
  __syncthreads();
  float* kc = a.kc0 + (size_t)l * a.cache_stride;
  float* vc = a.vc0 + (size_t)l * a.cache_stride;
  if (h % group == 0) {  // one writer per kv head; the others use their own copy
    for (uint32_t d = threadIdx.x; d < hd; d += kThreads) {
      kc[((size_t)kvh * hd + d) * a.max_pos + a.pos] = kv[d];
      vc[((size_t)kvh * a.max_pos + a.pos) * hd + d] = vv[d];
    }
  }
  // scores_j = dot_seq(q, k_j) * scale (main.rs:440-445)
  const float* kb = kc + (size_t)kvh * hd * a.max_pos;
  const float4* q4 = reinterpret_cast<const float4*>(qv);
  for (uint32_t j = threadIdx.x; j < len; j += kThreads) {
    float acc = 0.0f;
    if (j == a.pos) {
      for (uint32_t d = 0; d < hd; ++d) {
        float p = qv[d] * kv[d];
        acc = acc + p;
      }
    } else if (in_lds) {
#pragma unroll 4
      for (uint32_t d4 = 0; d4 < hd / 4; ++d4) {
        float4 qq = q4[d4];
        const float* kr = kl + (size_t)(4 * d4) * pos4 + j;
        float p;
        p = qq.x * kr[0]; acc = acc + p;
        p = qq.y * kr[pos4]; acc = acc + p;
        p = qq.z * kr[2 * pos4]; acc = acc + p;
        p = qq.w * kr[3 * pos4]; acc = acc + p;
      }
    } else {
#pragma unroll 8
      for (uint32_t d = 0; d < hd; ++d) {
        float p = qv[d] * kb[(size_t)d * a.max_pos + j];
        acc = acc + p;
      }
    }
    ss[j] = acc * a.scale;
  }
  __syncthreads();
  // softmax_seq (math.rs:425-442): first-wins max, pinned exp, strict-chain
  // denominator, true divide.
  Cand best = {0.0f, UINT32_MAX};
  for (uint32_t j = threadIdx.x; j < len; j += kThreads) {
    float v = ss[j];
    if (v == v) best = cand_pick(best, Cand{v, j});
  }
  best = cand_wave(best);
  Cand* red = reinterpret_cast<Cand*>(misc + 4);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = best;
  __syncthreads();
  Cand b = red[0];
  for (uint32_t i = 1; i < kThreads / 64; ++i) b = cand_pick(b, red[i]);
  const float mx = (ss[0] != ss[0]) ? ss[0] : b.v;
  __syncthreads();
  for (uint32_t j = threadIdx.x; j < len; j += kThreads) {
    float dlt = ss[j] - mx;
    ss[j] = exp_pinned(dlt);
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    float acc = 0.0f;
    uint32_t j = 0;
    for (; j + 4 <= len; j += 4) {
      float4 e = *reinterpret_cast<const float4*>(ss + j);
      acc = acc + e.x;
      acc = acc + e.y;
      acc = acc + e.z;
      acc = acc + e.w;
    }
    for (; j < len; ++j) acc = acc + ss[j];
    if (threadIdx.x == 0) misc[1] = acc;
  }
  __syncthreads();
  const float den = misc[1];
  for (uint32_t j = threadIdx.x; j < len; j += kThreads) {
    float pj = ss[j] / den;
    ss[j] = pj;
  }
  __syncthreads();
  // V mix out_d = fold_j (p_j * v_j[d]) (main.rs:454-463)
  const float* vb = in_lds ? vl : vc + (size_t)kvh * a.max_pos * hd;
  for (uint32_t d = threadIdx.x; d < hd; d += kThreads) {
    float acc = 0.0f;
    const uint32_t np = a.pos;  // cached positions; position pos from LDS
#pragma unroll 8
    for (uint32_t j = 0; j < np; ++j) {
      float p = ss[j] * vb[(size_t)j * hd + d];
      acc = acc + p;
    }
    float p = ss[np] * vv[d];
    acc = acc + p;
    st_ag(ac.att + (size_t)h * hd + d, acc);
  }
  signal_add(a.cnt + (size_t)l * kCountersPerLayer + C_ATT, 1);
  stamp(a, l, C_ATT, h, 2);
}

__device__ void prefetch_rows(const float* W, uint32_t R, uint32_t K, uint32_t blk, float* dst) {
  const size_t blkf = (size_t)R * K;
  copy_block_to_lds(reinterpret_cast<float4*>(dst), reinterpret_cast<const float4*>(W + blk * blkf),
                    (uint32_t)(blkf / 4));
}

// o_proj block + residual h1 = h + o (main.rs:470-472).
__device__ void run_o(const DecodeArgs& a, uint32_t l, uint32_t t, Lds& s, uint32_t tok) {
  const Act ac = act_of(a, l);
  stamp(a, l, C_O, t, 0);
  wait_ge(a.cnt + (size_t)l * kCountersPerLayer + C_ATT, a.epoch * a.nh, a.err);
  stamp(a, l, C_O, t, 1);
  float* x = s.v;
  load_vec(x, ac.att, a.qd, true);
  __syncthreads();
  if (threadIdx.x < 64) {
    float acc = chain_lds(s.w, a.Ro, x, a.qd, threadIdx.x);
    uint32_t row = t * a.Ro + threadIdx.x;
    if (threadIdx.x < a.Ro && row < a.H) {
      const float* hp = hin_of(a, l, tok);
      float hv = l > 0 ? ld_ag(hp + row) : hp[row];
      st_ag(ac.h1 + row, hv + acc);
    }
  }
  signal_add(a.cnt + (size_t)l * kCountersPerLayer + C_O, 1);
  stamp(a, l, C_O, t, 2);
}

// gate/up block (wave 0 gate rows, wave 1 up rows) after
// post_attention_layernorm; hid = silu(gate) * up (main.rs:478-487).
__device__ void run_gu(const DecodeArgs& a, uint32_t l, uint32_t t, Lds& s) {
  const LayerW& Lw = a.layers[l];
  const Act ac = act_of(a, l);
  stamp(a, l, C_GU, t, 0);
  wait_ge(a.cnt + (size_t)l * kCountersPerLayer + C_O, a.epoch * a.no, a.err);
  stamp(a, l, C_GU, t, 1);
  float* x = s.v;
  float* ln = x + a.H;
  float* gx = ln + a.H;  // 64 floats: gate results
  float* s_inv = gx + 64;
  load_vec(x, ac.h1, a.H, true);
  __syncthreads();
  rmsnorm_lds(x, Lw.ln2, a.eps, a.H, ln, ln, s_inv);
  const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const size_t blkf = (size_t)a.Rg * a.H;
  float acc = 0.0f;
  if (wv < 2) acc = chain_lds(s.w + wv * blkf, a.Rg, ln, a.H, lane);
  if (wv == 0) gx[lane] = acc;
  __syncthreads();
  if (wv == 1) {
    uint32_t row = t * a.Rg + lane;
    if (lane < a.Rg && row < a.I) {
      float sg = silu_pinned(gx[lane]);
      st_ag(ac.hid + row, sg * acc);
    }
  }
  signal_add(a.cnt + (size_t)l * kCountersPerLayer + C_GU, 1);
  stamp(a, l, C_GU, t, 2);
}

// down block + residual h_next = h1 + down (main.rs:489-491).
__device__ void run_d(const DecodeArgs& a, uint32_t l, uint32_t t, Lds& s) {
  const Act ac = act_of(a, l);
  stamp(a, l, C_D, t, 0);
  wait_ge(a.cnt + (size_t)l * kCountersPerLayer + C_GU, a.epoch * a.ng, a.err);
  stamp(a, l, C_D, t, 1);
  float* x = s.v;
  load_vec(x, ac.hid, a.I, true);
  __syncthreads();
  if (threadIdx.x < 64) {
    float acc = chain_lds(s.w, a.Rd, x, a.I, threadIdx.x);
    uint32_t row = t * a.Rd + threadIdx.x;
    if (threadIdx.x < a.Rd && row < a.H) st_ag(ac.hout + row, ld_ag(ac.h1 + row) + acc);
  }
  signal_add(a.cnt + (size_t)l * kCountersPerLayer + C_D, 1);
  stamp(a, l, C_D, t, 2);
}

// Final norm, LM-head rows (4 waves = 4 blocks at a time), per-block argmax
// candidates; the last workgroup to finish reduces them.
__device__ void run_lm(const DecodeArgs& a, Lds& s) {
  const uint32_t L = a.L;
  stamp(a, L - 1, 5, blockIdx.x, 0);
  wait_ge(a.cnt + (size_t)(L - 1) * kCountersPerLayer + C_D, a.epoch * a.nd, a.err);
  stamp(a, L - 1, 5, blockIdx.x, 1);
  float* x = s.v;
  float* hn = x + a.H;
  float* misc = hn + a.H;
  load_vec(x, act_of(a, L - 1).hout, a.H, true);
  __syncthreads();
  rmsnorm_lds(x, a.fnorm, a.eps, a.H, hn, hn, misc);
  const uint32_t wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  uint32_t done = 0;
  for (uint32_t base = blockIdx.x * 4; base < a.nl; base += a.nwg * 4) {
    const uint32_t b = base + wv;
    if (b < a.nl) {
      float acc = chain_global(a.lm + (size_t)b * a.Rl * a.H, a.Rl, hn, a.H, lane);
      const uint32_t row = b * a.Rl + lane;
      Cand c = {0.0f, UINT32_MAX};
      if (lane < a.Rl && row < a.V) {
        a.logits[row] = acc;
        if (acc == acc) c = Cand{acc, row};
      }
      c = cand_wave(c);
      if (lane == 0) {
        st_ag(a.cand + 2 * b, __float_as_uint(c.v));
        st_ag(a.cand + 2 * b + 1, c.i);
      }
      if (b == 0 && lane == 0) {  // NaN at index 0 wins outright (strict > scan)
        st_ag(a.cand + 2 * a.nl, acc != acc ? 1u : 0u);
      }
    }
    done += (base < a.nl) ? min(4u, a.nl - base) : 0u;
  }
  stamp(a, L - 1, 5, blockIdx.x, 2);
  // ticket: the workgroup whose blocks complete the set reduces them
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  uint32_t* ticket = a.cnt + (size_t)L * kCountersPerLayer;
  __shared__ uint32_t s_last;
  if (threadIdx.x == 0) {
    uint32_t before = __hip_atomic_fetch_add(ticket, done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (before + done == a.lm_epoch * a.nl) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  Cand c = {0.0f, UINT32_MAX};
  for (uint32_t b = threadIdx.x; b < a.nl; b += kThreads) {
    Cand o = {__uint_as_float(ld_ag(a.cand + 2 * b)), ld_ag(a.cand + 2 * b + 1)};
    c = cand_pick(c, o);
  }
  c = cand_wave(c);
  Cand* red = reinterpret_cast<Cand*>(misc + 4);
  if (lane == 0) red[wv] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    Cand r = red[0];
    for (uint32_t i = 1; i < kThreads / 64; ++i) r = cand_pick(r, red[i]);
    uint32_t first_nan = ld_ag(a.cand + 2 * a.nl);
    *a.tok_out = (first_nan || r.i == UINT32_MAX) ? 0u : r.i;
  }
  stamp(a, L - 1, 5, blockIdx.x, 3);
}

__global__ __launch_bounds__(256) void k_decode(DecodeArgs a) {
  extern __shared__ float4 lds4[];
  Lds s;
  s.w = reinterpret_cast<float*>(lds4);
  const size_t wbytes = decode_wregion_bytes(a);
  s.v = reinterpret_cast<float*>(reinterpret_cast<char*>(lds4) + wbytes);
  const uint32_t wg = blockIdx.x;
  // role of this workgroup in every layer
  int role = -1;
  uint32_t t = 0;
  if (wg >= a.base_q && wg < a.base_q + a.nq) { role = C_QKV; t = wg - a.base_q; }
  else if (wg >= a.base_a && wg < a.base_a + a.nh) { role = C_ATT; t = wg - a.base_a; }
  else if (wg >= a.base_o && wg < a.base_o + a.no) { role = C_O; t = wg - a.base_o; }
  else if (wg >= a.base_g && wg < a.base_g + a.ng) { role = C_GU; t = wg - a.base_g; }
  else if (wg >= a.base_d && wg < a.base_d + a.nd) { role = C_D; t = wg - a.base_d; }

  uint32_t tok = 0;
  if (role == C_QKV || role == C_O) {  // the layer-0 tasks that read the embedding row
    tok = *a.tok_in;
    if (tok >= a.V) {
      if (threadIdx.x == 0) atomicOr(a.err, 1u);
      tok = 0;
    }
  }
  for (uint32_t l = 0; l < a.L; ++l) {
    const LayerW& Lw = a.layers[l];
    switch (role) {
      case C_QKV:
        prefetch_qkv(a, l, t, s);
        __syncthreads();
        run_qkv(a, l, t, s, tok);
        break;
      case C_ATT:
        run_att(a, l, t, s, wbytes / 4);
        break;
      case C_O:
        prefetch_rows(Lw.wo, a.Ro, a.qd, t, s.w);
        __syncthreads();
        run_o(a, l, t, s, tok);
        break;
      case C_GU: {
        prefetch_rows(Lw.wg, a.Rg, a.H, t, s.w);
        prefetch_rows(Lw.wu, a.Rg, a.H, t, s.w + (size_t)a.Rg * a.H);
        __syncthreads();
        run_gu(a, l, t, s);
        break;
      }
      case C_D:
        prefetch_rows(Lw.wd, a.Rd, a.I, t, s.w);
        __syncthreads();
        run_d(a, l, t, s);
        break;
      default:
        break;
    }
    __syncthreads();
  }
  if (a.want_logits) run_lm(a, s);
}

}  // namespace

size_t decode_act_floats(uint32_t H, uint32_t I, uint32_t qd, uint32_t kvd) {
  return layer_stride(H, I, qd, kvd);
}

size_t decode_lds_bytes(const DecodeArgs& a) {
  size_t wbytes = decode_wregion_bytes(a);
  size_t vec = 2 * (size_t)a.H + 64 + 64;
  size_t vi = a.I, vq = a.qd, va = 4 * (size_t)a.hd + 64;
  vec = vec > vi ? vec : vi;
  vec = vec > vq ? vec : vq;
  vec = vec > va ? vec : va;
  return wbytes + vec * 4 + 256;
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t s) {
  const size_t lds = decode_lds_bytes(a);
  static size_t configured = 0;
  if (lds > configured) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&k_decode),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    configured = lds;
  }
  hipLaunchKernelGGL(k_decode, dim3(a.nwg), dim3(kThreads), lds, s, a);
  return hipGetLastError();
}

}  // namespace cis2
