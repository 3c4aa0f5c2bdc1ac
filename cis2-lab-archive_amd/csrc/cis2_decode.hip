// cis2_decode.hip — persistent per-token decode kernel for gfx950.
//
// One launch computes one position of one sequence: all layers, the LM head
// and the greedy argmax (code/cis2-fp/src/main.rs:355-529 and :1161-1169;
// C++ mirror code/cis2-fp/gpu/cis2_model.h:685-774).  Every workgroup owns
// one fixed task per layer phase, copies the weights that task needs into
// its LDS while it waits, and consumes the previous phase's outputs as soon
// as they are written:
//
//   QKV  row blocks of q/k/v (+ input_layernorm, recomputed per task)
//   ATT  one workgroup per query head: optional QK-norm, RoPE, KV store,
//        scores, softmax, V mix
//   O    row blocks of o_proj, + residual
//   GU   row blocks of gate and up (+ post_attention_layernorm per task),
//        hid = silu(gate) * up
//   D    row blocks of down_proj, + residual
//   LM   final norm, LM-head rows, per-block argmax candidates; the last
//        workgroup to finish reduces them to the next token id.
//
// Arithmetic order is the per-op kernels' (cis2_kernels.hip): one lane owns
// an output and folds its terms left to right from 0.  Dot products are
// split into two passes: every wave forms the rounded products (one
// rounding each, so any order gives the same bits) in LDS, then the owning
// lane adds them strictly in order, one add per step.
//
// Hand-over: every value that crosses workgroups is one 64-bit word
// {f32 bits, launch epoch} written with a single agent-scope (sc1) store;
// the consumer re-reads (sc1) the words it needs until all carry the
// current epoch.  An aligned 64-bit store is single-copy atomic, so a
// matching tag implies the matching value: no counters, fences or cache
// maintenance between phases.  Waits have a spin cap that raises an error
// flag instead of hanging, and stop early once any task raised it.
//
// Pointers carry their address space (LDS = 3, global = 1) so that every
// access is a ds_* or global_* instruction, never flat_*.
#include "cis2_decode.hpp"
#include "cis2_device_math.hpp"
#include "cis2_kernels.hpp"

namespace cis2 {

namespace {

#define AS_LDS __attribute__((address_space(3)))
#define AS_GLB __attribute__((address_space(1)))
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned long long u64;
typedef AS_LDS float lf;
typedef AS_LDS f4 lf4;
typedef const AS_GLB float gf;
typedef const AS_GLB f4 gf4;
typedef AS_GLB u64 gw;

// threadIdx.x through an opaque copy: values derived from it are formed
// where they are used instead of being hoisted out of the layer loop and
// kept live for the whole persistent kernel (which otherwise runs out of
// registers and spills).
__device__ __forceinline__ uint32_t tid_x() {
  uint32_t t = threadIdx.x;
  asm volatile("" : "+v"(t));
  __builtin_assume(t < 256u);  // every kernel here runs 256-thread workgroups
  return t;
}
__device__ __forceinline__ gf* G(const float* p) { return (gf*)p; }
__device__ __forceinline__ gf4* G4(const float* p) { return (gf4*)p; }
__device__ __forceinline__ AS_GLB float* GW(float* p) { return (AS_GLB float*)p; }
__device__ __forceinline__ AS_GLB uint32_t* GU(uint32_t* p) { return (AS_GLB uint32_t*)p; }

constexpr uint32_t kThreads = 256;

enum { P_QKV = kPhaseQKV, P_ATT = kPhaseATT, P_O = kPhaseO, P_GU = kPhaseGU, P_D = kPhaseD,
       P_LM = 5 };

// Per-layer tagged activations.
struct Act {
  gw *q, *k, *v, *att, *h1, *hid, *hout;
};

__host__ __device__ inline size_t layer_words(uint32_t H, uint32_t I, uint32_t qd, uint32_t kvd) {
  size_t s = 2 * (size_t)qd + 2 * (size_t)kvd + 2 * (size_t)H + I;
  return (s + 63) & ~(size_t)63;
}

__device__ __forceinline__ Act act_of(const DecodeArgs& a, uint32_t l) {
  gw* b = (gw*)a.act + (size_t)l * layer_words(a.H, a.I, a.qd, a.kvd);
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

// Row stride (floats) of the attention task's LDS copies of K and V for a
// position count: the least value >= pos rounded up to 4 that is 4 mod 32,
// so that 64 lanes reading 16 bytes each from 64 rows hit distinct banks.
__host__ __device__ inline uint32_t att_row_stride(uint32_t pos) {
  const uint32_t p4 = (pos + 3) & ~3u;
  return p4 + ((36u - (p4 & 31u)) & 31u);
}

// Row stride (floats) of the attention task's transposed LDS copy of K (one
// row of head dims per position): hd rounded up to 4, plus 4, so that 16
// lanes reading 16 bytes each from 16 consecutive rows cover all 64 banks.
__host__ __device__ inline uint32_t att_k_stride(uint32_t hd) { return ((hd + 3) & ~3u) + 4; }

// LDS floats of the attention task: scores (max_pos + 64), K as rows of
// positions 0..pos-1 (rounded up to 4) and V as rows of head dims.
__host__ __device__ inline size_t att_lds_floats(uint32_t hd, uint32_t pos, uint32_t max_pos) {
  return (size_t)max_pos + 64 + (size_t)((pos + 3) & ~3u) * att_k_stride(hd) +
         (size_t)hd * att_row_stride(pos);
}

// Positions per tile when a head's cached K/V do not fit in LDS: the
// largest multiple of 32 whose [hd][TP+4] tile fits beside the scores (row
// stride TP+4 is 4 mod 32: conflict-free 16-byte row reads); 0 if < 32.
__host__ __device__ inline uint32_t att_tile_positions(uint32_t hd, uint32_t max_pos,
                                                       size_t wfloats) {
  const size_t room = wfloats > (size_t)max_pos + 64 ? wfloats - max_pos - 64 : 0;
  const size_t per = room / hd;
  if (per < 36) return 0;
  size_t tp = (per - 4) & ~(size_t)31;
  if (tp > 1024) tp = 1024;
  return (uint32_t)tp;
}

// Split attention: output dims per mix task, and the floats of the tree
// partials that follow the scores (one per 32 positions, rounded to 16 B).
constexpr uint32_t kAttDV = 8;
__host__ __device__ inline size_t att_part_floats(uint32_t max_pos) {
  return ((size_t)max_pos / 32 + 1 + 3) & ~(size_t)3;
}
// A mix task's LDS in the weight region (floats): its head's scores
// ([max_pos + 64]), their tree partials, then a ring of nr V tiles
// ([16][tp + 4], the products formed in place).  The plan takes a ring of
// 4 tiles (two in flight beyond the tile in use and the one being
// formed), else 3, with the largest tile (a multiple of 32, at most 1024
// positions) that fits.  tp = 0: no plan fits.
__host__ __device__ inline void att_mix_plan(uint32_t max_pos, size_t wfloats, uint32_t* tp,
                                             uint32_t* nr) {
  *tp = 0;
  *nr = 0;
  const size_t used = (size_t)max_pos + 64 + att_part_floats(max_pos);
  if (wfloats <= used) return;
  const size_t room = wfloats - used;
  for (uint32_t r = 4; r >= 3; --r) {
    const size_t ts = room / ((size_t)r * kAttDV);
    if (ts < 36) continue;
    size_t t = (ts - 4) & ~(size_t)31;
    if (t > 1024) t = 1024;
    *tp = (uint32_t)t;
    *nr = r;
    return;
  }
}

// Floats of the vector region (input vectors and scratch of every role),
// rounded up to 16 bytes.
__host__ __device__ inline size_t decode_vec_floats(const DecodeArgs& a) {
  size_t vec = 2 * (size_t)a.H + 64 + 64;                          // QKV, GU, LM
  const size_t vo = (size_t)a.qd + a.Ro, vd = (size_t)a.I + a.Rd;  // O, D
  const size_t ng = a.nkv ? a.nh / a.nkv : 1;                      // ATT (score task)
  const size_t va = (2 * ng + 4) * a.hd + 64;
  vec = vec > vo ? vec : vo;
  vec = vec > vd ? vec : vd;
  vec = vec > va ? vec : va;
  return (vec + 3) & ~(size_t)3;
}

// Bytes of the LDS region that holds a task's weight block(s), or the
// attention task's scores and cached K/V (up to what LDS can give).
__host__ __device__ inline size_t decode_wregion_bytes(const DecodeArgs& a) {
  size_t q = (size_t)a.Rq * a.H, o = (size_t)a.Ro * a.qd, g = 2 * (size_t)a.Rg * a.H,
         d = (size_t)a.Rd * a.I, lm = (size_t)a.Rl * a.H;
  size_t m = q > o ? q : o;
  m = m > g ? m : g;
  m = m > d ? m : d;
  m = m > lm ? m : lm;
  m = m > a.wslot ? m : a.wslot;
  // Attention: scores always in LDS; K/V rows in LDS for the positions that
  // fit in 150 KiB, read from HBM beyond that.
  size_t att = att_lds_floats(a.hd, a.max_pos, a.max_pos);
  // what LDS leaves after the vectors, the product pad, slack and static LDS
  const size_t rest = decode_vec_floats(a) * 4 + 64 * 16 + 256 + 64;
  size_t cap = rest < 160 * 1024 ? (160 * 1024 - rest) / 4 : 0;
  cap &= ~(size_t)63;
  if (cap < (size_t)a.max_pos + 64) cap = (size_t)a.max_pos + 64;
  if (att > cap) att = cap;
  m = m > att ? m : att;
  return ((m * 4 + 255) / 256) * 256;
}

__device__ __forceinline__ uint32_t ld_ag(const uint32_t* p) {
  return __hip_atomic_load((const AS_GLB uint32_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_ag(uint32_t* p, uint32_t v) {
  __hip_atomic_store(GU(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_err(uint32_t* err, uint32_t bit) {
  __hip_atomic_fetch_or(GU(err), bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ u64 get_word(const gw* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void put_word(gw* p, float v, uint32_t epoch) {
  __hip_atomic_store(p, ((u64)epoch << 32) | (u64)__float_as_uint(v), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void stamp(const DecodeArgs& a, uint32_t l, uint32_t ph, uint32_t t,
                                      uint32_t slot) {
  if (a.tline && tid_x() == 0 && t < kTimelineTasks)
    ((AS_GLB uint64_t*)a.tline)[(((size_t)l * 6 + ph) * kTimelineTasks + t) * 4 + slot] =
        __builtin_amdgcn_s_memrealtime();
}

// s_waitcnt vmcnt(0) (expcnt, lgkmcnt fields at their maxima: no wait).
// The builtin is a side effect without a memory operand, so the empty asm
// statements pin the LDS accesses of the caller (the reads of rows that
// this wave's global_load_lds copies filled) after it.
__device__ __forceinline__ void wait_vm0() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0x0F70);
  asm volatile("" ::: "memory");
}

// s_waitcnt vmcnt(n) for a run-time n.  n is clamped to the counter's 63:
// once every load has been issued at most 63 are outstanding, and they are
// the newest ones, so when more than 63 loads followed the ones waited for,
// those have completed.
__device__ __forceinline__ void wait_vmcnt(uint32_t n) {
  switch (n < 63u ? n : 63u) {
#define CIS2_VMW(k) \
  case k:           \
    __builtin_amdgcn_s_waitcnt(0x0F70 | ((k) & 15) | (((k) >> 4) << 14)); \
    break;
    CIS2_VMW(0) CIS2_VMW(1) CIS2_VMW(2) CIS2_VMW(3) CIS2_VMW(4) CIS2_VMW(5) CIS2_VMW(6)
    CIS2_VMW(7) CIS2_VMW(8) CIS2_VMW(9) CIS2_VMW(10) CIS2_VMW(11) CIS2_VMW(12) CIS2_VMW(13)
    CIS2_VMW(14) CIS2_VMW(15) CIS2_VMW(16) CIS2_VMW(17) CIS2_VMW(18) CIS2_VMW(19) CIS2_VMW(20)
    CIS2_VMW(21) CIS2_VMW(22) CIS2_VMW(23) CIS2_VMW(24) CIS2_VMW(25) CIS2_VMW(26) CIS2_VMW(27)
    CIS2_VMW(28) CIS2_VMW(29) CIS2_VMW(30) CIS2_VMW(31) CIS2_VMW(32) CIS2_VMW(33) CIS2_VMW(34)
    CIS2_VMW(35) CIS2_VMW(36) CIS2_VMW(37) CIS2_VMW(38) CIS2_VMW(39) CIS2_VMW(40) CIS2_VMW(41)
    CIS2_VMW(42) CIS2_VMW(43) CIS2_VMW(44) CIS2_VMW(45) CIS2_VMW(46) CIS2_VMW(47) CIS2_VMW(48)
    CIS2_VMW(49) CIS2_VMW(50) CIS2_VMW(51) CIS2_VMW(52) CIS2_VMW(53) CIS2_VMW(54) CIS2_VMW(55)
    CIS2_VMW(56) CIS2_VMW(57) CIS2_VMW(58) CIS2_VMW(59) CIS2_VMW(60) CIS2_VMW(61) CIS2_VMW(62)
    default: __builtin_amdgcn_s_waitcnt(0x0F70 | 15 | (3 << 14)); break;
#undef CIS2_VMW
  }
}

// Workgroup barrier for LDS data only: waits for this wave's LDS
// operations, not for its outstanding global loads (HIP's __syncthreads
// waits for those too).  The empty asm statements keep the compiler from
// moving memory accesses across the barrier.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Waits until the n tagged words addr(0..n-1) carry `epoch` and copies their
// values to dst(0..n-1).  The first PW waves poll, up to M words in flight
// per thread (longer vectors are gathered in slices).  Waves at or past PW,
// which may have weight or tile copies into LDS outstanding (loads complete
// in issue order, so a poll issued behind them would wait for them), do not
// poll: they wait for their copies and join the closing barrier.
template <int M = 12, uint32_t PW = 4, class F, class D>
__device__ __forceinline__ void gather_map(uint32_t n, uint32_t epoch, uint32_t* err,
                                           uint32_t cap, F addr, D dst) {
  constexpr uint32_t NT = PW * 64;
  const uint32_t tid = tid_x();
  if (tid < NT) {
    for (uint32_t base = 0; base < n; base += M * NT) {
      u64 w[M];
      uint32_t spins = 0;
      while (true) {
#pragma unroll
        for (int u = 0; u < M; ++u) {
          const uint32_t i = base + tid + u * NT;
          if (i < n) w[u] = get_word(addr(i));
        }
        bool ok = true;
#pragma unroll
        for (int u = 0; u < M; ++u) {
          const uint32_t i = base + tid + u * NT;
          if (i < n && (uint32_t)(w[u] >> 32) != epoch) ok = false;
        }
        if (ok) break;
        __builtin_amdgcn_s_sleep(1);
        ++spins;
        if ((spins & 255u) == 0 && ld_ag(err) != 0u) break;  // another task failed
        if (spins > cap) {  // a.spin_cap: about 0.5 s by default
          raise_err(err, 2u);
          break;
        }
      }
#pragma unroll
      for (int u = 0; u < M; ++u) {
        const uint32_t i = base + tid + u * NT;
        if (i < n) *dst(i) = __uint_as_float((uint32_t)w[u]);
      }
    }
    // every global_load_lds copy this wave issued before has landed in
    // LDS too (loads complete in issue order)
    wait_vm0();
  } else {
    wait_vm0();
  }
  __syncthreads();
}
// The same into dst[0..n-1].
template <int M = 12, uint32_t PW = 4, class F>
__device__ __forceinline__ void gather(lf* dst, uint32_t n, uint32_t epoch, uint32_t* err,
                                       uint32_t cap, F addr) {
  gather_map<M, PW>(n, epoch, err, cap, addr, [=](uint32_t i) { return dst + i; });
}

template <int M = 12, uint32_t PW = 4>
__device__ __forceinline__ void gather_vec(lf* dst, const gw* src, uint32_t n,
                                           const DecodeArgs& a) {
  gather<M, PW>(dst, n, a.epoch, a.err, a.spin_cap, [=](uint32_t i) { return src + i; });
}

// Copies n4 f4 (element i from src(i), global memory) to dst[i] with up to
// 36 loads in flight per thread: a 144 KiB block in one round trip per
// workgroup.
template <class F>
__device__ __forceinline__ void copy_to_lds(lf4* dst, uint32_t n4, F src) {
  constexpr uint32_t B = 36;
  for (uint32_t i = tid_x(); i < n4; i += B * kThreads) {
    f4 t[B];
#pragma unroll
    for (uint32_t u = 0; u < B; ++u)
      if (i + u * kThreads < n4) t[u] = *src(i + u * kThreads);
#pragma unroll
    for (uint32_t u = 0; u < B; ++u)
      if (i + u * kThreads < n4) dst[i + u * kThreads] = t[u];
  }
}

// n4 16-byte elements from src(i) (global) to dst(i) (LDS), up to 16 loads
// in flight per thread.
template <class F, class G>
__device__ __forceinline__ void copy_map(uint32_t n4, F src, G dst) {
  constexpr uint32_t B = 16;
  for (uint32_t i = tid_x(); i < n4; i += B * kThreads) {
    f4 t[B];
#pragma unroll
    for (uint32_t u = 0; u < B; ++u)
      if (i + u * kThreads < n4) t[u] = *src(i + u * kThreads);
#pragma unroll
    for (uint32_t u = 0; u < B; ++u)
      if (i + u * kThreads < n4) *dst(i + u * kThreads) = t[u];
  }
}

// Positions [j0, j0 + n) of the hd rows of one kv head's cache ([hd][max_pos]
// at `rows`) into LDS rows of stride TS; n is rounded up to 4 (the extra
// positions stay inside max_pos and are never used).
__device__ __forceinline__ void copy_cache_tile(lf* dst, const float* rows, uint32_t max_pos,
                                                uint32_t hd, uint32_t j0, uint32_t n,
                                                uint32_t TS) {
  const uint32_t nq = (n + 3) >> 2, mp4 = max_pos >> 2, ts4 = TS >> 2, j04 = j0 >> 2;
  gf4* r4 = G4(rows);
  lf4* d4 = (lf4*)dst;
  copy_map(hd * nq,
           [=](uint32_t i) {
             const uint32_t d = i / nq, q = i - d * nq;
             return r4 + (size_t)d * mp4 + j04 + q;
           },
           [=](uint32_t i) {
             const uint32_t d = i / nq, q = i - d * nq;
             return d4 + (size_t)d * ts4 + q;
           });
}

// In place rows[d][q] *= factor for the 16-byte groups q < nq of rows
// d < nrows (row stride s4 groups).  Short rows: items i = d*nq + q are
// spread over all threads, four per thread; long rows: lanes take a row's
// groups.  Either way the loads (row groups and factors) are issued before
// any product.  scale_rows_by_row multiplies row d by the scalar f[d]
// (scores: q[d] * k_j[d]); scale_rows_by_col multiplies group q by the four
// values f4[q] (V mix: p_j * v_j[d]).  Each product is f * v, one rounding.
template <bool BY_ROW>
__device__ __forceinline__ void scale_rows(lf4* rows, uint32_t s4, uint32_t nrows, uint32_t nq,
                                           const lf* f, const lf4* f4c) {
  if (nq >= 48) {
    // long rows: lanes take the groups of a row (most lanes busy), waves take
    // rows wv, wv + 4, ...; 8 rows' groups and factors are read first
    const uint32_t wv = tid_x() >> 6, lane = tid_x() & 63;
    constexpr uint32_t RB = 8;
    for (uint32_t q = lane; q < nq; q += 64) {
      f4 cq = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (!BY_ROW) cq = f4c[q];
      for (uint32_t d0 = wv; d0 < nrows; d0 += 4 * RB) {
        f4 v[RB], c[RB];
#pragma unroll
        for (uint32_t u = 0; u < RB; ++u) {
          if (d0 + 4 * u < nrows) {
            v[u] = rows[(size_t)(d0 + 4 * u) * s4 + q];
            if constexpr (BY_ROW) {
              const float fd = f[d0 + 4 * u];
              c[u] = f4{fd, fd, fd, fd};
            } else {
              c[u] = cq;
            }
          }
        }
#pragma unroll
        for (uint32_t u = 0; u < RB; ++u) {
          if (d0 + 4 * u < nrows) {
            f4 r;
            r.x = c[u].x * v[u].x;
            r.y = c[u].y * v[u].y;
            r.z = c[u].z * v[u].z;
            r.w = c[u].w * v[u].w;
            rows[(size_t)(d0 + 4 * u) * s4 + q] = r;
          }
        }
      }
    }
    return;
  }
  // short rows: items over all threads
  const uint32_t total = nrows * nq;
  constexpr uint32_t B = 4;
  for (uint32_t i0 = tid_x(); i0 < total; i0 += B * kThreads) {
    f4 v[B], c[B];
    uint32_t off[B];
#pragma unroll
    for (uint32_t u = 0; u < B; ++u) {
      const uint32_t i = min(i0 + u * kThreads, total - 1);  // past the end: re-read the last
      const uint32_t d = i / nq, q = i - d * nq;
      off[u] = d * s4 + q;
      v[u] = rows[off[u]];
      if constexpr (BY_ROW) {
        const float fd = f[d];
        c[u] = f4{fd, fd, fd, fd};
      } else {
        c[u] = f4c[q];
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < B; ++u) {
      if (i0 + u * kThreads < total) {
        f4 r;
        r.x = c[u].x * v[u].x;
        r.y = c[u].y * v[u].y;
        r.z = c[u].z * v[u].z;
        r.w = c[u].w * v[u].w;
        rows[off[u]] = r;
      }
    }
  }
}
__device__ __forceinline__ void scale_rows_by_row(lf4* rows, uint32_t s4, uint32_t nrows,
                                                  uint32_t nq, const lf* f) {
  scale_rows<true>(rows, s4, nrows, nq, f, nullptr);
}
__device__ __forceinline__ void scale_rows_by_col(lf4* rows, uint32_t s4, uint32_t nrows,
                                                  uint32_t nq, const lf4* f4c) {
  scale_rows<false>(rows, s4, nrows, nq, nullptr, f4c);
}

// Row block blk ([K/4][R][4] floats) of a blocked matrix into LDS.
__device__ __forceinline__ void prefetch_rows(const float* W, uint32_t R, uint32_t K, uint32_t blk,
                                              lf* dst) {
  const size_t blkf = (size_t)R * K;
  gf4* src = G4(W + blk * blkf);
  copy_to_lds((lf4*)dst, (uint32_t)(blkf / 4), [=](uint32_t i) { return src + i; });
}

// Row block blk into LDS without holding the waves: 16-byte global->LDS
// loads (global_load_lds_dwordx4); each wave instruction fills 64
// consecutive 16-byte slots.  The data is in LDS once vmcnt reaches 0, and
// readable by other waves after a barrier.
// Weight blocks are copied into LDS by waves 2 and 3 (the DMA waves) while
// waves 0 and 1 poll for the task's inputs.
__device__ __forceinline__ void prefetch_rows_async(const float* W, uint32_t R, uint32_t K,
                                                    uint32_t blk, lf* dst) {
  const uint32_t n4 = R * K / 4;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6), lane = tid_x() & 63;
  if (wv < 2) return;
  gf4* src = G4(W + (size_t)blk * R * K);
  for (uint32_t i0 = (wv - 2) * 64; i0 < n4; i0 += 128) {  // i0: wave-uniform
    if (i0 + lane < n4)
      __builtin_amdgcn_global_load_lds((const AS_GLB void*)(src + i0 + lane),
                                       (AS_LDS void*)((lf4*)dst + i0), 16, 0, 0);
  }
}

// ---------------------------------------------------------------------------
// Strict chains over LDS with reads kept in flight
// ---------------------------------------------------------------------------

// acc + p[0].x + p[0].y + ... + p[n-1].w (element i at p[i * st]), strictly
// left to right.  A ring of D reads stays in flight, so a step costs its four
// adds rather than an LDS round trip.  The ring is filled unconditionally
// (n >= D) and each slot is refilled right after its adds, in an order the
// scheduler may not change: that lets the wait before each step be
// lgkmcnt(D-1) instead of a full drain.
template <uint32_t D = 15>
__device__ __forceinline__ float chain4(const lf4* p, uint32_t n, uint32_t st, float acc) {
  if (n < D) {
    for (uint32_t g = 0; g < n; ++g) {
      const f4 v = p[(size_t)g * st];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
    return acc;
  }
  f4 ring[D];
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) ring[u] = p[(size_t)u * st];
  uint32_t g = 0;
  for (; g + 2 * D <= n; g += D) {
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      const f4 v = ring[u];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
      ring[u] = p[(size_t)(g + u + D) * st];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // ring holds [g, g + D) and D <= n - g < 2D
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) {
    const f4 v = ring[u];
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
    if (g + u + D < n) ring[u] = p[(size_t)(g + u + D) * st];
  }
  g += D;
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) {
    if (g + u < n) {
      const f4 v = ring[u];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
  }
  return acc;
}

// acc + p[0] + p[st] + ... + p[(n-1)*st], strictly in order, same ring scheme.
template <uint32_t D = 12>
__device__ __forceinline__ float chain1(const lf* p, uint32_t n, uint32_t st, float acc) {
  if (n < D) {
    for (uint32_t g = 0; g < n; ++g) acc = acc + p[(size_t)g * st];
    return acc;
  }
  float ring[D];
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) ring[u] = p[(size_t)u * st];
  uint32_t g = 0;
  for (; g + 2 * D <= n; g += D) {
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      acc = acc + ring[u];
      ring[u] = p[(size_t)(g + u + D) * st];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) {
    acc = acc + ring[u];
    if (g + u + D < n) ring[u] = p[(size_t)(g + u + D) * st];
  }
  g += D;
#pragma unroll
  for (uint32_t u = 0; u < D; ++u)
    if (g + u < n) acc = acc + ring[u];
  return acc;
}

// chain4's order with the reads in two register sets of U groups: the next
// set's reads go out before the current set's 4U adds, one wait per set (a
// ring waits before every group); no read past group n-1.  About 15-20 %
// fewer cycles per add than chain4 on chains of 100+ groups (isolated,
// MI355X); chain4 stays ahead on short chunks.
template <uint32_t U = 8>
__device__ __forceinline__ float chain_pp(const lf4* p, uint32_t n, uint32_t st, float acc) {
  auto add1 = [&](f4 v) {
    acc = acc + v.x;
    acc = acc + v.y;
    acc = acc + v.z;
    acc = acc + v.w;
  };
  if (n < U) {
    for (uint32_t g = 0; g < n; ++g) {
      const f4 v = p[(size_t)g * st];
      add1(v);
    }
    return acc;
  }
  f4 a[U], b[U];
#pragma unroll
  for (uint32_t u = 0; u < U; ++u) a[u] = p[(size_t)u * st];
  uint32_t g = 0;
  for (; g + 3 * U <= n; g += 2 * U) {
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) b[u] = p[(size_t)(g + U + u) * st];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) add1(a[u]);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) a[u] = p[(size_t)(g + 2 * U + u) * st];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (uint32_t u = 0; u < U; ++u) add1(b[u]);
    __builtin_amdgcn_sched_barrier(0);
  }
  // a holds groups g .. g+U-1; n - g in [U, 3U)
#pragma unroll
  for (uint32_t u = 0; u < U; ++u)
    if (g + U + u < n) b[u] = p[(size_t)(g + U + u) * st];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (uint32_t u = 0; u < U; ++u) add1(a[u]);
  g += U;
#pragma unroll
  for (uint32_t u = 0; u < U; ++u)
    if (g + u < n) add1(b[u]);
  g += U;
  for (; g < n; ++g) {
    const f4 v = p[(size_t)g * st];
    add1(v);
  }
  return acc;
}

// chain_pp's order over 16 * npair groups (16 bytes, ST groups apart, the
// group address per lane), as one assembly loop over two fixed sets of 8
// groups (v[192:223], v[224:255]): the next set's 8 reads go out, one wait
// for the current set (issued a set earlier), its 32 adds.  Left to the
// compiler, the same loop inside the decode kernel kept the sum or the
// loop address in a register of the set read last and drained the reads
// (lgkmcnt(0)) once or twice per 64 adds: 8 to 10 cycles per add against
// 6.1 here (MI355X, one wave, 4096 adds).  The block starts with a full
// drain, so the counts inside are exact (LDS reads return in order); it
// reads 8 groups past the range (never added: the caller keeps that LDS
// readable) and drains them before the registers are released.  The adds
// are the same IEEE adds in the same order and operand order.  npair >= 1,
// wave-uniform.
#define CIS2_LD(R0, R3, K, BASE) \
  "ds_read_b128 v[" #R0 ":" #R3 "], %[ad] offset:" BASE "+" #K "*%[s]\n\t"
#define CIS2_ADD4(A, B, C, D)                                                   \
  "v_add_f32 %[acc], v" #A ", %[acc]\n\tv_add_f32 %[acc], v" #B ", %[acc]\n\t" \
  "v_add_f32 %[acc], v" #C ", %[acc]\n\tv_add_f32 %[acc], v" #D ", %[acc]\n\t"
#define CIS2_SET_A(BASE) CIS2_LD(192, 195, 0, BASE) CIS2_LD(196, 199, 1, BASE) CIS2_LD(200, 203, 2, BASE) CIS2_LD(204, 207, 3, BASE) CIS2_LD(208, 211, 4, BASE) CIS2_LD(212, 215, 5, BASE) CIS2_LD(216, 219, 6, BASE) CIS2_LD(220, 223, 7, BASE)
#define CIS2_SET_B(BASE) CIS2_LD(224, 227, 0, BASE) CIS2_LD(228, 231, 1, BASE) CIS2_LD(232, 235, 2, BASE) CIS2_LD(236, 239, 3, BASE) CIS2_LD(240, 243, 4, BASE) CIS2_LD(244, 247, 5, BASE) CIS2_LD(248, 251, 6, BASE) CIS2_LD(252, 255, 7, BASE)
#define CIS2_ADDS_A CIS2_ADD4(192, 193, 194, 195) CIS2_ADD4(196, 197, 198, 199) CIS2_ADD4(200, 201, 202, 203) CIS2_ADD4(204, 205, 206, 207) CIS2_ADD4(208, 209, 210, 211) CIS2_ADD4(212, 213, 214, 215) CIS2_ADD4(216, 217, 218, 219) CIS2_ADD4(220, 221, 222, 223)
#define CIS2_ADDS_B CIS2_ADD4(224, 225, 226, 227) CIS2_ADD4(228, 229, 230, 231) CIS2_ADD4(232, 233, 234, 235) CIS2_ADD4(236, 237, 238, 239) CIS2_ADD4(240, 241, 242, 243) CIS2_ADD4(244, 245, 246, 247) CIS2_ADD4(248, 249, 250, 251) CIS2_ADD4(252, 253, 254, 255)
template <uint32_t ST>
__device__ __forceinline__ float chain_lds16(const AS_LDS void* p, uint32_t npair, float acc) {
  uint32_t ad = (uint32_t)(uintptr_t)p;
  asm volatile(
      "s_waitcnt lgkmcnt(0)\n\t" CIS2_SET_A("0")
      "1:\n\t" CIS2_SET_B("8*%[s]")
      "s_waitcnt lgkmcnt(8)\n\t" CIS2_ADDS_A
      "v_add_u32 %[ad], 16*%[s], %[ad]\n\t" CIS2_SET_A("0")
      "s_waitcnt lgkmcnt(8)\n\t" CIS2_ADDS_B
      "s_sub_u32 %[n], %[n], 1\n\t"
      "s_cmp_lg_u32 %[n], 0\n\t"
      "s_cbranch_scc1 1b\n\t"
      "s_waitcnt lgkmcnt(0)"
      : [acc] "+v"(acc), [ad] "+v"(ad), [n] "+s"(npair)
      : [s] "i"(ST * 16)
      : "memory", "scc", "v192", "v193", "v194", "v195", "v196", "v197", "v198", "v199", "v200", "v201", "v202", "v203", "v204", "v205", "v206", "v207", "v208", "v209", "v210", "v211", "v212", "v213", "v214", "v215", "v216", "v217", "v218", "v219", "v220", "v221", "v222", "v223", "v224", "v225", "v226", "v227", "v228", "v229", "v230", "v231", "v232", "v233", "v234", "v235", "v236", "v237", "v238", "v239", "v240", "v241", "v242", "v243", "v244", "v245", "v246", "v247", "v248", "v249", "v250", "v251", "v252", "v253", "v254", "v255");
  return acc;
}
#undef CIS2_LD
#undef CIS2_ADD4
#undef CIS2_SET_A
#undef CIS2_SET_B
#undef CIS2_ADDS_A
#undef CIS2_ADDS_B

// Strict sum of n contiguous LDS floats (16-byte aligned; 32 readable
// floats after them).
__device__ __forceinline__ float chain_vec(const lf* p, uint32_t n, float acc) {
  const uint32_t np = __builtin_amdgcn_readfirstlane(n >> 6);
  if (np > 0) {
    acc = chain_lds16<1>(p, np, acc);
    p += (size_t)np * 64;
    n -= np * 64;
  }
  acc = chain_pp(reinterpret_cast<const lf4*>(p), n >> 2, 1, acc);
  for (uint32_t i = n & ~3u; i < n; ++i) acc = acc + p[i];
  return acc;
}

// chain4's order with reads past the end allowed: the caller keeps D
// groups of readable LDS after group n-1 (at the same stride), so the ring
// is refilled unconditionally at fixed offsets (no address arithmetic and
// no branches per step; the extra reads are never added); the last partial
// round adds its groups under uniform tests.  n wave-uniform.
template <uint32_t D = 8>
__device__ __forceinline__ float chain4s(const lf4* p, uint32_t n, uint32_t st, float acc) {
  f4 ring[D];
#pragma unroll
  for (uint32_t u = 0; u < D; ++u) ring[u] = p[(size_t)u * st];
  uint32_t g = 0;
  for (; g + D <= n; g += D) {
#pragma unroll
    for (uint32_t u = 0; u < D; ++u) {
      const f4 v = ring[u];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
      ring[u] = p[(size_t)(g + u + D) * st];
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (uint32_t u = 0; u + 1 < D; ++u) {
    if (g + u < n) {
      const f4 v = ring[u];
      acc = acc + v.x;
      acc = acc + v.y;
      acc = acc + v.z;
      acc = acc + v.w;
    }
  }
  return acc;
}

// Strict sum of n contiguous LDS floats (16-byte aligned) with 60 readable
// floats after them.
__device__ __forceinline__ float chain_vec_s(const lf* p, uint32_t n, float acc) {
  acc = chain4s<15>(reinterpret_cast<const lf4*>(p), n >> 2, 1, acc);
  for (uint32_t i = n & ~3u; i < n; ++i) acc = acc + p[i];
  return acc;
}

// ---------------------------------------------------------------------------
// GEMV on LDS-resident row blocks ([K/4][R][4] floats per block)
// ---------------------------------------------------------------------------

// Product pass over wave instructions [i0, i1) of nb blocks (block b at
// W4 + b*bf4): instruction `ins` covers groups [ins*GP, ins*GP + GP)
// (GP = 64/R), lane l forming W[g][r] *= x4[g] for g = ins*GP + l/R,
// r = l%R.  Lanes past GP*R, or past the last group, read and write their
// own slot of `pad` instead, so no lane is ever masked off.  Waves w, w+nw,
// ... (w wave-uniform) take turns over the instructions; the reads of B
// instructions are issued before their writes (in-place writes would
// otherwise order every read behind the previous write).
#ifndef PROD_BATCH
#define PROD_BATCH 12
#endif
template <uint32_t R>
__device__ __forceinline__ void prod_ins(lf4* W4, const lf4* x4, uint32_t bf4, uint32_t nb,
                                         uint32_t KG, uint32_t i0, uint32_t i1, uint32_t w,
                                         uint32_t nw, lf4* pad) {
  constexpr uint32_t GP = 64 / R, B = PROD_BATCH;
  const uint32_t lane = tid_x() & 63;
  const uint32_t lg = lane / R, lr = lane - (lane / R) * R;
  const bool live = lane < GP * R;
  for (uint32_t b = 0; b < nb; ++b) {
    lf4* base = W4 + (size_t)b * bf4;
    for (uint32_t ins = i0 + w; ins < i1; ins += B * nw) {
      lf4* dst[B];
      f4 wv[B], xv[B];
#pragma unroll
      for (uint32_t u = 0; u < B; ++u) {
        const uint32_t ii = ins + u * nw;
        const uint32_t g = ii * GP + lg;
        const bool ok = live && g < KG;
        dst[u] = ok ? base + (size_t)g * R + lr : pad + lane;
        const lf4* xs = ok ? x4 + g : (const lf4*)(pad + lane);
        if (ii < i1) {
          wv[u] = *dst[u];
          xv[u] = *xs;
        }
      }
#pragma unroll
      for (uint32_t u = 0; u < B; ++u) {
        if (ins + u * nw < i1) {
          f4 v = wv[u];
          v.x = v.x * xv[u].x;
          v.y = v.y * xv[u].y;
          v.z = v.z * xv[u].z;
          v.w = v.w * xv[u].w;
          *dst[u] = v;
        }
      }
    }
  }
}

// y[r] = fold_k (W[r][k] * x[k]) for nb LDS blocks (block b at W + b*R*K).
// The product pass is cut into NC chunks of wave instructions: all waves
// form chunk 0, then waves [0, nb) add chunk c (a strict chain per lane,
// reads kept in flight) while the other waves form chunk c+1.  Returns row
// `lane` of block `wave` in waves < nb (lanes >= R: row R-1).
template <uint32_t R, uint32_t CD = 8>
__device__ __forceinline__ float gemv_lds_t(lf* W, const lf* x, uint32_t K, uint32_t nb,
                                            lf4* pad) {
  constexpr uint32_t NC = 4, GP = 64 / R;
  // sizes are wave-uniform: keep them (and every bound derived from them) scalar
  const uint32_t KG = __builtin_amdgcn_readfirstlane(K >> 2), lane = tid_x() & 63;
  nb = __builtin_amdgcn_readfirstlane(nb);
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  lf4* W4 = (lf4*)W;
  const lf4* x4 = (const lf4*)x;
  const uint32_t bf4 = KG * R, nins = (KG + GP - 1) / GP;
  const uint32_t r = lane < R ? lane : R - 1;
  prod_ins<R>(W4, x4, bf4, nb, KG, 0, nins / NC, wv, kThreads / 64, pad);
  lds_barrier();
  float acc = 0.0f;
  for (uint32_t c = 0; c < NC; ++c) {
    const uint32_t i0 = nins * c / NC, i1 = nins * (c + 1) / NC;
    if (wv < nb) {
      const uint32_t g0 = i0 * GP, g1 = min(i1 * GP, KG);
      const lf4* cp = W4 + (size_t)wv * bf4 + (size_t)g0 * R + r;
      // CD = 0: chain_lds16's pairs, then chain_pp (8 groups of readable
      // LDS past each chunk at stride R), else a ring of CD
      if constexpr (CD == 0) {
        const uint32_t ng = g1 - g0, np = ng >> 4;
        if (np > 0) acc = chain_lds16<R>(cp, np, acc);
        acc = chain_pp(cp + (size_t)np * 16 * R, ng - np * 16, R, acc);
      }
      else
        acc = chain4<CD>(cp, g1 - g0, R, acc);
    } else if (c + 1 < NC) {
      prod_ins<R>(W4, x4, bf4, nb, KG, i1, nins * (c + 2) / NC, wv - nb, kThreads / 64 - nb,
                  pad);
    }
    lds_barrier();
  }
  return acc;
}

// Same order for any other block height (runtime stride, no overlap).
__device__ float gemv_lds_any(uint32_t R, lf* W, const lf* x, uint32_t K, uint32_t nb) {
  const uint32_t KG = K >> 2, wv = tid_x() >> 6, lane = tid_x() & 63;
  lf4* W4 = (lf4*)W;
  const lf4* x4 = (const lf4*)x;
  const uint32_t bf4 = KG * R;
  for (uint32_t i = tid_x(); i < nb * bf4; i += kThreads) {
    const f4 xv = x4[(i % bf4) / R];
    f4 w = W4[i];
    w.x = w.x * xv.x;
    w.y = w.y * xv.y;
    w.z = w.z * xv.z;
    w.w = w.w * xv.w;
    W4[i] = w;
  }
  __syncthreads();
  float acc = 0.0f;
  if (wv < nb) acc = chain4(W4 + (size_t)wv * bf4 + (lane < R ? lane : R - 1), KG, R, 0.0f);
  __syncthreads();
  return acc;
}

__device__ __noinline__ float gemv_lds_generic(uint32_t R, lf* W, const lf* x, uint32_t K,
                                               uint32_t nb) {
  return gemv_lds_any(R, W, x, K, nb);
}

// Inlined GEMV for the block heights a call site can see (the persistent
// kernel's layouts: R = min(32, 36864/K), gate/up R/2); any other height
// takes the generic out-of-line path.
template <uint32_t CD, uint32_t R0, uint32_t... Rs>
__device__ __forceinline__ float gemv_lds(uint32_t R, lf* W, const lf* x, uint32_t K, uint32_t nb,
                                          lf4* pad) {
  if (R == R0) return gemv_lds_t<R0, CD>(W, x, K, nb, pad);
  if constexpr (sizeof...(Rs) > 0) {
    return gemv_lds<CD, Rs...>(R, W, x, K, nb, pad);
  } else {
    return gemv_lds_generic(R, W, x, K, nb);
  }
}

// Tree order (v0.4 candidate, code/cis2-fp/src/math.rs:60-125) on LDS row
// blocks: item (block b, k block kb, row r) forms its row's 32 products
// W[r][k] * x[k], k in [32kb, 32kb + 32), in registers (+0 past K), reduces
// them by tree32 and leaves the result in its first weight slot; lane r of
// wave b then folds its row's block results from 0.  Each product is one
// rounding, so forming them in the item gives the bits of a separate product
// pass, with a quarter of its LDS traffic (the weights are read once, x by
// broadcast, no products written back).  R = 0: height given at run time (Rr).
template <uint32_t R>
__device__ __forceinline__ float gemv_tree_t(uint32_t Rr, lf* W, const lf* x, uint32_t K,
                                             uint32_t nb, lf4* pad) {
  const uint32_t Rv = R ? R : Rr;
  const uint32_t KG = __builtin_amdgcn_readfirstlane(K >> 2), lane = tid_x() & 63;
  nb = __builtin_amdgcn_readfirstlane(nb);
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  lf4* W4 = (lf4*)W;
  const lf4* x4 = (const lf4*)x;
  const uint32_t bf4 = KG * Rv;
  const uint32_t KB = (KG + 7) / 8, items = nb * KB * Rv;
  for (uint32_t it = tid_x(); it < items; it += kThreads) {
    const uint32_t r = it % Rv, q = it / Rv, kb = q % KB, b = q / KB;
    lf4* p = W4 + (size_t)b * bf4 + (size_t)kb * 8 * Rv + r;
    const lf4* xp = x4 + (size_t)kb * 8;
    f4 wv4[8], xv4[8];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      if (kb * 8 + j < KG) {
        wv4[j] = p[(size_t)j * Rv];
        xv4[j] = xp[j];
      }
    }
    float lv[32];
#pragma unroll
    for (uint32_t j = 0; j < 8; ++j) {
      const bool in = kb * 8 + j < KG;
      lv[4 * j] = in ? wv4[j].x * xv4[j].x : 0.0f;
      lv[4 * j + 1] = in ? wv4[j].y * xv4[j].y : 0.0f;
      lv[4 * j + 2] = in ? wv4[j].z * xv4[j].z : 0.0f;
      lv[4 * j + 3] = in ? wv4[j].w * xv4[j].w : 0.0f;
    }
    ((lf*)p)[0] = tree32(lv);
  }
  lds_barrier();
  float acc = 0.0f;
  if (wv < nb)
    acc = chain1((const lf*)(W4 + (size_t)wv * bf4 + (lane < Rv ? lane : Rv - 1)), KB, 32 * Rv,
                 0.0f);
  lds_barrier();
  return acc;
}

__device__ __noinline__ float gemv_tree_generic(uint32_t R, lf* W, const lf* x, uint32_t K,
                                                uint32_t nb, lf4* pad) {
  return gemv_tree_t<0>(R, W, x, K, nb, pad);
}

template <uint32_t R0, uint32_t... Rs>
__device__ __forceinline__ float gemv_tree(uint32_t R, lf* W, const lf* x, uint32_t K,
                                           uint32_t nb, lf4* pad) {
  if (R == R0) return gemv_tree_t<R0>(R, W, x, K, nb, pad);
  if constexpr (sizeof...(Rs) > 0) {
    return gemv_tree<Rs...>(R, W, x, K, nb, pad);
  } else {
    return gemv_tree_generic(R, W, x, K, nb, pad);
  }
}

// The GEMV of a call site in the reduction order TR selects; CD: reads kept
// in flight by the sequential order's chain.
template <bool TR, uint32_t CD, uint32_t... Rs>
__device__ __forceinline__ float gemv_sel(uint32_t R, lf* W, const lf* x, uint32_t K,
                                          uint32_t nb, lf4* pad) {
  if constexpr (TR) {
    return gemv_tree<Rs...>(R, W, x, K, nb, pad);
  } else {
    return gemv_lds<CD, Rs...>(R, W, x, K, nb, pad);
  }
}

// tree32 over the LDS values p[i * st], i < min(n, 32) (+0 past n).
__device__ __forceinline__ float tree_part(const lf* p, uint32_t n, uint32_t st) {
  float lv[32];
#pragma unroll
  for (uint32_t i = 0; i < 32; ++i) lv[i] = i < n ? p[(size_t)i * st] : 0.0f;
  return tree32(lv);
}
// tree_part of 32 contiguous 16-byte-aligned floats, the whole block
// readable (the values past n count as +0).
__device__ __forceinline__ float tree_part_v(const lf* p, uint32_t n) {
  float lv[32];
  const lf4* p4 = (const lf4*)p;
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    const f4 v = p4[i];
    lv[4 * i] = v.x;
    lv[4 * i + 1] = v.y;
    lv[4 * i + 2] = v.z;
    lv[4 * i + 3] = v.w;
  }
#pragma unroll
  for (uint32_t i = 0; i < 32; ++i) lv[i] = i < n ? lv[i] : 0.0f;
  return tree32(lv);
}
// Tree-order sum over n strided LDS values p[i * st] (scores: one column of
// products): 32-value blocks by tree32, the block results folded from acc.
__device__ __forceinline__ float tree_col(const lf* p, uint32_t n, uint32_t st, float acc) {
  for (uint32_t i0 = 0; i0 < n; i0 += 32) acc = acc + tree_part(p + (size_t)i0 * st, n - i0, st);
  return acc;
}

// RMSNorm of an LDS vector (code/cis2-fp/src/main.rs:245-260): squares
// into `tmp`, one strict chain in wave 0, mean by a true divide,
// inv = 1/sqrt(mean + eps), out = (x*inv)*w.  `out` may alias `tmp` or x.
// Waves 0 and 1 scale: the norm weights a thread scales with (elements
// tid_x() + 128u) are loaded into registers before the input is waited for
// (load_normw), so the scaling pass after the chain reads no global memory
// (n <= 1024; longer vectors read the tail from global memory).  Waves 2
// and 3 load nothing here: a load issued behind their weight copies would
// wait for every copy.
constexpr uint32_t kNormRegs = 8, kNormThreads = 128;
struct NormW {
  float v[kNormRegs];
  const float* g;
};
__device__ __forceinline__ NormW load_normw(const float* w_, uint32_t n) {
  NormW r;
  r.g = w_;
  gf* w = G(w_);
  const uint32_t tid = tid_x();
#pragma unroll
  for (uint32_t u = 0; u < kNormRegs; ++u) {
    const uint32_t i = tid + u * kNormThreads;
    r.v[u] = tid < kNormThreads && i < n ? w[i] : 0.0f;
  }
  return r;
}
// Tree order (TR): the squares of block t of 32 are reduced by tree32 into
// tmp[t], and the block results folded from 0.
template <bool TR>
__device__ __forceinline__ void rmsnorm_lds(const lf* x, const NormW& w, float eps, uint32_t n,
                                            lf* tmp, lf* out, lf* s_inv) {
  const uint32_t nb = (n + 31) / 32;
  if constexpr (TR) {
    for (uint32_t t = tid_x(); t < nb; t += kThreads) {
      float lv[32];
#pragma unroll
      for (uint32_t i = 0; i < 32; ++i) {
        const float v = 32 * t + i < n ? x[32 * t + i] : 0.0f;
        lv[i] = v * v;
      }
      tmp[t] = tree32(lv);
    }
  } else {
    for (uint32_t i = tid_x(); i < n; i += kThreads) {
      float v = x[i];
      tmp[i] = v * v;
    }
  }
  __syncthreads();
  if (tid_x() < 64) {
    const float acc = TR ? chain1(tmp, nb, 1, 0.0f) : chain_vec(tmp, n, 0.0f);
    float mean = acc / (float)n;
    float arg = mean + eps;
    float inv = rsqrt_cr(arg);
    if (tid_x() == 0) *s_inv = inv;
  }
  __syncthreads();
  const float inv = *s_inv;
  const uint32_t tid = tid_x();
  if (tid < kNormThreads) {
#pragma unroll
    for (uint32_t u = 0; u < kNormRegs; ++u) {
      const uint32_t i = tid + u * kNormThreads;
      if (i < n) {
        float sx = x[i] * inv;
        out[i] = sx * w.v[u];
      }
    }
    for (uint32_t i = tid + kNormRegs * kNormThreads; i < n; i += kNormThreads) {
      float sx = x[i] * inv;
      out[i] = sx * G(w.g)[i];
    }
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
// DPP min step (dpp_move, max_step and wave_max: cis2_device_math.hpp).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t min_step(uint32_t x) {
  const uint32_t y = dpp_move<CTRL, ROWMASK>(x, x);
  return y < x ? y : x;
}
__device__ __forceinline__ uint32_t wave_min(uint32_t x) {
  x = min_step<0x111, 0xF>(x);
  x = min_step<0x112, 0xF>(x);
  x = min_step<0x114, 0xF>(x);
  x = min_step<0x118, 0xF>(x);
  x = min_step<0x142, 0xA>(x);
  x = min_step<0x143, 0xC>(x);
  return __builtin_amdgcn_readlane(x, 63);
}
// The wave's cand_pick winner in registers: the largest value, then the
// lowest index holding a value equal to it (+0 == -0, as the strict-> scan
// sees them).  The returned value may be either zero of a +-0 tie; callers
// that need the winner's own bits re-read them at the index.
__device__ __forceinline__ Cand cand_wave_dpp(Cand c) {
  const float m = wave_max(c.i == UINT32_MAX ? -__builtin_inff() : c.v);
  const uint32_t i = (c.i != UINT32_MAX && c.v == m) ? c.i : UINT32_MAX;
  return Cand{m, wave_min(i)};
}
// Block-wide pick over the 4 waves' candidates (scratch: 8 words in LDS).
__device__ __forceinline__ Cand cand_block(Cand c, AS_LDS uint32_t* red) {
  c = cand_wave_dpp(c);
  if ((tid_x() & 63) == 0) {
    red[2 * (tid_x() >> 6)] = __float_as_uint(c.v);
    red[2 * (tid_x() >> 6) + 1] = c.i;
  }
  __syncthreads();
  Cand b = {__uint_as_float(red[0]), red[1]};
  for (uint32_t i = 1; i < kThreads / 64; ++i)
    b = cand_pick(b, Cand{__uint_as_float(red[2 * i]), red[2 * i + 1]});
  __syncthreads();
  return b;
}

// LDS layout: [weights | vectors].
struct Lds {
  lf* w;     // weight block(s); attention: scores, K rows, V rows
  lf* v;     // the task's input vector(s) and scratch
  lf4* pad;  // 64 slots the product pass's idle lanes write instead
};

// ---------------------------------------------------------------------------
// Phase tasks
// ---------------------------------------------------------------------------

struct QkvGeom {
  const float* W;
  const float* bias;
  gw* out;
  uint32_t M, blk;
};
__device__ __forceinline__ QkvGeom qkv_geom(const DecodeArgs& a, const LayerW& Lw, const Act& ac,
                                            uint32_t t) {
  if (t < a.nq_q) return QkvGeom{Lw.wq, Lw.bq, ac.q, a.qd, t};
  if (t < a.nq_q + a.nq_k) return QkvGeom{Lw.wk, Lw.bk, ac.k, a.kvd, t - a.nq_q};
  return QkvGeom{Lw.wv, Lw.bv, ac.v, a.kvd, t - a.nq_q - a.nq_k};
}

// One row block of q, k or v: input_layernorm, GEMV, bias (main.rs:405-413).
template <bool TR>
__device__ __forceinline__ void run_qkv(const DecodeArgs& a, uint32_t l, uint32_t t, const Lds& s,
                                       uint32_t tok, lf* wl, bool pre) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const QkvGeom g = qkv_geom(a, Lw, ac, t);
  lf* x = s.v;
  lf* ln = s.v + a.H;
  lf* s_inv = s.v + 2 * a.H;
  if (!pre) prefetch_rows_async(g.W, a.Rq, a.H, g.blk, wl);
  const NormW nw = load_normw(Lw.ln1, a.H);
  stamp(a, l, P_QKV, t, 0);
  if (l == 0) {
    gf* e = G(a.embed) + (size_t)tok * a.H;
    for (uint32_t i = tid_x(); i < a.H; i += kThreads) x[i] = e[i];
    __syncthreads();
  } else {
    gather_vec<8, 2>(x, act_of(a, l - 1).hout, a.H, a);
  }
  stamp(a, l, P_QKV, t, 1);
  rmsnorm_lds<TR>(x, nw, a.eps, a.H, ln, ln, s_inv);
  stamp(a, l, P_QKV, t, 3);
  const float acc = gemv_sel<TR, 8, 32, 8, 16>(a.Rq, wl, ln, a.H, 1, s.pad);
  const uint32_t row = g.blk * a.Rq + tid_x();
  if (tid_x() < a.Rq && row < g.M) {
    const float r = g.bias ? acc + G(g.bias)[row] : acc;
    put_word(g.out + row, r, a.epoch);
  }
  stamp(a, l, P_QKV, t, 2);
}

// Copies positions [0, pos) of one kv head's cached K and V (both
// [hd][max_pos] in HBM, written by earlier launches) into LDS: K transposed
// into rows of KS floats, one per position (kt[j * KS + d] = k_j[d]), V as
// rows of stride S, one per head dim (vl[d * S + j] = v_j[d]).  Positions up
// to pos rounded to 4 are copied; the ones >= pos are never used.  The
// global reads run along positions (16 bytes per thread, 16 in flight).
__device__ __forceinline__ void prefetch_kv(const DecodeArgs& a, uint32_t l, uint32_t kvh, lf* kt,
                                            uint32_t KS, lf* vl, uint32_t S) {
  const uint32_t hd = a.hd, kq = (a.pos + 3) >> 2, mp4 = a.max_pos >> 2, n4 = hd * kq;
  gf4* kc = G4(a.kc0 + (size_t)l * a.cache_stride);
  gf4* kb = kc + (size_t)kvh * hd * mp4;
  gf4* vb = kc + (size_t)a.kvd * mp4 + (size_t)kvh * hd * mp4;
  lf4* v4 = (lf4*)vl;
  const uint32_t s4 = S >> 2;
  constexpr uint32_t B = 16;
  for (uint32_t i0 = tid_x(); i0 < n4; i0 += B * kThreads) {
    f4 tk[B], tv[B];
#pragma unroll
    for (uint32_t u = 0; u < B; ++u) {
      const uint32_t i = i0 + u * kThreads;
      if (i < n4) {
        const uint32_t d = i / kq, q = i - d * kq;
        tk[u] = kb[(size_t)d * mp4 + q];
        tv[u] = vb[(size_t)d * mp4 + q];
      }
    }
#pragma unroll
    for (uint32_t u = 0; u < B; ++u) {
      const uint32_t i = i0 + u * kThreads;
      if (i < n4) {
        const uint32_t d = i / kq, q = i - d * kq;
        lf* dst = kt + (size_t)(4 * q) * KS + d;
        dst[0] = tk[u].x;
        dst[KS] = tk[u].y;
        dst[2 * KS] = tk[u].z;
        dst[3 * KS] = tk[u].w;
        v4[(size_t)d * s4 + q] = tv[u];
      }
    }
  }
}

// dot(q, k) * 1 over hd head dims in the order TR selects (q and k: LDS,
// 16-byte aligned, hd a multiple of 4): blocks of 32 products, each summed
// in order from the running value (dot_seq) or reduced by tree32 and added
// (dot_tree).  Every product is one rounding, so forming a block's
// products before its adds gives dot_seq's bits.
template <bool TR>
__device__ __forceinline__ float score_dot(const lf* q, const lf* k, uint32_t hd) {
  const lf4* q4 = (const lf4*)q;
  const lf4* k4 = (const lf4*)k;
  float acc = 0.0f;
  for (uint32_t b = 0; b < hd; b += 32) {
    float p[32];
#pragma unroll
    for (uint32_t g = 0; g < 8; ++g) {
      const uint32_t d = b + 4 * g;
      f4 qv = {0.0f, 0.0f, 0.0f, 0.0f}, kv = {0.0f, 0.0f, 0.0f, 0.0f};
      if (d < hd) {
        qv = q4[d >> 2];
        kv = k4[d >> 2];
      }
      p[4 * g] = d < hd ? qv.x * kv.x : 0.0f;
      p[4 * g + 1] = d < hd ? qv.y * kv.y : 0.0f;
      p[4 * g + 2] = d < hd ? qv.z * kv.z : 0.0f;
      p[4 * g + 3] = d < hd ? qv.w * kv.w : 0.0f;
    }
    if constexpr (TR) {
      acc = acc + tree32(p);
    } else {
      const uint32_t n = hd - b < 32 ? hd - b : 32;
#pragma unroll
      for (uint32_t i = 0; i < 32; ++i)
        if (i < n) acc = acc + p[i];
    }
  }
  return acc;
}

// Attention for query head h (code/cis2-fp/src/main.rs:415-467).
// The inputs of query head h at this position, in LDS: q at qv[0..hd), the
// head's k at qv[hd..2hd), v at qv[2hd..3hd) (gathered from the QKV tasks),
// then Qwen3's per-head QK-norm (after bias, before RoPE;
// labs/w1x-qwen3/scripts/qwen3-port.diff:66-80) and RoPE rotate-half of q
// and k (main.rs:285-307): o1 = x1*c + (-x2)*s, o2 = x2*c + x1*s.  Ends with
// a barrier.  tmp and misc: hd and 64 floats of scratch.
template <bool TR>
__device__ __forceinline__ void att_head_inputs(const DecodeArgs& a, uint32_t l, uint32_t h,
                                                lf* qv, lf* tmp, lf* misc) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const uint32_t hd = a.hd, kvh = h / (a.nh / a.nkv), pos = a.pos;
  lf* kv = qv + hd;
  NormW nq, nk;
  if (Lw.qn) nq = load_normw(Lw.qn, hd);
  if (Lw.kn) nk = load_normw(Lw.kn, hd);
  // cos/sin of this position for the pair this thread rotates (hd <= 256)
  const uint32_t half = hd / 2;
  float rc = 0.0f, rsn = 0.0f;
  if (tid_x() < 2 * half) {
    const uint32_t i = tid_x() < half ? tid_x() : tid_x() - half;
    gf* cs = G(a.rope_cs) + (size_t)pos * half * 2;
    rc = cs[2 * i];
    rsn = cs[2 * i + 1];
  }
  gather(qv, 3 * hd, a.epoch, a.err, a.spin_cap, [=](uint32_t i) {
    const uint32_t seg = i >= hd ? (i >= 2 * hd ? 2u : 1u) : 0u, d = i - seg * hd;
    return seg == 0 ? ac.q + (size_t)h * hd + d
                    : (seg == 1 ? ac.k : ac.v) + (size_t)kvh * hd + d;
  });
  if (Lw.qn) rmsnorm_lds<TR>(qv, nq, a.eps, hd, tmp, qv, misc);
  if (Lw.kn) rmsnorm_lds<TR>(kv, nk, a.eps, hd, tmp, kv, misc);
  if (tid_x() < 2 * half) {
    const uint32_t idx = tid_x();
    lf* hv = idx < half ? qv : kv;
    uint32_t i = idx < half ? idx : idx - half;
    float c = rc, sn = rsn;
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
}

// softmax over ss[0..len) in place: first-wins max, pinned exp, the
// denominator as one strict chain (softmax_seq, math.rs:425-442) or tree32
// block results folded from 0 (softmax_tree, math.rs:448-465; partials at
// part[0..ceil(len/32))), then a true divide.  misc[1] and red: scratch.
// Starts after and ends with a barrier.
template <bool TR>
__device__ __forceinline__ void softmax_lds(lf* ss, uint32_t len, lf* part, lf* misc,
                                            AS_LDS uint32_t* red) {
  Cand best = {0.0f, UINT32_MAX};
  for (uint32_t j = tid_x(); j < len; j += kThreads) {
    float v = ss[j];
    if (v == v) best = cand_pick(best, Cand{v, j});
  }
  const Cand b = cand_block(best, red);
  // the first maximum's own bits (a NaN at position 0 wins outright)
  const float mx = (ss[0] != ss[0] || b.i == UINT32_MAX) ? ss[0] : ss[b.i];
  for (uint32_t j = tid_x(); j < len; j += kThreads) {
    float dlt = ss[j] - mx;
    ss[j] = exp_pinned(dlt);
  }
  __syncthreads();
  if constexpr (TR) {
    const uint32_t nbk = (len + 31) / 32;
    for (uint32_t t = tid_x(); t < nbk; t += kThreads)
      part[t] = tree_part(ss + 32 * t, len - 32 * t, 1);
    __syncthreads();
    if (tid_x() < 64) {
      const float acc = chain1(part, nbk, 1, 0.0f);
      if (tid_x() == 0) misc[1] = acc;
    }
  } else if (tid_x() < 64) {
    const float acc = chain_vec(ss, len, 0.0f);
    if (tid_x() == 0) misc[1] = acc;
  }
  __syncthreads();
  const float den = misc[1];
  for (uint32_t j = tid_x(); j < len; j += kThreads) {
    float pj = ss[j] / den;
    ss[j] = pj;
  }
  __syncthreads();
}

// The rotated k and the raw v of this position into kv head kvh's caches.
__device__ __forceinline__ void store_kv_pos(const DecodeArgs& a, uint32_t l, uint32_t kvh,
                                             const lf* kv, const lf* vv) {
  AS_GLB float* kc = GW(a.kc0 + (size_t)l * a.cache_stride);
  AS_GLB float* vc = GW(a.vc0 + (size_t)l * a.cache_stride);
  for (uint32_t d = tid_x(); d < a.hd; d += kThreads) {
    kc[((size_t)kvh * a.hd + d) * a.max_pos + a.pos] = kv[d];
    vc[((size_t)kvh * a.hd + d) * a.max_pos + a.pos] = vv[d];
  }
}

// Orders this wave's LDS writes before its later LDS reads by other lanes
// (a wave's LDS operations complete in issue order; this keeps the compiler
// from moving accesses across the point).
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Softmax and V mix of one head by the whole workgroup, after the scores
// of positions 0..pos are in ss[] (written before a barrier):
//  1. every wave finds the maximum over all scores itself (a DPP wave
//     reduction over the non-NaN scores; a NaN at position 0, or scores
//     that are all NaN, give NaN): no cross-wave step.  This is the value
//     of the first maximum; where its bits could differ (+0 against -0),
//     e_j = exp(s_j - max) does not: both give exp(+-0) = 1;
//  2. the pinned exp of every position, spread over the block;
//  3. wave 0 forms the denominator (a strict chain, or tree32 blocks folded
//     from 0; partials in `part`) into misc[1];
//  4. the true divide p_j = e_j / den, spread over the block;
//  5. lane d of the chain waves (one wave per 64 dims) runs the V mix
//     out_d = fold_j (p_j * v_j[d]) over its cached V row in LDS (row d at
//     vl + d*S, positions < pos) and then this position's own v: it forms
//     each product itself, p_j taken by DPP broadcast (row_newbcast) from a
//     register that holds 16 consecutive probabilities in every 16-lane
//     row, the next 16 positions' reads in flight.
// A barrier separates steps 1-4.  hd <= 192.  The chains read up to 60
// floats past the scores and up to 32 past the last V row (the scores
// region has 64 spare floats; the vector region follows the V rows).
// Lane k of this lane's 16-lane row (DPP row_newbcast:k).
template <uint32_t K>
__device__ __forceinline__ float bcast16(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x150 + (int)K, 0xF, 0xF, false));
}
// acc + v[0].x * P_0 + v[0].y * P_1 + ... + v[3].w * P_15 in order (P_k:
// lane k of this lane's 16-lane row), each product rounded, then the add.
template <uint32_t K>
__device__ __forceinline__ void mix_step(float& acc, float P, const f4 (&v)[4]) {
  const f4 w = v[K / 4];
  const float x = K % 4 == 0 ? w.x : K % 4 == 1 ? w.y : K % 4 == 2 ? w.z : w.w;
  const float t = x * bcast16<K>(P);
  acc = acc + t;
}
template <uint32_t K = 0>
__device__ __forceinline__ void mix16(float& acc, float P, const f4 (&v)[4]) {
  if constexpr (K < 16) {
    mix_step<K>(acc, P, v);
    mix16<K + 1>(acc, P, v);
  }
}
// The first rem (< 16) steps of mix16.
template <uint32_t K>
__device__ __forceinline__ void mix_tail(float& acc, float P, const f4 (&v)[4], uint32_t rem) {
  if constexpr (K < 15) {
    if (K < rem) {
      mix_step<K>(acc, P, v);
      mix_tail<K + 1>(acc, P, v, rem);
    }
  }
}

template <bool TR>
__device__ __forceinline__ void att_tail_block(const DecodeArgs& a, gw* out, lf* ss, uint32_t len,
                                               uint32_t pos, lf* vl, uint32_t S, const lf* vv,
                                               lf* part, lf* misc) {
  const uint32_t lane = tid_x() & 63, hd = a.hd;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  const float s0 = ss[0];
  float m = -__builtin_inff();
  for (uint32_t j0 = 0; j0 < len; j0 += 256) {  // four reads in flight per lane
    float v[4];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) {
      const uint32_t j = j0 + u * 64 + lane;
      v[u] = j < len ? ss[j] : -__builtin_inff();
    }
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) m = v[u] > m ? v[u] : m;  // false for NaN
  }
  const float mx = s0 != s0 ? s0 : wave_max(m);
  lds_barrier();
  for (uint32_t j = tid_x(); j < len; j += kThreads) {
    const float dlt = ss[j] - mx;
    ss[j] = exp_pinned(dlt);
  }
  lds_barrier();
  if (wv == 0) {
    float den;
    if constexpr (TR) {
      const uint32_t nbk = (len + 31) / 32;
      for (uint32_t t = lane; t < nbk; t += 64) part[t] = tree_part_v(ss + 32 * t, len - 32 * t);
      wave_lds_order();
      den = chain1(part, nbk, 1, 0.0f);
    } else {
      den = chain_vec_s(ss, len, 0.0f);
    }
    if (lane == 0) misc[1] = den;
  }
  lds_barrier();
  const float den = misc[1];
  for (uint32_t j = tid_x(); j < len; j += kThreads) {
    const float pj = ss[j] / den;
    ss[j] = pj;
  }
  lds_barrier();
  const uint32_t ncw = (hd + 63) >> 6, s4 = S >> 2;  // chain waves
  if (wv < ncw) {  // every lane runs (the broadcasts read whole rows)
    const uint32_t d = (wv << 6) + lane, dr = d < hd ? d : hd - 1, k = lane & 15;
    const lf4* vr = (const lf4*)vl + (size_t)dr * s4;
    const uint32_t nb = pos >> 4;  // whole blocks of 16 positions
    float acc = 0.0f;
    // two register sets, each block's reads issued one block ahead
    float PA = ss[k], PB;
    f4 vA[4], vB[4];
#pragma unroll
    for (uint32_t u = 0; u < 4; ++u) vA[u] = vr[u];
    uint32_t m = 0;
    for (; m + 2 <= nb; m += 2) {
      PB = ss[16 * (m + 1) + k];
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u) vB[u] = vr[4 * (m + 1) + u];
      mix16(acc, PA, vA);
      PA = ss[16 * (m + 2) + k];
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u) vA[u] = vr[4 * (m + 2) + u];
      mix16(acc, PB, vB);
    }
    if (m < nb) {  // one whole block left
      PB = ss[16 * (m + 1) + k];
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u) vB[u] = vr[4 * (m + 1) + u];
      mix16(acc, PA, vA);
      PA = PB;
#pragma unroll
      for (uint32_t u = 0; u < 4; ++u) vA[u] = vB[u];
    }
    // the last partial block: positions 16*nb .. pos-1 (uniform tests)
    mix_tail<0>(acc, PA, vA, pos - 16 * nb);
    if (d < hd) {
      const float t = ss[pos] * vv[d];
      acc = acc + t;
      put_word(out + d, acc, a.epoch);
    }
  }
}

template <bool TR>
__device__ __forceinline__ void run_att(const DecodeArgs& a, uint32_t l, uint32_t h, const Lds& s,
                        size_t wfloats) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const uint32_t hd = a.hd, group = a.nh / a.nkv, kvh = h / group, pos = a.pos, len = pos + 1;
  const uint32_t wv = tid_x() >> 6, lane = tid_x() & 63;
  lf* qv = s.v;
  lf* kv = qv + hd;
  lf* vv = kv + hd;
  lf* tmp = vv + hd;
  lf* misc = tmp + hd;  // [0] inv, [1] den, [4..] reduction scratch
  AS_LDS uint32_t* red = (AS_LDS uint32_t*)(misc + 4);
  lf* ss = s.w;  // scores / probabilities
  lf* kt = ss + a.max_pos + 64;  // K: one row of KS floats per cached position
  const uint32_t S = att_row_stride(pos), KS = att_k_stride(hd);
  lf* vl = kt + (size_t)((pos + 3) & ~3u) * KS;  // V: one row of S floats per head dim
  const bool in_lds =
      hd % 4 == 0 && hd <= 192 && att_lds_floats(hd, pos, a.max_pos) <= wfloats;
  stamp(a, l, P_ATT, h, 0);
  if (in_lds) prefetch_kv(a, l, kvh, kt, KS, vl, S);
  att_head_inputs<TR>(a, l, h, qv, tmp, misc);
  stamp(a, l, P_ATT, h, 1);
  if (h % group == 0) store_kv_pos(a, l, kvh, kv, vv);  // one writer per kv head
  // scores_j = dot_seq(q, k_j) * scale (main.rs:440-445)
  if (in_lds) {
    // the lane of position j forms q[d] * k_j[d] from its K row and adds
    // them in order (or by tree32 blocks)
    for (uint32_t j = tid_x(); j < len; j += kThreads) {
      const lf* kr = j < pos ? kt + (size_t)j * KS : kv;
      const float sj = score_dot<TR>(qv, kr, hd) * a.scale;
      ss[j] = sj;
    }
  } else {
    // The cached K/V do not fit in LDS: stream tiles of TP positions.  Per
    // tile, the products q[d] * k_j[d] are formed in place and each
    // position's lane adds its hd products in order.
    const uint32_t TP = att_tile_positions(hd, a.max_pos, wfloats), TS = TP + 4;
    const float* kb = a.kc0 + (size_t)l * a.cache_stride + (size_t)kvh * hd * a.max_pos;
    lf* kt = ss + a.max_pos + 64;
    for (uint32_t j0 = 0; j0 < pos; j0 += TP) {
      const uint32_t n = min(TP, pos - j0);
      copy_cache_tile(kt, kb, a.max_pos, hd, j0, n, TS);
      __syncthreads();
      scale_rows_by_row((lf4*)kt, TS >> 2, hd, (n + 3) >> 2, qv);
      __syncthreads();
      for (uint32_t jj = tid_x(); jj < n; jj += kThreads)
        ss[j0 + jj] = (TR ? tree_col(kt + jj, hd, TS, 0.0f) : chain1(kt + jj, hd, TS, 0.0f)) *
                      a.scale;
      __syncthreads();
    }
    for (uint32_t d = tid_x(); d < hd; d += kThreads) tmp[d] = qv[d] * kv[d];
    __syncthreads();
    if (tid_x() == 0)
      ss[pos] = (TR ? tree_col(tmp, hd, 1, 0.0f) : chain1(tmp, hd, 1, 0.0f)) * a.scale;
  }
  if (in_lds) {
    // the scores are in ss; the block finishes the head (tree partials in
    // the K region, which no one reads any more)
    __syncthreads();
    stamp(a, l, P_ATT, h, 3);
    att_tail_block<TR>(a, ac.att + (size_t)h * hd, ss, len, pos, vl, S, vv, kt, misc);
    __syncthreads();
    stamp(a, l, P_ATT, h, 2);
    return;
  }
  __syncthreads();
  softmax_lds<TR>(ss, len, ss + a.max_pos + 64, misc, red);
  stamp(a, l, P_ATT, h, 3);
  // V mix out_d = fold_j (p_j * v_j[d]) (main.rs:454-463)
  {
    // Tiles of TP positions: products p_j * v_j[d] in place, then lane d
    // continues its one left-to-right chain over the tile.
    const uint32_t TP = att_tile_positions(hd, a.max_pos, wfloats), TS = TP + 4;
    const float* vb = a.vc0 + (size_t)l * a.cache_stride + (size_t)kvh * hd * a.max_pos;
    lf* vt = ss + a.max_pos + 64;
    float acc = 0.0f;
    for (uint32_t j0 = 0; j0 < pos; j0 += TP) {
      const uint32_t n = min(TP, pos - j0);
      copy_cache_tile(vt, vb, a.max_pos, hd, j0, n, TS);
      __syncthreads();
      const lf4* p4 = (const lf4*)(ss + j0);
      scale_rows_by_col((lf4*)vt, TS >> 2, hd, (n + 3) >> 2, p4);
      __syncthreads();
      if (tid_x() < hd) acc = chain_vec(vt + (size_t)tid_x() * TS, n, acc);
      __syncthreads();
    }
    if (tid_x() < hd) {
      const uint32_t d = tid_x();
      float p = ss[pos] * vv[d];
      acc = acc + p;
      put_word(ac.att + (size_t)h * hd + d, acc, a.epoch);
    }
  }
  __syncthreads();
  stamp(a, l, P_ATT, h, 2);
}

// The inputs of kv head kvh's score task, in LDS: the G = nh/nkv query
// heads of the group at qv[g*hd ..), the kv head's k at qv[G*hd ..) and v
// after it; Qwen3's per-head QK-norm (after bias, before RoPE;
// labs/w1x-qwen3/scripts/qwen3-port.diff:66-80) and RoPE rotate-half of
// every q head and k (main.rs:285-307): o1 = x1*c + (-x2)*s,
// o2 = x2*c + x1*s.  The G+1 sums of squares run as separate chains, one
// per wave.  cs: hd floats (this position's cos/sin pairs), tmp: (G+1)*hd
// floats, misc: 64.  Ends with a barrier.
template <bool TR>
__device__ __forceinline__ void att_group_inputs(const DecodeArgs& a, uint32_t l, uint32_t kvh,
                                                 lf* qv, lf* cs, lf* tmp, lf* misc) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const uint32_t hd = a.hd, ng = a.nh / a.nkv, nv = ng + 1, half = hd / 2;
  NormW nq, nk;
  if (Lw.qn) nq = load_normw(Lw.qn, hd);
  if (Lw.kn) nk = load_normw(Lw.kn, hd);
  float csv = 0.0f;
  if (tid_x() < hd) csv = G(a.rope_cs)[(size_t)a.pos * hd + tid_x()];
  const uint32_t nq_w = ng * hd;
  // waves 0..1 poll while the DMA waves' K tile copies land
  gather<4, 2>(qv, (ng + 2) * hd, a.epoch, a.err, a.spin_cap, [=](uint32_t i) {
    return i < nq_w ? ac.q + (size_t)kvh * nq_w + i
                    : (i < nq_w + hd ? ac.k : ac.v) + (size_t)kvh * hd + (i - nq_w) % hd;
  });
  if (tid_x() < hd) cs[tid_x()] = csv;
  if (Lw.qn || Lw.kn) {  // rmsnorm of each vector that has weights
    const uint32_t nb = (hd + 31) / 32;
    if constexpr (TR) {
      for (uint32_t t = tid_x(); t < nv * nb; t += kThreads) {
        const uint32_t v = t / nb, b = t - v * nb;
        const lf* x = qv + (size_t)v * hd + 32 * b;
        float lv[32];
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) {
          const float xv = 32 * b + i < hd ? x[i] : 0.0f;
          lv[i] = xv * xv;
        }
        tmp[t] = tree32(lv);
      }
    } else {
      for (uint32_t i = tid_x(); i < nv * hd; i += kThreads) {
        const float xv = qv[i];
        tmp[i] = xv * xv;
      }
    }
    __syncthreads();
    for (uint32_t v = tid_x() >> 6; v < nv; v += kThreads / 64) {
      const float acc = TR ? chain1(tmp + (size_t)v * nb, nb, 1, 0.0f)
                           : chain_vec(tmp + (size_t)v * hd, hd, 0.0f);
      float mean = acc / (float)hd;
      float arg = mean + a.eps;
      float inv = rsqrt_cr(arg);
      if ((tid_x() & 63) == 0) misc[v] = inv;
    }
    __syncthreads();
    for (uint32_t v = 0; v < nv; ++v) {
      const float inv = misc[v];
      const float* wg = v < ng ? Lw.qn : Lw.kn;
      if (!wg) continue;
      for (uint32_t i = tid_x(); i < hd; i += kThreads) {
        const float wv = i < kNormThreads ? (v < ng ? nq.v[0] : nk.v[0]) : G(wg)[i];
        float sx = qv[(size_t)v * hd + i] * inv;
        qv[(size_t)v * hd + i] = sx * wv;
      }
    }
  }
  __syncthreads();
  for (uint32_t idx = tid_x(); idx < nv * half; idx += kThreads) {
    const uint32_t v = idx / half, i = idx - v * half;
    lf* hv = qv + (size_t)v * hd;
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
}

// ---------------------------------------------------------------------------
// Split attention, for contexts whose K/V rows do not fit one workgroup's
// LDS.  The phase's tasks are natt_s score tasks and then natt_v mix tasks
// (every workgroup runs its score tasks before its mix tasks, so waits stay
// acyclic):
//   score task (kvh, c): positions c*P .. c*P+P-1 of every query head of kv
//     head kvh; the cached K columns are copied into LDS with
//     global_load_lds, kScoreKT positions at a time (the first tile's copies
//     issued before the input gather), then thread j forms dot_seq(q, k_j)
//     (or dot_tree) * scale for the group's heads two at a time from its
//     column, each published as a tagged word; the chunk holding `pos` uses
//     this position's own k and stores k and v into the caches.
//   mix task (h, dc): output dims d0 = dc*kAttDV .. d0+kAttDV-1 of head h:
//     gathers all of the head's scores, runs the softmax (the same order as
//     one task; the exps of the next block formed while wave 0 chains the
//     denominator over the current one), divides once, then lane d of wave 0
//     continues its one left-to-right V-mix chain over tiles of its V rows;
//     waves 1..3 copy the tiles into a ring in LDS with global_load_lds and
//     form each tile's products one tile ahead of the chain.
// Each head's K and V are read by many workgroups at once instead of
// streaming through one.
// ---------------------------------------------------------------------------
constexpr uint32_t kScoreKB = 128;       // most head dims of a score task
constexpr uint32_t kScoreKT = kThreads;  // positions per K tile: one per thread

// acc0 (and acc1 when TWO) continue over q0[d] * k[d] (q1[d] * k[d]),
// d < hd: one left-to-right chain per head (dot_seq, math.rs:56-62) or
// tree32 blocks folded in order (dot_tree, math.rs:75-93).  k is this
// thread's column of the LDS K tile (k[d] at kp[d * kScoreKT]); q0 and q1
// are 16-byte aligned LDS vectors read as broadcasts.  Blocks of 32 dims:
// the block's k and q values are read into registers, then its products
// formed and added.
template <bool TR, bool TWO>
__device__ __forceinline__ void score_cols(const lf* q0, const lf* q1, const lf* kp, uint32_t hd,
                                           float& acc0, float& acc1) {
  constexpr uint32_t B = TR ? 32 : 16;  // dims per block (tree32 blocks in tree order)
  auto qe = [](const f4 (&q)[B / 4], uint32_t i) {
    const f4 v = q[i / 4];
    return i % 4 == 0 ? v.x : i % 4 == 1 ? v.y : i % 4 == 2 ? v.z : v.w;
  };
#pragma unroll
  for (uint32_t b = 0; b < kScoreKB; b += B) {
    if (b < hd) {
      float k[B];
      f4 qa[B / 4], qb[B / 4];
#pragma unroll
      for (uint32_t i = 0; i < B; ++i)
        if (b + i < hd) k[i] = kp[(b + i) * kScoreKT];
#pragma unroll
      for (uint32_t u = 0; u < B / 4; ++u)
        if (b + 4 * u < hd) {
          qa[u] = ((const lf4*)(q0 + b))[u];
          if (TWO) qb[u] = ((const lf4*)(q1 + b))[u];
        }
      if constexpr (TR) {
        float l32[32];
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) l32[i] = b + i < hd ? qe(qa, i) * k[i] : 0.0f;
        acc0 = acc0 + tree32(l32);
        if (TWO) {
#pragma unroll
          for (uint32_t i = 0; i < 32; ++i) l32[i] = b + i < hd ? qe(qb, i) * k[i] : 0.0f;
          acc1 = acc1 + tree32(l32);
        }
      } else {
#pragma unroll
        for (uint32_t i = 0; i < B; ++i) {
          if (b + i < hd) {
            const float p = qe(qa, i) * k[i];
            acc0 = acc0 + p;
            if (TWO) {
              const float p1 = qe(qb, i) * k[i];
              acc1 = acc1 + p1;
            }
          }
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Copies kv head kvh's cached K rows (`krows`, row stride max_pos),
// positions js .. js+n-1 rounded up to 4 (all < max_pos: js and max_pos are
// multiples of 4 and js + n <= pos), into LDS rows of kScoreKT floats:
// tile[d * kScoreKT + (j - js)] = k_j[d], d < hd.  global_load_lds_dwordx4,
// one wave instruction per dim row (n <= kScoreKT = 4 * 64), issued by the
// DMA waves 2 and 3 in turn; nothing is waited for (the data is in LDS once
// the issuing wave's vmcnt reaches 0).
__device__ __forceinline__ void copy_k_tile(lf* tile, const float* krows, uint32_t max_pos,
                                            uint32_t hd, uint32_t js, uint32_t n) {
  const uint32_t n4 = (n + 3) >> 2, lane = tid_x() & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  if (w < 2) return;  // the DMA waves copy (rows d = w - 2, w, ...)
  // one running source pointer (no per-row address kept live across layers)
  const float* src = krows + (size_t)(w - 2) * max_pos + js + 4 * lane;
  const size_t step = (size_t)2 * max_pos;
#pragma unroll 1
  for (uint32_t d = w - 2; d < hd; d += 2, src += step)
    if (lane < n4)
      __builtin_amdgcn_global_load_lds((const AS_GLB void*)src,
                                       (AS_LDS void*)((lf4*)(tile + (size_t)d * kScoreKT)), 16, 0, 0);
}

template <bool TR>
__device__ __forceinline__ void run_att_score(const DecodeArgs& a, uint32_t l, uint32_t t,
                                              const Lds& s) {
  const uint32_t C = a.att_chunks, kvh = t / C, c = t - kvh * C, P = a.att_cpos;
  const uint32_t hd = a.hd, ng = a.nh / a.nkv, pos = a.pos, len = pos + 1;
  const uint32_t j0 = c * P, jend = min(len, j0 + P);
  stamp(a, l, P_ATT, t, 0);
  if (j0 >= len) {  // no positions in this chunk yet
    stamp(a, l, P_ATT, t, 1);
    stamp(a, l, P_ATT, t, 3);
    stamp(a, l, P_ATT, t, 2);
    return;
  }
  lf* qv = s.v;                  // the group's q heads [ng][hd]
  lf* kv = qv + (size_t)ng * hd;  // this position's k, then v
  lf* vv = kv + hd;
  lf* cs = vv + hd;                     // cos/sin pairs [hd]
  lf* tmp = cs + hd;                    // [(ng+1)*hd]
  lf* misc = tmp + (size_t)(ng + 1) * hd;
  // the cached K columns of kScoreKT positions at a time, [hd][kScoreKT]
  // in the weight region; the first tile's copies land during the gather
  // of this position's q, k and v
  lf* ktile = s.w;
  const float* krows = a.kc0 + (size_t)l * a.cache_stride + (size_t)kvh * hd * a.max_pos;
  auto issue = [&](uint32_t js) {
    const uint32_t je = min(pos, js + kScoreKT);
    if (je > js) copy_k_tile(ktile, krows, a.max_pos, hd, js, je - js);
  };
  issue(j0);
  att_group_inputs<TR>(a, l, kvh, qv, cs, tmp, misc);
  stamp(a, l, P_ATT, t, 1);
  if (pos < j0 + P) store_kv_pos(a, l, kvh, kv, vv);
  gw* sc = (gw*)a.scw + ((size_t)l * a.nh + (size_t)kvh * ng) * a.max_pos;
  for (uint32_t js = j0; js < jend; js += kScoreKT) {
    if (js != j0) {
      lds_barrier();  // every thread is done with the previous tile
      issue(js);
    }
    wait_vm0();
    lds_barrier();
    if (pos >= js && pos < js + kScoreKT) {  // this position's own k into its column
      for (uint32_t d = tid_x(); d < hd; d += kThreads) ktile[d * kScoreKT + (pos - js)] = kv[d];
      lds_barrier();
    }
    const uint32_t jt = js + tid_x();
    if (jt < jend) {
      const lf* kp = ktile + tid_x();
      for (uint32_t g0 = 0; g0 < ng; g0 += 2) {
        float a0 = 0.0f, a1 = 0.0f;
        const lf* q0 = qv + (size_t)g0 * hd;
        if (g0 + 1 < ng) {
          score_cols<TR, true>(q0, q0 + hd, kp, hd, a0, a1);
          put_word(sc + (size_t)(g0 + 1) * a.max_pos + jt, a1 * a.scale, a.epoch);
        } else {
          score_cols<TR, false>(q0, q0, kp, hd, a0, a1);
        }
        put_word(sc + (size_t)g0 * a.max_pos + jt, a0 * a.scale, a.epoch);
      }
    }
  }
  stamp(a, l, P_ATT, t, 3);
  stamp(a, l, P_ATT, t, 2);
}

// The V-tile rows of loader wave w (1..3 of a workgroup): rows d < nd with
// d % 3 == w - 1.  copy_v_rows copies positions j0 .. j0+n-1 (rounded up to
// 4, inside max_pos) of those rows of a kv head's V cache (row stride
// max_pos) into LDS rows of stride TS with global_load_lds_dwordx4, one wave
// instruction per row and 256 positions; the data is in LDS once this
// wave's vmcnt has counted those instructions.  Only the wave that copied a
// row touches it until the next barrier.
__device__ __forceinline__ void copy_v_rows(lf* dst, const float* vrows, uint32_t max_pos,
                                            uint32_t nd, uint32_t j0, uint32_t n, uint32_t TS) {
  const uint32_t n4 = (n + 3) >> 2, lane = tid_x() & 63;
  const uint32_t w = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  for (uint32_t d = w - 1; d < nd; d += 3)
    for (uint32_t q0 = 0; q0 < n4; q0 += 64)
      if (q0 + lane < n4)
        __builtin_amdgcn_global_load_lds(
            (const AS_GLB void*)(G4(vrows + (size_t)d * max_pos + j0) + q0 + lane),
            (AS_LDS void*)((lf4*)(dst + (size_t)d * TS) + q0), 16, 0, 0);
}

// Softmax of one head's scores ss[0..len) up to the denominator (the
// divide follows in the V mix):
//  1. the value of the first maximum (a DPP block reduction over the
//     non-NaN scores; a NaN at position 0, or scores that are all NaN, give
//     NaN); where its bits could differ (+0 against -0), e_j =
//     exp(s_j - max) does not: both give exp(+-0) = 1;
//  2. e_j = exp(s_j - max) in place;
//  3. the denominator: a strict chain (sequential order) that wave 0 runs
//     over blocks of 1024 positions while waves 1..3 form the next block's
//     e_j; or tree32 blocks (partials in `part`) folded from 0 (tree
//     order).
// Returns the denominator in every thread (after a barrier).
// `step` runs in every wave after each block of the chain (tree order:
// once, after the exps): the caller issues its V copies there, a block at a
// time, so the copies do not hold up the waves that form the exps.
template <bool TR, class S>
__device__ __forceinline__ float softmax_head(lf* ss, uint32_t len, lf* part, lf* misc,
                                              AS_LDS uint32_t* red, S step) {
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  // (four reads in flight per thread; the pick keeps the largest value and
  // the lowest index among equals, whatever the order it sees them in)
  Cand best = {0.0f, UINT32_MAX};
  for (uint32_t j0 = tid_x(); j0 < len; j0 += 4 * kThreads) {
    float v[4];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k)
      if (j0 + k * kThreads < len) v[k] = ss[j0 + k * kThreads];
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k)
      if (j0 + k * kThreads < len && v[k] == v[k]) best = cand_pick(best, Cand{v[k], j0 + k * kThreads});
  }
  const Cand b = cand_block(best, red);
  const float mx = (ss[0] != ss[0] || b.i == UINT32_MAX) ? ss[0] : ss[b.i];
  // e_j for positions [j0, j1) by threads t0, t0 + nthr, ...: each
  // thread's reads before its writes
  auto exps = [&](uint32_t j0, uint32_t j1, uint32_t t0, uint32_t nthr) {
    for (uint32_t jb = j0 + t0; jb < j1; jb += 4 * nthr) {
      float v[4];
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k)
        if (jb + k * nthr < j1) v[k] = ss[jb + k * nthr];
#pragma unroll
      for (uint32_t k = 0; k < 4; ++k)
        if (jb + k * nthr < j1) {
          const float dlt = v[k] - mx;
          ss[jb + k * nthr] = exp_pinned(dlt);
        }
    }
  };
  if constexpr (TR) {
    exps(0, len, tid_x(), kThreads);
    __syncthreads();
    step();
    const uint32_t nbk = (len + 31) / 32;
    for (uint32_t t = tid_x(); t < nbk; t += kThreads)
      part[t] = tree_part(ss + 32 * t, len - 32 * t, 1);
    __syncthreads();
    if (wv == 0) {
      const float acc = chain1(part, nbk, 1, 0.0f);
      if (tid_x() == 0) misc[1] = acc;
    }
  } else {
    constexpr uint32_t EB = 1024;
    const uint32_t nb = (len + EB - 1) / EB;
    exps(0, min(len, EB), tid_x(), kThreads);
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t bb = 0; bb < nb; ++bb) {
      if (wv == 0)
        acc = chain_vec(ss + bb * EB, min(EB, len - bb * EB), acc);
      else if (bb + 1 < nb)
        exps((bb + 1) * EB, min(len, (bb + 2) * EB), tid_x() - 64, kThreads - 64);
      lds_barrier();
      step();
    }
    if (tid_x() == 0) misc[1] = acc;
  }
  __syncthreads();
  return misc[1];
}

// Mix task u = (query head h, dim slice dc): output dims d0 = dc*kAttDV ..
// d0+kAttDV-1 of head h:
//  - the head's scores are gathered; waves 1..3 then start copying the
//    first V tiles (a ring of nr tiles of tp positions, each wave its own
//    rows) while softmax_head forms e_j and the denominator;
//  - the whole workgroup divides: p_j = e_j / den in place;
//  - lane d of wave 0 then runs one left-to-right V-mix chain
//    out_d = fold_j (p_j * v_j[d]) over tile i while waves 1..3 form tile
//    i+1's products p_j * v_j[d] in place from their own rows (waiting only
//    for those rows' copies) and copy tile i+nr-1 into the slot tile i-1
//    left;
//  - this position's own v (gathered) is added last (main.rs:454-463).
// One barrier per tile.
template <bool TR>
__device__ __forceinline__ void run_att_mix(const DecodeArgs& a, uint32_t l, uint32_t u,
                                            const Lds& s) {
  const Act ac = act_of(a, l);
  const uint32_t DVc = a.att_dvc, h = u / DVc, dc = u - h * DVc;
  const uint32_t hd = a.hd, kvh = h / (a.nh / a.nkv), pos = a.pos, len = pos + 1;
  const uint32_t d0 = dc * kAttDV, nd = hd % kAttDV == 0 ? kAttDV : min(kAttDV, hd - d0);
  const uint32_t t = a.natt_s + u;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6), lane = tid_x() & 63;
  const bool loader = wv != 0;  // waves 1..3 copy V tiles and form products
  lf* vv = s.v;        // v of this position, dims d0.. [kAttDV]
  lf* misc = vv + 64;  // [1] den, [4..] reduction scratch
  AS_LDS uint32_t* red = (AS_LDS uint32_t*)(misc + 4);
  lf* ss = s.w;                    // scores -> e_j -> p_j [max_pos + 64]
  lf* part = ss + a.max_pos + 64;  // tree partials
  const uint32_t TP = a.att_tp, TS = TP + 4, NR = a.att_nr, nt = (pos + TP - 1) / TP;
  lf* ring = part + att_part_floats(a.max_pos);  // NR tiles [kAttDV][TS]
  auto tile = [=](uint32_t i) { return ring + (size_t)(i % NR) * kAttDV * TS; };
  auto tile_n = [=](uint32_t i) { return min(TP, pos - i * TP); };
  const float* vrows = a.vc0 + (size_t)l * a.cache_stride + ((size_t)kvh * hd + d0) * a.max_pos;
  // copy instructions of this wave per tile: its rows (d < nd, d % 3 ==
  // wv - 1) times one per 256 positions
  const uint32_t myrows = (loader && nd >= wv) ? (nd - wv + 3) / 3 : 0;
  auto copies = [=](uint32_t i) { return myrows * ((tile_n(i) + 255) / 256); };
  stamp(a, l, P_ATT, t, 0);
  uint32_t issued = 0;  // tiles whose copies have been issued (the same in every wave)
  auto refill = [&]() {
    if (issued < nt) {
      if (loader) copy_v_rows(tile(issued), vrows, a.max_pos, nd, issued * TP, tile_n(issued), TS);
      ++issued;
    }
  };
  gather_map<17>(len, a.epoch, a.err, a.spin_cap,
                 [=](uint32_t i) { return (const gw*)a.scw + ((size_t)l * a.nh + h) * a.max_pos + i; },
                 [=](uint32_t i) { return ss + i; });
  gather(vv, nd, a.epoch, a.err, a.spin_cap,
         [=](uint32_t i) { return ac.v + (size_t)kvh * hd + d0 + i; });
  stamp(a, l, P_ATT, t, 1);
  // the ring less the tile formed next lands during the softmax, a tile per
  // chain block (issued after the gathers: a poll issued behind the copies
  // would wait for them)
  auto ahead = [&]() {
    if (issued + 1 < NR) refill();
  };
  const float den = softmax_head<TR>(ss, len, part, misc, red, ahead);
  while (issued < nt && issued + 1 < NR) refill();
  stamp(a, l, P_ATT, t, 3);
  // p_j = e_j / den for positions [0, pos), by all waves (each thread's
  // reads before its writes); this position's own p stays in registers
  {
    constexpr uint32_t B = 4;
    for (uint32_t jb = tid_x(); jb < pos; jb += B * kThreads) {
      float e[B];
#pragma unroll
      for (uint32_t k = 0; k < B; ++k)
        if (jb + k * kThreads < pos) e[k] = ss[jb + k * kThreads];
#pragma unroll
      for (uint32_t k = 0; k < B; ++k)
        if (jb + k * kThreads < pos) {
          const float pj = e[k] / den;
          ss[jb + k * kThreads] = pj;
        }
    }
  }
  const float p_pos = ss[pos] / den;
  lds_barrier();
  // products of this wave's rows of tile i in place: v_j[d] <- p_j * v_j[d]
  auto products = [&](uint32_t i) {
    const uint32_t n4 = (tile_n(i) + 3) >> 2;
    const lf4* p4 = (const lf4*)(ss + i * TP);
    lf* tt = tile(i);
    for (uint32_t d = wv - 1; d < nd; d += 3) {
      lf4* r4 = (lf4*)(tt + (size_t)d * TS);
      for (uint32_t q = lane; q < n4; q += 64) {
        const f4 f = p4[q], v = r4[q];
        f4 y;
        y.x = f.x * v.x;
        y.y = f.y * v.y;
        y.z = f.z * v.z;
        y.w = f.w * v.w;
        r4[q] = y;
      }
    }
  };
  // tile `need` is in LDS once only the copies issued after it are outstanding
  auto landed = [&](uint32_t need) {
    uint32_t after = 0;
    for (uint32_t k = need + 1; k < issued; ++k) after += copies(k);
    wait_vmcnt(after);
  };
  if (nt > 0) {
    if (loader) {
      landed(0);
      products(0);
    }
    refill();  // the slot before tile 0's in the ring
    lds_barrier();
  }
  float acc = 0.0f;
  for (uint32_t i = 0; i < nt; ++i) {
    if (!loader) {
      if (lane < nd) acc = chain_vec(tile(i) + (size_t)lane * TS, tile_n(i), acc);
    } else if (i + 1 < nt) {
      landed(i + 1);
      products(i + 1);
    }
    // tile i-1's slot is free (chained before the last barrier)
    if (i >= 1) refill();
    lds_barrier();
  }
  if (!loader && lane < nd) {
    const float p = p_pos * vv[lane];
    acc = acc + p;
    put_word(ac.att + (size_t)h * hd + d0 + lane, acc, a.epoch);
  }
  stamp(a, l, P_ATT, t, 2);
}

// o_proj block + residual h1 = h + o (main.rs:470-472).  OCD: the chain's
// form (gemv_lds_t's CD: 0 for the assembly pair loop, which pays off on
// chunks of 64+ groups, i.e. reduction lengths of 1024 and up).
template <bool TR, uint32_t OCD = 8>
__device__ __forceinline__ void run_o(const DecodeArgs& a, uint32_t l, uint32_t t, const Lds& s,
                                     uint32_t tok, lf* wl, bool pre) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const uint32_t qd = a.qd, r0 = t * a.Ro, nr = min(a.Ro, a.H - r0);
  lf* x = s.v;        // attention output [qd]
  lf* hres = x + qd;  // this block's residual rows [nr]
  if (!pre) prefetch_rows_async(Lw.wo, a.Ro, qd, t, wl);
  stamp(a, l, P_O, t, 0);
  if (l == 0) {
    gf* e = G(a.embed) + (size_t)tok * a.H + r0;
    for (uint32_t i = tid_x(); i < nr; i += kThreads) hres[i] = e[i];
    gather_vec<17, 2>(x, ac.att, qd, a);
  } else {
    const gw* hin = act_of(a, l - 1).hout + r0;
    const gw* att = ac.att;
    gather<17, 2>(x, qd + nr, a.epoch, a.err, a.spin_cap,
                  [=](uint32_t i) { return i < qd ? att + i : hin + (i - qd); });
  }
  stamp(a, l, P_O, t, 1);
  const float acc = gemv_sel<TR, OCD, 32, 18, 8>(a.Ro, wl, x, qd, 1, s.pad);
  stamp(a, l, P_O, t, 3);
  if (tid_x() < nr) put_word(ac.h1 + r0 + tid_x(), hres[tid_x()] + acc, a.epoch);
  stamp(a, l, P_O, t, 2);
}

// gate/up block (wave 0 gate rows, wave 1 up rows) after
// post_attention_layernorm; hid = silu(gate) * up (main.rs:478-487).
template <bool TR>
__device__ __forceinline__ void run_gu(const DecodeArgs& a, uint32_t l, uint32_t t, const Lds& s,
                                      lf* wl, bool pre) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  lf* x = s.v;
  lf* ln = x + a.H;
  lf* gx = ln + a.H;  // 64 floats: gate results
  lf* s_inv = gx + 64;
  if (!pre) {
    prefetch_rows_async(Lw.wg, a.Rg, a.H, t, wl);
    prefetch_rows_async(Lw.wu, a.Rg, a.H, t, wl + a.Rg * a.H);
  }
  const NormW nw = load_normw(Lw.ln2, a.H);
  stamp(a, l, P_GU, t, 0);
  gather_vec<8, 2>(x, ac.h1, a.H, a);
  stamp(a, l, P_GU, t, 1);
  rmsnorm_lds<TR>(x, nw, a.eps, a.H, ln, ln, s_inv);
  stamp(a, l, P_GU, t, 3);
  const float acc = gemv_sel<TR, 8, 16, 8>(a.Rg, wl, ln, a.H, 2, s.pad);
  const uint32_t wv = tid_x() >> 6, lane = tid_x() & 63;
  if (wv == 0) gx[lane] = acc;
  __syncthreads();
  if (wv == 1) {
    const uint32_t row = t * a.Rg + lane;
    if (lane < a.Rg && row < a.I) {
      const float sg = silu_pinned(gx[lane]);
      put_word(ac.hid + row, sg * acc, a.epoch);
    }
  }
  stamp(a, l, P_GU, t, 2);
}

// down block + residual h_next = h1 + down (main.rs:489-491).
template <bool TR>
__device__ __forceinline__ void run_d(const DecodeArgs& a, uint32_t l, uint32_t t, const Lds& s,
                                     lf* wl, bool pre) {
  const LayerW Lw = a.layers[l];
  const Act ac = act_of(a, l);
  const uint32_t I = a.I, r0 = t * a.Rd, nr = min(a.Rd, a.H - r0);
  lf* x = s.v;       // hid [I]
  lf* hres = x + I;  // residual rows [nr]
  if (!pre) prefetch_rows_async(Lw.wd, a.Rd, I, t, wl);
  stamp(a, l, P_D, t, 0);
  const gw* h1 = ac.h1 + r0;
  const gw* hid = ac.hid;
  gather<25, 2>(x, I + nr, a.epoch, a.err, a.spin_cap,
                [=](uint32_t i) { return i < I ? hid + i : h1 + (i - I); });
  stamp(a, l, P_D, t, 1);
  // the 1536- to 3072-long chain keeps 12 reads in flight (8 elsewhere:
  // deeper rings slowed the shorter GEMVs, measured)
  const float acc = gemv_sel<TR, 0, 32, 24, 12, 8>(a.Rd, wl, x, I, 1, s.pad);
  stamp(a, l, P_D, t, 3);
  if (tid_x() < nr) put_word(ac.hout + r0 + tid_x(), hres[tid_x()] + acc, a.epoch);
  stamp(a, l, P_D, t, 2);
}

// Final norm, LM-head row blocks (one LDS block at a time; the first is
// copied before the wait), per-block argmax candidates; the workgroup whose
// blocks complete the set reduces the candidates to the next token id
// (strict >, first maximum wins, NaN at index 0 wins; main.rs:1161-1169).
// Sequential-order LM head with every lane on a row: lane r of half-wave
// h of wave w takes row r of this workgroup's block 8j + 2w + h in round j
// (blocks b = wg, wg + nwg, ...; 32 rows each) and runs that row's strict
// chain acc + W[row][k] * hn[k], k ascending, with its own products, the
// weights streamed from HBM straight into registers (a ring of kLmRing
// 16-byte groups in flight per lane) and hn read from LDS (one broadcast
// read per four k).  No product pass, no LDS staging of weights and no
// barrier inside the loop, so all four waves keep HBM reads in flight.  The
// ring's first loads are issued before the final norm, whose gather hides
// their latency.  Needs 32-row blocks and K a multiple of 4 * kLmRing.
constexpr uint32_t kLmRing = 16;
struct LmRows {
  uint32_t nbw, total, slot, r;  // blocks of this workgroup, steps, block slot, row
  f4 ring[kLmRing];
};
__device__ __forceinline__ gf4* lm_row_addr(const DecodeArgs& a, const LmRows& m, uint32_t t) {
  const uint32_t KG = a.H >> 2, rd = t / KG, g = t - rd * KG;
  uint32_t i = rd * 8 + m.slot;
  if (i >= m.nbw) i = m.nbw - 1;  // idle lanes stream a valid block (never published)
  const uint32_t b = blockIdx.x + i * a.nwg;
  return G4(a.lm) + ((size_t)b * KG + g) * 32 + m.r;
}
__device__ __forceinline__ void lm_rows_start(const DecodeArgs& a, LmRows& m) {
  const uint32_t wg = blockIdx.x, lane = tid_x() & 63;
  m.nbw = wg < a.nl ? (a.nl - 1 - wg) / a.nwg + 1 : 0;
  m.total = ((m.nbw + 7) / 8) * (a.H >> 2);
  m.slot = (tid_x() >> 6) * 2 + (lane >> 5);
  m.r = lane & 31;
  if (m.nbw == 0) return;
#pragma unroll
  for (uint32_t u = 0; u < kLmRing; ++u) m.ring[u] = *lm_row_addr(a, m, u);
}
// The rows' chains, logits and per-block candidates; returns the number of
// blocks this workgroup published.
__device__ __forceinline__ uint32_t lm_rows_run(const DecodeArgs& a, LmRows& m, const lf* hn) {
  const uint32_t KG = a.H >> 2, lane = tid_x() & 63;
  if (m.nbw == 0) return 0;
  AS_GLB float* logits = GW(a.logits);
  const lf4* hn4 = (const lf4*)hn;
  float acc = 0.0f;
  for (uint32_t t0 = 0; t0 < m.total; t0 += kLmRing) {
    const uint32_t g0 = t0 % KG;
#pragma unroll
    for (uint32_t u = 0; u < kLmRing; ++u) {
      const f4 w = m.ring[u];
      const f4 xv = hn4[g0 + u];
      float p;
      p = w.x * xv.x;
      acc = acc + p;
      p = w.y * xv.y;
      acc = acc + p;
      p = w.z * xv.z;
      acc = acc + p;
      p = w.w * xv.w;
      acc = acc + p;
      if (t0 + u + kLmRing < m.total) m.ring[u] = *lm_row_addr(a, m, t0 + u + kLmRing);
    }
    if (g0 + kLmRing == KG) {  // a round ends: publish every lane's row
      const uint32_t i = (t0 / KG) * 8 + m.slot;
      const bool live = i < m.nbw;
      const uint32_t b = blockIdx.x + i * a.nwg, row = b * 32 + m.r;
      Cand c = {0.0f, UINT32_MAX};
      if (live && row < a.V) {
        logits[row] = acc;
        if (acc == acc) c = Cand{acc, row};
      }
      if (live && row == 0) st_ag(a.cand + 2 * a.nl, acc != acc ? 1u : 0u);
#pragma unroll
      for (uint32_t h = 0; h < 2; ++h) {  // the candidate of each half-wave's block
        const Cand ch = cand_wave_dpp((lane >> 5) == h ? c : Cand{0.0f, UINT32_MAX});
        const uint32_t ih = (t0 / KG) * 8 + (tid_x() >> 6) * 2 + h;
        if (lane == 0 && ih < m.nbw)
          __hip_atomic_store((gw*)a.cand + blockIdx.x + ih * a.nwg,
                             ((u64)ch.i << 32) | __float_as_uint(ch.v), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
      }
      acc = 0.0f;
    }
  }
  return m.nbw;
}

template <bool TR>
__device__ __forceinline__ void run_lm(const DecodeArgs& a, const Lds& s) {
  const uint32_t L = a.L, wg = blockIdx.x;
  const uint32_t wv = tid_x() >> 6, lane = tid_x() & 63;
  lf* x = s.v;
  lf* hn = x + a.H;
  lf* misc = hn + a.H;
  AS_LDS uint32_t* red = (AS_LDS uint32_t*)(misc + 4);
  const bool rows = !TR && a.Rl == 32 && a.H % (4 * kLmRing) == 0;
  LmRows lr;
  if (rows) lm_rows_start(a, lr);
  else if (wg < a.nl) prefetch_rows(a.lm, a.Rl, a.H, wg, s.w);
  const NormW nw = load_normw(a.fnorm, a.H);
  stamp(a, L - 1, P_LM, wg, 0);
  gather_vec(x, act_of(a, L - 1).hout, a.H, a);
  stamp(a, L - 1, P_LM, wg, 1);
  rmsnorm_lds<TR>(x, nw, a.eps, a.H, hn, hn, misc);
  AS_GLB float* logits = GW(a.logits);
  uint32_t done = 0;
  if (rows) done = lm_rows_run(a, lr, hn);
  // logits and argmax candidate of block b (wave 0)
  auto publish = [&](uint32_t b, float acc) {
    if (wv == 0) {
      const uint32_t row = b * a.Rl + lane;
      Cand c = {0.0f, UINT32_MAX};
      if (lane < a.Rl && row < a.V) {
        logits[row] = acc;
        if (acc == acc) c = Cand{acc, row};
      }
      c = cand_wave_dpp(c);
      if (lane == 0) {
        __hip_atomic_store((gw*)a.cand + b, ((u64)c.i << 32) | __float_as_uint(c.v),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (b == 0 && lane == 0) st_ag(a.cand + 2 * a.nl, acc != acc ? 1u : 0u);
    }
  };
  const size_t blkf = (size_t)a.Rl * a.H;
  if (rows) {
  } else if (2 * blkf * 4 <= decode_wregion_bytes(a)) {
    // two LDS buffers: block b + nwg streams in while block b is computed;
    // block b's results are published after the wait, so the wait covers
    // only loads and stores issued one GEMV earlier
    lf* cur = s.w;
    lf* nxt = s.w + blkf;
    uint32_t prev = UINT32_MAX;
    float prev_acc = 0.0f;
    for (uint32_t b = wg; b < a.nl; b += a.nwg) {
      if (prev != UINT32_MAX) publish(prev, prev_acc);
      if (b + a.nwg < a.nl) prefetch_rows_async(a.lm, a.Rl, a.H, b + a.nwg, nxt);
      prev_acc = gemv_sel<TR, 8, 32>(a.Rl, cur, hn, a.H, 1, s.pad);
      prev = b;
      ++done;
      wait_vm0();
      __syncthreads();
      lf* t = cur;
      cur = nxt;
      nxt = t;
    }
    if (prev != UINT32_MAX) publish(prev, prev_acc);
  } else {
    for (uint32_t b = wg; b < a.nl; b += a.nwg) {
      if (b != wg) {
        prefetch_rows(a.lm, a.Rl, a.H, b, s.w);
        __syncthreads();
      }
      const float acc = gemv_sel<TR, 8, 32>(a.Rl, s.w, hn, a.H, 1, s.pad);
      publish(b, acc);
      ++done;
      __syncthreads();
    }
  }
  stamp(a, L - 1, P_LM, wg, 2);
  if (done == 0) return;  // no blocks here (fewer blocks than workgroups)
  // ticket: all candidate stores are complete before the ticket moves
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  __shared__ uint32_t s_last;
  if (tid_x() == 0) {
    uint32_t before =
        __hip_atomic_fetch_add(GU(a.cnt), done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (before + done == a.lm_epoch * a.nl) ? 1u : 0u;
  }
  __syncthreads();
  if (!s_last) return;
  // every block's (value, index) pair as one 64-bit word, eight per thread
  // in flight
  Cand c = {0.0f, UINT32_MAX};
  const gw* cw = (const gw*)a.cand;
  for (uint32_t b0 = tid_x(); b0 < a.nl; b0 += 8 * kThreads) {
    u64 w[8];
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u)
      if (b0 + u * kThreads < a.nl) w[u] = get_word(cw + b0 + u * kThreads);
#pragma unroll
    for (uint32_t u = 0; u < 8; ++u)
      if (b0 + u * kThreads < a.nl)
        c = cand_pick(c, Cand{__uint_as_float((uint32_t)w[u]), (uint32_t)(w[u] >> 32)});
  }
  const Cand r = cand_block(c, red);
  if (tid_x() == 0) {
    const uint32_t first_nan = ld_ag(a.cand + 2 * a.nl);
    *GU(a.tok_out) = (first_nan || r.i == UINT32_MAX) ? 0u : r.i;
  }
  stamp(a, L - 1, P_LM, wg, 3);
}

// Floats of a task's weight blocks in LDS (attention: none).
__device__ __forceinline__ uint32_t task_wfloats(const DecodeArgs& a, uint32_t ph) {
  switch (ph) {
    case P_QKV: return a.Rq * a.H;
    case P_O: return a.Ro * a.qd;
    case P_GU: return 2 * a.Rg * a.H;
    case P_D: return a.Rd * a.I;
    default: return 0;
  }
}
// Loads of layer l's weight blocks of a workgroup's tasks into their LDS
// slots (global_load_lds, nothing waited for: the tasks' gathers wait for
// every earlier load before their barrier).
__device__ __forceinline__ void load_task_weights(const DecodeArgs& a, uint32_t l,
                                                  const uint32_t* task, uint32_t ntask,
                                                  const uint32_t* woff, const Lds& s) {
  const LayerW Lw = a.layers[l];
  for (uint32_t i = 0; i < ntask; ++i) {
    const uint32_t ph = task[i] >> 12, t = task[i] & 0xFFFu;
    lf* wl = s.w + woff[i];
    switch (ph) {
      case P_QKV: {
        const QkvGeom g = qkv_geom(a, Lw, act_of(a, l), t);
        prefetch_rows_async(g.W, a.Rq, a.H, g.blk, wl);
        break;
      }
      case P_O: prefetch_rows_async(Lw.wo, a.Ro, a.qd, t, wl); break;
      case P_GU:
        prefetch_rows_async(Lw.wg, a.Rg, a.H, t, wl);
        prefetch_rows_async(Lw.wu, a.Rg, a.H, t, wl + a.Rg * a.H);
        break;
      case P_D: prefetch_rows_async(Lw.wd, a.Rd, a.I, t, wl); break;
      default: break;
    }
  }
}

// One 256-thread workgroup per CU (the LDS footprint allows no second one),
// so one wave per SIMD: the compiler may use the whole register file.
// Model shapes compiled with their dimensions and row-block heights as
// constants (loop bounds, chunk sizes and GEMV dispatch then fold at compile
// time: 35-55 % fewer cycles per GEMV than with run-time K).  Shape 0 takes
// them from the arguments and serves every other configuration.
struct KShape {
  uint32_t H, I, qd, hd, Rq, Ro, Rg, Rd, Rl;
};
constexpr KShape kShapes[] = {
    {0, 0, 0, 0, 0, 0, 0, 0, 0},
    {576, 1536, 576, 64, 8, 8, 8, 8, 32},         // SmolLM2-135M
    {768, 3072, 768, 64, 16, 8, 16, 8, 32},       // llama-160m
    {1024, 3072, 2048, 128, 16, 8, 16, 8, 32},    // Qwen3-0.6B
};

// The O projection's chain form for a shape instance: the assembly loop
// where its reduction length (qd) is 1024 or more, else the ring.
constexpr uint32_t o_chain_cd(int sh) { return sh > 0 && kShapes[sh].qd >= 1024 ? 0u : 8u; }

__host__ __device__ inline bool shape_matches(const DecodeArgs& a, const KShape& k) {
  return a.H == k.H && a.I == k.I && a.qd == k.qd && a.hd == k.hd && a.Rq == k.Rq &&
         a.Ro == k.Ro && a.Rg == k.Rg && a.Rd == k.Rd && a.Rl == k.Rl;
}

template <bool TR, int SH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_decode(DecodeArgs a) {
  if constexpr (SH > 0) {  // the launch checked that the arguments equal these
    constexpr KShape k = kShapes[SH];
    a.H = k.H;
    a.I = k.I;
    a.qd = k.qd;
    a.hd = k.hd;
    a.Rq = k.Rq;
    a.Ro = k.Ro;
    a.Rg = k.Rg;
    a.Rd = k.Rd;
    a.Rl = k.Rl;
  }
  // 16-byte element type: the dynamic region follows the static LDS variables
  // (s_last) at a 16-byte boundary, so every ds_read/write_b128 is aligned
  // (a misaligned b128 access is split and runs several times slower).
  extern __shared__ f4 lds_dyn[];
  Lds s;
  s.w = (lf*)lds_dyn;
  const size_t wbytes = decode_wregion_bytes(a);
  s.v = s.w + wbytes / 4;
  s.pad = (lf4*)(s.v + decode_vec_floats(a));
  const uint32_t wg = blockIdx.x;
  // profiling: workgroup entry and exit in the layer-0 LM slots (the LM
  // phase stamps the last layer's)
  if (a.L > 1) stamp(a, 0, P_LM, wg, 0);
  // this position's token (written by the previous launch's argmax): its
  // load goes out with the task list's, ahead of any weight copy
  const uint32_t tok_in = *(const AS_GLB uint32_t*)a.tok_in;
  // this workgroup's tasks (the same in every layer), in phase order
  uint32_t task[kMaxTasks];
  uint32_t ntask = 0;
  bool reads_tok = false;
#pragma unroll
  for (uint32_t i = 0; i < kMaxTasks; ++i) {
    task[i] = __builtin_amdgcn_readfirstlane(((const AS_GLB uint16_t*)a.wg_tasks)[wg * kMaxTasks + i]);
    if (task[i] != kNoTask) {
      ntask = i + 1;
      const uint32_t ph = task[i] >> 12;
      reads_tok |= ph == P_QKV || ph == P_O;  // the layer-0 tasks that read the embedding row
    }
  }
  // Workgroups without an attention task keep every task's weight blocks
  // in a slot of their own and load the next layer's after their last task
  // of a layer (layer 0's at the start), so no task waits for its weights;
  // a workgroup with an attention task loads each block at its task's start.
  uint32_t woff[kMaxTasks];
  bool slots = true;
  {
    uint32_t tot = 0;
#pragma unroll
    for (uint32_t i = 0; i < kMaxTasks; ++i) {
      woff[i] = tot;
      if (i < ntask) {
        const uint32_t ph = task[i] >> 12;
        if (ph == P_ATT) slots = false;
        tot += task_wfloats(a, ph);
        if (tot % 4) slots = false;  // slots start 16-byte aligned
      }
    }
    if ((size_t)tot * 4 > wbytes) slots = false;
  }
  if (slots) load_task_weights(a, 0, task, ntask, woff, s);
  uint32_t tok = 0;
  if (reads_tok) {
    tok = tok_in;
    if (tok >= a.V) {
      if (tid_x() == 0) raise_err(a.err, 1u);
      tok = 0;
    }
  }
  for (uint32_t l = 0; l < a.L; ++l) {
    for (uint32_t i = 0; i < ntask; ++i) {
      const uint32_t ph = task[i] >> 12, t = task[i] & 0xFFFu;
      lf* wl = slots ? s.w + woff[i] : s.w;
      switch (ph) {
        case P_QKV: run_qkv<TR>(a, l, t, s, tok, wl, slots); break;
        case P_ATT:
          if (!a.att_split) run_att<TR>(a, l, t, s, wbytes / 4);
          else if (t < a.natt_s) run_att_score<TR>(a, l, t, s);
          else run_att_mix<TR>(a, l, t - a.natt_s, s);
          break;
        case P_O: run_o<TR, o_chain_cd(SH)>(a, l, t, s, tok, wl, slots); break;
        case P_GU: run_gu<TR>(a, l, t, s, wl, slots); break;
        case P_D: run_d<TR>(a, l, t, s, wl, slots); break;
        default: break;
      }
      __syncthreads();
    }
    if (slots && l + 1 < a.L) load_task_weights(a, l + 1, task, ntask, woff, s);
  }
  if (a.want_logits) run_lm<TR>(a, s);
  if (a.L > 1) stamp(a, 0, P_LM, wg, 2);
}

// ---------------------------------------------------------------------------
// Standalone strict-order GEMV y = W x (the per-row dot_seq of
// code/cis2-fp/src/main.rs:228-243) on the blocked layout: one workgroup
// per R-row block copies the block and x into LDS in one round trip, then
// runs the same pipelined product pass and strict chains as the decode
// kernel.
// ---------------------------------------------------------------------------
// KC != 0: K fixed at compile time (the kernel takes K == KC).
template <uint32_t R, uint32_t KC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemv_blk(const float* __restrict__ W, const float* __restrict__ x, float* y, uint32_t M,
                uint32_t Krt) {
  const uint32_t K = KC ? KC : Krt;
  extern __shared__ f4 lds_dyn[];
  lf* w = (lf*)lds_dyn;
  lf* xs = w + (size_t)R * K;
  lf4* pad = (lf4*)(xs + K);
  const uint32_t b = blockIdx.x;
  const size_t blkf = (size_t)R * K;
  gf4* src = G4(W + b * blkf);
  gf4* x4 = G4(x);
  const uint32_t n4 = (uint32_t)(blkf / 4), k4 = K >> 2;
  copy_to_lds((lf4*)w, n4 + k4, [=](uint32_t i) { return i < n4 ? src + i : x4 + (i - n4); });
  __syncthreads();
  const float acc = gemv_lds_t<R, 0>(w, xs, K, 1, pad);
  const uint32_t row = b * R + tid_x();
  if (tid_x() < R && row < M) GW(y)[row] = acc;
}

// 16-byte global->LDS loads (global_load_lds_dwordx4) of the 64-slot runs
// [64 ins, 64 ins + 64) of src into the same slots of dst, for ins = i0 + w,
// i0 + w + nw, ... < i1.  Every run is one wave instruction and lane l
// always writes slot 64 ins + l, so dst needs 63 slots of room past n4;
// lanes past n4 read slot n4 - 1 (no lane is skipped, so the count of
// load instructions is exact).  Returns that count (wave-uniform).
__device__ __forceinline__ uint32_t load_runs(gf4* src, lf4* dst, uint32_t n4, uint32_t i0,
                                              uint32_t i1, uint32_t w, uint32_t nw) {
  const uint32_t lane = tid_x() & 63;
  uint32_t cnt = 0;
  for (uint32_t ins = i0 + w; ins < i1; ins += nw) {
    const uint32_t s0 = ins * 64;
    __builtin_amdgcn_global_load_lds((const AS_GLB void*)(src + min(s0 + lane, n4 - 1)),
                                     (AS_LDS void*)(dst + s0), 16, 0, 0);
    ++cnt;
  }
  return cnt;
}

// The lone GEMV, pipelined (the standalone plan's kernel for K fixed at
// compile time): every wave issues, right at the start and in chunk order,
// the loads of exactly the W slots its own product instructions multiply,
// straight into LDS, so no wave waits for another wave's loads and the
// chain starts one HBM round trip after the launch instead of after the
// whole block has arrived.  Product instruction ins covers the 64 16-byte
// slots [64 ins, 64 ins + 64) of the block (group ins*GP + l/R, row l%R, as
// in prod_ins).  x is loaded by all waves first.  Chunk 0's instructions are
// spread over all four waves, later chunks over waves 1-3.  After chunk 0's
// products, lane r of wave 0 adds row r's products of chunk c strictly in
// order while waves 1-3 form chunk c+1's.
template <uint32_t R, uint32_t K>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1)))
void k_gemv_pipe(const float* __restrict__ W, const float* __restrict__ x, float* y, uint32_t M) {
  constexpr uint32_t NC = 3, GP = 64 / R, NW = kThreads / 64, KG = K / 4;
  constexpr uint32_t NINS = (KG + GP - 1) / GP, N4 = KG * R;
  static_assert(K % 4 == 0 && 64 % R == 0, "shape");
  // first product instruction of chunk c: NC equal chunks.  Measured at
  // 1536x576 (MI355X, us per launch): NC 1: 4.80, 2: 4.41, 3: 4.30, 4: 4.57,
  // 6: 5.14, 9: 7.50; unequal chunks ending on 16-group multiples were
  // slower than equal ones (4.80-5.06 against 4.56 at NC 4)
  auto bound = [](uint32_t c) { return NINS * c / NC; };
  extern __shared__ f4 lds_dyn[];
  lf4* w4 = (lf4*)lds_dyn;   // the block, then 64 slots of room
  lf4* xs = w4 + N4 + 64;    // x, then 64 slots of room
  lf4* pad = xs + KG + 64;   // prod_ins's idle-lane slots
  const uint32_t b = blockIdx.x;
  const uint32_t wv = __builtin_amdgcn_readfirstlane(tid_x() >> 6);
  gf4* src = G4(W + (size_t)b * R * K);
  uint32_t cnt[NC];
  cnt[0] = load_runs(G4(x), xs, KG, 0, (KG + 63) / 64, wv, NW);
  cnt[0] += load_runs(src, w4, N4, 0, bound(1), wv, NW);
  for (uint32_t c = 1; c < NC; ++c)
    cnt[c] = wv == 0 ? 0u : load_runs(src, w4, N4, bound(c), bound(c + 1), wv - 1, NW - 1);
  uint32_t rest = 0;  // this wave's loads of chunks 1.. (chunk 0 lands first)
  for (uint32_t c = 1; c < NC; ++c) rest += cnt[c];
  wait_vmcnt(rest);
  lds_barrier();
  prod_ins<R>(w4, xs, N4, 1, KG, 0, bound(1), wv, NW, pad);
  lds_barrier();
  const uint32_t lane = tid_x() & 63, r = lane < R ? lane : R - 1;
  float acc = 0.0f;
  for (uint32_t c = 0; c < NC; ++c) {
    const uint32_t i0 = bound(c), i1 = bound(c + 1);
    if (wv == 0) {
      // 16-group pairs in the assembly loop (its reads past the chunk land
      // in the next chunk's slots, or past the block in the room after it
      // and x), then any rest in a ring
      const uint32_t g0 = i0 * GP, g1 = min(i1 * GP, KG), ng = g1 - g0, np = ng >> 4;
      const lf4* cp = w4 + (size_t)g0 * R + r;
      if (np > 0) acc = chain_lds16<R>(cp, np, acc);
      acc = chain4<8>(cp + (size_t)np * 16 * R, ng - np * 16, R, acc);
    } else if (c + 1 < NC) {
      uint32_t later = 0;
      for (uint32_t c2 = c + 2; c2 < NC; ++c2) later += cnt[c2];
      wait_vmcnt(later);
      prod_ins<R>(w4, xs, N4, 1, KG, i1, bound(c + 2), wv - 1, NW - 1, pad);
    }
    lds_barrier();
  }
  const uint32_t row = b * R + tid_x();
  if (tid_x() < R && row < M) GW(y)[row] = acc;
}

// A batch of n independent GEMVs in one launch (gridDim.y = n): GEMV i is
// y_i = W_c x_i with W_c the replica c = (first + i) % copies, x_i at
// x + i*K, y_i at y + i*M.  The block's work is k_gemv_blk's; several
// workgroups share a CU, so one block's copy overlaps another's chains and
// the launch streams weights at HBM rate.
template <uint32_t R, uint32_t KC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 4)))
void k_gemv_many(const float* __restrict__ W, uint64_t w_per, uint32_t copies, uint32_t first,
                 const float* __restrict__ x, float* y, uint32_t M, uint32_t Krt) {
  const uint32_t K = KC ? KC : Krt;
  extern __shared__ f4 lds_dyn[];
  lf* w = (lf*)lds_dyn;
  lf* xs = w + (size_t)R * K;
  lf4* pad = (lf4*)(xs + K);
  const uint32_t b = blockIdx.x, i = blockIdx.y;
  const uint32_t c = (first + i) % copies;
  const size_t blkf = (size_t)R * K;
  gf4* src = G4(W + c * w_per + b * blkf);
  gf4* x4 = G4(x + (size_t)i * K);
  const uint32_t n4 = (uint32_t)(blkf / 4), k4 = K >> 2;
  copy_to_lds((lf4*)w, n4 + k4, [=](uint32_t j) { return j < n4 ? src + j : x4 + (j - n4); });
  __syncthreads();
  // the ring chain: chain_lds16's fixed registers (v192..v255) would hold
  // the kernel at one workgroup per CU, and the overlap of one block's copy
  // with another's chains is what keeps this launch at HBM rate
  const float acc = gemv_lds_t<R>(w, xs, K, 1, pad);
  const uint32_t row = b * R + tid_x();
  if (tid_x() < R && row < M) GW(y + (size_t)i * M)[row] = acc;
}

}  // namespace

size_t gemv_blk_lds_bytes(uint32_t K, uint32_t R) {
  // the block, x, prod_ins's 64 idle-lane slots, and room for the chains'
  // reads of 8 groups past the block
  return ((size_t)R * K + K) * 4 + 64 * 16 + (size_t)8 * R * 16;
}

template <uint32_t R, uint32_t KC>
static hipError_t launch_gemv_blk_t(const float* W, const float* x, float* y, uint32_t M,
                                    uint32_t K, size_t lds, hipStream_t s) {
  hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&k_gemv_blk<R, KC>), lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemv_blk<R, KC>), dim3((M + R - 1) / R), dim3(kThreads), lds, s, W, x,
                     y, M, K);
  return hipGetLastError();
}

template <uint32_t R, uint32_t K>
static hipError_t launch_gemv_pipe_t(const float* W, const float* x, float* y, uint32_t M,
                                     hipStream_t s) {
  const size_t lds = ((size_t)R * K + K + 3 * 256) * 4;  // block, x, 64 slots after each, pad
  hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&k_gemv_pipe<R, K>), lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemv_pipe<R, K>), dim3((M + R - 1) / R), dim3(kThreads), lds, s, W, x, y,
                     M);
  return hipGetLastError();
}

hipError_t launch_gemv_blk(const float* W, const float* x, float* y, uint32_t M, uint32_t K,
                           uint32_t R, hipStream_t s) {
  const size_t lds = gemv_blk_lds_bytes(K, R);
  if (K % 4 || lds > 160 * 1024 - 64) return hipErrorInvalidValue;
  // the hidden size of SmolLM2-135M (K = 576: the 1536x576 up-projection)
  // compiled with K fixed; any other K at run time
  if (R == 16 && K == 576) return launch_gemv_pipe_t<16, 576>(W, x, y, M, s);
  if (R == 16 && K == 1536) return launch_gemv_pipe_t<16, 1536>(W, x, y, M, s);
  if (R == 16) return launch_gemv_blk_t<16, 0>(W, x, y, M, K, lds, s);
  if (R == 32) return K == 576 ? launch_gemv_blk_t<32, 576>(W, x, y, M, K, lds, s)
                               : launch_gemv_blk_t<32, 0>(W, x, y, M, K, lds, s);
  return hipErrorInvalidValue;
}

template <uint32_t R, uint32_t KC>
static hipError_t launch_gemv_many_t(const float* W, uint64_t w_per, uint32_t copies,
                                     uint32_t first, uint32_t n, const float* x, float* y,
                                     uint32_t M, uint32_t K, size_t lds, hipStream_t s) {
  hipError_t e = ensure_dynamic_lds(reinterpret_cast<const void*>(&k_gemv_many<R, KC>), lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_gemv_many<R, KC>), dim3((M + R - 1) / R, n), dim3(kThreads), lds, s, W,
                     w_per, copies, first, x, y, M, K);
  return hipGetLastError();
}

hipError_t launch_gemv_many(const float* W, uint64_t w_per, uint32_t copies, uint32_t first,
                            uint32_t n, const float* x, float* y, uint32_t M, uint32_t K,
                            uint32_t R, hipStream_t s) {
  // k_gemv_many's ring chain reads nothing past the block: no room after it
  // (four workgroups per CU at K = 576)
  const size_t lds = gemv_blk_lds_bytes(K, R) - (size_t)8 * R * 16;
  if (n == 0) return hipSuccess;
  if (K % 4 || lds > 160 * 1024 - 64 || copies == 0 || n > 65535) return hipErrorInvalidValue;
  if (R == 16) return K == 576 ? launch_gemv_many_t<16, 576>(W, w_per, copies, first, n, x, y, M, K, lds, s)
                               : launch_gemv_many_t<16, 0>(W, w_per, copies, first, n, x, y, M, K, lds, s);
  return hipErrorInvalidValue;
}

size_t decode_act_floats(uint32_t H, uint32_t I, uint32_t qd, uint32_t kvd) {
  return 2 * layer_words(H, I, qd, kvd);
}

bool decode_att_ok(const DecodeArgs& a) {
  const size_t wfloats = decode_wregion_bytes(a) / 4;
  // split: the score task stages kScoreKT positions of K ([hd][kScoreKT],
  // hd <= kScoreKB, a multiple of 4) in the weight region
  if (a.att_split)
    return a.att_tp >= 32 && a.att_nr >= 3 && a.nh % a.nkv == 0 && a.nh / a.nkv < 64 &&
           a.hd <= kScoreKB &&
           a.hd % 4 == 0 && (size_t)a.hd * kScoreKT <= wfloats;
  // the one-task form keeps K and V in LDS when they fit (head_dim a
  // multiple of 4), else streams tiles of at least 32 positions
  return (a.hd % 4 == 0 && a.hd <= 192 &&
          att_lds_floats(a.hd, a.max_pos, a.max_pos) <= wfloats) ||
         att_tile_positions(a.hd, a.max_pos, wfloats) >= 32;
}

bool decode_att_needs_split(const DecodeArgs& a) {
  return att_lds_floats(a.hd, a.max_pos, a.max_pos) > decode_wregion_bytes(a) / 4;
}

void decode_att_plan(DecodeArgs& a, bool split) {
  a.att_split = split ? 1u : 0u;
  // positions per score task (one kv head's query heads): 256 (one per
  // thread) when every kv head's chunks fit one per workgroup, else the
  // fewest 64-multiples up to 512 that do (a workgroup holding two score
  // tasks of a layer would finish its second one late, and every mix task
  // of the group waits for it)
  uint32_t cp = kThreads;
  const uint32_t per_kv = a.nkv ? a.nwg / a.nkv : 0;
  if (per_kv > 0 && a.nkv * ((a.max_pos + cp - 1) / cp) > a.nwg) {
    cp = (a.max_pos + per_kv - 1) / per_kv;
    cp = (cp + 63) & ~63u;
    if (cp > 2 * kThreads) cp = 2 * kThreads;
  }
  a.att_cpos = cp;
  a.att_chunks = (a.max_pos + cp - 1) / cp;
  a.natt_s = a.nkv * a.att_chunks;
  a.att_dvc = (a.hd + kAttDV - 1) / kAttDV;
  a.natt_v = a.nh * a.att_dvc;
  att_mix_plan(a.max_pos, decode_wregion_bytes(a) / 4, &a.att_tp, &a.att_nr);
}

size_t decode_lds_bytes(const DecodeArgs& a) {
  // weight region | vectors | product-pass pad (64 x 16 B) | slack
  return decode_wregion_bytes(a) + decode_vec_floats(a) * 4 + 64 * 16 + 256;
}

// The k_decode instance for the arguments' order and shape.
static const void* decode_kernel(const DecodeArgs& a) {
  if (a.tree) {  // the v0.4-candidate order, with the same compile-time shapes
    if (shape_matches(a, kShapes[1])) return reinterpret_cast<const void*>(&k_decode<true, 1>);
    if (shape_matches(a, kShapes[2])) return reinterpret_cast<const void*>(&k_decode<true, 2>);
    if (shape_matches(a, kShapes[3])) return reinterpret_cast<const void*>(&k_decode<true, 3>);
    return reinterpret_cast<const void*>(&k_decode<true, 0>);
  }
  if (shape_matches(a, kShapes[1])) return reinterpret_cast<const void*>(&k_decode<false, 1>);
  if (shape_matches(a, kShapes[2])) return reinterpret_cast<const void*>(&k_decode<false, 2>);
  if (shape_matches(a, kShapes[3])) return reinterpret_cast<const void*>(&k_decode<false, 3>);
  return reinterpret_cast<const void*>(&k_decode<false, 0>);
}

hipError_t decode_coresident(const DecodeArgs& a, uint32_t ncu, bool* ok) {
  *ok = false;
  const void* fn = decode_kernel(a);
  const size_t lds = decode_lds_bytes(a);
  hipError_t e = ensure_dynamic_lds(fn, lds);
  if (e != hipSuccess) return e;
  int per_cu = 0;
  e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, (int)kThreads, lds);
  if (e != hipSuccess) return e;
  *ok = per_cu > 0 && (uint64_t)per_cu * ncu >= a.nwg;
  return hipSuccess;
}

// A plain launch of a grid the context checked at creation to fit the
// device at once (decode_coresident).  Not a cooperative launch: once one
// process has made a cooperative launch on a GPU, every other process's
// cooperative launch there fails ("cannot be performed in the present
// state", measured on MI355X), which would stop a second worker process.
// Should other work hold CUs so that some workgroups start late, the phase
// waits' spin cap ends the launch with an error instead of a hang.
hipError_t launch_decode(const DecodeArgs& a, hipStream_t s) {
  const void* fn = decode_kernel(a);
  const size_t lds = decode_lds_bytes(a);
  hipError_t e = ensure_dynamic_lds(fn, lds);
  if (e != hipSuccess) return e;
  void* args[] = {const_cast<DecodeArgs*>(&a)};
  return hipLaunchKernel(fn, dim3(a.nwg), dim3(kThreads), args, lds, s);
}

}  // namespace cis2
