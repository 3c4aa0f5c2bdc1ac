// cis2_sample.hip — seeded sampling of CIS-2 v0.4 draft section 14 on
// gfx950 (code/patches/cis2-spec__seeded-sampling.patch:57-196): a
// stateless Gumbel-max draw over the fp32 logits with MurmurHash3 noise,
// temperature, rank-order top-k and top-p.
//
// Per step, on the library's stream:
//   1. k_rank_keys: s_i = l_i / T and a 64-bit key per index whose
//      ascending order is the draft's rank order (s descending, then index
//      ascending; -0 and +0 tie).  Skipped when neither top-k nor top-p is
//      active (every index is kept, no order is needed).
//   2. bitonic sort of the keys: tiles of 4096 keys sorted and merged in
//      LDS, strides of a tile or more as grid-wide compare-exchange passes.
//      With top-k <= 4096 only the candidates are sorted: every tile is
//      sorted, its first K keys gathered, and those sorted.
//   3. k_keep: one workgroup; top-k cuts the ranks, then top-p runs its two
//      strict rank-order chains (the denominator, then the running sum,
//      stopping at the first rank whose predecessor sum reaches top_p).
//   4. k_draw / k_draw_final: z = s + g over the kept indices, first index
//      of the maximum (section 11.2's strict > scan from index 0).
// Every value is the one the draft's arithmetic gives: true divides, the
// pinned ln and exp, sequential f32 sums in rank order.
#include "cis2_sample.hpp"

#include <mutex>

#include "cis2_device_math.hpp"

namespace cis2 {

namespace {

constexpr uint32_t kTile = 4096;  // keys per LDS tile (32 KiB)

__device__ __forceinline__ uint32_t rotl32(uint32_t x, int r) { return (x << r) | (x >> (32 - r)); }

// One 4-byte block of MurmurHash3_x86_32.
__device__ __forceinline__ uint32_t mm_block(uint32_t h, uint32_t k) {
  k *= 0xcc9e2d51u;
  k = rotl32(k, 15);
  k *= 0x1b873593u;
  h ^= k;
  h = rotl32(h, 13);
  return h * 5u + 0xe6546b64u;
}

// Draft 14.2: MurmurHash3_x86_32 with hash seed 0x43495332 of the 16-byte
// key seed (u64 LE) || step (u32 LE) || index (u32 LE): four blocks, no
// tail, the length, fmix32.  Then m = (h >> 9) * 2 + 1, u = f32(m) * 2^-24
// (exact), g = 0 - ln(0 - ln(u)).
__device__ __forceinline__ float gumbel(uint64_t seed, uint32_t step, uint32_t idx) {
  uint32_t h = 0x43495332u;
  h = mm_block(h, (uint32_t)seed);
  h = mm_block(h, (uint32_t)(seed >> 32));
  h = mm_block(h, step);
  h = mm_block(h, idx);
  h ^= 16u;
  h ^= h >> 16;
  h *= 0x85ebca6bu;
  h ^= h >> 13;
  h *= 0xc2b2ae35u;
  h ^= h >> 16;
  const uint32_t m = (h >> 9) * 2u + 1u;
  const float u = (float)m * 5.9604644775390625e-08f;  // 2^-24
  const float inner = 0.0f - ln_pinned(u);
  return 0.0f - ln_pinned(inner);
}

// Ascending key order = rank order of draft 14.3 step 2.
__device__ __forceinline__ uint64_t rank_key(float s, uint32_t i) {
  uint32_t b = __float_as_uint(s);
  if (b == 0x80000000u) b = 0u;  // -0 ties with +0
  const uint32_t asc = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)(~asc) << 32) | i;
}

__global__ __launch_bounds__(256) void k_rank_keys(const float* __restrict__ l, uint32_t V,
                                                   uint32_t Vp, float T, uint64_t* key,
                                                   uint32_t* err) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= Vp) return;
  if (i < V) {
    const float s = l[i] / T;
    if (s != s) atomicOr(err, 0x100u);
    key[i] = rank_key(s, i);
  } else {
    key[i] = ~0ull;  // padding sorts last
  }
}

// Bitonic compare-exchange of the pair (i, i + j) in direction bit k of
// the global index i (ascending when clear).
__device__ __forceinline__ void cmpx(uint64_t& a, uint64_t& b, bool asc) {
  if ((a > b) == asc) {
    const uint64_t t = a;
    a = b;
    b = t;
  }
}

// One tile of kTile keys in LDS: k_level 0 sorts it completely (levels
// 2..kTile); otherwise it runs the strides kTile/2..1 of level k_level.
// asc_all: every tile ascending (for the top-k selection), instead of the
// alternating directions a following merge level needs.
__global__ __launch_bounds__(1024) void k_bitonic_tile(uint64_t* key, uint32_t k_level,
                                                       uint32_t asc_all) {
  __shared__ uint64_t t[kTile];
  const uint32_t base = blockIdx.x * kTile;
  for (uint32_t j = threadIdx.x; j < kTile; j += 1024) t[j] = key[base + j];
  __syncthreads();
  auto pass = [&](uint32_t k, uint32_t j) {
    for (uint32_t x = threadIdx.x; x < kTile / 2; x += 1024) {
      const uint32_t i = 2 * x - (x & (j - 1));
      cmpx(t[i], t[i + j], (((asc_all ? 0u : base) + i) & k) == 0);
    }
    __syncthreads();
  };
  if (k_level == 0) {
    for (uint32_t k = 2; k <= kTile; k <<= 1)
      for (uint32_t j = k >> 1; j > 0; j >>= 1) pass(k, j);
  } else {
    for (uint32_t j = kTile >> 1; j > 0; j >>= 1) pass(k_level, j);
  }
  for (uint32_t j = threadIdx.x; j < kTile; j += 1024) key[base + j] = t[j];
}

// One grid-wide pass of stride j (>= kTile) of level k.
__global__ __launch_bounds__(256) void k_bitonic_pass(uint64_t* key, uint32_t Vp, uint32_t k,
                                                      uint32_t j) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= Vp / 2) return;
  const uint32_t i = 2 * x - (x & (j - 1));
  uint64_t a = key[i], b = key[i + j];
  const bool asc = (i & k) == 0;
  if ((a > b) == asc) {
    key[i] = b;
    key[i + j] = a;
  }
}

// Top-k selection: the first K keys of every ascending-sorted tile (they
// hold every key of the global top K) into cand[0 .. ntiles*K), the rest of
// cand[0 .. Cp) padded to sort last.
__global__ __launch_bounds__(256) void k_gather_top(const uint64_t* __restrict__ key, uint32_t K,
                                                    uint32_t ntiles, uint32_t Cp, uint64_t* cand) {
  const uint32_t x = blockIdx.x * blockDim.x + threadIdx.x;
  if (x >= Cp) return;
  cand[x] = x < ntiles * K ? key[(x / K) * kTile + x % K] : ~0ull;
}

// Draft 14.3 steps 3-4 over the sorted keys (one workgroup): K = top-k
// cut; with top_p < 1, m = s of rank 0, e_r = exp(s_r - m), denom =
// sum_seq(e) in rank order, p_r = e_r / denom, c_r = c_{r-1} + p_r from 0,
// and the kept ranks end at the first r > 0 with !(c_{r-1} < top_p).
// The ranks pass through LDS in tiles of kKeepTile: lane 0 runs the strict
// chain over one tile (16 LDS reads in flight) while waves 1.. form the
// next tile's terms in the other buffer.  c never decreases (p_r >= 0), so a group of four needs a
// per-rank test only when its third sum fails.
constexpr uint32_t kKeepTile = 8192;

__global__ __launch_bounds__(1024) void k_keep(const uint64_t* __restrict__ key,
                                               const float* __restrict__ l, float T, uint32_t K,
                                               float top_p, float* e, uint32_t* nkeep) {
  // two tile buffers: wave 0 chains one while waves 1.. form the next
  __shared__ __attribute__((aligned(16))) float t[2][kKeepTile];
  __shared__ float s_den;
  __shared__ uint32_t s_keep;
  if (!(top_p < 1.0f)) {
    if (threadIdx.x == 0) *nkeep = K;
    return;
  }
  const float m = l[(uint32_t)key[0]] / T;
  const uint32_t nt = (K + kKeepTile - 1) / kKeepTile, wv = threadIdx.x >> 6;
  const uint32_t fid = threadIdx.x - 64, fn = blockDim.x - 64;  // formers: waves 1..
  auto len = [&](uint32_t tile) { return min(kKeepTile, K - tile * kKeepTile); };
  // e_r = exp(s_r - m) of one tile, into LDS and (for the second pass) HBM
  auto form_e = [&](uint32_t tile, float* dst, uint32_t id, uint32_t nthr) {
    const uint32_t base = tile * kKeepTile, n = len(tile);
    for (uint32_t j = id; j < n; j += nthr) {
      const float s = l[(uint32_t)key[base + j]] / T;
      const float d = s - m;
      const float ev = exp_pinned(d);
      dst[j] = ev;
      e[base + j] = ev;
    }
  };
  // the denominator
  float den = 0.0f;
  form_e(0, t[0], threadIdx.x, blockDim.x);
  __syncthreads();
  for (uint32_t tile = 0; tile < nt; ++tile) {
    if (wv == 0) {
      if (threadIdx.x == 0) {
        const float4* t4 = reinterpret_cast<const float4*>(t[tile & 1]);
        const uint32_t n = len(tile), n4 = n / 4;
        uint32_t g = 0;
        for (; g + 16 <= n4; g += 16) {
          float4 v[16];
#pragma unroll
          for (uint32_t u = 0; u < 16; ++u) v[u] = t4[g + u];
#pragma unroll
          for (uint32_t u = 0; u < 16; ++u) {
            den = den + v[u].x;
            den = den + v[u].y;
            den = den + v[u].z;
            den = den + v[u].w;
          }
        }
        for (uint32_t r = 4 * g; r < n; ++r) den = den + t[tile & 1][r];
      }
    } else if (tile + 1 < nt) {
      form_e(tile + 1, t[(tile + 1) & 1], fid, fn);
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    s_den = den;
    s_keep = 0xFFFFFFFFu;
  }
  __syncthreads();
  den = s_den;
  // p_r = e_r / den of one tile, into LDS
  auto form_p = [&](uint32_t tile, float* dst, uint32_t id, uint32_t nthr) {
    const uint32_t base = tile * kKeepTile, n = len(tile);
    for (uint32_t j = id; j < n; j += nthr) {
      const float p = e[base + j] / den;
      dst[j] = p;
    }
  };
  // the running sum up to the first failing rank
  float c = 0.0f;
  form_p(0, t[0], threadIdx.x, blockDim.x);
  __syncthreads();
  for (uint32_t tile = 0; tile < nt; ++tile) {
    if (wv == 0) {
      if (threadIdx.x == 0) {
        const float* tb = t[tile & 1];
        const float4* t4 = reinterpret_cast<const float4*>(tb);
        const uint32_t base = tile * kKeepTile, n = len(tile), n4 = n / 4;
        uint32_t keep = 0xFFFFFFFFu, g = 0;
        for (; g < n4 && keep == 0xFFFFFFFFu; g += 16) {
          float4 v[16];
#pragma unroll
          for (uint32_t u = 0; u < 16; ++u)
            if (g + u < n4) v[u] = t4[g + u];
#pragma unroll
          for (uint32_t u = 0; u < 16; ++u) {
            if (g + u < n4 && keep == 0xFFFFFFFFu) {
              const uint32_t r = base + 4 * (g + u);
              const float c0 = c + v[u].x;
              const float c1 = c0 + v[u].y;
              const float c2 = c1 + v[u].z;
              const float c3 = c2 + v[u].w;
              if (!(c2 < top_p)) {  // the prefix ends inside ranks r..r+3
                if (r > 0 && !(c < top_p)) keep = r;
                else if (!(c0 < top_p)) keep = r + 1;
                else if (!(c1 < top_p)) keep = r + 2;
                else keep = r + 3;
              }
              c = c3;
            }
          }
        }
        for (uint32_t j = 4 * n4; j < n && keep == 0xFFFFFFFFu; ++j) {
          const uint32_t r = base + j;
          if (r > 0 && !(c < top_p)) keep = r;
          else c = c + tb[j];
        }
        s_keep = keep;
      }
    } else if (tile + 1 < nt) {
      form_p(tile + 1, t[(tile + 1) & 1], fid, fn);
    }
    __syncthreads();
    if (s_keep != 0xFFFFFFFFu) break;
  }
  if (threadIdx.x == 0) *nkeep = s_keep == 0xFFFFFFFFu ? K : s_keep;
}

// (z, index) candidate packed so that a larger value is the better one:
// z descending, then index ascending (only finite or -inf z occur).
struct ZI {
  float z;
  uint32_t i;
};
__device__ __forceinline__ ZI zi_pick(ZI a, ZI b) {
  return (b.z > a.z || (b.z == a.z && b.i < a.i)) ? b : a;
}
__device__ __forceinline__ ZI zi_block(ZI c, ZI* red) {
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, nw = blockDim.x >> 6;
  for (uint32_t o = 32; o > 0; o >>= 1) {
    ZI d{__shfl_xor(c.z, o), __shfl_xor(c.i, o)};
    c = zi_pick(c, d);
  }
  if (lane == 0) red[wv] = c;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (uint32_t w = 1; w < nw; ++w) c = zi_pick(c, red[w]);
    red[0] = c;
  }
  __syncthreads();
  return red[0];
}

// Draft 14.4 over the kept ranks (or every index when nothing is cut):
// z = s + g, per-workgroup best (z, index).
__global__ __launch_bounds__(256) void k_draw(const uint64_t* __restrict__ key,
                                              const float* __restrict__ l, float T, uint32_t V,
                                              const uint32_t* __restrict__ nkeep, uint32_t all,
                                              uint64_t seed, uint32_t step, uint64_t* cand,
                                              uint32_t* err) {
  __shared__ ZI red[4];
  const uint32_t n = all ? V : *nkeep;
  ZI best{-__builtin_inff(), UINT32_MAX};
  bool nan = false;
  for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < n; r += gridDim.x * blockDim.x) {
    const uint32_t i = all ? r : (uint32_t)key[r];
    const float s = l[i] / T;
    nan |= s != s;
    const float z = s + gumbel(seed, step, i);
    best = zi_pick(best, ZI{z, i});
  }
  if (nan) atomicOr(err, 0x100u);
  best = zi_block(best, red);
  if (threadIdx.x == 0)
    cand[blockIdx.x] = ((uint64_t)best.i << 32) | __float_as_uint(best.z);
}

// The first index of the maximum z: the scan of section 11.2 starts at
// index 0 (z = -inf when masked), so the candidates reduce from (-inf, 0).
// nkeep_out (optional): the size of the kept set (V when nothing is cut).
__global__ __launch_bounds__(256) void k_draw_final(const uint64_t* __restrict__ cand,
                                                    uint32_t n, uint32_t* out,
                                                    const uint32_t* __restrict__ nkeep,
                                                    uint32_t all, uint32_t V,
                                                    uint32_t* nkeep_out) {
  __shared__ ZI red[4];
  ZI best{-__builtin_inff(), 0u};
  for (uint32_t b = threadIdx.x; b < n; b += blockDim.x) {
    const uint64_t c = cand[b];
    const ZI o{__uint_as_float((uint32_t)c), (uint32_t)(c >> 32)};
    if (o.i != UINT32_MAX) best = zi_pick(best, o);
  }
  best = zi_block(best, red);
  if (threadIdx.x == 0) {
    *out = best.i;
    if (nkeep_out) *nkeep_out = all ? V : *nkeep;
  }
}

__global__ void k_fill_u32(uint32_t* p, uint32_t n, uint32_t v) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

uint32_t sample_sort_len(uint32_t V) {
  uint32_t n = kTile;
  while (n < V) n <<= 1;
  return n;
}

hipError_t launch_sample(const float* logits, uint32_t V, const SampleParams& p, uint32_t step,
                         const SampleBufs& b, uint32_t* out, uint32_t* err, hipStream_t s,
                         uint32_t* nkeep_out) {
  if (V == 0 || b.V != V || b.Vp < sample_sort_len(V)) return hipErrorInvalidValue;
  const uint32_t K = (p.top_k > 0 && p.top_k < V) ? p.top_k : V;
  const bool all = K == V && !(p.top_p < 1.0f);
  const uint64_t* order = b.key;  // ascending rank keys, at least the first K sorted
  if (!all) {
    const uint32_t Vp = b.Vp, ntiles = Vp / kTile;
    hipLaunchKernelGGL(k_rank_keys, dim3((Vp + 255) / 256), dim3(256), 0, s, logits, V, Vp,
                       p.temperature, b.key, err);
    auto sort = [&](uint64_t* keys, uint32_t n) {  // n: a power of two >= kTile
      hipLaunchKernelGGL(k_bitonic_tile, dim3(n / kTile), dim3(1024), 0, s, keys, 0u, 0u);
      for (uint32_t k = 2 * kTile; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j >= kTile; j >>= 1)
          hipLaunchKernelGGL(k_bitonic_pass, dim3(n / 2 / 256), dim3(256), 0, s, keys, n, k, j);
        hipLaunchKernelGGL(k_bitonic_tile, dim3(n / kTile), dim3(1024), 0, s, keys, k, 0u);
      }
    };
    if (K < V && K <= kTile && ntiles > 1) {
      // top-k: sort the tiles, keep each tile's first K, sort those
      hipLaunchKernelGGL(k_bitonic_tile, dim3(ntiles), dim3(1024), 0, s, b.key, 0u, 1u);
      const uint32_t Cp = sample_sort_len(ntiles * K);
      hipLaunchKernelGGL(k_gather_top, dim3((Cp + 255) / 256), dim3(256), 0, s, b.key, K, ntiles,
                         Cp, b.key2);
      sort(b.key2, Cp);
      order = b.key2;
    } else {
      sort(b.key, Vp);
    }
    hipLaunchKernelGGL(k_keep, dim3(1), dim3(1024), 0, s, order, logits, p.temperature, K,
                       p.top_p, b.e, b.nkeep);
  }
  hipLaunchKernelGGL(k_draw, dim3(kSampleBlocks), dim3(256), 0, s, order, logits,
                     p.temperature, V, b.nkeep, all ? 1u : 0u, p.seed, step, b.cand, err);
  hipLaunchKernelGGL(k_draw_final, dim3(1), dim3(256), 0, s, b.cand, kSampleBlocks, out,
                     b.nkeep, all ? 1u : 0u, V, nkeep_out);
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Scratch of the no-allocation draw (cis2_sample_logits_noalloc): one copy
// of this array per GPU, held until the process ends, carved into the
// sampler's buffers for vocabularies up to kNoAllocMaxVocab.  In host code
// `scratch` names a host-side stand-in, never device memory: every host use
// goes through the address hipGetSymbolAddress returns for the device.
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kScrKeyWords = kNoAllocMaxVocab;        // [Vp] rank keys (Vp <= max vocab)
constexpr size_t kScrEWords = kNoAllocMaxVocab / 2;      // [V] f32 terms, two per word
constexpr size_t kScrCandWords = kSampleBlocks;          // per-workgroup candidates
constexpr size_t kScrFlagWords = 8;                      // nkeep (u32), error flag (u32)
constexpr size_t kScratchWords = 2 * kScrKeyWords + kScrEWords + kScrCandWords + kScrFlagWords;
static_assert(kNoAllocMaxVocab % kTile == 0, "the sort length of the largest vocabulary");
static_assert(kScratchWords * 8 == kNoAllocScratchBytes, "scratch size as declared");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];  // this GPU's address of `scratch`, or null
std::mutex g_scratch_use[kMaxDevices];  // held by a draw for its whole use of the scratch
}  // namespace

static __device__ __align__(256) uint64_t scratch[kScratchWords];

hipError_t sample_scratch_init() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (g_scratch_dev[dev]) return hipSuccess;
  void* ptr = nullptr;
  e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!ptr) return hipErrorInvalidSymbol;
  g_scratch_dev[dev] = ptr;
  return hipSuccess;
}

std::mutex* sample_scratch_lock(int dev) {
  return dev >= 0 && dev < kMaxDevices ? &g_scratch_use[dev] : nullptr;
}

hipError_t sample_scratch_bufs(int dev, uint32_t V, SampleBufs* b, uint32_t** err) {
  if (V == 0 || V > kNoAllocMaxVocab) return hipErrorInvalidValue;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* base = nullptr;
  {
    std::lock_guard<std::mutex> g(g_scratch_mu);
    base = g_scratch_dev[dev];
  }
  if (!base) return hipErrorNotInitialized;
  uint64_t* w = static_cast<uint64_t*>(base);
  b->V = V;
  b->Vp = sample_sort_len(V);
  b->key = w;
  b->key2 = w + kScrKeyWords;
  b->e = reinterpret_cast<float*>(w + 2 * kScrKeyWords);
  b->cand = w + 2 * kScrKeyWords + kScrEWords;
  uint32_t* flags = reinterpret_cast<uint32_t*>(b->cand + kScrCandWords);
  b->nkeep = flags;
  *err = flags + 1;
  return hipSuccess;
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t n, uint32_t v, hipStream_t s) {
  if (n == 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_u32, dim3((n + 255) / 256), dim3(256), 0, s, p, n, v);
  return hipGetLastError();
}

}  // namespace cis2
