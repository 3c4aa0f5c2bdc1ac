// cis2_sha256.cpp — SHA-256 with an x86 SHA-extensions fast path.
#include "cis2_sha256.hpp"

#include <cpuid.h>
#include <immintrin.h>
#include <string.h>

namespace cis2 {
namespace {

const uint32_t K256[64] = {
    0x428a2f98u, 0x71374491u, 0xb5c0fbcfu, 0xe9b5dba5u, 0x3956c25bu, 0x59f111f1u,
    0x923f82a4u, 0xab1c5ed5u, 0xd807aa98u, 0x12835b01u, 0x243185beu, 0x550c7dc3u,
    0x72be5d74u, 0x80deb1feu, 0x9bdc06a7u, 0xc19bf174u, 0xe49b69c1u, 0xefbe4786u,
    0x0fc19dc6u, 0x240ca1ccu, 0x2de92c6fu, 0x4a7484aau, 0x5cb0a9dcu, 0x76f988dau,
    0x983e5152u, 0xa831c66du, 0xb00327c8u, 0xbf597fc7u, 0xc6e00bf3u, 0xd5a79147u,
    0x06ca6351u, 0x14292967u, 0x27b70a85u, 0x2e1b2138u, 0x4d2c6dfcu, 0x53380d13u,
    0x650a7354u, 0x766a0abbu, 0x81c2c92eu, 0x92722c85u, 0xa2bfe8a1u, 0xa81a664bu,
    0xc24b8b70u, 0xc76c51a3u, 0xd192e819u, 0xd6990624u, 0xf40e3585u, 0x106aa070u,
    0x19a4c116u, 0x1e376c08u, 0x2748774cu, 0x34b0bcb5u, 0x391c0cb3u, 0x4ed8aa4au,
    0x5b9cca4fu, 0x682e6ff3u, 0x748f82eeu, 0x78a5636fu, 0x84c87814u, 0x8cc70208u,
    0x90befffau, 0xa4506cebu, 0xbef9a3f7u, 0xc67178f2u};

inline uint32_t rotr(uint32_t x, int n) { return (x >> n) | (x << (32 - n)); }

void blocks_portable(uint32_t st[8], const uint8_t* p, size_t nblk) {
  for (; nblk; --nblk, p += 64) {
    uint32_t w[64];
    for (int i = 0; i < 16; ++i)
      w[i] = (uint32_t)p[4 * i] << 24 | (uint32_t)p[4 * i + 1] << 16 |
             (uint32_t)p[4 * i + 2] << 8 | p[4 * i + 3];
    for (int i = 16; i < 64; ++i) {
      uint32_t s0 = rotr(w[i - 15], 7) ^ rotr(w[i - 15], 18) ^ (w[i - 15] >> 3);
      uint32_t s1 = rotr(w[i - 2], 17) ^ rotr(w[i - 2], 19) ^ (w[i - 2] >> 10);
      w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = st[0], b = st[1], c = st[2], d = st[3], e = st[4], f = st[5], g = st[6],
             h = st[7];
    for (int i = 0; i < 64; ++i) {
      uint32_t t1 = h + (rotr(e, 6) ^ rotr(e, 11) ^ rotr(e, 25)) + ((e & f) ^ (~e & g)) +
                    K256[i] + w[i];
      uint32_t t2 = (rotr(a, 2) ^ rotr(a, 13) ^ rotr(a, 22)) + ((a & b) ^ (a & c) ^ (b & c));
      h = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    st[0] += a; st[1] += b; st[2] += c; st[3] += d;
    st[4] += e; st[5] += f; st[6] += g; st[7] += h;
  }
}

// SHA-NI: state kept as (ABEF, CDGH); 16 groups of four rounds, the
// schedule W[4g..4g+3] = msg2(msg1(W[g-4],W[g-3]) + W[4g-7..4g-4], W[g-1]).
__attribute__((target("sha,sse4.1"))) void blocks_shani(uint32_t st[8], const uint8_t* p,
                                                        size_t nblk) {
  const __m128i bswap = _mm_set_epi64x(0x0c0d0e0f08090a0bULL, 0x0405060700010203ULL);
  __m128i t = _mm_loadu_si128(reinterpret_cast<const __m128i*>(&st[0]));
  __m128i s1 = _mm_loadu_si128(reinterpret_cast<const __m128i*>(&st[4]));
  t = _mm_shuffle_epi32(t, 0xB1);
  s1 = _mm_shuffle_epi32(s1, 0x1B);
  __m128i s0 = _mm_alignr_epi8(t, s1, 8);
  s1 = _mm_blend_epi16(s1, t, 0xF0);
  for (; nblk; --nblk, p += 64) {
    const __m128i a0 = s0, c0 = s1;
    __m128i m[16];
    for (int g = 0; g < 16; ++g) {
      if (g < 4) {
        m[g] = _mm_shuffle_epi8(_mm_loadu_si128(reinterpret_cast<const __m128i*>(p + 16 * g)),
                                bswap);
      } else {
        __m128i x = _mm_sha256msg1_epu32(m[g - 4], m[g - 3]);
        x = _mm_add_epi32(x, _mm_alignr_epi8(m[g - 1], m[g - 2], 4));
        m[g] = _mm_sha256msg2_epu32(x, m[g - 1]);
      }
      __m128i msg = _mm_add_epi32(m[g], _mm_loadu_si128(reinterpret_cast<const __m128i*>(&K256[4 * g])));
      s1 = _mm_sha256rnds2_epu32(s1, s0, msg);
      msg = _mm_shuffle_epi32(msg, 0x0E);
      s0 = _mm_sha256rnds2_epu32(s0, s1, msg);
    }
    s0 = _mm_add_epi32(s0, a0);
    s1 = _mm_add_epi32(s1, c0);
  }
  t = _mm_shuffle_epi32(s0, 0x1B);
  s1 = _mm_shuffle_epi32(s1, 0xB1);
  s0 = _mm_blend_epi16(t, s1, 0xF0);
  s1 = _mm_alignr_epi8(s1, t, 8);
  _mm_storeu_si128(reinterpret_cast<__m128i*>(&st[0]), s0);
  _mm_storeu_si128(reinterpret_cast<__m128i*>(&st[4]), s1);
}

bool have_shani() {
  unsigned a, b, c, d;
  if (!__get_cpuid_count(7, 0, &a, &b, &c, &d)) return false;
  bool sha = (b >> 29) & 1u;
  if (!__get_cpuid(1, &a, &b, &c, &d)) return false;
  bool sse41 = (c >> 19) & 1u, ssse3 = (c >> 9) & 1u;
  return sha && sse41 && ssse3;
}

typedef void (*blocks_fn)(uint32_t*, const uint8_t*, size_t);
blocks_fn pick() { return have_shani() ? blocks_shani : blocks_portable; }
const blocks_fn g_blocks = pick();

}  // namespace

const char* sha256_impl() { return g_blocks == blocks_shani ? "sha-ni" : "portable"; }

void Sha256::reset() {
  static const uint32_t iv[8] = {0x6a09e667u, 0xbb67ae85u, 0x3c6ef372u, 0xa54ff53au,
                                 0x510e527fu, 0x9b05688cu, 0x1f83d9abu, 0x5be0cd19u};
  memcpy(h, iv, sizeof iv);
  total = 0;
  fill = 0;
}

void Sha256::update(const void* data, size_t n) {
  const uint8_t* p = static_cast<const uint8_t*>(data);
  total += n;
  if (fill) {
    size_t take = 64 - fill < n ? 64 - fill : n;
    memcpy(buf + fill, p, take);
    fill += take; p += take; n -= take;
    if (fill == 64) { g_blocks(h, buf, 1); fill = 0; }
  }
  if (n >= 64) {
    size_t nb = n / 64;
    g_blocks(h, p, nb);
    p += nb * 64; n -= nb * 64;
  }
  if (n) { memcpy(buf, p, n); fill = n; }
}

void Sha256::update_u32le(uint32_t v) {
  uint8_t b[4] = {(uint8_t)v, (uint8_t)(v >> 8), (uint8_t)(v >> 16), (uint8_t)(v >> 24)};
  update(b, 4);
}

void Sha256::finish(uint8_t out[32]) {
  uint64_t bits = total * 8;
  uint8_t pad[72];
  size_t padlen = (fill < 56) ? (56 - fill) : (120 - fill);
  memset(pad, 0, sizeof pad);
  pad[0] = 0x80;
  for (int i = 0; i < 8; ++i) pad[padlen + i] = (uint8_t)(bits >> (56 - 8 * i));
  uint64_t keep = total;
  update(pad, padlen + 8);
  total = keep;
  for (int i = 0; i < 8; ++i) {
    out[4 * i] = (uint8_t)(h[i] >> 24);
    out[4 * i + 1] = (uint8_t)(h[i] >> 16);
    out[4 * i + 2] = (uint8_t)(h[i] >> 8);
    out[4 * i + 3] = (uint8_t)h[i];
  }
}

void sha256(const void* data, size_t n, uint8_t out[32]) {
  Sha256 s;
  s.update(data, n);
  s.finish(out);
}

}  // namespace cis2
