// cis2_sha256.hpp — SHA-256 (FIPS 180-4) for the witness fold and digests.
// Uses the x86 SHA extensions when the CPU has them (checked at run time),
// otherwise a portable compression function; both give identical digests.
#pragma once
#include <stddef.h>
#include <stdint.h>

namespace cis2 {

struct Sha256 {
  uint32_t h[8];
  uint64_t total;
  uint8_t buf[64];
  size_t fill;

  Sha256() { reset(); }
  void reset();
  void update(const void* data, size_t n);
  void update_u32le(uint32_t v);
  void finish(uint8_t out[32]);
};

void sha256(const void* data, size_t n, uint8_t out[32]);
// Which compression path is in use ("sha-ni" or "portable").
const char* sha256_impl();

}  // namespace cis2
