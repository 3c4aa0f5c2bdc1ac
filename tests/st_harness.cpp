// Loader harness for the malformed-file tests: opens a safetensors file with
// the CLI's streaming reader (cis2_checkpoint.hpp) and reads the first and
// last byte of every tensor, as the reference lab's fuzz harnesses read the
// opening and closing element of each (labs/rust-3/PREREG-from-ledger.md).
// With --all it reads every tensor whole, one at a time, and reports the
// peak resident set size.  Exit 0: accepted; exit 2: refused with a FATAL
// line.  Built with AddressSanitizer and UBSan by
// tests/test_safetensors_mutants.py.
#include <sys/resource.h>

#include "cis2_checkpoint.hpp"

int main(int argc, char** argv) {
  if (argc < 2 || argc > 3) return 3;
  const bool all = argc == 3 && !strcmp(argv[2], "--all");
  cis2::Checkpoint ck;
  ck.open(argv[1]);
  unsigned sum = 0;
  uint64_t largest = 0;
  std::vector<uint16_t> buf;
  for (const auto& t : ck.tensors()) {
    const uint64_t n = t.last - t.first;
    if (n == 0) continue;
    largest = n > largest ? n : largest;
    unsigned char a = 0, b = 0;
    ck.read_bytes(t, 0, &a, 1);
    ck.read_bytes(t, n - 1, &b, 1);
    sum += a + b;
    if (all && t.dtype == "BF16") {
      ck.read_bf16(t, buf);
      for (uint16_t v : buf) sum += v;
    }
  }
  struct rusage ru;
  getrusage(RUSAGE_SELF, &ru);
  printf("accepted %zu tensors (%u) largest_bytes=%llu peak_rss_kb=%ld\n", ck.tensors().size(),
         sum & 1, (unsigned long long)largest, ru.ru_maxrss);
  return 0;
}
