// Loader harness for the malformed-file tests: opens a safetensors file with
// the CLI's reader (cis2_artifacts.hpp) and reads the first and last element
// of every tensor, as the reference lab's fuzz harnesses do
// (labs/rust-3/PREREG-from-ledger.md: "reads the opening and closing element
// of each").  Exit 0: accepted; exit 2: refused with a FATAL line.  Built
// with AddressSanitizer and UBSan by tests/test_safetensors_mutants.py.
#include "cis2_artifacts.hpp"

int main(int argc, char** argv) {
  if (argc != 2) return 3;
  cis2::SafeTensors st;
  st.open(argv[1]);
  unsigned sum = 0;
  for (const auto& t : st.tensors) {
    if (t.end == t.begin) continue;
    const unsigned char* p = reinterpret_cast<const unsigned char*>(st.blob.data()) + st.data_off;
    sum += p[t.begin] + p[t.end - 1];
  }
  printf("accepted %zu tensors (%u)\n", st.tensors.size(), sum & 1);
  return 0;
}
