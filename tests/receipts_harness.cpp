// Harness for the receipt-log tests: drives cis2_receipts.hpp (the CLI's
// receipt log) on the CPU.
//   canon FILE              canonical form of the JSON document in FILE
//   append LOG FIELDS_FILE  append a record whose fields are the members of
//                           the JSON object in FIELDS_FILE; prints log_hash
//   verify LOG [ID]         prints the chain check; exit 0 ok, 1 broken
#include <stdio.h>

#include "cis2_checkpoint.hpp"
#include "cis2_receipts.hpp"

using namespace cis2;

int main(int argc, char** argv) {
  if (argc < 3) return 3;
  const std::string cmd = argv[1];
  if (cmd == "canon") {
    const JsonDoc d = parse_json_text(slurp(argv[2]));
    printf("%s", serialize(d, d.root(), ",", ":").c_str());
    return 0;
  }
  if (cmd == "append" && argc == 4) {
    const JsonDoc d = parse_json_text(slurp(argv[3]));
    std::vector<ReceiptField> f;
    for (const JsonNode* c : d.children(d.root()))
      f.emplace_back(c->key, serialize(d, *c, ",", ":"));
    const auto r = append_receipt(argv[2], f);
    printf("%s\n", r.second.c_str());
    return r.first ? 0 : 1;
  }
  if (cmd == "verify") {
    FILE* fp = fopen(argv[2], "rb");
    const std::string text = fp ? (fclose(fp), slurp(argv[2])) : std::string();
    const std::string id = argc > 3 ? argv[3] : "";
    const ChainResult r = verify_chain_text(text, argc > 3 ? &id : nullptr);
    printf("%s\n", r.message.c_str());
    return r.ok ? 0 : 1;
  }
  return 3;
}
