// cis2_checkpoint.hpp — host-side access to the files the CIS-2 driver
// reads: config.json, model.safetensors (BF16) and the decimal --ids file.
//
// model.safetensors is streamed: open() reads only the 8-byte length and the
// JSON header and validates every entry against the file's size; each
// tensor is then read with one seek and one read into a caller's buffer, so
// the host never holds more than one tensor (the reference's per-tensor
// loader, code/cis2-fp/src/stream_widen.rs:1-33).  Files are hashed through
// a 1 MiB buffer.  A malformed input ends the process with a FATAL: line on
// stderr and exit status 2, the reference driver's error contract
// (code/cis2-fp/gpu/cis2_host.cpp:26-45).
#pragma once
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#include <algorithm>
#include <string>
#include <utility>
#include <vector>

#include "cis2_json.hpp"
#include "cis2_sha256.hpp"

namespace cis2 {

[[noreturn]] inline void fatal(const std::string& msg) {
  fprintf(stderr, "FATAL: %s\n", msg.c_str());
  exit(2);
}
inline void fatal_cb(const std::string& msg) { fatal(msg); }

// A file read whole (config.json, the --ids file: a few KB).
inline std::string slurp(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) fatal("cannot open " + path);
  std::string s;
  std::vector<char> buf(1 << 16);
  size_t n;
  while ((n = fread(buf.data(), 1, buf.size(), f)) > 0) s.append(buf.data(), n);
  const bool bad = ferror(f) != 0;
  fclose(f);
  if (bad) fatal("read error on " + path);
  return s;
}

// SHA-256 of a file through a 1 MiB buffer.
inline void hash_file(const std::string& path, uint8_t out[32]) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) fatal("cannot open " + path);
  Sha256 h;
  std::vector<unsigned char> buf(1 << 20);
  size_t n;
  while ((n = fread(buf.data(), 1, buf.size(), f)) > 0) h.update(buf.data(), n);
  const bool bad = ferror(f) != 0;
  fclose(f);
  if (bad) fatal("read error on " + path);
  h.finish(out);
}

inline JsonDoc parse_json_text(const std::string& text) {
  return JsonDoc::parse(text.data(), text.size(), fatal_cb);
}

// A JSON number that is a whole number in [0, limit]; false otherwise.
inline bool whole_number(const JsonNode* v, double limit, uint64_t* out) {
  if (!v || v->type != JsonNode::Number) return false;
  const double x = v->number;
  if (!(x >= 0.0) || !(x <= limit)) return false;
  const uint64_t u = (uint64_t)x;
  if ((double)u != x) return false;
  *out = u;
  return true;
}

// ---- model.safetensors -------------------------------------------------------
class Checkpoint {
 public:
  struct Tensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t elements = 0;
    uint64_t first = 0, last = 0;  // byte range [first, last) of the data section
  };

  // Largest header the reader accepts (safetensors writers stay below it).
  static constexpr uint64_t kMaxHeaderBytes = 100ull << 20;

  Checkpoint() = default;
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;
  ~Checkpoint() { close(); }

  // Reads and checks the header: its length within the file, a JSON object
  // (no duplicate keys), every entry an object with a known dtype, a shape
  // of whole numbers whose product (without overflow) times the element
  // size is the entry's byte count, offsets of whole numbers inside the data
  // section, and no two entries' bytes overlapping.  Nothing is accepted
  // whose declared sizes disagree with the file.
  void open(const std::string& path) {
    close();
    path_ = path;
    fp_ = fopen(path.c_str(), "rb");
    if (!fp_) fatal("cannot open " + path);
    struct stat sb;
    if (fstat(fileno(fp_), &sb) != 0) fatal("cannot stat " + path);
    size_ = (uint64_t)sb.st_size;
    unsigned char len8[8];
    if (size_ < 8 || fread(len8, 1, 8, fp_) != 8) fatal("safetensors: file shorter than 8 bytes");
    uint64_t hlen = 0;
    for (int i = 7; i >= 0; --i) hlen = hlen << 8 | len8[i];
    if (hlen > size_ - 8) fatal("safetensors: header length beyond the end of the file");
    // the header is read whole before it is parsed: refuse a declared length
    // beyond what any writer produces before allocating it
    if (hlen > kMaxHeaderBytes) fatal("safetensors: header length above the 100 MiB limit");
    std::string text((size_t)hlen, '\0');
    if (hlen && fread(&text[0], 1, (size_t)hlen, fp_) != hlen)
      fatal("safetensors: short read of the header");
    data_at_ = 8 + hlen;
    const JsonDoc doc = parse_json_text(text);
    const JsonNode& top = doc.root();
    if (top.type != JsonNode::Object) fatal("safetensors: header is not a JSON object");
    const uint64_t data_bytes = size_ - data_at_;
    for (const JsonNode* e : doc.children(top)) {
      if (e->key == "__metadata__") {
        if (e->type != JsonNode::Object) fatal("safetensors: __metadata__ is not an object");
        continue;
      }
      tensors_.push_back(entry(doc, *e, data_bytes));
    }
    std::vector<std::pair<uint64_t, uint64_t>> spans;
    for (const Tensor& t : tensors_)
      if (t.last > t.first) spans.emplace_back(t.first, t.last);
    std::sort(spans.begin(), spans.end());
    for (size_t i = 1; i < spans.size(); ++i)
      if (spans[i].first < spans[i - 1].second) fatal("safetensors: two tensors share bytes");
  }

  void close() {
    if (fp_) fclose(fp_);
    fp_ = nullptr;
    tensors_.clear();
  }

  const std::vector<Tensor>& tensors() const { return tensors_; }
  const Tensor* find(const std::string& name) const {
    for (const Tensor& t : tensors_)
      if (t.name == name) return &t;
    return nullptr;
  }

  // The checks of Cis2SafeTensors::load_bf16 (code/cis2-fp/gpu/cis2_model.h:340-360):
  // dtype BF16 and exactly the expected shape.
  void require_bf16(const Tensor& t, const std::vector<uint64_t>& shape) const {
    if (t.dtype != "BF16") fatal("tensor " + t.name + " dtype " + t.dtype + ", expected BF16");
    if (t.shape != shape) fatal("tensor " + t.name + " shape mismatch");
  }

  // The tensor's BF16 elements (little-endian in the file) into dst.
  void read_bf16(const Tensor& t, std::vector<uint16_t>& dst) {
    dst.resize((size_t)t.elements);
    read_bytes(t, 0, dst.data(), t.last - t.first);
#if defined(__BYTE_ORDER__) && __BYTE_ORDER__ == __ORDER_BIG_ENDIAN__
    for (uint16_t& v : dst) v = (uint16_t)(v << 8 | v >> 8);
#endif
  }

  // n bytes at offset `off` of the tensor's payload.
  void read_bytes(const Tensor& t, uint64_t off, void* dst, uint64_t n) {
    if (!fp_) fatal("safetensors: not open");
    if (off > t.last - t.first || n > t.last - t.first - off)
      fatal("tensor " + t.name + ": read outside its bytes");
    if (n == 0) return;
    if (fseeko(fp_, (off_t)(data_at_ + t.first + off), SEEK_SET) != 0 ||
        fread(dst, 1, (size_t)n, fp_) != n)
      fatal("tensor " + t.name + ": short read from " + path_);
  }

 private:
  FILE* fp_ = nullptr;
  std::string path_;
  uint64_t size_ = 0, data_at_ = 0;
  std::vector<Tensor> tensors_;

  static uint64_t element_bytes(const std::string& d) {
    static const std::pair<const char*, uint64_t> k[] = {
        {"BOOL", 1}, {"U8", 1},  {"I8", 1},  {"F8_E5M2", 1}, {"F8_E4M3", 1}, {"I16", 2},
        {"U16", 2},  {"F16", 2}, {"BF16", 2}, {"I32", 4},    {"U32", 4},     {"F32", 4},
        {"I64", 8},  {"U64", 8}, {"F64", 8}};
    for (const auto& e : k)
      if (d == e.first) return e.second;
    return 0;
  }

  static Tensor entry(const JsonDoc& doc, const JsonNode& e, uint64_t data_bytes) {
    const std::string& n = e.key;
    if (e.type != JsonNode::Object) fatal("tensor " + n + " entry is not an object");
    const JsonNode* dt = doc.member(e, "dtype");
    const JsonNode* sh = doc.member(e, "shape");
    const JsonNode* of = doc.member(e, "data_offsets");
    if (!dt || dt->type != JsonNode::String) fatal("tensor " + n + " has no dtype string");
    if (!sh || sh->type != JsonNode::Array) fatal("tensor " + n + " has no shape list");
    if (!of || of->type != JsonNode::Array || of->count != 2)
      fatal("tensor " + n + " has no [begin, end] data_offsets");
    Tensor t;
    t.name = n;
    t.dtype = dt->text;
    const uint64_t esz = element_bytes(t.dtype);
    if (esz == 0) fatal("tensor " + n + " unknown dtype " + t.dtype);
    constexpr double kWhole = 9007199254740991.0;  // 2^53 - 1: exact in a double
    uint64_t elements = 1;
    for (const JsonNode* d : doc.children(*sh)) {
      uint64_t v = 0;
      if (!whole_number(d, kWhole, &v)) fatal("tensor " + n + " shape entry is not a whole number");
      if (v != 0 && elements > UINT64_MAX / v) fatal("tensor " + n + " shape product overflows");
      elements *= v;
      t.shape.push_back(v);
    }
    const std::vector<const JsonNode*> o = doc.children(*of);
    if (!whole_number(o[0], kWhole, &t.first) || !whole_number(o[1], kWhole, &t.last) ||
        t.last < t.first || t.last > data_bytes)
      fatal("tensor " + n + " byte range outside the data section");
    if (elements > UINT64_MAX / esz || elements * esz != t.last - t.first)
      fatal("tensor " + n + " byte count disagrees with its shape and dtype");
    t.elements = elements;
    return t;
  }
};

// ---- architecture gate on config.json alone (code/cis2-fp/src/main.rs:545-644) ----
// Refuses by name every configuration outside the specified subset, so that
// no digest is ever printed for arithmetic this build does not implement.
// Returns the refusal reason, or "" to accept.  Same checks, order and
// messages as the reference's gate (callers match them), with one
// extension: model_type "qwen3" (the archived Qwen3 port,
// labs/w1x-qwen3/scripts/qwen3-port.diff, which reads head_dim from the
// config and applies the per-head QK-norm) is in the subset, and for it an
// explicit head_dim is honoured instead of refused.
inline std::string debug_quoted(const std::string& v) {  // Rust {:?} of a &str (ASCII)
  std::string o = "\"";
  for (char ch : v) {
    if (ch == '"' || ch == '\\') o.push_back('\\');
    o.push_back(ch);
  }
  return o + "\"";
}
inline bool config_u64(const JsonNode* v, uint64_t* out) {  // serde's as_u64
  return whole_number(v, 18446744073709549568.0, out);
}
inline std::string shortest_f64(double x) {  // Rust Display of an f64: shortest round trip
  char b[64];
  for (int prec = 1; prec <= 17; ++prec) {
    snprintf(b, sizeof b, "%.*g", prec, x);
    if (strtod(b, nullptr) == x) break;
  }
  return b;
}
inline std::string gate_architecture(const JsonDoc& doc) {
  const JsonNode& c = doc.root();
  auto field = [&](const char* k) { return doc.member(c, k); };
  auto set = [&](const char* k) {
    const JsonNode* v = field(k);
    return v && v->type != JsonNode::Null;
  };
  std::string mt;
  if (const JsonNode* v = field("model_type"); v && v->type == JsonNode::String) {
    mt = v->text;
    if (mt != "llama" && mt != "qwen2" && mt != "qwen3")
      return "model_type=" + debug_quoted(mt) +
             " is not in the CIS-2 specified subset [\"llama\", \"qwen2\", \"qwen3\"]";
  }
  if (const JsonNode* v = field("torch_dtype"); v && v->type == JsonNode::String && v->text != "bfloat16")
    return "torch_dtype=" + debug_quoted(v->text) +
           "; CIS-2 pins bf16-on-disk weights (\xc2\xa7" "3.5)";
  uint64_t h = 0, nh = 0;
  if (config_u64(field("hidden_size"), &h) && config_u64(field("num_attention_heads"), &nh)) {
    if (nh == 0) return "num_attention_heads=0";
    const uint64_t derived = h / nh;
    uint64_t used = derived, explicit_hd = 0;
    if (config_u64(field("head_dim"), &explicit_hd)) {
      if (mt == "qwen3") {
        used = explicit_hd;
      } else if (explicit_hd != derived) {
        return "config declares head_dim=" + std::to_string(explicit_hd) +
               " but this implementation derives hidden_size/num_attention_heads=" +
               std::to_string(derived) +
               "; the decode path uses the derived value, so the explicit one would be "
               "silently ignored";
      }
    }
    if (used % 2 != 0)
      return (used == derived ? "derived head_dim=" : "head_dim=") + std::to_string(used) +
             " is odd; RoPE pairs require even";
  }
  if (const JsonNode* v = field("partial_rotary_factor"); v && v->type == JsonNode::Number && v->number != 1.0)
    return "partial_rotary_factor=" + shortest_f64(v->number) + "; only full rotary is specified";
  if (set("rope_scaling")) return "rope_scaling is set; only unscaled RoPE is specified";
  if (const JsonNode* v = field("use_sliding_window"); v && v->type == JsonNode::Bool && v->flag)
    return "use_sliding_window=true; only full causal attention is specified";
  if (set("quantization_config"))
    return "quantization_config is present; CIS-2 reads unquantized bf16 weights";
  for (const char* k : {"attention_multiplier", "embedding_multiplier", "residual_multiplier",
                        "logits_scaling", "attn_logit_softcapping", "final_logit_softcapping",
                        "query_pre_attn_scalar"})
    if (set(k))
      return std::string(k) +
             " is set; this implementation hardcodes rsqrt(head_dim) attention scaling and no "
             "logit scaling, so the result would be silently wrong";
  for (const char* k : {"num_local_experts", "num_experts", "n_routed_experts", "moe_intermediate_size"})
    if (set(k)) return std::string(k) + " is set; MoE routing is not specified";
  return "";
}

// ---- --ids file: decimal ids separated by whitespace or commas ---------------
inline std::vector<uint32_t> read_ids(const std::string& path) {
  const std::string t = slurp(path);
  std::vector<uint32_t> ids;
  size_t i = 0;
  auto sep = [](char ch) { return ch == ' ' || ch == '\t' || ch == '\n' || ch == '\r' || ch == ','; };
  while (i < t.size()) {
    if (sep(t[i])) {
      ++i;
      continue;
    }
    uint64_t v = 0;
    size_t j = i;
    while (j < t.size() && t[j] >= '0' && t[j] <= '9' && v <= 0xFFFFFFFFull) v = v * 10 + (uint64_t)(t[j++] - '0');
    if (j == i) fatal(path + ": expected a decimal token id at byte " + std::to_string(i));
    if (v > 0xFFFFFFFFull) fatal(path + ": token id beyond 32 bits at byte " + std::to_string(i));
    ids.push_back((uint32_t)v);
    i = j;
  }
  if (ids.empty()) fatal(path + ": no token ids");
  return ids;
}

}  // namespace cis2
