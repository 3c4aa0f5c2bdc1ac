// cis2_artifacts.hpp — host-side readers for the artifacts the CIS-2 driver
// consumes: config.json, model.safetensors (BF16), and the decimal --ids
// file.  Error behaviour follows the reference driver: a malformed input is
// reported on stderr with a FATAL: prefix and the process exits with status 2
// (code/cis2-fp/gpu/cis2_model.h:255-359, cis2_host.cpp:26-45).
#pragma once
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <set>
#include <string>
#include <utility>
#include <vector>

namespace cis2 {

[[noreturn]] inline void fatal(const std::string& msg) {
  fprintf(stderr, "FATAL: %s\n", msg.c_str());
  exit(2);
}

// ---- JSON (the subset config.json and safetensors headers use) -----------
struct JValue {
  enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
  bool b = false;
  double num = 0.0;  // strtod: correctly rounded decimal -> binary64
  std::string str;
  std::vector<JValue> arr;
  std::vector<std::pair<std::string, JValue>> obj;
  const JValue* find(const char* key) const {
    if (kind != OBJ) return nullptr;
    for (auto& kv : obj)
      if (kv.first == key) return &kv.second;
    return nullptr;
  }
};

class JParser {
 public:
  JParser(const char* b, const char* e) : p_(b), e_(e) {}
  // Nesting deeper than this is refused (a header is two levels deep; an
  // unbounded recursion would let a crafted file overflow the stack).
  static constexpr int kMaxDepth = 64;
  JValue value(int depth = 0) {
    skip();
    if (p_ >= e_) fatal("JSON parse error: unexpected end");
    if (depth > kMaxDepth) fatal("JSON parse error: nesting too deep");
    JValue v;
    char ch = *p_;
    if (ch == '{') {
      v.kind = JValue::OBJ;
      ++p_;
      skip();
      if (p_ < e_ && *p_ == '}') { ++p_; return v; }
      std::set<std::string> seen;
      while (true) {
        skip();
        std::string k = string();
        if (!seen.insert(k).second) fatal("JSON parse error: duplicate key " + k);
        skip();
        if (p_ >= e_ || *p_ != ':') fatal("JSON parse error: expected ':'");
        ++p_;
        v.obj.emplace_back(std::move(k), value(depth + 1));
        skip();
        if (p_ < e_ && *p_ == ',') { ++p_; continue; }
        if (p_ < e_ && *p_ == '}') { ++p_; return v; }
        fatal("JSON parse error: expected ',' or '}'");
      }
    }
    if (ch == '[') {
      v.kind = JValue::ARR;
      ++p_;
      skip();
      if (p_ < e_ && *p_ == ']') { ++p_; return v; }
      while (true) {
        v.arr.push_back(value(depth + 1));
        skip();
        if (p_ < e_ && *p_ == ',') { ++p_; continue; }
        if (p_ < e_ && *p_ == ']') { ++p_; return v; }
        fatal("JSON parse error: expected ',' or ']'");
      }
    }
    if (ch == '"') { v.kind = JValue::STR; v.str = string(); return v; }
    if (lit("true")) { v.kind = JValue::BOOL; v.b = true; return v; }
    if (lit("false")) { v.kind = JValue::BOOL; v.b = false; return v; }
    if (lit("null")) return v;
    std::string num;
    while (p_ < e_ && *p_ && strchr("+-0123456789.eE", *p_)) num.push_back(*p_++);
    if (num.empty()) fatal("JSON parse error: expected a value");
    char* stop = nullptr;
    v.kind = JValue::NUM;
    v.num = strtod(num.c_str(), &stop);
    if (*stop) fatal("JSON parse error: bad number " + num);
    return v;
  }

 private:
  void skip() {
    while (p_ < e_ && (*p_ == ' ' || *p_ == '\n' || *p_ == '\r' || *p_ == '\t')) ++p_;
  }
  bool lit(const char* w) {
    size_t n = strlen(w);
    if ((size_t)(e_ - p_) >= n && memcmp(p_, w, n) == 0) { p_ += n; return true; }
    return false;
  }
  std::string string() {
    if (p_ >= e_ || *p_ != '"') fatal("JSON parse error: expected string");
    ++p_;
    std::string s;
    while (p_ < e_ && *p_ != '"') {
      char c = *p_++;
      if (c != '\\') { s.push_back(c); continue; }
      if (p_ >= e_) fatal("JSON parse error: truncated escape");
      char x = *p_++;
      switch (x) {
        case 'n': s.push_back('\n'); break;
        case 't': s.push_back('\t'); break;
        case 'r': s.push_back('\r'); break;
        case 'b': s.push_back('\b'); break;
        case 'f': s.push_back('\f'); break;
        case 'u': {
          if (e_ - p_ < 4) fatal("JSON parse error: truncated \\u");
          unsigned cp = (unsigned)strtoul(std::string(p_, 4).c_str(), nullptr, 16);
          p_ += 4;
          s.push_back(cp < 0x80 ? (char)cp : '?');
          break;
        }
        default: s.push_back(x);
      }
    }
    if (p_ >= e_) fatal("JSON parse error: unterminated string");
    ++p_;
    return s;
  }
  const char* p_;
  const char* e_;
};

inline std::string read_file(const std::string& path) {
  FILE* f = fopen(path.c_str(), "rb");
  if (!f) fatal("cannot open " + path);
  std::string s;
  char buf[1 << 16];
  size_t n;
  while ((n = fread(buf, 1, sizeof buf, f)) > 0) s.append(buf, n);
  fclose(f);
  return s;
}

inline JValue parse_json(const std::string& text) {
  JParser p(text.data(), text.data() + text.size());
  return p.value();
}

// ---- safetensors -------------------------------------------------------------
struct TensorView {
  std::string name, dtype;
  std::vector<uint64_t> shape;
  uint64_t begin = 0, end = 0;
};

struct SafeTensors {
  std::string blob;
  uint64_t data_off = 0;
  std::vector<TensorView> tensors;

  // Element size of a safetensors dtype, 0 when unknown.
  static uint64_t dtype_size(const std::string& d) {
    if (d == "BOOL" || d == "U8" || d == "I8" || d == "F8_E5M2" || d == "F8_E4M3") return 1;
    if (d == "I16" || d == "U16" || d == "F16" || d == "BF16") return 2;
    if (d == "I32" || d == "U32" || d == "F32") return 4;
    if (d == "I64" || d == "U64" || d == "F64") return 8;
    return 0;
  }
  // A JSON number that is an exact non-negative integer below 2^53.
  static bool as_index(const JValue& v, uint64_t* out) {
    if (v.kind != JValue::NUM || !(v.num >= 0.0) || v.num >= 9007199254740992.0 ||
        v.num != (double)(uint64_t)v.num)
      return false;
    *out = (uint64_t)v.num;
    return true;
  }

  // Reads the file and checks the whole header before any tensor is used:
  // header length within the file, a JSON object without duplicate keys,
  // every entry with a known dtype, integer shape and offsets, shape
  // product (no overflow) x element size == end - begin, every range inside
  // the data section and no two ranges overlapping.  Any violation is
  // fatal: a file whose declared sizes disagree with its length is never
  // accepted.
  void open(const std::string& path) {
    blob = read_file(path);
    if (blob.size() < 8) fatal("safetensors too short");
    uint64_t hlen = 0;
    for (int i = 0; i < 8; ++i) hlen |= (uint64_t)(unsigned char)blob[i] << (8 * i);
    if (hlen > blob.size() - 8) fatal("safetensors header length out of range");
    JValue j = parse_json(blob.substr(8, hlen));
    if (j.kind != JValue::OBJ) fatal("safetensors header not an object");
    data_off = 8 + hlen;
    const uint64_t data_len = blob.size() - data_off;
    for (auto& kv : j.obj) {
      if (kv.first == "__metadata__") {
        if (kv.second.kind != JValue::OBJ) fatal("safetensors __metadata__ not an object");
        continue;
      }
      const std::string& n = kv.first;
      const JValue *dt = kv.second.find("dtype"), *sh = kv.second.find("shape"),
                   *of = kv.second.find("data_offsets");
      if (kv.second.kind != JValue::OBJ || !dt || dt->kind != JValue::STR || !sh ||
          sh->kind != JValue::ARR || !of || of->kind != JValue::ARR || of->arr.size() != 2)
        fatal("tensor " + n + " entry malformed");
      TensorView t;
      t.name = n;
      t.dtype = dt->str;
      const uint64_t esz = dtype_size(t.dtype);
      if (!esz) fatal("tensor " + n + " unknown dtype " + t.dtype);
      uint64_t count = 1;
      for (auto& d : sh->arr) {
        uint64_t v = 0;
        if (!as_index(d, &v)) fatal("tensor " + n + " shape not a list of integers");
        if (v && count > UINT64_MAX / v) fatal("tensor " + n + " shape product overflows");
        count *= v;
        t.shape.push_back(v);
      }
      if (!as_index(of->arr[0], &t.begin) || !as_index(of->arr[1], &t.end) || t.end < t.begin ||
          t.end > data_len)
        fatal("tensor " + n + " byte range invalid");
      if (count > UINT64_MAX / esz || count * esz != t.end - t.begin)
        fatal("tensor " + n + " element count mismatch");
      tensors.push_back(t);
    }
    std::vector<std::pair<uint64_t, uint64_t>> r;
    for (auto& t : tensors)
      if (t.end > t.begin) r.emplace_back(t.begin, t.end);
    std::sort(r.begin(), r.end());
    for (size_t i = 1; i < r.size(); ++i)
      if (r[i].first < r[i - 1].second) fatal("safetensors tensor byte ranges overlap");
  }
  const TensorView* find(const std::string& n) const {
    for (auto& t : tensors)
      if (t.name == n) return &t;
    return nullptr;
  }
  // Validated BF16 payload of a tensor (dtype, shape, byte range), as
  // Cis2SafeTensors::load_bf16 checks them (cis2_model.h:340-360).
  const uint16_t* bf16(const TensorView& t, const std::vector<uint64_t>& expect) const {
    if (t.dtype != "BF16") fatal("tensor " + t.name + " dtype " + t.dtype + ", expected BF16");
    if (t.shape != expect) fatal("tensor " + t.name + " shape mismatch");
    uint64_t nbytes = t.end - t.begin;
    if (t.end < t.begin || nbytes % 2 || data_off + t.end > blob.size())
      fatal("tensor " + t.name + " byte range invalid");
    uint64_t want = 1;
    for (auto d : expect) want *= d;
    if (nbytes / 2 != want) fatal("tensor " + t.name + " element count mismatch");
    return reinterpret_cast<const uint16_t*>(blob.data() + data_off + t.begin);
  }
};

// ---- architecture gate on config.json alone (code/cis2-fp/src/main.rs:545-644) ----
// Refuses by name every configuration outside the specified subset, so that
// no digest is ever printed for arithmetic this build does not implement.
// Returns the refusal reason, or "" to accept.  Same checks, order and
// messages as the reference's gate, with one extension: model_type "qwen3"
// (the archived Qwen3 port, labs/w1x-qwen3/scripts/qwen3-port.diff, which
// reads head_dim from the config and applies the per-head QK-norm) is in
// the subset, and for it an explicit head_dim is honoured instead of
// refused.
inline std::string json_debug_str(const std::string& v) {  // Rust {:?} of a &str
  std::string o = "\"";
  for (char ch : v) {
    if (ch == '"' || ch == '\\') o.push_back('\\');
    o.push_back(ch);
  }
  return o + "\"";
}
inline bool json_u64(const JValue* v, uint64_t* out) {  // serde as_u64
  if (!v || v->kind != JValue::NUM || !(v->num >= 0.0) || v->num > 18446744073709549568.0 ||
      v->num != (double)(uint64_t)v->num)
    return false;
  *out = (uint64_t)v->num;
  return true;
}
inline std::string json_f64_display(double x) {  // Rust Display of an f64 (shortest round trip)
  char b[64];
  for (int prec = 1; prec <= 17; ++prec) {
    snprintf(b, sizeof b, "%.*g", prec, x);
    if (strtod(b, nullptr) == x) break;
  }
  return b;
}
inline std::string gate_architecture(const JValue& c) {
  auto present = [&](const char* k) {
    const JValue* v = c.find(k);
    return v && v->kind != JValue::NUL;
  };
  std::string mt;
  if (const JValue* v = c.find("model_type"); v && v->kind == JValue::STR) {
    mt = v->str;
    if (mt != "llama" && mt != "qwen2" && mt != "qwen3")
      return "model_type=" + json_debug_str(mt) +
             " is not in the CIS-2 specified subset [\"llama\", \"qwen2\", \"qwen3\"]";
  }
  if (const JValue* v = c.find("torch_dtype"); v && v->kind == JValue::STR && v->str != "bfloat16")
    return "torch_dtype=" + json_debug_str(v->str) +
           "; CIS-2 pins bf16-on-disk weights (\xc2\xa7" "3.5)";
  uint64_t h = 0, nh = 0;
  if (json_u64(c.find("hidden_size"), &h) && json_u64(c.find("num_attention_heads"), &nh)) {
    if (nh == 0) return "num_attention_heads=0";
    const uint64_t derived = h / nh;
    uint64_t used = derived, explicit_hd = 0;
    if (json_u64(c.find("head_dim"), &explicit_hd)) {
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
  if (const JValue* v = c.find("partial_rotary_factor"); v && v->kind == JValue::NUM && v->num != 1.0)
    return "partial_rotary_factor=" + json_f64_display(v->num) + "; only full rotary is specified";
  if (present("rope_scaling")) return "rope_scaling is set; only unscaled RoPE is specified";
  if (const JValue* v = c.find("use_sliding_window"); v && v->kind == JValue::BOOL && v->b)
    return "use_sliding_window=true; only full causal attention is specified";
  if (present("quantization_config"))
    return "quantization_config is present; CIS-2 reads unquantized bf16 weights";
  for (const char* k : {"attention_multiplier", "embedding_multiplier", "residual_multiplier",
                        "logits_scaling", "attn_logit_softcapping", "final_logit_softcapping",
                        "query_pre_attn_scalar"})
    if (present(k))
      return std::string(k) +
             " is set; this implementation hardcodes rsqrt(head_dim) attention scaling and no "
             "logit scaling, so the result would be silently wrong";
  for (const char* k : {"num_local_experts", "num_experts", "n_routed_experts", "moe_intermediate_size"})
    if (present(k)) return std::string(k) + " is set; MoE routing is not specified";
  return "";
}

// ---- --ids file: decimal ids separated by whitespace or commas ------------------
inline std::vector<uint32_t> read_ids(const std::string& path) {
  std::string t = read_file(path);
  std::vector<uint32_t> ids;
  size_t i = 0;
  while (i < t.size()) {
    while (i < t.size() && t[i] && strchr("\n\r \t,", t[i])) ++i;
    if (i >= t.size()) break;
    size_t j = i;
    while (j < t.size() && t[j] >= '0' && t[j] <= '9') ++j;
    if (j == i) fatal(path + ": expected a decimal token id at byte " + std::to_string(i));
    ids.push_back((uint32_t)strtoul(t.substr(i, j - i).c_str(), nullptr, 10));
    i = j;
  }
  if (ids.empty()) fatal(path + ": no token ids");
  return ids;
}

}  // namespace cis2
