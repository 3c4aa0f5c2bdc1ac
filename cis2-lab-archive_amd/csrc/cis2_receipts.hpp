// cis2_receipts.hpp — the hash-chained, append-only receipt log of the
// CIS-2 service (code/cis2-llm/server/app/receipts.py:31-97), for the CLI.
//
// A log is a file of JSON lines.  Every record carries prev_hash (the
// previous record's log_hash; 64 zero hex digits for the first) and
// log_hash = sha256 of the record without log_hash in canonical form:
// keys sorted, separators "," and ":", non-ASCII and control characters
// escaped as \uXXXX, integers as written, floats in their shortest
// round-trip form — the bytes Python's json.dumps(sort_keys=True,
// separators=(",", ":")) gives, so logs written by the service and by this
// driver verify with either.  Appends take an exclusive lock on the file
// (flock), so concurrent writers keep the chain linear.  Tampering with a
// record breaks its log_hash; removing one breaks the next prev_hash.
#pragma once
#include <fcntl.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/file.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <charconv>
#include <string>
#include <utility>
#include <vector>

#include "cis2_json.hpp"
#include "cis2_sha256.hpp"

namespace cis2 {

constexpr const char* kGenesisHash =
    "0000000000000000000000000000000000000000000000000000000000000000";

inline std::string hex_of(const uint8_t* d, size_t n) {
  static const char* k = "0123456789abcdef";
  std::string s;
  for (size_t i = 0; i < n; ++i) {
    s.push_back(k[d[i] >> 4]);
    s.push_back(k[d[i] & 15]);
  }
  return s;
}

// ---- canonical serialization -------------------------------------------------

// A JSON string literal with every character outside printable ASCII
// (0x20..0x7e) escaped, as json.dumps(ensure_ascii=True) writes it (UTF-8
// decoded to code points, astral ones as surrogate pairs).
inline std::string quoted_ascii(const std::string& s) {
  std::string o = "\"";
  char buf[16];
  auto u = [&](uint32_t cp) {
    snprintf(buf, sizeof buf, "\\u%04x", cp);
    o += buf;
  };
  for (size_t i = 0; i < s.size();) {
    const unsigned char c = (unsigned char)s[i];
    uint32_t cp = c;
    size_t len = 1;
    if (c >= 0xF0 && i + 3 < s.size()) {
      cp = ((c & 7u) << 18) | ((s[i + 1] & 0x3Fu) << 12) | ((s[i + 2] & 0x3Fu) << 6) | (s[i + 3] & 0x3Fu);
      len = 4;
    } else if (c >= 0xE0 && i + 2 < s.size()) {
      cp = ((c & 15u) << 12) | ((s[i + 1] & 0x3Fu) << 6) | (s[i + 2] & 0x3Fu);
      len = 3;
    } else if (c >= 0xC0 && i + 1 < s.size()) {
      cp = ((c & 31u) << 6) | (s[i + 1] & 0x3Fu);
      len = 2;
    }
    i += len;
    switch (cp) {
      case '"': o += "\\\""; continue;
      case '\\': o += "\\\\"; continue;
      case '\n': o += "\\n"; continue;
      case '\r': o += "\\r"; continue;
      case '\t': o += "\\t"; continue;
      case '\b': o += "\\b"; continue;
      case '\f': o += "\\f"; continue;
      default: break;
    }
    if (cp < 0x20 || (cp >= 0x7F && cp < 0x10000)) {
      u(cp);
    } else if (cp >= 0x10000) {
      u(0xD800 + ((cp - 0x10000) >> 10));
      u(0xDC00 + ((cp - 0x10000) & 0x3FF));
    } else {
      o.push_back((char)cp);
    }
  }
  return o + "\"";
}

// Shortest round-trip decimal of a double, laid out as Python's float repr
// (fixed notation for decimal exponents -4 < e <= 16, else d.ddde+XX).
// The digits are the shortest string that reads back as x and, among those,
// the one nearest x (std::to_chars): at 2^-24 that is 5.960464477539063e-08,
// which is not the correctly rounded 16-digit value (...062e-08 does not
// read back: below a power of two the neighbouring doubles are closer).
inline std::string float_repr(double x) {
  if (std::isnan(x)) return "NaN";
  if (std::isinf(x)) return x > 0 ? "Infinity" : "-Infinity";
  char b[64];
  const auto r = std::to_chars(b, b + sizeof b - 1, x, std::chars_format::scientific);
  *r.ptr = '\0';
  // b = [-]d.ddde[+-]XX: split the digits and the exponent
  std::string t(b);
  const bool neg = t[0] == '-';
  if (neg) t.erase(0, 1);
  const size_t e = t.find('e');
  std::string digits = t.substr(0, e);
  digits.erase(std::remove(digits.begin(), digits.end(), '.'), digits.end());
  while (digits.size() > 1 && digits.back() == '0') digits.pop_back();
  const int exp10 = atoi(t.c_str() + e + 1);
  const int decpt = exp10 + 1;  // value = 0.digits x 10^decpt
  const int n = (int)digits.size();
  std::string o = neg ? "-" : "";
  if (decpt > -4 && decpt <= 16) {
    if (decpt <= 0) {
      o += "0." + std::string((size_t)-decpt, '0') + digits;
    } else if (decpt >= n) {
      o += digits + std::string((size_t)(decpt - n), '0') + ".0";
    } else {
      o += digits.substr(0, (size_t)decpt) + "." + digits.substr((size_t)decpt);
    }
  } else {
    o += digits.substr(0, 1);
    if (n > 1) o += "." + digits.substr(1);
    snprintf(b, sizeof b, "e%c%02d", exp10 < 0 ? '-' : '+', exp10 < 0 ? -exp10 : exp10);
    o += b;
  }
  return o;
}

// A JSON number as Python re-serializes it: an integer lexeme keeps its
// digits (-0 becomes 0), anything with a fraction or exponent is a float.
inline std::string number_repr(const JsonNode& n) {
  const std::string& t = n.text;
  if (t.find_first_of(".eE") == std::string::npos) return t == "-0" ? "0" : t;
  return float_repr(n.number);
}

// Canonical (sep_item, sep_key = "," ":") or display (", " ": ") form of a
// node; object members sorted by key (UTF-8 byte order = code-point order).
inline std::string serialize(const JsonDoc& d, const JsonNode& n, const char* item_sep,
                             const char* key_sep, const char* skip_key = nullptr) {
  switch (n.type) {
    case JsonNode::Null: return "null";
    case JsonNode::Bool: return n.flag ? "true" : "false";
    case JsonNode::Number: return number_repr(n);
    case JsonNode::String: return quoted_ascii(n.text);
    case JsonNode::Array: {
      std::string o = "[";
      bool first = true;
      for (const JsonNode* c : d.children(n)) {
        if (!first) o += item_sep;
        first = false;
        o += serialize(d, *c, item_sep, key_sep);
      }
      return o + "]";
    }
    case JsonNode::Object: {
      std::vector<const JsonNode*> m = d.children(n);
      std::sort(m.begin(), m.end(), [](const JsonNode* a, const JsonNode* b) { return a->key < b->key; });
      std::string o = "{";
      bool first = true;
      for (const JsonNode* c : m) {
        if (skip_key && c->key == skip_key) continue;
        if (!first) o += item_sep;
        first = false;
        o += quoted_ascii(c->key) + key_sep + serialize(d, *c, item_sep, key_sep);
      }
      return o + "}";
    }
  }
  return "null";
}

inline std::string sha256_hex(const std::string& s) {
  uint8_t h[32];
  sha256(s.data(), s.size(), h);
  return hex_of(h, 32);
}

// ---- the log -----------------------------------------------------------------

struct ChainResult {
  bool ok;
  std::string message;
  std::string last_hash;  // log_hash of the last record checked (genesis when none)
  size_t records;
};

// Recomputes the chain over the file's JSON lines (blank lines skipped); with
// upto_id, stops after the record whose receipt_id equals it.  Messages are
// the service verifier's (code/cis2-llm/server/app/receipts.py:75-97).
inline ChainResult verify_chain_text(const std::string& text, const std::string* upto_id = nullptr) {
  size_t i = 0, pos = 0;
  std::string prev = kGenesisHash;
  while (pos <= text.size()) {
    size_t nl = text.find('\n', pos);
    if (nl == std::string::npos) nl = text.size();
    std::string line = text.substr(pos, nl - pos);
    pos = nl + 1;
    const size_t b = line.find_first_not_of(" \t\r");
    if (b == std::string::npos) {
      if (nl == text.size()) break;
      continue;
    }
    struct Thrower {
      static void on(const std::string& m) { throw m; }
    };
    JsonDoc d;
    try {
      d = JsonDoc::parse(line.data(), line.size(), Thrower::on);
    } catch (const std::string& m) {
      return ChainResult{false, "line " + std::to_string(i) + ": not a JSON record (" + m + ")",
                         prev, i};
    }
    const JsonNode& rec = d.root();
    const JsonNode* lh = d.member(rec, "log_hash");
    const JsonNode* ph = d.member(rec, "prev_hash");
    const std::string recomputed = sha256_hex(serialize(d, rec, ",", ":", "log_hash"));
    if (rec.type != JsonNode::Object || !ph || ph->type != JsonNode::String || ph->text != prev)
      return ChainResult{false, "line " + std::to_string(i) + ": prev_hash mismatch", prev, i};
    if (!lh || lh->type != JsonNode::String || lh->text != recomputed)
      return ChainResult{false, "line " + std::to_string(i) + ": log_hash mismatch (tampered record)",
                         prev, i};
    prev = lh->text;
    ++i;
    if (upto_id) {
      const JsonNode* id = d.member(rec, "receipt_id");
      if (id && id->type == JsonNode::String && id->text == *upto_id)
        return ChainResult{true, "chain OK through line " + std::to_string(i - 1), prev, i};
    }
    if (nl == text.size()) break;
  }
  if (upto_id) return ChainResult{false, "receipt_id " + *upto_id + " not found", prev, i};
  return ChainResult{true, i ? "chain OK" : "empty log", prev, i};
}

// One field of a new record: its name and its value as JSON text.
using ReceiptField = std::pair<std::string, std::string>;

inline std::string json_string(const std::string& s) { return quoted_ascii(s); }
inline std::string json_u32_list(const std::vector<uint32_t>& v) {
  std::string o = "[";
  for (size_t i = 0; i < v.size(); ++i) o += (i ? "," : "") + std::to_string(v[i]);
  return o + "]";
}

// 32 hex digits of a random version-4 UUID (uuid.uuid4().hex).
inline std::string new_receipt_id() {
  uint8_t b[16] = {0};
  FILE* f = fopen("/dev/urandom", "rb");
  const bool got = f && fread(b, 1, 16, f) == 16;
  if (f) fclose(f);
  if (!got) {  // no random device: time and address, still unique per process
    const uint64_t t = (uint64_t)time(nullptr) ^ ((uint64_t)(uintptr_t)&b << 20);
    memcpy(b, &t, 8);
  }
  b[6] = (uint8_t)((b[6] & 0x0F) | 0x40);
  b[8] = (uint8_t)((b[8] & 0x3F) | 0x80);
  return hex_of(b, 16);
}

inline std::string utc_now_iso() {
  char b[32];
  const time_t t = time(nullptr);
  struct tm g;
  gmtime_r(&t, &g);
  strftime(b, sizeof b, "%Y-%m-%dT%H:%M:%SZ", &g);
  return b;
}

// Appends a record made of `fields` (none named prev_hash or log_hash) to
// the log at path under an exclusive lock, after checking the existing
// chain; returns (false, reason) when the log is broken or unwritable, else
// (true, the new record's log_hash).
inline std::pair<bool, std::string> append_receipt(const std::string& path,
                                                   std::vector<ReceiptField> fields) {
  const int fd = open(path.c_str(), O_RDWR | O_CREAT | O_APPEND, 0644);
  if (fd < 0) return {false, "cannot open " + path};
  if (flock(fd, LOCK_EX) != 0) {
    close(fd);
    return {false, "cannot lock " + path};
  }
  std::string text;
  {
    char buf[1 << 16];
    ssize_t n;
    lseek(fd, 0, SEEK_SET);
    while ((n = read(fd, buf, sizeof buf)) > 0) text.append(buf, (size_t)n);
  }
  const ChainResult c = verify_chain_text(text);
  if (!c.ok) {
    close(fd);
    return {false, "existing log is broken: " + c.message};
  }
  fields.emplace_back("prev_hash", json_string(c.last_hash));
  std::sort(fields.begin(), fields.end());
  auto render = [&](const char* item_sep, const char* key_sep, const std::string* log_hash) {
    std::string o = "{";
    std::vector<ReceiptField> all = fields;
    if (log_hash) all.emplace_back("log_hash", json_string(*log_hash));
    std::sort(all.begin(), all.end());
    for (size_t i = 0; i < all.size(); ++i) {
      // values are re-serialized so that the record's text is canonical
      struct Thrower {
        static void on(const std::string& m) { throw m; }
      };
      const JsonDoc v = JsonDoc::parse(all[i].second.data(), all[i].second.size(), Thrower::on);
      o += (i ? item_sep : "") + quoted_ascii(all[i].first) + key_sep +
           serialize(v, v.root(), item_sep, key_sep);
    }
    return o + "}";
  };
  std::string line, log_hash;
  try {
    log_hash = sha256_hex(render(",", ":", nullptr));
    line = render(", ", ": ", &log_hash) + "\n";
  } catch (const std::string& m) {
    close(fd);
    return {false, "bad field value: " + m};
  }
  if (!text.empty() && text.back() != '\n') line = "\n" + line;
  const ssize_t w = write(fd, line.data(), line.size());
  const bool ok = w == (ssize_t)line.size() && fsync(fd) == 0;
  close(fd);
  if (!ok) return {false, "short write to " + path};
  return {true, log_hash};
}

}  // namespace cis2
