// cis2_json.hpp — strict JSON (RFC 8259) for the two documents the driver
// reads: config.json and the safetensors header.
//
// Two stages.  A tokenizer turns bytes into tokens (punctuation, literals,
// numbers checked against the JSON number grammar, strings with every
// escape validated and decoded to UTF-8, surrogate pairs joined).  A
// table-free state machine with an explicit stack (no recursion, so no
// input can exhaust the C++ stack) appends the values to a flat node array;
// containers link their children by index.  Anything outside the grammar —
// a raw control character in a string, an unknown escape, a non-hex \u
// digit, a lone surrogate, a duplicate key, nesting deeper than kMaxDepth,
// bytes after the document — is an error.  Errors are reported through a
// caller-supplied handler that must not return (the driver prints a FATAL
// line and exits with status 2).
#pragma once
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <unordered_set>
#include <vector>

namespace cis2 {

struct JsonNode {
  enum Type : uint8_t { Null, Bool, Number, String, Array, Object };
  Type type = Null;
  bool flag = false;     // Bool
  double number = 0.0;   // Number: strtod of the lexeme (correctly rounded)
  std::string text;      // String: decoded UTF-8; Number: the lexeme as written
  std::string key;       // member name, when the parent is an Object
  int32_t first = -1;    // first child (Array, Object)
  int32_t next = -1;     // next sibling
  uint32_t count = 0;    // children (Array, Object)
};

class JsonDoc {
 public:
  static constexpr int kMaxDepth = 64;
  using OnError = void (*)(const std::string& msg);

  // Parses bytes [p, p + n); calls on_error (which must not return) on any
  // violation.  The root is node 0.
  static JsonDoc parse(const char* p, size_t n, OnError on_error) {
    JsonDoc d;
    Parser(p, n, on_error, d.nodes_).run();
    return d;
  }

  const JsonNode& at(int32_t i) const { return nodes_[(size_t)i]; }
  const JsonNode& root() const { return nodes_[0]; }
  // The member `key` of object node i, or nullptr (also when i is no object).
  const JsonNode* member(int32_t i, const char* key) const {
    const JsonNode& o = nodes_[(size_t)i];
    if (o.type != JsonNode::Object) return nullptr;
    for (int32_t c = o.first; c >= 0; c = nodes_[(size_t)c].next)
      if (nodes_[(size_t)c].key == key) return &nodes_[(size_t)c];
    return nullptr;
  }
  const JsonNode* member(const JsonNode& o, const char* key) const {
    return member(index_of(o), key);
  }
  int32_t index_of(const JsonNode& n) const { return (int32_t)(&n - nodes_.data()); }
  // Children of a container, in document order.
  std::vector<const JsonNode*> children(const JsonNode& o) const {
    std::vector<const JsonNode*> out;
    for (int32_t c = o.first; c >= 0; c = nodes_[(size_t)c].next) out.push_back(&nodes_[(size_t)c]);
    return out;
  }

 private:
  std::vector<JsonNode> nodes_;

  enum class Tok { BeginObject, EndObject, BeginArray, EndArray, Colon, Comma, Str, Num, True,
                   False, Null, Eof };

  class Parser {
   public:
    Parser(const char* p, size_t n, OnError err, std::vector<JsonNode>& out)
        : b_(p), p_(p), e_(p + n), err_(err), out_(out) {}

    void run() {
      State st = Value;
      std::string key;
      bool have_key = false;
      while (true) {
        if (st == Done) {
          skip_ws();
          if (p_ < e_) fail("bytes after the document");
          return;
        }
        const Tok t = lex();
        if (t == Tok::Eof) fail("unexpected end of input");
        switch (st) {
          case FirstKeyOrEnd:
            if (t == Tok::EndObject) { close(); st = after_close(); break; }
            [[fallthrough]];
          case Key:
            if (t != Tok::Str) fail("expected a member name");
            key = tok_text_;
            if (!stack_.back().keys.insert(key).second) fail("duplicate key \"" + key + "\"");
            have_key = true;
            st = ColonNext;
            break;
          case ColonNext:
            if (t != Tok::Colon) fail("expected ':'");
            st = Value;
            break;
          case CommaOrEnd:
            if (t == Tok::Comma) {
              st = stack_.back().object ? Key : Value;
            } else if (t == (stack_.back().object ? Tok::EndObject : Tok::EndArray)) {
              close();
              st = after_close();
            } else {
              fail(stack_.back().object ? "expected ',' or '}'" : "expected ',' or ']'");
            }
            break;
          case Value: {
            if (t == Tok::EndArray && !stack_.empty() && !stack_.back().object &&
                out_[(size_t)stack_.back().node].count == 0 && !have_key) {
              close();  // the empty array
              st = after_close();
              break;
            }
            const int32_t n = add(have_key ? &key : nullptr);
            have_key = false;
            JsonNode& v = out_[(size_t)n];
            switch (t) {
              case Tok::BeginObject:
              case Tok::BeginArray:
                v.type = t == Tok::BeginObject ? JsonNode::Object : JsonNode::Array;
                if ((int)stack_.size() >= kMaxDepth) fail("nesting deeper than 64 levels");
                stack_.push_back(Open{n, -1, t == Tok::BeginObject, {}});
                st = t == Tok::BeginObject ? FirstKeyOrEnd : Value;
                break;
              case Tok::Str: v.type = JsonNode::String; v.text = tok_text_; st = after_value(); break;
              case Tok::Num:
                v.type = JsonNode::Number;
                v.number = tok_num_;
                v.text = tok_text_;
                st = after_value();
                break;
              case Tok::True: v.type = JsonNode::Bool; v.flag = true; st = after_value(); break;
              case Tok::False: v.type = JsonNode::Bool; st = after_value(); break;
              case Tok::Null: st = after_value(); break;
              default: fail("expected a value");
            }
            break;
          }
          default: fail("parser state");
        }
      }
    }

   private:
    // what the next token may be
    enum State { Value, FirstKeyOrEnd, Key, ColonNext, CommaOrEnd, Done };
    struct Open {
      int32_t node, last;  // container node, its last child so far
      bool object;
      std::unordered_set<std::string> keys;
    };
    const char *b_, *p_, *e_;
    OnError err_;
    std::vector<JsonNode>& out_;
    std::vector<Open> stack_;
    std::string tok_text_;
    double tok_num_ = 0.0;

    [[noreturn]] void fail(const std::string& what) {
      err_("JSON: " + what + " at byte " + std::to_string(p_ - b_));
      abort();  // on_error does not return
    }
    // appends a value node under the open container (or as the root)
    int32_t add(const std::string* key) {
      const int32_t n = (int32_t)out_.size();
      out_.emplace_back();
      if (key) out_.back().key = *key;
      if (!stack_.empty()) {
        Open& o = stack_.back();
        JsonNode& parent = out_[(size_t)o.node];
        if (o.last < 0) parent.first = n;
        else out_[(size_t)o.last].next = n;
        o.last = n;
        ++parent.count;
      } else if (n != 0) {
        fail("a second document");
      }
      return n;
    }
    void close() { stack_.pop_back(); }
    State after_value() const { return stack_.empty() ? Done : CommaOrEnd; }
    State after_close() const { return after_value(); }

    void skip_ws() {
      while (p_ < e_ && (*p_ == ' ' || *p_ == '\t' || *p_ == '\n' || *p_ == '\r')) ++p_;
    }
    bool word(const char* w) {
      const size_t n = strlen(w);
      if ((size_t)(e_ - p_) < n || memcmp(p_, w, n) != 0) return false;
      p_ += n;
      return true;
    }
    Tok lex() {
      skip_ws();
      if (p_ >= e_) return Tok::Eof;
      switch (*p_) {
        case '{': ++p_; return Tok::BeginObject;
        case '}': ++p_; return Tok::EndObject;
        case '[': ++p_; return Tok::BeginArray;
        case ']': ++p_; return Tok::EndArray;
        case ':': ++p_; return Tok::Colon;
        case ',': ++p_; return Tok::Comma;
        case '"': lex_string(); return Tok::Str;
        default: break;
      }
      if (word("true")) return Tok::True;
      if (word("false")) return Tok::False;
      if (word("null")) return Tok::Null;
      if (*p_ == '-' || (*p_ >= '0' && *p_ <= '9')) {
        lex_number();
        return Tok::Num;
      }
      fail("unexpected character");
    }
    // -? (0 | [1-9][0-9]*) (. [0-9]+)? ([eE] [+-]? [0-9]+)?
    void lex_number() {
      const char* s = p_;
      auto digits = [&]() {
        const char* d = p_;
        while (p_ < e_ && *p_ >= '0' && *p_ <= '9') ++p_;
        return p_ - d;
      };
      if (*p_ == '-') ++p_;
      if (p_ < e_ && *p_ == '0') {
        ++p_;
      } else if (digits() == 0) {
        fail("malformed number");
      }
      if (p_ < e_ && *p_ == '.') {
        ++p_;
        if (digits() == 0) fail("malformed number");
      }
      if (p_ < e_ && (*p_ == 'e' || *p_ == 'E')) {
        ++p_;
        if (p_ < e_ && (*p_ == '+' || *p_ == '-')) ++p_;
        if (digits() == 0) fail("malformed number");
      }
      tok_text_.assign(s, p_);
      tok_num_ = strtod(tok_text_.c_str(), nullptr);
    }
    uint32_t hex4() {
      if (e_ - p_ < 4) fail("truncated \\u escape");
      uint32_t v = 0;
      for (int i = 0; i < 4; ++i) {
        const char c = *p_++;
        uint32_t d;
        if (c >= '0' && c <= '9') d = (uint32_t)(c - '0');
        else if (c >= 'a' && c <= 'f') d = (uint32_t)(c - 'a' + 10);
        else if (c >= 'A' && c <= 'F') d = (uint32_t)(c - 'A' + 10);
        else fail("non-hex digit in a \\u escape");
        v = v * 16 + d;
      }
      return v;
    }
    void put_utf8(uint32_t cp) {
      std::string& s = tok_text_;
      if (cp < 0x80) {
        s.push_back((char)cp);
      } else if (cp < 0x800) {
        s.push_back((char)(0xC0 | (cp >> 6)));
        s.push_back((char)(0x80 | (cp & 0x3F)));
      } else if (cp < 0x10000) {
        s.push_back((char)(0xE0 | (cp >> 12)));
        s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
        s.push_back((char)(0x80 | (cp & 0x3F)));
      } else {
        s.push_back((char)(0xF0 | (cp >> 18)));
        s.push_back((char)(0x80 | ((cp >> 12) & 0x3F)));
        s.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
        s.push_back((char)(0x80 | (cp & 0x3F)));
      }
    }
    void lex_string() {
      ++p_;  // opening quote
      tok_text_.clear();
      while (true) {
        if (p_ >= e_) fail("unterminated string");
        const unsigned char c = (unsigned char)*p_++;
        if (c == '"') return;
        if (c < 0x20) fail("control character in a string");
        if (c != '\\') {
          tok_text_.push_back((char)c);
          continue;
        }
        if (p_ >= e_) fail("unterminated string");
        const char x = *p_++;
        switch (x) {
          case '"': case '\\': case '/': tok_text_.push_back(x); break;
          case 'b': tok_text_.push_back('\b'); break;
          case 'f': tok_text_.push_back('\f'); break;
          case 'n': tok_text_.push_back('\n'); break;
          case 'r': tok_text_.push_back('\r'); break;
          case 't': tok_text_.push_back('\t'); break;
          case 'u': {
            uint32_t cp = hex4();
            if (cp >= 0xDC00 && cp <= 0xDFFF) fail("lone low surrogate");
            if (cp >= 0xD800 && cp <= 0xDBFF) {
              if (e_ - p_ < 2 || p_[0] != '\\' || p_[1] != 'u') fail("lone high surrogate");
              p_ += 2;
              const uint32_t lo = hex4();
              if (lo < 0xDC00 || lo > 0xDFFF) fail("lone high surrogate");
              cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
            }
            put_utf8(cp);
            break;
          }
          default: fail("unknown escape");
        }
      }
    }
  };
};

}  // namespace cis2
