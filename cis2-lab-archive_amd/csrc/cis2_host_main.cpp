// cis2_host_main.cpp — command-line driver over the gfx950 C ABI with the
// flags and stdout line protocol of the reference driver
// (code/cis2-fp/gpu/cis2_host.cpp:61-249; Rust src/main.rs:1231-1262), so
// the service runner's regexes (code/cis2-llm/server/app/runner.py:25-31)
// and digest/trace gates (code/cis2-fp/gpu/Makefile:160-184) apply as is.
//
//   cis2_host --weights-dir DIR --ids FILE [--gen-toks N] [--trace FILE]
//             [--prompt-idx I] [--reduction sequential|tree] [--sample SEED,T,K,P]
//             [--verify2] [--receipt-log FILE] [--layer-digests]
//   cis2_host --verify-chain FILE [--receipt-id ID]
//
// Debug surface of the reference CLI (code/cis2-fp/src/main.rs:315-335,
// 355-529, 1099-1212), none of it part of CIS2_REF: --layer-digests prints
// LAYER_DIGEST lines for the last prompt position; CIS2_DUMP_LAYERS (any
// value) prints CIS2_DUMP lines on stderr for the last prompt position and
// the first generated one; CIS2_DUMP_STEP0_LOGITS / CIS2_DUMP_LASTSTEP_LOGITS
// name files that receive the step-0 and the final step's fp32 logits.
#include "cis2_amd.h"
#include "cis2_checkpoint.hpp"
#include "cis2_receipts.hpp"
#include "cis2_sha256.hpp"

#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

using namespace cis2;

namespace {

std::string hex(const uint8_t* d, size_t n) {
  static const char* k = "0123456789abcdef";
  std::string s;
  for (size_t i = 0; i < n; ++i) {
    s.push_back(k[d[i] >> 4]);
    s.push_back(k[d[i] & 15]);
  }
  return s;
}

std::string ids_list(const std::vector<uint32_t>& v) {
  std::string s = "[";
  for (size_t i = 0; i < v.size(); ++i) {
    if (i) s += ", ";
    s += std::to_string(v[i]);
  }
  return s + "]";
}

struct TraceSink {
  FILE* fp = nullptr;
};

// The ops of one forward pass that the debug surface reports, as the
// reference's trace names them, with the digests a capture pass recorded.
struct Capture {
  uint32_t pos_lo = 0, pos_hi = 0;  // positions kept: [pos_lo, pos_hi]
  struct Line {
    int pos, layer;
    std::string op, sha;
  };
  std::vector<Line> lines;
};
void capture_cb(int pos, int layer, const char* op, const uint8_t sha[32], void* user) {
  Capture* c = static_cast<Capture*>(user);
  if (pos < (int)c->pos_lo || pos > (int)c->pos_hi) return;
  const std::string o = op;
  if (o == "embedding" || o == "resid1" || o == "resid2" || o == "final_norm" || o == "logits")
    c->lines.push_back({pos, layer, o, hex(sha, 32)});
}

// Raw little-endian fp32 values to a file (the reference's logit dumps).
void write_f32(const std::string& path, const std::vector<float>& v) {
  FILE* f = fopen(path.c_str(), "wb");
  if (!f || fwrite(v.data(), 4, v.size(), f) != v.size()) fatal("write " + path);
  fclose(f);
}
void trace_cb(int pos, int layer, const char* op, const uint8_t sha[32], void* user) {
  TraceSink* t = static_cast<TraceSink*>(user);
  fprintf(t->fp, "pos=%d layer=%d op=%s sha256=%s\n", pos, layer, op, hex(sha, 32).c_str());
}

// A config.json dimension: a whole number that fits 32 bits.
uint32_t dim_key(const JsonDoc& cfg, const char* k) {
  uint64_t v = 0;
  const JsonNode* n = cfg.member(cfg.root(), k);
  if (!n) fatal(std::string("config.json missing ") + k);
  if (!config_u64(n, &v) || v > 0xFFFFFFFFull)
    fatal(std::string("config.json ") + k + " is not a 32-bit whole number");
  return (uint32_t)v;
}

// "SEED,T,K,P": seed u64 (decimal or 0x hex), T and P by strtof (correctly
// rounded decimal to f32, draft 14.1), K u32.  False when malformed or out
// of range.
bool parse_sample(const char* txt, cis2_sampling* out) {
  std::string t(txt);
  std::vector<std::string> f;
  size_t b = 0;
  for (size_t e; (e = t.find(',', b)) != std::string::npos; b = e + 1) f.push_back(t.substr(b, e - b));
  f.push_back(t.substr(b));
  if (f.size() != 4) return false;
  for (const std::string& x : f)
    if (x.empty()) return false;
  char* end = nullptr;
  errno = 0;
  const unsigned long long seed = strtoull(f[0].c_str(), &end, 0);
  if (*end || errno || f[0][0] == '-') return false;
  const float T = strtof(f[1].c_str(), &end);
  if (*end) return false;
  errno = 0;
  const unsigned long k = strtoul(f[2].c_str(), &end, 10);
  if (*end || errno || k > 0xFFFFFFFFul || f[2][0] == '-') return false;
  const float P = strtof(f[3].c_str(), &end);
  if (*end) return false;
  if (!(T > 0.0f) || T == HUGE_VALF || !(P > 0.0f) || !(P <= 1.0f)) return false;
  out->mode = 1;
  out->seed = seed;
  out->temperature = T;
  out->top_k = (uint32_t)k;
  out->top_p = P;
  return true;
}

// Command-line settings with the reference driver's defaults
// (code/cis2-fp/gpu/cis2_host.cpp:61-85).
struct Options {
  std::string weights_dir = "weights", ids_path, trace_path;
  int gen_toks = 16, prompt_idx = 0;
  uint32_t reduction = 0;  // --reduction sequential|tree (code/cis2-fp/src/main.rs:775-782)
  // --sample SEED,T,K,P: seeded sampling (v0.4 draft section 14; the lab
  // driver's flag, labs/w1x-sample/feed/cm-hq__cis2-sample-hq-r2/job.sh:22-28)
  cis2_sampling samp{};
  // cis2-verify2 line protocol (code/cis2-fp/verify2/src/main.rs:353-500, parsed
  // by code/cis2-llm/server/app/runner.py:25-31): --verify2, or this binary
  // invoked under the name cis2-verify2
  bool verify2 = false;
  // hash-chained receipt log (code/cis2-llm/server/app/receipts.py:31-97):
  // --receipt-log FILE appends this run's receipt; --verify-chain FILE
  // [--receipt-id ID] checks a log (through ID) and exits 0 / 1
  std::string receipt_log, verify_chain, receipt_id;
  // --layer-digests (code/cis2-fp/src/main.rs:743-751): LAYER_DIGEST lines of
  // the last prompt position's forward pass
  bool layer_digests = false;
};

bool whole_int(const char* t, int* out) {
  char* end = nullptr;
  errno = 0;
  const long v = strtol(t, &end, 10);
  if (!*t || *end || errno || v < INT32_MIN || v > INT32_MAX) return false;
  *out = (int)v;
  return true;
}

// Flags as a table: name, whether a value follows, and what the value sets.
// Returns an error message, or "" when the command line is accepted.
std::string parse_options(int argc, char** argv, Options& o) {
  const std::string self = argv[0];
  o.verify2 = self.substr(self.rfind('/') == std::string::npos ? 0 : self.rfind('/') + 1) ==
              "cis2-verify2";
  struct Flag {
    const char* name;
    bool value;
    std::string (*apply)(Options&, const char*);
  };
  static const Flag flags[] = {
      {"--weights-dir", true, [](Options& o, const char* v) { o.weights_dir = v; return std::string(); }},
      {"--ids", true, [](Options& o, const char* v) { o.ids_path = v; return std::string(); }},
      {"--trace", true, [](Options& o, const char* v) { o.trace_path = v; return std::string(); }},
      {"--gen-toks", true, [](Options& o, const char* v) {
         return whole_int(v, &o.gen_toks) ? std::string() : "--gen-toks: not an integer: " + std::string(v);
       }},
      {"--prompt-idx", true, [](Options& o, const char* v) {
         return whole_int(v, &o.prompt_idx) ? std::string() : "--prompt-idx: not an integer: " + std::string(v);
       }},
      {"--reduction", true, [](Options& o, const char* v) {
         const std::string r = v;
         if (r != "sequential" && r != "tree")
           return "--reduction: expected 'sequential' or 'tree', got " + r;
         o.reduction = r == "tree" ? 1u : 0u;
         return std::string();
       }},
      {"--sample", true, [](Options& o, const char* v) {
         return parse_sample(v, &o.samp)
                    ? std::string()
                    : "--sample: expected SEED,T,K,P with T finite > 0 and P in (0,1], got " +
                          std::string(v);
       }},
      {"--verify2", false, [](Options& o, const char*) { o.verify2 = true; return std::string(); }},
      {"--layer-digests", false, [](Options& o, const char*) { o.layer_digests = true; return std::string(); }},
      {"--receipt-log", true, [](Options& o, const char* v) { o.receipt_log = v; return std::string(); }},
      {"--verify-chain", true, [](Options& o, const char* v) { o.verify_chain = v; return std::string(); }},
      {"--receipt-id", true, [](Options& o, const char* v) { o.receipt_id = v; return std::string(); }},
  };
  for (int i = 1; i < argc; ++i) {
    const Flag* f = nullptr;
    for (const Flag& c : flags)
      if (!strcmp(argv[i], c.name)) f = &c;
    if (!f || (f->value && i + 1 >= argc)) return std::string("unknown CLI argument: ") + argv[i];
    const std::string err = f->apply(o, f->value ? argv[++i] : nullptr);
    if (!err.empty()) return err;
  }
  return "";
}

}  // namespace

int main(int argc, char** argv) {
  Options opt;
  if (const std::string err = parse_options(argc, argv, opt); !err.empty()) {
    fprintf(stderr, "FATAL: %s\n", err.c_str());
    return 2;
  }
  if (!opt.verify_chain.empty()) {  // no model, no device: check the log and exit
    FILE* f = fopen(opt.verify_chain.c_str(), "rb");
    if (!f) fatal("cannot open " + opt.verify_chain);
    fclose(f);
    const std::string text = slurp(opt.verify_chain);
    const ChainResult r =
        verify_chain_text(text, opt.receipt_id.empty() ? nullptr : &opt.receipt_id);
    printf("CIS2_CHAIN %s records=%zu head=%s message=%s\n", r.ok ? "PASS" : "FAIL", r.records,
           r.last_hash.c_str(), r.message.c_str());
    return r.ok ? 0 : 1;
  }
  const std::string& ids_path = opt.ids_path;
  const std::string& trace_path = opt.trace_path;
  const int gen_toks = opt.gen_toks, prompt_idx = opt.prompt_idx;
  const uint32_t reduction = opt.reduction;
  const cis2_sampling& samp = opt.samp;
  const bool verify2 = opt.verify2;
  if (ids_path.empty() && !verify2) fatal("--ids FILE is required");
  if (gen_toks < 0) fatal("--gen-toks must be >= 0");
  const std::string wpath = opt.weights_dir + "/model.safetensors";
  const std::string tpath = opt.weights_dir + "/tokenizer.json";
  const std::string cpath = opt.weights_dir + "/config.json";
  const JsonDoc cfgj = parse_json_text(slurp(cpath));
  // scope gate on config.json alone, before any weights are opened or hashed
  // (code/cis2-fp/src/main.rs:817-823)
  const std::string reason = gate_architecture(cfgj);
  if (!reason.empty()) {
    fprintf(stderr, "CIS2_REF_UNSUPPORTED reason=%s\n", reason.c_str());
    fprintf(stderr, "This checkpoint is outside the CIS-2 specified subset; no digest emitted.\n");
    return 2;
  }
  uint8_t hdr[96];
  hash_file(wpath, hdr);
  hash_file(tpath, hdr + 32);
  hash_file(cpath, hdr + 64);

  cis2_config cfg;
  memset(&cfg, 0, sizeof cfg);
  cfg.hidden = dim_key(cfgj, "hidden_size");
  cfg.inter = dim_key(cfgj, "intermediate_size");
  cfg.n_layers = dim_key(cfgj, "num_hidden_layers");
  cfg.n_heads = dim_key(cfgj, "num_attention_heads");
  cfg.n_kv_heads = dim_key(cfgj, "num_key_value_heads");
  cfg.vocab = dim_key(cfgj, "vocab_size");
  const JsonNode* eps = cfgj.member(cfgj.root(), "rms_norm_eps");
  const JsonNode* theta = cfgj.member(cfgj.root(), "rope_theta");
  if (!eps || eps->type != JsonNode::Number) fatal("config.json missing rms_norm_eps");
  if (!theta || theta->type != JsonNode::Number) fatal("config.json missing rope_theta");
  cfg.eps = (float)eps->number;  // one narrowing, as `as f32` does
  cfg.rope_theta = theta->number;
  if (cfg.n_heads == 0) fatal("num_attention_heads must be > 0");
  // head_dim: hidden / heads, as the reference derives it
  // (code/cis2-fp/gpu/cis2_host.cpp:114); an explicit value only for qwen3
  // (labs/w1x-qwen3/scripts/qwen3-port.diff:104-110; the gate refuses any
  // other explicit value that differs), absent or null = derived
  cfg.head_dim = cfg.hidden / cfg.n_heads;
  {
    const JsonNode* mt = cfgj.member(cfgj.root(), "model_type");
    uint64_t hd = 0;
    if (mt && mt->type == JsonNode::String && mt->text == "qwen3" &&
        config_u64(cfgj.member(cfgj.root(), "head_dim"), &hd)) {
      if (hd == 0 || hd > 0xFFFFFFFFull) fatal("config.json head_dim out of range");
      cfg.head_dim = (uint32_t)hd;
    }
  }
  cfg.tied = 1;
  if (const JsonNode* t = cfgj.member(cfgj.root(), "tie_word_embeddings"))
    cfg.tied = (t->type == JsonNode::Bool) ? (t->flag ? 1 : 0) : 1;
  // verify2 without --ids: the section 13.1 prompt, "Once upon a time" under
  // the SmolLM2 tokenizer (verify2/src/main.rs:436-444)
  std::vector<uint32_t> prompt =
      ids_path.empty() ? std::vector<uint32_t>{6403, 1980, 253, 655} : read_ids(ids_path);
  cfg.max_pos = (uint32_t)(prompt.size() + gen_toks);
  cfg.max_seqs = 1;
  cfg.reduction_mode = reduction;

  // The header and every tensor's dtype and shape are checked before the
  // device is touched, so a bad file fails fast and identically everywhere;
  // the payloads are then read and uploaded one tensor at a time.
  Checkpoint ck;
  ck.open(wpath);
  const uint64_t H = cfg.hidden, I = cfg.inter, V = cfg.vocab;
  const uint64_t QD = (uint64_t)cfg.n_heads * cfg.head_dim,
                 KV = (uint64_t)cfg.n_kv_heads * cfg.head_dim, HD = cfg.head_dim;
  std::vector<const Checkpoint::Tensor*> plan;
  auto need = [&](const std::string& name, std::vector<uint64_t> shape, bool optional) {
    const Checkpoint::Tensor* t = ck.find(name);
    if (!t) {
      if (optional) return;
      fatal("tensor " + name + " missing");
    }
    ck.require_bf16(*t, shape);
    plan.push_back(t);
  };
  need("model.embed_tokens.weight", {V, H}, false);
  for (uint32_t l = 0; l < cfg.n_layers; ++l) {
    std::string p = "model.layers." + std::to_string(l) + ".";
    need(p + "input_layernorm.weight", {H}, false);
    need(p + "post_attention_layernorm.weight", {H}, false);
    need(p + "self_attn.q_proj.weight", {QD, H}, false);
    need(p + "self_attn.k_proj.weight", {KV, H}, false);
    need(p + "self_attn.v_proj.weight", {KV, H}, false);
    need(p + "self_attn.o_proj.weight", {H, QD}, false);
    need(p + "mlp.gate_proj.weight", {I, H}, false);
    need(p + "mlp.up_proj.weight", {I, H}, false);
    need(p + "mlp.down_proj.weight", {H, I}, false);
    need(p + "self_attn.q_proj.bias", {QD}, true);
    need(p + "self_attn.k_proj.bias", {KV}, true);
    need(p + "self_attn.v_proj.bias", {KV}, true);
    need(p + "self_attn.q_norm.weight", {HD}, true);
    need(p + "self_attn.k_norm.weight", {HD}, true);
  }
  need("model.norm.weight", {H}, false);
  if (!cfg.tied) need("lm_head.weight", {V, H}, false);

  cis2_ctx* ctx = nullptr;
  int rc = cis2_ctx_create(&cfg, &ctx);
  if (rc) fatal(std::string("cis2_ctx_create: ") + cis2_strerror(rc));
  if (samp.mode) {
    rc = cis2_set_sampling(ctx, &samp);
    if (rc) fatal(std::string("--sample: ") + cis2_last_error(ctx));
  }
  fprintf(stderr, "cis2_host: %zu tensors, read one at a time and widened on the device\n",
          plan.size());
  {
    std::vector<uint16_t> buf;  // one tensor's payload at a time
    for (const Checkpoint::Tensor* t : plan) {
      ck.read_bf16(*t, buf);
      rc = cis2_upload_bf16(ctx, t->name.c_str(), buf.data(), t->elements);
      if (rc) fatal("upload " + t->name + ": " + cis2_last_error(ctx));
    }
  }
  ck.close();
  rc = cis2_check_ready(ctx);
  if (rc) fatal(cis2_last_error(ctx));
  fprintf(stderr, "[prompt %d] token ids (%zu toks): %s\n", prompt_idx, prompt.size(),
          ids_list(prompt).c_str());

  // Debug capture (the reference's --layer-digests and CIS2_DUMP_LAYERS):
  // one traced pass of the prompt (and the first generated step for the
  // dump), before the decode; the per-op path it runs gives the decode's
  // bits.  Its digests are printed where the reference prints them: the
  // LAYER_DIGEST lines before any other stdout line, the CIS2_DUMP lines on
  // stderr.
  const bool dump_layers = getenv("CIS2_DUMP_LAYERS") != nullptr && !verify2;
  Capture cap;
  if ((opt.layer_digests || dump_layers) && !verify2) {
    const uint32_t last = (uint32_t)prompt.size() - 1;
    const uint32_t extra = dump_layers && gen_toks > 0 ? 1u : 0u;
    cap.pos_lo = last;
    cap.pos_hi = last + extra;
    cis2_trace_enable(ctx, capture_cb, &cap);
    std::vector<uint32_t> cids(prompt.size() + extra);
    uint8_t cw[32], ca[32];
    rc = cis2_decode(ctx, 0, prompt.data(), (uint32_t)prompt.size(), extra, hdr, cids.data(), cw,
                     ca, nullptr);
    cis2_trace_enable(ctx, nullptr, nullptr);
    if (rc) fatal(std::string("debug capture: ") + cis2_last_error(ctx));
    if (opt.layer_digests)
      for (const Capture::Line& l : cap.lines) {
        if (l.pos != (int)last) continue;
        if (l.op == "embedding") printf("LAYER_DIGEST embed %s\n", l.sha.c_str());
        else if (l.op == "resid2") printf("LAYER_DIGEST block_%d %s\n", l.layer, l.sha.c_str());
        else if (l.op == "final_norm") printf("LAYER_DIGEST final_norm %s\n", l.sha.c_str());
        else if (l.op == "logits") printf("LAYER_DIGEST logits %s\n", l.sha.c_str());
      }
    if (dump_layers)
      for (const Capture::Line& l : cap.lines) {
        std::string layer, field;
        if (l.op == "embedding") layer = "embed", field = "token_embedding";
        else if (l.op == "resid1") layer = "block" + std::to_string(l.layer), field = "post_attention_hidden";
        else if (l.op == "resid2") layer = "block" + std::to_string(l.layer), field = "post_mlp_hidden";
        else if (l.op == "final_norm") layer = "final_norm", field = "final_norm_output";
        else layer = "logits", field = "pre_argmax_logits";
        fprintf(stderr, "CIS2_DUMP layer=%s field=%s pos=%d digest=%s\n", layer.c_str(),
                field.c_str(), l.pos, l.sha.c_str());
      }
    fflush(stdout);
  }

  TraceSink sink;
  if (!trace_path.empty()) {
    sink.fp = fopen(trace_path.c_str(), "wb");
    if (!sink.fp) fatal("cannot write " + trace_path);
    cis2_trace_enable(ctx, trace_cb, &sink);
  }
  std::vector<uint32_t> ids(prompt.size() + gen_toks);
  uint8_t wit[32], adig[32];
  rc = cis2_decode(ctx, 0, prompt.data(), (uint32_t)prompt.size(), (uint32_t)gen_toks, hdr,
                   ids.data(), wit, adig, nullptr);
  if (rc) fatal(std::string("decode: ") + cis2_last_error(ctx));
  if (sink.fp) fclose(sink.fp);
  cis2_trace_enable(ctx, nullptr, nullptr);
  // the reference's logit dumps (main.rs:1145-1160, 1197-1212): step 0's
  // logits (the last prompt position's forward pass) and the final step's
  // (the forward pass of the last generated id); each pass is recomputed
  // from the decode's K/V cache with the same bits and rewrites its own
  // position only
  auto dump_logits = [&](const char* env, uint32_t pos, uint32_t tok, const char* what) {
    const char* path = getenv(env);
    if (!path || verify2) return;
    std::vector<float> lg(cfg.vocab);
    uint32_t seq = 0, am = 0;
    rc = cis2_forward(ctx, 1, &seq, &pos, &tok, lg.data(), &am);
    if (rc) fatal(std::string(env) + ": " + cis2_last_error(ctx));
    write_f32(path, lg);
    fprintf(stderr, "[debug] wrote %s logits (%zu f32 values) to %s\n", what, lg.size(), path);
  };
  dump_logits("CIS2_DUMP_STEP0_LOGITS", (uint32_t)prompt.size() - 1, prompt.back(), "step-0");
  dump_logits("CIS2_DUMP_LASTSTEP_LOGITS", (uint32_t)prompt.size() + gen_toks - 1,
              ids[prompt.size() + gen_toks - 1], "final-step");
  if (verify2) {
    // section 12.4: the whole decode twice in one process, identical results
    // (verify2/src/main.rs:446-477), then the verifier's five lines
    std::vector<uint32_t> ids2(ids.size());
    uint8_t wit2[32], adig2[32];
    rc = cis2_decode(ctx, 0, prompt.data(), (uint32_t)prompt.size(), (uint32_t)gen_toks, hdr,
                     ids2.data(), wit2, adig2, nullptr);
    if (rc) fatal(std::string("decode: ") + cis2_last_error(ctx));
    if (memcmp(wit, wit2, 32)) fatal("section 12.4: witness digest differs across same-process runs");
    if (memcmp(adig, adig2, 32)) fatal("section 12.4: argmax digest differs across same-process runs");
    if (ids != ids2) fatal("section 12.4: generated token ids differ across same-process runs");
    uint8_t table[32], invf[32];
    cis2_digests(ctx, table, invf);
    printf("CIS2_VERIFY2 digest=%s prompt_toks=%zu gen_toks=%d dtype=fp32\n", hex(wit, 32).c_str(),
           prompt.size(), gen_toks);
    printf("argmax_digest=%s\n", hex(adig, 32).c_str());
    printf("table_digest=%s\n", hex(table, 32).c_str());
    printf("inv_freq table_digest=%s\n", hex(invf, 32).c_str());
    std::vector<uint32_t> gen(ids.begin() + prompt.size(), ids.end());
    printf("generated_token_ids=%s\n", ids_list(gen).c_str());
    cis2_ctx_destroy(ctx);
    return 0;
  }
  if (!opt.receipt_log.empty()) {
    uint8_t table[32], invf[32];
    cis2_digests(ctx, table, invf);
    const JsonNode* mt = cfgj.member(cfgj.root(), "model_type");
    std::vector<uint32_t> gen(ids.begin() + (long)prompt.size(), ids.end());
    std::vector<ReceiptField> f = {
        {"receipt_id", json_string(new_receipt_id())},
        {"created", json_string(utc_now_iso())},
        {"model", json_string("cis2-" + (mt && mt->type == JsonNode::String ? mt->text : "llama") +
                              "-fp32")},
        {"cis2_version", json_string(reduction ? "v0.4-candidate-tree" : "v0.3b")},
        {"reduction_mode", json_string(reduction ? "tree" : "sequential")},
        {"backend", json_string("gfx950")},
        {"witness_digest", json_string(hex(wit, 32))},
        {"argmax_digest", json_string(hex(adig, 32))},
        {"table_digest", json_string(hex(table, 32))},
        {"inv_freq_table_digest", json_string(hex(invf, 32))},
        {"weights_sha256", json_string(hex(hdr, 32))},
        {"tokenizer_sha256", json_string(hex(hdr + 32, 32))},
        {"config_sha256", json_string(hex(hdr + 64, 32))},
        {"prompt_idx", std::to_string(prompt_idx)},
        {"prompt_token_ids", json_u32_list(prompt)},
        {"generated_token_ids", json_u32_list(gen)},
    };
    if (samp.mode) {
      uint32_t tb, pb;
      memcpy(&tb, &samp.temperature, 4);
      memcpy(&pb, &samp.top_p, 4);
      char sb[160];
      snprintf(sb, sizeof sb,
               "{\"seed\":%llu,\"temperature_bits\":%u,\"top_k\":%u,\"top_p_bits\":%u}",
               (unsigned long long)samp.seed, tb, samp.top_k, pb);
      f.emplace_back("sampling", sb);
    }
    const auto ar = append_receipt(opt.receipt_log, f);
    if (!ar.first) fatal("--receipt-log: " + ar.second);
    fprintf(stderr, "receipt appended to %s: log_hash=%s\n", opt.receipt_log.c_str(),
            ar.second.c_str());
  }
  for (int s = 0; s < gen_toks; ++s)
    fprintf(stderr, "[run1] step %d: token_id=%u\n", s, ids[prompt.size() + s]);
  if (samp.mode)  // the sampled ids, one line per step (what the lab's ids16 hash reads)
    for (int s = 0; s < gen_toks; ++s) printf("step %d next_id=%u\n", s, ids[prompt.size() + s]);

  uint8_t table[32], invf[32];
  cis2_digests(ctx, table, invf);
  printf("weights_sha256=%s\n", hex(hdr, 32).c_str());
  printf("tokenizer_sha256=%s\n", hex(hdr + 32, 32).c_str());
  printf("config_sha256=%s\n", hex(hdr + 64, 32).c_str());
  printf("table_digest=%s\n", hex(table, 32).c_str());
  printf("inv_freq_table_digest=%s\n", hex(invf, 32).c_str());
  printf("prompt_idx=%d prompt_tokens=%s\n", prompt_idx, ids_list(prompt).c_str());
  printf("prompt_idx=%d run1_tokens=%s\n", prompt_idx, ids_list(ids).c_str());
  printf("prompt_idx=%d run1_witness_digest=%s\n", prompt_idx, hex(wit, 32).c_str());
  printf("prompt_idx=%d run1_argmax_digest=%s\n", prompt_idx, hex(adig, 32).c_str());
  if (samp.mode) {
    uint32_t tb, pb;
    memcpy(&tb, &samp.temperature, 4);
    memcpy(&pb, &samp.top_p, 4);
    printf("prompt_idx=%d sample_mode=1 seed=%llu temperature=%08x top_k=%u top_p=%08x\n",
           prompt_idx, (unsigned long long)samp.seed, tb, samp.top_k, pb);
  }
  const char* mode = reduction ? "tree" : "sequential";
  printf("prompt_idx=%d reduction_mode=%s\n", prompt_idx, mode);
  printf("CIS2_REF digest=%s prompt_idx=%d prompt_toks=%zu gen_toks=%d dtype=fp32 "
         "reduction_mode=%s\n",
         hex(wit, 32).c_str(), prompt_idx, prompt.size(), gen_toks, mode);
  cis2_ctx_destroy(ctx);
  return 0;
}
