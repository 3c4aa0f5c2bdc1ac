// cis2_runtime.hip — the C ABI of include/cis2_amd.h: device memory,
// tensor upload, the per-token kernel sequence, the greedy decode loop with
// the pipelined witness fold, tracing, and the standalone GEMV plan.
#include "cis2_amd.h"
#include "cis2_decode.hpp"
#include "cis2_kernels.hpp"
#include "cis2_rows.hpp"
#include "cis2_sample.hpp"
#include "cis2_sha256.hpp"

#include <errno.h>
#include <fcntl.h>
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/file.h>
#include <unistd.h>

#include <algorithm>
#include <map>
#include <string>
#include <thread>
#include <vector>

using namespace cis2;

namespace {

// Pinned constants in the declared order of the table digest (spec §6.6;
// code/cis2-fp/src/math.rs:472-500): f32 words, with PI_2 as 8 bytes.
void table_digest(uint8_t out[32]) {
  Sha256 s;
  const uint32_t head[9] = {0x3fb8aa3bu, 0x3f318000u, 0xb95e8083u, 0x39506967u, 0x3ab743ceu,
                            0x3c088908u, 0x3d2aa9c1u, 0x3e2aaaaau, 0x3f000000u};
  for (uint32_t w : head) s.update_u32le(w);
  const uint64_t pio2 = 0x3ff921fb54442d18ull;
  s.update_u32le((uint32_t)pio2);
  s.update_u32le((uint32_t)(pio2 >> 32));
  const uint32_t tail[18] = {0xbe2aaaa3u, 0x3c08839eu, 0xb94ca1f9u, 0x3d2aaaa5u, 0xbab6061au,
                             0x37ccf5ceu, 0x3f3504f3u, 0xb95e8083u, 0x3f318000u, 0x3d9021bbu,
                             0xbdebd1b8u, 0x3def251bu, 0xbdfe5d4fu, 0x3e11e9bfu, 0xbe2aae50u,
                             0x3e4cceadu, 0xbe7ffffcu, 0x3eaaaaaau};
  for (uint32_t w : tail) s.update_u32le(w);
  s.finish(out);
}

enum Kind { VEC, GEMV, EMBED, LMHEAD };
struct Slot {
  float** ptr;
  uint64_t count;
  Kind kind;
  uint32_t M, K, R;  // R: rows per block of the blocked GEMV layout
  bool required;
};

struct Layer {
  float *ln1 = nullptr, *ln2 = nullptr, *wq = nullptr, *wk = nullptr, *wv = nullptr,
        *wo = nullptr, *wg = nullptr, *wu = nullptr, *wd = nullptr;
  float *bq = nullptr, *bk = nullptr, *bv = nullptr, *qn = nullptr, *kn = nullptr;
};

const int kRing = 4;

// A greedy decode in progress (cis2_decode_begin/steps/end).
struct Session {
  bool active = false;
  uint32_t seq = 0, n_prompt = 0, max_steps = 0;
  uint32_t enqueued = 0, folded = 0;
  bool fast = false;  // persistent kernel (argmax fused) vs per-op kernels
  Sha256 w;
  std::vector<uint32_t> ids;
  std::vector<uint8_t> step_dig;
};

// Device buffers of the row-batched forward pass (grown on demand).
struct RowsBuf {
  uint32_t cap = 0, lcap = 0;  // rows / logit rows allocated
  float *h = nullptr, *h2 = nullptr, *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
        *att = nullptr, *hid = nullptr;  // [cap][width]
  float *lx = nullptr, *logits = nullptr;                            // [lcap][H], [lcap][V]
  uint32_t *seq = nullptr, *pos = nullptr, *tok = nullptr;           // [cap]
  uint32_t *lrows = nullptr, *arg = nullptr;                         // [lcap]
  // the decode steps' second logit / argmax buffer, [cap2][V] and [cap2]
  float* logits2 = nullptr;
  uint32_t* arg2 = nullptr;
  uint32_t cap2 = 0;
  // prefill attention tiles (device copy of htiles) and their scratch
  std::vector<AttTile> htiles;
  AttTile* tiles = nullptr;
  uint32_t tcap = 0;
  float* ascr = nullptr;
  size_t acap = 0;
  std::vector<void*> mem, lmem, mem2, tmem;
};

}  // namespace

struct cis2_ctx {
  cis2_config cfg;
  int dev = 0;  // the HIP device current at creation
  uint32_t qd = 0, kvd = 0;
  float scale = 0.0f;
  hipStream_t st = nullptr;
  hipStream_t cs = nullptr;  // device-to-host copies that overlap the next pass
  std::vector<Layer> L;
  float *embed = nullptr, *lm_head = nullptr, *final_norm = nullptr;
  float *inv_freq = nullptr, *rope_cs = nullptr;
  float* kv = nullptr;  // [max_seqs][n_layers][K | V][kvd * max_pos]
  float *h = nullptr, *h2 = nullptr, *x = nullptr, *q = nullptr, *k = nullptr, *v = nullptr,
        *att = nullptr, *o = nullptr, *g = nullptr, *u = nullptr, *hid = nullptr,
        *dn = nullptr, *logits = nullptr, *scores = nullptr, *probs = nullptr;
  uint32_t* d_tok = nullptr;     // [2]: input token of the current step, argmax out
  // second token slot and logit buffer of the decode session's alternating
  // steps (step s reads logits / token set s % 2 while the next pass writes
  // the other set)
  uint32_t* d_tok2 = nullptr;
  float* logits2 = nullptr;
  uint32_t* d_err = nullptr;
  uint32_t* d_prompt = nullptr;  // [max_pos]: prompt ids of the sequence being prefilled
  std::map<std::string, Slot> slots;
  std::map<std::string, bool> present;
  uint8_t table_dig[32], invf_dig[32];
  cis2_trace_fn trace = nullptr;
  void* trace_user = nullptr;
  std::string err;
  // decode ring (pinned host)
  float* ring = nullptr;
  uint32_t* ring_tok = nullptr;
  hipEvent_t ring_ev[kRing];
  hipEvent_t ring_ready[kRing];  // main stream: step's logits and token final
  Session sess;
  // persistent decode kernel state
  uint32_t Rq = 0, Ro = 0, Rg = 0, Rd = 0, Rl = 0;
  bool fast_ok = false;      // this configuration fits the persistent kernel
  bool force_ops = false;    // CIS2_PATH=ops: per-op kernels only
  bool seq_prefill = false;  // CIS2_PREFILL=seq: prefill position by position
  uint32_t ncu = 0;
  LayerW* d_layers = nullptr;
  bool layers_dirty = true;
  float* act = nullptr;
  uint32_t* counters = nullptr;
  uint32_t* cand = nullptr;
  uint32_t epoch = 0, lm_epoch = 0;
  DecodeArgs dargs;
  // Persistent launches of this GPU are taken one session at a time across
  // processes: an exclusive flock on <dir>/cis2amd-<pci bus id>.lock, held
  // from the first persistent launch of a session until its end
  // (CIS2_DECODE_LOCK=0: never taken; CIS2_LOCK_DIR: the directory, /tmp by
  // default).  -1: not held.
  int lock_fd = -1;
  bool lock_off = false;
  std::string lock_path;
  // steps whose persistent launch hit the spin cap and were recomputed on the
  // per-op path (cis2_recoveries)
  uint32_t recoveries = 0;
  uint64_t* tline = nullptr;  // CIS2_TIMELINE=<file>: per-task timestamps of every launch
  FILE* tline_file = nullptr;
  std::vector<uint16_t> wg_tasks;  // [nwg][kMaxTasks] task table of the persistent kernel
  // cis2_profile: event pairs around decode-kernel launches
  bool prof_on = false;
  std::vector<hipEvent_t> prof_ev;  // [2 * kProfMax], created on first use
  std::vector<uint32_t> prof_pos;
  // seeded sampling (cis2_set_sampling): parameters and device scratch
  bool samp_on = false;
  SampleParams samp{};
  SampleBufs sbuf;
  RowsBuf rows;
  std::vector<void*> allocs;
};

constexpr size_t kProfMax = 65536;
// Rows per block of the standalone GEMV plan's layout (one workgroup each).
constexpr uint32_t kPlanR = 16;
// Above this many row blocks (two per CU on MI355X) a lone GEMV runs on the
// streaming batch kernel.
constexpr uint32_t kPlanStreamBlocks = 512;

struct cis2_gemv_plan {
  uint32_t M, K, copies;
  float *W = nullptr, *x = nullptr, *y = nullptr;
  float *xb = nullptr, *yb = nullptr;  // [ncap][K], [ncap][M]: batched launches
  uint32_t ncap = 0;
  hipStream_t st = nullptr;
  hipEvent_t e0 = nullptr, e1 = nullptr;
};

namespace {

int fail(cis2_ctx* c, int code, const std::string& msg) {
  if (c) c->err = msg;
  return code;
}
int hipfail(cis2_ctx* c, hipError_t e, const char* what) {
  return fail(c, CIS2_E_DEVICE, std::string(what) + ": " + hipGetErrorString(e));
}
#define HIPCHK(c, expr, what)                       \
  do {                                              \
    hipError_t _e = (expr);                         \
    if (_e != hipSuccess) return hipfail(c, _e, what); \
  } while (0)

float* dalloc(cis2_ctx* c, size_t nfloats) {
  void* p = nullptr;
  if (hipMalloc(&p, nfloats * sizeof(float) + 16) != hipSuccess) return nullptr;
  c->allocs.push_back(p);
  return static_cast<float*>(p);
}

void add_slot(cis2_ctx* c, const std::string& name, float** ptr, uint64_t count, Kind kind,
              uint32_t M, uint32_t K, bool required, uint32_t R = 64) {
  c->slots[name] = Slot{ptr, count, kind, M, K, R, required};
}

// Checkpoint tensor names as the reference loader reads them
// (code/cis2-fp/gpu/cis2_host.cpp:133-158; Qwen3 q/k norms
// labs/w1x-qwen3/scripts/qwen3-port.diff:139-141).
void build_registry(cis2_ctx* c) {
  const cis2_config& f = c->cfg;
  const uint32_t H = f.hidden, I = f.inter, V = f.vocab, QD = c->qd, KV = c->kvd;
  add_slot(c, "model.embed_tokens.weight", &c->embed, (uint64_t)V * H, EMBED, V, H, true, c->Rl);
  add_slot(c, "model.norm.weight", &c->final_norm, H, VEC, 0, 0, true);
  if (!f.tied)
    add_slot(c, "lm_head.weight", &c->lm_head, (uint64_t)V * H, LMHEAD, V, H, true, c->Rl);
  for (uint32_t l = 0; l < f.n_layers; ++l) {
    Layer& Ly = c->L[l];
    char p[64];
    snprintf(p, sizeof p, "model.layers.%u.", l);
    std::string s(p);
    add_slot(c, s + "input_layernorm.weight", &Ly.ln1, H, VEC, 0, 0, true);
    add_slot(c, s + "post_attention_layernorm.weight", &Ly.ln2, H, VEC, 0, 0, true);
    add_slot(c, s + "self_attn.q_proj.weight", &Ly.wq, (uint64_t)QD * H, GEMV, QD, H, true, c->Rq);
    add_slot(c, s + "self_attn.k_proj.weight", &Ly.wk, (uint64_t)KV * H, GEMV, KV, H, true, c->Rq);
    add_slot(c, s + "self_attn.v_proj.weight", &Ly.wv, (uint64_t)KV * H, GEMV, KV, H, true, c->Rq);
    add_slot(c, s + "self_attn.o_proj.weight", &Ly.wo, (uint64_t)H * QD, GEMV, H, QD, true, c->Ro);
    add_slot(c, s + "mlp.gate_proj.weight", &Ly.wg, (uint64_t)I * H, GEMV, I, H, true, c->Rg);
    add_slot(c, s + "mlp.up_proj.weight", &Ly.wu, (uint64_t)I * H, GEMV, I, H, true, c->Rg);
    add_slot(c, s + "mlp.down_proj.weight", &Ly.wd, (uint64_t)H * I, GEMV, H, I, true, c->Rd);
    add_slot(c, s + "self_attn.q_proj.bias", &Ly.bq, QD, VEC, 0, 0, false);
    add_slot(c, s + "self_attn.k_proj.bias", &Ly.bk, KV, VEC, 0, 0, false);
    add_slot(c, s + "self_attn.v_proj.bias", &Ly.bv, KV, VEC, 0, 0, false);
    add_slot(c, s + "self_attn.q_norm.weight", &Ly.qn, f.head_dim, VEC, 0, 0, false);
    add_slot(c, s + "self_attn.k_norm.weight", &Ly.kn, f.head_dim, VEC, 0, 0, false);
  }
}

float* kcache(cis2_ctx* c, uint32_t seq, uint32_t l) {
  size_t per = (size_t)c->kvd * c->cfg.max_pos;
  return c->kv + ((size_t)seq * c->cfg.n_layers + l) * 2 * per;
}
float* vcache(cis2_ctx* c, uint32_t seq, uint32_t l) {
  return kcache(c, seq, l) + (size_t)c->kvd * c->cfg.max_pos;
}

// Per-op trace hook: synchronise, pull the op output, hash it.
int emit(cis2_ctx* c, int pos, int layer, const char* op, const float* dev, size_t n) {
  if (!c->trace) return CIS2_OK;
  HIPCHK(c, hipStreamSynchronize(c->st), "trace sync");
  std::vector<float> hbuf(n);
  HIPCHK(c, hipMemcpy(hbuf.data(), dev, n * sizeof(float), hipMemcpyDeviceToHost), "trace copy");
  uint8_t d[32];
  sha256(hbuf.data(), n * sizeof(float), d);
  c->trace(pos, layer, op, d, c->trace_user);
  return CIS2_OK;
}
#define EMIT(pos, layer, op, dev, n)                       \
  do {                                                     \
    int _r = emit(c, (pos), (layer), (op), (dev), (n));    \
    if (_r) return _r;                                     \
  } while (0)
#define LAUNCH(expr, what) HIPCHK(c, (expr), what)

// One decode step for `seq` at `pos`; the input token is read on the device
// from *d_tokp.  Op order: code/cis2-fp/src/main.rs:355-529 (C++ mirror
// gpu/cis2_model.h:685-760; Qwen3 QK-norm qwen3-port.diff:66-80).
int forward_one(cis2_ctx* c, uint32_t seq, uint32_t pos, const uint32_t* d_tokp,
                bool want_logits) {
  const cis2_config& f = c->cfg;
  const uint32_t H = f.hidden, I = f.inter, hd = f.head_dim, QD = c->qd, KV = c->kvd;
  hipStream_t s = c->st;
  const bool tr = c->trace != nullptr;
  const bool tree = c->cfg.reduction_mode == 1;
  LAUNCH(launch_embed(c->embed, d_tokp, c->h, H, f.vocab, c->d_err, s), "embed");
  EMIT(pos, -1, "embedding", c->h, H);
  for (uint32_t l = 0; l < f.n_layers; ++l) {
    const Layer& Ly = c->L[l];
    float* kc = kcache(c, seq, l);
    float* vc = vcache(c, seq, l);
    LAUNCH(launch_rmsnorm(c->h, Ly.ln1, f.eps, H, 1, c->x, s, tree), "norm1");
    EMIT(pos, l, "norm1", c->x, H);
    GemvSeg qkv[3] = {{Ly.wq, c->x, Ly.bq, c->q, QD, H, 0, c->Rq},
                      {Ly.wk, c->x, Ly.bk, c->k, KV, H, 0, c->Rq},
                      {Ly.wv, c->x, Ly.bv, c->v, KV, H, 0, c->Rq}};
    LAUNCH(launch_gemv(qkv, 3, s, tree), "qkv");
    EMIT(pos, l, "q", c->q, QD);
    EMIT(pos, l, "k", c->k, KV);
    EMIT(pos, l, "v", c->v, KV);
    if (Ly.qn) {
      LAUNCH(launch_rmsnorm(c->q, Ly.qn, f.eps, hd, f.n_heads, c->q, s, tree), "q_norm");
      EMIT(pos, l, "q_norm", c->q, QD);
    }
    if (Ly.kn) {
      LAUNCH(launch_rmsnorm(c->k, Ly.kn, f.eps, hd, f.n_kv_heads, c->k, s, tree), "k_norm");
      EMIT(pos, l, "k_norm", c->k, KV);
    }
    LAUNCH(launch_rope_store(c->q, c->k, c->v, c->rope_cs, pos, f.n_heads, f.n_kv_heads, hd,
                             f.max_pos, kc, vc, s),
           "rope");
    EMIT(pos, l, "rope_q", c->q, QD);
    EMIT(pos, l, "rope_k", c->k, KV);
    LAUNCH(launch_attention(c->q, kc, vc, pos, f.n_heads, f.n_kv_heads, hd, f.max_pos,
                            c->scale, c->att, tr ? c->scores : nullptr,
                            tr ? c->probs : nullptr, s, tree),
           "attention");
    EMIT(pos, l, "scores", c->scores, (size_t)f.n_heads * (pos + 1));
    EMIT(pos, l, "softmax", c->probs, (size_t)f.n_heads * (pos + 1));
    EMIT(pos, l, "attn_out", c->att, QD);
    GemvSeg os[1] = {{Ly.wo, c->att, c->h, c->h2, H, QD, 1, c->Ro}};
    if (tr) {  // the trace needs o_proj on its own
      GemvSeg ot[1] = {{Ly.wo, c->att, nullptr, c->o, H, QD, 0, c->Ro}};
      LAUNCH(launch_gemv(ot, 1, s, tree), "o_proj");
      EMIT(pos, l, "o_proj", c->o, H);
    }
    LAUNCH(launch_gemv(os, 1, s, tree), "o_proj+resid");
    std::swap(c->h, c->h2);
    EMIT(pos, l, "resid1", c->h, H);
    LAUNCH(launch_rmsnorm(c->h, Ly.ln2, f.eps, H, 1, c->x, s, tree), "norm2");
    EMIT(pos, l, "norm2", c->x, H);
    LAUNCH(launch_gate_up_silu(Ly.wg, Ly.wu, c->x, c->g, c->u, c->hid, I, H, c->Rg, s, tree),
           "gate_up");
    EMIT(pos, l, "gate", c->g, I);
    EMIT(pos, l, "up", c->u, I);
    EMIT(pos, l, "silu_mul", c->hid, I);
    if (tr) {
      GemvSeg dt[1] = {{Ly.wd, c->hid, nullptr, c->dn, H, I, 0, c->Rd}};
      LAUNCH(launch_gemv(dt, 1, s, tree), "down");
      EMIT(pos, l, "down", c->dn, H);
    }
    GemvSeg ds[1] = {{Ly.wd, c->hid, c->h, c->h2, H, I, 1, c->Rd}};
    LAUNCH(launch_gemv(ds, 1, s, tree), "down+resid");
    std::swap(c->h, c->h2);
    EMIT(pos, l, "resid2", c->h, H);
  }
  if (want_logits || tr) {
    LAUNCH(launch_rmsnorm(c->h, c->final_norm, f.eps, H, 1, c->x, s, tree), "final_norm");
    EMIT(pos, -1, "final_norm", c->x, H);
    GemvSeg lm[1] = {{c->lm_head, c->x, nullptr, c->logits, f.vocab, H, 0, c->Rl}};
    LAUNCH(launch_gemv(lm, 1, s, tree), "lm_head");
    EMIT(pos, -1, "logits", c->logits, f.vocab);
  }
  return CIS2_OK;
}

int check_err_flag(cis2_ctx* c) {
  uint32_t e = 0;
  HIPCHK(c, hipMemcpy(&e, c->d_err, 4, hipMemcpyDeviceToHost), "error flag");
  if (e) {
    (void)hipMemsetAsync(c->d_err, 0, 4, c->st);
    (void)hipStreamSynchronize(c->st);
    if (e & 2u)
      return fail(c, CIS2_E_DEVICE,
                  "persistent decode kernel: a phase wait hit its spin cap "
                  "(workgroups not co-resident)");
    if (e & 0x100u) return fail(c, CIS2_E_NUMERIC, "NaN among logits / temperature in a sampled draw");
    return fail(c, CIS2_E_RANGE, "token id out of range on the device");
  }
  return CIS2_OK;
}

// The GPU's persistent-decode lock (see cis2_ctx::lock_fd): taken before
// the first persistent launch of a session, kept until decode_unlock.  A
// second process (or context) decoding on the same GPU waits here instead
// of launching a grid that would share the CUs with this one (its
// workgroups could then wait on each other until the spin cap).  A lock
// that cannot be taken (unwritable directory) is skipped: the spin-cap
// recovery still keeps such runs correct.
static void decode_lock(cis2_ctx* c) {
  if (c->lock_off || c->lock_fd >= 0) return;
  const int fd = open(c->lock_path.c_str(), O_RDWR | O_CREAT | O_CLOEXEC, 0666);
  if (fd < 0) return;
  while (flock(fd, LOCK_EX) != 0) {
    if (errno != EINTR) {
      close(fd);
      return;
    }
  }
  c->lock_fd = fd;
}
static void decode_unlock(cis2_ctx* c) {
  if (c->lock_fd < 0) return;
  close(c->lock_fd);
  c->lock_fd = -1;
}

// Waits for every queued launch and copy, then clears the device error
// word; *bits receives what it held.
static int drain_and_clear_err(cis2_ctx* c, uint32_t* bits) {
  HIPCHK(c, hipStreamSynchronize(c->st), "drain");
  if (c->cs) HIPCHK(c, hipStreamSynchronize(c->cs), "drain copies");
  HIPCHK(c, hipMemcpy(bits, c->d_err, 4, hipMemcpyDeviceToHost), "error flag");
  HIPCHK(c, hipMemsetAsync(c->d_err, 0, 4, c->st), "error flag clear");
  HIPCHK(c, hipStreamSynchronize(c->st), "error flag clear");
  return CIS2_OK;
}

// Fills the persistent-kernel arguments once the weights are in place.
int prepare_fast(cis2_ctx* c) {
  if (!c->layers_dirty) return CIS2_OK;
  const cis2_config& f = c->cfg;
  std::vector<LayerW> hl(f.n_layers);
  for (uint32_t l = 0; l < f.n_layers; ++l) {
    const Layer& L = c->L[l];
    hl[l] = LayerW{L.ln1, L.ln2, L.wq, L.wk, L.wv, L.wo, L.wg, L.wu, L.wd,
                   L.bq, L.bk, L.bv, L.qn, L.kn};
  }
  HIPCHK(c, hipMemcpy(c->d_layers, hl.data(), hl.size() * sizeof(LayerW), hipMemcpyHostToDevice),
         "layer table");
  DecodeArgs& a = c->dargs;
  a.layers = c->d_layers;
  a.embed = c->embed;
  a.lm = c->lm_head;
  a.fnorm = c->final_norm;
  c->layers_dirty = false;
  return CIS2_OK;
}

// One position through the persistent kernel; the token is read from
// *tokp on the device and the argmax is written to c->d_tok[0].
int forward_fast(cis2_ctx* c, uint32_t seq, uint32_t pos, uint32_t* tokp, bool want_logits,
                 float* logits_out = nullptr, uint32_t* tok_out = nullptr) {
  int r = prepare_fast(c);
  if (r) return r;
  DecodeArgs& a = c->dargs;
  const size_t per_layer = (size_t)2 * c->kvd * c->cfg.max_pos;
  a.kc0 = c->kv + (size_t)seq * c->cfg.n_layers * per_layer;
  a.vc0 = a.kc0 + (size_t)c->kvd * c->cfg.max_pos;
  a.tok_in = tokp;
  a.tok_out = tok_out ? tok_out : c->d_tok;
  a.logits = logits_out ? logits_out : c->logits;
  a.pos = pos;
  if (c->epoch == UINT32_MAX) {  // tags would repeat: clear them and restart at 1
    HIPCHK(c, hipMemsetAsync(c->act, 0,
                             (size_t)c->cfg.n_layers *
                                 decode_act_floats(c->cfg.hidden, c->cfg.inter, c->qd,
                                                   c->kvd) * sizeof(float),
                             c->st),
           "tag reset");
    if (a.scw)
      HIPCHK(c, hipMemsetAsync(a.scw, 0,
                               (size_t)c->cfg.n_layers * c->cfg.n_heads * c->cfg.max_pos * 8,
                               c->st),
             "score tag reset");
    c->epoch = 0;
  }
  a.epoch = ++c->epoch;
  if (want_logits) ++c->lm_epoch;
  a.lm_epoch = c->lm_epoch;
  a.want_logits = want_logits ? 1u : 0u;
  a.tline = c->tline;
  const size_t pi = c->prof_pos.size();
  const bool prof = c->prof_on && pi < kProfMax;
  if (prof) HIPCHK(c, hipEventRecord(c->prof_ev[2 * pi], c->st), "profile event");
  LAUNCH(launch_decode(a, c->st), "decode kernel");
  if (prof) {
    HIPCHK(c, hipEventRecord(c->prof_ev[2 * pi + 1], c->st), "profile event");
    c->prof_pos.push_back(pos);
  }
  if (c->tline_file) {  // profiling mode: synchronous, one record per launch
    const size_t n = (size_t)c->cfg.n_layers * 6 * kTimelineTasks * 4;
    std::vector<uint64_t> hbuf(n);
    HIPCHK(c, hipStreamSynchronize(c->st), "timeline sync");
    HIPCHK(c, hipMemcpy(hbuf.data(), c->tline, n * 8, hipMemcpyDeviceToHost), "timeline copy");
    uint32_t hdr[4] = {pos, c->cfg.n_layers, kTimelineTasks, want_logits ? 1u : 0u};
    fwrite(hdr, sizeof hdr, 1, c->tline_file);
    fwrite(hbuf.data(), 8, n, c->tline_file);
  }
  return CIS2_OK;
}

// The path a step takes: the persistent kernel, or the per-op kernels when
// tracing (every op's output is observed) or when the configuration does
// not fit the persistent kernel.
bool use_fast(const cis2_ctx* c) { return c->fast_ok && !c->force_ops && !c->trace; }

// ---- row-batched forward pass ----------------------------------------------

template <class T>
T* rows_alloc(std::vector<void*>& mem, size_t n) {
  void* p = nullptr;
  if (hipMalloc(&p, n * sizeof(T) + 16) != hipSuccess) return nullptr;
  mem.push_back(p);
  return static_cast<T*>(p);
}

// Row buffers for n rows and nl logit rows.
int rows_reserve(cis2_ctx* c, uint32_t n, uint32_t nl) {
  RowsBuf& b = c->rows;
  const cis2_config& f = c->cfg;
  if (n > b.cap) {
    HIPCHK(c, hipStreamSynchronize(c->st), "rows sync");
    for (void* p : b.mem) (void)hipFree(p);
    b.mem.clear();
    b.cap = 0;
    const size_t H = f.hidden, I = f.inter, QD = c->qd, KV = c->kvd;
    bool ok = (b.h = rows_alloc<float>(b.mem, n * H)) && (b.h2 = rows_alloc<float>(b.mem, n * H)) &&
              (b.x = rows_alloc<float>(b.mem, n * H)) && (b.q = rows_alloc<float>(b.mem, n * QD)) &&
              (b.k = rows_alloc<float>(b.mem, n * KV)) && (b.v = rows_alloc<float>(b.mem, n * KV)) &&
              (b.att = rows_alloc<float>(b.mem, n * QD)) && (b.hid = rows_alloc<float>(b.mem, n * I)) &&
              (b.seq = rows_alloc<uint32_t>(b.mem, n)) && (b.pos = rows_alloc<uint32_t>(b.mem, n)) &&
              (b.tok = rows_alloc<uint32_t>(b.mem, n));
    if (!ok) return fail(c, CIS2_E_OOM, "row buffers");
    b.cap = n;
  }
  if (nl > b.lcap) {
    HIPCHK(c, hipStreamSynchronize(c->st), "rows sync");
    for (void* p : b.lmem) (void)hipFree(p);
    b.lmem.clear();
    b.lcap = 0;
    bool ok = (b.lx = rows_alloc<float>(b.lmem, (size_t)nl * f.hidden)) &&
              (b.logits = rows_alloc<float>(b.lmem, (size_t)nl * f.vocab)) &&
              (b.lrows = rows_alloc<uint32_t>(b.lmem, nl)) &&
              (b.arg = rows_alloc<uint32_t>(b.lmem, nl));
    if (!ok) return fail(c, CIS2_E_OOM, "logit row buffers");
    b.lcap = nl;
  }
  return CIS2_OK;
}

// The forward pass of n rows whose descriptors are already in c->rows
// (seq, pos, and the token of row r at tok[r]), every op over all rows
// before the next (code/cis2-fp/src/main.rs:355-529): K and V of every row
// reach the caches before any row's attention, so rows of one sequence see
// each other causally.  max_len = 1 + the largest position.  The final
// norm, LM head and argmax run for the nl rows listed in rows.lrows:
// logits[i] and arg[i] belong to row lrows[i].
// Row counts up to which forward_rows applies the layer norms inside the
// projections that read them.
constexpr uint32_t kFuseNormRows = 256;

// The logits and argmax go to b.logits / b.arg unless `logits` / `arg` name
// other buffers of at least nl rows.
// ntiles > 0: the attention runs over the ntiles tiles in c->rows.tiles
// (runs of rows of one sequence at consecutive positions).
// one_per_seq: every row belongs to a different sequence (decode steps), so
// RoPE and the cache store may run inside the attention launch.
int forward_rows(cis2_ctx* c, uint32_t n, const uint32_t* d_tok, uint32_t max_len, uint32_t nl,
                 float* logits = nullptr, uint32_t* arg = nullptr, uint32_t ntiles = 0,
                 bool one_per_seq = false) {
  const cis2_config& f = c->cfg;
  RowsBuf& b = c->rows;
  const uint32_t H = f.hidden, I = f.inter, hd = f.head_dim, QD = c->qd, KV = c->kvd;
  const bool tree = f.reduction_mode == 1;
  hipStream_t s = c->st;
  const RowsDesc rd{b.seq, b.pos, d_tok, n};
  const size_t per = (size_t)KV * f.max_pos;           // one layer's K (or V) of one sequence
  const uint64_t seq_stride = (uint64_t)f.n_layers * 2 * per;
  LAUNCH(launch_embed_rows(c->embed, rd, H, f.vocab, b.h, c->d_err, s), "rows embed");
  // for few rows (decode steps) the RMSNorms run inside the launches that
  // consume them; each workgroup then repeats the norm chain of its rows,
  // which is latency hidden by the launch it saves only while the grid is
  // small
  const bool fuse_norm = n <= kFuseNormRows;
  for (uint32_t l = 0; l < f.n_layers; ++l) {
    const Layer& Ly = c->L[l];
    float* kc = c->kv + (size_t)l * 2 * per;
    float* vc = kc + per;
    // q, k and v in one launch over norm1(h): the norm inside the launch
    // for few rows, as its own pass for many
    BgemmOpts o1;
    o1.tree = tree;
    const float* xin = b.h;
    if (fuse_norm) {
      o1.norm_w = Ly.ln1;
      o1.eps = f.eps;
    } else {
      LAUNCH(launch_rmsnorm(b.h, Ly.ln1, f.eps, H, n, b.x, s, tree), "rows norm1");
      xin = b.x;
    }
    const BgemmSeg qkv[3] = {
        {Ly.wq, QD, H, c->Rq, xin, H, b.q, QD, Ly.bq, 0, Ly.bq ? kEpiBias : kEpiNone},
        {Ly.wk, KV, H, c->Rq, xin, H, b.k, KV, Ly.bk, 0, Ly.bk ? kEpiBias : kEpiNone},
        {Ly.wv, KV, H, c->Rq, xin, H, b.v, KV, Ly.bv, 0, Ly.bv ? kEpiBias : kEpiNone}};
    LAUNCH(launch_bgemm_multi(qkv, 3, n, o1, s), "rows qkv");
    if (Ly.qn) LAUNCH(launch_rmsnorm(b.q, Ly.qn, f.eps, hd, n * f.n_heads, b.q, s, tree), "rows q_norm");
    if (Ly.kn) LAUNCH(launch_rmsnorm(b.k, Ly.kn, f.eps, hd, n * f.n_kv_heads, b.k, s, tree), "rows k_norm");
    // decode steps: RoPE and the cache store inside the attention launch
    // when its shape allows (hipErrorNotSupported: nothing launched)
    hipError_t fe = hipErrorNotSupported;
    if (one_per_seq && !ntiles)
      fe = launch_rope_attention_rows(b.q, b.k, b.v, c->rope_cs, rd, max_len, f.n_heads,
                                      f.n_kv_heads, hd, f.max_pos, kc, vc, seq_stride, c->scale,
                                      b.att, tree, s);
    if (fe != hipErrorNotSupported) {
      LAUNCH(fe, "rows rope + attention");
    } else {
      LAUNCH(launch_rope_store_rows(b.q, b.k, b.v, c->rope_cs, rd, f.n_heads, f.n_kv_heads, hd,
                                    f.max_pos, kc, vc, seq_stride, s),
             "rows rope");
      if (ntiles)
        LAUNCH(launch_attention_tiles(b.q, kc, vc, b.tiles, ntiles, max_len, f.n_heads,
                                      f.n_kv_heads, hd, f.max_pos, seq_stride, c->scale, b.att,
                                      b.ascr, s),
               "rows attention tiles");
      else
        LAUNCH(launch_attention_rows(b.q, kc, vc, rd, max_len, f.n_heads, f.n_kv_heads, hd,
                                     f.max_pos, seq_stride, c->scale, b.att, tree, s),
               "rows attention");
    }
    const BgemmSeg so{Ly.wo, H, QD, c->Ro, b.att, QD, b.h2, H, b.h, H, kEpiResidual};
    LAUNCH(launch_bgemm(so, n, tree, s), "rows o_proj");
    std::swap(b.h, b.h2);
    // gate and up as two chains per thread, silu(gate) * up stored
    BgemmOpts o2;
    o2.tree = tree;
    o2.W2 = Ly.wu;
    const float* x2 = b.h;
    if (fuse_norm) {
      o2.norm_w = Ly.ln2;
      o2.eps = f.eps;
    } else {
      LAUNCH(launch_rmsnorm(b.h, Ly.ln2, f.eps, H, n, b.x, s, tree), "rows norm2");
      x2 = b.x;
    }
    const BgemmSeg sg{Ly.wg, I, H, c->Rg, x2, H, b.hid, I, nullptr, 0, kEpiNone};
    LAUNCH(launch_bgemm_multi(&sg, 1, n, o2, s), "rows gate_up");
    const BgemmSeg sd{Ly.wd, H, I, c->Rd, b.hid, I, b.h2, H, b.h, H, kEpiResidual};
    LAUNCH(launch_bgemm(sd, n, tree, s), "rows down");
    std::swap(b.h, b.h2);
  }
  if (nl) {
    LAUNCH(launch_gather_rows(b.h, b.lrows, nl, H, b.lx, s), "rows gather");
    LAUNCH(launch_rmsnorm(b.lx, c->final_norm, f.eps, H, nl, b.lx, s, tree), "rows final_norm");
    if (!logits) logits = b.logits;
    if (!arg) arg = b.arg;
    const BgemmSeg sl{c->lm_head, f.vocab, H, c->Rl, b.lx, H, logits, f.vocab, nullptr, 0,
                      kEpiNone};
    LAUNCH(launch_bgemm(sl, nl, tree, s), "rows lm_head");
    LAUNCH(launch_argmax_rows(logits, nl, f.vocab, arg, s), "rows argmax");
  }
  return CIS2_OK;
}

// Uploads row descriptors (and the logit-row list) and runs forward_rows.
// Rows that attend in tiles: the prefill of many rows (runs of one sequence
// at consecutive positions, up to kAttTileRows per tile) in the sequential
// order, for the shapes the tiled kernel has; *ntiles = 0 otherwise.
// CIS2_ATT_TILES=1 / 0 forces the tiles on / off (the bits are the same).
int plan_tiles(cis2_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
               uint32_t max_len, uint32_t* ntiles) {
  const cis2_config& f = c->cfg;
  RowsBuf& b = c->rows;
  *ntiles = 0;
  const char* pe = getenv("CIS2_ATT_TILES");
  const bool force = pe && pe[0] == '1', off = pe && pe[0] == '0';
  if (off || f.reduction_mode != 0 ||
      !attention_tiles_supported(f.n_heads, f.n_kv_heads, f.head_dim))
    return CIS2_OK;
  if (!force && (uint64_t)n * f.n_kv_heads < 4 * (uint64_t)c->ncu) return CIS2_OK;
  b.htiles.clear();
  for (uint32_t i = 0; i < n;) {
    uint32_t k = 1;
    while (i + k < n && k < kAttTileRows && seq[i + k] == seq[i] && pos[i + k] == pos[i] + k) ++k;
    b.htiles.push_back(AttTile{i, k, seq[i], pos[i]});
    i += k;
  }
  const uint32_t nt = (uint32_t)b.htiles.size();
  // short runs, or too few tile workgroups to fill the GPU: per-row attention
  if (!force && ((uint64_t)nt * 8 > n || (uint64_t)nt * f.n_kv_heads < c->ncu)) return CIS2_OK;
  const size_t scr = attention_tiles_scratch_floats(nt, f.n_heads, f.n_kv_heads, max_len);
  if (nt > b.tcap || scr > b.acap) {
    HIPCHK(c, hipStreamSynchronize(c->st), "tiles sync");
    for (void* p : b.tmem) (void)hipFree(p);
    b.tmem.clear();
    b.tcap = 0;
    b.acap = 0;
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)nt * sizeof(AttTile)) != hipSuccess)
      return fail(c, CIS2_E_OOM, "attention tiles");
    b.tmem.push_back(p);
    b.tiles = static_cast<AttTile*>(p);
    if (hipMalloc(&p, scr * sizeof(float)) != hipSuccess)
      return fail(c, CIS2_E_OOM, "attention tile scratch");
    b.tmem.push_back(p);
    b.ascr = static_cast<float*>(p);
    b.tcap = nt;
    b.acap = scr;
  }
  HIPCHK(c, hipMemcpyAsync(b.tiles, b.htiles.data(), (size_t)nt * sizeof(AttTile),
                           hipMemcpyHostToDevice, c->st),
         "tiles upload");
  *ntiles = nt;
  return CIS2_OK;
}

int forward_rows_host(cis2_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                      const uint32_t* tok, uint32_t nl, const uint32_t* lrows) {
  int r = rows_reserve(c, n, nl);
  if (r) return r;
  RowsBuf& b = c->rows;
  uint32_t max_len = 0;
  for (uint32_t i = 0; i < n; ++i) max_len = std::max(max_len, pos[i] + 1);
  HIPCHK(c, hipMemcpyAsync(b.seq, seq, (size_t)n * 4, hipMemcpyHostToDevice, c->st), "rows seq");
  HIPCHK(c, hipMemcpyAsync(b.pos, pos, (size_t)n * 4, hipMemcpyHostToDevice, c->st), "rows pos");
  HIPCHK(c, hipMemcpyAsync(b.tok, tok, (size_t)n * 4, hipMemcpyHostToDevice, c->st), "rows tok");
  if (nl)
    HIPCHK(c, hipMemcpyAsync(b.lrows, lrows, (size_t)nl * 4, hipMemcpyHostToDevice, c->st),
           "rows lrows");
  uint32_t ntiles = 0;
  r = plan_tiles(c, n, seq, pos, max_len, &ntiles);
  if (r) return r;
  std::vector<uint32_t> ss(seq, seq + n);
  std::sort(ss.begin(), ss.end());
  const bool one_per_seq = std::adjacent_find(ss.begin(), ss.end()) == ss.end();
  return forward_rows(c, n, b.tok, max_len, nl, nullptr, nullptr, ntiles, one_per_seq);
}

// Checks a row set: sequence and position ranges, token ranges, and no two
// rows at the same (sequence, position).
int check_rows(cis2_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
               const uint32_t* tok) {
  std::vector<uint64_t> keys(n);
  for (uint32_t i = 0; i < n; ++i) {
    if (seq[i] >= c->cfg.max_seqs) return fail(c, CIS2_E_ARG, "sequence index out of range");
    if (pos[i] >= c->cfg.max_pos) return fail(c, CIS2_E_RANGE, "position beyond max_pos");
    if (tok && tok[i] >= c->cfg.vocab) return fail(c, CIS2_E_RANGE, "token id >= vocab");
    keys[i] = (uint64_t)seq[i] << 32 | pos[i];
  }
  std::sort(keys.begin(), keys.end());
  if (std::adjacent_find(keys.begin(), keys.end()) != keys.end())
    return fail(c, CIS2_E_ARG, "two rows at the same sequence and position");
  return CIS2_OK;
}

// Folds `rows` logit rows into their witness streams on up to 16 host
// threads: for row i, the V logit bit patterns (u32 LE) then next id.
void fold_rows(std::vector<Sha256>& w, const float* logits, const uint32_t* ids, uint32_t rows,
               uint32_t V) {
  const uint32_t nt = std::max(1u, std::min<uint32_t>(rows, std::min(16u, std::max(
                                                           1u, std::thread::hardware_concurrency()))));
  auto job = [&](uint32_t t) {
    for (uint32_t i = t; i < rows; i += nt) {
      w[i].update(logits + (size_t)i * V, (size_t)V * sizeof(float));
      w[i].update_u32le(ids[i]);
    }
  };
  if (nt == 1) {
    job(0);
    return;
  }
  std::vector<std::thread> th;
  for (uint32_t t = 0; t < nt; ++t) th.emplace_back(job, t);
  for (auto& x : th) x.join();
}

}  // namespace

// Spreads the tasks of every phase over the workgroups: each task goes to a
// workgroup with the fewest tasks of its phase (a phase with more tasks than
// workgroups: split attention's score and mix tasks, so that no workgroup
// runs two score tasks while another runs none), then the fewest tasks so
// far, preferring one whose previous task is not in the phase just before
// (so its next weight copy has a phase of time to land; a down task's
// successor is the next layer's QKV task).  Every list is in phase order,
// which makes the waits acyclic: a task only waits for tasks of earlier
// (layer, phase), or, for split attention's mix tasks, for score tasks of
// the same phase, which come first in every list (lower task indices are
// assigned first).  False when some workgroup would need more than
// kMaxTasks or a task index exceeds 12 bits.
// XCDs of the MI355X (8 chiplets of 32 CUs, each with its own L2).
constexpr uint32_t kXcds = 8;
// The kv head whose cached K/V rows attention task t reads: task h of the
// one-task form is query head h; in the split form the score tasks are
// (kv head, chunk) and the mix tasks (query head, dim slice).
static uint32_t att_kv_head(const DecodeArgs& a, uint32_t t) {
  const uint32_t group = a.nh / a.nkv;
  if (!a.att_split) return t / group;
  if (t < a.natt_s) return t / a.att_chunks;
  return (t - a.natt_s) / a.att_dvc / group;
}

static bool assign_tasks(const DecodeArgs& a, std::vector<uint16_t>& table) {
  const uint32_t natt = a.att_split ? a.natt_s + a.natt_v : a.nh;
  const uint32_t n[kPhases] = {a.nq, natt, a.no, a.ng, a.nd};
  const uint32_t W = a.nwg;
  table.assign((size_t)W * kMaxTasks, kNoTask);
  std::vector<uint32_t> cnt(W, 0), same(W, 0);
  std::vector<int> last(W, -2);
  std::vector<bool> has_qkv(W, false);
  for (uint32_t p = 0; p < kPhases; ++p) {
    if (n[p] >= 4096) return false;
    std::fill(same.begin(), same.end(), 0u);
    auto adjacent = [&](uint32_t w) {
      return last[w] == (int)p - 1 || (p == kPhaseD && has_qkv[w]);
    };
    // split attention: the mix tasks (long) are placed first, one per
    // workgroup while there are workgroups left, then the score tasks
    // (short) beside them; each workgroup's list is then put back in task
    // order, so its score tasks run before its mix task
    const bool mix_first = p == kPhaseATT && a.att_split;
    for (uint32_t k = 0; k < n[p]; ++k) {
      const uint32_t t = mix_first ? (k < a.natt_v ? a.natt_s + k : k - a.natt_v) : k;
      // attention tasks of one kv head go to one XCD (workgroups are
      // dispatched to the XCDs round-robin: workgroup w runs on XCD
      // w % kXcds), so the tasks that read the same cached K and V rows
      // share that XCD's L2 and the rows come from HBM about once
      const int pref = p == kPhaseATT ? (int)(att_kv_head(a, t) % kXcds) : -1;
      auto on_pref = [&](uint32_t w) { return pref >= 0 && (int)(w % kXcds) == pref; };
      uint32_t best = W;
      for (uint32_t w = 0; w < W; ++w) {
        // one task of a phase per workgroup, unless the phase has more
        // tasks than workgroups
        if (cnt[w] >= kMaxTasks || (same[w] > 0 && n[p] <= W)) continue;
        if (best == W) { best = w; continue; }
        if (same[w] != same[best]) {
          if (same[w] < same[best]) best = w;
          continue;
        }
        if (on_pref(w) != on_pref(best)) {
          if (on_pref(w)) best = w;
          continue;
        }
        const bool adj_w = adjacent(w), adj_b = adjacent(best);
        if (cnt[w] < cnt[best] || (cnt[w] == cnt[best] && !adj_w && adj_b)) best = w;
      }
      if (best == W) return false;
      table[(size_t)best * kMaxTasks + cnt[best]] = (uint16_t)(p << 12 | t);
      ++cnt[best];
      ++same[best];
      last[best] = (int)p;
      if (p == kPhaseQKV) has_qkv[best] = true;
    }
    if (mix_first)
      for (uint32_t w = 0; w < W; ++w) {
        uint16_t* row = &table[(size_t)w * kMaxTasks];
        std::sort(row + cnt[w] - same[w], row + cnt[w]);
      }
  }
  return true;
}

// Floats of the largest set of weight blocks a workgroup without an
// attention task keeps in LDS (the persistent kernel's per-task slots).
static uint32_t task_slot_floats(const DecodeArgs& a, const std::vector<uint16_t>& table) {
  uint64_t best = 0;
  for (size_t w = 0; w * kMaxTasks < table.size(); ++w) {
    uint64_t tot = 0;
    bool att = false;
    for (uint32_t i = 0; i < kMaxTasks; ++i) {
      const uint16_t v = table[w * kMaxTasks + i];
      if (v == kNoTask) break;
      switch (v >> 12) {
        case kPhaseQKV: tot += (uint64_t)a.Rq * a.H; break;
        case kPhaseATT: att = true; break;
        case kPhaseO: tot += (uint64_t)a.Ro * a.qd; break;
        case kPhaseGU: tot += 2ull * a.Rg * a.H; break;
        case kPhaseD: tot += (uint64_t)a.Rd * a.I; break;
        default: break;
      }
    }
    if (!att && tot > best) best = tot;
  }
  return best > UINT32_MAX ? UINT32_MAX : (uint32_t)best;
}

extern "C" {

const char* cis2_strerror(int code) {
  switch (code) {
    case CIS2_OK: return "ok";
    case CIS2_E_ARG: return "invalid argument";
    case CIS2_E_UNSUPPORTED: return "unsupported configuration";
    case CIS2_E_MISSING_TENSOR: return "required tensor missing";
    case CIS2_E_SHAPE: return "tensor element count mismatch";
    case CIS2_E_NAME: return "unknown tensor name";
    case CIS2_E_FPENV: return "device FTZ/DAZ self-test failed";
    case CIS2_E_DEVICE: return "HIP device error";
    case CIS2_E_OOM: return "out of memory";
    case CIS2_E_RANGE: return "position or token out of range";
    case CIS2_E_NUMERIC: return "NaN logit in a sampled draw";
    default: return "unknown error";
  }
}

const char* cis2_last_error(const cis2_ctx* ctx) { return ctx ? ctx->err.c_str() : ""; }

void cis2_ctx_destroy(cis2_ctx* c) {
  if (!c) return;
  if (c->st) (void)hipStreamSynchronize(c->st);
  if (c->cs) (void)hipStreamSynchronize(c->cs);
  if (c->lock_fd >= 0) close(c->lock_fd);  // closing the descriptor releases the flock
  for (void* p : c->allocs) (void)hipFree(p);
  for (void* p : c->rows.mem) (void)hipFree(p);
  for (void* p : c->rows.lmem) (void)hipFree(p);
  for (void* p : c->rows.mem2) (void)hipFree(p);
  for (void* p : c->rows.tmem) (void)hipFree(p);
  if (c->tline_file) fclose(c->tline_file);
  for (hipEvent_t e : c->prof_ev)
    if (e) (void)hipEventDestroy(e);
  if (c->ring) (void)hipHostFree(c->ring);
  if (c->ring_tok) (void)hipHostFree(c->ring_tok);
  for (int i = 0; i < kRing; ++i) {
    if (c->ring_ev[i]) (void)hipEventDestroy(c->ring_ev[i]);
    if (c->ring_ready[i]) (void)hipEventDestroy(c->ring_ready[i]);
  }
  if (c->cs) {
    (void)hipStreamSynchronize(c->cs);
    (void)hipStreamDestroy(c->cs);
  }
  if (c->st) (void)hipStreamDestroy(c->st);
  delete c;
}

int cis2_ctx_create(const cis2_config* cfg, cis2_ctx** out) {
  if (!cfg || !out) return CIS2_E_ARG;
  *out = nullptr;
  cis2_config f = *cfg;
  if (f.hidden == 0 || f.inter == 0 || f.n_layers == 0 || f.n_heads == 0 || f.n_kv_heads == 0 ||
      f.head_dim == 0 || f.vocab == 0 || f.max_pos == 0 || f.max_seqs == 0)
    return CIS2_E_ARG;
  if (f.reduction_mode > 1) return CIS2_E_UNSUPPORTED;
  if (f.n_heads % f.n_kv_heads || f.head_dim % 2 || f.hidden % 4 || f.inter % 4 ||
      (f.n_heads * f.head_dim) % 4 || f.max_pos > 16384 || f.head_dim > 1024)
    return CIS2_E_UNSUPPORTED;
  // capacity rounded up to 4 positions: the K cache rows are copied as float4
  f.max_pos = (f.max_pos + 3u) & ~3u;
  cis2_ctx* c = new cis2_ctx();
  memset(c->ring_ev, 0, sizeof c->ring_ev);
  c->cfg = f;
  c->qd = f.n_heads * f.head_dim;
  c->kvd = f.n_kv_heads * f.head_dim;
  c->L.resize(f.n_layers);
  if (hipGetDevice(&c->dev) != hipSuccess ||
      hipStreamCreateWithFlags(&c->st, hipStreamNonBlocking) != hipSuccess) {
    cis2_ctx_destroy(c);
    return CIS2_E_DEVICE;
  }
  // this GPU's preallocated sampler scratch (cis2_sample_logits_noalloc)
  if (sample_scratch_init() != hipSuccess) {
    cis2_ctx_destroy(c);
    return CIS2_E_DEVICE;
  }
  // FTZ/DAZ self-test on the device (spec §1.3).
  {
    uint32_t* probe = nullptr;
    uint32_t hv[2] = {1u, 1u};
    if (hipMalloc(&probe, 8) != hipSuccess) { cis2_ctx_destroy(c); return CIS2_E_OOM; }
    hipError_t e = launch_fpenv_probe(probe, c->st);
    if (e == hipSuccess) e = hipMemcpy(hv, probe, 8, hipMemcpyDeviceToHost);
    (void)hipFree(probe);
    if (e != hipSuccess) { cis2_ctx_destroy(c); return CIS2_E_DEVICE; }
    if (hv[0] != 0u || hv[1] != 0u) { cis2_ctx_destroy(c); return CIS2_E_FPENV; }
  }
  const uint32_t H = f.hidden, I = f.inter, V = f.vocab;
  const size_t wide = H > c->qd ? H : c->qd;
  float** bufs[] = {&c->h, &c->h2, &c->x, &c->o, &c->dn};
  for (float** b : bufs)
    if (!(*b = dalloc(c, wide))) { cis2_ctx_destroy(c); return CIS2_E_OOM; }
  if (!(c->q = dalloc(c, c->qd)) || !(c->att = dalloc(c, c->qd)) || !(c->k = dalloc(c, c->kvd)) ||
      !(c->v = dalloc(c, c->kvd)) || !(c->g = dalloc(c, I)) || !(c->u = dalloc(c, I)) ||
      !(c->hid = dalloc(c, I)) || !(c->logits = dalloc(c, V)) ||
      !(c->scores = dalloc(c, (size_t)f.n_heads * f.max_pos)) ||
      !(c->probs = dalloc(c, (size_t)f.n_heads * f.max_pos)) ||
      !(c->inv_freq = dalloc(c, f.head_dim / 2)) ||
      !(c->rope_cs = dalloc(c, (size_t)f.head_dim * f.max_pos)) ||
      !(c->kv = dalloc(c, (size_t)f.max_seqs * f.n_layers * 2 * c->kvd * f.max_pos))) {
    cis2_ctx_destroy(c);
    return CIS2_E_OOM;
  }
  void* tp = nullptr;
  if (hipMalloc(&tp, 16) != hipSuccess) { cis2_ctx_destroy(c); return CIS2_E_OOM; }
  c->allocs.push_back(tp);
  c->d_tok = static_cast<uint32_t*>(tp);
  c->d_err = c->d_tok + 2;
  (void)hipMemsetAsync(tp, 0, 16, c->st);
  if (hipMalloc(&tp, 16) != hipSuccess) { cis2_ctx_destroy(c); return CIS2_E_OOM; }
  c->allocs.push_back(tp);
  c->d_tok2 = static_cast<uint32_t*>(tp);
  (void)hipMemsetAsync(tp, 0, 16, c->st);
  if (!(c->logits2 = dalloc(c, V))) { cis2_ctx_destroy(c); return CIS2_E_OOM; }
  if (hipMalloc(&tp, (size_t)f.max_pos * sizeof(uint32_t)) != hipSuccess) {
    cis2_ctx_destroy(c);
    return CIS2_E_OOM;
  }
  c->allocs.push_back(tp);
  c->d_prompt = static_cast<uint32_t*>(tp);
  (void)hipMemsetAsync(c->kv, 0, (size_t)f.max_seqs * f.n_layers * 2 * c->kvd * f.max_pos * sizeof(float), c->st);
  // Pinned inv_freq and rotation table; theta narrowed to f32 once
  // (code/cis2-fp/src/main.rs:849-858).
  if (launch_rope_table((float)f.rope_theta, f.head_dim, f.max_pos, c->inv_freq, c->rope_cs,
                        c->st) != hipSuccess ||
      hipStreamSynchronize(c->st) != hipSuccess) {
    cis2_ctx_destroy(c);
    return CIS2_E_DEVICE;
  }
  std::vector<float> invf(f.head_dim / 2);
  (void)hipMemcpy(invf.data(), c->inv_freq, invf.size() * sizeof(float), hipMemcpyDeviceToHost);
  sha256(invf.data(), invf.size() * sizeof(float), c->invf_dig);
  table_digest(c->table_dig);
  // scale = rsqrt_cr((f32)head_dim), computed on the device like every
  // other pinned value (code/cis2-fp/src/main.rs:372).
  {
    float hdv = (float)f.head_dim, sc = 0.0f;
    if (cis2_math_map(5, &hdv, &sc, 1) != CIS2_OK) { cis2_ctx_destroy(c); return CIS2_E_DEVICE; }
    c->scale = sc;
  }
  if (hipHostMalloc(reinterpret_cast<void**>(&c->ring), (size_t)kRing * V * sizeof(float)) !=
          hipSuccess ||
      hipHostMalloc(reinterpret_cast<void**>(&c->ring_tok), kRing * 2 * sizeof(uint32_t)) !=
          hipSuccess) {
    cis2_ctx_destroy(c);
    return CIS2_E_OOM;
  }
  for (int i = 0; i < kRing; ++i)
    if (hipEventCreateWithFlags(&c->ring_ev[i], hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&c->ring_ready[i], hipEventDisableTiming) != hipSuccess) {
      cis2_ctx_destroy(c);
      return CIS2_E_DEVICE;
    }
  // Persistent decode kernel: row-block sizes, task counts, workgroup roles.
  // The GEMV layout's row-block sizes are shared by both paths: R <= 32 when
  // the persistent kernel fits with them, else R <= 64.
  {
    int dev = 0, ncu = 0, lds = 0;
    (void)hipGetDevice(&dev);
    (void)hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev);
    (void)hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev);
    c->ncu = (uint32_t)ncu;
    const char* pe = getenv("CIS2_PATH");
    c->force_ops = pe && !strcmp(pe, "ops");
    const char* pl = getenv("CIS2_DECODE_LOCK");
    c->lock_off = pl && !strcmp(pl, "0");
    {
      char bus[64] = {0};
      if (hipDeviceGetPCIBusId(bus, (int)sizeof bus - 1, dev) != hipSuccess || !bus[0])
        snprintf(bus, sizeof bus, "dev%d", dev);
      for (char* q = bus; *q; ++q)
        if (*q == ':' || *q == '/' || *q == '.') *q = '_';
      const char* ld = getenv("CIS2_LOCK_DIR");
      c->lock_path = std::string(ld && *ld ? ld : "/tmp") + "/cis2amd-" + bus + ".lock";
    }
    const char* pf = getenv("CIS2_PREFILL");
    c->seq_prefill = pf && !strcmp(pf, "seq");
    DecodeArgs& a = c->dargs;
    // cap: the largest block height; small: GEMV blocks of at most 8 rows
    // (gate/up 8 each) and 32-row LM blocks, taken when every GEMV phase
    // still has at most one task per workgroup
    auto plan = [&](uint32_t cap, bool small) {
      memset(&a, 0, sizeof a);
      a.H = H; a.I = I; a.V = V; a.L = f.n_layers; a.nh = f.n_heads; a.nkv = f.n_kv_heads;
      a.hd = f.head_dim; a.qd = c->qd; a.kvd = c->kvd; a.max_pos = f.max_pos;
      a.Rq = rows_per_block(H, cap);
      a.Ro = rows_per_block(c->qd, cap);
      a.Rg = rows_per_block(H, cap) / 2 > 0 ? rows_per_block(H, cap) / 2 : 1;
      a.Rd = rows_per_block(I, cap);
      a.Rl = rows_per_block(H, cap);
      if (small) {
        // the smallest of 8, 16, 32 rows that keeps the phase at one task
        // per workgroup (and the block within rows_per_block's bound)
        auto pick = [&](uint32_t M, uint32_t K, uint32_t mats) {
          for (uint32_t r = 8; r <= 32; r *= 2)
            if ((M + r - 1) / r <= c->ncu && r * mats <= rows_per_block(K, 64)) return r;
          return 0u;
        };
        a.Rq = pick(c->qd + 2 * c->kvd, H, 1);
        a.Ro = pick(H, c->qd, 1);
        a.Rg = pick(I, H, 2);
        a.Rd = pick(H, I, 1);
        a.Rl = rows_per_block(H, 32);
        if (!a.Rq || !a.Ro || !a.Rg || !a.Rd) return false;
      }
      a.nq_q = (c->qd + a.Rq - 1) / a.Rq;
      a.nq_k = (c->kvd + a.Rq - 1) / a.Rq;
      a.nq = a.nq_q + 2 * a.nq_k;
      a.no = (H + a.Ro - 1) / a.Ro;
      a.ng = (I + a.Rg - 1) / a.Rg;
      a.nd = (H + a.Rd - 1) / a.Rd;
      a.nl = (V + a.Rl - 1) / a.Rl;
      a.nwg = c->ncu;
      a.cache_stride = (uint64_t)2 * c->kvd * f.max_pos;
      a.eps = f.eps;
      a.scale = c->scale;
      a.tree = f.reduction_mode;
      a.rope_cs = c->rope_cs;
      a.logits = c->logits;
      a.err = c->d_err;
      a.spin_cap = kDefaultSpinCap;
      if (const char* sc = getenv("CIS2_SPIN_CAP")) {
        const unsigned long v = strtoul(sc, nullptr, 10);
        if (v >= 1 && v <= kDefaultSpinCap) a.spin_cap = (uint32_t)v;
      }
      // attention split over score and mix tasks when a head's K/V rows at
      // max_pos do not fit one workgroup (CIS2_ATT=split / one: forced)
      const char* pa = getenv("CIS2_ATT");
      decode_att_plan(a, pa && !strcmp(pa, "split")  ? true
                         : pa && !strcmp(pa, "one") ? false
                                                    : decode_att_needs_split(a));
      if (small && (a.nq > a.nwg || a.no > a.nwg || a.ng > a.nwg || a.nd > a.nwg)) return false;
      if (!assign_tasks(a, c->wg_tasks)) return false;
      // dynamic LDS plus the kernel's static LDS (a few words) within one CU
      const size_t cap_lds = lds > 0 && (size_t)lds < 160 * 1024 ? (size_t)lds : 160 * 1024;
      a.wslot = task_slot_floats(a, c->wg_tasks);
      if (decode_lds_bytes(a) + 64 > cap_lds) a.wslot = 0;  // slots where they fit only
      const size_t need_lds = decode_lds_bytes(a) + 64;
      return lds > 0 && need_lds <= cap_lds && a.hd <= 256 &&  // RoPE: one pair per thread
             // split attention's score tasks address a kv head's K rows as one buffer
             (!a.att_split || (uint64_t)a.hd * a.max_pos * 4 <= 0x7FFFFFFFu) &&
             decode_att_ok(a);
    };
    c->fast_ok = plan(32, true) || plan(32, false) || plan(64, false);
    if (c->fast_ok) {  // every workgroup resident at once, or the per-op path
      bool res = false;
      if (decode_coresident(a, c->ncu, &res) != hipSuccess || !res) c->fast_ok = false;
    }
    c->Rq = a.Rq; c->Ro = a.Ro; c->Rg = a.Rg; c->Rd = a.Rd; c->Rl = a.Rl;
    void* p = nullptr;
    if (hipMalloc(&p, c->wg_tasks.size() * sizeof(uint16_t)) != hipSuccess) {
      cis2_ctx_destroy(c);
      return CIS2_E_OOM;
    }
    c->allocs.push_back(p);
    (void)hipMemcpy(p, c->wg_tasks.data(), c->wg_tasks.size() * sizeof(uint16_t),
                    hipMemcpyHostToDevice);
    a.wg_tasks = static_cast<const uint16_t*>(p);
    const size_t act_f = (size_t)f.n_layers * decode_act_floats(H, I, c->qd, c->kvd);
    const size_t cnt_n = 64;
    if (!(c->act = dalloc(c, act_f)) || hipMalloc(&p, cnt_n * 4) != hipSuccess) {
      cis2_ctx_destroy(c);
      return CIS2_E_OOM;
    }
    c->allocs.push_back(p);
    c->counters = static_cast<uint32_t*>(p);
    (void)hipMemsetAsync(c->counters, 0, cnt_n * 4, c->st);
    (void)hipMemsetAsync(c->act, 0, act_f * sizeof(float), c->st);  // tag 0: never a launch epoch
    if (hipMalloc(&p, ((size_t)2 * a.nl + 4) * 4) != hipSuccess) {
      cis2_ctx_destroy(c);
      return CIS2_E_OOM;
    }
    c->allocs.push_back(p);
    c->cand = static_cast<uint32_t*>(p);
    if (hipMalloc(&p, (size_t)f.n_layers * sizeof(LayerW)) != hipSuccess) {
      cis2_ctx_destroy(c);
      return CIS2_E_OOM;
    }
    c->allocs.push_back(p);
    c->d_layers = static_cast<LayerW*>(p);
    a.act = c->act;
    a.cnt = c->counters;
    a.cand = c->cand;
    if (a.att_split) {
      const size_t nw = (size_t)f.n_layers * f.n_heads * f.max_pos;
      if (hipMalloc(&p, nw * 8) != hipSuccess) {
        cis2_ctx_destroy(c);
        return CIS2_E_OOM;
      }
      c->allocs.push_back(p);
      (void)hipMemsetAsync(p, 0, nw * 8, c->st);  // tag 0: never a launch epoch
      a.scw = static_cast<uint64_t*>(p);
    }
    if (const char* tl = getenv("CIS2_TIMELINE")) {
      const size_t n = (size_t)f.n_layers * 6 * kTimelineTasks * 4;
      if (hipMalloc(&p, n * 8) == hipSuccess) {
        c->allocs.push_back(p);
        c->tline = static_cast<uint64_t*>(p);
        (void)hipMemsetAsync(c->tline, 0, n * 8, c->st);
        c->tline_file = fopen(tl, "wb");
        // the task table beside it (<file>.tasks: nwg rows of kMaxTasks
        // phase << 12 | task words, 0xFFFF ends a row)
        if (FILE* tf = fopen((std::string(tl) + ".tasks").c_str(), "wb")) {
          fwrite(c->wg_tasks.data(), sizeof(uint16_t), c->wg_tasks.size(), tf);
          fclose(tf);
        }
      }
    }
  }
  // every zero fill above runs on the context's stream (which does not
  // synchronize with the null stream): complete before the first launch
  if (hipStreamSynchronize(c->st) != hipSuccess) {
    cis2_ctx_destroy(c);
    return CIS2_E_DEVICE;
  }
  build_registry(c);
  *out = c;
  return CIS2_OK;
}

int cis2_upload_bf16(cis2_ctx* c, const char* name, const uint16_t* bf16, uint64_t n) {
  if (!c || !name || !bf16) return CIS2_E_ARG;
  auto it = c->slots.find(name);
  if (it == c->slots.end()) return fail(c, CIS2_E_NAME, std::string("unknown tensor ") + name);
  Slot& s = it->second;
  if (n != s.count)
    return fail(c, CIS2_E_SHAPE, std::string("tensor ") + name + " element count mismatch");
  uint16_t* stage = nullptr;
  HIPCHK(c, hipMalloc(&stage, n * sizeof(uint16_t)), "stage alloc");
  hipError_t e = hipMemcpy(stage, bf16, n * sizeof(uint16_t), hipMemcpyHostToDevice);
  float* wide = nullptr;
  if (e == hipSuccess) e = hipMalloc(&wide, n * sizeof(float));
  if (e == hipSuccess) e = launch_widen(stage, wide, n, c->st);
  float* dst = *s.ptr;
  if (e == hipSuccess && s.kind == VEC) {
    if (!dst && !(dst = dalloc(c, n))) e = hipErrorOutOfMemory;
    if (e == hipSuccess) e = hipMemcpyAsync(dst, wide, n * sizeof(float), hipMemcpyDeviceToDevice, c->st);
  } else if (e == hipSuccess && s.kind == EMBED) {
    if (!dst && !(dst = dalloc(c, n))) e = hipErrorOutOfMemory;
    if (e == hipSuccess) e = hipMemcpyAsync(dst, wide, n * sizeof(float), hipMemcpyDeviceToDevice, c->st);
    if (e == hipSuccess && c->cfg.tied) {
      if (!c->lm_head && !(c->lm_head = dalloc(c, blocked_floats(s.M, s.K, s.R))))
        e = hipErrorOutOfMemory;
      if (e == hipSuccess) e = launch_relayout(wide, c->lm_head, s.M, s.K, s.R, c->st);
    }
  } else if (e == hipSuccess) {  // GEMV / LMHEAD: blocked layout
    if (!dst && !(dst = dalloc(c, blocked_floats(s.M, s.K, s.R)))) e = hipErrorOutOfMemory;
    if (e == hipSuccess) e = launch_relayout(wide, dst, s.M, s.K, s.R, c->st);
  }
  if (e == hipSuccess) e = hipStreamSynchronize(c->st);
  (void)hipFree(stage);
  if (wide) (void)hipFree(wide);
  if (e != hipSuccess) return hipfail(c, e, "upload");
  *s.ptr = dst;
  c->present[name] = true;
  c->layers_dirty = true;
  return CIS2_OK;
}

int cis2_check_ready(cis2_ctx* c) {
  if (!c) return CIS2_E_ARG;
  for (auto& kv : c->slots)
    if (kv.second.required && !c->present.count(kv.first))
      return fail(c, CIS2_E_MISSING_TENSOR, "tensor " + kv.first + " missing");
  if (!c->lm_head) return fail(c, CIS2_E_MISSING_TENSOR, "LM head missing");
  return CIS2_OK;
}

int cis2_digests(cis2_ctx* c, uint8_t table[32], uint8_t inv_freq[32]) {
  if (!c || !table || !inv_freq) return CIS2_E_ARG;
  memcpy(table, c->table_dig, 32);
  memcpy(inv_freq, c->invf_dig, 32);
  return CIS2_OK;
}

int cis2_reset_seq(cis2_ctx* c, uint32_t seq) {
  if (!c || seq >= c->cfg.max_seqs) return CIS2_E_ARG;
  size_t per = (size_t)c->cfg.n_layers * 2 * c->kvd * c->cfg.max_pos;
  HIPCHK(c, hipMemsetAsync(c->kv + seq * per, 0, per * sizeof(float), c->st), "reset");
  HIPCHK(c, hipStreamSynchronize(c->st), "reset sync");
  return CIS2_OK;
}

int cis2_profile(cis2_ctx* c, int on) {
  if (!c) return CIS2_E_ARG;
  if (on && c->prof_ev.empty()) {
    c->prof_ev.assign(2 * kProfMax, nullptr);
    for (auto& e : c->prof_ev) HIPCHK(c, hipEventCreate(&e), "profile events");
  }
  if (on) c->prof_pos.clear();
  c->prof_on = on != 0;
  return CIS2_OK;
}

int cis2_recoveries(cis2_ctx* c, uint32_t* count) {
  if (!c || !count) return CIS2_E_ARG;
  *count = c->recoveries;
  return CIS2_OK;
}

int cis2_profile_read(cis2_ctx* c, uint64_t* launches, double* total_ms, uint32_t* positions,
                      uint64_t cap) {
  if (!c || !launches || !total_ms) return CIS2_E_ARG;
  const size_t n = c->prof_pos.size();
  double tot = 0.0;
  if (n) HIPCHK(c, hipEventSynchronize(c->prof_ev[2 * n - 1]), "profile sync");
  for (size_t i = 0; i < n; ++i) {
    float ms = 0.0f;
    HIPCHK(c, hipEventElapsedTime(&ms, c->prof_ev[2 * i], c->prof_ev[2 * i + 1]), "profile time");
    tot += ms;
    if (positions && i < cap) positions[i] = c->prof_pos[i];
  }
  *launches = n;
  *total_ms = tot;
  return CIS2_OK;
}

int cis2_trace_enable(cis2_ctx* c, cis2_trace_fn fn, void* user) {
  if (!c) return CIS2_E_ARG;
  c->trace = fn;
  c->trace_user = user;
  return CIS2_OK;
}

int cis2_forward(cis2_ctx* c, uint32_t n, const uint32_t* seq, const uint32_t* pos,
                 const uint32_t* tok, float* logits_host, uint32_t* argmax_out) {
  if (!c || !seq || !pos || !tok) return CIS2_E_ARG;
  int r = cis2_check_ready(c);
  if (r) return r;
  if (n > 1 && !c->trace) {  // all rows in one row-batched pass
    r = check_rows(c, n, seq, pos, tok);
    if (r) return r;
    std::vector<uint32_t> lr(n);
    for (uint32_t i = 0; i < n; ++i) lr[i] = i;
    r = forward_rows_host(c, n, seq, pos, tok, n, lr.data());
    if (r) return r;
    HIPCHK(c, hipStreamSynchronize(c->st), "rows sync");
    if (logits_host)
      HIPCHK(c, hipMemcpy(logits_host, c->rows.logits, (size_t)n * c->cfg.vocab * sizeof(float),
                          hipMemcpyDeviceToHost),
             "logits copy");
    if (argmax_out)
      HIPCHK(c, hipMemcpy(argmax_out, c->rows.arg, (size_t)n * 4, hipMemcpyDeviceToHost),
             "argmax copy");
    return check_err_flag(c);
  }
  const bool held = c->lock_fd >= 0;  // a decode session of this context holds the lock
  for (uint32_t i = 0; i < n; ++i) {
    if (seq[i] >= c->cfg.max_seqs) return fail(c, CIS2_E_ARG, "sequence index out of range");
    if (pos[i] >= c->cfg.max_pos) return fail(c, CIS2_E_RANGE, "position beyond max_pos");
    if (tok[i] >= c->cfg.vocab) return fail(c, CIS2_E_RANGE, "token id >= vocab");
    HIPCHK(c, hipMemcpyAsync(c->d_tok, &tok[i], 4, hipMemcpyHostToDevice, c->st), "token");
    bool ops = !use_fast(c);
    if (!ops) {
      decode_lock(c);
      r = forward_fast(c, seq[i], pos[i], c->d_tok, true);
      if (r) return r;
      HIPCHK(c, hipMemcpyAsync(c->d_tok + 1, c->d_tok, 4, hipMemcpyDeviceToDevice, c->st),
             "argmax copy");
      // a persistent launch that hit the spin cap: this row again on the
      // per-op path (it rewrites the position's K/V rows in every layer)
      uint32_t bits = 0;
      r = drain_and_clear_err(c, &bits);
      if (r) return r;
      if (bits & ~2u) HIPCHK(c, hipMemcpy(c->d_err, &bits, 4, hipMemcpyHostToDevice), "error flag");
      if (bits & 2u) {
        c->recoveries++;
        ops = true;
        HIPCHK(c, hipMemcpyAsync(c->d_tok, &tok[i], 4, hipMemcpyHostToDevice, c->st), "token");
      }
    }
    if (ops) {
      r = forward_one(c, seq[i], pos[i], c->d_tok, true);
      if (r) return r;
      if (argmax_out) LAUNCH(launch_argmax(c->logits, c->cfg.vocab, c->d_tok + 1, c->st), "argmax");
    }
    HIPCHK(c, hipStreamSynchronize(c->st), "forward sync");
    if (logits_host)
      HIPCHK(c, hipMemcpy(logits_host + (size_t)i * c->cfg.vocab, c->logits,
                          (size_t)c->cfg.vocab * sizeof(float), hipMemcpyDeviceToHost),
             "logits copy");
    if (argmax_out)
      HIPCHK(c, hipMemcpy(&argmax_out[i], c->d_tok + 1, 4, hipMemcpyDeviceToHost), "argmax copy");
  }
  if (!held) decode_unlock(c);
  return check_err_flag(c);
}

// Receipt header of a sampled decode (draft 14.5): "CIS2-SAMPLE-1", seed
// (u64 LE), temperature bits, top_k, top_p bits (u32 LE).
static void fold_sample_header(Sha256& w, const SampleParams& p) {
  w.update("CIS2-SAMPLE-1", 13);
  w.update_u32le((uint32_t)p.seed);
  w.update_u32le((uint32_t)(p.seed >> 32));
  uint32_t tb, pb;
  memcpy(&tb, &p.temperature, 4);
  memcpy(&pb, &p.top_p, 4);
  w.update_u32le(tb);
  w.update_u32le(p.top_k);
  w.update_u32le(pb);
}

int cis2_set_sampling(cis2_ctx* c, const cis2_sampling* sp) {
  if (!c) return CIS2_E_ARG;
  if (c->sess.active) return fail(c, CIS2_E_ARG, "sampling cannot change during a decode session");
  if (!sp || sp->mode == 0) {
    c->samp_on = false;
    return CIS2_OK;
  }
  const float T = sp->temperature, P = sp->top_p;
  if (sp->mode != 1 || !(T > 0.0f) || T == __builtin_inff() || !(P > 0.0f) || !(P <= 1.0f))
    return fail(c, CIS2_E_ARG, "invalid sampling parameters (mode 1, T finite > 0, top_p in (0,1])");
  const uint32_t V = c->cfg.vocab;
  SampleBufs& b = c->sbuf;
  if (b.V != V) {
    const uint32_t Vp = sample_sort_len(V);
    void *k = nullptr, *k2 = nullptr, *e = nullptr, *cd = nullptr, *nk = nullptr;
    if (hipMalloc(&k, (size_t)Vp * 8) != hipSuccess || hipMalloc(&k2, (size_t)Vp * 8) != hipSuccess ||
        hipMalloc(&e, (size_t)V * 4) != hipSuccess ||
        hipMalloc(&cd, (size_t)kSampleBlocks * 8) != hipSuccess || hipMalloc(&nk, 64) != hipSuccess) {
      for (void* q : {k, k2, e, cd, nk})
        if (q) (void)hipFree(q);
      return fail(c, CIS2_E_OOM, "sampling scratch");
    }
    for (void* q : {k, k2, e, cd, nk}) c->allocs.push_back(q);
    b.V = V;
    b.Vp = Vp;
    b.key = static_cast<uint64_t*>(k);
    b.key2 = static_cast<uint64_t*>(k2);
    b.e = static_cast<float*>(e);
    b.cand = static_cast<uint64_t*>(cd);
    b.nkeep = static_cast<uint32_t*>(nk);
  }
  c->samp = SampleParams{sp->seed, T, sp->top_k, P};
  c->samp_on = true;
  return CIS2_OK;
}

int cis2_sample_logits(cis2_ctx* c, const float* logits_host, uint32_t n, const uint32_t* steps,
                       uint32_t* ids_out, uint32_t* nkeep_out) {
  if (!c || !logits_host || !steps || !ids_out) return CIS2_E_ARG;
  if (!c->samp_on) return fail(c, CIS2_E_ARG, "sampling is not enabled (cis2_set_sampling)");
  if (c->sess.active) return fail(c, CIS2_E_ARG, "a decode session holds the logit buffer");
  const uint32_t V = c->cfg.vocab;
  for (uint32_t i = 0; i < n; ++i) {
    HIPCHK(c, hipMemcpyAsync(c->logits, logits_host + (size_t)i * V, (size_t)V * 4,
                             hipMemcpyHostToDevice, c->st),
           "logits upload");
    LAUNCH(launch_sample(c->logits, V, c->samp, steps[i], c->sbuf, c->d_tok + 1, c->d_err, c->st),
           "sample");
    HIPCHK(c, hipMemcpyAsync(&ids_out[i], c->d_tok + 1, 4, hipMemcpyDeviceToHost, c->st), "id copy");
    if (nkeep_out) {
      const uint32_t K = (c->samp.top_k > 0 && c->samp.top_k < V) ? c->samp.top_k : V;
      if (K == V && !(c->samp.top_p < 1.0f))
        nkeep_out[i] = V;
      else
        HIPCHK(c, hipMemcpyAsync(&nkeep_out[i], c->sbuf.nkeep, 4, hipMemcpyDeviceToHost, c->st),
               "nkeep copy");
    }
    HIPCHK(c, hipStreamSynchronize(c->st), "sample sync");
  }
  return check_err_flag(c);
}

int cis2_sample_logits_noalloc(cis2_ctx* c, const float* logits_dev, uint32_t n,
                               const uint32_t* steps, uint32_t* ids_dev, uint32_t* nkeep_dev) {
  if (!c) return CIS2_E_ARG;
  if (n == 0) return CIS2_OK;
  if (!logits_dev || !steps || !ids_dev) return fail(c, CIS2_E_ARG, "null argument");
  if (!c->samp_on) return fail(c, CIS2_E_ARG, "sampling is not enabled (cis2_set_sampling)");
  const uint32_t V = c->cfg.vocab;
  if (V > kNoAllocMaxVocab)
    return fail(c, CIS2_E_ARG, "vocabulary exceeds the no-allocation scratch (262144 entries)");
  std::mutex* mu = sample_scratch_lock(c->dev);
  if (!mu) return fail(c, CIS2_E_DEVICE, "device index out of range");
  // one draw at a time per GPU: the scratch is shared by every context there
  std::lock_guard<std::mutex> hold(*mu);
  SampleBufs b;
  uint32_t* err = nullptr;
  HIPCHK(c, sample_scratch_bufs(c->dev, V, &b, &err), "sampler scratch");
  // the scratch keeps the previous call's contents: only the error flag must
  // start at zero (every other word is written before it is read)
  LAUNCH(launch_fill_u32(err, 1, 0u, c->st), "clear error flag");
  for (uint32_t i = 0; i < n; ++i)
    LAUNCH(launch_sample(logits_dev + (size_t)i * V, V, c->samp, steps[i], b, ids_dev + i, err,
                         c->st, nkeep_dev ? nkeep_dev + i : nullptr),
           "sample");
  uint32_t flag = 0;
  HIPCHK(c, hipMemcpyAsync(&flag, err, 4, hipMemcpyDeviceToHost, c->st), "error flag");
  HIPCHK(c, hipStreamSynchronize(c->st), "sample sync");
  if (flag & 0x100u)
    return fail(c, CIS2_E_NUMERIC, "NaN among logits / temperature in a sampled draw");
  return CIS2_OK;
}

// Greedy decode + witness (code/cis2-fp/gpu/cis2_host.cpp:176-218).  The
// host enqueues step s, then folds step s - (kRing-1) while the GPU runs:
// argmax and the next token stay on the device, the logits stream to a
// pinned ring slot with an event per slot.
// Internal return of fold_step: the step's logits came from a persistent
// launch that hit the spin cap (recover_step redoes it).
constexpr int kNeedsRecovery = 1000;

static int fold_step(cis2_ctx* c) {
  Session& S = c->sess;
  const uint32_t V = c->cfg.vocab;
  const uint32_t step = S.folded;
  const int slot = step % kRing;
  HIPCHK(c, hipEventSynchronize(c->ring_ev[slot]), "ring wait");
  // the error word as it stood after the pass that produced these logits
  if (S.fast && (c->ring_tok[slot * 2 + 1] & 2u)) return kNeedsRecovery;
  const float* lg = c->ring + (size_t)slot * V;
  const uint32_t nid = c->ring_tok[slot * 2];
  S.w.update(lg, (size_t)V * sizeof(float));
  S.w.update_u32le(nid);
  sha256(lg, (size_t)V * sizeof(float), S.step_dig.data() + 32 * (size_t)step);
  S.ids[S.n_prompt + step] = nid;
  S.folded++;
  return CIS2_OK;
}

// Step `step`'s logits came from a persistent launch that hit the spin cap
// (its grid was not all resident at once: another process's work held
// CUs).  Every later launch of the session read a token that launch never
// wrote, so all of them are discarded: once the queues are drained and the
// error word cleared, the position before `step` is recomputed on the
// per-op path (same arithmetic, so the same bits; it rewrites that
// position's K/V rows in every layer), and the session continues from
// `step` on the per-op path, which recomputes every later position as it
// re-enqueues it.
static int recover_step(cis2_ctx* c, uint32_t step) {
  Session& S = c->sess;
  uint32_t bits = 0;
  int r = drain_and_clear_err(c, &bits);
  if (r) return r;
  if (bits & ~2u)
    return fail(c, (bits & 0x100u) ? CIS2_E_NUMERIC : CIS2_E_RANGE,
                "device error during a recovered decode step");
  S.fast = false;
  c->recoveries++;
  const uint32_t pos = S.n_prompt + step - 1;  // step >= 1: step 0 comes from the prefill
  HIPCHK(c, hipMemcpyAsync(c->d_tok, &S.ids[pos], 4, hipMemcpyHostToDevice, c->st), "token");
  r = forward_one(c, S.seq, pos, c->d_tok, true);
  if (r) return r;
  HIPCHK(c, hipStreamSynchronize(c->st), "recovery sync");
  S.enqueued = step;
  S.folded = step;
  return check_err_flag(c);
}

int cis2_decode_begin(cis2_ctx* c, uint32_t seq, const uint32_t* prompt, uint32_t n_prompt,
                      uint32_t max_steps, const uint8_t hdr[96]) {
  if (!c || !prompt || !hdr) return CIS2_E_ARG;
  if (n_prompt == 0 || seq >= c->cfg.max_seqs) return fail(c, CIS2_E_ARG, "bad prompt or seq");
  if ((uint64_t)n_prompt + max_steps > c->cfg.max_pos)
    return fail(c, CIS2_E_RANGE, "prompt + gen_toks exceeds max_pos");
  for (uint32_t i = 0; i < n_prompt; ++i)
    if (prompt[i] >= c->cfg.vocab) return fail(c, CIS2_E_RANGE, "prompt token id >= vocab");
  int r = cis2_check_ready(c);
  if (r) return r;
  r = cis2_reset_seq(c, seq);
  if (r) return r;
  decode_unlock(c);  // a session left without cis2_decode_end
  Session& S = c->sess;
  S = Session();
  S.seq = seq;
  S.n_prompt = n_prompt;
  S.max_steps = max_steps;
  S.ids.assign(prompt, prompt + n_prompt);
  S.ids.resize((size_t)n_prompt + max_steps);
  S.step_dig.assign(32 * (size_t)max_steps, 0);
  S.w.update(hdr, 96);
  S.w.update(c->table_dig, 32);
  S.w.update(c->invf_dig, 32);
  for (uint32_t i = 0; i < n_prompt; ++i) S.w.update_u32le(prompt[i]);
  if (c->samp_on) fold_sample_header(S.w, c->samp);
  // Prefill: every prompt position; only the last needs its logits.
  HIPCHK(c, hipMemcpy(c->d_prompt, prompt, (size_t)n_prompt * 4, hipMemcpyHostToDevice),
         "prompt upload");
  S.fast = use_fast(c);
  if (S.fast) decode_lock(c);
  if (n_prompt > 1 && !c->trace && !c->seq_prefill) {
    // all prompt positions in one row-batched pass (bit-identical to the
    // position-by-position prefill); the last row's logits and argmax go
    // where the decode steps expect them
    std::vector<uint32_t> sq(n_prompt, seq), ps(n_prompt);
    for (uint32_t p = 0; p < n_prompt; ++p) ps[p] = p;
    const uint32_t last = n_prompt - 1;
    r = forward_rows_host(c, n_prompt, sq.data(), ps.data(), prompt, 1, &last);
    if (r) return r;
    HIPCHK(c, hipMemcpyAsync(c->logits, c->rows.logits, (size_t)c->cfg.vocab * sizeof(float),
                             hipMemcpyDeviceToDevice, c->st),
           "prefill logits");
    HIPCHK(c, hipMemcpyAsync(c->d_tok, c->rows.arg, 4, hipMemcpyDeviceToDevice, c->st),
           "prefill argmax");
  } else {
    for (int pass = 0; pass < 2; ++pass) {
      for (uint32_t p = 0; p < n_prompt; ++p) {
        r = S.fast ? forward_fast(c, seq, p, c->d_prompt + p, p + 1 == n_prompt)
                   : forward_one(c, seq, p, c->d_prompt + p, p + 1 == n_prompt);
        if (r) return r;
      }
      if (!S.fast) break;
      // a persistent prefill launch that hit the spin cap: the whole prompt
      // again on the per-op path (each position rewrites its K/V rows)
      uint32_t bits = 0;
      r = drain_and_clear_err(c, &bits);
      if (r) return r;
      if (!(bits & 2u)) {
        if (bits) HIPCHK(c, hipMemcpy(c->d_err, &bits, 4, hipMemcpyHostToDevice), "error flag");
        break;
      }
      S.fast = false;
      c->recoveries++;
    }
  }
  HIPCHK(c, hipStreamSynchronize(c->st), "prefill sync");
  S.active = true;
  return check_err_flag(c);
}

int cis2_decode_steps(cis2_ctx* c, uint32_t n) {
  if (!c) return CIS2_E_ARG;
  Session& S = c->sess;
  if (!S.active) return fail(c, CIS2_E_ARG, "no decode session");
  if ((uint64_t)S.enqueued + n > S.max_steps) return fail(c, CIS2_E_RANGE, "steps beyond max_steps");
  const uint32_t V = c->cfg.vocab;
  const uint32_t target = S.enqueued + n;
  hipStream_t s = c->st;
  int r = CIS2_OK;
  if (S.fast && !c->trace && !c->cs)
    HIPCHK(c, hipStreamCreateWithFlags(&c->cs, hipStreamNonBlocking), "copy stream");
  // one fold: 0 folded, 1 a recovery reset the session to an earlier step
  // (the loops restart from there), -1 error (in r)
  auto fold = [&]() -> int {
    r = fold_step(c);
    if (r == kNeedsRecovery) {
      r = recover_step(c, S.folded);
      return r ? -1 : 1;
    }
    return r ? -1 : 0;
  };
  while (true) {
    bool restart = false;
    while (S.enqueued < target && !restart) {
      // Persistent-kernel steps alternate between two logit buffers and two
      // token slots: step t's logits and token (set t % 2) are copied to the
      // host ring on the copy stream while pass t (which writes set
      // (t+1) % 2) runs; pass t waits only for the copy of step t-1, whose
      // set it overwrites.  The per-op path keeps one set and copies in
      // stream order.
      const bool alt = S.fast && !c->trace;
      const uint32_t step = S.enqueued;
      const int slot = step % kRing;
      if (step >= S.folded + kRing) {  // slot reuse: fold what it held first
        const int f = fold();
        if (f < 0) return r;
        if (f > 0) {
          restart = true;
          break;
        }
      }
      const bool odd = alt && (step & 1);
      float* lcur = odd ? c->logits2 : c->logits;
      float* lnext = alt ? (odd ? c->logits : c->logits2) : c->logits;
      uint32_t* tcur = odd ? c->d_tok2 : c->d_tok;
      uint32_t* tnext = alt ? (odd ? c->d_tok : c->d_tok2) : c->d_tok;
      // the persistent kernel already left the argmax of these logits in the
      // token slot; a sampled draw replaces it (generation step = this step)
      if (c->samp_on)
        LAUNCH(launch_sample(lcur, V, c->samp, step, c->sbuf, tcur, c->d_err, s), "sample");
      else if (!S.fast)
        LAUNCH(launch_argmax(c->logits, V, c->d_tok, s), "argmax");
      hipStream_t cp = alt ? c->cs : s;
      if (alt) {
        HIPCHK(c, hipEventRecord(c->ring_ready[slot], s), "step event");
        HIPCHK(c, hipStreamWaitEvent(cp, c->ring_ready[slot], 0), "copy wait");
      }
      HIPCHK(c, hipMemcpyAsync(c->ring + (size_t)slot * V, lcur, (size_t)V * sizeof(float),
                               hipMemcpyDeviceToHost, cp),
             "logits d2h");
      HIPCHK(c, hipMemcpyAsync(c->ring_tok + slot * 2, tcur, 4, hipMemcpyDeviceToHost, cp),
             "token d2h");
      // the error word after the pass that produced these logits
      HIPCHK(c, hipMemcpyAsync(c->ring_tok + slot * 2 + 1, c->d_err, 4, hipMemcpyDeviceToHost,
                               cp),
             "error d2h");
      HIPCHK(c, hipEventRecord(c->ring_ev[slot], cp), "ring event");
      if (alt && step > 0)  // set (step+1) % 2 held step-1's results: copied by now
        HIPCHK(c, hipStreamWaitEvent(s, c->ring_ev[(step - 1) % kRing], 0), "set reuse wait");
      r = S.fast ? forward_fast(c, S.seq, S.n_prompt + step, tcur, true, lnext, tnext)
                 : forward_one(c, S.seq, S.n_prompt + step, c->d_tok, true);
      if (r) return r;
      S.enqueued++;
    }
    while (!restart && S.folded < S.enqueued) {
      const int f = fold();
      if (f < 0) return r;
      restart = f > 0;
    }
    if (restart) continue;
    HIPCHK(c, hipStreamSynchronize(s), "decode sync");
    if (S.fast && S.enqueued > 0) {
      // the last pass (whose logits the next call folds) hit the spin cap
      uint32_t e = 0;
      HIPCHK(c, hipMemcpy(&e, c->d_err, 4, hipMemcpyDeviceToHost), "error flag");
      if (e & 2u) {
        r = recover_step(c, S.enqueued);
        if (r) return r;
        continue;  // S.enqueued == target: the loops fall through to here
      }
    }
    return check_err_flag(c);
  }
}

int cis2_decode_end(cis2_ctx* c, uint32_t* out_ids, uint8_t witness[32],
                    uint8_t argmax_digest[32], uint8_t* step_digests) {
  if (!c || !out_ids || !witness || !argmax_digest) return CIS2_E_ARG;
  Session& S = c->sess;
  if (!S.active) return fail(c, CIS2_E_ARG, "no decode session");
  while (S.folded < S.enqueued) {
    int r = fold_step(c);
    if (r) return r;
  }
  S.active = false;
  decode_unlock(c);
  const uint32_t total = S.n_prompt + S.enqueued;
  S.w.finish(witness);
  Sha256 a;
  for (uint32_t i = 0; i < total; ++i) a.update_u32le(S.ids[i]);
  a.finish(argmax_digest);
  memcpy(out_ids, S.ids.data(), (size_t)total * 4);
  if (step_digests) memcpy(step_digests, S.step_dig.data(), 32 * (size_t)S.enqueued);
  return CIS2_OK;
}

int cis2_decode(cis2_ctx* c, uint32_t seq, const uint32_t* prompt, uint32_t n_prompt,
                uint32_t gen_toks, const uint8_t hdr[96], uint32_t* out_ids, uint8_t witness[32],
                uint8_t argmax_digest[32], uint8_t* step_digests) {
  if (!c || !prompt || !hdr || !out_ids || !witness || !argmax_digest) return CIS2_E_ARG;
  int r = cis2_decode_begin(c, seq, prompt, n_prompt, gen_toks, hdr);
  if (!r) r = cis2_decode_steps(c, gen_toks);
  if (!r) r = cis2_decode_end(c, out_ids, witness, argmax_digest, step_digests);
  c->sess.active = false;
  if (c->st) (void)hipStreamSynchronize(c->st);
  decode_unlock(c);
  return r;
}

// The generation steps of decode_group, after its prefill has left logit
// set 0 (each sequence's last prompt row) in rb.logits / rb.arg.  Logit set
// t (t >= 1) comes from a rows pass over row b = sequence b at position
// lens[b] + t - 1 whose input tokens are set t-1's argmax ids.  Sets
// alternate between two device buffers, so pass t runs while set t-1 is
// copied to pinned host memory on a second stream and folded into the
// witnesses on the host; pass t+1 waits only for the copy of set t-1 (the
// buffer it overwrites).  Both passes are captured once as HIP graphs
// (CIS2_GRAPH=0: launched op by op); the positions advance on the device
// at the end of each pass.
static int decode_steps(cis2_ctx* c, uint32_t G, const uint32_t* lens, const uint32_t* off,
                        uint32_t gen, std::vector<Sha256>& w, std::vector<Sha256>& a,
                        uint32_t* out_ids) {
  const uint32_t V = c->cfg.vocab;
  RowsBuf& rb = c->rows;
  int rc = rows_reserve(c, G, G);
  if (rc) return rc;
  if (G > rb.cap2) {
    HIPCHK(c, hipStreamSynchronize(c->st), "rows sync");
    for (void* p : rb.mem2) (void)hipFree(p);
    rb.mem2.clear();
    rb.cap2 = 0;
    if (!(rb.logits2 = rows_alloc<float>(rb.mem2, (size_t)G * V)) ||
        !(rb.arg2 = rows_alloc<uint32_t>(rb.mem2, G)))
      return fail(c, CIS2_E_OOM, "second logit buffer");
    rb.cap2 = G;
  }
  if (!c->cs) HIPCHK(c, hipStreamCreateWithFlags(&c->cs, hipStreamNonBlocking), "copy stream");
  // buffer of set t: (t + 1) & 1; set 0 is the prefill's
  float* logb[2] = {rb.logits2, rb.logits};
  uint32_t* argb[2] = {rb.arg2, rb.arg};
  std::vector<uint32_t> dseq(G), dpos(G), ident(G);
  uint32_t max_len = 0;
  for (uint32_t b = 0; b < G; ++b) {
    dseq[b] = b;
    ident[b] = b;
    dpos[b] = lens[b];
    max_len = std::max(max_len, lens[b] + gen - 1);  // the last pass's largest pos + 1
  }
  HIPCHK(c, hipMemcpyAsync(rb.seq, dseq.data(), (size_t)G * 4, hipMemcpyHostToDevice, c->st),
         "rows upload");
  HIPCHK(c, hipMemcpyAsync(rb.lrows, ident.data(), (size_t)G * 4, hipMemcpyHostToDevice, c->st),
         "rows upload");
  HIPCHK(c, hipMemcpyAsync(rb.pos, dpos.data(), (size_t)G * 4, hipMemcpyHostToDevice, c->st),
         "rows upload");
  // one pass into buffer j: tokens from buffer 1 - j
  auto pass = [&](uint32_t j) -> int {
    int r = forward_rows(c, G, argb[1 - j], max_len, G, logb[j], argb[j], 0, true);
    if (r) return r;
    HIPCHK(c, launch_advance_rows(rb.pos, G, c->st), "rows advance");
    return CIS2_OK;
  };
  hipGraphExec_t gx[2] = {nullptr, nullptr};
  const char* ge = getenv("CIS2_GRAPH");
  bool graphs = gen > 1 && !(ge && ge[0] == '0');
  for (uint32_t j = 0; j < 2 && graphs; ++j) {
    if (hipStreamBeginCapture(c->st, hipStreamCaptureModeThreadLocal) != hipSuccess) {
      graphs = false;
      break;
    }
    const int r = pass(j);
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(c->st, &g);
    if (r == CIS2_OK && e == hipSuccess && g &&
        hipGraphInstantiate(&gx[j], g, nullptr, nullptr, 0) != hipSuccess)
      gx[j] = nullptr;
    if (g) (void)hipGraphDestroy(g);
    if (!gx[j]) {  // not capturable here: launch op by op
      (void)hipGetLastError();
      c->err.clear();
      graphs = false;
    }
  }
  float* host = nullptr;
  uint32_t* hid = nullptr;
  hipEvent_t evd[2] = {nullptr, nullptr}, evc[2] = {nullptr, nullptr};
  if (hipHostMalloc((void**)&host, 2 * (size_t)G * V * sizeof(float), 0) != hipSuccess ||
      hipHostMalloc((void**)&hid, 2 * (size_t)G * 4, 0) != hipSuccess)
    rc = fail(c, CIS2_E_OOM, "pinned logits");
  for (int i = 0; i < 2 && rc == CIS2_OK; ++i)
    if (hipEventCreateWithFlags(&evd[i], hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&evc[i], hipEventDisableTiming) != hipSuccess)
      rc = fail(c, CIS2_E_DEVICE, "event create");
  // waits for set t's copy and folds it into the witnesses
  auto consume = [&](uint32_t t) -> int {
    const uint32_t j = (t + 1) & 1;
    if (hipEventSynchronize(evc[j]) != hipSuccess) return fail(c, CIS2_E_DEVICE, "logits wait");
    const float* hl = host + (size_t)j * G * V;
    const uint32_t* hi = hid + (size_t)j * G;
    fold_rows(w, hl, hi, G, V);
    for (uint32_t b = 0; b < G; ++b) {
      a[b].update_u32le(hi[b]);
      out_ids[off[b] + (size_t)b * gen + lens[b] + t] = hi[b];
    }
    return CIS2_OK;
  };
  for (uint32_t t = 0; t < gen && rc == CIS2_OK; ++t) {
    const uint32_t j = (t + 1) & 1;
    if (t >= 1) {
      if (t >= 2 && hipStreamWaitEvent(c->st, evc[j], 0) != hipSuccess) {
        rc = fail(c, CIS2_E_DEVICE, "copy wait");
        break;
      }
      if (graphs) {
        if (hipGraphLaunch(gx[j], c->st) != hipSuccess) {
          rc = fail(c, CIS2_E_DEVICE, "graph launch");
          break;
        }
      } else if ((rc = pass(j)) != CIS2_OK) {
        break;
      }
    }
    if (hipEventRecord(evd[j], c->st) != hipSuccess ||
        hipStreamWaitEvent(c->cs, evd[j], 0) != hipSuccess ||
        hipMemcpyAsync(host + (size_t)j * G * V, logb[j], (size_t)G * V * sizeof(float),
                       hipMemcpyDeviceToHost, c->cs) != hipSuccess ||
        hipMemcpyAsync(hid + (size_t)j * G, argb[j], (size_t)G * 4, hipMemcpyDeviceToHost,
                       c->cs) != hipSuccess ||
        hipEventRecord(evc[j], c->cs) != hipSuccess) {
      rc = fail(c, CIS2_E_DEVICE, "logits copy");
      break;
    }
    if (t >= 1) rc = consume(t - 1);
  }
  if (rc == CIS2_OK) rc = consume(gen - 1);
  // drain both streams before the pinned buffers go
  if (hipStreamSynchronize(c->st) != hipSuccess && rc == CIS2_OK)
    rc = fail(c, CIS2_E_DEVICE, "decode sync");
  if (hipStreamSynchronize(c->cs) != hipSuccess && rc == CIS2_OK)
    rc = fail(c, CIS2_E_DEVICE, "copy sync");
  for (int i = 0; i < 2; ++i) {
    if (evd[i]) (void)hipEventDestroy(evd[i]);
    if (evc[i]) (void)hipEventDestroy(evc[i]);
    if (gx[i]) (void)hipGraphExecDestroy(gx[i]);
  }
  if (host) (void)hipHostFree(host);
  if (hid) (void)hipHostFree(hid);
  return rc;
}

// Greedy decode of `G` sequences (cache slots 0..G-1) in row-batched
// passes: one prefill over every prompt position of every sequence, then
// one row per sequence per step.  Per sequence, the witness and argmax
// digest are built exactly as cis2_decode builds them.
static int decode_group(cis2_ctx* c, uint32_t G, const uint32_t* prompts, const uint32_t* lens,
                        uint32_t gen, const uint8_t hdr[96], uint32_t* out_ids, uint8_t* witness,
                        uint8_t* argmax_digest) {
  const uint32_t V = c->cfg.vocab;
  std::vector<uint32_t> seq, pos, tok, lrows(G), off(G + 1, 0);
  for (uint32_t b = 0; b < G; ++b) {
    if (lens[b] == 0) return fail(c, CIS2_E_ARG, "empty prompt");
    if ((uint64_t)lens[b] + gen > c->cfg.max_pos)
      return fail(c, CIS2_E_RANGE, "prompt + gen_toks exceeds max_pos");
    off[b + 1] = off[b] + lens[b];
    for (uint32_t p = 0; p < lens[b]; ++p) {
      if (prompts[off[b] + p] >= V) return fail(c, CIS2_E_RANGE, "prompt token id >= vocab");
      seq.push_back(b);
      pos.push_back(p);
      tok.push_back(prompts[off[b] + p]);
    }
    lrows[b] = off[b + 1] - 1;
  }
  for (uint32_t b = 0; b < G; ++b) {
    int r = cis2_reset_seq(c, b);
    if (r) return r;
  }
  std::vector<Sha256> w(G), a(G);
  for (uint32_t b = 0; b < G; ++b) {
    w[b].update(hdr, 96);
    w[b].update(c->table_dig, 32);
    w[b].update(c->invf_dig, 32);
    for (uint32_t p = 0; p < lens[b]; ++p) {
      w[b].update_u32le(prompts[off[b] + p]);
      a[b].update_u32le(prompts[off[b] + p]);
    }
  }
  // prefill: all prompt rows; logits of each sequence's last prompt row
  int r = forward_rows_host(c, (uint32_t)seq.size(), seq.data(), pos.data(), tok.data(), G,
                            lrows.data());
  if (r) return r;
  if (gen == 0) {
    HIPCHK(c, hipStreamSynchronize(c->st), "prefill sync");
  } else {
    r = decode_steps(c, G, lens, off.data(), gen, w, a, out_ids);
    if (r) return r;
  }
  for (uint32_t b = 0; b < G; ++b) {
    memcpy(out_ids + off[b] + (size_t)b * gen, prompts + off[b], (size_t)lens[b] * 4);
    w[b].finish(witness + 32 * (size_t)b);
    a[b].finish(argmax_digest + 32 * (size_t)b);
  }
  return check_err_flag(c);
}

int cis2_decode_batch(cis2_ctx* c, uint32_t nseq, const uint32_t* prompts,
                      const uint32_t* prompt_lens, uint32_t gen_toks, const uint8_t hdr[96],
                      uint32_t* out_ids, uint8_t* witness, uint8_t* argmax_digest) {
  if (!c || !prompts || !prompt_lens || !hdr || !out_ids || !witness || !argmax_digest)
    return CIS2_E_ARG;
  if (c->samp_on) return fail(c, CIS2_E_UNSUPPORTED, "the batched decode is greedy only");
  int r = cis2_check_ready(c);
  if (r) return r;
  size_t in_off = 0, out_off = 0;
  if (nseq == 1 || c->trace) {  // one sequence (or tracing): the single-row path
    for (uint32_t b = 0; b < nseq; ++b) {
      r = cis2_decode(c, b % c->cfg.max_seqs, prompts + in_off, prompt_lens[b], gen_toks, hdr,
                      out_ids + out_off, witness + 32 * (size_t)b,
                      argmax_digest + 32 * (size_t)b, nullptr);
      if (r) return r;
      in_off += prompt_lens[b];
      out_off += (size_t)prompt_lens[b] + gen_toks;
    }
    return CIS2_OK;
  }
  // groups of up to max_seqs sequences, one KV-cache slot each
  for (uint32_t b0 = 0; b0 < nseq; b0 += c->cfg.max_seqs) {
    const uint32_t G = std::min(c->cfg.max_seqs, nseq - b0);
    r = decode_group(c, G, prompts + in_off, prompt_lens + b0, gen_toks, hdr, out_ids + out_off,
                     witness + 32 * (size_t)b0, argmax_digest + 32 * (size_t)b0);
    if (r) return r;
    for (uint32_t b = 0; b < G; ++b) {
      in_off += prompt_lens[b0 + b];
      out_off += (size_t)prompt_lens[b0 + b] + gen_toks;
    }
  }
  return CIS2_OK;
}

// Teacher-forced verification of a claimed continuation in one row-batched
// pass (code/cis2-fp/verify3/model.c:923-1005): the rows are positions
// 0 .. n_prompt + n_gen - 2 of sequence `seq` fed prompt ++ claimed; the
// logits of position n_prompt - 1 + s predict claimed[s].  Witness and
// argmax digest fold each step's logits and their argmax (not the claimed
// id), as the reference does; first_mismatch is the first s whose argmax
// differs from claimed[s], or -1.
int cis2_verify_prefill(cis2_ctx* c, uint32_t seq, const uint32_t* prompt, uint32_t n_prompt,
                        const uint32_t* claimed, uint32_t n_gen, const uint8_t hdr[96],
                        uint32_t* generated, uint8_t witness[32], uint8_t argmax_digest[32],
                        int64_t* first_mismatch, float* logits_host) {
  if (!c || !prompt || (n_gen && !claimed) || !hdr || (n_gen && !generated) || !witness ||
      !argmax_digest || !first_mismatch)
    return CIS2_E_ARG;
  if (c->samp_on) return fail(c, CIS2_E_UNSUPPORTED, "the teacher-forced verifier is greedy only");
  if (n_prompt == 0 || seq >= c->cfg.max_seqs) return fail(c, CIS2_E_ARG, "bad prompt or seq");
  if ((uint64_t)n_prompt + n_gen > (uint64_t)c->cfg.max_pos + 1)
    return fail(c, CIS2_E_RANGE, "prompt + claimed tokens exceed max_pos");
  const uint32_t V = c->cfg.vocab;
  for (uint32_t i = 0; i < n_prompt; ++i)
    if (prompt[i] >= V) return fail(c, CIS2_E_RANGE, "prompt token id >= vocab");
  for (uint32_t i = 0; i < n_gen; ++i)
    if (claimed[i] >= V) return fail(c, CIS2_E_RANGE, "claimed token id >= vocab");
  int r = cis2_check_ready(c);
  if (r) return r;
  r = cis2_reset_seq(c, seq);
  if (r) return r;
  *first_mismatch = -1;
  Sha256 w, a;
  w.update(hdr, 96);
  w.update(c->table_dig, 32);
  w.update(c->invf_dig, 32);
  for (uint32_t i = 0; i < n_prompt; ++i) {
    w.update_u32le(prompt[i]);
    a.update_u32le(prompt[i]);
  }
  if (n_gen) {
    const uint32_t n = n_prompt + n_gen - 1;
    std::vector<uint32_t> sq(n, seq), ps(n), tk(n), lr(n_gen);
    for (uint32_t p = 0; p < n; ++p) {
      ps[p] = p;
      tk[p] = p < n_prompt ? prompt[p] : claimed[p - n_prompt];
    }
    for (uint32_t s = 0; s < n_gen; ++s) lr[s] = n_prompt - 1 + s;
    r = forward_rows_host(c, n, sq.data(), ps.data(), tk.data(), n_gen, lr.data());
    if (r) return r;
    std::vector<float> lg((size_t)n_gen * V);
    HIPCHK(c, hipStreamSynchronize(c->st), "prefill sync");
    HIPCHK(c, hipMemcpy(lg.data(), c->rows.logits, lg.size() * sizeof(float),
                        hipMemcpyDeviceToHost),
           "logits copy");
    HIPCHK(c, hipMemcpy(generated, c->rows.arg, (size_t)n_gen * 4, hipMemcpyDeviceToHost),
           "argmax copy");
    for (uint32_t s = 0; s < n_gen; ++s) {
      w.update(lg.data() + (size_t)s * V, (size_t)V * sizeof(float));
      w.update_u32le(generated[s]);
      a.update_u32le(generated[s]);
      if (*first_mismatch < 0 && generated[s] != claimed[s]) *first_mismatch = s;
    }
    if (logits_host) memcpy(logits_host, lg.data(), lg.size() * sizeof(float));
  }
  w.finish(witness);
  a.finish(argmax_digest);
  return check_err_flag(c);
}

// ---- standalone GEMV ------------------------------------------------------

int cis2_gemv_plan_create(uint32_t M, uint32_t K, uint32_t copies, const float* W,
                          cis2_gemv_plan** out) {
  if (!W || !out || M == 0 || K == 0 || K % 4 || copies == 0) return CIS2_E_ARG;
  if (gemv_blk_lds_bytes(K, kPlanR) > 160 * 1024 - 64) return CIS2_E_UNSUPPORTED;
  cis2_gemv_plan* p = new cis2_gemv_plan();
  p->M = M; p->K = K; p->copies = copies;
  const size_t per = blocked_floats(M, K, kPlanR);
  float* rowmajor = nullptr;
  hipError_t e = hipStreamCreateWithFlags(&p->st, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipMalloc(&p->W, per * copies * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&p->x, (size_t)K * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&p->y, ((size_t)M + 64) * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&rowmajor, (size_t)M * K * sizeof(float));
  if (e == hipSuccess) e = hipMemcpy(rowmajor, W, (size_t)M * K * sizeof(float), hipMemcpyHostToDevice);
  for (uint32_t i = 0; e == hipSuccess && i < copies; ++i)
    e = launch_relayout(rowmajor, p->W + per * i, M, K, kPlanR, p->st);
  if (e == hipSuccess) e = hipStreamSynchronize(p->st);
  if (e == hipSuccess) e = hipEventCreate(&p->e0);
  if (e == hipSuccess) e = hipEventCreate(&p->e1);
  if (rowmajor) (void)hipFree(rowmajor);
  if (e != hipSuccess) {
    cis2_gemv_plan_destroy(p);
    return e == hipErrorOutOfMemory ? CIS2_E_OOM : CIS2_E_DEVICE;
  }
  *out = p;
  return CIS2_OK;
}

// One GEMV of the plan on replica c.  A matrix of many row blocks (an LM
// head: more than two blocks per CU) streams through the batch kernel,
// whose workgroups share CUs so one block's loads overlap another's chains;
// a smaller one runs the pipelined lone-GEMV kernel, one block per CU.
static hipError_t plan_launch(cis2_gemv_plan* p, uint32_t c, const float* x, float* y) {
  const size_t per = blocked_floats(p->M, p->K, kPlanR);
  if ((p->M + kPlanR - 1) / kPlanR > kPlanStreamBlocks)
    return launch_gemv_many(p->W, per, p->copies, c % p->copies, 1, x, y, p->M, p->K, kPlanR,
                            p->st);
  return launch_gemv_blk(p->W + per * (c % p->copies), x, y, p->M, p->K, kPlanR, p->st);
}

int cis2_gemv_plan_run(cis2_gemv_plan* p, const float* x, float* y) {
  if (!p || !x || !y) return CIS2_E_ARG;
  hipError_t e = hipMemcpyAsync(p->x, x, (size_t)p->K * sizeof(float), hipMemcpyHostToDevice, p->st);
  if (e == hipSuccess) e = plan_launch(p, 0, p->x, p->y);
  if (e == hipSuccess) e = hipMemcpyAsync(y, p->y, (size_t)p->M * sizeof(float), hipMemcpyDeviceToHost, p->st);
  if (e == hipSuccess) e = hipStreamSynchronize(p->st);
  return e == hipSuccess ? CIS2_OK : CIS2_E_DEVICE;
}

int cis2_gemv_plan_time(cis2_gemv_plan* p, uint32_t iters, float* ms) {
  if (!p || !ms || iters == 0) return CIS2_E_ARG;
  hipError_t e = hipSuccess;
  for (uint32_t i = 0; e == hipSuccess && i < p->copies; ++i)  // warm-up pass
    e = plan_launch(p, i, p->x, p->y);
  if (e == hipSuccess) e = hipEventRecord(p->e0, p->st);
  for (uint32_t i = 0; e == hipSuccess && i < iters; ++i) e = plan_launch(p, i, p->x, p->y);
  if (e == hipSuccess) e = hipEventRecord(p->e1, p->st);
  if (e == hipSuccess) e = hipEventSynchronize(p->e1);
  float t = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&t, p->e0, p->e1);
  if (e != hipSuccess) return CIS2_E_DEVICE;
  *ms = t / (float)iters;
  return CIS2_OK;
}

// Device buffers for n GEMVs' inputs and outputs.
static hipError_t plan_reserve(cis2_gemv_plan* p, uint32_t n) {
  if (n <= p->ncap) return hipSuccess;
  hipError_t e = hipStreamSynchronize(p->st);
  if (p->xb) (void)hipFree(p->xb);
  if (p->yb) (void)hipFree(p->yb);
  p->xb = p->yb = nullptr;
  p->ncap = 0;
  if (e == hipSuccess) e = hipMalloc(&p->xb, (size_t)n * p->K * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&p->yb, (size_t)n * p->M * sizeof(float) + 256);
  if (e == hipSuccess) {
    p->ncap = n;
    // defined inputs for the timing runs
    e = hipMemsetAsync(p->xb, 0, (size_t)n * p->K * sizeof(float), p->st);
  }
  return e;
}

int cis2_gemv_plan_run_batch(cis2_gemv_plan* p, uint32_t n, const float* x, float* y) {
  if (!p || (n && (!x || !y)) || n > 65535) return CIS2_E_ARG;
  if (n == 0) return CIS2_OK;
  hipError_t e = plan_reserve(p, n);
  if (e == hipSuccess)
    e = hipMemcpyAsync(p->xb, x, (size_t)n * p->K * sizeof(float), hipMemcpyHostToDevice, p->st);
  if (e == hipSuccess)
    e = launch_gemv_many(p->W, blocked_floats(p->M, p->K, kPlanR), p->copies, 0, n, p->xb, p->yb,
                         p->M, p->K, kPlanR, p->st);
  if (e == hipSuccess)
    e = hipMemcpyAsync(y, p->yb, (size_t)n * p->M * sizeof(float), hipMemcpyDeviceToHost, p->st);
  if (e == hipSuccess) e = hipStreamSynchronize(p->st);
  return e == hipSuccess ? CIS2_OK : (e == hipErrorOutOfMemory ? CIS2_E_OOM : CIS2_E_DEVICE);
}

int cis2_gemv_plan_time_batch(cis2_gemv_plan* p, uint32_t n, uint32_t iters, float* ms) {
  if (!p || !ms || iters == 0 || n == 0 || n > 65535) return CIS2_E_ARG;
  const uint64_t per = blocked_floats(p->M, p->K, kPlanR);
  hipError_t e = plan_reserve(p, n);
  auto launch = [&](uint32_t it) {
    return launch_gemv_many(p->W, per, p->copies, (uint32_t)(((uint64_t)it * n) % p->copies), n,
                            p->xb, p->yb, p->M, p->K, kPlanR, p->st);
  };
  if (e == hipSuccess) e = launch(0);  // warm-up
  if (e == hipSuccess) e = hipEventRecord(p->e0, p->st);
  for (uint32_t i = 0; e == hipSuccess && i < iters; ++i) e = launch(i + 1);
  if (e == hipSuccess) e = hipEventRecord(p->e1, p->st);
  if (e == hipSuccess) e = hipEventSynchronize(p->e1);
  float t = 0.0f;
  if (e == hipSuccess) e = hipEventElapsedTime(&t, p->e0, p->e1);
  if (e != hipSuccess) return e == hipErrorOutOfMemory ? CIS2_E_OOM : CIS2_E_DEVICE;
  *ms = t / (float)iters;
  return CIS2_OK;
}

void cis2_gemv_plan_destroy(cis2_gemv_plan* p) {
  if (!p) return;
  if (p->st) (void)hipStreamSynchronize(p->st);
  if (p->xb) (void)hipFree(p->xb);
  if (p->yb) (void)hipFree(p->yb);
  if (p->W) (void)hipFree(p->W);
  if (p->x) (void)hipFree(p->x);
  if (p->y) (void)hipFree(p->y);
  if (p->e0) (void)hipEventDestroy(p->e0);
  if (p->e1) (void)hipEventDestroy(p->e1);
  if (p->st) (void)hipStreamDestroy(p->st);
  delete p;
}

// ---- verification hooks -----------------------------------------------------

int cis2_math_map(int fn, const float* in, float* out, uint64_t n) {
  if (!in || !out || fn < 0 || fn > 6) return CIS2_E_ARG;
  if (n == 0) return CIS2_OK;
  float *di = nullptr, *dout = nullptr;
  hipError_t e = hipMalloc(&di, n * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&dout, n * sizeof(float));
  if (e == hipSuccess) e = hipMemcpy(di, in, n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_math_map(fn, di, dout, n, 0);
  if (e == hipSuccess) e = hipMemcpy(out, dout, n * sizeof(float), hipMemcpyDeviceToHost);
  if (di) (void)hipFree(di);
  if (dout) (void)hipFree(dout);
  return e == hipSuccess ? CIS2_OK : CIS2_E_DEVICE;
}

int cis2_math_chunk_hashes(int fn, uint32_t c0, uint32_t nchunks, uint64_t* out) {
  if (!out || fn < 0 || fn > 6 || nchunks == 0 || (uint64_t)c0 + nchunks > 256) return CIS2_E_ARG;
  unsigned long long* d = nullptr;
  hipError_t e = hipMalloc(&d, nchunks * sizeof(unsigned long long));
  if (e == hipSuccess) e = hipMemset(d, 0, nchunks * sizeof(unsigned long long));
  for (uint32_t i = 0; e == hipSuccess && i < nchunks; ++i)
    e = launch_math_hash(fn, (c0 + i) << 24, 1u << 24, d + i, 0);
  if (e == hipSuccess) e = hipMemcpy(out, d, nchunks * sizeof(uint64_t), hipMemcpyDeviceToHost);
  if (d) (void)hipFree(d);
  return e == hipSuccess ? CIS2_OK : CIS2_E_DEVICE;
}

int cis2_div_map(const float* a, const float* b, float* out, uint64_t n) {
  if (!a || !b || !out) return CIS2_E_ARG;
  if (n == 0) return CIS2_OK;
  float *da = nullptr, *db = nullptr, *dout = nullptr;
  hipError_t e = hipMalloc(&da, n * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&db, n * sizeof(float));
  if (e == hipSuccess) e = hipMalloc(&dout, n * sizeof(float));
  if (e == hipSuccess) e = hipMemcpy(da, a, n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(db, b, n * sizeof(float), hipMemcpyHostToDevice);
  if (e == hipSuccess) e = launch_div_map(da, db, dout, n, 0);
  if (e == hipSuccess) e = hipMemcpy(out, dout, n * sizeof(float), hipMemcpyDeviceToHost);
  if (da) (void)hipFree(da);
  if (db) (void)hipFree(db);
  if (dout) (void)hipFree(dout);
  return e == hipSuccess ? CIS2_OK : CIS2_E_DEVICE;
}

void cis2_sha256(const void* data, uint64_t n, uint8_t out[32]) { sha256(data, n, out); }

int cis2_wait_probe(uint32_t bad[2]) {
  if (!bad) return CIS2_E_ARG;
  return run_wait_probes(bad) == hipSuccess ? CIS2_OK : CIS2_E_DEVICE;
}

int cis2_fpenv_probe(uint32_t out[2]) {
  if (!out) return CIS2_E_ARG;
  uint32_t* d = nullptr;
  hipError_t e = hipMalloc(&d, 8);
  if (e == hipSuccess) e = launch_fpenv_probe(d, 0);
  if (e == hipSuccess) e = hipMemcpy(out, d, 8, hipMemcpyDeviceToHost);
  if (d) (void)hipFree(d);
  return e == hipSuccess ? CIS2_OK : CIS2_E_DEVICE;
}

}  // extern "C"
