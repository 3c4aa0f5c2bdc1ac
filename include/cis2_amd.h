/* include/cis2_amd.h — C ABI of the MI355X (gfx950) CIS-2 pinned-order fp32
 * decoder forward pass.
 *
 * The reference exposes the forward pass in-process as
 *   Rust  forward_token(&Model, &mut [KvCache], pos, token_id, ..) -> Vec<f32>
 *         (code/cis2-fp/src/main.rs:355-364)
 *   C++   cis2_forward_token(const Cis2Model&, Cis2Workspace&, int pos,
 *                            uint32_t tok, Cis2Trace*)
 *         (code/cis2-fp/gpu/cis2_model.h:685-686)
 * and its callers drive it through the greedy decode / witness loop of
 * code/cis2-fp/gpu/cis2_host.cpp:61-249 (Rust: src/main.rs:1025-1263).
 * This header is the FFI a host (Rust via bindgen, C++, Python ctypes) binds
 * instead: plain pointers and sizes, no exceptions, no exit().
 *
 * Contract
 *   - Ownership: the caller owns every host buffer it passes; the context
 *     owns all device memory (weights, KV caches, scratch).
 *   - Errors: every call returns CIS2_OK (0) or a negative CIS2_E_* code;
 *     cis2_last_error() gives the message of the last failure on a context.
 *   - Threading: one context is used by one host thread at a time; calls
 *     block until their results are in host memory (as the reference's
 *     synchronous ops do).
 *   - Numerics: IEEE binary32, round to nearest even, FTZ/DAZ, no FMA
 *     contraction, pinned exp/sin/cos/ln, strict left-to-right reductions
 *     (CIS-2 v0.3b, reduction_mode 0) or the v0.4-candidate tree order
 *     (reduction_mode 1: 32-leaf pairwise blocks folded left to right,
 *     code/cis2-fp/src/math.rs:60-125).  Results are bit-identical to the
 *     reference CPU path in either mode.
 */
#ifndef CIS2_AMD_H
#define CIS2_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CIS2_ABI_VERSION 1

enum {
  CIS2_OK = 0,
  CIS2_E_ARG = -1,             /* null pointer, out-of-range index, bad size */
  CIS2_E_UNSUPPORTED = -2,     /* config the pinned path does not cover      */
  CIS2_E_MISSING_TENSOR = -3,  /* a required tensor was never uploaded       */
  CIS2_E_SHAPE = -4,           /* element count does not match the config    */
  CIS2_E_NAME = -5,            /* tensor name not part of the architecture   */
  CIS2_E_FPENV = -6,           /* device FTZ/DAZ self-test failed            */
  CIS2_E_DEVICE = -7,          /* HIP runtime error                          */
  CIS2_E_OOM = -8,             /* device or pinned host allocation failed    */
  CIS2_E_RANGE = -9,           /* position beyond max_pos / token >= vocab   */
  CIS2_E_NUMERIC = -10         /* NaN logit in a sampled draw                */
};

typedef struct cis2_ctx cis2_ctx;

/* Model configuration.  The field meanings follow config.json as the
 * reference reads it (code/cis2-fp/gpu/cis2_host.cpp:97-117, Qwen3
 * head_dim: labs/w1x-qwen3/scripts/qwen3-port.diff:104-110). */
typedef struct {
  uint32_t hidden;          /* hidden_size                                   */
  uint32_t inter;           /* intermediate_size                             */
  uint32_t n_layers;        /* num_hidden_layers                             */
  uint32_t n_heads;         /* num_attention_heads                           */
  uint32_t n_kv_heads;      /* num_key_value_heads                           */
  uint32_t head_dim;        /* head_dim key, else hidden / n_heads           */
  uint32_t vocab;           /* vocab_size                                    */
  uint32_t tied;            /* tie_word_embeddings (1: LM head = embedding)  */
  uint32_t max_pos;         /* KV-cache capacity per sequence (<= 16384)     */
  uint32_t max_seqs;        /* independent sequences (KV caches), >= 1       */
  uint32_t reduction_mode;  /* 0 sequential (v0.3b); 1 tree (v0.4 candidate)  */
  float eps;                /* (float)rms_norm_eps, narrowed once            */
  double rope_theta;        /* rope_theta as parsed (narrowed on use)        */
} cis2_config;

/* Called once per (position, layer, op) when tracing is on; `layer` is -1
 * for embedding, final_norm and logits; sha256 is over the little-endian
 * f32 bit patterns of the op's output (code/cis2-fp/gpu/cis2_model.h:482-496,
 * op order gpu/README.md:216-222). */
typedef void (*cis2_trace_fn)(int pos, int layer, const char *op,
                              const uint8_t sha256[32], void *user);

/* Creates a context on the current HIP device, allocates device memory for
 * the weights, KV caches and scratch, runs the device FTZ/DAZ self-test and
 * builds the pinned inv_freq / rotation tables.  Replaces Cis2Workspace::alloc
 * + cis2_build_inv_freq + cis2_fpenv_init (cis2_model.h:645-671, :456-476;
 * cis2_fpenv.h:110-117). */
int cis2_ctx_create(const cis2_config *cfg, cis2_ctx **out);
void cis2_ctx_destroy(cis2_ctx *ctx);
const char *cis2_strerror(int code);
const char *cis2_last_error(const cis2_ctx *ctx);

/* Uploads one BF16 tensor (little-endian u16, row-major as stored in
 * model.safetensors) by its checkpoint name; the device widens it exactly
 * (bits << 16) and lays GEMV weights out for coalesced streaming.  Replaces
 * Cis2SafeTensors::load_bf16 (cis2_model.h:340-374).  Optional tensors
 * (q/k/v biases, Qwen3 q_norm/k_norm) switch their op on when present. */
int cis2_upload_bf16(cis2_ctx *ctx, const char *name, const uint16_t *bf16, uint64_t n);
/* Returns CIS2_OK once every required tensor is present. */
int cis2_check_ready(cis2_ctx *ctx);

/* Table digest (spec §6.6) and inv_freq table digest (spec §7.2), as the
 * witness header binds them (cis2_host.cpp:119-124). */
int cis2_digests(cis2_ctx *ctx, uint8_t table[32], uint8_t inv_freq[32]);

/* Clears a sequence's KV cache (a fresh prompt). */
int cis2_reset_seq(cis2_ctx *ctx, uint32_t seq);

/* One forward pass per listed row: sequence seq[i] at position pos[i] with
 * input token tok[i].  logits_host (n * vocab floats) and argmax_out (n
 * ids, strict-> first maximum) may each be NULL.  Replaces one call of
 * cis2_forward_token + cis2_download + cis2_argmax per row
 * (cis2_model.h:685-774).  With n > 1 the rows run as one row-batched
 * pass: every row's K/V reach the caches before any row's attention, so
 * rows of one sequence at different positions are causal among themselves
 * (a teacher-forced prefill); no two rows may share a (seq, pos)
 * (CIS2_E_ARG).  Each row's results equal its single-row call bit for bit. */
int cis2_forward(cis2_ctx *ctx, uint32_t n, const uint32_t *seq, const uint32_t *pos,
                 const uint32_t *tok, float *logits_host, uint32_t *argmax_out);

/* Greedy decode with the CIS-2 witness fold, exactly the reference driver's
 * loop (cis2_host.cpp:176-218; src/main.rs:1084-1226): prefill every prompt
 * position, then gen_toks times { argmax of the logits already computed ->
 * fold logits (u32 LE bits) and the id into the witness -> forward the id }.
 * hdr = sha256(model.safetensors) ++ sha256(tokenizer.json) ++
 * sha256(config.json) (96 raw bytes).  out_ids receives prompt ++ generated
 * ids (n_prompt + gen_toks).  step_digests (optional, 32*gen_toks bytes)
 * receives sha256 of the logits folded at each step.  The argmax runs on
 * the device; logits stream to pinned host memory and are hashed while the
 * GPU computes the next step. */
int cis2_decode(cis2_ctx *ctx, uint32_t seq, const uint32_t *prompt, uint32_t n_prompt,
                uint32_t gen_toks, const uint8_t hdr[96], uint32_t *out_ids,
                uint8_t witness[32], uint8_t argmax_digest[32], uint8_t *step_digests);

/* The same decode split into steps, for callers that interleave their own
 * work (or time the steady state): begin = witness header + prefill;
 * steps = n more greedy steps; end = finish the digests.  begin + steps(a) +
 * steps(b) + end gives exactly cis2_decode(.., a + b, ..).  One session per
 * context at a time.  out_ids must hold n_prompt + total steps ids. */
int cis2_decode_begin(cis2_ctx *ctx, uint32_t seq, const uint32_t *prompt, uint32_t n_prompt,
                      uint32_t max_steps, const uint8_t hdr[96]);
int cis2_decode_steps(cis2_ctx *ctx, uint32_t n);
int cis2_decode_end(cis2_ctx *ctx, uint32_t *out_ids, uint8_t witness[32],
                    uint8_t argmax_digest[32], uint8_t *step_digests);

/* Seeded sampling (CIS-2 v0.4 draft section 14,
 * code/patches/cis2-spec__seeded-sampling.patch:57-196; the reference
 * driver's `--sample seed,T,K,P`, labs/w1x-sample/feed/cm-hq__cis2-sample-hq-r2/
 * job.sh:22-28).  mode 1 replaces the greedy argmax of cis2_decode /
 * cis2_decode_begin..end by a stateless Gumbel-max draw: s = l / T,
 * rank-order top-k and top-p, z = s + g(seed, step, index) with
 * MurmurHash3_x86_32 noise and the pinned ln, first index of max z.  The
 * witness absorbs "CIS2-SAMPLE-1", seed (u64 LE), T, top_k, top_p (bit
 * patterns, u32 LE) after the prompt ids; the argmax digest is fed the
 * drawn ids.  mode 0 (or s == NULL) restores greedy decoding, whose
 * receipts are unchanged.  Invalid parameters (T not finite or <= 0,
 * top_p outside (0, 1]) give CIS2_E_ARG.  The batched decode and the
 * teacher-forced verifier stay greedy (CIS2_E_UNSUPPORTED in mode 1). */
typedef struct {
  uint32_t mode;      /* 0 greedy, 1 seeded sampling                   */
  uint32_t top_k;     /* 0 or >= vocab: disabled                       */
  uint64_t seed;
  float temperature;  /* finite, > 0                                   */
  float top_p;        /* (0, 1]; 1.0: disabled                         */
} cis2_sampling;
int cis2_set_sampling(cis2_ctx *ctx, const cis2_sampling *s);

/* The same draw on n host logit rows (vocab floats each) with the
 * context's sampling parameters, row i at generation step steps[i]:
 * ids_out[i] = drawn id, nkeep_out[i] (optional) = size of the kept set.
 * For hosts that hold logits themselves, and for tests. */
int cis2_sample_logits(cis2_ctx *ctx, const float *logits_host, uint32_t n,
                       const uint32_t *steps, uint32_t *ids_out, uint32_t *nkeep_out);

/* ---- No-allocation draw (no counterpart in the reference) ----------------
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc): the draw of
 * cis2_sample_logits on n DEVICE-resident logit rows (logits_dev: n * vocab
 * floats), row i at step steps[i] (host array), with the context's sampling
 * parameters.  ids_dev[i] (device) receives the drawn id and nkeep_dev[i]
 * (device, optional) the size of the kept set; the results equal
 * cis2_sample_logits on the same rows bit for bit.  The call allocates
 * nothing: its scratch is one static array per GPU of 5,244,992 bytes
 * (two sort-key arrays, the f32 terms, candidates, flags), which serves
 * vocabularies up to 262,144 (larger: CIS2_E_ARG) and is held until the
 * process ends.  Every call on a GPU shares that GPU's array: a call holds
 * a per-GPU lock from clearing its error flag until its results are back,
 * so calls from several host threads on one GPU take turns (each process
 * has its own array).  Blocks until the draws are done; a NaN logit gives
 * CIS2_E_NUMERIC. */
int cis2_sample_logits_noalloc(cis2_ctx *ctx, const float *logits_dev, uint32_t n,
                               const uint32_t *steps, uint32_t *ids_dev, uint32_t *nkeep_dev);

/* Batched greedy decode: nseq independent sequences with their own prompts
 * (ragged lengths allowed), each decoded for gen_toks steps.  Groups of up
 * to max_seqs sequences run together (KV-cache slots 0..max_seqs-1): one
 * row-batched prefill of all their prompt positions, then one row per
 * sequence per step, each at its own position.  Every row's
 * outputs equal its bs=1 cis2_decode outputs bit for bit (the reference's
 * per-row batch semantics: code/patches/cis2-fp__cm_gpu3-batched-full.patch
 * :443-458,687-763).  prompts = concatenated ids, prompt_lens[nseq];
 * out_ids = concatenated (prompt_len+gen_toks) rows; witness/argmax digests
 * 32*nseq bytes. */
int cis2_decode_batch(cis2_ctx *ctx, uint32_t nseq, const uint32_t *prompts,
                      const uint32_t *prompt_lens, uint32_t gen_toks, const uint8_t hdr[96],
                      uint32_t *out_ids, uint8_t *witness, uint8_t *argmax_digest);

/* Teacher-forced verification of a claimed continuation in one row-batched
 * pass over prompt ++ claimed (cis2_verify_receipt_prefill,
 * code/cis2-fp/verify3/model.c:923-1005; first_mismatch_pos as
 * verify3/prefilltest.c:60-76).  The logits at position n_prompt-1+s
 * predict claimed[s]; generated[s] receives their argmax.  witness and
 * argmax_digest are built as cis2_decode builds them, from the logits and
 * their argmax ids, so an honest claim reproduces the decode's digests.
 * *first_mismatch = first s with generated[s] != claimed[s], else -1.
 * logits_host (optional) receives n_gen * vocab floats.  Uses KV-cache slot
 * `seq` (cleared first); n_prompt + n_gen - 1 <= max_pos. */
int cis2_verify_prefill(cis2_ctx *ctx, uint32_t seq, const uint32_t *prompt, uint32_t n_prompt,
                        const uint32_t *claimed, uint32_t n_gen, const uint8_t hdr[96],
                        uint32_t *generated, uint8_t witness[32], uint8_t argmax_digest[32],
                        int64_t *first_mismatch, float *logits_host);

/* Per-op tracing (--trace); NULL disables.  Tracing synchronises after every
 * op, so it is a verification mode, not a fast path. */
int cis2_trace_enable(cis2_ctx *ctx, cis2_trace_fn fn, void *user);

/* ---- Kernel timing (measurement; no counterpart in the reference) --------
 * While on, every launch of the persistent decode kernel is bracketed by a
 * pair of HIP events on the library's stream (at most 65536 launches are
 * kept).  cis2_profile(ctx, 1) also clears the record.
 * cis2_profile_read waits for the recorded launches and returns their count
 * and summed device time; positions[i] (optional, `cap` entries) receive the
 * position each launch computed. */
int cis2_profile(cis2_ctx *ctx, int on);
int cis2_profile_read(cis2_ctx *ctx, uint64_t *launches, double *total_ms, uint32_t *positions,
                      uint64_t cap);

/* ---- Sharing the GPU (no counterpart in the reference: its decode is one
 * CPU process) ---------------------------------------------------------------
 * The persistent decode kernel needs its whole grid resident at once.  Its
 * launches are therefore taken one decode session at a time per GPU, across
 * processes: an exclusive flock on CIS2_LOCK_DIR (default /tmp)/cis2amd-<pci
 * bus id>.lock is held from a session's first persistent launch
 * (cis2_decode_begin) until cis2_decode_end (cis2_forward: for the call);
 * CIS2_DECODE_LOCK=0 turns it off.  Should a launch still find CUs held by
 * other work and hit its bounded wait (the spin cap, about 0.5 s; the
 * CIS2_SPIN_CAP environment variable at context creation sets it in sleeps),
 * the step is recomputed on the per-op path with the same bits and the
 * session continues there.  *count receives how many steps of this context
 * were recovered so. */
int cis2_recoveries(cis2_ctx *ctx, uint32_t *count);

/* ---- Standalone pinned-order GEMV (the 4-row-interleaved reference kernel
 * of labs/rust-5, whose bits equal matvec/dot_seq: src/main.rs:228-243,
 * math.rs:40-48) --------------------------------------------------------- */
typedef struct cis2_gemv_plan cis2_gemv_plan;
/* Uploads `copies` replicas of the row-major [M,K] matrix W (host) in the
 * blocked device layout; replicas let a benchmark rotate through more bytes
 * than the 256 MB Infinity Cache holds. */
int cis2_gemv_plan_create(uint32_t M, uint32_t K, uint32_t copies, const float *W,
                          cis2_gemv_plan **out);
/* y = W x with host x[K] and y[M]. */
int cis2_gemv_plan_run(cis2_gemv_plan *p, const float *x, float *y);
/* Times `iters` device-resident launches cycling through the replicas on one
 * stream (HIP events on that stream); returns the mean ms per launch. */
int cis2_gemv_plan_time(cis2_gemv_plan *p, uint32_t iters, float *ms_per_launch);
/* n independent GEMVs in one launch: y_i = W_(i mod copies) x_i with host
 * x[n][K] and y[n][M], each bit-equal to cis2_gemv_plan_run on x_i (a
 * GEMV stream, as the layers of a model issue them back to back; the
 * reference runs one GEMV per call, rust-5 src/main.rs). n <= 65535. */
int cis2_gemv_plan_run_batch(cis2_gemv_plan *p, uint32_t n, const float *x, float *y);
/* Times `iters` launches of n GEMVs each over device-resident inputs,
 * consecutive launches on consecutive replicas; returns the mean ms per
 * launch. */
int cis2_gemv_plan_time_batch(cis2_gemv_plan *p, uint32_t n, uint32_t iters,
                              float *ms_per_launch);
void cis2_gemv_plan_destroy(cis2_gemv_plan *p);

/* SHA-256 of a host buffer (the witness header binds sha256 of
 * model.safetensors, tokenizer.json and config.json). */
void cis2_sha256(const void *data, uint64_t n, uint8_t out[32]);

/* ---- Verification hooks (device pinned math) --------------------------- */
/* fn: 0 exp, 1 sin, 2 cos, 3 ln, 4 silu, 5 rsqrt, 6 sqrt.  out[i] = fn(in[i]). */
int cis2_math_map(int fn, const float *in, float *out, uint64_t n);
/* Order-free hashes of fn over all inputs of chunks [c0, c0+nchunks) of
 * 2^24 bit patterns each: sum mix64(bits(fn(x)) ^ bits(x)*0x9E3779B97F4A7C15). */
int cis2_math_chunk_hashes(int fn, uint32_t c0, uint32_t nchunks, uint64_t *out);
/* out[i] = a[i] / b[i] on the device (correctly rounded, FTZ). */
int cis2_div_map(const float *a, const float *b, float *out, uint64_t n);
/* Device FTZ/DAZ probes: bits of 2^-126*1e-10 and of (2^-149 + 0.0). */
int cis2_fpenv_probe(uint32_t out[2]);
/* Wait-counter capacity probes (verification; no counterpart in the
 * reference): bad[0] receives the wrong registers after one wave issues 128
 * vector loads and then a single s_waitcnt vmcnt(0), bad[1] the wrong words
 * after 40 LDS reads and a single lgkmcnt(0).  The counters' fields hold 63
 * and 15 operations; the decode kernel keeps up to 128 loads per thread in
 * flight, which is exact only if the hardware holds further issue at a
 * field's maximum: both counts are then 0. */
int cis2_wait_probe(uint32_t bad[2]);

#ifdef __cplusplus
}
#endif
#endif
