/* oracle/cis2_oracle.h — CPU restatement of the CIS-2 v0.3b pinned-order
 * fp32 decoder forward pass (and the v0.4-candidate tree order).
 *
 * TEST INFRASTRUCTURE ONLY.  tests/, the smoke() entry point and
 * bench.py's cpu_baseline leg load this library to produce the expected
 * bits.  The product path (the HIP library) never links, loads or
 * calls it.
 *
 * Every function cites the reference file:line whose semantics it restates.
 * Paths are relative to the reference archive root (code/cis2-fp/...).
 *
 * Parity pins (how each part of this oracle is checked, see tests/):
 *   - math (exp/sin/cos/ln/silu/rsqrt): exhaustive 2^32-input comparison
 *     against the reference's own cis2_math.h compiled here, recorded as
 *     chunk-hash fixtures; closed-form KATs (rsqrt(64), table digest,
 *     SmolLM2 inv_freq digest).
 *   - dot_seq / GEMV: the 25 published rust-5 output hashes
 *     (labs/rust-5/reports/rust-5/box1/gate.out), brute force on tiny
 *     inputs, and the order-sensitivity KAT.
 *   - tree reduction: closed form ((1+2)+(3+4))+5 and a brute-force
 *     restatement on ragged lengths; digests of the reference compiled with
 *     -DCIS2_REDUCTION_TREE.
 *   - forward/decode/witness: CIS2_REF digests, token lists and --trace
 *     hashes of the reference C++ driver (gpu/cis2_host.cpp) compiled here
 *     and run on the same synthetic artifacts.
 */
#ifndef CIS2_ORACLE_H
#define CIS2_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- floating-point environment (per thread) ------------------------- */
/* Pins MXCSR FTZ|DAZ on the calling thread, reads it back and runs the
 * two adversarial probes.  Returns 0 on success. */
int orc_fpenv_pin(void);
void orc_fpenv_release(void);

/* ---- scalar pinned math ---------------------------------------------- */
enum { ORC_FN_EXP = 0, ORC_FN_SIN = 1, ORC_FN_COS = 2, ORC_FN_LN = 3,
       ORC_FN_SILU = 4, ORC_FN_RSQRT = 5, ORC_FN_SQRT = 6, ORC_FN_COUNT = 7 };
float orc_exp(float x);
float orc_sin(float x);
float orc_cos(float x);
float orc_ln(float x);
float orc_silu(float x);
float orc_rsqrt(float x);
float orc_sqrt(float x);
/* out[i] = a[i] / b[i] (one correctly rounded divss under FTZ|DAZ) */
void orc_div_map(const float *a, const float *b, float *out, size_t n);
/* out[i] = fn(in[i]) */
void orc_math_map(int fn, const float *in, float *out, size_t n);
/* Chunk hash over the 2^32 inputs [chunk<<shift, (chunk+1)<<shift):
 * sum over i of mix64(bits(fn(x_i)) ^ (i * 0x9E3779B97F4A7C15)).  The same
 * order-free hash is computed on the device. */
uint64_t orc_math_chunk_hash(int fn, uint32_t first, uint32_t count);
uint64_t orc_mix64(uint64_t z);

/* ---- reductions -------------------------------------------------------- */
float orc_dot_seq(const float *a, const float *b, int n);
float orc_sum_seq(const float *a, int n);
float orc_dot_tree(const float *a, const float *b, int n);
float orc_sum_tree(const float *a, int n);
/* y = W x with W row-major [M,K]; mode 0 sequential, 1 tree.  Row-parallel
 * over `threads` threads (rows are independent, so the bits do not depend
 * on the thread count). */
void orc_gemv(const float *W, const float *x, float *y, int M, int K, int mode,
              int threads);
void orc_softmax(float *v, int n, int mode);
uint32_t orc_argmax(const float *v, int n);

/* ---- digests ------------------------------------------------------------ */
void orc_sha256(const void *data, size_t n, uint8_t out[32]);
void orc_table_digest(uint8_t out[32]);
/* inv_freq[i] for i < head_dim/2 and its digest. */
void orc_inv_freq(double rope_theta, int head_dim, float *out, uint8_t digest[32]);

/* ---- model --------------------------------------------------------------- */
typedef struct {
  int hidden, inter, n_layers, n_heads, n_kv_heads, head_dim, vocab;
  int tied;          /* 1: LM head = embed_tokens */
  int max_pos;       /* KV-cache capacity in positions */
  int reduction;     /* 0 sequential (v0.3b), 1 tree (v0.4 candidate) */
  int threads;       /* worker threads for row-parallel work (>=1) */
  float eps;         /* already narrowed to f32 */
  double rope_theta;
} orc_config;

typedef struct orc_model orc_model;

typedef void (*orc_trace_fn)(int pos, int layer, const char *op,
                             const uint8_t sha[32], void *user);

orc_model *orc_model_create(const orc_config *cfg);
void orc_model_destroy(orc_model *m);
/* Widen a BF16 tensor (little-endian u16 array) into the model.  Returns
 * 0, or -1 unknown name, -2 element count mismatch. */
int orc_model_set_bf16(orc_model *m, const char *name, const uint16_t *bits,
                       size_t n);
/* Which tensors the config expects: name of the i-th tensor and its element
 * count; returns NULL past the end.  Optional tensors (biases, q/k norms)
 * are not listed. */
const char *orc_model_tensor(const orc_model *m, int i, size_t *count);
void orc_model_digests(const orc_model *m, uint8_t table[32], uint8_t inv_freq[32]);
void orc_model_reset(orc_model *m);
/* One forward pass at `pos` for `token`; writes vocab logits. */
int orc_forward(orc_model *m, int pos, uint32_t token, float *logits,
                orc_trace_fn cb, void *user);
/* The final-norm output (hidden floats) of the last orc_forward: the
 * vector the LM head multiplies.  Used to construct coverage rows. */
int orc_model_hidden(const orc_model *m, float *out);

/* Planted mistakes for tests that show a fixture detects them; 0 (the
 * default) runs the oracle as specified.
 *   ORC_MUT_ARGMAX_GE  greedy argmax with >= (the last maximum wins)
 *   ORC_MUT_NO_FTZ     FTZ/DAZ left off (subnormal inputs and results kept) */
#define ORC_MUT_ARGMAX_GE 1
#define ORC_MUT_NO_FTZ 2
void orc_set_mutation(int m);

/* Greedy decode exactly as the reference driver: prefill every prompt
 * position, then gen_toks steps of argmax -> witness fold -> forward.
 * hdr = sha256 of model.safetensors, tokenizer.json, config.json.
 * out_ids receives prompt ids followed by the generated ids.
 * step_digests (optional, gen_toks*32 bytes) receives sha256 of the logits
 * folded at each step.  Returns 0 or a negative error. */
int orc_decode(orc_model *m, const uint32_t *prompt, int n_prompt, int gen_toks,
               const uint8_t hdr[96], uint32_t *out_ids, uint8_t witness[32],
               uint8_t argmax_digest[32], uint8_t *step_digests,
               orc_trace_fn cb, void *user);

/* ---- seeded sampling (CIS-2 v0.4 draft section 14) ------------------
 * code/patches/cis2-spec__seeded-sampling.patch:57-196
 * (docs/CIS2_SPEC_v0.4-draft-seeded-sampling.md).  Pinned by the draft's
 * known answers: MurmurHash3 of the empty key (seeds 0 and 1), the four
 * (seed, step, index) -> hash, u, g rows of 14.6 and the 14.6 toy vector
 * (kept set, z bit patterns, next_id); the rank and top-p rules by a
 * brute-force restatement on small vocabularies (tests/). */
/* MurmurHash3_x86_32 (Appleby, public domain) of len bytes. */
uint32_t orc_murmur3_32(const void *key, size_t len, uint32_t seed);
/* hash, uniform and Gumbel noise of (seed, step, vocab index), 14.2. */
void orc_sample_noise(uint64_t seed, uint32_t step, uint32_t index, uint32_t *h,
                      float *u, float *g);
/* 0 when (temperature, top_k, top_p) are valid (14.1), else -1. */
int orc_sample_params_ok(float temperature, uint32_t top_k, float top_p);
/* Next id drawn from V logits at generation step `step` (14.3-14.4).
 * z (optional, V floats) receives the z values (masked: -inf), nkeep
 * (optional) the size of the kept set.  Returns UINT32_MAX for invalid
 * parameters or a NaN among l / temperature. */
uint32_t orc_sample(const float *logits, int V, uint64_t seed, uint32_t step,
                    float temperature, uint32_t top_k, float top_p, float *z,
                    uint32_t *nkeep);
/* orc_decode with the draw of orc_sample in place of the argmax, and the
 * section 14.5 receipt header after the prompt ids. */
int orc_decode_sampled(orc_model *m, const uint32_t *prompt, int n_prompt, int gen_toks,
                       const uint8_t hdr[96], uint64_t seed, float temperature,
                       uint32_t top_k, float top_p, uint32_t *out_ids, uint8_t witness[32],
                       uint8_t argmax_digest[32], uint8_t *step_digests);

#ifdef __cplusplus
}
#endif
#endif
