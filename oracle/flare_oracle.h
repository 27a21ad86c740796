/*
 * flare_oracle.h -- CPU restatement of flarellm's x86_64 decode kernels.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (flarellm_amd/, include/)
 * links, loads or calls this library.  It is the checker used by tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg.
 *
 * Every function restates the non-aarch64, non-wasm branch of the reference
 * (the branch that runs on an x86 host), citing file:line relative to the
 * reference checkout.  All arithmetic is IEEE binary32 with no contraction
 * (built with -ffp-contract=off) in the reference's loop order, so that the
 * oracle reproduces the reference bit-for-bit wherever the reference itself is
 * deterministic.  Transcendentals (powf, sinf, cosf, expf) come from the host
 * libm, which is what Rust's f32::{powf,sin_cos,exp} lower to on
 * x86_64-linux-gnu.
 */
#ifndef FLARE_ORACLE_H
#define FLARE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* WeightFormat subset on the hot path (flare-core/src/model.rs WeightFormat). */
enum { OR_F32 = 0, OR_Q8_0 = 1, OR_Q4K = 2, OR_Q6K = 3 };
/* KV cache storage modes (see or_model_create). */
enum { OR_KV_F32 = 0, OR_KV_F16 = 1, OR_KV_KIVI2 = 2, OR_KV_Q8 = 3, OR_KV_KIVI32 = 4 };

/* ---- scalar codecs ---------------------------------------------------- */
float or_f16_to_f32(uint16_t bits);
uint16_t or_f32_to_f16_rne(float f);
void or_dequant_q8_0_block(const uint8_t *blk, float out[32]);
void or_dequant_q4k_block(const uint8_t *blk, float out[256]);
void or_dequant_q6k_block(const uint8_t *blk, float out[256]);
void or_unpack_q4k_scales(const uint8_t *raw12, uint8_t sc[8], uint8_t mn[8]);
/* Dequantize a whole row-major tensor of `rows` rows x `bpr` blocks. */
int or_dequant_tensor(const uint8_t *data, int format, size_t rows, size_t bpr, float *out);

/* ---- activation quantizers -------------------------------------------- */
void or_quantize_input_q8_0(const float *x, size_t n, float *scales, int8_t *q);
void or_rmsnorm_quantize_q8_0(const float *x, const float *w, size_t n, float eps,
                              float *scales, int8_t *q);
void or_rmsnorm(const float *x, const float *w, size_t n, float eps, float *out);

/* ---- quantized matvecs -------------------------------------------------- */
/* Per-block integer dot products (the bit-exact parity target). */
void or_block_dots_q8_0(const uint8_t *w, const int8_t *xq, size_t rows, size_t bpr,
                        int32_t *dots /* rows*bpr */);
/* Q4_K: per superblock 8 entries, ordered (sub0 lo, sub0 hi, sub1 lo, ...):
 * entry 2*sub = dot_lo(sub), 2*sub+1 = dot_hi(sub) where hi uses sc[sub+4]. */
void or_block_dots_q4k(const uint8_t *w, const int8_t *xq, size_t rows, size_t bpr,
                       int32_t *dots /* rows*bpr*8 */);
void or_matvec_q8_0_preq(const uint8_t *w, const float *xs, const int8_t *xq, size_t rows,
                         size_t bpr, float *out);
void or_matvec_q4k_q8(const uint8_t *w, const float *xs, const int8_t *xq, size_t rows,
                      size_t cols, float *out);
/* Threads for the row-parallel loops (matvecs, argmax scores, attention
 * heads, dequantization).  Default 1 = the reference's single-threaded x86
 * path; results are identical for every thread count. */
void or_set_threads(int n);
/* Summation order of the float reductions: 0 = the reference's sequential
 * order (default), 1 = pairwise.  Order 1 is a measuring stick (how far two
 * valid summation orders drift apart on a model), not the reference. */
void or_set_order(int order);
int or_get_threads(void);
void or_matvec_argmax_q8_0_preq(const uint8_t *w, const float *xs, const int8_t *xq,
                                size_t rows, size_t bpr, int64_t *idx, float *val);
void or_matvec_argmax_q4k_q8_preq(const uint8_t *w, const float *xs, const int8_t *xq,
                                  size_t rows, size_t cols, int64_t *idx, float *val);
void or_matvec_argmax_f32(const float *mat, const float *vec, size_t rows, size_t cols,
                          int64_t *idx, float *val);
void or_matvec_f32(const float *mat, const float *vec, size_t rows, size_t cols, float *out);

/* ---- elementwise / attention ------------------------------------------- */
void or_rope_row(size_t head_dim, size_t pos, float theta, float *cos_out, float *sin_out);
void or_apply_rope(float *data, size_t num_heads, size_t head_dim, size_t pos, float theta);
void or_silu_mul(const float *gate, const float *up, size_t n, float *out);
void or_gqa_attention(const float *q, const float *k_cache, const float *v_cache,
                      size_t num_heads, size_t num_kv_heads, size_t head_dim, size_t seq_len,
                      float *out);

/* ---- KIVI 2-bit cache helpers (reference semantics) -------------------- */
void or_kivi_quantize_to_packed(const float *v, size_t n, uint8_t *packed, float *scale,
                                float *minv);

/* ---- KV forms of the long-context attention benchmark ------------------
 * OR_KV_Q8: every (token, kv head) row quantized per 32 values with the
 * quantize_input_q8_0_into arithmetic and the scale rounded to binary16.
 * OR_KV_KIVI32: rows rounded to binary16; tokens below
 * or_kivi32_qlen(T) replaced by their 2-bit group dequantization (K per
 * channel over 32 tokens, V per token over 32 channels, quantize_to_packed
 * arithmetic, (scale, min) rounded to binary16). */
size_t or_kivi32_qlen(size_t T);
/* Rows K, V: token-major [T][nkv][D] f32 as written.  Writes the values a
 * decode attention over T tokens reads, same layout. */
void or_kv_view(int kv_mode, const float *K, const float *V, size_t T, size_t nkv, size_t D,
                float *Kout, float *Vout);

/* ---- whole-model greedy decode ----------------------------------------- */
typedef struct {
    int hidden, layers, heads, kv_heads, head_dim, inter, vocab, max_seq;
    float eps, theta;
    int layer_format;  /* OR_Q8_0 or OR_Q4K for the 7 projections */
    int embed_format;  /* OR_Q8_0, OR_Q4K, OR_Q6K or OR_F32 */
    int output_format; /* -1 = tied to embedding, else format of output.weight */
    int kv_mode;       /* OR_KV_* */
} or_config;

/* Per-layer raw weights in GGUF byte layout (rows = out features). */
typedef struct {
    const uint8_t *wq, *wk, *wv, *wo, *w_gate, *w_up, *w_down;
    const float *attn_norm, *ffn_norm;
} or_layer;

typedef struct or_model or_model;

or_model *or_model_create(const or_config *cfg, const or_layer *layers,
                          const uint8_t *embedding, const uint8_t *output_weight,
                          const float *output_norm);
void or_model_destroy(or_model *m);
void or_model_reset(or_model *m);
/* Model::forward_greedy: returns argmax token, writes the winning logit. */
int64_t or_forward_greedy(or_model *m, uint32_t token, size_t pos, float *val);
/* Model::forward: full logits (vocab floats). */
void or_forward_logits(or_model *m, uint32_t token, size_t pos, float *logits);
/* Read-only access to the final normed hidden state of the last step. */
const float *or_model_final_normed(const or_model *m);
/* Greedy generation loop over Generator::step semantics (prompt processed one
 * token at a time). Writes n_gen tokens. */
void or_generate_greedy(or_model *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                        uint32_t *out);

/* ---- sampling (flare-core/src/sampling.rs) ----------------------------- */
/* Generator::step's transforms and sampler (generate.rs:210-230) on a copy
 * of logits[n]: apply_repeat_penalty (sampling.rs:83-96) over prev[n_prev],
 * apply_temperature (73-81), then sample_greedy (101-111) when temperature
 * is 0, else sample_top_p (131-181) when top_p < 1, else sample_min_p
 * (228-268) when min_p > 0, else sample_top_k (186-217) when top_k > 0, else
 * sample_top_p(1.0).  rng_val is the uniform draw.  Candidate sets are
 * ordered by descending probability, ties by ascending index. */
int64_t or_sample(const float *logits, size_t n, float temperature, float top_p, int top_k,
                  float repeat_penalty, float min_p, const uint32_t *prev, size_t n_prev,
                  float rng_val);

#ifdef __cplusplus
}
#endif
#endif
