/*
 * flare_hip.h -- C-ABI of the MI355X decode backend for flarellm.
 *
 * This is the drop-in boundary that replaces flarellm's
 * `flare_core::model::ComputeBackend` decode hooks
 * (flare-core/src/model.rs:176-618) and the free quantized kernels that
 * `Model::forward_layers` calls directly on the CPU path
 * (flare-core/src/model.rs:1955-2561).  Citations are path:line in the
 * flarellm source tree.
 *
 * Conventions
 *  - Every entry point returns 0 on success or a negative FL_E* code; the
 *    message is available from fl_last_error(ctx) (ctx may be NULL for
 *    errors raised before a context exists).  This replaces the reference's
 *    panics (model.rs:321, 474-477; flare-gpu/src/backend.rs:4907-4910).
 *  - One context = one GPU + one HIP stream.  A context is not thread-safe,
 *    like the reference's single `&mut Model`.
 *  - Weight bytes cross the boundary in GGUF block layout exactly as
 *    `RawWeight { data, format, num_rows, blocks_per_row }`
 *    (model.rs:123-130, flare-loader/src/gguf.rs:616-653).  They are host
 *    pointers and are copied (and, for Q8_0/Q6_K, re-laid-out) on upload.
 *  - "Op" entry points (fl_op_*) take DEVICE pointers and enqueue on the
 *    context stream; call fl_sync() before reading results on the host.
 *  - Activations quantized to Q8_0 are three device arrays: int8 quants[n],
 *    float scales[n/32] and int32 block sums[n/32] (sum of the 32 quants,
 *    used by the Q4_K min term).  quants+scales are the reference's
 *    `QuantizedInput` (model.rs:5468-5472).
 */
#ifndef FLARE_HIP_H
#define FLARE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FL_ABI_VERSION 1

/* status codes */
#define FL_OK 0
#define FL_E_INVALID (-1)     /* bad argument / unsupported shape */
#define FL_E_UNSUPPORTED (-2) /* format or path not implemented */
#define FL_E_HIP (-3)         /* HIP runtime error */
#define FL_E_STATE (-4)       /* call order violated (e.g. no weights) */
#define FL_E_OOM (-5)         /* device allocation failed */

/* WeightFormat subset on the decode hot path (model.rs WeightFormat). */
#define FL_F32 0
#define FL_Q8_0 1
#define FL_Q4K 2
#define FL_Q6K 3

/* KV cache storage. F32 = flare-core KvCache (kv_cache.rs:431-546);
 * F16 = flare-gpu GpuKvCache f16 (flare-gpu/src/kv_cache.rs:51-66). */
#define FL_KV_F32 0
#define FL_KV_F16 1
/* Q8: int8 + binary16 scale per 32 values of a (token, kv head) row, the
 * quantize_input_q8_0_into arithmetic (model.rs:5557-5570).  The reference
 * README lists a Q8 KV cache (README.md:70) with no implementation; this is the
 * long-context benchmark's form. */
#define FL_KV_Q8 2
/* KIVI 2-bit in the long-context benchmark's form: K quantized per channel over groups
 * of 32 tokens, V per token over groups of 32 channels, with the
 * quantize_to_packed arithmetic of flare-core/src/kv_cache.rs:336-371
 * ((max-min)/3, round, clamp 0..3, 4 codes per byte LSB first) and
 * (scale, min) kept as binary16.  The newest tokens stay binary16 in a
 * 192-slot ring: tokens [0, Q) come from the 2-bit groups and [Q, T) from the
 * ring, Q = 32*floor((T-129)/32) for T > 128 (else 0).  The reference's own
 * QuantizedKvCache (kv_cache.rs:35-323: 32-token f32 window, per-token K codes
 * read with running per-channel stats) is not reproduced. */
#define FL_KV_KIVI2 3

typedef struct fl_ctx fl_ctx;
typedef struct fl_weight fl_weight;

/* RawWeight (model.rs:123-130). */
typedef struct {
    const void *data; /* host pointer to GGUF tensor bytes */
    size_t nbytes;
    int format;       /* FL_Q8_0 / FL_Q4K / FL_Q6K / FL_F32 */
    int num_rows;     /* out features (last GGUF dim) */
    int blocks_per_row;
} fl_raw_weight;

/* ModelConfig fields used by forward_single_token_gpu (model.rs:555) and
 * flare-core/src/config.rs:17-54. */
typedef struct {
    int hidden_dim, num_layers, num_heads, num_kv_heads, head_dim, intermediate_dim,
        vocab_size, max_seq_len;
    float rms_norm_eps, rope_theta;
} fl_model_config;

/* ---- context ------------------------------------------------------------ */
int fl_abi_version(void);
/* Create a context on HIP device `device`.  No reference counterpart: the
 * reference constructs its backend with WebGpuBackend::new. */
int fl_ctx_create(int device, fl_ctx **out);
void fl_ctx_destroy(fl_ctx *ctx);
const char *fl_last_error(const fl_ctx *ctx);
/* The hipStream_t all work of this context is enqueued on. */
void *fl_ctx_stream(fl_ctx *ctx);
int fl_sync(fl_ctx *ctx);
/* ComputeBackend::name (model.rs:615). */
const char *fl_backend_name(void);

/* Execution switches of a context (measurement and testing; no reference
 * counterpart).  FL_OPT_VERIFY_FUSE (default 1): fl_verify runs the Q4_K QKV
 * post-processing and SiLU*up inside the GEMMs' last-arriving K split (0: as
 * separate kernels; both sum the K-split partials in the same order, so the
 * results are identical).  FL_OPT_VERIFY_GRAPH (default 1): replay fl_verify
 * as a captured HIP graph (0: enqueue kernel by kernel).  Drops captured
 * graphs. */
#define FL_OPT_VERIFY_FUSE 1
#define FL_OPT_VERIFY_GRAPH 2
/* FL_OPT_EXACT (default 0): the decode step (fl_decode_step, fl_generate)
 * and the Q8-input op matvecs compute in the x86 reference's floating-point
 * order -- row sums folded block by block, sequential sums of squares,
 * sequential online-softmax attention, expf as the C library computes it,
 * the f32 output dot in column order -- so logits equal the CPU reference's
 * bit for bit.  The matvecs are the same streaming kernels with an in-order
 * fold; attention and the f32 output projection run simple sequential
 * kernels (slow).  fl_verify and fl_prefill then run their tokens as
 * sequential decode steps (the reference's sequential verification; its
 * forward_prefill equals sequential steps, generate.rs:657), and fl_op_sample
 * sums in the reference's order.  F32 / F16 KV caches only.  Default:
 * tree-order sums (fast; outputs within 1e-3 relative). */
#define FL_OPT_EXACT 3
/* FL_OPT_FUSE_ATTN (default 0): with an fp16 KV cache, the decode step runs
 * each layer's QKV matvec and attention as one launch whose attention
 * workgroups stream the K / V cache while the QKV workgroups compute, then
 * wait for them (outputs identical to the two launches).  Measured slower on
 * MI355X (the attention role's registers halve the QKV role's occupancy), so
 * off by default. */
#define FL_OPT_FUSE_ATTN 4
int fl_set_option(fl_ctx *ctx, int option, int value);

/* Layer probe (testing surface; no reference counterpart).  With layer >= 0,
 * every following fl_decode_step / fl_decode_step_embed / fl_verify runs its
 * kernels without a captured graph and copies, as the production kernels
 * compute them, the intermediates of that layer into host_buf
 * (fl_probe_layout bytes, kept alive by the caller), for up to 16 tokens:
 * x_in, q (after RoPE), the slots' K and V rows, the attention output and
 * its Q8_0 codes / scales, x after wo, the hidden vector's Q8_0 codes /
 * scales, x after down (decode step), the final residual, and (verify pass)
 * the Q8_0 codes / scales of both RMSNorm outputs the GEMMs read.  So a test
 * can check each operation of the production path against the CPU reference
 * applied to the path's own inputs.  layer = -1 turns it off.
 * fl_probe_layout fills offsets[0..15] (byte offsets of the regions x_in, q,
 * k, v, attn, attn scales, x_mid, h scales, x_out, x_final, attn codes,
 * h codes, norm codes, norm scales, FFN-norm codes, FFN-norm scales; each
 * region [16 tokens][size]) and returns the total size (-1 without a
 * model). */
int fl_probe_layer(fl_ctx *ctx, int layer, void *host_buf);
int fl_probe_layout(const fl_ctx *ctx, size_t *offsets, int n);

/* ---- weights -------------------------------------------------------------- */
/* Upload one RawWeight for use with the fl_op_matvec* entry points (the
 * weight argument of ComputeBackend::batched_dequant_matmul, model.rs:468). */
int fl_weight_upload(fl_ctx *ctx, const fl_raw_weight *w, fl_weight **out);
void fl_weight_free(fl_ctx *ctx, fl_weight *w);

/* ---- per-op entry points (device pointers) --------------------------------- */
/* quantize_input_q8_0_into (model.rs:5534-5571). n % 32 == 0. */
int fl_op_quantize_q8(fl_ctx *ctx, const float *x, int n, int8_t *q, float *scales,
                      int32_t *sums);
/* rmsnorm_quantize_q8_0_into (model.rs:5581-5640) when order == 0:
 * normed = (x*w)*inv_rms; order == 1 is rmsnorm_into followed by
 * quantize_input_q8_0_into (model.rs:2040-2095, the Q4_K path):
 * normed = (x*inv_rms)*w. */
int fl_op_rmsnorm_quantize_q8(fl_ctx *ctx, const float *x, const float *w, int n, float eps,
                              int order, int8_t *q, float *scales, int32_t *sums);
/* rmsnorm_into (model.rs:7456-7477). */
int fl_op_rmsnorm(fl_ctx *ctx, const float *x, const float *w, int n, float eps, float *out);
/* matvec_q8_0_preq_into (model.rs:7976-8103) / matvec_q4k_q8_into
 * (model.rs:9672-9779) over a Q8_0-quantized input. */
int fl_op_matvec_q8in(fl_ctx *ctx, const fl_weight *w, const int8_t *q, const float *scales,
                      const int32_t *sums, float *out);
/* CpuBackend::batched_dequant_matmul (model.rs:740-1036) over n_tokens
 * (1..64; more than 16 take the prefill kernel) Q8_0-quantized input rows: q [n][cols] int8, scales / sums
 * [n][cols/32]; out [n][rows] f32.  Every row of out is the single-token
 * matvec_q8_0_preq_into / matvec_q4k_q8_into of that input row (the same
 * per-block integer dots, formed on int8 MFMA).  Synchronises. */
int fl_op_batched_matvec_q8in(fl_ctx *ctx, const fl_weight *w, int n_tokens, const int8_t *q,
                              const float *scales, const int32_t *sums, float *out);
/* ComputeBackend::batched_dequant_matmul(&RawWeight, input, batch)
 * (model.rs:468; CPU semantics model.rs:740-1036): input [batch][cols] f32
 * rows (device), each quantized on the device with quantize_input_q8_0_into,
 * then the quantized matvec of every row: out [batch][rows] (device).  Q8_0 /
 * Q4_K weights; any batch (16 rows per int8-MFMA GEMM).  Synchronises. */
int fl_op_batched_dequant_matmul(fl_ctx *ctx, const fl_weight *w, const float *input, int batch,
                                 float *out);
/* ComputeBackend::prefill_attention_gpu (model.rs:336-368; softcap 0):
 * causal attention of seq_len tokens, token t over keys / values 0..t, each
 * as cpu_grouped_query_attention (model.rs:9849-9966).  q [seq_len][nh*hd],
 * k, v [seq_len][nkv*hd], out [seq_len][nh*hd]: f32 device arrays.
 * Synchronises. */
int fl_op_prefill_attention(fl_ctx *ctx, const float *q, const float *k, const float *v, int seq_len,
                            int num_heads, int num_kv_heads, int head_dim, float *out);
/* The per-block integer dot products of the batched quantized GEMMs above
 * (the same kernels, K split and launches as fl_op_batched_matvec_q8in),
 * read back from the MFMA results: dots[t][row][b] for token t and 32-value
 * block b (Q4_K: b = 8 * super-block + sub-block, sub-blocks 4-7 the high
 * nibbles).  The integer part of batched_dequant_matmul's per-token
 * matvec_q8_0_preq_into / matvec_q4k_q8_into (model.rs:8082-8099, 8997-9014);
 * the parity surface of the verify and prefill GEMMs.  dots: device memory,
 * n_tokens * rows * K/32 int32. */
int fl_op_batched_block_dots(fl_ctx *ctx, const fl_weight *w, int n_tokens, const int8_t *q, const float *scales,
                             const int32_t *sums, int32_t *dots);
/* fl_op_batched_matvec_q8in without any allocation: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * kernels, K split and results as fl_op_batched_matvec_q8in; the K-split
 * partials live in a file-scope device array of 4 Mi floats (16 MiB, one copy
 * per GPU), so calls needing more (splits x n_tokens x rows) are rejected
 * with FL_E_INVALID.  Enqueues on the context stream and returns (no
 * synchronisation).  Every call on one GPU shares that array: calls that
 * overlap in time on one GPU (other streams or contexts) race. */
int fl_op_batched_matvec_q8in_noalloc(fl_ctx *ctx, const fl_weight *w, int n_tokens, const int8_t *q,
                                      const float *scales, const int32_t *sums, float *out);
/* Dequantized-weight x f32-input matvec for n_tokens (1..8) input rows at
 * once (the speculative-verify logits path: matvec_into / matvec_argmax_f32,
 * model.rs:7549 and 8668, per row): x [n][cols], out [n][rows], device
 * pointers.  Q6_K and Q8_0 weights, f16 MFMA with exact weight codes and
 * split (high + residual) f16 inputs. */
int fl_op_batched_matvec_f32in(fl_ctx *ctx, const fl_weight *w, int n_tokens, const float *x,
                               float *out);
/* Dequantized-weight x f32-input matvec (the f32 logits path,
 * matvec_into model.rs:7549 on dequantize_tensor output, gguf.rs:717). */
int fl_op_matvec_f32in(fl_ctx *ctx, const fl_weight *w, const float *x, float *out);
/* Per-block integer dot products of the device dot routine (the bit-exact
 * parity surface of model.rs:8082-8099 and 8997-9014).  Q8_0: rows*bpr
 * int32; Q4_K: rows*bpr*8 int32 ordered (sub0 lo, sub0 hi, sub1 lo, ...). */
int fl_op_block_dots(fl_ctx *ctx, const fl_weight *w, const int8_t *q, int32_t *dots);
/* Dequantize a whole weight to f32 (dequantize_tensor, gguf.rs:717-880). */
int fl_op_dequant(fl_ctx *ctx, const fl_weight *w, float *out);
/* Fused argmax over the output projection: matvec_argmax_q8_0_preq
 * (model.rs:8450), matvec_argmax_q4k_q8_preq (8569) with a Q8 input;
 * matvec_argmax_f32 (8668) with an f32 input (x != NULL, q == NULL).
 * Result: out_idx_val[0] = index (as int64), first maximum on ties;
 * *out_val = winning value. Both device pointers. */
int fl_op_matvec_argmax(fl_ctx *ctx, const fl_weight *w, const int8_t *q, const float *scales,
                        const int32_t *sums, const float *x, int64_t *out_idx, float *out_val);
/* apply_rope_with_table (model.rs:7256-7297) in place on num_heads*head_dim
 * floats, using the host-built libm table of RopeTable::new (7190-7212). */
int fl_op_rope(fl_ctx *ctx, float *data, int num_heads, int head_dim, int pos, float theta);
/* silu_mul_into (model.rs:9783-9796). */
int fl_op_silu_mul(fl_ctx *ctx, const float *gate, const float *up, int n, float *out);
/* cpu_grouped_query_attention_into (model.rs:9849-9966) over a ring cache
 * laid out [slot][num_kv_heads][head_dim] (kv_cache.rs:431-472), attending to
 * slots 0..seq_len-1; kv_format FL_KV_F32 or FL_KV_F16. num_splits <= 0 picks
 * the split count automatically. */
int fl_op_attention(fl_ctx *ctx, const float *q, const void *k_cache, const void *v_cache,
                    int kv_format, int num_heads, int num_kv_heads, int head_dim, int seq_len,
                    int num_splits, float *out);

/* ---- model: ComputeBackend decode hooks ----------------------------------- */
/* init_gpu_kv_cache (model.rs:274) + the config forward_single_token_gpu
 * receives per call (model.rs:555).  Must precede fl_upload_weights. */
int fl_model_init(fl_ctx *ctx, const fl_model_config *cfg, int kv_format);
/* upload_weights_to_gpu (model.rs:526) taking raw layers as
 * Model::set_raw_weights does (model.rs:1411-1452).  layers: 7*num_layers
 * weights ordered wq, wk, wv, wo, w_gate, w_up, w_down per layer; all seven
 * share one format (FL_Q8_0 or FL_Q4K).  attn_norms / ffn_norms: num_layers
 * host pointers to hidden_dim floats.  output: NULL when tied to the
 * embedding (flare-loader/src/weights.rs:50-51). */
int fl_upload_weights(fl_ctx *ctx, const fl_raw_weight *layers, const float *const *attn_norms,
                      const float *const *ffn_norms, const float *output_norm,
                      const fl_raw_weight *embedding, const fl_raw_weight *output);
/* has_gpu_weights (model.rs:537) / has_gpu_kv_cache (model.rs:299). */
int fl_has_weights(const fl_ctx *ctx);
int fl_has_kv_cache(const fl_ctx *ctx);
/* gpu_kv_write (model.rs:287): store one token's K and V (host floats,
 * num_kv_heads*head_dim each) at ring slot `position` of `layer`. */
int fl_kv_write(fl_ctx *ctx, int layer, int position, const float *key, const float *value);
/* Write n consecutive token rows (host floats, [n][num_kv_heads*head_dim]
 * each for K and V) at positions pos0..pos0+n-1 of `layer`: gpu_kv_write
 * (model.rs:287) for n rows at once.  Q8 rows are quantized on the device;
 * KIVI rows enter the ring and the groups that leave it are quantized. */
int fl_kv_write_batch(fl_ctx *ctx, int layer, int pos0, int n, const float *keys, const float *values);
/* grouped_query_attention_from_gpu_cache (model.rs:311): decode attention of
 * one query token (host floats, num_heads*head_dim, RoPE applied) over slots
 * 0..seq_len-1 of `layer`'s cache; writes num_heads*head_dim host floats.
 * seq_len must be the number of tokens written (the KIVI ring holds only the
 * newest ones). */
int fl_gqa_from_cache(fl_ctx *ctx, int layer, const float *q, int seq_len, float *out);
/* Model::reset / KvCache::clear (model.rs:1591, kv_cache.rs:534-545). */
int fl_reset(fl_ctx *ctx);
/* forward_greedy (model.rs:1872-1942) when out_logits == NULL, else
 * forward_single_token_gpu (model.rs:555) + argmax: writes vocab_size host
 * floats of logits.  The token is processed at position `pos` (the KV ring
 * slot), attending to pos+1 slots. */
int fl_decode_step(fl_ctx *ctx, uint32_t token, int pos, float *out_logits, int32_t *out_token,
                   float *out_val);
/* forward_single_token_gpu(token_embedding, pos, ...) (model.rs:555-557)
 * exactly: the step's input is the caller's f32 embedding row (hidden_dim
 * host floats) instead of a token id; otherwise as fl_decode_step. */
int fl_decode_step_embed(fl_ctx *ctx, const float *embedding, int pos, float *out_logits,
                         int32_t *out_token, float *out_val);
/* Greedy generation (Generator::step loop, flare-core/src/generate.rs:186-206):
 * feeds the n_prompt tokens one per step from position 0, then writes n_gen
 * generated tokens to out_tokens.  Runs device-resident: one HIP graph replay
 * per token, one host synchronisation at the end. */
int fl_generate(fl_ctx *ctx, const uint32_t *prompt, int n_prompt, int n_gen,
                uint32_t *out_tokens);

/* Speculative verify: n_tokens (1..16) draft tokens at positions
 * pos0..pos0+n_tokens-1 through the model in one pass: every projection as
 * batched_dequant_matmul (model.rs:740-1036, int8 MFMA), causal attention
 * (the default prefill_attention_gpu, model.rs:336-368: token i attends
 * 0..pos0+i), their K/V written to the cache, then the fused argmax per token
 * (forward_greedy, model.rs:1872-1942).  out_tokens[i] (and out_vals[i] if
 * not NULL) is the greedy token after draft i -- what n_tokens sequential
 * fl_decode_step calls return; Generator::speculative_step
 * (generate.rs:244-312) accepts drafts while they match.  Cache slots beyond
 * the accepted prefix are simply rewritten by later steps. */
int fl_verify(fl_ctx *ctx, const uint32_t *tokens, int n_tokens, int pos0, int32_t *out_tokens,
              float *out_vals);

/* Model::forward_prefill (model.rs:2578-3040): n_tokens prompt tokens at
 * positions pos0..pos0+n_tokens-1 in batched passes of up to 16 tokens (the
 * fl_verify pass: int8-MFMA projections, causal attention over the cache
 * and the tokens before each one in the batch, K/V written to the cache),
 * then the output projection of the last token only.  The reference starts
 * from an empty cache (pos0 = 0); pos0 > 0 continues a cache whose slots
 * 0..pos0-1 are written.  out_logits (vocab_size host floats) may be NULL:
 * then only the fused argmax runs; *out_token / *out_val (either may be
 * NULL) receive the greedy token after the last prompt token. */
int fl_prefill(fl_ctx *ctx, const uint32_t *tokens, int n_tokens, int pos0, float *out_logits,
               int32_t *out_token, float *out_val);

/* n_steps greedy steps (forward_greedy, model.rs:1872-1942) starting with
 * `token` at position `pos`, device-resident (one HIP graph replay per step,
 * one host synchronisation at the end): out_tokens[i] is the greedy token
 * after step pos+i, which is the input of step pos+i+1.  The Generator's
 * plain greedy steps (generate.rs:186-206) after fl_prefill. */
int fl_decode_run(fl_ctx *ctx, uint32_t token, int pos, int n_steps, uint32_t *out_tokens);

/* Enqueue n_steps more device-resident greedy steps after fl_generate (no
 * host synchronisation; tokens land in the device token buffer). */
int fl_decode_continue(fl_ctx *ctx, int n_steps);
/* Copy tokens[start, start+n) of the device token buffer (prompt tokens
 * followed by generated tokens) to the host. */
int fl_read_tokens(fl_ctx *ctx, int start, int n, uint32_t *out);

/* ---- sampling (flare-core/src/sampling.rs) ------------------------------------ */
/* SamplingParams (sampling.rs:19-54) without the self-speculation fields
 * (layer-skipping drafts are not built). */
typedef struct {
    float temperature, top_p;
    int top_k;
    float repeat_penalty, min_p;
    int speculative; /* n-gram speculative decoding (greedy only) */
} fl_sampling_params;
/* SamplingParams::default (sampling.rs:56-70). */
void fl_sampling_params_default(fl_sampling_params *p);
/* One token from a logits row on the device, as Generator::step does after
 * its forward (generate.rs:210-230): apply_repeat_penalty over prev_tokens
 * (host array, every occurrence counts), apply_temperature, then
 * sample_greedy (temperature 0) / sample_top_p / sample_min_p / sample_top_k
 * by the reference's priority, with rng_val as the uniform draw.  logits: n
 * device floats (left unchanged).  Candidate sets are ordered by descending
 * probability, ties by ascending index (top-k: the reference walks them in
 * select_nth_unstable's order instead).  Synchronises. */
int fl_op_sample(fl_ctx *ctx, const float *logits, int n, const fl_sampling_params *params,
                 const uint32_t *prev_tokens, int n_prev, float rng_val, int32_t *out_token);
/* forward_single_token_gpu (model.rs:555) for `token` at `pos`, then
 * fl_op_sample over the device logits: no logits readback. */
int fl_decode_step_sample(fl_ctx *ctx, uint32_t token, int pos, const fl_sampling_params *params,
                          const uint32_t *prev_tokens, int n_prev, float rng_val, int32_t *out_token);

/* ---- generation loop (flare-core/src/generate.rs), host code ----------------- */
/* NgramCache (generate.rs:37-103): n = 2, 3, 4; at most 5 drafts; cleared
 * when it exceeds 10 000 entries.  Host only (no GPU needed). */
typedef struct fl_ngram fl_ngram;
fl_ngram *fl_ngram_create(void);
void fl_ngram_destroy(fl_ngram *c);
/* record (generate.rs:55-75): the n-grams ending at tokens[n-1]. */
void fl_ngram_record(fl_ngram *c, const uint32_t *tokens, size_t n);
/* record_prompt_ngrams (generate.rs:166-182): every n-gram of tokens. */
void fl_ngram_record_all(fl_ngram *c, const uint32_t *tokens, size_t n);
/* lookup_drafts (generate.rs:79-92): writes up to 5 drafts, returns the count. */
int fl_ngram_lookup(const fl_ngram *c, const uint32_t *tokens, size_t n, uint32_t *out);
size_t fl_ngram_entries(const fl_ngram *c);

/* SpeculativeStats (generate.rs:22-30). */
typedef struct {
    uint64_t attempts, drafted, accepted;
} fl_spec_stats;
typedef float (*fl_rng_fn)(void *user);
/* on_token (generate.rs:409-416): return 0 to stop. */
typedef int (*fl_token_fn)(uint32_t token, size_t step, void *user);
/* Generator (generate.rs:106-560) over a context holding a model, positions
 * from 0.  Speculative steps verify the n-gram drafts in one fl_verify pass
 * over the inputs the reference's sequential forwards take
 * ([last, d0, .., d(k-2)]); accepted tokens, positions and statistics are
 * the reference's.  Self-speculation (layer skipping) is not built. */
typedef struct fl_generator fl_generator;
int fl_generator_create(fl_ctx *ctx, const fl_sampling_params *params, fl_generator **out);
void fl_generator_destroy(fl_generator *g);
/* Generator::prefill (generate.rs:139-163) through fl_prefill; out_logits
 * (vocab floats) may be NULL. */
int fl_generator_prefill(fl_generator *g, const uint32_t *prompt, int n, float *out_logits);
/* Generator::step (generate.rs:186-238): the forward of the last token at
 * the current position, then greedy / sampled token. */
int fl_generator_step(fl_generator *g, float rng_val, uint32_t *out_token);
/* Generator::generate (generate.rs:409-531): prefill, then up to max_tokens
 * tokens (speculative steps when enabled and greedy), stopping at eos (< 0:
 * none) or when on_token returns 0.  out_tokens holds max_tokens entries;
 * *n_out = tokens written.  rng / on_token may be NULL. */
int fl_generator_generate(fl_generator *g, const uint32_t *prompt, int n_prompt, int max_tokens,
                          int64_t eos, fl_rng_fn rng, void *rng_user, fl_token_fn on_token,
                          void *token_user, uint32_t *out_tokens, int *n_out);
/* speculative_stats (generate.rs:555-557). */
int fl_generator_stats(const fl_generator *g, fl_spec_stats *out);
/* position / tokens (generate.rs:547-553): tokens returns the count and
 * copies up to cap of them when out != NULL. */
int fl_generator_position(const fl_generator *g);
int fl_generator_tokens(const fl_generator *g, uint32_t *out, int cap);

/* ---- GGUF files (flare-loader/src/gguf.rs), host code ------------------------- */
/* A parsed GGUF v2 / v3 file (GgufFile::parse_header, gguf.rs:131-204): magic,
 * version, the reference's limits (1e6 tensors, 1e5 metadata entries, 1 MiB
 * strings), metadata, tensor infos, tensor data at the next 32-byte boundary.
 * fl_gguf_open memory-maps the file read-only; fl_gguf_open_memory copies a
 * buffer.  Errors: FL_E_INVALID / FL_E_UNSUPPORTED with fl_last_error(NULL). */
typedef struct fl_gguf fl_gguf;
int fl_gguf_open(const char *path, fl_gguf **out);
int fl_gguf_open_memory(const void *data, size_t len, fl_gguf **out);
void fl_gguf_close(fl_gguf *g);
int fl_gguf_version(const fl_gguf *g);
uint64_t fl_gguf_data_offset(const fl_gguf *g);
int fl_gguf_tensor_count(const fl_gguf *g);
/* find_tensor (gguf.rs:207): index, or -1. */
int fl_gguf_find_tensor(const fl_gguf *g, const char *name);
/* TensorInfo (gguf.rs:103-124): dims (up to 8) in file order [cols, rows, ...],
 * ggml type id, offset within the data section, byte size (0 when the type's
 * block size is unknown). */
int fl_gguf_tensor_info(const fl_gguf *g, int index, const char **name, int *n_dims, uint64_t *dims,
                        uint32_t *ggml_type, uint64_t *offset, uint64_t *nbytes);
/* Metadata as an integer (meta_usize: u8/u16/u32/u64/i32/i64, gguf.rs:218),
 * a float (meta_f32: f32/f64, gguf.rs:240) or a string (NULL if absent). */
int fl_gguf_meta_u64(const fl_gguf *g, const char *key, uint64_t *out);
int fl_gguf_meta_f32(const fl_gguf *g, const char *key, float *out);
const char *fl_gguf_meta_str(const fl_gguf *g, const char *key);
/* to_model_config (gguf.rs:241-346): llama / qwen2 / mistral / phi3 / gemma2
 * (*arch = 0..4), vocab from token_embd.weight's second dimension, the
 * reference's defaults for optional keys; head_dim = hidden / heads. */
int fl_gguf_model_config(const fl_gguf *g, fl_model_config *cfg, int *arch);
/* read_raw_weight (gguf.rs:616-653) without a copy: data points into the
 * mapping; num_rows = last dimension, blocks_per_row = ceil(cols / block).
 * Q8_0, Q4_K, Q6_K and F32 tensors (the formats of this backend's path). */
int fl_gguf_raw_weight(const fl_gguf *g, const char *name, fl_raw_weight *out);
/* An F32 / F16 tensor of n elements as f32 (norm weights). */
int fl_gguf_tensor_f32(const fl_gguf *g, const char *name, float *out, size_t n);
/* A whole model from a GGUF file: the config (max_seq_len > 0 overrides the
 * context length), init_gpu_kv_cache, the blk.N.* weights and norms
 * (weights.rs:30-66, gguf.rs:661-688; output tied to token_embd when absent),
 * upload_weights_to_gpu streaming from the mapping.  llama / mistral only. */
int fl_model_load_gguf(fl_ctx *ctx, const fl_gguf *g, int kv_format, int max_seq_len);

/* ---- measurement helpers ---------------------------------------------------- */
/* Enqueue `iters` launches of one decode kernel for `which` (0=qkv, 1=wo,
 * 2=gate_up, 3=down, 4=output argmax, 5=attention at the current position;
 * 6..9 = the verify GEMM of qkv / wo / gate_up / down for 8 tokens, over the
 * verify activation buffers) on the context stream, launch i using layer (first_layer + i) % num_layers,
 * reading the model's live activation buffers.  Writes the algorithmic HBM
 * bytes of one launch (GGUF weight bytes; K+V bytes for attention) to
 * *bytes_per_launch.  No counterpart in the reference: measurement only. */
int fl_bench_layer_kernel(fl_ctx *ctx, int which, int first_layer, int iters, double *bytes_per_launch);
/* Enqueue `iters` decode attention launches over slots 0..seq_len-1 (layer
 * i % num_layers, the query left by the last fl_gqa_from_cache / decode step)
 * and synchronise; writes the algorithmic K+V bytes of one launch.  Needs no
 * weights.  Measurement only. */
int fl_bench_attention(fl_ctx *ctx, int seq_len, int iters, double *bytes_per_launch);
/* Name of the device kernel fl_bench_layer_kernel launches for `which`. */
const char *fl_bench_kernel_name(fl_ctx *ctx, int which);

/* ---- synthetic model generation (host only; no reference counterpart: the
 * reference loads real GGUF files) --------------------------------------- */
/* Fill out[n] with N(mean, std) floats from a counter-based generator keyed
 * by (seed, index), so any slice is reproducible independently. */
void fl_synth_normal(uint64_t seed, uint64_t offset, size_t n, float mean, float std, float *out);
/* Quantize rows x cols f32 into GGUF block bytes of `format`. Returns the
 * byte count written (0 on bad shape).  Q4_K uses flarellm's layout
 * (model.rs:8700-8719, quantize.rs:386-423). */
size_t fl_synth_quantize(const float *src, size_t rows, size_t cols, int format, uint8_t *out);
size_t fl_format_row_bytes(int format, size_t cols);

#ifdef __cplusplus
}
#endif
#endif
