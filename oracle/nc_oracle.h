/*
 * nc_oracle.h -- CPU oracle for the speculative-decoding verify path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is a plain C++ restatement of the
 * reference's portable (x86, scalar) CPU path: the same per-element operation
 * order, the same f32 roundings, glibc libm for expf/powf/sinf/cosf, no FMA
 * contraction (built with -ffp-contract=off).  It is the checker the GPU
 * product is compared against.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product library never links it.
 *
 * Every function names the reference file:line it restates.  Paths are
 * relative to the reference repository root (src/...).
 *
 * Parity pinning (what fixes each function independently of this code):
 *   or_f16_to_f32 / or_f32_to_f16_trunc : reference known answers (q8.rs:5156-5195)
 *                                          + exhaustive IEEE half decode in tests
 *   or_dot_q4_0_q8_0                     : nibble-order known answer (q8.rs:4514-4530),
 *                                          dot_i8_scalar = 12 (q8.rs:4343-4348), brute force
 *   or_quantize_q8_0                     : closed-form ties (round half away from zero)
 *   or_matmul_q4_0                       : brute-force dequantised reference <= 1e-5
 *                                          (inference.rs:6028-6075) + exact block dots
 *   or_matmul_q4_k                       : dequantised reference <= 1e-4 (inference.rs:6517-6558)
 *   or_matmul_q5_k                       : the reference's dequantised fixture <= 1e-4
 *                                          (inference.rs:6561-6603), float64 decode, batch == single
 *   or_matmul_q8_0                       : block-dot known answer (q8.rs:5050-5058), float64
 *                                          dequantised reference, an order-fixing cancellation row
 *   or_quantize_q4_0_tied                : reconstruction error <= |d| (q8.rs:4187-4245)
 *   or_rms_norm / or_rope / or_softmax   : closed forms (inference.rs:7423-7468)
 *   model forward                        : batch == single-token per row (inference.rs:6866-6912),
 *                                          draft == target => acceptance exactly 1.0
 *   philox                               : Salmon et al. SC'11 known-answer vectors
 * The oracle-drafter and Philox stochastic acceptance have no reference
 * counterpart: "parity unpinned" versus the reference (they are pinned only by
 * this build's own specification and the Philox known-answer vectors).
 */
#ifndef NC_ORACLE_H
#define NC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------- block formats (src/q8.rs) ---------------- */
float or_f16_to_f32(uint16_t bits);            /* q8.rs:3626 fast_f16_to_f32 */
uint16_t or_f32_to_f16_trunc(float value);     /* q8.rs:3644 fast_f32_to_f16 */
int32_t or_dot_q4_0_q8_0(const uint8_t* block18, const int8_t* x32); /* q8.rs:2699 */
int32_t or_dot_i8(const int8_t* a, const int8_t* b, int64_t n);      /* q8.rs:3376 */
/* Q4_K: per 32-sub-block W_j = sum nib*x, A_j = sum x (q8.rs:1339-1376). */
void or_q4_k_subblock_ints(const uint8_t* block144, const int8_t* x256, int32_t* W8, int32_t* A8);
float or_q4_k_dot(const uint8_t* block144, const int8_t* x256, const float* xs8); /* q8.rs:1339 */
/* Q4_K dequantisation (q8.rs:1240-1264). */
void or_q4_k_dequantize(const uint8_t* block144, float* out256);
int or_dequantize_f32(int type, const uint8_t* bytes, int64_t n, float* out);
float or_q6_k_dot(const uint8_t* block210, const int8_t* x256, const float* xs8);
void or_matmul_q6_k(float* out, const int8_t* x, const float* xs, const uint8_t* w, int64_t N, int64_t M, int64_t K,
                    int nthreads);

/* inference.rs:935-1029 (scalar x86 path): per 32-block f32 scale amax/127. */
void or_quantize_q8_0(const float* x, int64_t n, int8_t* q, float* scales);
/* q8.rs:2442-2488: tied-head requantisation to Q4_0 (truncating f16 scale). */
void or_quantize_q4_0_tied(const float* values, int64_t rows, int64_t cols, uint8_t* out18);

/* ---------------- matmuls (src/inference.rs) ---------------- */
/* inference.rs:1385-1418 / 1525-1574: out[t][r] = sum_b ((ws*xs)*dot) in block order.
 * w = row-major GGUF Q4_0 blocks [M][K/32][18]. out is token-major [N][M]. */
void or_matmul_q4_0(float* out, const int8_t* x, const float* xs, const uint8_t* w,
                    int64_t N, int64_t M, int64_t K, int nthreads);
/* int32 per-block dots [N][M][K/32] (q8.rs:2699 for every block). */
void or_matmul_q8_0(float* out, const int8_t* x, const float* xs, const uint8_t* w, int64_t N, int64_t M, int64_t K,
                    int nthreads);
void or_matmul_q5_k(float* out, const int8_t* x, const float* xs, const uint8_t* w, int64_t N, int64_t M, int64_t K,
                    int nthreads);
float or_q5_k_dot(const uint8_t* blk, const int8_t* x, const float* xs);
void or_matmul_q4_0_blockdots(int32_t* dots, const int8_t* x, const uint8_t* w,
                              int64_t N, int64_t M, int64_t K, int nthreads);
/* inference.rs:2006-2132 (x86 path): w = [M][K/256][144]. */
void or_matmul_q4_k(float* out, const int8_t* x, const float* xs, const uint8_t* w,
                    int64_t N, int64_t M, int64_t K, int nthreads);

/* ---------------- elementwise / row ops (src/inference.rs) ---------------- */
void or_rms_norm(float* out, const float* x, const float* w, int64_t n, float eps); /* :697 */
/* :731-798 / :860-933; style 0 = NORM (pairs 2i,2i+1), 1 = NEOX. */
void or_rope(float* data, int64_t pos, int64_t heads, int64_t head_dim, int64_t rope_dim,
             float freq_base, int style);
/* (sin, cos) table entry for pair i at pos (inference.rs:880-901). */
void or_rope_sincos(int64_t pos, int64_t i, int64_t rope_dim, float freq_base, float* s, float* c);
/* Llama-3 scaled RoPE (inference.rs:874-893; scaling = {factor, original_context_length,
 * low_freq_factor, high_freq_factor} or NULL for none). */
float or_rope_theta(int64_t i, int64_t rope_dim, float freq_base, const float* scaling);
void or_rope_sincos_scaled(int64_t pos, int64_t i, int64_t rope_dim, float freq_base, const float* scaling,
                           float* s, float* c);
void or_rope_scaled(float* data, int64_t pos, int64_t heads, int64_t head_dim, int64_t rope_dim,
                    float freq_base, int style, const float* scaling);
void or_softmax(float* x, int64_t n);          /* :3522-3540 */
float or_expf(float x);                        /* Rust f32::exp == glibc expf */
int64_t or_expf_mismatches(uint32_t first, int64_t count, const float* vals, int nthreads, uint32_t* first_bad);
void or_silu_mul(float* out, const float* gate, const float* up, int64_t n); /* :3367-3390 */
int64_t or_argmax(const float* logits, int64_t n); /* :4834-4845 first max wins */
float or_rand_simple(uint64_t* state);             /* inference.rs:4876-4883 LCG draw */
/* inference.rs:4834-4873 sample_logits (temp <= 0: argmax, no draw) */
int64_t or_sample_logits(const float* logits, int64_t V, float temp, uint64_t* state);
/* One attention head over an f32 KV slice, inference.rs:4242-4292 (x86 path).
 * k_cache/v_cache: [>=pos+1][kv_width]; scores scratch >= pos+1. */
void or_attention_head(float* out_head, float* scores, const float* q_head,
                       const float* k_cache, const float* v_cache, int64_t pos,
                       int64_t kv_width, int64_t kv_h, int64_t head_dim, float scale);

/* Split-order attention head (the device's NC_ATTN_SPLIT; no reference counterpart): 64-position
 * chunks with per-chunk max / sum of exp / exp-weighted V, combined in chunk order; v past plast
 * (the pass's last position) read as 0.  out_head is overwritten. */
void or_attention_head_split(float* out_head, const float* q_head, const float* k_cache, const float* v_cache,
                             int64_t pos, int64_t plast, int64_t kv_width, int64_t kv_h, int64_t head_dim,
                             float scale);

/* ---------------- Philox4x32-10 (Salmon et al., SC'11) ---------------- */
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* ---------------- model + session ---------------- */
typedef struct or_model or_model;
typedef struct or_session or_session;

/* Loads a GGUF file (or an in-memory GGUF image).  Returns NULL on error and
 * writes a message into err.  Mirrors gguf.rs:454-551 + model.rs:48-186, 461-545. */
or_model* or_model_load(const char* path, int nthreads, char* err, int errlen);
or_model* or_model_load_memory(const void* data, size_t size, int nthreads, char* err, int errlen);
void or_model_free(or_model* m);
/* out[0..15]: context_length, d, layers, ffn, heads, kv_heads, head_dim, rope_dim,
 * vocab, attn_width, kv_width, has_output_weight, weight_type(2=Q4_0,12=Q4_K), 0,0,0 */
void or_model_info(const or_model* m, int64_t* out16);
/* rope_freq_base, rms_eps */
void or_model_info_f(const or_model* m, float* out2);
/* Copies the tied/untied head as Q4_0 GGUF blocks [V][d/32][18] (tied heads are
 * requantised per q8.rs:2442); returns bytes written or -1. */
int64_t or_model_head_q4_0(const or_model* m, uint8_t* out, int64_t cap);

/* Host threads the model's matmuls and attention heads use (row-parallel as rayon). */
void or_model_set_threads(or_model* m, int nthreads);

or_session* or_session_create(or_model* m, int64_t max_ctx, int64_t max_batch);
/* Attention order of the session's passes: 0 the reference's (default), 1 the split order of
 * or_attention_head_split (the checker of the device's NC_ATTN_SPLIT). */
void or_session_set_attention(or_session* s, int order);
/* N(0, 1) KV fill (no reference counterpart): or_synth_kv_values writes
 * elements [start, start + count) (even) of the stream of layer `layer`'s keys (kind 0) or values
 * (kind 1): Philox4x32-10, counter (pair index, 2 * layer + kind, purpose 10), key seed, Box-Muller
 * in double, rounded to f32.  or_session_fill_kv puts row p = elements [p * kv_width, (p + 1) *
 * kv_width) into KV rows [0, n) of every layer, so a pass at start_pos = n attends over n
 * positions of N(0, 1) keys and values, the same ones the device's nc_session_fill_kv writes. */
void or_synth_kv_values(uint64_t seed, int32_t layer, int32_t kind, int64_t start, int64_t count, float* out);
void or_session_fill_kv(or_session* s, int64_t n, uint64_t seed);
void or_session_free(or_session* s);
/* prefill_pass_batch (inference.rs:3695-3744): writes KV for start_pos..+n and
 * keeps per-row final hidden states. */
void or_prefill_pass_batch(or_session* s, const uint32_t* toks, int64_t n, int64_t start_pos);
/* forward_pass (inference.rs:3649, 4460-4832): single token, logits in session. */
void or_forward_pass(or_session* s, uint32_t tok, int64_t pos);
/* compute_logits_from_hidden (inference.rs:4783) for batch row `row`. */
void or_batch_row_logits(or_session* s, int64_t row, float* logits_out);
const float* or_session_logits(const or_session* s);
const float* or_session_batch_hidden(const or_session* s);

/* k+1 greedy verify (cluster_tcp_smoke.rs:905-979 semantics): one batched pass
 * over toks[0..n) at start_pos, then argmax of every row's logits.
 * preds[n]; margins[n] = top1 - top2 logit (may be NULL). */
void or_verify_greedy(or_session* s, const uint32_t* toks, int64_t n, int64_t start_pos,
                      uint32_t* preds, float* margins, float* logits_out /* [n][V] or NULL */);

/* Greedy decode baseline: prompt prefill (main.rs:9415-9485 chunks of
 * prefill_batch, last prompt token via forward_pass) then n_new greedy tokens
 * (plain loop). out[n_new]. Returns 0. */
int or_generate_greedy(or_session* s, const uint32_t* prompt, int64_t n_prompt, int64_t n_new,
                       int64_t prefill_batch, uint32_t* out);

/* The plain decode loop at temperature temp (main.rs:9894-9928, greedy at temp <= 0): each
 * token drawn with or_sample_logits (*rng_state, may be NULL at temp <= 0) from the live
 * logits; decoding ends before a stop token (stop[n_stop]), at the session context or after
 * n_new tokens.  Returns the number of tokens written to out. */
int64_t or_generate_plain(or_session* s, const uint32_t* prompt, int64_t n_prompt, int64_t n_new, float temp,
                          uint64_t* rng_state, const uint32_t* stop, int64_t n_stop, int64_t prefill_batch,
                          uint32_t* out);

/* Draft-model speculative decoding (speculative.rs:299-494) for n_new tokens.
 * target/draft sessions; temp <= 0 greedy.  out[n_new]; stats[2] = drafted,
 * accepted; steps_out = number of steps.  Returns number of tokens written. */
int64_t or_generate_speculative_draft(or_session* target, or_session* draft,
                                      const uint32_t* prompt, int64_t n_prompt, int64_t n_new,
                                      int64_t draft_k, int64_t prefill_batch,
                                      uint32_t* out, int64_t* stats, int64_t* steps_out);
/* The same at temperature temp > 0: every draw through or_sample_logits with the LCG state
 * *rng_state, in the reference's order (drafts, then one per verified position, then the
 * trailing token), acceptance by id match.  stop[n_stop]: is_stop_token (a drafted stop token
 * ends drafting, an accepted one ends verification with no trailing draw) and the generate
 * loop's turn end (tokens after the first stop token of a step are dropped, the stop token
 * itself too, and decoding ends). */
int64_t or_generate_speculative_draft_temp(or_session* target, or_session* draft, const uint32_t* prompt,
                                           int64_t n_prompt, int64_t n_new, int64_t draft_k, float temp,
                                           uint64_t* rng_state, const uint32_t* stop, int64_t n_stop,
                                           int64_t prefill_batch, uint32_t* out, int64_t* stats,
                                           int64_t* steps_out);

/* k+1 speculative decoding with the seeded oracle drafter (no reference
 * counterpart): draft i of a step at position p copies greedy[p - n_prompt]
 * when u(seed, p) < alpha, else a uniform id.  Emits the target greedy stream.
 * stats[2] = drafted, accepted. Returns tokens written. */
int64_t or_generate_speculative_oracle(or_session* target, const uint32_t* prompt, int64_t n_prompt,
                                       int64_t n_new, int64_t k, float alpha, uint64_t seed,
                                       const uint32_t* greedy, int64_t prefill_batch,
                                       uint32_t* out, int64_t* stats, int64_t* steps_out);

/* NGramDrafter::draft (speculative.rs:81-103): writes up to max_tokens proposals to out,
 * returns how many. */
int64_t or_ngram_draft(const uint32_t* history, int64_t len, int64_t min_ngram, int64_t max_ngram,
                       int64_t max_tokens, uint32_t* out);
/* n-gram prompt-lookup speculation, greedy: ngram_speculative_step (speculative.rs:122-286)
 * driven by main.rs:9729-9776 in the k+1 verify form (cluster_tcp_smoke.rs:905-979); the
 * stream stops before the first of the n_stop stop tokens.  stats[2] = drafted, accepted.
 * Returns tokens written (<= n_new). */
int64_t or_generate_speculative_ngram(or_session* target, const uint32_t* prompt, int64_t n_prompt,
                                      int64_t n_new, int64_t k, int64_t min_ngram, int64_t max_ngram,
                                      const uint32_t* stop, int64_t n_stop, int64_t prefill_batch,
                                      uint32_t* out, int64_t* stats, int64_t* steps_out);
/* At temperature temp > 0 (temp <= 0: the greedy loop above): the step itself, t0 and every
 * verified row drawn with or_sample_logits (*rng_state) in its order, a mismatch run as a
 * corrective forward. */
int64_t or_generate_speculative_ngram_temp(or_session* target, const uint32_t* prompt, int64_t n_prompt,
                                           int64_t n_new, int64_t k, int64_t min_ngram, int64_t max_ngram,
                                           float temp, uint64_t* rng_state, const uint32_t* stop, int64_t n_stop,
                                           int64_t prefill_batch, uint32_t* out, int64_t* stats,
                                           int64_t* steps_out);

/* Oracle-drafter proposal for absolute position p (shared spec with the product). */
uint32_t or_oracle_draft(uint64_t seed, int64_t p, float alpha, const uint32_t* greedy,
                         int64_t n_prompt, int64_t n_greedy, uint32_t vocab);
/* Seeded uniform prompt ids: ids[i] = philox(seed, i) mod vocab. */
void or_uniform_prompt(uint64_t seed, int64_t n, uint32_t vocab, uint32_t* ids);

/* Stochastic (temperature) speculative acceptance with Philox uniforms, one
 * k+1 verify.  p_logits [k+1][V] target logits, q_probs [k][V] draft probs,
 * drafts[k].  Writes accepted count, next token.  See the product header for
 * the exact specification (no reference counterpart). */
void or_stochastic_accept(const float* p_logits, const float* q_probs, const uint32_t* drafts,
                          int64_t k, int64_t V, float temp, uint64_t seed, int64_t start_pos,
                          int64_t* n_accepted, uint32_t* next_token);
/* Softmax with temperature used by the stochastic spec: probs[V]. */
void or_temperature_probs(const float* logits, int64_t V, float temp, float* probs);
/* Fixed-point inverse-CDF sample: weights W_j = floor(probs_j * 2^40), u = k24 / 2^24
 * (k24 = floor(u * 2^24)); returns the first j whose inclusive prefix of W exceeds
 * floor(k24 * sum(W) / 2^24); 0 when every weight is zero. */
uint32_t or_sample_inverse_cdf(const float* probs, int64_t V, float u);
/* Draft-model speculative sampling at temperature temp in the k+1 form (draft and
 * target sessions share the vocabulary).  out[n_new]; stats[2] = drafted, accepted.
 * Returns tokens written. */
int64_t or_generate_speculative_stochastic(or_session* target, or_session* draft, const uint32_t* prompt,
                                           int64_t n_prompt, int64_t n_new, int64_t k, float temp,
                                           uint64_t seed, int64_t prefill_batch, uint32_t* out,
                                           int64_t* stats, int64_t* steps_out);

#ifdef __cplusplus
}
#endif
#endif
