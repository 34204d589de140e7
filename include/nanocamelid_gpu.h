/*
 * nanocamelid_gpu.h -- C ABI of the MI355X speculative-decoding verify path.
 *
 * One shared library, libnanocamelid_hip.so, built with hipcc for gfx950.
 * Plain pointers and sizes only; opaque handles; every function returns an int
 * status (NC_OK = 0, negative on error) and never aborts.  nc_last_error()
 * returns the thread-local message of the last failure.  The library is meant to
 * be bound from the reference's Rust host through a thin `-sys` crate; every
 * entry point cites the reference interface it replaces (paths relative to the
 * reference repository root).
 *
 * Ownership: host buffers are borrowed for the duration of a call.  Device
 * memory (weights, KV cache, workspaces) is owned by model/session handles and
 * released by the matching *_free.  A model is immutable after load and may be
 * shared read-only by sessions; a session is used by one host thread at a time
 * and owns one HIP stream.  Steps allocate nothing.
 */
#ifndef NANOCAMELID_GPU_H
#define NANOCAMELID_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- status codes */
#define NC_OK 0
#define NC_EINVAL (-1)  /* bad argument (shape, null pointer, unsupported format) */
#define NC_ENOMEM (-2)  /* device or host allocation failed */
#define NC_EHIP (-3)    /* a HIP runtime call failed */
#define NC_EFORMAT (-4) /* malformed or unsupported GGUF */
#define NC_ERANGE (-5)  /* batch/context bounds (inference.rs:3712-3722 asserts) */

/* GGUF tensor type ids used by this path (gguf.rs:83-115). */
#define NC_TYPE_F32 0
#define NC_TYPE_Q4_0 2
#define NC_TYPE_Q8_0 8
#define NC_TYPE_Q4_K 12
#define NC_TYPE_Q5_K 13
#define NC_TYPE_Q6_K 14

typedef struct nc_ctx nc_ctx;         /* device context: device id, default stream */
typedef struct nc_qmat nc_qmat;       /* device-resident repacked quantized matrix */
typedef struct nc_model nc_model;     /* device-resident Llama weights */
typedef struct nc_session nc_session; /* KV cache + workspaces + stream of one sequence */

/* Thread-local message for the last non-zero status returned on this thread. */
const char* nc_last_error(void);
/* Library version string. */
const char* nc_version(void);

/* ---------------------------------------------------------------- context */
/* Opens device `device` (HIP ordinal).  No reference counterpart: the reference
 * is CPU-only; this is the device handle the Rust `-sys` crate holds.  Also allocates the
 * operator entry points' scratch (block sums for up to 16 rows of 65536 columns, temperature
 * softmax partials for 16 rows): those calls allocate nothing at these sizes; a larger call
 * grows the scratch once. */
int nc_ctx_create(int device, nc_ctx** out);
void nc_ctx_free(nc_ctx* ctx);
/* Blocks until all work queued on the context's default stream finished. */
int nc_ctx_synchronize(nc_ctx* ctx);

/* Dot-product path of the quantized matmuls on 16-row tiles, for every call made through this
 * context and its models' sessions; the counterpart of the reference's Q8DotKernelSelector
 * (src/q8.rs:42-46), which picks scalar / NEON / SDOT block dots.  AUTO (the default) takes
 * v_dot4c, the faster path at every measured shape and width; MFMA computes the same int32
 * block dots with v_mfma_i32_16x16x32_i8 (bit-identical results).  Set it between calls, not
 * while work of the context is queued. */
#define NC_GEMM_KERNEL_AUTO 0
#define NC_GEMM_KERNEL_DOT4 1
#define NC_GEMM_KERNEL_MFMA 2
int nc_ctx_set_gemm_kernel(nc_ctx* ctx, int kernel);

/* Summation order of the attention in the verify and decode passes (nc_verify_greedy,
 * nc_forward1 and the decode loops) of this context's sessions; replaces the softmax and
 * weighted-V loops of the reference's attention (src/inference.rs:3522-3540, :3603-3623).
 * SEQUENTIAL (the default): the reference's left-to-right sums, bit-identical.  SPLIT: each
 * row's positions in 64-position chunks, per chunk a max, a sum of exp and an exp-weighted V
 * sum, the chunks combined in a fixed order.  Attention outputs equal the sequential ones up
 * to f32 rounding; the Q8_0 quantisation that follows can turn such a difference into one
 * quantisation step, so logits are not bit-identical to the reference's and a greedy stream
 * can leave the reference's where its top-2 margin is that small.  A row's result does not
 * depend on the batch it is in, so speculative and plain decoding emit one stream.  Keys and
 * values are read once per KV head and chunk for all heads and rows of a pass.  Prompt passes
 * (nc_prefill) keep the sequential order.  Set it between calls. */
#define NC_ATTN_SEQUENTIAL 0
#define NC_ATTN_SPLIT 1
int nc_ctx_set_attention(nc_ctx* ctx, int order);

/* How the sessions of this context launch a verify / decode pass (nc_verify_greedy,
 * nc_verify_stochastic, nc_forward1 and the decode loops; not prompt passes).  DIRECT (the
 * default): every kernel is launched one by one.  GRAPH: the pass's kernels after the one that
 * writes its positions and tokens are captured into a HIP graph on the first pass of each kind
 * (width, head or not, dot-product path, attention variant: the attention kernels change at a few
 * row lengths and, past 1536 positions, every 512 positions) and replayed after that, which takes
 * the host's per-kernel launch cost off the pass.  Both run the same kernels on the same data, so
 * results are bit-identical.  The passes of the benchmarked models are bound by the GPU, not by
 * the launches (the 8B verify step measured 2.52 ms direct and 2.54 ms replayed, captures
 * included), hence the default.  Passes with per-kernel or per-stage timing enabled, and models
 * whose q, k and v are separate matrices, always launch directly.  No counterpart in the
 * reference (its passes are CPU loops).  Set it between calls. */
#define NC_PASS_DIRECT 0
#define NC_PASS_GRAPH 1
int nc_ctx_set_pass_launch(nc_ctx* ctx, int mode);

/* ---------------------------------------------------------------- operator boundary */
/* Uploads a row-major GGUF quantized matrix (rows x cols, GGUF dims [cols, rows])
 * and repacks it into the device layout.  Replaces the load-time matrix
 * construction load_q4_0_matrix / decode_q4_k_blocks (src/model.rs:1369-1401,
 * src/model.rs:1270) that feeds QuantizedMatrix (src/model.rs:294-310).
 * type: NC_TYPE_Q4_0, NC_TYPE_Q4_K, NC_TYPE_Q5_K (matmul_q5_k_batch src/inference.rs:2513-2640),
 * NC_TYPE_Q8_0 (matmul_q8_0_batch src/inference.rs:1343-1383; both batches of 1..16 tokens, more
 * in 16-token slices) or NC_TYPE_Q6_K (the Q6_K output projection
 * of llama.cpp files, matmul_q6_k_batch src/inference.rs:1882-2000; batches of 1..16 tokens).
 * cols % 32 == 0 (Q4_K, Q5_K, Q6_K: % 256; Q6_K: cols <= 16384). */
int nc_qmat_upload(nc_ctx* ctx, int type, int64_t rows, int64_t cols, const void* gguf_blocks_host,
                   nc_qmat** out);
void nc_qmat_free(nc_qmat* w);
/* Bytes of the repacked device copy (algorithmic bytes of the weight stream). */
int64_t nc_qmat_device_bytes(const nc_qmat* w);

/* out[t][r] = sum_b ((w_scale[r][b] * x_scales[t][b]) * dot_i32(w[r][b], x[t][b])), the sum
 * taken in block order b = 0, 1, ... in f32 exactly as the reference's per-row loop.
 * Replaces matmul_quantized_batch (src/inference.rs:1246-1303) and, for batch_size 1,
 * matmul_quantized (src/inference.rs:1201-1244).  All pointers are device pointers:
 * x_i8 [batch][cols] int8, x_scales [batch][cols/32] f32, out [batch][rows] f32
 * (token-major, as write_batch_out src/inference.rs:1333-1341).  batch_size >= 1, no upper
 * limit (matmul_quantized_batch takes any batch): up to 16 tokens run on the verify kernels;
 * more run on the int8 MFMA prompt matmul (Q4_0; slices of up to 256 tokens through buffers
 * that nc_ctx_create allocates, 18 MiB) or as 16-token slices (Q4_K, Q6_K).  Calls that share
 * a context and overlap on different streams race on those buffers.
 * stream: a hipStream_t or NULL for the context's default stream. */
int nc_matmul_quantized_batch(nc_ctx* ctx, const nc_qmat* w, const int8_t* x_i8, const float* x_scales,
                              float* out, int batch_size, int64_t rows, int64_t cols, void* stream);
/* Allocation-free variant of nc_matmul_quantized_batch (no reference counterpart: it is for
 * callers that cannot allocate device memory, such as code under HIP graph capture or serving
 * loops that forbid hipMalloc).  Same arguments, semantics and results; its only scratch is a
 * static per-device array sized for batch_size * cols <= 16 * 65536 (larger: NC_ERANGE;
 * batch_size above 16: NC_EINVAL).  It
 * calls no hipMalloc/hipFree.  Calls that overlap on one device share that array and race. */
int nc_matmul_quantized_batch_noalloc(nc_ctx* ctx, const nc_qmat* w, const int8_t* x_i8, const float* x_scales,
                                      float* out, int batch_size, int64_t rows, int64_t cols, void* stream);
/* Debug/parity variant: writes the int32 per-block dot products (Q4_0:
 * sum (nib-8)*x per 32-block, q8.rs:2699; Q4_K: W_j = sum nib*x per 32-sub-block,
 * q8.rs:1339-1376) as dots[t][r][cols/32] (device pointer). */
int nc_matmul_blockdots(nc_ctx* ctx, const nc_qmat* w, const int8_t* x_i8, int32_t* dots, int batch_size,
                        int64_t rows, int64_t cols, void* stream);
/* Debug/parity hook: out[i] = the device's exp of the float with bits first_bits + i, for
 * 0 <= i < count (device pointer; count <= 2^32).  The device restates glibc's expf, which is
 * what the reference's f32::exp calls in softmax (src/inference.rs:3522-3540) and SiLU
 * (src/inference.rs:3367-3390); this entry point lets a test compare the two on every input. */
int nc_debug_expf(nc_ctx* ctx, uint32_t first_bits, int64_t count, float* out, void* stream);
/* Debug hook: after nc_temperature_probs_batch or nc_sample_logits_batch on this context (and on
 * this stream), fast[r] (host) = 1 if row r's exact left-to-right sum came from the evaluation
 * that runs the vocabulary's segments in parallel, 0 if from the segment-after-segment one (a
 * row whose checks failed, or a vocabulary above 262144).  Synchronises the stream. */
int nc_debug_temperature_paths(nc_ctx* ctx, int32_t rows, int32_t* fast, void* stream);
/* Debug hook: passes this session captured into HIP graphs and passes it replayed from them
 * (NC_PASS_GRAPH; both stay 0 under NC_PASS_DIRECT). */
int nc_debug_pass_graphs(nc_session* s, int64_t* captures, int64_t* replays);
/* Per-32-block Q8_0 activation quantiser: scale = amax/127 (f32), q = round-half-away
 * (x * (1/scale)) clamped to +-127.  Replaces quantize_f32_to_q8_0_batch
 * (src/inference.rs:967-989, scalar path :991-1029).  Device pointers. */
int nc_quantize_q8_0_batch(nc_ctx* ctx, const float* x, int8_t* x_i8, float* x_scales, int batch_size,
                           int64_t dim, void* stream);

/* RMSNorm then Q8_0 quantisation of each row: scale = 1/sqrt(sum/dim + eps) with the sum of
 * squares taken left to right in f32 (bit-identical), y = x*scale*w, then the per-32-block
 * quantiser above.  Replaces rms_norm_batch (src/inference.rs:949-967, row op :697-706)
 * followed by quantize_f32_to_q8_0_batch (:967-989), as run_layer_range_batch does at
 * :3802-3808.  Device pointers: x [batch][dim], w [dim], x_i8 [batch][dim],
 * x_scales [batch][dim/32].  dim one of 256, 512, 768, 1024, 1536, 2048, 3072, 4096, 5120, 6144,
 * 8192. */
int nc_rms_norm_q8_0_batch(nc_ctx* ctx, const float* x, const float* w, float eps, int8_t* x_i8, float* x_scales,
                           int batch_size, int64_t dim, void* stream);

/* ---------------------------------------------------------------- stochastic acceptance
 * No reference counterpart: the reference's temperature path matches sampled tokens
 * (src/speculative.rs:403) and samples with a global LCG (src/inference.rs:4834-4883).
 * This library's specification (restated by the CPU oracle, checked bit for bit):
 *   probs    p_j = e_j * (1/S), e_j = expf((l_j - max)/temp), S = sum e_j left to right in
 *            f32 (the reference's softmax formula, src/inference.rs:3522-3540, 4857-4862);
 *   uniform  u = (philox4x32_10(ctr = {pos, pos >> 32, purpose, 0}, key = seed).x >> 8) / 2^24,
 *            purposes: draft sample 1, accept 2, resample 3, bonus 7;
 *   accept   draft i (row at start_pos + i) iff u_accept * q_i(x) < p_i(x);
 *   sample   W_j = floor(w_j * 2^40), first j whose inclusive prefix of W exceeds
 *            floor(k24 * sum W / 2^24), k24 = u * 2^24.  At the first rejection the next
 *            token is drawn from w = max(0, p_i - q_i) (from p_i if that has no mass) with
 *            the resample uniform; after k acceptances from p_k with the bonus uniform. */
/* sample_logits (src/inference.rs:4834-4873) of rows 1..16 rows of logits (device, row stride
 * vocab): temp <= 0 the first maximum; temp > 0 e_j = expf((l_j - max)/temp), S = sum e_j left
 * to right, r = u * S with u = rand_simple() (one draw of *rng_state per row, in row order), then
 * r -= e_j until r <= 0 (the last id if never), every f32 operation as the reference's.  work:
 * rows x vocab device floats (temp > 0).  tokens: host ids[rows]. */
int nc_sample_logits_batch(nc_ctx* ctx, const float* logits, int32_t rows, int64_t vocab, float temp,
                           uint64_t* rng_state, float* work, uint32_t* tokens, void* stream);
/* probs[r][j] for rows x vocab (device pointers, row stride vocab); temp > 0. */
int nc_temperature_probs_batch(nc_ctx* ctx, const float* logits, float* probs, int32_t rows, int64_t vocab, float temp,
                               void* stream);
/* k+1 acceptance over device buffers: p_probs [k+1][vocab] target probabilities of the rows
 * at start_pos .. start_pos+k, q_probs [k][vocab] draft probabilities, drafts [k] ids.
 * result (device, 3 x int32) = {n_accepted, next_token, start_pos + n_accepted + 1}.
 * k 0..15; a draft id >= vocab counts as rejected.  nc_sample_logits_batch,
 * nc_temperature_probs_batch and nc_stochastic_accept use the context's device scratch: calls
 * on one context are ordered on their stream, and calls on different streams must not overlap. */
int nc_stochastic_accept(nc_ctx* ctx, const float* p_probs, const float* q_probs, const uint32_t* drafts, int32_t k,
                         int64_t vocab, uint64_t seed, int64_t start_pos, int32_t* result, void* stream);

/* ---------------------------------------------------------------- model */
typedef struct nc_model_config {
    int64_t context_length, embedding_length, block_count, feed_forward_length;
    int64_t head_count, head_count_kv, head_dim, rope_dimension_count, vocab_size;
    int64_t attention_output_width, kv_width;
    int32_t weight_type;  /* GGUF type of blk.0.attn_q.weight: NC_TYPE_Q4_0, NC_TYPE_Q4_K, NC_TYPE_Q5_K,
                             NC_TYPE_Q8_0 or NC_TYPE_Q6_K.
                           Files that mix types (llama.cpp Q4_K_M) keep each matrix's own type; this
                           field names the first layer's attention-query type only. */
    int32_t tied_head;    /* 1 when the head was requantised from token_embd */
    float rope_freq_base, rms_norm_epsilon;
    int64_t device_weight_bytes; /* repacked matrices incl. head */
    int64_t verify_weight_bytes; /* algorithmic weight bytes streamed by one verify pass */
    /* Llama-3 RoPE frequency scaling, llama.rope.scaling.{factor, original_context_length,
     * low_freq_factor, high_freq_factor} (rope_scaling_from_gguf src/main.rs:8522-8535).
     * rope_scaling = 1 when all four keys are present, as cached_rope_angles
     * (src/inference.rs:875-893) requires before it scales; the values are 0 otherwise. */
    int32_t rope_scaling;
    float rope_scaling_factor, rope_scaling_original_context_length;
    float rope_scaling_low_freq_factor, rope_scaling_high_freq_factor;
} nc_model_config;

typedef struct nc_load_opts {
    int32_t nthreads;     /* host threads for dequant/requant/repack (0 = all cores) */
    int32_t reserved[7];
} nc_load_opts;

/* Parses a GGUF file / in-memory image, builds LlamaModelConfig and uploads the
 * weights.  Replaces gguf::read_file (src/gguf.rs:454-551),
 * LlamaModelConfig::from_gguf (src/model.rs:48-186), validate_model_tensors
 * (src/model.rs:851-1036) and LlamaWeights::load (src/model.rs:461-545), including the
 * tied-head Q4_0 requantisation (src/q8.rs:2442-2488).  The file is memory-mapped, never
 * copied whole into host memory.  Token embeddings and norms may be F32, F16, BF16, Q8_0,
 * Q4_0, Q4_1, Q5_0, Q5_1, Q4_K, Q5_K or Q6_K (decoded as load_f32_or_f16,
 * src/model.rs:1081-1229); the layer matrices and an untied head must be Q4_0 or Q4_K.
 * Fused q|k|v or gate|up tensors, attention biases and mixture-of-experts layers, which the
 * reference also reads, are refused with NC_EFORMAT.  opts may be NULL. */
int nc_model_load_gguf(nc_ctx* ctx, const char* path, const nc_load_opts* opts, nc_model** out);
int nc_model_load_gguf_memory(nc_ctx* ctx, const void* data, size_t size, const nc_load_opts* opts,
                              nc_model** out);
int nc_model_get_config(const nc_model* m, nc_model_config* out);
/* Header-only checks of an in-memory GGUF image, no GPU: gguf::read_file (src/gguf.rs:454-551),
 * LlamaModelConfig::from_gguf (src/model.rs:48-186) and validate_model_tensors
 * (src/model.rs:851-1036), plus the shape limits of this build; fills *out on success.  The
 * same checks nc_model_load_gguf makes before reading any weight. */
int nc_gguf_read_config(const void* data, size_t size, nc_model_config* out);

/* The ids that end a turn for the file's tokenizer: is_generation_stop_token
 * (src/main.rs:8518-8520) is membership in SpecialTokens::eog, built by Tokenizer::from_gguf
 * (src/tokenizer.rs:287-323) from eos, eot, eom and Phi-3's "<|end|>": metadata
 * tokenizer.ggml.{eos,eot,eom}_token_id, else eos = 2 ("llama" SentencePiece vocabularies) or
 * the id of "<|end_of_text|>" ("gpt2" BPE), eot = the id of "<|eot_id|>".  Sorted, distinct,
 * written to out[0..*n) (these are the stop ids the decode loops take).  NC_EFORMAT when the
 * file has no usable tokenizer model or token list, or a special id (bos, eos, unk, eot, eom,
 * sep, pad, mask) lies outside the vocabulary, as the reference's tokenizer load refuses it;
 * NC_ERANGE (with *n set) when max is too small.  Host only; needs no device. */
int nc_gguf_stop_tokens(const void* data, size_t size, uint32_t* out, int32_t max, int32_t* n);
/* gguf::read_file's tensor descriptors (src/gguf.rs:498-550): the count (negative: error
 * code), and for tensor `index` its name, dimension count, dims (unused ones 1), GGML type id,
 * absolute data offset and byte size (tensor_nbytes, src/gguf.rs:737-763). */
int64_t nc_gguf_tensor_count(const void* data, size_t size);
int nc_gguf_tensor_info(const void* data, size_t size, int64_t index, char* name, int64_t name_cap, int32_t* n_dims,
                        uint64_t* dims, int32_t* type, uint64_t* offset, uint64_t* nbytes);
/* Host-side decode of n_values of one GGUF tensor's bytes to f32, exactly as the loader
 * decodes token embeddings and norms: load_f32_or_f16 (src/model.rs:1081-1229) for GGML
 * types 0 (F32), 1 (F16), 30 (BF16), 8 (Q8_0), 2 (Q4_0), 3 (Q4_1), 6 (Q5_0), 7 (Q5_1),
 * 12 (Q4_K), 13 (Q5_K), 14 (Q6_K).  Host pointers; needs no GPU. */
int nc_dequantize_f32(int32_t type, const void* blocks, int64_t n_values, float* out);
void nc_model_free(nc_model* m);

/* ---------------------------------------------------------------- session */
/* KV cache [layers][kv_heads][max_ctx][head_dim] f32 plus batch workspaces for up to
 * max_batch rows.  Replaces LlamaKvCache::new + LlamaWorkspace/LlamaBatchWorkspace
 * (src/inference.rs:505-695).  max_batch 1..16.  max_ctx 1..min(context_length,
 * NC_MAX_CONTEXT): the attention kernels take score rows of at most NC_MAX_CONTEXT positions,
 * so a longer session is refused here (NC_ERANGE) instead of failing inside a pass. */
#define NC_MAX_CONTEXT 16384
int nc_session_create(nc_model* m, int64_t max_ctx, int32_t max_batch, nc_session** out);
void nc_session_free(nc_session* s);

/* Batched forward of n tokens at positions start_pos.. (KV written for every row),
 * final hidden rows kept for nc_session_hidden.  Replaces prefill_pass_batch
 * (src/inference.rs:3695-3744); n > max_batch is processed in max_batch chunks as
 * prefill_tokens does (src/main.rs:9415-9485).  want_logits != 0: the head runs on the
 * last chunk's rows (their logits are then readable with nc_session_logits, rows
 * 0 .. min(n, max_batch)-1 of that chunk); want_logits == 0: no head pass at all, as
 * prefill_pass_batch computes no logits.  Token ids >= vocab_size: NC_ERANGE before any
 * launch (the reference panics on the embedding index, src/inference.rs:3728-3733). */
int nc_prefill(nc_session* s, const uint32_t* toks, int32_t n, int64_t start_pos, int32_t want_logits);
/* Single-token forward (src/inference.rs:3649-3670 forward_pass).  logits_host may be
 * NULL; *pred_out (nullable) receives argmax (first max wins, inference.rs:4836-4846). */
int nc_forward1(nc_session* s, uint32_t tok, int64_t pos, float* logits_host, uint32_t* pred_out);

typedef struct nc_verify_result {
    int32_t n_accepted; /* drafts accepted (longest matching prefix) */
    uint32_t next_token; /* the target's token after the accepted prefix */
    int64_t new_pos;     /* start_pos + n_accepted + 1 */
} nc_verify_result;

/* k+1 greedy verify: toks[0] = the pending token at start_pos, toks[1..n) = drafts.
 * One batched forward, per-row head + argmax, and acceptance, all on the device; only
 * the result struct returns to the host.  KV rows past new_pos are dead (implicit
 * rollback, src/speculative.rs:184-187).  Semantics of cluster_tcp_smoke.rs:905-979 /
 * ngram_speculative_step (src/speculative.rs:122-286).  preds_host (nullable) receives
 * the n per-row predictions. */
int nc_verify_greedy(nc_session* s, const uint32_t* toks, int32_t n, int64_t start_pos,
                     nc_verify_result* result, uint32_t* preds_host);
/* k+1 stochastic verify: toks[0] = the pending token at start_pos, toks[1..n) = drafts
 * sampled from q_probs (device, [n-1][vocab] draft probabilities at temperature temp).  One
 * batched forward, then temperature probabilities and the acceptance above on the device;
 * only the result struct returns.  The stochastic counterpart of nc_verify_greedy. */
int nc_verify_stochastic(nc_session* s, const uint32_t* toks, int32_t n, int64_t start_pos, const float* q_probs,
                         float temp, uint64_t seed, nc_verify_result* result);
/* Copies row `row` of the last pass's logits ([vocab] f32) to host
 * (compute_logits_from_hidden, src/inference.rs:4783-4832). */
int nc_session_logits(nc_session* s, int32_t row, float* logits_host);
/* Copies the last pass's final hidden rows ([n][d] f32, before the output norm). */
int nc_session_hidden(nc_session* s, int32_t n, float* hidden_host);

/* ---------------------------------------------------------------- decode loops */
typedef struct nc_decode_stats {
    int64_t steps, drafted, accepted, emitted;
    double decode_seconds; /* wall time of the decode loop (prefill excluded) */
    double prefill_seconds;
} nc_decode_stats;

/* Plain greedy decode: prompt prefill (prefix in max_batch chunks, last token single)
 * then n_new greedy tokens.  Mirrors the plain loop of src/main.rs:9676-9706. */
int nc_generate_greedy(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new,
                       uint32_t* out, nc_decode_stats* stats);

/* The plain decode loop with sampling and stop tokens (src/main.rs:9894-9928): each token is
 * drawn with sample_logits (src/inference.rs:4834-4873) from the live logits, one
 * rand_simple draw (*rng_state) per token at temp > 0; decoding ends before a stop token
 * (stop[n_stop]; n_stop = 0: none, and the ids are not emitted), at the session context or
 * after n_new tokens.  stats->emitted is the number of tokens written to out.  temp <= 0
 * with no stop tokens is nc_generate_greedy (rng_state may then be NULL). */
int nc_generate_plain(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new, float temp,
                      uint64_t* rng_state, const uint32_t* stop, int32_t n_stop, uint32_t* out,
                      nc_decode_stats* stats);

/* k+1 speculative decode with the seeded oracle drafter (no reference counterpart;
 * the drafter exists only for the benchmark configs): the draft for absolute
 * position p copies greedy[p - n_prompt] (greedy = the target's recorded greedy
 * continuation, n_greedy tokens) when philox_u(seed, p) < alpha, else a philox
 * uniform id.  Emits the target's greedy stream.  Stops after n_new tokens or
 * max_steps verify steps (max_steps <= 0: no step bound). */
int nc_generate_speculative_oracle(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new,
                                   int32_t max_steps, int32_t k, float alpha, uint64_t seed,
                                   const uint32_t* greedy, int32_t n_greedy, uint32_t* out,
                                   nc_decode_stats* stats);

/* Prompt-lookup drafting, NGramDrafter::draft (src/speculative.rs:81-103): the longest
 * suffix n-gram of history (max_ngram down to min_ngram; the reference defaults are 4 and 3)
 * with an earlier occurrence, most recent occurrence first, proposes the tokens that followed
 * it: at most max_tokens, never past the end of the history.  Writes them to out and returns
 * how many (0: no proposal).  Host only; needs no device. */
int32_t nc_ngram_draft(const uint32_t* history, int64_t len, int32_t min_ngram, int32_t max_ngram, int32_t max_tokens,
                       uint32_t* out);

/* n-gram speculative decode, greedy: ngram_speculative_step (src/speculative.rs:122-286)
 * driven by the generate loop (src/main.rs:9729-9776: k clamped to the token budget minus
 * one), in the k+1 verify form (src/bin/cluster_tcp_smoke.rs:905-979).  Each step verifies
 * the pending token plus up to k drafts that nc_ngram_draft proposes from prompt + emitted
 * tokens; no proposal means a one-row pass.  The emitted stream is the target's greedy
 * stream, cut before the first of the n_stop stop tokens (a stop token is neither emitted
 * nor consumed).  stats->emitted (<= n_new) is the number of tokens written to out. */
int nc_generate_speculative_ngram(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new, int32_t k,
                                  int32_t min_ngram, int32_t max_ngram, const uint32_t* stop, int32_t n_stop,
                                  uint32_t* out, nc_decode_stats* stats);

/* The same at temperature temp > 0 (temp <= 0: the greedy loop above): each step draws t0
 * from the live logits with sample_logits (src/inference.rs:4834-4873), verifies t0 plus the
 * drafts in one pass, draws one token per verified row in order (a matching draw accepts the
 * draft, a different one is emitted and run as a corrective forward, a stop token ends the
 * turn), and when every draft matches the last row's logits predict the next step's t0.
 * *rng_state is the reference's LCG state (rand_simple), one draw per sample in the step's
 * order. */
int nc_generate_speculative_ngram_temp(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new,
                                       int32_t k, int32_t min_ngram, int32_t max_ngram, float temp,
                                       uint64_t* rng_state, const uint32_t* stop, int32_t n_stop, uint32_t* out,
                                       nc_decode_stats* stats);

/* Draft-model speculative decode, greedy, as speculative_decoding_step
 * (src/speculative.rs:299-494) driven by the generate loop (src/main.rs:9799-9870):
 * k draft forwards, one k-row target verify, acceptance against the live target
 * prediction, then a corrective/bonus single-token forward on both models. */
int nc_generate_speculative_draft(nc_session* target, nc_session* draft, const uint32_t* prompt,
                                  int32_t n_prompt, int32_t n_new, int32_t draft_k, uint32_t* out,
                                  nc_decode_stats* stats);

/* The same step at temperature temp (src/speculative.rs:299-494 with temp > 0): drafts are
 * drawn with sample_logits (src/inference.rs:4834-4873) from the draft's logits, the target
 * draws its own token at each verified position with sample_logits, a draft is accepted iff
 * the two ids match, and the first mismatch (or, after k matches, the trailing draw) is
 * emitted and run on both models.  *rng_state is the reference's LCG state (rand_simple,
 * src/inference.rs:4876-4883; the reference starts it at 0x123456789abcdef0), advanced by one
 * draw per sample the reference makes, in its order.  temp <= 0: the greedy loop above.
 * stop[n_stop] (n_stop = 0: none) are the step's is_stop_token ids (speculative.rs:305-447):
 * a drafted stop token ends drafting without a draft forward, an accepted one ends the
 * verification with no trailing draw; as the generate loop (src/main.rs:9852-9866), the
 * first stop token among a step's tokens ends decoding and is not written to out. */
int nc_generate_speculative_draft_temp(nc_session* target, nc_session* draft, const uint32_t* prompt,
                                       int32_t n_prompt, int32_t n_new, int32_t draft_k, float temp,
                                       uint64_t* rng_state, const uint32_t* stop, int32_t n_stop, uint32_t* out,
                                       nc_decode_stats* stats);

/* Draft-model speculative sampling at temperature temp > 0, k+1 form (no reference
 * counterpart; the draft-model loop shape follows src/speculative.rs:299-494).  Both models
 * prefill the prompt; the first token is drawn from the target's last prompt row with the
 * bonus uniform at position n_prompt-1.  Per step at position pos with pending token t0:
 * the draft runs t0, d_0 .. d_{k-2} at pos .. pos+k-1 and samples d_i from its temperature
 * probabilities with u(seed, pos+i, draft); the target verifies [t0, d_0 .. d_{k-1}]; the
 * acceptance above emits d_0 .. d_{a-1} and the next token.  After a full acceptance the
 * draft first runs d_{k-1}.  k is clamped to max_batch-1 and the context of both sessions.
 * Drafts stay on the device; one 16-byte result and the step's ids return per step. */
int nc_generate_speculative_stochastic(nc_session* target, nc_session* draft, const uint32_t* prompt,
                                       int32_t n_prompt, int32_t n_new, int32_t k, float temp, uint64_t seed,
                                       uint32_t* out, nc_decode_stats* stats);

/* ---------------------------------------------------------------- synthetic models */
typedef struct nc_synth_spec {
    int32_t layers, embedding_length, head_count, head_count_kv, feed_forward_length, vocab_size;
    int32_t context_length;
    int32_t weight_type; /* NC_TYPE_Q4_0, NC_TYPE_Q4_K, NC_TYPE_Q5_K or NC_TYPE_Q8_0 for layer matrices and
                            token_embd */
    int32_t tied;        /* 1: no output.weight (head requantised at load) */
    int32_t norm_mode;   /* 0: norm weights 1.0; 1: N(1, 0.1) */
    float rope_freq_base, rms_norm_epsilon, weight_std;
    uint64_t seed;
    /* rope_scaling_factor > 0: also write llama.rope.scaling.factor (f32),
     * .original_context_length (u32), .low_freq_factor and .high_freq_factor (f32). */
    float rope_scaling_factor, rope_scaling_low_freq_factor, rope_scaling_high_freq_factor;
    uint32_t rope_scaling_original_context_length;
} nc_synth_spec;

/* Size in bytes of the GGUF v3 image nc_synth_write would produce. */
int nc_synth_size(const nc_synth_spec* spec, uint64_t* size_out);
/* Writes a seeded random-init Llama GGUF v3 image (alignment 32): weights drawn from
 * N(0, weight_std) with a Philox4x32-10 counter stream and Box-Muller, quantised to
 * Q4_0 (llama.cpp rule: d = max/-8, round-to-nearest-even f16 scale) or Q4_K.
 * Deterministic for a given spec regardless of nthreads. */
int nc_synth_write(const nc_synth_spec* spec, void* dst, uint64_t size, int32_t nthreads);

/* Benchmark helper (config 1; no reference counterpart): launches the quantized matmul
 * `iters` times back to back on the context stream, round robin over `ncopies` weight copies
 * of one shape (so the weights stream from HBM, not the 256 MB last-level cache), each launch
 * bracketed by events stamped by its own dispatch; us_out[iters] receives every launch's kernel
 * duration in microseconds.  Device pointers as nc_matmul_quantized_batch. */
int nc_bench_matmul(nc_ctx* ctx, const nc_qmat* const* w, int32_t ncopies, const int8_t* x_i8, const float* x_scales,
                    float* out, int32_t batch_size, int32_t iters, float* us_out);

/* Philox4x32-10 helpers shared by the drafter and the synthetic prompt.
 * ids[i] = philox(seed, i, purpose 4).x mod vocab. */
int nc_uniform_prompt(uint64_t seed, int64_t n, uint32_t vocab, uint32_t* ids);
uint32_t nc_oracle_draft(uint64_t seed, int64_t p, float alpha, const uint32_t* greedy, int64_t n_prompt,
                         int64_t n_greedy, uint32_t vocab);

/* Benchmark and test helpers for BASELINE config 4's "KV cache filled with N(0, 1) keys and
 * values" (no reference counterpart).  nc_synth_kv_values (host only): N(0, 1) values, Philox4x32-10
 * with counter (pair index, stream 2 * layer + kind, purpose 10) and key seed, Box-Muller in
 * double, rounded to f32; elements [start, start + count) of the stream (start, count even) into
 * out.  kind 0 = keys, 1 = values.  nc_session_fill_kv: rows [0, n) of every layer's key and
 * value cache from those streams, element i of row p being element p * kv_width + i; a pass at
 * start_pos = n then attends over n positions of N(0, 1) keys and values.  Synchronous. */
int nc_synth_kv_values(uint64_t seed, int32_t layer, int32_t kind, int64_t start, int64_t count, float* out);
int nc_session_fill_kv(nc_session* s, int64_t n, uint64_t seed);

/* ---------------------------------------------------------------- timing hooks */
/* Average device time (ms) per launch of the named kernel family recorded with HIP
 * events on the session stream since the last reset; used by the benchmark's
 * roofline.  family: "gemm_q4_0" (all verify matmuls).  Prompt prefill passes are
 * never timed: only decode and verify passes count.  Returns launches counted. */
int64_t nc_session_kernel_timing(nc_session* s, const char* family, double* total_ms, int64_t* bytes);
/* enable: bit 0 = the matmul timing above; bit 1 = per-stage timing (HIP events between the
 * stages of every verify and decode pass, the reference's NANOCAMELID_TRACE stage breakdown,
 * inference.rs:179-229).  Either resets its totals. */
int nc_session_timing_enable(nc_session* s, int32_t enable);
/* Per-stage totals since the last enable: returns the number of stages; for 0 <= index < that
 * number writes the stage's name (the reference's trace stage names, joined with '+' where the
 * device runs them as one kernel), its total ms and the number of times it ran. */
int32_t nc_session_stage_timing(nc_session* s, int32_t index, char* name, int32_t name_cap, double* total_ms,
                                int64_t* calls);

#ifdef __cplusplus
}
#endif
#endif
