// Host-side internals of libnanocamelid_hip (not part of the C ABI).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

#include "../../include/nanocamelid_gpu.h"

namespace nc {

// ---------------------------------------------------------------- errors
void set_error(const std::string& msg);
int fail(int code, const std::string& msg);

#define NC_HIP(call)                                                                   \
    do {                                                                               \
        hipError_t _e = (call);                                                        \
        if (_e != hipSuccess)                                                          \
            return ::nc::fail(NC_EHIP, std::string(#call) + ": " + hipGetErrorString(_e)); \
    } while (0)

// ---------------------------------------------------------------- stage timing
// While t_stage_ev1 is set (a session's stage timing), kernels launched through NC_LAUNCH are
// dispatched with events stamped by the dispatch itself: t_stage_ev0 records the first such
// kernel's start (and is then cleared), t_stage_ev1 every kernel's end, so the pair spans the
// kernels of one stage and nothing between launches.
extern thread_local hipEvent_t t_stage_ev0, t_stage_ev1;
#define NC_LAUNCH(K, G, B, L, S, ...)                                                          \
    do {                                                                                       \
        if (::nc::t_stage_ev1) {                                                               \
            hipExtLaunchKernelGGL(K, G, B, L, S, ::nc::t_stage_ev0, ::nc::t_stage_ev1, 0, __VA_ARGS__); \
            ::nc::t_stage_ev0 = nullptr;                                                       \
        } else {                                                                               \
            hipLaunchKernelGGL(K, G, B, L, S, __VA_ARGS__);                                    \
        }                                                                                      \
    } while (0)

// ---------------------------------------------------------------- weight layouts
// Q4_0 device layout ("tile-group"): rows padded to 64-row tiles; per (tile, group of 8
// blocks) a 9216-byte chunk = 8 x [64 lanes x 16 B nibbles] followed by the f16 scales as
// 2 x [64 lanes x 4 scales] (blocks 0-3, then 4-7).  Lane l of a wave loads row 64*tile + l;
// a round of 4 blocks reads 4 KB of nibbles and 512 contiguous bytes of scales.
constexpr int kTileRows = 64;
constexpr int kQ40GroupBlocks = 8;
constexpr int kQ40ChunkBytes = kQ40GroupBlocks * 1024 + 1024;  // 9216
// Q4_K device layout: per (tile, super-block) 9 x [64 lanes x 16 B]: slot 0 = d, dmin and
// the 12 packed scale bytes, slots 1..8 = the 128 nibble bytes.
constexpr int kQ4KChunkBytes = 9 * 1024;

// Q4_0 "R16" layout (matrices with fewer than 512 64-row tiles, so that a launch still
// spans every CU): rows padded to 16-row tiles; blocks taken in quads (block b = 4*qd + j)
// and groups of 8 quads.  Per (tile16, group) a 9216-byte chunk of 8 quads, each 1152 bytes:
// [64 lanes x 16 B nibbles] with lane = 16*j + r holding block 4*qd + j of row 16*tile + r,
// then the 64 f16 scales of the same blocks in [r / 4][j][r % 4] order.  One wave load covers
// 4 blocks x 16 rows and its scales are one contiguous 128-byte line.
constexpr int kTileRowsR16 = 16;
constexpr int kQ40R16QuadBytes = 1024 + 128;  // 1152; 8 per chunk = kQ40ChunkBytes
// Q8_0 layout: rows padded to 64-row tiles; per (tile, group of 4 blocks) an 8704-byte chunk =
// [4 blocks][2 halves][64 lanes x 16 B] of int8 weights (lane l = row 64*tile + l), then the
// f16 scales as [4 blocks][64 lanes].  Every load of a wave is 1 KB (or 128 B) contiguous.
constexpr int kQ80GroupBlocks = 4;
constexpr int kQ80ChunkBytes = kQ80GroupBlocks * 2048 + kQ80GroupBlocks * 128;  // 8704
enum Layout : int { LAYOUT_R64 = 0, LAYOUT_R16 = 1, LAYOUT_R16K = 2, LAYOUT_Q6K = 3, LAYOUT_Q80 = 4 };  // R16K: Q4_K on 16-row tiles

struct QMatDev {
    int type = NC_TYPE_Q4_0;
    int layout = LAYOUT_R64;
    int64_t rows = 0, cols = 0;
    int64_t tiles = 0;       // padded rows / 64 (R16: / 16)
    int64_t units = 0;       // Q4_0, Q8_0: blocks per row; Q4_K: super-blocks per row
    int64_t groups = 0;      // Q4_0: ceil(blocks / 8) (R16: ceil(blocks / 32)); Q8_0: ceil(blocks / 4)
    uint8_t* dev = nullptr;  // repacked bytes
    int64_t dev_bytes = 0;
    int64_t algo_bytes = 0;  // rows * cols * 18/32 (Q4_0) or 144/256 (Q4_K)
};

// Repacks row-major GGUF blocks of `rows_src` rows into the device layout, writing tile
// rows [row_off, row_off + rows_src) of `dst` (host staging buffer of the whole matrix).
// interleave_pairs: rows_src rows are the gate half (tile lanes 0..31) or up half
// (lanes 32..63) of an interleaved SwiGLU matrix (half = 0 or 1), else -1.
void repack_q4_0(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups,
                 int64_t row_off, int half);
void repack_q4_k(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t row_off, int half,
                 int nslot = 9);
void repack_q4_0_r16(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups, int64_t row_off,
                     int half);
int64_t q40_r16_layout_bytes(int64_t rows, int64_t cols);
int64_t q40_layout_bytes(int64_t rows, int64_t cols);
int64_t q4k_layout_bytes(int64_t rows, int64_t cols);
int64_t q4k_r16_layout_bytes(int64_t rows, int64_t cols);
// Q4_K on 16-row tiles: per (tile, quad of 4 super-blocks) 9 x [64 lanes x 16 B], lane
// 16*q + r = super-block 4*quad + q of row r.  half >= 0: rows of an interleaved gate (0) or up
// (1) matrix, placed in 64-row groups as the Q4_0 repacks do.
int64_t q80_layout_bytes(int64_t rows, int64_t cols);
void repack_q8_0(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups, int64_t row_off,
                 int half);
void repack_q4_k_r16(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups,
                     int64_t row_off, int half = -1);

// ---------------------------------------------------------------- GEMM launch
enum Epi : int {
    EPI_STORE = 0,      // out[n*ld + row] = acc
    EPI_RESIDUAL = 1,   // out[n*ld + row] = acc + out[n*ld + row]
    EPI_QKV_ROPE = 2,   // RoPE on q/k rows, q -> q_out, k/v -> KV cache
    EPI_SWIGLU_Q8 = 3,  // silu(gate)*up then Q8_0 quantisation -> activations
    EPI_HEAD = 4,       // logits + per-tile argmax partials
};

struct GemmParams {
    const uint8_t* w = nullptr;
    int ntiles = 0, units = 0, groups = 0, M = 0, K = 0, N = 0;
    const int8_t* x = nullptr;     // [N][K]
    const float* xs = nullptr;     // [N][K/32]
    const int32_t* xs8 = nullptr;  // [N][K/32] -8 * (sum of the 32 int8 values of each block)
    int epi = EPI_STORE;
    float* out = nullptr;
    int ld_out = 0;
    // EPI_QKV_ROPE
    float* q_out = nullptr;
    int aw = 0, kw = 0, hd = 0, rope_half = 0, max_ctx = 0, kv_heads = 0;
    const float* rope_tab = nullptr;  // [max_ctx][rope_half][2] = (sin, cos)
    float* kcache = nullptr;          // layer base of [kv_heads][hd/4][max_ctx][4] (dim quads)
    float* vcache = nullptr;          // layer base of [kv_heads][max_ctx/4][hd][4] (position quads)
    const int32_t* d_pos = nullptr;   // start position of row 0
    // EPI_SWIGLU_Q8
    int8_t* xq_out = nullptr;
    float* xs_out = nullptr;
    int32_t* xs8_out = nullptr;
    int F = 0;
    // EPI_HEAD
    float* part_val = nullptr;  // [N][ntiles]
    int32_t* part_idx = nullptr;
    int kernel = NC_GEMM_KERNEL_AUTO;  // dot-product path for 16-row tiles (nc_ctx_set_gemm_kernel)
};

// ev0/ev1: optional events stamped at the kernel's own start and end (timing).
int launch_gemm(const QMatDev& w, const GemmParams& p, hipStream_t stream, hipEvent_t ev0 = nullptr,
                hipEvent_t ev1 = nullptr);
int launch_blockdots(const QMatDev& w, const int8_t* x, int32_t* dots, int N, hipStream_t stream);
// Q6_K matmul (plain outputs or the head's logits + argmax partials); rows per head tile
int launch_gemm_q6k(const QMatDev& w, const GemmParams& p, hipStream_t stream);
int q6k_rows_per_tile(int64_t cols);

// ---------------------------------------------------------------- layer kernels
int launch_rmsnorm_q8(const float* hidden, const float* weight, int N, int d, float eps, int8_t* xq, float* xs,
                      int32_t* xs8, hipStream_t stream);
// Activation side buffers: xs = per-block f32 scale, xs8 = -8 * per-block int8 sum.
int launch_quantize_q8(const float* x, int N, int dim, int8_t* xq, float* xs, int32_t* xs8, hipStream_t stream);
int launch_expf_range(uint32_t first, int64_t count, float* out, hipStream_t stream);
int launch_block_sums(const int8_t* x, int N, int dim, int32_t* xs8, hipStream_t stream);
struct TokenArgs {
    uint32_t t[16];
};
// Writes d_pos[0] = pos and, when toks != NULL, d_toks[0..n) = toks (n <= 16).
int launch_set_pass_state(int32_t* d_pos, int32_t pos, uint32_t* d_toks, const uint32_t* toks, int n, hipStream_t st);
int launch_embed(const float* table, const uint32_t* toks, int N, int d, float* hidden, hipStream_t stream);
struct AttnParams {
    const float* q = nullptr;  // [N][H*hd]
    const float* kcache = nullptr;  // layer base [Hkv][hd/4][max_ctx][4]: 4 dims of a position per 16 B
    const float* vcache = nullptr;  // layer base [Hkv][max_ctx/4][hd][4]: 4 positions of a dim per 16 B
    float* scores = nullptr;  // [N][H][max_ctx]
    int8_t* xq = nullptr;     // [N][H*hd] quantised attention output
    float* xs = nullptr;
    int32_t* xs8 = nullptr;
    const int32_t* d_pos = nullptr;
    int N = 0, H = 0, Hkv = 0, hd = 0, max_ctx = 0, max_pos = 0;
    float scale = 0.f;
    // split-position order (NC_ATTN_SPLIT): per (row, head, 64-position chunk) partials
    bool split = false;
    float* part_o = nullptr;   // [N][H][nchunks][hd]
    float* part_ml = nullptr;  // [N][H][nchunks][2] chunk max, chunk sum of exp
    int nchunks = 0;
};
int launch_attention(const AttnParams& a, hipStream_t stream);
// Launch variant of launch_attention: passes with equal values launch the same kernels with the
// same grids and blocks (the kernels read the rows' positions from d_pos, not from max_pos), so
// a captured pass replays correctly at every start position of its variant.
int64_t attention_variant(const AttnParams& a);

// ---------------------------------------------------------------- prompt (prefill) path
// Q4_0 batch matmul for any number of tokens on int8 MFMA: out[n * ld_out + row] (R16 and R64
// layouts) over xm / xsm, the activations x / xs repacked by launch_prompt_repack (xm:
// 16 * ceil(N/16) * K bytes, xsm: 16 * ceil(N/16) * ceil(K/128) * 4 floats).
int launch_gemm_prompt(const QMatDev& w, const int8_t* x, const float* xs, float* out, int ld_out, int N,
                       hipStream_t stream, const void* xm, const float* xsm);
// xam (optional, as xsm): the float sums of each 32-value block's int8 values (Q4_K's A_j)
int launch_prompt_repack(const int8_t* x, const float* xs, int N, int K, void* xm, float* xsm, hipStream_t stream,
                         float* xam = nullptr);
// Q4_K batch matmul for any number of tokens on int8 MFMA (R16K and R64 layouts) over
// activations repacked with their block sums
int launch_gemm_prompt_q4k(const QMatDev& w, float* out, int ld_out, int N, hipStream_t stream, const void* xm,
                           const float* xsm, const float* xam);
// The verify GEMMs' epilogues as separate kernels over a prompt matmul's f32 output y.
int launch_prompt_qkv_rope(const float* y, int N, int start, int aw, int kw, int hd, int rope_half,
                           const float* rope_tab, float* q_out, float* kcache, float* vcache, int max_ctx,
                           hipStream_t stream);
int launch_prompt_residual(const float* y, float* hidden, int N, int d, hipStream_t stream);
int launch_prompt_swiglu_q8(const float* y, int N, int F, int8_t* xq, float* xs, int32_t* xs8, hipStream_t stream,
                            bool split = false);
int launch_prompt_positions(int32_t* d, int start, int stride, int count, hipStream_t stream);
constexpr int kPromptRows = 256;   // tokens per prompt pass
constexpr int kPromptGroup = 64;   // rows per attention launch inside a prompt pass (score buffer rows)
constexpr int kPromptMin = 32;     // shorter prompts run as verify-sized passes
int launch_argmax_final(const float* part_val, const int32_t* part_idx, int N, int ntiles, uint32_t* preds,
                        hipStream_t stream);
int launch_accept_greedy(const uint32_t* toks, const uint32_t* preds, int n, int32_t* d_pos, int32_t* result,
                         uint32_t* next_tok_slot, hipStream_t stream);

// ---------------------------------------------------------------- stochastic acceptance
// probs[r][j] = expf((l_j - max)/temp) * (1 / sum), the sum exact left to right (rows x V).
// Temperature probabilities of `rows` rows; scratch: temperature_scratch_floats(rows) floats of
// device memory owned by the caller (stream-ordered reuse), 256-byte aligned; the samplers below
// use its first part, so a sample may follow the probabilities it reads on the same stream.
size_t temperature_scratch_floats(int rows);
// sample_logits (inference.rs:4834-4873) of `rows` rows (<= kSampleMaxRows): temp > 0 draws row r
// with the uniform u[r] (the reference's inverse-CDF walk, bit-exact); temp <= 0 takes the first
// maximum.  probs: rows x ld_p floats of work (the rows' e_j), scratch as above; out: device ids.
constexpr int kSampleMaxRows = 17;
struct SampleUniforms {
    float u[kSampleMaxRows];
};
int launch_sample_logits(const float* logits, int64_t ld_in, int rows, int V, float temp, const float* u, float* probs,
                         int64_t ld_p, float* scratch, uint32_t* out, hipStream_t stream);
int launch_temperature_probs(const float* logits, int64_t ld_in, float* probs, int64_t ld_out, int rows, int V,
                             float temp, float* scratch, hipStream_t st);
// fast[r] (host) = which evaluation gave row r's sum in the last temperature pass on scratch.
int temperature_row_paths(const float* scratch, int rows, int32_t* fast, hipStream_t st);
// p [k+1][ld] target probs, q [k][ld] draft probs, drafts[k] (device); result = {n_accepted,
// next_token, start_pos + n_accepted + 1}; d_pos (nullable) receives the new position.
int launch_accept_stochastic(const float* p, const float* q, int64_t ld, const uint32_t* drafts, int k, int V,
                             uint64_t seed, int64_t start_pos, int32_t* result, int32_t* d_pos, float* scratch,
                             hipStream_t st);
// One fixed-point inverse-CDF sample of probs[V] with the Philox uniform (seed, pos, purpose).
int launch_sample_probs(const float* probs, int V, uint64_t seed, int64_t pos, uint32_t purpose, uint32_t* out0,
                        uint32_t* out1, float* scratch, hipStream_t st);

// Address of the allocation-free entry point's scratch array on the current device
// (hipGetSymbolAddress of a file-scope __device__ array; each device has its own copy).
int static_scratch_address(int32_t** out);
// Capacity of that array in int32 entries: per-block sums of up to 16 rows x 65536 columns.
constexpr size_t kStaticScratchInts = 16 * 65536 / 32;

}  // namespace nc

// ---------------------------------------------------------------- C ABI handles (opaque in the header)
struct nc_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    // Scratch of the operator-level entry points, allocated by nc_ctx_create for up to 16
    // rows of 65536 columns (every Llama projection); a larger call grows it once.
    int32_t* xsum = nullptr;  // -8 * per-block int8 sums of the activations
    size_t xsum_cap = 0;
    float* tp_scratch = nullptr;  // temperature softmax partials
    size_t tp_cap = 0;
    // activations of the prompt matmul (more than 16 tokens) repacked in MFMA operand order
    // with their scales and block sums, for kPromptRows tokens of 65536 columns per slice;
    // allocated by nc_ctx_create
    int8_t* pxm = nullptr;
    float* pxsm = nullptr;
    float* pxam = nullptr;
    // device address of the static scratch array on this context's device (never freed)
    int32_t* static_scratch = nullptr;
    int gemm_kernel = NC_GEMM_KERNEL_AUTO;  // dot-product path of the quantized matmuls
    int attn_order = NC_ATTN_SEQUENTIAL;     // summation order of the verify passes' attention
    int pass_launch = NC_PASS_DIRECT;         // NC_PASS_GRAPH: session passes replayed from HIP graphs
};

struct nc_qmat {
    nc_ctx* ctx = nullptr;
    nc::QMatDev m;
};
