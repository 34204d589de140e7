// Host runtime of libnanocamelid_hip: device context, weight repacking and upload,
// the Llama model loader, sessions (KV cache + workspaces + stream), the verify pass,
// the decode loops and the C ABI declared in include/nanocamelid_gpu.h.
#include <algorithm>
#include <array>
#include <chrono>
#include <cmath>
#include <cstring>
#include <memory>
#include <thread>
#include <unordered_map>

#include "gguf.h"
#include "nc_internal.h"

#include <cerrno>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

// ---------------------------------------------------------------- handles
// nc_ctx and nc_qmat are defined in nc_internal.h (shared with noalloc.hip).
namespace {
constexpr size_t kCtxScratchCols = 65536;
}

namespace {

struct LayerDev {
    float* attn_norm = nullptr;
    float* ffn_norm = nullptr;
    nc::QMatDev qkv, wo, gateup, down;
    // q, k, v (gate, up) as separate matrices when their types differ or are not Q4_0 / Q4_K
    // (llama.cpp's Q4_K_M files keep attn_v and ffn_down in Q6_K on some layers): each matmul
    // then stores plain rows and the epilogue runs as its own kernel
    bool split_qkv = false, split_gateup = false;
    nc::QMatDev q, k, v, gate, up;
    // every matrix of the layer, for loops over them (unused ones have dev == nullptr)
    std::array<nc::QMatDev*, 9> all() { return {&qkv, &wo, &gateup, &down, &q, &k, &v, &gate, &up}; }
    std::array<const nc::QMatDev*, 9> all() const { return {&qkv, &wo, &gateup, &down, &q, &k, &v, &gate, &up}; }
};

}  // namespace

struct nc_model {
    nc_ctx* ctx = nullptr;
    nc_model_config cfg{};
    float* tok_emb = nullptr;  // [V][d] f32 (model.rs:467 token_embeddings)
    float* out_norm = nullptr;
    nc::QMatDev head;
    std::vector<LayerDev> layers;
    std::vector<void*> allocs;
};

struct nc_session {
    nc_model* m = nullptr;
    nc_ctx* ctx = nullptr;
    hipStream_t stream = nullptr;
    int64_t max_ctx = 0;
    int64_t ctx_stride = 0;  // max_ctx rounded up to 4: KV rows, V position quads, score rows
    int max_batch = 0;
    int64_t maxw = 0;
    float *kcache = nullptr, *vcache = nullptr;  // K [L][Hkv][hd/4][ctx_stride][4], V [L][Hkv][ctx_stride/4][hd][4]
    float* hidden = nullptr;                     // [B][d]
    int8_t* xq = nullptr;                        // [B][maxw]
    float* xs = nullptr;                         // [B][maxw/32]
    int32_t* xs8 = nullptr;  // -8 * per-block int8 sums
    float* q = nullptr;       // [B][aw]
    float* scores = nullptr;  // [B][H][ctx_stride]
    float* attn_part_o = nullptr;   // [B][H][attn_chunks][hd] split-order attention partials
    float* attn_part_ml = nullptr;  // [B][H][attn_chunks][2]
    int attn_chunks = 0;
    float* logits = nullptr;  // [B][V]
    float* probs = nullptr;   // [B][V] temperature probabilities of the last pass's rows
    float* qbuf = nullptr;    // [B][V] draft probabilities of the current speculative step
    float* tp_scratch = nullptr;  // temperature softmax scratch for B rows
    float* part_val = nullptr;
    int32_t* part_idx = nullptr;
    uint32_t* d_toks = nullptr;
    uint32_t* d_preds = nullptr;
    int32_t* d_pos = nullptr;
    int32_t* d_result = nullptr;
    uint32_t* d_samp = nullptr;  // [kSampleMaxRows] ids drawn by sample_logits
    float* ybuf = nullptr;       // [B][max(q|k|v rows, 2F, d)] plain matmul rows of split layers
    float* rope_tab = nullptr;
    // pinned host mirrors
    uint32_t* h_toks = nullptr;
    uint32_t* h_preds = nullptr;
    int32_t* h_result = nullptr;
    int32_t* h_pos = nullptr;
    int last_n = 0;
    uint32_t staged[16] = {};
    int n_staged = 0;  // staged tokens land in d_toks[0..n_staged); the rest stay as they are
    bool pending_toks = false;
    // captured passes (everything after the pass-state kernel), by pass_graph_key
    std::unordered_map<uint64_t, hipGraphExec_t> graphs;
    int64_t graph_captures = 0, graph_replays = 0;
    // per-stage timing (events between the pass's stages, named as the reference's trace stages)
    bool stage_timing = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> stage_ev;  // first kernel's start, last kernel's end
    std::vector<int> stage_of;                                // stage id of each recorded pair
    size_t stage_used = 0;
    std::vector<double> stage_ms;
    std::vector<int64_t> stage_calls;
    // per-kernel timing (HIP events on the session stream)
    bool timing = false;
    std::vector<std::pair<hipEvent_t, hipEvent_t>> ev;
    size_t ev_used = 0;
    double gemm_ms = 0.0;
    int64_t gemm_launches = 0, gemm_bytes = 0, pending_bytes = 0;
    // prompt passes of up to kPromptRows tokens (allocated by the first prompt that uses them)
    bool prompt_ready = false;
    float* p_hidden = nullptr;   // [R][d]
    int8_t* p_xq = nullptr;      // [R][maxw]
    float* p_xs = nullptr;       // [R][maxw/32]
    int32_t* p_xs8 = nullptr;    // [R][maxw/32]
    float* p_y = nullptr;        // [R][max(q|k|v rows, 2F, d)] matmul outputs
    float* p_q = nullptr;        // [R][aw]
    float* p_scores = nullptr;   // [kPromptGroup][H][ctx_stride]
    uint32_t* p_toks = nullptr;  // [max_ctx] the prompt's ids
    int32_t* p_pos = nullptr;    // [R / kPromptGroup] start positions of the attention row groups
    int8_t* p_xm = nullptr;      // matmul activations repacked in MFMA operand order
    float* p_xsm = nullptr;
    float* p_xam = nullptr;      // their block sums (Q4_K)
    std::vector<void*> allocs;
};

namespace nc {

// ---------------------------------------------------------------- errors
static thread_local std::string t_err;
void set_error(const std::string& msg) { t_err = msg; }
int fail(int code, const std::string& msg) {
    t_err = msg;
    return code;
}

static void parallel_for(int64_t n, int nthreads, const std::function<void(int64_t, int64_t)>& fn) {
    if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
    if (n < 1024 || nthreads == 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> th;
    const int64_t chunk = (n + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        const int64_t lo = t * chunk, hi = std::min(n, lo + chunk);
        if (lo >= hi) break;
        th.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto& t : th) t.join();
}

// ---------------------------------------------------------------- repacking
int64_t q40_layout_bytes(int64_t rows, int64_t cols) {
    const int64_t tiles = (rows + 63) / 64, groups = (cols / 32 + 7) / 8;
    return tiles * groups * kQ40ChunkBytes;
}
int64_t q4k_layout_bytes(int64_t rows, int64_t cols) { return (rows + 63) / 64 * (cols / 256) * kQ4KChunkBytes; }
int64_t q4k_r16_layout_bytes(int64_t rows, int64_t cols) {
    return (rows + 15) / 16 * ((cols / 256 + 3) / 4) * kQ4KChunkBytes;
}

static inline int64_t dst_row(int64_t r, int64_t row_off, int half) {
    return half < 0 ? row_off + r : (r / 32) * 64 + (r % 32) + 32 * half;
}

void repack_q4_0(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups, int64_t row_off,
                 int half) {
    const int64_t nb = cols / 32;
    parallel_for(rows_src, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const int64_t R = dst_row(r, row_off, half);
            const int64_t t = R / 64, l = R % 64;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t* blk = src + (r * nb + b) * 18;
                uint8_t* chunk = dst + (t * groups + b / 8) * kQ40ChunkBytes;
                std::memcpy(chunk + (b % 8) * 1024 + l * 16, blk + 2, 16);
                std::memcpy(chunk + 8192 + (b % 8 / 4) * 512 + l * 8 + (b % 4) * 2, blk, 2);
            }
        }
    });
}

int64_t q80_layout_bytes(int64_t rows, int64_t cols) {
    return (rows + 63) / 64 * ((cols / 32 + kQ80GroupBlocks - 1) / kQ80GroupBlocks) * kQ80ChunkBytes;
}

// Q8_0 block = f16 scale + 32 int8 (34 bytes, Q8_0Block::from_bytes q8.rs:479-487).
void repack_q8_0(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups, int64_t row_off,
                 int half) {
    const int64_t nb = cols / 32;
    parallel_for(rows_src, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const int64_t R = dst_row(r, row_off, half);
            const int64_t t = R / 64, l = R % 64;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t* blk = src + (r * nb + b) * 34;
                uint8_t* chunk = dst + (t * groups + b / kQ80GroupBlocks) * kQ80ChunkBytes;
                const int64_t u = b % kQ80GroupBlocks;
                std::memcpy(chunk + (2 * u) * 1024 + l * 16, blk + 2, 16);
                std::memcpy(chunk + (2 * u + 1) * 1024 + l * 16, blk + 18, 16);
                std::memcpy(chunk + kQ80GroupBlocks * 2048 + u * 128 + l * 2, blk, 2);
            }
        }
    });
}

int64_t q40_r16_layout_bytes(int64_t rows, int64_t cols) {
    const int64_t tiles = (rows + 15) / 16, groups = (cols / 32 + 31) / 32;
    return tiles * groups * kQ40ChunkBytes;
}

void repack_q4_0_r16(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups,
                     int64_t row_off, int half) {
    const int64_t nb = cols / 32;
    parallel_for(rows_src, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const int64_t R = dst_row(r, row_off, half);
            const int64_t t = R / 16, rr = R % 16;
            for (int64_t b = 0; b < nb; b++) {
                const uint8_t* blk = src + (r * nb + b) * 18;
                const int64_t qd = b / 4, j = b % 4, lane = 16 * j + rr;
                uint8_t* quad = dst + (t * groups + qd / 8) * kQ40ChunkBytes + (qd % 8) * kQ40R16QuadBytes;
                std::memcpy(quad + lane * 16, blk + 2, 16);
                // scales in [row / 4][block j][row % 4] order: each 4-row group's 16 scales are
                // 32 contiguous bytes (the MFMA kernel's lane group reads them in two 16-byte loads)
                std::memcpy(quad + 1024 + 2 * (16 * (rr / 4) + 4 * j + (rr % 4)), blk, 2);
            }
        }
    });
}

// Q4_K (nslot 9, 144-byte blocks) and Q5_K (nslot 11, 176-byte blocks) on 64-row tiles: per
// (tile, super-block) nslot x [64 lanes x 16 B], slot i = bytes 16i..16i+15 of the block.
void repack_q4_k(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t row_off, int half,
                 int nslot) {
    const int64_t nsb = cols / 256;
    parallel_for(rows_src, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const int64_t R = dst_row(r, row_off, half);
            const int64_t t = R / 64, l = R % 64;
            for (int64_t s = 0; s < nsb; s++) {
                const uint8_t* blk = src + (r * nsb + s) * 16 * nslot;
                uint8_t* chunk = dst + (t * nsb + s) * (int64_t)nslot * 1024;
                for (int i = 0; i < nslot; i++) std::memcpy(chunk + i * 1024 + l * 16, blk + i * 16, 16);
            }
        }
    });
}

void repack_q4_k_r16(const uint8_t* src, int64_t rows_src, int64_t cols, uint8_t* dst, int64_t groups,
                     int64_t row_off, int half) {
    const int64_t nsb = cols / 256;
    parallel_for(rows_src, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const int64_t R = dst_row(r, row_off, half), t = R / 16, rr = R % 16;
            for (int64_t s = 0; s < nsb; s++) {
                const uint8_t* blk = src + (r * nsb + s) * 144;
                uint8_t* chunk = dst + (t * groups + s / 4) * kQ4KChunkBytes + (16 * (s % 4) + rr) * 16;
                for (int i = 0; i < 9; i++) std::memcpy(chunk + i * 1024, blk + i * 16, 16);
            }
        }
    });
}

struct Part {
    const uint8_t* src;
    int64_t rows;
    int64_t row_off;
    int half;
};

// Builds one device matrix from one or more GGUF row blocks (fused q|k|v, interleaved
// gate/up, or a single matrix).
// Q6_K blocks (ql 128 | qh 64 | scales 16 | d 2 bytes) split into aligned planes
static void repack_q6_k_planes(const uint8_t* src, int64_t nblk, uint8_t* dst) {
    parallel_for(nblk, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t i = lo; i < hi; i++) {
            const uint8_t* b = src + i * 210;
            std::memcpy(dst + i * 128, b, 128);
            std::memcpy(dst + nblk * 128 + i * 64, b + 128, 64);
            std::memcpy(dst + nblk * 192 + i * 16, b + 192, 16);
            std::memcpy(dst + nblk * 208 + i * 2, b + 208, 2);
        }
    });
}

static int upload_matrix(int type, int64_t rows, int64_t cols, const std::vector<Part>& parts, QMatDev& out) {
    if (cols % 32 || ((type == NC_TYPE_Q4_K || type == NC_TYPE_Q5_K || type == NC_TYPE_Q6_K) && cols % 256))
        return fail(NC_EINVAL, "matrix columns must be a multiple of 32 (Q4_K, Q5_K, Q6_K: 256)");
    if (type == NC_TYPE_Q6_K) {
        if (parts.size() != 1 || parts[0].half >= 0 || parts[0].rows != rows || cols > 16384)
            return fail(NC_EINVAL, "Q6_K: single matrices of at most 16384 columns");
        out.type = type;
        out.layout = LAYOUT_Q6K;
        out.rows = rows;
        out.cols = cols;
        out.units = cols / 256;
        out.tiles = (rows + q6k_rows_per_tile(cols) - 1) / q6k_rows_per_tile(cols);
        out.groups = 0;
        out.algo_bytes = rows * (cols / 256) * 210;
        out.dev_bytes = out.algo_bytes + 4;
        std::vector<uint8_t> host(out.dev_bytes, 0);
        repack_q6_k_planes(parts[0].src, rows * (cols / 256), host.data());
        NC_HIP(hipMalloc((void**)&out.dev, out.dev_bytes));
        NC_HIP(hipMemcpy(out.dev, host.data(), out.dev_bytes, hipMemcpyHostToDevice));
        return NC_OK;
    }
    out.type = type;
    out.rows = rows;
    out.cols = cols;
    if (type == NC_TYPE_Q8_0) {
        out.layout = LAYOUT_Q80;
        out.units = cols / 32;
        out.tiles = (rows + 63) / 64;
        out.groups = (out.units + kQ80GroupBlocks - 1) / kQ80GroupBlocks;
        out.dev_bytes = q80_layout_bytes(rows, cols);
        out.algo_bytes = rows * cols / 32 * 34;
        std::vector<uint8_t> host(out.dev_bytes, 0);
        for (const auto& p : parts) repack_q8_0(p.src, p.rows, cols, host.data(), out.groups, p.row_off, p.half);
        NC_HIP(hipMalloc((void**)&out.dev, out.dev_bytes));
        NC_HIP(hipMemcpy(out.dev, host.data(), out.dev_bytes, hipMemcpyHostToDevice));
        return NC_OK;
    }
    // R16 for Q4_0 matrices below 1024 64-row tiles: every layer matrix up to the 70B shape
    // (57344 x 8192 as a plain matmul, us at N = 1 / 5 / 9 / 16: R64 47.7 / 78.1 / 110.2 / 288.3,
    // R16 43.6 / 70.1 / 92.1 / 129.0; the 70B verify pass 34.6 -> 30.5 ms), while the 128256 x 4096
    // head stays on R64 (R16 78.7 against 69.5 us at N = 5).  An interleaved gate/up pair keeps
    // its 64-row groups (gate rows 32t.. in rows 0-31 of group t, up rows in 32-63): with R16
    // those are four consecutive 16-row tiles, which one workgroup covers.
    // Q4_K likewise on 16-row tiles below 256 64-row tiles; an interleaved gate/up pair below
    // 1024 64-row groups (its SwiGLU epilogue takes four consecutive 16-row tiles).
    const bool single = std::all_of(parts.begin(), parts.end(), [](const Part& q) { return q.half < 0; });
    // NC_R16_MAX_TILES=<n>: tuning override of the 64-row tile count below which Q4_0 takes R16
    static const int64_t r16_max = [] {
        const char* e = getenv("NC_R16_MAX_TILES");
        return e ? std::max<int64_t>(1, atoll(e)) : (int64_t)1024;
    }();
    out.layout = type == NC_TYPE_Q4_0 && (rows + 63) / 64 < r16_max ? LAYOUT_R16 : LAYOUT_R64;
    if (type == NC_TYPE_Q4_K && (rows + 63) / 64 < (single ? 256 : 1024)) out.layout = LAYOUT_R16K;
    out.units = type == NC_TYPE_Q4_0 ? cols / 32 : cols / 256;
    if (out.layout == LAYOUT_R16) {
        out.tiles = (rows + 15) / 16;
        out.groups = (out.units + 31) / 32;
        out.dev_bytes = q40_r16_layout_bytes(rows, cols);
    } else if (out.layout == LAYOUT_R16K) {
        out.tiles = (rows + 15) / 16;
        out.groups = (out.units + 3) / 4;
        out.dev_bytes = q4k_r16_layout_bytes(rows, cols);
    } else {
        out.tiles = (rows + 63) / 64;
        out.groups = type == NC_TYPE_Q4_0 ? (out.units + 7) / 8 : 0;
        out.dev_bytes = type == NC_TYPE_Q4_0 ? q40_layout_bytes(rows, cols)
                        : type == NC_TYPE_Q5_K ? q4k_layout_bytes(rows, cols) / 9 * 11
                                               : q4k_layout_bytes(rows, cols);
    }
    out.algo_bytes = type == NC_TYPE_Q4_0 ? rows * cols / 32 * 18
                     : type == NC_TYPE_Q5_K ? rows * cols / 256 * 176
                                            : rows * cols / 256 * 144;
    std::vector<uint8_t> host(out.dev_bytes, 0);
    for (const auto& p : parts) {
        if (out.layout == LAYOUT_R16) repack_q4_0_r16(p.src, p.rows, cols, host.data(), out.groups, p.row_off, p.half);
        else if (out.layout == LAYOUT_R16K) repack_q4_k_r16(p.src, p.rows, cols, host.data(), out.groups, p.row_off, p.half);
        else if (type == NC_TYPE_Q4_0) repack_q4_0(p.src, p.rows, cols, host.data(), out.groups, p.row_off, p.half);
        else repack_q4_k(p.src, p.rows, cols, host.data(), p.row_off, p.half, type == NC_TYPE_Q5_K ? 11 : 9);
    }
    NC_HIP(hipMalloc((void**)&out.dev, out.dev_bytes));
    NC_HIP(hipMemcpy(out.dev, host.data(), out.dev_bytes, hipMemcpyHostToDevice));
    return NC_OK;
}

// ---------------------------------------------------------------- f16 helpers (host)

// q8.rs:3644-3673 fast_f32_to_f16 (truncating), used by the tied-head requantisation.
static uint16_t f32_to_f16_trunc(float value) {
    uint32_t bits;
    std::memcpy(&bits, &value, 4);
    const uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    const int32_t exponent = (int32_t)((bits >> 23) & 0xffu);
    const uint32_t fraction = bits & 0x007fffffu;
    if (exponent == 0) return sign;
    if (exponent == 0xff) return (uint16_t)(sign | 0x7c00u | (fraction ? ((fraction >> 13) | 1u) : 0u));
    const int32_t he = exponent - 127 + 15;
    if (he >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (he <= 0) {
        if (he < -10) return sign;
        return (uint16_t)(sign | (uint16_t)((fraction | 0x00800000u) >> (14 - he)));
    }
    return (uint16_t)(sign | (uint16_t)(he << 10) | (uint16_t)(fraction >> 13));
}

// Rust `f32 as i32` (saturating truncation, NaN -> 0).
static inline int32_t f32_as_i32(float v) {
    if (v != v) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

// quantize_f32_matrix_to_q4_0_blocks (q8.rs:2442-2488) for the tied LM head.
static void requant_tied_head(const float* emb, int64_t rows, int64_t cols, uint8_t* out) {
    const int64_t bpr = cols / 32;
    parallel_for(rows, 0, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++)
            for (int64_t b = 0; b < bpr; b++) {
                const float* c = emb + r * cols + b * 32;
                float amax = 0.0f, mx = 0.0f;
                for (int i = 0; i < 32; i++) {
                    const float a = std::fabs(c[i]);
                    if (a > amax) {
                        amax = a;
                        mx = c[i];
                    }
                }
                const float d = mx / -8.0f;
                const float id = d != 0.0f ? 1.0f / d : 0.0f;
                uint8_t* blk = out + (r * bpr + b) * 18;
                const uint16_t sb = f32_to_f16_trunc(d);
                blk[0] = (uint8_t)(sb & 0xff);
                blk[1] = (uint8_t)(sb >> 8);
                for (int j = 0; j < 16; j++) {
                    const float x0 = c[j] * id + 8.5f, x1 = c[j + 16] * id + 8.5f;
                    int q0 = f32_as_i32(x0), q1 = f32_as_i32(x1);
                    q0 = q0 < 0 ? 0 : (q0 > 15 ? 15 : q0);
                    q1 = q1 < 0 ? 0 : (q1 > 15 ? 15 : q1);
                    blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
                }
            }
    });
}

// load_f32_or_f16 (model.rs:1081-1230) for the types this path meets.
// load_f32_or_f16 (model.rs:1081-1229): the tensor decoded to f32 (dequant.cpp).
static int tensor_to_f32(const GgufFile& g, const std::string& name, std::vector<float>& out) {
    const GgufTensor* t = g.find(name);
    if (!t) return fail(NC_EFORMAT, "tensor " + name + " not found in GGUF");
    std::string err;
    const uint8_t* p = g.bytes(*t, err);
    if (!p) return fail(NC_EFORMAT, err);
    uint64_t el = 1;
    for (auto d : t->dims) el *= d;
    out.resize(el);
    int rc = dequant_f32(t->type, p, el, out.data(), 0);
    return rc ? fail(rc, name + ": " + t_err) : NC_OK;
}

// ---------------------------------------------------------------- tensor validation
// validate_model_tensors (model.rs:851-1036) for the dense Llama layout this build runs:
// every tensor the model needs is present with the descriptor shape the reference accepts
// ([input, output] or its transpose for matrices, [width] for norms) and the token rows of
// the embedding and the head fill their byte size exactly.  Layouts the reference also reads
// but this build does not run (fused q|k|v or gate|up, attention biases, mixture-of-experts
// layers) are refused here, before anything is uploaded.
static std::string dims_str(const std::vector<uint64_t>& d) {
    std::string s = "[";
    for (size_t i = 0; i < d.size(); i++) s += (i ? ", " : "") + std::to_string(d[i]);
    return s + "]";
}

static int require_shape(const GgufFile& g, const std::string& name, const std::vector<uint64_t>& want,
                         const std::string& role, const GgufTensor** out = nullptr) {
    const GgufTensor* t = g.find(name);
    if (!t) return fail(NC_EFORMAT, "tensor " + name + " not found in GGUF");
    if (t->dims != want)
        return fail(NC_EFORMAT, role + " tensor " + name + " expected descriptor shape " + dims_str(want) + ", got " +
                                    dims_str(t->dims));
    if (out) *out = t;
    return NC_OK;
}

static int require_matrix(const GgufFile& g, const std::string& name, uint64_t in, uint64_t outw,
                          const std::string& role, const GgufTensor** out = nullptr) {
    const GgufTensor* t = g.find(name);
    if (!t) return fail(NC_EFORMAT, "tensor " + name + " not found in GGUF");
    const std::vector<uint64_t> direct{in, outw}, transposed{outw, in};
    if (t->dims != direct && t->dims != transposed)
        return fail(NC_EFORMAT, role + " tensor " + name + " expected descriptor shape " + dims_str(direct) + " or " +
                                    dims_str(transposed) + ", got " + dims_str(t->dims));
    if (out) *out = t;
    return NC_OK;
}

// validate_token_row_storage_layout (model.rs:1477-1530)
static int require_token_rows(const GgufTensor& t, uint64_t hidden, uint64_t vocab, const std::string& role) {
    uint64_t row_values;
    if (t.dims.size() == 2 && t.dims[0] == hidden && t.dims[1] == vocab) row_values = hidden;
    else if (t.dims.size() == 2 && t.dims[0] == vocab && t.dims[1] == hidden) row_values = hidden;
    else return NC_OK;
    uint64_t bs, ts;
    if (!gguf_type_layout(t.type, &bs, &ts))
        return fail(NC_EFORMAT, role + " tensor " + t.name + " has unsupported storage type for token-row validation");
    if (row_values % bs)
        return fail(NC_EFORMAT, role + " tensor " + t.name + " token-row width " + std::to_string(row_values) +
                                    " is not divisible by block size " + std::to_string(bs));
    const uint64_t expected = row_values / bs * ts * vocab;
    if (t.nbytes != expected)
        return fail(NC_EFORMAT, role + " tensor " + t.name + " byte size " + std::to_string(t.nbytes) +
                                    " does not match " + std::to_string(vocab) + " token rows (" + std::to_string(expected) +
                                    " bytes)");
    return NC_OK;
}

static int validate_model_tensors(const GgufFile& g, const nc_model_config& c) {
    const uint64_t d = c.embedding_length, V = c.vocab_size, F = c.feed_forward_length;
    const uint64_t aw = c.attention_output_width, kw = c.kv_width;
    const GgufTensor* t = nullptr;
    int rc;
    if ((rc = require_matrix(g, "token_embd.weight", d, V, "token embedding", &t)) ||
        (rc = require_token_rows(*t, d, V, "token embedding")) ||
        (rc = require_shape(g, "output_norm.weight", {d}, "output norm")))
        return rc;
    if (g.find("output.weight")) {
        if ((rc = require_matrix(g, "output.weight", d, V, "output projection", &t)) ||
            (rc = require_token_rows(*t, d, V, "output projection")))
            return rc;
    }
    for (int64_t i = 0; i < c.block_count; i++) {
        const std::string b = "blk." + std::to_string(i) + ".", L = "layer " + std::to_string(i) + " ";
        if ((rc = require_shape(g, b + "attn_norm.weight", {d}, L + "attention norm"))) return rc;
        if (g.find(b + "attn_qkv.weight"))
            return fail(NC_EFORMAT, "tensor " + b + "attn_qkv.weight: fused q|k|v layers are not supported");
        for (const char* bias : {"attn_q.bias", "attn_k.bias", "attn_v.bias"})
            if (g.find(b + bias)) return fail(NC_EFORMAT, "tensor " + b + bias + ": attention biases are not supported");
        if ((rc = require_matrix(g, b + "attn_q.weight", d, aw, L + "attention q")) ||
            (rc = require_matrix(g, b + "attn_k.weight", d, kw, L + "attention k")) ||
            (rc = require_matrix(g, b + "attn_v.weight", d, kw, L + "attention v")) ||
            (rc = require_matrix(g, b + "attn_output.weight", aw, d, L + "attention output")) ||
            (rc = require_shape(g, b + "ffn_norm.weight", {d}, L + "ffn norm")))
            return rc;
        if (g.find(b + "ffn_gate.0.weight") || g.find(b + "ffn_gate_inp.weight"))
            return fail(NC_EFORMAT, "layer " + std::to_string(i) + ": mixture-of-experts layers are not supported");
        if (!g.find(b + "ffn_gate.weight"))
            return fail(NC_EFORMAT, "layer " + std::to_string(i) + ": fused ffn gate|up (no ffn_gate.weight) is not supported");
        if ((rc = require_matrix(g, b + "ffn_gate.weight", d, F, L + "ffn gate")) ||
            (rc = require_matrix(g, b + "ffn_up.weight", d, F, L + "ffn up")) ||
            (rc = require_matrix(g, b + "ffn_down.weight", F, d, L + "ffn down")))
            return rc;
    }
    return NC_OK;
}

template <typename T>
static int dev_alloc(std::vector<void*>& list, T** p, size_t count) {
    if (count == 0) count = 1;
    hipError_t e = hipMalloc((void**)p, count * sizeof(T));
    if (e != hipSuccess) return fail(NC_ENOMEM, std::string("hipMalloc: ") + hipGetErrorString(e));
    list.push_back(*p);
    return NC_OK;
}

static int upload_f32(std::vector<void*>& list, const std::vector<float>& h, float** d) {
    int rc = dev_alloc(list, d, h.size());
    if (rc) return rc;
    NC_HIP(hipMemcpy(*d, h.data(), h.size() * 4, hipMemcpyHostToDevice));
    return NC_OK;
}

static const GgufTensor* matrix_desc(const GgufFile& g, const std::string& name, int64_t rows, int64_t cols, int* err,
                                     bool allow_q6k = false) {
    const GgufTensor* t = g.find(name);
    if (!t) {
        *err = fail(NC_EFORMAT, "missing tensor " + name);
        return nullptr;
    }
    if (t->dims.size() != 2 || (int64_t)t->dims[0] != cols || (int64_t)t->dims[1] != rows) {
        *err = fail(NC_EFORMAT, "tensor " + name + ": transposed (output-major) storage " + dims_str(t->dims) +
                                    " is not supported");
        return nullptr;
    }
    if (t->type != NC_TYPE_Q4_0 && t->type != NC_TYPE_Q4_K && t->type != NC_TYPE_Q5_K && t->type != NC_TYPE_Q8_0 &&
        !(allow_q6k && t->type == NC_TYPE_Q6_K)) {
        *err = fail(NC_EFORMAT, "tensor " + name + ": only Q4_0, Q4_K, Q5_K, Q8_0" + (allow_q6k ? " and Q6_K" : "") +
                                    " matrices are supported, got GGML type " + std::to_string(t->type));
        return nullptr;
    }
    std::string e;
    if (!g.bytes(*t, e)) {
        *err = fail(NC_EFORMAT, e);
        return nullptr;
    }
    return t;
}

static void free_model(nc_model* m) {
    if (!m) return;
    for (void* p : m->allocs) (void)hipFree(p);
    if (m->head.dev) (void)hipFree(m->head.dev);
    for (auto& l : m->layers)
        for (auto* q : l.all())
            if (q->dev) (void)hipFree(q->dev);
    delete m;
}

// LlamaModelConfig::from_gguf (model.rs:48-186) plus this build's support checks and
// validate_model_tensors: everything decided from the header, before any weight is read.
static int read_config(const GgufFile& g, nc_model_config& c) {
    c = nc_model_config{};
    if (g.get_str("general.architecture") != "llama")
        return fail(NC_EFORMAT, "unsupported architecture: " + g.get_str("general.architecture"));
    // LlamaModelConfig::from_gguf (model.rs:48-186)
    uint32_t v;
    const std::string P = "llama.";
    if (!g.get_u32(P + "context_length", &v)) return fail(NC_EFORMAT, "missing llama.context_length");
    c.context_length = v;
    if (!g.get_u32(P + "embedding_length", &v)) return fail(NC_EFORMAT, "missing llama.embedding_length");
    c.embedding_length = v;
    if (!g.get_u32(P + "block_count", &v)) return fail(NC_EFORMAT, "missing llama.block_count");
    c.block_count = v;
    if (!g.get_u32(P + "feed_forward_length", &v)) return fail(NC_EFORMAT, "missing llama.feed_forward_length");
    c.feed_forward_length = v;
    if (!g.get_u32(P + "attention.head_count", &v) || v == 0) return fail(NC_EFORMAT, "bad attention.head_count");
    c.head_count = v;
    c.head_count_kv = g.get_u32(P + "attention.head_count_kv", &v) ? v : c.head_count;
    if (c.embedding_length % c.head_count || c.head_count_kv == 0 || c.head_count % c.head_count_kv)
        return fail(NC_EFORMAT, "inconsistent head geometry");
    float f;
    c.rope_freq_base = g.get_f32(P + "rope.freq_base", &f) ? f : 10000.0f;
    {  // rope_scaling_from_gguf (main.rs:8522-8535): used only when all four keys are present
        float fac = 0, lo = 0, hi = 0;
        uint32_t orig = 0;
        const bool a = g.get_f32(P + "rope.scaling.factor", &fac);
        const bool b = g.get_u32(P + "rope.scaling.original_context_length", &orig);
        const bool cc = g.get_f32(P + "rope.scaling.low_freq_factor", &lo);
        const bool dd = g.get_f32(P + "rope.scaling.high_freq_factor", &hi);
        c.rope_scaling = a && b && cc && dd ? 1 : 0;
        if (c.rope_scaling) {
            c.rope_scaling_factor = fac;
            c.rope_scaling_original_context_length = (float)orig;
            c.rope_scaling_low_freq_factor = lo;
            c.rope_scaling_high_freq_factor = hi;
        }
    }
    c.rms_norm_epsilon = g.get_f32(P + "attention.layer_norm_rms_epsilon", &f) ? f : 1e-5f;
    const GgufTensor* te = g.find("token_embd.weight");
    if (!te || te->dims.size() != 2) return fail(NC_EFORMAT, "missing token_embd.weight");
    c.vocab_size = g.get_u32(P + "vocab_size", &v) ? v
                   : ((int64_t)te->dims[0] == c.embedding_length ? (int64_t)te->dims[1] : (int64_t)te->dims[0]);
    c.head_dim = g.get_u32(P + "attention.key_length", &v) ? v : c.embedding_length / c.head_count;
    c.rope_dimension_count = g.get_u32(P + "rope.dimension_count", &v) ? v : c.head_dim;
    if (c.rope_dimension_count == 0 || c.rope_dimension_count > c.head_dim || c.rope_dimension_count % 2)
        return fail(NC_EFORMAT, "invalid rope.dimension_count");
    c.attention_output_width = c.head_count * c.head_dim;
    c.kv_width = c.head_count_kv * c.head_dim;
    const int64_t d = c.embedding_length, F = c.feed_forward_length;
    const int64_t aw = c.attention_output_width, kw = c.kv_width;
    if (aw % 64 || kw % 64 || F % 32 || d % 256)
        return fail(NC_EINVAL, "model widths must be multiples of 64 (attention), 32 (ffn), 256 (embedding)");
    if (c.head_dim != 64 && c.head_dim != 128) return fail(NC_EINVAL, "head_dim must be 64 or 128");
    if (c.head_count / c.head_count_kv > 8) return fail(NC_EINVAL, "at most 8 query heads per KV head");
    if (const int rc = validate_model_tensors(g, c)) return rc;
    // the first layer's attention-query type; each matrix keeps its own type when a file
    // mixes them (llama.cpp Q4_K_M), so this does not describe the other matrices
    const GgufTensor* tq = g.find("blk.0.attn_q.weight");
    c.weight_type = tq ? (int32_t)tq->type : -1;
    return NC_OK;
}

static int load_model(nc_ctx* ctx, const uint8_t* data, size_t size, const nc_load_opts* opts, nc_model** out) {
    GgufFile g;
    std::string err;
    if (!gguf_parse(data, size, g, err)) return fail(NC_EFORMAT, err);
    std::unique_ptr<nc_model, void (*)(nc_model*)> m(new nc_model(), free_model);
    m->ctx = ctx;
    nc_model_config& c = m->cfg;
    int rc0 = read_config(g, c);
    if (rc0) return rc0;
    const int64_t d = c.embedding_length, F = c.feed_forward_length, V = c.vocab_size;
    const int64_t aw = c.attention_output_width, kw = c.kv_width;
    // weights (LlamaWeights::load, model.rs:461-545)
    std::vector<float> emb;
    int rc = tensor_to_f32(g, "token_embd.weight", emb);
    if (rc) return rc;
    if ((int64_t)emb.size() != V * d) return fail(NC_EFORMAT, "token_embd.weight size mismatch");
    if ((rc = upload_f32(m->allocs, emb, &m->tok_emb))) return rc;
    std::vector<float> tmp;
    if ((rc = tensor_to_f32(g, "output_norm.weight", tmp))) return rc;
    if ((int64_t)tmp.size() != d) return fail(NC_EFORMAT, "output_norm.weight size mismatch");
    if ((rc = upload_f32(m->allocs, tmp, &m->out_norm))) return rc;
    if (const GgufTensor* ot = g.find("output.weight")) {
        int e = 0;
        if (!matrix_desc(g, "output.weight", V, d, &e, true)) return e;
        if ((rc = upload_matrix((int)ot->type, V, d, {{g.data + ot->offset, V, 0, -1}}, m->head))) return rc;
        c.tied_head = 0;
    } else {
        // model.rs:471-532: tied head requantised to Q4_0 from the f32 embeddings
        std::vector<uint8_t> blocks((size_t)V * (d / 32) * 18);
        requant_tied_head(emb.data(), V, d, blocks.data());
        if ((rc = upload_matrix(NC_TYPE_Q4_0, V, d, {{blocks.data(), V, 0, -1}}, m->head))) return rc;
        c.tied_head = 1;
    }
    emb.clear();
    emb.shrink_to_fit();
    m->layers.resize(c.block_count);
    for (int64_t i = 0; i < c.block_count; i++) {
        LayerDev& L = m->layers[i];
        const std::string b = "blk." + std::to_string(i) + ".";
        if ((rc = tensor_to_f32(g, b + "attn_norm.weight", tmp))) return rc;
        if ((rc = upload_f32(m->allocs, tmp, &L.attn_norm))) return rc;
        if ((rc = tensor_to_f32(g, b + "ffn_norm.weight", tmp))) return rc;
        if ((rc = upload_f32(m->allocs, tmp, &L.ffn_norm))) return rc;
        // each matrix keeps its own type, as matmul_quantized_batch dispatches per matrix
        // (inference.rs:1246-1303)
        int e = 0;
        const GgufTensor* tq = matrix_desc(g, b + "attn_q.weight", aw, d, &e, true);
        const GgufTensor* tk = tq ? matrix_desc(g, b + "attn_k.weight", kw, d, &e, true) : nullptr;
        const GgufTensor* tv = tk ? matrix_desc(g, b + "attn_v.weight", kw, d, &e, true) : nullptr;
        const GgufTensor* to = tv ? matrix_desc(g, b + "attn_output.weight", d, aw, &e, true) : nullptr;
        const GgufTensor* tg = to ? matrix_desc(g, b + "ffn_gate.weight", F, d, &e, true) : nullptr;
        const GgufTensor* tu = tg ? matrix_desc(g, b + "ffn_up.weight", F, d, &e, true) : nullptr;
        const GgufTensor* tdn = tu ? matrix_desc(g, b + "ffn_down.weight", d, F, &e, true) : nullptr;
        if (!tdn) return e;
        const int ty = (int)tq->type;
        const auto fusable = [](uint32_t t) {
            return t == NC_TYPE_Q4_0 || t == NC_TYPE_Q4_K || t == NC_TYPE_Q5_K || t == NC_TYPE_Q8_0;
        };
        const auto one = [&](const GgufTensor* t, int64_t rows, int64_t cols, QMatDev& out) {
            return upload_matrix((int)t->type, rows, cols, {{g.data + t->offset, rows, 0, -1}}, out);
        };
        if (fusable(tq->type) && tk->type == tq->type && tv->type == tq->type) {
            if ((rc = upload_matrix(ty, aw + 2 * kw, d,
                                    {{g.data + tq->offset, aw, 0, -1}, {g.data + tk->offset, kw, aw, -1},
                                     {g.data + tv->offset, kw, aw + kw, -1}},
                                    L.qkv)))
                return rc;
        } else {
            L.split_qkv = true;
            if ((rc = one(tq, aw, d, L.q)) || (rc = one(tk, kw, d, L.k)) || (rc = one(tv, kw, d, L.v))) return rc;
        }
        if ((rc = one(to, d, aw, L.wo))) return rc;
        if (fusable(tg->type) && tu->type == tg->type) {
            if ((rc = upload_matrix((int)tg->type, 2 * F, d,
                                    {{g.data + tg->offset, F, 0, 0}, {g.data + tu->offset, F, 0, 1}}, L.gateup)))
                return rc;
        } else {
            L.split_gateup = true;
            if ((rc = one(tg, F, d, L.gate)) || (rc = one(tu, F, d, L.up))) return rc;
        }
        if ((rc = one(tdn, d, F, L.down))) return rc;
    }
    int64_t devb = m->head.dev_bytes, algo = m->head.algo_bytes;
    for (auto& L : m->layers)
        for (auto* q : L.all()) {
            devb += q->dev_bytes;
            algo += q->algo_bytes;
        }
    c.device_weight_bytes = devb;
    c.verify_weight_bytes = algo;
    (void)opts;
    *out = m.release();
    return NC_OK;
}

// ---------------------------------------------------------------- session pass
static int timed_gemm(nc_session* s, const QMatDev& w, const GemmParams& p) {
    if (!s->timing) return launch_gemm(w, p, s->stream);
    if (s->ev_used == s->ev.size()) {
        NC_HIP(hipStreamSynchronize(s->stream));
        for (auto& e : s->ev) {
            float ms = 0;
            NC_HIP(hipEventElapsedTime(&ms, e.first, e.second));
            s->gemm_ms += ms;
        }
        s->gemm_bytes += s->pending_bytes;
        s->pending_bytes = 0;
        s->ev_used = 0;
    }
    auto& e = s->ev[s->ev_used++];
    int rc = launch_gemm(w, p, s->stream, e.first, e.second);
    s->gemm_launches++;
    // algorithmic bytes: weights + int8 activations + f32 scales + f32 outputs
    s->pending_bytes += w.algo_bytes + (int64_t)p.N * w.cols + 4 * (int64_t)p.N * (w.cols / 32) + 4 * (int64_t)p.N * w.rows;
    return rc;
}

static int flush_timing(nc_session* s) {
    if (!s->timing || s->ev_used == 0) return NC_OK;
    NC_HIP(hipStreamSynchronize(s->stream));
    for (size_t i = 0; i < s->ev_used; i++) {
        float ms = 0;
        NC_HIP(hipEventElapsedTime(&ms, s->ev[i].first, s->ev[i].second));
        s->gemm_ms += ms;
    }
    s->gemm_bytes += s->pending_bytes;
    s->pending_bytes = 0;
    s->ev_used = 0;
    return NC_OK;
}

// A matmul of the session's quantised rows (xq / xs / xs8) stored as plain f32 rows.
static GemmParams plain_rows(const nc_session* s, int n, float* out, int ld_out) {
    GemmParams p;
    p.kernel = s->ctx->gemm_kernel;
    p.x = s->xq;
    p.xs = s->xs;
    p.xs8 = s->xs8;
    p.N = n;
    p.epi = EPI_STORE;
    p.out = out;
    p.ld_out = ld_out;
    return p;
}

// hidden += matmul (the residual adds, inference.rs:3985, 4073): in the epilogue, or for
// Q6_K matrices (plain and head outputs only) as plain rows and a separate add.
static int residual_gemm(nc_session* s, const QMatDev& w, GemmParams& p, int n) {
    if (w.type != NC_TYPE_Q6_K) return timed_gemm(s, w, p);
    GemmParams pp = p;
    pp.epi = EPI_STORE;
    pp.out = s->ybuf;
    pp.ld_out = (int)w.rows;
    int rc = timed_gemm(s, w, pp);
    if (!rc) rc = launch_prompt_residual(s->ybuf, p.out, n, (int)w.rows, s->stream);
    return rc;
}

// Stages of a verify / decode pass, named as the reference's NANOCAMELID_TRACE stages
// (inference.rs:179-229, recorded at :3732-4109 and :4460-4832); stages the device fuses into one
// kernel carry the names of all of them.
static const char* const kStageNames[] = {
    "batch.embed_lookup",
    "batch.attn_norm+batch.attn_quant",
    "batch.wq+batch.wk+batch.wv+batch.rope_store_kv",
    "batch.attention+batch.wo_quant",
    "batch.wo",
    "batch.ffn_norm+batch.ffn_quant",
    "batch.w1+batch.w3+batch.silu_mul+batch.down_quant",
    "batch.w2",
    "decode.head_norm+decode.head_quant",
    "decode.head",
};
constexpr int kStages = (int)(sizeof(kStageNames) / sizeof(kStageNames[0]));
enum Stage { ST_EMBED, ST_ATTN_NORM, ST_QKV, ST_ATTENTION, ST_WO, ST_FFN_NORM, ST_GATEUP, ST_DOWN, ST_HEAD_NORM, ST_HEAD };

thread_local hipEvent_t t_stage_ev0 = nullptr, t_stage_ev1 = nullptr;

// Resolves the recorded stages: each pair spans the kernels of one stage (dispatch-stamped).
static int flush_stages(nc_session* s) {
    if (s->stage_used == 0) return NC_OK;
    NC_HIP(hipStreamSynchronize(s->stream));
    for (size_t i = 0; i < s->stage_used; i++) {
        float ms = 0;
        NC_HIP(hipEventElapsedTime(&ms, s->stage_ev[i].first, s->stage_ev[i].second));
        s->stage_ms[s->stage_of[i]] += ms;
        s->stage_calls[s->stage_of[i]]++;
    }
    s->stage_used = 0;
    return NC_OK;
}

// Ends the current stage and, for stage >= 0, starts the next: the kernels launched until the
// next mark stamp its event pair (NC_LAUNCH).
static void stage_mark(nc_session* s, int stage) {
    t_stage_ev0 = t_stage_ev1 = nullptr;
    if (!s->stage_timing || stage < 0) return;
    const size_t i = s->stage_used++;
    t_stage_ev0 = s->stage_ev[i].first;
    t_stage_ev1 = s->stage_ev[i].second;
    s->stage_of[i] = stage;
}

// Before a pass: room for its stages (the embedding, 7 per layer, 2 for the head), else resolve
// the recorded ones.
static int stage_reserve(nc_session* s) {
    if (!s->stage_timing) return NC_OK;
    const size_t need = 3 + 7 * (size_t)s->m->cfg.block_count;
    if (s->stage_used + need > s->stage_ev.size()) return flush_stages(s);
    return NC_OK;
}

// One forward over the n tokens already in d_toks at positions start_pos..: embedding,
// all layers (run_layer_range_batch, inference.rs:3747-4111), final norm, head and
// per-row argmax.  Writes d_preds and logits.
static int pass_body(nc_session* s, int n, int64_t start_pos, bool head) {
    nc_model* m = s->m;
    const nc_model_config& c = m->cfg;
    const int d = (int)c.embedding_length, aw = (int)c.attention_output_width, kw = (int)c.kv_width;
    const int F = (int)c.feed_forward_length, hd = (int)c.head_dim, Hkv = (int)c.head_count_kv;
    hipStream_t st = s->stream;
    int rc = launch_embed(m->tok_emb, s->d_toks, n, d, s->hidden, st);
    if (rc) return rc;
    const size_t layer_kv = (size_t)Hkv * s->ctx_stride * hd;
    for (int64_t li = 0; li < c.block_count; li++) {
        const LayerDev& L = m->layers[li];
        stage_mark(s, ST_ATTN_NORM);
        if ((rc = launch_rmsnorm_q8(s->hidden, L.attn_norm, n, d, c.rms_norm_epsilon, s->xq, s->xs, s->xs8, st)))
            return rc;
        stage_mark(s, ST_QKV);
        GemmParams p;
        p.kernel = s->ctx->gemm_kernel;
        p.x = s->xq;
        p.xs = s->xs;
        p.xs8 = s->xs8;
        p.N = n;
        p.epi = EPI_QKV_ROPE;
        p.q_out = s->q;
        p.aw = aw;
        p.kw = kw;
        p.hd = hd;
        p.rope_half = (int)c.rope_dimension_count / 2;
        p.max_ctx = (int)s->ctx_stride;
        p.kv_heads = Hkv;
        p.rope_tab = s->rope_tab;
        p.kcache = s->kcache + li * layer_kv;
        p.vcache = s->vcache + li * layer_kv;
        p.d_pos = s->d_pos;
        if (!L.split_qkv) {
            if ((rc = timed_gemm(s, L.qkv, p))) return rc;
        } else {
            // q, k, v rows side by side in ybuf, then RoPE and the cache stores as one kernel
            const int ldy = aw + 2 * kw;
            const std::pair<const QMatDev*, int> parts[3] = {{&L.q, 0}, {&L.k, aw}, {&L.v, aw + kw}};
            for (const auto& [w, off] : parts)
                if ((rc = timed_gemm(s, *w, plain_rows(s, n, s->ybuf + off, ldy)))) return rc;
            if ((rc = launch_prompt_qkv_rope(s->ybuf, n, (int)start_pos, aw, kw, hd, p.rope_half, s->rope_tab, s->q,
                                             p.kcache, p.vcache, (int)s->ctx_stride, st)))
                return rc;
        }
        AttnParams a;
        a.q = s->q;
        a.kcache = p.kcache;
        a.vcache = p.vcache;
        a.scores = s->scores;
        a.xq = s->xq;
        a.xs = s->xs;
        a.xs8 = s->xs8;
        a.d_pos = s->d_pos;
        a.N = n;
        a.H = (int)c.head_count;
        a.Hkv = Hkv;
        a.hd = hd;
        a.max_ctx = (int)s->ctx_stride;
        a.max_pos = (int)(start_pos + n - 1);
        a.scale = 1.0f / std::sqrt((float)hd);  // inference.rs:3927
        a.split = s->ctx->attn_order == NC_ATTN_SPLIT;
        a.part_o = s->attn_part_o;
        a.part_ml = s->attn_part_ml;
        a.nchunks = s->attn_chunks;
        stage_mark(s, ST_ATTENTION);
        if ((rc = launch_attention(a, st))) return rc;
        stage_mark(s, ST_WO);
        GemmParams po;
        po.kernel = s->ctx->gemm_kernel;
        po.x = s->xq;
        po.xs = s->xs;
        po.xs8 = s->xs8;
        po.N = n;
        po.epi = EPI_RESIDUAL;
        po.out = s->hidden;
        po.ld_out = d;
        if ((rc = residual_gemm(s, L.wo, po, n))) return rc;
        stage_mark(s, ST_FFN_NORM);
        if ((rc = launch_rmsnorm_q8(s->hidden, L.ffn_norm, n, d, c.rms_norm_epsilon, s->xq, s->xs, s->xs8, st)))
            return rc;
        stage_mark(s, ST_GATEUP);
        GemmParams pg;
        pg.kernel = s->ctx->gemm_kernel;
        pg.x = s->xq;
        pg.xs = s->xs;
        pg.xs8 = s->xs8;
        pg.N = n;
        pg.epi = EPI_SWIGLU_Q8;
        pg.F = F;
        // In-place would race (readers of row n's block b vs writers); use the upper half.
        pg.xq_out = s->xq + (size_t)s->max_batch * s->maxw;
        pg.xs_out = s->xs + (size_t)s->max_batch * (s->maxw / 32);
        pg.xs8_out = s->xs8 + (size_t)s->max_batch * (s->maxw / 32);
        if (!L.split_gateup && (L.gateup.layout != LAYOUT_R16K || n <= 9)) {
            if ((rc = timed_gemm(s, L.gateup, pg))) return rc;
        } else if (!L.split_gateup) {
            // Q4_K four-tile groups take at most 9 tokens: interleaved rows, then SwiGLU + Q8_0
            if ((rc = timed_gemm(s, L.gateup, plain_rows(s, n, s->ybuf, 2 * F))) ||
                (rc = launch_prompt_swiglu_q8(s->ybuf, n, F, pg.xq_out, pg.xs_out, pg.xs8_out, st, false)))
                return rc;
        } else {
            // gate rows then up rows in ybuf, then SwiGLU and the Q8_0 blocks as one kernel
            if ((rc = timed_gemm(s, L.gate, plain_rows(s, n, s->ybuf, 2 * F))) ||
                (rc = timed_gemm(s, L.up, plain_rows(s, n, s->ybuf + F, 2 * F))) ||
                (rc = launch_prompt_swiglu_q8(s->ybuf, n, F, pg.xq_out, pg.xs_out, pg.xs8_out, st, true)))
                return rc;
        }
        GemmParams pd;
        pd.kernel = s->ctx->gemm_kernel;
        pd.x = pg.xq_out;
        pd.xs = pg.xs_out;
        pd.xs8 = pg.xs8_out;
        pd.N = n;
        pd.epi = EPI_RESIDUAL;
        pd.out = s->hidden;
        pd.ld_out = d;
        stage_mark(s, ST_DOWN);
        if ((rc = residual_gemm(s, L.down, pd, n))) return rc;
    }
    s->last_n = head ? n : 0;
    if (!head) return NC_OK;  // a prompt chunk whose logits nobody reads (prefill_pass_batch)
    // compute_logits_from_hidden (inference.rs:4783-4832) for every row + argmax
    stage_mark(s, ST_HEAD_NORM);
    if ((rc = launch_rmsnorm_q8(s->hidden, m->out_norm, n, d, c.rms_norm_epsilon, s->xq, s->xs, s->xs8, st)))
        return rc;
    stage_mark(s, ST_HEAD);
    GemmParams ph;
    ph.kernel = s->ctx->gemm_kernel;
    ph.x = s->xq;
    ph.xs = s->xs;
    ph.xs8 = s->xs8;
    ph.N = n;
    ph.epi = EPI_HEAD;
    ph.out = s->logits;
    ph.ld_out = (int)c.vocab_size;
    ph.part_val = s->part_val;
    ph.part_idx = s->part_idx;
    if ((rc = timed_gemm(s, m->head, ph))) return rc;
    if ((rc = launch_argmax_final(s->part_val, s->part_idx, n, (int)m->head.tiles, s->d_preds, st))) return rc;
    s->last_n = n;
    return NC_OK;
}

// The attention parameters of a pass that decide its launches (attention_variant).
static AttnParams pass_attention_shape(const nc_session* s, int n, int64_t start_pos) {
    const nc_model_config& c = s->m->cfg;
    AttnParams a;
    a.N = n;
    a.H = (int)c.head_count;
    a.Hkv = (int)c.head_count_kv;
    a.hd = (int)c.head_dim;
    a.max_pos = (int)(start_pos + n - 1);
    a.split = s->ctx->attn_order == NC_ATTN_SPLIT;
    a.nchunks = s->attn_chunks;
    return a;
}

// Every launch of pass_body is fixed by the pass width, whether the head runs, the dot-product
// path and the attention variant: the kernels take the start position and the tokens from
// d_pos / d_toks, which the pass-state kernel writes before each replay.  Layers whose q, k and v
// come from separate matrices take the start position as a kernel argument (the RoPE kernel of
// the prompt path), so their passes always launch directly.
static bool pass_graph_ok(const nc_session* s) {
    if (s->ctx->pass_launch != NC_PASS_GRAPH || s->timing || s->stage_timing) return false;
    for (const LayerDev& L : s->m->layers)
        if (L.split_qkv) return false;
    return true;
}

static uint64_t pass_graph_key(const nc_session* s, int n, int64_t start_pos, bool head) {
    return (uint64_t)n | (uint64_t)head << 5 | (uint64_t)s->ctx->gemm_kernel << 6 |
           (uint64_t)attention_variant(pass_attention_shape(s, n, start_pos)) << 8;
}

// Captured passes kept per session; past this many (contexts crossing many 512-position
// score-grid steps) the cache starts over.
constexpr size_t kMaxPassGraphs = 48;

// pass_body as one HIP graph: captured on the first pass of its key, then replayed.  A graph
// holds kernel nodes only (no memset or copy nodes).
static int pass_body_graph(nc_session* s, int n, int64_t start_pos, bool head) {
    const uint64_t key = pass_graph_key(s, n, start_pos, head);
    auto it = s->graphs.find(key);
    if (it == s->graphs.end()) {
        if (s->graphs.size() >= kMaxPassGraphs) {
            NC_HIP(hipStreamSynchronize(s->stream));
            for (auto& g : s->graphs) NC_HIP(hipGraphExecDestroy(g.second));
            s->graphs.clear();
        }
        hipGraph_t g = nullptr;
        NC_HIP(hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal));
        const int rc = pass_body(s, n, start_pos, head);
        const hipError_t e = hipStreamEndCapture(s->stream, &g);
        if (rc || e != hipSuccess) {
            if (g) (void)hipGraphDestroy(g);
            return rc ? rc : fail(NC_EHIP, std::string("pass capture: ") + hipGetErrorString(e));
        }
        hipGraphExec_t x = nullptr;
        const hipError_t ei = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
        (void)hipGraphDestroy(g);
        if (ei != hipSuccess) return fail(NC_EHIP, std::string("pass graph instantiate: ") + hipGetErrorString(ei));
        it = s->graphs.emplace(key, x).first;
        s->graph_captures++;
    }
    NC_HIP(hipGraphLaunch(it->second, s->stream));
    s->graph_replays++;
    s->last_n = head ? n : 0;
    return NC_OK;
}

// One forward over the n tokens staged by upload_toks (or already in d_toks) at positions
// start_pos..: the pass-state kernel (positions and staged tokens, by kernel arguments), then
// pass_body, launched directly or replayed from its captured graph.
static int run_pass(nc_session* s, int n, int64_t start_pos, bool head = true) {
    if (n < 1 || n > s->max_batch) return fail(NC_ERANGE, "batch exceeds the session's max_batch");
    if (start_pos < 0 || start_pos + n > s->max_ctx) return fail(NC_ERANGE, "batch end exceeds the session context");
    int rc = stage_reserve(s);
    if (rc) return rc;
    struct StageEnd {  // no stage stays open past the pass, whatever path returns
        ~StageEnd() { t_stage_ev0 = t_stage_ev1 = nullptr; }
    } stage_end;
    stage_mark(s, ST_EMBED);
    rc = launch_set_pass_state(s->d_pos, (int32_t)start_pos, s->d_toks, s->pending_toks ? s->staged : nullptr,
                               s->pending_toks ? s->n_staged : 0, s->stream);
    if (rc) return rc;
    s->pending_toks = false;
    if (pass_graph_ok(s)) return pass_body_graph(s, n, start_pos, head);
    return pass_body(s, n, start_pos, head);
}

// Stages the next pass's tokens; run_pass writes them to the device together with the
// start position through kernel arguments.
static int upload_toks(nc_session* s, const uint32_t* toks, int n) {
    if (n < 1 || n > 16) return fail(NC_ERANGE, "batch must be 1..16 tokens");
    // The embedding gather indexes tok_emb[tok * d]: an id past the vocabulary is refused on
    // the host before anything launches (the reference panics on the slice index,
    // inference.rs:3728-3733).
    for (int i = 0; i < n; i++)
        if (toks[i] >= (uint32_t)s->m->cfg.vocab_size)
            return fail(NC_ERANGE, "token id " + std::to_string(toks[i]) + " >= vocab_size " +
                                       std::to_string(s->m->cfg.vocab_size));
    std::memcpy(s->staged, toks, n * sizeof(uint32_t));
    s->n_staged = n;
    s->pending_toks = true;
    return NC_OK;
}

static int fetch_preds(nc_session* s, int n, uint32_t* out) {
    NC_HIP(hipMemcpyAsync(s->h_preds, s->d_preds, n * sizeof(uint32_t), hipMemcpyDeviceToHost, s->stream));
    NC_HIP(hipStreamSynchronize(s->stream));
    std::memcpy(out, s->h_preds, n * sizeof(uint32_t));
    return NC_OK;
}

// rand_simple (inference.rs:4876-4883): the reference's LCG, state advanced before each draw;
// u32::MAX as f32 is 4294967296.0f.
static float lcg_next(uint64_t* state) {
    *state = *state * 6364136223846793005ull + 1ull;
    const uint32_t x = (uint32_t)(*state >> 32);
    return (float)x / (float)UINT32_MAX;
}

// sample_logits (inference.rs:4834-4873) of rows row0 .. row0 + rows - 1 of the session's last
// pass, row r with the uniform u[r] (temp > 0; temp <= 0: first maximum, no uniform).
static int sample_session_rows(nc_session* s, int row0, int rows, float temp, const float* u, uint32_t* out) {
    const int V = (int)s->m->cfg.vocab_size;
    if (rows < 1 || row0 < 0 || row0 + rows > s->max_batch) return fail(NC_EINVAL, "sample_logits: rows outside the pass");
    int rc = launch_sample_logits(s->logits + (size_t)row0 * V, V, rows, V, temp, u, s->probs, V, s->tp_scratch, s->d_samp,
                                  s->stream);
    if (rc) return rc;
    NC_HIP(hipMemcpyAsync(s->h_preds, s->d_samp, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, s->stream));
    NC_HIP(hipStreamSynchronize(s->stream));
    std::memcpy(out, s->h_preds, rows * sizeof(uint32_t));
    return NC_OK;
}

// ---------------------------------------------------------------- prompt passes
// Matrices with an MFMA prompt matmul: Q4_0 (R16 or R64 tiles) and Q4_K (R16K or R64).
static bool prompt_matrix_ok(const QMatDev& q) {
    if (q.type == NC_TYPE_Q4_0) return q.layout == LAYOUT_R16 || q.layout == LAYOUT_R64;
    if (q.type == NC_TYPE_Q4_K) return q.layout == LAYOUT_R16K || q.layout == LAYOUT_R64;
    return false;
}

// Prompt passes take every layer matrix on a prompt kernel, or Q5_K, Q6_K and Q8_0 ones in 16-row slices.
static bool prompt_path_ok(const nc_model* m) {
    for (const LayerDev& L : m->layers)
        for (const QMatDev* q : L.all())
            if (q->dev && !prompt_matrix_ok(*q) && q->type != NC_TYPE_Q6_K && q->type != NC_TYPE_Q8_0 &&
                q->type != NC_TYPE_Q5_K)
                return false;
    return true;
}

// Prompt matmul of n tokens (Q4_0 or Q4_K) over activations repacked into xm / xsm (/ xam).
static int prompt_matmul(const QMatDev& w, const int8_t* xq, const float* xs, float* out, int ld_out, int n,
                         hipStream_t st, int8_t* xm, float* xsm, float* xam) {
    const bool k = w.type == NC_TYPE_Q4_K;
    int rc = launch_prompt_repack(xq, xs, n, (int)w.cols, xm, xsm, st, k ? xam : nullptr);
    if (rc) return rc;
    return k ? launch_gemm_prompt_q4k(w, out, ld_out, n, st, xm, xsm, xam)
             : launch_gemm_prompt(w, xq, xs, out, ld_out, n, st, xm, xsm);
}

static int ensure_prompt_bufs(nc_session* s) {
    if (s->prompt_ready) return NC_OK;
    const nc_model_config& c = s->m->cfg;
    const size_t R = kPromptRows;
    const size_t yw = std::max({c.attention_output_width + 2 * c.kv_width, 2 * c.feed_forward_length,
                                c.embedding_length});
    int rc;
    if ((rc = dev_alloc(s->allocs, &s->p_hidden, R * c.embedding_length)) ||
        (rc = dev_alloc(s->allocs, &s->p_xq, R * s->maxw)) || (rc = dev_alloc(s->allocs, &s->p_xs, R * (s->maxw / 32))) ||
        (rc = dev_alloc(s->allocs, &s->p_xs8, R * (s->maxw / 32))) || (rc = dev_alloc(s->allocs, &s->p_y, R * yw)) ||
        (rc = dev_alloc(s->allocs, &s->p_q, R * c.attention_output_width)) ||
        (rc = dev_alloc(s->allocs, &s->p_scores, (size_t)kPromptGroup * c.head_count * s->ctx_stride)) ||
        (rc = dev_alloc(s->allocs, &s->p_toks, (size_t)s->max_ctx)) ||
        (rc = dev_alloc(s->allocs, &s->p_pos, R / kPromptGroup)) || (rc = dev_alloc(s->allocs, &s->p_xm, R * s->maxw)) ||
        (rc = dev_alloc(s->allocs, &s->p_xsm, R * ((s->maxw + 127) / 128) * 4)) ||
        (rc = dev_alloc(s->allocs, &s->p_xam, R * ((s->maxw + 127) / 128) * 4)))
        return rc;
    s->prompt_ready = true;
    return NC_OK;
}

// Prompt matmul of the pass's activations (repacked first into MFMA operand order).
// A prompt pass's matmul into rows of stride ld (default: the matrix's rows): the MFMA prompt
// kernels, or for Q5_K, Q6_K and Q8_0 matrices (no prompt kernel) the verify kernel on 16-row slices.
static int prompt_gemm(nc_session* s, const QMatDev& w, const int8_t* xq, const float* xs, float* out, int n,
                       int ld = 0) {
    if (ld == 0) ld = (int)w.rows;
    if (prompt_matrix_ok(w)) return prompt_matmul(w, xq, xs, out, ld, n, s->stream, s->p_xm, s->p_xsm, s->p_xam);
    for (int i = 0; i < n; i += 16) {
        GemmParams p;
        p.x = xq + (size_t)i * w.cols;
        p.xs = xs + (size_t)i * (w.cols / 32);
        p.xs8 = s->p_xs8 + (size_t)i * (w.cols / 32);
        p.N = std::min(16, n - i);
        p.epi = EPI_STORE;
        p.out = out + (size_t)i * ld;
        p.ld_out = ld;
        if (const int rc = launch_gemm(w, p, s->stream)) return rc;
    }
    return NC_OK;
}

// q, k, v rows of a prompt pass side by side in p_y ([n][aw + 2 kw]), fused or split.
static int prompt_qkv(nc_session* s, const LayerDev& L, int n, int aw, int kw) {
    if (!L.split_qkv) return prompt_gemm(s, L.qkv, s->p_xq, s->p_xs, s->p_y, n);
    const int ld = aw + 2 * kw;
    int rc;
    if ((rc = prompt_gemm(s, L.q, s->p_xq, s->p_xs, s->p_y, n, ld)) ||
        (rc = prompt_gemm(s, L.k, s->p_xq, s->p_xs, s->p_y + aw, n, ld)) ||
        (rc = prompt_gemm(s, L.v, s->p_xq, s->p_xs, s->p_y + aw + kw, n, ld)))
        return rc;
    return NC_OK;
}

// gate and up rows of a prompt pass in p_y: interleaved when fused, gate then up when split.
static int prompt_gateup(nc_session* s, const LayerDev& L, int n, int F) {
    if (!L.split_gateup) return prompt_gemm(s, L.gateup, s->p_xq, s->p_xs, s->p_y, n);
    int rc;
    if ((rc = prompt_gemm(s, L.gate, s->p_xq, s->p_xs, s->p_y, n, 2 * F)) ||
        (rc = prompt_gemm(s, L.up, s->p_xq, s->p_xs, s->p_y + F, n, 2 * F)))
        return rc;
    return NC_OK;
}

// One prompt pass over n <= kPromptRows ids p_toks[off..off+n) at positions start..: the
// layers of run_pass (run_layer_range_batch, inference.rs:3747-4111) with the MFMA prompt
// matmul and the epilogues as separate kernels; no head (prefill_pass_batch discards the
// prompt's logits).  Attention runs in row groups of kPromptGroup (the score rows).
static int run_prompt_pass(nc_session* s, int off, int n, int64_t start) {
    nc_model* m = s->m;
    const nc_model_config& c = m->cfg;
    const int d = (int)c.embedding_length, aw = (int)c.attention_output_width, kw = (int)c.kv_width;
    const int F = (int)c.feed_forward_length, hd = (int)c.head_dim, Hkv = (int)c.head_count_kv;
    hipStream_t st = s->stream;
    const int ngroups = (n + kPromptGroup - 1) / kPromptGroup;
    int rc;
    if ((rc = launch_embed(m->tok_emb, s->p_toks + off, n, d, s->p_hidden, st)) ||
        (rc = launch_prompt_positions(s->p_pos, (int)start, kPromptGroup, ngroups, st)))
        return rc;
    const size_t layer_kv = (size_t)Hkv * s->ctx_stride * hd;
    for (int64_t li = 0; li < c.block_count; li++) {
        const LayerDev& L = m->layers[li];
        float* kc = s->kcache + li * layer_kv;
        float* vc = s->vcache + li * layer_kv;
        if ((rc = launch_rmsnorm_q8(s->p_hidden, L.attn_norm, n, d, c.rms_norm_epsilon, s->p_xq, s->p_xs, s->p_xs8, st)) ||
            (rc = prompt_qkv(s, L, n, aw, kw)) ||
            (rc = launch_prompt_qkv_rope(s->p_y, n, (int)start, aw, kw, hd, (int)c.rope_dimension_count / 2,
                                         s->rope_tab, s->p_q, kc, vc, (int)s->ctx_stride, st)))
            return rc;
        for (int gi = 0; gi < ngroups; gi++) {
            const int g0 = gi * kPromptGroup, ng = std::min(kPromptGroup, n - g0);
            AttnParams a;
            a.q = s->p_q + (size_t)g0 * aw;
            a.kcache = kc;
            a.vcache = vc;
            a.scores = s->p_scores;
            a.xq = s->p_xq + (size_t)g0 * aw;
            a.xs = s->p_xs + (size_t)g0 * (aw / 32);
            a.xs8 = s->p_xs8 + (size_t)g0 * (aw / 32);
            a.d_pos = s->p_pos + gi;
            a.N = ng;
            a.H = (int)c.head_count;
            a.Hkv = Hkv;
            a.hd = hd;
            a.max_ctx = (int)s->ctx_stride;
            a.max_pos = (int)(start + g0 + ng - 1);
            a.scale = 1.0f / std::sqrt((float)hd);  // inference.rs:3927
            if ((rc = launch_attention(a, st))) return rc;
        }
        if ((rc = prompt_gemm(s, L.wo, s->p_xq, s->p_xs, s->p_y, n)) ||
            (rc = launch_prompt_residual(s->p_y, s->p_hidden, n, d, st)) ||
            (rc = launch_rmsnorm_q8(s->p_hidden, L.ffn_norm, n, d, c.rms_norm_epsilon, s->p_xq, s->p_xs, s->p_xs8, st)) ||
            (rc = prompt_gateup(s, L, n, F)) ||
            // the gate/up matmul has read every activation before the SwiGLU kernel overwrites them
            (rc = launch_prompt_swiglu_q8(s->p_y, n, F, s->p_xq, s->p_xs, s->p_xs8, st, L.split_gateup)) ||
            (rc = prompt_gemm(s, L.down, s->p_xq, s->p_xs, s->p_y, n)) ||
            (rc = launch_prompt_residual(s->p_y, s->p_hidden, n, d, st)))
            return rc;
    }
    s->last_n = 0;
    return NC_OK;
}

// prefill_tokens (main.rs:9415-9485): chunks of max_batch rows.  Returns the last row's
// greedy prediction in *last_pred.  Q4_0 models run all but the last max_batch tokens (all of
// them when no logits are wanted) as prompt passes of up to kPromptRows tokens; every token's
// arithmetic is the same in any chunking, so the KV cache and logits are the same bits.
static int prefill_chunks(nc_session* s, const uint32_t* toks, int n, int64_t start_pos, uint32_t* last_pred,
                          bool last_logits = false) {
    // per-kernel timing covers decode and verify passes only, never the prompt
    struct TimingOff {
        nc_session* s;
        bool was, was_stage;
        ~TimingOff() {
            s->timing = was;
            s->stage_timing = was_stage;
        }
    } guard{s, s->timing, s->stage_timing};
    s->timing = false;
    s->stage_timing = false;
    int rc;
    for (int i = 0; i < n; i++)  // every id is checked before the first chunk runs
        if (toks[i] >= (uint32_t)s->m->cfg.vocab_size)
            return fail(NC_ERANGE, "prompt token id " + std::to_string(toks[i]) + " >= vocab_size");
    if (start_pos < 0 || start_pos + n > s->max_ctx) return fail(NC_ERANGE, "prompt exceeds the session context");
    const bool head = last_pred || last_logits;
    int i = 0;
    const int tail = head ? std::min(n, s->max_batch) : 0;  // rows whose pass computes the head
    if (n - tail >= kPromptMin && prompt_path_ok(s->m)) {
        if ((rc = ensure_prompt_bufs(s))) return rc;
        // synchronous: an earlier prompt pass on the session stream may still read p_toks
        NC_HIP(hipStreamSynchronize(s->stream));
        NC_HIP(hipMemcpy(s->p_toks, toks, (size_t)(n - tail) * sizeof(uint32_t), hipMemcpyHostToDevice));
        for (; i < n - tail; i += kPromptRows) {
            const int len = std::min(kPromptRows, n - tail - i);
            if ((rc = run_prompt_pass(s, i, len, start_pos + i))) return rc;
        }
        i = n - tail;  // the verify-sized passes take the rest
    }
    for (; i < n; i += s->max_batch) {
        const int len = std::min(s->max_batch, n - i);
        if ((rc = upload_toks(s, toks + i, len))) return rc;
        if ((rc = run_pass(s, len, start_pos + i, head && i + len == n))) return rc;
    }
    if (last_pred) {
        uint32_t preds[16];
        if ((rc = fetch_preds(s, s->last_n, preds))) return rc;
        *last_pred = preds[s->last_n - 1];
    }
    return NC_OK;
}

static int verify_step(nc_session* s, int n, int64_t start_pos, nc_verify_result* r) {
    int rc = run_pass(s, n, start_pos);
    if (rc) return rc;
    if ((rc = launch_accept_greedy(s->d_toks, s->d_preds, n, s->d_pos, s->d_result, nullptr, s->stream))) return rc;
    NC_HIP(hipMemcpyAsync(s->h_result, s->d_result, 4 * sizeof(int32_t), hipMemcpyDeviceToHost, s->stream));
    NC_HIP(hipStreamSynchronize(s->stream));
    r->n_accepted = s->h_result[0];
    r->next_token = (uint32_t)s->h_result[1];
    r->new_pos = s->h_result[2];
    return NC_OK;
}

// Stochastic k+1 acceptance of the pass just run (rows 0..n-1 at start_pos): temperature
// probabilities of every row, then the accept/resample kernel.  q: [n-1][V] draft probs.
static int accept_stochastic_step(nc_session* s, int n, int64_t start_pos, const float* q, float temp, uint64_t seed) {
    const int V = (int)s->m->cfg.vocab_size;
    int rc = launch_temperature_probs(s->logits, V, s->probs, V, n, V, temp, s->tp_scratch, s->stream);
    if (rc) return rc;
    return launch_accept_stochastic(s->probs, q, V, s->d_toks + 1, n - 1, V, seed, start_pos, s->d_result, s->d_pos,
                                    s->tp_scratch, s->stream);
}

static int fetch_result(nc_session* s, int n_toks, nc_verify_result* r, uint32_t* toks_out) {
    NC_HIP(hipMemcpyAsync(s->h_result, s->d_result, 4 * sizeof(int32_t), hipMemcpyDeviceToHost, s->stream));
    if (toks_out)
        NC_HIP(hipMemcpyAsync(s->h_toks, s->d_toks, n_toks * sizeof(uint32_t), hipMemcpyDeviceToHost, s->stream));
    NC_HIP(hipStreamSynchronize(s->stream));
    r->n_accepted = s->h_result[0];
    r->next_token = (uint32_t)s->h_result[1];
    r->new_pos = s->h_result[2];
    if (toks_out) std::memcpy(toks_out, s->h_toks, n_toks * sizeof(uint32_t));
    return NC_OK;
}

static double now_s() {
    return std::chrono::duration<double>(std::chrono::steady_clock::now().time_since_epoch()).count();
}

}  // namespace nc

using namespace nc;

// ================================================================ C ABI
extern "C" {

const char* nc_last_error(void) { return t_err.c_str(); }
const char* nc_version(void) { return "nanocamelid-mi355x 0.1 (gfx950)"; }

int nc_ctx_create(int device, nc_ctx** out) {
    if (!out) return fail(NC_EINVAL, "out is null");
    NC_HIP(hipSetDevice(device));
    auto* c = new nc_ctx();
    c->device = device;
    // device address of the allocation-free entry point's static scratch array (noalloc.hip)
    int rc0 = static_scratch_address(&c->static_scratch);
    if (rc0) {
        delete c;
        return rc0;
    }
    hipError_t e = hipStreamCreate(&c->stream);
    if (e == hipSuccess) {
        c->xsum_cap = 16 * kCtxScratchCols / 32;
        e = hipMalloc((void**)&c->xsum, c->xsum_cap * sizeof(int32_t));
    }
    if (e == hipSuccess) {
        c->tp_cap = temperature_scratch_floats(16);
        e = hipMalloc((void**)&c->tp_scratch, c->tp_cap * sizeof(float));
    }
    if (e == hipSuccess) e = hipMalloc((void**)&c->pxm, kPromptRows * kCtxScratchCols);
    if (e == hipSuccess) e = hipMalloc((void**)&c->pxsm, kPromptRows * (kCtxScratchCols / 128 + 1) * 4 * sizeof(float));
    if (e == hipSuccess) e = hipMalloc((void**)&c->pxam, kPromptRows * (kCtxScratchCols / 128 + 1) * 4 * sizeof(float));
    if (e != hipSuccess) {
        nc_ctx_free(c);
        return fail(NC_EHIP, std::string("nc_ctx_create: ") + hipGetErrorString(e));
    }
    *out = c;
    return NC_OK;
}

void nc_ctx_free(nc_ctx* c) {
    if (!c) return;
    (void)hipSetDevice(c->device);
    if (c->xsum) (void)hipFree(c->xsum);
    if (c->tp_scratch) (void)hipFree(c->tp_scratch);
    if (c->pxm) (void)hipFree(c->pxm);
    if (c->pxsm) (void)hipFree(c->pxsm);
    if (c->pxam) (void)hipFree(c->pxam);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
}

int nc_ctx_set_attention(nc_ctx* c, int order) {
    if (!c || (order != NC_ATTN_SEQUENTIAL && order != NC_ATTN_SPLIT))
        return fail(NC_EINVAL, "nc_ctx_set_attention: unknown summation order");
    c->attn_order = order;
    return NC_OK;
}

int nc_ctx_set_pass_launch(nc_ctx* c, int mode) {
    if (!c || (mode != NC_PASS_GRAPH && mode != NC_PASS_DIRECT))
        return fail(NC_EINVAL, "nc_ctx_set_pass_launch: unknown launch mode");
    c->pass_launch = mode;
    return NC_OK;
}

int nc_ctx_set_gemm_kernel(nc_ctx* c, int kernel) {
    if (!c || kernel < NC_GEMM_KERNEL_AUTO || kernel > NC_GEMM_KERNEL_MFMA)
        return fail(NC_EINVAL, "nc_ctx_set_gemm_kernel: unknown kernel");
    c->gemm_kernel = kernel;
    return NC_OK;
}

int nc_ctx_synchronize(nc_ctx* c) {
    if (!c) return fail(NC_EINVAL, "ctx is null");
    NC_HIP(hipSetDevice(c->device));
    NC_HIP(hipStreamSynchronize(c->stream));
    return NC_OK;
}

int nc_qmat_upload(nc_ctx* ctx, int type, int64_t rows, int64_t cols, const void* blocks, nc_qmat** out) {
    if (!ctx || !blocks || !out || rows <= 0 || cols <= 0) return fail(NC_EINVAL, "nc_qmat_upload: bad arguments");
    if (type != NC_TYPE_Q4_0 && type != NC_TYPE_Q4_K && type != NC_TYPE_Q5_K && type != NC_TYPE_Q8_0 &&
        type != NC_TYPE_Q6_K)
        return fail(NC_EINVAL, "nc_qmat_upload: type must be Q4_0, Q4_K, Q5_K, Q8_0 or Q6_K");
    NC_HIP(hipSetDevice(ctx->device));
    auto* q = new nc_qmat();
    q->ctx = ctx;
    int rc = upload_matrix(type, rows, cols, {{(const uint8_t*)blocks, rows, 0, -1}}, q->m);
    if (rc) {
        if (q->m.dev) (void)hipFree(q->m.dev);
        delete q;
        return rc;
    }
    *out = q;
    return NC_OK;
}

void nc_qmat_free(nc_qmat* q) {
    if (!q) return;
    if (q->m.dev) (void)hipFree(q->m.dev);
    delete q;
}

int64_t nc_qmat_device_bytes(const nc_qmat* q) { return q ? q->m.dev_bytes : -1; }

static int ensure_xsum(nc_ctx* ctx, size_t count) {
    if (ctx->xsum_cap >= count) return NC_OK;
    if (ctx->xsum) NC_HIP(hipFree(ctx->xsum));
    ctx->xsum = nullptr;
    ctx->xsum_cap = 0;
    NC_HIP(hipMalloc((void**)&ctx->xsum, count * sizeof(int32_t)));
    ctx->xsum_cap = count;
    return NC_OK;
}

// Tokens per slice of the operator-level prompt matmul: the context's repack buffers hold
// kPromptRows tokens of kCtxScratchCols columns (0: columns too wide for a 16-token slice).
static int prompt_slice_tokens(int64_t cols) {
    return (int)std::min<int64_t>(kPromptRows, (int64_t)kPromptRows * (int64_t)kCtxScratchCols / cols / 16 * 16);
}

// The prompt matmul (Q4_0 or Q4_K) of batch_size > 16 tokens through the context's repack
// buffers, in slices of prompt_slice_tokens (every token's outputs are the same bits in any
// slicing).
static int ctx_prompt_matmul(nc_ctx* ctx, const QMatDev& w, const int8_t* x, const float* xs, float* out, int n,
                             hipStream_t st) {
    const int cols = (int)w.cols, T = prompt_slice_tokens(cols);
    for (int i = 0; i < n; i += T) {
        const int len = std::min(T, n - i);
        int rc = prompt_matmul(w, x + (size_t)i * cols, xs + (size_t)i * (cols / 32), out + (size_t)i * w.rows,
                               (int)w.rows, len, st, ctx->pxm, ctx->pxsm, ctx->pxam);
        if (rc) return rc;
    }
    return NC_OK;
}

int nc_matmul_quantized_batch(nc_ctx* ctx, const nc_qmat* w, const int8_t* x_i8, const float* x_scales, float* out,
                              int batch_size, int64_t rows, int64_t cols, void* stream) {
    if (!ctx || !w || !x_i8 || !x_scales || !out) return fail(NC_EINVAL, "nc_matmul_quantized_batch: null argument");
    if (rows != w->m.rows || cols != w->m.cols) return fail(NC_EINVAL, "nc_matmul_quantized_batch: shape mismatch");
    if (batch_size < 1) return fail(NC_EINVAL, "nc_matmul_quantized_batch: batch must be >= 1");
    NC_HIP(hipSetDevice(ctx->device));
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    // more than 16 tokens: the MFMA prompt matmul (Q4_0), or 16-token slices (Q4_K)
    if (batch_size > 16 && prompt_matrix_ok(w->m) && prompt_slice_tokens(cols) >= 16)
        return ctx_prompt_matmul(ctx, w->m, x_i8, x_scales, out, batch_size, st);
    for (int i = 0; i < batch_size; i += 16) {
        const int nb = std::min(16, batch_size - i);
        int rc = ensure_xsum(ctx, (size_t)nb * (cols / 32));
        if (rc) return rc;
        if ((rc = launch_block_sums(x_i8 + (size_t)i * cols, nb, (int)cols, ctx->xsum, st))) return rc;
        GemmParams p;
        p.kernel = ctx->gemm_kernel;
        p.x = x_i8 + (size_t)i * cols;
        p.xs = x_scales + (size_t)i * (cols / 32);
        p.xs8 = ctx->xsum;
        p.N = nb;
        p.epi = EPI_STORE;
        p.out = out + (size_t)i * rows;
        p.ld_out = (int)rows;
        if ((rc = launch_gemm(w->m, p, st))) return rc;
    }
    return NC_OK;
}

int nc_bench_matmul(nc_ctx* ctx, const nc_qmat* const* w, int32_t ncopies, const int8_t* x_i8, const float* x_scales,
                    float* out, int32_t batch_size, int32_t iters, float* us_out) {
    if (!ctx || !w || ncopies < 1 || !x_i8 || !x_scales || !out || !us_out || iters < 1)
        return fail(NC_EINVAL, "nc_bench_matmul: bad arguments");
    if (batch_size < 1) return fail(NC_EINVAL, "nc_bench_matmul: batch must be >= 1");
    for (int i = 0; i < ncopies; i++)
        if (!w[i] || w[i]->m.rows != w[0]->m.rows || w[i]->m.cols != w[0]->m.cols)
            return fail(NC_EINVAL, "nc_bench_matmul: weight copies differ in shape");
    if (batch_size > 16 && (!prompt_matrix_ok(w[0]->m) || prompt_slice_tokens(w[0]->m.cols) < 16))
        return fail(NC_EINVAL, "nc_bench_matmul: more than 16 tokens only for Q4_0 / Q4_K matrices of <= 1M columns");
    NC_HIP(hipSetDevice(ctx->device));
    hipStream_t st = ctx->stream;
    const int64_t cols = w[0]->m.cols, rows = w[0]->m.rows;
    int rc = NC_OK;
    if (batch_size <= 16) {
        rc = ensure_xsum(ctx, (size_t)batch_size * (cols / 32));
        if (rc || (rc = launch_block_sums(x_i8, batch_size, (int)cols, ctx->xsum, st))) return rc;
    }
    GemmParams p;
    p.kernel = ctx->gemm_kernel;
    p.x = x_i8;
    p.xs = x_scales;
    p.xs8 = ctx->xsum;
    p.N = batch_size;
    p.epi = EPI_STORE;
    p.out = out;
    p.ld_out = (int)rows;
    std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
    for (auto& e : ev) NC_HIP(hipEventCreate(&e));
    for (int i = 0; i < iters && !rc; i++) {
        if (batch_size <= 16) {
            rc = launch_gemm(w[i % ncopies]->m, p, st, ev[2 * i], ev[2 * i + 1]);
        } else if (hipEventRecord(ev[2 * i], st) != hipSuccess ||
                   (rc = ctx_prompt_matmul(ctx, w[i % ncopies]->m, x_i8, x_scales, out, batch_size, st)) ||
                   hipEventRecord(ev[2 * i + 1], st) != hipSuccess) {
            if (!rc) rc = fail(NC_EHIP, "nc_bench_matmul: event record");
        }
    }
    if (!rc && hipStreamSynchronize(st) != hipSuccess) rc = fail(NC_EHIP, "nc_bench_matmul: stream failed");
    for (int i = 0; i < iters && !rc; i++) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) != hipSuccess) rc = fail(NC_EHIP, "nc_bench_matmul: event");
        us_out[i] = ms * 1000.0f;
    }
    for (auto& e : ev) (void)hipEventDestroy(e);
    return rc;
}

int nc_matmul_blockdots(nc_ctx* ctx, const nc_qmat* w, const int8_t* x_i8, int32_t* dots, int batch_size, int64_t rows,
                        int64_t cols, void* stream) {
    if (!ctx || !w || !x_i8 || !dots) return fail(NC_EINVAL, "nc_matmul_blockdots: null argument");
    if (rows != w->m.rows || cols != w->m.cols) return fail(NC_EINVAL, "nc_matmul_blockdots: shape mismatch");
    NC_HIP(hipSetDevice(ctx->device));
    return launch_blockdots(w->m, x_i8, dots, batch_size, stream ? (hipStream_t)stream : ctx->stream);
}

int nc_debug_expf(nc_ctx* ctx, uint32_t first_bits, int64_t count, float* out, void* stream) {
    if (!ctx || (!out && count > 0)) return fail(NC_EINVAL, "nc_debug_expf: null argument");
    NC_HIP(hipSetDevice(ctx->device));
    return launch_expf_range(first_bits, count, out, stream ? (hipStream_t)stream : ctx->stream);
}

int nc_debug_pass_graphs(nc_session* s, int64_t* captures, int64_t* replays) {
    if (!s || !captures || !replays) return fail(NC_EINVAL, "nc_debug_pass_graphs: null argument");
    *captures = s->graph_captures;
    *replays = s->graph_replays;
    return NC_OK;
}

int nc_debug_temperature_paths(nc_ctx* ctx, int32_t rows, int32_t* fast, void* stream) {
    if (!ctx || !fast || rows < 1 || temperature_scratch_floats(rows) > ctx->tp_cap)
        return fail(NC_EINVAL, "nc_debug_temperature_paths: bad arguments");
    NC_HIP(hipSetDevice(ctx->device));
    return temperature_row_paths(ctx->tp_scratch, rows, fast, stream ? (hipStream_t)stream : ctx->stream);
}

int nc_quantize_q8_0_batch(nc_ctx* ctx, const float* x, int8_t* x_i8, float* x_scales, int batch_size, int64_t dim,
                           void* stream) {
    if (!ctx || !x || !x_i8 || !x_scales || dim % 32) return fail(NC_EINVAL, "nc_quantize_q8_0_batch: bad arguments");
    NC_HIP(hipSetDevice(ctx->device));
    int rc = ensure_xsum(ctx, (size_t)batch_size * (dim / 32));
    if (rc) return rc;
    return launch_quantize_q8(x, batch_size, (int)dim, x_i8, x_scales, ctx->xsum, stream ? (hipStream_t)stream : ctx->stream);
}

int nc_rms_norm_q8_0_batch(nc_ctx* ctx, const float* x, const float* w, float eps, int8_t* x_i8, float* x_scales,
                           int batch_size, int64_t dim, void* stream) {
    if (!ctx || !x || !w || !x_i8 || !x_scales || batch_size < 1 || dim < 256)
        return fail(NC_EINVAL, "nc_rms_norm_q8_0_batch: bad arguments");
    NC_HIP(hipSetDevice(ctx->device));
    int rc = ensure_xsum(ctx, (size_t)batch_size * (dim / 32));
    if (rc) return rc;
    return launch_rmsnorm_q8(x, w, batch_size, (int)dim, eps, x_i8, x_scales, ctx->xsum,
                             stream ? (hipStream_t)stream : ctx->stream);
}

int nc_temperature_probs_batch(nc_ctx* ctx, const float* logits, float* probs, int32_t rows, int64_t vocab, float temp,
                               void* stream) {
    if (!ctx || !logits || !probs || rows < 1 || vocab < 1 || vocab > INT32_MAX || !(temp > 0.0f))
        return fail(NC_EINVAL, "nc_temperature_probs_batch: bad arguments");
    NC_HIP(hipSetDevice(ctx->device));
    const size_t need = temperature_scratch_floats(rows);
    if (ctx->tp_cap < need) {
        if (ctx->tp_scratch) NC_HIP(hipFree(ctx->tp_scratch));
        ctx->tp_scratch = nullptr;
        ctx->tp_cap = 0;
        NC_HIP(hipMalloc((void**)&ctx->tp_scratch, need * sizeof(float)));
        ctx->tp_cap = need;
    }
    return launch_temperature_probs(logits, vocab, probs, vocab, rows, (int)vocab, temp, ctx->tp_scratch,
                                    stream ? (hipStream_t)stream : ctx->stream);
}

int nc_stochastic_accept(nc_ctx* ctx, const float* p_probs, const float* q_probs, const uint32_t* drafts, int32_t k,
                         int64_t vocab, uint64_t seed, int64_t start_pos, int32_t* result, void* stream) {
    if (!ctx || !p_probs || !result || k < 0 || k > 15 || (k > 0 && (!q_probs || !drafts)) || vocab < 1 ||
        vocab > INT32_MAX || start_pos < 0)
        return fail(NC_EINVAL, "nc_stochastic_accept: bad arguments");
    NC_HIP(hipSetDevice(ctx->device));
    return launch_accept_stochastic(p_probs, q_probs, vocab, drafts, k, (int)vocab, seed, start_pos, result, nullptr,
                                    ctx->tp_scratch, stream ? (hipStream_t)stream : ctx->stream);
}

int nc_model_load_gguf_memory(nc_ctx* ctx, const void* data, size_t size, const nc_load_opts* opts, nc_model** out) {
    if (!ctx || !data || !out) return fail(NC_EINVAL, "nc_model_load_gguf_memory: null argument");
    NC_HIP(hipSetDevice(ctx->device));
    return load_model(ctx, (const uint8_t*)data, size, opts, out);
}

// LlamaWeights::load maps the file (model.rs:461-467); so does this: the header is parsed from
// the mapping and each matrix is repacked from it into a staging buffer of that matrix alone,
// so no copy of the whole file is ever made in host memory.
int nc_model_load_gguf(nc_ctx* ctx, const char* path, const nc_load_opts* opts, nc_model** out) {
    if (!ctx || !path || !out) return fail(NC_EINVAL, "nc_model_load_gguf: null argument");
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return fail(NC_EINVAL, std::string("cannot open ") + path + ": " + std::strerror(errno));
    struct stat st;
    if (::fstat(fd, &st) != 0 || st.st_size <= 0) {
        ::close(fd);
        return fail(NC_EFORMAT, std::string("cannot stat ") + path);
    }
    const size_t size = (size_t)st.st_size;
    void* map = ::mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (map == MAP_FAILED) return fail(NC_EFORMAT, std::string("cannot map ") + path + ": " + std::strerror(errno));
    (void)::madvise(map, size, MADV_WILLNEED);
    const int rc = nc_model_load_gguf_memory(ctx, map, size, opts, out);
    ::munmap(map, size);
    return rc;
}

int nc_gguf_read_config(const void* data, size_t size, nc_model_config* out) {
    if (!data || !out) return fail(NC_EINVAL, "nc_gguf_read_config: null argument");
    GgufFile g;
    std::string err;
    if (!gguf_parse((const uint8_t*)data, size, g, err)) return fail(NC_EFORMAT, err);
    nc_model_config c;
    int rc = read_config(g, c);
    if (rc) return rc;
    *out = c;
    return NC_OK;
}

int nc_gguf_stop_tokens(const void* data, size_t size, uint32_t* out, int32_t max, int32_t* n) {
    if (!data || !n || max < 0 || (max > 0 && !out)) return fail(NC_EINVAL, "nc_gguf_stop_tokens: bad arguments");
    GgufFile g;
    std::string err;
    if (!gguf_parse((const uint8_t*)data, size, g, err)) return fail(NC_EFORMAT, err);
    std::vector<uint32_t> ids;
    if (!gguf_stop_tokens(g, ids, err)) return fail(NC_EFORMAT, err);
    *n = (int32_t)ids.size();
    if ((int64_t)ids.size() > max) return fail(NC_ERANGE, "nc_gguf_stop_tokens: more ids than max");
    std::copy(ids.begin(), ids.end(), out);
    return NC_OK;
}

int64_t nc_gguf_tensor_count(const void* data, size_t size) {
    if (!data) return fail(NC_EINVAL, "nc_gguf_tensor_count: null argument");
    GgufFile g;
    std::string err;
    if (!gguf_parse((const uint8_t*)data, size, g, err)) return fail(NC_EFORMAT, err);
    return (int64_t)g.tensors.size();
}

int nc_gguf_tensor_info(const void* data, size_t size, int64_t index, char* name, int64_t name_cap, int32_t* n_dims,
                        uint64_t* dims, int32_t* type, uint64_t* offset, uint64_t* nbytes) {
    if (!data || !name || name_cap < 1 || !n_dims || !dims || !type || !offset || !nbytes)
        return fail(NC_EINVAL, "nc_gguf_tensor_info: null argument");
    GgufFile g;
    std::string err;
    if (!gguf_parse((const uint8_t*)data, size, g, err)) return fail(NC_EFORMAT, err);
    if (index < 0 || index >= (int64_t)g.tensors.size()) return fail(NC_ERANGE, "nc_gguf_tensor_info: index out of range");
    const GgufTensor& t = g.tensors[(size_t)index];
    const size_t n = std::min((size_t)name_cap - 1, t.name.size());
    std::memcpy(name, t.name.data(), n);
    name[n] = 0;
    *n_dims = (int32_t)t.dims.size();
    for (size_t i = 0; i < 4; i++) dims[i] = i < t.dims.size() ? t.dims[i] : 1;
    *type = (int32_t)t.type;
    *offset = t.offset;
    *nbytes = t.nbytes;
    return NC_OK;
}

int nc_model_get_config(const nc_model* m, nc_model_config* out) {
    if (!m || !out) return fail(NC_EINVAL, "null argument");
    *out = m->cfg;
    return NC_OK;
}

void nc_model_free(nc_model* m) { free_model(m); }

void nc_session_free(nc_session* s) {
    if (!s) return;
    (void)hipSetDevice(s->ctx->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    for (auto& e : s->ev) {
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
    }
    for (auto& e : s->stage_ev) {
        (void)hipEventDestroy(e.first);
        (void)hipEventDestroy(e.second);
    }
    for (auto& g : s->graphs) (void)hipGraphExecDestroy(g.second);
    for (void* p : s->allocs) (void)hipFree(p);
    for (void* p : {(void*)s->h_toks, (void*)s->h_preds, (void*)s->h_result, (void*)s->h_pos})
        if (p) (void)hipHostFree(p);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
}

int nc_session_create(nc_model* m, int64_t max_ctx, int32_t max_batch, nc_session** out) {
    if (!m || !out) return fail(NC_EINVAL, "null argument");
    if (max_batch < 1 || max_batch > 16) return fail(NC_EINVAL, "max_batch must be 1..16");
    if (max_ctx < 1 || max_ctx > m->cfg.context_length)
        return fail(NC_ERANGE, "max_ctx must be in 1..context_length");
    if (max_ctx > NC_MAX_CONTEXT)
        return fail(NC_ERANGE, "max_ctx exceeds the attention kernels' " + std::to_string(NC_MAX_CONTEXT) +
                                   "-position score rows");
    NC_HIP(hipSetDevice(m->ctx->device));
    std::unique_ptr<nc_session, void (*)(nc_session*)> s(new nc_session(), nc_session_free);
    s->m = m;
    s->ctx = m->ctx;
    s->max_ctx = max_ctx;
    s->ctx_stride = (max_ctx + 3) / 4 * 4;
    s->attn_chunks = (int)((max_ctx + 63) / 64);  // 64-position chunks of the split-order attention
    s->max_batch = max_batch;
    NC_HIP(hipStreamCreate(&s->stream));
    const nc_model_config& c = m->cfg;
    const int64_t B = max_batch;
    s->maxw = std::max({c.embedding_length, c.feed_forward_length, c.attention_output_width});
    const size_t kv = (size_t)c.block_count * c.head_count_kv * s->ctx_stride * c.head_dim;
    int rc;
    if ((rc = dev_alloc(s->allocs, &s->kcache, kv)) || (rc = dev_alloc(s->allocs, &s->vcache, kv)) ||
        (rc = dev_alloc(s->allocs, &s->hidden, B * c.embedding_length)) ||
        (rc = dev_alloc(s->allocs, &s->xq, 2 * B * s->maxw)) ||
        (rc = dev_alloc(s->allocs, &s->xs, 2 * B * (s->maxw / 32))) ||
        (rc = dev_alloc(s->allocs, &s->xs8, 2 * B * (s->maxw / 32))) ||
        (rc = dev_alloc(s->allocs, &s->q, B * c.attention_output_width)) ||
        (rc = dev_alloc(s->allocs, &s->scores, (size_t)B * c.head_count * s->ctx_stride)) ||
        (rc = dev_alloc(s->allocs, &s->attn_part_o, (size_t)B * c.head_count * s->attn_chunks * c.head_dim)) ||
        (rc = dev_alloc(s->allocs, &s->attn_part_ml, (size_t)B * c.head_count * s->attn_chunks * 2)) ||
        (rc = dev_alloc(s->allocs, &s->logits, (size_t)B * c.vocab_size)) ||
        (rc = dev_alloc(s->allocs, &s->probs, (size_t)B * c.vocab_size)) ||
        (rc = dev_alloc(s->allocs, &s->qbuf, (size_t)B * c.vocab_size)) ||
        (rc = dev_alloc(s->allocs, &s->tp_scratch, temperature_scratch_floats(B))) ||
        (rc = dev_alloc(s->allocs, &s->part_val, B * m->head.tiles)) ||
        (rc = dev_alloc(s->allocs, &s->part_idx, B * m->head.tiles)) ||
        (rc = dev_alloc(s->allocs, &s->d_toks, B)) || (rc = dev_alloc(s->allocs, &s->d_preds, B)) ||
        (rc = dev_alloc(s->allocs, &s->d_pos, 4)) || (rc = dev_alloc(s->allocs, &s->d_result, 4)) ||
        (rc = dev_alloc(s->allocs, &s->d_samp, (size_t)kSampleMaxRows)) ||
        (rc = dev_alloc(s->allocs, &s->ybuf,
                        B * std::max({c.attention_output_width + 2 * c.kv_width, 2 * c.feed_forward_length,
                                      c.embedding_length}))))
        return rc;
    NC_HIP(hipMemset(s->kcache, 0, kv * 4));
    NC_HIP(hipMemset(s->vcache, 0, kv * 4));
    NC_HIP(hipHostMalloc((void**)&s->h_toks, 64 * sizeof(uint32_t), hipHostMallocDefault));
    NC_HIP(hipHostMalloc((void**)&s->h_preds, 64 * sizeof(uint32_t), hipHostMallocDefault));
    NC_HIP(hipHostMalloc((void**)&s->h_result, 16 * sizeof(int32_t), hipHostMallocDefault));
    NC_HIP(hipHostMalloc((void**)&s->h_pos, 16 * sizeof(int32_t), hipHostMallocDefault));
    // RoPE (sin, cos) table, cached_rope_angles (inference.rs:860-901), from glibc on the
    // host: theta = base.powf(-(2i)/rope_dim), Llama-3 frequency scaling when the model
    // carries it (inference.rs:875-893), (sin, cos) = (pos*theta).sin_cos().
    const int64_t half = c.rope_dimension_count / 2;
    std::vector<float> tab((size_t)max_ctx * half * 2);
    static float (*volatile p_sinf)(float) = sinf;
    static float (*volatile p_cosf)(float) = cosf;
    static float (*volatile p_powf)(float, float) = powf;
    std::vector<float> theta(half);
    for (int64_t i = 0; i < half; i++) {
        float th = p_powf(c.rope_freq_base, -((float)(i * 2)) / (float)c.rope_dimension_count);
        if (c.rope_scaling) {
            const float factor = c.rope_scaling_factor, orig = c.rope_scaling_original_context_length;
            const float low = c.rope_scaling_low_freq_factor, high = c.rope_scaling_high_freq_factor;
            const float wavelength = (2.0f * 3.14159265358979323846f) / th;
            const float low_wl = orig / low, high_wl = orig / high;
            if (wavelength >= high_wl) {
                if (wavelength > low_wl) {
                    th = th / factor;
                } else {
                    const float smooth = (orig / wavelength - low) / (high - low);
                    th = ((1.0f - smooth) * th / factor) + (smooth * th);
                }
            }
        }
        theta[i] = th;
    }
    for (int64_t pos = 0; pos < max_ctx; pos++)
        for (int64_t i = 0; i < half; i++) {
            const float angle = (float)pos * theta[i];
            tab[(pos * half + i) * 2] = p_sinf(angle);
            tab[(pos * half + i) * 2 + 1] = p_cosf(angle);
        }
    if ((rc = upload_f32(s->allocs, tab, &s->rope_tab))) return rc;
    s->ev.resize(4096);
    for (auto& e : s->ev) {
        NC_HIP(hipEventCreate(&e.first));
        NC_HIP(hipEventCreate(&e.second));
    }
    *out = s.release();
    return NC_OK;
}

int nc_prefill(nc_session* s, const uint32_t* toks, int32_t n, int64_t start_pos, int32_t want_logits) {
    if (!s || !toks || n < 1) return fail(NC_EINVAL, "nc_prefill: bad arguments");
    NC_HIP(hipSetDevice(s->ctx->device));
    int rc = prefill_chunks(s, toks, n, start_pos, nullptr, want_logits != 0);
    if (rc) return rc;
    NC_HIP(hipStreamSynchronize(s->stream));
    return flush_timing(s);
}

int nc_forward1(nc_session* s, uint32_t tok, int64_t pos, float* logits_host, uint32_t* pred_out) {
    if (!s) return fail(NC_EINVAL, "null session");
    NC_HIP(hipSetDevice(s->ctx->device));
    int rc = upload_toks(s, &tok, 1);
    if (rc || (rc = run_pass(s, 1, pos))) return rc;
    if (logits_host) {
        NC_HIP(hipMemcpyAsync(logits_host, s->logits, s->m->cfg.vocab_size * 4, hipMemcpyDeviceToHost, s->stream));
    }
    uint32_t pred;
    if ((rc = fetch_preds(s, 1, &pred))) return rc;
    if (pred_out) *pred_out = pred;
    return flush_timing(s);
}

int nc_verify_greedy(nc_session* s, const uint32_t* toks, int32_t n, int64_t start_pos, nc_verify_result* result,
                     uint32_t* preds_host) {
    if (!s || !toks || !result || n < 1) return fail(NC_EINVAL, "nc_verify_greedy: bad arguments");
    NC_HIP(hipSetDevice(s->ctx->device));
    int rc = upload_toks(s, toks, n);
    if (rc || (rc = verify_step(s, n, start_pos, result))) return rc;
    if (preds_host && (rc = fetch_preds(s, n, preds_host))) return rc;
    return flush_timing(s);
}

int nc_verify_stochastic(nc_session* s, const uint32_t* toks, int32_t n, int64_t start_pos, const float* q_probs,
                         float temp, uint64_t seed, nc_verify_result* result) {
    if (!s || !toks || !result || n < 1 || (n > 1 && !q_probs) || !(temp > 0.0f))
        return fail(NC_EINVAL, "nc_verify_stochastic: bad arguments");
    NC_HIP(hipSetDevice(s->ctx->device));
    int rc = upload_toks(s, toks, n);
    if (rc || (rc = run_pass(s, n, start_pos)) || (rc = accept_stochastic_step(s, n, start_pos, q_probs, temp, seed)) ||
        (rc = fetch_result(s, n, result, nullptr)))
        return rc;
    return flush_timing(s);
}

int nc_session_logits(nc_session* s, int32_t row, float* logits_host) {
    if (!s || !logits_host || row < 0 || row >= s->last_n) return fail(NC_EINVAL, "nc_session_logits: bad row");
    NC_HIP(hipSetDevice(s->ctx->device));
    NC_HIP(hipMemcpyAsync(logits_host, s->logits + (size_t)row * s->m->cfg.vocab_size, s->m->cfg.vocab_size * 4,
                          hipMemcpyDeviceToHost, s->stream));
    NC_HIP(hipStreamSynchronize(s->stream));
    return NC_OK;
}

int nc_session_hidden(nc_session* s, int32_t n, float* hidden_host) {
    if (!s || !hidden_host || n < 1 || n > s->max_batch) return fail(NC_EINVAL, "nc_session_hidden: bad arguments");
    NC_HIP(hipSetDevice(s->ctx->device));
    NC_HIP(hipMemcpyAsync(hidden_host, s->hidden, (size_t)n * s->m->cfg.embedding_length * 4, hipMemcpyDeviceToHost,
                          s->stream));
    NC_HIP(hipStreamSynchronize(s->stream));
    return NC_OK;
}

int nc_generate_greedy(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new, uint32_t* out,
                       nc_decode_stats* stats) {
    if (!s || !prompt || !out || n_prompt < 1 || n_new < 1) return fail(NC_EINVAL, "nc_generate_greedy: bad arguments");
    if (n_prompt + n_new > s->max_ctx) return fail(NC_ERANGE, "prompt + new tokens exceed the session context");
    NC_HIP(hipSetDevice(s->ctx->device));
    const double t0 = now_s();
    uint32_t pending;
    int rc = prefill_chunks(s, prompt, n_prompt, 0, &pending);
    if (rc) return rc;
    const double t1 = now_s();
    int64_t pos = n_prompt, steps = 0;
    out[0] = pending;
    for (int i = 1; i < n_new; i++) {
        nc_verify_result r;
        if ((rc = upload_toks(s, &pending, 1)) || (rc = verify_step(s, 1, pos, &r))) return rc;
        pending = r.next_token;
        out[i] = pending;
        pos = r.new_pos;
        steps++;
    }
    const double t2 = now_s();
    if (stats) {
        *stats = nc_decode_stats{steps, 0, 0, n_new, t2 - t1, t1 - t0};
    }
    return flush_timing(s);
}

int nc_generate_plain(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new, float temp,
                      uint64_t* rng_state, const uint32_t* stop, int32_t n_stop, uint32_t* out, nc_decode_stats* stats) {
    const bool t = temp > 0.0f;
    if (!s || !prompt || !out || n_prompt < 1 || n_new < 1 || n_stop < 0 || (n_stop > 0 && !stop) ||
        (t && !rng_state))
        return fail(NC_EINVAL, "nc_generate_plain: bad arguments");
    if (!t && n_stop == 0) return nc_generate_greedy(s, prompt, n_prompt, n_new, out, stats);
    if (n_prompt >= s->max_ctx) return fail(NC_ERANGE, "prompt fills the session context");
    NC_HIP(hipSetDevice(s->ctx->device));
    const auto is_stop = [&](uint32_t id) { return std::find(stop, stop + n_stop, id) != stop + n_stop; };
    const double t0 = now_s();
    // main.rs:9676-9706 prefill; the last row's logits (and argmax) are the live ones
    uint32_t pending;
    int rc = prefill_chunks(s, prompt, n_prompt, 0, &pending, t);
    if (rc) return rc;
    int live = s->last_n - 1;
    const double t1 = now_s();
    int64_t pos = n_prompt, produced = 0, steps = 0;
    // the plain loop (main.rs:9894-9928): sample, end at a stop token, the context end or
    // n_new, emit, end at n_new, forward
    for (;;) {
        uint32_t id = pending;
        if (t) {
            const float u = lcg_next(rng_state);
            if ((rc = sample_session_rows(s, live, 1, temp, &u, &id))) return rc;
        }
        if (is_stop(id) || pos >= s->max_ctx || produced >= n_new) break;
        out[produced++] = id;
        if (produced >= n_new) break;
        if ((rc = nc_forward1(s, id, pos, nullptr, &pending))) return rc;
        live = 0;
        pos++;
        steps++;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, 0, 0, produced, t2 - t1, t1 - t0};
    return flush_timing(s);
}

int nc_generate_speculative_oracle(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new,
                                   int32_t max_steps, int32_t k, float alpha, uint64_t seed, const uint32_t* greedy,
                                   int32_t n_greedy, uint32_t* out, nc_decode_stats* stats) {
    if (!s || !prompt || !out || !greedy || n_prompt < 1 || n_new < 1 || k < 0)
        return fail(NC_EINVAL, "nc_generate_speculative_oracle: bad arguments");
    if (n_prompt + n_new > s->max_ctx) return fail(NC_ERANGE, "prompt + new tokens exceed the session context");
    NC_HIP(hipSetDevice(s->ctx->device));
    const uint32_t V = (uint32_t)s->m->cfg.vocab_size;
    // the drafter copies greedy[] into verify batches: every id must be a vocabulary id
    for (int32_t i = 0; i < n_greedy; i++)
        if (greedy[i] >= V) return fail(NC_ERANGE, "greedy record holds an id >= vocab_size");
    const double t0 = now_s();
    uint32_t pending;
    int rc = prefill_chunks(s, prompt, n_prompt, 0, &pending);
    if (rc) return rc;
    const double t1 = now_s();
    int64_t pos = n_prompt, produced = 0, steps = 0, drafted = 0, accepted = 0;
    out[produced++] = pending;
    uint32_t batch[16];
    while (produced < n_new && (max_steps <= 0 || steps < max_steps)) {
        int64_t kk = std::min<int64_t>(k, s->max_batch - 1);
        kk = std::min<int64_t>(kk, s->max_ctx - pos - 1);
        if (kk < 0) break;
        batch[0] = pending;
        for (int64_t i = 1; i <= kk; i++) batch[i] = nc_oracle_draft(seed, pos + i, alpha, greedy, n_prompt, n_greedy, V);
        nc_verify_result r;
        if ((rc = upload_toks(s, batch, (int)kk + 1)) || (rc = verify_step(s, (int)kk + 1, pos, &r))) return rc;
        drafted += kk;
        accepted += r.n_accepted;
        for (int i = 1; i <= r.n_accepted && produced < n_new; i++) out[produced++] = batch[i];
        pending = r.next_token;
        if (produced < n_new) out[produced++] = pending;
        pos = r.new_pos;
        steps++;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, drafted, accepted, produced, t2 - t1, t1 - t0};
    return flush_timing(s);
}

int32_t nc_ngram_draft(const uint32_t* history, int64_t len, int32_t min_ngram, int32_t max_ngram, int32_t max_tokens,
                       uint32_t* out) {
    // NGramDrafter::draft (speculative.rs:81-103): the longest suffix n-gram, max_ngram down
    // to min_ngram, that occurred earlier in the history (the most recent earlier occurrence
    // wins) proposes the tokens that followed it, at most max_tokens and never past the end.
    if (max_tokens <= 0 || min_ngram <= 0 || len <= min_ngram || !history || !out) return 0;
    const int64_t max_n = std::min<int64_t>(max_ngram, len - 1);
    for (int64_t n = max_n; n >= min_ngram; n--) {
        const uint32_t* pat = history + len - n;
        for (int64_t start = len - n - 1; start >= 0; start--) {
            if (!std::equal(pat, pat + n, history + start)) continue;
            const int64_t from = start + n, to = std::min<int64_t>(from + max_tokens, len);
            std::copy(history + from, history + to, out);
            return (int32_t)(to - from);  // from < len, so at least one token
        }
    }
    return 0;
}

int nc_generate_speculative_ngram(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new, int32_t k,
                                  int32_t min_ngram, int32_t max_ngram, const uint32_t* stop, int32_t n_stop,
                                  uint32_t* out, nc_decode_stats* stats) {
    if (!s || !prompt || !out || n_prompt < 1 || n_new < 1 || k < 0 || min_ngram < 1 || max_ngram < min_ngram ||
        n_stop < 0 || (n_stop > 0 && !stop))
        return fail(NC_EINVAL, "nc_generate_speculative_ngram: bad arguments");
    if (n_prompt >= s->max_ctx) return fail(NC_ERANGE, "prompt fills the session context");
    NC_HIP(hipSetDevice(s->ctx->device));
    auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    const double t0 = now_s();
    uint32_t pending;
    int rc = prefill_chunks(s, prompt, n_prompt, 0, &pending);
    if (rc) return rc;
    const double t1 = now_s();
    // ngram_speculative_step (speculative.rs:122-286) driven by main.rs:9729-9776, greedy, in
    // the k+1 verify form (cluster_tcp_smoke.rs:905-979): [pending] + drafts from the history
    // ending in pending; accepted = matching prefix; next pending = pred[accepted], which is
    // the step's corrective token and the next step's t0 at once.  The emitted stream is the
    // target's greedy stream cut before the first stop token (never emitted nor consumed).
    std::vector<uint32_t> history(prompt, prompt + n_prompt);
    history.reserve((size_t)n_prompt + n_new);
    int64_t pos = n_prompt, produced = 0, steps = 0, drafted = 0, accepted = 0;
    uint32_t batch[16];
    while (produced < n_new && !is_stop(pending)) {
        out[produced++] = pending;
        history.push_back(pending);
        if (produced >= n_new || pos + 1 >= s->max_ctx) break;
        // main.rs:9736-9737: a step emits at most the token budget (t0 is already counted)
        int64_t kk = std::min<int64_t>(k, n_new - produced);
        kk = std::min<int64_t>(kk, s->max_batch - 1);
        kk = std::min<int64_t>(kk, s->max_ctx - pos - 1);
        batch[0] = pending;
        const int nd = kk > 0 ? nc_ngram_draft(history.data(), (int64_t)history.size(), min_ngram, max_ngram, (int)kk,
                                               batch + 1)
                              : 0;
        nc_verify_result r;
        if ((rc = upload_toks(s, batch, nd + 1)) || (rc = verify_step(s, nd + 1, pos, &r))) return rc;
        drafted += nd;
        bool stopped = false;
        int counted = r.n_accepted;  // the step stops counting at a stop prediction
        for (int i = 1; i <= r.n_accepted && produced < n_new; i++) {
            if (is_stop(batch[i])) {
                stopped = true;
                counted = i;
                break;
            }
            out[produced++] = batch[i];
            history.push_back(batch[i]);
        }
        accepted += counted;
        pending = r.next_token;
        pos = r.new_pos;
        steps++;
        if (stopped) break;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, drafted, accepted, produced, t2 - t1, t1 - t0};
    return flush_timing(s);
}

int nc_generate_speculative_ngram_temp(nc_session* s, const uint32_t* prompt, int32_t n_prompt, int32_t n_new,
                                       int32_t k, int32_t min_ngram, int32_t max_ngram, float temp,
                                       uint64_t* rng_state, const uint32_t* stop, int32_t n_stop, uint32_t* out,
                                       nc_decode_stats* stats) {
    if (!(temp > 0.0f))
        return nc_generate_speculative_ngram(s, prompt, n_prompt, n_new, k, min_ngram, max_ngram, stop, n_stop, out,
                                             stats);
    if (!s || !prompt || !out || !rng_state || n_prompt < 1 || n_new < 1 || k < 0 || min_ngram < 1 ||
        max_ngram < min_ngram || n_stop < 0 || (n_stop > 0 && !stop))
        return fail(NC_EINVAL, "nc_generate_speculative_ngram_temp: bad arguments");
    if (n_prompt >= s->max_ctx) return fail(NC_ERANGE, "prompt fills the session context");
    NC_HIP(hipSetDevice(s->ctx->device));
    auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    const double t0 = now_s();
    int rc = prefill_chunks(s, prompt, n_prompt, 0, nullptr, true);
    if (rc) return rc;
    int live = s->last_n - 1;  // row of the live logits in the last pass
    const double t1 = now_s();
    // main.rs:9729-9776 over ngram_speculative_step (speculative.rs:122-286): t0 drawn from the
    // live logits (a stop token ends the turn unemitted); drafts from the history ending in t0;
    // one pass over t0 + drafts; one draw per verified row in order (drawn provisionally for
    // every row, kept as far as the verification reaches): a stop prediction ends the turn, a
    // mismatch emits the prediction and runs it as a corrective forward, and when every draft
    // matches the last row's logits are the next step's live logits.
    std::vector<uint32_t> history(prompt, prompt + n_prompt);
    history.reserve((size_t)n_prompt + n_new + 1);
    int64_t pos = n_prompt, produced = 0, steps = 0, drafted = 0, accepted = 0;
    uint32_t batch[16], tt[16];
    float uv[16];
    for (;;) {
        if (pos >= s->max_ctx || produced >= n_new) break;
        const int64_t ck = std::min<int64_t>(k, n_new - produced - 1);
        const float u0 = lcg_next(rng_state);
        if ((rc = sample_session_rows(s, live, 1, temp, &u0, &batch[0]))) return rc;
        if (is_stop(batch[0])) break;
        history.push_back(batch[0]);
        // drafts are truncated to the batch and the context (speculative.rs:154-159); asking the
        // drafter for no more than that gives the same prefix and keeps batch in bounds
        const int64_t cap = std::min<int64_t>(ck, std::min<int64_t>(s->max_batch - 1, s->max_ctx - (pos + 1)));
        const int64_t nd = cap > 0 ? nc_ngram_draft(history.data(), (int64_t)history.size(), min_ngram, max_ngram,
                                                    (int)cap, batch + 1)
                                   : 0;
        steps++;
        if (nd <= 0) {
            if ((rc = nc_forward1(s, batch[0], pos, nullptr, nullptr))) return rc;
            live = 0;
            out[produced++] = batch[0];
            pos++;
            continue;
        }
        drafted += nd;
        if ((rc = upload_toks(s, batch, (int)nd + 1)) || (rc = run_pass(s, (int)nd + 1, pos))) return rc;
        uint64_t st = *rng_state;
        for (int64_t r = 0; r < nd; r++) uv[r] = lcg_next(&st);
        if ((rc = sample_session_rows(s, 0, (int)nd, temp, uv, tt))) return rc;
        out[produced++] = batch[0];
        int64_t i = 0;
        bool hit_stop = false, done = false;
        for (; i < nd; i++) {
            if (batch[1 + i] == tt[i]) accepted++;
            if (is_stop(tt[i])) {  // neither emitted nor consumed
                hit_stop = done = true;
                pos += i + 1;
                break;
            }
            out[produced++] = tt[i];
            history.push_back(tt[i]);
            if (batch[1 + i] != tt[i]) {  // corrective forward
                if ((rc = nc_forward1(s, tt[i], pos + i + 1, nullptr, nullptr))) return rc;
                live = 0;
                pos += i + 2;
                done = true;
                break;
            }
        }
        const int64_t used = done ? i + 1 : nd;  // draws the verification made
        for (int64_t r = 0; r < used; r++) (void)lcg_next(rng_state);
        if (!done) {
            live = (int)nd;
            pos += nd + 1;
        }
        if (hit_stop) break;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, drafted, accepted, produced, t2 - t1, t1 - t0};
    return flush_timing(s);
}

}  // extern "C"

namespace nc {
// The greedy draft-model loop with stop tokens (is_stop_token of speculative.rs:305-447 and
// the generate loop's turn end, main.rs:9852-9866; n_stop = 0: none).
static int draft_loop_greedy(nc_session* tg, nc_session* dr, const uint32_t* prompt, int32_t n_prompt, int32_t n_new,
                             int32_t draft_k, const uint32_t* stop, int32_t n_stop, uint32_t* out,
                             nc_decode_stats* stats) {
    if (!tg || !dr || tg == dr || !prompt || !out || n_prompt < 1 || n_new < 1 || draft_k < 1 || n_stop < 0 ||
        (n_stop > 0 && !stop))
        return fail(NC_EINVAL, "nc_generate_speculative_draft: bad arguments");
    const auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    // drafts produced by one model are fed to the other's embedding: the vocabularies must agree
    if (tg->m->cfg.vocab_size != dr->m->cfg.vocab_size) return fail(NC_EINVAL, "target and draft vocabularies differ");
    if (tg->ctx->device != dr->ctx->device) return fail(NC_EINVAL, "target and draft must share a device");
    NC_HIP(hipSetDevice(tg->ctx->device));
    const double t0 = now_s();
    uint32_t tlive, dlive;
    // main.rs:9643-9706: prefill both models; live predictions for position n_prompt
    int rc = prefill_chunks(dr, prompt, n_prompt, 0, &dlive);
    if (rc || (rc = prefill_chunks(tg, prompt, n_prompt, 0, &tlive))) return rc;
    const double t1 = now_s();
    int64_t pos = n_prompt, produced = 0, steps = 0, drafted = 0, accepted = 0;
    uint32_t drafts[16], preds[16];
    bool saw_stop = false;  // the turn has ended (main.rs:9852-9866)
    while (!saw_stop && produced < n_new && pos < tg->max_ctx) {
        // speculative.rs:318-321 clamp
        int64_t k = std::min<int64_t>(draft_k, n_new - produced);
        k = std::min<int64_t>(k, tg->max_batch);
        k = std::min<int64_t>(k, tg->max_ctx - (pos + 1));
        k = std::min<int64_t>(k, dr->max_ctx - (pos + 1));
        if (k <= 0) break;
        // 1. drafting: sample from the draft's live prediction, then a draft forward; a
        // stop token is drafted but not run on the draft and ends drafting (speculative.rs:327-350)
        int64_t nd = 0;
        while (nd < k) {
            drafts[nd] = dlive;
            if (is_stop(drafts[nd++])) break;
            if ((rc = nc_forward1(dr, drafts[nd - 1], pos + nd - 1, nullptr, &dlive))) return rc;
        }
        // 2. batched target pass over the drafts
        if ((rc = upload_toks(tg, drafts, (int)nd)) || (rc = run_pass(tg, (int)nd, pos)) ||
            (rc = fetch_preds(tg, (int)nd, preds)))
            return rc;
        // 3. verification (speculative.rs:384-447); an accepted stop token ends it with no
        // trailing token and ends the turn
        drafted += nd;
        int64_t i = 0;
        bool stop_accepted = false;
        for (; i < nd; i++) {
            const uint32_t tt = i == 0 ? tlive : preds[i - 1];
            if (drafts[i] != tt) break;
            accepted++;
            if (is_stop(tt)) {
                stop_accepted = true;
                break;
            }
            if (produced < n_new) out[produced++] = drafts[i];
        }
        steps++;
        if (stop_accepted) {
            pos += i + 1;
            saw_stop = true;
            break;
        }
        uint32_t fix;
        int64_t at;
        if (i < nd) {
            fix = i == 0 ? tlive : preds[i - 1];  // corrective token
            at = pos + i;
        } else {
            fix = preds[nd - 1];  // 4. trailing verified token
            at = pos + nd;
        }
        if ((rc = nc_forward1(tg, fix, at, nullptr, &tlive)) || (rc = nc_forward1(dr, fix, at, nullptr, &dlive))) return rc;
        if (is_stop(fix)) saw_stop = true;  // not part of the stream
        else if (produced < n_new) out[produced++] = fix;
        pos = at + 1;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, drafted, accepted, produced, t2 - t1, t1 - t0};
    return flush_timing(tg);
}
}  // namespace nc

extern "C" {

int nc_generate_speculative_draft(nc_session* tg, nc_session* dr, const uint32_t* prompt, int32_t n_prompt,
                                  int32_t n_new, int32_t draft_k, uint32_t* out, nc_decode_stats* stats) {
    return draft_loop_greedy(tg, dr, prompt, n_prompt, n_new, draft_k, nullptr, 0, out, stats);
}

int nc_generate_speculative_draft_temp(nc_session* tg, nc_session* dr, const uint32_t* prompt, int32_t n_prompt,
                                       int32_t n_new, int32_t draft_k, float temp, uint64_t* rng_state,
                                       const uint32_t* stop, int32_t n_stop, uint32_t* out, nc_decode_stats* stats) {
    // sample_logits at temp <= 0 is the argmax and draws nothing: the greedy loop
    if (!(temp > 0.0f)) return draft_loop_greedy(tg, dr, prompt, n_prompt, n_new, draft_k, stop, n_stop, out, stats);
    if (!tg || !dr || tg == dr || !prompt || !out || !rng_state || n_prompt < 1 || n_new < 1 || draft_k < 1 ||
        n_stop < 0 || (n_stop > 0 && !stop))
        return fail(NC_EINVAL, "nc_generate_speculative_draft_temp: bad arguments");
    const auto is_stop = [&](uint32_t t) { return std::find(stop, stop + n_stop, t) != stop + n_stop; };
    if (tg->m->cfg.vocab_size != dr->m->cfg.vocab_size) return fail(NC_EINVAL, "target and draft vocabularies differ");
    if (tg->ctx->device != dr->ctx->device) return fail(NC_EINVAL, "target and draft must share a device");
    NC_HIP(hipSetDevice(tg->ctx->device));
    const double t0 = now_s();
    // main.rs:9643-9706: prefill both models; their last rows' logits are the live ones
    int rc = prefill_chunks(dr, prompt, n_prompt, 0, nullptr, true);
    if (rc || (rc = prefill_chunks(tg, prompt, n_prompt, 0, nullptr, true))) return rc;
    int dlive = dr->last_n - 1, tlive = tg->last_n - 1;  // rows of the live logits in the last pass
    const double t1 = now_s();
    int64_t pos = n_prompt, produced = 0, steps = 0, drafted = 0, accepted = 0;
    uint32_t drafts[16], tt[17];
    float uv[17];
    bool saw_stop = false;  // the turn has ended (main.rs:9852-9866)
    while (!saw_stop && produced < n_new && pos < tg->max_ctx) {
        // speculative.rs:318-321 clamp
        int64_t k = std::min<int64_t>(draft_k, n_new - produced);
        k = std::min<int64_t>(k, tg->max_batch);
        k = std::min<int64_t>(k, tg->max_ctx - (pos + 1));
        k = std::min<int64_t>(k, dr->max_ctx - (pos + 1));
        if (k <= 0) break;
        // 1. drafting (speculative.rs:327-350): one draw per draft from the draft's live logits;
        // a stop token is drafted but not run on the draft and ends drafting
        int64_t nd = 0;
        while (nd < k) {
            const float u = lcg_next(rng_state);
            if ((rc = sample_session_rows(dr, dlive, 1, temp, &u, &drafts[nd]))) return rc;
            if (is_stop(drafts[nd++])) break;
            if ((rc = nc_forward1(dr, drafts[nd - 1], pos + nd - 1, nullptr, nullptr))) return rc;
            dlive = 0;
        }
        k = nd;
        // 2. the first verification draw, from the target's live logits, before the batch pass
        // replaces them (speculative.rs:384-403)
        const uint64_t st0 = *rng_state;
        uint64_t st = st0;
        uv[0] = lcg_next(&st);
        if ((rc = sample_session_rows(tg, tlive, 1, temp, uv, &tt[0]))) return rc;
        // 3. batched target pass over the drafts (speculative.rs:365-373); row r predicts
        // position pos + r + 1, so draw r + 1 samples it, provisionally: only the draws the
        // verification reaches are kept
        if ((rc = upload_toks(tg, drafts, (int)k)) || (rc = run_pass(tg, (int)k, pos))) return rc;
        for (int64_t r = 0; r < k; r++) uv[1 + r] = lcg_next(&st);
        if ((rc = sample_session_rows(tg, 0, (int)k, temp, uv + 1, &tt[1]))) return rc;
        // 4. verification (speculative.rs:384-447) and the trailing token (:450-489); an accepted
        // stop token ends verification with no trailing draw and ends the turn
        drafted += k;
        int64_t i = 0;
        bool stop_accepted = false;
        for (; i < k && drafts[i] == tt[i]; i++) {
            accepted++;
            if (is_stop(drafts[i])) {
                stop_accepted = true;
                break;
            }
            if (produced < n_new) out[produced++] = drafts[i];
        }
        st = st0;
        for (int64_t r = 0; r <= i; r++) (void)lcg_next(&st);  // draws 0 .. i were made
        *rng_state = st;
        steps++;
        if (stop_accepted) {
            pos += i + 1;
            saw_stop = true;
            break;
        }
        const uint32_t fix = tt[i];  // corrective (i < k) or trailing (i == k) token
        const int64_t at = pos + i;
        if ((rc = nc_forward1(tg, fix, at, nullptr, nullptr)) || (rc = nc_forward1(dr, fix, at, nullptr, nullptr)))
            return rc;
        if (is_stop(fix)) saw_stop = true;  // not part of the stream
        else if (produced < n_new) out[produced++] = fix;
        tlive = dlive = 0;
        pos = at + 1;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, drafted, accepted, produced, t2 - t1, t1 - t0};
    return flush_timing(tg);
}

int nc_sample_logits_batch(nc_ctx* ctx, const float* logits, int32_t rows, int64_t vocab, float temp,
                           uint64_t* rng_state, float* work, uint32_t* tokens, void* stream) {
    if (!ctx || !logits || !tokens || rows < 1 || rows > 16 || vocab < 1 || vocab > INT32_MAX)
        return fail(NC_EINVAL, "nc_sample_logits_batch: bad arguments");
    const bool t = temp > 0.0f;
    if (t && (!rng_state || !work)) return fail(NC_EINVAL, "nc_sample_logits_batch: temperature needs rng_state and work");
    NC_HIP(hipSetDevice(ctx->device));
    hipStream_t st = stream ? (hipStream_t)stream : ctx->stream;
    float u[16] = {};
    if (t)
        for (int r = 0; r < rows; r++) u[r] = lcg_next(rng_state);  // rows in order, one draw each
    uint32_t* d_out = (uint32_t*)ctx->xsum;  // >= 16 ids of the context's operator scratch
    int rc = launch_sample_logits(logits, vocab, rows, (int)vocab, temp, u, work, vocab, ctx->tp_scratch, d_out, st);
    if (rc) return rc;
    NC_HIP(hipMemcpyAsync(tokens, d_out, rows * sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    NC_HIP(hipStreamSynchronize(st));
    return NC_OK;
}

int nc_generate_speculative_stochastic(nc_session* tg, nc_session* dr, const uint32_t* prompt, int32_t n_prompt,
                                       int32_t n_new, int32_t k, float temp, uint64_t seed, uint32_t* out,
                                       nc_decode_stats* stats) {
    if (!tg || !dr || tg == dr || !prompt || !out || n_prompt < 1 || n_new < 1 || k < 0 || !(temp > 0.0f))
        return fail(NC_EINVAL, "nc_generate_speculative_stochastic: bad arguments");
    if (tg->m->cfg.vocab_size != dr->m->cfg.vocab_size) return fail(NC_EINVAL, "target and draft vocabularies differ");
    if (tg->ctx->device != dr->ctx->device) return fail(NC_EINVAL, "target and draft must share a device");
    if (n_prompt >= tg->max_ctx || n_prompt >= dr->max_ctx) return fail(NC_ERANGE, "prompt fills the session context");
    NC_HIP(hipSetDevice(tg->ctx->device));
    const int V = (int)tg->m->cfg.vocab_size;
    const double t0 = now_s();
    int rc = prefill_chunks(dr, prompt, n_prompt, 0, nullptr);
    if (rc || (rc = prefill_chunks(tg, prompt, n_prompt, 0, nullptr, true))) return rc;
    NC_HIP(hipStreamSynchronize(dr->stream));
    // The draft's kernels run on the target's stream for the decode loop: the draft samples
    // feed the target's token buffer and probability rows without cross-stream waits.
    struct StreamShare {
        nc_session* d;
        hipStream_t own;
        ~StreamShare() { d->stream = own; }
    } share{dr, dr->stream};
    dr->stream = tg->stream;
    hipStream_t st = tg->stream;
    // first token: the target's last prompt row, u(seed, n_prompt - 1, bonus)
    if ((rc = launch_temperature_probs(tg->logits + (size_t)(tg->last_n - 1) * V, V, tg->probs, V, 1, V, temp,
                                       tg->tp_scratch, st)) ||
        (rc = launch_sample_probs(tg->probs, V, seed, n_prompt - 1, kPurposeBonus, (uint32_t*)(tg->d_result + 1),
                                  nullptr, tg->tp_scratch, st)))
        return rc;
    NC_HIP(hipMemcpyAsync(tg->h_result, tg->d_result, 4 * sizeof(int32_t), hipMemcpyDeviceToHost, st));
    NC_HIP(hipStreamSynchronize(st));
    uint32_t pending = (uint32_t)tg->h_result[1];
    const double t1 = now_s();
    int64_t pos = n_prompt, produced = 0, steps = 0, drafted = 0, accepted = 0;
    uint32_t last_draft = 0, toks[16];
    // catch_up: the last step drafted and accepted every draft, so the draft model has not
    // run its last draft d_{k-1} (at pos - 1).  kk only shrinks with pos, so once a step
    // drafts nothing (k = 0, or the context end) the draft model is never needed again.
    bool catch_up = false;
    out[produced++] = pending;
    while (produced < n_new) {
        int64_t kk = std::min<int64_t>(k, tg->max_batch - 1);
        kk = std::min<int64_t>(kk, tg->max_ctx - pos - 1);
        kk = std::min<int64_t>(kk, dr->max_ctx - pos - 1);
        if (kk < 0) break;
        if (kk > 0 && catch_up) {
            if ((rc = upload_toks(dr, &last_draft, 1)) || (rc = run_pass(dr, 1, pos - 1))) return rc;
        }
        // k draft forwards; draft i's sample becomes the next draft input and target row i+1
        for (int64_t i = 0; i < kk; i++) {
            if (i == 0 && (rc = upload_toks(dr, &pending, 1))) return rc;
            if ((rc = run_pass(dr, 1, pos + i)) ||
                (rc = launch_temperature_probs(dr->logits, V, tg->qbuf + (size_t)i * V, V, 1, V, temp,
                                               tg->tp_scratch, st)) ||
                (rc = launch_sample_probs(tg->qbuf + (size_t)i * V, V, seed, pos + i, kPurposeDraft, tg->d_toks + 1 + i,
                                          dr->d_toks, tg->tp_scratch, st)))
                return rc;
        }
        // target verify of [pending, d_0 .. d_{kk-1}]: only row 0 comes from the host
        nc_verify_result r;
        if ((rc = upload_toks(tg, &pending, 1)) || (rc = run_pass(tg, (int)kk + 1, pos)) ||
            (rc = accept_stochastic_step(tg, (int)kk + 1, pos, tg->qbuf, temp, seed)) ||
            (rc = fetch_result(tg, (int)kk + 1, &r, toks)))
            return rc;
        drafted += kk;
        accepted += r.n_accepted;
        for (int i = 1; i <= r.n_accepted && produced < n_new; i++) out[produced++] = toks[i];
        if (produced < n_new) out[produced++] = r.next_token;
        if (kk > 0) last_draft = toks[kk];
        catch_up = kk > 0 && r.n_accepted == kk;
        pending = r.next_token;
        pos = r.new_pos;
        steps++;
    }
    const double t2 = now_s();
    if (stats) *stats = nc_decode_stats{steps, drafted, accepted, produced, t2 - t1, t1 - t0};
    return flush_timing(tg);
}

int nc_synth_size(const nc_synth_spec* spec, uint64_t* size_out) {
    if (!spec || !size_out) return fail(NC_EINVAL, "null argument");
    return synth_size(*spec, size_out);
}

int nc_synth_write(const nc_synth_spec* spec, void* dst, uint64_t size, int32_t nthreads) {
    if (!spec || !dst) return fail(NC_EINVAL, "null argument");
    if (spec->embedding_length % spec->head_count || spec->embedding_length % 256 || spec->feed_forward_length % 256)
        return fail(NC_EINVAL, "synth: widths must be multiples of 256");
    if (spec->weight_type != NC_TYPE_Q4_0 && spec->weight_type != NC_TYPE_Q4_K && spec->weight_type != NC_TYPE_Q5_K &&
        spec->weight_type != NC_TYPE_Q8_0)
        return fail(NC_EINVAL, "synth: weight_type must be Q4_0, Q4_K, Q5_K or Q8_0");
    return synth_write(*spec, (uint8_t*)dst, size, nthreads);
}

int nc_uniform_prompt(uint64_t seed, int64_t n, uint32_t vocab, uint32_t* ids) {
    if (!ids || vocab == 0) return fail(NC_EINVAL, "bad arguments");
    for (int64_t i = 0; i < n; i++) ids[i] = philox_word(seed, (uint64_t)i, kPurposePrompt) % vocab;
    return NC_OK;
}

uint32_t nc_oracle_draft(uint64_t seed, int64_t p, float alpha, const uint32_t* greedy, int64_t n_prompt,
                         int64_t n_greedy, uint32_t vocab) {
    const float u = philox_uniform(seed, (uint64_t)p, kPurposeOracleU);
    const int64_t gi = p - n_prompt;
    if (u < alpha && gi >= 0 && gi < n_greedy) return greedy[gi];
    return philox_word(seed, (uint64_t)p, kPurposeOracleId) % vocab;
}

int nc_synth_kv_values(uint64_t seed, int32_t layer, int32_t kind, int64_t start, int64_t count, float* out) {
    if (!out || layer < 0 || (kind != 0 && kind != 1) || start < 0 || count < 0 || (start | count) & 1)
        return fail(NC_EINVAL, "nc_synth_kv_values: bad arguments");
    synth_normal_values(seed, (uint32_t)(2 * layer + kind), (uint64_t)start, (uint64_t)count, kPurposeKvFill, out);
    return NC_OK;
}

// Keys and values of rows [0, n) of every layer from nc_synth_kv_values: element i of row p of
// layer l's keys (kind 0) or values (kind 1) is stream 2l + kind, element p * kv_width + i.
// Layers are drawn on host threads and copied into the device layouts (keys in dim quads
// [Hkv][hd/4][ctx][4], values in position quads [Hkv][ctx/4][hd][4]); the rest of the cache keeps
// its contents, except the positions n.. of a value quad that n cuts, which are zeroed.
int nc_session_fill_kv(nc_session* s, int64_t n, uint64_t seed) {
    if (!s || n < 0 || n > s->max_ctx) return fail(NC_EINVAL, "nc_session_fill_kv: n outside [0, max_ctx]");
    if (n == 0) return NC_OK;
    const nc_model_config& c = s->m->cfg;
    const int64_t L = c.block_count, Hkv = c.head_count_kv, hd = c.head_dim, kw = c.kv_width;
    const int64_t stride = s->ctx_stride, layer_kv = Hkv * hd * stride, nq = (n + 3) / 4;
    NC_HIP(hipStreamSynchronize(s->stream));
    const int nth = (int)std::max<unsigned>(1, std::min<unsigned>(16, std::thread::hardware_concurrency()));
    std::vector<std::vector<float>> kst(nth), vst(nth);
    for (int64_t l0 = 0; l0 < L; l0 += nth) {
        const int cnt = (int)std::min<int64_t>(nth, L - l0);
        std::vector<std::thread> th;
        for (int t = 0; t < cnt; t++)
            th.emplace_back([&, t] {
                const int64_t l = l0 + t;
                std::vector<float> row(kw);
                std::vector<float>& K = kst[t];
                std::vector<float>& V = vst[t];
                K.assign((size_t)Hkv * (hd / 4) * n * 4, 0.0f);
                V.assign((size_t)Hkv * nq * hd * 4, 0.0f);
                for (int64_t p = 0; p < n; p++) {
                    synth_normal_values(seed, (uint32_t)(2 * l), (uint64_t)(p * kw), (uint64_t)kw, kPurposeKvFill,
                                        row.data());
                    for (int64_t i = 0; i < kw; i++) {
                        const int64_t h = i / hd, d = i % hd;
                        K[((size_t)(h * (hd / 4) + d / 4) * n + p) * 4 + (d & 3)] = row[i];
                    }
                    synth_normal_values(seed, (uint32_t)(2 * l + 1), (uint64_t)(p * kw), (uint64_t)kw, kPurposeKvFill,
                                        row.data());
                    for (int64_t i = 0; i < kw; i++) {
                        const int64_t h = i / hd, d = i % hd;
                        V[((size_t)(h * nq + p / 4) * hd + d) * 4 + (p & 3)] = row[i];
                    }
                }
            });
        for (auto& x : th) x.join();
        for (int t = 0; t < cnt; t++) {
            const int64_t l = l0 + t;
            NC_HIP(hipMemcpy2D(s->kcache + l * layer_kv, (size_t)stride * 16, kst[t].data(), (size_t)n * 16,
                               (size_t)n * 16, (size_t)Hkv * (hd / 4), hipMemcpyHostToDevice));
            NC_HIP(hipMemcpy2D(s->vcache + l * layer_kv, (size_t)(stride / 4) * hd * 16, vst[t].data(),
                               (size_t)nq * hd * 16, (size_t)nq * hd * 16, (size_t)Hkv, hipMemcpyHostToDevice));
        }
    }
    return NC_OK;
}

int nc_session_timing_enable(nc_session* s, int32_t enable) {
    if (!s) return fail(NC_EINVAL, "null session");
    int rc = flush_timing(s);
    if (rc || (rc = flush_stages(s))) return rc;
    if ((enable & 3) == 3) return fail(NC_EINVAL, "nc_session_timing_enable: matmul and stage timing are exclusive");
    if ((enable & 2) && s->stage_ev.empty()) {
        s->stage_ev.resize(4096);
        s->stage_of.resize(4096);
        for (auto& e : s->stage_ev) {
            NC_HIP(hipEventCreate(&e.first));
            NC_HIP(hipEventCreate(&e.second));
        }
    }
    s->stage_timing = (enable & 2) != 0;
    s->stage_ms.assign(kStages, 0.0);
    s->stage_calls.assign(kStages, 0);
    s->timing = (enable & 1) != 0;
    s->gemm_ms = 0.0;
    s->gemm_launches = 0;
    s->gemm_bytes = 0;
    s->pending_bytes = 0;
    return NC_OK;
}

int32_t nc_session_stage_timing(nc_session* s, int32_t index, char* name, int32_t name_cap, double* total_ms,
                                int64_t* calls) {
    if (!s) return fail(NC_EINVAL, "null session");
    if (int rc = flush_stages(s)) return rc;
    if (index >= 0 && index < kStages) {
        if (name && name_cap > 0) {
            std::strncpy(name, kStageNames[index], (size_t)name_cap - 1);
            name[name_cap - 1] = 0;
        }
        if (total_ms) *total_ms = s->stage_ms.empty() ? 0.0 : s->stage_ms[index];
        if (calls) *calls = s->stage_calls.empty() ? 0 : s->stage_calls[index];
    }
    return kStages;
}

int64_t nc_session_kernel_timing(nc_session* s, const char* family, double* total_ms, int64_t* bytes) {
    if (!s || !family) return fail(NC_EINVAL, "bad arguments");
    if (flush_timing(s)) return -1;
    if (std::strcmp(family, "gemm_q4_0") != 0) return fail(NC_EINVAL, "unknown kernel family");
    if (total_ms) *total_ms = s->gemm_ms;
    if (bytes) *bytes = s->gemm_bytes;
    return s->gemm_launches;
}

}  // extern "C"
