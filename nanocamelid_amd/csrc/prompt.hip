// Prompt (prefill) path on gfx950: the Q4_0 x Q8_0 batch matmul for many tokens at once on
// int8 MFMA, and the elementwise steps that the verify GEMMs fuse into their epilogues (RoPE
// and the KV-cache scatter, the residual add, SwiGLU + Q8_0), as separate kernels over the
// matmul's f32 output.
//
// Each output is the reference's f32 chain over the row's blocks in order
// (matmul_q4_0_batch, inference.rs:1385-1418, and the swizzled form :1525-1574):
//   sum = 0; for b: sum += (w_scale[b] * x_scale[b]) * (float)dot_b
// so any number of tokens gives the bits of the 1-token loop.  The int32 block dots come from
// v_mfma_i32_16x16x32_i8 on the raw nibbles (0..15) with the accumulator input set to
// -8 * sum(x) of the block, itself one MFMA of a constant -8 operand with the same activations:
//   A (16 rows x 32, weights): lane (g, r) holds row r's nibble bytes 4g..4g+3, i.e. weights
//     4g..4g+3 (low nibbles) and 16+4g..16+4g+3 (high nibbles);
//   B (32 x 16 tokens, activations): lane (g, c) holds token c's x[4g..4g+3], x[16+4g..+3];
//   D lane (g, c): token c, rows 4g..4g+3.
// A wave owns 32 rows x 32 tokens (2 x 2 MFMA tiles, 16 chains per lane); a workgroup of four
// waves covers 64 rows x 64 tokens, so each weight byte is read by two waves of one workgroup
// and each activation by two.  Unlike the verify kernels (one to sixteen tokens, bound by the
// weight stream), the work here is the chain arithmetic: four VALU operations per (row, token,
// block); the MFMAs run beside them.
#include "nc_internal.h"
#include "nc_device.h"

namespace nc {

typedef int p_v4i __attribute__((ext_vector_type(4)));

struct PromptGemm {
    const uint8_t* w = nullptr;
    int64_t w_bytes = 0;
    int groups = 0;   // chunks per tile row (R16: 32 blocks each, R64: 8)
    int tiles16 = 0;  // 16-row tiles present in storage
    int M = 0, nb = 0, N = 0, ld_out = 0;
    const int8_t* x = nullptr;  // [N][32 * nb]
    const float* xs = nullptr;  // [N][nb]
    // the same activations repacked in MFMA operand order (prompt_repack_kernel), or null:
    // xm [N/16][nb][lane (g, c)] 8 bytes, xsm [N/16][nb/4][c] the 4 scales of a quad
    const uint2* xm = nullptr;
    const float4* xsm = nullptr;
    float* out = nullptr;       // out[n * ld_out + row]
};

template <int LAYOUT, int D, int RT>
__global__ __launch_bounds__(256) void gemm_q4_0_prompt_kernel(PromptGemm p) {
    // wave index through readfirstlane: the tile bases below are then scalar (buffer-load
    // soffsets) instead of per-lane values that the compiler would loop over
    const int lane = threadIdx.x & 63, wv = wave_id_uniform();
    const int g = lane >> 4, r = lane & 15;  // A/B lane (g, r); D lane (g, c = r)
    // RT = 2: a wave covers 32 rows x 32 tokens, a workgroup 64 x 64; RT = 1 (matrices whose
    // 32 x 32 tiles would leave a SIMD one wave): 16 rows x 32 tokens, a workgroup 64 x 32
    const int row0 = RT == 2 ? blockIdx.x * 64 + (wv & 1) * 32 : blockIdx.x * 64 + wv * 16;
    const int tok0 = RT == 2 ? blockIdx.y * 64 + (wv >> 1) * 32 : blockIdx.y * 32;
    if (row0 >= p.M || tok0 >= p.N) return;  // wave-uniform; the kernel has no barriers
    const int K = 32 * p.nb, nq = (p.nb + 3) / 4;
    int rt[RT];
#pragma unroll
    for (int i = 0; i < RT; i++) rt[i] = min(row0 / 16 + i, p.tiles16 - 1);  // storage is padded to 16 rows
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc((void*)p.w, 0, (int)p.w_bytes, 0x00020000);
    const int n16 = (p.N + 15) / 16;  // 16-token tiles of the repacked activations
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xm, 0, n16 * K * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xsm, 0, n16 * nq * 256, 0x00020000);
    int tt[2];  // 16-token tiles (repacked layout), clamped into the buffer
#pragma unroll
    for (int k = 0; k < 2; k++) tt[k] = min(tok0 / 16 + k, n16 - 1);
    // per-lane parts of the addresses
    int nvo[RT], svo[RT];
#pragma unroll
    for (int i = 0; i < RT; i++) {
        if constexpr (LAYOUT == LAYOUT_R16) {
            nvo[i] = r * 16 + 4 * g;  // + 256 j within the quad
            svo[i] = 1024 + 32 * g;   // scales [row / 4][j][row % 4]
        } else {
            const int sub = rt[i] & 3;
            nvo[i] = (16 * sub + r) * 16 + 4 * g;  // + 1024 * (block % 8)
            svo[i] = 8192 + (16 * sub + 4 * g) * 8;  // scales [row][block % 4], + 512 per half-chunk
        }
    }
    auto tile_base = [&](int i, int qd) -> int {
        if constexpr (LAYOUT == LAYOUT_R16)
            return (rt[i] * p.groups + (qd >> 3)) * kQ40ChunkBytes + (qd & 7) * kQ40R16QuadBytes;
        else
            return ((rt[i] >> 2) * p.groups + (qd >> 1)) * kQ40ChunkBytes;
    };
    uint32_t nib[D][RT][4], sw[D][RT][8], xa[D][2][4], xb[D][2][4];
    float4 xsv[D][2];
#define NC_PQ_LOAD(QD, SLOT)                                                                                    \
    do {                                                                                                        \
        const int qd_ = min((QD), nq - 1);                                                                      \
        _Pragma("unroll") for (int i = 0; i < RT; i++) {                                                         \
            const int tb_ = tile_base(i, qd_);                                                                  \
            _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                     \
                const int jo_ = LAYOUT == LAYOUT_R16 ? 256 * j : 1024 * ((qd_ & 1) * 4 + j);                   \
                nib[SLOT][i][j] = __builtin_amdgcn_raw_buffer_load_b32(wres, nvo[i] + jo_, tb_, 0);             \
            }                                                                                                   \
            const int so_ = LAYOUT == LAYOUT_R16 ? 0 : 512 * (qd_ & 1);                                         \
            const uint4 s0_ = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, svo[i] + so_, tb_, 0)); \
            const uint4 s1_ = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, svo[i] + so_ + 16, tb_, 0)); \
            sw[SLOT][i][0] = s0_.x; sw[SLOT][i][1] = s0_.y; sw[SLOT][i][2] = s0_.z; sw[SLOT][i][3] = s0_.w;     \
            sw[SLOT][i][4] = s1_.x; sw[SLOT][i][5] = s1_.y; sw[SLOT][i][6] = s1_.z; sw[SLOT][i][7] = s1_.w;     \
        }                                                                                                       \
        _Pragma("unroll") for (int k = 0; k < 2; k++) {                                                         \
            _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                     \
                const uint2 v_ = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(                \
                    xres, lane * 8, (tt[k] * p.nb + 4 * qd_ + j) * 512, 0));                                    \
                xa[SLOT][k][j] = v_.x;                                                                          \
                xb[SLOT][k][j] = v_.y;                                                                          \
            }                                                                                                   \
            xsv[SLOT][k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(                   \
                sres, r * 16, (tt[k] * nq + qd_) * 256, 0));                                                    \
        }                                                                                                       \
    } while (0)
    float acc[RT][2][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][k][v] = 0.0f;
    const long minus8 = (long)0xF8F8F8F8F8F8F8F8ull;
    const p_v4i zero = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < D - 1; s++) NC_PQ_LOAD(s, s);
    for (int q0 = 0; q0 < nq; q0 += D) {
#pragma unroll
        for (int s = 0; s < D; s++) {
            const int qd = q0 + s;
            NC_PQ_LOAD(qd + D - 1, (s + D - 1) % D);
            if (qd < nq) {  // uniform
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (4 * qd + j >= p.nb) break;  // uniform
                    long bx[2];
                    p_v4i corr[2];
                    float xsj[2];
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        bx[k] = (long)((uint64_t)xa[s][k][j] | ((uint64_t)xb[s][k][j] << 32));
                        corr[k] = __builtin_amdgcn_mfma_i32_16x16x32_i8(minus8, bx[k], zero, 0, 0, 0);
                        xsj[k] = j == 0 ? xsv[s][k].x : j == 1 ? xsv[s][k].y : j == 2 ? xsv[s][k].z : xsv[s][k].w;
                    }
#pragma unroll
                    for (int i = 0; i < RT; i++) {
                        const uint32_t wn = nib[s][i][j];
                        const long a = (long)((uint64_t)(wn & 0x0F0F0F0Fu) | ((uint64_t)((wn >> 4) & 0x0F0F0F0Fu) << 32));
                        float ws[4];
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            // R16: [g][j][v] halves; R64: [v][j] halves
                            const uint32_t dw = LAYOUT == LAYOUT_R16 ? sw[s][i][2 * j + (v >> 1)] : sw[s][i][2 * v + (j >> 1)];
                            const int hi = LAYOUT == LAYOUT_R16 ? (v & 1) : (j & 1);
                            ws[v] = f16_to_f32((uint16_t)(hi ? dw >> 16 : dw & 0xffff));
                        }
#pragma unroll
                        for (int k = 0; k < 2; k++) {
                            const p_v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bx[k], corr[k], 0, 0, 0);
#pragma unroll
                            for (int v = 0; v < 4; v++) acc[i][k][v] = acc[i][k][v] + (ws[v] * xsj[k]) * (float)d[v];
                        }
                    }
                }
            }
        }
    }
#undef NC_PQ_LOAD
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int n = tok0 + 16 * k + r;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const int row = row0 + 16 * i + 4 * g;
            float* o = p.out + (size_t)n * p.ld_out + row;
            if (row + 3 < p.M && (p.ld_out & 3) == 0) {
                *(float4*)o = make_float4(acc[i][k][0], acc[i][k][1], acc[i][k][2], acc[i][k][3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (row + v < p.M) o[v] = acc[i][k][v];
            }
        }
    }
}

// Row tiles per wave: 2 (32 x 32 wave tiles) when that gives every SIMD at least two waves
// (2048 waves on 256 CUs), else 1 (16 x 32: twice the waves for the same work).
static int prompt_row_tiles(int64_t rows, int N) {
    return ((rows + 31) / 32) * ((N + 31) / 32) >= 2048 ? 2 : 1;
}

int launch_gemm_prompt(const QMatDev& w, const int8_t* x, const float* xs, float* out, int ld_out, int N,
                       hipStream_t st, const void* xm, const float* xsm) {
    if (w.type != NC_TYPE_Q4_0 || (w.layout != LAYOUT_R16 && w.layout != LAYOUT_R64))
        return fail(NC_EINVAL, "prompt matmul: Q4_0 matrices only");
    if (!xm || !xsm) return fail(NC_EINVAL, "prompt matmul: repacked activations required");
    if (N < 1 || (int64_t)N * w.cols >= (int64_t)1 << 31 || w.dev_bytes >= (int64_t)1 << 31)
        return fail(NC_ERANGE, "prompt matmul: operands exceed 2 GiB");
    PromptGemm p;
    p.w = w.dev;
    p.w_bytes = w.dev_bytes;
    p.groups = (int)w.groups;
    p.tiles16 = (int)(w.layout == LAYOUT_R16 ? w.tiles : 4 * w.tiles);
    p.M = (int)w.rows;
    p.nb = (int)(w.cols / 32);
    p.N = N;
    p.ld_out = ld_out;
    p.x = x;
    p.xs = xs;
    p.xm = (const uint2*)xm;
    p.xsm = (const float4*)xsm;
    p.out = out;
    if (prompt_row_tiles(w.rows, N) == 2) {
        const dim3 grid((unsigned)((w.rows + 63) / 64), (unsigned)((N + 63) / 64));
        if (w.layout == LAYOUT_R16) NC_LAUNCH((gemm_q4_0_prompt_kernel<LAYOUT_R16, 2, 2>), grid, dim3(256), 0, st, p);
        else NC_LAUNCH((gemm_q4_0_prompt_kernel<LAYOUT_R64, 2, 2>), grid, dim3(256), 0, st, p);
    } else {
        const dim3 grid((unsigned)((w.rows + 63) / 64), (unsigned)((N + 31) / 32));
        if (w.layout == LAYOUT_R16) NC_LAUNCH((gemm_q4_0_prompt_kernel<LAYOUT_R16, 2, 1>), grid, dim3(256), 0, st, p);
        else NC_LAUNCH((gemm_q4_0_prompt_kernel<LAYOUT_R64, 2, 1>), grid, dim3(256), 0, st, p);
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- Q4_K prompt matmul
// matmul_q4_k_batch (inference.rs:2006-2132, x86 path :2083-2130) for many tokens: per row and
// token, super-blocks in order, each the f32 sum from 0.0 over its eight 32-value sub-blocks j of
//   xs_j * (sc_j * (float)W_j - mn_j * (float)A_j),   sc_j = d * s_j, mn_j = dmin * m_j
// (q8.rs:1339-1376 dot_q8_scaled_preloaded, scales by q4_k_scale_min q8.rs:2009-2018), with
// W_j = sum nib * x (unsigned nibbles) and A_j = sum x of the sub-block; that super-block sum is
// added to the row's sum.  W_j comes from v_mfma_i32_16x16x32_i8 on the raw nibbles (K = 32 = one
// sub-block): sub-block 2p is the low nibbles of bytes 32p..32p+31, 2p + 1 the high nibbles, so
// lane (g, r)'s dwords at bytes 32p + 4g and 32p + 16 + 4g give both A operands.  A_j as a float
// comes with the repacked activations (xam).  Lane (g, r) decodes its row's scales and mins of
// sub-blocks 2g and 2g + 1 into a per-wave LDS table from which the D lanes (g, c) read rows
// 4g..4g+3.  A wave covers 32 rows x 32 tokens, a workgroup 64 x 64; weights stay in the verify
// layouts (R16K: 16-row tiles, chunks of 4 super-blocks; R64: 64-row tiles, one super-block per
// chunk), each chunk 9 slots of [64 lanes x 16 B], slot 0 the header (d, dmin, 12 scale bytes).
struct PromptGemmK {
    const uint8_t* w = nullptr;
    int64_t w_bytes = 0;
    int nsb = 0, groups = 0, tiles16 = 0;  // super-blocks per row; R16K chunks per tile; 16-row tiles stored
    int M = 0, N = 0, ld_out = 0;
    const uint2* xm = nullptr;    // activations in MFMA operand order (prompt_repack_kernel)
    const float4* xsm = nullptr;  // x_scale of each sub-block, 4 per float4
    const float4* xam = nullptr;  // (float) sum of each sub-block's int8 values, 4 per float4
    float* out = nullptr;         // out[n * ld_out + row]
};

__device__ __forceinline__ void q4k_scale_min_dev(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t* s, uint32_t* m) {
    // 12 scale bytes in three dwords; byte k = (dw[k / 4] >> 8 (k % 4)) & 255 (q8.rs:2009-2018)
    auto byte = [&](int k) -> uint32_t {
        const uint32_t d = k < 4 ? s0 : k < 8 ? s1 : s2;
        return (d >> (8 * (k & 3))) & 0xffu;
    };
    if (j < 4) {
        *s = byte(j) & 63;
        *m = byte(j + 4) & 63;
    } else {
        *s = (byte(j + 4) & 0x0f) | ((byte(j - 4) >> 6) << 4);
        *m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}

template <int LAYOUT, int RT>
__global__ __launch_bounds__(256) void gemm_q4_k_prompt_kernel(PromptGemmK p) {
    __shared__ __align__(16) float tab[4][2][8][2][16];  // per wave: [tile][sub-block][sc, mn][row]
    const int lane = threadIdx.x & 63, wv = wave_id_uniform();
    const int g = lane >> 4, r = lane & 15;
    // RT = 2: a wave covers 32 rows x 32 tokens, a workgroup 64 x 64; RT = 1 (matrices whose
    // 32 x 32 tiles would leave a SIMD one wave): 16 rows x 32 tokens, a workgroup 64 x 32
    const int row0 = RT == 2 ? blockIdx.x * 64 + (wv & 1) * 32 : blockIdx.x * 64 + wv * 16;
    const int tok0 = RT == 2 ? blockIdx.y * 64 + (wv >> 1) * 32 : blockIdx.y * 32;
    if (row0 >= p.M || tok0 >= p.N) return;  // wave-uniform; the kernel has no barriers
    const int n16 = (p.N + 15) / 16, nq = 2 * p.nsb;  // 16-token tiles, quads of sub-blocks
    int tt[2];
#pragma unroll
    for (int k = 0; k < 2; k++) tt[k] = min(tok0 / 16 + k, n16 - 1);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc((void*)p.w, 0, (int)p.w_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xm, 0, n16 * p.nsb * 256 * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xsm, 0, n16 * nq * 256, 0x00020000);
    const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc((void*)p.xam, 0, n16 * nq * 256, 0x00020000);
    // chunk offset of (16-row tile i, super-block sb) and this lane's part of a slot
    auto chunk = [&](int i, int sb) -> int {
        if constexpr (LAYOUT == LAYOUT_R16K) {
            const int t16 = min(row0 / 16 + i, p.tiles16 - 1);  // storage is padded to 16 rows
            return (t16 * p.groups + sb / 4) * kQ4KChunkBytes + 256 * (sb & 3);
        } else {
            return ((row0 / 64) * p.nsb + sb) * kQ4KChunkBytes + ((row0 & 63) + 16 * i) * 16;
        }
    };
    // one stage = half a super-block (sub-blocks 4h..4h+3): per tile the nibble dwords of two
    // pairs and the header; per token tile four B operands, the x_scales and the sums
    uint32_t hd[2][RT][4], nb0[2][RT][2], nb1[2][RT][2], xa[2][2][4], xb[2][2][4];
    float4 xsv[2][2], xav[2][2];
#define NC_PK_LOAD(ST, SLOT)                                                                                    \
    do {                                                                                                        \
        const int st_ = min((ST), nq - 1), sb_ = st_ >> 1, h_ = st_ & 1;                                        \
        _Pragma("unroll") for (int i = 0; i < RT; i++) {                                                         \
            const int c_ = chunk(i, sb_);                                                                       \
            const uint4 hv_ = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, r * 16, c_, 0)); \
            hd[SLOT][i][0] = hv_.x; hd[SLOT][i][1] = hv_.y; hd[SLOT][i][2] = hv_.z; hd[SLOT][i][3] = hv_.w;     \
            _Pragma("unroll") for (int pp = 0; pp < 2; pp++) {                                                  \
                const int pr_ = 2 * h_ + pp;                                                                    \
                nb0[SLOT][i][pp] = __builtin_amdgcn_raw_buffer_load_b32(wres, r * 16 + 4 * g, c_ + (2 * pr_ + 1) * 1024, 0); \
                nb1[SLOT][i][pp] = __builtin_amdgcn_raw_buffer_load_b32(wres, r * 16 + 4 * g, c_ + (2 * pr_ + 2) * 1024, 0); \
            }                                                                                                   \
        }                                                                                                       \
        _Pragma("unroll") for (int k = 0; k < 2; k++) {                                                         \
            _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                     \
                const uint2 v_ = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(                \
                    xres, lane * 8, (tt[k] * 8 * p.nsb + 4 * st_ + j) * 512, 0));                               \
                xa[SLOT][k][j] = v_.x;                                                                          \
                xb[SLOT][k][j] = v_.y;                                                                          \
            }                                                                                                   \
            xsv[SLOT][k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(sres, r * 16, (tt[k] * nq + st_) * 256, 0)); \
            xav[SLOT][k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ares, r * 16, (tt[k] * nq + st_) * 256, 0)); \
        }                                                                                                       \
    } while (0)
    float acc[RT][2][4], part[RT][2][4];
#pragma unroll
    for (int i = 0; i < RT; i++)
#pragma unroll
        for (int k = 0; k < 2; k++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][k][v] = 0.0f;
    const p_v4i zero = {0, 0, 0, 0};
    float(*wt)[8][2][16] = tab[wv];
    NC_PK_LOAD(0, 0);
    for (int s0 = 0; s0 < nq; s0 += 2) {
#pragma unroll
        for (int s = 0; s < 2; s++) {
            const int st = s0 + s;  // s == st & 1 (nq is even)
            NC_PK_LOAD(st + 1, (s + 1) & 1);
            if (s == 0) {
                // this lane's row r, sub-blocks 2g and 2g + 1: scales and mins into the table
#pragma unroll
                for (int i = 0; i < RT; i++) {
                    const float d = f16_to_f32((uint16_t)(hd[0][i][0] & 0xffff));
                    const float dmin = f16_to_f32((uint16_t)(hd[0][i][0] >> 16));
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        uint32_t sv, mv;
                        q4k_scale_min_dev(2 * g + e, hd[0][i][1], hd[0][i][2], hd[0][i][3], &sv, &mv);
                        wt[i][2 * g + e][0][r] = d * (float)sv;
                        wt[i][2 * g + e][1][r] = dmin * (float)mv;
                    }
                }
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
                for (int i = 0; i < RT; i++)
#pragma unroll
                    for (int k = 0; k < 2; k++)
#pragma unroll
                        for (int v = 0; v < 4; v++) part[i][k][v] = 0.0f;
            }
#pragma unroll
            for (int jj = 0; jj < 4; jj++) {
                const int j = 4 * s + jj, pp = jj >> 1, hi = jj & 1;  // sub-block j of the super-block
                long bx[2];
                float xsj[2], xaj[2];
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    bx[k] = (long)((uint64_t)xa[s][k][jj] | ((uint64_t)xb[s][k][jj] << 32));
                    const float4 xs4 = xsv[s][k], xa4 = xav[s][k];
                    xsj[k] = jj == 0 ? xs4.x : jj == 1 ? xs4.y : jj == 2 ? xs4.z : xs4.w;
                    xaj[k] = jj == 0 ? xa4.x : jj == 1 ? xa4.y : jj == 2 ? xa4.z : xa4.w;
                }
#pragma unroll
                for (int i = 0; i < RT; i++) {
                    const uint32_t w0 = hi ? (nb0[s][i][pp] >> 4) : nb0[s][i][pp];
                    const uint32_t w1 = hi ? (nb1[s][i][pp] >> 4) : nb1[s][i][pp];
                    const long a = (long)((uint64_t)(w0 & 0x0F0F0F0Fu) | ((uint64_t)(w1 & 0x0F0F0F0Fu) << 32));
                    const float4 sc4 = *(const float4*)&wt[i][j][0][4 * g];
                    const float4 mn4 = *(const float4*)&wt[i][j][1][4 * g];
                    const float scv[4] = {sc4.x, sc4.y, sc4.z, sc4.w}, mnv[4] = {mn4.x, mn4.y, mn4.z, mn4.w};
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const p_v4i dw = __builtin_amdgcn_mfma_i32_16x16x32_i8(a, bx[k], zero, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++) {
                            const float av = scv[v] * (float)dw[v];
                            const float bv = mnv[v] * xaj[k];
                            part[i][k][v] = part[i][k][v] + xsj[k] * (av - bv);
                        }
                    }
                }
            }
            if (s == 1) {
#pragma unroll
                for (int i = 0; i < RT; i++)
#pragma unroll
                    for (int k = 0; k < 2; k++)
#pragma unroll
                        for (int v = 0; v < 4; v++) acc[i][k][v] = acc[i][k][v] + part[i][k][v];
                // every lane has read this super-block's table before the next one is written
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            }
        }
    }
#undef NC_PK_LOAD
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int n = tok0 + 16 * k + r;
        if (n >= p.N) continue;
#pragma unroll
        for (int i = 0; i < RT; i++) {
            const int row = row0 + 16 * i + 4 * g;
            float* o = p.out + (size_t)n * p.ld_out + row;
            if (row + 3 < p.M && (p.ld_out & 3) == 0) {
                *(float4*)o = make_float4(acc[i][k][0], acc[i][k][1], acc[i][k][2], acc[i][k][3]);
            } else {
#pragma unroll
                for (int v = 0; v < 4; v++)
                    if (row + v < p.M) o[v] = acc[i][k][v];
            }
        }
    }
}

int launch_gemm_prompt_q4k(const QMatDev& w, float* out, int ld_out, int N, hipStream_t st, const void* xm,
                           const float* xsm, const float* xam) {
    if (w.type != NC_TYPE_Q4_K || (w.layout != LAYOUT_R16K && w.layout != LAYOUT_R64))
        return fail(NC_EINVAL, "Q4_K prompt matmul: Q4_K matrices only");
    if (!xm || !xsm || !xam) return fail(NC_EINVAL, "Q4_K prompt matmul: repacked activations required");
    if (N < 1 || (int64_t)N * w.cols >= (int64_t)1 << 31 || w.dev_bytes >= (int64_t)1 << 31)
        return fail(NC_ERANGE, "Q4_K prompt matmul: operands exceed 2 GiB");
    PromptGemmK p;
    p.w = w.dev;
    p.w_bytes = w.dev_bytes;
    p.nsb = (int)(w.cols / 256);
    p.groups = (int)w.groups;
    p.tiles16 = (int)(w.layout == LAYOUT_R16K ? w.tiles : 4 * w.tiles);
    p.M = (int)w.rows;
    p.N = N;
    p.ld_out = ld_out;
    p.xm = (const uint2*)xm;
    p.xsm = (const float4*)xsm;
    p.xam = (const float4*)xam;
    p.out = out;
    if (prompt_row_tiles(w.rows, N) == 2) {
        const dim3 grid((unsigned)((w.rows + 63) / 64), (unsigned)((N + 63) / 64));
        if (w.layout == LAYOUT_R16K) NC_LAUNCH((gemm_q4_k_prompt_kernel<LAYOUT_R16K, 2>), grid, dim3(256), 0, st, p);
        else NC_LAUNCH((gemm_q4_k_prompt_kernel<LAYOUT_R64, 2>), grid, dim3(256), 0, st, p);
    } else {
        const dim3 grid((unsigned)((w.rows + 63) / 64), (unsigned)((N + 31) / 32));
        if (w.layout == LAYOUT_R16K) NC_LAUNCH((gemm_q4_k_prompt_kernel<LAYOUT_R16K, 1>), grid, dim3(256), 0, st, p);
        else NC_LAUNCH((gemm_q4_k_prompt_kernel<LAYOUT_R64, 1>), grid, dim3(256), 0, st, p);
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// Activations in MFMA operand order for the prompt matmul: xm unit (tile t, block b, lane
// (g, c)) = token 16t + c's bytes 32b + 4g..+3 and 32b + 16 + 4g..+3 (zero past N), so a wave
// reads a block's B operand as 512 contiguous bytes; xsm (t, quad q, c) = token 16t + c's scales
// of blocks 4q..4q+3 (zero past the row).  Units of x first, then of the scales.
__global__ void prompt_repack_kernel(const int8_t* x, const float* xs, int N, int nb, uint2* xm, float4* xsm,
                                     float4* xam) {
    const int64_t id = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int n16 = (N + 15) / 16, nq = (nb + 3) / 4, K = 32 * nb;
    const int64_t nx = (int64_t)n16 * nb * 64;
    if (id < nx) {
        const int lane = (int)(id & 63), g = lane >> 4, c = lane & 15;
        const int64_t tb = id >> 6;
        const int b = (int)(tb % nb), n = (int)(tb / nb) * 16 + c;
        uint2 v = make_uint2(0u, 0u);
        if (n < N) {
            const int8_t* row = x + (size_t)n * K + 32 * b + 4 * g;
            v.x = *(const uint32_t*)row;
            v.y = *(const uint32_t*)(row + 16);
        }
        xm[id] = v;
        return;
    }
    const int64_t id2 = id - nx;
    if (id2 >= (int64_t)n16 * nq * 16) return;
    const int c = (int)(id2 & 15);
    const int64_t tq = id2 >> 4;
    const int q = (int)(tq % nq), n = (int)(tq / nq) * 16 + c;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (n < N) {
        const float* sr = xs + (size_t)n * nb + 4 * q;
        v.x = sr[0];
        if (4 * q + 1 < nb) v.y = sr[1];
        if (4 * q + 2 < nb) v.z = sr[2];
        if (4 * q + 3 < nb) v.w = sr[3];
    }
    xsm[id2] = v;
    if (xam) {  // (float) sum of each block's int8 values (exact: |sum| <= 32 * 128)
        float sa[4] = {0.f, 0.f, 0.f, 0.f};
        if (n < N) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (4 * q + e >= nb) break;
                const int* blk = (const int*)(x + (size_t)n * K + 32 * (4 * q + e));
                int sum = 0;
#pragma unroll
                for (int d = 0; d < 8; d++) sum = __builtin_amdgcn_sdot4(blk[d], 0x01010101, sum, false);
                sa[e] = (float)sum;
            }
        }
        xam[id2] = make_float4(sa[0], sa[1], sa[2], sa[3]);
    }
}

int launch_prompt_repack(const int8_t* x, const float* xs, int N, int K, void* xm, float* xsm, hipStream_t st,
                         float* xam) {
    const int nb = K / 32, n16 = (N + 15) / 16, nq = (nb + 3) / 4;
    const int64_t total = (int64_t)n16 * nb * 64 + (int64_t)n16 * nq * 16;
    NC_LAUNCH(prompt_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, xs, N, nb,
                       (uint2*)xm, (float4*)xsm, (float4*)xam);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- elementwise steps
// inference.rs:3894-3924: RoPE (NORM pairs 2i, 2i+1 of each head) on the q and k rows of the
// fused q|k|v output, then q to q_out and k, v into the KV cache at positions start + n.
// The same arithmetic as the verify GEMMs' EPI_QKV_ROPE epilogue.
__global__ void prompt_qkv_rope_kernel(const float* y, int ld, int start, int aw, int kw, int hd, int rope_half,
                                       const float* rope_tab, float* q_out, float* kcache, float* vcache,
                                       int max_ctx) {
    const int n = blockIdx.y;
    const int row = blockIdx.x * blockDim.x + threadIdx.x;
    if (row >= aw + 2 * kw) return;
    const float* yr = y + (size_t)n * ld;
    float v = yr[row];
    const int pos = start + n;
    const bool is_q = row < aw, is_k = !is_q && row < aw + kw;
    const int rr = is_q ? row : (is_k ? row - aw : row - aw - kw);
    if (is_q || is_k) {
        const int i = (rr % hd) >> 1;
        if (i < rope_half) {
            const float* sc = rope_tab + ((size_t)pos * rope_half + i) * 2;
            const float sn = sc[0], cs = sc[1];
            const float x0 = yr[row & ~1], x1 = yr[row | 1];
            v = (row & 1) ? (x0 * sn + x1 * cs) : (x0 * cs - x1 * sn);
        }
    }
    if (is_q) {
        q_out[(size_t)n * aw + rr] = v;
    } else {
        const int kvh = rr / hd, d = rr % hd;
        if (is_k) kcache[(((size_t)kvh * (hd / 4) + d / 4) * max_ctx + pos) * 4 + (d & 3)] = v;
        else vcache[(((size_t)kvh * (max_ctx / 4) + pos / 4) * hd + d) * 4 + (pos & 3)] = v;
    }
}

int launch_prompt_qkv_rope(const float* y, int N, int start, int aw, int kw, int hd, int rope_half,
                           const float* rope_tab, float* q_out, float* kcache, float* vcache, int max_ctx,
                           hipStream_t st) {
    if ((aw | kw) & 1) return fail(NC_EINVAL, "prompt RoPE: widths must be even");
    const int rows = aw + 2 * kw;
    NC_LAUNCH(prompt_qkv_rope_kernel, dim3((rows + 255) / 256, N), dim3(256), 0, st, y, rows, start, aw, kw,
                       hd, rope_half, rope_tab, q_out, kcache, vcache, max_ctx);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// hidden += matmul output (inference.rs:3985, 4073; add_residual_batch :4122), as the
// EPI_RESIDUAL epilogue: h = y + h.
__global__ void prompt_residual_kernel(const float* y, float* hidden, int64_t total) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < total) hidden[i] = y[i] + hidden[i];
}

int launch_prompt_residual(const float* y, float* hidden, int N, int d, hipStream_t st) {
    const int64_t total = (int64_t)N * d;
    NC_LAUNCH(prompt_residual_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, y, hidden, total);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// fused_silu_mul (inference.rs:3367-3390) on the interleaved gate|up output (64-row group t:
// gate rows 32t..32t+31 in rows 64t..64t+31, the matching up rows in 64t+32..64t+63) or, with
// split, on gate rows 0..F-1 followed by up rows F..2F-1; then quantize_f32_to_q8_0 of each
// 32-wide block (inference.rs:4034-4041), as the EPI_SWIGLU_Q8 epilogue.  One half-wave per
// (token, block).
__global__ void prompt_swiglu_q8_kernel(const float* y, int F, int total_blocks, int8_t* xq, float* xs,
                                        int32_t* xs8, int split) {
    const int hb = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // (token, block) index
    if (hb >= total_blocks) return;                                 // whole half-waves exit together
    const int l = threadIdx.x & 31;
    const int nbf = F / 32, n = hb / nbf, t = hb % nbf;
    const float* yr = y + (size_t)n * 2 * F + (split ? 32 * t : 64 * t);
    const float g = yr[l], up = yr[(split ? F : 32) + l];
    const float sig = 1.0f / (1.0f + expf_glibc(-g));
    const float v = g * sig * up;
    const float amax = halfwave_amax(v);
    float scale;
    const int q = quantize_lane_q8(v, amax, &scale);
    const int qs = halfwave_isum(q);
    xq[(size_t)n * F + 32 * t + l] = (int8_t)q;
    if (l == 0) {
        xs[hb] = scale;
        xs8[hb] = -8 * qs;
    }
}

int launch_prompt_swiglu_q8(const float* y, int N, int F, int8_t* xq, float* xs, int32_t* xs8, hipStream_t st,
                            bool split) {
    if (F % 32) return fail(NC_EINVAL, "prompt SwiGLU: width must be a multiple of 32");
    const int total = N * (F / 32);
    NC_LAUNCH(prompt_swiglu_q8_kernel, dim3((total * 32 + 255) / 256), dim3(256), 0, st, y, F, total, xq, xs,
                       xs8, split ? 1 : 0);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// Start positions of the attention row groups of a prompt pass: d[i] = start + i * stride.
__global__ void prompt_positions_kernel(int32_t* d, int start, int stride, int count) {
    const int i = threadIdx.x;
    if (i < count) d[i] = start + i * stride;
}

int launch_prompt_positions(int32_t* d, int start, int stride, int count, hipStream_t st) {
    if (count < 1 || count > 256) return fail(NC_EINVAL, "prompt positions: 1..256 groups");
    NC_LAUNCH(prompt_positions_kernel, dim3(1), dim3(256), 0, st, d, start, stride, count);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
