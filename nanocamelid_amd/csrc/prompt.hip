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

template <int LAYOUT, int D, bool XM>
__global__ __launch_bounds__(256) void gemm_q4_0_prompt_kernel(PromptGemm p) {
    // wave index through readfirstlane: the tile bases below are then scalar (buffer-load
    // soffsets) instead of per-lane values that the compiler would loop over
    const int lane = threadIdx.x & 63, wv = wave_id_uniform();
    const int g = lane >> 4, r = lane & 15;  // A/B lane (g, r); D lane (g, c = r)
    const int row0 = blockIdx.x * 64 + (wv & 1) * 32;
    const int tok0 = blockIdx.y * 64 + (wv >> 1) * 32;
    if (row0 >= p.M || tok0 >= p.N) return;  // wave-uniform; the kernel has no barriers
    const int K = 32 * p.nb, nq = (p.nb + 3) / 4;
    int rt[2], tk[2];
#pragma unroll
    for (int i = 0; i < 2; i++) rt[i] = min(row0 / 16 + i, p.tiles16 - 1);  // storage is padded to 16 rows
#pragma unroll
    for (int k = 0; k < 2; k++) tk[k] = min(tok0 + 16 * k + r, p.N - 1);
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc((void*)p.w, 0, (int)p.w_bytes, 0x00020000);
    const int n16 = (p.N + 15) / 16;  // 16-token tiles of the repacked activations
    const __amdgpu_buffer_rsrc_t xres = XM ? __builtin_amdgcn_make_buffer_rsrc((void*)p.xm, 0, n16 * K * 16, 0x00020000)
                                           : __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, p.N * K, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = XM ? __builtin_amdgcn_make_buffer_rsrc((void*)p.xsm, 0, n16 * nq * 256, 0x00020000)
                                           : __builtin_amdgcn_make_buffer_rsrc((void*)p.xs, 0, p.N * p.nb * 4, 0x00020000);
    int tt[2];  // 16-token tiles (repacked layout), clamped into the buffer
#pragma unroll
    for (int k = 0; k < 2; k++) tt[k] = min(tok0 / 16 + k, n16 - 1);
    // per-lane parts of the addresses
    int nvo[2], svo[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        if constexpr (LAYOUT == LAYOUT_R16) {
            nvo[i] = r * 16 + 4 * g;  // + 256 j within the quad
            svo[i] = 1024 + 32 * g;   // scales [row / 4][j][row % 4]
        } else {
            const int sub = rt[i] & 3;
            nvo[i] = (16 * sub + r) * 16 + 4 * g;  // + 1024 * (block % 8)
            svo[i] = 8192 + (16 * sub + 4 * g) * 8;  // scales [row][block % 4], + 512 per half-chunk
        }
    }
    const int xvo[2] = {tk[0] * K + 4 * g, tk[1] * K + 4 * g};
    const int mvo[2] = {tk[0] * p.nb * 4, tk[1] * p.nb * 4};
    auto tile_base = [&](int i, int qd) -> int {
        if constexpr (LAYOUT == LAYOUT_R16)
            return (rt[i] * p.groups + (qd >> 3)) * kQ40ChunkBytes + (qd & 7) * kQ40R16QuadBytes;
        else
            return ((rt[i] >> 2) * p.groups + (qd >> 1)) * kQ40ChunkBytes;
    };
    uint32_t nib[D][2][4], sw[D][2][8], xa[D][2][4], xb[D][2][4];
    float4 xsv[D][2];
#define NC_PQ_LOAD(QD, SLOT)                                                                                    \
    do {                                                                                                        \
        const int qd_ = min((QD), nq - 1);                                                                      \
        _Pragma("unroll") for (int i = 0; i < 2; i++) {                                                         \
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
            if constexpr (XM) {                                                                                 \
                _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                 \
                    const uint2 v_ = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(            \
                        xres, lane * 8, (tt[k] * p.nb + 4 * qd_ + j) * 512, 0));                                \
                    xa[SLOT][k][j] = v_.x;                                                                      \
                    xb[SLOT][k][j] = v_.y;                                                                      \
                }                                                                                               \
                xsv[SLOT][k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(               \
                    sres, r * 16, (tt[k] * nq + qd_) * 256, 0));                                                \
            } else {                                                                                            \
                _Pragma("unroll") for (int j = 0; j < 4; j++) {                                                 \
                    xa[SLOT][k][j] = __builtin_amdgcn_raw_buffer_load_b32(xres, xvo[k], 128 * qd_ + 32 * j, 0); \
                    xb[SLOT][k][j] = __builtin_amdgcn_raw_buffer_load_b32(xres, xvo[k] + 16, 128 * qd_ + 32 * j, 0); \
                }                                                                                               \
                xsv[SLOT][k] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(sres, mvo[k], 16 * qd_, 0)); \
            }                                                                                                   \
        }                                                                                                       \
    } while (0)
    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
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
                    for (int i = 0; i < 2; i++) {
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
        for (int i = 0; i < 2; i++) {
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

int launch_gemm_prompt(const QMatDev& w, const int8_t* x, const float* xs, float* out, int ld_out, int N,
                       hipStream_t st, const void* xm, const float* xsm) {
    if (w.type != NC_TYPE_Q4_0 || (w.layout != LAYOUT_R16 && w.layout != LAYOUT_R64))
        return fail(NC_EINVAL, "prompt matmul: Q4_0 matrices only");
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
    const dim3 grid((unsigned)((w.rows + 63) / 64), (unsigned)((N + 63) / 64));
    if (xm && xsm) {
        if (w.layout == LAYOUT_R16) hipLaunchKernelGGL((gemm_q4_0_prompt_kernel<LAYOUT_R16, 2, true>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((gemm_q4_0_prompt_kernel<LAYOUT_R64, 2, true>), grid, dim3(256), 0, st, p);
    } else {
        if (w.layout == LAYOUT_R16) hipLaunchKernelGGL((gemm_q4_0_prompt_kernel<LAYOUT_R16, 2, false>), grid, dim3(256), 0, st, p);
        else hipLaunchKernelGGL((gemm_q4_0_prompt_kernel<LAYOUT_R64, 2, false>), grid, dim3(256), 0, st, p);
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// Activations in MFMA operand order for the prompt matmul: xm unit (tile t, block b, lane
// (g, c)) = token 16t + c's bytes 32b + 4g..+3 and 32b + 16 + 4g..+3 (zero past N), so a wave
// reads a block's B operand as 512 contiguous bytes; xsm (t, quad q, c) = token 16t + c's scales
// of blocks 4q..4q+3 (zero past the row).  Units of x first, then of the scales.
__global__ void prompt_repack_kernel(const int8_t* x, const float* xs, int N, int nb, uint2* xm, float4* xsm) {
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
}

int launch_prompt_repack(const int8_t* x, const float* xs, int N, int K, void* xm, float* xsm, hipStream_t st) {
    const int nb = K / 32, n16 = (N + 15) / 16, nq = (nb + 3) / 4;
    const int64_t total = (int64_t)n16 * nb * 64 + (int64_t)n16 * nq * 16;
    hipLaunchKernelGGL(prompt_repack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, xs, N, nb,
                       (uint2*)xm, (float4*)xsm);
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
    hipLaunchKernelGGL(prompt_qkv_rope_kernel, dim3((rows + 255) / 256, N), dim3(256), 0, st, y, rows, start, aw, kw,
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
    hipLaunchKernelGGL(prompt_residual_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, y, hidden, total);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// fused_silu_mul (inference.rs:3367-3390) on the interleaved gate|up output (64-row group t:
// gate rows 32t..32t+31 in rows 64t..64t+31, the matching up rows in 64t+32..64t+63), then
// quantize_f32_to_q8_0 of each 32-wide block (inference.rs:4034-4041), as the EPI_SWIGLU_Q8
// epilogue.  One half-wave per (token, block).
__global__ void prompt_swiglu_q8_kernel(const float* y, int F, int total_blocks, int8_t* xq, float* xs,
                                        int32_t* xs8) {
    const int hb = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // (token, block) index
    if (hb >= total_blocks) return;                                 // whole half-waves exit together
    const int l = threadIdx.x & 31;
    const int nbf = F / 32, n = hb / nbf, t = hb % nbf;
    const float* yr = y + (size_t)n * 2 * F + 64 * t;
    const float g = yr[l], up = yr[32 + l];
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

int launch_prompt_swiglu_q8(const float* y, int N, int F, int8_t* xq, float* xs, int32_t* xs8, hipStream_t st) {
    if (F % 32) return fail(NC_EINVAL, "prompt SwiGLU: width must be a multiple of 32");
    const int total = N * (F / 32);
    hipLaunchKernelGGL(prompt_swiglu_q8_kernel, dim3((total * 32 + 255) / 256), dim3(256), 0, st, y, F, total, xq, xs,
                       xs8);
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
    hipLaunchKernelGGL(prompt_positions_kernel, dim3(1), dim3(256), 0, st, d, start, stride, count);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
