// Skinny quantized GEMM for the k+1-column verify batch on gfx950.
//
//   out[n][r] = sum_b fl( fl(w_scale[r][b] * x_scale[n][b]) * (float)dot_i32(w[r][b], x[n][b]) )
//
// with the f32 sum taken strictly in block order b = 0, 1, ... (Q4_0:
// inference.rs:1553-1573; Q4_K: per super-block partials in order,
// inference.rs:2083-2130), so results are bit-identical to the reference's
// portable path.
//
// Mapping: one 64-row tile per workgroup, lane = row.  Weight bytes come from a
// repacked layout where every wave-wide load is 1 KB contiguous.  Q4_0: the activation
// block of a token is wave-uniform; each 16-lane row loads it once (one dword per lane)
// and v_dot4c_i32_i8 with a DPP row broadcast feeds it to every lane, so activations
// cost no LDS traffic and no extra VALU moves.  Q4_K reads activations with scalar loads.
// With S > 1 waves per workgroup the K range is split round-robin in rounds of
// S*U blocks: each wave writes its per-block terms to LDS and the chain threads
// (lane = row, wave = token group) add them in block order.  int32 dots are exact,
// every float op is IEEE with no contraction.
#include <cstdlib>
#include <utility>

#include <hip/hip_ext.h>

#include "nc_device.h"
#include "nc_internal.h"

namespace nc {

typedef const int __attribute__((address_space(4)))* sptr_i32;
typedef const float __attribute__((address_space(4)))* sptr_f32;

template <typename T>
__device__ __forceinline__ sptr_i32 as_scalar_i32(const T* p) {
    return (sptr_i32)(const void __attribute__((address_space(4)))*)(uintptr_t)p;
}
template <typename T>
__device__ __forceinline__ sptr_f32 as_scalar_f32(const T* p) {
    return (sptr_f32)(const void __attribute__((address_space(4)))*)(uintptr_t)p;
}

__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// ---------------------------------------------------------------- epilogues
// Thread (wave w, lane l) owns row 64*tile + l and tokens n = w + j*S.
template <int NMAX, int S>
__device__ __forceinline__ void gemm_epilogue(const GemmParams& p, const float* acc, int tile, int wave, int lane) {
    constexpr int TPW = (NMAX + S - 1) / S;
    const int row = tile * kTileRows + lane;
#pragma unroll
    for (int j = 0; j < TPW; j++) {
        const int n = wave + j * S;
        if (n >= p.N) break;  // wave-uniform
        float v = acc[j];
        switch (p.epi) {
            case EPI_STORE:
                if (row < p.M) p.out[(size_t)n * p.ld_out + row] = v;
                break;
            case EPI_RESIDUAL:
                // hidden = matmul; hidden += residual (inference.rs:3985, 4073; add_residual_batch :4122)
                if (row < p.M) {
                    float* o = p.out + (size_t)n * p.ld_out + row;
                    *o = v + *o;
                }
                break;
            case EPI_QKV_ROPE: {
                // inference.rs:3894-3924: RoPE on q and k rows (NORM pairs 2i, 2i+1 are
                // adjacent lanes), then q to the q buffer and k, v to the KV cache.
                const int pos = p.d_pos[0] + n;
                const int base = tile * kTileRows;  // tiles never straddle q/k/v
                const bool is_q = base < p.aw;
                const bool is_k = !is_q && base < p.aw + p.kw;
                const int rr = is_q ? row : (is_k ? row - p.aw : row - p.aw - p.kw);
                float partner = __shfl_xor(v, 1, 64);
                if (is_q || is_k) {
                    const int i = (rr % p.hd) >> 1;
                    if (i < p.rope_half) {
                        const float* sc = p.rope_tab + ((size_t)pos * p.rope_half + i) * 2;
                        const float s = sc[0], c = sc[1];
                        const float x0 = (lane & 1) ? partner : v;
                        const float x1 = (lane & 1) ? v : partner;
                        v = (lane & 1) ? (x0 * s + x1 * c) : (x0 * c - x1 * s);
                    }
                }
                if (is_q) {
                    p.q_out[(size_t)n * p.aw + rr] = v;
                } else {
                    const int kvh = rr / p.hd, d = rr % p.hd;
                    if (is_k) p.kcache[(((size_t)kvh * (p.hd / 4) + d / 4) * p.max_ctx + pos) * 4 + (d & 3)] = v;
                    else p.vcache[(((size_t)kvh * (p.max_ctx / 4) + pos / 4) * p.hd + d) * 4 + (pos & 3)] = v;
                }
                break;
            }
            case EPI_SWIGLU_Q8: {
                // Interleaved tile: lanes 0..31 gate rows f = 32*tile + l, lanes 32..63 the up rows.
                // fused_silu_mul (inference.rs:3367-3390) then quantize_f32_to_q8_0 of the
                // 32-wide block f = 32*tile .. +31 (inference.rs:4034-4041).
                float up = __shfl(v, (lane & 31) + 32, 64);
                float g = v;
                float sig = 1.0f / (1.0f + expf_glibc(-g));
                float y = g * sig * up;
                float amax = halfwave_amax(y);
                float scale;
                int q = quantize_lane_q8(y, amax, &scale);
                int qs = halfwave_isum(q);
                if (lane < 32) {
                    const int f = tile * 32 + lane;
                    p.xq_out[(size_t)n * p.F + f] = (int8_t)q;
                    if (lane == 0) {
                        p.xs_out[(size_t)n * (p.F / 32) + tile] = scale;
                        p.xs8_out[(size_t)n * (p.F / 32) + tile] = -8 * qs;
                    }
                }
                break;
            }
            case EPI_HEAD: {
                // logits row + first-max argmax partial of this tile (inference.rs:4836-4846).
                if (row < p.M) p.out[(size_t)n * p.ld_out + row] = v;
                float bv = row < p.M ? v : -__builtin_inff();
                int bi = row < p.M ? row : 0x7fffffff;
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) {
                    float ov = __shfl_xor(bv, off, 64);
                    int oi = __shfl_xor(bi, off, 64);
                    if (ov > bv || (ov == bv && oi < bi)) {
                        bv = ov;
                        bi = oi;
                    }
                }
                if (lane == 0) {
                    p.part_val[(size_t)n * p.ntiles + tile] = bv;
                    p.part_idx[(size_t)n * p.ntiles + tile] = bi;
                }
                break;
            }
        }
    }
}

// ---------------------------------------------------------------- Q4_0
// Activation delivery by DPP row broadcast.  For block b, each row of 16 lanes loads the
// 16 dwords {x[2p][b] (8 dwords), x[2p+1][b] (8 dwords)} of token pair p (every row holds
// the same 64 bytes, one global_load_dword per lane), and one "meta" dword per lane:
// lane j < 8 holds x_scale[j][b], lane 8 + j holds -8 * sum(x[j][b]) (tokens 8q..8q+7).
// v_dot4c_i32_i8 with DPP row_newbcast:j reads lane j of each row as its src0, so the
// activation dword reaches every lane without scalar loads, LDS, or extra VALU moves.

// 8 int8 dot4 steps of one (block, token): acc += sum_i dot4(x dword (J0 + i), w_i).
// The leading s_nop covers the VALU-write -> DPP-read hazard in case the compiler
// materialised the activation register with a VALU move.  The trailing s_nop 2 covers
// the DOT-write -> other-VALU-read hazard (3 wait states on gfx950): the compiler's
// hazard recognizer cannot see inside the asm, and without it the first consumer of the
// result reads the accumulator as it was two dot4c steps earlier.
template <int J0>
__device__ __forceinline__ int dot32_bcast(int acc, int xp, int w0, int w1, int w2, int w3, int w4, int w5, int w6,
                                           int w7) {
    asm("s_nop 1\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %2 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %3 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %4 row_newbcast:%12 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %5 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %6 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %7 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %8 row_newbcast:%16 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %1, %9 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 2"
        : "+v"(acc)
        : "v"(xp), "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(w4), "v"(w5), "v"(w6), "v"(w7), "n"(J0), "n"(J0 + 1),
          "n"(J0 + 2), "n"(J0 + 3), "n"(J0 + 4), "n"(J0 + 5), "n"(J0 + 6), "n"(J0 + 7));
    return acc;
}

template <int J>
__device__ __forceinline__ int bcast_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, 0x150 + J, 0xf, 0xf, false);
}
template <int J>
__device__ __forceinline__ float bcast_f(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x150 + J, 0xf, 0xf, false));
}

// Two tokens of a pair (2p, 2p+1) share the activation register xp: their 8-step chains
// are interleaved (acc0 reads lanes 0..7 of each row, acc1 lanes 8..15) so that each
// dot4c's dependency on its own accumulator is hidden behind the other chain.
// The scale products are folded into the same asm: besides the two dot chains, c0 = x_scale[n0] * ws and c1 = x_scale[n1] * ws, each one
// v_mul_f32_dpp that reads the token's x_scale from lane X0 / X1 of the meta dword (the same
// IEEE product as a broadcast followed by a multiply).  The leading s_nop covers a VALU write
// of meta or xp just before the asm.
template <int X0, int X1>
__device__ __forceinline__ void dot32_bcast_pair_scaled(int& acc0, int& acc1, float& c0, float& c1, int xp, int meta,
                                                        float ws, int w0, int w1, int w2, int w3, int w4, int w5,
                                                        int w6, int w7) {
    asm("s_nop 1\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %7 row_newbcast:0 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %7 row_newbcast:8 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %8 row_newbcast:1 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %8 row_newbcast:9 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %9 row_newbcast:2 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %9 row_newbcast:10 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %10 row_newbcast:3 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %10 row_newbcast:11 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %11 row_newbcast:4 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %11 row_newbcast:12 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %12 row_newbcast:5 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %12 row_newbcast:13 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %13 row_newbcast:6 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %13 row_newbcast:14 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %6, %14 row_newbcast:7 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %1, %6, %14 row_newbcast:15 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %2, %4, %5 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %3, %4, %5 row_newbcast:%16 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 2"
        : "+v"(acc0), "+v"(acc1), "=&v"(c0), "=&v"(c1)
        : "v"(meta), "v"(ws), "v"(xp), "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(w4), "v"(w5), "v"(w6), "v"(w7),
          "n"(X0), "n"(X1));
}

// One token's dot chain with its scale product folded in: c = x_scale (lane X of meta) * ws.
template <int J0, int X>
__device__ __forceinline__ int dot32_bcast_scaled(int acc, float& c, int xp, int meta, float ws, int w0, int w1, int w2,
                                                  int w3, int w4, int w5, int w6, int w7) {
    asm("s_nop 1\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %5 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %6 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %7 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %8 row_newbcast:%16 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %9 row_newbcast:%17 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %10 row_newbcast:%18 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %11 row_newbcast:%19 row_mask:0xf bank_mask:0xf\n\t"
        "v_dot4c_i32_i8_dpp %0, %4, %12 row_newbcast:%20 row_mask:0xf bank_mask:0xf\n\t"
        "v_mul_f32_dpp %1, %2, %3 row_newbcast:%21 row_mask:0xf bank_mask:0xf\n\t"
        "s_nop 2"
        : "+v"(acc), "=&v"(c)
        : "v"(meta), "v"(ws), "v"(xp), "v"(w0), "v"(w1), "v"(w2), "v"(w3), "v"(w4), "v"(w5), "v"(w6), "v"(w7),
          "n"(J0), "n"(J0 + 1), "n"(J0 + 2), "n"(J0 + 3), "n"(J0 + 4), "n"(J0 + 5), "n"(J0 + 6), "n"(J0 + 7), "n"(X));
    return acc;
}

// Term of token n (compile-time) for one block: t = (ws * xs) * (float)sum (nib - 8) * x.
template <int n>
__device__ __forceinline__ float term_q40(const int* xp, const int* meta, const int (&lo)[4], const int (&hi)[4],
                                          float ws) {
    int d = bcast_i<8 + (n & 7)>(meta[n >> 3]);  // -8 * sum x: sum (nib-8)*x = sum nib*x - 8 sum x
    float c;                                       // x_scale * ws (IEEE product, commutative)
    d = dot32_bcast_scaled<8 * (n & 1), n & 7>(d, c, xp[n >> 1], meta[n >> 3], ws, lo[0], lo[1], lo[2], lo[3], hi[0],
                                                hi[1], hi[2], hi[3]);
    return c * (float)d;  // == (ws * xs) * d
}

// R64: a ring of D rounds of weights, scales and activations is kept in flight per wave.
// NMAX is the batch width itself for N <= 9.  With S > 1 the terms go to a double-
// buffered LDS array, one barrier per round, and the chain threads add them in block order.
// Terms of all NMAX tokens of one block (token pairs through dot32_bcast_pair).
template <int NMAX>
__device__ __forceinline__ void terms_q40(float (&t)[NMAX], const int* xp, const int* meta, const int (&lo)[4],
                                          const int (&hi)[4], float ws) {
    [&]<int... P>(std::integer_sequence<int, P...>) {
        (([&] {
             constexpr int n0 = 2 * P, n1 = 2 * P + 1;
             if constexpr (n1 < NMAX) {
                 int d0 = bcast_i<8 + (n0 & 7)>(meta[n0 >> 3]);
                 int d1 = bcast_i<8 + (n1 & 7)>(meta[n1 >> 3]);
                 float c0, c1;  // x_scale * ws (meta[n0 >> 3] == meta[n1 >> 3]: n0, n1 differ in bit 0)
                 dot32_bcast_pair_scaled<n0 & 7, n1 & 7>(d0, d1, c0, c1, xp[P], meta[n0 >> 3], ws, lo[0], lo[1],
                                                         lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]);
                 t[n0] = c0 * (float)d0;
                 t[n1] = c1 * (float)d1;
             } else {
                 t[n0] = term_q40<n0>(xp, meta, lo, hi, ws);
             }
         }()),
         ...);
    }(std::make_integer_sequence<int, (NMAX + 1) / 2>{});
}

template <int NMAX, int S, int D>
__global__ __launch_bounds__(64 * S) void gemm_q4_0_kernel(GemmParams p) {
    constexpr int U = 4;                       // blocks per wave per round
    constexpr int RB = S * U;                  // blocks per round
    constexpr int TPW = (NMAX + S - 1) / S;    // chain tokens per thread
    constexpr int NP = (NMAX + 1) / 2;         // token-pair activation dwords per block
    constexpr int NM = (NMAX + 7) / 8;         // meta dwords per block
    extern __shared__ float lds[];             // [2][RB][NMAX][64] terms when S > 1
    const int tile = blockIdx.x;
    const int wave = wave_id_uniform();
    const int lane = threadIdx.x & 63;
    const int j16 = lane & 15;
    const int N = p.N;
    const int nb = p.units;
    const uint8_t* wt = p.w + (size_t)tile * p.groups * kQ40ChunkBytes;
    float acc[TPW];
#pragma unroll
    for (int t = 0; t < TPW; t++) acc[t] = 0.0f;
    // per-lane activation addresses: pair q -> token 2q + (j16 >> 3), dword j16 & 7;
    // meta: lanes 0..7 read x_scale, lanes 8..15 read -8*sum(x) of token 8q + (j16 & 7)
    const int* xbase = (const int*)p.x + (j16 & 7);
    const int xtok = j16 >> 3;
    const int mtok = j16 & 7;
    const int* mbase = j16 >= 8 ? p.xs8 : (const int*)p.xs;
    const int nrounds = (nb + RB - 1) / RB;

    uint4 rw[D][U];
    uint2 rs[D];
    int rx[D][U][NP], rm[D][U][NM];
    // Loads are issued unconditionally (indices clamped into the padded matrix, data past the
    // end is never used): straight-line load sequences keep the compiler's wait counts exact,
    // so consuming one ring slot never drains the slots still in flight.
    const int bmax = 8 * p.groups - U;  // last round start inside the padded groups (U | 8)
#define NC_R64_LOAD(R, SLOT)                                                                        \
    do {                                                                                            \
        const int b0_ = min(min((R), nrounds - 1) * RB + wave * U, bmax);                           \
        const uint8_t* chunk_ = wt + (size_t)(b0_ >> 3) * kQ40ChunkBytes;                           \
        const int u0_ = b0_ & 7;                                                                    \
        _Pragma("unroll") for (int u = 0; u < U; u++) rw[SLOT][u] =                                 \
            *(const uint4*)(chunk_ + (u0_ + u) * 1024 + lane * 16);                                 \
        rs[SLOT] = *(const uint2*)(chunk_ + 8192 + (u0_ >> 2) * 512 + lane * 8);                    \
        _Pragma("unroll") for (int u = 0; u < U; u++) {                                             \
            const int b_ = min(b0_ + u, nb - 1);                                                    \
            _Pragma("unroll") for (int q = 0; q < NP; q++) {                                        \
                const int t_ = min(2 * q + xtok, N - 1);                                            \
                rx[SLOT][u][q] = xbase[((size_t)t_ * p.K + (size_t)b_ * 32) / 4];                   \
            }                                                                                       \
            _Pragma("unroll") for (int q = 0; q < NM; q++) {                                        \
                const int t_ = min(8 * q + mtok, N - 1);                                            \
                rm[SLOT][u][q] = mbase[(size_t)t_ * nb + b_];                                       \
            }                                                                                       \
        }                                                                                           \
    } while (0)

#pragma unroll
    for (int k = 0; k < D - 1; k++) NC_R64_LOAD(k, k);
    for (int r0 = 0; r0 < nrounds; r0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0 + k;
            NC_R64_LOAD(r + D - 1, (k + D - 1) % D);
            if (r < nrounds) {  // uniform
                float* buf = lds + (size_t)(r & 1) * RB * NMAX * 64;
                const int b0 = r * RB + wave * U;
#pragma unroll
                for (int u = 0; u < U; u++) {
                    if (b0 + u < nb) {  // uniform
                        const uint4 v = rw[k][u];
                        const int lo[4] = {(int)(v.x & 0x0F0F0F0Fu), (int)(v.y & 0x0F0F0F0Fu),
                                           (int)(v.z & 0x0F0F0F0Fu), (int)(v.w & 0x0F0F0F0Fu)};
                        const int hi[4] = {(int)((v.x >> 4) & 0x0F0F0F0Fu), (int)((v.y >> 4) & 0x0F0F0F0Fu),
                                           (int)((v.z >> 4) & 0x0F0F0F0Fu), (int)((v.w >> 4) & 0x0F0F0F0Fu)};
                        const uint32_t sw = u < 2 ? rs[k].x : rs[k].y;
                        const float ws = f16_to_f32((uint16_t)((u & 1) ? (sw >> 16) : (sw & 0xffff)));
                        // every token of the instantiation, without branches (tokens >= N read
                        // clamped activations and are never stored): straight-line code keeps
                        // the load wait counts precise
                        float t[NMAX];
                        terms_q40<NMAX>(t, rx[k][u], rm[k][u], lo, hi, ws);
#pragma unroll
                        for (int n = 0; n < NMAX; n++) {
                            if constexpr (S == 1) acc[n] = acc[n] + t[n];
                            else buf[((wave * U + u) * NMAX + n) * 64 + lane] = t[n];
                        }
                    }
                }
                if constexpr (S > 1) {
                    __syncthreads();
                    const int nblk = min(RB, nb - r * RB);
#pragma unroll
                    for (int t = 0; t < TPW; t++) {
                        const int n = wave + t * S;
                        if (n < N) {
                            float a = acc[t];
                            const float* src = buf + n * 64 + lane;
                            int bl = 0;
                            for (; bl + 8 <= nblk; bl += 8) {
                                float v[8];
#pragma unroll
                                for (int i = 0; i < 8; i++) v[i] = src[(bl + i) * NMAX * 64];
#pragma unroll
                                for (int i = 0; i < 8; i++) a = a + v[i];
                            }
                            for (; bl < nblk; bl++) a = a + src[bl * NMAX * 64];
                            acc[t] = a;
                        }
                    }
                }
            }
        }
    }
#undef NC_R64_LOAD
    gemm_epilogue<NMAX, S>(p, acc, tile, wave, lane);
}

// ---------------------------------------------------------------- Q8_0 (64-row tiles)
// matmul_q8_0_batch (inference.rs:1343-1383): per row and token, sum += ws * xs * dot over the
// 32-blocks in order, dot = the signed int8 block dot (dot_i8_scalar, q8.rs:3376-3382), ws the
// block's f16 scale.  Lane l owns row 64*tile + l; in round r wave w takes block r*S + w (its
// 32 weight bytes as two 16-byte loads, its scale); the token's 32 activation bytes and x_scale
// are wave-uniform, read as scalar loads.  Terms of the S blocks of a round go through a
// double-buffered LDS array and are added in block order by the chain threads (thread
// (w, l): tokens w, w + S, ...), one barrier per round; the epilogues are the 64-row ones.
template <int NMAX, int S>
__global__ __launch_bounds__(64 * S) void gemm_q8_0_kernel(GemmParams p) {
    constexpr int TPW = (NMAX + S - 1) / S;  // chain tokens per thread
    constexpr int D = 2;                      // ring of rounds in flight
    extern __shared__ float lds[];            // [2][S][NMAX][64] terms when S > 1
    const int tile = blockIdx.x;
    const int wave = wave_id_uniform();
    const int lane = threadIdx.x & 63;
    const int N = p.N, nb = p.units;
    const uint8_t* wt = p.w + (size_t)tile * p.groups * kQ80ChunkBytes;
    const int nrounds = (nb + S - 1) / S;
    float acc[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) acc[j] = 0.0f;
    uint4 rw[D][2];
    uint32_t rs[D];
    // loads are unconditional, with the block index clamped into the row (a clamped block's
    // term is never added)
#define NC_Q80_LOAD(R, SLOT)                                                                       \
    do {                                                                                           \
        const int b_ = min(min((R), nrounds - 1) * S + wave, nb - 1);                              \
        const uint8_t* c_ = wt + (size_t)(b_ / kQ80GroupBlocks) * kQ80ChunkBytes;                  \
        const int u_ = b_ % kQ80GroupBlocks;                                                       \
        rw[SLOT][0] = *(const uint4*)(c_ + (2 * u_) * 1024 + lane * 16);                           \
        rw[SLOT][1] = *(const uint4*)(c_ + (2 * u_ + 1) * 1024 + lane * 16);                       \
        rs[SLOT] = *(const uint16_t*)(c_ + kQ80GroupBlocks * 2048 + u_ * 128 + lane * 2);          \
    } while (0)
    NC_Q80_LOAD(0, 0);
    for (int r0 = 0; r0 < nrounds; r0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0 + k;
            if (r >= nrounds) break;  // uniform
            NC_Q80_LOAD(r + 1, (k + 1) % D);
            const int b = r * S + wave;
            float* buf = lds + (size_t)(r & 1) * S * NMAX * 64;
            if (b < nb) {  // uniform
                const float ws = f16_to_f32((uint16_t)rs[k]);
                const int wv[8] = {(int)rw[k][0].x, (int)rw[k][0].y, (int)rw[k][0].z, (int)rw[k][0].w,
                                   (int)rw[k][1].x, (int)rw[k][1].y, (int)rw[k][1].z, (int)rw[k][1].w};
                float t[NMAX];
#pragma unroll
                for (int n = 0; n < NMAX; n++) {
                    // tokens >= N read the last token's activations and are never stored
                    const int nn = min(n, N - 1);
                    sptr_i32 xw = as_scalar_i32(p.x + (size_t)nn * p.K + (size_t)b * 32);
                    sptr_f32 xsp = as_scalar_f32(p.xs + (size_t)nn * nb + b);
                    int dot = 0;
#pragma unroll
                    for (int i = 0; i < 8; i++) dot = __builtin_amdgcn_sdot4(wv[i], xw[i], dot, false);
                    t[n] = ws * xsp[0] * (float)dot;
                }
#pragma unroll
                for (int n = 0; n < NMAX; n++) {
                    if constexpr (S == 1) acc[n] = acc[n] + t[n];
                    else buf[(wave * NMAX + n) * 64 + lane] = t[n];
                }
            }
            if constexpr (S > 1) {
                // buffer r & 1 is rewritten in round r + 2, after every thread passed round r + 1's
                // barrier
                __syncthreads();
                const int nblk = min(S, nb - r * S);
#pragma unroll
                for (int j = 0; j < TPW; j++) {
                    const int n = wave + j * S;
                    if (n < N) {
                        float a = acc[j];
                        for (int bl = 0; bl < nblk; bl++) a = a + buf[(bl * NMAX + n) * 64 + lane];
                        acc[j] = a;
                    }
                }
            }
        }
    }
#undef NC_Q80_LOAD
    gemm_epilogue<NMAX, S>(p, acc, tile, wave, lane);
}

// ---------------------------------------------------------------- Q4_0, 16-row tiles (R16)
// Workgroup = one 16-row tile, S waves.  A wave instruction covers one quad of blocks:
// lane = 16*j + r holds block 4*qd + j of row r, so each DPP row of 16 lanes is one block
// and its activation dwords / meta are broadcast inside the row exactly as above.  Rounds
// of S*U quads: wave w takes quads w*U .. w*U+U-1 of the round; a ring of D rounds of
// weights, scales and activations is kept in flight per wave.  Terms go to a double-
// buffered LDS array [round block][token][row]; after the round's barrier the chain
// threads (thread c: token c/16, row c%16) add them in block order.
template <int NMAX>
__device__ __forceinline__ void gemm_epilogue_r16(const GemmParams& p, float v, int n, int tile, int r) {
    const int row = tile * kTileRowsR16 + r;
    switch (p.epi) {
        case EPI_STORE:
            if (row < p.M) p.out[(size_t)n * p.ld_out + row] = v;
            break;
        case EPI_RESIDUAL:
            if (row < p.M) {
                float* o = p.out + (size_t)n * p.ld_out + row;
                *o = v + *o;
            }
            break;
        case EPI_QKV_ROPE: {
            // inference.rs:3894-3924 (see gemm_epilogue): pair rows 2i, 2i+1 are lanes r, r^1
            const int pos = p.d_pos[0] + n;
            const int base = tile * kTileRowsR16;
            const bool is_q = base < p.aw;
            const bool is_k = !is_q && base < p.aw + p.kw;
            const int rr = is_q ? row : (is_k ? row - p.aw : row - p.aw - p.kw);
            const float partner = __shfl_xor(v, 1, 64);
            if (is_q || is_k) {
                const int i = (rr % p.hd) >> 1;
                if (i < p.rope_half) {
                    const float* sc = p.rope_tab + ((size_t)pos * p.rope_half + i) * 2;
                    const float sn = sc[0], cs = sc[1];
                    const float x0 = (r & 1) ? partner : v;
                    const float x1 = (r & 1) ? v : partner;
                    v = (r & 1) ? (x0 * sn + x1 * cs) : (x0 * cs - x1 * sn);
                }
            }
            if (is_q) {
                p.q_out[(size_t)n * p.aw + rr] = v;
            } else {
                const int kvh = rr / p.hd, d = rr % p.hd;
                if (is_k) p.kcache[(((size_t)kvh * (p.hd / 4) + d / 4) * p.max_ctx + pos) * 4 + (d & 3)] = v;
                else p.vcache[(((size_t)kvh * (p.max_ctx / 4) + pos / 4) * p.hd + d) * 4 + (pos & 3)] = v;
            }
            break;
        }
        case EPI_HEAD: {
            // logits row + first-max argmax partial of this 16-row tile (inference.rs:4836-4846)
            if (row < p.M) p.out[(size_t)n * p.ld_out + row] = v;
            float bv = row < p.M ? v : -__builtin_inff();
            int bi = row < p.M ? row : 0x7fffffff;
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) {
                const float ov = __shfl_xor(bv, off, 64);
                const int oi = __shfl_xor(bi, off, 64);
                if (ov > bv || (ov == bv && oi < bi)) {
                    bv = ov;
                    bi = oi;
                }
            }
            if (r == 0) {
                p.part_val[(size_t)n * p.ntiles + tile] = bv;
                p.part_idx[(size_t)n * p.ntiles + tile] = bi;
            }
            break;
        }
        default:
            break;  // EPI_SWIGLU_Q8: the four-tile variant finishes it in its own epilogue
    }
}

// ---------------------------------------------------------------- R16 chain threads
// The block-ordered f32 chains of a 16-row tile: after each round's barrier, thread (token cn,
// row cr) adds that round's BR terms [BR][NMAX][16] of LDS buffer r & 1 in block order
// (inference.rs:1553-1573), so the sum is bit-identical to the reference's per-row loop.

// LDS floats per tile of a tile group: the double-buffered terms [2][BR][NMAX][16], padded by 16
// floats in four-tile groups so that a chain wave's four 16-lane rows (one per tile) read
// disjoint LDS banks (unpadded, the tiles' buffers sit a multiple of 64 banks apart).
template <int BR, int NMAX, int TPG>
constexpr int r16_tile_lds() {
    return 2 * BR * NMAX * 16 + (TPG > 1 ? 16 : 0);
}

// One round's chain step: adds the round's nblk terms of (token cn, row cr) in block order.
template <int NMAX, int BR>
__device__ __forceinline__ float r16_chain_step(const float* buf, int nblk, int cn, int cr, float acc) {
    const float* src = buf + cn * 16 + cr;
    // groups of 16 terms read ahead of their dependent adds
    int bl = 0;
    for (; bl + 16 <= nblk; bl += 16) {
        float v[16];
#pragma unroll
        for (int i = 0; i < 16; i++) v[i] = src[(bl + i) * NMAX * 16];
#pragma unroll
        for (int i = 0; i < 16; i++) acc = acc + v[i];
    }
    for (; bl < nblk; bl++) acc = acc + src[bl * NMAX * 16];
    return acc;
}

// Dedicated chain wave of a four-tile group, token cn: one barrier per round, then its step;
// lane = 16 * tile + row, so the wave holds the token's 32 gate and 32 up outputs and finishes
// SwiGLU and the Q8_0 block with shuffles.
template <int NMAX, int BR>
__device__ __forceinline__ void r16_chain_wave_tpg4(const GemmParams& p, const float* lds_all, int cn) {
    const int lane = threadIdx.x & 63;
    const int sub = lane >> 4, cr = lane & 15;
    const int nb = p.units;
    const int nrounds = ((nb + 3) / 4 + BR / 4 - 1) / (BR / 4);
    const bool active = cn < p.N;  // wave-uniform
    float acc = 0.0f;
    for (int r = 0; r < nrounds; r++) {
        __syncthreads();  // round r's terms are in buffer r & 1 of every tile
        if (active)
            acc = r16_chain_step<NMAX, BR>(lds_all + (size_t)sub * r16_tile_lds<BR, NMAX, 4>() + (r & 1) * BR * NMAX * 16,
                                           min(BR, nb - r * BR), cn, cr, acc);
    }
    if (active) {
        // EPI_SWIGLU_Q8 (fused_silu_mul inference.rs:3367-3390, then quantize_f32_to_q8_0 of
        // the 32-wide block, inference.rs:4034-4041): lanes 0-31 gate, 32-63 up
        const int l = lane & 31;
        const float g = __shfl(acc, l, 64);
        const float up = __shfl(acc, 32 + l, 64);
        const float sig = 1.0f / (1.0f + expf_glibc(-g));
        const float y = g * sig * up;
        const float amax = halfwave_amax(y);
        float scale;
        const int q = quantize_lane_q8(y, amax, &scale);
        const int qs = halfwave_isum(q);
        if (lane < 32) {
            const int blk = blockIdx.x;
            p.xq_out[(size_t)cn * p.F + blk * 32 + lane] = (int8_t)q;
            if (lane == 0) {
                p.xs_out[(size_t)cn * (p.F / 32) + blk] = scale;
                p.xs8_out[(size_t)cn * (p.F / 32) + blk] = -8 * qs;
            }
        }
    }
}

// Dedicated chain wave(s) of a one-tile group with S term waves: chain thread c = (token
// c / 16, row c % 16).
template <int NMAX, int BR, int S>
__device__ __forceinline__ void r16_chain_wave_tpg1(const GemmParams& p, const float* lds_all) {
    const int c = threadIdx.x - 64 * S;
    const int cn = c >> 4, cr = c & 15;
    const int nb = p.units;
    const int nrounds = ((nb + 3) / 4 + BR / 4 - 1) / (BR / 4);
    const bool active = c < 16 * NMAX && cn < p.N;
    float acc = 0.0f;
    for (int r = 0; r < nrounds; r++) {
        __syncthreads();  // round r's terms are in buffer r & 1
        if (active) acc = r16_chain_step<NMAX, BR>(lds_all + (size_t)(r & 1) * BR * NMAX * 16, min(BR, nb - r * BR),
                                                   cn, cr, acc);
    }
    if (active) gemm_epilogue_r16<NMAX>(p, acc, cn, blockIdx.x, cr);
}

// EPI_SWIGLU_Q8 of a four-tile group whose chains ran on the term waves: rows 0-31 gate,
// 32-63 up of output block blockIdx.x (fused_silu_mul inference.rs:3367-3390, then
// quantize_f32_to_q8_0 of the 32-wide block, inference.rs:4034-4041).
template <int NMAX>
__device__ __forceinline__ void r16_swiglu_epilogue(const GemmParams& p, float* lds_all, bool chain, int sub, int cn,
                                                    int cr, float acc, int wave_all) {
    float* outv = lds_all;  // [64 rows][NMAX]
    __syncthreads();        // every chain has read its last round's terms
    if (chain) outv[(sub * 16 + cr) * NMAX + cn] = acc;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int n = wave_all;  // one wave per token, lanes 0-31 = the 32 outputs
    if (n < p.N) {
        const int l = lane & 31;
        const float g = outv[l * NMAX + n];
        const float up = outv[(32 + l) * NMAX + n];
        const float sig = 1.0f / (1.0f + expf_glibc(-g));
        const float y = g * sig * up;
        const float amax = halfwave_amax(y);
        float scale;
        const int q = quantize_lane_q8(y, amax, &scale);
        const int qs = halfwave_isum(q);
        if (lane < 32) {
            const int blk = blockIdx.x;
            p.xq_out[(size_t)n * p.F + blk * 32 + lane] = (int8_t)q;
            if (lane == 0) {
                p.xs_out[(size_t)n * (p.F / 32) + blk] = scale;
                p.xs8_out[(size_t)n * (p.F / 32) + blk] = -8 * qs;
            }
        }
    }
}

// TPG = 4: one workgroup covers four consecutive tiles (64 rows) with a group of S waves
// each, sharing the per-round barrier; used for the interleaved gate,up matrix, whose 64-row
// groups hold 32 gate rows and the 32 matching up rows, so that SwiGLU and the Q8_0
// quantisation of the 32-wide output block finish inside the workgroup.
//
// CW > 0: the chain threads are CW extra waves that only add terms, so the term-computing
// waves carry no chain work.  A wave issues one VALU instruction per 8 cycles at most, so
// chain work placed on a computing wave lengthens that wave's round by its BR dependent adds
// and their LDS reads, and every round's barrier waits for it.  TPG = 1: chain thread c of
// the extra waves is (token c / 16, row c % 16).  TPG = 4: one chain wave per token (CW =
// NMAX), lane = 16 * tile + row, so the wave holds the token's 32 gate and 32 up outputs and
// finishes SwiGLU and the Q8_0 block with shuffles.
template <int NMAX, int S, int U, int D, int TPG, int CW = 0>
__global__ __launch_bounds__(64 * (S * TPG + CW)) void gemm_q4_0_r16_kernel(GemmParams p) {
    static_assert(CW > 0 ? 16 * NMAX <= 64 * CW : 16 * NMAX <= 64 * S, "chain threads must fit their waves");
    static_assert(U == 1 || U == 2 || U == 4, "quads per wave per round");
    static_assert(TPG == 1 || TPG == 4, "tiles per workgroup");
    static_assert(CW == 0 || TPG == 1 || CW == NMAX, "four-tile groups: one chain wave per token");
    constexpr int QR = S * U;                // quads per round
    constexpr int BR = 4 * QR;               // blocks per round
    constexpr int NP = (NMAX + 1) / 2;       // token-pair activation dwords per block
    constexpr int NM = (NMAX + 7) / 8;       // meta dwords per block
    extern __shared__ float lds_all[];       // per tile group: [2][BR][NMAX][16]
    const int wave_all = wave_id_uniform();
    if constexpr (CW > 0 && TPG == 4) {
        if (wave_all >= S * TPG) {  // chain wave of token wave_all - S * TPG
            r16_chain_wave_tpg4<NMAX, BR>(p, lds_all, wave_all - S * TPG);
            return;
        }
    }
    if constexpr (CW > 0 && TPG == 1) {
        if (wave_all >= S) {  // dedicated chain wave
            r16_chain_wave_tpg1<NMAX, BR, S>(p, lds_all);
            return;
        }
    }
    const int sub = wave_all / S;            // tile of the group (TPG = 4)
    const int wave = wave_all % S;
    const int tile = blockIdx.x * TPG + sub;
    float* lds = lds_all + (size_t)sub * r16_tile_lds<BR, NMAX, TPG>();
    const int tig = threadIdx.x - sub * 64 * S;  // thread index within the tile's group
    const int lane = threadIdx.x & 63;
    const int j = lane >> 4, i16 = lane & 15;
    const int N = p.N, nb = p.units;
    const int nq = (nb + 3) / 4;
    const uint8_t* wt = p.w + (size_t)tile * p.groups * kQ40ChunkBytes;
    const int xtok = i16 >> 3, mtok = i16 & 7;
    const int nrounds = (nq + QR - 1) / QR;

    uint4 rw[D][U];
    uint32_t rs[D][U];
    int rx[D][U][NP], rm[D][U][NM];
    // Unconditional loads (see the R64 kernel): exact wait counts across the ring.  Weights
    // and activations are buffer loads.  The weight chunk offset is wave-uniform (scalar) and
    // clamped to the padded groups; activations (and block scales on the buffer path) take a
    // per-lane 32-bit offset that is range-checked against the real [N][K] / [N][K/32]
    // extents, so a token past N or a block past the last row reads 0 instead of being
    // clamped (those terms are never added).
    const int qmax = 8 * p.groups - U;  // last wave-round start inside the padded groups (U | 8)
    const __amdgpu_buffer_rsrc_t wres =
        __builtin_amdgcn_make_buffer_rsrc((void*)wt, 0, p.groups * kQ40ChunkBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, N * p.K, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs, 0, N * nb * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t s8res = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs8, 0, N * nb * 4, 0x00020000);
    // a quad's nibbles, then its 64 scales ([row / 4][block][row % 4]: this lane's is (j, i16))
    const int wvo = lane * 16, svo = 2 * (16 * (i16 >> 2) + 4 * j + (i16 & 3));
    int xvo[NP], mvo[NM], mt[NM];
#pragma unroll
    for (int q = 0; q < NP; q++) xvo[q] = (2 * q + xtok) * p.K + 32 * j + 4 * (i16 & 7);
#pragma unroll
    for (int q = 0; q < NM; q++) {
        mvo[q] = ((8 * q + mtok) * nb + j) * 4;
        mt[q] = min(8 * q + mtok, N - 1);
    }
    // Block scales: lanes 0-7 of a row take xs, lanes 8-15 xs8.  For 3..8 rows two buffer
    // loads and a select measured faster than one load through a per-lane pointer; for
    // other widths the single clamped load is faster.
    constexpr bool kMetaBuf = NMAX >= 3 && NMAX <= 8;
    const bool meta_s = i16 < 8;
    const int* mbase = meta_s ? (const int*)p.xs : p.xs8;
#define NC_R16_LOAD(R, SLOT)                                                                         \
    do {                                                                                             \
        const int qd0_ = min(min((R), nrounds - 1) * QR + wave * U, qmax);                           \
        const int cb_ = (qd0_ >> 3) * kQ40ChunkBytes;                                                \
        _Pragma("unroll") for (int u = 0; u < U; u++) {                                              \
            const int qo_ = cb_ + ((qd0_ + u) & 7) * kQ40R16QuadBytes;                               \
            rw[SLOT][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wvo, qo_, 0)); \
            rs[SLOT][u] = __builtin_amdgcn_raw_buffer_load_b16(wres, svo, qo_ + 1024, 0);            \
        }                                                                                            \
        _Pragma("unroll") for (int u = 0; u < U; u++) {                                              \
            _Pragma("unroll") for (int q = 0; q < NP; q++) rx[SLOT][u][q] = (int)                     \
                __builtin_amdgcn_raw_buffer_load_b32(xres, xvo[q] + 128 * (qd0_ + u), 0, 0);         \
            _Pragma("unroll") for (int q = 0; q < NM; q++) {                                         \
                if constexpr (kMetaBuf) {                                                            \
                    const int mo_ = mvo[q] + 16 * (qd0_ + u);                                        \
                    const int ms_ = (int)__builtin_amdgcn_raw_buffer_load_b32(sres, mo_, 0, 0);      \
                    const int m8_ = (int)__builtin_amdgcn_raw_buffer_load_b32(s8res, mo_, 0, 0);     \
                    rm[SLOT][u][q] = meta_s ? ms_ : m8_;                                             \
                } else {                                                                             \
                    const int b_ = min(4 * (qd0_ + u) + j, nb - 1);                                  \
                    rm[SLOT][u][q] = mbase[(size_t)mt[q] * nb + b_];                                 \
                }                                                                                    \
            }                                                                                        \
        }                                                                                            \
    } while (0)

#pragma unroll
    for (int k = 0; k < D - 1; k++) NC_R16_LOAD(k, k);
    float acc = 0.0f;
    const int cn = tig >> 4, cr = tig & 15;  // chain thread: token, row
    for (int r0 = 0; r0 < nrounds; r0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0 + k;
            NC_R16_LOAD(r + D - 1, (k + D - 1) % D);
            if (r < nrounds) {  // uniform
                float* buf = lds + (size_t)(r & 1) * BR * NMAX * 16;
                const int qd0 = r * QR + wave * U;
#pragma unroll
                for (int u = 0; u < U; u++) {
                    if (qd0 + u < nq) {  // uniform
                        const uint4 v = rw[k][u];
                        const int lo[4] = {(int)(v.x & 0x0F0F0F0Fu), (int)(v.y & 0x0F0F0F0Fu),
                                           (int)(v.z & 0x0F0F0F0Fu), (int)(v.w & 0x0F0F0F0Fu)};
                        const int hi[4] = {(int)((v.x >> 4) & 0x0F0F0F0Fu), (int)((v.y >> 4) & 0x0F0F0F0Fu),
                                           (int)((v.z >> 4) & 0x0F0F0F0Fu), (int)((v.w >> 4) & 0x0F0F0F0Fu)};
                        const float ws = f16_to_f32((uint16_t)rs[k][u]);
                        float* dst = buf + ((size_t)((wave * U + u) * 4 + j) * NMAX) * 16 + i16;
                        float t[NMAX];
                        terms_q40<NMAX>(t, rx[k][u], rm[k][u], lo, hi, ws);
#pragma unroll
                        for (int n = 0; n < NMAX; n++) dst[n * 16] = t[n];
                    }
                }
                __syncthreads();
                if (CW == 0 && tig < 16 * NMAX && cn < N) acc = r16_chain_step<NMAX, BR>(buf, min(BR, nb - r * BR), cn, cr, acc);
            }
        }
    }
#undef NC_R16_LOAD
    if constexpr (TPG == 1) {
        if (CW == 0 && tig < 16 * NMAX && cn < N) gemm_epilogue_r16<NMAX>(p, acc, cn, tile, cr);
    } else if constexpr (CW == 0) {
        r16_swiglu_epilogue<NMAX>(p, lds_all, tig < 16 * NMAX && cn < N, sub, cn, cr, acc, wave_all);
    }
}

// ---------------------------------------------------------------- Q4_0, 16-row tiles, int8 MFMA
// Same tiles, rounds, LDS term buffers, chain threads and epilogues as gemm_q4_0_r16_kernel; the
// per-block int32 dots come from v_mfma_i32_16x16x32_i8 instead of v_dot4c:
//   A (16 x 32, weights): lane (g, r) holds row r's K subset g = nibble bytes 4g..4g+3 of the
//     block, i.e. weights 4g..4g+3 (low nibbles) and 16+4g..16+4g+3 (high nibbles);
//   B (32 x 16, activations): lane (g, c) holds token c's x[4g..4g+3] and x[16+4g..16+4g+3];
//   C = -8 * sum(x) of (token c, block), so D = sum (nib - 8) * x exactly (|D| <= 32512);
//   D lane (g, c) = token c, rows 4g..4g+3 (byte k of an A lane meets byte k of the B lane in
//     the same 16-lane group: measured, and covered by the bit-exact tests).
// Operands arrive compactly, each datum loaded once per wave: the quad's nibbles as before
// (lane (j, r) = block j of row r) and a 4x4 transpose of the 16-lane groups (two permlane32
// and two permlane16 swaps) gives lane (g, r) dword g of every block; token c's 128 activation
// bytes of the quad as two 16-byte pieces per lane plus the same transpose; one dword of the
// quad's 128 scale bytes per lane, and x_scale / -8*sum of (token, block) per lane, spread
// with ds_bpermute.  Each lane then forms 16 terms (4 rows x 4 blocks of its token), the
// reference's (w_scale * x_scale) * (float)dot.  One MFMA covers 16 tokens, so every width
// 1..16 costs the same.  Measured on the 8B shapes it is bit-exact but not faster than the
// v_dot4c kernel at any width (the round structure and operand delivery bound both), so the
// dispatch selects it only on request (nc_ctx_set_gemm_kernel).
typedef int nc_v4i __attribute__((ext_vector_type(4)));

// out register b of lane (g, x) = in register g of lane (b, x) (g, b: 16-lane groups)
__device__ __forceinline__ void rows_transpose4(uint32_t& r0, uint32_t& r1, uint32_t& r2, uint32_t& r3) {
    const auto p02 = __builtin_amdgcn_permlane32_swap(r0, r2, false, false);
    const auto p13 = __builtin_amdgcn_permlane32_swap(r1, r3, false, false);
    const auto q01 = __builtin_amdgcn_permlane16_swap(p02[0], p13[0], false, false);
    const auto q23 = __builtin_amdgcn_permlane16_swap(p02[1], p13[1], false, false);
    r0 = q01[0];
    r1 = q01[1];
    r2 = q23[0];
    r3 = q23[1];
}

template <int NMAX, int S, int D, int TPG, int CW>
__global__ __launch_bounds__(64 * (S * TPG + CW)) void gemm_q4_0_mfma_kernel(GemmParams p) {
    static_assert(CW > 0 ? 16 * NMAX <= 64 * CW : 16 * NMAX <= 64 * S, "chain threads must fit their waves");
    static_assert(TPG == 1 || TPG == 4, "tiles per workgroup");
    static_assert(CW == 0 || TPG == 1 || CW == NMAX, "four-tile groups: one chain wave per token");
    constexpr int QR = S;       // quads per round (one per term wave)
    constexpr int BR = 4 * QR;  // blocks per round
    extern __shared__ float lds_all[];  // per tile: [2][BR][NMAX][16] terms
    const int wave_all = wave_id_uniform();
    if constexpr (CW > 0 && TPG == 4) {
        if (wave_all >= S * TPG) {
            r16_chain_wave_tpg4<NMAX, BR>(p, lds_all, wave_all - S * TPG);
            return;
        }
    }
    if constexpr (CW > 0 && TPG == 1) {
        if (wave_all >= S) {
            r16_chain_wave_tpg1<NMAX, BR, S>(p, lds_all);
            return;
        }
    }
    const int sub = wave_all / S;  // tile of the group (TPG = 4)
    const int wave = wave_all % S;
    const int tile = blockIdx.x * TPG + sub;
    float* lds = lds_all + (size_t)sub * r16_tile_lds<BR, NMAX, TPG>();
    const int tig = threadIdx.x - sub * 64 * S;
    const int lane = threadIdx.x & 63;
    const int g = lane >> 4, c = lane & 15;
    const int N = p.N, nb = p.units;
    const int nq = (nb + 3) / 4;
    const uint8_t* wt = p.w + (size_t)tile * p.groups * kQ40ChunkBytes;
    const int nrounds = (nq + QR - 1) / QR;
    const int qmax = 8 * p.groups - 1;
    const __amdgpu_buffer_rsrc_t wres =
        __builtin_amdgcn_make_buffer_rsrc((void*)wt, 0, p.groups * kQ40ChunkBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, N * p.K, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs, 0, N * nb * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t s8res = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs8, 0, N * nb * 4, 0x00020000);
    const int wvo = lane * 16;
    const int svo = 1024 + 4 * (lane & 31);  // one dword of the quad's 128 scale bytes per lane
    const int xvo = c * p.K + 16 * g;        // token c's 16-byte piece g (and g + 4) of the quad
    const int mvo = (c * nb + g) * 4;        // x_scale / -8*sum of (token c, block g of the quad)
    // bpermute sources: scales dwords 8g..8g+7 (rows 4g..4g+3 of the 4 blocks), meta of (c, block b)
    const int sperm = 32 * g;                // byte address of lane 8g
    uint4 rw[D], rxa[D], rxb[D];
    uint32_t rs[D], rms[D], rm8[D];
#define NC_MF_LOAD(R, SLOT)                                                                          \
    do {                                                                                             \
        const int qd_ = min(min((R), nrounds - 1) * QR + wave, qmax);                                \
        const int qo_ = (qd_ >> 3) * kQ40ChunkBytes + (qd_ & 7) * kQ40R16QuadBytes;                  \
        rw[SLOT] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wvo, qo_, 0)); \
        rs[SLOT] = __builtin_amdgcn_raw_buffer_load_b32(wres, svo, qo_, 0);                          \
        rxa[SLOT] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, xvo + 128 * qd_, 0, 0)); \
        rxb[SLOT] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(xres, xvo + 128 * qd_ + 64, 0, 0)); \
        rms[SLOT] = __builtin_amdgcn_raw_buffer_load_b32(sres, mvo + 16 * qd_, 0, 0);               \
        rm8[SLOT] = __builtin_amdgcn_raw_buffer_load_b32(s8res, mvo + 16 * qd_, 0, 0);              \
    } while (0)
#pragma unroll
    for (int k = 0; k < D - 1; k++) NC_MF_LOAD(k, k);
    float acc = 0.0f;
    const int cn = tig >> 4, cr = tig & 15;  // chain thread: token, row
    for (int r0 = 0; r0 < nrounds; r0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0 + k;
            NC_MF_LOAD(r + D - 1, (k + D - 1) % D);
            if (r < nrounds) {  // uniform
                float* buf = lds + (size_t)(r & 1) * BR * NMAX * 16;
                if (r * QR + wave < nq) {  // uniform
                    uint32_t w0 = rw[k].x, w1 = rw[k].y, w2 = rw[k].z, w3 = rw[k].w;
                    rows_transpose4(w0, w1, w2, w3);  // wb = dword g of block b, row c
                    const uint32_t wb[4] = {w0, w1, w2, w3};
                    // activations: after the transposes, lane (g, c) holds dwords g and 4 + g of
                    // token c's blocks 0, 1 (from pieces 0..3) and 2, 3 (pieces 4..7)
                    uint32_t a0 = rxa[k].x, a1 = rxa[k].y, a2 = rxa[k].z, a3 = rxa[k].w;
                    uint32_t b0 = rxb[k].x, b1 = rxb[k].y, b2 = rxb[k].z, b3 = rxb[k].w;
                    rows_transpose4(a0, a1, a2, a3);
                    rows_transpose4(b0, b1, b2, b3);
                    const uint32_t xd[8] = {a0, a1, a2, a3, b0, b1, b2, b3};
                    // weight scales of rows 4g..4g+3 x 4 blocks: dwords 8g..8g+7 of the 128 bytes
                    uint32_t sw[8];
#pragma unroll
                    for (int i = 0; i < 8; i++)
                        sw[i] = (uint32_t)__builtin_amdgcn_ds_bpermute(sperm + 4 * i, (int)rs[k]);
#pragma unroll
                    for (int b = 0; b < 4; b++) {
                        const float xsb = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (16 * b + c), (int)rms[k]));
                        const int x8b = __builtin_amdgcn_ds_bpermute(4 * (16 * b + c), (int)rm8[k]);
                        const uint64_t a = (uint64_t)(wb[b] & 0x0F0F0F0Fu) |
                                           ((uint64_t)((wb[b] >> 4) & 0x0F0F0F0Fu) << 32);
                        const uint64_t bx = (uint64_t)xd[2 * b] | ((uint64_t)xd[2 * b + 1] << 32);
                        const nc_v4i cinit = {x8b, x8b, x8b, x8b};
                        const nc_v4i d = __builtin_amdgcn_mfma_i32_16x16x32_i8((long)a, (long)bx, cinit, 0, 0, 0);
                        float4 t;
                        t.x = (f16_to_f32((uint16_t)(sw[2 * b] & 0xffff)) * xsb) * (float)d[0];
                        t.y = (f16_to_f32((uint16_t)(sw[2 * b] >> 16)) * xsb) * (float)d[1];
                        t.z = (f16_to_f32((uint16_t)(sw[2 * b + 1] & 0xffff)) * xsb) * (float)d[2];
                        t.w = (f16_to_f32((uint16_t)(sw[2 * b + 1] >> 16)) * xsb) * (float)d[3];
                        if (c < NMAX) *(float4*)(buf + ((wave * 4 + b) * NMAX + c) * 16 + 4 * g) = t;
                    }
                }
                __syncthreads();
                if (CW == 0 && tig < 16 * NMAX && cn < N)
                    acc = r16_chain_step<NMAX, BR>(buf, min(BR, nb - r * BR), cn, cr, acc);
            }
        }
    }
#undef NC_MF_LOAD
    if constexpr (TPG == 1) {
        if (CW == 0 && tig < 16 * NMAX && cn < N) gemm_epilogue_r16<NMAX>(p, acc, cn, tile, cr);
    } else if constexpr (CW == 0) {
        r16_swiglu_epilogue<NMAX>(p, lds_all, tig < 16 * NMAX && cn < N, sub, cn, cr, acc, wave_all);
    }
}

// ---------------------------------------------------------------- Q4_K
// q8.rs:2008-2018 q4_k_scale_min on the 12 packed scale bytes held in three words.
__device__ __forceinline__ uint32_t kbyte(uint32_t w0, uint32_t w1, uint32_t w2, int i) {
    const uint32_t w = i < 4 ? w0 : (i < 8 ? w1 : w2);
    return (w >> ((i & 3) * 8)) & 0xff;
}

// Q5 = true: Q5_K super-blocks (q8.rs:1380-1397: slot 0 as Q4_K, slots 1-2 the 32 high-bit bytes,
// slots 3-10 the nibbles), chunks of 11 x 1 KB; a sub-block's 5-bit value is its nibble plus 16
// when bit 2*pair (low half) / 2*pair + 1 (high half) of qh[l] is set, and the term is the same
// xs_j * (sc_j * W_j - mn_j * A_j) (matmul_q5_k_batch's x86 path, q8.rs:1551-1594).
template <int NMAX, int S, int D, bool Q5 = false>
__global__ __launch_bounds__(64 * S) void gemm_q4_k_kernel(GemmParams p) {
    constexpr int NSLOT = Q5 ? 11 : 9;       // 16-byte slots per super-block and lane
    constexpr int QS = Q5 ? 3 : 1;           // first nibble slot
    constexpr int CHUNK = NSLOT * 1024;
    constexpr int TPW = (NMAX + S - 1) / S;  // chain tokens per thread
    extern __shared__ float lds[];           // [2][S][NMAX][64] super-block terms when S > 1
    const int tile = blockIdx.x;
    const int wave = wave_id_uniform();
    const int lane = threadIdx.x & 63;
    const int N = p.N;
    const int nsb = p.units;
    const int nb = nsb * 8;
    const uint8_t* wt = p.w + (size_t)tile * nsb * CHUNK + lane * 16;
    float acc[TPW];
#pragma unroll
    for (int j = 0; j < TPW; j++) acc[j] = 0.0f;
    // round r: wave w takes super-block r*S + w; a ring of D super-blocks (9 x 16 B per lane)
    // is in flight.  Loads are unconditional with clamped indices (straight-line load code
    // keeps the wait counts exact); a clamped super-block's term is never added.
    const int nrounds = (nsb + S - 1) / S;
    uint4 rw[D][NSLOT];
#define NC_K_LOAD(R, SLOT)                                                                           \
    do {                                                                                             \
        const int sb_ = min(min((R), nrounds - 1) * S + wave, nsb - 1);                              \
        const uint8_t* c_ = wt + (size_t)sb_ * CHUNK;                                                \
        _Pragma("unroll") for (int i = 0; i < NSLOT; i++) rw[SLOT][i] = *(const uint4*)(c_ + i * 1024); \
    } while (0)
#pragma unroll
    for (int k = 0; k < D - 1; k++) NC_K_LOAD(k, k);
    for (int r0 = 0; r0 < nrounds; r0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0 + k;
            NC_K_LOAD(r + D - 1, (k + D - 1) % D);
            if (r < nrounds) {  // uniform
                const int sb = r * S + wave;
                const int sbc = min(sb, nsb - 1);
                const uint4* v = rw[k];
                const float d = f16_to_f32((uint16_t)(v[0].x & 0xffff));
                const float dmin = f16_to_f32((uint16_t)(v[0].x >> 16));
                float sc[8], mn[8];
#pragma unroll
                for (int j = 0; j < 8; j++) {
                    uint32_t s, m;
                    if (j < 4) {
                        s = kbyte(v[0].y, v[0].z, v[0].w, j) & 63;
                        m = kbyte(v[0].y, v[0].z, v[0].w, j + 4) & 63;
                    } else {
                        s = (kbyte(v[0].y, v[0].z, v[0].w, j + 4) & 0x0f) |
                            ((kbyte(v[0].y, v[0].z, v[0].w, j - 4) >> 6) << 4);
                        m = (kbyte(v[0].y, v[0].z, v[0].w, j + 4) >> 4) | ((kbyte(v[0].y, v[0].z, v[0].w, j) >> 6) << 4);
                    }
                    sc[j] = d * (float)s;
                    mn[j] = dmin * (float)m;
                }
                // every token of the instantiation, without branches (tokens >= N read clamped
                // activations and are never stored)
                float t[NMAX];
                if constexpr (!Q5) {
#pragma unroll
                    for (int n = 0; n < NMAX; n++) {
                        const int nn = min(n, N - 1);
                        sptr_i32 xw = as_scalar_i32(p.x + (size_t)nn * p.K + (size_t)sbc * 256);
                        sptr_f32 xsp = as_scalar_f32(p.xs + (size_t)nn * nb + (size_t)sbc * 8);
                        sptr_i32 xap = as_scalar_i32(p.xs8 + (size_t)nn * nb + (size_t)sbc * 8);
                        float part = 0.0f;
#pragma unroll
                        for (int pr = 0; pr < 4; pr++) {
                            const uint4 q0 = v[QS + 2 * pr], q1 = v[QS + 1 + 2 * pr];
                            const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                            int wl = 0, wh = 0;
#pragma unroll
                            for (int i = 0; i < 8; i++) {
                                wl = dot4((int)(qw[i] & 0x0F0F0F0Fu), xw[pr * 16 + i], wl);
                                wh = dot4((int)((qw[i] >> 4) & 0x0F0F0F0Fu), xw[pr * 16 + 8 + i], wh);
                            }
                            // q8.rs:1372-1375: sum += xs * (sc*W - mn*A), low then high half
                            const int jl = 2 * pr, jh = 2 * pr + 1;
                            part = part + xsp[jl] * (sc[jl] * (float)wl - mn[jl] * (float)(xap[jl] / -8));
                            part = part + xsp[jh] * (sc[jh] * (float)wh - mn[jh] * (float)(xap[jh] / -8));
                        }
                        t[n] = part;
                    }
                } else {
                    // pairs outside, tokens inside: each pair's 5-bit values are built once; every
                    // token's sum still takes its pairs in order, low then high half
                    const uint32_t qh[8] = {v[1].x, v[1].y, v[1].z, v[1].w, v[2].x, v[2].y, v[2].z, v[2].w};
#pragma unroll
                    for (int n = 0; n < NMAX; n++) t[n] = 0.0f;
#pragma unroll
                    for (int pr = 0; pr < 4; pr++) {
                        const uint4 q0 = v[QS + 2 * pr], q1 = v[QS + 1 + 2 * pr];
                        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                        int lo[8], hi[8];
#pragma unroll
                        for (int i = 0; i < 8; i++) {
                            // qh bytes 4i..4i+3: bit 2*pr adds 16 to the low value, 2*pr + 1 to the high
                            lo[i] = (int)((qw[i] & 0x0F0F0F0Fu) | (((qh[i] >> (2 * pr)) & 0x01010101u) << 4));
                            hi[i] = (int)(((qw[i] >> 4) & 0x0F0F0F0Fu) | (((qh[i] >> (2 * pr + 1)) & 0x01010101u) << 4));
                        }
                        const int jl = 2 * pr, jh = 2 * pr + 1;
#pragma unroll
                        for (int n = 0; n < NMAX; n++) {
                            const int nn = min(n, N - 1);
                            sptr_i32 xw = as_scalar_i32(p.x + (size_t)nn * p.K + (size_t)sbc * 256);
                            sptr_f32 xsp = as_scalar_f32(p.xs + (size_t)nn * nb + (size_t)sbc * 8);
                            sptr_i32 xap = as_scalar_i32(p.xs8 + (size_t)nn * nb + (size_t)sbc * 8);
                            int wl = 0, wh = 0;
#pragma unroll
                            for (int i = 0; i < 8; i++) {
                                wl = dot4(lo[i], xw[pr * 16 + i], wl);
                                wh = dot4(hi[i], xw[pr * 16 + 8 + i], wh);
                            }
                            // q8.rs:1587-1590: sum += xs * (sc*W - mn*A), low then high half
                            t[n] = t[n] + xsp[jl] * (sc[jl] * (float)wl - mn[jl] * (float)(xap[jl] / -8));
                            t[n] = t[n] + xsp[jh] * (sc[jh] * (float)wh - mn[jh] * (float)(xap[jh] / -8));
                        }
                    }
                }
                if constexpr (S == 1) {
                    if (sb < nsb) {  // uniform
#pragma unroll
                        for (int n = 0; n < NMAX; n++) acc[n] = acc[n] + t[n];
                    }
                } else {
                    // double-buffered terms: one barrier per round (round r+2 rewrites this
                    // buffer only after every thread passed round r+1's barrier)
                    float* buf = lds + (size_t)(r & 1) * S * NMAX * 64;
#pragma unroll
                    for (int n = 0; n < NMAX; n++) buf[(wave * NMAX + n) * 64 + lane] = t[n];
                    __syncthreads();
                    const int nblk = min(S, nsb - r * S);
#pragma unroll
                    for (int j = 0; j < TPW; j++) {
                        const int n = wave + j * S;
                        if (n < N) {
                            float a = acc[j];
                            for (int bl = 0; bl < nblk; bl++) a = a + buf[(bl * NMAX + n) * 64 + lane];
                            acc[j] = a;
                        }
                    }
                }
            }
        }
    }
#undef NC_K_LOAD
    gemm_epilogue<NMAX, S>(p, acc, tile, wave, lane);
}

// ---------------------------------------------------------------- Q4_K, 16-row tiles (R16)
// Workgroup = one 16-row tile, S waves.  A wave instruction covers a quad of 4 super-blocks:
// lane = 16*q + r holds super-block 4*g + q of row r (9 x 16 bytes: slot 0 = d, dmin and the
// 12 packed scale bytes, slots 1..8 the 128 nibble bytes).  Round: wave w takes quad
// r*S + w.  Each DPP row of 16 lanes is one super-block, so its activations are broadcast
// inside the row: for token n, dword c*16 + j of the super-block's 256 int8 activations sits
// in lane 16*q + j of register ax[n][c], and one meta dword per lane carries the sub-block
// scales (lanes j < 8: x_scale of sub-block j) and sums (lanes 8 + j: -8 * sum of x).  Per
// token the super-block term follows q8.rs:1372-1375 sub-block by sub-block (low half then
// high half of each nibble pair); the terms go through LDS and the chain threads (token n,
// row r) add them in super-block order.  Loads are unconditional buffer loads: weights at a
// scalar chunk offset (clamped to the padded quads), activations and meta at per-lane offsets
// range-checked against [N][K] and [N][K/32] (a token past N reads 0 and is never stored).
template <int NMAX, int S, int D>
__global__ __launch_bounds__(64 * S) void gemm_q4_k_r16_kernel(GemmParams p) {
    static_assert(16 * NMAX <= 64 * S, "chain threads must fit the workgroup");
    extern __shared__ float lds[];  // [2][4*S][NMAX][16] super-block terms
    const int tile = blockIdx.x;
    const int wave = wave_id_uniform();
    const int lane = threadIdx.x & 63;
    const int q = lane >> 4, j = lane & 15;
    const int N = p.N, nsb = p.units, nb = nsb * 8;
    const int nquads = (nsb + 3) / 4;    // padded to p.groups quads per tile
    const int nrounds = (nquads + S - 1) / S;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.w + (size_t)tile * p.groups * kQ4KChunkBytes), 0, p.groups * kQ4KChunkBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, N * p.K, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs, 0, N * nb * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t s8res = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs8, 0, N * nb * 4, 0x00020000);
    const int wvo = lane * 16;
    const int xvo = q * 256 + j * 4;          // + n*K + c*64 + quad*1024
    const int mvo = q * 32 + (j & 7) * 4;     // + n*nb*4 + quad*128
    const bool meta_s = j < 8;
    uint4 rw[D][9];
    int ax[D][NMAX][4], am[D][NMAX];
#define NC_K16_LOAD(R, SLOT)                                                                         \
    do {                                                                                             \
        const int g_ = min(min((R), nrounds - 1) * S + wave, p.groups - 1);                          \
        _Pragma("unroll") for (int i = 0; i < 9; i++) rw[SLOT][i] = __builtin_bit_cast(               \
            uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wvo, g_ * kQ4KChunkBytes + i * 1024, 0)); \
        _Pragma("unroll") for (int n = 0; n < NMAX; n++) {                                           \
            _Pragma("unroll") for (int c = 0; c < 4; c++) ax[SLOT][n][c] = (int)                      \
                __builtin_amdgcn_raw_buffer_load_b32(xres, xvo + n * p.K + c * 64 + g_ * 1024, 0, 0); \
            const int mo_ = mvo + n * nb * 4 + g_ * 128;                                             \
            const int ms_ = (int)__builtin_amdgcn_raw_buffer_load_b32(sres, mo_, 0, 0);              \
            const int m8_ = (int)__builtin_amdgcn_raw_buffer_load_b32(s8res, mo_, 0, 0);             \
            am[SLOT][n] = meta_s ? ms_ : m8_;                                                        \
        }                                                                                            \
    } while (0)
#pragma unroll
    for (int k = 0; k < D - 1; k++) NC_K16_LOAD(k, k);
    float acc = 0.0f;
    const int cn = threadIdx.x >> 4, cr = threadIdx.x & 15;  // chain thread: token, row
    for (int r0 = 0; r0 < nrounds; r0 += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0 + k;
            NC_K16_LOAD(r + D - 1, (k + D - 1) % D);
            if (r < nrounds) {  // uniform
                float* buf = lds + (size_t)(r & 1) * 4 * S * NMAX * 16;
                const uint4* v = rw[k];
                const float d = f16_to_f32((uint16_t)(v[0].x & 0xffff));
                const float dmin = f16_to_f32((uint16_t)(v[0].x >> 16));
                float sc[8], mn[8];
#pragma unroll
                for (int jj = 0; jj < 8; jj++) {  // q8.rs:2008-2018 q4_k_scale_min
                    uint32_t sv, mv;
                    if (jj < 4) {
                        sv = kbyte(v[0].y, v[0].z, v[0].w, jj) & 63;
                        mv = kbyte(v[0].y, v[0].z, v[0].w, jj + 4) & 63;
                    } else {
                        sv = (kbyte(v[0].y, v[0].z, v[0].w, jj + 4) & 0x0f) |
                             ((kbyte(v[0].y, v[0].z, v[0].w, jj - 4) >> 6) << 4);
                        mv = (kbyte(v[0].y, v[0].z, v[0].w, jj + 4) >> 4) |
                             ((kbyte(v[0].y, v[0].z, v[0].w, jj) >> 6) << 4);
                    }
                    sc[jj] = d * (float)sv;
                    mn[jj] = dmin * (float)mv;
                }
                float part[NMAX];
#pragma unroll
                for (int n = 0; n < NMAX; n++) part[n] = 0.0f;
                auto pair_step = [&]<int PR>() {
                    const uint4 q0 = v[1 + 2 * PR], q1 = v[2 + 2 * PR];
                    const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
                    int lo[8], hi[8];
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        lo[i] = (int)(qw[i] & 0x0F0F0F0Fu);
                        hi[i] = (int)((qw[i] >> 4) & 0x0F0F0F0Fu);
                    }
                    constexpr int jl = 2 * PR, jh = 2 * PR + 1;
                    [&]<int... Ns>(std::integer_sequence<int, Ns...>) {
                        (([&] {
                             constexpr int n = Ns;
                             // W = sum(nib * x) over the pair's low / high 32 elements: x dwords
                             // 16*PR + i (lanes i) and 16*PR + 8 + i (lanes 8 + i) of ax[.][n][PR]
                             const int wl = dot32_bcast<0>(0, ax[k][n][PR], lo[0], lo[1], lo[2], lo[3], lo[4], lo[5],
                                                           lo[6], lo[7]);
                             const int wh = dot32_bcast<8>(0, ax[k][n][PR], hi[0], hi[1], hi[2], hi[3], hi[4], hi[5],
                                                           hi[6], hi[7]);
                             const float xl = bcast_f<jl>(__int_as_float(am[k][n]));
                             const float xh = bcast_f<jh>(__int_as_float(am[k][n]));
                             const int al = bcast_i<8 + jl>(am[k][n]) / -8;  // A_j = sum of x
                             const int ah = bcast_i<8 + jh>(am[k][n]) / -8;
                             // q8.rs:1372-1375: sum += xs * (sc*W - mn*A), low then high half
                             part[n] = part[n] + xl * (sc[jl] * (float)wl - mn[jl] * (float)al);
                             part[n] = part[n] + xh * (sc[jh] * (float)wh - mn[jh] * (float)ah);
                         }()),
                         ...);
                    }(std::make_integer_sequence<int, NMAX>{});
                };
                pair_step.template operator()<0>();
                pair_step.template operator()<1>();
                pair_step.template operator()<2>();
                pair_step.template operator()<3>();
#pragma unroll
                for (int n = 0; n < NMAX; n++) buf[((wave * 4 + q) * NMAX + n) * 16 + j] = part[n];
                __syncthreads();
                if (threadIdx.x < 16 * NMAX && cn < N) {
                    const int nblk = min(4 * S, nsb - r * 4 * S);
                    for (int bl = 0; bl < nblk; bl++) acc = acc + buf[(bl * NMAX + cn) * 16 + cr];
                }
            }
        }
    }
#undef NC_K16_LOAD
    if (threadIdx.x < 16 * NMAX && cn < N) gemm_epilogue_r16<NMAX>(p, acc, cn, tile, cr);
}

// ---------------------------------------------------------------- Q4_K, 16-row tiles, pair-split
// The R16K layout with the work of a super-block quad split over four waves, one per pair of
// sub-blocks, so that four 16-row tiles (the interleaved gate,up's 64-row group, whose SwiGLU
// epilogue needs all four) fit one workgroup of 16 waves.  Workgroup = TPG 16-row tiles x QL
// quad lanes x 4 pair waves; in round
// r, wave (tile tt, quad lane ql, pair pr) takes quad r*QL + ql of tile tt: slot 0 (d, dmin and
// the packed scales) and the pair's two nibble slots, one activation dword per token (the pair's
// 64 int8 values of the lane's super-block, broadcast by DPP rows) and the meta dword.  It
// computes the two sub-block values xs_j * (sc_j*W_j - mn_j*A_j) (q8.rs:1372-1375) of every
// token and stores them in LDS as [tile][super-block][sub-block][token][row].  After a barrier
// the super-block sums 0 + v_0 + ... + v_7 are taken in sub-block order (one thread per tile,
// super-block, token and row), and after a second barrier the chain threads add them in
// super-block order: the same f32 operations in the same order as the one-wave-per-quad kernel.
// TPG = 4: the interleaved gate,up matrix (32 gate rows and their 32 up rows per four tiles);
// the SwiGLU + Q8_0 epilogue finishes the group's 32 outputs.  Two barriers per round make one
// buffer enough: round r+1 writes values only after every thread passed round r's second
// barrier, which follows the last read of round r's values.
template <int NMAX, int QL, int TPG>
constexpr int kps_sbl() { return 4 * QL; }  // super-blocks per tile per round
template <int NMAX, int QL, int TPG>
constexpr int kps_lds_floats() {
    return TPG * kps_sbl<NMAX, QL, TPG>() * 8 * NMAX * 16 + TPG * kps_sbl<NMAX, QL, TPG>() * NMAX * 16;
}

template <int NMAX, int QL, int TPG, int PR>
__device__ __forceinline__ void gemm_q4_k_ps_body(const GemmParams& p, float* lds) {
    constexpr int SBL = kps_sbl<NMAX, QL, TPG>();
    constexpr int NT = 256 * QL * TPG;  // threads per workgroup
    constexpr int jl = 2 * PR, jh = 2 * PR + 1;
    float* vals = lds;                                // [TPG][SBL][8][NMAX][16]
    float* parts = lds + TPG * SBL * 8 * NMAX * 16;   // [TPG][SBL][NMAX][16]
    const int w = wave_id_uniform();
    const int lane = threadIdx.x & 63;
    const int q = lane >> 4, j = lane & 15;
    const int ql = (w >> 2) % QL, tt = w / (4 * QL);
    const int tile = blockIdx.x * TPG + tt;
    const int N = p.N, nsb = p.units, nb = nsb * 8;
    const int nquads = p.groups;
    const int nrounds = (nquads + QL - 1) / QL;
    const __amdgpu_buffer_rsrc_t wres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(p.w + (size_t)tile * p.groups * kQ4KChunkBytes), 0, p.groups * kQ4KChunkBytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t xres = __builtin_amdgcn_make_buffer_rsrc((void*)p.x, 0, N * p.K, 0x00020000);
    const __amdgpu_buffer_rsrc_t sres = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs, 0, N * nb * 4, 0x00020000);
    const __amdgpu_buffer_rsrc_t s8res = __builtin_amdgcn_make_buffer_rsrc((void*)p.xs8, 0, N * nb * 4, 0x00020000);
    const int wvo = lane * 16;
    const int xvo = q * 256 + j * 4 + PR * 64;  // + n*K + quad*1024
    const int mvo = q * 32 + (j & 7) * 4;       // + n*nb*4 + quad*128
    const bool meta_s = j < 8;
    constexpr int D = 2;  // ring of rounds in flight
    uint4 rs[D], r0[D], r1[D];
    int ax[D][NMAX], am[D][NMAX];
#define NC_KPS_LOAD(R, SLOT)                                                                               \
    do {                                                                                                   \
        const int g_ = min((R) * QL + ql, p.groups - 1);                                                   \
        rs[SLOT] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(wres, wvo, g_ * kQ4KChunkBytes, 0)); \
        r0[SLOT] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(                        \
                                                 wres, wvo, g_ * kQ4KChunkBytes + (1 + 2 * PR) * 1024, 0));  \
        r1[SLOT] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(                        \
                                                 wres, wvo, g_ * kQ4KChunkBytes + (2 + 2 * PR) * 1024, 0));  \
        _Pragma("unroll") for (int n = 0; n < NMAX; n++) {                                                 \
            ax[SLOT][n] = (int)__builtin_amdgcn_raw_buffer_load_b32(xres, xvo + n * p.K + g_ * 1024, 0, 0); \
            const int mo_ = mvo + n * nb * 4 + g_ * 128;                                                   \
            const int ms_ = (int)__builtin_amdgcn_raw_buffer_load_b32(sres, mo_, 0, 0);                    \
            const int m8_ = (int)__builtin_amdgcn_raw_buffer_load_b32(s8res, mo_, 0, 0);                   \
            am[SLOT][n] = meta_s ? ms_ : m8_;                                                              \
        }                                                                                                  \
    } while (0)
    NC_KPS_LOAD(0, 0);
    // chain thread c: TPG = 1 token c / 16, row c % 16; TPG = 4 token c / 64 (one wave per
    // token, as the SwiGLU epilogue wants), tile (c % 64) / 16, row c % 16
    const int c = threadIdx.x;
    const int cn = TPG == 1 ? c >> 4 : c >> 6;
    const int ct = TPG == 1 ? 0 : (c & 63) >> 4;
    const int cr = c & 15;
    const bool chain = c < TPG * NMAX * 16 && cn < N;
    float acc = 0.0f;
    for (int r0i = 0; r0i < nrounds; r0i += D) {
#pragma unroll
        for (int k = 0; k < D; k++) {
            const int r = r0i + k;
            if (r >= nrounds) break;  // uniform
            NC_KPS_LOAD(min(r + 1, nrounds - 1), (k + 1) % D);
            const int g = r * QL + ql;
            if (g < nquads) {  // uniform per wave
                const uint4 v = rs[k];
                const float d = f16_to_f32((uint16_t)(v.x & 0xffff));
                const float dmin = f16_to_f32((uint16_t)(v.x >> 16));
                // q8.rs:2008-2018 q4_k_scale_min for sub-blocks jl and jh
                uint32_t sl, ml, sh, mh;
                if constexpr (jl < 4) {
                    sl = kbyte(v.y, v.z, v.w, jl) & 63;
                    ml = kbyte(v.y, v.z, v.w, jl + 4) & 63;
                    sh = kbyte(v.y, v.z, v.w, jh) & 63;
                    mh = kbyte(v.y, v.z, v.w, jh + 4) & 63;
                } else {
                    sl = (kbyte(v.y, v.z, v.w, jl + 4) & 0x0f) | ((kbyte(v.y, v.z, v.w, jl - 4) >> 6) << 4);
                    ml = (kbyte(v.y, v.z, v.w, jl + 4) >> 4) | ((kbyte(v.y, v.z, v.w, jl) >> 6) << 4);
                    sh = (kbyte(v.y, v.z, v.w, jh + 4) & 0x0f) | ((kbyte(v.y, v.z, v.w, jh - 4) >> 6) << 4);
                    mh = (kbyte(v.y, v.z, v.w, jh + 4) >> 4) | ((kbyte(v.y, v.z, v.w, jh) >> 6) << 4);
                }
                const float scl = d * (float)sl, mnl = dmin * (float)ml;
                const float sch = d * (float)sh, mnh = dmin * (float)mh;
                const uint32_t qw[8] = {r0[k].x, r0[k].y, r0[k].z, r0[k].w, r1[k].x, r1[k].y, r1[k].z, r1[k].w};
                int lo[8], hi[8];
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    lo[i] = (int)(qw[i] & 0x0F0F0F0Fu);
                    hi[i] = (int)((qw[i] >> 4) & 0x0F0F0F0Fu);
                }
                float* vb = vals + ((size_t)(tt * SBL + ql * 4 + q) * 8) * NMAX * 16 + j;
                [&]<int... Ns>(std::integer_sequence<int, Ns...>) {
                    (([&] {
                         constexpr int n = Ns;
                         const int wl = dot32_bcast<0>(0, ax[k][n], lo[0], lo[1], lo[2], lo[3], lo[4], lo[5], lo[6],
                                                       lo[7]);
                         const int wh = dot32_bcast<8>(0, ax[k][n], hi[0], hi[1], hi[2], hi[3], hi[4], hi[5], hi[6],
                                                       hi[7]);
                         const float xl = bcast_f<jl>(__int_as_float(am[k][n]));
                         const float xh = bcast_f<jh>(__int_as_float(am[k][n]));
                         const int al = bcast_i<8 + jl>(am[k][n]) / -8;  // A_j = sum of x
                         const int ah = bcast_i<8 + jh>(am[k][n]) / -8;
                         vb[(jl * NMAX + n) * 16] = xl * (scl * (float)wl - mnl * (float)al);
                         vb[(jh * NMAX + n) * 16] = xh * (sch * (float)wh - mnh * (float)ah);
                     }()),
                     ...);
                }(std::make_integer_sequence<int, NMAX>{});
            }
            __syncthreads();
            // super-block sums in sub-block order, starting from 0 as the reference's per-
            // super-block loop does
            const int sb0 = r * QL * 4;  // first super-block of the round
            for (int i = c; i < TPG * SBL * NMAX * 16; i += NT) {
                const int sbl = (i / (NMAX * 16)) % SBL;
                if (sb0 + sbl < nsb) {
                    const int tsb = i / (NMAX * 16);  // tile * SBL + sbl
                    const int nr = i % (NMAX * 16);   // token * 16 + row
                    const float* vv = vals + (size_t)tsb * 8 * NMAX * 16 + nr;
                    float part = 0.0f;
#pragma unroll
                    for (int s = 0; s < 8; s++) part = part + vv[s * NMAX * 16];
                    parts[i] = part;
                }
            }
            __syncthreads();
            if (chain) {
                const int nblk = min(SBL, nsb - sb0);
                const float* pp = parts + (size_t)ct * SBL * NMAX * 16 + cn * 16 + cr;
                for (int bl = 0; bl < nblk; bl++) acc = acc + pp[bl * NMAX * 16];
            }
        }
    }
#undef NC_KPS_LOAD
    if constexpr (TPG == 1) {
        if (chain) gemm_epilogue_r16<NMAX>(p, acc, cn, tile, cr);
    } else {
        r16_swiglu_epilogue<NMAX>(p, lds, chain, ct, cn, cr, acc, w);
    }
}

template <int NMAX, int QL, int TPG>
__global__ __launch_bounds__(256 * QL * TPG) void gemm_q4_k_ps_kernel(GemmParams p) {
    static_assert(TPG == 1 || (TPG == 4 && QL == 1), "tile groups: one tile with 1..4 quad lanes, or four tiles");
    static_assert(NMAX <= 9, "LDS holds the sub-block values of at most 9 tokens");
    __shared__ float lds[kps_lds_floats<NMAX, QL, TPG>()];
    switch (wave_id_uniform() & 3) {  // the wave's sub-block pair (uniform)
        case 0: gemm_q4_k_ps_body<NMAX, QL, TPG, 0>(p, lds); break;
        case 1: gemm_q4_k_ps_body<NMAX, QL, TPG, 1>(p, lds); break;
        case 2: gemm_q4_k_ps_body<NMAX, QL, TPG, 2>(p, lds); break;
        default: gemm_q4_k_ps_body<NMAX, QL, TPG, 3>(p, lds); break;
    }
}

// ---------------------------------------------------------------- per-block dots (parity debug)
__global__ void blockdots_q4_0_kernel(const uint8_t* w, int groups, int r16, int M, int K, const int8_t* x, int N,
                                      int32_t* dots) {
    const int nb = K / 32;
    const int64_t total = (int64_t)N * M * nb;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int b = (int)(i % nb);
        const int r = (int)((i / nb) % M);
        const int n = (int)(i / ((int64_t)nb * M));
        const uint8_t* nib;
        if (r16) {
            const int qd = b / 4, lane = 16 * (b & 3) + (r & 15);
            nib = w + ((size_t)(r / 16) * groups + qd / 8) * kQ40ChunkBytes + (qd & 7) * kQ40R16QuadBytes + lane * 16;
        } else {
            nib = w + ((size_t)(r / 64) * groups + b / 8) * kQ40ChunkBytes + (b & 7) * 1024 + (r & 63) * 16;
        }
        const int8_t* xb = x + (size_t)n * K + (size_t)b * 32;
        int d = 0;
        for (int j = 0; j < 16; j++) {
            d += ((int)(nib[j] & 0x0f) - 8) * (int)xb[j];
            d += ((int)(nib[j] >> 4) - 8) * (int)xb[j + 16];
        }
        dots[i] = d;
    }
}

__global__ void blockdots_q4_k_kernel(const uint8_t* w, int nsb, int groups, int r16, int M, int K, const int8_t* x,
                                      int N, int32_t* dots) {
    const int nb = K / 32;
    const int64_t total = (int64_t)N * M * nb;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int j = (int)(i % nb);
        const int r = (int)((i / nb) % M);
        const int n = (int)(i / ((int64_t)nb * M));
        const int sb = j / 8, sj = j % 8, pr = sj / 2, half = sj % 2;
        const uint8_t* chunk = r16 ? w + ((size_t)(r / 16) * groups + sb / 4) * kQ4KChunkBytes +
                                         (16 * (sb % 4) + (r & 15)) * 16
                                   : w + ((size_t)(r / 64) * nsb + sb) * kQ4KChunkBytes + (r & 63) * 16;
        const int8_t* xb = x + (size_t)n * K + (size_t)j * 32;
        int d = 0;
        for (int l = 0; l < 32; l++) {
            const uint8_t byte = chunk[(1 + 2 * pr + l / 16) * 1024 + (l % 16)];
            d += (int)(half ? (byte >> 4) : (byte & 0x0f)) * (int)xb[l];
        }
        dots[i] = d;
    }
}

// ---------------------------------------------------------------- dispatch
namespace {


// ev0/ev1 (optional): events stamped by the dispatch itself at kernel start and end
// (hipExtLaunchKernelGGL), so their elapsed time is the kernel's own duration.
template <int NMAX, int S>
int launch_one(const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    if (w.type == NC_TYPE_Q4_0) {
        if constexpr (S > 4) {
            return fail(NC_EINVAL, "gemm: Q4_0 uses at most 4 K-split waves");
        } else {
            // ring depth: one round ahead when K is split over waves (deeper rings measured
            // slower: the extra loads issued up front delay every wave's first round), two for S = 1
            constexpr int D = S == 1 ? 3 : 2;
            const size_t lds = S > 1 ? (size_t)2 * S * 4 * NMAX * 64 * sizeof(float) : 0;
            if (ev0)
                hipExtLaunchKernelGGL((gemm_q4_0_kernel<NMAX, S, D>), dim3(p.ntiles), dim3(64 * S), lds, st, ev0,
                                      ev1, 0, p);
            else
                NC_LAUNCH((gemm_q4_0_kernel<NMAX, S, D>), dim3(p.ntiles), dim3(64 * S), lds, st, p);
        }
    } else if (w.type == NC_TYPE_Q5_K) {
        constexpr int D = 2;
        const size_t lds = S > 1 ? (size_t)2 * S * NMAX * 64 * sizeof(float) : 0;
        if (ev0)
            hipExtLaunchKernelGGL((gemm_q4_k_kernel<NMAX, S, D, true>), dim3(p.ntiles), dim3(64 * S), lds, st, ev0,
                                  ev1, 0, p);
        else
            NC_LAUNCH((gemm_q4_k_kernel<NMAX, S, D, true>), dim3(p.ntiles), dim3(64 * S), lds, st, p);
    } else {
        constexpr int D = 2;  // one super-block ahead
        const size_t lds = S > 1 ? (size_t)2 * S * NMAX * 64 * sizeof(float) : 0;
        if (ev0)
            hipExtLaunchKernelGGL((gemm_q4_k_kernel<NMAX, S, D>), dim3(p.ntiles), dim3(64 * S), lds, st, ev0, ev1, 0,
                                  p);
        else
            NC_LAUNCH((gemm_q4_k_kernel<NMAX, S, D>), dim3(p.ntiles), dim3(64 * S), lds, st, p);
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// R16: S waves so that the chain threads (16 per token) fit; U = 1 quad per wave-round and
// one round in flight ahead of the one being computed (the fastest of the measured
// S x U x D shapes on every layer matrix of the 8B model).
template <int NMAX>
int launch_r16(const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    constexpr int U = 1, D = 2;
    if (p.epi == EPI_SWIGLU_Q8) {
        // four 16-row tiles per workgroup, 4 waves each (the fastest 16-row shape measured on
        // the 28672 x 4096 gate,up matrix)
        // up to 8 rows: 2 waves per tile and one chain wave per token; wider: 4 waves per tile
        // with the chains on the first two waves of each tile
        constexpr int TPG = 4, CW = NMAX <= 8 ? NMAX : 0, S = CW ? 2 : 4;
        if (p.ntiles % TPG) return fail(NC_EINVAL, "gemm: SwiGLU rows must fill whole 64-row groups");
        const size_t lds = (size_t)TPG * r16_tile_lds<4 * S * U, NMAX, TPG>() * sizeof(float);
        if (ev0)
            hipExtLaunchKernelGGL((gemm_q4_0_r16_kernel<NMAX, S, U, D, TPG, CW>), dim3(p.ntiles / TPG),
                                  dim3(64 * (S * TPG + CW)), lds, st, ev0, ev1, 0, p);
        else
            NC_LAUNCH((gemm_q4_0_r16_kernel<NMAX, S, U, D, TPG, CW>), dim3(p.ntiles / TPG),
                               dim3(64 * (S * TPG + CW)), lds, st, p);
    } else {
        // 8 waves (two per SIMD hide each other's dependency latency); 16 when K is long
        // (at least 64 quads): half the rounds, each with its barrier and chain step
        // (4096 x 14336 at N = 5: 11.81 -> 10.44 us; 6144 x 4096 is slower with 16), for
        // widths whose round buffers stay within 48 KB of LDS
        constexpr int CW = (16 * NMAX + 63) / 64;  // dedicated chain waves
        auto go = [&]<int S>() {
            const size_t lds = (size_t)2 * 4 * S * U * NMAX * 16 * sizeof(float);
            if (ev0)
                hipExtLaunchKernelGGL((gemm_q4_0_r16_kernel<NMAX, S, U, D, 1, CW>), dim3(p.ntiles),
                                      dim3(64 * (S + CW)), lds, st, ev0, ev1, 0, p);
            else
                NC_LAUNCH((gemm_q4_0_r16_kernel<NMAX, S, U, D, 1, CW>), dim3(p.ntiles), dim3(64 * (S + CW)),
                                   lds, st, p);
        };
        if constexpr (NMAX <= 6) {
            if ((p.units + 3) / 4 >= 64)
                go.template operator()<12>();
            else
                go.template operator()<8>();
        } else {
            go.template operator()<8>();
        }
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// R16 with MFMA dots: the same launch shapes as launch_r16 (term waves per tile, dedicated
// chain waves where they fit).
template <int NMAX>
int launch_r16_mfma(const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    constexpr int D = 2;
    if (p.epi == EPI_SWIGLU_Q8) {
        // four 16-row tiles per workgroup; up to 8 rows one chain wave per token, wider the
        // chains run on the first waves of each tile
        constexpr int TPG = 4, CW = NMAX <= 8 ? NMAX : 0, S = CW ? 2 : 4;
        if (p.ntiles % TPG) return fail(NC_EINVAL, "gemm: SwiGLU rows must fill whole 64-row groups");
        const size_t lds = (size_t)TPG * r16_tile_lds<4 * S, NMAX, TPG>() * sizeof(float);
        if (ev0)
            hipExtLaunchKernelGGL((gemm_q4_0_mfma_kernel<NMAX, S, D, TPG, CW>), dim3(p.ntiles / TPG),
                                  dim3(64 * (S * TPG + CW)), lds, st, ev0, ev1, 0, p);
        else
            NC_LAUNCH((gemm_q4_0_mfma_kernel<NMAX, S, D, TPG, CW>), dim3(p.ntiles / TPG),
                               dim3(64 * (S * TPG + CW)), lds, st, p);
    } else {
        constexpr int CW = (16 * NMAX + 63) / 64;
        auto go = [&]<int S>() {
            const size_t lds = (size_t)2 * 4 * S * NMAX * 16 * sizeof(float);
            if (ev0)
                hipExtLaunchKernelGGL((gemm_q4_0_mfma_kernel<NMAX, S, D, 1, CW>), dim3(p.ntiles), dim3(64 * (S + CW)),
                                      lds, st, ev0, ev1, 0, p);
            else
                NC_LAUNCH((gemm_q4_0_mfma_kernel<NMAX, S, D, 1, CW>), dim3(p.ntiles), dim3(64 * (S + CW)),
                                   lds, st, p);
        };
        if constexpr (NMAX <= 6) {
            if ((p.units + 3) / 4 >= 64)
                go.template operator()<12>();
            else
                go.template operator()<8>();
        } else {
            go.template operator()<8>();
        }
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

template <int NMAX>
int launch_s(int S, const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    switch (S) {
        case 1: return launch_one<NMAX, 1>(w, p, st, ev0, ev1);
        case 2: return launch_one<NMAX, 2>(w, p, st, ev0, ev1);
        default: return launch_one<NMAX, 4>(w, p, st, ev0, ev1);
    }
}

// Q4_K: more K-split waves than the Q4_0 path (a super-block is 9 KB per wave and the 3B/8B
// Q4_K matrices have few 64-row tiles): 12 waves when K is 12 super-blocks (one round),
// else 8, else 4.
template <int NMAX>
int launch_k(int S, const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    switch (S) {
        case 1: return launch_one<NMAX, 1>(w, p, st, ev0, ev1);
        case 2: return launch_one<NMAX, 2>(w, p, st, ev0, ev1);
        case 4: return launch_one<NMAX, 4>(w, p, st, ev0, ev1);
        case 8: return launch_one<NMAX, 8>(w, p, st, ev0, ev1);
        default: return launch_one<NMAX, 12>(w, p, st, ev0, ev1);
    }
}

// Q4_K on 16-row tiles: 8 waves (one quad of super-blocks each per round) when K has at least
// 8 quads, else 4 (enough chain threads for 16 tokens); a ring of 2 rounds, 1 at 16 rows
// (registers).
template <int NMAX>
int launch_k16(const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    constexpr int D = NMAX <= 9 ? 2 : 1;
    auto go = [&]<int S>() {
        const size_t lds = (size_t)2 * 4 * S * NMAX * 16 * sizeof(float);
        if (ev0)
            hipExtLaunchKernelGGL((gemm_q4_k_r16_kernel<NMAX, S, D>), dim3(p.ntiles), dim3(64 * S), lds, st, ev0, ev1, 0,
                                  p);
        else
            NC_LAUNCH((gemm_q4_k_r16_kernel<NMAX, S, D>), dim3(p.ntiles), dim3(64 * S), lds, st, p);
    };
    if constexpr (NMAX <= 9) {
        // The interleaved gate,up as four-tile groups with the SwiGLU epilogue on the pair-split
        // kernel (3B, N = 5: 14.9 us against 15.4 for the 64-row kernel in the verify step).
        // Plain matrices stay one wave per quad: the pair-split kernel with 1-4 quad lanes
        // measured no faster inside the step (3B q,k,v 10.2 / wo 7.1 us against 9.7 / 6.8).
        auto ps = [&]<int QL, int TPG>() {
            const dim3 grid(p.ntiles / TPG), block(256 * QL * TPG);
            if (ev0)
                hipExtLaunchKernelGGL((gemm_q4_k_ps_kernel<NMAX, QL, TPG>), grid, block, 0, st, ev0, ev1, 0, p);
            else
                NC_LAUNCH((gemm_q4_k_ps_kernel<NMAX, QL, TPG>), grid, block, 0, st, p);
        };
        // NC_Q4K_PS=<1..4>: tuning override, plain matrices on the pair-split kernel with that many
        // quad lanes; read at each launch, so a sweep or a test can switch it within a process
        const char* ps_env = getenv("NC_Q4K_PS");
        const int forced = ps_env ? atoi(ps_env) : 0;
        if (p.epi == EPI_SWIGLU_Q8) {
            if (p.ntiles % 4) return fail(NC_EINVAL, "gemm: interleaved gate,up needs whole 64-row groups");
            ps.template operator()<1, 4>();
        } else if (forced == 1) {
            ps.template operator()<1, 1>();
        } else if (forced == 2) {
            ps.template operator()<2, 1>();
        } else if (forced == 3) {
            ps.template operator()<3, 1>();
        } else if (forced == 4) {
            ps.template operator()<4, 1>();
        } else if (w.groups >= 8) {
            go.template operator()<8>();
        } else {
            go.template operator()<4>();
        }
    } else {
        if (p.epi == EPI_SWIGLU_Q8)
            return fail(NC_EINVAL, "gemm: the 16-row Q4_K SwiGLU epilogue takes at most 9 tokens");
        if (w.groups >= 8) go.template operator()<8>();
        else go.template operator()<4>();
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace

template <int NMAX>
int launch_q80(const QMatDev& w, const GemmParams& p, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    // K-split waves: enough that ~1000+ waves stream the matrix, at most one per block
    int S = 1;
    while (S < 8 && w.tiles * S < 1024 && 2 * S <= w.units) S *= 2;
    auto go = [&]<int SS>() {
        const size_t lds = SS > 1 ? (size_t)2 * SS * NMAX * 64 * sizeof(float) : 0;
        if (ev0)
            hipExtLaunchKernelGGL((gemm_q8_0_kernel<NMAX, SS>), dim3(p.ntiles), dim3(64 * SS), lds, st, ev0, ev1, 0, p);
        else
            NC_LAUNCH((gemm_q8_0_kernel<NMAX, SS>), dim3(p.ntiles), dim3(64 * SS), lds, st, p);
    };
    switch (S) {
        case 1: go.template operator()<1>(); break;
        case 2: go.template operator()<2>(); break;
        case 4: go.template operator()<4>(); break;
        default: go.template operator()<8>(); break;
    }
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// R64 waves per workgroup: enough K-split waves that ~1000+ waves stream the matrix
// (1, 2 or 4; LDS terms double-buffered: 2 * S * 4 * NMAX * 64 floats).
static int pick_waves(int64_t tiles) {
    int S = 1;
    while (S < 4 && tiles * S < 1024) S *= 2;
    return S;
}

// Instantiated batch widths: exact for 1..9 (k <= 8 verify widths, decode), 16 above.
#define NC_GEMM_FOR_NMAX(F, N_, ...)                  \
    switch ((N_) <= 9 ? (N_) : 16) {                  \
        case 1: return F<1>(__VA_ARGS__);             \
        case 2: return F<2>(__VA_ARGS__);             \
        case 3: return F<3>(__VA_ARGS__);             \
        case 4: return F<4>(__VA_ARGS__);             \
        case 5: return F<5>(__VA_ARGS__);             \
        case 6: return F<6>(__VA_ARGS__);             \
        case 7: return F<7>(__VA_ARGS__);             \
        case 8: return F<8>(__VA_ARGS__);             \
        case 9: return F<9>(__VA_ARGS__);             \
        default: return F<16>(__VA_ARGS__);           \
    }

int launch_gemm(const QMatDev& w, const GemmParams& p0, hipStream_t st, hipEvent_t ev0, hipEvent_t ev1) {
    GemmParams p = p0;
    p.w = w.dev;
    p.ntiles = (int)w.tiles;
    p.units = (int)w.units;
    p.groups = (int)w.groups;
    p.M = (int)w.rows;
    p.K = (int)w.cols;
    if (p.N < 1 || p.N > 16) return fail(NC_EINVAL, "gemm: batch must be 1..16");
    if (w.layout == LAYOUT_Q6K) {
        if (ev0) NC_HIP(hipEventRecord(ev0, st));
        const int rc = launch_gemm_q6k(w, p, st);
        if (!rc && ev1) NC_HIP(hipEventRecord(ev1, st));
        return rc;
    }
    if (w.layout == LAYOUT_R16) {
        // dot products by v_dot4c (AUTO: the faster path at every measured shape and width) or,
        // on request, by int8 MFMA
        if (p.kernel == NC_GEMM_KERNEL_MFMA) {
            NC_GEMM_FOR_NMAX(launch_r16_mfma, p.N, w, p, st, ev0, ev1)
        }
        NC_GEMM_FOR_NMAX(launch_r16, p.N, w, p, st, ev0, ev1)
    }
    if (w.layout == LAYOUT_R16K) {
        NC_GEMM_FOR_NMAX(launch_k16, p.N, w, p, st, ev0, ev1)
    }
    if (w.layout == LAYOUT_Q80) {
        NC_GEMM_FOR_NMAX(launch_q80, p.N, w, p, st, ev0, ev1)
    }
    if (w.type == NC_TYPE_Q4_K || w.type == NC_TYPE_Q5_K) {
        const int nsb = (int)w.units;
        int S = nsb == 12 ? 12 : (nsb >= 8 ? 8 : 4);
        if (w.tiles * S > 4096) S = pick_waves(w.tiles);
        NC_GEMM_FOR_NMAX(launch_k, p.N, S, w, p, st, ev0, ev1)
    }
    int S = pick_waves(w.tiles);
    // NC_GEMM_WAVES=<1|2|4>: tuning override of the R64 K-split width
    static const int forced = [] {
        const char* e = getenv("NC_GEMM_WAVES");
        return e ? atoi(e) : 0;
    }();
    if (forced == 1 || forced == 2 || forced == 4) S = forced;
    NC_GEMM_FOR_NMAX(launch_s, p.N, S, w, p, st, ev0, ev1)
}

int launch_blockdots(const QMatDev& w, const int8_t* x, int32_t* dots, int N, hipStream_t st) {
    if (w.type != NC_TYPE_Q4_0 && w.type != NC_TYPE_Q4_K) return fail(NC_EINVAL, "blockdots: Q4_0 and Q4_K only");
    const int64_t total = (int64_t)N * w.rows * (w.cols / 32);
    const int blocks = (int)std::min<int64_t>((total + 255) / 256, 65536);
    if (w.type == NC_TYPE_Q4_0)
        hipLaunchKernelGGL(blockdots_q4_0_kernel, dim3(blocks), dim3(256), 0, st, w.dev, (int)w.groups,
                           (int)(w.layout == LAYOUT_R16), (int)w.rows,
                           (int)w.cols, x, N, dots);
    else
        hipLaunchKernelGGL(blockdots_q4_k_kernel, dim3(blocks), dim3(256), 0, st, w.dev, (int)w.units, (int)w.groups,
                           (int)(w.layout == LAYOUT_R16K), (int)w.rows, (int)w.cols, x, N, dots);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
