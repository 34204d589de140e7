// Q6_K x Q8_0 batch matmul on gfx950, for the Q6_K output projection that llama.cpp writes
// into most quantised files (its Q4_0 and Q4_K_M mixes among them).
//
// The reference's portable path (matmul_q6_k_batch, inference.rs:1882-2000, with
// Q6KBlock::dot_q8_scaled, q8.rs:2093-2150) sums every element's term in f32, in a fixed
// order, per 256-value super-block, then adds the super-block sums along the row:
//   ws[i] = d * sc[i];  c = ws[group] * x_scale[32-block]
//   block: s = 0; for half, for l in 0..32, for k in 0..4: s += (c * (float)q) * (float)x
//   row:   sum = 0; for b: sum += s_b
// Lane (row, super-block b) evaluates one block's chain for every token (the 6-bit values are
// unpacked once and reused across tokens); the row's chain then reads the block sums of its
// lanes in order through cross-lane reads.  A wave holds 64 / (K/256) rows.
//
// Device layout: the GGUF blocks split into planes so every lane's loads are aligned 16-byte
// pieces: ql [rows*nb][128], qh [rows*nb][64], scales [rows*nb][16], d [rows*nb] (f16).
#include "nc_internal.h"
#include "nc_device.h"

namespace nc {

struct Q6Planes {
    const uint8_t *ql, *qh, *sc;
    const uint16_t* d;
};

__host__ __device__ inline Q6Planes q6k_planes(const uint8_t* base, int64_t nblk) {
    Q6Planes p;
    p.ql = base;
    p.qh = base + nblk * 128;
    p.sc = base + nblk * 192;
    p.d = (const uint16_t*)(base + nblk * 208);
    return p;
}

template <int NMAX>
__global__ __launch_bounds__(256) void gemm_q6_k_kernel(GemmParams p, int nb, int rpw) {
    __shared__ float tile_val[NMAX][4 * 64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int rb = lane / nb, b = lane % nb;
    const int rows_wg = 4 * rpw;
    const int row = blockIdx.x * rows_wg + wv * rpw + rb;
    const bool active = rb < rpw && row < p.M;
    const int rr = min(row, p.M - 1);  // inactive lanes read a valid block and store nothing
    const int64_t nblk = (int64_t)p.M * nb, blk = (int64_t)rr * nb + min(b, nb - 1);
    const Q6Planes w = q6k_planes(p.w, nblk);
    const int N = p.N, K = p.K, nx = K / 32;
    const uint4 scv = *(const uint4*)(w.sc + blk * 16);
    const int8_t* sc8 = (const int8_t*)&scv;
    const float d = f16_to_f32(w.d[blk]);
    float ws[16];
#pragma unroll
    for (int i = 0; i < 16; i++) ws[i] = d * (float)sc8[i];
    float bsum[NMAX];
#pragma unroll
    for (int t = 0; t < NMAX; t++) bsum[t] = 0.0f;
#pragma unroll
    for (int half = 0; half < 2; half++) {
        uint32_t ql[16], qh[8];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint4 v = *(const uint4*)(w.ql + blk * 128 + 64 * half + 16 * i);
            ql[4 * i] = v.x; ql[4 * i + 1] = v.y; ql[4 * i + 2] = v.z; ql[4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 2; i++) {
            const uint4 v = *(const uint4*)(w.qh + blk * 64 + 32 * half + 16 * i);
            qh[4 * i] = v.x; qh[4 * i + 1] = v.y; qh[4 * i + 2] = v.z; qh[4 * i + 3] = v.w;
        }
        // c[t][k][lc]: lc = 0 for l < 16 (the "low" scale of the 32-value group), 1 above
        float c[NMAX][4][2];
#pragma unroll
        for (int t = 0; t < NMAX; t++) {
            if (t < N) {
                const float4 xs4 = *(const float4*)(p.xs + (size_t)t * nx + 8 * b + 4 * half);
                const float xsk[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    c[t][k][0] = ws[8 * half + 2 * k] * xsk[k];
                    c[t][k][1] = ws[8 * half + 2 * k + 1] * xsk[k];
                }
            }
        }
        const int8_t* xb = p.x + 256 * b + 128 * half;
#pragma unroll 2
        for (int l0 = 0; l0 < 32; l0 += 4) {
            uint32_t xw[NMAX][4];
#pragma unroll
            for (int t = 0; t < NMAX; t++)
                if (t < N) {
#pragma unroll
                    for (int k = 0; k < 4; k++) xw[t][k] = *(const uint32_t*)(xb + (size_t)t * K + 32 * k + l0);
                }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int l = l0 + j, lc = l >> 4;
                const uint32_t lo = (ql[l >> 2] >> (8 * (l & 3))) & 0xff;
                const uint32_t hi32 = (ql[(l + 32) >> 2] >> (8 * (l & 3))) & 0xff;
                const uint32_t hb = (qh[l >> 2] >> (8 * (l & 3))) & 0xff;
                float qf[4];
                qf[0] = (float)((int)((lo & 0x0f) | ((hb & 3) << 4)) - 32);
                qf[1] = (float)((int)((hi32 & 0x0f) | (((hb >> 2) & 3) << 4)) - 32);
                qf[2] = (float)((int)((lo >> 4) | (((hb >> 4) & 3) << 4)) - 32);
                qf[3] = (float)((int)((hi32 >> 4) | (((hb >> 6) & 3) << 4)) - 32);
#pragma unroll
                for (int t = 0; t < NMAX; t++) {
                    if (t < N) {
#pragma unroll
                        for (int k = 0; k < 4; k++) {
                            const float xf = (float)(int8_t)((xw[t][k] >> (8 * j)) & 0xff);
                            bsum[t] = bsum[t] + (c[t][k][lc] * qf[k]) * xf;
                        }
                    }
                }
            }
        }
    }
    // the row's chain over its super-blocks, in order, from the lanes rb*nb .. rb*nb + nb - 1
    float rowsum[NMAX];
#pragma unroll
    for (int t = 0; t < NMAX; t++) {
        float acc = 0.0f;
        for (int bb = 0; bb < nb; bb++) acc = acc + __shfl(bsum[t], rb * nb + bb, 64);
        rowsum[t] = acc;
    }
    const bool writer = active && b == 0;
    if (p.epi == EPI_HEAD) {
        // logits, then the first maximum over this workgroup's rows per token
        // (inference.rs:4836-4846): value, then the lower index on ties
#pragma unroll
        for (int t = 0; t < NMAX; t++) {
            if (t < N) {
                if (writer) p.out[(size_t)t * p.ld_out + row] = rowsum[t];
                if (b == 0 && rb < rpw) tile_val[t][wv * rpw + rb] = active ? rowsum[t] : -__builtin_inff();
            }
        }
        __syncthreads();
        if ((int)threadIdx.x < N) {
            const int t = threadIdx.x;
            float bv = -__builtin_inff();
            int bi = 0x7fffffff;
            for (int i = 0; i < rows_wg; i++) {
                const int r = blockIdx.x * rows_wg + i;
                if (r >= p.M) break;
                const float v = tile_val[t][i];
                if (v > bv || (v == bv && r < bi)) {
                    bv = v;
                    bi = r;
                }
            }
            p.part_val[(size_t)t * p.ntiles + blockIdx.x] = bv;
            p.part_idx[(size_t)t * p.ntiles + blockIdx.x] = bi;
        }
    } else {
#pragma unroll
        for (int t = 0; t < NMAX; t++)
            if (t < N && writer) p.out[(size_t)t * p.ld_out + row] = rowsum[t];
    }
}

// Rows per workgroup of the Q6_K kernel (4 waves of 64 / (cols / 256) rows); the head's
// argmax partials come one per workgroup.
int q6k_rows_per_tile(int64_t cols) { return 4 * (int)(64 / (cols / 256)); }

int launch_gemm_q6k(const QMatDev& w, const GemmParams& p0, hipStream_t st) {
    GemmParams p = p0;
    const int nb = (int)(w.cols / 256);
    if (w.cols % 256 || nb < 1 || nb > 64) return fail(NC_EINVAL, "Q6_K matmul: cols must be 256..16384, multiple of 256");
    if (p.epi != EPI_STORE && p.epi != EPI_HEAD) return fail(NC_EINVAL, "Q6_K matmul: plain or head outputs only");
    const int rpw = 64 / nb;
    p.w = w.dev;
    p.M = (int)w.rows;
    p.K = (int)w.cols;
    p.ntiles = (int)w.tiles;
    const dim3 grid((unsigned)w.tiles);
#define NC_Q6K(NM) NC_LAUNCH((gemm_q6_k_kernel<NM>), grid, dim3(256), 0, st, p, nb, rpw)
    if (p.N <= 1) NC_Q6K(1);
    else if (p.N <= 4) NC_Q6K(4);
    else if (p.N <= 8) NC_Q6K(8);
    else if (p.N <= 16) NC_Q6K(16);
    else return fail(NC_EINVAL, "Q6_K matmul: batch must be 1..16");
#undef NC_Q6K
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
