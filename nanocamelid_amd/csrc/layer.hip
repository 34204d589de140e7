// Row ops of the verify forward on gfx950: fused RMSNorm + Q8_0 quantisation,
// activation quantisation, embedding gather, causal GQA attention over the
// HBM-resident f32 KV cache (with the Q8_0 quantisation of its output fused in),
// the head argmax reduction and greedy acceptance.
//
// Every f32 chain that the reference evaluates sequentially gives the same bits here:
// the RMSNorm sum of squares goes through exact_chain_sum (a parallel evaluation that is
// verified step by step against the sequential recurrence); each attention dot product,
// the softmax denominator and the weighted V sum are evaluated in order.  The parallel
// parts are the order-free ones (max, elementwise maps, integer sums, independent
// rows/heads/positions).
#include "nc_device.h"
#include "nc_chain.h"
#include "nc_internal.h"

namespace nc {

// Writes the Q8_0 block (32 values, one per lane of a half-wave) quantised as
// inference.rs:1012-1029, plus -8 * (the block's int8 sum) used by the Q4_0 GEMM.
__device__ __forceinline__ void store_q8_block(float y, int lane32, int8_t* q_dst, float* s_dst, int32_t* s8_dst) {
    const float amax = halfwave_amax(y);
    float scale;
    const int q = quantize_lane_q8(y, amax, &scale);
    const int qs = halfwave_isum(q);
    q_dst[lane32] = (int8_t)q;
    if (lane32 == 0) {
        *s_dst = scale;
        *s8_dst = -8 * qs;
    }
}

// ---------------------------------------------------------------- RMSNorm + Q8_0
// rms_norm (inference.rs:697-706): sum += x*x sequentially, scale = 1/sqrt(sum/n + eps),
// y = x*scale*w; then quantize_f32_to_q8_0 of y (inference.rs:3802-3808).  The sequential
// sum is evaluated by exact_chain_sum (bit-identical to the left-to-right loop).  One
// workgroup of 256 threads per row; thread t owns elements [t*E, t*E + E).
template <int E>
__global__ __launch_bounds__(256) void rmsnorm_q8_kernel(const float* hidden, const float* weight, float eps,
                                                          int8_t* xq, float* xs, int32_t* xsum) {
    constexpr int T = 256, d = T * E;
    __shared__ ChainScratch<T> sc;
    __shared__ float a_lds[d];
    const int n = blockIdx.x;
    const float* x = hidden + (size_t)n * d;
    float a[E];
#pragma unroll
    for (int j = 0; j < E; j++) {
        const float v = x[threadIdx.x * E + j];
        a[j] = v * v;
    }
    const float sum = exact_chain_sum<E, T>(a, sc, a_lds);
    const float scale = 1.0f / __builtin_sqrtf(sum / (float)d + eps);
    const int lane32 = threadIdx.x & 31;
    const int half = threadIdx.x >> 5;  // 8 half-waves
    for (int b = half; b < d / 32; b += T / 32) {
        const int i = b * 32 + lane32;
        const float y = x[i] * scale * weight[i];
        store_q8_block(y, lane32, xq + (size_t)n * d + b * 32, xs + (size_t)n * (d / 32) + b,
                       xsum + (size_t)n * (d / 32) + b);
    }
}

int launch_rmsnorm_q8(const float* hidden, const float* weight, int N, int d, float eps, int8_t* xq, float* xs,
                      int32_t* xsum, hipStream_t st) {
#define NC_RMS_CASE(E)                                                                                      \
    case E:                                                                                                 \
        hipLaunchKernelGGL(rmsnorm_q8_kernel<E>, dim3(N), dim3(256), 0, st, hidden, weight, eps, xq, xs, xsum); \
        break;
    switch (d % 256 ? 0 : d / 256) {
        NC_RMS_CASE(1)
        NC_RMS_CASE(2)
        NC_RMS_CASE(3)
        NC_RMS_CASE(4)
        NC_RMS_CASE(6)
        NC_RMS_CASE(8)
        NC_RMS_CASE(12)
        NC_RMS_CASE(16)
        NC_RMS_CASE(20)
        NC_RMS_CASE(24)
        NC_RMS_CASE(32)
        default:
            return fail(NC_EINVAL, "rmsnorm: width must be 256 * {1,2,3,4,6,8,12,16,20,24,32}");
    }
#undef NC_RMS_CASE
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- plain Q8_0 quantiser
__global__ void quantize_q8_kernel(const float* x, int dim, int nblocks_total, int8_t* xq, float* xs, int32_t* xsum) {
    const int gb = (blockIdx.x * blockDim.x + threadIdx.x) >> 5;  // global block id
    if (gb >= nblocks_total) return;                               // whole half-wave exits together
    const int lane32 = threadIdx.x & 31;
    const float y = x[(size_t)gb * 32 + lane32];
    store_q8_block(y, lane32, xq + (size_t)gb * 32, xs + gb, xsum + gb);
}

int launch_quantize_q8(const float* x, int N, int dim, int8_t* xq, float* xs, int32_t* xsum, hipStream_t st) {
    if (dim % 32) return fail(NC_EINVAL, "quantize: width must be a multiple of 32");
    const int total = N * (dim / 32);
    hipLaunchKernelGGL(quantize_q8_kernel, dim3((total * 32 + 255) / 256), dim3(256), 0, st, x, dim, total, xq, xs, xsum);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

__global__ void block_sums_kernel(const int8_t* x, int total_blocks, int32_t* xsum) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= total_blocks) return;
    const int8_t* p = x + (size_t)b * 32;
    int s = 0;
    for (int j = 0; j < 32; j++) s += p[j];
    xsum[b] = -8 * s;
}

int launch_block_sums(const int8_t* x, int N, int dim, int32_t* xsum, hipStream_t st) {
    const int total = N * (dim / 32);
    hipLaunchKernelGGL(block_sums_kernel, dim3((total + 255) / 256), dim3(256), 0, st, x, total, xsum);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- pass state
// Start position and the batch's token ids travel as kernel arguments (copied at
// launch), so back-to-back passes never race on a host staging buffer.
__global__ void set_pass_state_kernel(int32_t* d_pos, int32_t pos, uint32_t* d_toks, TokenArgs toks, int n) {
    const int i = threadIdx.x;
    if (i == 0) d_pos[0] = pos;
    if (i < n) d_toks[i] = toks.t[i];
}

int launch_set_pass_state(int32_t* d_pos, int32_t pos, uint32_t* d_toks, const uint32_t* toks, int n, hipStream_t st) {
    TokenArgs a{};
    for (int i = 0; i < n && i < 16; i++) a.t[i] = toks ? toks[i] : 0u;
    hipLaunchKernelGGL(set_pass_state_kernel, dim3(1), dim3(64), 0, st, d_pos, pos, d_toks, a, toks ? n : 0);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- embedding gather
__global__ void embed_kernel(const float* table, const uint32_t* toks, int d, float* hidden) {
    const int n = blockIdx.y;
    const size_t src = (size_t)toks[n] * d;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < d; i += gridDim.x * blockDim.x)
        hidden[(size_t)n * d + i] = table[src + i];
}

int launch_embed(const float* table, const uint32_t* toks, int N, int d, float* hidden, hipStream_t st) {
    hipLaunchKernelGGL(embed_kernel, dim3((d + 255) / 256, N), dim3(256), 0, st, table, toks, d, hidden);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- attention
// Phase 1: scores[n][h][p] = dot(q[n][h], k[p]) * scale for p <= pos_n
// (inference.rs:4252-4257; dot_f32_scalar folds a*b from -0.0 in index order).
// Workgroup = one KV head x 64 positions: the K tile is staged once in LDS (rows padded
// to HD+4 floats so the per-lane row reads are bank-conflict free) and shared by the
// G query-head waves; lane = position p, each lane keeps k_p in VGPRs across rows n.
template <int HD>
__global__ __launch_bounds__(1024) void attn_scores_kernel(AttnParams a) {
    constexpr int RS = HD + 4;
    __shared__ float kt[64 * RS];
    const int kvh = blockIdx.y;
    const int G = a.H / a.Hkv;
    const int g = wave_id_uniform();
    const int h = kvh * G + g;
    const int lane = threadIdx.x & 63;
    const int pos0 = a.d_pos[0];
    const int last = pos0 + a.N - 1;
    for (int tile = blockIdx.x; tile * 64 <= last; tile += gridDim.x) {
        __syncthreads();  // previous tile's readers are done with kt
        const int rows = min(64, last + 1 - tile * 64);
        const float4* src = (const float4*)(a.kcache + ((size_t)kvh * a.max_ctx + (size_t)tile * 64) * HD);
        for (int i = threadIdx.x; i < rows * (HD / 4); i += blockDim.x) {
            const int r = i / (HD / 4), c = i % (HD / 4);
            *(float4*)&kt[r * RS + c * 4] = src[(size_t)r * (HD / 4) + c];
        }
        __syncthreads();
        const int p = tile * 64 + lane;
        float k[HD];
        if (p <= last) {
#pragma unroll
            for (int i = 0; i < HD / 4; i++) {
                const float4 v = *(const float4*)&kt[lane * RS + i * 4];
                k[4 * i] = v.x;
                k[4 * i + 1] = v.y;
                k[4 * i + 2] = v.z;
                k[4 * i + 3] = v.w;
            }
        }
        for (int n = 0; n < a.N; n++) {
            if (tile * 64 > pos0 + n) continue;  // uniform: whole tile beyond this row
            const float __attribute__((address_space(4)))* q =
                (const float __attribute__((address_space(4)))*)(const void __attribute__((address_space(4)))*)(
                    uintptr_t)(a.q + (size_t)n * a.H * HD + (size_t)h * HD);
            float dot = -0.0f;
#pragma unroll
            for (int i = 0; i < HD; i++) dot = dot + q[i] * k[i];
            if (p <= pos0 + n) a.scores[((size_t)n * a.H + h) * a.max_ctx + p] = dot * a.scale;
        }
    }
}

// Phase 2 (fused): softmax over 0..=pos (inference.rs:3522-3540) and the weighted V sum
// (add_weighted_f32_scalar, inference.rs:3603-3623) for two (row, head) units per
// workgroup; half-wave u owns unit u and 32 output dims.  max is order free; e_p =
// expf(s_p - max) goes to LDS; lane 0 of the half-wave adds e_0, e_1, ... in order;
// prob_p = e_p * (1/sum); out[d] = ((0 + prob_0*v_0[d]) + prob_1*v_1[d]) + ... in order.
// The output block of 32 dims is then quantised to Q8_0 for the wo matmul.
__global__ __launch_bounds__(64) void attn_softmax_pv_kernel(AttnParams a) {
    extern __shared__ float e[];  // [2][a.max_pos + 1 rounded up to 4]
    const int kvh = blockIdx.x;
    const int dchunk = blockIdx.y;
    const int G = a.H / a.Hkv;
    const int lane = threadIdx.x & 63;
    const int u = lane >> 5, lane32 = lane & 31;
    const int unit = blockIdx.z * 2 + u;  // (n, g) pair
    const bool active = unit < a.N * G;  // half-wave uniform
    const int n = active ? unit / G : 0, g = active ? unit % G : 0;
    const int h = kvh * G + g;
    const int L = a.d_pos[0] + n + 1;
    const int stride = ((a.max_pos + 1) + 3) & ~3;
    float* eu = e + u * stride;
    const float* s = a.scores + ((size_t)n * a.H + h) * a.max_ctx;
    float mx = -__builtin_inff();
    if (active)
        for (int p = lane32; p < L; p += 32) {
            const float v = s[p];
            mx = v > mx ? v : mx;
        }
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off, 64);
        mx = o > mx ? o : mx;
    }
    if (active)
        for (int p = lane32; p < L; p += 32) eu[p] = expf_glibc(s[p] - mx);
    __syncthreads();
    float inv = 0.0f;
    if (active && lane32 == 0) {
        float sum = 0.0f;
        int p = 0;
        for (; p + 32 <= L; p += 32) {
            float4 v[8];
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = *(const float4*)&eu[p + 4 * j];
#pragma unroll
            for (int j = 0; j < 8; j++) {
                sum = sum + v[j].x;
                sum = sum + v[j].y;
                sum = sum + v[j].z;
                sum = sum + v[j].w;
            }
        }
        for (; p < L; p++) sum = sum + eu[p];
        inv = 1.0f / sum;
    }
    inv = __shfl(inv, u * 32, 64);
    if (!active) return;  // no barriers below
    const int d = dchunk * 32 + lane32;
    const float* v = a.vcache + (size_t)kvh * a.max_ctx * a.hd + d;
    float acc = 0.0f;
    int p = 0;
    for (; p + 16 <= L; p += 16) {
        float vv[16], pr[16];
#pragma unroll
        for (int j = 0; j < 16; j++) vv[j] = v[(size_t)(p + j) * a.hd];
#pragma unroll
        for (int j = 0; j < 16; j++) pr[j] = eu[p + j] * inv;
#pragma unroll
        for (int j = 0; j < 16; j++) acc = acc + pr[j] * vv[j];
    }
    for (; p < L; p++) acc = acc + (eu[p] * inv) * v[(size_t)p * a.hd];
    const int aw = a.H * a.hd;
    const int col = h * a.hd + dchunk * 32;
    store_q8_block(acc, lane32, a.xq + (size_t)n * aw + col, a.xs + (size_t)n * (aw / 32) + col / 32,
                   a.xs8 + (size_t)n * (aw / 32) + col / 32);
}

int launch_attention(const AttnParams& a, hipStream_t st) {
    const int G = a.H / a.Hkv;
    if (G > 16 || a.H % a.Hkv) return fail(NC_EINVAL, "attention: at most 16 query heads per KV head supported");
    const int tiles = (a.max_pos + 64) / 64;
    if (a.hd == 128)
        hipLaunchKernelGGL(attn_scores_kernel<128>, dim3(tiles, a.Hkv), dim3(64 * G), 0, st, a);
    else if (a.hd == 64)
        hipLaunchKernelGGL(attn_scores_kernel<64>, dim3(tiles, a.Hkv), dim3(64 * G), 0, st, a);
    else
        return fail(NC_EINVAL, "attention: head_dim must be 64 or 128");
    NC_HIP(hipGetLastError());
    const size_t lds = 2 * (size_t)(((a.max_pos + 1) + 3) & ~3) * sizeof(float);
    if (lds > 160 * 1024) return fail(NC_ERANGE, "attention: context too long for the fused softmax kernel");
    hipLaunchKernelGGL(attn_softmax_pv_kernel, dim3(a.Hkv, a.hd / 32, (a.N * G + 1) / 2), dim3(64), lds, st, a);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- head argmax + acceptance
// First maximum over the per-tile partials (tiles are in row order).
__global__ void argmax_final_kernel(const float* pv, const int32_t* pi, int ntiles, uint32_t* preds) {
    const int n = blockIdx.x;
    __shared__ float sv[256];
    __shared__ int si[256];
    float bv = -__builtin_inff();
    int bi = 0x7fffffff;
    for (int t = threadIdx.x; t < ntiles; t += blockDim.x) {
        const float v = pv[(size_t)n * ntiles + t];
        const int i = pi[(size_t)n * ntiles + t];
        if (v > bv || (v == bv && i < bi)) {
            bv = v;
            bi = i;
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int off = 128; off >= 1; off >>= 1) {
        if (threadIdx.x < off) {
            const float ov = sv[threadIdx.x + off];
            const int oi = si[threadIdx.x + off];
            if (ov > sv[threadIdx.x] || (ov == sv[threadIdx.x] && oi < si[threadIdx.x])) {
                sv[threadIdx.x] = ov;
                si[threadIdx.x] = oi;
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) preds[n] = (uint32_t)(si[0] == 0x7fffffff ? 0 : si[0]);
}

int launch_argmax_final(const float* part_val, const int32_t* part_idx, int N, int ntiles, uint32_t* preds,
                        hipStream_t st) {
    hipLaunchKernelGGL(argmax_final_kernel, dim3(N), dim3(256), 0, st, part_val, part_idx, ntiles, preds);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// cluster_tcp_smoke.rs:954-979: accepted = longest prefix with draft[i] == pred[i],
// next = pred[accepted], pos += accepted + 1.  result = {accepted, next, new_pos}.
__global__ void accept_greedy_kernel(const uint32_t* toks, const uint32_t* preds, int n, int32_t* d_pos,
                                     int32_t* result, uint32_t* next_tok_slot) {
    if (threadIdx.x != 0) return;
    int a = 0;
    while (a < n - 1 && toks[a + 1] == preds[a]) a++;
    const uint32_t next = preds[a];
    const int np = d_pos[0] + a + 1;
    result[0] = a;
    result[1] = (int32_t)next;
    result[2] = np;
    d_pos[0] = np;
    if (next_tok_slot) next_tok_slot[0] = next;
}

int launch_accept_greedy(const uint32_t* toks, const uint32_t* preds, int n, int32_t* d_pos, int32_t* result,
                         uint32_t* next_tok_slot, hipStream_t st) {
    hipLaunchKernelGGL(accept_greedy_kernel, dim3(1), dim3(64), 0, st, toks, preds, n, d_pos, result, next_tok_slot);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
