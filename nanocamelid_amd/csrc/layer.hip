// Row ops of the verify forward on gfx950: fused RMSNorm + Q8_0 quantisation,
// activation quantisation, embedding gather, causal GQA attention over the
// HBM-resident f32 KV cache (with the Q8_0 quantisation of its output fused in),
// the head argmax reduction and greedy acceptance.
//
// Every f32 chain that the reference evaluates sequentially gives the same bits here:
// the RMSNorm sum of squares and the softmax denominator go through exact_chain_sum (a
// parallel evaluation that is verified step by step against the sequential recurrence);
// each attention dot product and the weighted V sum are evaluated in order.  The parallel
// parts are the order-free ones (max, elementwise maps, integer sums, independent
// rows/heads/positions).  The one exception is opt-in: the split-position attention
// (NC_ATTN_SPLIT) sums in a fixed chunked order of its own.
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
// Q8_0 quantisation of a row held in LDS (quantize_f32_to_q8_0, inference.rs:1012-1029):
// 8 lanes per 32-block, 4 values per lane, all blocks of the row in one pass.
template <int T>
__device__ __forceinline__ void quantize_row_lds_q8(const float* y, int d, int8_t* q, float* s, int32_t* s8) {
    for (int g = threadIdx.x; g < d / 4; g += T) {  // d % 32 == 0: 8-lane groups stay whole
        const float4 v = *(const float4*)(y + 4 * g);
        float amax = __builtin_fabsf(v.x);
        amax = __builtin_fabsf(v.y) > amax ? __builtin_fabsf(v.y) : amax;
        amax = __builtin_fabsf(v.z) > amax ? __builtin_fabsf(v.z) : amax;
        amax = __builtin_fabsf(v.w) > amax ? __builtin_fabsf(v.w) : amax;
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) {
            const float o = __shfl_xor(amax, off, 8);
            amax = o > amax ? o : amax;
        }
        float scale;
        const int q0 = quantize_lane_q8(v.x, amax, &scale);
        const int q1 = quantize_lane_q8(v.y, amax, &scale);
        const int q2 = quantize_lane_q8(v.z, amax, &scale);
        const int q3 = quantize_lane_q8(v.w, amax, &scale);
        int qs = q0 + q1 + q2 + q3;
#pragma unroll
        for (int off = 1; off < 8; off <<= 1) qs += __shfl_xor(qs, off, 8);
        *(int*)(q + 4 * g) = (q0 & 0xff) | ((q1 & 0xff) << 8) | ((q2 & 0xff) << 16) | ((q3 & 0xff) << 24);
        if ((g & 7) == 0) {
            s[g >> 3] = scale;
            s8[g >> 3] = -8 * qs;
        }
    }
}

// Exact max / sum over aligned groups of W lanes (W = 1, 2, 4, ..., 32).
template <int W>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (W >= 2) {
        const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xb1, 0xf, 0xf, false));
        v = o > v ? o : v;
    }
    if constexpr (W >= 4) {
        const float o = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4e, 0xf, 0xf, false));
        v = o > v ? o : v;
    }
#pragma unroll
    for (int off = 4; off < W; off <<= 1) {
        const float o = __shfl_xor(v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}
template <int W>
__device__ __forceinline__ int group_sum(int v) {
    if constexpr (W >= 2) v += __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false);
    if constexpr (W >= 4) v += __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false);
#pragma unroll
    for (int off = 4; off < W; off <<= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// Q8_0 quantisation (inference.rs:1012-1029) of a row whose 32-blocks are split across
// 32/E consecutive lanes holding E values each (register resident, no LDS).
template <int E>
__device__ __forceinline__ void quantize_regs_q8(const float (&y)[E], int8_t* q_row, float* s_row, int32_t* s8_row) {
    constexpr int W = 32 / E;
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < E; j++) amax = __builtin_fabsf(y[j]) > amax ? __builtin_fabsf(y[j]) : amax;
    amax = group_max<W>(amax);
    const float scale = amax / 127.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    int qv[E];
    int qs = 0;
#pragma unroll
    for (int j = 0; j < E; j++) {
        float r = round_half_away(y[j] * inv);
        r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
        qv[j] = scale > 0.0f ? (int)r : 0;
        qs += qv[j];
    }
    qs = group_sum<W>(qs);
    int8_t* dst = q_row + threadIdx.x * E;
    if constexpr (E >= 4) {
#pragma unroll
        for (int j = 0; j < E; j += 4)
            *(int*)(dst + j) = (qv[j] & 0xff) | ((qv[j + 1] & 0xff) << 8) | ((qv[j + 2] & 0xff) << 16) |
                               ((qv[j + 3] & 0xff) << 24);
    } else {
#pragma unroll
        for (int j = 0; j < E; j++) dst[j] = (int8_t)qv[j];
    }
    if (threadIdx.x % W == 0) {
        const int b = threadIdx.x / W;
        s_row[b] = scale;
        s8_row[b] = -8 * qs;
    }
}

// rms_norm (inference.rs:697-706): sum += x*x sequentially, scale = 1/sqrt(sum/n + eps),
// y = x*scale*w; then quantize_f32_to_q8_0 of y (inference.rs:3802-3808).  The sequential
// sum is evaluated by exact_chain_sum (bit-identical to the left-to-right loop).  One
// workgroup of T threads (256 or 1024) per row; thread t owns elements [t*E, t*E + E).
template <int E, int T>
__global__ __launch_bounds__(T) void rmsnorm_q8_kernel(const float* hidden, const float* weight, float eps,
                                                        int8_t* xq, float* xs, int32_t* xsum) {
    constexpr int d = T * E;
    __shared__ ChainScratch<T> sc;
    __shared__ __align__(16) float a_lds[d];
    const int n = blockIdx.x;
    const float* x = hidden + (size_t)n * d;
    float xv[E], wv[E], a[E];
#pragma unroll
    for (int j = 0; j < E; j++) {
        xv[j] = x[threadIdx.x * E + j];
        wv[j] = weight[threadIdx.x * E + j];
    }
#pragma unroll
    for (int j = 0; j < E; j++) a[j] = xv[j] * xv[j];
    const float sum = exact_chain_sum<E, T>(a, sc, a_lds);
    const float scale = 1.0f / __builtin_sqrtf(sum / (float)d + eps);
    float y[E];
#pragma unroll
    for (int j = 0; j < E; j++) y[j] = xv[j] * scale * wv[j];
    int8_t* q_row = xq + (size_t)n * d;
    float* s_row = xs + (size_t)n * (d / 32);
    int32_t* s8_row = xsum + (size_t)n * (d / 32);
    if constexpr (32 % E == 0) {
        quantize_regs_q8<E>(y, q_row, s_row, s8_row);
    } else {
#pragma unroll
        for (int j = 0; j < E; j++) a_lds[threadIdx.x * E + j] = y[j];
        __syncthreads();
        quantize_row_lds_q8<T>(a_lds, d, q_row, s_row, s8_row);
    }
}

int launch_rmsnorm_q8(const float* hidden, const float* weight, int N, int d, float eps, int8_t* xq, float* xs,
                      int32_t* xsum, hipStream_t st) {
    // One workgroup per row.  Wide rows use 512 threads (measured fastest: 5 rows at d = 4096
    // 4.9 us against 6.0 us for 1024 threads, at d = 8192 6.4 against 6.8 us; 256 threads were
    // slower still), small ones 256.
#define NC_RMS(E, T)                                                                                     \
    NC_LAUNCH((rmsnorm_q8_kernel<E, T>), dim3(N), dim3(T), 0, st, hidden, weight, eps, xq, xs, xsum); \
    break;
    switch (d) {
        case 256: NC_RMS(1, 256)
        case 512: NC_RMS(2, 256)
        case 768: NC_RMS(3, 256)
        case 1024: NC_RMS(4, 256)
        case 1536: NC_RMS(6, 256)
        case 2048: NC_RMS(4, 512)
        case 3072: NC_RMS(6, 512)
        case 4096: NC_RMS(8, 512)
        case 5120: NC_RMS(10, 512)
        case 6144: NC_RMS(12, 512)
        case 8192: NC_RMS(16, 512)
        default:
            return fail(NC_EINVAL, "rmsnorm: width must be one of 256, 512, 768, 1024, 1536, 2048, 3072, 4096, "
                                   "5120, 6144, 8192");
    }
#undef NC_RMS
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

// expf_glibc over consecutive input bit patterns first, first + 1, ... (a parity check of the
// device restatement against the host's glibc expf, which Rust's f32::exp calls)
__global__ void expf_range_kernel(uint32_t first, int64_t count, float* out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = expf_glibc(__uint_as_float(first + (uint32_t)i));
}

int launch_expf_range(uint32_t first, int64_t count, float* out, hipStream_t st) {
    if (count < 0 || count > ((int64_t)1 << 32)) return fail(NC_ERANGE, "expf range: 0..2^32 values");
    if (count == 0) return NC_OK;
    const int64_t blocks = std::min<int64_t>((count + 255) / 256, 65536);
    NC_LAUNCH(expf_range_kernel, dim3((unsigned)blocks), dim3(256), 0, st, first, count, out);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int launch_quantize_q8(const float* x, int N, int dim, int8_t* xq, float* xs, int32_t* xsum, hipStream_t st) {
    if (dim % 32) return fail(NC_EINVAL, "quantize: width must be a multiple of 32");
    const int total = N * (dim / 32);
    NC_LAUNCH(quantize_q8_kernel, dim3((total * 32 + 255) / 256), dim3(256), 0, st, x, dim, total, xq, xs, xsum);
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
    NC_LAUNCH(block_sums_kernel, dim3((total + 255) / 256), dim3(256), 0, st, x, total, xsum);
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
    NC_LAUNCH(set_pass_state_kernel, dim3(1), dim3(64), 0, st, d_pos, pos, d_toks, a, toks ? n : 0);
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
    NC_LAUNCH(embed_kernel, dim3((d + 255) / 256, N), dim3(256), 0, st, table, toks, d, hidden);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// ---------------------------------------------------------------- attention
// Phase 1: scores[n][h][p] = dot(q[n][h], k[p]) * scale for p <= pos_n
// (inference.rs:4252-4257; dot_f32_scalar folds a*b from -0.0 in index order).
// Workgroup = one KV head x 64 positions: the K tile is staged once in LDS (rows padded
// to HD+4 floats so the per-lane row reads are bank-conflict free) and shared by the
// G query-head waves; lane = position p reads its key row from LDS (4 floats a step).
// RB rows' dot chains are interleaved (each chain is sequential in i, the rows are
// independent); their q vectors sit in LDS and are read as wave-wide broadcasts.
template <int HD, int RB>
__global__ __launch_bounds__(512) void attn_scores_kernel(AttnParams a) {
    constexpr int RS = HD + 4;
    __shared__ float kt[64 * RS];
    __shared__ __align__(16) float qs[8][RB][HD];  // [head in group][row][dim]
    const int kvh = blockIdx.x;  // KV head fastest: one XCD per KV head (see attn_fused_kernel)
    const int G = a.H / a.Hkv;
    const int g = wave_id_uniform();
    const int h = kvh * G + g;
    const int lane = threadIdx.x & 63;
    const int pos0 = a.d_pos[0];
    const int last = pos0 + a.N - 1;
    for (int tile = blockIdx.y; tile * 64 <= last; tile += gridDim.y) {
        __syncthreads();  // previous tile's readers are done with kt
        if (tile * 64 > pos0 + min(a.N, ((int)blockIdx.z + 1) * RB) - 1) break;  // no row of this block reaches it
        const int rows = min(64, last + 1 - tile * 64);
        // keys are stored as dim quads [HD/4][max_ctx][4]: quad c of the tile's rows is
        // 16 * rows contiguous bytes
        const float4* src = (const float4*)a.kcache + (size_t)kvh * (HD / 4) * a.max_ctx + (size_t)tile * 64;
        for (int i = threadIdx.x; i < rows * (HD / 4); i += blockDim.x) {
            const int c = i / rows, r = i % rows;
            *(float4*)&kt[r * RS + c * 4] = src[(size_t)c * a.max_ctx + r];
        }
        __syncthreads();
        const int p = tile * 64 + lane;
        const float* krow = &kt[lane * RS];  // this lane's key row (stale for p > last: unused)
        // this block's rows: n = blockIdx.z*RB .. +RB-1 whose window reaches this tile
        // (n >= tile*64 - pos0; uniform over the block)
        const int n_first = max((int)blockIdx.z * RB, tile * 64 - pos0);
        for (int n0 = n_first; n0 < min(a.N, ((int)blockIdx.z + 1) * RB); n0 += RB) {
            // this wave's head: q rows n0 .. n0+RB-1 into LDS (each wave owns its slice)
#pragma unroll
            for (int r = 0; r < RB; r++) {
                const int n = min(n0 + r, a.N - 1);
                const float* qrow = a.q + (size_t)n * a.H * HD + (size_t)h * HD;
                for (int i = lane; i < HD; i += 64) qs[g][r][i] = qrow[i];
            }
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float dot[RB];
#pragma unroll
            for (int r = 0; r < RB; r++) dot[r] = -0.0f;
#pragma unroll 4
            for (int i = 0; i < HD; i += 4) {
                const float4 kv = *(const float4*)&krow[i];
#pragma unroll
                for (int r = 0; r < RB; r++) {
                    const float4 qv = *(const float4*)&qs[g][r][i];
                    dot[r] = dot[r] + qv.x * kv.x;
                    dot[r] = dot[r] + qv.y * kv.y;
                    dot[r] = dot[r] + qv.z * kv.z;
                    dot[r] = dot[r] + qv.w * kv.w;
                }
            }
#pragma unroll
            for (int r = 0; r < RB; r++) {
                const int n = n0 + r;
                if (n < a.N && p <= pos0 + n) a.scores[((size_t)n * a.H + h) * a.max_ctx + p] = dot[r] * a.scale;
            }
            __builtin_amdgcn_wave_barrier();  // readers done before the next group overwrites qs
        }
    }
}

// Phase 2 (fused), one workgroup of T threads per (row n, head h) unit: softmax over
// 0..=pos (inference.rs:3522-3540) then the weighted V sum (add_weighted_f32_scalar,
// inference.rs:3603-3623) and the Q8_0 quantisation of the output for the wo matmul.
//   max: order free (block reduction); e_p = expf(s_p - max) in parallel;
//   sum = e_0 + e_1 + ... left to right: exact_chain_sum (bit-identical);
//   prob_p = e_p * (1/sum);  out[d] = ((0 + prob_0*v_0[d]) + prob_1*v_1[d]) + ... in order,
//   one lane per output dim d, V rows streamed with a software-pipelined prefetch.
// Thread t owns positions [t*E, t*E + E) of the score row (zeros past the row's end).
// softmax (inference.rs:3522-3540) of the score row srow[0 .. L): max, e = expf(s - max),
// the sum of e left to right (exact_chain_sum), p = e * (1 / sum).  Thread t returns the
// probabilities of positions t*E .. t*E + E - 1 (0 past L).  Every thread of the block calls
// it; lds_terms: T*E floats used by the chain.
// X = 1: the row continues for up to T more positions, thread t holding position T*E + t; its
// e joins the chain after the first T*E terms (exact_chain_sum from the carried sum, with
// lds_terms + T*E as its T floats of scratch) and its probability is returned in *px.
template <int E, int T, int X = 0>
__device__ __forceinline__ void softmax_row(const float* srow, int L, float (&pr)[E], ChainScratch<T>& sc,
                                            float* lds_terms, float* red, float* px = nullptr) {
    const int t = threadIdx.x;
    float sv[E];
#pragma unroll
    for (int j = 0; j < E; j++) {
        const int p = t * E + j;
        sv[j] = p < L ? srow[p] : -__builtin_inff();
    }
    const int px_pos = T * E + t;
    const float svx = X && px_pos < L ? srow[px_pos] : -__builtin_inff();
    float mx = sv[0];
#pragma unroll
    for (int j = 1; j < E; j++) mx = sv[j] > mx ? sv[j] : mx;
    if (X) mx = svx > mx ? svx : mx;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(mx, off, 64);
        mx = o > mx ? o : mx;
    }
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = red[0];
#pragma unroll
    for (int w = 1; w < T / 64; w++) mx = red[w] > mx ? red[w] : mx;
    float e[E];
#pragma unroll
    for (int j = 0; j < E; j++) e[j] = t * E + j < L ? expf_glibc(sv[j] - mx) : 0.0f;
    float sum = exact_chain_sum<E, T>(e, sc, lds_terms);
    float ex[1] = {0.0f};
    if constexpr (X) {
        ex[0] = px_pos < L ? expf_glibc(svx - mx) : 0.0f;
        sum = exact_chain_sum<1, T>(ex, sc, lds_terms + T * E, sum);
    }
    const float inv = 1.0f / sum;
#pragma unroll
    for (int j = 0; j < E; j++) pr[j] = e[j] * inv;
    if constexpr (X) *px = ex[0] * inv;
}

// The weighted V sum of unit (n, h) over positions 0..L-1 (probabilities in LDS) and the
// Q8_0 quantisation of its output block; threads past the head dim return at once.
template <int HD, bool PIPE>
__device__ __forceinline__ void weighted_v_q8(const AttnParams& a, int n, int h, int kvh, int L, const float* probs) {
    const int t = threadIdx.x;
    if (t >= HD) return;
    // Weighted V sum, lane = output dim t.  V is stored in position quads: one 16-byte load
    // brings positions 4q..4q+3 of this lane's dim (consecutive lanes read consecutive 16
    // bytes).  A ring of D batches of B quads keeps (D-1)*B*4 positions in flight.  The loads
    // are buffer loads whose quad offset is wave-uniform (scalar registers) and clamped, so
    // they are unconditional, need no per-lane address arithmetic, and keep the wait counts
    // exact; each batch's loads are pinned in order.  The batch's probabilities are read
    // from LDS one batch ahead, so neither latency is exposed in the chain.  V rows come from
    // HBM (a decode step streams the weights between two reads of a layer's cache), where
    // three batches in flight (D = 4) run the chain at ~17 cycles per position against ~25
    // for one; with the rows hot in L2 the two are equal.
    // PIPE selects a software-pipelined loop (below) for launches where several chains share
    // a SIMD; with one chain per SIMD the plain loop is as fast or faster.
    constexpr int HDv = HD;
    typedef float f4v __attribute__((ext_vector_type(4)));
    const char* vbase = (const char*)(a.vcache + (size_t)kvh * a.max_ctx * HD);
    const __amdgpu_buffer_rsrc_t vres =
        __builtin_amdgcn_make_buffer_rsrc((void*)vbase, 0, a.max_ctx * HD * 4, 0x00020000);
    const int voff = t * 16;
    constexpr int B = 8, D = 4;
    static_assert(D % 2 == 0, "probability slots follow the unrolled batch index");
    const int nq = L >> 2;    // whole position quads
    const int nbt = nq / B;   // whole batches
    float acc = 0.0f;
    if (nbt > 0) {
        f4v ring[D][B];
        f4v pq[2][B];
#define NC_PV_LOAD(BT, SLOT)                                                                        \
        {                                                                                           \
            const int bq_ = min((BT), nbt - 1) * B;                                                 \
            _Pragma("unroll") for (int j = 0; j < B; j++) ring[SLOT][j] = __builtin_bit_cast(        \
                f4v, __builtin_amdgcn_raw_buffer_load_b128(vres, voff, (bq_ + j) * (HD * 16), 0));  \
            __builtin_amdgcn_sched_barrier(0);                                                      \
        }
#define NC_PV_PROBS(BT, SLOT)                                                                       \
        {                                                                                           \
            const float* pp_ = &probs[min((BT), nbt - 1) * B * 4];                                  \
            _Pragma("unroll") for (int j = 0; j < B; j++) pq[SLOT][j] = *(const f4v*)(pp_ + 4 * j); \
        }
        if constexpr (!PIPE) {
#pragma unroll
        for (int k = 0; k < D - 1; k++) NC_PV_LOAD(k, k)
        NC_PV_PROBS(0, 0)
        for (int b0 = 0; b0 < nbt; b0 += D) {
#pragma unroll
            for (int k = 0; k < D; k++) {
                const int b = b0 + k;
                NC_PV_LOAD(b + D - 1, (k + D - 1) % D)
                NC_PV_PROBS(b + 1, (k + 1) & 1)
                if (b < nbt) {
#pragma unroll
                    for (int j = 0; j < B; j++) {
                        const f4v p4 = pq[k & 1][j];
                        const f4v v = ring[k][j];
                        acc = acc + p4.x * v.x;
                        acc = acc + p4.y * v.y;
                        acc = acc + p4.z * v.z;
                        acc = acc + p4.w * v.w;
                    }
                }
            }
        }
        } else {
        // Software pipeline: while batch b's products are added (a dependent chain, one add per
        // add latency), batch b+1's products are formed in the issue slots between the adds.
        // Each inline-asm group alternates "acc += prod" with "prod' = p * v" of the next batch,
        // the same IEEE operations in the same order as the sequential loop.
        f4v pr[B];  // products of the batch being added
#pragma unroll
        for (int k = 0; k < D - 1; k++) NC_PV_LOAD(k, k)
        NC_PV_PROBS(0, 0)
        NC_PV_PROBS(1, 1)
#pragma unroll
        for (int j = 0; j < B; j++) pr[j] = pq[0][j] * ring[0][j];
        for (int b0 = 0; b0 < nbt; b0 += D) {
#pragma unroll
            for (int k = 0; k < D; k++) {
                const int b = b0 + k;
                NC_PV_LOAD(b + D - 1, (k + D - 1) % D)
                if (b < nbt) {
#pragma unroll
                    for (int j = 0; j < B; j++) {
                        const f4v p4 = pq[(k + 1) & 1][j];
                        const f4v v = ring[(k + 1) % D][j];
                        float c0 = pr[j].x, c1 = pr[j].y, c2 = pr[j].z, c3 = pr[j].w;
                        asm volatile(
                            "v_add_f32 %0, %0, %1\n\t"
                            "v_mul_f32 %1, %5, %9\n\t"
                            "v_add_f32 %0, %0, %2\n\t"
                            "v_mul_f32 %2, %6, %10\n\t"
                            "v_add_f32 %0, %0, %3\n\t"
                            "v_mul_f32 %3, %7, %11\n\t"
                            "v_add_f32 %0, %0, %4\n\t"
                            "v_mul_f32 %4, %8, %12"
                            : "+v"(acc), "+v"(c0), "+v"(c1), "+v"(c2), "+v"(c3)
                            : "v"(p4.x), "v"(p4.y), "v"(p4.z), "v"(p4.w), "v"(v.x), "v"(v.y), "v"(v.z), "v"(v.w));
                        pr[j] = f4v{c0, c1, c2, c3};
                    }
                }
                NC_PV_PROBS(b + 2, k & 1)
            }
        }
        }
#undef NC_PV_PROBS
#undef NC_PV_LOAD
    }
    {
        // the remaining whole quads (fewer than B) and the last partial quad: one batch of
        // loads (quads clamped to the last one holding a position) and probabilities, then
        // the chain; a position past the row leaves acc unchanged (a select, not a branch)
        const int q0 = nbt * B;
        const int qlast = (L - 1) >> 2;
        f4v tv[B], tp[B];
#pragma unroll
        for (int j = 0; j < B; j++) {
            const int q = min(q0 + j, qlast);
            tv[j] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(vres, voff, q * (HD * 16), 0));
            tp[j] = *(const f4v*)&probs[4 * q];
        }
#pragma unroll
        for (int j = 0; j < B; j++) {
            const int p0 = (q0 + j) * 4;
            acc = p0 < L ? acc + tp[j].x * tv[j].x : acc;
            acc = p0 + 1 < L ? acc + tp[j].y * tv[j].y : acc;
            acc = p0 + 2 < L ? acc + tp[j].z * tv[j].z : acc;
            acc = p0 + 3 < L ? acc + tp[j].w * tv[j].w : acc;
        }
    }
    const int aw = a.H * HDv;
    const int col = h * HDv + (t & ~31);
    store_q8_block(acc, t & 31, a.xq + (size_t)n * aw + col, a.xs + (size_t)n * (aw / 32) + col / 32,
                   a.xs8 + (size_t)n * (aw / 32) + col / 32);
}

template <int E, int T, int HD, bool PIPE, int X = 0>
__global__ __launch_bounds__(T) void attn_softmax_pv_kernel(AttnParams a) {
    __shared__ ChainScratch<T> sc;
    __shared__ __align__(16) float probs[T * E + X * T];
    __shared__ float red[T / 64];
    // unit order: KV head fastest, so that with round-robin dispatch over the 8 XCDs (and 8
    // KV heads) every unit of a KV head lands on one XCD and its keys and values stay in that
    // XCD's L2 instead of being re-read through the shared cache
    const int G = a.H / a.Hkv;
    const int kvh = blockIdx.x % a.Hkv, j = blockIdx.x / a.Hkv;
    const int n = j / G, h = kvh * G + j % G;
    const int L = a.d_pos[0] + n + 1;
    const int t = threadIdx.x;
    const float* srow = a.scores + ((size_t)n * a.H + h) * a.max_ctx;
    float pr[E], px = 0.0f;
    softmax_row<E, T, X>(srow, L, pr, sc, probs, red, &px);
#pragma unroll
    for (int j = 0; j < E; j++) probs[t * E + j] = pr[j];
    if (X) probs[T * E + t] = px;
    __syncthreads();
    weighted_v_q8<HD, PIPE>(a, n, h, kvh, L, probs);  // no barriers below
}

// Attention of one (row n, head h) unit in one kernel, for rows of at most T*E <= 1536
// positions: the scores (as attn_scores_kernel: dot from -0.0 over the head dims in order,
// then * scale) go to LDS, then the softmax and the weighted V sum as attn_softmax_pv_kernel.
// Thread t scores positions t, t + T, ..., so a wave's key loads are consecutive positions:
// keys are stored as dim quads [HD/4][max_ctx][4], one 16-byte load brings 4 dims of a
// position and a wave load is 1 KB contiguous.  A ring of KD dim quads of loads is in
// flight; a position past the row reads outside the buffer (0, no memory access) and its
// score is not stored.
template <int E, int T, int HD>
__global__ __launch_bounds__(T) void attn_fused_kernel(AttnParams a) {
    static_assert(T * E <= 1536, "rows up to 1536 positions");
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ ChainScratch<T> sc;
    __shared__ __align__(16) float probs[T * E];  // scores, then probabilities
    __shared__ float red[T / 64];
    __shared__ __align__(16) float qs[HD];
    // unit order: KV head fastest, so that with round-robin dispatch over the 8 XCDs (and 8
    // KV heads) every unit of a KV head lands on one XCD and its keys and values stay in that
    // XCD's L2 instead of being re-read through the shared cache
    const int G = a.H / a.Hkv;
    const int kvh = blockIdx.x % a.Hkv, j = blockIdx.x / a.Hkv;
    const int n = j / G, h = kvh * G + j % G;
    const int L = a.d_pos[0] + n + 1;
    const int t = threadIdx.x;
    if (t < HD) qs[t] = a.q[((size_t)n * a.H + h) * HD + t];
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.kcache + (size_t)kvh * a.max_ctx * HD), 0, a.max_ctx * HD * 4, 0x00020000);
    int koff[E];
#pragma unroll
    for (int m = 0; m < E; m++) koff[m] = t + T * m < L ? (t + T * m) * 16 : 0x40000000;
    const int qstride = a.max_ctx * 16;  // bytes between dim quads
    constexpr int KD = E <= 2 ? 8 : 4;   // dim quads in the ring (4 x E loads at E = 4: registers)
    constexpr int NQ = HD / 4;
    static_assert(NQ % KD == 0, "ring divides the dim quads");
    f4v kr[KD][E];
#define NC_K_LOAD(I, SLOT)                                                                              \
    {                                                                                                   \
        const int so_ = min((I), NQ - 1) * qstride;                                                     \
        _Pragma("unroll") for (int m = 0; m < E; m++) kr[SLOT][m] =                                     \
            __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(kres, koff[m], so_, 0));       \
        __builtin_amdgcn_sched_barrier(0);                                                              \
    }
#pragma unroll
    for (int k = 0; k < KD - 1; k++) NC_K_LOAD(k, k)
    __syncthreads();  // q in LDS
    float dot[E];
#pragma unroll
    for (int m = 0; m < E; m++) dot[m] = -0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < NQ; i0 += KD) {
#pragma unroll
        for (int k = 0; k < KD; k++) {
            const int i = i0 + k;
            NC_K_LOAD(i + KD - 1, (k + KD - 1) % KD)
            const f4v qv = *(const f4v*)&qs[4 * i];
#pragma unroll
            for (int m = 0; m < E; m++) {
                const f4v kv = kr[k][m];
                dot[m] = dot[m] + qv.x * kv.x;
                dot[m] = dot[m] + qv.y * kv.y;
                dot[m] = dot[m] + qv.z * kv.z;
                dot[m] = dot[m] + qv.w * kv.w;
            }
        }
    }
#undef NC_K_LOAD
#pragma unroll
    for (int m = 0; m < E; m++)
        if (t + T * m < L) probs[t + T * m] = dot[m] * a.scale;
    __syncthreads();
    float pr[E];
    softmax_row<E, T>(probs, L, pr, sc, probs, red);
#pragma unroll
    for (int j = 0; j < E; j++) probs[t * E + j] = pr[j];
    __syncthreads();
    weighted_v_q8<HD, false>(a, n, h, kvh, L, probs);  // no barriers below
}

// ---------------------------------------------------------------- split-position attention
// NC_ATTN_SPLIT.  The reference's attention (inference.rs:3522-3540 softmax, 3603-3623 weighted
// V sum) with its sums taken in a fixed split order instead of left to right: the positions of
// a row are cut into chunks of kSplitChunk, and per (query, chunk)
//   m_c = max s_p,  l_c = sum_p exp(s_p - m_c),  o_c[d] = sum_p exp(s_p - m_c) * v_p[d];
// the combine step takes M = max m_c, w_c = exp(m_c - M), out = (sum_c w_c o_c) / (sum_c w_c l_c).
// Equal to the sequential softmax and weighted sum up to f32 rounding.  Chunks sit at absolute
// positions and each query's arithmetic is the same whichever workgroup computes it, so a row's
// output does not depend on the batch it is in.  One workgroup = (KV head, query group, chunk):
// the chunk's keys and values are read from HBM once for all query heads and rows of the group
// (the sequential kernels read them once per (row, head) unit), and a long row is spread over
// as many workgroups as it has chunks.
constexpr int kSplitChunk = 64;

// Workgroup of 4 waves over CPW consecutive chunks of one KV head and WGQ = QG * 4 / CPW
// queries: wave w takes chunk CPW * blockIdx.z + w % CPW and queries (w / CPW) * QG .. + QG - 1
// of the group.  CPW = 4: every key and value of a chunk is read once per workgroup (long rows);
// CPW = 1 or 2: four or two waves share a chunk, when the queries fill more than one group.  Query j of group z is
// qi = z * WGQ + j = g * N + n (head kvh * G + g, row n).  Score phase: lane = position of the
// chunk.  Value phase: lane = output dims lane (and lane + 64 at HD = 128).
template <int HD, int QG, int CPW>
__global__ __launch_bounds__(256) void attn_split_kernel(AttnParams a) {
    constexpr int C = kSplitChunk, NQ = HD / 4, DL = HD / 64, WGQ = QG * 4 / CPW;
    typedef float f4v __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float qs[WGQ][HD];
    __shared__ __align__(16) float es[4][QG][C];
    const int G = a.H / a.Hkv, GN = G * a.N;
    const int kvh = blockIdx.x, z = blockIdx.y;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int c = CPW * blockIdx.z + w % CPW;  // this wave's chunk (past the last: all masked)
    const int q0 = z * WGQ + (w / CPW) * QG;   // this wave's first query
    const int pos0 = a.d_pos[0];
    const int plast = pos0 + a.N - 1;
    const bool chunk_live = c * C <= plast;  // uniform
    const int p0 = c * C;
    for (int e = t; e < WGQ * HD; e += 256) {
        const int i = e / HD, d = e % HD, qi = z * WGQ + i;
        float v = 0.0f;
        if (qi < GN) v = a.q[((size_t)(qi % a.N) * a.H + kvh * G + qi / a.N) * HD + d];
        qs[i][d] = v;
    }
    __syncthreads();
    // scores s_p = (q . k_p) * scale of this lane's position; keys are dim quads
    // [HD/4][max_ctx][4], so a wave's 16-byte loads of one dim quad are 1 KB contiguous.  A lane
    // past the pass's last row takes an offset outside the buffer (reads 0, no access).
    const int p = p0 + lane;
    const int kvo = p <= plast ? p * 16 : 0x40000000;
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.kcache + (size_t)kvh * a.max_ctx * HD), 0, a.max_ctx * HD * 4, 0x00020000);
    const int qstride = a.max_ctx * 16;
    float dot[QG];
#pragma unroll
    for (int k = 0; k < QG; k++) dot[k] = 0.0f;
    constexpr int KB = QG <= 8 ? 8 : 4;  // dim quads per batch of loads (registers allowing)
#pragma unroll 1
    for (int h0 = 0; h0 < NQ; h0 += KB) {
        f4v kv[KB];
#pragma unroll
        for (int i = 0; i < KB; i++)
            kv[i] = __builtin_bit_cast(f4v, __builtin_amdgcn_raw_buffer_load_b128(kres, kvo, (h0 + i) * qstride, 0));
#pragma unroll
        for (int i = 0; i < KB; i++) {
#pragma unroll
            for (int k = 0; k < QG; k++) {
                const f4v qv = *(const f4v*)&qs[(w / CPW) * QG + k][4 * (h0 + i)];
                dot[k] = __builtin_fmaf(qv.x, kv[i].x, dot[k]);
                dot[k] = __builtin_fmaf(qv.y, kv[i].y, dot[k]);
                dot[k] = __builtin_fmaf(qv.z, kv[i].z, dot[k]);
                dot[k] = __builtin_fmaf(qv.w, kv[i].w, dot[k]);
            }
        }
    }
    // chunk softmax partials: a position past the query's row is masked
#pragma unroll
    for (int k = 0; k < QG; k++) {
        const int qi = q0 + k;
        const bool live = qi < GN && p <= pos0 + qi % a.N;
        const float s = live ? dot[k] * a.scale : -__builtin_inff();
        float m = s;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float o = __shfl_xor(m, off, 64);
            m = o > m ? o : m;
        }
        const float e = live ? expf_glibc(s - m) : 0.0f;
        float l = e;
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) l = l + __shfl_xor(l, off, 64);
        es[w][k][lane] = e;
        if (lane == 0 && qi < GN && chunk_live) {
            const size_t u = ((size_t)(qi % a.N) * a.H + kvh * G + qi / a.N) * a.nchunks + c;
            a.part_ml[2 * u] = m;  // -inf (and l = 0) when the whole chunk is past the row
            a.part_ml[2 * u + 1] = l;
        }
    }
    __syncthreads();
    // o_c[d] = sum_p e_p * v_p[d]; values are position quads [max_ctx/4][HD][4].  Quads past the
    // one holding the pass's last row are not read (the quad index is clamped to it) and
    // positions past that row are zeroed (never-written cache rows may hold any bits; e = 0 there)
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(a.vcache + (size_t)kvh * a.max_ctx * HD), 0, a.max_ctx * HD * 4, 0x00020000);
    const int qlast = plast >> 2;
    float o[QG][DL];
#pragma unroll
    for (int k = 0; k < QG; k++)
#pragma unroll
        for (int dl = 0; dl < DL; dl++) o[k][dl] = 0.0f;
    constexpr int PB = QG <= 4 ? 8 : (QG <= 8 ? 4 : 2);  // position quads per batch of loads
#pragma unroll 1
    for (int b0 = 0; b0 < C / 4; b0 += PB) {
        f4v vv[PB][DL];
#pragma unroll
        for (int j = 0; j < PB; j++)
#pragma unroll
            for (int dl = 0; dl < DL; dl++)
                vv[j][dl] = __builtin_bit_cast(
                    f4v, __builtin_amdgcn_raw_buffer_load_b128(vres, (lane + 64 * dl) * 16,
                                                               min(p0 / 4 + b0 + j, qlast) * (HD * 16), 0));
#pragma unroll
        for (int j = 0; j < PB; j++) {
            const int pq = p0 + 4 * (b0 + j);
            if (pq + 3 > plast) {  // uniform: the quad holding the pass's last row, or past it
#pragma unroll
                for (int dl = 0; dl < DL; dl++) {
                    vv[j][dl].x = pq <= plast ? vv[j][dl].x : 0.0f;
                    vv[j][dl].y = pq + 1 <= plast ? vv[j][dl].y : 0.0f;
                    vv[j][dl].z = pq + 2 <= plast ? vv[j][dl].z : 0.0f;
                    vv[j][dl].w = 0.0f;
                }
            }
#pragma unroll
            for (int k = 0; k < QG; k++) {
                const f4v e4 = *(const f4v*)&es[w][k][4 * (b0 + j)];
#pragma unroll
                for (int dl = 0; dl < DL; dl++) {
                    o[k][dl] = __builtin_fmaf(e4.x, vv[j][dl].x, o[k][dl]);
                    o[k][dl] = __builtin_fmaf(e4.y, vv[j][dl].y, o[k][dl]);
                    o[k][dl] = __builtin_fmaf(e4.z, vv[j][dl].z, o[k][dl]);
                    o[k][dl] = __builtin_fmaf(e4.w, vv[j][dl].w, o[k][dl]);
                }
            }
        }
    }
    if (!chunk_live) return;
#pragma unroll
    for (int k = 0; k < QG; k++) {
        const int qi = q0 + k;
        if (qi < GN) {  // uniform
            const size_t u = ((size_t)(qi % a.N) * a.H + kvh * G + qi / a.N) * a.nchunks + c;
#pragma unroll
            for (int dl = 0; dl < DL; dl++) a.part_o[u * HD + lane + 64 * dl] = o[k][dl];
        }
    }
}

// Combine of a (row n, head h) unit's chunk partials, then the Q8_0 quantisation of its output
// block for the wo matmul; thread = output dim.  The chunk max M and the weights
// w_c = expf(m_c - M) are formed in parallel into LDS; the sums l = fma(w_c, l_c, l) and
// o = fma(w_c, o_c, o) run in chunk order, the partial outputs loaded a batch ahead.
constexpr int kSplitMaxChunks = NC_MAX_CONTEXT / kSplitChunk;
template <int HD>
__global__ __launch_bounds__(HD) void attn_combine_kernel(AttnParams a) {
    __shared__ float wl[2][kSplitMaxChunks];  // w_c, l_c
    __shared__ float red[HD / 64];
    const int n = blockIdx.x / a.H, h = blockIdx.x % a.H;
    const int t = threadIdx.x;
    const int nc = (a.d_pos[0] + n) / kSplitChunk + 1;  // chunks holding positions 0..pos
    const size_t u0 = ((size_t)n * a.H + h) * a.nchunks;
    const float* ml = a.part_ml + 2 * u0;
    const float* po = a.part_o + u0 * HD + t;
    constexpr int B = 32;  // partial outputs in flight
    float v[B];            // the first batch is loaded before the max and the weights
#pragma unroll
    for (int j = 0; j < B; j++) v[j] = po[(size_t)min(j, nc - 1) * HD];
    float M = -__builtin_inff();
    for (int c = t; c < nc; c += HD) M = ml[2 * c] > M ? ml[2 * c] : M;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float o = __shfl_xor(M, off, 64);
        M = o > M ? o : M;
    }
    if ((t & 63) == 0) red[t >> 6] = M;
    __syncthreads();
    M = red[0];
#pragma unroll
    for (int i = 1; i < HD / 64; i++) M = red[i] > M ? red[i] : M;
    for (int c = t; c < nc; c += HD) {
        wl[0][c] = expf_glibc(ml[2 * c] - M);  // chunk 0 always holds position 0: M finite
        wl[1][c] = ml[2 * c + 1];
    }
    __syncthreads();
    float l = 0.0f, o = 0.0f;
    for (int c0 = 0; c0 < nc; c0 += B) {
        if (c0 > 0) {
#pragma unroll
            for (int j = 0; j < B; j++) v[j] = po[(size_t)min(c0 + j, nc - 1) * HD];
        }
#pragma unroll
        for (int j = 0; j < B; j++) {
            if (c0 + j < nc) {  // uniform
                l = __builtin_fmaf(wl[0][c0 + j], wl[1][c0 + j], l);
                o = __builtin_fmaf(wl[0][c0 + j], v[j], o);
            }
        }
    }
    const float y = o / l;
    const int aw = a.H * HD;
    const int col = h * HD + (t & ~31);
    store_q8_block(y, t & 31, a.xq + (size_t)n * aw + col, a.xs + (size_t)n * (aw / 32) + col / 32,
                   a.xs8 + (size_t)n * (aw / 32) + col / 32);
}

static int launch_attention_split(const AttnParams& a, hipStream_t st) {
    const int G = a.H / a.Hkv, GN = G * a.N;
    const int nch = a.max_pos / kSplitChunk + 1;
    if (nch > a.nchunks) return fail(NC_ERANGE, "attention: row longer than the split partials hold");
    // Queries per wave QG (4, 8, 12 or 16): the largest that still gives ~1024 chunk waves (one
    // per SIMD), since every query group re-reads the chunk's keys and values; 16 at most
    // (registers).  Chunks per workgroup CPW: with chunk waves to spare (long rows, config 4:
    // 24.2 against 28.9 ms per pass) each wave takes its own chunk; otherwise query groups that
    // share a chunk share a workgroup, its waves reading the chunk through one CU's cache
    // (config 2: 1466 tok/s, config 3: 291 tok/s).
    auto waves = [&](int q) { return a.Hkv * nch * ((GN + q - 1) / q); };
    int qg = 4;
    for (int q : {16, 12, 8})
        if (q <= (GN + 3) / 4 * 4 && waves(q) >= 1024) {  // no more slots than queries
            qg = q;
            break;
        }
    const int subsets = (GN + qg - 1) / qg;
    const int cpw = subsets == 1 || waves(qg) >= 2048 ? 4 : (subsets >= 4 ? 1 : 2), wgq = qg * 4 / cpw;
    const dim3 grid(a.Hkv, (GN + wgq - 1) / wgq, (nch + cpw - 1) / cpw);
#define NC_SPLIT_QG(HD, CPW)                                                                               \
    switch (qg) {                                                                                          \
        case 4: NC_LAUNCH((attn_split_kernel<HD, 4, CPW>), grid, dim3(256), 0, st, a); break;    \
        case 8: NC_LAUNCH((attn_split_kernel<HD, 8, CPW>), grid, dim3(256), 0, st, a); break;    \
        case 12: NC_LAUNCH((attn_split_kernel<HD, 12, CPW>), grid, dim3(256), 0, st, a); break;  \
        default: NC_LAUNCH((attn_split_kernel<HD, 16, CPW>), grid, dim3(256), 0, st, a); break;  \
    }
#define NC_SPLIT(HD)                                                                            \
    if (cpw == 4) {                                                                             \
        NC_SPLIT_QG(HD, 4)                                                                      \
    } else if (cpw == 2) {                                                                      \
        NC_SPLIT_QG(HD, 2)                                                                      \
    } else {                                                                                    \
        NC_SPLIT_QG(HD, 1)                                                                      \
    }                                                                                           \
    NC_HIP(hipGetLastError());                                                                  \
    NC_LAUNCH((attn_combine_kernel<HD>), dim3(a.N * a.H), dim3(HD), 0, st, a);
    if (a.hd == 128) {
        NC_SPLIT(128)
    } else {
        NC_SPLIT(64)
    }
#undef NC_SPLIT
#undef NC_SPLIT_QG
    NC_HIP(hipGetLastError());
    return NC_OK;
}

// Kernel choice of the sequential-order attention for a pass whose longest row holds len
// positions (the branches of launch_attention below).
enum AttnTier {
    AT_FUSED_1_512, AT_FUSED_3_256, AT_FUSED_4_256, AT_FUSED_5_256, AT_FUSED_3_512,  // one kernel
    AT_PV_32_256_X1, AT_PV_4_512, AT_PV_8_512, AT_PV_16_512, AT_PV_32_512,           // scores, then
    AT_PV_8_256, AT_PV_16_256, AT_PV_32_256,                                         // softmax + V
    AT_TOO_LONG
};

static int attention_tier(const AttnParams& a) {
    const int len = a.max_pos + 1;  // the longest score row of the pass
    if (len <= 1536) {
        // one kernel per pass: each (row, head) unit scores its own keys (rows up to 1536
        // positions: the units of a KV head, all on one XCD, re-read its keys from that XCD's
        // L2, which costs less than a second launch and the scores' round trip through memory)
        // positions per thread E matched to the row (fewer score slots past the row); rows of
        // at most 512 and of 1281..1536 positions on 512 threads (two waves per SIMD in the
        // score phase; measured faster there, slower for 513..1280)
        return len <= 512 ? AT_FUSED_1_512 : len <= 768 ? AT_FUSED_3_256 : len <= 1024 ? AT_FUSED_4_256
             : len <= 1280 ? AT_FUSED_5_256 : AT_FUSED_3_512;
    }
    if (len > 16384) return AT_TOO_LONG;
    // more units than CUs on rows just past 8192 positions (a verify over an 8192-position
    // cache): the 256-thread tier with one extra position per thread (70B shape, 9 rows x 64
    // heads at 8201 positions)
    if (a.N * a.H > 256 && len > 8192 && len <= 8192 + 256) return AT_PV_32_256_X1;
    // at most one unit per CU: 512 threads, two waves per SIMD through the max, exp and sum
    // phases (a wave issues one VALU instruction per 8 cycles at most; 2000 positions 27.2 ->
    // 26.4 us, 8000 84.2 -> 78.4 us for one row), and the plain weighted-V loop
    if (a.N * a.H <= 256 || len > 8192)
        return len <= 2048 ? AT_PV_4_512 : len <= 4096 ? AT_PV_8_512 : len <= 8192 ? AT_PV_16_512 : AT_PV_32_512;
    // more units than CUs: 256 threads, so that three units fit on a CU at once (168 VGPRs
    // allow three waves per SIMD; at 512 threads only one unit fits and 576 units ran in three
    // rounds), and the software-pipelined weighted-V loop, which is faster when several chains
    // share a SIMD.  70B shape, 9 rows x 64 heads at 8101 positions: softmax + weighted V 213
    // -> 126 us, 9 rows x 64 heads at 2001: 78 -> 51 us (both kernels)
    return len <= 2048 ? AT_PV_8_256 : len <= 4096 ? AT_PV_16_256 : AT_PV_32_256;
}

// Score-kernel workgroups along the positions: the row's 64-position tiles rounded up to a
// multiple of 8 (the kernel strides over the tiles and a workgroup past the last tile does
// nothing), so that one grid serves 512 consecutive positions.
static int score_tile_groups(const AttnParams& a) { return ((a.max_pos + 64) / 64 + 7) / 8 * 8; }

int64_t attention_variant(const AttnParams& a) {
    if (a.split) return ((int64_t)1 << 40) | (a.max_pos / kSplitChunk + 1);
    const int tier = attention_tier(a);
    return ((int64_t)tier << 24) | (tier >= AT_PV_32_256_X1 ? score_tile_groups(a) : 0);
}

int launch_attention(const AttnParams& a, hipStream_t st) {
    const int G = a.H / a.Hkv;
    if (G > 8 || a.H % a.Hkv) return fail(NC_EINVAL, "attention: at most 8 query heads per KV head supported");
    if (a.hd != 64 && a.hd != 128) return fail(NC_EINVAL, "attention: head_dim must be 64 or 128");
    if (a.split) return launch_attention_split(a, st);
    const int tier = attention_tier(a);
    if (tier == AT_TOO_LONG) return fail(NC_ERANGE, "attention: context longer than 16384 positions");
    const dim3 grid(a.N * a.H);
    if (tier <= AT_FUSED_3_512) {
#define NC_FUSED(E, T)                                                                               \
    if (a.hd == 128) NC_LAUNCH((attn_fused_kernel<E, T, 128>), grid, dim3(T), 0, st, a);    \
    else NC_LAUNCH((attn_fused_kernel<E, T, 64>), grid, dim3(T), 0, st, a);                 \
    break;
        switch (tier) {
            case AT_FUSED_1_512: NC_FUSED(1, 512)
            case AT_FUSED_3_256: NC_FUSED(3, 256)
            case AT_FUSED_4_256: NC_FUSED(4, 256)
            case AT_FUSED_5_256: NC_FUSED(5, 256)
            default: NC_FUSED(3, 512)
        }
#undef NC_FUSED
        NC_HIP(hipGetLastError());
        return NC_OK;
    }
    // longer rows: scores by (KV head, 64-position tile) blocks that share each key tile
    // between the query heads and rows of a group, then one kernel for softmax and V sum
    // rows per block: one or two interleaved dot chains per lane; row groups are spread over
    // blockIdx.z so that every SIMD gets a short chain instead of a few SIMDs getting long ones
    const int rb = a.N >= 2 ? 2 : 1;
    const int tiles = score_tile_groups(a);
#define NC_SCORES(HD, RB)                                                                         \
    NC_LAUNCH((attn_scores_kernel<HD, RB>), dim3(a.Hkv, tiles, (a.N + (RB)-1) / (RB)), dim3(64 * G), 0, \
                       st, a);                                                                    \
    break;
#define NC_SCORES_HD(HD)            \
    switch (rb) {                   \
        case 1: NC_SCORES(HD, 1)    \
        default: NC_SCORES(HD, 2)   \
    }
    if (a.hd == 128) {
        NC_SCORES_HD(128)
    } else {
        NC_SCORES_HD(64)
    }
#undef NC_SCORES_HD
#undef NC_SCORES
    NC_HIP(hipGetLastError());
#define NC_PV(E, T, PIPE, X)                                                                              \
    if (a.hd == 128) NC_LAUNCH((attn_softmax_pv_kernel<E, T, 128, PIPE, X>), grid, dim3(T), 0, st, a); \
    else NC_LAUNCH((attn_softmax_pv_kernel<E, T, 64, PIPE, X>), grid, dim3(T), 0, st, a);              \
    break;
    switch (tier) {
        case AT_PV_32_256_X1: NC_PV(32, 256, true, 1)
        case AT_PV_4_512: NC_PV(4, 512, false, 0)
        case AT_PV_8_512: NC_PV(8, 512, false, 0)
        case AT_PV_16_512: NC_PV(16, 512, false, 0)
        case AT_PV_32_512: NC_PV(32, 512, false, 0)
        case AT_PV_8_256: NC_PV(8, 256, true, 0)
        case AT_PV_16_256: NC_PV(16, 256, true, 0)
        default: NC_PV(32, 256, true, 0)
    }
#undef NC_PV
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
    NC_LAUNCH(argmax_final_kernel, dim3(N), dim3(256), 0, st, part_val, part_idx, ntiles, preds);
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
    NC_LAUNCH(accept_greedy_kernel, dim3(1), dim3(64), 0, st, toks, preds, n, d_pos, result, next_tok_slot);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
