// Sampling on the device: the reference's sample_logits, and stochastic speculative acceptance.
//
// sample_logits (inference.rs:4834-4873) is restated exactly (lcg_walk_kernel, below): the
// uniform comes from the caller's copy of the reference's LCG, and the reference's f32 walk
// over the vocabulary is evaluated bit for bit.  Its speculative temperature path matches
// sampled tokens (speculative.rs:403).  The speculative sampler here is the library's own
// specification: temperature softmax over the vocabulary, the min(1, p/q) acceptance test and
// fixed-point inverse-CDF sampling driven by Philox4x32-10 uniforms:
//
//   probs     p_j = e_j * (1 / S),  e_j = expf((l_j - max) / T),  S = sum_j e_j taken left
//             to right in f32 (the reference's softmax formula, inference.rs:3522-3540,
//             4857-4862), evaluated exactly with the segmented parallel chain;
//   uniforms  u = (philox(seed, position, purpose).x >> 8) / 2^24, counter = (position,
//             purpose), key = seed;
//   accept    draft x of row i (position start+i) iff u_accept * q_i(x) < p_i(x);
//   sample    weights W_j = floor(w_j * 2^40) (exact integers), target =
//             floor(k24 * sum W / 2^24), result = first j whose inclusive prefix of W
//             exceeds target.  Integer prefix sums do not depend on evaluation order,
//             so one workgroup scans the vocabulary in parallel.
//
// The CPU oracle restates the same specification; the tests compare the two bit for bit.
#include <hip/hip_runtime.h>

#include "gguf.h"
#include "nc_chain.h"
#include "nc_device.h"
#include "nc_internal.h"

namespace nc {

// Philox4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): round multipliers 0xD2511F53 and
// 0xCD9E8D57, Weyl key increments 0x9E3779B9 and 0xBB67AE85, ten rounds.  Returns word 0.
__device__ inline uint32_t philox_word_dev(uint64_t seed, uint64_t pos, uint32_t purpose) {
    uint32_t c0 = (uint32_t)pos, c1 = (uint32_t)(pos >> 32), c2 = purpose, c3 = 0;
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
#pragma unroll
    for (int r = 0; r < 10; r++) {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    return c0;
}

__device__ inline uint32_t philox_u24(uint64_t seed, int64_t pos, uint32_t purpose) {
    return philox_word_dev(seed, (uint64_t)pos, purpose) >> 8;
}

__device__ inline uint64_t fixed_weight(float w) { return w > 0.0f ? (uint64_t)(w * 1099511627776.0f) : 0ull; }

// ---------------------------------------------------------------- temperature softmax
constexpr int kSmT = 1024;             // threads per row
constexpr int kSmE = 16;               // chain terms per thread per segment
constexpr int kSmSeg = kSmT * kSmE;    // terms per exact-chain segment

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// The order-free passes (max, e_j, p_j = e_j * (1/S)) run on kTpCh workgroups per row; only
// the exact sequential sum S runs on one workgroup per row.  e_j is kept in the output row
// between the passes.  scratch: per row kTpCh chunk maxima, then 1/S.
constexpr int kTpCh = 64;
constexpr int kTpT = 256;
constexpr int kTpStride = kTpCh + 2;  // per row: chunk maxima, 1/S, S

__device__ inline int tp_chunk(int V) { return (V + kTpCh - 1) / kTpCh; }

__global__ __launch_bounds__(kTpT) void tp_max_kernel(const float* logits, int64_t ld_in, int V, float* scratch) {
    __shared__ float wm[kTpT / 64];
    const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
    const float* l = logits + (size_t)row * ld_in;
    const int lo = min(c * tp_chunk(V), V), hi = min(lo + tp_chunk(V), V);
    float mx = -INFINITY;
    for (int i = lo + t; i < hi; i += kTpT) mx = fmaxf(mx, l[i]);
    mx = wave_max(mx);
    if ((t & 63) == 0) wm[t >> 6] = mx;
    __syncthreads();
    if (t == 0) {
#pragma unroll
        for (int w = 1; w < kTpT / 64; w++) mx = fmaxf(mx, wm[w]);
        scratch[(size_t)row * kTpStride + c] = mx;
    }
}

// e_j = expf((l_j - max) / T) (inference.rs:4857-4862), written to the output row.  The max
// does not depend on evaluation order (finite logits; +-0 give identical terms).
__global__ __launch_bounds__(kTpT) void tp_exp_kernel(const float* logits, int64_t ld_in, float* probs, int64_t ld_out,
                                                      int V, float temp, const float* scratch) {
    const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
    const float* pm = scratch + (size_t)row * kTpStride;
    static_assert(kTpCh == 64, "one chunk maximum per lane");
    float mx = pm[t & 63];
    mx = wave_max(mx);  // every wave reduces all kTpCh chunk maxima
    const float* l = logits + (size_t)row * ld_in;
    float* e = probs + (size_t)row * ld_out;
    const int lo = min(c * tp_chunk(V), V), hi = min(lo + tp_chunk(V), V);
    for (int i = lo + t; i < hi; i += kTpT) e[i] = expf_glibc((l[i] - mx) / temp);
}

// S = sum e_j left to right, one exact segment of kSmSeg terms at a time; scratch gets 1/S and S.
__global__ __launch_bounds__(kSmT) void tp_sum_kernel(const float* probs, int64_t ld_out, int V, float* scratch) {
    __shared__ ChainScratch<kSmT> sc;
    __shared__ __align__(16) float a_lds[kSmSeg];
    const float* e = probs + (size_t)blockIdx.x * ld_out;
    const int t = threadIdx.x;
    float sum = 0.0f;
    for (int base = 0; base < V; base += kSmSeg) {
        float a[kSmE];
#pragma unroll
        for (int j = 0; j < kSmE; j++) {
            const int i = base + t * kSmE + j;
            a[j] = i < V ? e[i] : 0.0f;
        }
        sum = exact_chain_sum<kSmE, kSmT>(a, sc, a_lds, sum);
    }
    if (t == 0) {
        scratch[(size_t)blockIdx.x * kTpStride + kTpCh] = 1.0f / sum;
        scratch[(size_t)blockIdx.x * kTpStride + kTpCh + 1] = sum;
    }
}

// p_j = e_j * (1 / S) (inference.rs:3535-3539), in place.
__global__ __launch_bounds__(kTpT) void tp_norm_kernel(float* probs, int64_t ld_out, int V, const float* scratch) {
    const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
    const float inv = scratch[(size_t)row * kTpStride + kTpCh];
    float* e = probs + (size_t)row * ld_out;
    const int lo = min(c * tp_chunk(V), V), hi = min(lo + tp_chunk(V), V);
    for (int i = lo + t; i < hi; i += kTpT) e[i] = e[i] * inv;
}

// ---------------------------------------------------------------- the reference's sampler
// sample_logits for temperature > 0 (inference.rs:4846-4873): with e_j = expf((l_j - max) / T)
// and S = sum e_j left to right (the passes above), r = u * S with u from the caller's LCG
// (rand_simple, inference.rs:4876-4883), then r -= e_j for j = 0, 1, ... and the first j with
// r <= 0 is the sample (V - 1 if none).  r_j = fl(r_{j-1} - e_j) is the negation of the chain
// q_j = fl(q_{j-1} + e_j) from q = -r (round to nearest is symmetric), so exact_chain_sum
// evaluates it bit for bit from a negative start and finds its first j with q_j >= 0.
__global__ __launch_bounds__(kSmT) void lcg_walk_kernel(const float* probs, int64_t ld, int V, const float* scratch,
                                                        SampleUniforms uu, uint32_t* out) {
    __shared__ ChainScratch<kSmT> sc;
    __shared__ __align__(16) float a_lds[kSmSeg];
    const int row = blockIdx.x, t = threadIdx.x;
    const float* e = probs + (size_t)row * ld;
    const float S = scratch[(size_t)row * kTpStride + kTpCh + 1];
    float q = -(uu.u[row] * S);
    int found = -1;
    for (int base = 0; base < V; base += kSmSeg) {
        float a[kSmE];
#pragma unroll
        for (int j = 0; j < kSmE; j++) {
            const int i = base + t * kSmE + j;
            a[j] = i < V ? e[i] : 0.0f;  // zeros past the row leave the chain and its sign unchanged
        }
        q = exact_chain_sum<kSmE, kSmT, true>(a, sc, a_lds, q);
        if (sc.first != 0x7fffffff) {  // uniform: read after the routine's last barrier
            found = base + sc.first;
            break;
        }
    }
    if (t == 0) out[row] = (uint32_t)(found >= 0 && found < V ? found : V - 1);
}

// Greedy sample_logits (inference.rs:4835-4845): the first maximum of each row.
__global__ __launch_bounds__(1024) void argmax_rows_kernel(const float* logits, int64_t ld, int V, uint32_t* out) {
    __shared__ float bvs[16];
    __shared__ int bis[16];
    const int row = blockIdx.x, t = threadIdx.x;
    const float* l = logits + (size_t)row * ld;
    float bv = -INFINITY;
    int bi = 0x7fffffff;
    for (int i = t; i < V; i += 1024) {
        const float v = l[i];
        if (v > bv) {  // ascending i per thread: the first of equal values stays
            bv = v;
            bi = i;
        }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const int oi = __shfl_xor(bi, o);
        if (ov > bv || (ov == bv && oi < bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if ((t & 63) == 0) {
        bvs[t >> 6] = bv;
        bis[t >> 6] = bi;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < 16; w++)
            if (bvs[w] > bv || (bvs[w] == bv && bis[w] < bi)) {
                bv = bvs[w];
                bi = bis[w];
            }
        out[row] = (uint32_t)(bi == 0x7fffffff ? 0 : bi);
    }
}

// ---------------------------------------------------------------- fixed-point sampler
constexpr int kSpT = 1024;

struct SampleScratch {
    uint64_t wtot[kSpT / 64];
    int found;
};

// Inclusive scan of a uint64 over the 64 lanes of a wave (shuffle based).
__device__ inline uint64_t wave_incl_scan_u64(uint64_t v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint64_t n = __shfl_up(v, o);
        if (lane >= o) v += n;
    }
    return v;
}

// Weight of id i: residual max(0, p_i - q_i) when q is given, else p_i.
__device__ inline uint64_t sample_weight(const float* p, const float* q, int i) {
    if (q) {
        const float d = p[i] - q[i];
        return fixed_weight(d > 0.0f ? d : 0.0f);
    }
    return fixed_weight(p[i]);
}

// Every thread of the block calls it; returns the sampled id, or -1 when all weights are 0.
// Wave w owns the contiguous ids [w*C, w*C + C) and reads them 64 at a time (lane l takes id
// base + 64*i + l: coalesced).  Phase 1: the wave totals (order-free integer sums) and their
// block scan fix the target and the wave whose range holds it.  Phase 2: that wave walks its
// range in 64-id tiles, an inclusive 64-bit scan per tile on top of the running prefix, and
// the first lane whose prefix exceeds the target is the answer.
__device__ int sample_fixed_block(const float* p, const float* q, int V, uint32_t k24, SampleScratch& ss) {
    constexpr int NW = kSpT / 64;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int C = (V + NW - 1) / NW;
    const int lo = min(w * C, V), hi = min(lo + C, V);
    uint64_t mine = 0;
    for (int i = lo + lane; i < hi; i += 64) mine += sample_weight(p, q, i);
    // wave total (order-free)
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mine += __shfl_xor(mine, o);
    if (lane == 0) ss.wtot[w] = mine;
    if (t == 0) ss.found = -1;
    __syncthreads();
    uint64_t base = 0, total = 0;
#pragma unroll
    for (int i = 0; i < NW; i++) {
        const uint64_t v = ss.wtot[i];
        if (i < w) base += v;
        total += v;
    }
    // target = floor(k24 * total / 2^24) < total, split so every product fits in 64 bits
    const uint64_t target = (((uint64_t)k24 * (total >> 32)) << 8) + (((uint64_t)k24 * (total & 0xffffffffull)) >> 24);
    if (total != 0 && base <= target && target < base + mine) {  // wave-uniform
        uint64_t run = base;  // inclusive prefix before this tile
        for (int t0 = lo; t0 < hi; t0 += 64) {
            const int i = t0 + lane;
            const uint64_t wv = i < hi ? sample_weight(p, q, i) : 0ull;
            const uint64_t incl = run + wave_incl_scan_u64(wv);
            const uint64_t hit = __ballot(i < hi && incl > target);
            if (hit) {
                if (lane == 0) ss.found = t0 + __ffsll((unsigned long long)hit) - 1;
                break;
            }
            run = __shfl(incl, 63);
        }
    }
    __syncthreads();
    const int r = ss.found;
    __syncthreads();  // ss is reused by the caller's next call
    return r;
}

// k+1 acceptance.  p: [k+1][ld] target probs of rows at start_pos .. start_pos+k; q: [k][ld]
// draft probs; drafts[k].  result = {n_accepted, next_token, start_pos + n_accepted + 1}.
__global__ __launch_bounds__(kSpT) void accept_stochastic_kernel(const float* p, const float* q, int64_t ld,
                                                                 const uint32_t* drafts, int k, int V, uint64_t seed,
                                                                 int64_t start_pos, int32_t* result, int32_t* d_pos) {
    __shared__ SampleScratch ss;
    __shared__ int s_a;
    const int t = threadIdx.x;
    if (t < 64) {
        bool reject = false;
        if (t < k) {
            const uint32_t x = drafts[t];
            const float u = (float)philox_u24(seed, start_pos + t, kPurposeAccept) * (1.0f / 16777216.0f);
            // an id outside the vocabulary has no probability under p: rejected
            reject = x >= (uint32_t)V || !(u * q[(size_t)t * ld + x] < p[(size_t)t * ld + x]);
        }
        const uint64_t m = __ballot(reject);
        if (t == 0) s_a = m ? __ffsll((unsigned long long)m) - 1 : k;
    }
    __syncthreads();
    const int a = s_a;
    int next;
    if (a < k) {
        const uint32_t k24 = philox_u24(seed, start_pos + a, kPurposeResample);
        const float* pa = p + (size_t)a * ld;
        next = sample_fixed_block(pa, q + (size_t)a * ld, V, k24, ss);
        if (next < 0) next = sample_fixed_block(pa, nullptr, V, k24, ss);
    } else {
        next = sample_fixed_block(p + (size_t)k * ld, nullptr, V, philox_u24(seed, start_pos + k, kPurposeBonus), ss);
    }
    if (t == 0) {
        const int np = (int)(start_pos + a + 1);
        result[0] = a;
        result[1] = next;
        result[2] = np;
        if (d_pos) d_pos[0] = np;
    }
}

// One sample from probs[V] with u(seed, pos, purpose); the id goes to out0 (and out1).
__global__ __launch_bounds__(kSpT) void sample_probs_kernel(const float* probs, int V, uint64_t seed, int64_t pos,
                                                            uint32_t purpose, uint32_t* out0, uint32_t* out1) {
    __shared__ SampleScratch ss;
    const int id = sample_fixed_block(probs, nullptr, V, philox_u24(seed, pos, purpose), ss);
    if (threadIdx.x == 0) {
        const uint32_t v = id < 0 ? 0u : (uint32_t)id;
        out0[0] = v;
        if (out1) out1[0] = v;
    }
}

size_t temperature_scratch_floats(int rows) { return (size_t)rows * kTpStride; }

int launch_sample_logits(const float* logits, int64_t ld_in, int rows, int V, float temp, const float* u, float* probs,
                         int64_t ld_p, float* scratch, uint32_t* out, hipStream_t st) {
    if (rows < 1 || rows > kSampleMaxRows || V < 1) return fail(NC_EINVAL, "sample_logits: 1..17 rows of vocab >= 1");
    if (!(temp > 0.0f)) {
        hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(1024), 0, st, logits, ld_in, V, out);
        NC_HIP(hipGetLastError());
        return NC_OK;
    }
    if (!u || !probs || !scratch) return fail(NC_EINVAL, "sample_logits: uniforms and work buffers required");
    SampleUniforms uu;
    for (int r = 0; r < kSampleMaxRows; r++) uu.u[r] = r < rows ? u[r] : 0.0f;
    const dim3 grid(kTpCh, rows);
    hipLaunchKernelGGL(tp_max_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, V, scratch);
    hipLaunchKernelGGL(tp_exp_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, probs, ld_p, V, temp, scratch);
    hipLaunchKernelGGL(tp_sum_kernel, dim3(rows), dim3(kSmT), 0, st, probs, ld_p, V, scratch);
    hipLaunchKernelGGL(lcg_walk_kernel, dim3(rows), dim3(kSmT), 0, st, probs, ld_p, V, scratch, uu, out);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int launch_temperature_probs(const float* logits, int64_t ld_in, float* probs, int64_t ld_out, int rows, int V,
                             float temp, float* scratch, hipStream_t st) {
    if (rows < 1 || V < 1 || !(temp > 0.0f)) return fail(NC_EINVAL, "temperature probs: rows, vocab and temp must be > 0");
    if (!scratch) return fail(NC_EINVAL, "temperature probs: no scratch");
    const dim3 grid(kTpCh, rows);
    hipLaunchKernelGGL(tp_max_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, V, scratch);
    hipLaunchKernelGGL(tp_exp_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, probs, ld_out, V, temp, scratch);
    hipLaunchKernelGGL(tp_sum_kernel, dim3(rows), dim3(kSmT), 0, st, probs, ld_out, V, scratch);
    hipLaunchKernelGGL(tp_norm_kernel, grid, dim3(kTpT), 0, st, probs, ld_out, V, scratch);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int launch_accept_stochastic(const float* p, const float* q, int64_t ld, const uint32_t* drafts, int k, int V,
                             uint64_t seed, int64_t start_pos, int32_t* result, int32_t* d_pos, hipStream_t st) {
    if (k < 0 || k > 63 || V < 1) return fail(NC_EINVAL, "stochastic accept: k must be 0..63");
    hipLaunchKernelGGL(accept_stochastic_kernel, dim3(1), dim3(kSpT), 0, st, p, q, ld, drafts, k, V, seed, start_pos,
                       result, d_pos);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int launch_sample_probs(const float* probs, int V, uint64_t seed, int64_t pos, uint32_t purpose, uint32_t* out0,
                        uint32_t* out1, hipStream_t st) {
    if (V < 1) return fail(NC_EINVAL, "sample: vocab must be > 0");
    hipLaunchKernelGGL(sample_probs_kernel, dim3(1), dim3(kSpT), 0, st, probs, V, seed, pos, purpose, out0, out1);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
