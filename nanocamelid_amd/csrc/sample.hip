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

// The order-free passes (max, e_j, p_j = e_j * (1/S)) run on kTpCh workgroups per row.  The
// exact sequential sum S runs its kSmSeg-term segments on one workgroup each (the evaluation
// of exact_chain_sum spread over the segments: tps_run, tps_walk, tps_verify, tps_finish) when
// the row has at most kTpSegMax segments, else on one workgroup per row, segment after
// segment.  e_j is kept in the output row between the passes.
constexpr int kTpCh = 64;
constexpr int kTpT = 256;
constexpr int kTpSegMax = 16;  // segments evaluated in parallel: V <= 262144
constexpr int kTpEntCap = 256;  // sensitive runs listed per segment

struct TpSegInfo {
    double dtot;      // sum of the segment's run increments (runs evaluated from the guesses)
    double shift_in;  // correction of the last sensitive run before the segment (0: none)
    int nsens;        // sensitive runs in the segment (more than kTpEntCap: not listed)
    int bad;          // a boundary check inside the segment failed
    float first;      // verified start of the segment's first run
    float last;       // end of its last run
};
struct TpEnt {
    double cstart, cend;  // uncorrected start and end of a sensitive run, relative to its segment
    double shift;         // true end - uncorrected end (global), after the walk
    int run;              // run index in the row (term run * kSmE is its first term)
    int pad;
};
// Per-row scratch of the temperature softmax.
struct TpRowScratch {
    float cmax[kTpCh];  // chunk maxima
    float inv, S;       // 1 / S and S
    int ok;             // the walk listed every sensitive run
    int fast;           // S came from the parallel evaluation (else from the sequential fallback)
    double csum[kTpCh];                      // chunk sums of e in double (the guesses' prefix)
    TpSegInfo seg[kTpSegMax];
    TpEnt ent[kTpSegMax * kTpEntCap];
    double crun[kTpSegMax * kSmT];  // uncorrected start of each run, relative to its segment
    int off[kTpSegMax * kSmT];      // sensitive runs before each run in its segment
};
constexpr int kTpStride = (int)((sizeof(TpRowScratch) + 255) / 256 * 64);  // floats per row

__host__ __device__ inline TpRowScratch* tp_row(float* scratch, int row) {
    return reinterpret_cast<TpRowScratch*>(scratch + (size_t)row * kTpStride);
}
__host__ __device__ inline const TpRowScratch* tp_row(const float* scratch, int row) {
    return reinterpret_cast<const TpRowScratch*>(scratch + (size_t)row * kTpStride);
}

// Chunk length: ceil(V / kTpCh) rounded up to a power of two, so that chunks tile every
// kSmSeg-term segment (kSmSeg is a power of two) and a segment's prefix is a sum of chunk sums.
__device__ inline int tp_chunk(int V) {
    int c = 256;
    while (c * kTpCh < V) c <<= 1;
    return c;
}

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
        tp_row(scratch, row)->cmax[c] = mx;
    }
}

// e_j = expf((l_j - max) / T) (inference.rs:4857-4862), written to the output row, and the
// chunk's sum of e in double (a fixed tree: only the guesses of the exact sum read it).  The
// max does not depend on evaluation order (finite logits; +-0 give identical terms).
__global__ __launch_bounds__(kTpT) void tp_exp_kernel(const float* logits, int64_t ld_in, float* probs, int64_t ld_out,
                                                      int V, float temp, float* scratch) {
    __shared__ double ws[kTpT / 64];
    const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
    TpRowScratch* R = tp_row(scratch, row);
    static_assert(kTpCh == 64, "one chunk maximum per lane");
    float mx = R->cmax[t & 63];
    mx = wave_max(mx);  // every wave reduces all kTpCh chunk maxima
    const float* l = logits + (size_t)row * ld_in;
    float* e = probs + (size_t)row * ld_out;
    const int lo = min(c * tp_chunk(V), V), hi = min(lo + tp_chunk(V), V);
    double sum = 0.0;
    for (int i = lo + t; i < hi; i += kTpT) {
        const float v = expf_glibc((l[i] - mx) / temp);
        e[i] = v;
        sum += (double)v;
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o);
    if ((t & 63) == 0) ws[t >> 6] = sum;
    __syncthreads();
    if (t == 0) {
        double c_sum = 0.0;
#pragma unroll
        for (int w = 0; w < kTpT / 64; w++) c_sum += ws[w];
        R->csum[c] = c_sum;
    }
}

// S = sum e_j left to right, one exact segment of kSmSeg terms after another.
__device__ float tp_sum_segments(const float* e, int V, ChainScratch<kSmT>& sc, float* a_lds) {
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
    return sum;
}

// One workgroup per row, segments in order; scratch gets 1/S and S.
__global__ __launch_bounds__(kSmT) void tp_sum_kernel(const float* probs, int64_t ld_out, int V, float* scratch) {
    __shared__ ChainScratch<kSmT> sc;
    __shared__ __align__(16) float a_lds[kSmSeg];
    const float sum = tp_sum_segments(probs + (size_t)blockIdx.x * ld_out, V, sc, a_lds);
    if (threadIdx.x == 0) {
        TpRowScratch* R = tp_row(scratch, blockIdx.x);
        R->inv = 1.0f / sum;
        R->S = sum;
        R->fast = 0;
    }
}

// The segments in parallel.  exact_chain_sum's five steps over a whole row of runs (a run is
// a thread's kSmE consecutive terms, a segment one workgroup's kSmT runs), with the block-wide
// scans split at segment boundaries:
//   tps_run     (segment x row workgroups) steps 1-3: guesses from the double prefix (the
//               chunk sums before the segment plus the block scan), the runs from the guesses
//               and their sensitivity, the uncorrected starts relative to the segment and the
//               segment's list of sensitive runs;
//   tps_walk    (one wave per row) step 4: the segment bases C_g (sums of the earlier
//               segments' increments, in order), then the walk over every listed run of the
//               row, which fixes each run's correction;
//   tps_verify  (segment x row) step 5: every run recomputed from its corrected start and
//               every boundary inside the segment checked;
//   tps_finish  (one workgroup per row) the boundaries between segments; if any check
//               failed, or a segment had more sensitive runs than it lists, S is evaluated
//               segment after segment as tp_sum_kernel does.
// As in exact_chain_sum, the result is the sequential chain whenever it is accepted: the
// verified starts equal the previous runs' ends at every boundary, so by induction the last
// end is s_{V-1}.
// A run's kSmE terms e[i0 ..], zeros past the row (they leave the chain unchanged); 16-byte
// loads when the run is whole and aligned.
__device__ inline void tps_load_run(const float* e, int V, int i0, float (&a)[kSmE]) {
    static_assert(kSmE % 4 == 0, "whole float4s per run");
    if (i0 + kSmE <= V && (reinterpret_cast<uintptr_t>(e + i0) & 15) == 0) {
        const float4* p = reinterpret_cast<const float4*>(e + i0);
#pragma unroll
        for (int c = 0; c < kSmE / 4; c++) {
            const float4 v = p[c];
            a[4 * c] = v.x;
            a[4 * c + 1] = v.y;
            a[4 * c + 2] = v.z;
            a[4 * c + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int j = 0; j < kSmE; j++) a[j] = i0 + j < V ? e[i0 + j] : 0.0f;
    }
}

__global__ __launch_bounds__(kSmT) void tps_run_kernel(const float* probs, int64_t ld, int V, float* scratch) {
    __shared__ double dtot[kSmT / 64], dtot2[kSmT / 64];
    __shared__ int itot[kSmT / 64];
    __shared__ double s_base;
    const int g = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    TpRowScratch* R = tp_row(scratch, row);
    const float* e = probs + (size_t)row * ld;
    const int base = g * kSmSeg;
    float a[kSmE];
    tps_load_run(e, V, base + t * kSmE, a);
    if (t == 0) {
        double P = 0.0;
        const int cb = base / tp_chunk(V);  // chunks tile the segments
        for (int c = 0; c < cb; c++) P += R->csum[c];
        s_base = P;
    }
    // 1. guess: the double prefix of every earlier term
    double run = 0.0;
#pragma unroll
    for (int j = 0; j < kSmE; j++) run += (double)a[j];
    const double lp = block_excl_scan_f64<kSmT>(run, dtot);  // its barrier publishes s_base
    const float gs = (float)(s_base + lp);
    // 2. the run from the guess
    float x;
    const bool sens = chain_run_sensitive<kSmE>(a, gs, false, x);
    const double d = (double)x - (double)gs;
    // 3. uncorrected start relative to the segment, sensitive count before the run
    int off, total_s;
    const double cl = block_excl_scan_f64_i32<kSmT>(d, sens ? 1 : 0, dtot2, itot, &off, &total_s);
    const int r = g * kSmT + t;
    R->crun[r] = cl;
    R->off[r] = off;
    if (sens && off < kTpEntCap) {
        TpEnt& en = R->ent[g * kTpEntCap + off];
        en.cstart = cl;
        en.cend = cl + d;
        en.run = r;
    }
    if (t == kSmT - 1) {
        R->seg[g].dtot = cl + d;
        R->seg[g].nsens = total_s;
    }
}

__global__ __launch_bounds__(64) void tps_walk_kernel(const float* probs, int64_t ld, int V, float* scratch) {
    constexpr int W = WalkRow<kSmE>::W;
    __shared__ WalkRow<kSmE> rows[64];
    __shared__ float walk_end[64];
    __shared__ double cbase[kTpSegMax + 1];
    __shared__ int eoff[kTpSegMax + 1];
    __shared__ double shifts[kTpSegMax * kTpEntCap];
    __shared__ int s_listed;
    const int row = blockIdx.x, t = threadIdx.x;
    TpRowScratch* R = tp_row(scratch, row);
    const float* e = probs + (size_t)row * ld;
    const int nseg = (V + kSmSeg - 1) / kSmSeg;
    if (t == 0) {
        double c = 0.0;
        int n = 0;
        bool listed = true;
        for (int g = 0; g < nseg; g++) {
            cbase[g] = c;
            eoff[g] = n;
            c += R->seg[g].dtot;
            const int ns = R->seg[g].nsens;
            listed = listed && ns <= kTpEntCap;
            n += min(ns, kTpEntCap);
        }
        cbase[nseg] = c;
        eoff[nseg] = n;
        s_listed = listed ? 1 : 0;
    }
    __syncthreads();
    if (!s_listed) {
        if (t == 0) R->ok = 0;
        return;
    }
    const int total = eoff[nseg];
    float S = 0.0f;  // true chain value after the last walked run (lane 0)
    for (int e0 = 0; e0 < total; e0 += 64) {
        const int me = e0 + t;
        const int cnt = min(64, total - e0);
        double ce = 0.0;
        if (me < total) {
            int g = 0;
            while (g + 1 < nseg && eoff[g + 1] <= me) g++;
            const TpEnt& en = R->ent[g * kTpEntCap + (me - eoff[g])];
            const double cs = cbase[g] + en.cstart;
            ce = cbase[g] + en.cend;
            double cprev = 0.0;  // uncorrected end of the previous listed run (the chain starts at 0)
            if (me > 0) {
                int gp = g;
                while (eoff[gp] > me - 1) gp--;
                cprev = cbase[gp] + R->ent[gp * kTpEntCap + (me - 1 - eoff[gp])].cend;
            }
            rows[t].v[0] = (float)(cs - cprev);  // exact advance over the insensitive runs between
            const int i0 = en.run * kSmE;
#pragma unroll
            for (int j = 0; j < kSmE; j++) rows[t].v[1 + j] = i0 + j < V ? e[i0 + j] : 0.0f;
#pragma unroll
            for (int j = kSmE + 1; j < W; j++) rows[t].v[j] = 0.0f;
        }
        __syncthreads();
        if (t == 0) S = chain_walk_rows<kSmE>(rows, cnt, S, walk_end);
        __syncthreads();
        if (me < total) shifts[me] = (double)walk_end[t] - ce;
        __syncthreads();  // rows and walk_end are rewritten by the next window
    }
    for (int g = t; g < nseg; g += 64) R->seg[g].shift_in = eoff[g] > 0 ? shifts[eoff[g] - 1] : 0.0;
    for (int i = t; i < total; i += 64) {
        int g = 0;
        while (g + 1 < nseg && eoff[g + 1] <= i) g++;
        R->ent[g * kTpEntCap + (i - eoff[g])].shift = shifts[i];
    }
    if (t == 0) R->ok = 1;
}

__global__ __launch_bounds__(kSmT) void tps_verify_kernel(const float* probs, int64_t ld, int V, float* scratch) {
    __shared__ float last[kSmT];
    __shared__ double s_cb;
    __shared__ int s_ok;
    const int g = blockIdx.x, row = blockIdx.y, t = threadIdx.x;
    TpRowScratch* R = tp_row(scratch, row);
    if (t == 0) {
        s_ok = R->ok;
        double c = 0.0;  // the walk's segment base, summed in the same order
        for (int h = 0; h < g; h++) c += R->seg[h].dtot;
        s_cb = c;
    }
    __syncthreads();
    if (!s_ok) return;  // uniform: tps_finish takes the sequential evaluation
    const float* e = probs + (size_t)row * ld;
    const int base = g * kSmSeg;
    float a[kSmE];
    tps_load_run(e, V, base + t * kSmE, a);
    const int r = g * kSmT + t;
    const int off = R->off[r];
    const double sh = off > 0 ? R->ent[g * kTpEntCap + off - 1].shift : R->seg[g].shift_in;
    const float start = (float)((s_cb + R->crun[r]) + sh);
    float y = start;
#pragma unroll
    for (int j = 0; j < kSmE; j++) y = y + a[j];
    last[t] = y;
    bool bad = (g == 0 && t == 0) ? start != 0.0f : false;
    __syncthreads();
    if (t > 0) bad |= start != last[t - 1];
    bad = __syncthreads_or(bad);
    if (t == 0) {
        R->seg[g].bad = bad ? 1 : 0;
        R->seg[g].first = start;
    }
    if (t == kSmT - 1) R->seg[g].last = y;
}

__global__ __launch_bounds__(kSmT) void tps_finish_kernel(const float* probs, int64_t ld, int V, float* scratch) {
    __shared__ ChainScratch<kSmT> sc;
    __shared__ __align__(16) float a_lds[kSmSeg];
    __shared__ int s_ok;
    __shared__ float s_sum;
    const int row = blockIdx.x, t = threadIdx.x;
    TpRowScratch* R = tp_row(scratch, row);
    if (t == 0) {
        const int nseg = (V + kSmSeg - 1) / kSmSeg;
        bool ok = R->ok != 0;
        for (int g = 0; ok && g < nseg; g++) ok = !R->seg[g].bad && (g == 0 || R->seg[g].first == R->seg[g - 1].last);
        s_ok = ok ? 1 : 0;
        s_sum = ok ? R->seg[nseg - 1].last : 0.0f;
    }
    __syncthreads();
    const bool ok = s_ok != 0;
    const float sum = ok ? s_sum : tp_sum_segments(probs + (size_t)row * ld, V, sc, a_lds);
    if (t == 0) {
        R->inv = 1.0f / sum;
        R->S = sum;
        R->fast = ok ? 1 : 0;
    }
}

// S and 1/S of every row, by the parallel segments when the row fits kTpSegMax of them.
static void launch_tp_sum(const float* probs, int64_t ld, int rows, int V, float* rs, hipStream_t st) {
    const int nseg = (V + kSmSeg - 1) / kSmSeg;
    if (nseg > kTpSegMax) {
        hipLaunchKernelGGL(tp_sum_kernel, dim3(rows), dim3(kSmT), 0, st, probs, ld, V, rs);
        return;
    }
    hipLaunchKernelGGL(tps_run_kernel, dim3(nseg, rows), dim3(kSmT), 0, st, probs, ld, V, rs);
    hipLaunchKernelGGL(tps_walk_kernel, dim3(rows), dim3(64), 0, st, probs, ld, V, rs);
    hipLaunchKernelGGL(tps_verify_kernel, dim3(nseg, rows), dim3(kSmT), 0, st, probs, ld, V, rs);
    hipLaunchKernelGGL(tps_finish_kernel, dim3(rows), dim3(kSmT), 0, st, probs, ld, V, rs);
}

// p_j = e_j * (1 / S) (inference.rs:3535-3539), in place.
__global__ __launch_bounds__(kTpT) void tp_norm_kernel(float* probs, int64_t ld_out, int V, const float* scratch) {
    const int row = blockIdx.y, c = blockIdx.x, t = threadIdx.x;
    const float inv = tp_row(scratch, row)->inv;
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
    const float S = tp_row(scratch, row)->S;
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
// Two launches.  sample_totals_kernel: kSpG workgroups, one contiguous chunk of ids each, sum
// the chunk's fixed-point weights (order-free integer sums) for the residual max(0, p - q) and
// for p; in acceptance mode every workgroup also decides the accepted prefix a (the same
// ballot over the k Philox tests) and workgroup 0 publishes it.  sample_pick_kernel: one
// workgroup scans the kSpG chunk totals, fixes the weight set, the target and the one chunk
// whose range holds it, and scans that chunk's ids with a block-wide inclusive 64-bit scan.
// The answer is the first id whose inclusive prefix exceeds the target, which does not
// depend on how the sums were split.
constexpr int kSpG = 256;   // chunk workgroups
constexpr int kSpTT = 256;  // threads per chunk workgroup
constexpr int kSpT = 1024;  // threads of the pick workgroup

// Device scratch of the sampler: chunk totals of both weight sets and the pick descriptor.
struct SampleScratch {
    uint64_t tot_r[kSpG];  // residual max(0, p - q) per chunk
    uint64_t tot_p[kSpG];  // p per chunk
    int32_t a;             // row to sample (acceptance: the accepted prefix length)
    uint32_t k24;          // 24-bit uniform of the draw
    int32_t use_q;         // 1: residual weights first, p if they are all 0
    int32_t pad;
};
constexpr size_t kSpScratchFloats = (sizeof(SampleScratch) + 255) / 256 * 64;  // 256-byte multiple

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

__device__ inline uint64_t wave_sum_u64(uint64_t v) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
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

__device__ inline int sample_chunk(int V) { return (V + kSpG - 1) / kSpG; }

// k+1 acceptance (k >= 0): p [k+1][ld] target probs of rows start_pos .. start_pos+k, q [k][ld]
// draft probs, drafts[k]; draft i is accepted iff u_accept * q_i(x) < p_i(x), and a is the
// first rejected row (k if none).  Sampling mode (k < 0): row 0 of p, u(seed, pos, purpose).
// Every workgroup sums its chunk of the row it will sample; workgroup 0 writes the descriptor
// and, in acceptance mode, result[0] = a, result[2] = start_pos + a + 1 and d_pos.
__global__ __launch_bounds__(kSpTT) void sample_totals_kernel(const float* p, const float* q, int64_t ld,
                                                              const uint32_t* drafts, int k, int V, uint64_t seed,
                                                              int64_t pos, uint32_t purpose, SampleScratch* ss,
                                                              int32_t* result, int32_t* d_pos) {
    __shared__ int s_a;
    __shared__ uint64_t wr[kSpTT / 64], wp[kSpTT / 64];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    if (t < 64) {
        int a = 0;
        if (k >= 0) {
            bool reject = false;
            if (t < k) {
                const uint32_t x = drafts[t];
                const float u = (float)philox_u24(seed, pos + t, kPurposeAccept) * (1.0f / 16777216.0f);
                // an id outside the vocabulary has no probability under p: rejected
                reject = x >= (uint32_t)V || !(u * q[(size_t)t * ld + x] < p[(size_t)t * ld + x]);
            }
            const uint64_t m = __ballot(reject);
            a = m ? __ffsll((unsigned long long)m) - 1 : k;
        }
        if (t == 0) s_a = a;
    }
    __syncthreads();
    const int a = s_a;
    const bool use_q = k >= 0 && a < k;
    const float* pa = p + (size_t)a * ld;
    const float* qa = use_q ? q + (size_t)a * ld : nullptr;
    const int C = sample_chunk(V);
    const int lo = min(blockIdx.x * C, V), hi = min(lo + C, V);
    uint64_t r = 0, pw = 0;
    for (int i = lo + t; i < hi; i += kSpTT) {
        const float pv = pa[i];
        pw += fixed_weight(pv);
        if (qa) {
            const float d = pv - qa[i];
            r += fixed_weight(d > 0.0f ? d : 0.0f);
        }
    }
    r = wave_sum_u64(r);
    pw = wave_sum_u64(pw);
    if (lane == 0) {
        wr[w] = r;
        wp[w] = pw;
    }
    __syncthreads();
    if (t == 0) {
        uint64_t sr = 0, sp = 0;
#pragma unroll
        for (int i = 0; i < kSpTT / 64; i++) {
            sr += wr[i];
            sp += wp[i];
        }
        ss->tot_r[blockIdx.x] = sr;
        ss->tot_p[blockIdx.x] = sp;
        if (blockIdx.x == 0) {
            uint32_t k24;
            if (k < 0)
                k24 = philox_u24(seed, pos, purpose);
            else
                k24 = philox_u24(seed, pos + a, use_q ? kPurposeResample : kPurposeBonus);
            ss->a = a;
            ss->k24 = k24;
            ss->use_q = use_q ? 1 : 0;
            if (k >= 0) {
                const int np = (int)(pos + a + 1);
                result[0] = a;
                result[2] = np;
                if (d_pos) d_pos[0] = np;
            }
        }
    }
}

// One workgroup: the draw described by ss.  Acceptance mode (result != null): result[1] = id,
// -1 when every weight is 0.  Sampling mode: out0 (and out1) = id, 0 when every weight is 0.
__global__ __launch_bounds__(kSpT) void sample_pick_kernel(const float* p, const float* q, int64_t ld, int V,
                                                           const SampleScratch* ss, int32_t* result, uint32_t* out0,
                                                           uint32_t* out1) {
    static_assert(kSpG == 4 * 64, "waves 0..3 hold one chunk total per lane");
    __shared__ uint64_t wt_r[4], wt_p[4], wt[kSpT / 64];
    __shared__ uint64_t s_base;
    __shared__ int s_chunk, s_found;
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int a = ss->a, use_q = ss->use_q;
    const uint32_t k24 = ss->k24;
    uint64_t ir = 0, ip = 0, vr = 0, vp = 0;
    if (w < 4) {
        vr = use_q ? ss->tot_r[t] : 0ull;
        vp = ss->tot_p[t];
        ir = wave_incl_scan_u64(vr);
        ip = wave_incl_scan_u64(vp);
        if (lane == 63) {
            wt_r[w] = ir;
            wt_p[w] = ip;
        }
    }
    if (t == 0) {
        s_chunk = -1;
        s_found = 0x7fffffff;
    }
    __syncthreads();
    uint64_t total_r = 0, total_p = 0, pre_r = 0, pre_p = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        if (i < w) {
            pre_r += wt_r[i];
            pre_p += wt_p[i];
        }
        total_r += wt_r[i];
        total_p += wt_p[i];
    }
    const bool res = total_r != 0;  // residual weights exist (use_q only: otherwise all 0)
    const uint64_t total = res ? total_r : total_p;
    // target = floor(k24 * total / 2^24) < total, split so every product fits in 64 bits
    const uint64_t target = (((uint64_t)k24 * (total >> 32)) << 8) + (((uint64_t)k24 * (total & 0xffffffffull)) >> 24);
    if (w < 4 && total != 0) {
        const uint64_t own = res ? vr : vp;
        const uint64_t base = (res ? pre_r + ir : pre_p + ip) - own;
        if (own != 0 && base <= target && target < base + own) {  // exactly one chunk
            s_chunk = t;
            s_base = base;
        }
    }
    __syncthreads();
    const int c = s_chunk;
    int found = -1;
    if (c >= 0) {
        const float* pa = p + (size_t)a * ld;
        const float* qa = res ? q + (size_t)a * ld : nullptr;
        const int C = sample_chunk(V);
        const int lo = min(c * C, V), hi = min(lo + C, V);
        uint64_t run = s_base;  // inclusive prefix before this tile
        for (int t0 = lo; t0 < hi; t0 += kSpT) {
            const int i = t0 + t;
            const uint64_t wv = i < hi ? sample_weight(pa, qa, i) : 0ull;
            const uint64_t incl = wave_incl_scan_u64(wv);
            if (lane == 63) wt[w] = incl;
            __syncthreads();
            uint64_t before = run, tile = 0;
#pragma unroll
            for (int j = 0; j < kSpT / 64; j++) {
                if (j < w) before += wt[j];
                tile += wt[j];
            }
            // prefixes only grow with i, so the first id past the target is the smallest hit
            if (i < hi && before + incl > target) atomicMin(&s_found, i);
            __syncthreads();
            if (s_found != 0x7fffffff) break;
            run += tile;
        }
        found = s_found == 0x7fffffff ? -1 : s_found;  // a hit exists: target < base + own
    }
    if (t == 0) {
        if (result)
            result[1] = found;
        else {
            const uint32_t v = found < 0 ? 0u : (uint32_t)found;
            out0[0] = v;
            if (out1) out1[0] = v;
        }
    }
}

size_t temperature_scratch_floats(int rows) { return kSpScratchFloats + (size_t)rows * kTpStride; }

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
    float* rs = scratch + kSpScratchFloats;
    const dim3 grid(kTpCh, rows);
    hipLaunchKernelGGL(tp_max_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, V, rs);
    hipLaunchKernelGGL(tp_exp_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, probs, ld_p, V, temp, rs);
    launch_tp_sum(probs, ld_p, rows, V, rs, st);
    hipLaunchKernelGGL(lcg_walk_kernel, dim3(rows), dim3(kSmT), 0, st, probs, ld_p, V, rs, uu, out);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int launch_temperature_probs(const float* logits, int64_t ld_in, float* probs, int64_t ld_out, int rows, int V,
                             float temp, float* scratch, hipStream_t st) {
    if (rows < 1 || V < 1 || !(temp > 0.0f)) return fail(NC_EINVAL, "temperature probs: rows, vocab and temp must be > 0");
    if (!scratch) return fail(NC_EINVAL, "temperature probs: no scratch");
    float* rs = scratch + kSpScratchFloats;
    const dim3 grid(kTpCh, rows);
    hipLaunchKernelGGL(tp_max_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, V, rs);
    hipLaunchKernelGGL(tp_exp_kernel, grid, dim3(kTpT), 0, st, logits, ld_in, probs, ld_out, V, temp, rs);
    launch_tp_sum(probs, ld_out, rows, V, rs, st);
    hipLaunchKernelGGL(tp_norm_kernel, grid, dim3(kTpT), 0, st, probs, ld_out, V, rs);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int temperature_row_paths(const float* scratch, int rows, int32_t* fast, hipStream_t st) {
    const float* rs = scratch + kSpScratchFloats;
    for (int r = 0; r < rows; r++)
        NC_HIP(hipMemcpyAsync(fast + r, &tp_row(rs, r)->fast, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    NC_HIP(hipStreamSynchronize(st));
    return NC_OK;
}

int launch_accept_stochastic(const float* p, const float* q, int64_t ld, const uint32_t* drafts, int k, int V,
                             uint64_t seed, int64_t start_pos, int32_t* result, int32_t* d_pos, float* scratch,
                             hipStream_t st) {
    if (k < 0 || k > 63 || V < 1) return fail(NC_EINVAL, "stochastic accept: k must be 0..63");
    if (!scratch || !result) return fail(NC_EINVAL, "stochastic accept: no scratch or result");
    SampleScratch* ss = reinterpret_cast<SampleScratch*>(scratch);
    hipLaunchKernelGGL(sample_totals_kernel, dim3(kSpG), dim3(kSpTT), 0, st, p, q, ld, drafts, k, V, seed, start_pos,
                       0u, ss, result, d_pos);
    hipLaunchKernelGGL(sample_pick_kernel, dim3(1), dim3(kSpT), 0, st, p, q, ld, V, ss, result, nullptr, nullptr);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

int launch_sample_probs(const float* probs, int V, uint64_t seed, int64_t pos, uint32_t purpose, uint32_t* out0,
                        uint32_t* out1, float* scratch, hipStream_t st) {
    if (V < 1) return fail(NC_EINVAL, "sample: vocab must be > 0");
    if (!scratch || !out0) return fail(NC_EINVAL, "sample: no scratch or output");
    SampleScratch* ss = reinterpret_cast<SampleScratch*>(scratch);
    hipLaunchKernelGGL(sample_totals_kernel, dim3(kSpG), dim3(kSpTT), 0, st, probs, nullptr, (int64_t)V, nullptr, -1,
                       V, seed, pos, purpose, ss, nullptr, nullptr);
    hipLaunchKernelGGL(sample_pick_kernel, dim3(1), dim3(kSpT), 0, st, probs, nullptr, (int64_t)V, V, ss, nullptr,
                       out0, out1);
    NC_HIP(hipGetLastError());
    return NC_OK;
}

}  // namespace nc
