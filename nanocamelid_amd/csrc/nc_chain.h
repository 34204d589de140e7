// Exact parallel evaluation of a sequential f32 sum of non-negative terms.
//
// The reference accumulates several sums strictly left to right in f32 (the RMSNorm
// sum of squares, inference.rs:697-706; the softmax denominator, inference.rs:3522-3540):
//
//     s_{-1} = 0,   s_i = fl32(s_{i-1} + a_i),   i = 0 .. n-1.
//
// On gfx950 one dependent v_add_f32 costs ~10 cycles, so a 4096-term chain is ~21 us
// when evaluated literally.  This routine returns the bit-identical s_{n-1} from a
// workgroup of T threads in a few parallel passes:
//
//  1. Guess.  P_i = sum_{j<=i} a_j in double (a block scan) and G_{i-1} = fl32(P_{i-1})
//     approximates the chain value before step i (it differs from s_{i-1} only by the
//     chain's accumulated rounding, a few ulps).
//  2. Increments.  If s_{i-1} and G_{i-1} lie in the same binade, the step neither
//     crosses into the next binade nor rounds a tie, then
//         fl32(s_{i-1} + a_i) - s_{i-1} = fl32(G_{i-1} + a_i) - G_{i-1} =: d_i,
//     because both states are multiples of the binade's ulp.  Steps where that can fail
//     (a binade boundary within a margin of 256 ulps of G, or a tie) are flagged
//     "sensitive"; there are ~20 of them in 4096 terms (most binade crossings happen
//     in the first few dozen terms, where the sum grows fastest).
//  3. c_i = sum_{j<=i} d_j (block scan in double; exact, since partial sums are
//     differences of f32 values).
//  4. Sensitive walk.  One wave visits the sensitive steps in order and computes their
//     true result from the corrected chain value before them, keeping the running
//     correction shift_k = s_k - c_k.  Every other step inherits the shift of the last
//     sensitive step before it.
//  5. Verify.  Every step is checked locally, in parallel: the corrected value must be an
//     f32 and equal fl32(previous corrected value + a_i).  If every step holds, the
//     corrected sequence IS the sequential chain (induction from s_{-1} = 0), whatever
//     the guesses were.  If any step fails (never seen on test data; it needs the chain
//     to drift > 256 ulps from the exact prefix), thread 0 recomputes the chain
//     sequentially.
//
// The result is therefore always bit-identical to the sequential loop; the guesses only
// decide how fast it is found.  Terms must be >= 0 (sums of squares, exponentials).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nc {

constexpr int kChainMaxSensitive = 256;

struct ChainEntry {
    double cprev;  // c_{k-1} (uncorrected)
    double cold;   // c_k (uncorrected)
    double shift;  // s_k - c_k after the walk
    float a;       // a_k
    int idx;       // k
};

template <int T>
struct ChainScratch {
    double dtot[T / 64];
    int itot[T / 64];
    float last[T];
    ChainEntry ent[kChainMaxSensitive];
    float result;
};

// Binade class of a non-negative value at f32 resolution: the unbiased binary exponent,
// with zero and the f32 subnormal range (one ulp, 2^-149) collapsed into one class.
__device__ __forceinline__ int chain_binade(double v) {
    if (!(v >= 1.1754943508222875e-38)) return -127;
    return (int)((__double_as_longlong(v) >> 52) & 0x7ff) - 1023;
}

// ulp of a non-negative f32 value (2^-149 in the subnormal range).
__device__ __forceinline__ double chain_ulp(float x) {
    const int e = (int)((__float_as_uint(x) >> 23) & 0xff);
    return __longlong_as_double((long long)(e > 0 ? e - 23 + 1023 - 127 : 1023 - 149) << 52);
}

__device__ __forceinline__ double chain_readlane(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffff), lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

template <int T>
__device__ __forceinline__ double chain_excl_scan_f64(double v, double* tot, double* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    double incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const double o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    double excl = __shfl_up(incl, 1, 64);
    if (lane == 0) excl = 0.0;
    if (lane == 63) tot[w] = incl;
    __syncthreads();
    double base = 0.0, all = 0.0;
#pragma unroll
    for (int i = 0; i < T / 64; i++) {
        const double t = tot[i];
        if (i < w) base += t;
        all += t;
    }
    __syncthreads();
    *total = all;
    return base + excl;
}

template <int T>
__device__ __forceinline__ int chain_excl_scan_i32(int v, int* tot, int* total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(incl, off, 64);
        if (lane >= off) incl += o;
    }
    if (lane == 63) tot[w] = incl;
    __syncthreads();
    int base = 0, all = 0;
#pragma unroll
    for (int i = 0; i < T / 64; i++) {
        const int t = tot[i];
        if (i < w) base += t;
        all += t;
    }
    __syncthreads();
    *total = all;
    return base + incl - v;
}

// Thread t holds terms a[0..E) = a_{tE} .. a_{tE+E-1} (n = T*E terms; pad with zeros, which
// leave the chain unchanged).  a_lds: n floats of LDS used by the fallback.  Every thread
// of the block must call it; returns s_{n-1} to all threads.
template <int E, int T>
__device__ float exact_chain_sum(const float (&a)[E], ChainScratch<T>& sc, float* a_lds) {
    static_assert(E >= 1 && E <= 32, "terms per thread");
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < E; j++) a_lds[t * E + j] = a[j];

    // 1. guesses from the exact-ish double prefix
    double w[E];
    double run = 0.0;
#pragma unroll
    for (int j = 0; j < E; j++) {
        run += (double)a[j];
        w[j] = run;
    }
    double totp;
    const double exclp = chain_excl_scan_f64<T>(run, sc.dtot, &totp);

    // 2. speculative increments and sensitivity (w[] becomes d[])
    uint32_t sens = 0;
    double prevp = exclp;
#pragma unroll
    for (int j = 0; j < E; j++) {
        const double pj = exclp + w[j];
        const float g = (float)prevp;
        const float r = g + a[j];
        const double dj = (double)r - (double)g;
        bool s = false;
        if (g != 0.0f) {  // g == 0 means every earlier term is 0, so the chain is exactly 0
            const double rem = ((double)g + (double)a[j]) - (double)r;
            s = __builtin_fabs(rem) == 0.5 * chain_ulp(r);
            const double m = 256.0 * chain_ulp(g);
            const double lo = (double)g - m, hi = (double)g + m + (double)a[j];
            s = s || chain_binade(lo) != chain_binade(hi);
        }
        if (s) sens |= 1u << j;
        w[j] = dj;
        prevp = pj;
    }

    // 3. uncorrected chain c = prefix of d
    run = 0.0;
#pragma unroll
    for (int j = 0; j < E; j++) {
        run += w[j];
        w[j] = run;
    }
    double totc;
    const double exclc = chain_excl_scan_f64<T>(run, sc.dtot, &totc);

    // 4. sensitive list in ascending order, then the walk
    int total_s;
    const int off = chain_excl_scan_i32<T>(__popc(sens), sc.itot, &total_s);
    const bool listed = total_s <= kChainMaxSensitive;
    if (listed) {
        int e = off;
#pragma unroll
        for (int j = 0; j < E; j++) {
            if (sens >> j & 1) {
                ChainEntry& ce = sc.ent[e++];
                ce.cprev = j == 0 ? exclc : exclc + w[j - 1];
                ce.cold = exclc + w[j];
                ce.a = a[j];
                ce.idx = t * E + j;
            }
        }
    }
    __syncthreads();
    if (listed && t < 64) {
        double acc = 0.0;
        for (int e0 = 0; e0 < total_s; e0 += 64) {
            const int me = e0 + t;
            double cp = 0.0, co = 0.0;
            float av = 0.0f;
            int ix = 0;
            if (me < total_s) {
                cp = sc.ent[me].cprev;
                co = sc.ent[me].cold;
                av = sc.ent[me].a;
                ix = sc.ent[me].idx;
            }
            double mine = 0.0;
            const int cnt = min(64, total_s - e0);
            for (int q = 0; q < cnt; q++) {  // q is wave-uniform: v_readlane, no LDS
                const double cpq = chain_readlane(cp, q), coq = chain_readlane(co, q);
                const float aq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(av), q));
                const int iq = __builtin_amdgcn_readlane(ix, q);
                const double prev = iq == 0 ? 0.0 : cpq + acc;
                const float tr = (float)prev + aq;
                acc = (double)tr - coq;
                if (t == q) mine = acc;
            }
            if (me < total_s) sc.ent[me].shift = mine;
        }
    }
    __syncthreads();

    // 5. corrected values and the local check of every step
    bool bad = !listed;
    float cn[E];
    if (listed) {
        double cur = off == 0 ? 0.0 : sc.ent[off - 1].shift;
        int e = off;
#pragma unroll
        for (int j = 0; j < E; j++) {
            if (sens >> j & 1) cur = sc.ent[e++].shift;
            const double v = exclc + w[j] + cur;
            cn[j] = (float)v;
            bad = bad || (double)cn[j] != v;
        }
        sc.last[t] = cn[E - 1];
    }
    __syncthreads();
    if (listed) {
        float prev = t == 0 ? 0.0f : sc.last[t - 1];
#pragma unroll
        for (int j = 0; j < E; j++) {
            bad = bad || (prev + a[j]) != cn[j];
            prev = cn[j];
        }
    }
    const bool any_bad = __syncthreads_or(bad);
    if (!any_bad) {
        if (t == T - 1) sc.result = cn[E - 1];
    } else if (t == 0) {
        float s = 0.0f;
        for (int i = 0; i < T * E; i++) s = s + a_lds[i];
        sc.result = s;
    }
    __syncthreads();
    return sc.result;
}

}  // namespace nc
