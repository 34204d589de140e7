// Exact parallel evaluation of a sequential f32 sum of non-negative terms.
//
// The reference accumulates several sums strictly left to right in f32 (the RMSNorm
// sum of squares, inference.rs:697-706; the softmax denominator, inference.rs:3522-3540):
//
//     s_{-1} = s0 (0 unless a carry-in is given),   s_i = fl32(s_{i-1} + a_i),   i = 0 .. n-1.
//
// On gfx950 one dependent v_add_f32 costs ~10 cycles, so a 4096-term chain is ~21 us
// when evaluated literally.  This routine returns the bit-identical s_{n-1} from a
// workgroup of T threads in a few parallel passes:
//
//  1. Guess.  P_i = sum_{j<=i} a_j in double (a block scan) and g_i = fl32(P_{i-1})
//     approximates the chain value before step i (it differs from s_{i-1} only by the
//     chain's accumulated rounding, a few ulps).
//  2. Increments.  If s_{i-1} lies within 256 ulps of g_i, in the same binade, and the
//     step neither reaches the next binade nor rounds an exact tie, then
//         fl32(s_{i-1} + a_i) - s_{i-1} = fl32(g_i + a_i) - g_i =: d_i,
//     because both states are multiples of the binade's ulp.  Steps where that can fail
//     are flagged "sensitive" by integer tests on the f32 bits; there are ~20 of them in
//     4096 terms of smooth data (binade crossings cluster in the first few dozen terms,
//     where the sum grows fastest).
//  3. c_i = sum_{j<=i} d_j (block scan in double).
//  4. Sensitive walk.  One wave visits the sensitive steps in order and computes their
//     true result from the corrected chain value before them (carried in f32, two
//     dependent adds per step), giving the correction shift_k = s_k - c_k.  Every other
//     step inherits the shift of the last sensitive step before it.
//  5. Verify.  With cn_i = fl32(c_i + shift), every step is checked locally and in
//     parallel: cn_i == fl32(cn_{i-1} + a_i), cn_{-1} = 0.  If all hold, cn IS the
//     sequential chain (induction), whatever the guesses were.  If any fails (it needs the
//     chain to drift > 256 ulps from the exact prefix, or more than kChainMaxSensitive
//     sensitive steps), thread 0 recomputes the chain sequentially.
//
// The result is therefore always bit-identical to the sequential loop; the guesses only
// decide how fast it is found.  Terms must be >= 0 (sums of squares, exponentials).
//
// Wave-level scans use gfx9 DPP (row_shr, row_bcast, wave_shr): no LDS round trips.
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
};

template <int T>
struct ChainScratch {
    double dtot[T / 64];
    int itot[T / 64];
    float last[T];
    ChainEntry ent[kChainMaxSensitive];
    float result;
};

// ---------------------------------------------------------------- DPP helpers (wave64)
enum : int {
    kDppRowShr1 = 0x111,
    kDppRowShr2 = 0x112,
    kDppRowShr4 = 0x114,
    kDppRowShr8 = 0x118,
    kDppWaveShr1 = 0x138,
    kDppRowBcast15 = 0x142,
    kDppRowBcast31 = 0x143,
};

// Lanes whose DPP source is invalid or whose row is masked off read 0.
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ int dpp0_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, ROWS, 0xf, false);
}
template <int CTRL, int ROWS = 0xf>
__device__ __forceinline__ double dpp0_d(double v) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(b & 0xffffffff), CTRL, ROWS, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, ROWS, 0xf, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Inclusive scans over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan_i32(int v) {
    v += dpp0_i<kDppRowShr1>(v);
    v += dpp0_i<kDppRowShr2>(v);
    v += dpp0_i<kDppRowShr4>(v);
    v += dpp0_i<kDppRowShr8>(v);
    v += dpp0_i<kDppRowBcast15, 0xa>(v);
    v += dpp0_i<kDppRowBcast31, 0xc>(v);
    return v;
}
__device__ __forceinline__ double wave_incl_scan_f64(double v) {
    v += dpp0_d<kDppRowShr1>(v);
    v += dpp0_d<kDppRowShr2>(v);
    v += dpp0_d<kDppRowShr4>(v);
    v += dpp0_d<kDppRowShr8>(v);
    v += dpp0_d<kDppRowBcast15, 0xa>(v);
    v += dpp0_d<kDppRowBcast31, 0xc>(v);
    return v;
}

__device__ __forceinline__ double chain_readlane(double v, int lane) {
    const long long b = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)(b & 0xffffffff), lane);
    const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

// Block-wide exclusive scan of a double (and optionally of an int in the same pass).
template <int T>
__device__ __forceinline__ double block_excl_scan_f64(double v, double* tot) {
    const int w = threadIdx.x >> 6;
    const double incl = wave_incl_scan_f64(v);
    const double excl = dpp0_d<kDppWaveShr1>(incl);
    if ((threadIdx.x & 63) == 63) tot[w] = incl;
    __syncthreads();
    double base = 0.0;
#pragma unroll
    for (int i = 0; i < T / 64; i++)
        if (i < w) base += tot[i];
    __syncthreads();
    return base + excl;
}
template <int T>
__device__ __forceinline__ double block_excl_scan_f64_i32(double v, int k, double* tot, int* itot, int* kexcl,
                                                           int* ktotal) {
    const int w = threadIdx.x >> 6;
    const double incl = wave_incl_scan_f64(v);
    const double excl = dpp0_d<kDppWaveShr1>(incl);
    const int kincl = wave_incl_scan_i32(k);
    if ((threadIdx.x & 63) == 63) {
        tot[w] = incl;
        itot[w] = kincl;
    }
    __syncthreads();
    double base = 0.0;
    int kbase = 0, kall = 0;
#pragma unroll
    for (int i = 0; i < T / 64; i++) {
        const int ki = itot[i];
        if (i < w) {
            base += tot[i];
            kbase += ki;
        }
        kall += ki;
    }
    __syncthreads();
    *kexcl = kbase + kincl - k;
    *ktotal = kall;
    return base + excl;
}

// Step i with guess g (the chain value before the step, approximately) and term a >= 0:
// returns d = fl32(g + a) - g exactly and whether the step is sensitive (see above).
// Branch free (selects only): every lane evaluates every test.
__device__ __forceinline__ double chain_increment(float g, float a, bool* sensitive) {
    const float r = g + a;
    const double d = (double)r - (double)g;
    const uint32_t bg = __float_as_uint(g), ba = __float_as_uint(a);
    const int eg = (int)(bg >> 23), ea = (int)(ba >> 23);
    const int mg = (int)(bg & 0x7fffff);
    const int sh = eg - (ea > 0 ? ea : 1);  // a's binary exponent below g's
    const uint32_t ma = (ba & 0x7fffffu) | (ea > 0 ? 0x800000u : 0u);
    const int shc = sh < 1 ? 1 : (sh > 31 ? 31 : sh);
    const uint32_t low = ma & ((1u << shc) - 1u);
    // exact tie of g + a at g's ulp (only possible for 2 <= sh <= 24)
    const bool tie = (sh >= 2) & (sh <= 24) & (low == (1u << (shc - 1)));
    const int a_ulps = sh > 24 ? 1 : (int)(ma >> shc) + 1;  // >= a / ulp(g)
    // sh < 2: a comparable to the running sum, the binade may change; eg == 0: subnormal
    // running sum; the margin tests: s may sit in the binade below, or s + a may reach the
    // next binade.
    const bool s = (sh < 2) | tie | (mg + a_ulps + 256 >= (1 << 23)) | (mg < 256) | (eg == 0);
    // g == 0: every earlier term is 0, the chain is exactly 0 and d = a.  a == 0: d = 0.
    *sensitive = s & (bg != 0) & (ba != 0);
    return d;
}

// Thread t holds terms a[0..E) = a_{tE} .. a_{tE+E-1} (n = T*E terms; pad with zeros, which
// leave the chain unchanged).  The chain starts from s_{-1} = s0 >= 0, so a long sum can be
// evaluated as consecutive segments, each starting from the previous segment's result.
// a_lds: n floats of LDS used by the fallback.  Every thread of the block must call it;
// returns s_{n-1} to all threads.
template <int E, int T>
__device__ float exact_chain_sum(const float (&a)[E], ChainScratch<T>& sc, float* a_lds, float s0 = 0.0f) {
    static_assert(E >= 1 && E <= 32, "terms per thread");
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < E; j++) a_lds[t * E + j] = a[j];

    // 1. guesses from the double prefix
    double w[E];
    double run = 0.0;
#pragma unroll
    for (int j = 0; j < E; j++) {
        run += (double)a[j];
        w[j] = run;
    }
    const double exclp = (double)s0 + block_excl_scan_f64<T>(run, sc.dtot);

    // 2. speculative increments and sensitivity (w[] becomes d[])
    uint32_t sens = 0;
    float g = (float)exclp;
#pragma unroll
    for (int j = 0; j < E; j++) {
        const float gnext = (float)(exclp + w[j]);
        bool s;
        w[j] = chain_increment(g, a[j], &s);
        if (s) sens |= 1u << j;
        g = gnext;
    }

    // 3. uncorrected chain c = prefix of d, with the sensitive count scanned in the same pass
    run = 0.0;
#pragma unroll
    for (int j = 0; j < E; j++) {
        run += w[j];
        w[j] = run;
    }
    int off, total_s;
    const double exclc = block_excl_scan_f64_i32<T>(run, __popc(sens), sc.dtot, sc.itot, &off, &total_s);

    // 4. sensitive list in ascending order, then the walk
    const bool listed = total_s <= kChainMaxSensitive;
    if (listed && sens) {
        int e = off;
#pragma unroll
        for (int j = 0; j < E; j++) {
            if (sens >> j & 1) {
                ChainEntry& ce = sc.ent[e++];
                ce.cprev = j == 0 ? exclc : exclc + w[j - 1];
                ce.cold = exclc + w[j];
                ce.a = a[j];
            }
        }
    }
    __syncthreads();
    if (listed && t < 64) {
        // s_{k-1} = s_j + (c_{k-1} - c_j) with j the previous sensitive step (the advance is
        // exact: nothing between j and k changes binade or ties), then s_k = fl32(s_{k-1} + a_k).
        float s_run = s0;      // s_j (s_{-1} = s0, c_{-1} = 0 before the first entry)
        double co_last = 0.0;  // c_j
        for (int e0 = 0; e0 < total_s; e0 += 64) {
            const int me = e0 + t;
            double cp = 0.0, co = 0.0;
            float av = 0.0f;
            if (me < total_s) {
                cp = sc.ent[me].cprev;
                co = sc.ent[me].cold;
                av = sc.ent[me].a;
            }
            double co_prev = dpp0_d<kDppWaveShr1>(co);
            if (t == 0) co_prev = co_last;
            const float adv = (float)(cp - co_prev);
            float mine = 0.0f;
            const int cnt = min(64, total_s - e0);
            for (int q0 = 0; q0 < cnt; q0 += 8) {  // q is wave-uniform: v_readlane, no LDS
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const int q = q0 + u;
                    if (q < cnt) {
                        const float advq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(adv), q));
                        const float aq = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(av), q));
                        s_run = (s_run + advq) + aq;
                        mine = t == q ? s_run : mine;
                    }
                }
            }
            if (me < total_s) sc.ent[me].shift = (double)mine - co;
            co_last = chain_readlane(co, cnt - 1);
        }
    }
    __syncthreads();

    // 5. corrected values and the local check of every step
    bool bad = !listed;
    float cn[E];
    if (listed) {
        double cur = off == 0 ? (double)s0 : sc.ent[off - 1].shift;
        int e = off;
#pragma unroll
        for (int j = 0; j < E; j++) {
            if (sens >> j & 1) cur = sc.ent[e++].shift;
            cn[j] = (float)(exclc + w[j] + cur);
        }
        sc.last[t] = cn[E - 1];
    }
    __syncthreads();
    if (listed) {
        float prev = t == 0 ? s0 : sc.last[t - 1];
#pragma unroll
        for (int j = 0; j < E; j++) {
            bad |= (prev + a[j]) != cn[j];
            prev = cn[j];
        }
    }
    const bool any_bad = __syncthreads_or(bad);
    if (!any_bad) {
        if (t == T - 1) sc.result = cn[E - 1];
    } else if (t == 0) {
        float s = s0;
        for (int i = 0; i < T * E; i++) s = s + a_lds[i];
        sc.result = s;
    }
    __syncthreads();
    return sc.result;
}

}  // namespace nc
