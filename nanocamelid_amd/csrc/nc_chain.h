// Exact parallel evaluation of a sequential f32 sum of non-negative terms.
//
// The reference accumulates several sums strictly left to right in f32 (the RMSNorm
// sum of squares, inference.rs:697-706; the softmax denominator, inference.rs:3522-3540):
//
//     s_{-1} = s0 (0 unless a carry-in is given),   s_i = fl32(s_{i-1} + a_i),   i = 0 .. n-1.
//
// On gfx950 a wave issues at most one VALU instruction per 8 cycles, so a dependent
// v_add_f32 chain costs 8 cycles per term and a 4096-term chain ~14 us when evaluated
// literally.  This routine returns the bit-identical s_{n-1} from a
// workgroup of T threads; thread t owns the segment of terms a_{tE} .. a_{tE+E-1}:
//
//  1. Guess.  G_t = fl32(s0 + sum of all earlier terms), the prefix taken in double (a
//     block scan): it differs from the true chain value at the segment start only by the
//     chain's accumulated rounding, a few ulps.
//  2. Segment from the guess.  Each thread runs its E additions sequentially from G_t,
//     giving the end value X_t and the increment D_t = X_t - G_t (exact in double).  If the
//     true start S_t lies within 256 ulps of G_t in the same binade, and the run neither
//     leaves that binade (start and end in the same binade, both 256 ulps from its edges)
//     nor rounds an exact tie (the Fast2Sum error of a step equals half an ulp), then
//     every step rounds the same way from S_t as from G_t, so the true end is S_t + D_t:
//     both states are multiples of the binade's ulp.  Segments where that can fail are
//     "sensitive" (typically the ~12 that contain a binade crossing of the growing sum).
//  3. C_t = s0 + sum of the earlier D (block scan in double): the start of segment t if no
//     earlier segment were sensitive.
//  4. Walk.  One wave visits the sensitive segments in order: it advances the true chain
//     value over the insensitive segments in between (their increments add exactly),
//     evaluates the sensitive segment term by term, and records the correction
//     shift_k = (true end) - (C_k + D_k).  A segment's start is then C_t + shift of the last
//     sensitive segment before it.
//  5. Verify.  Every thread recomputes its segment sequentially from that start; if each
//     start equals the previous segment's recomputed end (and the first equals s0), the
//     last end IS the sequential chain, by induction, whatever the guesses were.  If any
//     check fails (the chain drifted > 256 ulps from the exact prefix, or more than
//     kChainMaxSensitive segments are sensitive), thread 0 recomputes the chain sequentially.
//
// The result is therefore always bit-identical to the sequential loop; the guesses only
// decide how fast it is found.  Terms must be >= 0 (sums of squares, exponentials); the start
// may be negative (a subtraction chain r_i = r_{i-1} - a_i is the negation of this chain from
// -r, since round-to-nearest is symmetric).
//
// Wave-level scans use gfx9 DPP (row_shr, row_bcast, wave_shr): no LDS round trips.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nc {

constexpr int kChainMaxSensitive = 256;

struct ChainEntry {
    double cstart;  // C_k: uncorrected start of sensitive segment k
    double cend;    // C_k + D_k: its uncorrected end
    double shift;   // true end - cend, after the walk
    int seg;        // segment (thread) index
};

// A sensitive entry as the walk reads it: the advance over the insensitive segments before
// it, then its terms (padded to whole 16-byte rows).
template <int E>
struct WalkRow {
    static constexpr int W = (E + 1 + 3) / 4 * 4;
    float v[W];
};

template <int T>
struct ChainScratch {
    double dtot[T / 64];   // wave totals of the guess scan
    double dtot2[T / 64];  // wave totals of the increment scan
    int itot[T / 64];
    float last[T];
    ChainEntry ent[kChainMaxSensitive];
    float walk_end[64];  // chain value after each entry of the current 64-entry window
    int bad;             // set by any thread whose boundary check fails
    int first;           // FIND: first term index whose chain value is >= 0 (INT_MAX: none)
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

// Block-wide exclusive scan of a double (and optionally of an int in the same pass).  The
// wave totals array must not be written again before a later barrier (each scan of
// exact_chain_sum has its own, and the routine ends with a barrier).
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
    *kexcl = kbase + kincl - k;
    *ktotal = kall;
    return base + excl;
}

constexpr int kChainMargin = 256;  // ulps between a guess and the true state that are tolerated

// Step 2 for one thread: its E terms added in order from the guess g; x receives the end
// value.  Returns whether moving the run to the true start might not translate it exactly:
// the guess or the end lies within kChainMargin ulps of a binade edge, the run leaves the
// guess's binade, a step rounds an exact tie, or the binade is too small for the test.
// s0_neg: the chain started below zero, so a zero guess is a cancellation, not an exact start.
template <int E>
__device__ __forceinline__ bool chain_run_sensitive(const float (&a)[E], float g, bool s0_neg, float& x_out) {
    const uint32_t bg = __float_as_uint(g);
    const int eg = (int)(bg >> 23);  // sign and exponent: the binade test below includes the sign
    const int ea = eg & 0xff;
    // half an ulp of g's binade, 2^(ea - 151); only used when ea >= 25 (else sensitive anyway)
    const float half = __uint_as_float((uint32_t)(ea > 25 ? ea - 24 : 1) << 23);
    float x = g;
    bool tie = false;
#pragma unroll
    for (int j = 0; j < E; j++) {
        const float r = x + a[j];
        // Fast2Sum error of the step (exact while x >= a[j], i.e. whenever the binade holds)
        tie |= __builtin_fabsf(a[j] - (r - x)) == half;
        x = r;
    }
    x_out = x;
    const uint32_t bx = __float_as_uint(x);
    const int mg = (int)(bg & 0x7fffff), mx = (int)(bx & 0x7fffff);
    // Absorbed runs translate exactly from any start: all-zero terms, or (binade >= 2^-100)
    // every term below a quarter ulp of g's binade, which is below half an ulp of any start
    // within the margin (that start's binade is g's or a neighbour, whose ulp is at least
    // half of g's), so every step rounds back to its start.
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < E; j++) amax = fmaxf(amax, a[j]);
    const bool absorbed = (amax == 0.0f) | ((ea >= 27) & (amax < 0.5f * half));
    // g == 0 with s0 >= 0: every earlier term and s0 are 0, so the start is exact and the run
    // is the truth
    return !absorbed & ((bg != 0) | s0_neg) &
           ((ea < 25) | ((int)(bx >> 23) != eg) | (mg < kChainMargin) | (mx + kChainMargin >= (1 << 23)) | tie);
}

// The walk's serial part, run by one lane: adds rows[0 .. cnt) in order to S (a row holds the
// advance over the insensitive runs before its entry, then the entry's E terms) and records
// the value after each row in walk_end[q].  Three register sets rotate, so entry q's row is
// read from LDS two entries ahead and only the dependent adds are serial.
template <int E>
__device__ __forceinline__ float chain_walk_rows(const WalkRow<E>* rows, int cnt, float S, float* walk_end) {
    typedef float f4v __attribute__((ext_vector_type(4)));
    constexpr int W = WalkRow<E>::W;
    f4v r0[W / 4], r1[W / 4], r2[W / 4];
#define NC_WALK_READ(R, Q)                                                                          \
    {                                                                                               \
        const int q_ = min((Q), cnt - 1);                                                           \
        _Pragma("unroll") for (int c = 0; c < W / 4; c++) R[c] = *(const f4v*)&rows[q_].v[4 * c];  \
    }
#define NC_WALK_ADD(R, Q)                                                                           \
    {                                                                                               \
        _Pragma("unroll") for (int c = 0; c < W / 4; c++) {                                        \
            if (4 * c + 0 <= E) S = S + R[c].x;                                                     \
            if (4 * c + 1 <= E) S = S + R[c].y;                                                     \
            if (4 * c + 2 <= E) S = S + R[c].z;                                                     \
            if (4 * c + 3 <= E) S = S + R[c].w;                                                     \
        }                                                                                           \
        walk_end[(Q)] = S;                                                                          \
    }
    // (the padding after the E terms is never added)
    NC_WALK_READ(r0, 0)
    NC_WALK_READ(r1, 1)
    for (int q = 0; q < cnt; q += 3) {
        NC_WALK_READ(r2, q + 2)
        NC_WALK_ADD(r0, q)
        if (q + 1 >= cnt) break;
        NC_WALK_READ(r0, q + 3)
        NC_WALK_ADD(r1, q + 1)
        if (q + 2 >= cnt) break;
        NC_WALK_READ(r1, q + 4)
        NC_WALK_ADD(r2, q + 2)
    }
#undef NC_WALK_ADD
#undef NC_WALK_READ
    return S;
}

// Thread t holds terms a[0..E) = a_{tE} .. a_{tE+E-1} (n = T*E terms; pad with zeros, which
// leave the chain unchanged).  The chain starts from s_{-1} = s0, so a long sum can be
// evaluated as consecutive segments, each starting from the previous segment's result.  A
// negative s0 is allowed (terms stay >= 0): the state then rises through zero, whose
// neighbourhood only makes segments sensitive.  a_lds: n floats of LDS used by the walk and
// the fallback.  Every thread of the block must call it; returns s_{n-1} to all threads.
// FIND: sc.first also receives the first index i (0 .. n-1) with s_i >= 0, or INT_MAX.
template <int E, int T, bool FIND = false>
__device__ float exact_chain_sum(const float (&a)[E], ChainScratch<T>& sc, float* a_lds, float s0 = 0.0f) {
    static_assert(E >= 1 && E <= 32, "terms per thread");
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < E; j++) a_lds[t * E + j] = a[j];

    // 1. guess of the segment's start from the double prefix
    double run = 0.0;
#pragma unroll
    for (int j = 0; j < E; j++) run += (double)a[j];
    const double exclp = (double)s0 + block_excl_scan_f64<T>(run, sc.dtot);
    const float g = (float)exclp;  // segment 0: exactly s0

    // 2. the segment evaluated from the guess, with the tie and binade tests
    float x;
    const bool sens = chain_run_sensitive<E>(a, g, s0 < 0.0f, x);
    const double d = (double)x - (double)g;

    // 3. uncorrected starts C_t, with the sensitive count scanned in the same pass
    int off, total_s;
    const double cstart = (double)s0 + block_excl_scan_f64_i32<T>(d, sens ? 1 : 0, sc.dtot2, sc.itot, &off, &total_s);

    // 4. sensitive list in ascending order, then the walk (one wave)
    const bool listed = total_s <= kChainMaxSensitive;
    if (listed && sens) {
        ChainEntry& ce = sc.ent[off];
        ce.cstart = cstart;
        ce.cend = cstart + d;
        ce.seg = t;
    }
    if (t == 0) {
        sc.bad = 0;  // read after the verification barrier, two barriers on
        if (FIND) sc.first = 0x7fffffff;
    }
    __syncthreads();
    if (listed && t < 64) {
        // wave 0: lane q stages entry e0 + q (its advance over the insensitive segments before
        // it, which is exact, and its E terms) as one LDS row; lane 0 then walks the rows in
        // order with 16-byte reads issued two entries ahead, so only the dependent adds are
        // serial.
        constexpr int W = WalkRow<E>::W;
        __shared__ WalkRow<E> rows[64];
        float S = s0;  // true chain value at the end of the last walked segment (lane 0)
        for (int e0 = 0; e0 < total_s; e0 += 64) {
            const int me = e0 + t;
            const int cnt = min(64, total_s - e0);
            double ce = 0.0;
            if (me < total_s) {
                const double cs = sc.ent[me].cstart;
                ce = sc.ent[me].cend;
                const double cl = me == 0 ? (double)s0 : sc.ent[me - 1].cend;
                rows[t].v[0] = (float)(cs - cl);
                const float* ap = a_lds + sc.ent[me].seg * E;
#pragma unroll
                for (int j = 0; j < E; j++) rows[t].v[1 + j] = ap[j];
#pragma unroll
                for (int j = E + 1; j < W; j++) rows[t].v[j] = 0.0f;
            }
            // rows of this wave's lanes: LDS operations of one wave complete in order
            if (t == 0) S = chain_walk_rows<E>(rows, cnt, S, sc.walk_end);
            if (me < total_s) sc.ent[me].shift = (double)sc.walk_end[t] - ce;
        }
    }
    __syncthreads();

    // 5. corrected start, sequential recomputation, and the check of every boundary
    bool bad = !listed;
    float y = 0.0f;
    if (listed) {
        const double sh = off == 0 ? 0.0 : sc.ent[off - 1].shift;
        const float start = (float)(cstart + sh);
        y = start;
        int fi = -1;
#pragma unroll
        for (int j = 0; j < E; j++) {
            y = y + a[j];
            if (FIND && fi < 0 && y >= 0.0f) fi = j;
        }
        if (FIND && fi >= 0) atomicMin(&sc.first, t * E + fi);  // meaningful only if every check passes
        sc.last[t] = y;
        bad = t == 0 ? start != s0 : false;
        // the start is compared with the previous segment's end after the barrier
        run = (double)start;  // reuse a register for the start
    }
    __syncthreads();
    if (listed && t > 0) bad |= (float)run != sc.last[t - 1];
    if (bad) sc.bad = 1;
    __syncthreads();
    const bool any_bad = sc.bad != 0;
    if (!any_bad) {
        if (t == T - 1) sc.result = y;
    } else if (t == 0) {
        float v = s0;
        int fi = 0x7fffffff;
        for (int i = 0; i < T * E; i++) {
            v = v + a_lds[i];
            if (FIND && fi == 0x7fffffff && v >= 0.0f) fi = i;
        }
        sc.result = v;
        if (FIND) sc.first = fi;
    }
    __syncthreads();
    return sc.result;
}

}  // namespace nc
