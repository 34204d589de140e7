// Device helpers shared by the HIP kernels of the verify path (gfx950, wave64).
//
// Numerics are bit-faithful to the reference's portable x86 path: every f32
// expression is evaluated in the reference's order with IEEE rounding (the
// library is compiled with -ffp-contract=off and correctly rounded f32 divide
// and sqrt), and expf reproduces glibc's expf bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace nc {

constexpr int kWave = 64;

// tab[i] = bits(2^(i/32) rounded to double) - (i << 47): the exponent-adjusted table of
// the expf algorithm below (values generated from exp2l on the host).
static __constant__ uint64_t c_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

// expf of glibc >= 2.27 (the ARM optimized-routines algorithm by Szabolcs Nagy,
// as built with FMA contraction on x86-64): x*N/ln2 = k + r evaluated in double,
// 2^(k/N) from a 32-entry table, a degree-3 polynomial in r.  The product
// InvLn2N*x is fused into both of its uses and every a*b+c is an fma, which is
// the only formulation that matches the system expf on all 2^32 inputs (checked
// exhaustively on the host, and on the device by the parity tests).
__device__ __forceinline__ float expf_glibc(float x) {
    const double kInvLn2N = 0x1.71547652b82fep+0 * 32.0;
    const double kShift = 0x1.8p+52;
    const double kC0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double kC1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double kC2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux = __float_as_uint(x);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {  // |x| >= 88 or nan/inf  (top12(88.0f) == 0x42b)
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double kd = __builtin_fma(kInvLn2N, xd, kShift);
    uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd -= kShift;
    double r = __builtin_fma(kInvLn2N, xd, -kd);
    uint64_t t = c_exp2_tab[ki & 31];
    t += ki << 47;
    double s = __longlong_as_double((long long)t);
    double z = __builtin_fma(kC0, r, kC1);
    double r2 = r * r;
    double y = __builtin_fma(kC2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// Exact IEEE binary16 -> binary32 (q8.rs:3626 fast_f16_to_f32 for non-NaN codes).
__device__ __forceinline__ float f16_to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// Rust f32::round: half away from zero.
__device__ __forceinline__ float round_half_away(float v) { return __builtin_roundf(v); }

// Q8_0 activation block quantisation (inference.rs:1012-1029) of the value held by
// this lane within a 32-lane group.  Returns q; *scale_out = amax/127 (f32).
__device__ __forceinline__ int quantize_lane_q8(float v, float amax, float* scale_out) {
    float scale = amax / 127.0f;
    *scale_out = scale;
    if (scale > 0.0f) {
        float inv = 1.0f / scale;
        float q = round_half_away(v * inv);
        q = q < -127.0f ? -127.0f : (q > 127.0f ? 127.0f : q);
        return (int)q;
    }
    return 0;
}

// Max of |v| over each 32-lane half of the wave (exact: max is order independent).
__device__ __forceinline__ float halfwave_amax(float v) {
    float a = __builtin_fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        float o = __shfl_xor(a, off, 64);
        a = o > a ? o : a;
    }
    return a;
}

__device__ __forceinline__ int halfwave_isum(int v) {
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ int wave_id_uniform() {
    return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}

}  // namespace nc
