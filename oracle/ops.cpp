// Oracle: block formats, quantisers, matmuls and row ops.
// TEST INFRASTRUCTURE ONLY -- a restatement of the reference's portable x86 path
// (see nc_oracle.h for the pinning of each function).  Built with
// -O2 -ffp-contract=off so every f32 expression rounds exactly as Rust does.
#include "oracle_internal.h"

#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

extern "C" {

// q8.rs:3599-3623 f16_bits_to_f32 / q8.rs:3626-3641 fast_f16_to_f32:
// exact IEEE binary16 -> binary32, subnormals normalised, NaN payload kept.
float or_f16_to_f32(uint16_t bits) {
    uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    uint32_t exponent = (bits & 0x7c00u) >> 10;
    uint32_t fraction = bits & 0x03ffu;
    uint32_t out;
    if (exponent == 0) {
        if (fraction == 0) {
            out = sign;
        } else {
            uint32_t mantissa = fraction;
            int32_t e = -14;
            while ((mantissa & 0x0400u) == 0) {
                mantissa <<= 1;
                e -= 1;
            }
            mantissa &= 0x03ffu;
            out = sign | ((uint32_t)(e + 127) << 23) | (mantissa << 13);
        }
    } else if (exponent == 0x1f) {
        out = sign | 0x7f800000u | (fraction << 13);
    } else {
        out = sign | ((exponent + 112) << 23) | (fraction << 13);
    }
    return bits_f32(out);
}

// q8.rs:3644-3673 fast_f32_to_f16: truncating conversion (no rounding).
uint16_t or_f32_to_f16_trunc(float value) {
    uint32_t bits = f32_bits(value);
    uint16_t sign = (uint16_t)((bits >> 16) & 0x8000u);
    int32_t exponent = (int32_t)((bits >> 23) & 0xffu);
    uint32_t fraction = bits & 0x007fffffu;
    if (exponent == 0) return sign;
    if (exponent == 0xff) {
        if (fraction == 0) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7c00u | (uint16_t)(fraction >> 13) | 1u);
    }
    int32_t half_exponent = exponent - 127 + 15;
    if (half_exponent >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (half_exponent <= 0) {
        if (half_exponent < -10) return sign;
        uint32_t mantissa = (fraction | 0x00800000u) >> (14 - half_exponent);
        return (uint16_t)(sign | (uint16_t)mantissa);
    }
    return (uint16_t)(sign | (uint16_t)(half_exponent << 10) | (uint16_t)(fraction >> 13));
}

// q8.rs:3376-3382 dot_i8_scalar.
int32_t or_dot_i8(const int8_t* a, const int8_t* b, int64_t n) {
    int32_t s = 0;
    for (int64_t i = 0; i < n; i++) s += (int32_t)a[i] * (int32_t)b[i];
    return s;
}

// q8.rs:539-546 unpack_values + q8.rs:2699-2702 dot_q4_0_q8_0_scalar.
// Nibble j<16 is the low nibble of byte j, nibble 16+j the high nibble.
int32_t or_dot_q4_0_q8_0(const uint8_t* block18, const int8_t* x32) {
    int8_t w[32];
    const uint8_t* v = block18 + 2;
    for (int j = 0; j < 16; j++) {
        w[j] = (int8_t)((int)(v[j] & 0x0f) - 8);
        w[j + 16] = (int8_t)((int)(v[j] >> 4) - 8);
    }
    return or_dot_i8(w, x32, 32);
}

// q8.rs:2008-2018 q4_k_scale_min.
static inline void q4k_scale_min(int idx, const uint8_t* scales, uint8_t* sc, uint8_t* mn) {
    if (idx < 4) {
        *sc = scales[idx] & 63;
        *mn = scales[idx + 4] & 63;
    } else {
        *sc = (uint8_t)((scales[idx + 4] & 0x0f) | ((scales[idx - 4] >> 6) << 4));
        *mn = (uint8_t)((scales[idx + 4] >> 4) | ((scales[idx] >> 6) << 4));
    }
}

// Q4_K super-block layout q8.rs:1195-1207: d(f16) dmin(f16) scales[12] qs[128].
void or_q4_k_subblock_ints(const uint8_t* blk, const int8_t* x, int32_t* W8, int32_t* A8) {
    const uint8_t* qs = blk + 16;
    for (int pair = 0; pair < 4; pair++) {
        int32_t lw = 0, la = 0, hw = 0, ha = 0;
        for (int l = 0; l < 32; l++) {
            uint8_t byte = qs[pair * 32 + l];
            int32_t lx = x[pair * 64 + l];
            int32_t hx = x[pair * 64 + 32 + l];
            lw += (int32_t)(byte & 0x0f) * lx;
            la += lx;
            hw += (int32_t)(byte >> 4) * hx;
            ha += hx;
        }
        W8[2 * pair] = lw;
        A8[2 * pair] = la;
        W8[2 * pair + 1] = hw;
        A8[2 * pair + 1] = ha;
    }
}

// q8.rs:1211-1231 unpack + q8.rs:1339-1376 dot_q8_scaled_preloaded (the x86 path
// of matmul_q4_k_batch, inference.rs:2083-2130).  Sum starts at 0.0 per super-block.
float or_q4_k_dot(const uint8_t* blk, const int8_t* x, const float* xs8) {
    float d = or_f16_to_f32(load_u16(blk));
    float dmin = or_f16_to_f32(load_u16(blk + 2));
    const uint8_t* scales = blk + 4;
    float sc[8], mn[8];
    for (int pair = 0; pair < 4; pair++) {
        for (int h = 0; h < 2; h++) {
            uint8_t s, m;
            q4k_scale_min(pair * 2 + h, scales, &s, &m);
            sc[pair * 2 + h] = d * (float)s;
            mn[pair * 2 + h] = dmin * (float)m;
        }
    }
    int32_t W[8], A[8];
    or_q4_k_subblock_ints(blk, x, W, A);
    float sum = 0.0f;
    for (int j = 0; j < 8; j++) {
        float a = sc[j] * (float)W[j];
        float b = mn[j] * (float)A[j];
        sum += xs8[j] * (a - b);
    }
    return sum;
}

// Q5_K super-block layout q8.rs:1380-1397: d(f16) dmin(f16) scales[12] qh[32] qs[128]; the
// 5-bit value of element 64*pair + l (low half) / 64*pair + 32 + l (high half) is the nibble
// plus 16 when bit 2*pair / 2*pair + 1 of qh[l] is set.  q8.rs:1444-1468 unpack +
// q8.rs:1551-1594 dot_q8_scaled_preloaded (the x86 path of matmul_q5_k_batch,
// inference.rs:2587-2640): per pair the low then the high sub-block term
// xs_j * (sc_j * W_j - mn_j * A_j), added to a sum that starts at 0.0 per super-block.
float or_q5_k_dot(const uint8_t* blk, const int8_t* x, const float* xs) {
    const float d = or_f16_to_f32(load_u16(blk));
    const float dmin = or_f16_to_f32(load_u16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* qh = blk + 16;
    const uint8_t* qs = blk + 48;
    float sum = 0.0f;
    for (int pair = 0; pair < 4; pair++) {
        uint8_t ls, lm, hs, hm;
        q4k_scale_min(pair * 2, scales, &ls, &lm);
        q4k_scale_min(pair * 2 + 1, scales, &hs, &hm);
        const float lsc = d * (float)ls, hsc = d * (float)hs;
        const float lmn = dmin * (float)lm, hmn = dmin * (float)hm;
        int32_t lw = 0, la = 0, hw = 0, ha = 0;
        for (int l = 0; l < 32; l++) {
            const uint8_t byte = qs[pair * 32 + l];
            const int32_t lo = (byte & 0x0f) + ((qh[l] >> (2 * pair)) & 1 ? 16 : 0);
            const int32_t hi = (byte >> 4) + ((qh[l] >> (2 * pair + 1)) & 1 ? 16 : 0);
            const int32_t lx = x[pair * 64 + l], hx = x[pair * 64 + 32 + l];
            lw += lo * lx;
            la += lx;
            hw += hi * hx;
            ha += hx;
        }
        sum += xs[pair * 2] * (lsc * (float)lw - lmn * (float)la);
        sum += xs[pair * 2 + 1] * (hsc * (float)hw - hmn * (float)ha);
    }
    return sum;
}

// q8.rs:1233-1264 Q4KBlock::dequantize.
void or_q4_k_dequantize(const uint8_t* blk, float* out) {
    float d = or_f16_to_f32(load_u16(blk));
    float dmin = or_f16_to_f32(load_u16(blk + 2));
    const uint8_t* scales = blk + 4;
    const uint8_t* qs = blk + 16;
    for (int pair = 0; pair < 4; pair++) {
        uint8_t ls, lm, hs, hm;
        q4k_scale_min(pair * 2, scales, &ls, &lm);
        q4k_scale_min(pair * 2 + 1, scales, &hs, &hm);
        float lsc = d * (float)ls, hsc = d * (float)hs;
        float lmn = dmin * (float)lm, hmn = dmin * (float)hm;
        for (int l = 0; l < 32; l++) {
            uint8_t byte = qs[pair * 32 + l];
            out[pair * 64 + l] = lsc * (float)(byte & 0x0f) - lmn;
            out[pair * 64 + 32 + l] = hsc * (float)(byte >> 4) - hmn;
        }
    }
}

// load_f32_or_f16 (model.rs:1081-1229): one tensor's n values decoded to f32, written in the
// reference's per-type loop order.  Types: 0 F32, 1 F16, 30 BF16, 8 Q8_0, 2 Q4_0, 3 Q4_1,
// 6 Q5_0, 7 Q5_1, 12 Q4_K, 13 Q5_K, 14 Q6_K.  Returns 0, or -1 for any other type.
int or_dequantize_f32(int type, const uint8_t* p, int64_t n, float* out) {
    int64_t o = 0;
    switch (type) {
        case 0:
            std::memcpy(out, p, (size_t)n * 4);
            return 0;
        case 1:
            for (int64_t i = 0; i < n; i++) out[i] = or_f16_to_f32(load_u16(p + 2 * i));
            return 0;
        case 30:
            for (int64_t i = 0; i < n; i++) out[i] = bits_f32((uint32_t)load_u16(p + 2 * i) << 16);
            return 0;
        case 8:  // q8.rs:478-511: value * scale
            for (int64_t b = 0; b < n / 32; b++, p += 34) {
                const float scale = or_f16_to_f32(load_u16(p));
                for (int k = 0; k < 32; k++) out[o++] = (float)(int8_t)p[2 + k] * scale;
            }
            return 0;
        case 2:  // q8.rs:514-547 unpack_values (low nibbles then high) - 8, * scale
            for (int64_t b = 0; b < n / 32; b++, p += 18) {
                const float scale = or_f16_to_f32(load_u16(p));
                int8_t v[32];
                for (int k = 0; k < 16; k++) {
                    v[k] = (int8_t)((p[2 + k] & 0x0f) - 8);
                    v[k + 16] = (int8_t)((p[2 + k] >> 4) - 8);
                }
                for (int k = 0; k < 32; k++) out[o++] = (float)v[k] * scale;
            }
            return 0;
        case 3:  // q8.rs:549-599: value * scale + min
            for (int64_t b = 0; b < n / 32; b++, p += 20) {
                const float scale = or_f16_to_f32(load_u16(p)), mn = or_f16_to_f32(load_u16(p + 2));
                uint8_t v[32];
                for (int k = 0; k < 16; k++) {
                    v[k] = p[4 + k] & 0x0f;
                    v[k + 16] = p[4 + k] >> 4;
                }
                for (int k = 0; k < 32; k++) out[o++] = (float)v[k] * scale + mn;
            }
            return 0;
        case 6:  // q8.rs:601-649: 5-bit values - 16, * scale
        case 7:  // q8.rs:651-720: 5-bit values * scale + min
            for (int64_t b = 0; b < n / 32; b++) {
                const bool has_min = type == 7;
                const float scale = or_f16_to_f32(load_u16(p));
                const float mn = has_min ? or_f16_to_f32(load_u16(p + 2)) : 0.0f;
                const uint8_t* hb = p + (has_min ? 4 : 2);
                const uint32_t high = (uint32_t)hb[0] | ((uint32_t)hb[1] << 8) | ((uint32_t)hb[2] << 16) | ((uint32_t)hb[3] << 24);
                const uint8_t* qs = hb + 4;
                int v[32];
                for (int k = 0; k < 16; k++) {
                    v[k] = (qs[k] & 0x0f) | (int)(((high >> k) & 1u) << 4);
                    v[k + 16] = (qs[k] >> 4) | (int)(((high >> (k + 16)) & 1u) << 4);
                }
                for (int k = 0; k < 32; k++) out[o++] = has_min ? (float)v[k] * scale + mn : (float)(v[k] - 16) * scale;
                p += has_min ? 24 : 22;
            }
            return 0;
        case 12:
            for (int64_t b = 0; b < n / 256; b++) or_q4_k_dequantize(p + b * 144, out + b * 256);
            return 0;
        case 13:  // q8.rs:1467-1498 Q5KBlock::dequantize
            for (int64_t b = 0; b < n / 256; b++, p += 176) {
                const float d = or_f16_to_f32(load_u16(p)), dmin = or_f16_to_f32(load_u16(p + 2));
                const uint8_t* scales = p + 4;
                const uint8_t* high = p + 16;
                const uint8_t* vals = p + 48;
                float* ob = out + b * 256;
                uint8_t u1 = 1, u2 = 2;
                for (int pair = 0; pair < 4; pair++) {
                    uint8_t ls, lm, hs, hm;
                    q4k_scale_min(pair * 2, scales, &ls, &lm);
                    q4k_scale_min(pair * 2 + 1, scales, &hs, &hm);
                    const float lsc = d * (float)ls, hsc = d * (float)hs;
                    const float lmn = dmin * (float)lm, hmn = dmin * (float)hm;
                    for (int l = 0; l < 32; l++) {
                        const uint8_t byte = vals[pair * 32 + l];
                        const int low = (byte & 0x0f) + ((high[l] & u1) != 0 ? 16 : 0);
                        const int hi = (byte >> 4) + ((high[l] & u2) != 0 ? 16 : 0);
                        ob[pair * 64 + l] = lsc * (float)low - lmn;
                        ob[pair * 64 + 32 + l] = hsc * (float)hi - hmn;
                    }
                    u1 = (uint8_t)(u1 << 2);
                    u2 = (uint8_t)(u2 << 2);
                }
            }
            return 0;
        case 14:  // q8.rs:2063-2090 Q6KBlock::dequantize
            for (int64_t b = 0; b < n / 256; b++, p += 210) {
                const uint8_t* ql = p;
                const uint8_t* qh = p + 128;
                const int8_t* sc = (const int8_t*)(p + 192);
                const float d = or_f16_to_f32(load_u16(p + 208));
                float* ob = out + b * 256;
                int qlo = 0, qho = 0, so = 0;
                for (int nn = 0; nn < 256; nn += 128) {
                    for (int l = 0; l < 32; l++) {
                        const int is = l / 16;
                        const uint8_t h = qh[qho + l];
                        const int q1 = (int8_t)((ql[qlo + l] & 0x0f) | ((h & 0x03) << 4)) - 32;
                        const int q2 = (int8_t)((ql[qlo + l + 32] & 0x0f) | (((h >> 2) & 0x03) << 4)) - 32;
                        const int q3 = (int8_t)((ql[qlo + l] >> 4) | (((h >> 4) & 0x03) << 4)) - 32;
                        const int q4 = (int8_t)((ql[qlo + l + 32] >> 4) | (((h >> 6) & 0x03) << 4)) - 32;
                        ob[nn + l] = d * (float)sc[so + is] * (float)q1;
                        ob[nn + l + 32] = d * (float)sc[so + is + 2] * (float)q2;
                        ob[nn + l + 64] = d * (float)sc[so + is + 4] * (float)q3;
                        ob[nn + l + 96] = d * (float)sc[so + is + 6] * (float)q4;
                    }
                    qlo += 64;
                    qho += 32;
                    so += 8;
                }
            }
            return 0;
        default:
            return -1;
    }
}

// Rust `(f32).clamp(-127.0, 127.0) as i8` after `.round()` (roundf: half away from zero).
static inline int8_t round_clamp_i8(float v) {
    float q = std::round(v);
    if (q < -127.0f) q = -127.0f;
    if (q > 127.0f) q = 127.0f;
    return (int8_t)(int)q;
}

// inference.rs:991-1029 quantize_f32_to_q8_0_scalar + max_abs_scalar +
// quantize_q8_block_with_max_abs.  Scale stored as f32 (not f16).
void or_quantize_q8_0(const float* x, int64_t n, int8_t* q, float* scales) {
    int64_t blocks = n / 32;
    for (int64_t b = 0; b < blocks; b++) {
        const float* chunk = x + b * 32;
        float max_abs = 0.0f;
        for (int i = 0; i < 32; i++) {
            float a = std::fabs(chunk[i]);
            if (a > max_abs) max_abs = a;
        }
        float scale = max_abs / 127.0f;
        scales[b] = scale;
        if (scale > 0.0f) {
            float inv = 1.0f / scale;
            for (int i = 0; i < 32; i++) q[b * 32 + i] = round_clamp_i8(chunk[i] * inv);
        } else {
            for (int i = 0; i < 32; i++) q[b * 32 + i] = 0;
        }
    }
}

// q8.rs:2442-2488 quantize_f32_matrix_to_q4_0_blocks (tied LM head, model.rs:495-499).
void or_quantize_q4_0_tied(const float* values, int64_t rows, int64_t cols, uint8_t* out) {
    int64_t bpr = cols / 32;
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t b = 0; b < bpr; b++) {
            const float* chunk = values + r * cols + b * 32;
            float amax = 0.0f, mx = 0.0f;
            for (int i = 0; i < 32; i++) {
                float a = std::fabs(chunk[i]);
                if (a > amax) {
                    amax = a;
                    mx = chunk[i];
                }
            }
            float d = mx / -8.0f;
            float id = (d != 0.0f) ? 1.0f / d : 0.0f;
            uint8_t* blk = out + (r * bpr + b) * 18;
            uint16_t sb = or_f32_to_f16_trunc(d);
            blk[0] = (uint8_t)(sb & 0xff);
            blk[1] = (uint8_t)(sb >> 8);
            for (int j = 0; j < 16; j++) {
                float x0 = chunk[j] * id + 8.5f;
                float x1 = chunk[j + 16] * id + 8.5f;
                int q0 = clamp_i32(rust_f32_as_i32(x0), 0, 15);
                int q1 = clamp_i32(rust_f32_as_i32(x1), 0, 15);
                blk[2 + j] = (uint8_t)(q0 | (q1 << 4));
            }
        }
    }
}

}  // extern "C"

// Row-parallel partition mirroring rayon's per-row split (inference.rs:1318-1330):
// rows are independent and each row's accumulation order is unchanged.
void parallel_rows(int64_t rows, int nthreads, const std::function<void(int64_t, int64_t)>& fn) {
    if (nthreads <= 1 || rows < 256) {
        fn(0, rows);
        return;
    }
    std::vector<std::thread> ts;
    int64_t chunk = (rows + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        int64_t lo = t * chunk, hi = std::min<int64_t>(rows, lo + chunk);
        if (lo >= hi) break;
        ts.emplace_back([&fn, lo, hi] { fn(lo, hi); });
    }
    for (auto& th : ts) th.join();
}

extern "C" {

// inference.rs:1385-1418 matmul_q4_0_batch and :1525-1574 (swizzled, same per-row order):
// sum += ws * xs * dot, left to right, blocks in order, one f32 chain per (row, token).
void or_matmul_q4_0(float* out, const int8_t* x, const float* xs, const uint8_t* w,
                    int64_t N, int64_t M, int64_t K, int nthreads) {
    int64_t bpr = K / 32;
    parallel_rows(M, nthreads, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const uint8_t* wrow = w + r * bpr * 18;
            for (int64_t t = 0; t < N; t++) {
                const int8_t* xt = x + t * K;
                const float* st = xs + t * bpr;
                float sum = 0.0f;
                for (int64_t b = 0; b < bpr; b++) {
                    const uint8_t* blk = wrow + b * 18;
                    int32_t dot = or_dot_q4_0_q8_0(blk, xt + b * 32);
                    float ws = or_f16_to_f32(load_u16(blk));
                    sum += ws * st[b] * (float)dot;
                }
                out[t * M + r] = sum;
            }
        }
    });
}

// inference.rs:2513-2640 matmul_q5_k_batch (x86 path): per row and token, super-blocks in order,
// each contributing or_q5_k_dot (a 0.0-started partial sum).
void or_matmul_q5_k(float* out, const int8_t* x, const float* xs, const uint8_t* w,
                    int64_t N, int64_t M, int64_t K, int nthreads) {
    int64_t spr = K / 256;
    parallel_rows(M, nthreads, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            for (int64_t t = 0; t < N; t++) {
                float sum = 0.0f;
                for (int64_t sb = 0; sb < spr; sb++)
                    sum += or_q5_k_dot(w + (r * spr + sb) * 176, x + t * K + sb * 256, xs + t * (K / 32) + sb * 8);
                out[t * M + r] = sum;
            }
        }
    });
}

// inference.rs:1343-1383 matmul_q8_0_batch: per row and token, sum += ws * xs * dot over the
// 32-blocks in order, dot = dot_i8_scalar of the block's int8 weights and activations
// (q8.rs:3376-3382), ws = fast_f16_to_f32 of the block's scale (q8.rs:500-502); block =
// f16 scale then 32 int8 (Q8_0Block::from_bytes, q8.rs:479-487).
void or_matmul_q8_0(float* out, const int8_t* x, const float* xs, const uint8_t* w,
                    int64_t N, int64_t M, int64_t K, int nthreads) {
    int64_t bpr = K / 32;
    parallel_rows(M, nthreads, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            const uint8_t* wrow = w + r * bpr * 34;
            for (int64_t t = 0; t < N; t++) {
                const int8_t* xt = x + t * K;
                const float* st = xs + t * bpr;
                float sum = 0.0f;
                for (int64_t b = 0; b < bpr; b++) {
                    const uint8_t* blk = wrow + b * 34;
                    int32_t dot = 0;
                    for (int i = 0; i < 32; i++) dot += (int32_t)(int8_t)blk[2 + i] * (int32_t)xt[b * 32 + i];
                    const float ws = or_f16_to_f32(load_u16(blk));
                    sum += ws * st[b] * (float)dot;
                }
                out[t * M + r] = sum;
            }
        }
    });
}

void or_matmul_q4_0_blockdots(int32_t* dots, const int8_t* x, const uint8_t* w,
                              int64_t N, int64_t M, int64_t K, int nthreads) {
    int64_t bpr = K / 32;
    parallel_rows(M, nthreads, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++)
            for (int64_t t = 0; t < N; t++)
                for (int64_t b = 0; b < bpr; b++)
                    dots[(t * M + r) * bpr + b] =
                        or_dot_q4_0_q8_0(w + (r * bpr + b) * 18, x + t * K + b * 32);
    });
}

// inference.rs:2083-2130 (x86 path of matmul_q4_k_batch): per row/token, super-blocks in
// order, each contributing dot_q8_scaled_preloaded (a 0.0-started partial sum).
void or_matmul_q4_k(float* out, const int8_t* x, const float* xs, const uint8_t* w,
                    int64_t N, int64_t M, int64_t K, int nthreads) {
    int64_t spr = K / 256;
    parallel_rows(M, nthreads, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++) {
            for (int64_t t = 0; t < N; t++) {
                float sum = 0.0f;
                for (int64_t sb = 0; sb < spr; sb++) {
                    const uint8_t* blk = w + (r * spr + sb) * 144;
                    sum += or_q4_k_dot(blk, x + t * K + sb * 256, xs + t * (K / 32) + sb * 8);
                }
                out[t * M + r] = sum;
            }
        }
    });
}

// q8.rs:2093-2150 Q6KBlock::dot_q8_scaled: weight_scales[i] = d * scales[i]; per 128-value
// half n, c*_low / c*_high = weight_scale * x_scale of the 32-value group; then for l in 0..16
// (low scales) and l in 16..32 (high scales) the four terms of q1..q4 at x[n+l], x[n+l+32],
// x[n+l+64], x[n+l+96], each (c * q) * x, added to one f32 sum that starts at 0.
float or_q6_k_dot(const uint8_t* blk, const int8_t* x, const float* xs8) {
    const uint8_t* ql = blk;
    const uint8_t* qh = blk + 128;
    const int8_t* scales = (const int8_t*)(blk + 192);
    const float d = or_f16_to_f32(load_u16(blk + 208));
    float weight_scales[16];
    for (int i = 0; i < 16; i++) weight_scales[i] = d * (float)scales[i];
    float sum = 0.0f;
    int ql_off = 0, qh_off = 0, sc_off = 0;
    for (int n = 0; n < 256; n += 128) {
        const int xo = n / 32;
        const float c_low[4] = {weight_scales[sc_off] * xs8[xo], weight_scales[sc_off + 2] * xs8[xo + 1],
                                weight_scales[sc_off + 4] * xs8[xo + 2], weight_scales[sc_off + 6] * xs8[xo + 3]};
        const float c_high[4] = {weight_scales[sc_off + 1] * xs8[xo], weight_scales[sc_off + 3] * xs8[xo + 1],
                                 weight_scales[sc_off + 5] * xs8[xo + 2], weight_scales[sc_off + 7] * xs8[xo + 3]};
        for (int l = 0; l < 32; l++) {
            const float* c = l < 16 ? c_low : c_high;
            const uint8_t h = qh[qh_off + l];
            const int q1 = (int8_t)((ql[ql_off + l] & 0x0f) | ((h & 0x03) << 4)) - 32;
            const int q2 = (int8_t)((ql[ql_off + l + 32] & 0x0f) | (((h >> 2) & 0x03) << 4)) - 32;
            const int q3 = (int8_t)((ql[ql_off + l] >> 4) | (((h >> 4) & 0x03) << 4)) - 32;
            const int q4 = (int8_t)((ql[ql_off + l + 32] >> 4) | (((h >> 6) & 0x03) << 4)) - 32;
            sum += c[0] * (float)q1 * (float)x[n + l];
            sum += c[1] * (float)q2 * (float)x[n + l + 32];
            sum += c[2] * (float)q3 * (float)x[n + l + 64];
            sum += c[3] * (float)q4 * (float)x[n + l + 96];
        }
        ql_off += 64;
        qh_off += 32;
        sc_off += 8;
    }
    return sum;
}

// inference.rs:1882-2000 matmul_q6_k_batch (portable path): per row and token, the super-block
// dots added in order to a sum that starts at 0.
void or_matmul_q6_k(float* out, const int8_t* x, const float* xs, const uint8_t* w, int64_t N, int64_t M, int64_t K,
                    int nthreads) {
    const int64_t spr = K / 256;
    parallel_rows(M, nthreads, [&](int64_t lo, int64_t hi) {
        for (int64_t r = lo; r < hi; r++)
            for (int64_t t = 0; t < N; t++) {
                float sum = 0.0f;
                for (int64_t sb = 0; sb < spr; sb++)
                    sum += or_q6_k_dot(w + (r * spr + sb) * 210, x + t * K + sb * 256, xs + t * (K / 32) + sb * 8);
                out[t * M + r] = sum;
            }
    });
}

// inference.rs:697-706 rms_norm: sequential f32 sum of squares; out = x*scale*w.
void or_rms_norm(float* out, const float* x, const float* w, int64_t n, float eps) {
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) sum += x[i] * x[i];
    float scale = 1.0f / std::sqrt(sum / (float)n + eps);
    for (int64_t i = 0; i < n; i++) out[i] = x[i] * scale * w[i];
}

// inference.rs:880-901 cached_rope_angles (no rope scaling keys in these models):
// theta = base.powf(-(2i) / rope_dim); (sin, cos) = (pos * theta).sin_cos().
// inference.rs:874-893 (cached_rope_angles) / :763-786 (apply_rope): theta of pair i, with the
// Llama-3 frequency scaling when scaling = {factor, original_context_length, low_freq_factor,
// high_freq_factor} is given (all four present, as the reference requires).
float or_rope_theta(int64_t i, int64_t rope_dim, float freq_base, const float* scaling) {
    static float (*volatile p_powf)(float, float) = powf;
    float theta = p_powf(freq_base, -((float)(i * 2)) / (float)rope_dim);
    if (scaling) {
        const float factor = scaling[0], orig_len = scaling[1], low = scaling[2], high = scaling[3];
        const float wavelength = (2.0f * (float)M_PI) / theta;
        const float low_freq_wavelength = orig_len / low;
        const float high_freq_wavelength = orig_len / high;
        if (wavelength >= high_freq_wavelength) {
            if (wavelength > low_freq_wavelength) {
                theta /= factor;
            } else {
                const float smooth = (orig_len / wavelength - low) / (high - low);
                theta = ((1.0f - smooth) * theta / factor) + (smooth * theta);
            }
        }
    }
    return theta;
}

void or_rope_sincos_scaled(int64_t pos, int64_t i, int64_t rope_dim, float freq_base, const float* scaling, float* s,
                           float* c) {
    // Separate sinf and cosf calls as Rust's f32::sin_cos makes; the volatile pointers keep
    // the compiler from merging them into one sincosf call.
    static float (*volatile p_sinf)(float) = sinf;
    static float (*volatile p_cosf)(float) = cosf;
    float theta = or_rope_theta(i, rope_dim, freq_base, scaling);
    float angle = (float)pos * theta;
    *s = p_sinf(angle);
    *c = p_cosf(angle);
}

void or_rope_sincos(int64_t pos, int64_t i, int64_t rope_dim, float freq_base, float* s, float* c) {
    or_rope_sincos_scaled(pos, i, rope_dim, freq_base, nullptr, s, c);
}

// inference.rs:914-933 apply_rope_cached.
void or_rope_scaled(float* data, int64_t pos, int64_t heads, int64_t head_dim, int64_t rope_dim,
                    float freq_base, int style, const float* scaling) {
    int64_t half = rope_dim / 2;
    std::vector<float> sn(half), cs(half);
    for (int64_t i = 0; i < half; i++) or_rope_sincos_scaled(pos, i, rope_dim, freq_base, scaling, &sn[i], &cs[i]);
    for (int64_t h = 0; h < heads; h++) {
        int64_t hs = h * head_dim;
        for (int64_t i = 0; i < half; i++) {
            int64_t d0 = style == 0 ? hs + 2 * i : hs + i;
            int64_t d1 = style == 0 ? hs + 2 * i + 1 : hs + i + half;
            float x0 = data[d0], x1 = data[d1];
            data[d0] = x0 * cs[i] - x1 * sn[i];
            data[d1] = x0 * sn[i] + x1 * cs[i];
        }
    }
}

void or_rope(float* data, int64_t pos, int64_t heads, int64_t head_dim, int64_t rope_dim,
             float freq_base, int style) {
    or_rope_scaled(data, pos, heads, head_dim, rope_dim, freq_base, style, nullptr);
}

float or_expf(float x) { return expf(x); }

// inference.rs:4876-4883 rand_simple: state = state * 6364136223846793005 + 1 (wrapping),
// ((state >> 32) as u32) as f32 / (u32::MAX as f32).
float or_rand_simple(uint64_t* state) {
    *state = *state * 6364136223846793005ull + 1ull;
    const float x = (float)(uint32_t)(*state >> 32);
    return x / (float)UINT32_MAX;
}

// inference.rs:4834-4873 sample_logits: temp <= 0 the first maximum; else max, e_i =
// ((l_i - max) / temp).exp() summed left to right, r = rand_simple() * sum, then r -= e_i
// until r <= 0 (the last index if never).
int64_t or_sample_logits(const float* logits, int64_t V, float temp, uint64_t* state) {
    if (temp <= 0.0f) return or_argmax(logits, V);
    float mx = logits[0];
    for (int64_t i = 0; i < V; i++)
        if (logits[i] > mx) mx = logits[i];
    std::vector<float> e(V);
    float sum = 0.0f;
    for (int64_t i = 0; i < V; i++) {
        e[i] = expf((logits[i] - mx) / temp);
        sum += e[i];
    }
    float r = or_rand_simple(state) * sum;
    for (int64_t i = 0; i < V; i++) {
        r -= e[i];
        if (r <= 0.0f) return i;
    }
    return V - 1;
}

// Checker for the device restatement of expf: vals[i] against glibc expf of the float with
// bits first + i, bit for bit (NaN inputs: any NaN).  Returns the mismatch count and the first
// mismatching input's bits in *first_bad.
int64_t or_expf_mismatches(uint32_t first, int64_t count, const float* vals, int nthreads, uint32_t* first_bad) {
    std::vector<int64_t> bad(std::max(1, nthreads), 0);
    std::vector<int64_t> firsts(bad.size(), -1);
    parallel_rows(count, nthreads, [&](int64_t lo, int64_t hi) {
        const size_t slot = (size_t)(lo * (int64_t)bad.size() / std::max<int64_t>(count, 1));
        for (int64_t i = lo; i < hi; i++) {
            const uint32_t ub = first + (uint32_t)i;
            float x;
            std::memcpy(&x, &ub, 4);
            const float want = expf(x);
            uint32_t wb, gb;
            std::memcpy(&wb, &want, 4);
            std::memcpy(&gb, &vals[i], 4);
            const bool ok = std::isnan(x) ? std::isnan(vals[i]) : wb == gb;
            if (!ok) {
                if (firsts[slot] < 0) firsts[slot] = i;
                bad[slot]++;
            }
        }
    });
    int64_t total = 0, fb = -1;
    for (size_t k = 0; k < bad.size(); k++) {
        total += bad[k];
        if (firsts[k] >= 0 && (fb < 0 || firsts[k] < fb)) fb = firsts[k];
    }
    if (first_bad) *first_bad = fb < 0 ? 0 : first + (uint32_t)fb;
    return total;
}

// inference.rs:3522-3540 softmax.
void or_softmax(float* x, int64_t n) {
    float mx = -INFINITY;
    for (int64_t i = 0; i < n; i++)
        if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (int64_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    float inv = 1.0f / sum;
    for (int64_t i = 0; i < n; i++) x[i] *= inv;
}

// inference.rs:3367-3390 fused_silu_mul: g * (1/(1+exp(-g))) * u.
void or_silu_mul(float* out, const float* gate, const float* up, int64_t n) {
    for (int64_t i = 0; i < n; i++) {
        float g = gate[i];
        float sig = 1.0f / (1.0f + expf(-g));
        out[i] = g * sig * up[i];
    }
}

// inference.rs:4836-4846 greedy branch of sample_logits: strict '>' keeps the first max.
int64_t or_argmax(const float* logits, int64_t n) {
    float mv = logits[0];
    int64_t mi = 0;
    for (int64_t i = 0; i < n; i++)
        if (logits[i] > mv) {
            mv = logits[i];
            mi = i;
        }
    return mi;
}

// inference.rs:4242-4292 apply_attention_head, F32 KV, x86 branch:
// score_p = dot(q, k_p) * scale (dot_f32_scalar: sequential sum), softmax over 0..=pos,
// out += score_p * v_p for p in order (add_weighted_f32_scalar).  out_head must be zeroed
// by the caller (inference.rs:3929 fills attn_output with 0.0).
void or_attention_head(float* out_head, float* scores, const float* q_head,
                       const float* k_cache, const float* v_cache, int64_t pos,
                       int64_t kv_width, int64_t kv_h, int64_t head_dim, float scale) {
    for (int64_t p = 0; p <= pos; p++) {
        const float* k = k_cache + p * kv_width + kv_h * head_dim;
        float dot = -0.0f;  // Rust f32 Sum folds from -0.0
        for (int64_t i = 0; i < head_dim; i++) dot += q_head[i] * k[i];
        scores[p] = dot * scale;
    }
    or_softmax(scores, pos + 1);
    for (int64_t p = 0; p <= pos; p++) {
        const float* v = v_cache + p * kv_width + kv_h * head_dim;
        float s = scores[p];
        for (int64_t i = 0; i < head_dim; i++) out_head[i] += s * v[i];
    }
}

// Split-order attention head: the device's NC_ATTN_SPLIT order (no reference counterpart; the
// reference's order is or_attention_head above, which this equals up to f32 rounding).
// Positions 0..pos in chunks of 64; per chunk c, lanes j = p - 64c:
//   s_p = fmaf-chain dot(q, k_p) in dim order from 0, times scale;  m_c = max of the live s_p;
//   e_p = expf(s_p - m_c) (0 past pos);  l_c = the xor-butterfly sum of the 64 lanes' e
//   (offsets 32, 16, ..., 1);  o_c[i] = fmaf chain over the chunk's 64 positions in order of
//   e_p * v_p[i], v taken as 0 past plast (the pass's last position);
// then, in chunk order: M = max m_c, w_c = expf(m_c - M), l = fmaf(w_c, l_c, l),
// o[i] = fmaf(w_c, o_c[i], o[i]), out[i] = o[i] / l.  out_head is overwritten.
void or_attention_head_split(float* out_head, const float* q_head, const float* k_cache, const float* v_cache,
                             int64_t pos, int64_t plast, int64_t kv_width, int64_t kv_h, int64_t head_dim,
                             float scale) {
    const int64_t C = 64, nch = pos / C + 1;
    std::vector<float> mc(nch), lc(nch), oc((size_t)nch * head_dim);
    for (int64_t c = 0; c < nch; c++) {
        float sv[64], e[64];
        float m = -INFINITY;
        for (int64_t j = 0; j < C; j++) {
            const int64_t p = c * C + j;
            sv[j] = -INFINITY;
            if (p > pos) continue;
            const float* k = k_cache + p * kv_width + kv_h * head_dim;
            float dot = 0.0f;
            for (int64_t i = 0; i < head_dim; i++) dot = fmaf(q_head[i], k[i], dot);
            sv[j] = dot * scale;
            m = sv[j] > m ? sv[j] : m;
        }
        for (int64_t j = 0; j < C; j++) e[j] = c * C + j <= pos ? expf(sv[j] - m) : 0.0f;
        float b[64], nb[64];
        std::memcpy(b, e, sizeof b);
        for (int off = 32; off >= 1; off >>= 1) {
            for (int i = 0; i < 64; i++) nb[i] = b[i] + b[i ^ off];
            std::memcpy(b, nb, sizeof b);
        }
        mc[c] = m;
        lc[c] = b[0];
        for (int64_t i = 0; i < head_dim; i++) {
            float o = 0.0f;
            for (int64_t j = 0; j < C; j++) {
                const int64_t p = c * C + j;
                const float v = p <= plast ? v_cache[p * kv_width + kv_h * head_dim + i] : 0.0f;
                o = fmaf(e[j], v, o);
            }
            oc[(size_t)c * head_dim + i] = o;
        }
    }
    float M = mc[0];
    for (int64_t c = 1; c < nch; c++) M = mc[c] > M ? mc[c] : M;
    std::vector<float> w(nch);
    float l = 0.0f;
    for (int64_t c = 0; c < nch; c++) {
        w[c] = expf(mc[c] - M);
        l = fmaf(w[c], lc[c], l);
    }
    for (int64_t i = 0; i < head_dim; i++) {
        float o = 0.0f;
        for (int64_t c = 0; c < nch; c++) o = fmaf(w[c], oc[(size_t)c * head_dim + i], o);
        out_head[i] = o / l;
    }
}

// Philox4x32-10, Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
// 1, 2, 3", SC'11: round multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key increments
// 0x9E3779B9 / 0xBB67AE85, ten rounds.
void or_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; round++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t n0 = hi1 ^ c1 ^ k0;
        uint32_t n1 = lo1;
        uint32_t n2 = hi0 ^ c3 ^ k1;
        uint32_t n3 = lo0;
        c0 = n0;
        c1 = n1;
        c2 = n2;
        c3 = n3;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0;
    out[1] = c1;
    out[2] = c2;
    out[3] = c3;
}

}  // extern "C"
