// Host decoding of GGUF tensors to f32 at load time (token embeddings, norm vectors): the
// reference's load_f32_or_f16 (model.rs:1081-1229) for F32, F16, BF16, Q8_0, Q4_0, Q4_1, Q5_0,
// Q5_1, Q4_K, Q5_K and Q6_K, each value computed with the reference's expression and operand
// order so that the f32 bits match:
//   Q8_0, Q4_0, Q5_0: q * d                        (q8.rs:478-648, model.rs:1109-1155)
//   Q4_1, Q5_1:       q * d + m                    (q8.rs:549-720)
//   Q4_K, Q5_K:       (d * sc) * q - (dmin * mn)   (q8.rs:1271-1300, :1467-1498)
//   Q6_K:             d * sc * q                   (q8.rs:2063-2090)
// f16 fields decode as fast_f16_to_f32 (q8.rs:3626-3641), which keeps NaN payloads as they are.
#include <algorithm>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "gguf.h"

namespace nc {

namespace {

inline float bits_f32(uint32_t b) {
    float f;
    std::memcpy(&f, &b, 4);
    return f;
}

// fast_f16_to_f32 / f16_bits_to_f32 (q8.rs:3626-3641, model.rs:1541-1565)
inline float f16_decode(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1f, f = h & 0x3ffu;
    if (e == 0) {
        if (f == 0) return bits_f32(sign);
        uint32_t mant = f;
        int exp = -14;
        while ((mant & 0x400u) == 0) {
            mant <<= 1;
            exp -= 1;
        }
        mant &= 0x3ffu;
        return bits_f32(sign | ((uint32_t)(exp + 127) << 23) | (mant << 13));
    }
    if (e == 0x1f) return bits_f32(sign | 0x7f800000u | (f << 13));
    return bits_f32(sign | ((e + 112) << 23) | (f << 13));
}

inline uint16_t u16le(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

// q4_k_scale_min (q8.rs:2009-2018)
inline void k_scale_min(int j, const uint8_t* sc, uint8_t* s, uint8_t* m) {
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (uint8_t)((sc[j + 4] & 0x0f) | ((sc[j - 4] >> 6) << 4));
        *m = (uint8_t)((sc[j + 4] >> 4) | ((sc[j] >> 6) << 4));
    }
}

void block_q8_0(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b));
    for (int i = 0; i < 32; i++) o[i] = (float)(int8_t)b[2 + i] * d;
}

void block_q4_0(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b));
    for (int i = 0; i < 16; i++) {
        o[i] = (float)((int)(b[2 + i] & 0x0f) - 8) * d;
        o[i + 16] = (float)((int)(b[2 + i] >> 4) - 8) * d;
    }
}

void block_q4_1(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b)), m = f16_decode(u16le(b + 2));
    for (int i = 0; i < 16; i++) {
        o[i] = (float)(b[4 + i] & 0x0f) * d + m;
        o[i + 16] = (float)(b[4 + i] >> 4) * d + m;
    }
}

void block_q5_0(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b));
    const uint32_t hb = (uint32_t)b[2] | ((uint32_t)b[3] << 8) | ((uint32_t)b[4] << 16) | ((uint32_t)b[5] << 24);
    for (int i = 0; i < 16; i++) {
        const int lo = (b[6 + i] & 0x0f) | (((hb >> i) & 1) << 4);
        const int hi = (b[6 + i] >> 4) | (((hb >> (i + 16)) & 1) << 4);
        o[i] = (float)(lo - 16) * d;
        o[i + 16] = (float)(hi - 16) * d;
    }
}

void block_q5_1(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b)), m = f16_decode(u16le(b + 2));
    const uint32_t hb = (uint32_t)b[4] | ((uint32_t)b[5] << 8) | ((uint32_t)b[6] << 16) | ((uint32_t)b[7] << 24);
    for (int i = 0; i < 16; i++) {
        const int lo = (b[8 + i] & 0x0f) | (((hb >> i) & 1) << 4);
        const int hi = (b[8 + i] >> 4) | (((hb >> (i + 16)) & 1) << 4);
        o[i] = (float)lo * d + m;
        o[i + 16] = (float)hi * d + m;
    }
}

void block_q4_k(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b)), dmin = f16_decode(u16le(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qs = b + 16;
    for (int pr = 0; pr < 4; pr++) {
        uint8_t ls, lm, hs, hm;
        k_scale_min(2 * pr, sc, &ls, &lm);
        k_scale_min(2 * pr + 1, sc, &hs, &hm);
        const float lsc = d * (float)ls, hsc = d * (float)hs;
        const float lmn = dmin * (float)lm, hmn = dmin * (float)hm;
        for (int l = 0; l < 32; l++) {
            const uint8_t byte = qs[pr * 32 + l];
            o[pr * 64 + l] = lsc * (float)(byte & 0x0f) - lmn;
            o[pr * 64 + 32 + l] = hsc * (float)(byte >> 4) - hmn;
        }
    }
}

void block_q5_k(const uint8_t* b, float* o) {
    const float d = f16_decode(u16le(b)), dmin = f16_decode(u16le(b + 2));
    const uint8_t* sc = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    uint8_t u1 = 1, u2 = 2;
    for (int pr = 0; pr < 4; pr++) {
        uint8_t ls, lm, hs, hm;
        k_scale_min(2 * pr, sc, &ls, &lm);
        k_scale_min(2 * pr + 1, sc, &hs, &hm);
        const float lsc = d * (float)ls, hsc = d * (float)hs;
        const float lmn = dmin * (float)lm, hmn = dmin * (float)hm;
        for (int l = 0; l < 32; l++) {
            const uint8_t byte = qs[pr * 32 + l];
            const int lo = (byte & 0x0f) + ((qh[l] & u1) ? 16 : 0);
            const int hi = (byte >> 4) + ((qh[l] & u2) ? 16 : 0);
            o[pr * 64 + l] = lsc * (float)lo - lmn;
            o[pr * 64 + 32 + l] = hsc * (float)hi - hmn;
        }
        u1 = (uint8_t)(u1 << 2);
        u2 = (uint8_t)(u2 << 2);
    }
}

void block_q6_k(const uint8_t* b, float* o) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = f16_decode(u16le(b + 208));
    for (int half = 0; half < 2; half++) {
        const uint8_t* l_ = ql + 64 * half;
        const uint8_t* h_ = qh + 32 * half;
        const int8_t* s_ = sc + 8 * half;
        float* out = o + 128 * half;
        for (int l = 0; l < 32; l++) {
            const int is = l / 16;
            const int q1 = (int)((l_[l] & 0x0f) | ((h_[l] & 3) << 4)) - 32;
            const int q2 = (int)((l_[l + 32] & 0x0f) | (((h_[l] >> 2) & 3) << 4)) - 32;
            const int q3 = (int)((l_[l] >> 4) | (((h_[l] >> 4) & 3) << 4)) - 32;
            const int q4 = (int)((l_[l + 32] >> 4) | (((h_[l] >> 6) & 3) << 4)) - 32;
            out[l] = d * (float)s_[is] * (float)q1;
            out[l + 32] = d * (float)s_[is + 2] * (float)q2;
            out[l + 64] = d * (float)s_[is + 4] * (float)q3;
            out[l + 96] = d * (float)s_[is + 6] * (float)q4;
        }
    }
}

}  // namespace

bool dequant_supported(uint32_t type) {
    switch (type) {
        case 0: case 1: case 2: case 3: case 6: case 7: case 8: case 12: case 13: case 14: case 30: return true;
        default: return false;
    }
}

int dequant_f32(uint32_t type, const uint8_t* src, uint64_t n, float* out, int nthreads) {
    uint64_t bs, ts;
    if (!dequant_supported(type) || !gguf_type_layout(type, &bs, &ts))
        return fail(NC_EFORMAT, "unsupported type " + std::to_string(type) + " for an f32 load");
    if (n % bs) return fail(NC_EFORMAT, "value count is not a whole number of blocks");
    void (*fn)(const uint8_t*, float*) = nullptr;
    switch (type) {
        case 0:
            std::memcpy(out, src, n * 4);
            return NC_OK;
        case 1:
            for (uint64_t i = 0; i < n; i++) out[i] = f16_decode(u16le(src + 2 * i));
            return NC_OK;
        case 30:  // BF16: the high half of an f32
            for (uint64_t i = 0; i < n; i++) out[i] = bits_f32((uint32_t)u16le(src + 2 * i) << 16);
            return NC_OK;
        case 2: fn = block_q4_0; break;
        case 3: fn = block_q4_1; break;
        case 6: fn = block_q5_0; break;
        case 7: fn = block_q5_1; break;
        case 8: fn = block_q8_0; break;
        case 12: fn = block_q4_k; break;
        case 13: fn = block_q5_k; break;
        case 14: fn = block_q6_k; break;
    }
    const int64_t nblk = (int64_t)(n / bs);
    if (nthreads <= 0) nthreads = (int)std::max(1u, std::thread::hardware_concurrency());
    if (nblk < 4096) nthreads = 1;
    std::vector<std::thread> th;
    const int64_t chunk = (nblk + nthreads - 1) / nthreads;
    for (int t = 0; t < nthreads; t++) {
        const int64_t lo = t * chunk, hi = std::min(nblk, lo + chunk);
        if (lo >= hi) break;
        th.emplace_back([=] {
            for (int64_t i = lo; i < hi; i++) fn(src + i * ts, out + i * bs);
        });
    }
    for (auto& t : th) t.join();
    return NC_OK;
}

}  // namespace nc

// ================================================================ C ABI
extern "C" int nc_dequantize_f32(int32_t type, const void* blocks, int64_t n_values, float* out) {
    if (!blocks || !out || n_values < 0) return nc::fail(NC_EINVAL, "nc_dequantize_f32: bad arguments");
    return nc::dequant_f32((uint32_t)type, (const uint8_t*)blocks, (uint64_t)n_values, out, 0);
}
