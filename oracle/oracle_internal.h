// Oracle internals (TEST INFRASTRUCTURE ONLY): small bit helpers shared by the
// oracle translation units.
#ifndef NC_ORACLE_INTERNAL_H
#define NC_ORACLE_INTERNAL_H

#include <cmath>
#include <cstdint>
#include <cstring>
#include <functional>

#include "nc_oracle.h"

static inline float bits_f32(uint32_t u) {
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static inline uint32_t f32_bits(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    return u;
}
static inline uint16_t load_u16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline int32_t clamp_i32(int32_t v, int32_t lo, int32_t hi) {
    return v < lo ? lo : (v > hi ? hi : v);
}
// Rust `f32 as i32`: truncation toward zero, saturating, NaN -> 0.
static inline int32_t rust_f32_as_i32(float v) {
    if (std::isnan(v)) return 0;
    if (v >= 2147483648.0f) return INT32_MAX;
    if (v <= -2147483648.0f) return INT32_MIN;
    return (int32_t)v;
}

void parallel_rows(int64_t rows, int nthreads, const std::function<void(int64_t, int64_t)>& fn);

#endif
