// fill.cpp — host-side input generation and f16 conversion (no GPU).
//
// nc_fill_flash_input restates fillFlashInput (src/main.zig:1207-1211), the fill of the
// reference's smoke and compare cases. The seeded generators produce the synthetic inputs of the
// MI355X benchmark configurations: SplitMix64 (Steele, Lea, Flood, "Fast splittable pseudorandom
// number generators", OOPSLA 2014) used as a counter-based generator, so element i of tensor t
// under seed s is a pure function of (s, t, i); uniforms take the top 24 bits, normals use the
// Box-Muller transform on element pairs (2j, 2j+1).

#include <cmath>
#include <cstring>

#include "notcute_flash.h"

namespace {

constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint32_t tensor_id) {
    return mix64(seed + kGamma * (uint64_t(tensor_id) + 1));
}

inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }

inline double unit24(uint64_t r) { return double(r >> 40) * (1.0 / 16777216.0); }  // [0, 1)

}  // namespace

extern "C" {

uint16_t nc_f32_to_f16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {  // inf / nan (nan stays quiet, keeps the top payload bits)
        if (ax == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    const uint32_t e = ax >> 23;
    if (e >= 113) {  // f16 normal range or overflow
        uint32_t h = ((e - 112) << 10) | ((ax >> 13) & 0x3ffu);
        const uint32_t low = ax & 0x1fffu;
        if (low > 0x1000u || (low == 0x1000u && (h & 1u))) ++h;  // round to nearest even
        if (h >= 0x7c00u) h = 0x7c00u;                              // overflow -> inf
        return (uint16_t)(sign | h);
    }
    // f16 subnormal or zero: value / 2^-24 = full_mantissa * 2^(e - 126)
    const uint32_t shift = 126 - e;
    if (shift > 24) return (uint16_t)sign;
    const uint32_t full = (ax & 0x7fffffu) | 0x800000u;
    uint32_t h = full >> shift;
    const uint32_t rem = full & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

float nc_f16_to_f32(uint16_t h) {
    const uint32_t sign = uint32_t(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0x1f) {
        x = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        x = sign | ((e + 112) << 23) | (m << 13);
    } else if (m == 0) {
        x = sign;
    } else {  // subnormal: normalise
        uint32_t ex = 113;
        while ((m & 0x400u) == 0) {
            m <<= 1;
            --ex;
        }
        x = sign | (ex << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

void nc_fill_flash_input(uint16_t *data, size_t n, uint64_t mul, uint64_t add, float scale) {
    for (size_t i = 0; i < n; ++i) data[i] = nc_f32_to_f16((float)((i * mul + add) % 17) * scale);
}

uint16_t nc_f32_to_bf16(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);  // nan: keep it quiet
    x += 0x7fffu + ((x >> 16) & 1u);  // round to nearest even (carries into the exponent, up to inf)
    return (uint16_t)(x >> 16);
}

float nc_bf16_to_f32(uint16_t h) {
    const uint32_t x = uint32_t(h) << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

}  // extern "C"

namespace {

template <uint16_t (*ROUND)(float)>
void fill_uniform(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float lo, float hi) {
    const uint64_t key = stream_key(seed, tensor_id);
    const double span = double(hi) - double(lo);
    for (size_t i = 0; i < n; ++i) out[i] = ROUND((float)(double(lo) + span * unit24(draw(key, i))));
}

template <uint16_t (*ROUND)(float)>
void fill_normal(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float mean, float sigma) {
    const uint64_t key = stream_key(seed, tensor_id);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t j = 0; 2 * j < n; ++j) {
        const double u1 = double((draw(key, 2 * j) >> 40) + 1) * (1.0 / 16777216.0);  // (0, 1]
        const double u2 = unit24(draw(key, 2 * j + 1));
        const double rad = std::sqrt(-2.0 * std::log(u1));
        const double th = two_pi * u2;
        out[2 * j] = ROUND((float)(double(mean) + double(sigma) * rad * std::cos(th)));
        if (2 * j + 1 < n) out[2 * j + 1] = ROUND((float)(double(mean) + double(sigma) * rad * std::sin(th)));
    }
}

}  // namespace

extern "C" {

void nc_fill_uniform_f16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float lo, float hi) {
    fill_uniform<nc_f32_to_f16>(out, n, seed, tensor_id, lo, hi);
}

void nc_fill_normal_f16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float mean, float sigma) {
    fill_normal<nc_f32_to_f16>(out, n, seed, tensor_id, mean, sigma);
}

void nc_fill_uniform_bf16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float lo, float hi) {
    fill_uniform<nc_f32_to_bf16>(out, n, seed, tensor_id, lo, hi);
}

void nc_fill_normal_bf16(uint16_t *out, size_t n, uint64_t seed, uint32_t tensor_id, float mean, float sigma) {
    fill_normal<nc_f32_to_bf16>(out, n, seed, tensor_id, mean, sigma);
}

}  // extern "C"
