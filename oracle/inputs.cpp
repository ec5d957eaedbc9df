// inputs.cpp -- fp16 conversion and the reference's seeded input generators.
// TEST INFRASTRUCTURE ONLY (see oracle.h): never linked into the product.
#include <cstring>
#include <random>

#include "oracle.h"

namespace {

// IEEE binary32 -> binary16, round to nearest even, overflow to inf, NaN kept quiet.
// This is the rounding __float2half performs (src/attn_sm75.cu:399) and numpy's float16.
uint16_t f2h_one(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    const uint32_t e = ax >> 23;
    const uint32_t frac = ax & 0x7fffffu;
    if (e >= 143) return (uint16_t)(sign | 0x7c00u);  // |f| >= 65536 (and inf)
    if (e >= 113) {                                   // normal half
        uint32_t h = ((e - 112u) << 10) | (frac >> 13);
        const uint32_t rem = frac & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // carry may give inf
        return (uint16_t)(sign | h);
    }
    // subnormal half: value / 2^-24 = mant24 * 2^(e - 126)
    const uint32_t shift = 126u - e;
    if (shift >= 32) return (uint16_t)sign;
    const uint32_t mant24 = frac | 0x800000u;
    uint32_t r = mant24 >> shift;
    const uint32_t rem = mant24 & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    if (rem > halfway || (rem == halfway && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
}

float h2f_one(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {  // subnormal: normalise
            int ee = -1;
            do {
                ++ee;
                m <<= 1;
            } while (!(m & 0x400u));
            x = sign | ((uint32_t)(112 - ee) << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &x, 4);
    return f;
}

}  // namespace

extern "C" void orc_f2h(const float* src, uint16_t* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = f2h_one(src[i]);
}

extern "C" void orc_h2f(const uint16_t* src, float* dst, size_t n) {
    for (size_t i = 0; i < n; ++i) dst[i] = h2f_one(src[i]);
}

// src/attn_sm75.cu:393-406 (make_tensor) driven as in :473-476: one mt19937 shared by
// the Q, K, V tensors in that order; normal_distribution<float>(0, 0.5) per element.
extern "C" void orc_mt_normal_half(uint32_t seed, float mean, float stddev, size_t n,
                                   int ntensors, uint16_t* out) {
    std::mt19937 rng(seed);
    for (int t = 0; t < ntensors; ++t) {
        std::normal_distribution<float> dist(mean, stddev);  // fresh per tensor, as make_tensor
        uint16_t* dst = out + (size_t)t * n;
        for (size_t i = 0; i < n; ++i) dst[i] = f2h_one(dist(rng));
    }
}

// src/gdn_sm75.cu:1270-1279.
extern "C" void orc_gdn_lcg_inputs(int T, int Hq, int Hv, int d, float* q, float* k, float* v,
                                   float* g_log, float* beta) {
    uint32_t seed = 1;
    auto rnd = [&]() {
        seed = seed * 1664525u + 1013904223u;
        return ((float)(seed >> 8) / 16777216.f) - 0.5f;
    };
    const size_t nqk = (size_t)T * Hq * d, nv = (size_t)T * Hv * d, ng = (size_t)T * Hv;
    for (size_t i = 0; i < nqk; ++i) q[i] = rnd() * 0.2f;
    for (size_t i = 0; i < nqk; ++i) k[i] = rnd() * 0.2f;
    for (size_t i = 0; i < nv; ++i) v[i] = rnd() * 0.2f;
    for (size_t i = 0; i < ng; ++i) g_log[i] = -0.2f + rnd() * 0.05f;
    for (size_t i = 0; i < ng; ++i) beta[i] = 0.4f + (rnd() + 0.5f) * 0.4f;
}
