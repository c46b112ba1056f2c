// Q8_0 scalar helpers shared by host and device code.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace tvara_amd {

// half_to_float (quant.hpp:14-29): exact for normals, subnormals, inf and NaN,
// which is what the hardware f16 -> f32 conversion gives.
__host__ __device__ inline float half_bits_to_float(uint16_t h) {
#if defined(__HIP_DEVICE_COMPILE__)
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
#else
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000) << 16;
    uint32_t exponent = (h >> 10) & 31, mantissa = h & 1023, bits;
    if (exponent == 0) {
        if (!mantissa) {
            bits = sign;
        } else {
            int e = -14;
            while ((mantissa & 1024) == 0) {
                mantissa <<= 1;
                --e;
            }
            bits = sign | (static_cast<uint32_t>(e + 127) << 23) | ((mantissa & 1023) << 13);
        }
    } else if (exponent == 31) {
        bits = sign | 0x7f800000u | (mantissa << 13);
    } else {
        bits = sign | ((exponent + 112) << 23) | (mantissa << 13);
    }
    return __builtin_bit_cast(float, bits);
#endif
}

// float64 -> float16 bits, round to nearest even, directly from the f64 bits
// (a detour through f32 would round twice).
__host__ __device__ inline uint16_t double_to_half_bits(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint16_t sign = static_cast<uint16_t>((b >> 48) & 0x8000);
    const int biased = static_cast<int>((b >> 52) & 0x7ff);
    const uint64_t mant = b & 0xfffffffffffffull;
    if (biased == 0x7ff)
        return static_cast<uint16_t>(sign | 0x7c00 | (mant ? (0x200 | static_cast<uint16_t>(mant >> 42)) : 0));
    const int e = biased - 1023;
    if (e > 15) return static_cast<uint16_t>(sign | 0x7c00);
    if (e >= -14) {
        uint32_t h = (static_cast<uint32_t>(e + 15) << 10) | static_cast<uint32_t>(mant >> 42);
        const uint64_t rem = mant & ((1ull << 42) - 1), half = 1ull << 41;
        if (rem > half || (rem == half && (h & 1))) h += 1;
        return static_cast<uint16_t>(sign | h);
    }
    if (e < -25 || biased == 0) return sign;
    const uint64_t full = mant | (1ull << 52);
    const int shift = 28 - e;
    uint64_t hm = full >> shift;
    const uint64_t rem = full & ((1ull << shift) - 1), half = 1ull << (shift - 1);
    if (rem > half || (rem == half && (hm & 1))) hm += 1;
    return static_cast<uint16_t>(sign | hm);
}

// One element of the Q8_0 encoder of tools/make_api_fixture.py:131-137, given
// the group's max |x|: d = f16(max/127), q = clip(rint(x / f32(max/127)), -127, 127),
// q = 0 for an all-zero group.
__host__ __device__ inline void q8_encode_element(float x, float amax, uint16_t* d, int8_t* q) {
    const double scale = static_cast<double>(amax) / 127.0;
    *d = double_to_half_bits(scale);
    if (scale == 0.0) {
        *q = 0;
        return;
    }
    const float s = static_cast<float>(scale);
#if defined(__HIP_DEVICE_COMPILE__)
    float r = __builtin_rintf(__fdiv_rn(x, s));
#else
    float r = __builtin_rintf(x / s);
#endif
    r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
    *q = static_cast<int8_t>(r);
}

}  // namespace tvara_amd
