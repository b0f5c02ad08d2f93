// rac_q8.hpp — Q8_0 block helpers shared by the GEMV, the quantizer and the
// safetensors loader (lib/c/rac_q8_0.h layout: fp16 scale d, then 32 int8).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rac {

constexpr int kQ8Block = 32;
constexpr int kQ8Bytes = 34;

// The same value by the hardware conversion (v_cvt_f32_f16, fp16
// denormals preserved): equal to half_bits_to_float for every zero,
// subnormal, normal and infinite half; a signalling NaN comes back quiet.
// For a GEMV block scale that difference cannot show, since the scale only
// enters an fma, whose result is the same quiet NaN either way (the outputs
// agree bit for bit over all 65536 patterns).  Code that stores the
// converted value itself keeps half_bits_to_float.
__device__ __forceinline__ float half_bits_to_float_cvt(uint32_t h) {
    const uint16_t b = (uint16_t)h;
    _Float16 v;
    __builtin_memcpy(&v, &b, 2);
    return (float)v;
}

// rac_fp16_to_fp32 (rac_q8_0.c:21-45) as bit operations.
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint32_t sign = (h >> 15) & 1u, ex = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu, bits;
    if (ex == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            // normalise: shift until bit 10 is set
            const int lz = __builtin_clz(mant) - 21;   // leading zeros within the 11-bit field
            mant = (mant << lz) & 0x3ffu;
            bits = (sign << 31) | ((uint32_t)(-14 - lz + 127) << 23) | (mant << 13);
        }
    } else if (ex == 31) {
        bits = (sign << 31) | (0xffu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((ex - 15 + 127) << 23) | (mant << 13);
    }
    return __uint_as_float(bits);
}

// rac_fp32_to_fp16 (rac_q8_0.c:47-64): truncating conversion.
__device__ __forceinline__ uint32_t float_to_half_bits(float f) {
    const uint32_t b = __float_as_uint(f);
    const uint32_t sign = (b >> 16) & 0x8000u;
    const int ex = (int)((b >> 23) & 0xffu) - 127 + 15;
    uint32_t mant = b & 0x7fffffu;
    if (ex <= 0) {
        if (ex < -10) return sign;
        mant = (mant | 0x800000u) >> (1 - ex);
        return sign | (mant >> 13);
    }
    if (ex >= 31) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    return sign | ((uint32_t)ex << 10) | (mant >> 13);
}

// rac_q8_0_quantize_row (rac_q8_0.c:66-100) for one block of 32 values:
// d = amax / 127 stored as truncated fp16, q = (int)lrintf(v * (1 / d)).
__device__ __forceinline__ void q8_quantize_block(const float (&v)[kQ8Block], uint8_t* o) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < kQ8Block; i++) {
        const float a = __builtin_fabsf(v[i]);
        if (a > amax) amax = a;
    }
    const float d = amax / 127.0f;
    const float id = (d > 0.0f) ? 1.0f / d : 0.0f;
    const uint32_t h = float_to_half_bits(d);
    o[0] = (uint8_t)(h & 0xffu);
    o[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int i = 0; i < kQ8Block; i++) {
        const float t = __builtin_rintf(v[i] * id);
        // (int)lrintf(t) on the reference's x86-64 host: NaN and |t| >= 2^63
        // convert to LONG_MIN, whose low 32 bits are 0.  |t| exceeds 127 only
        // when id overflowed to inf (amax < 2^-121), so t is then +-inf or
        // NaN and q = 0; otherwise the clamp to [-127, 127] applies.
        const int q = (__builtin_fabsf(t) < 2147483648.0f) ? (int)__builtin_amdgcn_fmed3f(t, -127.0f, 127.0f) : 0;
        o[2 + i] = (uint8_t)(int8_t)q;
    }
}

}  // namespace rac
