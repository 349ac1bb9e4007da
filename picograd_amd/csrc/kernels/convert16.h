// f32 <-> f16/bf16 conversions on the raw bits, shared by the gfx950
// kernels (device code only).  f32 -> 16-bit rounds to nearest even as the
// reference's convert.h:15-104 does: bf16 = (x + 0x7FFF + lsb) >> 16 with
// NaN -> quiet NaN; f16 per IEEE 754 including subnormals (where the
// reference's f16 encoder rounds some subnormals differently, this one
// keeps the IEEE result).
#ifndef PGK_CONVERT16_H
#define PGK_CONVERT16_H

#include <hip/hip_runtime.h>
#include <stdint.h>

// f32 -> bf16: round to nearest even on the raw bits; a NaN becomes the
// positive quiet NaN 0x7FC0 | bit 16 (the reference's convert.h rule).
__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7F800000u) == 0x7F800000u && (x & 0x7FFFFFu) != 0)
        return (uint16_t)(0x7FC0u | ((x >> 16) & 1u));
    return (uint16_t)((x + 0x7FFFu + ((x >> 16) & 1u)) >> 16);
}

// f32 -> f16, IEEE round to nearest even including subnormals; NaN keeps
// its top payload bits and is quieted.
__device__ __forceinline__ uint16_t f32_to_f16(float f)
{
    uint32_t x = __float_as_uint(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ex = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (ex == 255) {
        if (man == 0)
            return (uint16_t)(sign | 0x7C00u);
        uint32_t q = sign | 0x7C00u | (man >> 13);
        if ((q & 0x3FFu) == 0)
            q |= 1u;
        return (uint16_t)(q | 0x200u);
    }
    int e = (int)ex - 112;
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (e <= 0) {
        if (e < -10)
            return (uint16_t)sign;
        man |= 0x800000u;
        uint32_t sh = (uint32_t)(1 - e) + 13u;
        uint32_t keep = man >> sh;
        uint32_t rem = man & ((1u << sh) - 1u);
        uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (keep & 1u)))
            keep++;
        return (uint16_t)(sign | keep);
    }
    uint32_t r = man + 0xFFFu + ((man >> 13) & 1u);
    if (r & 0x800000u) {
        r = 0;
        e++;
    }
    if (e >= 31)
        return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | ((uint32_t)e << 10) | (r >> 13));
}

// f16 -> f32 on the raw bits (exact; NaN payloads kept as they are)
__device__ __forceinline__ float f16_to_f32(uint16_t h)
{
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t ex = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t man = (uint32_t)h & 0x3FFu;
    if (ex == 0) {
        if (man == 0)
            return __uint_as_float(sign);
        int e = 1;
        while ((man & 0x400u) == 0) {
            man <<= 1;
            e--;
        }
        man &= 0x3FFu;
        return __uint_as_float(sign | ((uint32_t)(e + 112) << 23) | (man << 13));
    }
    if (ex == 31)
        return __uint_as_float(sign | 0x7F800000u | (man << 13));
    return __uint_as_float(sign | ((ex + 112u) << 23) | (man << 13));
}

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

__device__ __forceinline__ uint16_t to16(int dtype, float f)
{
    return dtype == 1 ? f32_to_f16(f) : f32_to_bf16(f);
}

__device__ __forceinline__ float from16(int dtype, uint16_t h)
{
    return dtype == 1 ? f16_to_f32(h) : bf16_to_f32(h);
}

#endif
