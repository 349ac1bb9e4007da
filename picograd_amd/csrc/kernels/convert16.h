// f32 <-> f16/bf16 conversions shared by the gfx950 kernels (device code
// only).  f32 -> 16-bit rounds to nearest even as the reference's
// convert.h:15-104 does: bf16 = (x + 0x7FFF + lsb) >> 16 with NaN -> quiet
// NaN; f16 per IEEE 754 including subnormals (where the reference's f16
// encoder rounds some subnormals differently, this one keeps the IEEE
// result).  The encoders are gfx950's hardware converts with the NaN rule
// applied on top; the decoders work on the raw bits.
#ifndef PGK_CONVERT16_H
#define PGK_CONVERT16_H

#ifdef __HIPCC_RTC__
// the JIT compiles this file's text with hiprtc, whose fixed-width types
// live in a namespace of its own
using __hip_internal::uint16_t;
using __hip_internal::uint32_t;
#else
#include <hip/hip_runtime.h>
#include <stdint.h>
#endif

// f32 -> bf16 by the hardware convert (v_cvt_pk_bf16_f32): round to nearest
// even, f32 subnormals kept (the kernels run in the default FP mode, which
// does not flush them), so every non-NaN input gets the integer rule's
// (x + 0x7FFF + lsb) >> 16.  A NaN becomes the positive quiet NaN
// 0x7FC0 | bit 16 (the reference's convert.h rule), not the instruction's.
__device__ __forceinline__ uint16_t bf16_nan(float f) { return (uint16_t)(0x7FC0u | ((__float_as_uint(f) >> 16) & 1u)); }

__device__ __forceinline__ uint16_t f32_to_bf16(float f)
{
    const uint16_t h = __builtin_bit_cast(uint16_t, (__bf16)f);
    return f != f ? bf16_nan(f) : h;
}

// two at once, a in the low half: one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float a, float b)
{
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 h2 __attribute__((ext_vector_type(2)));
    const f2 v = {a, b};
    uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
    h = a != a ? (h & 0xFFFF0000u) | bf16_nan(a) : h;
    h = b != b ? (h & 0xFFFFu) | ((uint32_t)bf16_nan(b) << 16) : h;
    return h;
}

// f32 -> f16 by the hardware convert (v_cvt_f16_f32): IEEE round to nearest
// even including f16 subnormals and overflow to infinity.  A NaN keeps its
// top 10 payload bits and is quieted, with payload 1 when those are all zero
// (the reference's convert.h:22-28 rule: sign | 0x7C00 | man >> 13, | 1 when
// that leaves no payload, | 0x200).
__device__ __forceinline__ uint16_t f32_to_f16(float f)
{
    const uint16_t h = __builtin_bit_cast(uint16_t, (_Float16)f);
    if (f != f) {
        const uint32_t x = __float_as_uint(f), m = (x & 0x7FFFFFu) >> 13;
        return (uint16_t)(((x >> 16) & 0x8000u) | 0x7E00u | m | (m == 0 ? 1u : 0u));
    }
    return h;
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

// a and b as two 16-bit values of one word, a in the low half
__device__ __forceinline__ uint32_t to16x2(int dtype, float a, float b)
{
    return dtype == 1 ? (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16) : f32x2_to_bf16x2(a, b);
}

__device__ __forceinline__ float from16(int dtype, uint16_t h)
{
    return dtype == 1 ? f16_to_f32(h) : bf16_to_f32(h);
}

#endif
