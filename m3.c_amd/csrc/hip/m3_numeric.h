/*
 * m3_numeric.h - bit-exact element conversions and operation semantics
 * shared by the gfx950 kernels and the host-side self tests.
 *
 * The conversions produce the same bits as the reference's host converters
 * (src/m3_op_numeric.c:27-130) for every input, including NaN payloads,
 * subnormals and ties, but are written branch-free for SIMD execution:
 *   - F16 -> F32 keeps signalling NaNs (sign | 0x7f800000 | frac << 13) and
 *     decodes subnormals exactly as frac * 2^-24;
 *   - F32 -> F16 rounds to nearest even; NaN becomes
 *     sign | 0x7e00 | max(frac >> 13, 1), overflow becomes infinity;
 *     subnormal results are rounded by one F32 addition of 0.5, which puts
 *     the F16 subnormal step 2^-24 at the F32 unit in the last place;
 *   - F32 -> BF16 adds 0x7fff plus the kept low bit; NaN keeps its top 16
 *     bits and sets 0x0040.
 * m3_binary_nan_fix makes a NaN result carry the bits the x86-64 build of
 * the reference's CPU provider produces, so that arithmetic on NaN inputs
 * matches it bit for bit.
 *
 * The file is valid C11 and HIP C++; under HIP every function is
 * __host__ __device__.
 */
#ifndef M3_NUMERIC_H
#define M3_NUMERIC_H

#if defined(__HIPCC_RTC__)
/* runtime compilation: no system headers; its runtime header declares the
 * fixed-width types in namespace __hip_internal */
using __hip_internal::int32_t;
using __hip_internal::uint16_t;
using __hip_internal::uint32_t;
using __hip_internal::uint64_t;
#else
#include <stdint.h>
#include <string.h>
#endif

#if defined(__HIPCC__)
#if !defined(__HIPCC_RTC__)
#include <hip/hip_runtime.h>
#endif
#define M3_HD static __host__ __device__ inline __attribute__((always_inline))
#else
#define M3_HD static inline
#endif

M3_HD uint32_t m3_f32_bits(float value)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint32_t, value);
#else
    uint32_t bits;

    memcpy(&bits, &value, sizeof(bits));
    return bits;
#endif
}

M3_HD float m3_bits_f32(uint32_t bits)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(float, bits);
#else
    float value;

    memcpy(&value, &bits, sizeof(value));
    return value;
#endif
}

M3_HD uint32_t m3_f16_to_f32_bits(uint32_t half)
{
    uint32_t sign = (half & 0x8000U) << 16U;
    uint32_t exponent = (half >> 10U) & 0x1fU;
    uint32_t fraction = half & 0x03ffU;
    uint32_t normal = ((exponent + 112U) << 23U) | (fraction << 13U);
    uint32_t special = 0x7f800000U | (fraction << 13U);
    /* frac * 2^-24 is exact in F32 and is +0 for frac == 0. */
    uint32_t tiny = m3_f32_bits((float)fraction * 0x1.0p-24F);
    uint32_t magnitude = exponent == 0U ? tiny
                         : exponent == 0x1fU ? special : normal;

    return sign | magnitude;
}

M3_HD uint32_t m3_f32_to_f16_bits(uint32_t bits)
{
    uint32_t sign = (bits >> 16U) & 0x8000U;
    uint32_t magnitude = bits & 0x7fffffffU;
    uint32_t rebased = magnitude - (112U << 23U);
    uint32_t normal =
        (rebased + 0x0fffU + ((rebased >> 13U) & 1U)) >> 13U;
    uint32_t subnormal =
        m3_f32_bits(m3_bits_f32(magnitude) + 0.5F) - 0x3f000000U;
    uint32_t nan_fraction = (magnitude >> 13U) & 0x03ffU;
    uint32_t nan = 0x7e00U | (nan_fraction == 0U ? 1U : nan_fraction);
    uint32_t result = magnitude >= 0x38800000U ? normal : subnormal;

    result = magnitude >= 0x47800000U ? 0x7c00U : result;
    result = magnitude > 0x7f800000U ? nan : result;
    return sign | result;
}

M3_HD uint32_t m3_bf16_to_f32_bits(uint32_t brain)
{
    return (brain & 0xffffU) << 16U;
}

M3_HD uint32_t m3_f32_to_bf16_bits(uint32_t bits)
{
    uint32_t rounded = (bits + 0x7fffU + ((bits >> 16U) & 1U)) >> 16U;
    uint32_t nan = (bits >> 16U) | 0x0040U;

    return (bits & 0x7fffffffU) > 0x7f800000U ? nan : rounded;
}

M3_HD int m3_f32_is_nan_bits(uint32_t bits)
{
    return (bits & 0x7fffffffU) > 0x7f800000U;
}

/* Bits of the NaN the x86-64 CPU provider returns for operands a and b
 * when the IEEE result is NaN; `result` is returned unchanged when it is
 * not NaN. A single NaN operand propagates quieted; an invalid operation
 * on non-NaN operands gives the default NaN 0xffc00000. When both operands
 * are NaN, IEEE 754 leaves the payload open: the reference's host loop
 * compiled by gcc for x86-64 evaluates a commutative operation (ADD, MUL)
 * as b (op) a and so returns b's NaN, and SUB/DIV return a's. */
M3_HD uint32_t m3_binary_nan_fix(uint32_t result, uint32_t a, uint32_t b,
                                 int commutative)
{
    int a_nan = m3_f32_is_nan_bits(a);
    int b_nan = m3_f32_is_nan_bits(b);
    uint32_t propagated = (a_nan && !(commutative && b_nan))
                              ? (a | 0x00400000U)
                          : b_nan ? (b | 0x00400000U)
                                  : 0xffc00000U;

    return m3_f32_is_nan_bits(result) ? propagated : result;
}

/* Element types and operations; values equal m3_dtype / m3_hip_binary_op. */
enum { M3N_F32 = 0, M3N_F16 = 1, M3N_BF16 = 2, M3N_I32 = 3 };
enum { M3N_ADD = 0, M3N_MUL = 1, M3N_SUB = 2, M3N_DIV = 3 };

/* Raw element (2 or 4 bytes, zero-extended) -> F32 value bits. */
M3_HD uint32_t m3_load_as_f32_bits(uint32_t raw, uint32_t dtype)
{
    return dtype == M3N_F32    ? raw
           : dtype == M3N_F16  ? m3_f16_to_f32_bits(raw)
           : dtype == M3N_BF16 ? m3_bf16_to_f32_bits(raw)
                               : m3_f32_bits((float)(int32_t)raw);
}

/* F32 value bits -> raw element of dtype (float to I32 truncates toward
 * zero; callers guarantee the value is finite and in range). */
M3_HD uint32_t m3_store_from_f32_bits(uint32_t bits, uint32_t dtype)
{
    return dtype == M3N_F32    ? bits
           : dtype == M3N_F16  ? m3_f32_to_f16_bits(bits)
           : dtype == M3N_BF16 ? m3_f32_to_bf16_bits(bits)
                               : (uint32_t)(int32_t)m3_bits_f32(bits);
}

/* F32 bits rounded through a 16-bit float dtype and back (identity for
 * F32), with the converters of CAST: the value a store of `bits` to that
 * dtype and a load back give (src/m3_op_numeric.c:210-222). */
M3_HD uint32_t m3_round_through_bits(uint32_t bits, uint32_t dtype)
{
    return dtype == M3N_F16
               ? m3_f16_to_f32_bits(m3_f32_to_f16_bits(bits))
           : dtype == M3N_BF16
               ? m3_bf16_to_f32_bits(m3_f32_to_bf16_bits(bits))
               : bits;
}

/* One F32 operation, IEEE round-to-nearest-even, no contraction. */
M3_HD uint32_t m3_binary_f32_bits(uint32_t op, uint32_t a, uint32_t b)
{
    float x = m3_bits_f32(a);
    float y = m3_bits_f32(b);
    float r;

    if (op == M3N_ADD) {
        r = x + y;
    } else if (op == M3N_MUL) {
        r = x * y;
    } else if (op == M3N_SUB) {
        r = x - y;
    } else {
        r = x / y;
    }
    return m3_binary_nan_fix(m3_f32_bits(r), a, b,
                             op == M3N_ADD || op == M3N_MUL);
}

#endif
