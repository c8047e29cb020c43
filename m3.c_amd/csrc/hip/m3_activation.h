/*
 * m3_activation.h - the GATED_SILU element function, shared by the gfx950
 * kernels (m3_hip_activation.hip) and the host checks that compare it
 * with the C library's arithmetic on every gate value. TANH elements are
 * m3_tanhf_uniform (m3_libm.h).
 *
 * Reference semantics (src/m3_op_execute_basic.c:104-122): gate and up
 * load as F32; activation = gate / (1 + expf(-gate)), each operation one
 * rounded F32 operation, then rounded through the gate's dtype
 * (src/m3_op_numeric.c:210-222); result = activation * up, stored in the
 * output's dtype.
 */
#ifndef M3_ACTIVATION_H
#define M3_ACTIVATION_H

#include "m3_libm.h"
#include "m3_numeric.h"

/* The unrounded activation gate / (1 + expf(-gate)). Its bits equal the
 * host's whenever they are not NaN. */
M3_HD float m3_silu_quotient(float gate)
{
    return gate / (1.0F + m3_expf_any(-gate));
}

/* The unrounded activation as the vector kernels form it: expf with the
 * table `table` (a copy in LDS on the device) and its overflow as a select
 * instead of a branch, and the division as m3_div_normal where its
 * operands allow it. Both operands are scaled by 2^-32 first (exact, and
 * the quotient is unchanged), so that the reciprocal of a denominator up
 * to 2^128 (gates down to -88.7) stays normal. Gates below 2^-60 in
 * magnitude (zeros, subnormals) take gate * 0.5, the exact quotient by
 * 1 + expf(-gate) = 2, and an infinite denominator takes gate * 0 (-0, or
 * NaN for gate = -inf). For
 * every gate whose activation is not NaN on the host the result has the
 * host's bits, except that on the device an infinite or near-overflow
 * quotient (gate near +inf, divided by 1) comes out NaN; NaN results carry
 * no defined payload. Callers recompute every NaN with m3_gated_silu_bits. */
M3_HD float m3_silu_quotient_fast(float gate, const uint64_t *table)
{
    const float threshold = 0x1.62e42ep6F; /* expf overflows above */
    const float minus = -gate;
    /* formed for every gate and then selected, not branched on */
    const float clamped = m3_expf_with_table(fminf(minus, threshold), table);
    const float exp_minus =
        minus > threshold ? m3_bits_f32(0x7f800000U) : clamped;
    const float denominator = 1.0F + exp_minus;
    float quotient =
        m3_div_normal(gate * 0x1p-32F, denominator * 0x1p-32F);

    quotient = fabsf(gate) < 0x1p-60F ? gate * 0.5F : quotient;
    return m3_f32_bits(denominator) == 0x7f800000U ? gate * 0.0F : quotient;
}

/* F32 bits rounded through BF16 and back, for bits that are not NaN. */
M3_HD uint32_t m3_round_through_bf16_finite(uint32_t bits)
{
    return (bits + 0x7fffU + ((bits >> 16U) & 1U)) & 0xffff0000U;
}

/* One GATED_SILU element as F32 bits, NaN bits included. On the host a NaN
 * gate passes through the division quieted (the dividend's NaN is taken),
 * the only invalid division, -inf / inf, gives 0xffc00000, and the product
 * activation * up takes the activation's NaN when both operands are NaN
 * (gcc evaluates it with the activation as the first operand): the rule of
 * m3_binary_nan_fix for a non-commutative operation, in both steps. */
M3_HD uint32_t m3_gated_silu_bits(float gate, float up, uint32_t gate_dtype)
{
    const float one_plus = 1.0F + m3_expf_any(-gate);
    const uint32_t quotient = m3_binary_nan_fix(
        m3_f32_bits(gate / one_plus), m3_f32_bits(gate),
        m3_f32_bits(one_plus), 0);
    const uint32_t activation = m3_round_through_bits(quotient, gate_dtype);
    const float product = m3_bits_f32(activation) * up;

    return m3_binary_nan_fix(m3_f32_bits(product), activation,
                             m3_f32_bits(up), 0);
}

#endif
