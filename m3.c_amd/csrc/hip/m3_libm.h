/*
 * m3_libm.h - single-precision exp and sin that return the same bits as the
 * C library the CPU provider of the reference calls on Linux.
 *
 * The reference computes softmax with expf and Snake1d with sinf from the
 * platform libm (src/m3_op_execute_basic.c:156,172,188). On this image that
 * is GNU libc 2.35 on x86-64, whose expf and sinf are the ARM
 * optimized-routines algorithms (Szabolcs Nagy, 2017; MIT licence),
 * dispatched to the variants built with FMA on CPUs that have it:
 *
 *   expf: x*N/ln2 = k + r with N = 32, |r| <= 1/2, both products fused;
 *         2^(k/N) from a 32-entry table T[i] = bits(RN(2^(i/32))) - i<<47
 *         with k folded into the exponent; 2^(r/N) by a cubic in double.
 *   sinf: |x| < pi/4 (by the top 12 bits) -> odd polynomial in double;
 *         |x| < 120 -> quadrant n = round(x*2/pi) by the 2^24-scaled
 *         integer trick, r = x - n*pi/2 fused; |x| >= 120 -> 96-bit
 *         fixed-point reduction with 192 bits of 2/pi; then the sine or
 *         cosine polynomial selected by the quadrant.
 *
 * These restatements were checked bit for bit against that libm: expf on
 * every non-NaN float up to log(2^128) (all 3,196,059,650 floats <= 0.5
 * and all floats in (-103.9, 88.7)) and sinf on all 2^32 floats, with zero
 * mismatches. The test suite re-checks a dense sample on every run.
 *
 * Valid C11 and HIP C++; under HIP every function is __host__ __device__.
 * All double operations must stay unfused except where fma() is written.
 */
#ifndef M3_LIBM_H
#define M3_LIBM_H

#include "m3_numeric.h"

#include <math.h>
#include <stdint.h>

#if defined(__HIPCC__)
#define M3_LIBM_CONST static __constant__
#else
#define M3_LIBM_CONST static const
#endif

M3_HD uint64_t m3_f64_bits(double value)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(uint64_t, value);
#else
    uint64_t bits;

    memcpy(&bits, &value, sizeof(bits));
    return bits;
#endif
}

M3_HD double m3_bits_f64(uint64_t bits)
{
#if defined(__HIPCC__)
    return __builtin_bit_cast(double, bits);
#else
    double value;

    memcpy(&value, &bits, sizeof(value));
    return value;
#endif
}

/* T[i] = bits(RN(2^(i/32))) - (i << 47). */
#define M3_EXPF_TABLE_INIT                                                    \
    {                                                                         \
        0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, \
        0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, \
        0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL, \
        0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL, \
        0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, \
        0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, \
        0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL, \
        0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL, \
        0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, \
        0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, \
        0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL                         \
    }

M3_LIBM_CONST uint64_t m3_expf_table[32] = M3_EXPF_TABLE_INIT;

/* expf for x that is not NaN and not above log(2^128) (the softmax domain is
 * x <= 0). `table` holds the 32 entries of M3_EXPF_TABLE_INIT; kernels pass
 * a copy in LDS. */
M3_HD float m3_expf_with_table(float x, const uint64_t *table)
{
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    /* The library returns +0 below log(2^-150) (and for -inf). Clamping the
     * argument at -128 gives the same result without a branch: the
     * arithmetic below then yields a double near 2^-184.7, which rounds to
     * +0 in the final conversion, and every x in (-128, log(2^-150)) also
     * rounds to +0 (checked on all floats). */
    double xd = (double)fmaxf(x, -128.0F);
    double kd;
    double r;
    double s;
    double z;
    double y;
    uint64_t ki;

    kd = fma(inv_ln2_n, xd, shift);
    ki = m3_f64_bits(kd);
    kd -= shift;
    r = fma(inv_ln2_n, xd, -kd);
    /* s = bits(T[ki % 32] + (ki << 47) mod 2^64). The addend's low word is
     * zero, so only the high word changes: high(T) + (low(ki) << 15). The
     * device form keeps the two words apart so that this stays a single
     * 32-bit shift-add. */
#if defined(__HIP_DEVICE_COMPILE__)
    {
        typedef uint32_t m3_words __attribute__((ext_vector_type(2)));
        m3_words entry = ((const m3_words *)table)[ki % 32U];

        entry.y += (uint32_t)ki << 15U;
        s = __builtin_bit_cast(double, entry);
    }
#else
    s = m3_bits_f64(table[ki % 32U] + (ki << 47U));
#endif
    z = fma(c0, r, c1);
    y = fma(c2, r, 1.0);
    y = fma(z, r * r, y);
    return (float)(y * s);
}

M3_HD float m3_expf(float x)
{
    return m3_expf_with_table(x, m3_expf_table);
}

/* 32-bit windows of the bytes of 2/pi = 0.a2f9836e4e441529fc27...: entry i
 * holds bytes max(0,i-3)..i. */
M3_LIBM_CONST uint32_t m3_sinf_two_over_pi[24] = {
    0x000000a2U, 0x0000a2f9U, 0x00a2f983U, 0xa2f9836eU, 0xf9836e4eU,
    0x836e4e44U, 0x6e4e4415U, 0x4e441529U, 0x441529fcU, 0x1529fc27U,
    0x29fc2757U, 0xfc2757d1U, 0x2757d1f5U, 0x57d1f534U, 0xd1f534ddU,
    0xf534ddc0U, 0x34ddc0dbU, 0xddc0db62U, 0xc0db6295U, 0xdb629599U,
    0x6295993cU, 0x95993c43U, 0x993c4390U, 0x3c439041U
};

/* Sine polynomial (even quadrant, odd = 0) or cosine polynomial (odd
 * quadrant), the cosine negated for quadrants 2 and 3. */
M3_HD double m3_sinf_eval(double x, double x2, int odd, int negate_cos)
{
    const double s1 = -0x1.555545995a603p-3;
    const double s2 = 0x1.1107605230bc4p-7;
    const double s3 = -0x1.994eb3774cf24p-13;
    double sign = negate_cos ? -1.0 : 1.0;

    if (!odd) {
        double x3 = x * x2;
        double t = fma(x2, s3, s2);
        double x7 = x3 * x2;
        double s = fma(x3, s1, x);

        return fma(x7, t, s);
    } else {
        double c0 = sign * 0x1p0;
        double c1 = sign * -0x1.ffffffd0c621cp-2;
        double c2 = sign * 0x1.55553e1068f19p-5;
        double c3 = sign * -0x1.6c087e89a359dp-10;
        double c4 = sign * 0x1.99343027bf8c3p-16;
        double x4 = x2 * x2;
        double t2 = fma(x2, c4, c3);
        double t1 = fma(x2, c1, c0);
        double x6 = x4 * x2;
        double c = fma(x4, c2, t1);

        return fma(x6, t2, c);
    }
}

M3_HD uint32_t m3_sinf_top12(float value)
{
    return (m3_f32_bits(value) >> 20U) & 0x7ffU;
}

/* sinf for |y| >= 120 and for infinities and NaN (which give NaN): the
 * 96-bit fixed-point reduction with 192 bits of 2/pi. */
M3_HD float m3_sinf_large(float y)
{
    const double pi63 = 0x1.921FB54442D18p-62;
    uint32_t xi = m3_f32_bits(y);
    const uint32_t *window;
    uint32_t shift;
    uint64_t lo;
    uint64_t mid;
    uint64_t hi;
    uint64_t q;
    double x;
    int n;
    int quadrant;
    double sign;

    if (m3_sinf_top12(y) >= m3_sinf_top12(INFINITY)) {
        return (y - y) / (y - y);
    }
    window = &m3_sinf_two_over_pi[(xi >> 26U) & 15U];
    shift = (xi >> 23U) & 7U;
    xi = (xi & 0xffffffU) | 0x800000U;
    xi <<= shift;
    hi = (uint64_t)(xi * window[0]);
    mid = (uint64_t)xi * window[4];
    lo = (uint64_t)xi * window[8];
    hi = (lo >> 32U) | (hi << 32U);
    hi += mid;
    q = (hi + (1ULL << 61U)) >> 62U;
    hi -= q << 62U;
    x = (double)(int64_t)hi * pi63;
    n = (int)q;
    quadrant = n + (int)(m3_f32_bits(y) >> 31U);
    sign = ((quadrant & 3) == 1 || (quadrant & 3) == 2) ? -1.0 : 1.0;
    return (float)m3_sinf_eval(x * sign, x * x, n & 1, (quadrant & 2) != 0);
}

/* sinf of the libm for |y| < 120 (m3_sinf_top12(y) < m3_sinf_top12(120)),
 * as one branch-free sequence that gives the library's result bit for bit
 * (checked on all floats through m3_sinf):
 *   - the library's separate path for |y| < 0.75 evaluates the sine
 *     polynomial on y itself; the reduction below gives n = 0 there and
 *     fma(-0, pi/2, y) = y exactly, so it is the same evaluation;
 *   - its |y| < 2^-12 path returns y, kept here as a final select (it also
 *     keeps the sign of -0);
 *   - the library negates the cosine coefficients for quadrants 2 and 3
 *     and evaluates the sine polynomial on -x for quadrants 1 and 2; with
 *     round-to-nearest both equal negating the polynomial's result, so
 *     quadrant n gives (n odd ? cosine : sine), negated when n & 2.
 * Both polynomials are evaluated and one is selected, so SIMD lanes in
 * different quadrants do not diverge. m3_sinf_medium_unsigned returns the
 * selected polynomial before the sign of quadrants 2 and 3 is applied, and
 * the quadrant in *quadrant. */
M3_HD double m3_sinf_medium_unsigned(float y, int32_t *quadrant)
{
    const double half_pi = 0x1.921FB54442D18p0;
    const double s1 = -0x1.555545995a603p-3;
    const double s2 = 0x1.1107605230bc4p-7;
    const double s3 = -0x1.994eb3774cf24p-13;
    const double c0 = 0x1p0;
    const double c1 = -0x1.ffffffd0c621cp-2;
    const double c2 = 0x1.55553e1068f19p-5;
    const double c3 = -0x1.6c087e89a359dp-10;
    const double c4 = 0x1.99343027bf8c3p-16;
    double x = (double)y;
    double r = x * 0x1.45F306DC9C883p+23;
    int32_t n = ((int32_t)r + 0x800000) >> 24;
    double x2;
    double sine;
    double cosine;

    x = fma(-(double)n, half_pi, x);
    x2 = x * x;
    {
        double x3 = x * x2;
        double t = fma(x2, s3, s2);
        double x7 = x3 * x2;
        double s = fma(x3, s1, x);

        sine = fma(x7, t, s);
    }
    {
        double x4 = x2 * x2;
        double t2 = fma(x2, c4, c3);
        double t1 = fma(x2, c1, c0);
        double x6 = x4 * x2;
        double c = fma(x4, c2, t1);

        cosine = fma(x6, t2, c);
    }
    *quadrant = n;
    return (n & 1) != 0 ? cosine : sine;
}

M3_HD float m3_sinf_medium(float y)
{
    int32_t n;
    double value = m3_sinf_medium_unsigned(y, &n);

    value = (n & 2) != 0 ? -value : value;
    return m3_sinf_top12(y) < m3_sinf_top12(0x1p-12F) ? y : (float)value;
}

/* |sinf(y)| for |y| < 120, for callers that only use the magnitude (a
 * square): the sign flip and the |y| < 2^-12 select of m3_sinf_medium are
 * left out. Below 2^-12 the polynomial's terms past y are under 2^-26 of y,
 * so (float) rounds back to +-y; the magnitude equals |m3_sinf(y)| for every
 * float with |y| < 120 (checked exhaustively). */
M3_HD float m3_sinf_medium_magnitude(float y)
{
    int32_t n;

    return (float)m3_sinf_medium_unsigned(y, &n);
}

/* sinf of the libm, for every float input (NaN and infinities give NaN). */
M3_HD float m3_sinf(float y)
{
    if (m3_sinf_top12(y) >= m3_sinf_top12(120.0F)) {
        return m3_sinf_large(y);
    }
    return m3_sinf_medium(y);
}

#endif
