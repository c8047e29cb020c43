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

/* True when `condition` holds in any lane of the wave on the device, and
 * simply `condition` on the host: straight-line code uses it to skip work
 * that no lane of a wave needs. */
#if defined(__HIP_DEVICE_COMPILE__)
#define M3_ANY_LANE(condition) (__any(condition) != 0)
#else
#define M3_ANY_LANE(condition) (condition)
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

/* expf of the libm for every float input: a NaN gives itself quieted (the
 * library returns x + x), inputs above log(2^128) = 0x1.62e42ep6 and +inf
 * overflow to +inf (the library's overflow path), and everything else,
 * -inf included, is m3_expf, which rounds to +0 below log(2^-150) as the
 * library's underflow path returns. */
M3_HD float m3_expf_any(float x)
{
    uint32_t bits = m3_f32_bits(x);

    if ((bits & 0x7fffffffU) > 0x7f800000U) {
        return m3_bits_f32(bits | 0x00400000U);
    }
    if (x > 0x1.62e42ep6F) {
        return m3_bits_f32(0x7f800000U);
    }
    return m3_expf(x);
}

/* expm1f and tanhf of the libm. GNU libc 2.35 computes both with the
 * single-precision fdlibm algorithms (Sun Microsystems, 1993; freely
 * redistributable), in float arithmetic without fused operations:
 *   expm1f: |x| >= 27 ln2 -> -1 (x < 0) or overflow above 0x1.62e3p6;
 *           reduction x = k ln2 + r (hi/lo split of ln2) for |x| > ln2/2;
 *           |x| < 2^-25 -> x; expm1(r) from a rational form in
 *           r/2 * r with a degree-5 polynomial in (r/2 * r); the result
 *           rebuilt with k folded into the exponent.
 *   tanhf:  |x| >= 22 -> +-1; |x| < 2^-55 -> x (1 + x);
 *           |x| >= 1 -> 1 - 2 / (expm1f(2|x|) + 2);
 *           else -> -t / (t + 2) with t = expm1f(-2|x|).
 * The statements below follow that published algorithm operation by
 * operation; checked bit for bit against the library on all 2^32 inputs. */
M3_HD float m3_expm1f(float x)
{
    const float huge = 1.0e+30F;
    const float tiny = 1.0e-30F;
    const float ln2_hi = 6.9313812256e-01F; /* 0x3f317180 */
    const float ln2_lo = 9.0580006145e-06F; /* 0x3717f7d1 */
    const float invln2 = 1.4426950216e+00F; /* 0x3fb8aa3b */
    const float q1 = -3.3333335072e-02F;    /* 0xbd088889 */
    const float q2 = 1.5873016091e-03F;     /* 0x3ad00d01 */
    const float q3 = -7.9365076090e-05F;    /* 0xb8a670cd */
    const float q4 = 4.0082177293e-06F;     /* 0x36867e54 */
    const float q5 = -2.0109921195e-07F;    /* 0xb457edbb */
    uint32_t hx = m3_f32_bits(x);
    const uint32_t xsb = hx & 0x80000000U;
    float hi;
    float lo;
    float c = 0.0F;
    float t;
    float e;
    float hxs;
    float hfx;
    float r1;
    float y;
    int32_t k;

    hx &= 0x7fffffffU;
    if (hx >= 0x4195b844U) { /* |x| >= 27 ln2 */
        if (hx >= 0x42b17218U) { /* |x| >= 88.721... */
            if (hx > 0x7f800000U) {
                return x + x; /* NaN */
            }
            if (hx == 0x7f800000U) {
                return xsb == 0U ? x : -1.0F;
            }
            if (x > 8.8721679688e+01F) { /* 0x42b17180 */
                return huge * huge; /* overflow */
            }
        }
        if (xsb != 0U) {
            return tiny - 1.0F;
        }
    }
    if (hx > 0x3eb17218U) { /* |x| > ln2 / 2 */
        if (hx < 0x3f851592U) { /* and |x| < 1.5 ln2 */
            if (xsb == 0U) {
                hi = x - ln2_hi;
                lo = ln2_lo;
                k = 1;
            } else {
                hi = x + ln2_hi;
                lo = -ln2_lo;
                k = -1;
            }
        } else {
            k = (int32_t)(invln2 * x + (xsb == 0U ? 0.5F : -0.5F));
            t = (float)k;
            hi = x - t * ln2_hi; /* exact */
            lo = t * ln2_lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000U) { /* |x| < 2^-25 */
        t = huge + x;
        return x - (t - (huge + x));
    } else {
        k = 0;
    }
    hfx = 0.5F * x;
    hxs = x * hfx;
    r1 = 1.0F + hxs * (q1 + hxs * (q2 + hxs * (q3 + hxs * (q4 + hxs * q5))));
    t = 3.0F - r1 * hfx;
    e = hxs * ((r1 - t) / (6.0F - x * t));
    if (k == 0) {
        return x - (x * e - hxs);
    }
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) {
        return 0.5F * (x - e) - 0.5F;
    }
    if (k == 1) {
        if (x < -0.25F) {
            return -2.0F * (e - (x + 0.5F));
        }
        return 1.0F + 2.0F * (x - e);
    }
    if (k <= -2 || k > 56) { /* exp(x) - 1 */
        y = 1.0F - (e - x);
        y = m3_bits_f32(m3_f32_bits(y) + ((uint32_t)k << 23U));
        return y - 1.0F;
    }
    if (k < 23) {
        t = m3_bits_f32(0x3f800000U - (0x1000000U >> k)); /* 1 - 2^-k */
        y = t - (e - x);
    } else {
        t = m3_bits_f32((uint32_t)(0x7f - k) << 23U); /* 2^-k */
        y = x - (e + t);
        y += 1.0F;
    }
    return m3_bits_f32(m3_f32_bits(y) + ((uint32_t)k << 23U));
}

M3_HD float m3_tanhf(float x)
{
    const uint32_t jx = m3_f32_bits(x);
    const uint32_t ix = jx & 0x7fffffffU;
    float t;
    float z;

    if (ix >= 0x7f800000U) { /* infinity or NaN */
        if ((jx & 0x80000000U) == 0U) {
            return 1.0F / x + 1.0F;
        }
        return 1.0F / x - 1.0F;
    }
    if (ix < 0x41b00000U) { /* |x| < 22 */
        if (ix == 0U) {
            return x;
        }
        if (ix < 0x24000000U) { /* |x| < 2^-55 */
            return x * (1.0F + x);
        }
        if (ix >= 0x3f800000U) { /* |x| >= 1 */
            t = m3_expm1f(2.0F * fabsf(x));
            z = 1.0F - 2.0F / (t + 2.0F);
        } else {
            t = m3_expm1f(-2.0F * fabsf(x));
            z = -t / (t + 2.0F);
        }
    } else {
        z = 1.0F - 1.0e-30F;
    }
    return (jx & 0x80000000U) == 0U ? z : -z;
}

/* a / b rounded to nearest even, for callers that guarantee a, b, 1 / b
 * and the quotient are normal (|b| < 2^126) and the quotient is far from
 * overflow. On the device this is the
 * Newton-Raphson iteration of the compiler's IEEE division (reciprocal
 * estimate, one refinement, two correction steps) without its operand
 * scaling and special-value fixup, which leave such operands unchanged;
 * on the host it is the C division. */
M3_HD float m3_div_normal(float a, float b)
{
#if defined(__HIP_DEVICE_COMPILE__)
    float y = __builtin_amdgcn_rcpf(b);
    const float e = fmaf(-b, y, 1.0F);
    float q;
    float r;

    y = fmaf(e, y, y);
    q = a * y;
    r = fmaf(-b, q, a);
    q = fmaf(r, y, q);
    r = fmaf(-b, q, a);
    return fmaf(r, y, q);
#else
    return a / b;
#endif
}

/* a / b for TANH's two divisions: the product of a and the hardware
 * reciprocal of b, corrected once by its residual (4 instructions;
 * m3_div_normal refines the reciprocal first and corrects twice, 8). That
 * is the correctly rounded quotient for most operand pairs but not for
 * all; the GPU test of TANH over every F32 input shows that no input of
 * tanhf reaches such a pair through either division. On the host it is the
 * C division. */
M3_HD float m3_div_one_step(float a, float b)
{
#if defined(__HIP_DEVICE_COMPILE__)
    const float y = __builtin_amdgcn_rcpf(b);
    const float q = a * y;

    return fmaf(fmaf(-b, q, a), y, q);
#else
    return a / b;
#endif
}

/* m3_expm1f for the arguments tanhf passes, v in (-2, 0) or [2, 44], as
 * straight-line code: every case of the reduction is the general one with
 * k = 0 (no reduction, c = 0), k = +-1 below 1.5 ln2, or k = round(v/ln2),
 * which gives the same hi, lo, x and c bit for bit; the reconstructions
 * of the cases k = 0, k = -1, k <= -2 and 2 <= k < 23 are all formed and
 * one is selected, and those of 23 <= k <= 56 and k > 56 (tanh's |x| of
 * 7.97 and more) only in a wave that has such an argument; below
 * |v| = 2^-25, where the library returns v, the k = 0 form gives v as
 * well. (k = 1 needs v in (ln2/2, 1.5 ln2), outside that domain, so
 * 1.5 ln2 > |v| > ln2 / 2 means k = -1.)
 * The quotient of the polynomial step has operands near -2 and 6, so
 * m3_div_normal applies. */
M3_HD float m3_expm1f_tanh(float v)
{
    const float ln2_hi = 6.9313812256e-01F;
    const float ln2_lo = 9.0580006145e-06F;
    const float invln2 = 1.4426950216e+00F;
    const float q1 = -3.3333335072e-02F;
    const float q2 = 1.5873016091e-03F;
    const float q3 = -7.9365076090e-05F;
    const float q4 = 4.0082177293e-06F;
    const float q5 = -2.0109921195e-07F;
    const uint32_t hv = m3_f32_bits(v);
    const uint32_t hx = hv & 0x7fffffffU;
    /* +-0.5 with v's sign */
    const float half = m3_bits_f32(0x3f000000U | (hv & 0x80000000U));
    /* |v| <= ln2 / 2: k = 0; |v| < 1.5 ln2: k = -1 (v < 0 there); no
     * other argument rounds to k = 0 or -1 */
    const int k_zero = hx <= 0x3eb17218U;
    const int k_minus_one = hx < 0x3f851592U;
    const int32_t k = k_zero ? 0
                      : k_minus_one ? -1
                                    : (int32_t)(invln2 * v + half);
    const float kf = (float)k;
    const float hi = v - kf * ln2_hi;
    const float lo = kf * ln2_lo;
    const float x = hi - lo;
    const float c = (hi - x) - lo;
    const float hfx = 0.5F * x;
    const float hxs = x * hfx;
    const float r1 =
        1.0F + hxs * (q1 + hxs * (q2 + hxs * (q3 + hxs * (q4 + hxs * q5))));
    const float t = 3.0F - r1 * hfx;
    const float e = hxs * m3_div_one_step(r1 - t, 6.0F - x * t);
    const float zero_k = x - (x * e - hxs);
    float f = x * (e - c) - c;
    const uint32_t kbits = (uint32_t)k << 23U;

    f -= hxs;
    const float minus_one_k = 0.5F * (x - f) - 0.5F;
    const float outer =
        m3_bits_f32(m3_f32_bits(1.0F - (f - x)) + kbits) - 1.0F;
    const float low_t =
        m3_bits_f32(0x3f800000U - (0x1000000U >> ((uint32_t)k & 31U)));
    const float low = m3_bits_f32(m3_f32_bits(low_t - (f - x)) + kbits);
    float result = k <= -2 ? outer : low;
    /* k >= 23 (tanh's |x| from 7.97 on): formed only in a wave that has
     * such an argument */
    const int high_case = k >= 23;

    if (M3_ANY_LANE(high_case)) {
        const float high_t = m3_bits_f32((uint32_t)(0x7f - k) << 23U);
        float high = x - (f + high_t);

        high += 1.0F;
        high = m3_bits_f32(m3_f32_bits(high) + kbits);
        result = k > 56 ? outer : high_case ? high : result;
    }
    result = k_minus_one ? minus_one_k : result;
    /* for |v| < 2^-25 the library returns v itself; zero_k is v there too
     * (x = v and x * e - hxs is below a quarter of v's ulp) */
    return k_zero ? zero_k : result;
}

/* m3_tanhf as straight-line code with one expm1f evaluation and one
 * division per input: its |x| >= 1 and |x| < 1 cases differ only in the
 * sign of the expm1f argument (2|x| or -2|x|) and in the numerator (2 or
 * -t) of the quotient by t + 2, so both are formed with selects. |x| is
 * clamped at 22 first (results there are the constant 1 - 1e-30, with the
 * sign), so expm1f sees only its tanhf domain. A NaN input returns that
 * NaN quieted, the bits 1/x + 1 gives on the host, without relying on how
 * the device propagates NaN operands. The quotient's operands are normal
 * wherever its result is used (numerator 2 or at least 2^-54 in
 * magnitude, denominator in [1.1, 2^64)). Same bits as m3_tanhf for every
 * input. */
M3_HD float m3_tanhf_straight(float x)
{
    const uint32_t jx = m3_f32_bits(x);
    const uint32_t ix = jx & 0x7fffffffU;
    const int big = ix >= 0x3f800000U;
    /* |x| clamped at 22 on its bits (NaN too: its result is set below) */
    const float magnitude = m3_bits_f32(ix < 0x41b00000U ? ix : 0x41b00000U);
    const float t = m3_expm1f_tanh((big ? 2.0F : -2.0F) * magnitude);
    const float q = m3_div_one_step(big ? 2.0F : -t, t + 2.0F);
    const uint32_t sign = jx & 0x80000000U;
    /* |x| >= 22, infinities and NaN, or |x| < 2^-55: handled only in a
     * wave that has such an input */
    const int rare = ix - 0x24000000U >= 0x41b00000U - 0x24000000U;
    float z = big ? 1.0F - q : q; /* +0 or positive */

    z = m3_bits_f32(m3_f32_bits(z) | sign);
    if (M3_ANY_LANE(rare)) {
        if (ix >= 0x41b00000U) { /* |x| >= 22 and infinities */
            z = m3_bits_f32(m3_f32_bits(1.0F - 1.0e-30F) | sign);
        }
        if (ix < 0x24000000U) { /* |x| < 2^-55, zeros and subnormals
                                 * included: 1 + x rounds to 1, so
                                 * x * (1 + x) is x */
            z = x;
        }
        if (ix > 0x7f800000U) {
            z = m3_bits_f32(jx | 0x00400000U);
        }
    }
    return z;
}

/* tanhf on its common domain, 2^-55 <= |x| < 0x1.f310e4p+2, where the
 * expm1f argument v = +-2|x| reduces with k <= 22: (v in [2, 15.6) for
 * |x| >= 1, k in [3, 22]; v in (-2, -2^-54] below, k in [-3, 0]).
 * The same operations as m3_tanhf_straight, arranged to share work:
 *   - k is round(v / ln2) as expm1f forms it for |v| >= 1.5 ln2, for every
 *     v here; on the ranges where expm1f fixes k = 0 or k = -1 instead,
 *     the rounded form gives the same k (and, at the one v, -0x1.62e43p-2,
 *     where it gives -1 for 0, the k = -1 reconstruction gives the same
 *     bits), so no selection of k is needed;
 *   - k ln2_hi is exact (ln2_hi has 17 significant bits, |k| < 64), so
 *     v - k ln2_hi is one fused operation with the same result;
 *   - with c = 0 (k = 0) expm1f's x * (e - c) - c - hxs is x * e - hxs,
 *     so its k = 0 result x - (x * e - hxs) is d = x - f, the value every
 *     other reconstruction starts from: 0.5 (x - f) - 0.5 (k = -1, with
 *     0.5 d exact, one fused operation), 1 - (f - x) = 1 + d (k <= -2,
 *     then scaled by 2^k and less 1) and (1 - 2^-k) - (f - x) (3 <= k <=
 *     22, then scaled by 2^k).
 * Every input of the domain gives m3_tanhf's bits (checked against the C
 * library on all of them on the host, and on the device with the one-step
 * divisions, whose operands here are m3_tanhf_straight's). */
M3_HD float m3_tanhf_common(float x)
{
    const float ln2_hi = 6.9313812256e-01F;
    const float ln2_lo = 9.0580006145e-06F;
    const float invln2 = 1.4426950216e+00F;
    const float q1 = -3.3333335072e-02F;
    const float q2 = 1.5873016091e-03F;
    const float q3 = -7.9365076090e-05F;
    const float q4 = 4.0082177293e-06F;
    const float q5 = -2.0109921195e-07F;
    const uint32_t jx = m3_f32_bits(x);
    const uint32_t ix = jx & 0x7fffffffU;
    const int big = ix >= 0x3f800000U;
    /* |x| clamped at 22 on its bits, so that the lanes outside the domain
     * (their results are replaced) keep k in range */
    const float magnitude = m3_bits_f32(ix < 0x41b00000U ? ix : 0x41b00000U);
    const float v = (big ? 2.0F : -2.0F) * magnitude;
    /* +-0.5 with v's sign */
    const float half = m3_bits_f32(0x3f000000U | (m3_f32_bits(v) &
                                                  0x80000000U));
    const int32_t k = (int32_t)(invln2 * v + half);
    const float kf = (float)k;
    const float hi = fmaf(-kf, ln2_hi, v);
    const float lo = kf * ln2_lo;
    const float r = hi - lo;
    const float c = (hi - r) - lo;
    const float hfx = 0.5F * r;
    const float hxs = r * hfx;
    const float r1 =
        1.0F + hxs * (q1 + hxs * (q2 + hxs * (q3 + hxs * (q4 + hxs * q5))));
    const float t = 3.0F - r1 * hfx;
    const float e = hxs * m3_div_one_step(r1 - t, 6.0F - r * t);
    float f = r * (e - c) - c;

    f -= hxs;
    const float d = r - f;
    /* 1 - 2^-k for k >= 3 and 1 for k <= -2 (the shift by 32 + k leaves
     * nothing; k = 0 and k = -1 do not use it), scaled by 2^k on the
     * bits */
    const float base =
        m3_bits_f32(0x3f800000U - (0x1000000U >> ((uint32_t)k & 31U)));
    const float scaled =
        m3_bits_f32(m3_f32_bits(base + d) + ((uint32_t)k << 23U));
    const float outer = scaled - 1.0F;
    const float em1 = big ? scaled
                      : k < -1 ? outer
                      : k == -1 ? fmaf(0.5F, d, -0.5F)
                                : d;
    const float q = m3_div_one_step(big ? 2.0F : -em1, em1 + 2.0F);
    const float z = big ? 1.0F - q : q; /* +0 or positive */

    /* z's magnitude with x's sign, as one bit-field insert */
    return m3_bits_f32((m3_f32_bits(z) & 0x7fffffffU) |
                       (jx & 0x80000000U));
}

/* The C library's tanhf for every input: m3_tanhf_common, and
 * m3_tanhf_straight for the inputs outside its domain (|x| from 7.8 on,
 * infinities and NaN, |x| below 2^-55), formed only in a wave that has
 * such an input. */
M3_HD float m3_tanhf_uniform(float x)
{
    const uint32_t ix = m3_f32_bits(x) & 0x7fffffffU;
    const int rare = ix - 0x24000000U >= 0x40f98872U - 0x24000000U;
    float z = m3_tanhf_common(x);

    if (M3_ANY_LANE(rare)) {
        const float straight = m3_tanhf_straight(x);

        z = rare ? straight : z;
    }
    return z;
}

#endif
