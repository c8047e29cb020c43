/*
 * m3_oracle.c - CPU restatement of the reference's host tensor ops.
 *
 * TEST INFRASTRUCTURE ONLY: what the tests compare the HIP provider with;
 * never part of the product. Built with -ffp-contract=off and without -ffast-math, as
 * the reference asks for (Makefile:7 builds with clang -O3 and no fast-math;
 * src/m3_op_execute_basic.c:182 turns contraction off for Snake1d).
 * Transcendentals are the platform libm's expf/sinf, which is what the
 * reference calls (src/m3_op_execute_basic.c:156,172,188).
 */
#include "m3_oracle.h"

#include <math.h>
#include <string.h>

static uint32_t bits_of(float value)
{
    uint32_t bits;

    memcpy(&bits, &value, sizeof(bits));
    return bits;
}

static float float_of(uint32_t bits)
{
    float value;

    memcpy(&value, &bits, sizeof(value));
    return value;
}

/* src/m3_op_numeric.c:27-53: exact widening; subnormals are normalised by
 * shifting until the hidden bit appears; Inf/NaN keep their fraction. */
uint32_t oracle_f16_to_f32(uint16_t half)
{
    uint32_t sign = ((uint32_t)half & 0x8000U) << 16;
    uint32_t exponent = ((uint32_t)half >> 10) & 0x1fU;
    uint32_t fraction = (uint32_t)half & 0x3ffU;

    if (exponent == 0U) {
        uint32_t biased = 113U;

        if (fraction == 0U) {
            return sign;
        }
        while ((fraction & 0x400U) == 0U) {
            fraction <<= 1;
            biased -= 1U;
        }
        return sign | (biased << 23) | ((fraction & 0x3ffU) << 13);
    }
    if (exponent == 31U) {
        return sign | 0x7f800000U | (fraction << 13);
    }
    return sign | ((exponent + 112U) << 23) | (fraction << 13);
}

/* src/m3_op_numeric.c:55-112: round to nearest even, NaN keeps the top
 * fraction bits with the quiet bit set (at least one payload bit), values
 * past the F16 range become infinity, small values round into subnormals. */
uint16_t oracle_f32_to_f16(uint32_t bits)
{
    uint32_t sign = (bits >> 16) & 0x8000U;
    uint32_t exponent = (bits >> 23) & 0xffU;
    uint32_t fraction = bits & 0x7fffffU;
    int e = (int)exponent - 127;

    if (exponent == 0xffU) {
        uint32_t kept;

        if (fraction == 0U) {
            return (uint16_t)(sign | 0x7c00U);
        }
        kept = fraction >> 13;
        if (kept == 0U) {
            kept = 1U;
        }
        return (uint16_t)(sign | 0x7c00U | 0x200U | kept);
    }
    if (e > 15) {
        return (uint16_t)(sign | 0x7c00U);
    }
    if (e >= -14) {
        uint32_t mantissa = fraction >> 13;
        uint32_t dropped = fraction & 0x1fffU;
        uint32_t biased = (uint32_t)(e + 15);

        if (dropped > 0x1000U || (dropped == 0x1000U && (mantissa & 1U))) {
            mantissa += 1U;
            if (mantissa == 0x400U) {
                mantissa = 0U;
                biased += 1U;
            }
        }
        if (biased >= 31U) {
            return (uint16_t)(sign | 0x7c00U);
        }
        return (uint16_t)(sign | (biased << 10) | mantissa);
    }
    if (e >= -25) {
        uint32_t significand = fraction | 0x800000U;
        uint32_t shift = (uint32_t)(-e - 1);
        uint32_t mantissa = significand >> shift;
        uint32_t dropped = significand & ((1U << shift) - 1U);
        uint32_t half_way = 1U << (shift - 1U);

        if (dropped > half_way ||
            (dropped == half_way && (mantissa & 1U))) {
            mantissa += 1U;
        }
        return (uint16_t)(sign | mantissa);
    }
    return (uint16_t)sign;
}

/* src/m3_op_numeric.c:114-117. */
uint32_t oracle_bf16_to_f32(uint16_t brain)
{
    return (uint32_t)brain << 16;
}

/* src/m3_op_numeric.c:119-130: NaN keeps its top half with 0x0040 set;
 * everything else rounds to nearest even by adding 0x7fff plus the kept
 * lowest bit. */
uint16_t oracle_f32_to_bf16(uint32_t bits)
{
    if ((bits & 0x7f800000U) == 0x7f800000U && (bits & 0x7fffffU) != 0U) {
        return (uint16_t)((bits >> 16) | 0x40U);
    }
    bits += 0x7fffU + ((bits >> 16) & 1U);
    return (uint16_t)(bits >> 16);
}

static size_t element_size(uint32_t dtype)
{
    return dtype == ORACLE_F16 || dtype == ORACLE_BF16 ? 2U : 4U;
}

static uint64_t element_count(const oracle_view *view)
{
    uint64_t count = 1U;
    uint32_t axis;

    for (axis = 0U; axis < view->rank; ++axis) {
        count *= view->shape[axis];
    }
    return count;
}

/* src/m3_op_numeric.c:132-148: row-major flat index -> byte offset. */
static uint64_t element_offset(const oracle_view *view, uint64_t flat)
{
    uint64_t offset = view->byte_offset;
    uint32_t axis = view->rank;

    while (axis > 0U) {
        axis -= 1U;
        offset += (flat % view->shape[axis]) * view->byte_strides[axis];
        flat /= view->shape[axis];
    }
    return offset;
}

/* src/m3_op_numeric.c:150-174: offset of the input element that broadcasts
 * onto output element `flat` (right-aligned; size-1 axes repeat). */
static uint64_t broadcast_offset(const oracle_view *input,
                                 const oracle_view *output, uint64_t flat)
{
    uint64_t offset = input->byte_offset;
    uint32_t axis = output->rank;
    int lead = (int)output->rank - (int)input->rank;

    while (axis > 0U) {
        uint64_t coordinate;
        int input_axis;

        axis -= 1U;
        coordinate = flat % output->shape[axis];
        flat /= output->shape[axis];
        input_axis = (int)axis - lead;
        if (input_axis >= 0 && input->shape[input_axis] != 1U) {
            offset += coordinate * input->byte_strides[input_axis];
        }
    }
    return offset;
}

/* src/m3_op_numeric.c:176-208: typed load as F32 (I32 converts). */
static float load_float(const oracle_view *view, uint64_t offset)
{
    const uint8_t *p = (const uint8_t *)view->data + offset;

    if (view->dtype == ORACLE_F32) {
        float v;

        memcpy(&v, p, sizeof(v));
        return v;
    }
    if (view->dtype == ORACLE_I32) {
        int32_t v;

        memcpy(&v, p, sizeof(v));
        return (float)v;
    }
    {
        uint16_t h;

        memcpy(&h, p, sizeof(h));
        return float_of(view->dtype == ORACLE_F16 ? oracle_f16_to_f32(h)
                                                  : oracle_bf16_to_f32(h));
    }
}

/* src/m3_op_numeric.c:224-243: typed store from F32 (I32 truncates). */
static void store_float(const oracle_view *view, uint64_t offset, float value)
{
    uint8_t *p = (uint8_t *)view->data + offset;

    if (view->dtype == ORACLE_F32) {
        memcpy(p, &value, sizeof(value));
    } else if (view->dtype == ORACLE_I32) {
        int32_t v = (int32_t)value;

        memcpy(p, &v, sizeof(v));
    } else {
        uint16_t h = view->dtype == ORACLE_F16
                         ? oracle_f32_to_f16(bits_of(value))
                         : oracle_f32_to_bf16(bits_of(value));

        memcpy(p, &h, sizeof(h));
    }
}

/* src/m3_op_execute_basic.c:61-77 (ADD/MUL); SUB and DIV are the same
 * loop with the other IEEE operations. */
int oracle_binary(uint32_t op, const oracle_view *left,
                  const oracle_view *right, const oracle_view *output)
{
    uint64_t count = element_count(output);
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        float a = load_float(left, broadcast_offset(left, output, i));
        float b = load_float(right, broadcast_offset(right, output, i));
        float r;

        switch (op) {
        case ORACLE_ADD:
            r = a + b;
            break;
        case ORACLE_MUL:
            r = a * b;
            break;
        case ORACLE_SUB:
            r = a - b;
            break;
        default:
            r = a / b;
            break;
        }
        store_float(output, element_offset(output, i), r);
    }
    return 0;
}

/* src/m3_op_execute_basic.c:11-26: element-wise byte copy. */
int oracle_copy(const oracle_view *input, const oracle_view *output)
{
    uint64_t count = element_count(input);
    size_t size = element_size(input->dtype);
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        memmove((uint8_t *)output->data + element_offset(output, i),
                (const uint8_t *)input->data + element_offset(input, i),
                size);
    }
    return 0;
}

/* src/m3_op_execute_basic.c:28-59. */
int oracle_cast(const oracle_view *input, const oracle_view *output)
{
    uint64_t count = element_count(input);
    uint64_t i;

    if (input->dtype == output->dtype) {
        return oracle_copy(input, output);
    }
    for (i = 0U; i < count; ++i) {
        uint64_t from = element_offset(input, i);
        uint64_t to = element_offset(output, i);

        if (input->dtype == ORACLE_I32) {
            int32_t v;

            memcpy(&v, (const uint8_t *)input->data + from, sizeof(v));
            store_float(output, to, (float)v);
        } else {
            store_float(output, to, load_float(input, from));
        }
    }
    return 0;
}

/* src/m3_op_execute_basic.c:124-180: three passes per row. */
int oracle_softmax(const oracle_view *input, const oracle_view *output)
{
    uint64_t total = element_count(input);
    uint64_t width = input->shape[input->rank - 1U];
    uint64_t row;

    for (row = 0U; width != 0U && row < total / width; ++row) {
        float maximum = -INFINITY;
        float sum = 0.0F;
        uint64_t infinities = 0U;
        uint64_t c;

        for (c = 0U; c < width; ++c) {
            float v = load_float(input, element_offset(input, row * width + c));

            if (v > maximum) {
                maximum = v;
            }
            if (v == INFINITY) {
                infinities += 1U;
            }
        }
        if (maximum != -INFINITY && maximum != INFINITY) {
            for (c = 0U; c < width; ++c) {
                float v = load_float(input,
                                     element_offset(input, row * width + c));

                sum += expf(v - maximum);
            }
        }
        for (c = 0U; c < width; ++c) {
            uint64_t flat = row * width + c;
            float v = load_float(input, element_offset(input, flat));
            float p;

            if (maximum == -INFINITY) {
                p = 0.0F;
            } else if (maximum == INFINITY) {
                p = v == INFINITY ? 1.0F / (float)infinities : 0.0F;
            } else {
                p = expf(v - maximum) / sum;
            }
            store_float(output, element_offset(output, flat), p);
        }
    }
    return 0;
}

/* src/m3_op_execute_basic.c:182-215: seven rounded F32 statements. */
#pragma STDC FP_CONTRACT OFF
static float snake_value(float x, float a)
{
    volatile float denominator = a + 0x1.12e0bep-30F;
    volatile float inverse = 1.0F / denominator;
    volatile float angle = a * x;
    volatile float sine = sinf(angle);
    volatile float square = sine * sine;
    volatile float scaled = inverse * square;
    volatile float result = x + scaled;

    return result;
}

int oracle_snake1d(const oracle_view *input, const oracle_view *alpha,
                   const oracle_view *output)
{
    uint64_t count = element_count(input);
    uint64_t length = input->shape[2];
    uint64_t channels = input->shape[1];
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        uint64_t channel = (i / length) % channels;
        float x = load_float(input, element_offset(input, i));
        float a = load_float(alpha, element_offset(alpha, channel));

        store_float(output, element_offset(output, i), snake_value(x, a));
    }
    return 0;
}

/* src/m3_op_numeric.c:210-222: F32 rounded through a 16-bit dtype and
 * back (identity for F32). */
static float round_to_dtype(uint32_t dtype, float value)
{
    if (dtype == ORACLE_F16) {
        return float_of(oracle_f16_to_f32(oracle_f32_to_f16(bits_of(value))));
    }
    if (dtype == ORACLE_BF16) {
        return float_of(
            oracle_bf16_to_f32(oracle_f32_to_bf16(bits_of(value))));
    }
    return dtype == ORACLE_F32 ? value : NAN;
}

/* src/m3_op_execute_basic.c:104-122: activation = gate / (1 + expf(-gate))
 * rounded to the gate's dtype, times up, stored in the output's dtype. */
int oracle_gated_silu(const oracle_view *gate, const oracle_view *up,
                      const oracle_view *output)
{
    uint64_t count = element_count(output);
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        float g = load_float(gate, element_offset(gate, i));
        float u = load_float(up, element_offset(up, i));
        float activation = round_to_dtype(gate->dtype,
                                          g / (1.0F + expf(-g)));
        float result = activation * u;

        store_float(output, element_offset(output, i), result);
    }
    return 0;
}

/* src/m3_op_execute_basic.c:217-229: tanhf of every element. */
int oracle_tanh(const oracle_view *input, const oracle_view *output)
{
    uint64_t count = element_count(input);
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        store_float(output, element_offset(output, i),
                    tanhf(load_float(input, element_offset(input, i))));
    }
    return 0;
}

/* src/m3_op_data_preflight.c:48-64. */
int oracle_preflight_nan(const oracle_view *view)
{
    uint64_t count = element_count(view);
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        if (isnan(load_float(view, element_offset(view, i)))) {
            return 2;
        }
    }
    return 0;
}

/* src/m3_op_data_preflight.c:8-28. */
int oracle_preflight_i32(const oracle_view *view)
{
    uint64_t count = element_count(view);
    uint64_t i;

    for (i = 0U; i < count; ++i) {
        float v = load_float(view, element_offset(view, i));

        if (!isfinite(v) || v < -2147483648.0F || v >= 2147483648.0F) {
            return 2;
        }
    }
    return 0;
}

void oracle_f32_to_f16_array(const uint32_t *in, uint16_t *out, size_t n)
{
    size_t i;

    for (i = 0U; i < n; ++i) {
        out[i] = oracle_f32_to_f16(in[i]);
    }
}

void oracle_f16_to_f32_array(const uint16_t *in, uint32_t *out, size_t n)
{
    size_t i;

    for (i = 0U; i < n; ++i) {
        out[i] = oracle_f16_to_f32(in[i]);
    }
}

void oracle_f32_to_bf16_array(const uint32_t *in, uint16_t *out, size_t n)
{
    size_t i;

    for (i = 0U; i < n; ++i) {
        out[i] = oracle_f32_to_bf16(in[i]);
    }
}
