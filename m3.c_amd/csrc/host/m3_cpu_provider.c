/*
 * m3_cpu_provider.c - the CPU provider: this library's kinds executed on
 * the host, over host-visible storage.
 *
 * The scheduler hands a list here when the caller disabled the GPU
 * provider (allow_metal = false), or for nodes the GPU provider was told
 * to leave to the CPU (M3_HIP_CPU_KINDS, see m3_provider.c); over device
 * storage the session runs such nodes on host mirrors (m3_session.c).
 * Nothing falls back here when the GPU is missing.
 *
 * Semantics are the reference host provider's (src/m3_op_execute_host.c:
 * 5-60, src/m3_op_execute_basic.c:11-215): commands run in list order,
 * each one's data check right before it (softmax input without NaN, a
 * float to I32 cast input finite and in [-2^31, 2^31); OUT_OF_RANGE, and
 * the list stops there). The element functions are the ones the gfx950
 * kernels are compiled from (m3_numeric.h, m3_libm.h, m3_activation.h),
 * so the CPU and GPU providers agree bit for bit; those headers are
 * checked against the reference's own host code over every input.
 *
 * Iteration. An output is contiguous, so its elements are visited in
 * row-major order by a cursor: an odometer over the output's extents that
 * carries a byte offset per operand, each operand's strides aligned to the
 * output's trailing axes with broadcast axes (absent, or of extent 1)
 * stepping 0. Advancing costs one add per operand in the common case; no
 * index is divided.
 */
#include "m3_internal.h"

#include "m3_activation.h"

#include <string.h>

#define M3_CURSOR_OPERANDS 3U

typedef struct {
    uint8_t rank;
    uint64_t extent[M3_TENSOR_MAX_RANK];
    uint64_t at[M3_TENSOR_MAX_RANK];
    size_t step[M3_CURSOR_OPERANDS][M3_TENSOR_MAX_RANK];
    size_t offset[M3_CURSOR_OPERANDS];
    uint32_t operands;
} m3_cursor;

static void m3_cursor_start(m3_cursor *c, uint8_t rank,
                            const uint64_t *extent)
{
    (void)memset(c, 0, sizeof(*c));
    c->rank = rank;
    (void)memcpy(c->extent, extent, (size_t)rank * sizeof(*extent));
}

/* Adds `view` as the next operand, read over the cursor's extents. */
static void m3_cursor_bind(m3_cursor *c, const m3_tensor_view *view)
{
    const uint32_t k = c->operands++;
    const uint8_t lead = (uint8_t)(c->rank - view->metadata.rank);
    uint8_t axis;

    for (axis = lead; axis < c->rank; ++axis) {
        const uint8_t own = (uint8_t)(axis - lead);

        c->step[k][axis] = view->metadata.shape[own] == 1U
                               ? 0U
                               : view->byte_strides[own];
    }
}

static void m3_cursor_advance(m3_cursor *c)
{
    int axis;
    uint32_t k;

    for (axis = (int)c->rank - 1; axis >= 0; --axis) {
        for (k = 0U; k < c->operands; ++k) {
            c->offset[k] += c->step[k][axis];
        }
        if (++c->at[axis] < c->extent[axis]) {
            return;
        }
        for (k = 0U; k < c->operands; ++k) {
            c->offset[k] -= c->step[k][axis] * (size_t)c->extent[axis];
        }
        c->at[axis] = 0U;
    }
}

/* ---- elements ----------------------------------------------------------- */

static const uint8_t *m3_host_in(const m3_tensor_view *view)
{
    return (const uint8_t *)m3_storage_const_data(view->storage) +
           view->byte_offset;
}

static uint8_t *m3_host_out(m3_tensor_view *view)
{
    return (uint8_t *)m3_storage_data(view->storage) + view->byte_offset;
}

static uint32_t m3_raw_at(const uint8_t *at, m3_dtype dtype)
{
    if (m3_dtype_size(dtype) == 4U) {
        uint32_t word;

        (void)memcpy(&word, at, sizeof(word));
        return word;
    } else {
        uint16_t half;

        (void)memcpy(&half, at, sizeof(half));
        return half;
    }
}

static void m3_raw_put(uint8_t *at, m3_dtype dtype, uint32_t raw)
{
    if (m3_dtype_size(dtype) == 4U) {
        (void)memcpy(at, &raw, sizeof(raw));
    } else {
        const uint16_t half = (uint16_t)raw;

        (void)memcpy(at, &half, sizeof(half));
    }
}

static float m3_value_at(const uint8_t *at, m3_dtype dtype)
{
    return m3_bits_f32(m3_load_as_f32_bits(m3_raw_at(at, dtype),
                                           (uint32_t)dtype));
}

static void m3_value_put(uint8_t *at, m3_dtype dtype, uint32_t f32_bits)
{
    m3_raw_put(at, dtype, m3_store_from_f32_bits(f32_bits, (uint32_t)dtype));
}

/* ---- data checks -------------------------------------------------------- */

static bool m3_cpu_any_nan(const m3_tensor_view *view)
{
    const uint8_t *base = m3_host_in(view);
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, view->metadata.rank, view->metadata.shape);
    m3_cursor_bind(&c, view);
    for (e = 0U; e < view->metadata.element_count; ++e) {
        const float v = m3_value_at(base + c.offset[0],
                                    view->metadata.dtype);

        if (v != v) {
            return true;
        }
        m3_cursor_advance(&c);
    }
    return false;
}

static bool m3_cpu_fits_i32(const m3_tensor_view *view)
{
    const uint8_t *base = m3_host_in(view);
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, view->metadata.rank, view->metadata.shape);
    m3_cursor_bind(&c, view);
    for (e = 0U; e < view->metadata.element_count; ++e) {
        const float v = m3_value_at(base + c.offset[0],
                                    view->metadata.dtype);

        /* NaN fails both comparisons */
        if (!(v >= -0x1p31F && v < 0x1p31F)) {
            return false;
        }
        m3_cursor_advance(&c);
    }
    return true;
}

static m3_status m3_cpu_check_data(const m3_command *command,
                                   m3_error *error)
{
    if (command->kind == M3_OP_SOFTMAX &&
        m3_cpu_any_nan(command->descriptor.softmax.input)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "softmax input holds a NaN");
    }
    if (command->kind == M3_OP_CAST &&
        command->descriptor.cast.output->metadata.dtype == M3_DTYPE_I32 &&
        command->descriptor.cast.input->metadata.dtype != M3_DTYPE_I32 &&
        !m3_cpu_fits_i32(command->descriptor.cast.input)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "cast to I32 meets a value that is not finite "
                            "or not in [-2^31, 2^31)");
    }
    return M3_STATUS_OK;
}

/* ---- operations --------------------------------------------------------- */

/* COPY, and CAST: a raw copy between equal dtypes; else through F32, with
 * I32 read as (float)i and written truncated toward zero. */
static void m3_cpu_convert(const m3_tensor_view *in, m3_tensor_view *out)
{
    const uint8_t *src = m3_host_in(in);
    uint8_t *dst = m3_host_out(out);
    const m3_dtype from = in->metadata.dtype;
    const m3_dtype to = out->metadata.dtype;
    const size_t out_size = m3_dtype_size(to);
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, out->metadata.rank, out->metadata.shape);
    m3_cursor_bind(&c, in);
    for (e = 0U; e < out->metadata.element_count; ++e) {
        const uint32_t raw = m3_raw_at(src + c.offset[0], from);

        m3_raw_put(dst + e * out_size, to,
                   from == to ? raw
                              : m3_store_from_f32_bits(
                                    m3_load_as_f32_bits(raw, (uint32_t)from),
                                    (uint32_t)to));
        m3_cursor_advance(&c);
    }
}

static uint32_t m3_cpu_op_code(m3_op_kind kind)
{
    return kind == M3_OP_ADD   ? M3N_ADD
           : kind == M3_OP_MUL ? M3N_MUL
           : kind == M3_OP_SUB ? M3N_SUB
                               : M3N_DIV;
}

static void m3_cpu_binary(uint32_t op, const m3_op_binary *b)
{
    const uint8_t *left = m3_host_in(b->left);
    const uint8_t *right = m3_host_in(b->right);
    uint8_t *dst = m3_host_out(b->output);
    const m3_tensor_metadata *out = &b->output->metadata;
    const size_t out_size = m3_dtype_size(out->dtype);
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, out->rank, out->shape);
    m3_cursor_bind(&c, b->left);
    m3_cursor_bind(&c, b->right);
    for (e = 0U; e < out->element_count; ++e) {
        const uint32_t l = m3_load_as_f32_bits(
            m3_raw_at(left + c.offset[0], b->left->metadata.dtype),
            (uint32_t)b->left->metadata.dtype);
        const uint32_t r = m3_load_as_f32_bits(
            m3_raw_at(right + c.offset[1], b->right->metadata.dtype),
            (uint32_t)b->right->metadata.dtype);

        m3_value_put(dst + e * out_size, out->dtype,
                     m3_binary_f32_bits(op, l, r));
        m3_cursor_advance(&c);
    }
}

/* Softmax of one row of `width` elements `column` bytes apart, into a
 * contiguous output row: maximum and +inf count, the left-to-right F32 sum
 * of expf(v - max), then expf(v - max) / sum; an all -inf row gives
 * zeros, a row whose maximum is +inf gives 1/k on its +inf entries. */
static void m3_cpu_softmax_row(const uint8_t *row, size_t column,
                               m3_dtype in_dtype, uint64_t width,
                               uint8_t *dst, m3_dtype out_dtype)
{
    const size_t out_size = m3_dtype_size(out_dtype);
    float maximum = -INFINITY;
    float sum = 0.0F;
    uint32_t infinities = 0U;
    uint64_t j;

    for (j = 0U; j < width; ++j) {
        const float v = m3_value_at(row + j * column, in_dtype);

        maximum = v > maximum ? v : maximum;
        infinities += v == INFINITY ? 1U : 0U;
    }
    if (maximum == -INFINITY || maximum == INFINITY) {
        const float share = maximum == INFINITY ? 1.0F / (float)infinities
                                                : 0.0F;

        for (j = 0U; j < width; ++j) {
            const float v = m3_value_at(row + j * column, in_dtype);

            m3_value_put(dst + j * out_size, out_dtype,
                         m3_f32_bits(v == INFINITY ? share : 0.0F));
        }
        return;
    }
    for (j = 0U; j < width; ++j) {
        sum = sum + m3_expf_any(m3_value_at(row + j * column, in_dtype) -
                            maximum);
    }
    for (j = 0U; j < width; ++j) {
        const float e = m3_expf_any(m3_value_at(row + j * column, in_dtype) -
                                maximum);

        m3_value_put(dst + j * out_size, out_dtype, m3_f32_bits(e / sum));
    }
}

static void m3_cpu_softmax(const m3_op_unary *op)
{
    const m3_tensor_view *in = op->input;
    const m3_tensor_metadata *meta = &in->metadata;
    const uint8_t last = (uint8_t)(meta->rank - 1U);
    const uint64_t width = meta->shape[last];
    const size_t row_bytes =
        (size_t)width * m3_dtype_size(op->output->metadata.dtype);
    const uint8_t *src = m3_host_in(in);
    uint8_t *dst = m3_host_out(op->output);
    m3_tensor_view row_axes;
    size_t rows;
    size_t r;
    m3_cursor c;

    if (width == 0U) {
        return;
    }
    rows = meta->element_count / (size_t)width;
    /* the cursor walks the rows: every axis but the last */
    row_axes = *in;
    row_axes.metadata.rank = last;
    m3_cursor_start(&c, last, meta->shape);
    m3_cursor_bind(&c, &row_axes);
    for (r = 0U; r < rows; ++r) {
        m3_cpu_softmax_row(src + c.offset[0], in->byte_strides[last],
                           meta->dtype, width, dst + r * row_bytes,
                           op->output->metadata.dtype);
        m3_cursor_advance(&c);
    }
}

/* Snake1d, the reference's seven rounded F32 statements:
 * d = a + 0x1.12e0bep-30; inv = 1 / d; ang = a * x; s = sinf(ang);
 * q = s * s; t = inv * q; y = x + t. */
static void m3_cpu_snake1d(const m3_op_snake1d *op)
{
    const uint8_t *xs = m3_host_in(op->input);
    const uint8_t *alphas = m3_host_in(op->alpha);
    float *out = (float *)(void *)m3_host_out(op->output);
    const m3_tensor_metadata *meta = &op->output->metadata;
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, meta->rank, meta->shape);
    m3_cursor_bind(&c, op->input);
    m3_cursor_bind(&c, op->alpha);
    for (e = 0U; e < meta->element_count; ++e) {
        float x;
        float a;
        float d;
        float inv;
        float ang;
        float s;
        float q;
        float t;
        float y;

        (void)memcpy(&x, xs + c.offset[0], sizeof(x));
        (void)memcpy(&a, alphas + c.offset[1], sizeof(a));
        d = a + m3_bits_f32(0x3089705fU);
        inv = 1.0F / d;
        ang = a * x;
        s = m3_sinf(ang);
        q = s * s;
        t = inv * q;
        y = x + t;
        (void)memcpy(&out[e], &y, sizeof(y));
        m3_cursor_advance(&c);
    }
}

static void m3_cpu_tanh(const m3_op_unary *op)
{
    const uint8_t *src = m3_host_in(op->input);
    float *out = (float *)(void *)m3_host_out(op->output);
    const m3_tensor_metadata *meta = &op->output->metadata;
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, meta->rank, meta->shape);
    m3_cursor_bind(&c, op->input);
    for (e = 0U; e < meta->element_count; ++e) {
        float x;
        float y;

        (void)memcpy(&x, src + c.offset[0], sizeof(x));
        y = m3_tanhf(x);
        (void)memcpy(&out[e], &y, sizeof(y));
        m3_cursor_advance(&c);
    }
}

static void m3_cpu_gated_silu(const m3_op_binary *op)
{
    const uint8_t *gates = m3_host_in(op->left);
    const uint8_t *ups = m3_host_in(op->right);
    uint8_t *dst = m3_host_out(op->output);
    const m3_tensor_metadata *meta = &op->output->metadata;
    const m3_dtype gate_dtype = op->left->metadata.dtype;
    const m3_dtype up_dtype = op->right->metadata.dtype;
    const size_t out_size = m3_dtype_size(meta->dtype);
    m3_cursor c;
    size_t e;

    m3_cursor_start(&c, meta->rank, meta->shape);
    m3_cursor_bind(&c, op->left);
    m3_cursor_bind(&c, op->right);
    for (e = 0U; e < meta->element_count; ++e) {
        const float gate = m3_value_at(gates + c.offset[0], gate_dtype);
        const float up = m3_value_at(ups + c.offset[1], up_dtype);

        m3_value_put(dst + e * out_size, meta->dtype,
                     m3_gated_silu_bits(gate, up, (uint32_t)gate_dtype));
        m3_cursor_advance(&c);
    }
}

bool m3_cpu_kind_supported(m3_op_kind kind)
{
    return m3_op_kind_supported(kind);
}

/* Every operand of `command` is host memory. */
static bool m3_cpu_reachable(const m3_command *command)
{
    const m3_tensor_view *views[3] = {NULL, NULL, NULL};
    const m3_op_binary *binary = m3_op_binary_of(command);
    size_t k;

    if (binary != NULL) {
        views[0] = binary->left;
        views[1] = binary->right;
        views[2] = binary->output;
    } else if (command->kind == M3_OP_SNAKE1D) {
        views[0] = command->descriptor.snake1d.input;
        views[1] = command->descriptor.snake1d.alpha;
        views[2] = command->descriptor.snake1d.output;
    } else if (command->kind == M3_OP_GATED_SILU) {
        views[0] = command->descriptor.gated_silu.left;
        views[1] = command->descriptor.gated_silu.right;
        views[2] = command->descriptor.gated_silu.output;
    } else {
        /* COPY, CAST, SOFTMAX and TANH share the unary layout */
        views[0] = command->descriptor.copy.input;
        views[2] = command->descriptor.copy.output;
    }
    for (k = 0U; k < 3U; ++k) {
        if (views[k] != NULL && views[k]->metadata.element_count != 0U &&
            !m3_storage_host_visible(views[k]->storage)) {
            return false;
        }
    }
    return true;
}

m3_status m3_cpu_execute(const m3_command *commands, size_t count,
                         m3_error *error)
{
    size_t i;

    for (i = 0U; i < count; ++i) {
        const m3_command *command = &commands[i];
        m3_status status;

        if (!m3_cpu_kind_supported(command->kind)) {
            return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                                "the CPU provider has no kind %d",
                                (int)command->kind);
        }
        if (!m3_cpu_reachable(command)) {
            return m3_error_set(error, M3_STATUS_INTERNAL,
                                "the CPU provider was given device memory");
        }
        status = m3_cpu_check_data(command, error);
        if (status != M3_STATUS_OK) {
            return status;
        }
        switch (command->kind) {
        case M3_OP_COPY:
            m3_cpu_convert(command->descriptor.copy.input,
                           command->descriptor.copy.output);
            break;
        case M3_OP_CAST:
            m3_cpu_convert(command->descriptor.cast.input,
                           command->descriptor.cast.output);
            break;
        case M3_OP_SOFTMAX:
            m3_cpu_softmax(&command->descriptor.softmax);
            break;
        case M3_OP_SNAKE1D:
            m3_cpu_snake1d(&command->descriptor.snake1d);
            break;
        case M3_OP_TANH:
            m3_cpu_tanh(&command->descriptor.tanh);
            break;
        case M3_OP_GATED_SILU:
            m3_cpu_gated_silu(&command->descriptor.gated_silu);
            break;
        default:
            m3_cpu_binary(m3_cpu_op_code(command->kind),
                          m3_op_binary_of(command));
            break;
        }
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}
