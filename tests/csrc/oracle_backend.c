/*
 * oracle_backend.c - TEST INFRASTRUCTURE: an m3 backend over host memory
 * whose execute hook evaluates commands with the oracle.
 *
 * Registered through m3_provider_set_gpu_factory, it stands in for the HIP
 * device on machines without a GPU so that the graph compiler, liveness
 * planner, scheduler and session I/O of libm3.so can be tested on the CPU.
 * It reports itself as M3_BACKEND_HIP so the scheduler treats it as the GPU
 * provider, records every executed list, and is never part of the product.
 * Elementwise programs (the session compiler's fused runs) are interpreted
 * from their words, whose operand addresses are host addresses here, with
 * the oracle's binary operation for each F32 operation; the words in
 * storage must equal the host copy.
 */
#include "m3_backend.h"
#include "m3_oracle.h"

#include <stdlib.h>
#include <string.h>

#define ORACLE_BACKEND_LOG 4096

typedef struct {
    int marker;
} oracle_backend_context;

static int g_log_kinds[ORACLE_BACKEND_LOG];
static int g_log_lists[ORACLE_BACKEND_LOG];
static size_t g_log_count;
static size_t g_list_count;
static size_t g_allocations;
static size_t g_fail_allocation_at; /* 0: never */
static size_t g_reserved;
static size_t g_programs;
static size_t g_periodic; /* periodic operands of the programs run */
/* Programs run their elements in increasing order, or in decreasing order
 * when set: a device runs a program's lanes in no fixed order, and a
 * store that lands on bytes another element still reads changes the
 * result in one of the two. */
static int g_decreasing;
/* When set, backends made afterwards declare their memory device memory
 * (write/read hooks, which copy and count): the session then runs CPU
 * provider nodes on host mirrors, as it does over HIP memory. */
static int g_device_memory;
/* When nonzero, the constructor makes nothing and returns this status, as
 * a GPU backend does on a machine without a usable device. */
static int g_create_status;
/* When nonzero, the list with this number (1 = the first one executed
 * after the reset) runs its commands and then fails with g_fail_status, as
 * a device error that surfaces when the list's completion is awaited. */
static size_t g_fail_list_at;
static int g_fail_status;
static size_t g_host_to_device;
static size_t g_device_to_host;

void oracle_backend_reset(void);
size_t oracle_backend_log(int *kinds, int *lists, size_t capacity);
size_t oracle_backend_lists(void);
size_t oracle_backend_reserved(void);
void oracle_backend_fail_allocation_at(size_t index);
size_t oracle_backend_programs(void);
size_t oracle_backend_periodic(void);
void oracle_backend_set_program_order(int decreasing);
void oracle_backend_set_device_memory(int on);
void oracle_backend_set_create_status(int status);
void oracle_backend_fail_list_at(size_t list, int status);
size_t oracle_backend_transfers(int to_device);
m3_status oracle_backend_create(m3_backend **backend, m3_error *error);

void oracle_backend_reset(void)
{
    g_log_count = 0U;
    g_list_count = 0U;
    g_allocations = 0U;
    g_fail_allocation_at = 0U;
    g_reserved = 0U;
    g_programs = 0U;
    g_periodic = 0U;
    g_host_to_device = 0U;
    g_device_to_host = 0U;
    g_create_status = 0;
    g_fail_list_at = 0U;
    g_fail_status = 0;
}

void oracle_backend_set_create_status(int status)
{
    g_create_status = status;
}

void oracle_backend_fail_list_at(size_t list, int status)
{
    g_fail_list_at = list;
    g_fail_status = status;
}

void oracle_backend_set_program_order(int decreasing)
{
    g_decreasing = decreasing;
}

void oracle_backend_set_device_memory(int on)
{
    g_device_memory = on;
}

size_t oracle_backend_transfers(int to_device)
{
    return to_device ? g_host_to_device : g_device_to_host;
}

size_t oracle_backend_programs(void)
{
    return g_programs;
}

size_t oracle_backend_periodic(void)
{
    return g_periodic;
}

size_t oracle_backend_log(int *kinds, int *lists, size_t capacity)
{
    size_t i;

    for (i = 0U; i < g_log_count && i < capacity; ++i) {
        kinds[i] = g_log_kinds[i];
        lists[i] = g_log_lists[i];
    }
    return g_log_count;
}

size_t oracle_backend_lists(void)
{
    return g_list_count;
}

size_t oracle_backend_reserved(void)
{
    return g_reserved;
}

void oracle_backend_fail_allocation_at(size_t index)
{
    g_fail_allocation_at = index;
}

static void destroy(void *context)
{
    free(context);
}

static m3_status allocate(void *context, size_t byte_count, size_t alignment,
                          void **handle, void **data, m3_error *error)
{
    size_t size = (byte_count + alignment - 1U) / alignment * alignment;
    void *memory;

    (void)context;
    *handle = NULL;
    *data = NULL;
    g_allocations += 1U;
    if (g_fail_allocation_at != 0U && g_allocations == g_fail_allocation_at) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "injected allocation failure");
    }
    if (byte_count == 0U) {
        return M3_STATUS_OK;
    }
    memory = aligned_alloc(alignment, size);
    if (memory == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY, "no memory");
    }
    memset(memory, 0, size);
    *handle = memory;
    *data = memory;
    return M3_STATUS_OK;
}

static void free_storage(void *context, void *handle, void *data)
{
    (void)context;
    (void)data;
    free(handle);
}

static m3_status reserve(void *context, size_t byte_count, m3_error *error)
{
    (void)context;
    (void)error;
    g_reserved += byte_count;
    return M3_STATUS_OK;
}

static void to_oracle(const m3_tensor_view *view, oracle_view *out)
{
    uint8_t axis;

    memset(out, 0, sizeof(*out));
    out->data = m3_storage_device_data(view->storage);
    out->byte_offset = view->byte_offset;
    out->dtype = (uint32_t)view->metadata.dtype;
    out->rank = view->metadata.rank;
    for (axis = 0U; axis < view->metadata.rank; ++axis) {
        out->shape[axis] = view->metadata.shape[axis];
        out->byte_strides[axis] = view->byte_strides[axis];
    }
}

/* One F32 operation through the oracle, on one-element views. */
static uint32_t oracle_op1(uint32_t op, uint32_t a, uint32_t b)
{
    uint32_t values[3] = {a, b, 0U};
    oracle_view v[3];
    int k;

    for (k = 0; k < 3; ++k) {
        memset(&v[k], 0, sizeof(v[k]));
        v[k].data = &values[k];
        v[k].dtype = ORACLE_F32;
        v[k].rank = 1U;
        v[k].shape[0] = 1U;
        v[k].byte_strides[0] = 4U;
    }
    (void)oracle_binary(op, &v[0], &v[1], &v[2]);
    return values[2];
}

static uint8_t *operand_address(const uint32_t *operands, uint32_t index)
{
    uint64_t low = operands[2U * index];
    uint64_t high = operands[2U * index + 1U] & 0x3fffffffU;

    return (uint8_t *)(uintptr_t)(((high << 32U) | low) & ~(uint64_t)1U);
}

/* Period of operand `index` from the period table (pairs of operand index
 * and period), 0 when it is not periodic. */
static uint64_t operand_period(const uint32_t *periods, uint32_t period_count,
                               uint32_t index)
{
    uint32_t k;

    for (k = 0U; k < period_count; ++k) {
        if (periods[2U * k] == index) {
            return periods[2U * k + 1U];
        }
    }
    return 0U;
}

/* Element e of operand `index` as F32 bits, converted from its dtype (bits
 * 30-31 of the high word) with the oracle's converters; a periodic operand
 * is read at e mod its period. */
static uint32_t operand_load(const uint32_t *operands, const uint32_t *periods,
                             uint32_t period_count, uint32_t index,
                             uint64_t e)
{
    const uint8_t *base = operand_address(operands, index);
    const uint64_t period = operand_period(periods, period_count, index);
    uint32_t dtype = operands[2U * index + 1U] >> 30U;
    uint16_t half;
    uint32_t bits;

    e = period != 0U ? e % period : e;
    if (dtype == ORACLE_F32) {
        memcpy(&bits, base + 4U * e, sizeof(bits));
        return bits;
    }
    memcpy(&half, base + 2U * e, sizeof(half));
    return dtype == ORACLE_F16 ? oracle_f16_to_f32(half)
                               : oracle_bf16_to_f32(half);
}

static void operand_store(const uint32_t *operands, uint32_t index,
                          uint64_t e, uint32_t bits)
{
    uint8_t *base = operand_address(operands, index);
    uint32_t dtype = operands[2U * index + 1U] >> 30U;
    uint16_t half;

    if (dtype == ORACLE_F32) {
        memcpy(base + 4U * e, &bits, sizeof(bits));
        return;
    }
    half = dtype == ORACLE_F16 ? oracle_f32_to_f16(bits)
                               : oracle_f32_to_bf16(bits);
    memcpy(base + 2U * e, &half, sizeof(half));
}

/* F32 bits stored to `dtype` and loaded back. */
static uint32_t round_through(uint32_t bits, uint32_t dtype)
{
    return dtype == ORACLE_F16    ? oracle_f16_to_f32(oracle_f32_to_f16(bits))
           : dtype == ORACLE_BF16 ? oracle_bf16_to_f32(
                                        oracle_f32_to_bf16(bits))
                                  : bits;
}

/* Runs an elementwise program (layout in m3_hip.h) element by element, in
 * the order g_decreasing selects. */
static int run_program(const m3_op_elementwise_program *program)
{
    const uint32_t *words = program->words;
    const uint32_t operand_count = words[1];
    const uint32_t code_words = words[2];
    const uint64_t count = (uint64_t)words[3] | ((uint64_t)words[4] << 32U);
    const uint32_t period_count = words[5];
    const uint32_t *operands = words + 8;
    const uint32_t *periods = operands + 2U * operand_count;
    const uint32_t *code = periods + 2U * period_count;
    const uint8_t *stored =
        (const uint8_t *)m3_storage_device_data(program->storage);
    uint64_t i;

    if (stored == NULL ||
        memcmp(stored + program->byte_offset, words,
               program->word_count * sizeof(uint32_t)) != 0 ||
        program->word_count !=
            8U + 2U * operand_count + 2U * period_count + code_words) {
        return (int)M3_STATUS_INTERNAL;
    }
    for (i = 0U; i < count; ++i) {
        const uint64_t e = g_decreasing ? count - 1U - i : i;
        uint32_t r[4] = {0U, 0U, 0U, 0U};
        uint32_t f[4] = {0U, 0U, 0U, 0U};
        uint32_t pc = 0U;

        while (pc < code_words) {
            uint32_t w = code[pc];

            if ((w & 3U) == 0U) { /* FETCH */
                uint32_t n = ((w >> 2U) & 3U) + 1U;
                uint32_t k;

                for (k = 0U; k < n; ++k) {
                    f[k] = operand_load(operands, periods, period_count,
                                        (code[pc + 1U] >> (8U * k)) & 0xffU,
                                        e);
                }
                pc += 2U;
            } else if ((w & 3U) == 1U || (w & 3U) == 3U) { /* OP, ROUND */
                int binary = (w & 3U) == 1U;
                uint32_t kinds[2] = {(w >> 8U) & 15U, (w >> 12U) & 15U};
                uint32_t x[2] = {0U, 0U};
                int k;

                for (k = 0; k < (binary ? 2 : 1); ++k) {
                    x[k] = kinds[k] < 4U   ? r[kinds[k]]
                           : kinds[k] < 8U ? f[kinds[k] - 4U]
                                           : operand_load(
                                                 operands, periods,
                                                 period_count,
                                                 (w >> 16U) & 0xffU, 0U);
                }
                r[(w >> 4U) & 3U] = round_through(
                    binary ? oracle_op1((w >> 2U) & 3U, x[0], x[1]) : x[0],
                    (w >> 24U) & 3U);
                pc += 1U;
            } else { /* STORE */
                operand_store(operands, (w >> 8U) & 0xffU, e,
                              r[(w >> 4U) & 3U]);
                pc += 1U;
            }
        }
    }
    g_programs += 1U;
    g_periodic += period_count;
    return 0;
}

static m3_status execute(void *context, const m3_command *commands,
                         size_t count, m3_scratch_arena *scratch,
                         m3_error *error)
{
    size_t i;

    (void)context;
    (void)scratch;
    for (i = 0U; i < count; ++i) {
        const m3_command *c = &commands[i];
        oracle_view a;
        oracle_view b;
        oracle_view o;
        int status = 0;

        if (c->kind == M3_OP_ELEMENTWISE_PROGRAM) {
            const m3_op_elementwise_program *program =
                &c->descriptor.elementwise_program;
            size_t k;

            /* the log lists the fused commands, in order */
            for (k = 0U; k < program->command_count &&
                         g_log_count < ORACLE_BACKEND_LOG;
                 ++k) {
                g_log_kinds[g_log_count] = (int)program->commands[k].kind;
                g_log_lists[g_log_count] = (int)g_list_count;
                g_log_count += 1U;
            }
            if (run_program(program) != 0) {
                return m3_error_set(error, M3_STATUS_INTERNAL,
                                    "oracle backend: malformed program");
            }
            continue;
        }
        if (g_log_count < ORACLE_BACKEND_LOG) {
            g_log_kinds[g_log_count] = (int)c->kind;
            g_log_lists[g_log_count] = (int)g_list_count;
            g_log_count += 1U;
        }
        switch (c->kind) {
        case M3_OP_ADD:
        case M3_OP_MUL:
        case M3_OP_SUB:
        case M3_OP_DIV: {
            const m3_op_binary *op = &c->descriptor.add;
            uint32_t code = c->kind == M3_OP_ADD   ? ORACLE_ADD
                            : c->kind == M3_OP_MUL ? ORACLE_MUL
                            : c->kind == M3_OP_SUB ? ORACLE_SUB
                                                   : ORACLE_DIV;

            to_oracle(op->left, &a);
            to_oracle(op->right, &b);
            to_oracle(op->output, &o);
            status = oracle_binary(code, &a, &b, &o);
            break;
        }
        case M3_OP_COPY:
        case M3_OP_CAST:
            to_oracle(c->descriptor.cast.input, &a);
            to_oracle(c->descriptor.cast.output, &o);
            status = oracle_cast(&a, &o);
            break;
        case M3_OP_SOFTMAX:
            to_oracle(c->descriptor.softmax.input, &a);
            to_oracle(c->descriptor.softmax.output, &o);
            status = oracle_preflight_nan(&a);
            if (status == 0) {
                status = oracle_softmax(&a, &o);
            }
            break;
        case M3_OP_SNAKE1D:
            to_oracle(c->descriptor.snake1d.input, &a);
            to_oracle(c->descriptor.snake1d.alpha, &b);
            to_oracle(c->descriptor.snake1d.output, &o);
            status = oracle_snake1d(&a, &b, &o);
            break;
        case M3_OP_GATED_SILU:
            to_oracle(c->descriptor.gated_silu.left, &a);
            to_oracle(c->descriptor.gated_silu.right, &b);
            to_oracle(c->descriptor.gated_silu.output, &o);
            status = oracle_gated_silu(&a, &b, &o);
            break;
        case M3_OP_TANH:
            to_oracle(c->descriptor.tanh.input, &a);
            to_oracle(c->descriptor.tanh.output, &o);
            status = oracle_tanh(&a, &o);
            break;
        default:
            return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                                "oracle backend: kind %d", (int)c->kind);
        }
        if (status != 0) {
            return m3_error_set(error, (m3_status)status,
                                "oracle backend preflight failed");
        }
    }
    g_list_count += 1U;
    if (g_fail_list_at != 0U && g_list_count == g_fail_list_at) {
        return m3_error_set(error, (m3_status)g_fail_status,
                            "test backend: the device reported an error "
                            "after list %zu",
                            g_list_count);
    }
    return M3_STATUS_OK;
}

static m3_status write_hook(void *context, void *data, size_t byte_offset,
                            const void *source, size_t byte_count,
                            m3_error *error)
{
    (void)context;
    (void)error;
    memcpy((uint8_t *)data + byte_offset, source, byte_count);
    g_host_to_device += 1U;
    return M3_STATUS_OK;
}

static m3_status read_hook(void *context, const void *data,
                           size_t byte_offset, void *destination,
                           size_t byte_count, m3_error *error)
{
    (void)context;
    (void)error;
    memcpy(destination, (const uint8_t *)data + byte_offset, byte_count);
    g_device_to_host += 1U;
    return M3_STATUS_OK;
}

m3_status oracle_backend_create(m3_backend **backend, m3_error *error)
{
    static const m3_backend_vtable host_vtable = {
        destroy, allocate, free_storage, execute, NULL, NULL, reserve};
    static const m3_backend_vtable device_vtable = {
        destroy,    allocate,  free_storage, execute,
        write_hook, read_hook, reserve};
    const m3_backend_vtable *chosen =
        g_device_memory ? &device_vtable : &host_vtable;
    m3_backend_info info;
    oracle_backend_context *context;
    m3_status status;

    if (g_create_status != 0) {
        return m3_error_set(error, (m3_status)g_create_status,
                            "test backend: made to fail with status %d",
                            g_create_status);
    }
    context = calloc(1U, sizeof(*context));
    if (context == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY, "no memory");
    }
    memset(&info, 0, sizeof(info));
    strcpy(info.name, "oracle test backend");
    info.kind = M3_BACKEND_HIP;
    info.unified_memory = true;
    info.maximum_storage_bytes = (uint64_t)SIZE_MAX;
    info.unified_memory = !g_device_memory;
    status = m3_backend_create_internal(chosen, context, &info, backend,
                                        error);
    if (status != M3_STATUS_OK) {
        free(context);
    }
    return status;
}
