/*
 * m3_backend_hip.c - the HIP execution provider as an m3 backend.
 *
 * Takes the place of the Metal backend of the reference
 * (src/m3_backend_metal.m); written in C11 against the backend vtable and
 * the thin C ABI of m3_hip.h.
 *
 * Storage. The session compiler reserves one arena (one hipMalloc) sized
 * for all of its slots and every slot is carved from it at 256-byte
 * alignment; allocations made without a reserved arena, or beyond it, get
 * their own hipMalloc. Device memory is zeroed when obtained. Storage is
 * not host-visible: m3_storage_write/read become stream-ordered copies.
 *
 * Execution of a command list (reference: m3_metal_execute_in_pool,
 * src/m3_backend_metal.m:178-217, and m3_metal_preflight_basic,
 * src/m3_backend_metal_basic.m:274-302). Checked inputs (a SOFTMAX input,
 * the input of a CAST from a float dtype to I32) that no command of the
 * list writes are scanned on the device (NaN for SOFTMAX, finite and
 * inside [-2^31, 2^31) for the cast) before any kernel is enqueued, with
 * one flag readback for the whole list, and the first failing one in list
 * order fails the list with no output modified (OUT_OF_RANGE). A checked
 * input that an earlier command of the list writes, which Metal rejects,
 * is checked as the reference CPU provider does, right before its command:
 * the scan is queued after its producers and a failure closes the list's
 * device-side gate, so that the command and every later one return
 * without running; the list then waits once, at its end, for the verdict
 * (the commands before the failing one have run). A view that
 * passed its check is remembered until its storage is written (host write,
 * kernel output) or freed, so an unchanged input is not scanned again.
 * Views the preflight has scanned are also watched: a host write to their
 * storage starts their scan on the device right after the copy
 * (m3_hip_scan_views_begin) and returns, and the next preflight collects
 * its flags instead of scanning, so the scan runs while the host is busy
 * between the write and the run. Then every command is enqueued in order
 * on the device stream and the list waits once at the end.
 */
#include "m3_backend_internal.h"

#include "m3_backend_hip.h"
#include "m3_hip.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define M3_HIP_ARENA_ALIGNMENT 256U
#define M3_HIP_MAX_ARENAS 16U
#define M3_HIP_MESSAGE 256U
#define M3_HIP_CLEAN_VIEWS 64U
#define M3_HIP_WATCHED_VIEWS 16U

typedef struct {
    uint8_t *base;
    size_t size;
    size_t used;
} m3_hip_arena;

typedef struct {
    m3_hip_device *device;
    m3_hip_arena arenas[M3_HIP_MAX_ARENAS];
    size_t arena_count;
    /* per-list preflight buffers, grown on demand */
    m3_hip_view *scan_views;
    uint32_t *scan_kinds;
    uint32_t *scan_flags;
    size_t scan_capacity;
    /* views whose last data check passed and whose storage has not been
     * written since (host write, kernel output or free) */
    m3_hip_view clean[M3_HIP_CLEAN_VIEWS];
    uint32_t clean_kinds[M3_HIP_CLEAN_VIEWS];
    size_t clean_count;
    size_t clean_next;
    /* views the preflight has scanned, rescanned early after host writes */
    m3_hip_view watched[M3_HIP_WATCHED_VIEWS];
    uint32_t watched_kinds[M3_HIP_WATCHED_VIEWS];
    size_t watched_count;
    /* the scan a host write started, until a preflight collects it; an
     * entry whose storage is written again before that is dropped */
    m3_hip_view started[M3_HIP_WATCHED_VIEWS];
    uint32_t started_kinds[M3_HIP_WATCHED_VIEWS];
    bool started_valid[M3_HIP_WATCHED_VIEWS];
    size_t started_count;
    uint32_t started_ticket;
    /* true when nothing was queued since the last list waited for its
     * produced checks' verdict: m3_hip_finish has nothing to wait for */
    bool settled;
} m3_hip_backend_context;

static bool m3_hip_same_view(const m3_hip_view *a, const m3_hip_view *b)
{
    uint32_t axis;

    if (a->base != b->base || a->byte_offset != b->byte_offset ||
        a->element_count != b->element_count || a->rank != b->rank ||
        a->dtype != b->dtype) {
        return false;
    }
    for (axis = 0U; axis < a->rank; ++axis) {
        if (a->shape[axis] != b->shape[axis] ||
            a->byte_strides[axis] != b->byte_strides[axis]) {
            return false;
        }
    }
    return true;
}

static bool m3_hip_known_clean(const m3_hip_backend_context *context,
                               const m3_hip_view *view, uint32_t kind)
{
    size_t i;

    for (i = 0U; i < context->clean_count; ++i) {
        if (context->clean_kinds[i] == kind &&
            m3_hip_same_view(&context->clean[i], view)) {
            return true;
        }
    }
    return false;
}

static void m3_hip_remember_clean(m3_hip_backend_context *context,
                                  const m3_hip_view *view, uint32_t kind)
{
    size_t slot;

    if (m3_hip_known_clean(context, view, kind)) {
        return;
    }
    if (context->clean_count < M3_HIP_CLEAN_VIEWS) {
        slot = context->clean_count++;
    } else {
        slot = context->clean_next;
        context->clean_next = (context->clean_next + 1U) % M3_HIP_CLEAN_VIEWS;
    }
    context->clean[slot] = *view;
    context->clean_kinds[slot] = kind;
}

/* Forgets every clean view over the storage that starts at `base`, and
 * the started scan of any. */
static void m3_hip_forget_storage(m3_hip_backend_context *context,
                                  const void *base)
{
    size_t i = 0U;

    for (i = 0U; i < context->started_count; ++i) {
        if (context->started[i].base == base) {
            context->started_valid[i] = false;
        }
    }
    i = 0U;

    while (i < context->clean_count) {
        if (context->clean[i].base == base) {
            context->clean_count -= 1U;
            context->clean[i] = context->clean[context->clean_count];
            context->clean_kinds[i] = context->clean_kinds[context->clean_count];
        } else {
            ++i;
        }
    }
    context->clean_next = 0U;
}

static m3_status m3_hip_status(int code, const char *message,
                               m3_error *error)
{
    switch (code) {
    case M3_HIP_OK:
        return M3_STATUS_OK;
    case M3_HIP_NO_DEVICE:
    case M3_HIP_UNSUPPORTED:
        return m3_error_set(error, M3_STATUS_UNSUPPORTED, "%s", message);
    case M3_HIP_OUT_OF_MEMORY:
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY, "%s", message);
    default:
        return m3_error_set(error, M3_STATUS_INTERNAL, "%s", message);
    }
}

/* Watches (view, kind) for early rescans after host writes. */
static void m3_hip_watch(m3_hip_backend_context *context,
                         const m3_hip_view *view, uint32_t kind)
{
    size_t i;

    for (i = 0U; i < context->watched_count; ++i) {
        if (context->watched_kinds[i] == kind &&
            m3_hip_same_view(&context->watched[i], view)) {
            return;
        }
    }
    if (context->watched_count < M3_HIP_WATCHED_VIEWS) {
        context->watched[context->watched_count] = *view;
        context->watched_kinds[context->watched_count] = kind;
        context->watched_count += 1U;
    }
}

/* Collects the scan a host write started, if any: every entry still valid
 * whose view passed is remembered clean (one that failed is left to the
 * preflight, which scans it again and reports it). */
static m3_status m3_hip_settle_started(m3_hip_backend_context *context,
                                       m3_error *error)
{
    uint32_t flags[M3_HIP_WATCHED_VIEWS];
    char message[M3_HIP_MESSAGE] = "";
    size_t count = context->started_count;
    size_t i;
    int code;

    if (count == 0U) {
        return M3_STATUS_OK;
    }
    context->started_count = 0U;
    code = m3_hip_scan_views_collect(context->device, context->started_ticket,
                                     count, flags, message, sizeof(message));
    if (code != M3_HIP_OK) {
        return m3_hip_status(code, message, error);
    }
    for (i = 0U; i < count; ++i) {
        if (context->started_valid[i] && flags[i] == 0U) {
            m3_hip_remember_clean(context, &context->started[i],
                                  context->started_kinds[i]);
        }
    }
    return M3_STATUS_OK;
}

static void m3_hip_destroy(void *opaque)
{
    m3_hip_backend_context *context = opaque;
    size_t i;

    /* queued commands may still use the arenas */
    (void)m3_hip_synchronize(context->device, NULL, 0U);
    for (i = 0U; i < context->arena_count; ++i) {
        m3_hip_arena_release(context->device, context->arenas[i].base);
    }
    m3_hip_device_close(context->device);
    free(context->scan_views);
    free(context->scan_kinds);
    free(context->scan_flags);
    free(context);
}

static m3_status m3_hip_reserve(void *opaque, size_t byte_count,
                                m3_error *error)
{
    m3_hip_backend_context *context = opaque;
    char message[M3_HIP_MESSAGE] = "";
    void *base = NULL;
    int code;

    context->settled = false;
    if (context->arena_count == M3_HIP_MAX_ARENAS) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "HIP backend arena table is full");
    }
    code = m3_hip_arena_reserve(context->device, byte_count, &base, message,
                                sizeof(message));
    if (code != M3_HIP_OK) {
        return m3_hip_status(code, message, error);
    }
    context->arenas[context->arena_count].base = base;
    context->arenas[context->arena_count].size = byte_count;
    context->arenas[context->arena_count].used = 0U;
    context->arena_count += 1U;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* The arena holding [address, address + 1), or NULL for memory that has
 * its own hipMalloc. */
static const m3_hip_arena *m3_hip_arena_of(
    const m3_hip_backend_context *context, const void *address)
{
    const uint8_t *at = address;
    size_t i;

    for (i = 0U; i < context->arena_count; ++i) {
        const m3_hip_arena *arena = &context->arenas[i];

        if (at >= arena->base && at < arena->base + arena->size) {
            return arena;
        }
    }
    return NULL;
}

/* handle and data are both the device address of the storage (the
 * backend's storages are reached through m3_storage_handle_internal);
 * storage carved from an arena is told apart by its address. */
static m3_status m3_hip_allocate(void *opaque, size_t byte_count,
                                 size_t alignment, void **handle, void **data,
                                 m3_error *error)
{
    m3_hip_backend_context *context = opaque;
    size_t granule = alignment > M3_HIP_ARENA_ALIGNMENT
                         ? alignment
                         : M3_HIP_ARENA_ALIGNMENT;
    char message[M3_HIP_MESSAGE] = "";
    void *base = NULL;
    int code;

    context->settled = false;
    *handle = NULL;
    *data = NULL;
    if (byte_count == 0U) {
        return M3_STATUS_OK;
    }
    if (context->arena_count != 0U) {
        m3_hip_arena *arena = &context->arenas[context->arena_count - 1U];
        size_t start = (arena->used + granule - 1U) & ~(granule - 1U);

        if (start >= arena->used && start <= arena->size &&
            byte_count <= arena->size - start) {
            arena->used = start + byte_count;
            *data = arena->base + start;
            *handle = *data;
            return M3_STATUS_OK;
        }
    }
    code = m3_hip_arena_reserve(context->device, byte_count, &base, message,
                                sizeof(message));
    if (code != M3_HIP_OK) {
        return m3_hip_status(code, message, error);
    }
    *handle = base;
    *data = base;
    return M3_STATUS_OK;
}

static void m3_hip_free_storage(void *opaque, void *handle, void *data)
{
    m3_hip_backend_context *context = opaque;
    size_t i = 0U;

    m3_hip_forget_storage(context, data);
    /* memory at this address may later hold other storage */
    while (i < context->watched_count) {
        if (context->watched[i].base == data) {
            context->watched_count -= 1U;
            context->watched[i] = context->watched[context->watched_count];
            context->watched_kinds[i] =
                context->watched_kinds[context->watched_count];
        } else {
            ++i;
        }
    }
    if (handle != NULL && m3_hip_arena_of(context, handle) == NULL) {
        /* queued commands may still use the memory */
        (void)m3_hip_synchronize(context->device, NULL, 0U);
        m3_hip_arena_release(context->device, handle);
    }
}

static m3_status m3_hip_write(void *opaque, void *data, size_t byte_offset,
                              const void *source, size_t byte_count,
                              m3_error *error)
{
    m3_hip_backend_context *context = opaque;
    char message[M3_HIP_MESSAGE] = "";
    m3_hip_view views[M3_HIP_WATCHED_VIEWS];
    uint32_t kinds[M3_HIP_WATCHED_VIEWS];
    size_t count = 0U;
    size_t i;
    m3_status status;
    int code;

    context->settled = false;
    m3_hip_forget_storage(context, data);
    code = m3_hip_copy_h2d(context->device, (uint8_t *)data + byte_offset,
                               source, byte_count, message, sizeof(message));
    if (code != M3_HIP_OK) {
        return m3_hip_status(code, message, error);
    }
    for (i = 0U; i < context->watched_count; ++i) {
        if (context->watched[i].base == data) {
            views[count] = context->watched[i];
            kinds[count] = context->watched_kinds[i];
            count += 1U;
        }
    }
    if (count == 0U) {
        return M3_STATUS_OK;
    }
    /* The data is written; starting its scan early is an optimization. If
     * settling the previous started scan (only the last one can be
     * collected) or starting this one fails, nothing is started and the
     * next preflight scans these views itself, reporting any device error
     * there. */
    status = m3_hip_settle_started(context, error);
    if (status == M3_STATUS_OK) {
        code = m3_hip_scan_views_begin(context->device, kinds, views, count,
                                       &context->started_ticket, message,
                                       sizeof(message));
    }
    if (status != M3_STATUS_OK || code != M3_HIP_OK) {
        m3_error_reset(error);
        return M3_STATUS_OK;
    }
    for (i = 0U; i < count; ++i) {
        context->started[i] = views[i];
        context->started_kinds[i] = kinds[i];
        context->started_valid[i] = true;
    }
    context->started_count = count;
    return M3_STATUS_OK;
}

static m3_status m3_hip_read(void *opaque, const void *data,
                             size_t byte_offset, void *destination,
                             size_t byte_count, m3_error *error)
{
    m3_hip_backend_context *context = opaque;
    char message[M3_HIP_MESSAGE] = "";
    int code = m3_hip_copy_d2h(context->device, destination,
                               (const uint8_t *)data + byte_offset,
                               byte_count, message, sizeof(message));

    context->settled = false;
    return code == M3_HIP_OK ? M3_STATUS_OK
                             : m3_hip_status(code, message, error);
}

static void m3_hip_view_of(const m3_tensor_view *view, m3_hip_view *out)
{
    uint8_t axis;

    (void)memset(out, 0, sizeof(*out));
    out->base = m3_storage_handle_internal(view->storage);
    out->byte_offset = (uint64_t)view->byte_offset;
    out->element_count = (uint64_t)view->metadata.element_count;
    out->rank = view->metadata.rank;
    out->dtype = (uint32_t)view->metadata.dtype;
    for (axis = 0U; axis < view->metadata.rank; ++axis) {
        out->shape[axis] = view->metadata.shape[axis];
        out->byte_strides[axis] = (uint64_t)view->byte_strides[axis];
    }
}

/* The binary descriptor of ADD, MUL, SUB and DIV commands, else NULL. */
static const m3_op_binary *m3_hip_binary_of(const m3_command *command)
{
    switch (command->kind) {
    case M3_OP_ADD:
        return &command->descriptor.add;
    case M3_OP_MUL:
        return &command->descriptor.mul;
    case M3_OP_SUB:
        return &command->descriptor.sub;
    case M3_OP_DIV:
        return &command->descriptor.div;
    default:
        return NULL;
    }
}

/* The view a command writes (NULL for an elementwise program, whose
 * outputs are those of its commands). */
static const m3_tensor_view *m3_hip_output_of(const m3_command *command)
{
    const m3_op_binary *binary = m3_hip_binary_of(command);

    if (binary != NULL) {
        return binary->output;
    }
    switch (command->kind) {
    case M3_OP_COPY:
    case M3_OP_CAST:
    case M3_OP_SOFTMAX:
    case M3_OP_TANH:
        /* the unary descriptors share one layout */
        return command->descriptor.copy.output;
    case M3_OP_SNAKE1D:
        return command->descriptor.snake1d.output;
    case M3_OP_GATED_SILU:
        return command->descriptor.gated_silu.output;
    default:
        return NULL;
    }
}

/* Input view that must pass a data check before the list runs, else NULL;
 * *kind receives the scan kind. */
static const m3_tensor_view *m3_hip_checked_input(const m3_command *command,
                                                  uint32_t *kind)
{
    if (command->kind == M3_OP_SOFTMAX) {
        *kind = M3_HIP_SCAN_NAN;
        return command->descriptor.softmax.input;
    }
    if (command->kind == M3_OP_CAST &&
        command->descriptor.cast.output->metadata.dtype == M3_DTYPE_I32 &&
        command->descriptor.cast.input->metadata.dtype != M3_DTYPE_I32) {
        *kind = M3_HIP_SCAN_I32_RANGE;
        return command->descriptor.cast.input;
    }
    return NULL;
}

/* True when `command` writes `storage`: its output, or for a fused
 * elementwise program the output of any fused command (also those the
 * program keeps in registers, which is conservative). */
static bool m3_hip_writes(const m3_command *command,
                          const m3_storage *storage)
{
    const m3_tensor_view *output = m3_hip_output_of(command);

    if (command->kind == M3_OP_ELEMENTWISE_PROGRAM) {
        const m3_op_elementwise_program *program =
            &command->descriptor.elementwise_program;
        size_t k;

        for (k = 0U; k < program->command_count; ++k) {
            if (m3_hip_writes(&program->commands[k], storage)) {
                return true;
            }
        }
        return false;
    }
    return output != NULL && output->storage == storage;
}

static bool m3_hip_written_before(const m3_command *commands, size_t index,
                                  const m3_storage *storage)
{
    size_t i;

    for (i = 0U; i < index; ++i) {
        if (m3_hip_writes(&commands[i], storage)) {
            return true;
        }
    }
    return false;
}

/* Drops the clean-scan memory of every storage `command` writes. */
static void m3_hip_forget_outputs(m3_hip_backend_context *context,
                                  const m3_command *command)
{
    const m3_tensor_view *output = m3_hip_output_of(command);

    if (command->kind == M3_OP_ELEMENTWISE_PROGRAM) {
        const m3_op_elementwise_program *program =
            &command->descriptor.elementwise_program;
        size_t k;

        for (k = 0U; k < program->command_count; ++k) {
            m3_hip_forget_outputs(context, &program->commands[k]);
        }
        return;
    }
    if (output != NULL) {
        m3_hip_forget_storage(context,
                              m3_storage_handle_internal(output->storage));
    }
}

static m3_status m3_hip_grow_scans(m3_hip_backend_context *context,
                                   size_t count, m3_error *error)
{
    m3_hip_view *views;
    uint32_t *kinds;
    uint32_t *flags;

    if (count <= context->scan_capacity) {
        return M3_STATUS_OK;
    }
    views = realloc(context->scan_views, count * sizeof(*views));
    if (views != NULL) {
        context->scan_views = views;
    }
    kinds = realloc(context->scan_kinds, count * sizeof(*kinds));
    if (kinds != NULL) {
        context->scan_kinds = kinds;
    }
    flags = realloc(context->scan_flags, count * sizeof(*flags));
    if (flags != NULL) {
        context->scan_flags = flags;
    }
    if (views == NULL || kinds == NULL || flags == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot grow HIP preflight state");
    }
    context->scan_capacity = count;
    return M3_STATUS_OK;
}

static m3_status m3_hip_scan_failure(uint32_t kind, m3_error *error)
{
    return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                        kind == M3_HIP_SCAN_NAN
                            ? "a softmax input element is NaN"
                            : "invalid value for a cast to I32: NaN, infinite or outside [-2^31, 2^31)");
}

/* The list-atomic part of the data preflight: every checked input that no
 * earlier command of the list writes is scanned before anything runs, and
 * the first failing one in list order fails the whole list with nothing
 * executed (the Metal contract, src/m3_backend_metal_basic.m:274-302).
 * Checked inputs that an earlier command writes are checked on the
 * device after their producers (m3_hip_check_produced). */
static m3_status m3_hip_preflight(m3_hip_backend_context *context,
                                  const m3_command *commands, size_t count,
                                  m3_error *error)
{
    size_t scans = 0U;
    size_t i;
    m3_status status = m3_hip_settle_started(context, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    for (i = 0U; i < count; ++i) {
        uint32_t kind = 0U;
        const m3_tensor_view *input = m3_hip_checked_input(&commands[i],
                                                           &kind);

        if (input == NULL || input->metadata.element_count == 0U ||
            m3_hip_written_before(commands, i, input->storage)) {
            continue;
        }
        status = m3_hip_grow_scans(context, scans + 1U, error);
        if (status != M3_STATUS_OK) {
            return status;
        }
        m3_hip_view_of(input, &context->scan_views[scans]);
        if (m3_hip_known_clean(context, &context->scan_views[scans], kind)) {
            continue;
        }
        context->scan_kinds[scans] = kind;
        scans += 1U;
    }
    for (i = 0U; i < scans; i += 64U) {
        char message[M3_HIP_MESSAGE] = "";
        size_t batch = scans - i < 64U ? scans - i : 64U;
        int code = m3_hip_scan_views(context->device, &context->scan_kinds[i],
                                     &context->scan_views[i], batch,
                                     &context->scan_flags[i], message,
                                     sizeof(message));

        if (code != M3_HIP_OK) {
            return m3_hip_status(code, message, error);
        }
    }
    for (i = 0U; i < scans; ++i) {
        m3_hip_watch(context, &context->scan_views[i],
                     context->scan_kinds[i]);
        if (context->scan_flags[i] == 0U) {
            m3_hip_remember_clean(context, &context->scan_views[i],
                                  context->scan_kinds[i]);
        }
    }
    for (i = 0U; i < scans; ++i) {
        if (context->scan_flags[i] != 0U) {
            return m3_hip_scan_failure(context->scan_kinds[i], error);
        }
    }
    return M3_STATUS_OK;
}

/* Queues the check of the input of commands[index] when it is a checked
 * input (softmax, float-to-I32 cast) that an earlier command of the list
 * writes: the scan runs on the stream after the commands enqueued so far,
 * so it sees the produced values, and a failing scan closes the list's
 * gate, so that this command and every later one return without running
 * (m3_hip_gate_open .. m3_hip_gate_close). The commands before `index`
 * have then run and it and the rest have not: the reference CPU provider's
 * order, preflight right before each command (src/m3_op_execute_host.c
 * :5-60), where Metal rejects such a list outright. *gated records that the
 * gate is open. */
static m3_status m3_hip_check_produced(m3_hip_backend_context *context,
                                       const m3_command *commands,
                                       size_t index, bool *gated,
                                       m3_error *error)
{
    uint32_t kind = 0U;
    const m3_tensor_view *input = m3_hip_checked_input(&commands[index],
                                                       &kind);
    char message[M3_HIP_MESSAGE] = "";
    m3_hip_view view;
    int code = M3_HIP_OK;

    if (input == NULL || input->metadata.element_count == 0U ||
        !m3_hip_written_before(commands, index, input->storage)) {
        return M3_STATUS_OK;
    }
    if (!*gated) {
        code = m3_hip_gate_open(context->device, message, sizeof(message));
        *gated = code == M3_HIP_OK;
    }
    if (code == M3_HIP_OK) {
        m3_hip_view_of(input, &view);
        code = m3_hip_gate_check(context->device, kind, &view, message,
                                 sizeof(message));
    }
    return code == M3_HIP_OK ? M3_STATUS_OK
                             : m3_hip_status(code, message, error);
}

/* The checked input of commands[index + 1] when commands[index] is an
 * elementwise program that writes it and the check is a NaN check: the
 * program can make that check as it stores the values
 * (m3_hip_launch_program_checked). NULL otherwise. */
static const m3_tensor_view *m3_hip_fusable_check(const m3_command *commands,
                                                  size_t count, size_t index,
                                                  uint32_t *kind)
{
    const m3_tensor_view *input;

    if (commands[index].kind != M3_OP_ELEMENTWISE_PROGRAM ||
        index + 1U >= count) {
        return NULL;
    }
    input = m3_hip_checked_input(&commands[index + 1U], kind);
    if (input == NULL || *kind != M3_HIP_SCAN_NAN ||
        input->metadata.element_count == 0U ||
        !m3_hip_writes(&commands[index], input->storage)) {
        return NULL;
    }
    return input;
}

/* Launches the elementwise program `command` with the NaN check of
 * `checked` made as it stores it when the program stores all of it
 * (*fused = true), else plainly (*fused = false). */
static int m3_hip_enqueue_checked(m3_hip_backend_context *context,
                                  const m3_command *command,
                                  const m3_tensor_view *checked,
                                  uint32_t kind, bool *fused, char *message,
                                  size_t capacity)
{
    const m3_op_elementwise_program *program =
        &command->descriptor.elementwise_program;
    m3_hip_view view;
    int made = 0;
    int code;

    m3_hip_view_of(checked, &view);
    code = m3_hip_launch_program_checked(
        context->device, program->words,
        (const uint8_t *)m3_storage_handle_internal(program->storage) +
            program->byte_offset,
        program->word_count, kind, &view, &made, message, capacity);
    *fused = code == M3_HIP_OK && made != 0;
    return code;
}

static int m3_hip_enqueue(m3_hip_backend_context *context,
                          const m3_command *command, char *message,
                          size_t capacity)
{
    const m3_op_binary *binary = m3_hip_binary_of(command);
    m3_hip_view a;
    m3_hip_view b;
    m3_hip_view c;

    if (command->kind == M3_OP_ELEMENTWISE_PROGRAM) {
        const m3_op_elementwise_program *program =
            &command->descriptor.elementwise_program;

        return m3_hip_launch_program(
            context->device, program->words,
            (const uint8_t *)m3_storage_handle_internal(program->storage) +
                program->byte_offset,
            program->word_count, message, capacity);
    }
    if (binary != NULL) {
        static const uint32_t ops[] = {M3_HIP_ADD, M3_HIP_MUL, M3_HIP_SUB,
                                       M3_HIP_DIV};
        uint32_t op = command->kind == M3_OP_ADD   ? ops[0]
                      : command->kind == M3_OP_MUL ? ops[1]
                      : command->kind == M3_OP_SUB ? ops[2]
                                                   : ops[3];

        m3_hip_view_of(binary->left, &a);
        m3_hip_view_of(binary->right, &b);
        m3_hip_view_of(binary->output, &c);
        return m3_hip_launch_binary(context->device, op, &a, &b, &c, message,
                                    capacity);
    }
    switch (command->kind) {
    case M3_OP_COPY:
        m3_hip_view_of(command->descriptor.copy.input, &a);
        m3_hip_view_of(command->descriptor.copy.output, &c);
        return m3_hip_launch_copy(context->device, &a, &c, message,
                                  capacity);
    case M3_OP_CAST:
        m3_hip_view_of(command->descriptor.cast.input, &a);
        m3_hip_view_of(command->descriptor.cast.output, &c);
        return m3_hip_launch_cast(context->device, &a, &c, message,
                                  capacity);
    case M3_OP_SOFTMAX:
        m3_hip_view_of(command->descriptor.softmax.input, &a);
        m3_hip_view_of(command->descriptor.softmax.output, &c);
        return m3_hip_launch_softmax(context->device, &a, &c, message,
                                     capacity);
    case M3_OP_SNAKE1D:
        m3_hip_view_of(command->descriptor.snake1d.input, &a);
        m3_hip_view_of(command->descriptor.snake1d.alpha, &b);
        m3_hip_view_of(command->descriptor.snake1d.output, &c);
        return m3_hip_launch_snake1d(context->device, &a, &b, &c, message,
                                     capacity);
    case M3_OP_TANH:
        m3_hip_view_of(command->descriptor.tanh.input, &a);
        m3_hip_view_of(command->descriptor.tanh.output, &c);
        return m3_hip_launch_tanh(context->device, &a, &c, message,
                                  capacity);
    case M3_OP_GATED_SILU:
        m3_hip_view_of(command->descriptor.gated_silu.left, &a);
        m3_hip_view_of(command->descriptor.gated_silu.right, &b);
        m3_hip_view_of(command->descriptor.gated_silu.output, &c);
        return m3_hip_launch_gated_silu(context->device, &a, &b, &c, message,
                                        capacity);

    default:
        (void)snprintf(message, capacity,
                       "HIP does not implement operation %d",
                       (int)command->kind);
        return M3_HIP_UNSUPPORTED;
    }
}

static m3_status m3_hip_execute(void *opaque, const m3_command *commands,
                                size_t count, m3_scratch_arena *scratch,
                                m3_error *error)
{
    m3_hip_backend_context *context = opaque;
    char message[M3_HIP_MESSAGE] = "";
    m3_status status;
    size_t i;
    int code = M3_HIP_OK;
    bool gated = false;
    bool fused = false; /* the command before checked this one's input */

    (void)scratch;
    context->settled = false;
    status = m3_hip_preflight(context, commands, count, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    for (i = 0U; i < count && code == M3_HIP_OK; ++i) {
        uint32_t kind = 0U;
        const m3_tensor_view *checked;

        if (fused) {
            /* its check was made as the program before it stored the
             * input: armed, its kernels close the gate instead of running
             * when that check failed */
            m3_hip_forget_outputs(context, &commands[i]);
            code = m3_hip_gate_pending(context->device, 1, message,
                                       sizeof(message));
            if (code == M3_HIP_OK) {
                const int run = m3_hip_enqueue(context, &commands[i],
                                               message, sizeof(message));

                code = m3_hip_gate_pending(context->device, 0, NULL, 0U);
                code = run != M3_HIP_OK ? run : code;
            }
            fused = false;
            continue;
        }
        status = m3_hip_check_produced(context, commands, i, &gated, error);
        if (status != M3_STATUS_OK) {
            break;
        }
        m3_hip_forget_outputs(context, &commands[i]);
        checked = m3_hip_fusable_check(commands, count, i, &kind);
        if (checked == NULL) {
            code = m3_hip_enqueue(context, &commands[i], message,
                                  sizeof(message));
            continue;
        }
        if (!gated) {
            code = m3_hip_gate_open(context->device, message,
                                    sizeof(message));
            gated = code == M3_HIP_OK;
        }
        if (code == M3_HIP_OK) {
            code = m3_hip_enqueue_checked(context, &commands[i], checked,
                                          kind, &fused, message,
                                          sizeof(message));
        }
    }
    if (gated) {
        /* the list's one host wait: the verdict of its produced checks */
        uint32_t failed = 0U;
        char close_message[M3_HIP_MESSAGE] = "";
        const int closed = m3_hip_gate_close(context->device, &failed,
                                             close_message,
                                             sizeof(close_message));

        if (status == M3_STATUS_OK && code == M3_HIP_OK) {
            if (closed != M3_HIP_OK) {
                return m3_hip_status(closed, close_message, error);
            }
            if (failed != 0U) {
                return m3_hip_scan_failure(failed - 1U, error);
            }
            context->settled = true;
        }
    }
    if (status != M3_STATUS_OK) {
        (void)m3_hip_synchronize(context->device, NULL, 0U);
        return status;
    }
    if (code == M3_HIP_OK) {
        /* queued (or, with produced checks, complete); m3_hip_finish, a
         * storage read or write, a data scan or destroy waits for it */
        m3_error_reset(error);
        return M3_STATUS_OK;
    }
    (void)m3_hip_synchronize(context->device, NULL, 0U);
    return m3_hip_status(code, message, error);
}

static m3_status m3_hip_finish(void *opaque, m3_error *error)
{
    m3_hip_backend_context *context = opaque;
    char message[M3_HIP_MESSAGE] = "";
    int code;

    if (context->settled) {
        return M3_STATUS_OK; /* the last list already waited */
    }
    code = m3_hip_synchronize(context->device, message, sizeof(message));

    return code == M3_HIP_OK ? M3_STATUS_OK
                             : m3_hip_status(code, message, error);
}

m3_status m3_backend_create_hip(m3_backend **backend, m3_error *error)
{
    static const m3_backend_vtable vtable = {
        m3_hip_destroy, m3_hip_allocate, m3_hip_free_storage, m3_hip_execute,
        m3_hip_write,   m3_hip_read,     m3_hip_reserve,      m3_hip_finish};
    m3_hip_backend_context *context;
    m3_backend_info info;
    char message[M3_HIP_MESSAGE] = "";
    uint64_t total = 0U;
    uint32_t units = 0U;
    m3_status status;
    int code;

    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "HIP backend output is null");
    }
    *backend = NULL;
    context = calloc(1U, sizeof(*context));
    if (context == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate HIP backend context");
    }
    code = m3_hip_device_open(0, &context->device, message, sizeof(message));
    if (code != M3_HIP_OK) {
        free(context);
        return m3_hip_status(code, message, error);
    }
    (void)memset(&info, 0, sizeof(info));
    code = m3_hip_device_properties(context->device, info.name,
                                    sizeof(info.name), &total, &units,
                                    message, sizeof(message));
    if (code != M3_HIP_OK) {
        m3_hip_destroy(context);
        return m3_hip_status(code, message, error);
    }
    if (info.name[0] == '\0') {
        (void)snprintf(info.name, sizeof(info.name), "HIP device 0");
    }
    info.kind = M3_BACKEND_HIP;
    info.unified_memory = false;
    info.recommended_working_set_bytes = total;
    info.maximum_storage_bytes = total;
    status = m3_backend_create_internal(&vtable, context, &info, backend,
                                        error);
    if (status != M3_STATUS_OK) {
        m3_hip_destroy(context);
    }
    return status;
}

bool m3_hip_owns_execute(m3_status (*execute)(void *, const m3_command *,
                                            size_t, m3_scratch_arena *,
                                            m3_error *))
{
    return execute == m3_hip_execute;
}

void *m3_hip_context_device(void *context)
{
    return context == NULL ? NULL
                           : (void *)((m3_hip_backend_context *)context)
                                 ->device;
}
