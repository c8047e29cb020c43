/*
 * m3_internal.h - declarations shared by the C11 host layer.
 */
#ifndef M3_INTERNAL_H
#define M3_INTERNAL_H

#include "m3_backend.h"
#include "m3_backend_hip.h"

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

/* ---- checked size arithmetic ------------------------------------------ */

static inline bool m3_size_add_checked(size_t a, size_t b, size_t *out)
{
    if (a > SIZE_MAX - b) {
        return false;
    }
    *out = a + b;
    return true;
}

static inline bool m3_size_mul_checked(size_t a, size_t b, size_t *out)
{
    if (a != 0U && b > SIZE_MAX / a) {
        return false;
    }
    *out = a * b;
    return true;
}

/* ---- op helpers (m3_op_validate.c) ------------------------------------ */

bool m3_op_dtype_is_float(m3_dtype dtype);
bool m3_op_same_shape(const m3_tensor_view *a, const m3_tensor_view *b);
/* Binary descriptor of ADD/MUL/SUB/DIV commands, else NULL. */
const m3_op_binary *m3_op_binary_of(const m3_command *command);
/* Output view written by a supported command, else NULL. */
const m3_tensor_view *m3_op_output_of(const m3_command *command);
/* True when the HIP provider runs this operation kind. */
bool m3_op_kind_supported(m3_op_kind kind);

/* ---- backend internals (m3_buffers.c) --------------------------------- */

const m3_backend_vtable *m3_backend_vtable_of(const m3_backend *backend);
/* True when the backend's storages are host memory. */
bool m3_backend_host_visible(const m3_backend *backend);

/* ---- CPU provider (m3_cpu_provider.c) --------------------------------- */

bool m3_cpu_kind_supported(m3_op_kind kind);
/* Runs a validated list over host storage, each command's data check
 * right before it. */
m3_status m3_cpu_execute(const m3_command *commands, size_t count,
                         m3_error *error);

/* ---- provider scheduler (m3_provider.c) ------------------------------- */

m3_status m3_backend_create_preferred(bool allow_gpu, bool allow_cpu,
                                      m3_backend **backend, m3_error *error);
m3_status m3_provider_select_regular(const m3_backend *storage_backend,
                                     bool allow_gpu, bool allow_cpu,
                                     const m3_command *commands,
                                     size_t command_count,
                                     m3_provider_kind *provider,
                                     m3_error *error);
m3_status m3_provider_execute_regular(m3_backend *storage_backend,
                                      m3_provider_kind provider,
                                      const m3_command *commands,
                                      size_t command_count,
                                      m3_scratch_arena *scratch,
                                      m3_error *error);

#endif
