/*
 * m3_buffers.c - backends and the storages they own.
 *
 * A backend is a provider's hooks (m3_backend_vtable, copied when the
 * backend is made) plus its context. The storages it has handed out sit
 * in a row table: each storage record knows its row, so releasing one
 * moves the last row into the hole, and releasing the backend walks the
 * table once and then destroys the context. Live and peak byte and
 * storage counts are kept beside the table.
 *
 * A backend whose hooks include write/read owns device memory: the host
 * cannot dereference its storages (m3_storage_data gives NULL) and every
 * transfer goes through the hooks, in stream order for the HIP backend.
 * Other backends own host memory and transfers are memcpy.
 *
 * What callers observe is kept from the reference (src/m3_backend.c:
 * 80-366): the statuses, the order in which arguments are checked, the
 * allocation statistics, and that executing a list first validates all of
 * it and checks the scratch it needs (m3_backend_execute).
 */
#include "m3_internal.h"

#include <stdlib.h>
#include <string.h>

#define M3_TABLE_FIRST_ROWS 16U

struct m3_storage {
    m3_backend *home;
    size_t row;
    void *handle;
    void *address; /* what the allocate hook returned as data */
    size_t bytes;
};

struct m3_backend {
    m3_backend_vtable hooks;
    void *context;
    m3_backend_info info;
    m3_storage **table;
    size_t rows;
    size_t capacity;
    size_t bytes_live;
    size_t bytes_peak;
    size_t rows_peak;
};

static bool m3_hooks_complete(const m3_backend_vtable *hooks)
{
    const bool has_write = hooks->write != NULL;
    const bool has_read = hooks->read != NULL;

    return hooks->destroy_context != NULL && hooks->allocate != NULL &&
           hooks->free_storage != NULL && hooks->execute != NULL &&
           has_write == has_read;
}

static bool m3_device_resident(const m3_backend *backend)
{
    return backend->hooks.write != NULL;
}

m3_status m3_backend_create_internal(const m3_backend_vtable *vtable,
                                     void *context,
                                     const m3_backend_info *info,
                                     m3_backend **backend_output,
                                     m3_error *error)
{
    m3_backend *made;

    if (backend_output == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no place to return the new backend");
    }
    *backend_output = NULL;
    if (vtable == NULL || context == NULL || info == NULL ||
        !m3_hooks_complete(vtable) || info->name[0] == '\0') {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "a backend needs its four required hooks (write "
                            "and read only as a pair), a context and a "
                            "named info record");
    }
    made = calloc(1U, sizeof(*made));
    if (made == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for a backend record");
    }
    made->hooks = *vtable;
    made->context = context;
    made->info = *info;
    *backend_output = made;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

void m3_backend_free(m3_backend *backend)
{
    size_t row;

    if (backend == NULL) {
        return;
    }
    for (row = backend->rows; row > 0U; --row) {
        m3_storage *storage = backend->table[row - 1U];

        backend->hooks.free_storage(backend->context, storage->handle,
                                    storage->address);
        free(storage);
    }
    free(backend->table);
    backend->hooks.destroy_context(backend->context);
    free(backend);
}

m3_status m3_backend_get_info(const m3_backend *backend,
                              m3_backend_info *info, m3_error *error)
{
    if (backend == NULL || info == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "backend info needs a backend and a result "
                            "record");
    }
    *info = backend->info;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_backend_get_allocation_stats(
    const m3_backend *backend, m3_backend_allocation_stats *stats,
    m3_error *error)
{
    if (backend == NULL || stats == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "allocation statistics need a backend and a "
                            "result record");
    }
    stats->live_allocated_bytes = backend->bytes_live;
    stats->peak_allocated_bytes = backend->bytes_peak;
    stats->live_storage_count = backend->rows;
    stats->peak_storage_count = backend->rows_peak;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_backend_reserve(m3_backend *backend, size_t byte_count,
                             m3_error *error)
{
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "cannot reserve an arena without a backend");
    }
    if (backend->hooks.reserve != NULL && byte_count != 0U) {
        return backend->hooks.reserve(backend->context, byte_count, error);
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_backend_finish(m3_backend *backend, m3_error *error)
{
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "cannot wait for work without a backend");
    }
    if (backend->hooks.finish != NULL) {
        return backend->hooks.finish(backend->context, error);
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* Scratch bytes still free in an arena a caller passed, or false when
 * the arena's fields contradict each other. No arena offers nothing. */
static bool m3_scratch_room(const m3_scratch_arena *scratch, size_t *room)
{
    *room = 0U;
    if (scratch == NULL) {
        return true;
    }
    if (scratch->offset > scratch->capacity ||
        (scratch->data == NULL && scratch->capacity != 0U)) {
        return false;
    }
    *room = scratch->capacity - scratch->offset;
    return true;
}

m3_status m3_backend_execute(m3_backend *backend, const m3_command *commands,
                             size_t command_count, m3_scratch_arena *scratch,
                             m3_error *error)
{
    size_t wanted = 0U;
    size_t room = 0U;
    m3_status status;

    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "cannot execute commands without a backend");
    }
    /* the whole list is validated before any of it runs */
    status = m3_commands_scratch_bytes(backend, commands, command_count,
                                       &wanted, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (!m3_scratch_room(scratch, &room)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "scratch arena offset or backing is "
                            "inconsistent");
    }
    if (wanted > room) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "command list wants %zu scratch bytes, %zu "
                            "are free",
                            wanted, room);
    }
    if (command_count != 0U) {
        status = backend->hooks.execute(backend->context, commands,
                                        command_count, scratch, error);
        if (status != M3_STATUS_OK) {
            return status;
        }
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

void *m3_backend_hip_device(const m3_backend *backend)
{
    return backend != NULL && m3_hip_owns_execute(backend->hooks.execute)
               ? m3_hip_context_device(backend->context)
               : NULL;
}

bool m3_backend_host_visible(const m3_backend *backend)
{
    return backend != NULL && !m3_device_resident(backend);
}

void *m3_backend_context_internal(const m3_backend *backend)
{
    return backend == NULL ? NULL : backend->context;
}

const m3_backend_vtable *m3_backend_vtable_of(const m3_backend *backend)
{
    return backend == NULL ? NULL : &backend->hooks;
}

/* ---- storages ----------------------------------------------------------- */

static bool m3_table_make_room(m3_backend *backend)
{
    size_t grown;
    m3_storage **moved;

    if (backend->rows < backend->capacity) {
        return true;
    }
    grown = backend->capacity == 0U ? M3_TABLE_FIRST_ROWS
                                    : backend->capacity * 2U;
    if (grown < backend->capacity || grown > SIZE_MAX / sizeof(*moved)) {
        return false;
    }
    moved = realloc(backend->table, grown * sizeof(*moved));
    if (moved == NULL) {
        return false;
    }
    backend->table = moved;
    backend->capacity = grown;
    return true;
}

static void m3_table_add(m3_backend *backend, m3_storage *storage)
{
    storage->home = backend;
    storage->row = backend->rows;
    backend->table[backend->rows] = storage;
    backend->rows += 1U;
    backend->bytes_live += storage->bytes;
    if (backend->bytes_live > backend->bytes_peak) {
        backend->bytes_peak = backend->bytes_live;
    }
    if (backend->rows > backend->rows_peak) {
        backend->rows_peak = backend->rows;
    }
}

static void m3_table_remove(m3_storage *storage)
{
    m3_backend *backend = storage->home;
    m3_storage *last = backend->table[backend->rows - 1U];

    backend->table[storage->row] = last;
    last->row = storage->row;
    backend->rows -= 1U;
    backend->bytes_live -= storage->bytes;
    storage->home = NULL;
}

m3_status m3_storage_allocate(m3_backend *backend, size_t byte_count,
                              size_t alignment, m3_storage **storage_output,
                              m3_error *error)
{
    m3_storage *storage;
    void *handle = NULL;
    void *address = NULL;
    m3_status status;

    if (storage_output == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no place to return the new storage");
    }
    *storage_output = NULL;
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "cannot allocate storage without a backend");
    }
    if (alignment < sizeof(void *) || (alignment & (alignment - 1U)) != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage alignment %zu is not a power of two "
                            "of at least pointer size",
                            alignment);
    }
    if ((uint64_t)byte_count > backend->info.maximum_storage_bytes) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "%zu bytes exceed the backend's largest storage",
                            byte_count);
    }
    if (byte_count > SIZE_MAX - backend->bytes_live ||
        backend->rows == SIZE_MAX) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "live storage totals would overflow");
    }
    storage = calloc(1U, sizeof(*storage));
    if (storage == NULL || !m3_table_make_room(backend)) {
        free(storage);
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for a storage record");
    }
    status = backend->hooks.allocate(backend->context, byte_count, alignment,
                                     &handle, &address, error);
    if (status != M3_STATUS_OK) {
        free(storage);
        return status;
    }
    if ((address == NULL && byte_count != 0U) ||
        ((uintptr_t)address & (alignment - 1U)) != 0U) {
        backend->hooks.free_storage(backend->context, handle, address);
        free(storage);
        return m3_error_set(error, M3_STATUS_INTERNAL,
                            "the backend's allocate hook returned %s memory",
                            address == NULL ? "no" : "misaligned");
    }
    storage->handle = handle;
    storage->address = address;
    storage->bytes = byte_count;
    m3_table_add(backend, storage);
    *storage_output = storage;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

void m3_storage_free(m3_storage *storage)
{
    m3_backend *backend;

    if (storage == NULL) {
        return;
    }
    backend = storage->home;
    if (backend != NULL) {
        m3_table_remove(storage);
        backend->hooks.free_storage(backend->context, storage->handle,
                                    storage->address);
    }
    free(storage);
}

size_t m3_storage_size(const m3_storage *storage)
{
    return storage == NULL ? 0U : storage->bytes;
}

bool m3_storage_host_visible(const m3_storage *storage)
{
    return storage != NULL && storage->home != NULL &&
           !m3_device_resident(storage->home);
}

void *m3_storage_data(m3_storage *storage)
{
    return m3_storage_host_visible(storage) ? storage->address : NULL;
}

const void *m3_storage_const_data(const m3_storage *storage)
{
    return m3_storage_host_visible(storage) ? storage->address : NULL;
}

void *m3_storage_device_data(const m3_storage *storage)
{
    return storage == NULL ? NULL : storage->address;
}

void *m3_storage_handle_internal(const m3_storage *storage)
{
    return storage == NULL ? NULL : storage->handle;
}

m3_backend *m3_storage_backend(const m3_storage *storage)
{
    return storage == NULL ? NULL : storage->home;
}

/* Checks shared by transfers in both directions; `direction` names the
 * transfer in messages. */
static m3_status m3_transfer_check(const m3_storage *storage,
                                   size_t byte_offset, size_t byte_count,
                                   const void *host, const char *direction,
                                   m3_error *error)
{
    if (storage == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage %s without a storage", direction);
    }
    if (byte_offset > storage->bytes ||
        byte_count > storage->bytes - byte_offset) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "storage %s of %zu bytes at offset %zu passes "
                            "the end of a %zu-byte storage",
                            direction, byte_count, byte_offset,
                            storage->bytes);
    }
    if (byte_count != 0U && host == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage %s has no host buffer", direction);
    }
    if (byte_count != 0U && storage->home == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage %s after its backend was released",
                            direction);
    }
    return M3_STATUS_OK;
}

m3_status m3_storage_write(m3_storage *storage, size_t byte_offset,
                           const void *source, size_t byte_count,
                           m3_error *error)
{
    m3_status status = m3_transfer_check(storage, byte_offset, byte_count,
                                         source, "write", error);

    if (status != M3_STATUS_OK || byte_count == 0U) {
        if (status == M3_STATUS_OK) {
            m3_error_reset(error);
        }
        return status;
    }
    if (m3_device_resident(storage->home)) {
        const m3_backend *home = storage->home;

        status = home->hooks.write(home->context, storage->address,
                                   byte_offset, source, byte_count, error);
        if (status != M3_STATUS_OK) {
            return status;
        }
    } else {
        (void)memcpy((uint8_t *)storage->address + byte_offset, source,
                     byte_count);
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_storage_read(const m3_storage *storage, size_t byte_offset,
                          void *destination, size_t byte_count,
                          m3_error *error)
{
    m3_status status = m3_transfer_check(storage, byte_offset, byte_count,
                                         destination, "read", error);

    if (status != M3_STATUS_OK || byte_count == 0U) {
        if (status == M3_STATUS_OK) {
            m3_error_reset(error);
        }
        return status;
    }
    if (m3_device_resident(storage->home)) {
        const m3_backend *home = storage->home;

        status = home->hooks.read(home->context, storage->address,
                                  byte_offset, destination, byte_count,
                                  error);
        if (status != M3_STATUS_OK) {
            return status;
        }
    } else {
        (void)memcpy(destination,
                     (const uint8_t *)storage->address + byte_offset,
                     byte_count);
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}
