/*
 * m3_backend.c - backend objects, storage bookkeeping and list execution.
 *
 * Behaviour follows src/m3_backend.c of the reference:
 *   lifetime contract and creation         :80-111
 *   m3_backend_execute (validate, scratch) :113-154
 *   storage allocation and statistics      :189-276
 *   range-checked write/read               :319-366
 * Storage whose backend provides write/read hooks is device memory: its
 * host address is NULL and transfers go through the hooks.
 */
#include "m3_internal.h"

#include <stdlib.h>
#include <string.h>

struct m3_storage {
    m3_backend *owner;
    void *handle;
    void *data;
    size_t byte_count;
    struct m3_storage *previous;
    struct m3_storage *next;
};

struct m3_backend {
    const m3_backend_vtable *vtable;
    void *context;
    m3_backend_info info;
    m3_backend_allocation_stats stats;
    m3_storage *storages;
    bool device_memory;
};

static bool m3_is_power_of_two(size_t value)
{
    return value != 0U && (value & (value - 1U)) == 0U;
}

m3_status m3_backend_create_internal(const m3_backend_vtable *vtable,
                                     void *context,
                                     const m3_backend_info *info,
                                     m3_backend **backend_output,
                                     m3_error *error)
{
    m3_backend *backend;

    if (backend_output == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "backend output is null");
    }
    *backend_output = NULL;
    if (vtable == NULL || vtable->destroy_context == NULL ||
        vtable->allocate == NULL || vtable->free_storage == NULL ||
        vtable->execute == NULL || context == NULL || info == NULL ||
        info->name[0] == '\0' ||
        (vtable->write == NULL) != (vtable->read == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "backend lifetime contract is incomplete");
    }
    backend = calloc(1U, sizeof(*backend));
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate backend state");
    }
    backend->vtable = vtable;
    backend->context = context;
    backend->info = *info;
    backend->device_memory = vtable->write != NULL;
    *backend_output = backend;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_backend_finish(m3_backend *backend, m3_error *error)
{
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "backend is null");
    }
    if (backend->vtable->finish == NULL) {
        m3_error_reset(error);
        return M3_STATUS_OK;
    }
    return backend->vtable->finish(backend->context, error);
}

m3_status m3_backend_execute(m3_backend *backend, const m3_command *commands,
                             size_t command_count, m3_scratch_arena *scratch,
                             m3_error *error)
{
    size_t needed = 0U;
    size_t available = 0U;
    m3_status status;

    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "execution backend is null");
    }
    status = m3_commands_scratch_bytes(backend, commands, command_count,
                                       &needed, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (scratch != NULL) {
        if (scratch->offset > scratch->capacity ||
            (scratch->capacity != 0U && scratch->data == NULL)) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "scratch arena state is invalid");
        }
        available = scratch->capacity - scratch->offset;
    }
    if (needed > available) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "execution needs %zu scratch bytes", needed);
    }
    if (command_count == 0U) {
        m3_error_reset(error);
        return M3_STATUS_OK;
    }
    status = backend->vtable->execute(backend->context, commands,
                                      command_count, scratch, error);
    if (status == M3_STATUS_OK) {
        m3_error_reset(error);
    }
    return status;
}

void m3_backend_free(m3_backend *backend)
{
    m3_storage *storage;

    if (backend == NULL) {
        return;
    }
    storage = backend->storages;
    backend->storages = NULL;
    while (storage != NULL) {
        m3_storage *next = storage->next;

        backend->vtable->free_storage(backend->context, storage->handle,
                                      storage->data);
        free(storage);
        storage = next;
    }
    backend->vtable->destroy_context(backend->context);
    free(backend);
}

m3_status m3_backend_get_info(const m3_backend *backend,
                              m3_backend_info *info, m3_error *error)
{
    if (backend == NULL || info == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "backend and info output are required");
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
                            "backend and stats output are required");
    }
    *stats = backend->stats;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_backend_reserve(m3_backend *backend, size_t byte_count,
                             m3_error *error)
{
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "reserve backend is null");
    }
    if (backend->vtable->reserve == NULL || byte_count == 0U) {
        m3_error_reset(error);
        return M3_STATUS_OK;
    }
    return backend->vtable->reserve(backend->context, byte_count, error);
}

const m3_backend_vtable *m3_backend_vtable_of(const m3_backend *backend)
{
    return backend == NULL ? NULL : backend->vtable;
}

void *m3_backend_context_internal(const m3_backend *backend)
{
    return backend == NULL ? NULL : backend->context;
}

m3_status m3_storage_allocate(m3_backend *backend, size_t byte_count,
                              size_t alignment, m3_storage **storage_output,
                              m3_error *error)
{
    m3_storage *storage;
    void *handle = NULL;
    void *data = NULL;
    m3_status status;

    if (storage_output == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage output is null");
    }
    *storage_output = NULL;
    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage backend is null");
    }
    if (!m3_is_power_of_two(alignment) || alignment < sizeof(void *)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage alignment is invalid");
    }
    if ((uint64_t)byte_count > backend->info.maximum_storage_bytes) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "storage exceeds backend allocation limit");
    }
    if (backend->stats.live_allocated_bytes > SIZE_MAX - byte_count ||
        backend->stats.live_storage_count == SIZE_MAX) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "backend allocation statistics overflow");
    }
    storage = calloc(1U, sizeof(*storage));
    if (storage == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate storage state");
    }
    status = backend->vtable->allocate(backend->context, byte_count,
                                       alignment, &handle, &data, error);
    if (status != M3_STATUS_OK) {
        free(storage);
        return status;
    }
    if ((byte_count != 0U && data == NULL) ||
        (data != NULL && (uintptr_t)data % alignment != 0U)) {
        backend->vtable->free_storage(backend->context, handle, data);
        free(storage);
        return m3_error_set(error, M3_STATUS_INTERNAL,
                            "backend returned null or misaligned storage");
    }
    storage->owner = backend;
    storage->handle = handle;
    storage->data = data;
    storage->byte_count = byte_count;
    storage->next = backend->storages;
    if (backend->storages != NULL) {
        backend->storages->previous = storage;
    }
    backend->storages = storage;
    backend->stats.live_allocated_bytes += byte_count;
    backend->stats.live_storage_count += 1U;
    if (backend->stats.live_allocated_bytes >
        backend->stats.peak_allocated_bytes) {
        backend->stats.peak_allocated_bytes =
            backend->stats.live_allocated_bytes;
    }
    if (backend->stats.live_storage_count > backend->stats.peak_storage_count) {
        backend->stats.peak_storage_count = backend->stats.live_storage_count;
    }
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
    backend = storage->owner;
    if (backend != NULL) {
        if (storage->previous != NULL) {
            storage->previous->next = storage->next;
        } else {
            backend->storages = storage->next;
        }
        if (storage->next != NULL) {
            storage->next->previous = storage->previous;
        }
        backend->stats.live_allocated_bytes -= storage->byte_count;
        backend->stats.live_storage_count -= 1U;
        backend->vtable->free_storage(backend->context, storage->handle,
                                      storage->data);
    }
    free(storage);
}

size_t m3_storage_size(const m3_storage *storage)
{
    return storage == NULL ? 0U : storage->byte_count;
}

bool m3_storage_host_visible(const m3_storage *storage)
{
    return storage != NULL && storage->owner != NULL &&
           !storage->owner->device_memory;
}

void *m3_storage_data(m3_storage *storage)
{
    return m3_storage_host_visible(storage) ? storage->data : NULL;
}

const void *m3_storage_const_data(const m3_storage *storage)
{
    return m3_storage_host_visible(storage) ? storage->data : NULL;
}

void *m3_storage_device_data(const m3_storage *storage)
{
    return storage == NULL ? NULL : storage->data;
}

void *m3_storage_handle_internal(const m3_storage *storage)
{
    return storage == NULL ? NULL : storage->handle;
}

m3_backend *m3_storage_backend(const m3_storage *storage)
{
    return storage == NULL ? NULL : storage->owner;
}

static m3_status m3_storage_range(const m3_storage *storage,
                                  size_t byte_offset, size_t byte_count,
                                  const void *memory, const char *what,
                                  m3_error *error)
{
    if (storage == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "%s storage is null", what);
    }
    if (byte_offset > storage->byte_count ||
        byte_count > storage->byte_count - byte_offset) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "storage %s range exceeds storage", what);
    }
    if (byte_count != 0U && memory == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage %s memory is null", what);
    }
    if (byte_count != 0U && storage->owner == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage %s has no backend", what);
    }
    return M3_STATUS_OK;
}

m3_status m3_storage_write(m3_storage *storage, size_t byte_offset,
                           const void *source, size_t byte_count,
                           m3_error *error)
{
    m3_status status = m3_storage_range(storage, byte_offset, byte_count,
                                        source, "write", error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (byte_count != 0U) {
        const m3_backend *owner = storage->owner;

        if (owner->device_memory) {
            status = owner->vtable->write(owner->context, storage->data,
                                          byte_offset, source, byte_count,
                                          error);
            if (status != M3_STATUS_OK) {
                return status;
            }
        } else {
            (void)memcpy((uint8_t *)storage->data + byte_offset, source,
                         byte_count);
        }
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_storage_read(const m3_storage *storage, size_t byte_offset,
                          void *destination, size_t byte_count,
                          m3_error *error)
{
    m3_status status = m3_storage_range(storage, byte_offset, byte_count,
                                        destination, "read", error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (byte_count != 0U) {
        const m3_backend *owner = storage->owner;

        if (owner->device_memory) {
            status = owner->vtable->read(owner->context, storage->data,
                                         byte_offset, destination,
                                         byte_count, error);
            if (status != M3_STATUS_OK) {
                return status;
            }
        } else {
            (void)memcpy(destination,
                         (const uint8_t *)storage->data + byte_offset,
                         byte_count);
        }
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}
