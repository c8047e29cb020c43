/*
 * m3_provider.c - provider scheduler: storage backend choice and per-list
 * provider selection.
 *
 * Mirrors src/m3_provider.c of the reference with the HIP provider in the
 * place of Metal:
 *   m3_backend_create_preferred  (:35-60)  GPU first when allowed
 *   m3_provider_select_regular   (:62-99)  GPU iff the storage backend is
 *                                          the GPU and every kind is
 *                                          supported
 *   m3_provider_execute_regular  (:101-129)
 * This library has no CPU provider. Where the reference would fall back to
 * its host backend, the scheduler returns M3_STATUS_UNSUPPORTED with a
 * message saying so; nothing is computed on the CPU.
 *
 * m3_provider_set_gpu_factory replaces the GPU backend constructor. Tests
 * use it to run the graph compiler and scheduler against a recording
 * backend on machines without a GPU; NULL restores m3_backend_create_hip.
 */
#include "m3_internal.h"

static m3_backend_factory m3_gpu_factory = NULL;

void m3_provider_set_gpu_factory(m3_backend_factory factory)
{
    m3_gpu_factory = factory;
}

m3_status m3_backend_create_preferred(bool allow_gpu, bool allow_cpu,
                                      m3_backend **backend, m3_error *error)
{
    m3_status status;

    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "preferred backend output is null");
    }
    *backend = NULL;
    if (!allow_gpu && !allow_cpu) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "at least one storage provider is required");
    }
    if (!allow_gpu) {
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "this library has no CPU provider; enable the "
                            "GPU provider (allow_metal)");
    }
    status = m3_gpu_factory != NULL ? m3_gpu_factory(backend, error)
                                    : m3_backend_create_hip(backend, error);
    if (status == M3_STATUS_UNSUPPORTED && allow_cpu) {
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "no HIP device is available and this library "
                            "has no CPU provider");
    }
    return status;
}

m3_status m3_provider_select_regular(const m3_backend *storage_backend,
                                     bool allow_gpu, bool allow_cpu,
                                     const m3_command *commands,
                                     size_t command_count,
                                     m3_provider_kind *provider,
                                     m3_error *error)
{
    m3_backend_info info;
    size_t index;
    m3_status status;

    if (storage_backend == NULL || provider == NULL ||
        (command_count != 0U && commands == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "regular provider selection is incomplete");
    }
    status = m3_backend_get_info(storage_backend, &info, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (allow_gpu && info.kind == M3_BACKEND_HIP) {
        for (index = 0U; index < command_count; ++index) {
            if (!m3_op_kind_supported(commands[index].kind)) {
                break;
            }
        }
        if (index == command_count) {
            *provider = M3_PROVIDER_HIP;
            m3_error_reset(error);
            return M3_STATUS_OK;
        }
        if (allow_cpu) {
            return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                                "operation kind %d needs the CPU provider, "
                                "which this library does not include",
                                (int)commands[index].kind);
        }
    }
    return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                        "no enabled provider supports the command list");
}

m3_status m3_provider_execute_regular(m3_backend *storage_backend,
                                      m3_provider_kind provider,
                                      const m3_command *commands,
                                      size_t command_count,
                                      m3_scratch_arena *scratch,
                                      m3_error *error)
{
    if (provider != M3_PROVIDER_HIP) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "provider cannot execute regular operations");
    }
    return m3_backend_execute(storage_backend, commands, command_count,
                              scratch, error);
}
