/*
 * m3_executor.c - command lists run outside any graph.
 *
 * The way the reference's flow and conditioning code drive the provider
 * (src/m3_command_executor.c:55-92): each call validates the list and
 * sizes its scratch, keeps a scratch buffer that only grows, lets the
 * scheduler pick the provider with every provider allowed, and executes.
 * On the HIP backend a list returns once its kernels are queued, so
 * single-command calls queue back to back; m3_backend_finish, or any read
 * of a storage, waits for them.
 */
#include "m3_internal.h"

#include <stdlib.h>
#include <string.h>

void m3_command_executor_init(m3_command_executor *executor,
                              m3_backend *backend)
{
    if (executor == NULL) {
        return;
    }
    executor->backend = backend;
    executor->scratch = NULL;
    executor->scratch_capacity = 0U;
}

void m3_command_executor_dispose(m3_command_executor *executor)
{
    if (executor == NULL) {
        return;
    }
    free(executor->scratch);
    m3_command_executor_init(executor, NULL);
}

/* Grows the executor's scratch to at least `bytes`. */
static m3_status m3_executor_scratch(m3_command_executor *executor,
                                     size_t bytes, m3_error *error)
{
    void *larger;

    if (bytes <= executor->scratch_capacity) {
        return M3_STATUS_OK;
    }
    larger = malloc(bytes);
    if (larger == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for %zu scratch bytes",
                            bytes);
    }
    free(executor->scratch);
    executor->scratch = larger;
    executor->scratch_capacity = bytes;
    return M3_STATUS_OK;
}

m3_status m3_command_executor_execute(m3_command_executor *executor,
                                      const m3_command *commands,
                                      size_t command_count, m3_error *error)
{
    m3_scratch_arena arena;
    m3_provider_kind provider = M3_PROVIDER_CPU;
    size_t wanted = 0U;
    m3_status status;

    if (executor == NULL || executor->backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "the executor has no backend");
    }
    status = m3_commands_scratch_bytes(executor->backend, commands,
                                       command_count, &wanted, error);
    if (status == M3_STATUS_OK) {
        status = m3_executor_scratch(executor, wanted, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_scratch_arena_init(&arena, executor->scratch,
                                       executor->scratch_capacity, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_provider_select_regular(executor->backend, true, true,
                                            commands, command_count,
                                            &provider, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_provider_execute_regular(executor->backend, provider,
                                             commands, command_count,
                                             &arena, error);
    }
    return status;
}
