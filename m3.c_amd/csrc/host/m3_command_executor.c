/*
 * m3_command_executor.c - command lists outside any graph.
 *
 * Same flow as src/m3_command_executor.c:55-92 of the reference: validate
 * and size scratch, grow the executor's scratch, select a provider with
 * every provider allowed, execute. Flow CFG/Euler arithmetic and the
 * conditioning softmax of the reference run through this path.
 */
#include "m3_internal.h"

#include <stdlib.h>
#include <string.h>

void m3_command_executor_init(m3_command_executor *executor,
                              m3_backend *backend)
{
    if (executor != NULL) {
        (void)memset(executor, 0, sizeof(*executor));
        executor->backend = backend;
    }
}

void m3_command_executor_dispose(m3_command_executor *executor)
{
    if (executor != NULL) {
        free(executor->scratch);
        m3_command_executor_init(executor, NULL);
    }
}

m3_status m3_command_executor_execute(m3_command_executor *executor,
                                      const m3_command *commands,
                                      size_t command_count, m3_error *error)
{
    m3_scratch_arena arena;
    m3_provider_kind provider;
    size_t needed = 0U;
    m3_status status;

    if (executor == NULL || executor->backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "command executor backend is required");
    }
    status = m3_commands_scratch_bytes(executor->backend, commands,
                                       command_count, &needed, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (needed > executor->scratch_capacity) {
        void *grown = malloc(needed);

        if (grown == NULL) {
            return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                                "cannot grow command scratch to %zu bytes",
                                needed);
        }
        free(executor->scratch);
        executor->scratch = grown;
        executor->scratch_capacity = needed;
    }
    status = m3_scratch_arena_init(&arena, executor->scratch,
                                   executor->scratch_capacity, error);
    if (status == M3_STATUS_OK) {
        status = m3_provider_select_regular(executor->backend, true, true,
                                            commands, command_count,
                                            &provider, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_provider_execute_regular(executor->backend, provider,
                                             commands, command_count, &arena,
                                             error);
    }
    return status;
}
