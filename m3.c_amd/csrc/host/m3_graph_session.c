/*
 * m3_graph_session.c - session I/O, execution and plan queries.
 *
 * Follows src/m3_graph_session.c of the reference:
 *   role and exact-size checks on I/O   :38-98
 *   partitioned run                     :100-150
 *   plan info and node provider         :152-184
 * A run groups each maximal stretch of consecutive nodes with the same
 * provider into one command list. With the HIP provider every node of a
 * stretch is enqueued on one stream and the list waits once at its end.
 * The list executed is the session's run list, in which fused runs of
 * elementwise nodes appear as one elementwise-program command each.
 */
#include "m3_graph_internal.h"

static m3_status m3_session_check_value(const m3_session *session,
                                        m3_graph_value_id value,
                                        m3_graph_value_role role,
                                        const char *what, m3_error *error)
{
    if (session == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "%s session is null", what);
    }
    if ((size_t)value >= session->value_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "%s value is out of range", what);
    }
    if (session->values[value].description.role != role) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "%s value has the wrong role", what);
    }
    return M3_STATUS_OK;
}

m3_status m3_session_write_input(m3_session *session, m3_graph_value_id value,
                                 const void *data, size_t byte_count,
                                 m3_error *error)
{
    m3_status status = m3_session_check_value(session, value, M3_GRAPH_INPUT,
                                              "input write", error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (byte_count != session->values[value].metadata.byte_count ||
        (byte_count != 0U && data == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "input write size does not match tensor");
    }
    return m3_storage_write(session->views[value].storage,
                            session->views[value].byte_offset, data,
                            byte_count, error);
}

m3_status m3_session_read_output(const m3_session *session,
                                 m3_graph_value_id value, void *data,
                                 size_t byte_count, m3_error *error)
{
    m3_status status = m3_session_check_value(session, value,
                                              M3_GRAPH_OUTPUT, "output read",
                                              error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (byte_count != session->values[value].metadata.byte_count ||
        (byte_count != 0U && data == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "output read size does not match tensor");
    }
    return m3_storage_read(session->views[value].storage,
                           session->views[value].byte_offset, data,
                           byte_count, error);
}

m3_status m3_session_run(m3_session *session, m3_error *error)
{
    size_t begin = 0U;

    if (session == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "session is null");
    }
    while (begin < session->run_count) {
        m3_scratch_arena scratch;
        size_t end = begin + 1U;
        m3_status status;

        while (end < session->run_count &&
               session->run_providers[end] == session->run_providers[begin]) {
            ++end;
        }
        status = m3_scratch_arena_init(&scratch, session->scratch,
                                       session->scratch_capacity, error);
        if (status == M3_STATUS_OK) {
            status = m3_provider_execute_regular(
                session->backend, session->run_providers[begin],
                &session->run_commands[begin], end - begin, &scratch,
                error);
        }
        if (status != M3_STATUS_OK) {
            return status;
        }
        begin = end;
    }
    /* a run is complete when it returns, as on the reference's providers */
    return m3_backend_finish(session->backend, error);
}

m3_status m3_session_get_plan_info(const m3_session *session,
                                   m3_session_plan_info *info,
                                   m3_error *error)
{
    if (session == NULL || info == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "session and plan info output are required");
    }
    info->value_count = session->value_count;
    info->node_count = session->node_count;
    info->storage_slot_count = session->slot_count;
    info->allocated_bytes = session->allocated_bytes;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_session_get_node_provider(const m3_session *session,
                                       size_t node_index,
                                       m3_provider_kind *provider,
                                       m3_error *error)
{
    if (session == NULL || provider == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "session and provider output are required");
    }
    if (node_index >= session->node_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "session node index is out of range");
    }
    *provider = session->providers[node_index];
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* The session's storage backend, for measurement tools that read the
 * provider's kernel timings. Not part of the reference API. */
m3_backend *m3_session_backend(const m3_session *session)
{
    return session == NULL ? NULL : session->backend;
}
