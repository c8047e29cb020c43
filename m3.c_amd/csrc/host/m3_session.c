/*
 * m3_session.c - compiling a graph into a session, running it, and its
 * input/output boundary.
 *
 * Compilation (m3_session_create), in layers:
 *   1. the liveness plan (m3_plan.c): data-flow checks and slots;
 *   2. the storage backend, chosen by the scheduler from the options
 *      (m3_backend_create_preferred), one arena reserved for all slots and
 *      each slot carved from it;
 *   3. one contiguous view per value over its slot; constants uploaded;
 *   4. one command per node and its provider (m3_provider_select_regular).
 *      A node on the CPU provider runs directly on host storage, or, when
 *      the storage is device memory, on host mirrors of the values it
 *      touches (a staged node);
 *   5. the run list (m3_graph_fuse.c).
 *
 * Running walks the run list in stretches of entries with the same
 * provider and hands each stretch to the scheduler as one command list.
 * Around a stretch of staged nodes the session moves data across PCIe
 * once per value and run: an input of the stretch whose mirror is not
 * fresh is copied device -> host first (the copy waits for the device to
 * have produced it), and a value the stretch writes is copied host ->
 * device afterwards only when it is an OUTPUT or a node on the GPU reads
 * it later. Constants are mirrored once, at creation. The run ends with
 * m3_backend_finish, so the outputs are complete when it returns.
 *
 * Observable contract kept from the reference (src/m3_graph_compile.c:
 * 442-531, src/m3_graph_session.c:38-184): statuses and check order of
 * every call, the plan numbers, and one list per same-provider stretch.
 */
#include "m3_session_internal.h"

#include <stdlib.h>
#include <string.h>

#define M3_SLOT_ALIGNMENT 64U

/* ---- compilation ------------------------------------------------------- */

static m3_status m3_session_arrays(m3_session *session, m3_error *error)
{
    const size_t values = session->value_count == 0U ? 1U
                                                     : session->value_count;
    const size_t nodes = session->node_count == 0U ? 1U : session->node_count;

    session->values = calloc(values, sizeof(*session->values));
    session->views = calloc(values, sizeof(*session->views));
    session->commands = calloc(nodes, sizeof(*session->commands));
    session->providers = calloc(nodes, sizeof(*session->providers));
    session->lanes = calloc(nodes, sizeof(*session->lanes));
    session->nodes = calloc(nodes, sizeof(*session->nodes));
    if (session->values == NULL || session->views == NULL ||
        session->commands == NULL || session->providers == NULL ||
        session->lanes == NULL || session->nodes == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for a session");
    }
    return M3_STATUS_OK;
}

/* Reserves the arena and carves one storage per slot from it. */
static m3_status m3_session_place_slots(m3_session *session, m3_error *error)
{
    const m3_plan *plan = &session->plan;
    size_t s;
    m3_status status;

    session->slots = calloc(plan->slot_count == 0U ? 1U : plan->slot_count,
                            sizeof(*session->slots));
    if (session->slots == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for the slot table");
    }
    status = m3_backend_reserve(session->backend, plan->arena_bytes, error);
    for (s = 0U; status == M3_STATUS_OK && s < plan->slot_count; ++s) {
        status = m3_storage_allocate(session->backend, plan->slot_bytes[s],
                                     M3_SLOT_ALIGNMENT, &session->slots[s],
                                     error);
    }
    return status;
}

static m3_status m3_session_build_views(m3_session *session,
                                        const m3_graph *graph,
                                        m3_error *error)
{
    size_t v;

    for (v = 0U; v < session->value_count; ++v) {
        const m3_value_spec *spec = &session->values[v];
        m3_storage *slot = session->slots[session->plan.slot_of[v]];
        m3_status status = m3_tensor_view_contiguous(
            &session->views[v], slot, spec->meta.dtype, spec->meta.rank,
            spec->meta.shape, 0U, error);

        if (status == M3_STATUS_OK &&
            spec->desc.role == M3_GRAPH_CONSTANT) {
            status = m3_storage_write(slot, 0U,
                                      m3_graph_value_at(graph, v)->constant,
                                      spec->meta.byte_count, error);
        }
        if (status != M3_STATUS_OK) {
            return status;
        }
    }
    return M3_STATUS_OK;
}

static m3_status m3_session_bind_nodes(m3_session *session, m3_error *error)
{
    const bool device = !m3_backend_host_visible(session->backend);
    size_t n;

    for (n = 0U; n < session->node_count; ++n) {
        size_t scratch = 0U;
        m3_status status = m3_graph_bind_command(
            &session->nodes[n], session->views, session->value_count,
            &session->commands[n], error);

        if (status == M3_STATUS_OK) {
            status = m3_provider_select_regular(
                session->backend, session->options.allow_metal,
                session->options.allow_cpu, &session->commands[n], 1U,
                &session->providers[n], error);
        }
        if (status == M3_STATUS_OK) {
            status = m3_commands_scratch_bytes(session->backend,
                                               &session->commands[n], 1U,
                                               &scratch, error);
        }
        if (status != M3_STATUS_OK) {
            return status;
        }
        session->lanes[n] = session->providers[n] != M3_PROVIDER_CPU
                                ? M3_LANE_GPU
                            : device ? M3_LANE_STAGED
                                     : M3_LANE_CPU;
    }
    return M3_STATUS_OK;
}

/* ---- staging ------------------------------------------------------------ */

static bool m3_node_reads(const m3_graph_node_desc *node, size_t value)
{
    size_t k;

    for (k = 0U; k < M3_GRAPH_NODE_INPUT_CAPACITY; ++k) {
        if (node->inputs[k] == value) {
            return true;
        }
    }
    return false;
}

static bool m3_node_touches(const m3_graph_node_desc *node, size_t value)
{
    return m3_node_reads(node, value) || node->outputs[0] == value;
}

/* Mirrors, mirror views and re-bound commands for the staged nodes. */
static m3_status m3_session_stage(m3_session *session, m3_error *error)
{
    size_t n;
    size_t v;
    bool any = false;
    m3_status status;

    for (n = 0U; n < session->node_count; ++n) {
        any = any || session->lanes[n] == M3_LANE_STAGED;
    }
    if (!any) {
        return M3_STATUS_OK;
    }
    session->mirrors = calloc(session->value_count,
                              sizeof(*session->mirrors));
    session->mirror_viewset = calloc(session->value_count,
                                     sizeof(*session->mirror_viewset));
    if (session->mirrors == NULL || session->mirror_viewset == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for staging state");
    }
    status = m3_backend_create_host(&session->mirror_backend, error);
    for (v = 0U; status == M3_STATUS_OK && v < session->value_count; ++v) {
        m3_mirror *mirror = &session->mirrors[v];
        const m3_value_spec *spec = &session->values[v];
        bool staged = false;

        for (n = 0U; n < session->node_count; ++n) {
            if (session->lanes[n] == M3_LANE_STAGED &&
                m3_node_touches(&session->nodes[n], v)) {
                staged = true;
            }
            /* written by a staged node, read later on the GPU */
            if (session->lanes[n] == M3_LANE_GPU &&
                m3_node_reads(&session->nodes[n], v)) {
                mirror->gpu_reads = true;
            }
        }
        session->mirror_viewset[v] = session->views[v];
        if (!staged) {
            continue;
        }
        status = m3_storage_allocate(session->mirror_backend,
                                     spec->meta.byte_count, M3_SLOT_ALIGNMENT,
                                     &mirror->storage, error);
        if (status == M3_STATUS_OK) {
            m3_tensor_view_init(&session->mirror_viewset[v]);
            status = m3_tensor_view_contiguous(
                &session->mirror_viewset[v], mirror->storage,
                spec->meta.dtype, spec->meta.rank, spec->meta.shape, 0U,
                error);
        }
        if (status == M3_STATUS_OK &&
            spec->desc.role == M3_GRAPH_CONSTANT) {
            status = m3_storage_read(session->views[v].storage, 0U,
                                     m3_storage_data(mirror->storage),
                                     spec->meta.byte_count, error);
            mirror->fresh = true;
            mirror->keep = true;
        }
    }
    for (n = 0U; status == M3_STATUS_OK && n < session->node_count; ++n) {
        if (session->lanes[n] == M3_LANE_STAGED) {
            status = m3_graph_bind_command(
                &session->nodes[n], session->mirror_viewset,
                session->value_count, &session->commands[n], error);
        }
    }
    return status;
}

/* Device -> mirror for every input of nodes [first, end) that is stale. */
static m3_status m3_stage_in(m3_session *session, size_t first, size_t end,
                             m3_error *error)
{
    size_t n;
    size_t k;

    for (n = first; n < end; ++n) {
        const m3_graph_node_desc *node = &session->nodes[n];

        for (k = 0U; k < M3_GRAPH_NODE_INPUT_CAPACITY; ++k) {
            const m3_graph_value_id v = node->inputs[k];
            m3_mirror *mirror;
            m3_status status;

            if (v == M3_GRAPH_VALUE_NONE) {
                continue;
            }
            mirror = &session->mirrors[v];
            if (mirror->fresh) {
                continue;
            }
            status = m3_storage_read(session->views[v].storage,
                                     session->views[v].byte_offset,
                                     m3_storage_data(mirror->storage),
                                     session->values[v].meta.byte_count,
                                     error);
            if (status != M3_STATUS_OK) {
                return status;
            }
            mirror->fresh = true;
        }
    }
    return M3_STATUS_OK;
}

/* Mirror -> device for the values nodes [first, end) wrote that leave the
 * CPU: OUTPUT values, and values a GPU node reads. */
static m3_status m3_stage_out(m3_session *session, size_t first, size_t end,
                              m3_error *error)
{
    size_t n;

    for (n = first; n < end; ++n) {
        const m3_graph_value_id v = session->nodes[n].outputs[0];
        m3_mirror *mirror = &session->mirrors[v];
        m3_status status;

        mirror->fresh = true;
        if (session->values[v].desc.role != M3_GRAPH_OUTPUT &&
            !mirror->gpu_reads) {
            continue;
        }
        status = m3_storage_write(session->views[v].storage,
                                  session->views[v].byte_offset,
                                  m3_storage_data(mirror->storage),
                                  session->values[v].meta.byte_count, error);
        if (status != M3_STATUS_OK) {
            return status;
        }
    }
    return M3_STATUS_OK;
}

/* ---- lifetime ----------------------------------------------------------- */

void m3_session_free(m3_session *session)
{
    size_t index;

    if (session == NULL) {
        return;
    }
    m3_session_free_runs(session);
    for (index = 0U; session->mirrors != NULL && index < session->value_count;
         ++index) {
        m3_storage_free(session->mirrors[index].storage);
    }
    m3_backend_free(session->mirror_backend);
    for (index = 0U; session->slots != NULL &&
                     index < session->plan.slot_count;
         ++index) {
        m3_storage_free(session->slots[index]);
    }
    m3_backend_free(session->backend);
    m3_plan_release(&session->plan);
    free(session->mirrors);
    free(session->mirror_viewset);
    free(session->slots);
    free(session->views);
    free(session->values);
    free(session->commands);
    free(session->providers);
    free(session->lanes);
    free(session->nodes);
    free(session);
}

m3_status m3_session_create(m3_session **session_output,
                            const m3_graph *graph,
                            const m3_session_options *options,
                            m3_error *error)
{
    m3_session *session;
    m3_status status;
    size_t v;

    if (session_output == NULL || *session_output != NULL || graph == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "a session needs a graph and the address of a "
                            "NULL session pointer");
    }
    session = calloc(1U, sizeof(*session));
    if (session == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for a session");
    }
    m3_session_options_init(&session->options);
    if (options != NULL) {
        session->options = *options;
    }
    if (!session->options.allow_neural_engine &&
        !session->options.allow_metal && !session->options.allow_cpu) {
        free(session);
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "the options enable no provider");
    }
    session->value_count = graph->values.count;
    session->node_count = graph->nodes.count;
    status = m3_session_arrays(session, error);
    for (v = 0U; status == M3_STATUS_OK && v < session->value_count; ++v) {
        session->values[v] = *m3_graph_value_at(graph, v);
        session->values[v].constant = NULL; /* the graph keeps the bytes */
    }
    if (status == M3_STATUS_OK && session->node_count != 0U) {
        (void)memcpy(session->nodes, graph->nodes.items,
                     session->node_count * sizeof(*session->nodes));
    }
    if (status == M3_STATUS_OK) {
        status = m3_plan_build(graph, &session->plan, error);
    }
    if (status == M3_STATUS_OK) {
        const m3_session_options *o = &session->options;

        status = m3_backend_create_preferred(
            o->allow_metal || o->allow_neural_engine,
            o->allow_cpu || o->allow_neural_engine, &session->backend, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_session_place_slots(session, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_session_build_views(session, graph, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_session_bind_nodes(session, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_session_stage(session, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_session_plan_runs(session, graph, error);
    }
    if (status != M3_STATUS_OK) {
        m3_session_free(session);
        return status;
    }
    *session_output = session;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* ---- boundary ----------------------------------------------------------- */

/* The view of a value the caller may write (INPUT) or read (OUTPUT),
 * with exactly its byte count. */
static m3_status m3_session_endpoint(const m3_session *session,
                                     m3_graph_value_id value,
                                     m3_graph_value_role role,
                                     const void *memory, size_t byte_count,
                                     m3_error *error)
{
    const char *what = role == M3_GRAPH_INPUT ? "input" : "output";

    if (session == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no session to move %s data", what);
    }
    if ((size_t)value >= session->value_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "value %u is not in the session",
                            (unsigned int)value);
    }
    if (session->values[value].desc.role != role) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "value %u is not an %s of the graph",
                            (unsigned int)value,
                            role == M3_GRAPH_INPUT ? "INPUT" : "OUTPUT");
    }
    if (byte_count != session->values[value].meta.byte_count ||
        (memory == NULL && byte_count != 0U)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "%s %u moves exactly %zu bytes", what,
                            (unsigned int)value,
                            session->values[value].meta.byte_count);
    }
    return M3_STATUS_OK;
}

m3_status m3_session_write_input(m3_session *session, m3_graph_value_id value,
                                 const void *data, size_t byte_count,
                                 m3_error *error)
{
    m3_status status = m3_session_endpoint(session, value, M3_GRAPH_INPUT,
                                           data, byte_count, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (session->mirrors != NULL) {
        session->mirrors[value].fresh = false;
    }
    return m3_storage_write(session->views[value].storage,
                            session->views[value].byte_offset, data,
                            byte_count, error);
}

m3_status m3_session_read_output(const m3_session *session,
                                 m3_graph_value_id value, void *data,
                                 size_t byte_count, m3_error *error)
{
    m3_status status = m3_session_endpoint(session, value, M3_GRAPH_OUTPUT,
                                           data, byte_count, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    return m3_storage_read(session->views[value].storage,
                           session->views[value].byte_offset, data,
                           byte_count, error);
}

/* ---- running ------------------------------------------------------------ */

static m3_lane m3_run_lane(const m3_session *session, size_t entry)
{
    return session->lanes[session->run_first_node[entry]];
}

m3_status m3_session_run(m3_session *session, m3_error *error)
{
    m3_scratch_arena scratch = {NULL, 0U, 0U};
    size_t first = 0U;
    size_t v;

    if (session == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no session to run");
    }
    for (v = 0U; session->mirrors != NULL && v < session->value_count; ++v) {
        session->mirrors[v].fresh = session->mirrors[v].keep;
    }
    while (first < session->run_count) {
        const m3_provider_kind provider = session->run_providers[first];
        const m3_lane lane = m3_run_lane(session, first);
        size_t end = first + 1U;
        m3_status status = M3_STATUS_OK;

        while (end < session->run_count &&
               session->run_providers[end] == provider &&
               m3_run_lane(session, end) == lane) {
            end += 1U;
        }
        if (lane == M3_LANE_STAGED) {
            /* staged entries are single nodes: programs are GPU-only */
            status = m3_stage_in(session, session->run_first_node[first],
                                 session->run_first_node[end - 1U] + 1U,
                                 error);
        }
        if (status == M3_STATUS_OK) {
            status = m3_provider_execute_regular(
                lane == M3_LANE_STAGED ? session->mirror_backend
                                       : session->backend,
                provider, &session->run_commands[first], end - first,
                &scratch, error);
        }
        if (status == M3_STATUS_OK && lane == M3_LANE_STAGED) {
            status = m3_stage_out(session, session->run_first_node[first],
                                  session->run_first_node[end - 1U] + 1U,
                                  error);
        }
        if (status != M3_STATUS_OK) {
            return status;
        }
        first = end;
    }
    return m3_backend_finish(session->backend, error);
}

m3_status m3_session_get_plan_info(const m3_session *session,
                                   m3_session_plan_info *info,
                                   m3_error *error)
{
    if (session == NULL || info == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "plan info needs a session and a result record");
    }
    info->value_count = session->value_count;
    info->node_count = session->node_count;
    info->storage_slot_count = session->plan.slot_count;
    info->allocated_bytes = session->plan.plain_bytes;
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
                            "node provider needs a session and a result");
    }
    if (node_index >= session->node_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "node %zu is past the session's %zu nodes",
                            node_index, session->node_count);
    }
    *provider = session->providers[node_index];
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_backend *m3_session_backend(const m3_session *session)
{
    return session == NULL ? NULL : session->backend;
}
