/*
 * m3_graph_compile.c - session compiler: topology check, liveness slot
 * planning, one device arena, views, constant upload, command binding and
 * provider selection.
 *
 * Follows src/m3_graph_compile.c of the reference:
 *   operation I/O schema                     :18-66
 *   topology (read-before-produce, single
 *   producer, last uses)                     :122-245
 *   best-fit slot reuse                      :260-324
 *   slot allocation, allocated_bytes         :326-348
 *   views and constant upload                :350-377
 *   bind + provider + validation per node    :379-440
 *   m3_session_create                        :442-531
 * After the nodes are bound, the run list (fused elementwise programs) is
 * planned by m3_graph_fuse.c.
 * The slot plan is the reference's: every INPUT, CONSTANT and OUTPUT value
 * owns a slot for the whole session; each TEMPORARY takes the smallest slot
 * that is free before its producer runs and large enough, or a new slot.
 * What differs is placement: the compiler sums the slot sizes (each rounded
 * up to 256 bytes), asks the backend for one arena of that size, and the
 * slots are carved from it in order. allocated_bytes stays the unpadded sum
 * of slot sizes.
 */
#include "m3_graph_internal.h"

#include <stdlib.h>
#include <string.h>

#define M3_SLOT_ALIGNMENT 64U
#define M3_ARENA_GRANULE 256U

typedef struct {
    size_t inputs;
    size_t outputs;
} m3_node_arity;

static m3_status m3_node_arity_of(m3_op_kind kind, m3_node_arity *arity,
                                  m3_error *error)
{
    arity->outputs = 1U;
    switch (kind) {
    case M3_OP_COPY:
    case M3_OP_CAST:
    case M3_OP_SOFTMAX:
    case M3_OP_TANH:
        arity->inputs = 1U;
        return M3_STATUS_OK;
    case M3_OP_ADD:
    case M3_OP_MUL:
    case M3_OP_SUB:
    case M3_OP_DIV:
    case M3_OP_SNAKE1D:
    case M3_OP_GATED_SILU:
        arity->inputs = 2U;
        return M3_STATUS_OK;
    default:
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "unsupported graph operation kind %d",
                            (int)kind);
    }
}

static m3_status m3_check_value_id(const m3_graph *graph,
                                   m3_graph_value_id value, const char *what,
                                   m3_error *error)
{
    if (value == M3_GRAPH_VALUE_NONE) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "required graph node %s is absent", what);
    }
    if ((size_t)value >= graph->value_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "graph node %s is out of range", what);
    }
    return M3_STATUS_OK;
}

static m3_status m3_check_node_ids(const m3_graph *graph,
                                   const m3_graph_node_desc *node,
                                   m3_node_arity *arity, m3_error *error)
{
    size_t index;
    m3_status status = m3_node_arity_of(node->kind, arity, error);

    for (index = 0U;
         status == M3_STATUS_OK && index < M3_GRAPH_NODE_INPUT_CAPACITY;
         ++index) {
        if (index >= arity->inputs) {
            if (node->inputs[index] != M3_GRAPH_VALUE_NONE) {
                status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                      "graph node has an extra input");
            }
        } else {
            status = m3_check_value_id(graph, node->inputs[index], "input",
                                       error);
        }
    }
    for (index = 0U;
         status == M3_STATUS_OK && index < M3_GRAPH_NODE_OUTPUT_CAPACITY;
         ++index) {
        if (index >= arity->outputs) {
            if (node->outputs[index] != M3_GRAPH_VALUE_NONE) {
                status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                      "graph node has an extra output");
            }
        } else {
            status = m3_check_value_id(graph, node->outputs[index], "output",
                                       error);
        }
    }
    return status;
}

/* Walks the nodes in order. producers[v] is the node writing v (SIZE_MAX
 * for inputs and constants); last_uses[v] is the last node reading or
 * writing v. */
static m3_status m3_graph_topology(const m3_graph *graph, size_t *producers,
                                   size_t *last_uses, m3_error *error)
{
    bool *ready = calloc(graph->value_count == 0U ? 1U : graph->value_count,
                         sizeof(*ready));
    m3_status status = M3_STATUS_OK;
    size_t v;
    size_t n;

    if (ready == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate graph topology state");
    }
    for (v = 0U; v < graph->value_count; ++v) {
        const m3_graph_value *value = &graph->values[v];

        producers[v] = SIZE_MAX;
        last_uses[v] = 0U;
        ready[v] = value->description.role == M3_GRAPH_INPUT ||
                   value->description.role == M3_GRAPH_CONSTANT;
        if (value->description.role == M3_GRAPH_CONSTANT &&
            !value->constant_set) {
            status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                  "graph constant has no data");
            break;
        }
    }
    for (n = 0U; status == M3_STATUS_OK && n < graph->node_count; ++n) {
        const m3_graph_node_desc *node = &graph->nodes[n];
        m3_node_arity arity = {0U, 0U};
        size_t i;

        status = m3_check_node_ids(graph, node, &arity, error);
        for (i = 0U; status == M3_STATUS_OK && i < arity.inputs; ++i) {
            m3_graph_value_id input = node->inputs[i];

            if (!ready[input]) {
                status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                      "graph node reads a value before it "
                                      "is produced");
            } else {
                last_uses[input] = n;
            }
        }
        for (i = 0U; status == M3_STATUS_OK && i < arity.outputs; ++i) {
            m3_graph_value_id output = node->outputs[i];
            m3_graph_value_role role = graph->values[output].description.role;
            size_t earlier;

            if (role != M3_GRAPH_TEMPORARY && role != M3_GRAPH_OUTPUT) {
                status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                      "graph node writes an input or "
                                      "constant value");
            } else if (producers[output] != SIZE_MAX) {
                status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                      "graph value has multiple producers");
            }
            for (earlier = 0U; status == M3_STATUS_OK && earlier < i;
                 ++earlier) {
                if (node->outputs[earlier] == output) {
                    status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                          "graph node repeats an output "
                                          "value");
                }
            }
            if (status == M3_STATUS_OK) {
                producers[output] = n;
                last_uses[output] = n;
                ready[output] = true;
            }
        }
    }
    for (v = 0U; status == M3_STATUS_OK && v < graph->value_count; ++v) {
        m3_graph_value_role role = graph->values[v].description.role;

        if ((role == M3_GRAPH_TEMPORARY || role == M3_GRAPH_OUTPUT) &&
            producers[v] == SIZE_MAX) {
            status = m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                  "graph value has no producer");
        }
    }
    free(ready);
    return status;
}

static size_t m3_new_slot(m3_session *session, size_t byte_count)
{
    size_t slot = session->slot_count;

    session->slots[slot].byte_count = byte_count;
    session->slot_count += 1U;
    return slot;
}

static m3_status m3_plan_slots(m3_session *session, const size_t *producers,
                               const size_t *last_uses, m3_error *error)
{
    /* busy_until[s]: last node that uses slot s (SIZE_MAX: never free). */
    size_t *busy_until = calloc(session->value_count == 0U
                                    ? 1U
                                    : session->value_count,
                                sizeof(*busy_until));
    size_t v;
    size_t n;

    if (busy_until == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate liveness slots");
    }
    for (v = 0U; v < session->value_count; ++v) {
        m3_session_value *value = &session->values[v];

        value->slot = SIZE_MAX;
        if (value->description.role != M3_GRAPH_TEMPORARY) {
            value->slot = m3_new_slot(session, value->metadata.byte_count);
            busy_until[value->slot] = SIZE_MAX;
        }
    }
    for (n = 0U; n < session->node_count; ++n) {
        for (v = 0U; v < session->value_count; ++v) {
            m3_session_value *value = &session->values[v];
            size_t need = value->metadata.byte_count;
            size_t best = SIZE_MAX;
            size_t s;

            if (value->description.role != M3_GRAPH_TEMPORARY ||
                producers[v] != n) {
                continue;
            }
            for (s = 0U; s < session->slot_count; ++s) {
                size_t size = session->slots[s].byte_count;

                if (busy_until[s] < n && size >= need &&
                    (best == SIZE_MAX ||
                     size < session->slots[best].byte_count)) {
                    best = s;
                }
            }
            if (best == SIZE_MAX) {
                best = m3_new_slot(session, need);
            }
            value->slot = best;
            busy_until[best] = last_uses[v];
        }
    }
    free(busy_until);
    m3_error_reset(error);
    return M3_STATUS_OK;
}

static m3_status m3_allocate_slots(m3_session *session, m3_error *error)
{
    size_t arena = 0U;
    size_t s;
    m3_status status;

    for (s = 0U; s < session->slot_count; ++s) {
        size_t bytes = session->slots[s].byte_count;
        size_t padded;

        if (bytes > SIZE_MAX - session->allocated_bytes ||
            !m3_size_add_checked(bytes, M3_ARENA_GRANULE - 1U, &padded) ||
            !m3_size_add_checked(arena, padded & ~(size_t)(M3_ARENA_GRANULE -
                                                           1U),
                                 &arena)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "graph allocation total overflows");
        }
        session->allocated_bytes += bytes;
    }
    status = m3_backend_reserve(session->backend, arena, error);
    for (s = 0U; status == M3_STATUS_OK && s < session->slot_count; ++s) {
        status = m3_storage_allocate(session->backend,
                                     session->slots[s].byte_count,
                                     M3_SLOT_ALIGNMENT,
                                     &session->slots[s].storage, error);
    }
    return status;
}

static m3_status m3_build_views(m3_session *session, const m3_graph *graph,
                                m3_error *error)
{
    size_t v;

    for (v = 0U; v < session->value_count; ++v) {
        const m3_session_value *value = &session->values[v];
        m3_status status = m3_tensor_view_contiguous(
            &session->views[v], session->slots[value->slot].storage,
            value->metadata.dtype, value->metadata.rank,
            value->metadata.shape, 0U, error);

        if (status == M3_STATUS_OK &&
            value->description.role == M3_GRAPH_CONSTANT) {
            status = m3_storage_write(session->views[v].storage, 0U,
                                      graph->values[v].constant_data,
                                      graph->values[v].constant_size, error);
        }
        if (status != M3_STATUS_OK) {
            return status;
        }
    }
    return M3_STATUS_OK;
}

static m3_status m3_compile_nodes(m3_session *session, const m3_graph *graph,
                                  m3_error *error)
{
    size_t n;

    for (n = 0U; n < session->node_count; ++n) {
        m3_command *command = &session->commands[n];
        size_t scratch = 0U;
        m3_status status = m3_graph_bind_command(&graph->nodes[n],
                                                 session->views,
                                                 session->value_count,
                                                 command, error);

        if (status == M3_STATUS_OK) {
            status = m3_provider_select_regular(
                session->backend, session->options.allow_metal,
                session->options.allow_cpu, command, 1U,
                &session->providers[n], error);
        }
        if (status == M3_STATUS_OK) {
            status = m3_commands_scratch_bytes(session->backend, command, 1U,
                                               &scratch, error);
        }
        if (status != M3_STATUS_OK) {
            return status;
        }
    }
    return M3_STATUS_OK;
}

void m3_session_free(m3_session *session)
{
    size_t s;

    if (session == NULL) {
        return;
    }
    m3_session_free_runs(session);
    for (s = 0U; session->slots != NULL && s < session->slot_count; ++s) {
        m3_storage_free(session->slots[s].storage);
    }
    free(session->scratch);
    free(session->commands);
    free(session->providers);
    free(session->slots);
    free(session->views);
    free(session->values);
    m3_backend_free(session->backend);
    free(session);
}

m3_status m3_session_create(m3_session **session_output,
                            const m3_graph *graph,
                            const m3_session_options *options,
                            m3_error *error)
{
    m3_session_options selected;
    m3_session *session;
    size_t *producers;
    size_t *last_uses;
    size_t values;
    size_t v;
    m3_status status = M3_STATUS_OK;

    if (session_output == NULL || *session_output != NULL || graph == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "session output must be empty and graph is "
                            "required");
    }
    m3_session_options_init(&selected);
    if (options != NULL) {
        selected = *options;
    }
    if (!selected.allow_neural_engine && !selected.allow_metal &&
        !selected.allow_cpu) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "session has no enabled provider");
    }
    session = calloc(1U, sizeof(*session));
    if (session == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate session");
    }
    session->options = selected;
    session->value_count = graph->value_count;
    session->node_count = graph->node_count;
    values = graph->value_count == 0U ? 1U : graph->value_count;
    session->values = calloc(values, sizeof(*session->values));
    session->views = calloc(values, sizeof(*session->views));
    session->slots = calloc(values, sizeof(*session->slots));
    session->providers = calloc(graph->node_count == 0U ? 1U
                                                        : graph->node_count,
                                sizeof(*session->providers));
    session->commands = calloc(graph->node_count == 0U ? 1U
                                                       : graph->node_count,
                               sizeof(*session->commands));
    producers = calloc(values, sizeof(*producers));
    last_uses = calloc(values, sizeof(*last_uses));
    if (session->values == NULL || session->views == NULL ||
        session->slots == NULL || session->providers == NULL ||
        session->commands == NULL || producers == NULL ||
        last_uses == NULL) {
        status = m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                              "cannot allocate session plan arrays");
    }
    for (v = 0U; status == M3_STATUS_OK && v < session->value_count; ++v) {
        session->values[v].description = graph->values[v].description;
        session->values[v].metadata = graph->values[v].metadata;
    }
    if (status == M3_STATUS_OK) {
        status = m3_graph_topology(graph, producers, last_uses, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_backend_create_preferred(
            selected.allow_metal || selected.allow_neural_engine,
            selected.allow_cpu || selected.allow_neural_engine,
            &session->backend, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_plan_slots(session, producers, last_uses, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_allocate_slots(session, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_build_views(session, graph, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_compile_nodes(session, graph, error);
    }
    if (status == M3_STATUS_OK) {
        status = m3_session_plan_runs(session, graph, error);
    }
    free(producers);
    free(last_uses);
    if (status != M3_STATUS_OK) {
        m3_session_free(session);
        return status;
    }
    *session_output = session;
    m3_error_reset(error);
    return M3_STATUS_OK;
}
