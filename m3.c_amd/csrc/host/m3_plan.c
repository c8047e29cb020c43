/*
 * m3_plan.c - data-flow checks and liveness slots of a graph.
 *
 * Data flow. Every CONSTANT must have its bytes. Nodes are then taken in
 * order, and each is held to its kind's arity (m3_plan_arity): the
 * operand positions it uses hold ids of the graph, the others hold
 * M3_GRAPH_VALUE_NONE; it reads only values that exist by then (INPUT and
 * CONSTANT values exist from the start, the rest once produced); it
 * writes only TEMPORARY or OUTPUT values, none twice. At the end every
 * TEMPORARY and OUTPUT value must have been produced. The first failing
 * rule, in that order, decides the status.
 *
 * Slots. A value's live range runs from its producer (or the start) to
 * the last node that reads or writes it. INPUT, CONSTANT and OUTPUT values
 * each own a slot for the whole session. Going through the nodes in
 * order, a TEMPORARY written by node n takes, among the slots whose live
 * range ended before n, the smallest one that holds it, or opens a slot of
 * its own size. This is the reference's rule (src/m3_graph_compile.c:
 * 260-324): plan info reports the same slot count and bytes, which the
 * reference's KAT pins (6 values, 4 nodes -> 5 slots, 80 bytes).
 *
 * The arena that holds the slots is sized here too: every slot rounded up
 * to the 256-byte granule the device allocator carves at.
 */
#include "m3_session_internal.h"

#include <stdlib.h>
#include <string.h>

#define M3_ARENA_GRANULE 256U

typedef struct {
    size_t reads;
    size_t writes;
} m3_arity;

/* Operand positions of the kinds this library compiles; UNSUPPORTED for
 * the others. */
static m3_status m3_plan_arity(m3_op_kind kind, m3_arity *arity,
                               m3_error *error)
{
    switch (kind) {
    case M3_OP_COPY:
    case M3_OP_CAST:
    case M3_OP_SOFTMAX:
    case M3_OP_TANH:
        *arity = (m3_arity){1U, 1U};
        return M3_STATUS_OK;
    case M3_OP_ADD:
    case M3_OP_MUL:
    case M3_OP_SUB:
    case M3_OP_DIV:
    case M3_OP_SNAKE1D:
    case M3_OP_GATED_SILU:
        *arity = (m3_arity){2U, 1U};
        return M3_STATUS_OK;
    default:
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "graph node kind %d is outside this library",
                            (int)kind);
    }
}

/* One operand position: `used` says whether the kind reads/writes it. */
static m3_status m3_plan_operand(m3_graph_value_id id, bool used,
                                 size_t value_count, size_t node,
                                 const char *role, m3_error *error)
{
    if (!used) {
        return id == M3_GRAPH_VALUE_NONE
                   ? M3_STATUS_OK
                   : m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                  "node %zu names an %s its kind does "
                                  "not take",
                                  node, role);
    }
    if (id == M3_GRAPH_VALUE_NONE) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "node %zu leaves a required %s empty", node,
                            role);
    }
    if ((size_t)id >= value_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "node %zu names %s %u, past the graph's values",
                            node, role, (unsigned int)id);
    }
    return M3_STATUS_OK;
}

static m3_status m3_plan_node_shape(const m3_graph_node_desc *node,
                                    size_t index, size_t value_count,
                                    m3_arity *arity, m3_error *error)
{
    m3_status status = m3_plan_arity(node->kind, arity, error);
    size_t k;

    for (k = 0U; status == M3_STATUS_OK && k < M3_GRAPH_NODE_INPUT_CAPACITY;
         ++k) {
        status = m3_plan_operand(node->inputs[k], k < arity->reads,
                                 value_count, index, "input", error);
    }
    for (k = 0U;
         status == M3_STATUS_OK && k < M3_GRAPH_NODE_OUTPUT_CAPACITY; ++k) {
        status = m3_plan_operand(node->outputs[k], k < arity->writes,
                                 value_count, index, "output", error);
    }
    return status;
}

/* Data flow of the graph (file comment); fills producer and last. */
static m3_status m3_plan_flow(const m3_graph *graph, size_t *producer,
                              size_t *last, m3_error *error)
{
    const size_t count = graph->values.count;
    size_t v;
    size_t n;

    for (v = 0U; v < count; ++v) {
        const m3_value_spec *spec = m3_graph_value_at(graph, v);

        producer[v] = M3_NO_NODE;
        last[v] = 0U;
        if (spec->desc.role == M3_GRAPH_CONSTANT && !spec->constant_given) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "constant %zu was never given its bytes",
                                v);
        }
    }
    for (n = 0U; n < graph->nodes.count; ++n) {
        const m3_graph_node_desc *node = m3_graph_node_at(graph, n);
        m3_arity arity = {0U, 0U};
        size_t k;
        m3_status status = m3_plan_node_shape(node, n, count, &arity, error);

        if (status != M3_STATUS_OK) {
            return status;
        }
        for (k = 0U; k < arity.reads; ++k) {
            const size_t in = node->inputs[k];
            const m3_graph_value_role role =
                m3_graph_value_at(graph, in)->desc.role;

            if (producer[in] == M3_NO_NODE && role != M3_GRAPH_INPUT &&
                role != M3_GRAPH_CONSTANT) {
                return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                    "node %zu reads value %zu before any "
                                    "node writes it",
                                    n, in);
            }
            last[in] = n;
        }
        for (k = 0U; k < arity.writes; ++k) {
            const size_t out = node->outputs[k];
            const m3_graph_value_role role =
                m3_graph_value_at(graph, out)->desc.role;
            size_t j;

            if (role != M3_GRAPH_TEMPORARY && role != M3_GRAPH_OUTPUT) {
                return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                    "node %zu writes value %zu, an INPUT "
                                    "or CONSTANT",
                                    n, out);
            }
            if (producer[out] != M3_NO_NODE) {
                return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                    "value %zu is written by nodes %zu "
                                    "and %zu",
                                    out, producer[out], n);
            }
            for (j = 0U; j < k; ++j) {
                if (node->outputs[j] == node->outputs[k]) {
                    return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                        "node %zu lists output %zu twice", n,
                                        out);
                }
            }
            producer[out] = n;
            last[out] = n;
        }
    }
    for (v = 0U; v < count; ++v) {
        const m3_graph_value_role role = m3_graph_value_at(graph, v)->desc.role;

        if (producer[v] == M3_NO_NODE &&
            (role == M3_GRAPH_TEMPORARY || role == M3_GRAPH_OUTPUT)) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "no node writes value %zu", v);
        }
    }
    return M3_STATUS_OK;
}

/* Slot assignment (file comment). free_after[s] is the last node using
 * slot s, SIZE_MAX for a slot owned for the whole session. */
static void m3_plan_slots(const m3_graph *graph, const size_t *producer,
                          const size_t *last, m3_plan *plan,
                          size_t *free_after)
{
    const size_t count = graph->values.count;
    size_t v;
    size_t n;

    for (v = 0U; v < count; ++v) {
        const m3_value_spec *spec = m3_graph_value_at(graph, v);

        plan->slot_of[v] = SIZE_MAX;
        if (spec->desc.role != M3_GRAPH_TEMPORARY) {
            plan->slot_bytes[plan->slot_count] = spec->meta.byte_count;
            free_after[plan->slot_count] = SIZE_MAX;
            plan->slot_of[v] = plan->slot_count++;
        }
    }
    for (n = 0U; n < graph->nodes.count; ++n) {
        const m3_graph_node_desc *node = m3_graph_node_at(graph, n);
        size_t k;

        for (k = 0U; k < M3_GRAPH_NODE_OUTPUT_CAPACITY; ++k) {
            const m3_graph_value_id out = node->outputs[k];
            size_t need;
            size_t best = SIZE_MAX;
            size_t s;

            if (out == M3_GRAPH_VALUE_NONE || producer[out] != n ||
                m3_graph_value_at(graph, out)->desc.role !=
                    M3_GRAPH_TEMPORARY) {
                continue;
            }
            need = m3_graph_value_at(graph, out)->meta.byte_count;
            for (s = 0U; s < plan->slot_count; ++s) {
                const bool idle = free_after[s] < n;
                const bool fits = plan->slot_bytes[s] >= need;

                if (idle && fits &&
                    (best == SIZE_MAX ||
                     plan->slot_bytes[s] < plan->slot_bytes[best])) {
                    best = s;
                }
            }
            if (best == SIZE_MAX) {
                best = plan->slot_count++;
                plan->slot_bytes[best] = need;
            }
            plan->slot_of[out] = best;
            free_after[best] = last[out];
        }
    }
}

static m3_status m3_plan_totals(m3_plan *plan, m3_error *error)
{
    size_t s;

    for (s = 0U; s < plan->slot_count; ++s) {
        const size_t bytes = plan->slot_bytes[s];
        size_t rounded;

        if (!m3_size_add_checked(plan->plain_bytes, bytes,
                                 &plan->plain_bytes) ||
            !m3_size_add_checked(bytes, M3_ARENA_GRANULE - 1U, &rounded) ||
            !m3_size_add_checked(plan->arena_bytes,
                                 rounded & ~(size_t)(M3_ARENA_GRANULE - 1U),
                                 &plan->arena_bytes)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "the graph's slots total more than size_t "
                                "holds");
        }
    }
    return M3_STATUS_OK;
}

void m3_plan_release(m3_plan *plan)
{
    if (plan != NULL) {
        free(plan->slot_of);
        free(plan->slot_bytes);
        (void)memset(plan, 0, sizeof(*plan));
    }
}

m3_status m3_plan_build(const m3_graph *graph, m3_plan *plan,
                        m3_error *error)
{
    const size_t count = graph->values.count;
    const size_t cells = count == 0U ? 1U : count;
    size_t *producer = malloc(cells * sizeof(*producer));
    size_t *last = malloc(cells * sizeof(*last));
    size_t *free_after = malloc(cells * sizeof(*free_after));
    m3_status status;

    (void)memset(plan, 0, sizeof(*plan));
    plan->count = count;
    plan->slot_of = malloc(cells * sizeof(*plan->slot_of));
    plan->slot_bytes = malloc(cells * sizeof(*plan->slot_bytes));
    if (producer == NULL || last == NULL || free_after == NULL ||
        plan->slot_of == NULL || plan->slot_bytes == NULL) {
        status = m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                              "out of host memory for the liveness plan");
    } else {
        status = m3_plan_flow(graph, producer, last, error);
    }
    if (status == M3_STATUS_OK) {
        m3_plan_slots(graph, producer, last, plan, free_after);
        status = m3_plan_totals(plan, error);
    }
    free(producer);
    free(last);
    free(free_after);
    if (status != M3_STATUS_OK) {
        m3_plan_release(plan);
    }
    return status;
}
