/*
 * m3_graph_builder.c - building graphs, and the output shapes of nodes.
 *
 * A graph only records: value specs and node descriptors are appended to
 * two lists, constant bytes are copied, and data flow is checked when a
 * session is compiled from the graph. Inference gives the shape (and for
 * some kinds the dtype) a node's output will have, for the kinds this
 * library runs.
 *
 * Observable contract kept from the reference builder (src/m3_graph.c:
 * 125-357, src/m3_graph_infer.c:41-272): the default descriptors and
 * options, the statuses of each call (OUT_OF_RANGE for a value id past
 * the graph, INVALID_ARGUMENT for a bad role or constant size, OVERFLOW
 * when ids run out, UNSUPPORTED for Core ML partitions and for inference
 * of kinds outside this library), and the inferred shapes: right-aligned
 * broadcast for ADD/MUL/SUB/DIV, the first input's shape otherwise; COPY
 * keeps the input dtype, SNAKE1D and TANH produce F32.
 */
#include "m3_session_internal.h"

#include <stdlib.h>
#include <string.h>

#define M3_LIST_FIRST 8U

/* Appends one item of `size` bytes, growing the list geometrically. */
static bool m3_list_push(m3_list *list, size_t size, const void *item)
{
    if (list->count == list->capacity) {
        size_t grown = list->capacity == 0U ? M3_LIST_FIRST
                                            : list->capacity * 2U;
        void *moved;

        if (grown < list->capacity || grown > SIZE_MAX / size) {
            return false;
        }
        moved = realloc(list->items, grown * size);
        if (moved == NULL) {
            return false;
        }
        list->items = moved;
        list->capacity = grown;
    }
    (void)memcpy((uint8_t *)list->items + list->count * size, item, size);
    list->count += 1U;
    return true;
}

void m3_graph_value_desc_init(m3_graph_value_desc *description,
                              m3_graph_value_role role, m3_dtype dtype,
                              uint8_t rank, const uint64_t *shape)
{
    uint8_t kept;

    if (description == NULL) {
        return;
    }
    (void)memset(description, 0, sizeof(*description));
    description->role = role;
    description->dtype = dtype;
    description->rank = rank;
    kept = rank < M3_TENSOR_MAX_RANK ? rank : (uint8_t)M3_TENSOR_MAX_RANK;
    if (shape != NULL && kept != 0U) {
        (void)memcpy(description->shape, shape, kept * sizeof(*shape));
    }
}

void m3_graph_node_desc_init(m3_graph_node_desc *description,
                             m3_op_kind kind)
{
    if (description == NULL) {
        return;
    }
    (void)memset(description, 0, sizeof(*description));
    description->kind = kind;
    /* M3_GRAPH_VALUE_NONE is all ones in every byte */
    (void)memset(description->inputs, 0xff, sizeof(description->inputs));
    (void)memset(description->outputs, 0xff, sizeof(description->outputs));
}

void m3_session_options_init(m3_session_options *options)
{
    if (options == NULL) {
        return;
    }
    *options = (m3_session_options){true, true, true};
}

m3_status m3_graph_create(m3_graph **graph, m3_error *error)
{
    if (graph == NULL || *graph != NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "pass the address of a NULL graph pointer");
    }
    *graph = calloc(1U, sizeof(**graph));
    if (*graph == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for a graph");
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

void m3_graph_free(m3_graph *graph)
{
    m3_value_spec *specs;
    size_t index;

    if (graph == NULL) {
        return;
    }
    specs = graph->values.items;
    for (index = 0U; index < graph->values.count; ++index) {
        free(specs[index].constant);
    }
    free(graph->values.items);
    free(graph->nodes.items);
    free(graph);
}

static bool m3_role_known(m3_graph_value_role role)
{
    return (unsigned int)role <= (unsigned int)M3_GRAPH_OUTPUT;
}

m3_status m3_graph_add_value(m3_graph *graph,
                             const m3_graph_value_desc *description,
                             m3_graph_value_id *value, m3_error *error)
{
    m3_value_spec spec;
    m3_status status;

    if (graph == NULL || description == NULL || value == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "adding a value needs a graph, a descriptor "
                            "and a place for the id");
    }
    if (!m3_role_known(description->role)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "value role %d is not INPUT, CONSTANT, "
                            "TEMPORARY or OUTPUT",
                            (int)description->role);
    }
    if (graph->values.count >= (size_t)M3_GRAPH_VALUE_NONE) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "the graph has used every value id");
    }
    (void)memset(&spec, 0, sizeof(spec));
    status = m3_tensor_metadata_init(&spec.meta, description->dtype,
                                     description->rank, description->shape,
                                     error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    spec.desc = *description;
    if (!m3_list_push(&graph->values, sizeof(spec), &spec)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for graph values");
    }
    *value = (m3_graph_value_id)(graph->values.count - 1U);
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_graph_set_constant(m3_graph *graph, m3_graph_value_id value,
                                const void *data, size_t byte_count,
                                m3_error *error)
{
    m3_value_spec *spec;
    uint8_t *copy = NULL;

    if (graph == NULL || (size_t)value >= graph->values.count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "constant value id %u is not in the graph",
                            (unsigned int)value);
    }
    spec = (m3_value_spec *)graph->values.items + value;
    if (spec->desc.role != M3_GRAPH_CONSTANT) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "value %u is not a CONSTANT",
                            (unsigned int)value);
    }
    if (byte_count != spec->meta.byte_count ||
        (data == NULL && byte_count != 0U)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "constant %u takes exactly %zu bytes of data",
                            (unsigned int)value, spec->meta.byte_count);
    }
    if (byte_count != 0U) {
        copy = malloc(byte_count);
        if (copy == NULL) {
            return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                                "out of host memory for a constant");
        }
        (void)memcpy(copy, data, byte_count);
    }
    free(spec->constant);
    spec->constant = copy;
    spec->constant_given = true;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_graph_add_node(m3_graph *graph,
                            const m3_graph_node_desc *description,
                            m3_error *error)
{
    if (graph == NULL || description == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "adding a node needs a graph and a descriptor");
    }
    if (!m3_list_push(&graph->nodes, sizeof(*description), description)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "out of host memory for graph nodes");
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_graph_add_coreml_partition(
    m3_graph *graph, const m3_coreml_partition_desc *description,
    m3_error *error)
{
    (void)graph;
    (void)description;
    return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                        "Core ML partitions need Apple frameworks, which "
                        "this library does not use");
}

/* ---- inference ---------------------------------------------------------- */

static m3_status m3_infer_operand(const m3_graph *graph,
                                  m3_graph_value_id value,
                                  const m3_tensor_metadata **meta,
                                  m3_error *error)
{
    if (value == M3_GRAPH_VALUE_NONE || (size_t)value >= graph->values.count) {
        *meta = NULL;
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "inference reads value %u, which the graph "
                            "does not have",
                            (unsigned int)value);
    }
    *meta = &m3_graph_value_at(graph, value)->meta;
    return M3_STATUS_OK;
}

/* Right-aligned broadcast of two shapes into `out`. */
static m3_status m3_infer_broadcast(const m3_tensor_metadata *a,
                                    const m3_tensor_metadata *b,
                                    m3_graph_value_desc *out,
                                    m3_error *error)
{
    const uint8_t rank = a->rank > b->rank ? a->rank : b->rank;
    uint8_t back;

    out->rank = rank;
    for (back = 1U; back <= rank; ++back) {
        const uint64_t da = back <= a->rank ? a->shape[a->rank - back] : 1U;
        const uint64_t db = back <= b->rank ? b->shape[b->rank - back] : 1U;

        if (da != db && da != 1U && db != 1U) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "extents %llu and %llu do not broadcast",
                                (unsigned long long)da,
                                (unsigned long long)db);
        }
        out->shape[rank - back] = da == 1U ? db : da;
    }
    return M3_STATUS_OK;
}

static m3_status m3_infer_output(const m3_graph *graph,
                                 const m3_graph_node_desc *node,
                                 size_t output_index,
                                 m3_graph_value_desc *out, m3_error *error)
{
    const m3_tensor_metadata *first = NULL;
    const m3_tensor_metadata *second = NULL;
    m3_status status = m3_infer_operand(graph, node->inputs[0], &first,
                                        error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (output_index != 0U && m3_op_kind_supported(node->kind)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "kind %d has a single output",
                            (int)node->kind);
    }
    switch (node->kind) {
    case M3_OP_ADD:
    case M3_OP_MUL:
    case M3_OP_SUB:
    case M3_OP_DIV:
        status = m3_infer_operand(graph, node->inputs[1], &second, error);
        return status != M3_STATUS_OK
                   ? status
                   : m3_infer_broadcast(first, second, out, error);
    case M3_OP_COPY:
        out->dtype = first->dtype;
        break;
    case M3_OP_SNAKE1D:
    case M3_OP_TANH:
        out->dtype = M3_DTYPE_F32;
        break;
    case M3_OP_CAST:
    case M3_OP_SOFTMAX:
    case M3_OP_GATED_SILU:
        break; /* the caller's dtype */
    default:
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "no output inference for kind %d",
                            (int)node->kind);
    }
    out->rank = first->rank;
    (void)memcpy(out->shape, first->shape, sizeof(out->shape));
    return M3_STATUS_OK;
}

m3_status m3_graph_add_inferred_value(m3_graph *graph,
                                      const m3_graph_node_desc *node,
                                      size_t output_index,
                                      m3_graph_value_role role,
                                      m3_dtype dtype,
                                      m3_graph_value_id *value,
                                      m3_error *error)
{
    m3_graph_value_desc out;
    m3_status status;

    if (graph == NULL || node == NULL || value == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "inference needs a graph, a node and a place "
                            "for the id");
    }
    if (role != M3_GRAPH_TEMPORARY && role != M3_GRAPH_OUTPUT) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "an inferred value is a TEMPORARY or an OUTPUT");
    }
    m3_graph_value_desc_init(&out, role, dtype, 0U, NULL);
    status = m3_infer_output(graph, node, output_index, &out, error);
    return status != M3_STATUS_OK
               ? status
               : m3_graph_add_value(graph, &out, value, error);
}
