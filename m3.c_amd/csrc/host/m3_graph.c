/*
 * m3_graph.c - graph construction and output-shape inference.
 *
 * Contracts follow the reference builder and inference:
 *   descriptor initialisers and options    src/m3_graph.c:125-170
 *   create/free, values, constants, nodes  src/m3_graph.c:172-357
 *   broadcast inference                    src/m3_graph_infer.c:41-63
 *   per-operation inference                src/m3_graph_infer.c:133-272
 * The graph copies descriptors and constant bytes; nothing is validated
 * against other values until a session is created. Inference covers the
 * operations this provider runs; other kinds report M3_STATUS_UNSUPPORTED.
 */
#include "m3_graph_internal.h"

#include <stdlib.h>
#include <string.h>

void m3_graph_value_desc_init(m3_graph_value_desc *description,
                              m3_graph_value_role role, m3_dtype dtype,
                              uint8_t rank, const uint64_t *shape)
{
    uint8_t axis;

    if (description == NULL) {
        return;
    }
    (void)memset(description, 0, sizeof(*description));
    description->role = role;
    description->dtype = dtype;
    description->rank = rank;
    for (axis = 0U; shape != NULL && axis < rank && axis < M3_TENSOR_MAX_RANK;
         ++axis) {
        description->shape[axis] = shape[axis];
    }
}

void m3_graph_node_desc_init(m3_graph_node_desc *description,
                             m3_op_kind kind)
{
    size_t index;

    if (description == NULL) {
        return;
    }
    (void)memset(description, 0, sizeof(*description));
    description->kind = kind;
    for (index = 0U; index < M3_GRAPH_NODE_INPUT_CAPACITY; ++index) {
        description->inputs[index] = M3_GRAPH_VALUE_NONE;
    }
    for (index = 0U; index < M3_GRAPH_NODE_OUTPUT_CAPACITY; ++index) {
        description->outputs[index] = M3_GRAPH_VALUE_NONE;
    }
}

void m3_session_options_init(m3_session_options *options)
{
    if (options != NULL) {
        options->allow_neural_engine = true;
        options->allow_metal = true;
        options->allow_cpu = true;
    }
}

m3_status m3_graph_create(m3_graph **graph, m3_error *error)
{
    m3_graph *created;

    if (graph == NULL || *graph != NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "graph output must be empty");
    }
    created = calloc(1U, sizeof(*created));
    if (created == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate graph");
    }
    *graph = created;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

void m3_graph_free(m3_graph *graph)
{
    size_t index;

    if (graph == NULL) {
        return;
    }
    for (index = 0U; index < graph->value_count; ++index) {
        free(graph->values[index].constant_data);
    }
    free(graph->values);
    free(graph->nodes);
    free(graph);
}

/* Doubles a growable array (starting at 8 entries). */
static bool m3_graph_grow(void **array, size_t *capacity, size_t entry_size)
{
    size_t wanted = *capacity == 0U ? 8U : *capacity * 2U;
    void *grown;

    if (wanted < *capacity || wanted > SIZE_MAX / entry_size) {
        return false;
    }
    grown = realloc(*array, wanted * entry_size);
    if (grown == NULL) {
        return false;
    }
    *array = grown;
    *capacity = wanted;
    return true;
}

m3_status m3_graph_add_value(m3_graph *graph,
                             const m3_graph_value_desc *description,
                             m3_graph_value_id *value, m3_error *error)
{
    m3_graph_value entry;
    m3_status status;

    if (graph == NULL || description == NULL || value == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "graph, value description, and output are "
                            "required");
    }
    if ((int)description->role < (int)M3_GRAPH_INPUT ||
        (int)description->role > (int)M3_GRAPH_OUTPUT) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "graph value role is invalid");
    }
    if (graph->value_count >= (size_t)M3_GRAPH_VALUE_NONE) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "graph value identifiers are exhausted");
    }
    (void)memset(&entry, 0, sizeof(entry));
    status = m3_tensor_metadata_init(&entry.metadata, description->dtype,
                                     description->rank, description->shape,
                                     error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    entry.description = *description;
    if (graph->value_count == graph->value_capacity &&
        !m3_graph_grow((void **)&graph->values, &graph->value_capacity,
                       sizeof(*graph->values))) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot grow graph values");
    }
    graph->values[graph->value_count] = entry;
    *value = (m3_graph_value_id)graph->value_count;
    graph->value_count += 1U;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_graph_set_constant(m3_graph *graph, m3_graph_value_id value,
                                const void *data, size_t byte_count,
                                m3_error *error)
{
    m3_graph_value *target;
    void *copy = NULL;

    if (graph == NULL || (size_t)value >= graph->value_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "constant graph value is out of range");
    }
    target = &graph->values[value];
    if (target->description.role != M3_GRAPH_CONSTANT ||
        byte_count != target->metadata.byte_count ||
        (byte_count != 0U && data == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "constant data does not match its graph value");
    }
    if (byte_count != 0U) {
        copy = malloc(byte_count);
        if (copy == NULL) {
            return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                                "cannot copy graph constant");
        }
        (void)memcpy(copy, data, byte_count);
    }
    free(target->constant_data);
    target->constant_data = copy;
    target->constant_size = byte_count;
    target->constant_set = true;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_graph_add_node(m3_graph *graph,
                            const m3_graph_node_desc *description,
                            m3_error *error)
{
    if (graph == NULL || description == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "graph and node description are required");
    }
    if (graph->node_count == graph->node_capacity &&
        !m3_graph_grow((void **)&graph->nodes, &graph->node_capacity,
                       sizeof(*graph->nodes))) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot grow graph nodes");
    }
    graph->nodes[graph->node_count] = *description;
    graph->node_count += 1U;
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
                        "Core ML partitions are not available on this "
                        "platform");
}

/* ---- inference --------------------------------------------------------- */

static m3_status m3_graph_infer_operand(const m3_graph *graph,
                                        m3_graph_value_id value,
                                        const m3_tensor_metadata **metadata,
                                        m3_error *error)
{
    *metadata = NULL;
    if (value == M3_GRAPH_VALUE_NONE || (size_t)value >= graph->value_count) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "inferred graph input is absent or out of "
                            "range");
    }
    *metadata = &graph->values[value].metadata;
    return M3_STATUS_OK;
}

static m3_status m3_graph_infer_shape(const m3_graph *graph,
                                      const m3_graph_node_desc *node,
                                      size_t output_index,
                                      m3_graph_value_desc *output,
                                      m3_error *error)
{
    const m3_tensor_metadata *first;
    const m3_tensor_metadata *second;
    m3_status status = m3_graph_infer_operand(graph, node->inputs[0], &first,
                                              error);
    uint8_t axis;

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (output_index != 0U && m3_op_kind_supported(node->kind)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "operation has no requested inferred output");
    }
    switch (node->kind) {
    case M3_OP_COPY:
    case M3_OP_CAST:
    case M3_OP_SOFTMAX:
    case M3_OP_SNAKE1D:
    case M3_OP_TANH:
        output->rank = first->rank;
        (void)memcpy(output->shape, first->shape, sizeof(output->shape));
        if (node->kind == M3_OP_COPY) {
            output->dtype = first->dtype;
        } else if (node->kind == M3_OP_SNAKE1D ||
                   node->kind == M3_OP_TANH) {
            output->dtype = M3_DTYPE_F32;
        }
        return M3_STATUS_OK;
    case M3_OP_GATED_SILU:
        /* the gate's shape; the dtype stays the requested one */
        output->rank = first->rank;
        (void)memcpy(output->shape, first->shape, sizeof(output->shape));
        return M3_STATUS_OK;
    case M3_OP_ADD:
    case M3_OP_MUL:
    case M3_OP_SUB:
    case M3_OP_DIV:
        status = m3_graph_infer_operand(graph, node->inputs[1], &second,
                                        error);
        if (status != M3_STATUS_OK) {
            return status;
        }
        output->rank = first->rank > second->rank ? first->rank
                                                  : second->rank;
        for (axis = 0U; axis < output->rank; ++axis) {
            int a = (int)axis - (int)(output->rank - first->rank);
            int b = (int)axis - (int)(output->rank - second->rank);
            uint64_t l = a < 0 ? 1U : first->shape[a];
            uint64_t r = b < 0 ? 1U : second->shape[b];

            if (l != r && l != 1U && r != 1U) {
                return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                    "inferred broadcast dimensions "
                                    "disagree");
            }
            output->shape[axis] = l == 1U ? r : l;
        }
        return M3_STATUS_OK;
    default:
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "cannot infer unsupported operation kind %d",
                            (int)node->kind);
    }
}

m3_status m3_graph_add_inferred_value(m3_graph *graph,
                                      const m3_graph_node_desc *node,
                                      size_t output_index,
                                      m3_graph_value_role role,
                                      m3_dtype dtype,
                                      m3_graph_value_id *value,
                                      m3_error *error)
{
    m3_graph_value_desc output;
    m3_status status;

    if (graph == NULL || node == NULL || value == NULL ||
        (role != M3_GRAPH_TEMPORARY && role != M3_GRAPH_OUTPUT)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "inferred graph value request is invalid");
    }
    (void)memset(&output, 0, sizeof(output));
    output.role = role;
    output.dtype = dtype;
    status = m3_graph_infer_shape(graph, node, output_index, &output, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    return m3_graph_add_value(graph, &output, value, error);
}
