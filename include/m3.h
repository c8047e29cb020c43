/*
 * m3.h - public graph/session API of the m3 tensor-op library, MI355X build.
 *
 * This header keeps the public surface of taconotsandwich/m3.c
 * (include/m3.h:20-259) so that existing callers compile unchanged: every
 * enumerator value, struct layout and prototype below matches the reference.
 * Two additions are appended after the last reference enumerator so that no
 * existing value moves:
 *   - M3_OP_SUB and M3_OP_DIV (elementwise subtraction and division; the
 *     reference has only ADD and MUL, include/m3.h:52-73);
 *   - M3_PROVIDER_HIP (the AMD GPU execution provider; the reference lists
 *     NEURAL_ENGINE, METAL and CPU, include/m3.h:80-84).
 * m3_session_options.allow_metal keeps its name and means "allow the
 * platform GPU provider"; in this library that provider is HIP on gfx950.
 *
 * The Music3 model engine (include/m3.h:155-291) is a model adapter and is
 * not part of this library.
 */
#ifndef M3_H
#define M3_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define M3_VERSION_MAJOR 0
#define M3_VERSION_MINOR 1
#define M3_VERSION_PATCH 0
#define M3_VERSION_STRING "0.1.0"

#define M3_TENSOR_MAX_RANK 8U
#define M3_GRAPH_NODE_INPUT_CAPACITY 5U
#define M3_GRAPH_NODE_OUTPUT_CAPACITY 2U
#define M3_GRAPH_VALUE_NONE UINT32_MAX

/* Reference: include/m3.h:20-31. */
typedef enum {
    M3_STATUS_OK = 0,
    M3_STATUS_INVALID_ARGUMENT = 1,
    M3_STATUS_OUT_OF_RANGE = 2,
    M3_STATUS_OVERFLOW = 3,
    M3_STATUS_OUT_OF_MEMORY = 4,
    M3_STATUS_IO = 5,
    M3_STATUS_INVALID_FORMAT = 6,
    M3_STATUS_UNSUPPORTED = 7,
    M3_STATUS_CANCELLED = 8,
    M3_STATUS_INTERNAL = 9
} m3_status;

#define M3_ERROR_MESSAGE_CAPACITY 256U

/* Reference: include/m3.h:35-38. */
typedef struct {
    m3_status status;
    char message[M3_ERROR_MESSAGE_CAPACITY];
} m3_error;

typedef struct {
    const char *data;
    size_t length;
} m3_text_view;

/* Reference: include/m3.h:45-50. */
typedef enum {
    M3_DTYPE_F32 = 0,
    M3_DTYPE_F16,
    M3_DTYPE_BF16,
    M3_DTYPE_I32
} m3_dtype;

/* Reference: include/m3.h:52-73; SUB and DIV appended. */
typedef enum {
    M3_OP_COPY = 0,
    M3_OP_CAST,
    M3_OP_ADD,
    M3_OP_MUL,
    M3_OP_EMBEDDING,
    M3_OP_MATMUL,
    M3_OP_LINEAR,
    M3_OP_RMS_NORM,
    M3_OP_LAYER_NORM,
    M3_OP_ROPE,
    M3_OP_ATTENTION,
    M3_OP_GATED_SILU,
    M3_OP_SOFTMAX,
    M3_OP_TOP_K,
    M3_OP_CATEGORICAL,
    M3_OP_CONV1D,
    M3_OP_CONV_TRANSPOSE1D,
    M3_OP_NEAREST_RESIZE1D,
    M3_OP_SNAKE1D,
    M3_OP_TANH,
    M3_OP_SUB,
    M3_OP_DIV
} m3_op_kind;

typedef enum {
    M3_ROPE_HALF_SPLIT = 0,
    M3_ROPE_INTERLEAVED
} m3_rope_mode;

/* Reference: include/m3.h:80-84; HIP appended. */
typedef enum {
    M3_PROVIDER_NEURAL_ENGINE = 0,
    M3_PROVIDER_METAL,
    M3_PROVIDER_CPU,
    M3_PROVIDER_HIP
} m3_provider_kind;

typedef enum {
    M3_GRAPH_INPUT = 0,
    M3_GRAPH_CONSTANT,
    M3_GRAPH_TEMPORARY,
    M3_GRAPH_OUTPUT
} m3_graph_value_role;

typedef uint32_t m3_graph_value_id;

/* Reference: include/m3.h:95-100. */
typedef struct {
    m3_dtype dtype;
    uint8_t rank;
    uint64_t shape[M3_TENSOR_MAX_RANK];
    m3_graph_value_role role;
} m3_graph_value_desc;

/* Reference: include/m3.h:102-133. The parameter union is kept whole so the
 * descriptor layout matches callers built against the reference. */
typedef struct {
    m3_op_kind kind;
    m3_graph_value_id inputs[M3_GRAPH_NODE_INPUT_CAPACITY];
    m3_graph_value_id outputs[M3_GRAPH_NODE_OUTPUT_CAPACITY];
    union {
        struct {
            float epsilon;
        } norm;
        struct {
            uint64_t position_offset;
            uint32_t rotary_dimension;
            m3_rope_mode mode;
        } rope;
        struct {
            float scale;
            int64_t causal_offset;
            bool causal;
        } attention;
        struct {
            uint64_t k;
        } top_k;
        struct {
            uint64_t groups;
            uint64_t stride;
            uint64_t dilation;
            uint64_t pad_left;
            uint64_t pad_right;
            uint64_t output_padding;
        } convolution;
        struct {
            uint64_t output_length;
        } resize;
    } parameters;
} m3_graph_node_desc;

typedef struct {
    const char *compiled_model_path;
    const m3_graph_value_id *inputs;
    const char *const *input_names;
    size_t input_count;
    const m3_graph_value_id *outputs;
    const char *const *output_names;
    size_t output_count;
} m3_coreml_partition_desc;

/* Reference: include/m3.h:147-151. allow_metal enables the platform GPU
 * provider (HIP here). */
typedef struct {
    bool allow_neural_engine;
    bool allow_metal;
    bool allow_cpu;
} m3_session_options;

typedef struct {
    size_t value_count;
    size_t node_count;
    size_t storage_slot_count;
    size_t allocated_bytes;
} m3_session_plan_info;

typedef struct m3_graph m3_graph;
typedef struct m3_session m3_session;

const char *m3_version(void);
const char *m3_status_string(m3_status status);
void m3_error_reset(m3_error *error);
const char *m3_error_message(const m3_error *error);

void m3_graph_value_desc_init(m3_graph_value_desc *description,
                              m3_graph_value_role role, m3_dtype dtype,
                              uint8_t rank, const uint64_t *shape);
void m3_graph_node_desc_init(m3_graph_node_desc *description,
                             m3_op_kind kind);
void m3_session_options_init(m3_session_options *options);

/* Graph construction. Reference: include/m3.h:209-229. */
m3_status m3_graph_create(m3_graph **graph, m3_error *error);
void m3_graph_free(m3_graph *graph);
m3_status m3_graph_add_value(m3_graph *graph,
                             const m3_graph_value_desc *description,
                             m3_graph_value_id *value, m3_error *error);
m3_status m3_graph_set_constant(m3_graph *graph,
                                m3_graph_value_id value,
                                const void *data, size_t byte_count,
                                m3_error *error);
m3_status m3_graph_add_inferred_value(
    m3_graph *graph, const m3_graph_node_desc *node,
    size_t output_index, m3_graph_value_role role, m3_dtype dtype,
    m3_graph_value_id *value, m3_error *error);

/* Regular nodes use the fixed input/output positions of their operation;
 * optional inputs use M3_GRAPH_VALUE_NONE. The graph copies the descriptor;
 * data flow is validated when a session is created. */
m3_status m3_graph_add_node(m3_graph *graph,
                            const m3_graph_node_desc *description,
                            m3_error *error);

/* Core ML partitions need Apple frameworks. In this library the call
 * records nothing and returns M3_STATUS_UNSUPPORTED. */
m3_status m3_graph_add_coreml_partition(
    m3_graph *graph, const m3_coreml_partition_desc *description,
    m3_error *error);

/* A session owns its storage backend and compiled plan; the graph may be
 * freed after creation. With allow_metal the storage is the HIP device's
 * and regular nodes run on the HIP provider (M3_STATUS_UNSUPPORTED when no
 * HIP device is present); with only allow_cpu the storage is host memory
 * and nodes run on the CPU provider. Sessions are not thread-safe.
 * Reference: include/m3.h:240-259. */
m3_status m3_session_create(m3_session **session, const m3_graph *graph,
                             const m3_session_options *options,
                             m3_error *error);
void m3_session_free(m3_session *session);
m3_status m3_session_write_input(m3_session *session,
                                  m3_graph_value_id value,
                                  const void *data, size_t byte_count,
                                  m3_error *error);
m3_status m3_session_read_output(const m3_session *session,
                                  m3_graph_value_id value,
                                  void *data, size_t byte_count,
                                  m3_error *error);
m3_status m3_session_run(m3_session *session, m3_error *error);
m3_status m3_session_get_plan_info(const m3_session *session,
                                    m3_session_plan_info *info,
                                    m3_error *error);
m3_status m3_session_get_node_provider(const m3_session *session,
                                        size_t node_index,
                                        m3_provider_kind *provider,
                                        m3_error *error);

#ifdef __cplusplus
}
#endif

#endif
