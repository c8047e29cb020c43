/*
 * m3_backend.h - execution-provider plug-in interface of the m3 tensor-op
 * library: tensor views, storage, backends and command lists.
 *
 * The names, layouts and semantics follow the internal headers of
 * taconotsandwich/m3.c so that a provider written against this header also
 * builds inside the reference tree:
 *   tensor metadata and views   src/m3_tensor.h:12-69
 *   storage and backends        src/m3_backend.h:13-60
 *   backend vtable              src/m3_backend_internal.h:9-18
 *   scratch arena               src/m3_scratch.h
 *   commands                    src/m3_op.h:14-173
 *   error setter                src/m3_error.h
 *
 * Additions, each appended so existing layouts and values stay fixed:
 *   - M3_BACKEND_HIP and m3_backend_create_hip(), the AMD GPU provider that
 *     takes the place of m3_backend_create_metal (src/m3_backend.h:38);
 *   - vtable hooks `write`, `read` and `reserve`. When `write`/`read` are
 *     set, storage is device memory that the host cannot dereference:
 *     m3_storage_data() returns NULL and m3_storage_write/read go through
 *     the hooks. `reserve` lets the session compiler ask for one arena that
 *     later allocations are carved from;
 *   - SUB and DIV command descriptors (M3_OP_SUB/M3_OP_DIV);
 *   - the internal command kind M3_OP_ELEMENTWISE_PROGRAM, which the
 *     session compiler forms from runs of ADD/SUB/MUL/DIV commands; it has
 *     no counterpart in the reference and never appears in a graph.
 */
#ifndef M3_BACKEND_H
#define M3_BACKEND_H

#include "m3.h"

#include <stdarg.h>
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- errors (src/m3_error.h) ------------------------------------------ */

/* Sets *error (which may be NULL) and returns status. */
m3_status m3_error_set(m3_error *error, m3_status status,
                       const char *format, ...)
#if defined(__GNUC__)
    __attribute__((format(printf, 3, 4)))
#endif
    ;
m3_status m3_error_set_v(m3_error *error, m3_status status,
                         const char *format, va_list arguments);

/* ---- tensors (src/m3_tensor.h:12-69) ---------------------------------- */

typedef struct {
    m3_dtype dtype;
    uint8_t rank;
    uint64_t shape[M3_TENSOR_MAX_RANK];
    size_t element_count;
    size_t byte_count;
} m3_tensor_metadata;

typedef struct m3_storage m3_storage;
typedef struct m3_backend m3_backend;

typedef struct {
    m3_tensor_metadata metadata;
    size_t byte_offset;
    size_t byte_strides[M3_TENSOR_MAX_RANK];
    m3_storage *storage;
} m3_tensor_view;

const char *m3_dtype_name(m3_dtype dtype);
size_t m3_dtype_size(m3_dtype dtype);
m3_status m3_tensor_metadata_init(m3_tensor_metadata *metadata,
                                  m3_dtype dtype, uint8_t rank,
                                  const uint64_t *shape, m3_error *error);
void m3_tensor_view_init(m3_tensor_view *tensor);
/* Views borrow storage and become invalid when the storage is freed. */
m3_status m3_tensor_view_contiguous(m3_tensor_view *tensor,
                                    m3_storage *storage,
                                    m3_dtype dtype, uint8_t rank,
                                    const uint64_t *shape,
                                    size_t byte_offset, m3_error *error);
m3_status m3_tensor_view_strided(m3_tensor_view *tensor,
                                 m3_storage *storage,
                                 m3_dtype dtype, uint8_t rank,
                                 const uint64_t *shape,
                                 const size_t *byte_strides,
                                 size_t byte_offset, m3_error *error);
bool m3_tensor_is_contiguous(const m3_tensor_view *tensor);
/* Validates the view; *data is the host address of its first element, or
 * NULL when the storage is device memory. */
m3_status m3_tensor_const_data(const m3_tensor_view *tensor,
                               const void **data, m3_error *error);
m3_status m3_tensor_data(m3_tensor_view *tensor, void **data,
                         m3_error *error);
m3_status m3_tensor_element_offset(const m3_tensor_view *tensor,
                                   const uint64_t *indices,
                                   size_t *byte_offset, m3_error *error);
m3_status m3_tensor_slice(const m3_tensor_view *source, uint8_t axis,
                          uint64_t start, uint64_t length,
                          m3_tensor_view *view, m3_error *error);
m3_status m3_tensor_reshape(const m3_tensor_view *source, uint8_t rank,
                            const uint64_t *shape, m3_tensor_view *view,
                            m3_error *error);
m3_status m3_tensor_permute(const m3_tensor_view *source,
                            const uint8_t *permutation,
                            m3_tensor_view *view, m3_error *error);

/* ---- scratch arena (src/m3_scratch.h) --------------------------------- */

typedef struct {
    uint8_t *data;
    size_t capacity;
    size_t offset;
} m3_scratch_arena;

m3_status m3_scratch_arena_init(m3_scratch_arena *arena, void *data,
                                size_t capacity, m3_error *error);
size_t m3_scratch_arena_mark(const m3_scratch_arena *arena);
m3_status m3_scratch_arena_rewind(m3_scratch_arena *arena, size_t mark,
                                  m3_error *error);

/* ---- commands (src/m3_op.h:14-148) ------------------------------------ */

typedef struct {
    const m3_tensor_view *input;
    m3_tensor_view *output;
} m3_op_unary;

typedef struct {
    const m3_tensor_view *left;
    const m3_tensor_view *right;
    m3_tensor_view *output;
} m3_op_binary;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *alpha;
    m3_tensor_view *output;
} m3_op_snake1d;

/* Descriptors of operations this provider does not run. They are declared
 * only so that m3_command has the reference layout. */
typedef struct {
    const m3_tensor_view *ids;
    const m3_tensor_view *table;
    m3_tensor_view *output;
} m3_op_embedding;

typedef struct {
    const m3_tensor_view *left;
    const m3_tensor_view *right;
    m3_tensor_view *output;
} m3_op_matmul;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *weight;
    const m3_tensor_view *bias;
    m3_tensor_view *output;
} m3_op_linear;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *scale;
    m3_tensor_view *output;
    float epsilon;
} m3_op_rms_norm;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *scale;
    const m3_tensor_view *bias;
    m3_tensor_view *output;
    float epsilon;
} m3_op_layer_norm;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *cosines;
    const m3_tensor_view *sines;
    m3_tensor_view *output;
    uint64_t position_offset;
    uint32_t rotary_dimension;
    m3_rope_mode mode;
} m3_op_rope;

typedef struct {
    const m3_tensor_view *query;
    const m3_tensor_view *key;
    const m3_tensor_view *value;
    const m3_tensor_view *mask;
    m3_tensor_view *output;
    float scale;
    int64_t causal_offset;
    bool causal;
} m3_op_attention;

typedef struct {
    const m3_tensor_view *logits;
    m3_tensor_view *values;
    m3_tensor_view *indices;
    uint64_t k;
} m3_op_top_k;

typedef struct {
    const m3_tensor_view *probabilities;
    const m3_tensor_view *uniforms;
    m3_tensor_view *output;
} m3_op_categorical;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *weight;
    const m3_tensor_view *bias;
    m3_tensor_view *output;
    uint64_t groups;
    uint64_t stride;
    uint64_t dilation;
    uint64_t pad_left;
    uint64_t pad_right;
} m3_op_conv1d;

typedef struct {
    const m3_tensor_view *input;
    const m3_tensor_view *weight;
    const m3_tensor_view *bias;
    m3_tensor_view *output;
    uint64_t groups;
    uint64_t stride;
    uint64_t dilation;
    uint64_t pad_left;
    uint64_t pad_right;
    uint64_t output_padding;
} m3_op_conv_transpose1d;

/* A run of F32 ADD/SUB/MUL/DIV commands over one element space that the
 * session compiler fused into one elementwise program (layout: see
 * m3_hip_launch_program in m3_hip.h). `commands` are the original
 * commands, in order: they are validated as usual and define the result.
 * `words` is the program in host memory; the same words are in `storage`
 * at `byte_offset`. Intermediate values that only the run reads are not
 * written to their slots. */
#define M3_OP_ELEMENTWISE_PROGRAM ((m3_op_kind)0x1000)

struct m3_command_s;

typedef struct {
    const struct m3_command_s *commands;
    size_t command_count;
    const uint32_t *words;
    size_t word_count;
    m3_storage *storage;
    size_t byte_offset;
} m3_op_elementwise_program;

typedef struct m3_command_s {
    m3_op_kind kind;
    union {
        m3_op_unary copy;
        m3_op_unary cast;
        m3_op_binary add;
        m3_op_binary mul;
        m3_op_embedding embedding;
        m3_op_matmul matmul;
        m3_op_linear linear;
        m3_op_rms_norm rms_norm;
        m3_op_layer_norm layer_norm;
        m3_op_rope rope;
        m3_op_attention attention;
        m3_op_binary gated_silu;
        m3_op_unary softmax;
        m3_op_top_k top_k;
        m3_op_categorical categorical;
        m3_op_conv1d conv1d;
        m3_op_conv_transpose1d conv_transpose1d;
        m3_op_unary nearest_resize1d;
        m3_op_snake1d snake1d;
        m3_op_unary tanh;
        m3_op_binary sub;
        m3_op_binary div;
        m3_op_elementwise_program elementwise_program;
    } descriptor;
} m3_command;

/* Commands borrow their views. Inputs may be strided; outputs are
 * contiguous. ADD/MUL/SUB/DIV load each operand as F32, apply one F32
 * operation and round once to the output dtype. SOFTMAX maps an all
 * -INFINITY row to zeros and splits probability equally among +INFINITY
 * entries when any are present. SNAKE1D rounds each of its seven F32
 * statements and uses the epsilon bits 0x3089705f. */

/* Structural validation of one command against a backend. */
m3_status m3_command_validate(const m3_backend *backend,
                              const m3_command *command, m3_error *error);
/* Validates a list and reports the scratch bytes it needs. */
m3_status m3_commands_scratch_bytes(const m3_backend *backend,
                                    const m3_command *commands,
                                    size_t command_count,
                                    size_t *scratch_bytes, m3_error *error);
/* Validates the whole list, then hands it to the backend's execute hook. */
m3_status m3_backend_execute(m3_backend *backend, const m3_command *commands,
                             size_t command_count, m3_scratch_arena *scratch,
                             m3_error *error);

/* ---- backends and storage (src/m3_backend.h:13-60) -------------------- */

#define M3_BACKEND_NAME_CAPACITY 128U

typedef enum {
    M3_BACKEND_HOST = 0,
    M3_BACKEND_METAL,
    M3_BACKEND_HIP
} m3_backend_kind;

typedef struct {
    char name[M3_BACKEND_NAME_CAPACITY];
    m3_backend_kind kind;
    bool unified_memory;
    uint64_t recommended_working_set_bytes;
    uint64_t maximum_storage_bytes;
} m3_backend_info;

typedef struct {
    size_t live_allocated_bytes;
    size_t peak_allocated_bytes;
    size_t live_storage_count;
    size_t peak_storage_count;
} m3_backend_allocation_stats;

/* Backend lifetime contract (src/m3_backend_internal.h:9-18) plus four
 * optional hooks. destroy_context, allocate, free_storage and execute are
 * required. write/read copy between host memory and storage `data` at a
 * byte offset; both set means the storage is device memory. reserve asks
 * for one arena of `byte_count` bytes from which later allocations may be
 * carved. finish waits until every command executed so far has completed
 * and reports a failure that surfaced while they ran; a backend with a
 * finish hook may return from execute once the commands are queued (write,
 * read and destroy_context still see their results). */
typedef struct {
    void (*destroy_context)(void *context);
    m3_status (*allocate)(void *context, size_t byte_count, size_t alignment,
                          void **handle, void **data, m3_error *error);
    void (*free_storage)(void *context, void *handle, void *data);
    m3_status (*execute)(void *context, const m3_command *commands,
                         size_t command_count, m3_scratch_arena *scratch,
                         m3_error *error);
    m3_status (*write)(void *context, void *data, size_t byte_offset,
                       const void *source, size_t byte_count,
                       m3_error *error);
    m3_status (*read)(void *context, const void *data, size_t byte_offset,
                      void *destination, size_t byte_count,
                      m3_error *error);
    m3_status (*reserve)(void *context, size_t byte_count, m3_error *error);
    m3_status (*finish)(void *context, m3_error *error);
} m3_backend_vtable;

m3_status m3_backend_create_internal(const m3_backend_vtable *vtable,
                                     void *context,
                                     const m3_backend_info *info,
                                     m3_backend **backend, m3_error *error);
/* Host memory executed by the CPU provider (src/m3_backend.h:37). The HIP
 * backend's constructor is in m3_backend_hip.h. */
m3_status m3_backend_create_host(m3_backend **backend, m3_error *error);
void m3_backend_free(m3_backend *backend);
m3_status m3_backend_get_info(const m3_backend *backend,
                              m3_backend_info *info, m3_error *error);
m3_status m3_backend_get_allocation_stats(
    const m3_backend *backend, m3_backend_allocation_stats *stats,
    m3_error *error);
/* Requests one arena for the allocations that follow (no-op for backends
 * without a reserve hook). */
m3_status m3_backend_reserve(m3_backend *backend, size_t byte_count,
                             m3_error *error);
void *m3_backend_context_internal(const m3_backend *backend);
/* Waits until every command executed on `backend` so far has completed
 * (no-op for backends that complete commands inside execute). Sessions
 * call it at the end of m3_session_run; callers of m3_backend_execute or
 * m3_command_executor_execute call it when they need the commands done
 * without reading a storage. */
m3_status m3_backend_finish(m3_backend *backend, m3_error *error);

m3_status m3_storage_allocate(m3_backend *backend, size_t byte_count,
                              size_t alignment, m3_storage **storage,
                              m3_error *error);
void m3_storage_free(m3_storage *storage);
size_t m3_storage_size(const m3_storage *storage);
/* Host address of the storage; NULL for device storage. */
void *m3_storage_data(m3_storage *storage);
const void *m3_storage_const_data(const m3_storage *storage);
/* Backend address of the storage (device pointer for device storage). */
void *m3_storage_device_data(const m3_storage *storage);
void *m3_storage_handle_internal(const m3_storage *storage);
m3_backend *m3_storage_backend(const m3_storage *storage);
bool m3_storage_host_visible(const m3_storage *storage);
m3_status m3_storage_write(m3_storage *storage, size_t byte_offset,
                           const void *source, size_t byte_count,
                           m3_error *error);
m3_status m3_storage_read(const m3_storage *storage, size_t byte_offset,
                          void *destination, size_t byte_count,
                          m3_error *error);

/* ---- non-graph command lists (src/m3_runtime_workspace.h:41-53) ------ */

/* Runs command lists outside any graph, the way flow and conditioning code
 * of the reference call the provider (src/m3_command_executor.c:55-92):
 * validate, size scratch, select a provider, execute. The backend is
 * borrowed and must outlive the executor. */
typedef struct {
    m3_backend *backend;
    void *scratch;
    size_t scratch_capacity;
} m3_command_executor;

void m3_command_executor_init(m3_command_executor *executor,
                              m3_backend *backend);
void m3_command_executor_dispose(m3_command_executor *executor);
m3_status m3_command_executor_execute(m3_command_executor *executor,
                                      const m3_command *commands,
                                      size_t command_count,
                                      m3_error *error);

/* ---- measurement and test seams (no reference counterpart) ----------- */

/* Replaces the constructor the scheduler uses for the GPU storage backend;
 * NULL restores m3_backend_create_hip. Lets the graph compiler run against
 * a recording backend on machines without a GPU. */
typedef m3_status (*m3_backend_factory)(m3_backend **backend,
                                        m3_error *error);
void m3_provider_set_gpu_factory(m3_backend_factory factory);
/* The storage backend a session owns. */
m3_backend *m3_session_backend(const m3_session *session);
/* The m3_hip_device behind a HIP backend, or NULL for other backends. */
void *m3_backend_hip_device(const m3_backend *backend);

#ifdef __cplusplus
}
#endif

#endif
