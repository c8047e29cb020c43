/*
 * m3_tensor.c - tensor metadata and strided views over backend storage.
 *
 * Contracts follow the reference tensor layer:
 *   metadata init with overflow checks      src/m3_tensor.c:38-102
 *   view construction and bounds checks     src/m3_tensor_runtime.c:94-220
 *   contiguity test                          src/m3_tensor_runtime.c:222-248
 *   slice / reshape / permute                src/m3_tensor_runtime.c:359-477
 * A view is valid when its offset and strides are multiples of the element
 * size and every element lies inside the storage. Failed view constructors
 * leave the output view zeroed.
 */
#include "m3_internal.h"

#include <string.h>

const char *m3_dtype_name(m3_dtype dtype)
{
    switch (dtype) {
    case M3_DTYPE_F32:
        return "F32";
    case M3_DTYPE_F16:
        return "F16";
    case M3_DTYPE_BF16:
        return "BF16";
    case M3_DTYPE_I32:
        return "I32";
    }
    return "unknown";
}

size_t m3_dtype_size(m3_dtype dtype)
{
    switch (dtype) {
    case M3_DTYPE_F32:
    case M3_DTYPE_I32:
        return 4U;
    case M3_DTYPE_F16:
    case M3_DTYPE_BF16:
        return 2U;
    }
    return 0U;
}

m3_status m3_tensor_metadata_init(m3_tensor_metadata *metadata,
                                  m3_dtype dtype, uint8_t rank,
                                  const uint64_t *shape, m3_error *error)
{
    size_t elements = 1U;
    size_t element_size;
    uint8_t axis;

    if (metadata == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor metadata output is null");
    }
    (void)memset(metadata, 0, sizeof(*metadata));
    element_size = m3_dtype_size(dtype);
    if (element_size == 0U) {
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "unsupported tensor dtype value %d", (int)dtype);
    }
    if (rank > M3_TENSOR_MAX_RANK) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "tensor rank %u exceeds maximum rank %u",
                            (unsigned int)rank,
                            (unsigned int)M3_TENSOR_MAX_RANK);
    }
    if (rank != 0U && shape == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor shape is null for rank %u",
                            (unsigned int)rank);
    }
    for (axis = 0U; axis < rank; ++axis) {
        if (shape[axis] > (uint64_t)SIZE_MAX) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "tensor dimension %u does not fit size_t",
                                (unsigned int)axis);
        }
        if (!m3_size_mul_checked(elements, (size_t)shape[axis], &elements)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "tensor element count overflows at "
                                "dimension %u", (unsigned int)axis);
        }
    }
    if (!m3_size_mul_checked(elements, element_size,
                             &metadata->byte_count)) {
        metadata->byte_count = 0U;
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "tensor byte count overflows size_t");
    }
    metadata->dtype = dtype;
    metadata->rank = rank;
    for (axis = 0U; axis < rank; ++axis) {
        metadata->shape[axis] = shape[axis];
    }
    metadata->element_count = elements;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* Row-major byte strides; all zero for an empty tensor. */
static m3_status m3_tensor_row_major_strides(const m3_tensor_metadata *meta,
                                             size_t *strides,
                                             m3_error *error)
{
    size_t stride = m3_dtype_size(meta->dtype);
    uint8_t axis = meta->rank;

    (void)memset(strides, 0, M3_TENSOR_MAX_RANK * sizeof(*strides));
    if (meta->element_count == 0U) {
        return M3_STATUS_OK;
    }
    while (axis > 0U) {
        --axis;
        strides[axis] = stride;
        if (!m3_size_mul_checked(stride, (size_t)meta->shape[axis],
                                 &stride)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "tensor stride overflows at axis %u",
                                (unsigned int)axis);
        }
    }
    return M3_STATUS_OK;
}

static m3_status m3_tensor_check(const m3_tensor_view *tensor,
                                 m3_error *error)
{
    m3_tensor_metadata fresh;
    size_t element_size;
    size_t storage_bytes;
    size_t last;
    const void *base;
    uint8_t axis;
    m3_status status;

    if (tensor == NULL || tensor->storage == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor view is not initialized");
    }
    status = m3_tensor_metadata_init(&fresh, tensor->metadata.dtype,
                                     tensor->metadata.rank,
                                     tensor->metadata.shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (fresh.element_count != tensor->metadata.element_count ||
        fresh.byte_count != tensor->metadata.byte_count) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor metadata counts are inconsistent");
    }
    storage_bytes = m3_storage_size(tensor->storage);
    if (tensor->byte_offset > storage_bytes) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "tensor byte offset exceeds storage");
    }
    element_size = m3_dtype_size(fresh.dtype);
    if (tensor->byte_offset % element_size != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor byte offset is misaligned");
    }
    base = m3_storage_device_data(tensor->storage);
    if (base != NULL && (uintptr_t)base % element_size != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor storage pointer is misaligned");
    }
    for (axis = 0U; axis < fresh.rank; ++axis) {
        if (tensor->byte_strides[axis] % element_size != 0U) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "tensor stride %u is misaligned",
                                (unsigned int)axis);
        }
    }
    if (fresh.element_count == 0U) {
        return M3_STATUS_OK;
    }
    last = tensor->byte_offset;
    for (axis = 0U; axis < fresh.rank; ++axis) {
        size_t reach;

        if (!m3_size_mul_checked((size_t)(fresh.shape[axis] - 1U),
                                 tensor->byte_strides[axis], &reach) ||
            !m3_size_add_checked(last, reach, &last)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "tensor view bounds overflow");
        }
    }
    if (!m3_size_add_checked(last, element_size, &last)) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "tensor view end overflows");
    }
    if (last > storage_bytes) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "tensor view exceeds storage");
    }
    return M3_STATUS_OK;
}

void m3_tensor_view_init(m3_tensor_view *tensor)
{
    if (tensor != NULL) {
        (void)memset(tensor, 0, sizeof(*tensor));
    }
}

static m3_status m3_tensor_fresh_output(m3_tensor_view *tensor,
                                        m3_error *error)
{
    if (tensor == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor output is null");
    }
    if (tensor->storage != NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor output already describes a view");
    }
    return M3_STATUS_OK;
}

static m3_status m3_tensor_finish(m3_tensor_view *tensor, m3_error *error)
{
    m3_status status = m3_tensor_check(tensor, error);

    if (status != M3_STATUS_OK) {
        m3_tensor_view_init(tensor);
        return status;
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_tensor_view_strided(m3_tensor_view *tensor,
                                 m3_storage *storage, m3_dtype dtype,
                                 uint8_t rank, const uint64_t *shape,
                                 const size_t *byte_strides,
                                 size_t byte_offset, m3_error *error)
{
    m3_tensor_metadata metadata;
    m3_status status = m3_tensor_fresh_output(tensor, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (storage == NULL || (rank != 0U && byte_strides == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor storage and strides are required");
    }
    status = m3_tensor_metadata_init(&metadata, dtype, rank, shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    tensor->metadata = metadata;
    tensor->byte_offset = byte_offset;
    tensor->storage = storage;
    if (rank != 0U) {
        (void)memcpy(tensor->byte_strides, byte_strides,
                     (size_t)rank * sizeof(*byte_strides));
    }
    return m3_tensor_finish(tensor, error);
}

m3_status m3_tensor_view_contiguous(m3_tensor_view *tensor,
                                    m3_storage *storage, m3_dtype dtype,
                                    uint8_t rank, const uint64_t *shape,
                                    size_t byte_offset, m3_error *error)
{
    m3_tensor_metadata metadata;
    size_t strides[M3_TENSOR_MAX_RANK];
    m3_status status = m3_tensor_metadata_init(&metadata, dtype, rank, shape,
                                               error);

    if (status == M3_STATUS_OK) {
        status = m3_tensor_row_major_strides(&metadata, strides, error);
    }
    if (status != M3_STATUS_OK) {
        return status;
    }
    return m3_tensor_view_strided(tensor, storage, dtype, rank, shape,
                                  strides, byte_offset, error);
}

bool m3_tensor_is_contiguous(const m3_tensor_view *tensor)
{
    size_t expected;
    uint8_t axis;

    if (tensor == NULL || tensor->storage == NULL) {
        return false;
    }
    if (tensor->metadata.element_count == 0U) {
        return true;
    }
    expected = m3_dtype_size(tensor->metadata.dtype);
    axis = tensor->metadata.rank;
    while (axis > 0U) {
        --axis;
        if (tensor->metadata.shape[axis] > 1U &&
            tensor->byte_strides[axis] != expected) {
            return false;
        }
        if (!m3_size_mul_checked(expected,
                                 (size_t)tensor->metadata.shape[axis],
                                 &expected)) {
            return false;
        }
    }
    return true;
}

m3_status m3_tensor_const_data(const m3_tensor_view *tensor,
                               const void **data, m3_error *error)
{
    const uint8_t *base;
    m3_status status;

    if (data == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor data output is null");
    }
    *data = NULL;
    status = m3_tensor_check(tensor, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    base = m3_storage_const_data(tensor->storage);
    if (base != NULL) {
        *data = base + tensor->byte_offset;
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_tensor_data(m3_tensor_view *tensor, void **data,
                         m3_error *error)
{
    const void *read_only = NULL;
    m3_status status;

    if (data == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor data output is null");
    }
    *data = NULL;
    status = m3_tensor_const_data(tensor, &read_only, error);
    if (status == M3_STATUS_OK) {
        *data = (void *)(uintptr_t)read_only;
    }
    return status;
}

m3_status m3_tensor_element_offset(const m3_tensor_view *tensor,
                                   const uint64_t *indices,
                                   size_t *byte_offset, m3_error *error)
{
    size_t offset;
    uint8_t axis;
    m3_status status;

    if (byte_offset == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor element offset output is null");
    }
    *byte_offset = 0U;
    status = m3_tensor_check(tensor, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (tensor->metadata.rank != 0U && indices == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor indices are null");
    }
    offset = tensor->byte_offset;
    for (axis = 0U; axis < tensor->metadata.rank; ++axis) {
        size_t step;

        if (indices[axis] >= tensor->metadata.shape[axis]) {
            return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                                "tensor index exceeds axis %u",
                                (unsigned int)axis);
        }
        if (!m3_size_mul_checked((size_t)indices[axis],
                                 tensor->byte_strides[axis], &step) ||
            !m3_size_add_checked(offset, step, &offset)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "tensor element offset overflows");
        }
    }
    *byte_offset = offset;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

static m3_status m3_tensor_derive_begin(const m3_tensor_view *source,
                                        m3_tensor_view *view,
                                        m3_error *error)
{
    m3_status status = m3_tensor_fresh_output(view, error);

    return status == M3_STATUS_OK ? m3_tensor_check(source, error) : status;
}

m3_status m3_tensor_slice(const m3_tensor_view *source, uint8_t axis,
                          uint64_t start, uint64_t length,
                          m3_tensor_view *view, m3_error *error)
{
    uint64_t shape[M3_TENSOR_MAX_RANK];
    size_t offset;
    m3_status status = m3_tensor_derive_begin(source, view, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (axis >= source->metadata.rank ||
        start > source->metadata.shape[axis] ||
        length > source->metadata.shape[axis] - start) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "tensor slice exceeds axis bounds");
    }
    if (!m3_size_mul_checked((size_t)start, source->byte_strides[axis],
                             &offset) ||
        !m3_size_add_checked(source->byte_offset, offset, &offset)) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "tensor slice offset overflows");
    }
    (void)memcpy(shape, source->metadata.shape, sizeof(shape));
    shape[axis] = length;
    *view = *source;
    view->byte_offset = offset;
    status = m3_tensor_metadata_init(&view->metadata, source->metadata.dtype,
                                     source->metadata.rank, shape, error);
    if (status != M3_STATUS_OK) {
        m3_tensor_view_init(view);
        return status;
    }
    return m3_tensor_finish(view, error);
}

m3_status m3_tensor_reshape(const m3_tensor_view *source, uint8_t rank,
                            const uint64_t *shape, m3_tensor_view *view,
                            m3_error *error)
{
    m3_tensor_metadata metadata;
    m3_status status = m3_tensor_derive_begin(source, view, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (!m3_tensor_is_contiguous(source)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "cannot reshape a non-contiguous tensor");
    }
    status = m3_tensor_metadata_init(&metadata, source->metadata.dtype, rank,
                                     shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (metadata.element_count != source->metadata.element_count) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "reshape changes tensor element count");
    }
    status = m3_tensor_row_major_strides(&metadata, view->byte_strides,
                                         error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    view->metadata = metadata;
    view->byte_offset = source->byte_offset;
    view->storage = source->storage;
    return m3_tensor_finish(view, error);
}

m3_status m3_tensor_permute(const m3_tensor_view *source,
                            const uint8_t *permutation,
                            m3_tensor_view *view, m3_error *error)
{
    bool used[M3_TENSOR_MAX_RANK] = {false};
    uint64_t shape[M3_TENSOR_MAX_RANK];
    m3_tensor_metadata metadata;
    uint8_t axis;
    m3_status status = m3_tensor_derive_begin(source, view, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (source->metadata.rank != 0U && permutation == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "tensor permutation is null");
    }
    for (axis = 0U; axis < source->metadata.rank; ++axis) {
        uint8_t from = permutation[axis];

        if (from >= source->metadata.rank || used[from]) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "tensor permutation axis %u is invalid",
                                (unsigned int)from);
        }
        used[from] = true;
        shape[axis] = source->metadata.shape[from];
    }
    status = m3_tensor_metadata_init(&metadata, source->metadata.dtype,
                                     source->metadata.rank, shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    *view = *source;
    view->metadata = metadata;
    for (axis = 0U; axis < source->metadata.rank; ++axis) {
        view->byte_strides[axis] = source->byte_strides[permutation[axis]];
    }
    return m3_tensor_finish(view, error);
}
