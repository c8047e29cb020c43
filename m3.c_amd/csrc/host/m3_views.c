/*
 * m3_views.c - tensor metadata and strided views over storages.
 *
 * A view is (metadata, byte offset, byte strides, storage). It is sound
 * when its metadata re-derives from dtype, rank and shape, its offset and
 * strides are whole elements, and the furthest element it can reach ends
 * inside its storage (m3_view_audit). Constructors and the derived views
 * (slice, reshape, permute) build the candidate view in place and audit it;
 * a rejected candidate leaves the output zeroed.
 *
 * The statuses and the order of the checks are those callers of the
 * reference observe (src/m3_tensor.c:38-102, src/m3_tensor_runtime.c:
 * 94-477): a bad dtype is UNSUPPORTED, a rank above 8 OUT_OF_RANGE, sizes
 * that do not fit size_t OVERFLOW, misalignment INVALID_ARGUMENT and a
 * view past its storage OUT_OF_RANGE.
 */
#include "m3_internal.h"

#include <string.h>

const char *m3_dtype_name(m3_dtype dtype)
{
    static const char *const names[] = {"F32", "F16", "BF16", "I32"};

    return (unsigned int)dtype < 4U ? names[dtype] : "unknown";
}

size_t m3_dtype_size(m3_dtype dtype)
{
    static const size_t sizes[] = {4U, 2U, 2U, 4U};

    return (unsigned int)dtype < 4U ? sizes[dtype] : 0U;
}

m3_status m3_tensor_metadata_init(m3_tensor_metadata *metadata,
                                  m3_dtype dtype, uint8_t rank,
                                  const uint64_t *shape, m3_error *error)
{
    const size_t element_size = m3_dtype_size(dtype);
    size_t count = 1U;
    uint8_t axis;

    if (metadata == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no metadata record to fill");
    }
    (void)memset(metadata, 0, sizeof(*metadata));
    if (element_size == 0U) {
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "dtype %d is not one of F32, F16, BF16, I32",
                            (int)dtype);
    }
    if (rank > M3_TENSOR_MAX_RANK) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "rank %u is above the limit of %u",
                            (unsigned int)rank,
                            (unsigned int)M3_TENSOR_MAX_RANK);
    }
    if (shape == NULL && rank != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "a rank-%u tensor needs a shape",
                            (unsigned int)rank);
    }
    for (axis = 0U; axis < rank; ++axis) {
        if (shape[axis] > (uint64_t)SIZE_MAX ||
            !m3_size_mul_checked(count, (size_t)shape[axis], &count)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "element count overflows size_t at axis %u",
                                (unsigned int)axis);
        }
    }
    if (!m3_size_mul_checked(count, element_size, &metadata->byte_count)) {
        metadata->byte_count = 0U;
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "%zu elements of %zu bytes overflow size_t",
                            count, element_size);
    }
    metadata->dtype = dtype;
    metadata->rank = rank;
    if (rank != 0U) {
        (void)memcpy(metadata->shape, shape, (size_t)rank * sizeof(*shape));
    }
    metadata->element_count = count;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* Dense row-major strides of `metadata`; every stride is 0 when the
 * tensor is empty. */
static m3_status m3_dense_strides(const m3_tensor_metadata *metadata,
                                  size_t strides[M3_TENSOR_MAX_RANK],
                                  m3_error *error)
{
    size_t step = m3_dtype_size(metadata->dtype);
    int axis;

    (void)memset(strides, 0, M3_TENSOR_MAX_RANK * sizeof(*strides));
    if (metadata->element_count == 0U) {
        return M3_STATUS_OK;
    }
    for (axis = (int)metadata->rank - 1; axis >= 0; --axis) {
        strides[axis] = step;
        if (!m3_size_mul_checked(step, (size_t)metadata->shape[axis],
                                 &step)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "row-major stride overflows at axis %d",
                                axis);
        }
    }
    return M3_STATUS_OK;
}

/* One past the last byte a non-empty view can touch. */
static m3_status m3_view_reach(const m3_tensor_view *view, size_t *end,
                               m3_error *error)
{
    size_t reach = view->byte_offset;
    uint8_t axis;

    for (axis = 0U; axis < view->metadata.rank; ++axis) {
        size_t span;

        if (!m3_size_mul_checked((size_t)view->metadata.shape[axis] - 1U,
                                 view->byte_strides[axis], &span) ||
            !m3_size_add_checked(reach, span, &reach)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "view extent overflows size_t");
        }
    }
    if (!m3_size_add_checked(reach,
                             m3_dtype_size(view->metadata.dtype), end)) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "view extent overflows size_t");
    }
    return M3_STATUS_OK;
}

/* Soundness of a view (see the file comment). */
static m3_status m3_view_audit(const m3_tensor_view *view, m3_error *error)
{
    m3_tensor_metadata derived;
    size_t element_size;
    size_t capacity;
    size_t end = 0U;
    uintptr_t base;
    uint8_t axis;
    m3_status status;

    if (view == NULL || view->storage == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "view has no storage");
    }
    status = m3_tensor_metadata_init(&derived, view->metadata.dtype,
                                     view->metadata.rank,
                                     view->metadata.shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (derived.element_count != view->metadata.element_count ||
        derived.byte_count != view->metadata.byte_count) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "view element or byte count disagrees with its "
                            "shape");
    }
    capacity = m3_storage_size(view->storage);
    if (view->byte_offset > capacity) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "view offset %zu is past its %zu-byte storage",
                            view->byte_offset, capacity);
    }
    element_size = m3_dtype_size(derived.dtype);
    if (view->byte_offset % element_size != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "view offset is not a whole number of "
                            "elements");
    }
    base = (uintptr_t)m3_storage_device_data(view->storage);
    if (base % element_size != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "storage address is not element aligned");
    }
    for (axis = 0U; axis < derived.rank; ++axis) {
        if (view->byte_strides[axis] % element_size != 0U) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "stride of axis %u is not a whole number of "
                                "elements",
                                (unsigned int)axis);
        }
    }
    if (derived.element_count == 0U) {
        return M3_STATUS_OK;
    }
    status = m3_view_reach(view, &end, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (end > capacity) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "view reaches byte %zu of a %zu-byte storage",
                            end, capacity);
    }
    return M3_STATUS_OK;
}

/* Keeps a candidate view that passes the audit, else zeroes it. */
static m3_status m3_view_settle(m3_tensor_view *view, m3_error *error)
{
    m3_status status = m3_view_audit(view, error);

    if (status != M3_STATUS_OK) {
        (void)memset(view, 0, sizeof(*view));
        return status;
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* A view output must exist and not already describe a view. */
static m3_status m3_view_blank(const m3_tensor_view *view, m3_error *error)
{
    if (view == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no view record to fill");
    }
    if (view->storage != NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "view record is in use; initialize it first");
    }
    return M3_STATUS_OK;
}

void m3_tensor_view_init(m3_tensor_view *tensor)
{
    if (tensor != NULL) {
        (void)memset(tensor, 0, sizeof(*tensor));
    }
}

m3_status m3_tensor_view_strided(m3_tensor_view *tensor,
                                 m3_storage *storage, m3_dtype dtype,
                                 uint8_t rank, const uint64_t *shape,
                                 const size_t *byte_strides,
                                 size_t byte_offset, m3_error *error)
{
    m3_tensor_metadata metadata;
    m3_status status = m3_view_blank(tensor, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (storage == NULL || (byte_strides == NULL && rank != 0U)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "a strided view needs a storage and strides");
    }
    status = m3_tensor_metadata_init(&metadata, dtype, rank, shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    tensor->metadata = metadata;
    tensor->storage = storage;
    tensor->byte_offset = byte_offset;
    if (rank != 0U) {
        (void)memcpy(tensor->byte_strides, byte_strides,
                     (size_t)rank * sizeof(*byte_strides));
    }
    return m3_view_settle(tensor, error);
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
        status = m3_dense_strides(&metadata, strides, error);
    }
    return status != M3_STATUS_OK
               ? status
               : m3_tensor_view_strided(tensor, storage, dtype, rank, shape,
                                        strides, byte_offset, error);
}

bool m3_tensor_is_contiguous(const m3_tensor_view *tensor)
{
    size_t dense[M3_TENSOR_MAX_RANK];
    uint8_t axis;

    if (tensor == NULL || tensor->storage == NULL) {
        return false;
    }
    if (tensor->metadata.element_count == 0U) {
        return true;
    }
    if (m3_dense_strides(&tensor->metadata, dense, NULL) != M3_STATUS_OK) {
        return false;
    }
    /* an axis of extent 1 is never stepped, whatever its stride */
    for (axis = 0U; axis < tensor->metadata.rank; ++axis) {
        if (tensor->metadata.shape[axis] != 1U &&
            tensor->byte_strides[axis] != dense[axis]) {
            return false;
        }
    }
    return true;
}

m3_status m3_tensor_const_data(const m3_tensor_view *tensor,
                               const void **data, m3_error *error)
{
    const uint8_t *host;
    m3_status status;

    if (data == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no place to return the data address");
    }
    *data = NULL;
    status = m3_view_audit(tensor, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    host = m3_storage_const_data(tensor->storage);
    *data = host == NULL ? NULL : host + tensor->byte_offset;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

m3_status m3_tensor_data(m3_tensor_view *tensor, void **data,
                         m3_error *error)
{
    const void *address = NULL;
    m3_status status;

    if (data == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no place to return the data address");
    }
    status = m3_tensor_const_data(tensor, &address, error);
    *data = (void *)(uintptr_t)address;
    return status;
}

m3_status m3_tensor_element_offset(const m3_tensor_view *tensor,
                                   const uint64_t *indices,
                                   size_t *byte_offset, m3_error *error)
{
    size_t at;
    uint8_t axis;
    m3_status status;

    if (byte_offset == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no place to return the element offset");
    }
    *byte_offset = 0U;
    status = m3_view_audit(tensor, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (indices == NULL && tensor->metadata.rank != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "element offset needs one index per axis");
    }
    at = tensor->byte_offset;
    for (axis = 0U; axis < tensor->metadata.rank; ++axis) {
        size_t step;

        if (indices[axis] >= tensor->metadata.shape[axis]) {
            return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                                "index %llu is outside axis %u of extent "
                                "%llu",
                                (unsigned long long)indices[axis],
                                (unsigned int)axis,
                                (unsigned long long)
                                    tensor->metadata.shape[axis]);
        }
        if (!m3_size_mul_checked((size_t)indices[axis],
                                 tensor->byte_strides[axis], &step) ||
            !m3_size_add_checked(at, step, &at)) {
            return m3_error_set(error, M3_STATUS_OVERFLOW,
                                "element offset overflows size_t");
        }
    }
    *byte_offset = at;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

/* Common start of the derived views: a blank output and a sound source. */
static m3_status m3_derive_start(const m3_tensor_view *source,
                                 const m3_tensor_view *view, m3_error *error)
{
    m3_status status = m3_view_blank(view, error);

    return status != M3_STATUS_OK ? status : m3_view_audit(source, error);
}

m3_status m3_tensor_slice(const m3_tensor_view *source, uint8_t axis,
                          uint64_t start, uint64_t length,
                          m3_tensor_view *view, m3_error *error)
{
    m3_tensor_view candidate;
    uint64_t shape[M3_TENSOR_MAX_RANK];
    size_t skip;
    m3_status status = m3_derive_start(source, view, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (axis >= source->metadata.rank ||
        start > source->metadata.shape[axis] ||
        length > source->metadata.shape[axis] - start) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "slice [%llu, +%llu) does not fit axis %u",
                            (unsigned long long)start,
                            (unsigned long long)length, (unsigned int)axis);
    }
    if (!m3_size_mul_checked((size_t)start, source->byte_strides[axis],
                             &skip) ||
        !m3_size_add_checked(source->byte_offset, skip, &skip)) {
        return m3_error_set(error, M3_STATUS_OVERFLOW,
                            "slice offset overflows size_t");
    }
    candidate = *source;
    (void)memcpy(shape, source->metadata.shape, sizeof(shape));
    shape[axis] = length;
    status = m3_tensor_metadata_init(&candidate.metadata,
                                     source->metadata.dtype,
                                     source->metadata.rank, shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    candidate.byte_offset = skip;
    *view = candidate;
    return m3_view_settle(view, error);
}

m3_status m3_tensor_reshape(const m3_tensor_view *source, uint8_t rank,
                            const uint64_t *shape, m3_tensor_view *view,
                            m3_error *error)
{
    m3_tensor_view candidate;
    m3_status status = m3_derive_start(source, view, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (!m3_tensor_is_contiguous(source)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "only a row-major view can be reshaped");
    }
    (void)memset(&candidate, 0, sizeof(candidate));
    status = m3_tensor_metadata_init(&candidate.metadata,
                                     source->metadata.dtype, rank, shape,
                                     error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (candidate.metadata.element_count != source->metadata.element_count) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "reshape from %zu to %zu elements",
                            source->metadata.element_count,
                            candidate.metadata.element_count);
    }
    status = m3_dense_strides(&candidate.metadata, candidate.byte_strides,
                              error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    candidate.storage = source->storage;
    candidate.byte_offset = source->byte_offset;
    *view = candidate;
    return m3_view_settle(view, error);
}

m3_status m3_tensor_permute(const m3_tensor_view *source,
                            const uint8_t *permutation,
                            m3_tensor_view *view, m3_error *error)
{
    m3_tensor_view candidate;
    uint64_t shape[M3_TENSOR_MAX_RANK];
    uint32_t taken = 0U;
    uint8_t axis;
    m3_status status = m3_derive_start(source, view, error);

    if (status != M3_STATUS_OK) {
        return status;
    }
    if (permutation == NULL && source->metadata.rank != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "permute needs one source axis per axis");
    }
    candidate = *source;
    for (axis = 0U; axis < source->metadata.rank; ++axis) {
        const uint8_t from = permutation[axis];

        if (from >= source->metadata.rank || (taken >> from & 1U) != 0U) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "permutation names axis %u twice or out of "
                                "range",
                                (unsigned int)from);
        }
        taken |= 1U << from;
        shape[axis] = source->metadata.shape[from];
        candidate.byte_strides[axis] = source->byte_strides[from];
    }
    status = m3_tensor_metadata_init(&candidate.metadata,
                                     source->metadata.dtype,
                                     source->metadata.rank, shape, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    *view = candidate;
    return m3_view_settle(view, error);
}
