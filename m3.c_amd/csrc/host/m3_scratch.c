/*
 * m3_scratch.c - host scratch arena handed to execute hooks.
 *
 * Same contract as src/m3_scratch.c:13-107 of the reference (init, mark,
 * rewind). The operations this provider runs need no scratch, so no
 * allocation entry is exported.
 */
#include "m3_internal.h"

m3_status m3_scratch_arena_init(m3_scratch_arena *arena, void *data,
                                size_t capacity, m3_error *error)
{
    if (arena == NULL || (capacity != 0U && data == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "scratch arena and nonempty backing are "
                            "required");
    }
    arena->data = data;
    arena->capacity = capacity;
    arena->offset = 0U;
    m3_error_reset(error);
    return M3_STATUS_OK;
}

size_t m3_scratch_arena_mark(const m3_scratch_arena *arena)
{
    return arena == NULL ? 0U : arena->offset;
}

m3_status m3_scratch_arena_rewind(m3_scratch_arena *arena, size_t mark,
                                  m3_error *error)
{
    if (arena == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "scratch arena is null");
    }
    if (mark > arena->offset) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "scratch rewind mark is ahead of current offset");
    }
    arena->offset = mark;
    m3_error_reset(error);
    return M3_STATUS_OK;
}
