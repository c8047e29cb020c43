/*
 * m3_scratch.c - the host scratch arena passed to execute hooks.
 *
 * An arena is a caller-owned byte range with a fill offset; marks are
 * offsets, and rewinding moves the offset back to an earlier mark (never
 * forward). The contract of the reference's arena (src/m3_scratch.c:
 * 13-107): init needs a backing for a nonzero capacity, a rewind ahead of
 * the offset is OUT_OF_RANGE. No operation of this library takes scratch,
 * so nothing here hands bytes out.
 */
#include "m3_internal.h"

m3_status m3_scratch_arena_init(m3_scratch_arena *arena, void *data,
                                size_t capacity, m3_error *error)
{
    if (arena == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no scratch arena record to fill");
    }
    if (data == NULL && capacity != 0U) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "a %zu-byte scratch arena needs a backing",
                            capacity);
    }
    *arena = (m3_scratch_arena){(uint8_t *)data, capacity, 0U};
    m3_error_reset(error);
    return M3_STATUS_OK;
}

size_t m3_scratch_arena_mark(const m3_scratch_arena *arena)
{
    return arena != NULL ? arena->offset : 0U;
}

m3_status m3_scratch_arena_rewind(m3_scratch_arena *arena, size_t mark,
                                  m3_error *error)
{
    if (arena == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no scratch arena to rewind");
    }
    if (mark > arena->offset) {
        return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                            "mark %zu is ahead of the arena offset %zu",
                            mark, arena->offset);
    }
    arena->offset = mark;
    m3_error_reset(error);
    return M3_STATUS_OK;
}
