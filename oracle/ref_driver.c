/*
 * ref_driver.c - runs one command on the compiled reference CPU provider.
 *
 * TEST INFRASTRUCTURE ONLY. Built by oracle/Makefile together with the
 * reference's own op-layer sources (read in place from the reference tree)
 * into oracle/_ref/libm3ref.so; used to pin the oracle restatement. Each
 * distinct host buffer becomes one reference host storage, so views that
 * share a buffer alias exactly as they would in the reference.
 */
#include "m3_backend.h"
#include "m3_op.h"
#include "m3_tensor.h"

#include <stdlib.h>
#include <string.h>

typedef struct {
    void *data;       /* host buffer */
    size_t bytes;     /* buffer size */
    uint64_t byte_offset;
    uint32_t dtype;
    uint32_t rank;
    uint64_t shape[8];
    uint64_t byte_strides[8];
} ref_view;

#define REF_MAX_VIEWS 4

int ref_execute(int kind, const ref_view *views, size_t count, char *message,
                size_t capacity);

int ref_execute(int kind, const ref_view *views, size_t count, char *message,
                size_t capacity)
{
    m3_backend *backend = NULL;
    m3_storage *storages[REF_MAX_VIEWS] = {NULL};
    void *owners[REF_MAX_VIEWS] = {NULL};
    size_t sizes[REF_MAX_VIEWS] = {0};
    size_t storage_count = 0U;
    m3_tensor_view tensors[REF_MAX_VIEWS];
    m3_command command;
    m3_error error;
    m3_status status;
    size_t i;

    m3_error_reset(&error);
    if (count == 0U || count > REF_MAX_VIEWS) {
        return (int)M3_STATUS_INVALID_ARGUMENT;
    }
    status = m3_backend_create_host(&backend, &error);
    for (i = 0U; status == M3_STATUS_OK && i < count; ++i) {
        size_t s;
        size_t strides[8];
        uint32_t axis;

        for (s = 0U; s < storage_count; ++s) {
            if (owners[s] == views[i].data) {
                break;
            }
        }
        if (s == storage_count) {
            status = m3_storage_allocate(backend, views[i].bytes, 64U,
                                         &storages[s], &error);
            if (status == M3_STATUS_OK) {
                status = m3_storage_write(storages[s], 0U, views[i].data,
                                          views[i].bytes, &error);
            }
            owners[s] = views[i].data;
            sizes[s] = views[i].bytes;
            storage_count += 1U;
        }
        for (axis = 0U; axis < views[i].rank && axis < 8U; ++axis) {
            strides[axis] = (size_t)views[i].byte_strides[axis];
        }
        m3_tensor_view_init(&tensors[i]);
        if (status == M3_STATUS_OK) {
            status = m3_tensor_view_strided(
                &tensors[i], storages[s], (m3_dtype)views[i].dtype,
                (uint8_t)views[i].rank, views[i].shape, strides,
                (size_t)views[i].byte_offset, &error);
        }
    }
    if (status == M3_STATUS_OK) {
        memset(&command, 0, sizeof(command));
        command.kind = (m3_op_kind)kind;
        switch (command.kind) {
        case M3_OP_ADD:
        case M3_OP_MUL:
            command.descriptor.add.left = &tensors[0];
            command.descriptor.add.right = &tensors[1];
            command.descriptor.add.output = &tensors[2];
            break;
        case M3_OP_GATED_SILU:
            command.descriptor.gated_silu.left = &tensors[0];
            command.descriptor.gated_silu.right = &tensors[1];
            command.descriptor.gated_silu.output = &tensors[2];
            break;
        case M3_OP_TANH:
            command.descriptor.tanh.input = &tensors[0];
            command.descriptor.tanh.output = &tensors[1];
            break;
        case M3_OP_SNAKE1D:
            command.descriptor.snake1d.input = &tensors[0];
            command.descriptor.snake1d.alpha = &tensors[1];
            command.descriptor.snake1d.output = &tensors[2];
            break;
        default:
            command.descriptor.copy.input = &tensors[0];
            command.descriptor.copy.output = &tensors[1];
            break;
        }
        status = m3_backend_execute(backend, &command, 1U, NULL, &error);
    }
    for (i = 0U; status == M3_STATUS_OK && i < storage_count; ++i) {
        status = m3_storage_read(storages[i], 0U, owners[i], sizes[i],
                                 &error);
    }
    if (message != NULL && capacity != 0U) {
        strncpy(message, m3_error_message(&error), capacity - 1U);
        message[capacity - 1U] = '\0';
    }
    for (i = 0U; i < storage_count; ++i) {
        m3_storage_free(storages[i]);
    }
    m3_backend_free(backend);
    return (int)status;
}
