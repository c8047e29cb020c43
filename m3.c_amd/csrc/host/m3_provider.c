/*
 * m3_provider.c - the scheduler: which backend holds a session's storage,
 * and which provider runs each command list.
 *
 * Storage. With the GPU provider allowed (allow_metal, or the neural
 * engine option, which here means "any provider") the storage is the HIP
 * device's. When the HIP backend cannot be made because there is no usable
 * device (its constructor says UNSUPPORTED) and the CPU provider is
 * allowed, the storage is host memory (m3_host_backend.c) and every list
 * runs on the CPU provider, as the reference falls back from Metal
 * (src/m3_provider.c:46-58); any other failure of the constructor is
 * returned as it is. With only the CPU provider allowed the storage is
 * host memory.
 *
 * Lists. A list goes to the GPU provider when the GPU is allowed, the
 * storage is the device's and the GPU takes every kind in it; otherwise to
 * the CPU provider when that is allowed and has every kind; otherwise the
 * list is UNSUPPORTED. The GPU takes every kind this library has, except
 * the kinds named in the environment variable M3_HIP_CPU_KINDS (a comma
 * list of COPY, CAST, ADD, MUL, SUB, DIV, SOFTMAX, SNAKE1D, TANH,
 * GATED_SILU), which go to the CPU provider. That switch exists to compare
 * the providers node by node and to run sessions that mix them; a session
 * reads it once, when it is created.
 *
 * This is the reference's scheduling (src/m3_provider.c:35-129) with HIP
 * in the place of Metal. It differs for kinds outside this library, which
 * the reference's CPU provider would run: here such a list is
 * UNSUPPORTED.
 *
 * m3_provider_set_gpu_factory replaces the GPU backend's constructor;
 * tests use it to compile sessions against a recording backend on
 * machines without a GPU.
 */
#include "m3_internal.h"

#include <stdlib.h>
#include <string.h>

static m3_backend_factory m3_gpu_factory = NULL;

void m3_provider_set_gpu_factory(m3_backend_factory factory)
{
    m3_gpu_factory = factory;
}

static const char *const m3_kind_names[] = {
    "COPY",      "CAST",        "ADD",        "MUL",
    "EMBEDDING", "MATMUL",      "LINEAR",     "RMS_NORM",
    "LAYER_NORM", "ROPE",       "ATTENTION",  "GATED_SILU",
    "SOFTMAX",   "TOP_K",       "CATEGORICAL", "CONV1D",
    "CONV_TRANSPOSE1D", "NEAREST_RESIZE1D", "SNAKE1D", "TANH",
    "SUB",       "DIV"};

/* True when `kind` is named in M3_HIP_CPU_KINDS. */
static bool m3_left_to_cpu(m3_op_kind kind)
{
    const char *list = getenv("M3_HIP_CPU_KINDS");
    const char *name;
    size_t length;

    if (list == NULL ||
        (unsigned int)kind >=
            sizeof(m3_kind_names) / sizeof(m3_kind_names[0])) {
        return false;
    }
    name = m3_kind_names[kind];
    length = strlen(name);
    while (*list != '\0') {
        const char *end = strchr(list, ',');
        const size_t token = end == NULL ? strlen(list)
                                         : (size_t)(end - list);

        if (token == length && strncmp(list, name, length) == 0) {
            return true;
        }
        list += token;
        list += *list == ',' ? 1 : 0;
    }
    return false;
}

static bool m3_gpu_takes(m3_op_kind kind)
{
    return m3_op_kind_supported(kind) && !m3_left_to_cpu(kind);
}

m3_status m3_backend_create_preferred(bool allow_gpu, bool allow_cpu,
                                      m3_backend **backend, m3_error *error)
{
    m3_status status;

    if (backend == NULL) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "no place to return the storage backend");
    }
    *backend = NULL;
    if (!allow_gpu && !allow_cpu) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "neither the GPU nor the CPU provider is "
                            "allowed");
    }
    if (!allow_gpu) {
        return m3_backend_create_host(backend, error);
    }
    status = m3_gpu_factory != NULL ? m3_gpu_factory(backend, error)
                                    : m3_backend_create_hip(backend, error);
    if (status != M3_STATUS_UNSUPPORTED) {
        return status;
    }
    *backend = NULL;
    if (allow_cpu) {
        /* No usable device: host storage and the CPU provider. */
        return m3_backend_create_host(backend, error);
    }
    {
        char cause[M3_ERROR_MESSAGE_CAPACITY] = "";

        if (error != NULL) {
            (void)memcpy(cause, error->message, sizeof(cause));
            cause[sizeof(cause) - 1U] = '\0';
        }
        return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                            "no HIP device and the CPU provider is not "
                            "allowed: %s", cause);
    }
}

m3_status m3_provider_select_regular(const m3_backend *storage_backend,
                                     bool allow_gpu, bool allow_cpu,
                                     const m3_command *commands,
                                     size_t command_count,
                                     m3_provider_kind *provider,
                                     m3_error *error)
{
    m3_backend_info info;
    bool gpu = allow_gpu;
    bool cpu = allow_cpu;
    size_t i;
    m3_status status;

    if (storage_backend == NULL || provider == NULL ||
        (commands == NULL && command_count != 0U)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "provider choice needs a backend, commands and "
                            "a place for the result");
    }
    status = m3_backend_get_info(storage_backend, &info, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    gpu = gpu && info.kind == M3_BACKEND_HIP;
    for (i = 0U; i < command_count; ++i) {
        gpu = gpu && m3_gpu_takes(commands[i].kind);
        cpu = cpu && m3_cpu_kind_supported(commands[i].kind);
    }
    if (gpu || cpu) {
        *provider = gpu ? M3_PROVIDER_HIP : M3_PROVIDER_CPU;
        m3_error_reset(error);
        return M3_STATUS_OK;
    }
    for (i = 0U; i < command_count; ++i) {
        if (!m3_op_kind_supported(commands[i].kind)) {
            return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                                "kind %d is outside this library",
                                (int)commands[i].kind);
        }
    }
    return m3_error_set(error, M3_STATUS_UNSUPPORTED,
                        "no allowed provider runs this command list");
}

m3_status m3_provider_execute_regular(m3_backend *storage_backend,
                                      m3_provider_kind provider,
                                      const m3_command *commands,
                                      size_t command_count,
                                      m3_scratch_arena *scratch,
                                      m3_error *error)
{
    size_t wanted = 0U;
    m3_status status;

    if (provider == M3_PROVIDER_HIP) {
        return m3_backend_execute(storage_backend, commands, command_count,
                                  scratch, error);
    }
    if (provider != M3_PROVIDER_CPU) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "provider %d does not run regular commands",
                            (int)provider);
    }
    status = m3_commands_scratch_bytes(storage_backend, commands,
                                       command_count, &wanted, error);
    if (status != M3_STATUS_OK) {
        return status;
    }
    if (wanted != 0U &&
        (scratch == NULL || scratch->offset > scratch->capacity ||
         wanted > scratch->capacity - scratch->offset)) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "the CPU provider wants %zu scratch bytes",
                            wanted);
    }
    return m3_cpu_execute(commands, command_count, error);
}
