/*
 * m3_hip_runtime.hip - device, stream, arena, copies, data scans and
 * launch timing of the m3 HIP execution provider.
 *
 * One device handle owns one HIP stream (default priority). Every copy,
 * fill, scan and kernel of the handle is ordered on that stream, which is
 * what makes a command list execute in list order and lets
 * m3_hip_synchronize stand for the reference's commit + wait
 * (src/m3_backend_metal.m:189-216).
 */
#include "m3_hip_internal.h"

#include <algorithm>
#include <chrono>
#include <cstdlib>
#include <cstring>
#include <new>

int m3_hip_fail(char *message, size_t capacity, int code, const char *format,
                ...)
{
    if (message != nullptr && capacity != 0U) {
        va_list arguments;

        va_start(arguments, format);
        (void)vsnprintf(message, capacity, format, arguments);
        va_end(arguments);
        message[capacity - 1U] = '\0';
    }
    return code;
}

int m3_hip_check(hipError_t status, const char *what, char *message,
                 size_t capacity)
{
    if (status == hipSuccess) {
        return M3_HIP_OK;
    }
    return m3_hip_fail(message, capacity,
                       status == hipErrorOutOfMemory ? M3_HIP_OUT_OF_MEMORY
                       : status == hipErrorNoDevice  ? M3_HIP_NO_DEVICE
                                                     : M3_HIP_RUNTIME,
                       "%s failed: %s", what, hipGetErrorString(status));
}

size_t m3_dtype_bytes(uint32_t dtype)
{
    return dtype == M3_HIP_F16 || dtype == M3_HIP_BF16 ? 2U : 4U;
}

bool m3_view_is_valid(const m3_hip_view *view)
{
    uint64_t count = 1U;

    if (view == nullptr || view->rank > M3_HIP_MAX_RANK ||
        view->dtype > M3_HIP_I32) {
        return false;
    }
    for (uint32_t axis = 0U; axis < view->rank; ++axis) {
        count *= view->shape[axis];
    }
    return count == view->element_count &&
           (count == 0U || view->base != nullptr);
}

bool m3_view_is_contiguous(const m3_hip_view *view)
{
    uint64_t expected = m3_dtype_bytes(view->dtype);

    if (view->element_count == 0U) {
        return true;
    }
    for (int axis = (int)view->rank - 1; axis >= 0; --axis) {
        if (view->shape[axis] > 1U && view->byte_strides[axis] != expected) {
            return false;
        }
        expected *= view->shape[axis];
    }
    return true;
}

bool m3_view_broadcasts_to(const m3_hip_view *input,
                           const m3_hip_view *output)
{
    if (input->rank > output->rank) {
        return false;
    }
    for (uint32_t axis = 0U; axis < input->rank; ++axis) {
        uint64_t dim = input->shape[axis];
        uint64_t target = output->shape[axis + output->rank - input->rank];

        if (dim != 1U && dim != target) {
            return false;
        }
    }
    return true;
}

uint32_t m3_grid_blocks(const m3_hip_device *device, uint64_t items,
                        uint32_t threads, uint32_t per_cu)
{
    uint64_t wanted = (items + threads - 1U) / threads;
    uint64_t cap = (uint64_t)device->compute_units * per_cu;

    if (wanted == 0U) {
        wanted = 1U;
    }
    return (uint32_t)std::min<uint64_t>(wanted, cap);
}

void m3_plan_index_space(const m3_hip_view *output,
                         const m3_hip_view *const *operands,
                         uint32_t operand_count, m3_index_plan *plan)
{
    uint32_t rank = output->rank;
    uint64_t shape[M3_HIP_MAX_RANK];
    int64_t strides[3][M3_HIP_MAX_RANK];
    uint32_t kept = 0U;

    for (uint32_t axis = 0U; axis < rank; ++axis) {
        shape[axis] = output->shape[axis];
        for (uint32_t k = 0U; k < operand_count; ++k) {
            const m3_hip_view *view = operands[k];
            int view_axis = (int)axis - (int)(rank - view->rank);
            bool present = view_axis >= 0 && view->shape[view_axis] != 1U;

            strides[k][axis] =
                present ? (int64_t)view->byte_strides[view_axis] : 0;
        }
    }
    /* Drop size-1 axes, then merge an axis into its outer neighbour when
     * every operand steps across the pair as one axis. */
    std::memset(plan, 0, sizeof(*plan));
    for (uint32_t axis = 0U; axis < rank; ++axis) {
        if (shape[axis] == 1U) {
            continue;
        }
        if (kept != 0U) {
            bool mergeable = true;

            for (uint32_t k = 0U; k < operand_count; ++k) {
                if (plan->strides[k][kept - 1U] !=
                    strides[k][axis] * (int64_t)shape[axis]) {
                    mergeable = false;
                    break;
                }
            }
            if (mergeable) {
                plan->shape[kept - 1U] *= shape[axis];
                for (uint32_t k = 0U; k < operand_count; ++k) {
                    plan->strides[k][kept - 1U] = strides[k][axis];
                }
                continue;
            }
        }
        plan->shape[kept] = shape[axis];
        for (uint32_t k = 0U; k < operand_count; ++k) {
            plan->strides[k][kept] = strides[k][axis];
        }
        ++kept;
    }
    if (kept == 0U) {
        plan->shape[0] = 1U;
        kept = 1U;
    }
    plan->rank = kept;
}

/* ---- device lifetime ---------------------------------------------------- */

/* Views one data scan takes: one flag word each. */
constexpr uint32_t kScanViews = 64U;

/* The flag words of m3_hip_scan_views_static: a file-scope device array
 * (each GPU holds its own copy until the process ends), so that scan
 * allocates nothing. Host code never uses this name as an address; it
 * uses the address hipGetSymbolAddress gives for the device, kept per
 * device ordinal below. */
static __device__ __align__(256) uint32_t scratch[kScanViews];

constexpr int kScratchOrdinals = 64;
/* scratch's address on device ordinal i, looked up at the first open of
 * that device (with the device current) */
static void *m3_scratch_address[kScratchOrdinals];
/* one m3_hip_scan_views_static call at a time per device */
static m3_scratch_guard<kScratchOrdinals> m3_scratch_in_use;

/* Device and pinned host allocations made by this library, counted so that
 * tests can show an entry point allocates nothing. */
static std::atomic<uint64_t> m3_allocations{0};

int m3_hip_malloc(void **memory, size_t bytes)
{
    const hipError_t status = hipMalloc(memory, bytes);

    if (status == hipSuccess) {
        m3_allocations.fetch_add(1U, std::memory_order_relaxed);
    }
    return (int)status;
}

int m3_hip_host_malloc(void **memory, size_t bytes, unsigned int flags)
{
    const hipError_t status = hipHostMalloc(memory, bytes, flags);

    if (status == hipSuccess) {
        m3_allocations.fetch_add(1U, std::memory_order_relaxed);
    }
    return (int)status;
}

extern "C" int m3_hip_allocation_count(uint64_t *count)
{
    if (count == nullptr) {
        return M3_HIP_INVALID;
    }
    *count = m3_allocations.load(std::memory_order_relaxed);
    return M3_HIP_OK;
}

extern "C" int m3_hip_device_count(int *count, char *message,
                                   size_t capacity)
{
    int found = 0;
    hipError_t status;

    if (count == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "device count output is null");
    }
    *count = 0;
    status = hipGetDeviceCount(&found);
    if (status == hipErrorNoDevice || (status == hipSuccess && found == 0)) {
        return M3_HIP_OK;
    }
    if (status != hipSuccess) {
        return m3_hip_check(status, "hipGetDeviceCount", message, capacity);
    }
    *count = found;
    return M3_HIP_OK;
}

extern "C" int m3_hip_device_open(int ordinal, m3_hip_device **device_output,
                                  char *message, size_t capacity)
{
    hipDeviceProp_t properties;
    m3_hip_device *device;
    int count = 0;
    int code;

    if (device_output == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "device output is null");
    }
    *device_output = nullptr;
    code = m3_hip_device_count(&count, message, capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    if (ordinal < 0 || ordinal >= count) {
        return m3_hip_fail(message, capacity, M3_HIP_NO_DEVICE,
                           "HIP device %d is not present (%d found)",
                           ordinal, count);
    }
    code = m3_hip_check(hipSetDevice(ordinal), "hipSetDevice", message,
                        capacity);
    if (code == M3_HIP_OK) {
        code = m3_hip_check(hipGetDeviceProperties(&properties, ordinal),
                            "hipGetDeviceProperties", message, capacity);
    }
    if (code != M3_HIP_OK) {
        return code;
    }
    device = new (std::nothrow) m3_hip_device();
    if (device == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_OUT_OF_MEMORY,
                           "cannot allocate HIP device state");
    }
    device->ordinal = ordinal;
    std::snprintf(device->name, sizeof(device->name), "%s (%s)",
                  properties.name, properties.gcnArchName);
    std::snprintf(device->arch, sizeof(device->arch), "%s",
                  properties.gcnArchName);
    if (ordinal < kScratchOrdinals && m3_scratch_address[ordinal] == nullptr) {
        void *address = nullptr;

        code = m3_hip_check(hipGetSymbolAddress(&address, HIP_SYMBOL(scratch)),
                            "hipGetSymbolAddress(scratch)", message, capacity);
        if (code != M3_HIP_OK) {
            delete device;
            return code;
        }
        m3_scratch_address[ordinal] = address;
    }
    device->static_scratch = ordinal < kScratchOrdinals
                                 ? (uint32_t *)m3_scratch_address[ordinal]
                                 : nullptr;
    device->total_bytes = (uint64_t)properties.totalGlobalMem;
    device->compute_units = (uint32_t)properties.multiProcessorCount;
    device->lds_per_block = (uint32_t)properties.sharedMemPerBlock;
    {
        int rate = 0;
        const char *late = std::getenv("M3_HIP_SOFTMAX_LATE_US");
        const char *hold = std::getenv("M3_HIP_SOFTMAX_HOLD_US");
        const char *wide = std::getenv("M3_HIP_SOFTMAX_WIDE_GRID");

        device->wall_clock_khz =
            hipDeviceGetAttribute(&rate, hipDeviceAttributeWallClockRate,
                                  ordinal) == hipSuccess && rate > 0
                ? (uint32_t)rate
                : 0U;
        device->softmax_late_us =
            late != nullptr && late[0] != '\0' ? std::strtof(late, nullptr)
                                                : -1.0F;
        device->softmax_hold_us =
            hold != nullptr && hold[0] != '\0' ? std::strtof(hold, nullptr)
                                                : -1.0F;
        device->softmax_wide_grid =
            wide != nullptr && wide[0] != '\0'
                ? (uint32_t)std::strtoul(wide, nullptr, 10)
                : 0U;
    }
    code = m3_hip_check(hipStreamCreateWithFlags(&device->stream,
                                                 hipStreamNonBlocking),
                        "hipStreamCreateWithFlags", message, capacity);
    if (code == M3_HIP_OK) {
        code = m3_hip_check(
            (hipError_t)m3_hip_host_malloc((void **)&device->host_flags,
                                           2U * kScanViews * sizeof(uint32_t),
                                           hipHostMallocCoherent),
            "hipHostMalloc", message, capacity);
    }
    if (code == M3_HIP_OK) {
        code = m3_silu_table_build(device, message, capacity);
    }
    if (code != M3_HIP_OK) {
        m3_hip_device_close(device);
        return code;
    }
    /* optional: without it m3_hip_synchronize waits on the stream alone */
    if (m3_hip_host_malloc((void **)&device->done_word, 64U,
                           hipHostMallocCoherent) == (int)hipSuccess) {
        __atomic_store_n(device->done_word, 0U, __ATOMIC_RELEASE);
    } else {
        (void)hipGetLastError();
        device->done_word = nullptr;
    }
    *device_output = device;
    return M3_HIP_OK;
}

extern "C" void m3_hip_device_close(m3_hip_device *device)
{
    if (device == nullptr) {
        return;
    }
    (void)hipSetDevice(device->ordinal);
    if (device->stream != nullptr) {
        (void)hipStreamSynchronize(device->stream);
    }
    for (m3_hip_pending_time &slot : device->pending) {
        (void)hipEventDestroy(slot.start);
        (void)hipEventDestroy(slot.stop);
    }
    for (hipEvent_t event : device->spare_events) {
        (void)hipEventDestroy(event);
    }
    m3_program_cache_release(device);
    m3_silu_table_release(device);
    if (device->scan_flags != nullptr) {
        (void)hipFree(device->scan_flags);
    }
    if (device->gate_words != nullptr) {
        (void)hipFree(device->gate_words);
    }
    if (device->host_gate != nullptr) {
        (void)hipHostFree(device->host_gate);
    }
    if (device->host_flags != nullptr) {
        (void)hipHostFree(device->host_flags);
    }
    if (device->done_word != nullptr) {
        (void)hipHostFree(device->done_word);
    }
    if (device->stream != nullptr) {
        (void)hipStreamDestroy(device->stream);
    }
    delete device;
}

extern "C" int m3_hip_host_waits(const m3_hip_device *device,
                                 uint64_t *waits)
{
    if (device == nullptr || waits == nullptr) {
        return M3_HIP_INVALID;
    }
    *waits = device->host_waits;
    return M3_HIP_OK;
}

extern "C" int m3_hip_device_properties(const m3_hip_device *device,
                                        char *name, size_t name_capacity,
                                        uint64_t *total_bytes,
                                        uint32_t *compute_units,
                                        char *message, size_t capacity)
{
    if (device == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "device is null");
    }
    if (name != nullptr && name_capacity != 0U) {
        std::snprintf(name, name_capacity, "%s", device->name);
    }
    if (total_bytes != nullptr) {
        *total_bytes = device->total_bytes;
    }
    if (compute_units != nullptr) {
        *compute_units = device->compute_units;
    }
    return M3_HIP_OK;
}

extern "C" void *m3_hip_stream(m3_hip_device *device)
{
    return device == nullptr ? nullptr : (void *)device->stream;
}

/* ---- memory ------------------------------------------------------------- */

__global__ void m3_fill_zero_kernel(uint4 *words, uint64_t word_count,
                                    uint8_t *tail, uint32_t tail_bytes)
{
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;

    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         i < word_count; i += stride) {
        words[i] = make_uint4(0U, 0U, 0U, 0U);
    }
    if (blockIdx.x == 0U && threadIdx.x < tail_bytes) {
        tail[threadIdx.x] = 0U;
    }
}

extern "C" int m3_hip_fill_zero(m3_hip_device *device,
                                void *device_destination, size_t byte_count,
                                char *message, size_t capacity)
{
    if (device == nullptr || (byte_count != 0U &&
                              device_destination == nullptr)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "fill destination is null");
    }
    if (byte_count == 0U) {
        return M3_HIP_OK;
    }
    /* Leading bytes up to 16-byte alignment are folded into the tail
     * handling by requiring aligned starts: arenas are 256-byte aligned. */
    if (((uintptr_t)device_destination & 15U) != 0U) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "fill destination is not 16-byte aligned");
    }
    uint64_t words = byte_count / 16U;
    uint32_t tail = (uint32_t)(byte_count % 16U);
    uint8_t *tail_pointer = (uint8_t *)device_destination + words * 16U;
    uint32_t blocks = m3_grid_blocks(device, words == 0U ? 1U : words, 256U,
                                     8U);

    return m3_hip_launch(
        device, "m3_fill_zero",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_fill_zero_kernel, dim3(blocks), dim3(256),
                                  0, device->stream, start, stop, 0U,
                                  (uint4 *)device_destination, words,
                                  tail_pointer, tail);
        },
        message, capacity);
}

extern "C" int m3_hip_arena_reserve(m3_hip_device *device, size_t byte_count,
                                    void **base, char *message,
                                    size_t capacity)
{
    void *memory = nullptr;
    int code;

    if (device == nullptr || base == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "arena device and output are required");
    }
    *base = nullptr;
    if (byte_count == 0U) {
        return M3_HIP_OK;
    }
    code = m3_hip_check((hipError_t)m3_hip_malloc(&memory, byte_count),
                        "hipMalloc", message,
                        capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    /* Fresh device memory is zeroed so that nothing reads stale bytes. */
    code = m3_hip_fill_zero(device, memory, byte_count, message, capacity);
    if (code != M3_HIP_OK) {
        (void)hipFree(memory);
        return code;
    }
    *base = memory;
    return M3_HIP_OK;
}

extern "C" void m3_hip_arena_release(m3_hip_device *device, void *base)
{
    if (base == nullptr) {
        return;
    }
    if (device != nullptr) {
        (void)hipStreamSynchronize(device->stream);
    }
    (void)hipFree(base);
}

/* A host-to-device copy of at most kSmallCopy bytes carried in the
 * kernel's arguments: stream-ordered like any launch, and the host buffer
 * is free as soon as the launch returns, so the caller does not wait. */
constexpr uint32_t kSmallCopy = 256U;

struct m3_small_copy_args {
    uint8_t *destination;
    uint32_t count;
    uint8_t bytes[kSmallCopy];
};

__global__ __launch_bounds__(256) void m3_small_copy_kernel(
    m3_small_copy_args a)
{
    if (threadIdx.x < a.count) {
        a.destination[threadIdx.x] = a.bytes[threadIdx.x];
    }
}

extern "C" int m3_hip_copy_h2d(m3_hip_device *device,
                               void *device_destination,
                               const void *host_source, size_t byte_count,
                               char *message, size_t capacity)
{
    int code;

    if (device == nullptr ||
        (byte_count != 0U &&
         (device_destination == nullptr || host_source == nullptr))) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "copy endpoints are required");
    }
    if (byte_count == 0U) {
        return M3_HIP_OK;
    }
    if (byte_count <= kSmallCopy) {
        m3_small_copy_args args;

        std::memset(&args, 0, sizeof(args));
        args.destination = (uint8_t *)device_destination;
        args.count = (uint32_t)byte_count;
        std::memcpy(args.bytes, host_source, byte_count);
        return m3_hip_launch(
            device, "m3_small_copy",
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_small_copy_kernel, dim3(1),
                                      dim3(kSmallCopy), 0, device->stream,
                                      start, stop, 0U, args);
            },
            message, capacity);
    }
    /* pageable source: the copy is complete before the buffer is free */
    code = m3_hip_check(hipMemcpyAsync(device_destination, host_source,
                                       byte_count, hipMemcpyHostToDevice,
                                       device->stream),
                        "hipMemcpyAsync(host to device)", message, capacity);
    device->host_waits += 1U;
    if (code == M3_HIP_OK) {
        code = m3_hip_check(hipStreamSynchronize(device->stream),
                            "hipStreamSynchronize", message, capacity);
    }
    return code;
}

extern "C" int m3_hip_copy_d2h(m3_hip_device *device, void *host_destination,
                               const void *device_source, size_t byte_count,
                               char *message, size_t capacity)
{
    int code;

    if (device == nullptr ||
        (byte_count != 0U &&
         (device_source == nullptr || host_destination == nullptr))) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "copy endpoints are required");
    }
    if (byte_count == 0U) {
        return M3_HIP_OK;
    }
    code = m3_hip_check(hipMemcpyAsync(host_destination, device_source,
                                       byte_count, hipMemcpyDeviceToHost,
                                       device->stream),
                        "hipMemcpyAsync(device to host)", message, capacity);
    device->host_waits += 1U;
    if (code == M3_HIP_OK) {
        code = m3_hip_check(hipStreamSynchronize(device->stream),
                            "hipStreamSynchronize", message, capacity);
    }
    return code;
}

/* Stores `sequence` into the completion word, system-coherent, once every
 * earlier launch on the stream has finished. */
__global__ __launch_bounds__(64) void m3_done_kernel(uint32_t *word,
                                                    uint32_t sequence)
{
    if (threadIdx.x == 0U) {
        /* no release needed: the stream orders this kernel after the
         * work, and the host reads results through copies */
        __hip_atomic_store(word, sequence, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

/* How long m3_hip_synchronize polls the completion word before it waits
 * on the stream instead. */
constexpr double kDonePollSeconds = 1.0e-3;

/* Completions seen through the completion word between two queries of
 * the stream's error state. A query (hipStreamQuery) measured 17.5 us on
 * MI355X against 8.4 us for a whole launch and polled completion, so it
 * is made once per this many polled completions, not after each. */
constexpr uint32_t kPollsPerErrorQuery = 64U;

/* After a completion seen through the completion word: every
 * kPollsPerErrorQuery of them, an error the stream has recorded (a
 * kernel fault, say) is reported; not ready (the runtime has not retired
 * the work yet) is no error. Storage reads, frees and destroy wait on the
 * stream itself, which reports such errors too. */
static int m3_hip_stream_errors(m3_hip_device *device, char *message,
                                size_t capacity)
{
    hipError_t state;

    device->unchecked_polls += 1U;
    if (device->unchecked_polls < kPollsPerErrorQuery) {
        return M3_HIP_OK;
    }
    device->unchecked_polls = 0U;
    state = hipStreamQuery(device->stream);
    if (state == hipSuccess || state == hipErrorNotReady) {
        return M3_HIP_OK;
    }
    return m3_hip_check(state, "stream (queued work)", message, capacity);
}

/* Polls the completion word for `sequence` for at most kDonePollSeconds;
 * true when it arrived or a later sequence did (sequences grow by one per
 * completion queued on the stream, which stores them in order). */
static bool m3_hip_poll_done(const m3_hip_device *device, uint32_t sequence)
{
    const auto start = std::chrono::steady_clock::now();

    for (uint32_t spin = 0U;; ++spin) {
        const uint32_t seen = __atomic_load_n(device->done_word,
                                              __ATOMIC_ACQUIRE);

        if ((int32_t)(seen - sequence) >= 0) {
            return true;
        }
        if ((spin & 255U) == 255U &&
            std::chrono::duration<double>(std::chrono::steady_clock::now() -
                                          start)
                    .count() > kDonePollSeconds) {
            return false;
        }
    }
}

extern "C" int m3_hip_synchronize(m3_hip_device *device, char *message,
                                  size_t capacity)
{
    if (device == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "device is null");
    }
    /* The stream's own completion signal reaches the host about 11 us
     * after a launch even for an empty kernel; a kernel queued behind the
     * work that stores a sequence number into coherent pinned memory is
     * seen by polling about 4 us sooner. The poll is bounded, and the
     * stream wait after it (on timeout, or when the word is unavailable)
     * also reports any device error. With timing on, the stream wait is
     * used instead: the runtime then retires each run's work before the
     * next launch, and the timing events of the next launch read the
     * kernel's own duration (they read about 2 us long when the runtime
     * has not yet retired the previous work). */
    device->host_waits += 1U;
    if (device->done_word != nullptr && !device->timing) {
        const uint32_t sequence = device->done_sequence + 1U;

        hipLaunchKernelGGL(m3_done_kernel, dim3(1), dim3(64), 0,
                           device->stream, device->done_word, sequence);
        if (hipGetLastError() == hipSuccess) {
            device->done_sequence = sequence;
            if (m3_hip_poll_done(device, sequence)) {
                return m3_hip_stream_errors(device, message, capacity);
            }
        }
    }
    return m3_hip_check(hipStreamSynchronize(device->stream),
                        "hipStreamSynchronize", message, capacity);
}

/* ---- data scans (preflight) -------------------------------------------- */

/*
 * A scan checks each of up to kScanViews views for its condition (no NaN
 * for a softmax input, finite and in [-2^31, 2^31) for a float-to-I32
 * cast input) and hands the host one flag per view, without a device to
 * host copy or a stream wait:
 *   - every scan call has an epoch; a wave that finds an offending element
 *     stores the epoch into its view's flag word (device memory, written
 *     only on failure, so the words need no clearing between scans);
 *   - one publish wave then writes "flag == epoch" for every view into
 *     the device's coherent pinned host flags, fences at system scope, and
 *     stores the call's completion sequence into the pinned completion
 *     word, which the host polls (as m3_hip_synchronize does) before it
 *     reads the flags; the stream wait remains the fallback.
 */

struct m3_scan_args {
    const uint8_t *base;
    uint64_t count;
    uint32_t rank;
    uint32_t dtype;
    uint32_t kind;
    uint32_t epoch;
    uint64_t shape[M3_HIP_MAX_RANK];
    int64_t strides[M3_HIP_MAX_RANK];
    uint32_t *flag;
};

__device__ __forceinline__ uint32_t m3_scan_load(const uint8_t *p,
                                                 uint32_t dtype)
{
    uint32_t raw = dtype == M3N_F16 || dtype == M3N_BF16
                       ? (uint32_t)*(const uint16_t *)p
                       : *(const uint32_t *)p;

    return m3_load_as_f32_bits(raw, dtype);
}

/* 1 when the element offends the scan's condition, else 0. */
__device__ __forceinline__ uint32_t m3_scan_offends(uint32_t bits,
                                                    uint32_t kind)
{
    if (kind == M3_HIP_SCAN_NAN) {
        return m3_f32_is_nan_bits(bits) ? 1U : 0U;
    }
    /* finite and -2^31 <= v < 2^31 */
    float v = m3_bits_f32(bits);

    return ((bits & 0x7f800000U) != 0x7f800000U && v >= -2147483648.0F &&
            v < 2147483648.0F)
               ? 0U
               : 1U;
}

/* A scan that also closes a command list's gate when it finds an
 * offending element (m3_hip_gate_check): words[0] is the gate word, `host`
 * the pinned report (epoch of the closed gate, kind of the check). No
 * words: a plain scan. */
struct m3_scan_gate {
    uint32_t *words;
    uint32_t *host;
    uint32_t epoch;
    uint32_t kind;
};

/* The lanes that found an offending element store the epoch (all store
 * the same word, so their order does not matter), and close the gate of
 * a gated scan unless an earlier check of the same gate closed it (the
 * waves of one scan store the same values, so their races are benign;
 * checks of one gate run in list order on the stream). */
__device__ __forceinline__ void m3_scan_mark(uint32_t found, uint32_t *flag,
                                             uint32_t epoch,
                                             const m3_scan_gate &gate)
{
    if (__any(found != 0U) && found != 0U) {
        *flag = epoch;
        if (gate.words != nullptr &&
            __hip_atomic_load(&gate.words[0], __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT) != gate.epoch) {
            __hip_atomic_store(&gate.words[0], gate.epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&gate.host[1], gate.kind, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
            __hip_atomic_store(&gate.host[0], gate.epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_SYSTEM);
            __threadfence_system();
        }
    }
}

__global__ void m3_scan_kernel(m3_scan_args args, m3_scan_gate gate)
{
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint32_t found = 0U;

    for (uint64_t flat = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         flat < args.count; flat += stride) {
        uint64_t rest = flat;
        int64_t offset = 0;

        for (int axis = (int)args.rank - 1; axis >= 0; --axis) {
            uint64_t dim = args.shape[axis];
            uint64_t coordinate = rest % dim;

            rest /= dim;
            offset += (int64_t)coordinate * args.strides[axis];
        }
        found |= m3_scan_offends(m3_scan_load(args.base + offset, args.dtype),
                                 args.kind);
    }
    m3_scan_mark(found, args.flag, args.epoch, gate);
}

/* Contiguous F32 scan: 16-byte loads. */
__global__ void m3_scan_f32_contiguous_kernel(const uint4 *data,
                                              uint64_t quads,
                                              const uint32_t *tail,
                                              uint32_t tail_count,
                                              uint32_t kind, uint32_t *flag,
                                              uint32_t epoch,
                                              m3_scan_gate gate)
{
    uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    uint32_t found = 0U;

    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         i < quads; i += stride) {
        uint4 v = data[i];

        found |= m3_scan_offends(v.x, kind) | m3_scan_offends(v.y, kind) |
                 m3_scan_offends(v.z, kind) | m3_scan_offends(v.w, kind);
    }
    if (blockIdx.x == 0U && threadIdx.x < tail_count) {
        found |= m3_scan_offends(tail[threadIdx.x], kind);
    }
    m3_scan_mark(found, flag, epoch, gate);
}

/* Zeroes `count` flag words (one wave). */
__global__ __launch_bounds__(64) void m3_scan_clear_kernel(uint32_t *flags,
                                                          uint32_t count)
{
    if (threadIdx.x < count) {
        flags[threadIdx.x] = 0U;
    }
}

/* One wave: host_flags[v] = (flags[v] == epoch) for the first `count`
 * views, a system-scope fence, then the completion sequence (when the
 * device has a completion word). */
__global__ __launch_bounds__(64) void m3_scan_publish_kernel(
    const uint32_t *flags, uint32_t count, uint32_t epoch,
    uint32_t *host_flags, uint32_t *done_word, uint32_t sequence)
{
    const uint32_t lane = threadIdx.x;

    if (lane < count) {
        __hip_atomic_store(&host_flags[lane], flags[lane] == epoch ? 1U : 0U,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __threadfence_system();
    if (lane == 0U && done_word != nullptr) {
        __hip_atomic_store(done_word, sequence, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

/* Queues the scan of one view for `kind`: a wave that finds an offending
 * element stores `epoch` into *flag and closes `gate` when it has words. */
static int m3_hip_scan_launch(m3_hip_device *device, uint32_t *flag,
                              uint32_t epoch, uint32_t kind,
                              const m3_hip_view *view,
                              const m3_scan_gate &gate, char *message,
                              size_t capacity)
{
    if (view->element_count == 0U) {
        return M3_HIP_OK;
    }
    const m3_hip_view *operands[1] = {view};
    m3_index_plan plan;
    const uint8_t *base = (const uint8_t *)view->base + view->byte_offset;

    m3_plan_index_space(view, operands, 1U, &plan);
    if (view->dtype == M3_HIP_F32 && plan.rank == 1U &&
        plan.strides[0][0] == 4 && ((uintptr_t)base & 15U) == 0U) {
        uint64_t quads = view->element_count / 4U;
        uint32_t tail = (uint32_t)(view->element_count % 4U);
        uint32_t blocks = m3_grid_blocks(device, quads == 0U ? 1U : quads,
                                         256U, 8U);

        return m3_hip_launch(
            device, "m3_scan_f32",
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_scan_f32_contiguous_kernel,
                                      dim3(blocks), dim3(256), 0,
                                      device->stream, start, stop, 0U,
                                      (const uint4 *)base, quads,
                                      (const uint32_t *)base + quads * 4U,
                                      tail, kind, flag, epoch, gate);
            },
            message, capacity);
    }
    m3_scan_args args;

    std::memset(&args, 0, sizeof(args));
    args.base = base;
    args.count = view->element_count;
    args.rank = plan.rank;
    args.dtype = view->dtype;
    args.kind = kind;
    args.epoch = epoch;
    args.flag = flag;
    for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
        args.shape[axis] = plan.shape[axis];
        args.strides[axis] = plan.strides[0][axis];
    }
    uint32_t blocks = m3_grid_blocks(device, view->element_count, 256U, 8U);

    return m3_hip_launch(
        device, "m3_scan_strided",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_scan_kernel, dim3(blocks), dim3(256), 0,
                                  device->stream, start, stop, 0U, args,
                                  gate);
        },
        message, capacity);
}

/* Queues the scan of views[0, count) into the flag words `flags` with
 * `epoch` and the publication of one flag per view into the pinned words
 * `published`; *sequence receives the completion sequence that follows
 * the publication. */
static int m3_hip_scan_queue(m3_hip_device *device, uint32_t *flags,
                             uint32_t epoch, const uint32_t *kinds,
                             const m3_hip_view *views, size_t count,
                             uint32_t *published, bool timed,
                             uint32_t *sequence_out, char *message,
                             size_t capacity)
{
    int code = M3_HIP_OK;
    uint32_t sequence = device->done_sequence;
    /* untimed launches take no timing events (whose pool may grow) */
    const bool was_timing = device->timing;

    device->timing = device->timing && timed;
    for (size_t i = 0U; code == M3_HIP_OK && i < count; ++i) {
        code = m3_hip_scan_launch(device, flags + i, epoch, kinds[i],
                                  &views[i], m3_scan_gate{}, message,
                                  capacity);
    }
    if (code == M3_HIP_OK) {
        sequence += 1U;
        code = m3_hip_launch(
            device, "m3_scan_publish",
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_scan_publish_kernel, dim3(1),
                                      dim3(64), 0, device->stream, start,
                                      stop, 0U, flags, (uint32_t)count,
                                      epoch, published, device->done_word,
                                      sequence);
            },
            message, capacity);
    }
    device->timing = was_timing;
    if (code != M3_HIP_OK) {
        return code;
    }
    if (device->done_word != nullptr) {
        device->done_sequence = sequence;
    }
    *sequence_out = sequence;
    return M3_HIP_OK;
}

/* Waits until the publication that completion `sequence` follows has
 * happened and copies its `count` flags from `published`. */
static int m3_hip_scan_wait(m3_hip_device *device, uint32_t sequence,
                            const uint32_t *published, size_t count,
                            uint32_t *result, char *message, size_t capacity)
{
    int code;

    device->host_waits += 1U;
    if (device->done_word != nullptr && !device->timing &&
        m3_hip_poll_done(device, sequence)) {
        code = m3_hip_stream_errors(device, message, capacity);
    } else {
        code = m3_hip_check(hipStreamSynchronize(device->stream),
                            "hipStreamSynchronize", message, capacity);
    }
    for (size_t i = 0U; code == M3_HIP_OK && i < count; ++i) {
        result[i] = __atomic_load_n(&published[i], __ATOMIC_ACQUIRE);
    }
    return code;
}

/* Scans views[0, count) into the flag words `flags` with `epoch` and
 * returns one flag per view in `result`. */
static int m3_hip_scan_into(m3_hip_device *device, uint32_t *flags,
                            uint32_t epoch, const uint32_t *kinds,
                            const m3_hip_view *views, size_t count,
                            uint32_t *result, bool timed, char *message,
                            size_t capacity)
{
    uint32_t sequence = 0U;
    int code = m3_hip_scan_queue(device, flags, epoch, kinds, views, count,
                                 device->host_flags, timed, &sequence,
                                 message, capacity);

    if (code != M3_HIP_OK) {
        return code;
    }
    return m3_hip_scan_wait(device, sequence, device->host_flags, count,
                            result, message, capacity);
}

static int m3_hip_scan_arguments(const m3_hip_device *device,
                                 const uint32_t *kinds,
                                 const m3_hip_view *views, size_t count,
                                 const uint32_t *flags, char *message,
                                 size_t capacity)
{
    if (device == nullptr || (count != 0U && (kinds == nullptr ||
                                              views == nullptr ||
                                              flags == nullptr))) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "scan arguments are incomplete");
    }
    if (count > kScanViews) {
        return m3_hip_fail(message, capacity, M3_HIP_UNSUPPORTED,
                           "at most %u views can be scanned at once (%zu "
                           "given)",
                           kScanViews, count);
    }
    for (size_t i = 0U; i < count; ++i) {
        if (!m3_view_is_valid(&views[i]) ||
            kinds[i] > M3_HIP_SCAN_I32_RANGE) {
            return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                               "scan view %zu is malformed", i);
        }
    }
    return M3_HIP_OK;
}

/* The device's flag words (allocated on first use) and the next epoch:
 * 0 is what the words hold after a clear and is never a scan's epoch; a
 * fresh array, and one whose epochs wrapped, is cleared first. */
static int m3_hip_scan_epoch(m3_hip_device *device, char *message,
                             size_t capacity)
{
    int code = M3_HIP_OK;
    bool fresh = false;

    if (device->scan_flags == nullptr) {
        code = m3_hip_check((hipError_t)m3_hip_malloc((void **)&device->scan_flags,
                                      kScanViews * sizeof(uint32_t)),
                            "hipMalloc(scan flags)", message, capacity);
        fresh = true;
    }
    /* 0 is what the words hold after a clear and is never a scan's epoch;
     * a fresh array, and one whose epochs wrapped, is cleared first */
    device->scan_epoch += 1U;
    if (device->scan_epoch == 0U) {
        device->scan_epoch = 1U;
        fresh = true;
    }
    if (code == M3_HIP_OK && fresh) {
        code = m3_hip_launch(
            device, "m3_scan_clear",
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_scan_clear_kernel, dim3(1),
                                      dim3(64), 0, device->stream, start,
                                      stop, 0U, device->scan_flags,
                                      kScanViews);
            },
            message, capacity);
    }
    return code;
}

extern "C" int m3_hip_scan_views(m3_hip_device *device, const uint32_t *kinds,
                                 const m3_hip_view *views, size_t count,
                                 uint32_t *flags, char *message,
                                 size_t capacity)
{
    int code = m3_hip_scan_arguments(device, kinds, views, count, flags,
                                     message, capacity);

    if (code != M3_HIP_OK || count == 0U) {
        return code;
    }
    code = m3_hip_scan_epoch(device, message, capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    return m3_hip_scan_into(device, device->scan_flags, device->scan_epoch,
                            kinds, views, count, flags, true, message,
                            capacity);
}

extern "C" int m3_hip_scan_views_begin(m3_hip_device *device,
                                       const uint32_t *kinds,
                                       const m3_hip_view *views,
                                       size_t count, uint32_t *ticket,
                                       char *message, size_t capacity)
{
    uint32_t sequence = 0U;
    int code;

    if (ticket == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "scan ticket output is null");
    }
    code = m3_hip_scan_arguments(device, kinds, views, count, ticket, message,
                                 capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    code = m3_hip_scan_epoch(device, message, capacity);
    if (code == M3_HIP_OK) {
        code = m3_hip_scan_queue(device, device->scan_flags,
                                 device->scan_epoch, kinds, views, count,
                                 device->host_flags + kScanViews, true,
                                 &sequence, message, capacity);
    }
    if (code != M3_HIP_OK) {
        device->async_count = 0U;
        return code;
    }
    device->async_ticket += 1U;
    device->async_sequence = sequence;
    device->async_count = (uint32_t)count;
    *ticket = device->async_ticket;
    return M3_HIP_OK;
}

extern "C" int m3_hip_scan_views_collect(m3_hip_device *device,
                                         uint32_t ticket, size_t count,
                                         uint32_t *flags, char *message,
                                         size_t capacity)
{
    if (device == nullptr || (count != 0U && flags == nullptr)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "scan collection arguments are incomplete");
    }
    if (ticket != device->async_ticket || count != device->async_count) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "scan ticket %u with %zu views is not the last "
                           "started scan",
                           ticket, count);
    }
    return m3_hip_scan_wait(device, device->async_sequence,
                            device->host_flags + kScanViews, count, flags,
                            message, capacity);
}

extern "C" int m3_hip_scan_views_static(m3_hip_device *device,
                                        const uint32_t *kinds,
                                        const m3_hip_view *views,
                                        size_t count, uint32_t *flags,
                                        char *message, size_t capacity)
{
    int code = m3_hip_scan_arguments(device, kinds, views, count, flags,
                                     message, capacity);

    if (code != M3_HIP_OK || count == 0U) {
        return code;
    }
    if (device->static_scratch == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_UNSUPPORTED,
                           "no static scan scratch on device %d",
                           device->ordinal);
    }
    if (!m3_scratch_in_use.acquire(device->ordinal)) {
        return m3_hip_fail(message, capacity, M3_HIP_UNSUPPORTED,
                           "the static scan scratch of device %d is in use "
                           "by another call",
                           device->ordinal);
    }
    /* other handles on this GPU share the words: start from zero, and
     * mark with epoch 1 */
    hipLaunchKernelGGL(m3_scan_clear_kernel, dim3(1), dim3(64), 0,
                       device->stream, device->static_scratch,
                       (uint32_t)count);
    code = m3_hip_check(hipGetLastError(), "m3_scan_clear", message,
                        capacity);
    if (code == M3_HIP_OK) {
        code = m3_hip_scan_into(device, device->static_scratch, 1U, kinds,
                                views, count, flags, false, message,
                                capacity);
    }
    m3_scratch_in_use.release(device->ordinal);
    return code;
}

/* ---- device-side gating of a command list ------------------------------ */

/* Zeroes gate words [first, first + count) on the stream. */
static int m3_hip_gate_clear(m3_hip_device *device, uint32_t first,
                             uint32_t count, char *message, size_t capacity)
{
    return m3_hip_launch(
        device, "m3_scan_clear",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_scan_clear_kernel, dim3(1), dim3(64), 0,
                                  device->stream, start, stop, 0U,
                                  device->gate_words + first, count);
        },
        message, capacity);
}

extern "C" int m3_hip_gate_open(m3_hip_device *device, char *message,
                                size_t capacity)
{
    int code = M3_HIP_OK;

    if (device == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "device is null");
    }
    if (device->gate.word != nullptr) {
        return M3_HIP_OK; /* already open: the list keeps its gate */
    }
    if (device->gate_words == nullptr) {
        code = m3_hip_check((hipError_t)m3_hip_malloc((void **)&device->gate_words,
                                      2U * sizeof(uint32_t)),
                            "hipMalloc(gate words)", message, capacity);
        if (code == M3_HIP_OK) {
            code = m3_hip_gate_clear(device, 0U, 2U, message, capacity);
        }
        if (code != M3_HIP_OK) {
            (void)hipFree(device->gate_words);
            device->gate_words = nullptr;
            return code;
        }
    }
    if (device->host_gate == nullptr) {
        code = m3_hip_check((hipError_t)m3_hip_host_malloc(
                                (void **)&device->host_gate,
                                2U * sizeof(uint32_t), hipHostMallocCoherent),
                            "hipHostMalloc(gate report)", message, capacity);
        if (code != M3_HIP_OK) {
            device->host_gate = nullptr;
            return code;
        }
        device->host_gate[0] = 0U;
        device->host_gate[1] = 0U;
    }
    /* 0 is what a cleared gate word holds and is never an epoch; when the
     * epochs wrap the words are cleared again */
    device->gate_epoch += 1U;
    if (device->gate_epoch == 0U) {
        device->gate_epoch = 1U;
        code = m3_hip_gate_clear(device, 0U, 2U, message, capacity);
        if (code != M3_HIP_OK) {
            return code;
        }
        __atomic_store_n(&device->host_gate[0], 0U, __ATOMIC_RELEASE);
    }
    device->gate = m3_hip_gate{};
    device->gate.word = device->gate_words;
    device->gate.epoch = device->gate_epoch;
    return M3_HIP_OK;
}

/* The next epoch of the open gate's check flag (word 1): each check of a
 * list stores its own epoch there when it fails. When the epochs wrap the
 * word is cleared again. */
int m3_hip_gate_flag_epoch(m3_hip_device *device, uint32_t *epoch,
                           char *message, size_t capacity)
{
    device->gate_scan_epoch += 1U;
    if (device->gate_scan_epoch == 0U) {
        device->gate_scan_epoch = 1U;
        const int code = m3_hip_gate_clear(device, 1U, 1U, message, capacity);

        if (code != M3_HIP_OK) {
            return code;
        }
    }
    *epoch = device->gate_scan_epoch;
    return M3_HIP_OK;
}

extern "C" int m3_hip_gate_pending(m3_hip_device *device, int armed,
                                   char *message, size_t capacity)
{
    if (device == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "device is null");
    }
    if (!armed) {
        device->gate.pending = nullptr;
        return M3_HIP_OK;
    }
    if (device->gate.word == nullptr || device->fused_epoch == 0U) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "no gate is open or no check was fused");
    }
    device->gate.pending = device->gate_words + 1U;
    device->gate.pending_epoch = device->fused_epoch;
    device->gate.report = device->host_gate;
    device->gate.kind = device->fused_kind;
    device->fused_epoch = 0U;
    return M3_HIP_OK;
}

extern "C" int m3_hip_gate_check(m3_hip_device *device, uint32_t kind,
                                 const m3_hip_view *view, char *message,
                                 size_t capacity)
{
    int code;

    if (device == nullptr || view == nullptr || !m3_view_is_valid(view) ||
        kind > M3_HIP_SCAN_I32_RANGE) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "gate check arguments are incomplete or "
                           "malformed");
    }
    if (device->gate.word == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "no gate is open on this device");
    }
    uint32_t epoch = 0U;

    code = m3_hip_gate_flag_epoch(device, &epoch, message, capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    const m3_scan_gate gate = {device->gate_words, device->host_gate,
                               device->gate.epoch, kind};

    return m3_hip_scan_launch(device, device->gate_words + 1U, epoch, kind,
                              view, gate, message, capacity);
}

extern "C" int m3_hip_gate_close(m3_hip_device *device,
                                 uint32_t *failed_kind, char *message,
                                 size_t capacity)
{
    if (device == nullptr || failed_kind == nullptr) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "gate close arguments are incomplete");
    }
    *failed_kind = 0U;
    if (device->gate.word == nullptr) {
        return M3_HIP_OK;
    }
    const uint32_t epoch = device->gate.epoch;

    device->gate = m3_hip_gate{};
    device->fused_epoch = 0U;
    int code = m3_hip_synchronize(device, message, capacity);

    if (code != M3_HIP_OK) {
        return code;
    }
    if (__atomic_load_n(&device->host_gate[0], __ATOMIC_ACQUIRE) == epoch) {
        *failed_kind = 1U + __atomic_load_n(&device->host_gate[1],
                                            __ATOMIC_ACQUIRE);
    }
    return M3_HIP_OK;
}

/* ---- timing ------------------------------------------------------------- */

static int m3_hip_take_event(m3_hip_device *device, hipEvent_t *event)
{
    if (!device->spare_events.empty()) {
        *event = device->spare_events.back();
        device->spare_events.pop_back();
        return M3_HIP_OK;
    }
    return hipEventCreate(event) == hipSuccess ? M3_HIP_OK : M3_HIP_RUNTIME;
}

int m3_hip_time_begin(m3_hip_device *device, const char *name,
                      m3_hip_pending_time *slot)
{
    slot->name = name;
    slot->start = nullptr;
    slot->stop = nullptr;
    if (!device->timing || !device->timing_events) {
        return M3_HIP_OK;
    }
    if (m3_hip_take_event(device, &slot->start) != M3_HIP_OK) {
        slot->start = nullptr;
        return M3_HIP_RUNTIME;
    }
    if (m3_hip_take_event(device, &slot->stop) != M3_HIP_OK) {
        device->spare_events.push_back(slot->start);
        slot->start = nullptr;
        slot->stop = nullptr;
        return M3_HIP_RUNTIME;
    }
    return M3_HIP_OK;
}

void m3_hip_time_end(m3_hip_device *device, m3_hip_pending_time *slot)
{
    if (slot->start == nullptr) {
        return;
    }
    device->pending.push_back(*slot);
}

extern "C" int m3_hip_timing_enable(m3_hip_device *device, int enabled)
{
    if (device == nullptr) {
        return M3_HIP_INVALID;
    }
    device->timing = enabled != 0;
    device->timing_events = enabled == 1;
    return M3_HIP_OK;
}

static void m3_hip_fold_pending(m3_hip_device *device)
{
    for (m3_hip_pending_time &slot : device->pending) {
        float ms = 0.0F;
        bool found = false;

        device->spare_events.push_back(slot.start);
        device->spare_events.push_back(slot.stop);
        /* a launch that failed never recorded its events: not counted */
        if (hipEventElapsedTime(&ms, slot.start, slot.stop) != hipSuccess) {
            (void)hipGetLastError();
            continue;
        }
        for (m3_hip_time_total &total : device->totals) {
            if (total.name == slot.name) {
                total.launches += 1U;
                total.total_ms += ms;
                if (total.samples.size() < kTimingSamples) {
                    total.samples.push_back(ms);
                }
                found = true;
                break;
            }
        }
        if (!found) {
            device->totals.push_back({slot.name, 1U, (double)ms, {ms}});
        }
    }
    device->pending.clear();
}

extern "C" int m3_hip_timing_reset(m3_hip_device *device)
{
    if (device == nullptr) {
        return M3_HIP_INVALID;
    }
    (void)hipStreamSynchronize(device->stream);
    m3_hip_fold_pending(device);
    device->totals.clear();
    return M3_HIP_OK;
}

extern "C" int m3_hip_timing_read(m3_hip_device *device,
                                  m3_hip_kernel_time *entries,
                                  size_t capacity, size_t *count,
                                  char *message, size_t message_capacity)
{
    int code;

    if (device == nullptr || count == nullptr ||
        (capacity != 0U && entries == nullptr)) {
        return m3_hip_fail(message, message_capacity, M3_HIP_INVALID,
                           "timing arguments are incomplete");
    }
    code = m3_hip_check(hipStreamSynchronize(device->stream),
                        "hipStreamSynchronize", message, message_capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    m3_hip_fold_pending(device);
    *count = device->totals.size();
    for (size_t i = 0U; i < device->totals.size() && i < capacity; ++i) {
        std::snprintf(entries[i].name, sizeof(entries[i].name), "%s",
                      device->totals[i].name.c_str());
        entries[i].launches = device->totals[i].launches;
        entries[i].total_ms = device->totals[i].total_ms;
    }
    return M3_HIP_OK;
}

extern "C" int m3_hip_timing_samples(m3_hip_device *device, const char *name,
                                     float *durations_ms, size_t capacity,
                                     size_t *count, char *message,
                                     size_t message_capacity)
{
    int code;

    if (device == nullptr || name == nullptr || count == nullptr ||
        (capacity != 0U && durations_ms == nullptr)) {
        return m3_hip_fail(message, message_capacity, M3_HIP_INVALID,
                           "timing sample arguments are incomplete");
    }
    code = m3_hip_check(hipStreamSynchronize(device->stream),
                        "hipStreamSynchronize", message, message_capacity);
    if (code != M3_HIP_OK) {
        return code;
    }
    m3_hip_fold_pending(device);
    *count = 0U;
    for (const m3_hip_time_total &total : device->totals) {
        if (total.name == name) {
            *count = total.samples.size();
            for (size_t i = 0U; i < total.samples.size() && i < capacity;
                 ++i) {
                durations_ms[i] = total.samples[i];
            }
            break;
        }
    }
    return M3_HIP_OK;
}
