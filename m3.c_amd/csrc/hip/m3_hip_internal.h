/*
 * m3_hip_internal.h - state and helpers shared by the HIP translation units
 * of the m3 execution provider (gfx950).
 */
#ifndef M3_HIP_INTERNAL_H
#define M3_HIP_INTERNAL_H

#include "m3_hip.h"
#include "m3_numeric.h"
#include "m3_scratch_guard.h"

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

/* One timed launch: events recorded around a kernel on the device stream. */
struct m3_hip_pending_time {
    const char *name;
    hipEvent_t start;
    hipEvent_t stop;
};

struct m3_hip_time_total {
    std::string name;
    uint64_t launches;
    double total_ms;
    std::vector<float> samples; /* each launch's duration, in launch order,
                                 * up to kTimingSamples of them */
};

/* Launch durations kept per kernel name between two timing resets. */
constexpr size_t kTimingSamples = 4096U;

/* The device-side gate of a command list. After a command whose checked
 * input (a softmax input, a float-to-I32 cast input) an earlier command of
 * the same list produced, every command kernel of the list is launched
 * with the list's gate; it returns at its start, before touching any
 * tensor, when the gate word holds the gate's epoch, which a failed check
 * stores there (m3_hip_gate_check). word == nullptr: no gate, one uniform
 * branch on a kernel argument. */
struct m3_hip_gate {
    uint32_t *word;
    uint32_t epoch;
    /* The check of this command's input that its producer made as it
     * stored it (m3_hip_launch_program_checked): *pending holds
     * pending_epoch when it found an offending value. The command then
     * closes the gate itself, reports the failure as a failing check does
     * (report[1] = kind, report[0] = epoch) and returns. pending ==
     * nullptr: none. */
    uint32_t *pending;
    uint32_t pending_epoch;
    uint32_t *report;
    uint32_t kind;
};

__device__ __forceinline__ bool m3_gate_closed(const m3_hip_gate &gate)
{
    if (gate.word == nullptr) {
        return false;
    }
    if (__hip_atomic_load(gate.word, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT) == gate.epoch) {
        return true;
    }
    if (gate.pending == nullptr ||
        __hip_atomic_load(gate.pending, __ATOMIC_RELAXED,
                          __HIP_MEMORY_SCOPE_AGENT) != gate.pending_epoch) {
        return false;
    }
    /* every wave of the command stores the same words */
    __hip_atomic_store(gate.word, gate.epoch, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&gate.report[1], gate.kind, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
    __hip_atomic_store(&gate.report[0], gate.epoch, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
    __threadfence_system();
    return true;
}

struct m3_hip_device {
    int ordinal;
    hipStream_t stream;
    char name[256];
    uint64_t total_bytes;
    uint32_t compute_units;
    uint32_t lds_per_block; /* bytes of LDS one workgroup may use */
    uint32_t wall_clock_khz; /* rate of s_memrealtime; 0 if unknown */
    /* M3_HIP_SOFTMAX_LATE_US at open (negative when unset): when a wave of
     * the lane-row softmax counts as late (m3_hip_softmax.hip) */
    float softmax_late_us;
    /* M3_HIP_SOFTMAX_HOLD_US at open (negative when unset): how long after
     * its start a wave of the lane-row softmax holds its stores */
    float softmax_hold_us;
    /* M3_HIP_SOFTMAX_WIDE_GRID at open (0 when unset): at most this many
     * workgroups in a launch of the long-row softmax, each then taking
     * several rows in turn */
    uint32_t softmax_wide_grid;
    /* device flags for data scans (a view's word holds the epoch of the
     * last scan that found an offending element in it), the epoch of the
     * next scan, and the flags' host mirror in coherent pinned memory */
    uint32_t *scan_flags;
    uint32_t scan_epoch;
    uint32_t *host_flags; /* two halves: blocking scans, started scans */
    /* the last scan started with m3_hip_scan_views_begin: its ticket, the
     * completion sequence after its publication, and its view count */
    uint32_t async_ticket;
    uint32_t async_sequence;
    uint32_t async_count;
    /* the gate that launches carry (no word outside m3_hip_gate_open ..
     * m3_hip_gate_close); device words: [0] the epoch of the last closed
     * gate, [1] the flag of the gate's scans; pinned words: [0] the epoch
     * of the last closed gate, [1] the kind of its failed check; the epoch
     * of the last gate opened */
    m3_hip_gate gate;
    uint32_t *gate_words;
    uint32_t *host_gate;
    uint32_t gate_epoch;
    uint32_t gate_scan_epoch;
    /* the check the last m3_hip_launch_program_checked made (its flag
     * epoch and kind), armed on the gate by m3_hip_gate_pending */
    uint32_t fused_epoch;
    uint32_t fused_kind;
    /* how many times the host has waited for the stream (synchronize,
     * scan readback, blocking copies) since the device was opened */
    uint64_t host_waits;
    /* the device address of the static scan scratch (m3_hip_runtime.hip) */
    uint32_t *static_scratch;
    /* completion word in coherent pinned host memory (may be null) and the
     * last sequence number a kernel was queued to store there */
    uint32_t *done_word;
    uint32_t done_sequence;
    uint32_t unchecked_polls; /* polled completions since the last query
                               * of the stream's error state */
    bool timing;
    /* timing mode 1 attaches events to every launch; mode 2 only retires
     * each run on the stream, as mode 1 does, so that an external profiler
     * sees the same dispatch pattern without the events */
    bool timing_events;
    std::vector<m3_hip_pending_time> pending;
    std::vector<hipEvent_t> spare_events;
    std::vector<m3_hip_time_total> totals;
    char arch[64]; /* gcnArchName, e.g. gfx950:sramecc+:xnack- */
    /* kernels generated for elementwise programs (m3_hip_program.hip) */
    struct m3_program_cache *programs;
    /* GATED_SILU's BF16 activation of every gate in the table's range
     * (m3_hip_activation.hip) */
    uint16_t *silu_bf16_table;
};

/* Unloads the generated kernels of a device (m3_hip_program.hip). */
void m3_program_cache_release(m3_hip_device *device);

/* Builds and frees the device's GATED_SILU BF16 activation table
 * (m3_hip_activation.hip); the build is queued on the device stream. */
int m3_silu_table_build(m3_hip_device *device, char *message,
                        size_t capacity);
void m3_silu_table_release(m3_hip_device *device);

/* hipMalloc and hipHostMalloc, counted (m3_hip_allocation_count); the
 * hipError_t as an int. */
int m3_hip_malloc(void **memory, size_t bytes);
int m3_hip_host_malloc(void **memory, size_t bytes, unsigned int flags);

/* Writes a formatted message into a caller buffer (which may be NULL). */
int m3_hip_fail(char *message, size_t capacity, int code, const char *format,
                ...) __attribute__((format(printf, 4, 5)));
/* Maps a HIP error to an m3_hip_code with a message naming `what`. */
int m3_hip_check(hipError_t status, const char *what, char *message,
                 size_t capacity);

/* The epoch the next check of the open gate stores into its flag word
 * (gate word 1) when it fails (m3_hip_runtime.hip). */
int m3_hip_gate_flag_epoch(m3_hip_device *device, uint32_t *epoch,
                           char *message, size_t capacity);

/* Timing of one kernel launch: when timing is on, begin hands out a pair of
 * events for the dispatch and end queues them for folding (no-ops when
 * timing is off, leaving both events null). */
int m3_hip_time_begin(m3_hip_device *device, const char *name,
                      m3_hip_pending_time *slot);
void m3_hip_time_end(m3_hip_device *device, m3_hip_pending_time *slot);

/* Launch helper: launch(start, stop) enqueues one kernel with
 * hipExtLaunchKernelGGL, which attaches the two events to the dispatch
 * itself, so a timed interval is the kernel's execution and excludes the
 * host's submission latency. The launch is then checked. */
template <typename Launch>
int m3_hip_launch(m3_hip_device *device, const char *name, Launch launch,
                  char *message, size_t capacity)
{
    m3_hip_pending_time slot = {name, nullptr, nullptr};
    int code = m3_hip_time_begin(device, name, &slot);

    if (code != M3_HIP_OK) {
        return m3_hip_fail(message, capacity, code,
                           "cannot take timing events for %s", name);
    }
    launch(slot.start, slot.stop);
    hipError_t status = hipGetLastError();
    m3_hip_time_end(device, &slot);
    return m3_hip_check(status, name, message, capacity);
}

/* Streaming stores for kernel outputs: nontemporal vector stores that
 * write through without keeping the lines in the caches. Every output of
 * this library is written once and not read back by the same kernel; on
 * gfx950 these stores sustain a higher copy rate than ordinary ones. */
typedef uint32_t m3_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t m3_u32x2 __attribute__((ext_vector_type(2)));
typedef float m3_f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void m3_stream_store(uint4 *p, uint4 v)
{
    m3_u32x4 w = {v.x, v.y, v.z, v.w};

    __builtin_nontemporal_store(w, (m3_u32x4 *)p);
}

__device__ __forceinline__ void m3_stream_store(uint2 *p, uint2 v)
{
    m3_u32x2 w = {v.x, v.y};

    __builtin_nontemporal_store(w, (m3_u32x2 *)p);
}

__device__ __forceinline__ void m3_stream_store(float4 *p, float4 v)
{
    m3_f32x4 w = {v.x, v.y, v.z, v.w};

    __builtin_nontemporal_store(w, (m3_f32x4 *)p);
}

/* Streaming loads for inputs that one kernel reads exactly once (not for
 * broadcast operands, which stay cached across the grid). */
__device__ __forceinline__ uint4 m3_stream_load(const uint4 *p)
{
    m3_u32x4 w = __builtin_nontemporal_load((const m3_u32x4 *)p);

    return make_uint4(w.x, w.y, w.z, w.w);
}

__device__ __forceinline__ uint2 m3_stream_load(const uint2 *p)
{
    m3_u32x2 w = __builtin_nontemporal_load((const m3_u32x2 *)p);

    return make_uint2(w.x, w.y);
}

__device__ __forceinline__ float4 m3_stream_load(const float4 *p)
{
    m3_f32x4 w = __builtin_nontemporal_load((const m3_f32x4 *)p);

    return make_float4(w.x, w.y, w.z, w.w);
}

/* Unsigned 32-bit division by an invariant divisor d >= 1:
 * q = (umulhi(n, mul) + n) >> shift with shift = ceil(log2 d) and
 * mul = floor(2^32 (2^shift - d) / d) + 1; the sum is formed in 64 bits,
 * so the quotient is exact for every 32-bit n. */
struct m3_fast_div {
    uint32_t divisor;
    uint32_t mul;
    uint32_t shift;
};

static inline m3_fast_div m3_fast_div_make(uint32_t divisor)
{
    m3_fast_div d;
    uint32_t shift = 0U;

    while (shift < 32U && (1ULL << shift) < divisor) {
        ++shift;
    }
    d.divisor = divisor;
    d.shift = shift;
    d.mul = (uint32_t)((((1ULL << shift) - divisor) << 32U) / divisor + 1U);
    return d;
}

__host__ __device__ __forceinline__ uint32_t m3_fast_div_q(m3_fast_div d,
                                                          uint32_t n)
{
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t hi = __umulhi(n, d.mul);
#else
    uint32_t hi = (uint32_t)(((uint64_t)n * d.mul) >> 32U);
#endif
    return (uint32_t)(((uint64_t)hi + n) >> d.shift);
}

/* Byte strides of an operand over the (coalesced) output index space. */
struct m3_index_plan {
    uint32_t rank;               /* coalesced rank, >= 1 */
    uint64_t shape[M3_HIP_MAX_RANK];
    int64_t strides[3][M3_HIP_MAX_RANK]; /* per operand, bytes */
};

/* Builds the output index space of `output` with the given operands mapped
 * onto it by right-aligned broadcasting (a size-1 operand axis has stride
 * 0), then merges adjacent axes that are contiguous for every operand and
 * drops size-1 axes. operand_count <= 3; operand 0 is usually the output. */
void m3_plan_index_space(const m3_hip_view *output,
                         const m3_hip_view *const *operands,
                         uint32_t operand_count, m3_index_plan *plan);

bool m3_view_is_valid(const m3_hip_view *view);
/* Row-major layout: every axis longer than one steps by the product of the
 * inner extents times the element size. */
bool m3_view_is_contiguous(const m3_hip_view *view);
/* Every axis of `input`, right-aligned, is 1 or equals the output axis. */
bool m3_view_broadcasts_to(const m3_hip_view *input,
                           const m3_hip_view *output);
size_t m3_dtype_bytes(uint32_t dtype);

/* Number of blocks for a grid-stride loop over `items` work items with
 * `threads` threads per block, capped at `per_cu` blocks per CU. */
uint32_t m3_grid_blocks(const m3_hip_device *device, uint64_t items,
                        uint32_t threads, uint32_t per_cu);

#endif
