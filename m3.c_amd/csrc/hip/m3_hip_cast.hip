/*
 * m3_hip_cast.hip - CAST and COPY for gfx950.
 *
 * Semantics are the reference's m3_host_cast / m3_host_copy
 * (src/m3_op_execute_basic.c:11-59) and Metal m3_cast / m3_copy
 * (src/m3_backend_metal_basic.m:29-63):
 *   - same dtype: the element bytes are copied;
 *   - I32 -> float: (float)i, rounded to nearest even, then stored like
 *     any F32 value (so I32 -> F16 rounds twice, as the reference does);
 *   - float -> I32: truncation toward zero (inputs were scanned first);
 *   - float -> float: exact widening to F32, then the bit-exact RNE
 *     narrowing of m3_numeric.h. NaN payloads follow the reference rules.
 * The output is contiguous. A contiguous, aligned input runs the vector
 * kernel (four elements per lane per group, two groups in flight, output
 * written with streaming stores), or, for the cheap conversions of a
 * tensor whose lanes are all resident at once, its held form (all loads,
 * then the stores after a timed wait);
 * strided inputs run a per-element kernel over the coalesced index space.
 */
#include "m3_hip_internal.h"

#include <cstring>

namespace {

constexpr uint32_t kThreads = 256U;
constexpr uint32_t kUnroll = 2U; /* groups in flight per lane, copies */
/* Groups in flight per lane of a conversion: 4 when it narrows (4-byte to
 * 16-bit elements), 2 otherwise. Against 2, in bench.py alternating
 * libraries on one box: F32 -> F16 17.4-17.5 against 17.6-17.8 us and
 * F32 -> BF16 16.9-17.0 against 17.0-17.1 us; the widening casts measured
 * the same or slower with 1 or 4. */
constexpr uint32_t m3_cast_unroll(uint32_t in_size, uint32_t out_size)
{
    return in_size > out_size ? 4U : 2U;
}
/* workgroups per CU of a conversion: up to 32, so that a 16M-element
 * cast runs each lane's groups in one pass instead of a grid-stride loop
 * (measured 2% faster for F16 -> F32 than 16 per CU) */
constexpr uint32_t kCastBlocksPerCu = 32U;

template <uint32_t DT>
struct m3_vec_io;

/* Four 4-byte elements: one 16-byte access, read with a streaming load
 * (each input byte is read once). */
template <>
struct m3_vec_io<4U> {
    using type = uint4;
    __device__ static type load(const type *p) { return m3_stream_load(p); }
    __device__ static uint4 unpack(type v) { return v; }
    __device__ static type pack(uint4 v) { return v; }
};

/* Four 2-byte elements: one 8-byte access, read with a streaming load
 * (F16 -> F32 17.8-18.0 against 18.3-18.5 us with an ordinary one, BF16 ->
 * F32 17.8-18.0 against 18.3-18.5 us; bench.py alternating libraries on
 * one box). */
template <>
struct m3_vec_io<2U> {
    using type = uint2;
    __device__ static type load(const type *p) { return m3_stream_load(p); }
    __device__ static uint4 unpack(type v)
    {
        return make_uint4(v.x & 0xffffU, v.x >> 16U, v.y & 0xffffU,
                          v.y >> 16U);
    }
    __device__ static type pack(uint4 v)
    {
        return make_uint2((v.x & 0xffffU) | (v.y << 16U),
                          (v.z & 0xffffU) | (v.w << 16U));
    }
};

constexpr uint32_t m3_size_of(uint32_t dtype)
{
    return dtype == M3N_F16 || dtype == M3N_BF16 ? 2U : 4U;
}

template <uint32_t IN, uint32_t OUT>
__device__ __forceinline__ uint32_t m3_convert(uint32_t raw)
{
    return m3_store_from_f32_bits(m3_load_as_f32_bits(raw, IN), OUT);
}

template <uint32_t IN, uint32_t OUT>
__global__ __launch_bounds__(256) void m3_cast_vec_kernel(
    const uint8_t *input, uint8_t *output, uint64_t count, uint64_t groups,
    m3_hip_gate gate)
{
    if (m3_gate_closed(gate)) {
        return; /* a check earlier in the list failed */
    }
    using in_io = m3_vec_io<m3_size_of(IN)>;
    using out_io = m3_vec_io<m3_size_of(OUT)>;
    const typename in_io::type *in = (const typename in_io::type *)input;
    typename out_io::type *out = (typename out_io::type *)output;
    constexpr uint32_t unroll = m3_cast_unroll(m3_size_of(IN), m3_size_of(OUT));
    const uint64_t step = (uint64_t)gridDim.x * kThreads * unroll;

    for (uint64_t first = (uint64_t)blockIdx.x * kThreads * unroll +
                          threadIdx.x;
         first < groups; first += step) {
        uint4 v[unroll];

#pragma unroll
        for (uint32_t u = 0U; u < unroll; ++u) {
            uint64_t g = first + u * kThreads;

            if (g < groups) {
                v[u] = in_io::unpack(in_io::load(&in[g]));
            }
        }
#pragma unroll
        for (uint32_t u = 0U; u < unroll; ++u) {
            uint64_t g = first + u * kThreads;

            if (g < groups) {
                uint4 r = make_uint4(m3_convert<IN, OUT>(v[u].x),
                                     m3_convert<IN, OUT>(v[u].y),
                                     m3_convert<IN, OUT>(v[u].z),
                                     m3_convert<IN, OUT>(v[u].w));

                m3_stream_store(&out[g], out_io::pack(r));
            }
        }
    }
    if (blockIdx.x == 0U && threadIdx.x < count - groups * 4U) {
        uint64_t f = groups * 4U + threadIdx.x;
        uint32_t raw = m3_size_of(IN) == 4U
                           ? ((const uint32_t *)input)[f]
                           : (uint32_t)((const uint16_t *)input)[f];
        uint32_t r = m3_convert<IN, OUT>(raw);

        if (m3_size_of(OUT) == 4U) {
            ((uint32_t *)output)[f] = r;
        } else {
            ((uint16_t *)output)[f] = (uint16_t)r;
        }
    }
}

struct m3_strided_args {
    const uint8_t *input;
    uint8_t *output;
    uint32_t in_dtype;
    uint32_t out_dtype;
    uint32_t rank;
    uint64_t count;
    uint64_t shape[M3_HIP_MAX_RANK];
    int64_t strides[M3_HIP_MAX_RANK];
    m3_hip_gate list_gate;
};

/* Strided input, contiguous output; `convert` false copies raw elements. */
__global__ __launch_bounds__(256) void m3_cast_strided_kernel(
    m3_strided_args a, bool convert)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    const uint32_t in_size = m3_size_of(a.in_dtype);
    const uint32_t out_size = m3_size_of(a.out_dtype);

    for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         f < a.count; f += step) {
        uint64_t rest = f;
        int64_t offset = 0;

        for (int axis = (int)a.rank - 1; axis >= 0; --axis) {
            uint64_t dim = a.shape[axis];
            uint64_t q = rest / dim;

            offset += (int64_t)(rest - q * dim) * a.strides[axis];
            rest = q;
        }
        uint32_t raw = in_size == 4U
                           ? *(const uint32_t *)(a.input + offset)
                           : (uint32_t) * (const uint16_t *)(a.input + offset);
        uint32_t r = convert ? m3_store_from_f32_bits(
                                   m3_load_as_f32_bits(raw, a.in_dtype),
                                   a.out_dtype)
                             : raw;

        if (out_size == 4U) {
            *(uint32_t *)(a.output + f * 4U) = r;
        } else {
            *(uint16_t *)(a.output + f * 2U) = (uint16_t)r;
        }
    }
}

/* Contiguous byte copy with 16-byte words; `tail` bytes finish it. */
__global__ __launch_bounds__(256) void m3_copy_bytes_kernel(
    const uint4 *input, uint4 *output, uint64_t words, const uint8_t *tail_in,
    uint8_t *tail_out, uint32_t tail, m3_hip_gate gate)
{
    if (m3_gate_closed(gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t step = (uint64_t)gridDim.x * kThreads * kUnroll;

    for (uint64_t first = (uint64_t)blockIdx.x * kThreads * kUnroll +
                          threadIdx.x;
         first < words; first += step) {
        uint4 v[kUnroll];

#pragma unroll
        for (uint32_t u = 0U; u < kUnroll; ++u) {
            uint64_t g = first + u * kThreads;

            if (g < words) {
                v[u] = m3_stream_load(&input[g]);
            }
        }
#pragma unroll
        for (uint32_t u = 0U; u < kUnroll; ++u) {
            uint64_t g = first + u * kThreads;

            if (g < words) {
                m3_stream_store(&output[g], v[u]);
            }
        }
    }
    if (blockIdx.x == 0U && threadIdx.x < tail) {
        tail_out[threadIdx.x] = tail_in[threadIdx.x];
    }
}

/* Groups of four elements per lane of the held form. */
constexpr int kHeldGroups = 8;
/* Workgroups per CU that are all resident at once in the held form (its
 * lanes take at most 64 VGPRs: eight waves per SIMD). */
constexpr uint32_t kHeldBlocksPerCu = 8U;

/* How long the held form of a conversion waits before its stores, as a
 * multiple of the time the launch's reads take at 8 TB/s; 0 where it is
 * not used. Measured in bench.py, alternating libraries on one box
 * (4096 x 4096): F16 -> F32 and BF16 -> F32 16.7-17.1 us at 1.4 against
 * 18.0-18.5 us with the streaming kernel (1.19: 17.1-17.5, 1.6: 17.5-17.8);
 * F32 -> BF16 16.3-16.4 against 16.7-17.0 us at 1.19 (1.4: 18.1). F32 ->
 * F16, whose conversion takes several times the instructions, measured
 * slower held at every factor (19.6-21.4 against 17.2-17.4 us): its
 * conversions, all after the loads, then delay the stores. */
constexpr double m3_cast_hold_factor(uint32_t in, uint32_t out)
{
    return (in == M3N_F16 || in == M3N_BF16) && out == M3N_F32 ? 1.4
           : in == M3N_F32 && out == M3N_BF16                  ? 1.19
                                                                : 0.0;
}

/* The held form of the vector conversion, for a launch whose workgroups
 * are all resident at once: each lane loads its kHeldGroups groups, forms
 * their results, and stores them only hold_ticks (s_memrealtime) after its
 * start, so that the launch's writes do not compete with its reads still
 * in flight (HBM serves a phase of reads, then one of writes). The wait is
 * bounded by the clock; results are those of m3_cast_vec_kernel. */
template <uint32_t IN, uint32_t OUT, int K>
__global__ __launch_bounds__(256) void m3_cast_held_kernel(
    const uint8_t *input, uint8_t *output, uint64_t count, uint64_t groups,
    uint32_t hold_ticks, m3_hip_gate gate)
{
    if (m3_gate_closed(gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t start = __builtin_amdgcn_s_memrealtime();
    using in_io = m3_vec_io<m3_size_of(IN)>;
    using out_io = m3_vec_io<m3_size_of(OUT)>;
    const typename in_io::type *in = (const typename in_io::type *)input;
    typename out_io::type *out = (typename out_io::type *)output;
    const uint64_t first = (uint64_t)blockIdx.x * kThreads * K + threadIdx.x;
    typename out_io::type result[K];

#pragma unroll
    for (int k = 0; k < K; ++k) {
        const uint64_t g = first + (uint64_t)k * kThreads;
        uint4 v = make_uint4(0U, 0U, 0U, 0U);

        if (g < groups) {
            v = in_io::unpack(in_io::load(&in[g]));
        }
        result[k] = out_io::pack(make_uint4(m3_convert<IN, OUT>(v.x),
                                            m3_convert<IN, OUT>(v.y),
                                            m3_convert<IN, OUT>(v.z),
                                            m3_convert<IN, OUT>(v.w)));
    }
    while (__builtin_amdgcn_s_memrealtime() - start < (uint64_t)hold_ticks) {
        __builtin_amdgcn_s_sleep(2);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const uint64_t g = first + (uint64_t)k * kThreads;

        if (g < groups) {
            m3_stream_store(&out[g], result[k]);
        }
    }
    if (blockIdx.x == 0U && threadIdx.x < count - groups * 4U) {
        uint64_t f = groups * 4U + threadIdx.x;
        uint32_t raw = m3_size_of(IN) == 4U
                           ? ((const uint32_t *)input)[f]
                           : (uint32_t)((const uint16_t *)input)[f];
        uint32_t r = m3_convert<IN, OUT>(raw);

        if (m3_size_of(OUT) == 4U) {
            ((uint32_t *)output)[f] = r;
        } else {
            ((uint16_t *)output)[f] = (uint16_t)r;
        }
    }
}

template <uint32_t IN, uint32_t OUT>
void m3_launch_cast_vec(m3_hip_device *device, const uint8_t *input,
                        uint8_t *output, uint64_t count, uint32_t blocks,
                        hipEvent_t start, hipEvent_t stop)
{
    constexpr double factor = m3_cast_hold_factor(IN, OUT);
    const uint64_t groups = count / 4U;
    const uint64_t held =
        (groups + kThreads * kHeldGroups - 1U) / (kThreads * kHeldGroups);

    const uint64_t slots =
        (uint64_t)device->compute_units * kHeldBlocksPerCu;

    /* held only when its workgroups fill at least half of what the device
     * holds at once (few workgroups of eight groups per lane would leave
     * most CUs idle) and fit in it */
    if (factor > 0.0 && device->wall_clock_khz != 0U && 2U * held >= slots &&
        held <= slots) {
        const double us = factor * (double)count * m3_size_of(IN) / 8.0e6;
        const uint32_t ticks =
            (uint32_t)(us * (double)device->wall_clock_khz / 1000.0);

        hipExtLaunchKernelGGL((m3_cast_held_kernel<IN, OUT, kHeldGroups>),
                              dim3((uint32_t)held), dim3(kThreads), 0,
                              device->stream, start, stop, 0U, input, output,
                              count, groups, ticks, device->gate);
        return;
    }
    hipExtLaunchKernelGGL((m3_cast_vec_kernel<IN, OUT>), dim3(blocks),
                          dim3(kThreads), 0, device->stream, start, stop, 0U,
                          input, output, count, count / 4U, device->gate);
}

typedef void (*m3_cast_launcher)(m3_hip_device *, const uint8_t *, uint8_t *,
                                 uint64_t, uint32_t, hipEvent_t, hipEvent_t);

m3_cast_launcher m3_cast_vec_launcher(uint32_t in, uint32_t out)
{
#define M3_CAST_CASE(I, O)                                                    \
    if (in == (I) && out == (O)) {                                           \
        return &m3_launch_cast_vec<(I), (O)>;                                \
    }
    M3_CAST_CASE(M3N_F32, M3N_F16)
    M3_CAST_CASE(M3N_F32, M3N_BF16)
    M3_CAST_CASE(M3N_F32, M3N_I32)
    M3_CAST_CASE(M3N_F16, M3N_F32)
    M3_CAST_CASE(M3N_F16, M3N_BF16)
    M3_CAST_CASE(M3N_F16, M3N_I32)
    M3_CAST_CASE(M3N_BF16, M3N_F32)
    M3_CAST_CASE(M3N_BF16, M3N_F16)
    M3_CAST_CASE(M3N_BF16, M3N_I32)
    M3_CAST_CASE(M3N_I32, M3N_F32)
    M3_CAST_CASE(M3N_I32, M3N_F16)
    M3_CAST_CASE(M3N_I32, M3N_BF16)
#undef M3_CAST_CASE
    return nullptr;
}

const char *m3_cast_kernel_name(uint32_t in, uint32_t out)
{
    static const char *const names[4][4] = {
        {"m3_copy", "m3_cast_f32_f16", "m3_cast_f32_bf16", "m3_cast_f32_i32"},
        {"m3_cast_f16_f32", "m3_copy", "m3_cast_f16_bf16", "m3_cast_f16_i32"},
        {"m3_cast_bf16_f32", "m3_cast_bf16_f16", "m3_copy",
         "m3_cast_bf16_i32"},
        {"m3_cast_i32_f32", "m3_cast_i32_f16", "m3_cast_i32_bf16",
         "m3_copy"}};

    return names[in][out];
}

int m3_launch_unary(m3_hip_device *device, const m3_hip_view *input,
                    const m3_hip_view *output, char *message,
                    size_t capacity)
{
    const uint8_t *in = (const uint8_t *)input->base + input->byte_offset;
    uint8_t *out = (uint8_t *)output->base + output->byte_offset;
    const m3_hip_view *operands[2] = {output, input};
    const char *name = m3_cast_kernel_name(input->dtype, output->dtype);
    bool same = input->dtype == output->dtype;
    m3_index_plan plan;
    uint64_t count = output->element_count;

    m3_plan_index_space(output, operands, 2U, &plan);
    bool input_contiguous =
        plan.rank == 1U &&
        plan.strides[1][0] == (int64_t)m3_dtype_bytes(input->dtype);

    if (input_contiguous && same && ((uintptr_t)in & 15U) == 0U &&
        ((uintptr_t)out & 15U) == 0U) {
        uint64_t bytes = count * m3_dtype_bytes(input->dtype);
        uint64_t words = bytes / 16U;
        uint32_t tail = (uint32_t)(bytes % 16U);
        uint32_t blocks = m3_grid_blocks(device, words == 0U ? 1U : words,
                                         kThreads * kUnroll, 16U);

        return m3_hip_launch(
            device, name,
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_copy_bytes_kernel, dim3(blocks),
                                      dim3(kThreads), 0, device->stream, start,
                                      stop, 0U, (const uint4 *)in,
                                      (uint4 *)out, words, in + words * 16U,
                                      out + words * 16U, tail, device->gate);
            },
            message, capacity);
    }
    if (input_contiguous && !same) {
        uint32_t in_align = 4U * (uint32_t)m3_dtype_bytes(input->dtype);
        uint32_t out_align = 4U * (uint32_t)m3_dtype_bytes(output->dtype);
        m3_cast_launcher launcher =
            m3_cast_vec_launcher(input->dtype, output->dtype);

        if (launcher != nullptr && ((uintptr_t)in % in_align) == 0U &&
            ((uintptr_t)out % out_align) == 0U) {
            uint64_t groups = count / 4U;
            uint32_t blocks = m3_grid_blocks(device,
                                             groups == 0U ? 1U : groups,
                                             kThreads * m3_cast_unroll(
                                                 in_align / 4U,
                                                 out_align / 4U),
                                             kCastBlocksPerCu);

            return m3_hip_launch(
                device, name,
                [&](hipEvent_t start, hipEvent_t stop) {
                    launcher(device, in, out, count, blocks, start, stop);
                },
                message, capacity);
        }
    }
    m3_strided_args args;

    std::memset(&args, 0, sizeof(args));
    args.list_gate = device->gate;
    args.input = in;
    args.output = out;
    args.in_dtype = input->dtype;
    args.out_dtype = output->dtype;
    args.rank = plan.rank;
    args.count = count;
    for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
        args.shape[axis] = plan.shape[axis];
        args.strides[axis] = plan.strides[1][axis];
    }
    uint32_t blocks = m3_grid_blocks(device, count, 256U, 16U);

    return m3_hip_launch(
        device, name,
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_cast_strided_kernel, dim3(blocks),
                                  dim3(256), 0, device->stream, start, stop,
                                  0U, args, !same);
        },
        message, capacity);
}

bool m3_unary_views_ok(const m3_hip_view *input, const m3_hip_view *output)
{
    if (!m3_view_is_valid(input) || !m3_view_is_valid(output) ||
        input->rank != output->rank || !m3_view_is_contiguous(output)) {
        return false;
    }
    for (uint32_t axis = 0U; axis < input->rank; ++axis) {
        if (input->shape[axis] != output->shape[axis]) {
            return false;
        }
    }
    return true;
}

} // namespace

extern "C" int m3_hip_launch_cast(m3_hip_device *device,
                                  const m3_hip_view *input,
                                  const m3_hip_view *output, char *message,
                                  size_t capacity)
{
    if (device == nullptr || !m3_unary_views_ok(input, output)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "cast launch arguments are malformed");
    }
    if (output->element_count == 0U) {
        return M3_HIP_OK;
    }
    return m3_launch_unary(device, input, output, message, capacity);
}

extern "C" int m3_hip_launch_copy(m3_hip_device *device,
                                  const m3_hip_view *input,
                                  const m3_hip_view *output, char *message,
                                  size_t capacity)
{
    if (device == nullptr || !m3_unary_views_ok(input, output) ||
        input->dtype != output->dtype) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "copy launch arguments are malformed");
    }
    if (output->element_count == 0U) {
        return M3_HIP_OK;
    }
    return m3_launch_unary(device, input, output, message, capacity);
}
