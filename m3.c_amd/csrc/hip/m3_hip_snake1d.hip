/*
 * m3_hip_snake1d.hip - Snake1d activation for gfx950, bit-exact with the
 * CPU provider of the reference.
 *
 * Reference semantics (src/m3_op_execute_basic.c:182-215): for x[B, C, L]
 * and alpha[1, C, 1], every output element is the result of seven F32
 * statements, each rounded, with contraction off:
 *   d = a + 0x1.12e0bep-30 (bits 0x3089705f); inv = 1 / d; ang = a * x;
 *   s = sinf(ang); q = s * s; t = inv * q; y = x + t.
 * sinf is m3_sinf, the C library algorithm restated bit for bit; the
 * division is the IEEE F32 quotient; this file is compiled with
 * -ffp-contract=off so no statement fuses. inv depends only on the channel
 * and is formed once per lane and loop iteration when the lane's groups lie
 * in one channel, else once per group of four outputs.
 *
 * The vector kernel handles contiguous, 16-byte aligned x and output with
 * L a multiple of 4: a lane takes four consecutive elements of one
 * channel, four groups in flight. Other layouts run per element over
 * stride tables.
 */
#include "m3_hip_internal.h"
#include "m3_libm.h"

#include <cstring>

namespace {

constexpr uint32_t kThreads = 256U;
constexpr uint32_t kUnroll = 4U;
/* Grid cap: 1,024 workgroups per CU, so the vector kernel runs one
 * workgroup per tile (1,024 groups of four elements) and the hardware
 * dispatcher spreads the tiles. Measured alternating in one process on
 * x[2,1536,65536]: 274 us against 292 us with 16 workgroups per CU. The
 * vector path takes fewer than 2^32 elements, so group indices plus one
 * grid stride (at most 2^28) stay below 2^32. */
constexpr uint32_t kBlocksPerCu = 1024U;

/* y = x + inverse * sin(a*x)^2 given sine = sin(a*x). */
__device__ __forceinline__ float m3_snake_finish(float x, float sine,
                                                 float inverse)
{
    float square = sine * sine;
    float scaled = inverse * square;

    return x + scaled;
}

__device__ __forceinline__ float m3_snake(float x, float a, float inverse)
{
    return m3_snake_finish(x, m3_sinf(a * x), inverse);
}

/* Four outputs of one channel. When no lane of the wave has an angle with
 * |a*x| >= 120 or a NaN angle (the common case by far), all four take the
 * branch-free sinf path, so the large-argument reduction costs one uniform
 * test per group instead of a divergent branch per element. That path
 * drops the sign of sinf: only its square is used, and the magnitude is
 * that of sinf for every |angle| < 120. */
__device__ __forceinline__ float4 m3_snake4(float4 x, float a, float inverse)
{
    const float4 angle = make_float4(a * x.x, a * x.y, a * x.z, a * x.w);
    /* one compare per element into a lane mask, the masks OR-ed as
     * scalars */
    const uint64_t large = __ballot(!(fabsf(angle.x) < 120.0F)) |
                           __ballot(!(fabsf(angle.y) < 120.0F)) |
                           __ballot(!(fabsf(angle.z) < 120.0F)) |
                           __ballot(!(fabsf(angle.w) < 120.0F));
    float4 sine;

    if (large != 0U) {
        sine = make_float4(m3_sinf(angle.x), m3_sinf(angle.y),
                           m3_sinf(angle.z), m3_sinf(angle.w));
    } else {
        sine = make_float4(m3_sinf_medium_magnitude(angle.x),
                           m3_sinf_medium_magnitude(angle.y),
                           m3_sinf_medium_magnitude(angle.z),
                           m3_sinf_medium_magnitude(angle.w));
    }
    return make_float4(m3_snake_finish(x.x, sine.x, inverse),
                       m3_snake_finish(x.y, sine.y, inverse),
                       m3_snake_finish(x.z, sine.z, inverse),
                       m3_snake_finish(x.w, sine.w, inverse));
}

__device__ __forceinline__ float m3_snake_inverse(float a)
{
    float denominator = a + m3_bits_f32(0x3089705fU);

    return 1.0F / denominator;
}

struct m3_snake_vec_args {
    const float4 *input;
    const uint8_t *alpha; /* alpha element of channel 0 */
    int64_t alpha_stride; /* bytes between channels */
    float4 *output;
    uint32_t groups;      /* elements / 4 */
    m3_fast_div length_in_groups; /* L / 4 */
    m3_fast_div channels;
    m3_hip_gate list_gate;
};

__global__ __launch_bounds__(256) void m3_snake1d_vec_kernel(
    m3_snake_vec_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint32_t step = gridDim.x * kThreads * kUnroll;

    for (uint32_t first = blockIdx.x * kThreads * kUnroll + threadIdx.x;
         first < a.groups; first += step) {
        const uint32_t last = first + (kUnroll - 1U) * kThreads;
        const uint32_t row = m3_fast_div_q(a.length_in_groups, first);
        float4 x[kUnroll];

        /* The row b*C + c of group g is nondecreasing in g, so when the
         * first and last group of a lane share a row, all of its groups
         * do: one channel, one alpha and one division for the lane. */
        if (__all(last < a.groups &&
                  m3_fast_div_q(a.length_in_groups, last) == row)) {
            const uint32_t channel =
                row - m3_fast_div_q(a.channels, row) * a.channels.divisor;
            const float alpha = *(const float *)(
                a.alpha + (int64_t)channel * a.alpha_stride);

#pragma unroll
            for (uint32_t u = 0U; u < kUnroll; ++u) {
                x[u] = m3_stream_load(&a.input[first + u * kThreads]);
            }
            const float inverse = m3_snake_inverse(alpha);

#pragma unroll
            for (uint32_t u = 0U; u < kUnroll; ++u) {
                m3_stream_store(&a.output[first + u * kThreads],
                                m3_snake4(x[u], alpha, inverse));
            }
            continue;
        }

        float alpha[kUnroll];

#pragma unroll
        for (uint32_t u = 0U; u < kUnroll; ++u) {
            uint32_t g = first + u * kThreads;

            if (g < a.groups) {
                uint32_t q = m3_fast_div_q(a.length_in_groups, g);
                uint32_t channel =
                    q - m3_fast_div_q(a.channels, q) * a.channels.divisor;

                x[u] = m3_stream_load(&a.input[g]);
                alpha[u] = *(const float *)(a.alpha +
                                            (int64_t)channel * a.alpha_stride);
            }
        }
#pragma unroll
        for (uint32_t u = 0U; u < kUnroll; ++u) {
            uint32_t g = first + u * kThreads;

            if (g < a.groups) {
                float inverse = m3_snake_inverse(alpha[u]);

                m3_stream_store(&a.output[g],
                                m3_snake4(x[u], alpha[u], inverse));
            }
        }
    }
}

struct m3_snake_general_args {
    const uint8_t *input;
    const uint8_t *alpha;
    float *output;
    uint64_t count;
    uint64_t shape[3];
    int64_t input_strides[3];
    int64_t alpha_stride;
    m3_hip_gate list_gate;
};

__global__ __launch_bounds__(256) void m3_snake1d_general_kernel(
    m3_snake_general_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;

    for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         f < a.count; f += step) {
        uint64_t l = f % a.shape[2];
        uint64_t rest = f / a.shape[2];
        uint64_t c = rest % a.shape[1];
        uint64_t b = rest / a.shape[1];
        float x = *(const float *)(a.input + (int64_t)b * a.input_strides[0] +
                                   (int64_t)c * a.input_strides[1] +
                                   (int64_t)l * a.input_strides[2]);
        float alpha = *(const float *)(a.alpha + (int64_t)c * a.alpha_stride);

        a.output[f] = m3_snake(x, alpha, m3_snake_inverse(alpha));
    }
}

} // namespace

extern "C" int m3_hip_launch_snake1d(m3_hip_device *device,
                                     const m3_hip_view *input,
                                     const m3_hip_view *alpha,
                                     const m3_hip_view *output,
                                     char *message, size_t capacity)
{
    if (device == nullptr || !m3_view_is_valid(input) ||
        !m3_view_is_valid(alpha) || !m3_view_is_valid(output) ||
        input->rank != 3U || alpha->rank != 3U || output->rank != 3U ||
        input->dtype != M3_HIP_F32 || alpha->dtype != M3_HIP_F32 ||
        output->dtype != M3_HIP_F32 || !m3_view_is_contiguous(output) ||
        alpha->shape[0] != 1U || alpha->shape[2] != 1U ||
        alpha->shape[1] != input->shape[1]) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "Snake1d launch arguments are malformed");
    }
    for (uint32_t axis = 0U; axis < 3U; ++axis) {
        if (input->shape[axis] != output->shape[axis]) {
            return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                               "Snake1d input and output shapes differ");
        }
    }
    if (output->element_count == 0U) {
        return M3_HIP_OK;
    }
    const uint8_t *in = (const uint8_t *)input->base + input->byte_offset;
    const uint8_t *al = (const uint8_t *)alpha->base + alpha->byte_offset;
    uint8_t *out = (uint8_t *)output->base + output->byte_offset;
    uint64_t length = input->shape[2];
    int64_t alpha_stride = input->shape[1] > 1U
                               ? (int64_t)alpha->byte_strides[1]
                               : 0;

    if (m3_view_is_contiguous(input) && length % 4U == 0U &&
        output->element_count < (1ULL << 32U) &&
        ((uintptr_t)in & 15U) == 0U && ((uintptr_t)out & 15U) == 0U) {
        m3_snake_vec_args args;

        std::memset(&args, 0, sizeof(args));
        args.list_gate = device->gate;
        args.input = (const float4 *)in;
        args.alpha = al;
        args.alpha_stride = alpha_stride;
        args.output = (float4 *)out;
        args.groups = (uint32_t)(output->element_count / 4U);
        args.length_in_groups = m3_fast_div_make((uint32_t)(length / 4U));
        args.channels = m3_fast_div_make((uint32_t)input->shape[1]);
        uint32_t blocks = m3_grid_blocks(device, args.groups,
                                         kThreads * kUnroll, kBlocksPerCu);

        return m3_hip_launch(
            device, "m3_snake1d",
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_snake1d_vec_kernel, dim3(blocks),
                                      dim3(kThreads), 0, device->stream, start,
                                      stop, 0U, args);
            },
            message, capacity);
    }

    m3_snake_general_args general;

    std::memset(&general, 0, sizeof(general));
    general.list_gate = device->gate;
    general.input = in;
    general.alpha = al;
    general.output = (float *)out;
    general.count = output->element_count;
    for (uint32_t axis = 0U; axis < 3U; ++axis) {
        general.shape[axis] = input->shape[axis];
        general.input_strides[axis] = (int64_t)input->byte_strides[axis];
    }
    general.alpha_stride = alpha_stride;
    uint32_t blocks = m3_grid_blocks(device, general.count, 256U, 16U);

    return m3_hip_launch(
        device, "m3_snake1d_strided",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_snake1d_general_kernel, dim3(blocks),
                                  dim3(256), 0, device->stream, start, stop,
                                  0U, general);
        },
        message, capacity);
}
