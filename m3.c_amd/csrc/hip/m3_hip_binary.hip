/*
 * m3_hip_binary.hip - broadcast elementwise ADD/MUL/SUB/DIV for gfx950.
 *
 * Semantics are the reference's m3_host_binary (src/m3_op_execute_basic.c:
 * 61-77) and Metal m3_binary_apply (src/m3_backend_metal_basic.m:66-104):
 * out[i] = round_out(float(left[b_l(i)]) (op) float(right[b_r(i)])) with
 * right-aligned broadcasting, one F32 operation per element, round to
 * nearest even on store.
 *
 * Launch planning (host side):
 *   1. the output index space is coalesced: size-1 axes are dropped and
 *      neighbouring axes merge when every operand steps across them as one
 *      axis (m3_plan_index_space);
 *   2. each input is classified by how its element offset depends on the
 *      flat output index f:
 *        FULL     offset = f                 (same layout as the output)
 *        TRAIL    offset = f mod P           (trailing-axis broadcast,
 *                                             e.g. x[8,1024,1536]*c[1536])
 *        ROW      offset = (f / I) mod P     (broadcast over inner axes,
 *                                             I a multiple of 4)
 *        SCALAR   offset = 0
 *        PERIODIC offset = (f / I) mod P     (any I, per-element loads)
 *   3. when both inputs classify and the output is contiguous and aligned,
 *      the vector kernel runs: each lane handles groups of 4 consecutive
 *      outputs with 16-byte (F32) or 8-byte (F16/BF16) loads and stores,
 *      two groups in flight per lane, grid-stride over the tensor; with
 *      F32 operands and a tensor whose lanes are all resident at once, its
 *      held form instead (all loads, then the stores after a timed wait);
 *      divisions by I and P use precomputed multiply-shift divisors;
 *   4. anything else runs the general kernel: per-element offsets from the
 *      coalesced stride table.
 * All operands are read as F32 bit patterns, so NaN payloads survive
 * loads; m3_binary_f32_bits applies the operation and the NaN rule.
 */
#include "m3_hip_internal.h"

#include <cstring>

namespace {

enum m3_bin_mode : uint32_t {
    M3_BIN_FULL = 0,
    M3_BIN_TRAIL = 1,
    M3_BIN_ROW = 2,
    M3_BIN_SCALAR = 3,
    M3_BIN_PERIODIC = 4
};

struct m3_bin_operand {
    const uint8_t *base; /* first element (byte offset applied) */
    uint32_t mode;
    uint32_t dtype;
    m3_fast_div inner;
    m3_fast_div period;
};

struct m3_bin_vec_args {
    m3_bin_operand left;
    m3_bin_operand right;
    uint8_t *out;
    uint32_t out_dtype;
    uint32_t count;  /* elements, < 2^32 */
    uint32_t groups; /* count / 4 */
    m3_hip_gate list_gate;
};

constexpr uint32_t kThreads = 256U;
constexpr uint32_t kUnroll = 2U; /* groups in flight per lane (measured best) */

__device__ __forceinline__ uint32_t m3_load_raw(const uint8_t *p,
                                                uint32_t dtype)
{
    return dtype == M3N_F32 ? *(const uint32_t *)p
                            : (uint32_t) * (const uint16_t *)p;
}

template <bool F32ONLY>
__device__ __forceinline__ uint32_t m3_operand_index(const m3_bin_operand &o,
                                                     uint32_t f)
{
    switch (o.mode) {
    case M3_BIN_FULL:
        return f;
    case M3_BIN_TRAIL:
        return f - m3_fast_div_q(o.period, f) * o.period.divisor;
    case M3_BIN_SCALAR:
        return 0U;
    default: {
        uint32_t q = m3_fast_div_q(o.inner, f);

        return q - m3_fast_div_q(o.period, q) * o.period.divisor;
    }
    }
}

template <bool F32ONLY>
__device__ __forceinline__ uint32_t m3_operand_element(const m3_bin_operand &o,
                                                       uint32_t f)
{
    uint32_t dtype = F32ONLY ? (uint32_t)M3N_F32 : o.dtype;
    uint32_t esize = dtype == M3N_F32 ? 4U : 2U;
    uint32_t raw = m3_load_raw(o.base + (uint64_t)m3_operand_index<F32ONLY>(
                                            o, f) * esize,
                               dtype);

    return m3_load_as_f32_bits(raw, dtype);
}

/* F32 bits of operand elements f..f+3 (f a multiple of 4). */
template <bool F32ONLY>
__device__ __forceinline__ uint4 m3_operand_load4(const m3_bin_operand &o,
                                                  uint32_t f)
{
    uint32_t dtype = F32ONLY ? (uint32_t)M3N_F32 : o.dtype;

    if (o.mode == M3_BIN_FULL || o.mode == M3_BIN_TRAIL) {
        uint32_t index = o.mode == M3_BIN_FULL
                             ? f
                             : f - m3_fast_div_q(o.period, f) *
                                       o.period.divisor;

        /* a full operand is read once per launch: streamed; a trailing
         * broadcast operand is reread by every row: cached */
        if (dtype == M3N_F32) {
            const uint4 *p = (const uint4 *)(o.base + (uint64_t)index * 4U);

            return o.mode == M3_BIN_FULL ? m3_stream_load(p) : *p;
        }
        const uint2 *h = (const uint2 *)(o.base + (uint64_t)index * 2U);
        const uint2 half = o.mode == M3_BIN_FULL ? m3_stream_load(h) : *h;

        return make_uint4(m3_load_as_f32_bits(half.x & 0xffffU, dtype),
                          m3_load_as_f32_bits(half.x >> 16U, dtype),
                          m3_load_as_f32_bits(half.y & 0xffffU, dtype),
                          m3_load_as_f32_bits(half.y >> 16U, dtype));
    }
    if (o.mode == M3_BIN_ROW || o.mode == M3_BIN_SCALAR) {
        uint32_t v = m3_operand_element<F32ONLY>(o, f);

        return make_uint4(v, v, v, v);
    }
    return make_uint4(m3_operand_element<F32ONLY>(o, f),
                      m3_operand_element<F32ONLY>(o, f + 1U),
                      m3_operand_element<F32ONLY>(o, f + 2U),
                      m3_operand_element<F32ONLY>(o, f + 3U));
}

template <bool F32ONLY>
__device__ __forceinline__ void m3_store4(uint8_t *out, uint32_t dtype,
                                          uint32_t f, uint4 v)
{
    if (F32ONLY || dtype == M3N_F32) {
        m3_stream_store((uint4 *)(out + (uint64_t)f * 4U), v);
        return;
    }
    uint2 packed;

    packed.x = m3_store_from_f32_bits(v.x, dtype) |
               (m3_store_from_f32_bits(v.y, dtype) << 16U);
    packed.y = m3_store_from_f32_bits(v.z, dtype) |
               (m3_store_from_f32_bits(v.w, dtype) << 16U);
    m3_stream_store((uint2 *)(out + (uint64_t)f * 2U), packed);
}

template <int OP, bool F32ONLY, int UNROLL = (int)kUnroll>
__global__ __launch_bounds__(256) void m3_binary_vec_kernel(m3_bin_vec_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint32_t out_dtype = F32ONLY ? (uint32_t)M3N_F32 : a.out_dtype;
    const uint32_t step = gridDim.x * kThreads * UNROLL;

    for (uint32_t first = blockIdx.x * kThreads * UNROLL + threadIdx.x;
         first < a.groups; first += step) {
        uint4 left[UNROLL];
        uint4 right[UNROLL];

#pragma unroll
        for (uint32_t u = 0U; u < UNROLL; ++u) {
            uint32_t g = first + u * kThreads;

            if (g < a.groups) {
                left[u] = m3_operand_load4<F32ONLY>(a.left, g * 4U);
                right[u] = m3_operand_load4<F32ONLY>(a.right, g * 4U);
            }
        }
#pragma unroll
        for (uint32_t u = 0U; u < UNROLL; ++u) {
            uint32_t g = first + u * kThreads;

            if (g < a.groups) {
                uint4 r;

                r.x = m3_binary_f32_bits(OP, left[u].x, right[u].x);
                r.y = m3_binary_f32_bits(OP, left[u].y, right[u].y);
                r.z = m3_binary_f32_bits(OP, left[u].z, right[u].z);
                r.w = m3_binary_f32_bits(OP, left[u].w, right[u].w);
                m3_store4<F32ONLY>(a.out, out_dtype, g * 4U, r);
            }
        }
    }
    /* Tail: the last count % 4 elements. */
    if (blockIdx.x == 0U && threadIdx.x < a.count - a.groups * 4U) {
        uint32_t f = a.groups * 4U + threadIdx.x;
        uint32_t r = m3_binary_f32_bits(
            OP, m3_operand_element<F32ONLY>(a.left, f),
            m3_operand_element<F32ONLY>(a.right, f));
        uint32_t raw = m3_store_from_f32_bits(r, out_dtype);

        if (out_dtype == M3N_F32) {
            *(uint32_t *)(a.out + (uint64_t)f * 4U) = raw;
        } else {
            *(uint16_t *)(a.out + (uint64_t)f * 2U) = (uint16_t)raw;
        }
    }
}

/* Groups of four outputs per lane of the held form, and its workgroups
 * per CU (120 VGPRs: four waves per SIMD, all resident at once). */
constexpr int kHeldGroups = 12;
constexpr uint32_t kHeldBlocksPerCu = 4U;
/* Its wait before the stores, as a multiple of the time the launch's
 * reads of its full operands take at 8 TB/s. Measured in bench.py on
 * MUL x[8,1024,1536] * c[1536], alternating libraries on one box: 17.6-17.9
 * us at 1.0 and 1.19 against 18.1-18.6 us with the streaming kernel (1.4:
 * 18.5-18.8; eight groups per lane, whose workgroups were not all
 * resident, 20-31 us). */
constexpr double kBinaryHoldFactor = 1.1;

/* The held form of the F32 vector kernel, for a launch whose workgroups
 * are all resident at once: each lane loads its kHeldGroups groups of both
 * operands, forms the results, and stores them only hold_ticks
 * (s_memrealtime) after its start, so that the launch's writes do not
 * compete with its reads still in flight. The wait is bounded by the
 * clock; results are those of m3_binary_vec_kernel. */
template <int OP, int K>
__global__ __launch_bounds__(256) void m3_binary_held_kernel(
    m3_bin_vec_args a, uint32_t hold_ticks)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t start = __builtin_amdgcn_s_memrealtime();
    const uint32_t first = blockIdx.x * kThreads * K + threadIdx.x;
    uint4 left[K];
    uint4 right[K];

#pragma unroll
    for (int k = 0; k < K; ++k) {
        const uint32_t g = first + (uint32_t)k * kThreads;

        if (g < a.groups) {
            left[k] = m3_operand_load4<true>(a.left, g * 4U);
            right[k] = m3_operand_load4<true>(a.right, g * 4U);
        } else {
            left[k] = make_uint4(0U, 0U, 0U, 0U);
            right[k] = left[k];
        }
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        left[k].x = m3_binary_f32_bits(OP, left[k].x, right[k].x);
        left[k].y = m3_binary_f32_bits(OP, left[k].y, right[k].y);
        left[k].z = m3_binary_f32_bits(OP, left[k].z, right[k].z);
        left[k].w = m3_binary_f32_bits(OP, left[k].w, right[k].w);
    }
    while (__builtin_amdgcn_s_memrealtime() - start < (uint64_t)hold_ticks) {
        __builtin_amdgcn_s_sleep(2);
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const uint32_t g = first + (uint32_t)k * kThreads;

        if (g < a.groups) {
            m3_store4<true>(a.out, M3N_F32, g * 4U, left[k]);
        }
    }
    /* Tail: the last count % 4 elements. */
    if (blockIdx.x == 0U && threadIdx.x < a.count - a.groups * 4U) {
        uint32_t f = a.groups * 4U + threadIdx.x;

        *(uint32_t *)(a.out + (uint64_t)f * 4U) = m3_binary_f32_bits(
            OP, m3_operand_element<true>(a.left, f),
            m3_operand_element<true>(a.right, f));
    }
}

struct m3_bin_general_args {
    const uint8_t *left;
    const uint8_t *right;
    uint8_t *out;
    uint32_t left_dtype;
    uint32_t right_dtype;
    uint32_t out_dtype;
    uint32_t rank;
    uint64_t count;
    uint64_t shape[M3_HIP_MAX_RANK];
    int64_t left_strides[M3_HIP_MAX_RANK];
    int64_t right_strides[M3_HIP_MAX_RANK];
    m3_hip_gate list_gate;
};

template <int OP>
__global__ __launch_bounds__(256) void m3_binary_general_kernel(
    m3_bin_general_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    const uint32_t out_size = a.out_dtype == M3N_F32 ? 4U : 2U;

    for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         f < a.count; f += stride) {
        uint64_t rest = f;
        int64_t lo = 0;
        int64_t ro = 0;

        for (int axis = (int)a.rank - 1; axis >= 0; --axis) {
            uint64_t dim = a.shape[axis];
            uint64_t q = rest / dim;
            uint64_t c = rest - q * dim;

            rest = q;
            lo += (int64_t)c * a.left_strides[axis];
            ro += (int64_t)c * a.right_strides[axis];
        }
        uint32_t x = m3_load_as_f32_bits(m3_load_raw(a.left + lo,
                                                     a.left_dtype),
                                         a.left_dtype);
        uint32_t y = m3_load_as_f32_bits(m3_load_raw(a.right + ro,
                                                     a.right_dtype),
                                         a.right_dtype);
        uint32_t raw =
            m3_store_from_f32_bits(m3_binary_f32_bits(OP, x, y), a.out_dtype);

        if (out_size == 4U) {
            *(uint32_t *)(a.out + f * 4U) = raw;
        } else {
            *(uint16_t *)(a.out + f * 2U) = (uint16_t)raw;
        }
    }
}

/* Classifies operand k of `plan` (strides in bytes, element size esize). */
bool m3_classify_operand(const m3_index_plan &plan, uint32_t k,
                         const m3_hip_view *view, m3_bin_operand *operand)
{
    const int64_t esize = (int64_t)m3_dtype_bytes(view->dtype);
    const uint8_t *base = (const uint8_t *)view->base + view->byte_offset;
    uint64_t contiguous = 1U; /* output-layout element stride of an axis */
    uint64_t expected[M3_HIP_MAX_RANK];
    int live = -1;
    uint32_t live_count = 0U;
    bool full = true;

    for (int axis = (int)plan.rank - 1; axis >= 0; --axis) {
        expected[axis] = contiguous;
        contiguous *= plan.shape[axis];
    }
    for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
        int64_t s = plan.strides[k][axis];

        if (s != (int64_t)expected[axis] * esize) {
            full = false;
        }
        if (s != 0) {
            live = (int)axis;
            live_count += 1U;
        }
    }
    std::memset(operand, 0, sizeof(*operand));
    operand->base = base;
    operand->dtype = view->dtype;
    if (full && contiguous < (1ULL << 32U)) {
        operand->mode = M3_BIN_FULL;
        return true;
    }
    if (live_count == 0U) {
        operand->mode = M3_BIN_SCALAR;
        return true;
    }
    if (live_count != 1U || plan.strides[k][live] != esize ||
        contiguous >= (1ULL << 32U)) {
        return false;
    }
    operand->inner = m3_fast_div_make((uint32_t)expected[live]);
    operand->period = m3_fast_div_make((uint32_t)plan.shape[live]);
    operand->mode = M3_BIN_PERIODIC;
    if (expected[live] == 1U && plan.shape[live] % 4U == 0U) {
        operand->mode = M3_BIN_TRAIL;
    } else if (expected[live] % 4U == 0U) {
        operand->mode = M3_BIN_ROW;
    }
    return true;
}

bool m3_vector_aligned(const m3_bin_operand &o)
{
    uint32_t bytes = o.dtype == M3N_F32 ? 16U : 8U;

    if (o.mode != M3_BIN_FULL && o.mode != M3_BIN_TRAIL) {
        return true;
    }
    return ((uintptr_t)o.base % bytes) == 0U;
}

template <int OP>
int m3_launch_binary_op(m3_hip_device *device, const m3_hip_view *left,
                        const m3_hip_view *right, const m3_hip_view *output,
                        char *message, size_t capacity)
{
    static const char *const names[4] = {"m3_binary_add", "m3_binary_mul",
                                         "m3_binary_sub", "m3_binary_div"};
    const m3_hip_view *operands[3] = {output, left, right};
    m3_index_plan plan;
    m3_bin_vec_args vec;
    uint8_t *out = (uint8_t *)output->base + output->byte_offset;
    uint32_t out_bytes = output->dtype == M3N_F32 ? 16U : 8U;

    m3_plan_index_space(output, operands, 3U, &plan);
    std::memset(&vec, 0, sizeof(vec));
    vec.list_gate = device->gate;
    if (output->element_count < (1ULL << 32U) &&
        ((uintptr_t)out % out_bytes) == 0U &&
        m3_classify_operand(plan, 1U, left, &vec.left) &&
        m3_classify_operand(plan, 2U, right, &vec.right) &&
        m3_vector_aligned(vec.left) && m3_vector_aligned(vec.right)) {
        bool f32 = left->dtype == M3N_F32 && right->dtype == M3N_F32 &&
                   output->dtype == M3N_F32;

        vec.out = out;
        vec.out_dtype = output->dtype;
        vec.count = (uint32_t)output->element_count;
        vec.groups = vec.count / 4U;
        uint32_t blocks = m3_grid_blocks(device,
                                         (uint64_t)vec.groups == 0U
                                             ? 1U
                                             : vec.groups,
                                         kThreads * kUnroll, 16U);

        const uint64_t held =
            ((uint64_t)vec.groups + kThreads * kHeldGroups - 1U) /
            (kThreads * kHeldGroups);
        /* held only when its workgroups fill at least half of what the
         * device holds at once (a smaller tensor in few workgroups of
         * twelve groups per lane runs slower than streamed: 2 MB MUL, 9.0
         * against 4.5 us) and fit in it */
        const uint64_t slots =
            (uint64_t)device->compute_units * kHeldBlocksPerCu;
        const bool hold = f32 && device->wall_clock_khz != 0U &&
                          2U * held >= slots && held <= slots;
        /* the full operands' bytes (broadcast ones are read from cache) */
        const double read_bytes =
            4.0 * (double)vec.count *
            (double)((vec.left.mode == M3_BIN_FULL) +
                     (vec.right.mode == M3_BIN_FULL));
        const uint32_t hold_ticks = (uint32_t)(
            kBinaryHoldFactor * read_bytes / 8.0e6 *
            (double)device->wall_clock_khz / 1000.0);

        return m3_hip_launch(
            device, names[OP],
            [&](hipEvent_t start, hipEvent_t stop) {
                if (hold) {
                    hipExtLaunchKernelGGL(
                        (m3_binary_held_kernel<OP, kHeldGroups>),
                        dim3((uint32_t)held), dim3(kThreads), 0,
                        device->stream, start, stop, 0U, vec, hold_ticks);
                } else if (f32) {
                    hipExtLaunchKernelGGL((m3_binary_vec_kernel<OP, true>),
                                          dim3(blocks), dim3(kThreads), 0,
                                          device->stream, start, stop, 0U,
                                          vec);
                } else {
                    hipExtLaunchKernelGGL((m3_binary_vec_kernel<OP, false>),
                                          dim3(blocks), dim3(kThreads), 0,
                                          device->stream, start, stop, 0U,
                                          vec);
                }
            },
            message, capacity);
    }

    m3_bin_general_args general;

    std::memset(&general, 0, sizeof(general));
    general.list_gate = device->gate;
    general.left = (const uint8_t *)left->base + left->byte_offset;
    general.right = (const uint8_t *)right->base + right->byte_offset;
    general.out = out;
    general.left_dtype = left->dtype;
    general.right_dtype = right->dtype;
    general.out_dtype = output->dtype;
    general.rank = plan.rank;
    general.count = output->element_count;
    for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
        general.shape[axis] = plan.shape[axis];
        general.left_strides[axis] = plan.strides[1][axis];
        general.right_strides[axis] = plan.strides[2][axis];
    }
    uint32_t blocks = m3_grid_blocks(device, general.count, 256U, 16U);

    return m3_hip_launch(
        device, names[OP],
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL((m3_binary_general_kernel<OP>), dim3(blocks),
                                  dim3(256), 0, device->stream, start, stop,
                                  0U, general);
        },
        message, capacity);
}

} // namespace

extern "C" int m3_hip_launch_binary(m3_hip_device *device, uint32_t op,
                                    const m3_hip_view *left,
                                    const m3_hip_view *right,
                                    const m3_hip_view *output, char *message,
                                    size_t capacity)
{
    if (device == nullptr || op > M3_HIP_DIV || !m3_view_is_valid(left) ||
        !m3_view_is_valid(right) || !m3_view_is_valid(output) ||
        left->dtype == M3_HIP_I32 || right->dtype == M3_HIP_I32 ||
        output->dtype == M3_HIP_I32 || !m3_view_is_contiguous(output) ||
        !m3_view_broadcasts_to(left, output) ||
        !m3_view_broadcasts_to(right, output)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "binary launch arguments are malformed");
    }
    if (output->element_count == 0U) {
        return M3_HIP_OK;
    }
    switch (op) {
    case M3_HIP_ADD:
        return m3_launch_binary_op<M3N_ADD>(device, left, right, output,
                                            message, capacity);
    case M3_HIP_MUL:
        return m3_launch_binary_op<M3N_MUL>(device, left, right, output,
                                            message, capacity);
    case M3_HIP_SUB:
        return m3_launch_binary_op<M3N_SUB>(device, left, right, output,
                                            message, capacity);
    default:
        return m3_launch_binary_op<M3N_DIV>(device, left, right, output,
                                            message, capacity);
    }
}
