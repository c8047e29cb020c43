/*
 * m3_hip_activation.hip - TANH and GATED_SILU for gfx950, bit-exact with
 * the CPU provider of the reference.
 *
 * Reference semantics:
 *   TANH       (src/m3_op_execute_basic.c:217-229) out = tanhf(in), F32;
 *              every element is m3_tanhf_uniform, the C library's tanhf
 *              restated bit for bit (m3_libm.h).
 *   GATED_SILU (src/m3_op_execute_basic.c:104-122) out = round_gate(gate /
 *              (1 + expf(-gate))) * up; m3_activation.h states it with
 *              the host's NaN bits.
 *
 * Both are elementwise and bound by HBM traffic at large sizes: TANH moves
 * 8 bytes per F32 element, GATED_SILU 12 (F32) or 6 (16-bit operands).
 * The vector kernels take contiguous, 16-byte (F32) or 8-byte (16-bit)
 * aligned operands of one dtype: a lane handles four consecutive elements
 * per group, kUnroll groups in flight, loads and stores streaming (every
 * element is read and written once). The last count % 4 elements are done
 * by the first lanes of block 0. Every other layout (strided inputs, mixed
 * dtypes for GATED_SILU) runs the general kernel over the coalesced index
 * space with per-element offsets.
 *
 * GATED_SILU's NaN rule costs a recomputation only in a wave where some
 * product is NaN: the plain arithmetic gives the host's bits for every
 * non-NaN result, and m3_gated_silu_bits gives them for all.
 *
 * All-BF16 GATED_SILU looks its activation up in a 16 KB table that each
 * device builds once (m3_gated_silu_bf16_kernel): a BF16 gate has only
 * 65,536 values, and the rounded activation depends on the gate alone.
 * That takes the kernel from 52 VALU instructions per element, clock-bound,
 * to 25, bound by HBM.
 */
#include "m3_activation.h"
#include "m3_hip_internal.h"
#include "m3_libm.h"

#include <cstring>

namespace {

constexpr uint32_t kThreads = 256U;
constexpr uint32_t kUnroll = 4U;
/* TANH's groups per lane: with ~100 instructions per element, two groups
 * in flight already cover the load latency, and the smaller tile lets the
 * dispatcher spread the work more evenly (3% faster than four, measured
 * alternating in one process on x[2,1536,65536]). */
constexpr uint32_t kTanhUnroll = 2U;
/* Grid cap of the vector kernels: 1,024 workgroups per CU, so every
 * tensor below 2^30 elements runs as one workgroup per tile (1,024 groups
 * of four elements) and the hardware dispatcher, not the grid-stride
 * loop, spreads the tiles. Measured against 16 per CU, alternating in one
 * process: GATED_SILU [16384, 3072] 94.5 against 100.5 us in F32 and 68.5
 * against 72.3 us in BF16; TANH x[2,1536,65536] 484 against 506 us. */
constexpr uint32_t kBlocksPerCu = 1024U;

/* Four consecutive elements of dtype D at group g of a contiguous array,
 * as F32. */
template <uint32_t D>
__device__ __forceinline__ void m3_load4(const uint8_t *base, uint32_t g,
                                         float v[4])
{
    if (D == M3N_F32) {
        uint4 w = m3_stream_load((const uint4 *)base + g);

        v[0] = m3_bits_f32(w.x);
        v[1] = m3_bits_f32(w.y);
        v[2] = m3_bits_f32(w.z);
        v[3] = m3_bits_f32(w.w);
    } else {
        uint2 w = m3_stream_load((const uint2 *)base + g);

        v[0] = m3_bits_f32(m3_load_as_f32_bits(w.x & 0xffffU, D));
        v[1] = m3_bits_f32(m3_load_as_f32_bits(w.x >> 16U, D));
        v[2] = m3_bits_f32(m3_load_as_f32_bits(w.y & 0xffffU, D));
        v[3] = m3_bits_f32(m3_load_as_f32_bits(w.y >> 16U, D));
    }
}

/* Stores four F32 results (as bits) rounded to dtype D at group g. */
template <uint32_t D>
__device__ __forceinline__ void m3_store4(uint8_t *base, uint32_t g,
                                          const uint32_t r[4])
{
    if (D == M3N_F32) {
        m3_stream_store((uint4 *)base + g, make_uint4(r[0], r[1], r[2], r[3]));
    } else {
        uint32_t lo = m3_store_from_f32_bits(r[0], D) |
                      (m3_store_from_f32_bits(r[1], D) << 16U);
        uint32_t hi = m3_store_from_f32_bits(r[2], D) |
                      (m3_store_from_f32_bits(r[3], D) << 16U);

        m3_stream_store((uint2 *)base + g, make_uint2(lo, hi));
    }
}

__device__ __forceinline__ uint32_t m3_load_element(const uint8_t *p,
                                                    uint32_t dtype)
{
    uint32_t raw = dtype == M3N_F32 ? *(const uint32_t *)p
                                    : (uint32_t) * (const uint16_t *)p;

    return m3_load_as_f32_bits(raw, dtype);
}

__device__ __forceinline__ void m3_store_element(uint8_t *p, uint32_t dtype,
                                                 uint32_t bits)
{
    uint32_t raw = m3_store_from_f32_bits(bits, dtype);

    if (dtype == M3N_F32) {
        *(uint32_t *)p = raw;
    } else {
        *(uint16_t *)p = (uint16_t)raw;
    }
}

/* ---- TANH ---------------------------------------------------------------- */

struct m3_tanh_vec_args {
    const uint8_t *input;
    uint8_t *output;
    uint32_t groups; /* count / 4 */
    uint32_t tail;   /* count % 4 */
    m3_hip_gate list_gate;
};

__global__ __launch_bounds__(256) void m3_tanh_vec_kernel(m3_tanh_vec_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint32_t step = gridDim.x * kThreads * kTanhUnroll;

    for (uint32_t first = blockIdx.x * kThreads * kTanhUnroll + threadIdx.x;
         first < a.groups; first += step) {
        float x[kTanhUnroll][4];

        /* unconditional loads (groups past the end re-read the last one)
         * so that all of them are in flight before the first use */
#pragma unroll
        for (uint32_t u = 0U; u < kTanhUnroll; ++u) {
            m3_load4<M3N_F32>(a.input, min(first + u * kThreads,
                                            a.groups - 1U), x[u]);
        }
#pragma unroll
        for (uint32_t u = 0U; u < kTanhUnroll; ++u) {
            uint32_t g = first + u * kThreads;

            if (g < a.groups) {
                uint32_t r[4];

#pragma unroll
                for (uint32_t k = 0U; k < 4U; ++k) {
                    r[k] = m3_f32_bits(m3_tanhf_uniform(x[u][k]));
                }
                m3_store4<M3N_F32>(a.output, g, r);
            }
        }
    }
    if (blockIdx.x == 0U && threadIdx.x < a.tail) {
        const uint64_t e = 4ULL * a.groups + threadIdx.x;
        float x = m3_bits_f32(*(const uint32_t *)(a.input + 4ULL * e));

        *(uint32_t *)(a.output + 4ULL * e) = m3_f32_bits(m3_tanhf_uniform(x));
    }
}

/* Coalesced index space: operand 0 is the contiguous output, 1 and 2 the
 * inputs (byte strides per axis). */
struct m3_activation_general_args {
    const uint8_t *inputs[2];
    uint8_t *output;
    uint32_t dtypes[3]; /* output, input 0, input 1 */
    uint32_t rank;
    uint64_t count;
    uint64_t shape[M3_HIP_MAX_RANK];
    int64_t strides[2][M3_HIP_MAX_RANK];
    m3_hip_gate list_gate;
};

__device__ __forceinline__ void m3_general_offsets(
    const m3_activation_general_args &a, uint64_t f, int64_t offsets[2])
{
    uint64_t rest = f;

    offsets[0] = 0;
    offsets[1] = 0;
    for (int axis = (int)a.rank - 1; axis >= 0; --axis) {
        uint64_t dim = a.shape[axis];
        uint64_t q = rest / dim;
        int64_t c = (int64_t)(rest - q * dim);

        offsets[0] += c * a.strides[0][axis];
        offsets[1] += c * a.strides[1][axis];
        rest = q;
    }
}

__global__ __launch_bounds__(256) void m3_tanh_general_kernel(
    m3_activation_general_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;

    for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         f < a.count; f += step) {
        int64_t offsets[2];

        m3_general_offsets(a, f, offsets);
        float x = m3_bits_f32(*(const uint32_t *)(a.inputs[0] + offsets[0]));

        *(uint32_t *)(a.output + 4ULL * f) = m3_f32_bits(m3_tanhf_uniform(x));
    }
}

/* ---- GATED_SILU ---------------------------------------------------------- */

struct m3_silu_vec_args {
    const uint8_t *gate;
    const uint8_t *up;
    uint8_t *output;
    uint32_t groups;
    uint32_t tail;
    m3_hip_gate list_gate;
};

/* Four GATED_SILU elements with a gate of dtype D, as F32 bits; `table`
 * is the expf table in LDS. */
template <uint32_t D>
__device__ __forceinline__ void m3_silu4(const float g[4], const float u[4],
                                         const uint64_t *table, uint32_t r[4])
{
    float p[4];

#pragma unroll
    for (uint32_t k = 0U; k < 4U; ++k) {
        float activation = m3_silu_quotient_fast(g[k], table);

        if (D == M3N_BF16) {
            activation = m3_bits_f32(
                m3_round_through_bf16_finite(m3_f32_bits(activation)));
        } else if (D == M3N_F16) {
            activation = m3_bits_f32(
                m3_round_through_bits(m3_f32_bits(activation), D));
        }
        p[k] = activation * u[k];
    }
    /* a NaN activation makes its product NaN, so one test covers both */
    if ((__ballot(p[0] != p[0]) | __ballot(p[1] != p[1]) |
         __ballot(p[2] != p[2]) | __ballot(p[3] != p[3])) != 0U) {
#pragma unroll
        for (uint32_t k = 0U; k < 4U; ++k) {
            p[k] = m3_bits_f32(m3_gated_silu_bits(g[k], u[k], D));
        }
    }
#pragma unroll
    for (uint32_t k = 0U; k < 4U; ++k) {
        r[k] = m3_f32_bits(p[k]);
    }
}

/* GATED_SILU BF16 through a table of activations. A BF16 gate has 65,536
 * bit patterns, and the activation, rounded through BF16, depends on the
 * gate alone; the table holds it for every gate of magnitude in
 * [2^-25, 2^7) (exponent fields 102-133, 32 binades of 128 values, both
 * signs: 8,192 entries, 16 KB), which covers every gate that is not tiny,
 * huge, infinite or NaN. The entries are the bits m3_gated_silu_bits gives
 * with up = 1 (exact: the product of a finite BF16 activation and 1), built
 * on the device when it is opened. Each workgroup copies the table into
 * LDS; an element then costs one LDS read instead of the ~35 instructions
 * of expf and the division. Gates outside the table take the arithmetic
 * of m3_silu4 in the waves where a lane has one, and NaN products the
 * exact recomputation, as in m3_gated_silu_vec_kernel. */
constexpr uint32_t kSiluTableFirstField = 102U; /* exponent field of 2^-25 */
constexpr uint32_t kSiluTableSpan = 32U << 7U;  /* entries per sign */
constexpr uint32_t kSiluTableEntries = 2U * kSiluTableSpan;

/* The BF16 bits of table entry i: bit 12 is the sign, the rest counts up
 * from the first exponent field. */
__host__ __device__ inline uint32_t m3_silu_table_gate(uint32_t i)
{
    return ((i & kSiluTableSpan) << 3U) |
           ((kSiluTableFirstField << 7U) + (i & (kSiluTableSpan - 1U)));
}

__global__ __launch_bounds__(256) void m3_silu_table_build_kernel(
    uint16_t *table)
{
    const uint32_t i = blockIdx.x * 256U + threadIdx.x;

    if (i < kSiluTableEntries) {
        const float gate = m3_bits_f32(m3_silu_table_gate(i) << 16U);

        table[i] = (uint16_t)(m3_gated_silu_bits(gate, 1.0F, M3N_BF16) >>
                              16U);
    }
}

/* The activation of BF16 gate bits `raw` as F32 bits from the LDS table;
 * *miss is set (and 0 returned) for a gate outside it. */
__device__ __forceinline__ uint32_t m3_silu_table_lookup(
    uint32_t raw, const uint16_t *table, bool *miss)
{
    const uint32_t index = (raw & 0x7fffU) - (kSiluTableFirstField << 7U);
    const bool inside = index < kSiluTableSpan;

    *miss = !inside;
    return inside ? (uint32_t)table[index | ((raw >> 3U) & kSiluTableSpan)]
                        << 16U
                  : 0U;
}

__global__ __launch_bounds__(256) void m3_gated_silu_bf16_kernel(
    m3_silu_vec_args a, const uint4 *source)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint32_t step = gridDim.x * kThreads * kUnroll;
    __shared__ uint16_t table[kSiluTableEntries];
    __shared__ uint64_t exp_table[32];

    for (uint32_t i = threadIdx.x; i < kSiluTableEntries / 8U; i += kThreads) {
        ((uint4 *)table)[i] = source[i];
    }
    if (threadIdx.x < 32U) {
        exp_table[threadIdx.x] = m3_expf_table[threadIdx.x];
    }
    __syncthreads();
    for (uint32_t first = blockIdx.x * kThreads * kUnroll + threadIdx.x;
         first < a.groups; first += step) {
        uint2 gate[kUnroll];
        uint2 up[kUnroll];

        /* unconditional loads (groups past the end re-read the last one)
         * so that all of them are in flight before the first use */
#pragma unroll
        for (uint32_t k = 0U; k < kUnroll; ++k) {
            const uint32_t index = min(first + k * kThreads, a.groups - 1U);

            gate[k] = m3_stream_load((const uint2 *)a.gate + index);
            up[k] = m3_stream_load((const uint2 *)a.up + index);
        }
#pragma unroll
        for (uint32_t k = 0U; k < kUnroll; ++k) {
            const uint32_t index = first + k * kThreads;

            if (index < a.groups) {
                const uint32_t raw[4] = {gate[k].x & 0xffffU, gate[k].x >> 16U,
                                         gate[k].y & 0xffffU, gate[k].y >> 16U};
                const float u[4] = {m3_bits_f32(up[k].x << 16U),
                                    m3_bits_f32(up[k].x & 0xffff0000U),
                                    m3_bits_f32(up[k].y << 16U),
                                    m3_bits_f32(up[k].y & 0xffff0000U)};
                uint32_t activation[4];
                bool miss[4];
                float p[4];
                uint32_t r[4];

#pragma unroll
                for (uint32_t e = 0U; e < 4U; ++e) {
                    activation[e] = m3_silu_table_lookup(raw[e], table,
                                                         &miss[e]);
                }
                if ((__ballot(miss[0]) | __ballot(miss[1]) |
                     __ballot(miss[2]) | __ballot(miss[3])) != 0U) {
#pragma unroll
                    for (uint32_t e = 0U; e < 4U; ++e) {
                        if (miss[e]) {
                            activation[e] = m3_round_through_bf16_finite(
                                m3_f32_bits(m3_silu_quotient_fast(
                                    m3_bits_f32(raw[e] << 16U), exp_table)));
                        }
                    }
                }
#pragma unroll
                for (uint32_t e = 0U; e < 4U; ++e) {
                    p[e] = m3_bits_f32(activation[e]) * u[e];
                }
                /* a NaN activation makes its product NaN, so one test
                 * covers both */
                if ((__ballot(p[0] != p[0]) | __ballot(p[1] != p[1]) |
                     __ballot(p[2] != p[2]) | __ballot(p[3] != p[3])) != 0U) {
#pragma unroll
                    for (uint32_t e = 0U; e < 4U; ++e) {
                        p[e] = m3_bits_f32(m3_gated_silu_bits(
                            m3_bits_f32(raw[e] << 16U), u[e], M3N_BF16));
                    }
                }
#pragma unroll
                for (uint32_t e = 0U; e < 4U; ++e) {
                    r[e] = m3_f32_bits(p[e]);
                }
                m3_store4<M3N_BF16>(a.output, index, r);
            }
        }
    }
    if (blockIdx.x == 0U && threadIdx.x < a.tail) {
        const uint64_t e = 4ULL * a.groups + threadIdx.x;
        float g = m3_bits_f32(m3_load_element(a.gate + 2U * e, M3N_BF16));
        float u = m3_bits_f32(m3_load_element(a.up + 2U * e, M3N_BF16));

        m3_store_element(a.output + 2U * e, M3N_BF16,
                         m3_gated_silu_bits(g, u, M3N_BF16));
    }
}

/* Gate, up and output all of dtype D, contiguous and aligned. */
template <uint32_t D>
__global__ __launch_bounds__(256) void m3_gated_silu_vec_kernel(
    m3_silu_vec_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint32_t step = gridDim.x * kThreads * kUnroll;
    constexpr uint32_t size = D == M3N_F32 ? 4U : 2U;
    __shared__ uint64_t table[32];

    if (threadIdx.x < 32U) {
        table[threadIdx.x] = m3_expf_table[threadIdx.x];
    }
    __syncthreads();
    for (uint32_t first = blockIdx.x * kThreads * kUnroll + threadIdx.x;
         first < a.groups; first += step) {
        float g[kUnroll][4];
        float u[kUnroll][4];

        /* unconditional loads (groups past the end re-read the last one)
         * so that all of them are in flight before the first use */
#pragma unroll
        for (uint32_t k = 0U; k < kUnroll; ++k) {
            const uint32_t index = min(first + k * kThreads, a.groups - 1U);

            m3_load4<D>(a.gate, index, g[k]);
            m3_load4<D>(a.up, index, u[k]);
        }
#pragma unroll
        for (uint32_t k = 0U; k < kUnroll; ++k) {
            uint32_t index = first + k * kThreads;

            if (index < a.groups) {
                uint32_t r[4];

                m3_silu4<D>(g[k], u[k], table, r);
                m3_store4<D>(a.output, index, r);
            }
        }
    }
    if (blockIdx.x == 0U && threadIdx.x < a.tail) {
        const uint64_t e = 4ULL * a.groups + threadIdx.x;
        float g = m3_bits_f32(m3_load_element(a.gate + size * e, D));
        float u = m3_bits_f32(m3_load_element(a.up + size * e, D));

        m3_store_element(a.output + size * e, D, m3_gated_silu_bits(g, u, D));
    }
}

__global__ __launch_bounds__(256) void m3_gated_silu_general_kernel(
    m3_activation_general_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
    const uint64_t out_size = a.dtypes[0] == M3N_F32 ? 4U : 2U;

    for (uint64_t f = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         f < a.count; f += step) {
        int64_t offsets[2];

        m3_general_offsets(a, f, offsets);
        float g = m3_bits_f32(
            m3_load_element(a.inputs[0] + offsets[0], a.dtypes[1]));
        float u = m3_bits_f32(
            m3_load_element(a.inputs[1] + offsets[1], a.dtypes[2]));

        m3_store_element(a.output + out_size * f, a.dtypes[0],
                         m3_gated_silu_bits(g, u, a.dtypes[1]));
    }
}

/* ---- launch planning ----------------------------------------------------- */

bool m3_same_shape(const m3_hip_view *a, const m3_hip_view *b)
{
    if (a->rank != b->rank) {
        return false;
    }
    for (uint32_t axis = 0U; axis < a->rank; ++axis) {
        if (a->shape[axis] != b->shape[axis]) {
            return false;
        }
    }
    return true;
}

bool m3_is_float(uint32_t dtype)
{
    return dtype == M3_HIP_F32 || dtype == M3_HIP_F16 ||
           dtype == M3_HIP_BF16;
}

/* Fills the general kernel's arguments from the coalesced index space of
 * `output` with inputs `first` and `second` (second may be null). */
void m3_general_args(const m3_hip_view *output, const m3_hip_view *first,
                     const m3_hip_view *second,
                     m3_activation_general_args *args)
{
    const m3_hip_view *operands[3] = {output, first,
                                      second != nullptr ? second : first};
    m3_index_plan plan;

    m3_plan_index_space(output, operands, 3U, &plan);
    std::memset(args, 0, sizeof(*args));
    args->inputs[0] = (const uint8_t *)first->base + first->byte_offset;
    args->inputs[1] =
        second != nullptr
            ? (const uint8_t *)second->base + second->byte_offset
            : args->inputs[0];
    args->output = (uint8_t *)output->base + output->byte_offset;
    args->dtypes[0] = output->dtype;
    args->dtypes[1] = first->dtype;
    args->dtypes[2] = second != nullptr ? second->dtype : first->dtype;
    args->rank = plan.rank;
    args->count = output->element_count;
    for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
        args->shape[axis] = plan.shape[axis];
        args->strides[0][axis] = plan.strides[1][axis];
        args->strides[1][axis] = plan.strides[2][axis];
    }
}

/* True when `view` is contiguous and its first element is aligned to
 * `alignment` bytes. */
bool m3_vector_ready(const m3_hip_view *view, uintptr_t alignment)
{
    uintptr_t address = (uintptr_t)view->base + view->byte_offset;

    return m3_view_is_contiguous(view) && address % alignment == 0U;
}

template <uint32_t D>
void m3_launch_silu_vec(m3_hip_device *device, const m3_silu_vec_args &args,
                        uint32_t blocks, hipEvent_t start, hipEvent_t stop)
{
    if (D == M3N_BF16) {
        hipExtLaunchKernelGGL(m3_gated_silu_bf16_kernel, dim3(blocks),
                              dim3(kThreads), 0, device->stream, start, stop,
                              0U, args,
                              (const uint4 *)device->silu_bf16_table);
        return;
    }
    hipExtLaunchKernelGGL((m3_gated_silu_vec_kernel<D>), dim3(blocks),
                          dim3(kThreads), 0, device->stream, start, stop, 0U,
                          args);
}

} // namespace

int m3_silu_table_build(m3_hip_device *device, char *message,
                        size_t capacity)
{
    int code = m3_hip_check((hipError_t)m3_hip_malloc((void **)&device->silu_bf16_table,
                                      kSiluTableEntries * sizeof(uint16_t)),
                            "hipMalloc(GATED_SILU table)", message, capacity);

    if (code != M3_HIP_OK) {
        device->silu_bf16_table = nullptr;
        return code;
    }
    hipLaunchKernelGGL(m3_silu_table_build_kernel,
                       dim3(kSiluTableEntries / 256U), dim3(256), 0,
                       device->stream, device->silu_bf16_table);
    return m3_hip_check(hipGetLastError(), "m3_silu_table_build", message,
                        capacity);
}

void m3_silu_table_release(m3_hip_device *device)
{
    if (device->silu_bf16_table != nullptr) {
        (void)hipFree(device->silu_bf16_table);
        device->silu_bf16_table = nullptr;
    }
}

extern "C" int m3_hip_launch_tanh(m3_hip_device *device,
                                  const m3_hip_view *input,
                                  const m3_hip_view *output, char *message,
                                  size_t capacity)
{
    if (device == nullptr || !m3_view_is_valid(input) ||
        !m3_view_is_valid(output) || input->dtype != M3_HIP_F32 ||
        output->dtype != M3_HIP_F32 || input->rank == 0U ||
        !m3_same_shape(input, output) || !m3_view_is_contiguous(output)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "tanh launch arguments are malformed");
    }
    const uint64_t count = output->element_count;

    if (count == 0U) {
        return M3_HIP_OK;
    }
    /* below 2^32 elements the vector kernel's 32-bit group indices, plus
     * one grid stride (at most 2^28), stay below 2^32 */
    if (m3_vector_ready(input, 16U) && m3_vector_ready(output, 16U) &&
        count < (1ULL << 32U)) {
        m3_tanh_vec_args args;

        args.list_gate = device->gate;
        args.input = (const uint8_t *)input->base + input->byte_offset;
        args.output = (uint8_t *)output->base + output->byte_offset;
        args.groups = (uint32_t)(count / 4U);
        args.tail = (uint32_t)(count % 4U);
        uint32_t blocks = m3_grid_blocks(
            device, args.groups == 0U ? 1U : args.groups,
            kThreads * kTanhUnroll, kBlocksPerCu);

        return m3_hip_launch(
            device, "m3_tanh",
            [&](hipEvent_t start, hipEvent_t stop) {
                hipExtLaunchKernelGGL(m3_tanh_vec_kernel, dim3(blocks),
                                      dim3(kThreads), 0, device->stream, start,
                                      stop, 0U, args);
            },
            message, capacity);
    }
    m3_activation_general_args args;

    m3_general_args(output, input, nullptr, &args);
    args.list_gate = device->gate;
    uint32_t blocks = m3_grid_blocks(device, count, 256U, 16U);

    return m3_hip_launch(
        device, "m3_tanh_strided",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_tanh_general_kernel, dim3(blocks),
                                  dim3(256), 0, device->stream, start, stop,
                                  0U, args);
        },
        message, capacity);
}

extern "C" int m3_hip_launch_gated_silu(m3_hip_device *device,
                                        const m3_hip_view *gate,
                                        const m3_hip_view *up,
                                        const m3_hip_view *output,
                                        char *message, size_t capacity)
{
    if (device == nullptr || !m3_view_is_valid(gate) ||
        !m3_view_is_valid(up) || !m3_view_is_valid(output) ||
        !m3_is_float(gate->dtype) || !m3_is_float(up->dtype) ||
        !m3_is_float(output->dtype) || !m3_same_shape(gate, up) ||
        !m3_same_shape(gate, output) || !m3_view_is_contiguous(output)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "gated SiLU launch arguments are malformed");
    }
    const uint64_t count = output->element_count;

    if (count == 0U) {
        return M3_HIP_OK;
    }
    const uint32_t dtype = output->dtype;
    const uintptr_t alignment = dtype == M3_HIP_F32 ? 16U : 8U;

    if (gate->dtype == dtype && up->dtype == dtype &&
        m3_vector_ready(gate, alignment) && m3_vector_ready(up, alignment) &&
        m3_vector_ready(output, alignment) &&
        count < (1ULL << 32U)) { /* 32-bit group indices, as for TANH */
        m3_silu_vec_args args;

        args.list_gate = device->gate;
        args.gate = (const uint8_t *)gate->base + gate->byte_offset;
        args.up = (const uint8_t *)up->base + up->byte_offset;
        args.output = (uint8_t *)output->base + output->byte_offset;
        args.groups = (uint32_t)(count / 4U);
        args.tail = (uint32_t)(count % 4U);
        uint32_t blocks = m3_grid_blocks(
            device, args.groups == 0U ? 1U : args.groups,
            kThreads * kUnroll, kBlocksPerCu);
        void (*launch)(m3_hip_device *, const m3_silu_vec_args &, uint32_t,
                       hipEvent_t, hipEvent_t) =
            dtype == M3_HIP_F32   ? &m3_launch_silu_vec<M3N_F32>
            : dtype == M3_HIP_F16 ? &m3_launch_silu_vec<M3N_F16>
                                  : &m3_launch_silu_vec<M3N_BF16>;
        const char *name = dtype == M3_HIP_F32   ? "m3_gated_silu"
                           : dtype == M3_HIP_F16 ? "m3_gated_silu_f16"
                                                 : "m3_gated_silu_bf16";

        return m3_hip_launch(
            device, name,
            [&](hipEvent_t start, hipEvent_t stop) {
                launch(device, args, blocks, start, stop);
            },
            message, capacity);
    }
    m3_activation_general_args args;

    m3_general_args(output, gate, up, &args);
    args.list_gate = device->gate;
    uint32_t blocks = m3_grid_blocks(device, count, 256U, 16U);

    return m3_hip_launch(
        device, "m3_gated_silu_strided",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_gated_silu_general_kernel, dim3(blocks),
                                  dim3(256), 0, device->stream, start, stop,
                                  0U, args);
        },
        message, capacity);
}
