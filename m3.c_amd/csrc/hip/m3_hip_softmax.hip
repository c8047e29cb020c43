/*
 * m3_hip_softmax.hip - last-axis softmax for gfx950, bit-exact with the
 * CPU provider of the reference.
 *
 * Reference semantics (src/m3_op_execute_basic.c:124-180): per row
 *   pass 1: maximum, and the count k of +inf entries;
 *   pass 2: sum = ((0 + e0) + e1) + ... in F32, e_j = expf(v_j - max),
 *           skipped when max is +-inf;
 *   pass 3: p_j = e_j / sum; an all -inf row gives zeros; a row whose
 *           maximum is +inf gives 1/k on its +inf entries and 0 elsewhere.
 * Rounding is reproduced, not approximated:
 *   - the maximum and k are order-independent, so they are reduced across
 *     the 64 lanes of a wavefront (DPP row operations);
 *   - e_j uses m3_expf (the libm algorithm restated bit for bit);
 *   - the sum keeps the reference's left-to-right F32 order: one
 *     dependent addition per column, the addends reaching the summing
 *     lanes through LDS or DPP broadcasts;
 *   - p_j is the IEEE F32 quotient e_j / sum, formed as
 *     RN_f32(e_j * RN_f64(1/sum)) where that is exact (m3_softmax_scale4).
 *
 * Kernels for rows contiguous along the last axis, by width; "VEC" rows
 * have aligned starts and a width that is a multiple of 4 and move in 16-
 * or 8-byte accesses, other rows element by element; row starts may be
 * evenly spaced or follow several outer axes (m3_softmax_row):
 *   - VEC rows of 513..1024 columns, and of 257..512 columns with 16-bit
 *     input or output: four rows per wave, one per 16-lane DPP row, the
 *     in-order sums carried in registers by additions whose addends are
 *     broadcast from lane to lane (row_newbcast), with no LDS traffic
 *     (m3_softmax_lane_rows_kernel).
 *   - other rows up to 2048 columns: wave-independent rows
 *     (m3_softmax_rows_kernel). A wave holds R rows in VGPRs, reduces max
 *     and k, forms e_j in place and streams 256-column chunks through a
 *     wave-private LDS tile where the in-order sums run; no workgroup
 *     barrier separates the phases, so waves overlap memory and
 *     arithmetic.
 *   - VEC rows with evenly spaced starts up to 8192 columns: a 256-thread
 *     workgroup owns a tile of whole rows in LDS (m3_softmax_tiled_kernel);
 *     phase 1 loads a row, reduces max and k and writes e_j to LDS; phase 2
 *     has one lane per row sum its row in order and form 1/sum in double;
 *     phase 3 reads e_j back, scales, rounds and stores coalesced. LDS rows
 *     are padded by 4 floats so the per-row walks hit distinct banks.
 *   - any other row: three streamed passes over 256-column chunks
 *     (m3_softmax_stream_kernel), carrying the in-order sum across chunks
 *     and reading the row again for the scale pass.
 * A last axis that is not contiguous runs one thread per row through the
 * three passes (m3_softmax_general_kernel).
 */
#include "m3_hip_internal.h"
#include "m3_libm.h"

#include <algorithm>
#include <cstring>
#include <utility>

namespace {

constexpr uint32_t kThreads = 256U;
constexpr uint32_t kWaves = kThreads / 64U;
constexpr uint32_t kStaticLds = 1024U; /* room for the static arrays */
constexpr uint32_t kTiledLdsCap = 65536U; /* dynamic LDS of the tiled kernel */
constexpr uint32_t kMaxTileRows = 16U;
constexpr uint32_t kMaxWidth = 8192U;
constexpr uint32_t kPad = 4U;
constexpr uint32_t kChunk = 256U;         /* columns per LDS chunk */
constexpr uint32_t kLine = kChunk + kPad; /* LDS floats per chunk row */
constexpr uint64_t kMaxGrid = 1U << 20;   /* workgroups; waves loop beyond */
constexpr uint64_t kMaxLaneGrid = 0x7fffffffU; /* grid x limit */
constexpr double kHbmBytesPerUs = 8.0e6; /* MI355X peak, 8 TB/s */
constexpr double kLateFactor = 0.95;
constexpr double kLateFloorUs = 3.0;
constexpr double kHoldFactor = 1.25;
constexpr uint32_t kLaneRowWavesPerSimd = 4U; /* amdgpu_waves_per_eu */
constexpr uint32_t kStreamRows = 4U; /* rows per workgroup, streamed kernel */

/* Four F32 -inf: what a load past the end of a row reads instead. Never
 * written; not const, so that it is in the global address space like the
 * rows and a select between the two stays a global load. */
__device__ float4 m3_minus_inf4 = {-INFINITY, -INFINITY, -INFINITY,
                                   -INFINITY};

struct m3_softmax_args {
    const uint8_t *input;
    uint8_t *output;
    uint64_t rows;
    uint64_t row_stride; /* input bytes between rows (outer_rank <= 1) */
    uint32_t width;
    uint32_t in_dtype;
    uint32_t out_dtype;
    uint32_t tile_rows;
    /* lane-row kernel: s_memrealtime ticks after its start past which a
     * wave still waiting for its rows counts as late */
    uint32_t late_ticks;
    /* lane-row kernel: s_memrealtime ticks after its start before which a
     * wave does not store its results (0: no hold) */
    uint32_t hold_ticks;
    /* Rows whose starts are not evenly spaced (outer_rank > 1): row r
     * starts at input + sum over axes of coordinate(r, axis) * stride. */
    uint32_t outer_rank;
    uint64_t outer_shape[M3_HIP_MAX_RANK];
    int64_t outer_strides[M3_HIP_MAX_RANK];
    m3_hip_gate list_gate;
};

/* Start of input row `row`. */
__device__ __forceinline__ const uint8_t *m3_softmax_row(
    const m3_softmax_args &a, uint64_t row)
{
    if (a.outer_rank <= 1U) {
        return a.input + row * a.row_stride;
    }
    int64_t offset = 0;
    uint64_t rest = row;

    for (int axis = (int)a.outer_rank - 1; axis >= 0; --axis) {
        const uint64_t dim = a.outer_shape[axis];
        const uint64_t q = rest / dim;

        offset += (int64_t)(rest - q * dim) * a.outer_strides[axis];
        rest = q;
    }
    return a.input + offset;
}

/* Wave64 reductions through DPP row operations, which stay in the VALU
 * (a shuffle is an LDS permute with its round-trip latency):
 *   quad_perm [1,0,3,2] and [2,3,0,1]  - quads,
 *   row_half_mirror, row_mirror        - 8 and 16 lanes,
 *   row_bcast:15 into rows 1 and 3     - pairs of rows,
 *   row_bcast:31 into rows 2 and 3     - lane 63 holds the whole wave.
 * `identity` is what the lanes of a row outside the row mask contribute.
 * The result is read from lane 63 into a scalar register. */
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t m3_dpp(uint32_t identity, uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_update_dpp((int)identity, (int)x, CTRL,
                                                 ROW_MASK, 0xF, false);
}

template <typename Op>
__device__ __forceinline__ uint32_t m3_wave_reduce(uint32_t v,
                                                   uint32_t identity, Op op)
{
    v = op(v, m3_dpp<0xB1, 0xF>(identity, v));
    v = op(v, m3_dpp<0x4E, 0xF>(identity, v));
    v = op(v, m3_dpp<0x141, 0xF>(identity, v));
    v = op(v, m3_dpp<0x140, 0xF>(identity, v));
    v = op(v, m3_dpp<0x142, 0xA>(identity, v));
    v = op(v, m3_dpp<0x143, 0xC>(identity, v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

__device__ __forceinline__ float m3_wave_max(float v)
{
    return m3_bits_f32(m3_wave_reduce(
        m3_f32_bits(v), m3_f32_bits(-INFINITY), [](uint32_t x, uint32_t y) {
            return m3_f32_bits(fmaxf(m3_bits_f32(x), m3_bits_f32(y)));
        }));
}

__device__ __forceinline__ uint32_t m3_wave_sum(uint32_t v)
{
    return m3_wave_reduce(v, 0U, [](uint32_t x, uint32_t y) { return x + y; });
}

__device__ __forceinline__ uint32_t m3_wave_max_u32(uint32_t v)
{
    return m3_wave_reduce(v, 0U,
                          [](uint32_t x, uint32_t y) { return max(x, y); });
}

/* A value that is equal in every lane of the wave, moved to a scalar
 * register so that branches on it are uniform (the compiler cannot prove
 * that a cross-lane reduction is uniform). */
__device__ __forceinline__ uint32_t m3_uniform_u32(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)v);
}

__device__ __forceinline__ float m3_uniform_f32(float v)
{
    return __builtin_bit_cast(float, m3_uniform_u32(m3_f32_bits(v)));
}

/* Lane `k`'s double, as a wave-uniform value. */
__device__ __forceinline__ double m3_lane_f64(double v, int k)
{
    uint64_t bits = __builtin_bit_cast(uint64_t, v);
    uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)bits, k);
    uint32_t hi =
        (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(bits >> 32U), k);

    return __builtin_bit_cast(double, ((uint64_t)hi << 32U) | lo);
}

/* Four 16-bit values widened to F32. */
__device__ __forceinline__ float4 m3_widen4(uint32_t lo, uint32_t hi,
                                            uint32_t dtype)
{
    return make_float4(
        m3_bits_f32(m3_load_as_f32_bits(lo & 0xffffU, dtype)),
        m3_bits_f32(m3_load_as_f32_bits(lo >> 16U, dtype)),
        m3_bits_f32(m3_load_as_f32_bits(hi & 0xffffU, dtype)),
        m3_bits_f32(m3_load_as_f32_bits(hi >> 16U, dtype)));
}

/* A load that is nontemporal (data read once) or ordinary (data read
 * again soon, which the caches may keep). */
template <bool NT, typename T>
__device__ __forceinline__ T m3_softmax_read(const T *p)
{
    if (NT) {
        return __builtin_nontemporal_load(p);
    }
    return *p;
}

/* Four consecutive row elements starting at column c, as F32, from an
 * aligned row (16 bytes for F32, 8 for 16-bit dtypes); nontemporal unless
 * NT is false. */
template <bool F32IO, bool NT = true>
__device__ __forceinline__ float4 m3_softmax_load4(const uint8_t *row,
                                                   uint64_t c, uint32_t dtype)
{
    if (F32IO || dtype == M3N_F32) {
        const m3_f32x4 w =
            m3_softmax_read<NT>((const m3_f32x4 *)(row + c * 4U));

        return make_float4(w[0], w[1], w[2], w[3]);
    }
    const m3_u32x2 h = m3_softmax_read<NT>((const m3_u32x2 *)(row + c * 2U));

    return m3_widen4(h[0], h[1], dtype);
}

/* Columns c..c+3 of a row of `width` elements at any alignment, element
 * by element; columns at or past the width read as -inf. */
template <bool F32IO>
__device__ __forceinline__ float4 m3_softmax_load4_masked(
    const uint8_t *row, uint32_t c, uint32_t width, uint32_t dtype)
{
    float x[4];

#pragma unroll
    for (uint32_t i = 0U; i < 4U; ++i) {
        const uint32_t col = min(c + i, width - 1U);
        float value;

        if (F32IO || dtype == M3N_F32) {
            value = *(const float *)(row + (uint64_t)col * 4U);
        } else {
            value = m3_bits_f32(m3_load_as_f32_bits(
                *(const uint16_t *)(row + (uint64_t)col * 2U), dtype));
        }
        x[i] = c + i < width ? value : -INFINITY;
    }
    return make_float4(x[0], x[1], x[2], x[3]);
}

/* Four results at column c, rounded to the output dtype (streaming
 * stores). */
template <bool F32IO>
__device__ __forceinline__ void m3_softmax_store4(uint8_t *row, uint64_t c,
                                                  uint32_t dtype, float4 p)
{
    if (F32IO || dtype == M3N_F32) {
        m3_stream_store((float4 *)(row + c * 4U), p);
        return;
    }
    uint2 packed;

    packed.x = m3_store_from_f32_bits(m3_f32_bits(p.x), dtype) |
               (m3_store_from_f32_bits(m3_f32_bits(p.y), dtype) << 16U);
    packed.y = m3_store_from_f32_bits(m3_f32_bits(p.z), dtype) |
               (m3_store_from_f32_bits(m3_f32_bits(p.w), dtype) << 16U);
    m3_stream_store((uint2 *)(row + c * 2U), packed);
}

/* Stores the columns of c..c+3 that are inside the width, element by
 * element (output rows of any width). */
template <bool F32IO>
__device__ __forceinline__ void m3_softmax_store4_masked(
    uint8_t *row, uint32_t c, uint32_t width, uint32_t dtype, float4 p)
{
    const float x[4] = {p.x, p.y, p.z, p.w};

#pragma unroll
    for (uint32_t i = 0U; i < 4U; ++i) {
        if (c + i >= width) {
            continue;
        }
        if (F32IO || dtype == M3N_F32) {
            __builtin_nontemporal_store(
                x[i], (float *)(row + (uint64_t)(c + i) * 4U));
        } else {
            __builtin_nontemporal_store(
                (uint16_t)m3_store_from_f32_bits(m3_f32_bits(x[i]), dtype),
                (uint16_t *)(row + (uint64_t)(c + i) * 2U));
        }
    }
}

/* Loads and stores of four columns, vectorised for aligned rows whose
 * width is a multiple of 4 (VEC) and element-wise otherwise. No load sits
 * under a branch: a column past the width loads from an address that is
 * always valid (m3_minus_inf4, or the row's first columns) and the result
 * is replaced, so the compiler can wait for each load alone instead of
 * for every load in flight. */
template <bool F32IO, bool VEC, bool NT = true>
__device__ __forceinline__ float4 m3_softmax_get4(const uint8_t *row,
                                                  uint32_t c, uint32_t width,
                                                  uint32_t dtype)
{
    if (!VEC) {
        return m3_softmax_load4_masked<F32IO>(row, c, width, dtype);
    }
    const bool inside = c < width;

    if (F32IO || dtype == M3N_F32) {
        const m3_f32x4 *source =
            inside ? (const m3_f32x4 *)(row + (uint64_t)c * 4U)
                   : (const m3_f32x4 *)&m3_minus_inf4;
        const m3_f32x4 w = m3_softmax_read<NT>(source);

        return make_float4(w[0], w[1], w[2], w[3]);
    }
    const float4 x =
        m3_softmax_load4<F32IO, NT>(row, inside ? c : 0U, dtype);

    return inside ? x
                  : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
}

template <bool F32IO, bool VEC>
__device__ __forceinline__ void m3_softmax_put4(uint8_t *row, uint32_t c,
                                                uint32_t width, uint32_t dtype,
                                                float4 p)
{
    if (VEC) {
        if (c < width) {
            m3_softmax_store4<F32IO>(row, c, dtype, p);
        }
        return;
    }
    m3_softmax_store4_masked<F32IO>(row, c, width, dtype, p);
}

/* p = e / sum, the IEEE F32 quotient, for e >= 0 and sum >= 1 given
 * inverse = RN_f64(1/sum).
 *
 * q = RN_f64(e * inverse) is within 2^-52 (relative) of e / sum, so
 * RN_f32(q) is the quotient unless e / sum lies within 2^-52 of an F32
 * rounding midpoint:
 *   - for a normal result the midpoints have 25 significant bits; e / sum
 *     equals one only when sum = 2^k (1/sum then exact, and q too), and
 *     otherwise stays at least 2^-49 away from it;
 *   - below 2^-126 the midpoints are (2k+1) * 2^-150, numbers with few
 *     significant bits, so e = sum * midpoint holds for ordinary sums
 *     (147 * 2^-149 / 98 = 3 * 2^-150) and q falls on either side of the
 *     tie. Such a quotient rounds to a positive subnormal, or to +0 only
 *     from the tie 2^-150, whose correct rounding is +0 (a non-tie
 *     quotient near 2^-150 is at least 2^-24 relative from it).
 * So RN_f32(q) is the quotient whenever it is +0 or normal, and a lane
 * whose result is a positive subnormal takes the F32 division instead,
 * behind a wave-uniform test (sum is recovered exactly as
 * RN_f32(1 / inverse)). The test is one v_cmp_class per element. */
__device__ __forceinline__ float m3_softmax_scale(float e, double inverse)
{
    constexpr int kPositiveSubnormal = 1 << 7;
    const float p = (float)((double)e * inverse);
    const bool tiny = __builtin_amdgcn_classf(p, kPositiveSubnormal);

    if (__any(tiny)) {
        if (tiny) {
            return e / (float)(1.0 / inverse);
        }
    }
    return p;
}

__device__ __forceinline__ float4 m3_softmax_scale4(float4 e, double inverse)
{
    constexpr int kPositiveSubnormal = 1 << 7;
    float4 p;

    p.x = (float)((double)e.x * inverse);
    p.y = (float)((double)e.y * inverse);
    p.z = (float)((double)e.z * inverse);
    p.w = (float)((double)e.w * inverse);
    const bool tx = __builtin_amdgcn_classf(p.x, kPositiveSubnormal);
    const bool ty = __builtin_amdgcn_classf(p.y, kPositiveSubnormal);
    const bool tz = __builtin_amdgcn_classf(p.z, kPositiveSubnormal);
    const bool tw = __builtin_amdgcn_classf(p.w, kPositiveSubnormal);

    if (__any(tx | ty | tz | tw)) {
        const float sum = (float)(1.0 / inverse);

        p.x = tx ? e.x / sum : p.x;
        p.y = ty ? e.y / sum : p.y;
        p.z = tz ? e.z / sum : p.z;
        p.w = tw ? e.w / sum : p.w;
    }
    return p;
}

/* The reference's left-to-right F32 sum of `width` values (a multiple of
 * 4) at `line` in LDS. Loads run one 16-element block ahead of the
 * dependent additions so LDS latency overlaps the chain. */
__device__ __forceinline__ float m3_row_sum_in_order(const float *line,
                                                     uint32_t width)
{
    float sum = 0.0F;
    uint32_t c = 0U;

    if (width >= 16U) {
        float4 current[4];
        float4 next[4];

#pragma unroll
        for (uint32_t k = 0U; k < 4U; ++k) {
            current[k] = *(const float4 *)(line + 4U * k);
        }
        for (c = 16U; c + 16U <= width; c += 16U) {
#pragma unroll
            for (uint32_t k = 0U; k < 4U; ++k) {
                next[k] = *(const float4 *)(line + c + 4U * k);
            }
#pragma unroll
            for (uint32_t k = 0U; k < 4U; ++k) {
                sum = sum + current[k].x;
                sum = sum + current[k].y;
                sum = sum + current[k].z;
                sum = sum + current[k].w;
            }
#pragma unroll
            for (uint32_t k = 0U; k < 4U; ++k) {
                current[k] = next[k];
            }
        }
#pragma unroll
        for (uint32_t k = 0U; k < 4U; ++k) {
            sum = sum + current[k].x;
            sum = sum + current[k].y;
            sum = sum + current[k].z;
            sum = sum + current[k].w;
        }
    }
    for (; c < width; c += 4U) {
        float4 e = *(const float4 *)(line + c);

        sum = sum + e.x;
        sum = sum + e.y;
        sum = sum + e.z;
        sum = sum + e.w;
    }
    return sum;
}

/* Per-row state shared through LDS between the phases. */
struct m3_row_state {
    float maximum;
    uint32_t infinities;
    double inverse;      /* 1/sum for finite rows */
    float one_over_count; /* 1/k for rows whose maximum is +inf */
    uint32_t pad;
};

template <bool F32IO>
__global__ __launch_bounds__(256) void m3_softmax_tiled_kernel(
    m3_softmax_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    extern __shared__ float lds[];
    __shared__ m3_row_state state[kMaxTileRows];
    __shared__ uint64_t exp_table[32];
    const uint32_t lane = threadIdx.x & 63U;
    const uint32_t wave = threadIdx.x >> 6U;
    const uint32_t width = a.width;
    const uint32_t pitch = width + kPad;
    const uint32_t in_dtype = F32IO ? (uint32_t)M3N_F32 : a.in_dtype;
    const uint32_t out_dtype = F32IO ? (uint32_t)M3N_F32 : a.out_dtype;
    const uint32_t out_size = out_dtype == M3N_F32 ? 4U : 2U;

    if (threadIdx.x < 32U) {
        exp_table[threadIdx.x] = m3_expf_table[threadIdx.x];
    }
    for (uint64_t tile = blockIdx.x; tile * a.tile_rows < a.rows;
         tile += gridDim.x) {
        const uint64_t first_row = tile * a.tile_rows;
        const uint32_t tile_rows =
            (uint32_t)min((uint64_t)a.tile_rows, a.rows - first_row);

        __syncthreads();
        /* Phase 1: max, +inf count and e_j for each row of this wave. */
        for (uint32_t r = wave; r < tile_rows; r += kWaves) {
            const uint8_t *row = a.input + (first_row + r) * a.row_stride;
            float *line = lds + (uint64_t)r * pitch;
            float maximum = -INFINITY;
            uint32_t infinities = 0U;

            for (uint32_t c = lane * 4U; c < width; c += 256U) {
                float4 v = m3_softmax_load4<F32IO>(row, c, in_dtype);

                maximum = fmaxf(maximum, fmaxf(fmaxf(v.x, v.y),
                                               fmaxf(v.z, v.w)));
                infinities += (v.x == INFINITY) + (v.y == INFINITY) +
                              (v.z == INFINITY) + (v.w == INFINITY);
                *(float4 *)(line + c) = v;
            }
            maximum = m3_wave_max(maximum);
            infinities = m3_wave_sum(infinities);
            if (maximum != INFINITY && maximum != -INFINITY) {
                for (uint32_t c = lane * 4U; c < width; c += 256U) {
                    float4 v = *(float4 *)(line + c);
                    float4 e;

                    e.x = m3_expf_with_table(v.x - maximum, exp_table);
                    e.y = m3_expf_with_table(v.y - maximum, exp_table);
                    e.z = m3_expf_with_table(v.z - maximum, exp_table);
                    e.w = m3_expf_with_table(v.w - maximum, exp_table);
                    *(float4 *)(line + c) = e;
                }
            }
            if (lane == 0U) {
                state[r].maximum = maximum;
                state[r].infinities = infinities;
            }
        }
        __syncthreads();
        /* Phase 2: the reference's left-to-right F32 sum, one lane per row. */
        if (threadIdx.x < tile_rows) {
            m3_row_state *s = &state[threadIdx.x];
            float maximum = s->maximum;

            if (maximum != INFINITY && maximum != -INFINITY) {
                s->inverse = 1.0 / (double)m3_row_sum_in_order(
                                       lds + (uint64_t)threadIdx.x * pitch,
                                       width);
            } else if (maximum == INFINITY) {
                s->one_over_count = 1.0F / (float)s->infinities;
            }
        }
        __syncthreads();
        /* Phase 3: scale, round to the output dtype, store. */
        for (uint32_t r = wave; r < tile_rows; r += kWaves) {
            const float *line = lds + (uint64_t)r * pitch;
            uint8_t *out = a.output + (first_row + r) * (uint64_t)width *
                                          out_size;
            const m3_row_state s = state[r];

            for (uint32_t c = lane * 4U; c < width; c += 256U) {
                float4 v = *(const float4 *)(line + c);
                float4 p;

                if (s.maximum == -INFINITY) {
                    p = make_float4(0.0F, 0.0F, 0.0F, 0.0F);
                } else if (s.maximum == INFINITY) {
                    p.x = v.x == INFINITY ? s.one_over_count : 0.0F;
                    p.y = v.y == INFINITY ? s.one_over_count : 0.0F;
                    p.z = v.z == INFINITY ? s.one_over_count : 0.0F;
                    p.w = v.w == INFINITY ? s.one_over_count : 0.0F;
                } else {
                    p = m3_softmax_scale4(v, s.inverse);
                }
                m3_softmax_store4<F32IO>(out, c, out_dtype, p);
            }
        }
    }
}

/* Adds four floats to s in order. */
__device__ __forceinline__ float m3_add4(float s, float4 e)
{
    s = s + e.x;
    s = s + e.y;
    s = s + e.z;
    return s + e.w;
}

/* Sum of the first n (a multiple of 4, at most 256) floats of an LDS line,
 * continuing the left-to-right F32 sum s. A full chunk keeps DEPTH 16-byte
 * loads in flight ahead of the dependent additions; a partial chunk (the
 * end of a trimmed row) issues four loads per 16 elements before adding
 * them, so LDS latency is paid once per 16 additions, not per 4. */
template <int DEPTH>
__device__ __forceinline__ float m3_chunk_sum(float s, const float *line,
                                              uint32_t n)
{
    if (n == kChunk) {
        float4 ahead[DEPTH];

#pragma unroll
        for (int i = 0; i < DEPTH; ++i) {
            ahead[i] = *(const float4 *)(line + 4 * i);
        }
#pragma unroll
        for (int i = 0; i < (int)kChunk / 4; ++i) {
            float4 e = ahead[i % DEPTH];

            if (i + DEPTH < (int)kChunk / 4) {
                ahead[i % DEPTH] = *(const float4 *)(line + 4 * (i + DEPTH));
            }
            s = m3_add4(s, e);
        }
        return s;
    }
    uint32_t c = 0U;

    for (; c + 16U <= n; c += 16U) {
        float4 a = *(const float4 *)(line + c);
        float4 b = *(const float4 *)(line + c + 4U);
        float4 d = *(const float4 *)(line + c + 8U);
        float4 f = *(const float4 *)(line + c + 12U);

        s = m3_add4(s, a);
        s = m3_add4(s, b);
        s = m3_add4(s, d);
        s = m3_add4(s, f);
    }
    for (; c < n; c += 4U) {
        s = m3_add4(s, *(const float4 *)(line + c));
    }
    return s;
}

/* Orders this wave's LDS writes before its later LDS reads of other lanes'
 * data (the LDS executes one wave's operations in issue order). */
__device__ __forceinline__ void m3_wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/* Scales and stores one row of a register-resident task: p_j = e_j / sum
 * for a finite maximum, zeros for an all -inf row, 1/k on the k +inf
 * entries of a row whose maximum is +inf. `v` holds e_j (finite rows) or
 * the inputs (other rows). */
template <int VPL, bool F32IO, bool VEC>
__device__ __forceinline__ void m3_softmax_emit_row(
    const float4 (&v)[VPL], float maximum, double inverse, uint8_t *out,
    uint32_t lane, uint32_t width, uint32_t out_dtype)
{
    if (maximum != INFINITY && maximum != -INFINITY) {
#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const uint32_t c = lane * 4U + kChunk * j;

            if (VEC && c >= width) {
                continue;
            }
            m3_softmax_put4<F32IO, VEC>(out, c, width, out_dtype,
                                        m3_softmax_scale4(v[j], inverse));
        }
        return;
    }
    float one_over_count = 0.0F;

    if (maximum == INFINITY) {
        uint32_t count = 0U;

#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            count += (v[j].x == INFINITY) + (v[j].y == INFINITY) +
                     (v[j].z == INFINITY) + (v[j].w == INFINITY);
        }
        one_over_count = 1.0F / (float)m3_wave_sum(count);
    }
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const uint32_t c = lane * 4U + kChunk * j;
        float4 p;

        if (VEC && c >= width) {
            continue;
        }
        p.x = v[j].x == INFINITY ? one_over_count : 0.0F;
        p.y = v[j].y == INFINITY ? one_over_count : 0.0F;
        p.z = v[j].z == INFINITY ? one_over_count : 0.0F;
        p.w = v[j].w == INFINITY ? one_over_count : 0.0F;
        m3_softmax_put4<F32IO, VEC>(out, c, width, out_dtype, p);
    }
}

/* Wave-independent rows (width <= 256 * VPL). Each wave takes R
 * consecutive rows at a time and keeps them in VGPRs, lane l holding
 * columns 4l + 256j .. 4l + 256j + 3 (VPL float4 per lane per row). It
 * reduces each row's maximum with DPP, forms e_j in place, then walks the
 * row in 256-column chunks, writing each chunk of its R rows to a
 * wave-private LDS tile where every lane continues the left-to-right sum
 * of row l % R. All 64 lanes run that chain: a wave instruction takes the
 * same issue slot at any lane count, and a full mask keeps the chain in
 * one basic block with its LDS reads. The sum stops after the wave's last
 * column holding something other than -inf: the later terms are +0 and
 * leave a nonnegative F32 sum unchanged, so masked (causal) rows cost
 * half. p_j is formed from the registers and streamed out. No workgroup
 * barrier is needed after the table copy, so the waves of a CU overlap
 * their loads, arithmetic and sums freely. VEC rows (aligned, width a
 * multiple of 4) move in 16-byte (F32) or 8-byte (16-bit) accesses; other
 * rows element by element, with columns past the width read as -inf. */
template <int VPL, int R, int DEPTH, bool F32IO, bool VEC>
__device__ __forceinline__ void m3_softmax_rows(const m3_softmax_args &a)
{
    __shared__ float tiles[kWaves][R][kLine];
    __shared__ uint64_t exp_table[32];
    const uint32_t lane = threadIdx.x & 63U;
    const uint32_t wave = m3_uniform_u32(threadIdx.x >> 6U);
    const uint32_t width = a.width;
    const uint32_t in_dtype = F32IO ? (uint32_t)M3N_F32 : a.in_dtype;
    const uint32_t out_dtype = F32IO ? (uint32_t)M3N_F32 : a.out_dtype;
    const uint32_t out_size = out_dtype == M3N_F32 ? 4U : 2U;
    const uint64_t out_pitch = (uint64_t)width * out_size;
    const uint64_t tasks = (a.rows + R - 1U) / R;
    float *tile = &tiles[wave][0][0];

    if (threadIdx.x < 32U) {
        exp_table[threadIdx.x] = m3_expf_table[threadIdx.x];
    }
    __syncthreads();
    for (uint64_t task = (uint64_t)blockIdx.x * kWaves + wave; task < tasks;
         task += (uint64_t)gridDim.x * kWaves) {
        const uint64_t first_row = task * R;
        /* rows of this task that exist (the last task may be partial) */
        const uint32_t present =
            (uint32_t)min((uint64_t)R, a.rows - first_row);
        float4 v[R][VPL];
        float maximum[R];
        uint32_t last = 0U; /* 1 + index of the last float4 not all -inf */

        /* Every load is issued and none is under a branch, so the wave
         * waits for each row's data alone: row 0 is reduced and
         * exponentiated while the later rows are still arriving. A row past
         * the end of the tensor (the last task) reads the task's first row
         * and is never stored. A VEC column past the width reads four F32
         * -inf from m3_minus_inf4 (16-bit inputs: column 0, replaced by
         * -inf). A variant serves widths above 256 * VPL / 2, so its chunks
         * j < VPL / 2 are always inside the row. */
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint8_t *row = m3_softmax_row(
                a, first_row + ((uint32_t)k < present ? (uint32_t)k : 0U));

#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                const uint32_t c = lane * 4U + kChunk * j;
                const bool inside = (VPL > 1 && j < VPL / 2) || c < width;

                if (!VEC) {
                    v[k][j] = m3_softmax_load4_masked<F32IO>(row, c, width,
                                                             in_dtype);
                } else if (F32IO || in_dtype == M3N_F32) {
                    const m3_f32x4 *source =
                        inside ? (const m3_f32x4 *)(row + (uint64_t)c * 4U)
                               : (const m3_f32x4 *)&m3_minus_inf4;
                    const m3_f32x4 w = __builtin_nontemporal_load(source);

                    v[k][j] = make_float4(w[0], w[1], w[2], w[3]);
                } else {
                    const float4 x = m3_softmax_load4<F32IO>(
                        row, inside ? c : 0U, in_dtype);

                    v[k][j] = inside ? x
                                     : make_float4(-INFINITY, -INFINITY,
                                                   -INFINITY, -INFINITY);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < R; ++k) {
            float m = -INFINITY;

#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                const float t = fmaxf(fmaxf(v[k][j].x, v[k][j].y),
                                      fmaxf(v[k][j].z, v[k][j].w));

                m = fmaxf(m, t);
                last = t != -INFINITY ? max(last, lane + 64U * j + 1U) : last;
            }
            m = m3_uniform_f32(m3_wave_max(m));
            maximum[k] = m;
            if (m != INFINITY && m != -INFINITY) {
#pragma unroll
                for (int j = 0; j < VPL; ++j) {
                    v[k][j].x = m3_expf_with_table(v[k][j].x - m, exp_table);
                    v[k][j].y = m3_expf_with_table(v[k][j].y - m, exp_table);
                    v[k][j].z = m3_expf_with_table(v[k][j].z - m, exp_table);
                    v[k][j].w = m3_expf_with_table(v[k][j].w - m, exp_table);
                }
            }
        }
        const uint32_t wave_length = m3_uniform_u32(m3_wave_max_u32(last)) * 4U;
        const float *line = tile + (lane % (uint32_t)R) * kLine;
        float sum = 0.0F;

#pragma unroll
        for (int j = 0; j < VPL; ++j) {
            const uint32_t base = kChunk * j;

            if (base >= wave_length) {
                break;
            }
#pragma unroll
            for (int k = 0; k < R; ++k) {
                *(float4 *)(tile + k * kLine + lane * 4U) = v[k][j];
            }
            m3_wave_sync();
            sum = m3_chunk_sum<DEPTH>(sum, line,
                                      min(wave_length - base, kChunk));
            m3_wave_sync();
        }
        const double inverse_of_lane = 1.0 / (double)sum;

#pragma unroll
        for (int k = 0; k < R; ++k) {
            if ((uint32_t)k >= present) {
                continue;
            }
            m3_softmax_emit_row<VPL, F32IO, VEC>(
                v[k], maximum[k], m3_lane_f64(inverse_of_lane, k),
                a.output + (first_row + (uint32_t)k) * out_pitch, lane, width,
                out_dtype);
        }
    }
}

template <int VPL, int R, int DEPTH, bool F32IO, bool VEC>
__global__ __launch_bounds__(256) void m3_softmax_rows_kernel(
    m3_softmax_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    m3_softmax_rows<VPL, R, DEPTH, F32IO, VEC>(a);
}

/* x of lane CTRL selects within this lane's 16-lane DPP row (`identity`
 * where the control names no lane). */
template <int CTRL>
__device__ __forceinline__ float m3_dpp_f32(float identity, float x)
{
    return m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
        (int)m3_f32_bits(identity), (int)m3_f32_bits(x), CTRL, 0xF, 0xF,
        false));
}

template <int CTRL>
__device__ __forceinline__ uint32_t m3_dpp_u32(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, 0xF, 0xF,
                                                 false);
}

/* Maximum and sum over the 16 lanes of a DPP row, in every lane of it:
 * quads, then the other quad of each half (row_half_mirror), then the
 * other half (row_mirror). */
__device__ __forceinline__ float m3_row16_max(float m)
{
    m = fmaxf(m, m3_dpp_f32<0xB1>(-INFINITY, m));
    m = fmaxf(m, m3_dpp_f32<0x4E>(-INFINITY, m));
    m = fmaxf(m, m3_dpp_f32<0x141>(-INFINITY, m));
    return fmaxf(m, m3_dpp_f32<0x140>(-INFINITY, m));
}

__device__ __forceinline__ uint32_t m3_row16_sum(uint32_t n)
{
    n += m3_dpp_u32<0xB1>(n);
    n += m3_dpp_u32<0x4E>(n);
    n += m3_dpp_u32<0x141>(n);
    return n + m3_dpp_u32<0x140>(n);
}

/* s + (e of lane N of this DPP row): row_newbcast:N hands every lane of
 * the row the addend of lane N, so the 16 lanes carry the same sum. */
template <int N>
__device__ __forceinline__ float m3_add_from_lane(float s, float e)
{
    return s + m3_dpp_f32<0x150 + N>(0.0F, e);
}

/* Continues the left-to-right sum over the 64 columns of one block: lane
 * N holds columns 4N..4N+3 of it in e. */
template <int... N>
__device__ __forceinline__ float m3_block_sum(float s, float4 e,
                                              std::integer_sequence<int, N...>)
{
    ((s = m3_add_from_lane<N>(s, e.x), s = m3_add_from_lane<N>(s, e.y),
      s = m3_add_from_lane<N>(s, e.z), s = m3_add_from_lane<N>(s, e.w)),
     ...);
    return s;
}

/* The same sum with the running value passed from lane to lane: step g,
 * the same four instructions in every lane, takes lane g - 1's sum
 * (row_ror:1; lane 0 takes lane 15's, the end of the previous block) and
 * adds lane g's four columns, so that lane g holds the in-order sum after
 * step g and lane 15 after the block. A dependent DPP addition takes about
 * 12 cycles and a plain one 4: 6 cycles per column against 12 for
 * m3_block_sum, whose DPP operand is the addend, not the sum. */
__device__ __forceinline__ float m3_block_sum_passed(float s, float4 e)
{
#pragma unroll
    for (int g = 0; g < 16; ++g) {
        s = m3_dpp_f32<0x121>(0.0F, s) + e.x;
        s = s + e.y;
        s = s + e.z;
        s = s + e.w;
    }
    return s;
}

/* Rows of 32Q + 1 .. 64Q columns (VEC: aligned, a multiple of 4 wide),
 * Q = 8 or 16, with the in-order sum carried in registers. A wave takes
 * four consecutive rows, one per 16-lane DPP row (lanes 16k..16k+15 hold
 * row k); lane i of a row holds columns 4i + 64j .. 4i + 64j + 3 (block
 * j = 0..Q-1), so each load instruction reads four runs of 256 bytes (F32)
 * or 128 bytes (16-bit). The maximum is reduced within the 16 lanes and
 * e_j formed in place; then the left-to-right sum is one dependent
 * addition per column, whose addend comes from the lane holding it
 * (m3_add_from_lane), and the four rows advance together. Against the
 * rows kernel this removes the LDS tile: there every lane group reads its
 * row's e_j back from LDS, at a bandwidth cost per CU that set the sum's
 * pace. As there, the sum stops after the wave's last float4 holding
 * something other than -inf (later terms are +0). Rows whose maximum is
 * +-inf are written from their inputs before the exponentials (zeros, or
 * 1/k on their k +inf entries) behind a wave-uniform test. FULL rows are
 * exactly 64Q wide; otherwise blocks of the second half may lie past the
 * width, read -inf there and are not stored. F32IO: F32 in and out, with
 * immediate-offset addressing; otherwise any float dtypes. One task per
 * wave: the grid covers them all (a loop over tasks took 30 more VGPRs and
 * ran slower).
 *
 * All waves issue their loads at once, and the waves whose rows the HBM
 * serves last decide when the kernel ends: by then most SIMDs are idle and
 * the sum's latency is what counts. A wave whose rows arrive more than
 * a.late_ticks after its start (s_memrealtime) therefore sums with
 * m3_block_sum_passed, half the latency per column; the others keep
 * m3_block_sum, which leaves more issue slots to the waves sharing their
 * SIMD. Both perform the same additions in the same order. */
template <int Q, bool FULL, bool F32IO>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void m3_softmax_lane_rows_kernel(m3_softmax_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    __shared__ uint64_t exp_table[32];
    const uint32_t lane = threadIdx.x & 63U;
    const uint32_t wave = m3_uniform_u32(threadIdx.x >> 6U);
    const uint32_t sub = lane & 15U;
    const uint32_t width = a.width;
    const uint32_t in_dtype = F32IO ? (uint32_t)M3N_F32 : a.in_dtype;
    const uint32_t out_dtype = F32IO ? (uint32_t)M3N_F32 : a.out_dtype;
    const uint64_t out_pitch =
        (uint64_t)width * (out_dtype == M3N_F32 ? 4U : 2U);
    const uint64_t tasks = (a.rows + 3U) / 4U;
    const uint64_t task = (uint64_t)blockIdx.x * kWaves + wave;
    const uint64_t start = __builtin_amdgcn_s_memrealtime();
    /* The expf table's load goes first and the rows' loads right after it,
     * ahead of the barrier that publishes the table in LDS. The barrier's
     * fences cover LDS only, so the rows stay in flight across it instead
     * of being issued after the table's round trip (0.35 us less on C2 in
     * bench.py, alternating libraries on one box). A wave past the last
     * task loads the last task's rows and stops at the barrier. */
    const uint64_t table_word = m3_expf_table[threadIdx.x & 31U];
    const uint64_t mine = task < tasks ? task : tasks - 1U;
    const uint64_t row = mine * 4U + (lane >> 4U);
    const bool present = task < tasks && row < a.rows;
    /* a row past the end of the tensor reads the task's first row */
    const uint8_t *in = m3_softmax_row(a, row < a.rows ? row : mine * 4U);
    uint8_t *out = a.output + row * out_pitch;
    float4 v[Q];

#pragma unroll
    for (int j = 0; j < Q; ++j) {
        const uint32_t c = sub * 4U + 64U * j;
        const bool inside = FULL || j < Q / 2 || c < width;

        if (F32IO) {
            const m3_f32x4 *source =
                inside ? (const m3_f32x4 *)(in + sub * 16U) + 16 * j
                       : (const m3_f32x4 *)&m3_minus_inf4;
            const m3_f32x4 w = __builtin_nontemporal_load(source);

            v[j] = make_float4(w[0], w[1], w[2], w[3]);
        } else {
            const float4 x =
                m3_softmax_load4<false>(in, inside ? c : 0U, in_dtype);

            v[j] = inside ? x
                          : make_float4(-INFINITY, -INFINITY, -INFINITY,
                                        -INFINITY);
        }
    }
    if (threadIdx.x < 32U) {
        exp_table[threadIdx.x] = table_word;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    if (task < tasks) {
        float m = -INFINITY;
        uint32_t last = 0U; /* 1 + index of the last float4 not all -inf */

#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const float t = fmaxf(fmaxf(v[j].x, v[j].y),
                                  fmaxf(v[j].z, v[j].w));

            m = fmaxf(m, t);
            last = t != -INFINITY ? sub + 16U * j + 1U : last;
        }
        m = m3_row16_max(m);
        const uint32_t length = m3_uniform_u32(m3_wave_max_u32(last));
        const bool finite = m != INFINITY && m != -INFINITY;
        /* every load has returned here (all were reduced); the wait makes
         * the clock read follow them */
        __builtin_amdgcn_s_waitcnt(0);
        const bool late =
            __builtin_amdgcn_s_memrealtime() - start > (uint64_t)a.late_ticks;
        /* stores p at block j when the block is inside the row */
        auto put = [&](int j, float4 p) {
            const uint32_t c = sub * 4U + 64U * j;

            if (!FULL && j >= Q / 2 && c >= width) {
                return;
            }
            if (F32IO) {
                m3_stream_store((float4 *)(out + sub * 16U) + 16 * j, p);
            } else {
                m3_softmax_store4<false>(out, c, out_dtype, p);
            }
        };

        if (M3_ANY_LANE(!finite)) {
            uint32_t count = 0U;

#pragma unroll
            for (int j = 0; j < Q; ++j) {
                count += (v[j].x == INFINITY) + (v[j].y == INFINITY) +
                         (v[j].z == INFINITY) + (v[j].w == INFINITY);
            }
            const float one_over_count = 1.0F / (float)m3_row16_sum(count);

            if (!finite && present) {
#pragma unroll
                for (int j = 0; j < Q; ++j) {
                    float4 p;

                    p.x = v[j].x == INFINITY ? one_over_count : 0.0F;
                    p.y = v[j].y == INFINITY ? one_over_count : 0.0F;
                    p.z = v[j].z == INFINITY ? one_over_count : 0.0F;
                    p.w = v[j].w == INFINITY ? one_over_count : 0.0F;
                    put(j, p);
                }
            }
        }
        /* e_j against a finite maximum (what the other rows get is not
         * used). Each block's four exponentials are completed in place
         * before the next block's start (the empty asm statement): left to
         * itself the scheduler interleaves the start of every block's expf
         * with the end of others and spills. */
        const float shift = finite ? m : 0.0F;

#pragma unroll
        for (int j = 0; j < Q; ++j) {
            v[j].x = m3_expf_with_table(v[j].x - shift, exp_table);
            v[j].y = m3_expf_with_table(v[j].y - shift, exp_table);
            v[j].z = m3_expf_with_table(v[j].z - shift, exp_table);
            v[j].w = m3_expf_with_table(v[j].w - shift, exp_table);
            asm volatile(""
                         : "+v"(v[j].x), "+v"(v[j].y), "+v"(v[j].z),
                           "+v"(v[j].w));
        }
        float sum = 0.0F;

        if (late) {
#pragma unroll
            for (int j = 0; j < Q; ++j) {
                if (16U * j < length) {
                    sum = m3_block_sum_passed(sum, v[j]);
                }
            }
            sum = m3_dpp_f32<0x15F>(0.0F, sum); /* lane 15's, to the row */
        } else {
#pragma unroll
            for (int j = 0; j < Q; ++j) {
                if (16U * j < length) {
                    sum = m3_block_sum(sum, v[j],
                                       std::make_integer_sequence<int, 16>());
                }
            }
        }
        /* A wave whose rows arrived early waits, up to a.hold_ticks after
         * its start, before it stores: its writes then do not compete with
         * the reads still in flight for other waves. Bounded by the clock,
         * so every wave goes on. */
        while (__builtin_amdgcn_s_memrealtime() - start <
               (uint64_t)a.hold_ticks) {
            __builtin_amdgcn_s_sleep(2);
        }
        if (finite && present) {
            const double inverse = 1.0 / (double)sum;

#pragma unroll
            for (int j = 0; j < Q; ++j) {
                put(j, m3_softmax_scale4(v[j], inverse));
            }
        }
    }
}

/* Float4 slot, in a line of the streamed kernel's ring, of the chunk's
 * float4 f = 4i + q (columns 16i + 4q .. +3): the summing lane i reads
 * slots 4i..4i+3, rotated by (i >> 1) + (i >> 3) so that the 16-byte reads
 * of the lanes that the LDS serves together fall on distinct banks. The
 * producers write through the same map. */
__device__ __forceinline__ uint32_t m3_ring_slot(uint32_t f)
{
    const uint32_t i = f >> 2U;

    return (i << 2U) | (((f & 3U) + (i >> 1U) + (i >> 3U)) & 3U);
}

/* Continues the left-to-right sum over one 256-column chunk of a ring line.
 * Lane i of each 16-lane DPP row holds columns 16i..16i+15 (e, in order),
 * and the running sum passes from lane to lane: step g, the same four
 * instructions in every lane, takes lane g - 1's sum (row_ror:1; lane 0
 * takes lane 15's, the end of the previous chunk) and adds lane g's
 * sixteen columns. Only lane g's result is the in-order sum after step g;
 * after the chunk lane 15 holds it. One DPP addition per sixteen columns:
 * a dependent DPP addition costs about three plain ones. */
__device__ __forceinline__ float m3_pass_along_sum(float s, const float4 (&e)[4])
{
#pragma unroll
    for (int g = 0; g < 16; ++g) {
        s = m3_dpp_f32<0x121>(0.0F, s) + e[0].x;
        s = s + e[0].y;
        s = s + e[0].z;
        s = s + e[0].w;
#pragma unroll
        for (int q = 1; q < 4; ++q) {
            s = m3_add4(s, e[q]);
        }
    }
    return s;
}

/* x where mask is all ones, +0 where it is zero. */
__device__ __forceinline__ float4 m3_keep4(float4 x, uint32_t mask)
{
    return make_float4(m3_bits_f32(m3_f32_bits(x.x) & mask),
                       m3_bits_f32(m3_f32_bits(x.y) & mask),
                       m3_bits_f32(m3_f32_bits(x.z) & mask),
                       m3_bits_f32(m3_f32_bits(x.w) & mask));
}

/* e_j of four inputs against the row maximum m. */
__device__ __forceinline__ float4 m3_exp4(float4 v, float m,
                                          const uint64_t *table)
{
    return make_float4(m3_expf_with_table(v.x - m, table),
                       m3_expf_with_table(v.y - m, table),
                       m3_expf_with_table(v.z - m, table),
                       m3_expf_with_table(v.w - m, table));
}

/* Rows of any width, streamed by a workgroup of four waves that owns R
 * consecutive rows and reads them three times in 256-column chunks, lane l
 * at columns 4l..4l+3 of a chunk:
 *   pass 1  wave w takes the chunks w, w+4, ...: maximum, +inf count and
 *           last column that is not -inf, combined through LDS;
 *   pass 2  the in-order sums. One wave runs the chains (DPP row k of its
 *           lanes sums row k, m3_pass_along_sum) while the other three
 *           produce the e_j of the next chunks into an LDS ring, one chunk
 *           each per step: the exponentials run beside the chains on other
 *           SIMDs instead of in front of them;
 *   pass 3  wave w takes the chunks w, w+4, ... again: e_j (the same
 *           function of the same input), scaled, rounded and stored.
 * The rows are read with ordinary loads, not nontemporal ones, so that the
 * caches may serve a pass's reads of lines the previous pass fetched.
 * The sums stop after the last column holding something other than -inf
 * in a row with a finite maximum (later terms are +0). Rows past the end
 * of the tensor repeat the task's first row and store its values again.
 * Rows whose starts are not evenly spaced come from the outer axes. */
template <bool F32IO, bool VEC>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(4))) void m3_softmax_stream_kernel(
    m3_softmax_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    constexpr int R = (int)kStreamRows;
    constexpr int P = (int)kWaves - 1; /* producer waves */
    __shared__ float ring[2 * P][R][kLine];
    __shared__ float part_max[kWaves][R];
    __shared__ uint32_t part_inf[kWaves][R];
    __shared__ uint32_t part_last[kWaves][R];
    __shared__ uint64_t exp_table[32];
    const uint32_t lane = threadIdx.x & 63U;
    const uint32_t wave = m3_uniform_u32(threadIdx.x >> 6U);
    const uint32_t width = a.width;
    const uint32_t in_dtype = F32IO ? (uint32_t)M3N_F32 : a.in_dtype;
    const uint32_t out_dtype = F32IO ? (uint32_t)M3N_F32 : a.out_dtype;
    const uint32_t out_size = out_dtype == M3N_F32 ? 4U : 2U;
    const uint64_t out_pitch = (uint64_t)width * out_size;
    const uint64_t tasks = (a.rows + R - 1U) / R;
    const uint32_t chunks = (width + kChunk - 1U) / kChunk;

    if (threadIdx.x < 32U) {
        exp_table[threadIdx.x] = m3_expf_table[threadIdx.x];
    }
    for (uint64_t task = blockIdx.x; task < tasks; task += gridDim.x) {
        const uint64_t first_row = task * R;
        const uint32_t present =
            (uint32_t)min((uint64_t)R, a.rows - first_row);
        const uint8_t *rows[R];
        uint8_t *outs[R];
        float maximum[R];
        uint32_t infinities[R];
        uint32_t last[R];

#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint64_t row =
                first_row + ((uint32_t)k < present ? (uint32_t)k : 0U);

            rows[k] = m3_softmax_row(a, row);
            outs[k] = a.output + row * out_pitch;
            maximum[k] = -INFINITY;
            infinities[k] = 0U;
            last[k] = 0U;
        }
        /* pass 1, last chunk first (pass 2 then starts on the chunks read
         * most recently, pass 3 ends there): two chunks per iteration keep
         * 2R loads in flight; a chunk index past the row reads -inf */
        for (uint32_t j = wave; j < chunks; j += 2U * kWaves) {
            float4 x[R][2];
            uint32_t chunk[2];

#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t t = j + (uint32_t)h * kWaves;

                chunk[h] = t < chunks ? chunks - 1U - t : chunks;
            }
#pragma unroll
            for (int k = 0; k < R; ++k) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    x[k][h] = m3_softmax_get4<F32IO, VEC, false>(
                        rows[k], chunk[h] * kChunk + lane * 4U, width,
                        in_dtype);
                }
            }
#pragma unroll
            for (int k = 0; k < R; ++k) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const float4 e = x[k][h];
                    const float t = fmaxf(fmaxf(e.x, e.y), fmaxf(e.z, e.w));

                    maximum[k] = fmaxf(maximum[k], t);
                    infinities[k] += (e.x == INFINITY) + (e.y == INFINITY) +
                                     (e.z == INFINITY) + (e.w == INFINITY);
                    last[k] = t != -INFINITY
                                  ? max(last[k], chunk[h] * 64U + lane + 1U)
                                  : last[k];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float m = m3_wave_max(maximum[k]);
            const uint32_t n = m3_wave_sum(infinities[k]);
            const uint32_t l = m3_wave_max_u32(last[k]);

            if (lane == 0U) {
                part_max[wave][k] = m;
                part_inf[wave][k] = n;
                part_last[wave][k] = l;
            }
        }
        __syncthreads();
        uint32_t length = 0U;
        uint32_t finite[R]; /* all ones for a finite maximum, else zero */

#pragma unroll
        for (int k = 0; k < R; ++k) {
            float m = part_max[0][k];
            uint32_t n = part_inf[0][k];
            uint32_t l = part_last[0][k];

#pragma unroll
            for (uint32_t w = 1U; w < kWaves; ++w) {
                m = fmaxf(m, part_max[w][k]);
                n += part_inf[w][k];
                l = max(l, part_last[w][k]);
            }
            maximum[k] = m3_uniform_f32(m);
            infinities[k] = m3_uniform_u32(n);
            finite[k] =
                maximum[k] != INFINITY && maximum[k] != -INFINITY ? ~0U : 0U;
            length = max(length, (m3_uniform_u32(l) * 4U) & finite[k]);
        }
        /* pass 2 */
        const uint32_t sum_chunks = (min(width, length) + kChunk - 1U) / kChunk;
        const uint32_t steps = (sum_chunks + P - 1U) / P;
        float sum = 0.0F;

        /* the consumer role rotates with the task so that the chains of the
         * workgroups sharing a CU run on different SIMDs */
        const uint32_t consumer = (uint32_t)(task % kWaves);
        const uint32_t producer = (wave + kWaves - consumer - 1U) % kWaves;

        /* a producer's inputs arrive two steps after their loads issue */
        const uint32_t seen = min(width, length);
        float4 x[2][R];

#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int k = 0; k < R; ++k) {
                x[h][k] = m3_softmax_get4<F32IO, VEC, false>(
                    rows[k], (h * P + producer) * kChunk + lane * 4U, seen,
                    in_dtype);
            }
        }
        for (uint32_t step = 0U; step <= steps; ++step) {
            if (wave != consumer) {
                /* producer p: chunk step * P + p into its ring slot (chunks
                 * past the sums, -inf, give zeros nobody reads) */
                float *slot = &ring[(step & 1U) * P + producer][0][0];
                const uint32_t ahead = (step + 2U) * P + producer;

#pragma unroll
                for (int k = 0; k < R; ++k) {
                    const float4 v = (step & 1U) != 0U ? x[1][k] : x[0][k];

                    *(float4 *)(slot + k * kLine + m3_ring_slot(lane) * 4U) =
                        m3_keep4(m3_exp4(v, maximum[k], exp_table),
                                 finite[k]);
                    __builtin_amdgcn_sched_barrier(0);
                }
#pragma unroll
                for (int k = 0; k < R; ++k) {
                    const float4 v = m3_softmax_get4<F32IO, VEC, false>(
                        rows[k], ahead * kChunk + lane * 4U, seen, in_dtype);

                    if ((step & 1U) != 0U) {
                        x[1][k] = v;
                    } else {
                        x[0][k] = v;
                    }
                }
            } else if (step > 0U) {
                /* consumer: the chunks of the previous step, in order; the
                 * 16 lanes of DPP row k sum row k, each reading its sixteen
                 * columns of a chunk once */
                const uint32_t first = (step - 1U) * P;
                const uint32_t i = lane & 15U;

#pragma unroll 1
                for (uint32_t c = 0U; c < P && first + c < sum_chunks; ++c) {
                    const float *line =
                        &ring[((step - 1U) & 1U) * P + c][lane >> 4U][0];
                    float4 e[4];

#pragma unroll
                    for (uint32_t q = 0U; q < 4U; ++q) {
                        e[q] = *(const float4 *)(line +
                                                 m3_ring_slot(4U * i + q) * 4U);
                    }
                    sum = m3_pass_along_sum(sum, e);
                }
            }
            __syncthreads();
        }
        /* the sums (lane 15 of each DPP row) reach the other waves
         * through LDS */
        if (wave == consumer && (lane & 15U) == 15U) {
            part_max[0][lane >> 4U] = sum;
        }
        __syncthreads();
        double inverse[R];
        float one_over_count[R];

#pragma unroll
        for (int k = 0; k < R; ++k) {
            inverse[k] = 1.0 / (double)part_max[0][k];
            one_over_count[k] =
                maximum[k] == INFINITY ? 1.0F / (float)infinities[k] : 0.0F;
        }
        /* pass 3, last chunk first, where pass 2 ended */
        for (uint32_t t = wave; t < chunks; t += kWaves) {
            const uint32_t j = chunks - 1U - t;
            float4 x[R];

#pragma unroll
            for (int k = 0; k < R; ++k) {
                x[k] = m3_softmax_get4<F32IO, VEC, false>(
                    rows[k], j * kChunk + lane * 4U, width, in_dtype);
            }
#pragma unroll
            for (int k = 0; k < R; ++k) {
                const float4 v = x[k];
                const float4 p = m3_softmax_scale4(
                    m3_exp4(v, maximum[k], exp_table), inverse[k]);
                float4 q;

                /* rows without a finite maximum: 1/k on +inf, else 0 */
                q.x = v.x == INFINITY ? one_over_count[k] : 0.0F;
                q.y = v.y == INFINITY ? one_over_count[k] : 0.0F;
                q.z = v.z == INFINITY ? one_over_count[k] : 0.0F;
                q.w = v.w == INFINITY ? one_over_count[k] : 0.0F;
                q = make_float4(
                    m3_bits_f32((m3_f32_bits(p.x) & finite[k]) |
                                (m3_f32_bits(q.x) & ~finite[k])),
                    m3_bits_f32((m3_f32_bits(p.y) & finite[k]) |
                                (m3_f32_bits(q.y) & ~finite[k])),
                    m3_bits_f32((m3_f32_bits(p.z) & finite[k]) |
                                (m3_f32_bits(q.z) & ~finite[k])),
                    m3_bits_f32((m3_f32_bits(p.w) & finite[k]) |
                                (m3_f32_bits(q.w) & ~finite[k])));
                m3_softmax_put4<F32IO, VEC>(outs[k], j * kChunk + lane * 4U,
                                            width, out_dtype, q);
            }
        }
        /* the LDS of this task is reused by the next */
        __syncthreads();
    }
}

/* ---- long rows: one read, the in-order sum in parallel ------------------ */

/* Sum of a float over the 16 lanes of each DPP row (any order: the value
 * is an estimate), in every lane of the row. */
__device__ __forceinline__ float m3_row16_sum_f32(float t)
{
    t = t + m3_dpp_f32<0xB1>(0.0F, t);
    t = t + m3_dpp_f32<0x4E>(0.0F, t);
    t = t + m3_dpp_f32<0x141>(0.0F, t);
    return t + m3_dpp_f32<0x140>(0.0F, t);
}

/* Inclusive prefix sum over the 64 lanes of a wave (lane l gets the sum of
 * lanes 0..l): row_shr within the 16-lane rows, then row_bcast:15 and
 * row_bcast:31 across them. */
__device__ __forceinline__ uint32_t m3_wave_scan_u32(uint32_t x)
{
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xF, 0xF,
                                               false); /* row_shr:1 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xF, 0xF,
                                               false); /* row_shr:2 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xF, 0xF,
                                               false); /* row_shr:4 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xF, 0xF,
                                               false); /* row_shr:8 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xA, 0xF,
                                               false); /* row_bcast:15 */
    x += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xC, 0xF,
                                               false); /* row_bcast:31 */
    return x;
}

/* Rows of up to 256 NW Q columns (VEC: aligned, a multiple of 4 wide),
 * read once and written once (m3_softmax_wide_kernel): a workgroup of NW
 * waves holds one row in VGPRs, wave w the contiguous columns [256Qw,
 * 256Q(w+1)); lane l of a wave holds columns 256j + 4l .. +3 of them in
 * block j (j < Q), and DPP row r of the wave (lanes 16r..16r+15) holds the
 * 64 columns 256j + 64r .. of block j, a "segment". Columns past the width
 * read -inf and give e = +0.
 *
 * The reference's in-order sum s_{c+1} = RN(s_c + e_c) (src/m3_op_execute_
 * basic.c:124-180) is computed exactly without a chain of `width`
 * dependent additions. While s stays inside one binade [2^k, 2^(k+1)), an
 * F32 value there is K ulp_k with K an integer in [2^23, 2^24) (ulp_k =
 * 2^(k-23); the binade "k = -126" is [0, 2^-125) with K in [0, 2^24), zero
 * and the subnormals included), and for e >= 0
 *     RN(K ulp_k + e) = (K + r) ulp_k,  r = RN_int(e / ulp_k)
 * as long as K + r < 2^24 and e / ulp_k is not an exact half-integer (a tie,
 * whose rounding would depend on the parity of K). Within a binade the sum
 * is therefore K plus an integer sum of the r, which any order computes.
 * For each segment the kernel guesses the binade of s at its start from an
 * estimate of the running sum (F32 totals of the segments before it) and
 * forms R = sum of r over its 64 columns, marking the segment when a
 * column is a tie or its r reaches 2^24. Then a walk over the segments in
 * column order keeps the exact s as bits: a segment whose guess matches
 * the binade of s, is not marked and ends inside the binade advances s by
 * R in integer arithmetic; any other segment (the first one, which starts
 * at s = 0; one where s crosses a power of two; a tie; a wrong guess) is
 * summed column by column in order (m3_segment_sum_lanes). Both give the
 * reference's bits; the guesses only decide how often the second form runs
 * (about 3% of the segments for softmax rows of 16,384 normal logits).
 *
 * The maximum, the count of +inf and the last column that is not -inf are
 * reduced across the workgroup first; blocks past that column skip the
 * exponentials. Rows whose maximum is +-inf are written from their inputs
 * (zeros, or 1/k on their k +inf entries). p = e / sum as in the other
 * kernels (m3_softmax_scale4), stored once. */
/* Loads one row's block j of this lane as F32 (columns past the width
 * read -inf). */
template <bool F32IO>
__device__ __forceinline__ float4 m3_wide_load(const uint8_t *in, uint32_t c,
                                               uint32_t width,
                                               uint32_t in_dtype)
{
    if (F32IO) {
        const m3_f32x4 *source =
            c < width ? (const m3_f32x4 *)(in + 4U * (uint64_t)c)
                      : (const m3_f32x4 *)&m3_minus_inf4;
        const m3_f32x4 w = __builtin_nontemporal_load(source);

        return make_float4(w[0], w[1], w[2], w[3]);
    }
    const float4 x = m3_softmax_load4<false>(in, c < width ? c : 0U, in_dtype);

    return c < width ? x
                     : make_float4(-INFINITY, -INFINITY, -INFINITY,
                                   -INFINITY);
}

/* One wave's share of a row's reductions for the wide kernel: maximum,
 * count of +inf and 1 + the last column that is not -inf over this lane's
 * columns first + 256j .. +3, reduced across the wave and posted by lane 0
 * into the workgroup's part arrays. */
template <int Q>
__device__ __forceinline__ void m3_wide_partials(const float4 (&x)[Q],
                                                 uint32_t first,
                                                 uint32_t lane,
                                                 uint32_t wave,
                                                 float *part_max,
                                                 uint32_t *part_inf,
                                                 uint32_t *part_last)
{
    float m = -INFINITY;
    uint32_t infinities = 0U;
    uint32_t last = 0U;

#pragma unroll
    for (int j = 0; j < Q; ++j) {
        const float t = fmaxf(fmaxf(x[j].x, x[j].y), fmaxf(x[j].z, x[j].w));

        m = fmaxf(m, t);
        infinities += (x[j].x == INFINITY) + (x[j].y == INFINITY) +
                      (x[j].z == INFINITY) + (x[j].w == INFINITY);
        last = t != -INFINITY ? first + 256U * j + 4U : last;
    }
    m = m3_wave_max(m);
    infinities = m3_wave_sum(infinities);
    last = m3_wave_max_u32(last);
    if (lane == 0U) {
        part_max[wave] = m;
        part_inf[wave] = infinities;
        part_last[wave] = last;
    }
}


/* The in-order sum continued over one 64-column segment whose values are
 * in registers: lane i of each DPP row holds the segment's columns 4i ..
 * 4i+3 in `e`; the running value passes from lane to lane (row_ror:1), so
 * that lane 15 holds the sum after the 64 values (the other DPP rows repeat
 * the same additions), and lane 15's result is returned. */
__device__ __forceinline__ uint32_t m3_segment_sum_lanes(uint32_t s_bits,
                                                         float4 e)
{
    float t = m3_bits_f32(s_bits);

#pragma unroll
    for (int g = 0; g < 16; ++g) {
        t = m3_dpp_f32<0x121>(0.0F, t) + e.x;
        t = t + e.y;
        t = t + e.z;
        t = t + e.w;
    }
    return (uint32_t)__builtin_amdgcn_readlane((int)m3_f32_bits(t), 15);
}

/* Segments per row whose exponentials the wide kernel keeps in LDS. */
constexpr uint32_t kWideSlots = 48U;
/* Relative distance from a power of two within which an estimated running
 * sum counts as possibly on the other side of it. The in-order F32 sum of
 * n non-negative terms is within (n - 1) 2^-24 of the exact sum, relative,
 * at most 2^-9 for n <= 32768; the estimates (F32 sums of F32 segment
 * totals, fewer than 100 dependent additions) are within 2^-17 of it. So
 * every segment where s crosses a power of two, or whose guessed binade
 * differs from that of s, has an estimate within this margin of one. */
constexpr float kWideMargin = 1.0F / 256.0F;

/* Sum of x over the lanes below this one (lane 0: +0), in any order: the
 * values shifted up one lane (wave_shr:1), then an inclusive scan through
 * row_shr and row_bcast. */
__device__ __forceinline__ float m3_wave_exclusive_sum_f32(float x)
{
    uint32_t b = (uint32_t)__builtin_amdgcn_update_dpp(
        0, (int)m3_f32_bits(x), 0x138, 0xF, 0xF, false); /* wave_shr:1 */
    float t = m3_bits_f32(b);

    t = t + m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
                0, (int)m3_f32_bits(t), 0x111, 0xF, 0xF, false));
    t = t + m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
                0, (int)m3_f32_bits(t), 0x112, 0xF, 0xF, false));
    t = t + m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
                0, (int)m3_f32_bits(t), 0x114, 0xF, 0xF, false));
    t = t + m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
                0, (int)m3_f32_bits(t), 0x118, 0xF, 0xF, false));
    t = t + m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
                0, (int)m3_f32_bits(t), 0x142, 0xA, 0xF, false));
    t = t + m3_bits_f32((uint32_t)__builtin_amdgcn_update_dpp(
                0, (int)m3_f32_bits(t), 0x143, 0xC, 0xF, false));
    return t;
}

/* This lane's index in its wave (0..63), from the lane masks: two vector
 * instructions, without the work-item id, formed where it is called (a
 * volatile statement, so that the compiler neither hoists it out of a loop
 * nor keeps it in a spilled register). */
__device__ __forceinline__ uint32_t m3_lane_index()
{
    uint32_t index;

    asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\t"
                 "v_mbcnt_hi_u32_b32 %0, -1, %0"
                 : "=v"(index));
    return index;
}

/* Index of the lowest set bit of a wave-uniform mask, 64 when there is
 * none (one scalar instruction; s_ff1 gives 0xFFFFFFFF for zero). */
__device__ __forceinline__ uint32_t m3_first_set(uint64_t mask)
{
    uint32_t index;

    asm("s_ff1_i32_b64 %0, %1" : "=s"(index) : "s"(mask));
    return index < 64U ? index : 64U;
}

/* The clamped exponent field of a non-negative F32 (1 for zero and the
 * subnormals, whose ulp is that of the smallest binade). */
__device__ __forceinline__ uint32_t m3_binade(float x)
{
    const uint32_t field = m3_f32_bits(x) >> 23U;

    return field < 1U ? 1U : field;
}

/* The long-row kernel described above. One row per workgroup at a time,
 * no loads ahead in registers and 13-31 KB of LDS, so that several
 * workgroups share a CU (eight to sixteen of two waves up to 8,192
 * columns, four to six of four waves up to 16,384, two or three of eight
 * waves beyond) and one's walk overlaps the others' loads and
 * exponentials. Each row goes through: the loads and the maximum (barrier),
 * the exponentials and the segment totals (barrier), the words, each wave
 * then posting a ready tag, the walk by wave 0, each 64-segment chunk as
 * soon as the waves holding it have posted (barrier), the scale and the
 * stores.
 *
 * The walk sums column by column only the first segment, the segments
 * where s crosses a power of two, marked segments and segments whose
 * guessed binade is wrong; all of these lie where the estimated running
 * sum is within kWideMargin of a power of two at the segment's start or
 * end, or crosses one inside it, or the segment is marked. The data waves
 * stage exactly those segments' exponentials in kSlots LDS lines; a
 * segment the walk needs that is not staged (more than kSlots
 * candidates in the row) has its exponentials formed again from the input
 * by the walking wave, the same expf of the same operands, so that the
 * bits never depend on the prediction. */
template <int Q, int NW, bool F32IO, int WAVES_PER_EU>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(WAVES_PER_EU))) void m3_softmax_wide_kernel(
    m3_softmax_args a)
{
    static_assert(4 * Q <= 64, "one segment of a wave per lane");
    static_assert((NW * Q) % 16 == 0, "whole 64-segment chunks");
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    constexpr uint32_t kSegments = (uint32_t)(NW * Q * 4);
    constexpr uint32_t kWaveSegments = (uint32_t)(4 * Q);
    __shared__ uint64_t exp_table[32];
    __shared__ float part_max[NW];
    __shared__ uint32_t part_inf[NW];
    __shared__ uint32_t part_last[NW];
    __shared__ float totals[NW][kWaveSegments];
    __shared__ uint32_t words[kSegments];
    __shared__ uint8_t slot_of[kSegments];
    __shared__ uint32_t ready[NW];
    __shared__ uint32_t slot_count;
    __shared__ uint32_t carry;
    /* rows of one 64-segment chunk keep 32 lines, which lets seven
     * two-wave workgroups share a CU */
    constexpr uint32_t kSlots = kSegments <= 64U ? 32U : kWideSlots;
    __shared__ float4 staged[kSlots][16];
    /* The walking wave's own values while it walks, so that its registers
     * serve the walk and the kernel fits in 96 VGPRs (five workgroups of
     * four waves per CU; eight waves of 48 values with F32 I/O: 80 VGPRs,
     * three per CU); the other classes keep them in registers, their
     * occupancy the same either way. */
    constexpr bool kPark = NW == 4 || (NW == 8 && Q == 12 && F32IO);
    __shared__ float4 parked[kPark ? Q : 1][64];
    const uint32_t width = a.width;
    const uint32_t in_dtype = F32IO ? (uint32_t)M3N_F32 : a.in_dtype;
    const uint32_t out_dtype = F32IO ? (uint32_t)M3N_F32 : a.out_dtype;
    const uint64_t out_pitch =
        (uint64_t)width * (out_dtype == M3N_F32 ? 4U : 2U);
    uint32_t tag = 0U; /* rows this workgroup has begun */

    if (threadIdx.x < 32U) {
        exp_table[threadIdx.x] = m3_expf_table[threadIdx.x];
    }
    if (threadIdx.x < (uint32_t)NW) {
        ready[threadIdx.x] = 0U;
    }
    const uint32_t wave_index = m3_uniform_u32(threadIdx.x >> 6U);
    for (uint64_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
        /* the lane's columns and masks are formed again each row, not kept
         * live (in spilled registers) across the loop */
        uint32_t lane = m3_lane_index();
        uint32_t wave = wave_index;

        asm volatile("" : "+v"(lane));
        asm volatile("" : "+s"(wave));
        const uint32_t drow = lane >> 4U;
        /* first column of this lane in block 0 */
        const uint32_t first = wave * 256U * Q + 4U * lane;
        const uint8_t *in = m3_softmax_row(a, row);
        uint8_t *out = a.output + row * out_pitch;
        float4 v[Q];

        ++tag;
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            v[j] = m3_wide_load<F32IO>(in, first + 256U * j, width, in_dtype);
        }
        /* maximum, +inf count and 1 + the last column that is not -inf
         * (counting the +inf entries of every row, not only of rows whose
         * maximum is +inf, keeps this kernel out of spilled registers) */
        m3_wide_partials<Q>(v, first, lane, wave, part_max, part_inf,
                            part_last);
        if (wave == 0U && lane == 0U) {
            slot_count = 0U;
        }
        __syncthreads();
        float m = part_max[0];
        uint32_t infinities = part_inf[0];
        uint32_t last = part_last[0];

#pragma unroll
        for (int w = 1; w < NW; ++w) {
            m = fmaxf(m, part_max[w]);
            infinities += part_inf[w];
            last = max(last, part_last[w]);
        }
        m = m3_uniform_f32(m);
        infinities = m3_uniform_u32(infinities);
        last = m3_uniform_u32(last);
        if (m == INFINITY || m == -INFINITY) {
            /* zeros, or 1/k on the k +inf entries */
            const float one_over_count =
                m == INFINITY ? 1.0F / (float)infinities : 0.0F;
            /* columns formed again here (this branch is rare), not kept
             * live from the loads */
            uint32_t column = first;

            asm volatile("" : "+v"(column));
#pragma unroll
            for (int j = 0; j < Q; ++j) {
                const uint32_t c = column + 256U * j;
                float4 p;

                p.x = v[j].x == INFINITY ? one_over_count : 0.0F;
                p.y = v[j].y == INFINITY ? one_over_count : 0.0F;
                p.z = v[j].z == INFINITY ? one_over_count : 0.0F;
                p.w = v[j].w == INFINITY ? one_over_count : 0.0F;
                if (c < width) {
                    m3_softmax_store4<F32IO>(out, c, out_dtype, p);
                }
            }
            __syncthreads(); /* every wave has read the part_* words */
            continue;
        }
        /* e_j; blocks wholly past the last column that is not -inf are
         * zero */
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            if (wave * 256U * Q + 256U * j < last) {
                v[j].x = m3_expf_with_table(v[j].x - m, exp_table);
                v[j].y = m3_expf_with_table(v[j].y - m, exp_table);
                v[j].z = m3_expf_with_table(v[j].z - m, exp_table);
                v[j].w = m3_expf_with_table(v[j].w - m, exp_table);
            } else {
                v[j] = make_float4(0.0F, 0.0F, 0.0F, 0.0F);
            }
            /* one block at a time: interleaving them costs registers */
            __builtin_amdgcn_sched_barrier(0);
        }
        /* estimates: the F32 total of each segment (any order); this
         * wave's segment 4j + r (block j, DPP row r) at totals[wave][4j+r] */
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const float t = m3_row16_sum_f32(((v[j].x + v[j].y) + v[j].z) +
                                             v[j].w);

            if ((lane & 15U) == 0U) {
                totals[wave][4U * j + drow] = t;
            }
        }
        __syncthreads();
        /* Per segment, one per lane (lane l: this wave's segment l): the
         * estimated running sum at its start (the totals before it, in
         * any order) and at its end, the guessed binade E of s at its start
         * and whether s may cross a power of two in it or lie on the other
         * side of one from the estimate (`near`). */
        uint32_t E_lane;
        uint64_t near;
        {
            float before = 0.0F;

            for (uint32_t i = lane; i < wave * kWaveSegments; i += 64U) {
                before += (&totals[0][0])[i];
            }
            before = m3_bits_f32(m3_wave_reduce(
                m3_f32_bits(before), 0U, [](uint32_t x, uint32_t y) {
                    return m3_f32_bits(m3_bits_f32(x) + m3_bits_f32(y));
                }));
            const float own =
                lane < kWaveSegments ? totals[wave][lane] : 0.0F;
            const float start = before + m3_wave_exclusive_sum_f32(own);
            const float end = start + own;

            E_lane = m3_binade(start);
            near = __ballot(lane < kWaveSegments &&
                            m3_binade(start * (1.0F - kWideMargin)) !=
                                m3_binade(end * (1.0F + kWideMargin)));
        }
        /* per segment: R = sum of RN_int(e / ulp) at the guessed binade,
         * marked (R = 0xFFFFFF) when a column is a tie, R reaches 2^24 - 1
         * or E is past the F32 range; word = (E << 24) | R. A segment is a
         * candidate for the column-by-column sum when it is marked or near
         * (bit 4j + DPP row, mod 64, of candidates[j / 16]). */
        constexpr int kGroups = (Q + 15) / 16;
        uint64_t candidates[kGroups];

#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            candidates[g] = 0ULL;
        }
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t E = (uint32_t)__builtin_amdgcn_ds_bpermute(
                (int)(4U * (4U * j + drow)), (int)E_lane);
            const int shift = 150 - (int)E;
            const float f0 = __builtin_ldexpf(v[j].x, shift);
            const float f1 = __builtin_ldexpf(v[j].y, shift);
            const float f2 = __builtin_ldexpf(v[j].z, shift);
            const float f3 = __builtin_ldexpf(v[j].w, shift);
            const float r0 = __builtin_rintf(f0);
            const float r1 = __builtin_rintf(f1);
            const float r2 = __builtin_rintf(f2);
            const float r3 = __builtin_rintf(f3);
            /* |f - RN_int(f)| <= 1/2, equal only at a tie */
            const float off = fmaxf(
                fmaxf(__builtin_fabsf(f0 - r0), __builtin_fabsf(f1 - r1)),
                fmaxf(__builtin_fabsf(f2 - r2), __builtin_fabsf(f3 - r3)));
            const float R = m3_row16_sum_f32(((r0 + r1) + r2) + r3);
            const uint64_t ties = __ballot(off == 0.5F);
            const bool mark = ((ties >> (16U * drow)) & 0xFFFFULL) != 0ULL ||
                              !(R < 16777215.0F) || E > 150U;
            const uint64_t marks = __ballot(mark);

#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const uint64_t bit =
                    ((marks >> (16U * d)) | (near >> (4U * j + d))) & 1ULL;

                candidates[j / 16] |= bit << (4U * (j % 16) + d);
            }
            if ((lane & 15U) == 0U) {
                words[wave * kWaveSegments + 4U * j + drow] =
                    (E << 24U) | (mark ? 0xFFFFFFU : (uint32_t)R);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        /* LDS lines for this wave's candidates, then their exponentials */
        uint32_t count = 0U;

#pragma unroll
        for (int g = 0; g < kGroups; ++g) {
            count += (uint32_t)__builtin_popcountll(candidates[g]);
        }
        uint32_t base = 0U;

        if (lane == 0U && count != 0U) {
            base = atomicAdd(&slot_count, count);
        }
        base = m3_uniform_u32(base);
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint64_t group = candidates[j / 16];
            const uint32_t bit = 4U * (j % 16) + drow;
            const uint32_t slot =
                base +
                (uint32_t)__builtin_popcountll(group & ((1ULL << bit) - 1ULL));
            const bool keep =
                ((group >> bit) & 1ULL) != 0ULL && slot < kSlots;

            if (keep) {
                staged[slot][lane & 15U] = v[j];
            }
            if ((lane & 15U) == 0U) {
                slot_of[wave * kWaveSegments + 4U * j + drow] =
                    keep ? (uint8_t)slot : 0xFFU;
            }
            if (j % 16 == 15) {
                base += (uint32_t)__builtin_popcountll(group);
            }
        }
        /* this wave's words, slots and lines are written: the walk may
         * read them */
        if (lane == 0U) {
            __hip_atomic_store(&ready[wave], tag, __ATOMIC_RELEASE,
                               __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        /* The walk by wave 0, each 64-segment chunk as soon as the waves
         * holding it have posted its words. The state (s, the run's start
         * t0, the prefix sum before it) stays in scalar registers; a step
         * takes two vector compares (the segments whose guess is s's binade,
         * the segment ends where K would reach 2^24) and three reads of a
         * lane (the prefix sums around the run's end and the next
         * segment's LDS line), so that it waits little behind the other
         * waves' vector work. A segment summed column by column reads its
         * staged line, or forms its exponentials again when it has none. */
        if (wave == 0U) {
            uint32_t s = 0U;
            /* the lane index (and the LDS addresses made from it) formed
             * again here, not kept in registers through the row */
            uint32_t wl = m3_lane_index();

            asm volatile("" : "+v"(wl));

            if (kPark) {
#pragma unroll
                for (int j = 0; j < Q; ++j) {
                    parked[kPark ? j : 0][wl] = v[j];
                }
            }
            __builtin_amdgcn_s_setprio(3);
            for (uint32_t chunk = 0U; chunk < kSegments / 64U; ++chunk) {
                const uint32_t w0 = 64U * chunk / kWaveSegments;
                const uint32_t w1 = (64U * chunk + 63U) / kWaveSegments;

                for (uint32_t w = w0 > 1U ? w0 : 1U; w <= w1; ++w) {
                    while (__hip_atomic_load(&ready[w], __ATOMIC_ACQUIRE,
                                             __HIP_MEMORY_SCOPE_WORKGROUP) !=
                           tag) {
                        __builtin_amdgcn_s_sleep(1);
                    }
                }
                const uint32_t word = words[64U * chunk + wl];
                const uint32_t line = slot_of[64U * chunk + wl];
                const uint32_t guess = word >> 24U;
                const uint32_t R = word & 0xFFFFFFU;
                /* prefix sums of R over the chunk: a run from t0 reaches
                 * K + P - offset at the end of segment l, offset = P[t0 - 1]
                 * (unsigned, so that marked segments before t0 cancel;
                 * every sum is below 2^30) */
                const uint32_t P = m3_wave_scan_u32(R);
                const uint64_t unmarked = __ballot(R != 0xFFFFFFU);
                uint32_t t0 = 0U;
                uint32_t offset = 0U;

                while (t0 < 64U) {
                    const uint32_t E = m3_binade(m3_bits_f32(s));
                    const uint32_t K = s - ((E - 1U) << 23U);
                    const uint32_t threshold = 0x1000000U - K + offset;
                    const uint64_t match = __ballot(guess == E);
                    const uint64_t reach = __ballot(P >= threshold);
                    const uint64_t from = ~0ULL << t0;
                    const uint64_t bad = ~(match & unmarked) & from;
                    const uint32_t stop = m3_first_set(bad);
                    const uint64_t below =
                        stop >= 64U ? ~0ULL : (1ULL << stop) - 1ULL;
                    /* over's bits lie below stop */
                    const uint64_t over = reach & from & below;
                    const uint32_t first_over = m3_first_set(over);
                    const uint32_t cross =
                        first_over < stop ? first_over : stop;

                    if (cross >= 64U) {
                        /* the run reaches the chunk's end */
                        s += (uint32_t)__builtin_amdgcn_readlane((int)P, 63) -
                             offset;
                        break;
                    }
                    /* the run [t0, cross) (possibly empty), then segment
                     * `cross` column by column */
                    const uint32_t before =
                        cross == 0U ? 0U
                                    : (uint32_t)__builtin_amdgcn_readlane(
                                          (int)P, (int)(cross - 1U));
                    const uint32_t after =
                        (uint32_t)__builtin_amdgcn_readlane((int)P,
                                                            (int)cross);
                    const uint32_t slot =
                        (uint32_t)__builtin_amdgcn_readlane((int)line,
                                                            (int)cross);
                    const uint32_t t = 64U * chunk + cross;
                    float4 e;

                    s += before - offset;
                    if (slot != 0xFFU) {
                        e = staged[slot][wl & 15U];
                    } else {
                        const uint32_t c = 64U * t + 4U * (wl & 15U);

                        e = m3_wide_load<F32IO>(in, c, width, in_dtype);
                        if (64U * t < last) {
                            e.x = m3_expf_with_table(e.x - m, exp_table);
                            e.y = m3_expf_with_table(e.y - m, exp_table);
                            e.z = m3_expf_with_table(e.z - m, exp_table);
                            e.w = m3_expf_with_table(e.w - m, exp_table);
                        } else {
                            e = make_float4(0.0F, 0.0F, 0.0F, 0.0F);
                        }
                    }
                    s = m3_segment_sum_lanes(s, e);
                    offset = after;
                    t0 = cross + 1U;
                }
            }
            if (wl == 0U) {
                carry = s;
            }
            __builtin_amdgcn_s_setprio(0);
            if (kPark) {
#pragma unroll
                for (int j = 0; j < Q; ++j) {
                    v[j] = parked[kPark ? j : 0][wl];
                }
            }
        }
        __syncthreads();
        const float sum = m3_bits_f32(m3_uniform_u32(carry));
        const double inverse = 1.0 / (double)sum;
        /* the store addresses are formed here: keeping the loads' 64-bit
         * offsets live through the row costs 32 VGPRs */
        uint32_t column = first;

        asm volatile("" : "+v"(column));
#pragma unroll
        for (int j = 0; j < Q; ++j) {
            const uint32_t c = column + 256U * j;

            if (c < width) {
                m3_softmax_store4<F32IO>(out, c, out_dtype,
                                         m3_softmax_scale4(v[j], inverse));
            }
        }
        /* the next row writes part_* and totals (read before the last
         * barrier), words, slot_of and staged (read by the walk, before
         * it), and carry only after two more barriers */
    }
}

typedef void (*m3_softmax_launcher)(dim3, hipStream_t, hipEvent_t,
                                    hipEvent_t, m3_softmax_args);

template <int VPL, int R, int DEPTH, bool F32IO, bool VEC>
void m3_launch_rows(dim3 grid, hipStream_t stream, hipEvent_t start,
                    hipEvent_t stop, m3_softmax_args args)
{
    hipExtLaunchKernelGGL((m3_softmax_rows_kernel<VPL, R, DEPTH, F32IO, VEC>),
                          grid, dim3(kThreads), 0, stream, start, stop, 0U,
                          args);
}

template <int Q, bool FULL, bool F32IO>
void m3_launch_lane_rows(dim3 grid, hipStream_t stream, hipEvent_t start,
                         hipEvent_t stop, m3_softmax_args args)
{
    hipExtLaunchKernelGGL((m3_softmax_lane_rows_kernel<Q, FULL, F32IO>), grid,
                          dim3(kThreads), 0, stream, start, stop, 0U, args);
}

/* Waves per SIMD the wide kernel is built for: seven (at most 72 VGPRs;
 * the compiler takes eight when 64 suffice) for two-wave workgroups of 32
 * values per lane, whose 9 KB of LDS let fourteen to sixteen share a CU;
 * six (at most 80) for four- and eight-wave workgroups of 48 with F32 I/O
 * (six and three per CU, the walking wave's values parked in LDS: faster
 * than five and two per CU, where for eight-wave workgroups of 40 three
 * per CU measured slower); five (at most 96) for two- and four-wave
 * workgroups of 64 values per lane with F32 I/O (ten and five per CU),
 * four-wave ones of 48 with 16-bit I/O and eight-wave ones of 40; four
 * (128 VGPRs) for the rest, which would spill registers at 96. */
template <int Q, int NW, bool F32IO>
constexpr int m3_wide_waves_per_eu()
{
    return NW == 2 && Q == 8 ? 7
           : Q == 12 && F32IO ? 6
           : (NW <= 4 && (F32IO || Q <= 12)) || (NW == 8 && Q <= 10) ? 5
                                                                    : 4;
}

template <int Q, int NW, bool F32IO>
void m3_launch_wide(dim3 grid, hipStream_t stream, hipEvent_t start,
                    hipEvent_t stop, m3_softmax_args args)
{
    hipExtLaunchKernelGGL((m3_softmax_wide_kernel<Q, NW, F32IO,
                                                  m3_wide_waves_per_eu<Q, NW, F32IO>()>),
                          grid, dim3(64 * NW), 0, stream, start, stop, 0U,
                          args);
}

template <bool F32IO, bool VEC>
void m3_launch_stream(dim3 grid, hipStream_t stream, hipEvent_t start,
                      hipEvent_t stop, m3_softmax_args args)
{
    hipExtLaunchKernelGGL((m3_softmax_stream_kernel<F32IO, VEC>), grid,
                          dim3(kThreads), 0, stream, start, stop, 0U, args);
}

struct m3_rows_variant {
    uint32_t vectors_per_lane;
    uint32_t rows_per_wave;
    m3_softmax_launcher f32;      /* F32 in and out, VEC rows */
    m3_softmax_launcher other;    /* any dtypes, VEC rows */
    m3_softmax_launcher elements; /* any dtypes, element-wise rows */
};

/* Wave-independent variants; the first whose width class fits is used.
 * Rows per wave and sum prefetch depth are chosen for four waves per SIMD
 * at widths up to 1024 with F32 in and out; the width-2048 instance and
 * the 16-bit-IO instances from width 1024 take more VGPRs and run three
 * waves per SIMD. */
const m3_rows_variant m3_rows_variants[] = {
    {1U, 8U, &m3_launch_rows<1, 8, 8, true, true>,
     &m3_launch_rows<1, 8, 8, false, true>,
     &m3_launch_rows<1, 8, 8, false, false>},
    {2U, 4U, &m3_launch_rows<2, 4, 8, true, true>,
     &m3_launch_rows<2, 4, 8, false, true>,
     &m3_launch_rows<2, 4, 8, false, false>},
    {4U, 4U, &m3_launch_rows<4, 4, 4, true, true>,
     &m3_launch_rows<4, 4, 4, false, true>,
     &m3_launch_rows<4, 4, 4, false, false>},
    {8U, 2U, &m3_launch_rows<8, 2, 4, true, true>,
     &m3_launch_rows<8, 2, 4, false, true>,
     &m3_launch_rows<8, 2, 4, false, false>},
};

struct m3_softmax_general_args {
    const uint8_t *input;
    uint8_t *output;
    uint64_t rows;
    uint32_t width;
    uint32_t in_dtype;
    uint32_t out_dtype;
    uint32_t outer_rank;
    int64_t column_stride;
    uint64_t outer_shape[M3_HIP_MAX_RANK];
    int64_t outer_strides[M3_HIP_MAX_RANK];
    m3_hip_gate list_gate;
};

__device__ __forceinline__ float m3_general_load(const uint8_t *p,
                                                 uint32_t dtype)
{
    uint32_t raw = dtype == M3N_F32 ? *(const uint32_t *)p
                                    : (uint32_t) * (const uint16_t *)p;

    return m3_bits_f32(m3_load_as_f32_bits(raw, dtype));
}

/* One thread per row: the reference's three passes over a strided row. */
__global__ __launch_bounds__(64) void m3_softmax_general_kernel(
    m3_softmax_general_args a)
{
    if (m3_gate_closed(a.list_gate)) {
        return; /* a check earlier in the list failed */
    }
    const uint32_t out_size = a.out_dtype == M3N_F32 ? 4U : 2U;
    const uint64_t step = (uint64_t)gridDim.x * blockDim.x;

    for (uint64_t row = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
         row < a.rows; row += step) {
        uint64_t rest = row;
        int64_t base = 0;
        float maximum = -INFINITY;
        float sum = 0.0F;
        uint32_t infinities = 0U;

        for (int axis = (int)a.outer_rank - 1; axis >= 0; --axis) {
            uint64_t dim = a.outer_shape[axis];
            uint64_t q = rest / dim;

            base += (int64_t)(rest - q * dim) * a.outer_strides[axis];
            rest = q;
        }
        const uint8_t *in = a.input + base;
        uint8_t *out = a.output + row * a.width * out_size;

        for (uint32_t c = 0U; c < a.width; ++c) {
            float v = m3_general_load(in + (int64_t)c * a.column_stride,
                                      a.in_dtype);

            maximum = v > maximum ? v : maximum;
            infinities += v == INFINITY;
        }
        if (maximum != INFINITY && maximum != -INFINITY) {
            for (uint32_t c = 0U; c < a.width; ++c) {
                float v = m3_general_load(in + (int64_t)c * a.column_stride,
                                          a.in_dtype);

                sum = sum + m3_expf(v - maximum);
            }
        }
        double inverse = 1.0 / (double)sum;
        float one_over_count = 1.0F / (float)infinities;

        for (uint32_t c = 0U; c < a.width; ++c) {
            float v = m3_general_load(in + (int64_t)c * a.column_stride,
                                      a.in_dtype);
            float p;

            if (maximum == -INFINITY) {
                p = 0.0F;
            } else if (maximum == INFINITY) {
                p = v == INFINITY ? one_over_count : 0.0F;
            } else {
                p = m3_softmax_scale(m3_expf(v - maximum), inverse);
            }
            uint32_t raw = m3_store_from_f32_bits(m3_f32_bits(p),
                                                  a.out_dtype);

            if (out_size == 4U) {
                *(uint32_t *)(out + (uint64_t)c * 4U) = raw;
            } else {
                *(uint16_t *)(out + (uint64_t)c * 2U) = (uint16_t)raw;
            }
        }
    }
}

} // namespace

extern "C" int m3_hip_launch_softmax(m3_hip_device *device,
                                     const m3_hip_view *input,
                                     const m3_hip_view *output,
                                     char *message, size_t capacity)
{
    if (device == nullptr || !m3_view_is_valid(input) ||
        !m3_view_is_valid(output) || input->rank == 0U ||
        input->rank != output->rank || input->dtype == M3_HIP_I32 ||
        output->dtype == M3_HIP_I32 || !m3_view_is_contiguous(output)) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "softmax launch arguments are malformed");
    }
    for (uint32_t axis = 0U; axis < input->rank; ++axis) {
        if (input->shape[axis] != output->shape[axis]) {
            return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                               "softmax input and output shapes differ");
        }
    }
    uint64_t width = input->shape[input->rank - 1U];

    if (width == 0U) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "softmax last axis must be nonempty");
    }
    if (output->element_count == 0U) {
        return M3_HIP_OK;
    }
    uint64_t rows = input->element_count / width;
    const uint8_t *in = (const uint8_t *)input->base + input->byte_offset;
    uint8_t *out = (uint8_t *)output->base + output->byte_offset;
    uint32_t in_size = (uint32_t)m3_dtype_bytes(input->dtype);
    uint32_t out_size = (uint32_t)m3_dtype_bytes(output->dtype);

    /* Outer axes (all but the last) of the input, coalesced. */
    m3_hip_view outer = *input;
    m3_index_plan plan;
    const m3_hip_view *operands[1] = {&outer};

    outer.rank = input->rank - 1U;
    m3_plan_index_space(&outer, operands, 1U, &plan);

    if (width > 0xffffffffULL) {
        return m3_hip_fail(message, capacity, M3_HIP_UNSUPPORTED,
                           "softmax rows longer than 2^32 are unsupported");
    }
    const bool uniform_rows = plan.rank == 1U || rows == 1U;
    const bool columns_contiguous =
        width == 1U ||
        input->byte_strides[input->rank - 1U] == (uint64_t)in_size;

    if (columns_contiguous) {
        m3_softmax_args args;
        /* VEC rows: every row start aligned for 4-element accesses */
        bool vec = width % 4U == 0U &&
                   ((uintptr_t)in % (4U * in_size)) == 0U &&
                   ((uintptr_t)out % (4U * out_size)) == 0U;
        const bool f32 =
            input->dtype == M3_HIP_F32 && output->dtype == M3_HIP_F32;

        std::memset(&args, 0, sizeof(args));
        args.list_gate = device->gate;
        args.input = in;
        args.output = out;
        args.rows = rows;
        args.width = (uint32_t)width;
        args.in_dtype = input->dtype;
        args.out_dtype = output->dtype;
        if (uniform_rows) {
            args.outer_rank = 1U;
            args.row_stride = rows == 1U ? 0U : (uint64_t)plan.strides[0][0];
            vec = vec && args.row_stride % (4U * in_size) == 0U;
        } else {
            args.outer_rank = plan.rank;
            for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
                args.outer_shape[axis] = plan.shape[axis];
                args.outer_strides[axis] = plan.strides[0][axis];
                vec = vec && (uint64_t)plan.strides[0][axis] %
                                     (4U * in_size) ==
                                 0U;
            }
        }
        /* VEC rows of 513..1024 columns, and of 257..512 columns with a
         * 16-bit input or output: the lane-row kernel, 16 or 8 float4 per
         * lane (index: [wide][full][f32]). F32 rows of 257..512 columns
         * measured the same or faster on the rows kernel (49.5 against
         * 49.6 us for [65536,512], 23.4 against 22.2 us for [32768,300]);
         * with 16-bit I/O the lane-row kernel is faster at every width
         * (56.6 against 73.3 us for [65536,512] BF16, 38.5 against 58.1 us
         * for [16384,1024] BF16). */
        static const m3_softmax_launcher lane_launchers[2][2][2] = {
            {{&m3_launch_lane_rows<8, false, false>,
              &m3_launch_lane_rows<8, false, true>},
             {&m3_launch_lane_rows<8, true, false>,
              &m3_launch_lane_rows<8, true, true>}},
            {{&m3_launch_lane_rows<16, false, false>,
              &m3_launch_lane_rows<16, false, true>},
             {&m3_launch_lane_rows<16, true, false>,
              &m3_launch_lane_rows<16, true, true>}}};
        const uint64_t lane_blocks =
            (rows + 4U * kWaves - 1U) / (4U * kWaves);
        const uint32_t lane_q = width > 1024U           ? 0U
                                : width > 512U          ? 16U
                                : width > 256U && !f32 ? 8U
                                                        : 0U;

        if (vec && lane_q != 0U && lane_blocks <= kMaxLaneGrid) {
            const dim3 grid((uint32_t)lane_blocks);
            /* late: 0.95 times the time the launch's reads take at peak
             * HBM bandwidth (8.0 us for [16,1024,1024] F32; in bench.py on
             * one box with the store hold, three rounds: 6.0 us 22.8-23.5,
             * 7.1 us 22.8-23.7, 8.0 us 22.7-22.9, 9.0 us 23.5), at least 3 us
             * (about the latency of a first load), unless
             * M3_HIP_SOFTMAX_LATE_US sets it */
            const double late_us =
                device->softmax_late_us >= 0.0F
                    ? (double)device->softmax_late_us
                    : std::max(kLateFloorUs,
                               kLateFactor * (double)rows * (double)width *
                                   in_size / kHbmBytesPerUs);
            const double ticks = late_us * device->wall_clock_khz / 1000.0;

            args.late_ticks = device->wall_clock_khz == 0U || ticks >= 4.0e9
                                  ? 0xffffffffU
                                  : (uint32_t)ticks;
            /* hold: 1.25 times the time the launch's reads take at peak
             * HBM bandwidth (10.5 us for [16,1024,1024] F32; in bench.py on
             * one box, three rounds: 9.0 us 23.1-23.4, 10.0 us 23.0-23.2,
             * 10.5 us 22.7-23.0, 11.0 us 23.5-23.9), when every
             * wave of the launch is resident at once so that all its reads
             * are issued at the start; otherwise none. M3_HIP_SOFTMAX_HOLD_US
             * sets it. */
            const uint64_t resident = (uint64_t)device->compute_units * 4U *
                                      kLaneRowWavesPerSimd;
            const double hold_us =
                device->softmax_hold_us >= 0.0F
                    ? (double)device->softmax_hold_us
                : (rows + 3U) / 4U <= resident
                    ? kHoldFactor * (double)rows * (double)width * in_size /
                          kHbmBytesPerUs
                    : 0.0;
            const double hold = hold_us * device->wall_clock_khz / 1000.0;

            args.hold_ticks = device->wall_clock_khz == 0U || hold >= 4.0e9
                                  ? 0U
                                  : (uint32_t)hold;
            const m3_softmax_launcher launcher =
                lane_launchers[lane_q == 16U][width == 64U * lane_q][f32];

            return m3_hip_launch(
                device, "m3_softmax_rows",
                [&](hipEvent_t start, hipEvent_t stop) {
                    launcher(grid, device->stream, start, stop, args);
                },
                message, capacity);
        }
        for (const m3_rows_variant &variant : m3_rows_variants) {
            if (width > kChunk * variant.vectors_per_lane) {
                continue;
            }
            uint64_t tasks =
                (rows + variant.rows_per_wave - 1U) / variant.rows_per_wave;
            uint64_t blocks = (tasks + kWaves - 1U) / kWaves;
            dim3 grid((uint32_t)(blocks < kMaxGrid ? blocks : kMaxGrid));
            m3_softmax_launcher launcher =
                !vec ? variant.elements : f32 ? variant.f32 : variant.other;

            return m3_hip_launch(
                device, "m3_softmax_rows",
                [&](hipEvent_t start, hipEvent_t stop) {
                    launcher(grid, device->stream, start, stop, args);
                },
                message, capacity);
        }
        /* VEC rows of 2049..32768 columns: a workgroup per row at a time,
         * each row read once, the in-order sum in parallel. */
        if (vec && width > 2048U && width <= 32768U) {
            /* the smallest row class that holds the width: NW waves of Q
             * float4 per lane, 256 NW Q columns; one workgroup per row (the
             * hardware hands a CU's next row to whichever of its workgroups
             * ends first) */
#define M3_WIDE_ENTRY(Q, NW)                                                  \
    {1024U * (Q) * (NW) / 4U,                                                 \
     {&m3_launch_wide<Q, NW, false>, &m3_launch_wide<Q, NW, true>}}
            static const struct {
                uint32_t columns;
                m3_softmax_launcher launch[2];
            } classes[] = {M3_WIDE_ENTRY(8, 2),  M3_WIDE_ENTRY(16, 2),
                           M3_WIDE_ENTRY(12, 4), M3_WIDE_ENTRY(16, 4),
                           M3_WIDE_ENTRY(10, 8), M3_WIDE_ENTRY(12, 8),
                           M3_WIDE_ENTRY(16, 8)};
#undef M3_WIDE_ENTRY
            uint32_t which = 0U;

            while (classes[which].columns < width) {
                ++which;
            }
            const uint64_t cap =
                device->softmax_wide_grid != 0U &&
                        device->softmax_wide_grid < kMaxGrid
                    ? device->softmax_wide_grid
                    : kMaxGrid;
            const dim3 grid((uint32_t)(rows < cap ? rows : cap));
            const m3_softmax_launcher launcher = classes[which].launch[f32];

            return m3_hip_launch(
                device, "m3_softmax_rows_wide",
                [&](hipEvent_t start, hipEvent_t stop) {
                    launcher(grid, device->stream, start, stop, args);
                },
                message, capacity);
        }
        /* Rows wider than the register variants: whole rows in LDS when
         * they fit the dynamic LDS a launch gets without opting in. */
        uint32_t pitch_bytes = ((uint32_t)width + kPad) * 4U;
        uint32_t budget = device->lds_per_block > kStaticLds
                              ? device->lds_per_block - kStaticLds
                              : 0U;

        budget = budget > kTiledLdsCap ? kTiledLdsCap : budget;
        uint32_t tile_rows = width <= kMaxWidth ? budget / pitch_bytes : 0U;

        tile_rows = tile_rows > kMaxTileRows ? kMaxTileRows : tile_rows;
        if (vec && uniform_rows && tile_rows != 0U) {
            args.tile_rows = tile_rows;
            uint64_t tiles = (rows + tile_rows - 1U) / tile_rows;
            uint32_t blocks =
                (uint32_t)(tiles < (uint64_t)device->compute_units * 8U
                               ? tiles
                               : (uint64_t)device->compute_units * 8U);
            size_t lds_bytes = (size_t)tile_rows * pitch_bytes;

            return m3_hip_launch(
                device, "m3_softmax_rows_lds",
                [&](hipEvent_t start, hipEvent_t stop) {
                    if (f32) {
                        hipExtLaunchKernelGGL((m3_softmax_tiled_kernel<true>),
                                              dim3(blocks), dim3(kThreads),
                                              lds_bytes, device->stream, start,
                                              stop, 0U, args);
                    } else {
                        hipExtLaunchKernelGGL((m3_softmax_tiled_kernel<false>),
                                              dim3(blocks), dim3(kThreads),
                                              lds_bytes, device->stream, start,
                                              stop, 0U, args);
                    }
                },
                message, capacity);
        }
        /* Any other row: streamed through three passes, a workgroup per
         * kStreamRows rows. */
        uint64_t tasks = (rows + kStreamRows - 1U) / kStreamRows;
        dim3 grid((uint32_t)(tasks < kMaxGrid ? tasks : kMaxGrid));
        m3_softmax_launcher launcher = !vec ? &m3_launch_stream<false, false>
                                       : f32 ? &m3_launch_stream<true, true>
                                             : &m3_launch_stream<false, true>;

        return m3_hip_launch(
            device, "m3_softmax_rows_streamed",
            [&](hipEvent_t start, hipEvent_t stop) {
                launcher(grid, device->stream, start, stop, args);
            },
            message, capacity);
    }

    m3_softmax_general_args general;

    std::memset(&general, 0, sizeof(general));
    general.list_gate = device->gate;
    general.input = in;
    general.output = out;
    general.rows = rows;
    general.width = (uint32_t)width;
    general.in_dtype = input->dtype;
    general.out_dtype = output->dtype;
    general.column_stride = (int64_t)input->byte_strides[input->rank - 1U];
    general.outer_rank = plan.rank;
    for (uint32_t axis = 0U; axis < plan.rank; ++axis) {
        general.outer_shape[axis] = plan.shape[axis];
        general.outer_strides[axis] = plan.strides[0][axis];
    }
    uint32_t blocks = m3_grid_blocks(device, rows, 64U, 16U);

    return m3_hip_launch(
        device, "m3_softmax_rows_strided",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_softmax_general_kernel, dim3(blocks),
                                  dim3(64), 0, device->stream, start, stop, 0U,
                                  general);
        },
        message, capacity);
}
