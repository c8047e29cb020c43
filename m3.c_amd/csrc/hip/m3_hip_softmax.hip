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
 *     the 64 lanes of a wavefront;
 *   - e_j uses m3_expf (the libm algorithm restated bit for bit);
 *   - the sum keeps the reference's left-to-right F32 order: one lane per
 *     row walks the row's e_j in LDS;
 *   - p_j is the IEEE F32 quotient e_j / sum, formed as
 *     RN_f32(e_j * RN_f64(1/sum)) where that is exact (m3_softmax_scale4).
 *
 * Kernels, chosen by layout and width (rows contiguous along the last axis
 * with a uniform row stride and width a multiple of 4 use the first two):
 *   - width <= 2048: wave-independent rows (m3_softmax_rows_kernel). A wave
 *     holds R rows in VGPRs, reduces max and k with shuffles, forms e_j in
 *     place and streams 256-column chunks through a wave-private LDS tile
 *     where one lane per row continues the in-order sum; no workgroup
 *     barrier separates the phases, so waves overlap memory and arithmetic.
 *   - width <= 8192: a 256-thread workgroup owns a tile of rows; each wave
 *     owns rows w, w+4, ... of the tile; phase 1 loads a row with 16-byte
 *     accesses (8-byte for 16-bit dtypes), reduces max and k, and writes
 *     e_j to LDS; phase 2 has one lane per row sum its row in order from
 *     LDS and form 1/sum in double; phase 3 reads e_j back, scales, rounds
 *     to the output dtype and stores coalesced. LDS rows are padded by 4
 *     floats so the per-row walks of phase 2 hit distinct banks.
 *   - any other layout: one thread per row through the three passes.
 */
#include "m3_hip_internal.h"
#include "m3_libm.h"

#include <cstring>

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
constexpr uint32_t kSumLanes = 16U;       /* lanes that run the in-order sums */

/* Four F32 -inf: what a load past the end of a row reads instead. Never
 * written; not const, so that it is in the global address space like the
 * rows and a select between the two stays a global load. */
__device__ float4 m3_minus_inf4 = {-INFINITY, -INFINITY, -INFINITY,
                                   -INFINITY};

struct m3_softmax_args {
    const uint8_t *input;
    uint8_t *output;
    uint64_t rows;
    uint64_t row_stride; /* input bytes between rows */
    uint32_t width;
    uint32_t in_dtype;
    uint32_t out_dtype;
    uint32_t tile_rows;
};

__device__ __forceinline__ float m3_wave_max(float v)
{
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) {
        v = fmaxf(v, __shfl_xor(v, mask, 64));
    }
    return v;
}

__device__ __forceinline__ uint32_t m3_wave_sum(uint32_t v)
{
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) {
        v += __shfl_xor(v, mask, 64);
    }
    return v;
}

__device__ __forceinline__ uint32_t m3_wave_max_u32(uint32_t v)
{
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) {
        v = max(v, (uint32_t)__shfl_xor((int)v, mask, 64));
    }
    return v;
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

/* Four consecutive row elements starting at column c, as F32. */
template <bool F32IO>
__device__ __forceinline__ float4 m3_softmax_load4(const uint8_t *row,
                                                   uint64_t c, uint32_t dtype)
{
    if (F32IO || dtype == M3N_F32) {
        return *(const float4 *)(row + c * 4U);
    }
    uint2 h = *(const uint2 *)(row + c * 2U);

    return make_float4(
        m3_bits_f32(m3_load_as_f32_bits(h.x & 0xffffU, dtype)),
        m3_bits_f32(m3_load_as_f32_bits(h.x >> 16U, dtype)),
        m3_bits_f32(m3_load_as_f32_bits(h.y & 0xffffU, dtype)),
        m3_bits_f32(m3_load_as_f32_bits(h.y >> 16U, dtype)));
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

/* Wave-independent rows (width <= 256 * VPL, a multiple of 4). Each wave
 * takes R consecutive rows at a time and keeps them in VGPRs (VPL float4
 * per lane per row): it reduces max with shuffles, forms e_j in place,
 * then walks the row in 256-column chunks, writing each chunk of its R
 * rows to a wave-private LDS tile where lanes 0..R-1 continue their row's
 * left-to-right sum. The sum stops after the row's last nonzero e_j: the
 * trailing terms are +0 and leave a nonnegative F32 sum unchanged, so the
 * result is identical while masked (causal) rows cost half. p_j is formed
 * from the registers and streamed out with nontemporal stores. No
 * workgroup barrier is needed after the table copy, so waves of one CU
 * overlap their loads, arithmetic and sums freely. */
template <int VPL, int R, int DEPTH, bool F32IO>
__device__ __forceinline__ void m3_softmax_rows(const m3_softmax_args &a)
{
    static_assert(R <= (int)kSumLanes, "one summing lane per row");
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
        const uint8_t *rows = a.input + first_row * a.row_stride;
        float4 v[R][VPL];
        float maximum[R];
        uint32_t length[R]; /* elements up to the last nonzero e_j */

        /* Every load is issued and none is under a branch, so the wave
         * waits for each row's data alone: row 0 is reduced and
         * exponentiated while the later rows are still arriving. A row past
         * the end of the tensor (the last task) reads the task's first row
         * and is never stored. A column past the width reads four F32 -inf
         * from m3_minus_inf4 (16-bit inputs: column 0, replaced by -inf).
         * A variant serves widths above 256 * VPL / 2, so its chunks
         * j < VPL / 2 are always inside the row. */
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const uint8_t *row =
                rows + (uint64_t)((uint32_t)k < present ? (uint32_t)k : 0U) *
                           a.row_stride;

#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                const uint32_t c = lane * 4U + kChunk * j;
                const bool inside = (VPL > 1 && j < VPL / 2) || c < width;

                if (F32IO || in_dtype == M3N_F32) {
                    const float4 *source =
                        inside ? (const float4 *)(row + (uint64_t)c * 4U)
                               : &m3_minus_inf4;

                    v[k][j] = *source;
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
            uint32_t last = 0U; /* 1 + index of the last nonzero float4 */

#pragma unroll
            for (int j = 0; j < VPL; ++j) {
                m = fmaxf(m, fmaxf(fmaxf(v[k][j].x, v[k][j].y),
                                   fmaxf(v[k][j].z, v[k][j].w)));
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

                    uint32_t nonzero =
                        m3_f32_bits(v[k][j].x) | m3_f32_bits(v[k][j].y) |
                        m3_f32_bits(v[k][j].z) | m3_f32_bits(v[k][j].w);

                    last = nonzero != 0U ? lane + 64U * j + 1U : last;
                }
            }
            length[k] = m3_uniform_u32(m3_wave_max_u32(last)) * 4U;
        }
        uint32_t wave_length = 0U;

#pragma unroll
        for (int k = 0; k < R; ++k) {
            wave_length = max(wave_length, length[k]);
        }
        /* The sums run on the 16 lanes of the wave's first lane group,
         * lane l summing row l % R: a dependent add issued with a full
         * 16-lane group measured about twice as fast on gfx950 as one
         * issued for fewer lanes. Every lane sums up to the longest row's
         * length; terms past a row's own length are +0 and leave its sum
         * unchanged. Lanes 0..R-1 hold the R row sums. */
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
            if (lane < kSumLanes) {
                sum = m3_chunk_sum<DEPTH>(sum, line,
                                          min(wave_length - base, kChunk));
            }
            m3_wave_sync();
        }
        const double inverse_of_lane = 1.0 / (double)sum;

        uint8_t *out = a.output + first_row * out_pitch +
                       (uint64_t)lane * 4U * out_size;

#pragma unroll
        for (int k = 0; k < R; ++k) {
            const float m = maximum[k];

            if ((uint32_t)k >= present) {
                continue;
            }
            if (m != INFINITY && m != -INFINITY) {
                const double inverse = m3_lane_f64(inverse_of_lane, k);

#pragma unroll
                for (int j = 0; j < VPL; ++j) {
                    const float4 e = v[k][j];
                    float4 p;

                    if (lane * 4U + kChunk * j >= width) {
                        continue;
                    }
                    p = m3_softmax_scale4(e, inverse);
                    m3_softmax_store4<F32IO>(out, (uint64_t)kChunk * j,
                                             out_dtype, p);
                }
            } else if (m == -INFINITY) {
                /* every entry is -inf: zeros */
#pragma unroll
                for (int j = 0; j < VPL; ++j) {
                    if (lane * 4U + kChunk * j < width) {
                        m3_softmax_store4<F32IO>(
                            out, (uint64_t)kChunk * j, out_dtype,
                            make_float4(0.0F, 0.0F, 0.0F, 0.0F));
                    }
                }
            } else {
                /* maximum +inf: 1/k on the k +inf entries, 0 elsewhere */
                uint32_t count = 0U;

#pragma unroll
                for (int j = 0; j < VPL; ++j) {
                    count += (v[k][j].x == INFINITY) +
                             (v[k][j].y == INFINITY) +
                             (v[k][j].z == INFINITY) +
                             (v[k][j].w == INFINITY);
                }
                const float one_over_count =
                    1.0F / (float)m3_wave_sum(count);

#pragma unroll
                for (int j = 0; j < VPL; ++j) {
                    const float4 e = v[k][j];
                    float4 p;

                    if (lane * 4U + kChunk * j >= width) {
                        continue;
                    }
                    p.x = e.x == INFINITY ? one_over_count : 0.0F;
                    p.y = e.y == INFINITY ? one_over_count : 0.0F;
                    p.z = e.z == INFINITY ? one_over_count : 0.0F;
                    p.w = e.w == INFINITY ? one_over_count : 0.0F;
                    m3_softmax_store4<F32IO>(out, (uint64_t)kChunk * j,
                                             out_dtype, p);
                }
            }
            out += out_pitch;
        }
    }
}

template <int VPL, int R, int DEPTH, bool F32IO>
__global__ __launch_bounds__(256) void m3_softmax_rows_kernel(
    m3_softmax_args a)
{
    m3_softmax_rows<VPL, R, DEPTH, F32IO>(a);
}

typedef void (*m3_softmax_launcher)(dim3, hipStream_t, hipEvent_t,
                                    hipEvent_t, m3_softmax_args);

template <int VPL, int R, int DEPTH, bool F32IO>
void m3_launch_rows(dim3 grid, hipStream_t stream, hipEvent_t start,
                    hipEvent_t stop, m3_softmax_args args)
{
    hipExtLaunchKernelGGL((m3_softmax_rows_kernel<VPL, R, DEPTH, F32IO>),
                          grid, dim3(kThreads), 0, stream, start, stop, 0U,
                          args);
}

struct m3_rows_variant {
    uint32_t vectors_per_lane;
    uint32_t rows_per_wave;
    m3_softmax_launcher f32;
    m3_softmax_launcher other;
};

/* Wave-independent variants; the first whose width class fits is used.
 * Rows per wave and sum prefetch depth are chosen for four waves per SIMD
 * (88, 98 and 120 VGPRs for the F32 instances up to width 1024); the
 * width-2048 instance and the 16-bit-IO instances from width 1024 take
 * 133-157 VGPRs, three waves per SIMD. */
const m3_rows_variant m3_rows_variants[] = {
    {1U, 8U, &m3_launch_rows<1, 8, 8, true>,
     &m3_launch_rows<1, 8, 8, false>},
    {2U, 4U, &m3_launch_rows<2, 4, 8, true>,
     &m3_launch_rows<2, 4, 8, false>},
    {4U, 4U, &m3_launch_rows<4, 4, 4, true>,
     &m3_launch_rows<4, 4, 4, false>},
    {8U, 2U, &m3_launch_rows<8, 2, 4, true>,
     &m3_launch_rows<8, 2, 4, false>},
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

    bool uniform_rows = plan.rank == 1U;
    uint64_t row_stride = uniform_rows ? (uint64_t)plan.strides[0][0] : 0U;
    bool columns_contiguous =
        width == 1U ||
        input->byte_strides[input->rank - 1U] == (uint64_t)in_size;

    if (rows == 1U) {
        uniform_rows = true;
        row_stride = 0U;
    }
    if (uniform_rows && columns_contiguous && width % 4U == 0U &&
        width <= kMaxWidth && row_stride % (4U * in_size) == 0U &&
        ((uintptr_t)in % (4U * in_size)) == 0U &&
        ((uintptr_t)out % (4U * out_size)) == 0U &&
        plan.strides[0][0] >= 0) {
        m3_softmax_args args;
        uint32_t pitch_bytes = ((uint32_t)width + kPad) * 4U;
        uint32_t budget = device->lds_per_block > kStaticLds
                              ? device->lds_per_block - kStaticLds
                              : 0U;
        bool f32 = input->dtype == M3_HIP_F32 && output->dtype == M3_HIP_F32;

        std::memset(&args, 0, sizeof(args));
        args.input = in;
        args.output = out;
        args.rows = rows;
        args.row_stride = row_stride;
        args.width = (uint32_t)width;
        args.in_dtype = input->dtype;
        args.out_dtype = output->dtype;
        for (const m3_rows_variant &variant : m3_rows_variants) {
            if (width > kChunk * variant.vectors_per_lane) {
                continue;
            }
            uint64_t tasks =
                (rows + variant.rows_per_wave - 1U) / variant.rows_per_wave;
            uint64_t blocks = (tasks + kWaves - 1U) / kWaves;
            dim3 grid((uint32_t)(blocks < kMaxGrid ? blocks : kMaxGrid));
            m3_softmax_launcher launcher = f32 ? variant.f32 : variant.other;

            return m3_hip_launch(
                device, "m3_softmax_rows",
                [&](hipEvent_t start, hipEvent_t stop) {
                    launcher(grid, device->stream, start, stop, args);
                },
                message, capacity);
        }
        /* Rows wider than the register variants: whole rows in LDS,
         * within the dynamic LDS a launch gets without opting in. */
        budget = budget > kTiledLdsCap ? kTiledLdsCap : budget;
        uint32_t tile_rows = budget / pitch_bytes;

        tile_rows = tile_rows > kMaxTileRows ? kMaxTileRows : tile_rows;
        if (tile_rows != 0U) {
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
    }

    m3_softmax_general_args general;

    std::memset(&general, 0, sizeof(general));
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
    if (width > 0xffffffffULL) {
        return m3_hip_fail(message, capacity, M3_HIP_UNSUPPORTED,
                           "softmax rows longer than 2^32 are unsupported");
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
