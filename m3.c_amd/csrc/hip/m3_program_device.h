/*
 * m3_program_device.h - device helpers of elementwise programs, shared by
 * the interpreter kernel (m3_hip_program.hip) and the kernels generated
 * from program words at run time (compiled with hipRTC, which receives
 * this header and m3_numeric.h as in-memory headers).
 *
 * Element e of an array operand of dtype D (F32, F16 or BF16, bits 30-31
 * of its high address word) is at its address + e * size(D), or at
 * index e mod M for a periodic operand of period M (a multiple of 4, so
 * the four elements of a group are consecutive there too); a lane
 * handles the four elements 4g..4g+3 and holds them as F32. The last,
 * partial group reads and writes only the elements below `count`. Loads
 * convert to F32 and stores from F32 with the converters of CAST; an
 * operation is one F32 operation rounded to nearest even with the NaN
 * results of m3_binary_f32_bits, then rounded through its output dtype
 * when that is F16 or BF16 (the value a store and a load back give).
 */
#ifndef M3_PROGRAM_DEVICE_H
#define M3_PROGRAM_DEVICE_H

#include "m3_numeric.h"

typedef float m3_program_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int m3_program_u32x2 __attribute__((ext_vector_type(2)));
/* Operand memory is global memory: accesses through these types are
 * global (not flat) loads and stores, so a wait for scalar loads (operand
 * addresses) does not also wait for the lane's vector loads. */
typedef float __attribute__((address_space(1))) m3_program_global_f32;
typedef m3_program_f32x4
    __attribute__((address_space(1))) m3_program_global_f32x4;
typedef unsigned short __attribute__((address_space(1))) m3_program_global_u16;
typedef m3_program_u32x2
    __attribute__((address_space(1))) m3_program_global_u32x2;

__device__ __forceinline__ const unsigned char *m3_program_address(
    const unsigned int *operands, unsigned int index)
{
    unsigned long long low = operands[2U * index];
    unsigned long long high = operands[2U * index + 1U] & 0x3fffffffU;

    return (const unsigned char *)(((high << 32U) | low) & ~1ULL);
}

/* Element type of operand `index` (M3N_F32, M3N_F16 or M3N_BF16). */
__device__ __forceinline__ unsigned int m3_program_dtype(
    const unsigned int *operands, unsigned int index)
{
    return operands[2U * index + 1U] >> 30U;
}

/* A scalar operand of dtype D: one element that no lane writes during the
 * launch, read through the constant address space so that it is a scalar
 * load and does not wait for the lane's outstanding vector loads. */
template <unsigned int D>
__device__ __forceinline__ float m3_program_scalar(
    const unsigned int *operands, unsigned int index)
{
    typedef const float __attribute__((address_space(4))) *constant_f32;
    typedef const unsigned short __attribute__((address_space(4))) *
        constant_u16;
    const unsigned long long address =
        (unsigned long long)m3_program_address(operands, index);

    if (D == M3N_F32) {
        return *(constant_f32)address;
    }
    return m3_bits_f32(
        m3_load_as_f32_bits((unsigned int)*(constant_u16)address, D));
}

/* True when the command list's gate is closed: a data check earlier in
 * the list failed and the program must not run (word 0: no gate). */
__device__ __forceinline__ bool m3_program_gate_closed(
    const unsigned int *word, unsigned int epoch)
{
    return word != 0 &&
           __hip_atomic_load(word, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT) == epoch;
}

__device__ __forceinline__ m3_program_f32x4 m3_program_splat(float v)
{
    m3_program_f32x4 r = {v, v, v, v};

    return r;
}

/* Loads elements 4g..4g+3 (those below `count`) of array operand `index`;
 * `period` is its period, or 0 when it is not periodic. */
template <bool FULL, unsigned int D>
__device__ __forceinline__ m3_program_f32x4
m3_program_load(const unsigned int *operands, unsigned int index,
                unsigned long long g, unsigned long long count,
                unsigned long long period)
{
    const unsigned long long first = 4ULL * g;
    const unsigned long long at = period != 0ULL ? first % period : first;
    m3_program_f32x4 v = {0.0F, 0.0F, 0.0F, 0.0F};

    if (D == M3N_F32) {
        const m3_program_global_f32 *p =
            (const m3_program_global_f32 *)(unsigned long long)
                m3_program_address(operands, index) +
            at;

        if (FULL) {
            /* an array operand is read once per launch; a broadcast one
             * (period) is read again and stays in the caches */
            if (period == 0ULL) {
                return __builtin_nontemporal_load(
                    (const m3_program_global_f32x4 *)p);
            }
            return *(const m3_program_global_f32x4 *)p;
        }
        v.x = p[0];
        if (first + 1U < count) {
            v.y = p[1];
        }
        if (first + 2U < count) {
            v.z = p[2];
        }
        if (first + 3U < count) {
            v.w = p[3];
        }
        return v;
    }
    const m3_program_global_u16 *p =
        (const m3_program_global_u16 *)(unsigned long long)
            m3_program_address(operands, index) +
        at;
    unsigned int h[4] = {0U, 0U, 0U, 0U};

    if (FULL) {
        const m3_program_u32x2 w =
            period == 0ULL
                ? __builtin_nontemporal_load((const m3_program_global_u32x2 *)p)
                : *(const m3_program_global_u32x2 *)p;

        h[0] = w.x & 0xffffU;
        h[1] = w.x >> 16U;
        h[2] = w.y & 0xffffU;
        h[3] = w.y >> 16U;
    } else {
        h[0] = p[0];
        if (first + 1U < count) {
            h[1] = p[1];
        }
        if (first + 2U < count) {
            h[2] = p[2];
        }
        if (first + 3U < count) {
            h[3] = p[3];
        }
    }
    v.x = m3_bits_f32(m3_load_as_f32_bits(h[0], D));
    v.y = m3_bits_f32(m3_load_as_f32_bits(h[1], D));
    v.z = m3_bits_f32(m3_load_as_f32_bits(h[2], D));
    v.w = m3_bits_f32(m3_load_as_f32_bits(h[3], D));
    return v;
}

/* 1 when a value that the store of group g writes is NaN: all four of a
 * whole group, the first count - 4g of the last, partial one (whose other
 * lanes are not stored). */
template <bool FULL>
__device__ __forceinline__ unsigned int m3_program_nan4(
    m3_program_f32x4 v, unsigned long long g, unsigned long long count)
{
    const unsigned long long first = 4ULL * g;

    return (v.x != v.x) | ((FULL || first + 1U < count) && v.y != v.y) |
           ((FULL || first + 2U < count) && v.z != v.z) |
           ((FULL || first + 3U < count) && v.w != v.w);
}

/* Stores are nontemporal for whole groups: program outputs are written
 * once and not read back by the launch. */
template <bool FULL, unsigned int D>
__device__ __forceinline__ void m3_program_store(
    const unsigned int *operands, unsigned int index, unsigned long long g,
    unsigned long long count, m3_program_f32x4 v)
{
    const unsigned long long first = 4ULL * g;

    if (D == M3N_F32) {
        m3_program_global_f32 *p =
            (m3_program_global_f32 *)(unsigned long long)m3_program_address(
                operands, index) +
            first;

        if (FULL) {
            __builtin_nontemporal_store(v, (m3_program_global_f32x4 *)p);
            return;
        }
        p[0] = v.x;
        if (first + 1U < count) {
            p[1] = v.y;
        }
        if (first + 2U < count) {
            p[2] = v.z;
        }
        if (first + 3U < count) {
            p[3] = v.w;
        }
        return;
    }
    m3_program_global_u16 *p =
        (m3_program_global_u16 *)(unsigned long long)m3_program_address(
            operands, index) +
        first;
    const unsigned int h[4] = {m3_store_from_f32_bits(m3_f32_bits(v.x), D),
                               m3_store_from_f32_bits(m3_f32_bits(v.y), D),
                               m3_store_from_f32_bits(m3_f32_bits(v.z), D),
                               m3_store_from_f32_bits(m3_f32_bits(v.w), D)};

    if (FULL) {
        const m3_program_u32x2 w = {h[0] | (h[1] << 16U),
                                    h[2] | (h[3] << 16U)};

        __builtin_nontemporal_store(w, (m3_program_global_u32x2 *)p);
        return;
    }
    p[0] = (unsigned short)h[0];
    if (first + 1U < count) {
        p[1] = (unsigned short)h[1];
    }
    if (first + 2U < count) {
        p[2] = (unsigned short)h[2];
    }
    if (first + 3U < count) {
        p[3] = (unsigned short)h[3];
    }
}

/* Four values rounded through dtype D (identity for F32). */
template <unsigned int D>
__device__ __forceinline__ m3_program_f32x4
m3_program_round4(m3_program_f32x4 v)
{
    if (D == M3N_F32) {
        return v;
    }
    m3_program_f32x4 r;

    r.x = m3_bits_f32(m3_round_through_bits(m3_f32_bits(v.x), D));
    r.y = m3_bits_f32(m3_round_through_bits(m3_f32_bits(v.y), D));
    r.z = m3_bits_f32(m3_round_through_bits(m3_f32_bits(v.z), D));
    r.w = m3_bits_f32(m3_round_through_bits(m3_f32_bits(v.w), D));
    return r;
}

template <unsigned int OP>
__device__ __forceinline__ float m3_program_apply(float a, float b)
{
    return OP == M3N_ADD ? a + b : OP == M3N_MUL ? a * b
                               : OP == M3N_SUB ? a - b
                                               : a / b;
}

/* One F32 operation on four elements. The NaN rule of m3_binary_f32_bits
 * is applied only when some lane of the wave produced a NaN. */
template <unsigned int OP>
__device__ __forceinline__ m3_program_f32x4
m3_program_apply4(m3_program_f32x4 a, m3_program_f32x4 b)
{
    m3_program_f32x4 r;

    r.x = m3_program_apply<OP>(a.x, b.x);
    r.y = m3_program_apply<OP>(a.y, b.y);
    r.z = m3_program_apply<OP>(a.z, b.z);
    r.w = m3_program_apply<OP>(a.w, b.w);
    if ((__ballot(r.x != r.x) | __ballot(r.y != r.y) |
         __ballot(r.z != r.z) | __ballot(r.w != r.w)) != 0U) {
        const int commutative = OP == M3N_ADD || OP == M3N_MUL;

        r.x = m3_bits_f32(m3_binary_nan_fix(m3_f32_bits(r.x),
                                            m3_f32_bits(a.x),
                                            m3_f32_bits(b.x), commutative));
        r.y = m3_bits_f32(m3_binary_nan_fix(m3_f32_bits(r.y),
                                            m3_f32_bits(a.y),
                                            m3_f32_bits(b.y), commutative));
        r.z = m3_bits_f32(m3_binary_nan_fix(m3_f32_bits(r.z),
                                            m3_f32_bits(a.z),
                                            m3_f32_bits(b.z), commutative));
        r.w = m3_bits_f32(m3_binary_nan_fix(m3_f32_bits(r.w),
                                            m3_f32_bits(a.w),
                                            m3_f32_bits(b.w), commutative));
    }
    return r;
}

#endif
