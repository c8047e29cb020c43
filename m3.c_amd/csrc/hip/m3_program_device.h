/*
 * m3_program_device.h - device helpers of elementwise programs, shared by
 * the interpreter kernel (m3_hip_program.hip) and the kernels generated
 * from program words at run time (compiled with hipRTC, which receives
 * this header and m3_numeric.h as in-memory headers).
 *
 * Element e of an array operand is the F32 at its address + 4e; a lane
 * handles the four elements 4g..4g+3. The last, partial group reads and
 * writes only the elements below `count`. Every operation is one F32
 * operation rounded to nearest even with the NaN results of
 * m3_binary_f32_bits.
 */
#ifndef M3_PROGRAM_DEVICE_H
#define M3_PROGRAM_DEVICE_H

#include "m3_numeric.h"

typedef float m3_program_f32x4 __attribute__((ext_vector_type(4)));
/* Operand memory is global memory: accesses through these types are
 * global (not flat) loads and stores, so a wait for scalar loads (operand
 * addresses) does not also wait for the lane's vector loads. */
typedef float __attribute__((address_space(1))) m3_program_global_f32;
typedef m3_program_f32x4
    __attribute__((address_space(1))) m3_program_global_f32x4;

__device__ __forceinline__ const unsigned char *m3_program_address(
    const unsigned int *operands, unsigned int index)
{
    unsigned long long low = operands[2U * index];
    unsigned long long high = operands[2U * index + 1U];

    return (const unsigned char *)(((high << 32U) | low) & ~1ULL);
}

/* A scalar operand: one F32 that no lane writes during the launch, read
 * through the constant address space so that it is a scalar load and does
 * not wait for the lane's outstanding vector loads. */
__device__ __forceinline__ float m3_program_scalar(
    const unsigned int *operands, unsigned int index)
{
    typedef const float __attribute__((address_space(4))) *constant_f32;

    return *(constant_f32)(unsigned long long)m3_program_address(operands,
                                                                  index);
}

__device__ __forceinline__ m3_program_f32x4 m3_program_splat(float v)
{
    m3_program_f32x4 r = {v, v, v, v};

    return r;
}

template <bool FULL>
__device__ __forceinline__ m3_program_f32x4
m3_program_load(const unsigned int *operands, unsigned int index,
                unsigned long long g, unsigned long long count)
{
    const m3_program_global_f32 *p =
        (const m3_program_global_f32 *)(unsigned long long)
            m3_program_address(operands, index) +
        4ULL * g;

    if (FULL) {
        return *(const m3_program_global_f32x4 *)p;
    }
    m3_program_f32x4 v = {0.0F, 0.0F, 0.0F, 0.0F};
    const unsigned long long first = 4ULL * g;

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

/* Stores are nontemporal for whole groups: program outputs are written
 * once and not read back by the launch. */
template <bool FULL>
__device__ __forceinline__ void m3_program_store(
    const unsigned int *operands, unsigned int index, unsigned long long g,
    unsigned long long count, m3_program_f32x4 v)
{
    m3_program_global_f32 *p =
        (m3_program_global_f32 *)(unsigned long long)m3_program_address(
            operands, index) +
        4ULL * g;

    if (FULL) {
        __builtin_nontemporal_store(v, (m3_program_global_f32x4 *)p);
        return;
    }
    const unsigned long long first = 4ULL * g;

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
