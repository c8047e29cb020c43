/*
 * m3_hip_program.hip - elementwise programs: a run of F32 ADD/SUB/MUL/DIV
 * commands fused by the session compiler, executed per element with the
 * intermediate values in registers.
 *
 * Per element every operation is the reference's (src/m3_op_execute_basic.c:
 * 61-77): load each operand as F32, one F32 operation rounded to nearest
 * even, store F32; NaN results carry the bits m3_binary_nan_fix gives. The
 * program replaces the memory round trip of every intermediate value that
 * only the fused run reads; the values it does store and the order of the
 * operations are those of the unfused commands, so the results are
 * identical bit for bit.
 *
 * Execution. A lane takes four consecutive elements (one 16-byte group) and
 * walks the instruction words, which are the same for every lane: they are
 * read with scalar loads and dispatched with wave-uniform branches, so the
 * interpreter costs scalar instructions, not divergence. Registers are
 * fixed VGPRs (R0..R3 values, F0..F3 fetched operands); a FETCH issues up to
 * four 16-byte loads back to back, which keeps several HBM requests in
 * flight per lane between dependent operations. The word layout is defined
 * with m3_hip_launch_program in m3_hip.h.
 */
#include "m3_hip_internal.h"
#include "m3_numeric.h"

#include <cstring>

namespace {

constexpr uint32_t kThreads = 256U;
constexpr uint32_t kBlocksPerCu = 64U;
constexpr uint32_t kScalarSource = 8U;

__device__ __forceinline__ const uint8_t *m3_operand_address(
    const uint32_t *operands, uint32_t index)
{
    uint64_t low = operands[2U * index];
    uint64_t high = operands[2U * index + 1U];

    return (const uint8_t *)(((high << 32U) | low) & ~(uint64_t)1U);
}

/* Four elements of an array operand starting at element 4g; the last,
 * partial group reads only the elements that exist. */
__device__ __forceinline__ m3_f32x4 m3_fetch4(const uint8_t *base,
                                             uint64_t g, bool full,
                                             uint64_t count)
{
    const float *p = (const float *)base + 4U * g;

    if (full) {
        return *(const m3_f32x4 *)p;
    }
    m3_f32x4 v = {0.0F, 0.0F, 0.0F, 0.0F};
    uint64_t first = 4U * g;

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

__device__ __forceinline__ void m3_store4(uint8_t *base, uint64_t g,
                                          bool full, uint64_t count,
                                          m3_f32x4 v)
{
    float *p = (float *)base + 4U * g;

    if (full) {
        __builtin_nontemporal_store(v, (m3_f32x4 *)p);
        return;
    }
    uint64_t first = 4U * g;

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

template <uint32_t OP>
__device__ __forceinline__ float m3_apply(float a, float b)
{
    return OP == M3N_ADD ? a + b : OP == M3N_MUL ? a * b
                               : OP == M3N_SUB ? a - b
                                               : a / b;
}

/* One F32 operation on four elements. The NaN rule of m3_binary_f32_bits
 * is applied only when some lane of the wave produced a NaN. */
template <uint32_t OP>
__device__ __forceinline__ m3_f32x4 m3_apply4(m3_f32x4 a, m3_f32x4 b)
{
    m3_f32x4 r;

    r.x = m3_apply<OP>(a.x, b.x);
    r.y = m3_apply<OP>(a.y, b.y);
    r.z = m3_apply<OP>(a.z, b.z);
    r.w = m3_apply<OP>(a.w, b.w);
    const uint64_t nan = __ballot(r.x != r.x) | __ballot(r.y != r.y) |
                         __ballot(r.z != r.z) | __ballot(r.w != r.w);

    if (nan != 0U) {
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

/* Register selection by value on native vectors: the registers stay in
 * VGPRs (a selection of HIP's float4 class, or through a pointer into a
 * register array, would put them in scratch memory). Kinds 0-3 are R0-R3,
 * 4-7 F0-F3. */
__device__ __forceinline__ m3_f32x4 m3_pick(uint32_t kind, m3_f32x4 r0,
                                            m3_f32x4 r1, m3_f32x4 r2,
                                            m3_f32x4 r3, m3_f32x4 f0,
                                            m3_f32x4 f1, m3_f32x4 f2,
                                            m3_f32x4 f3)
{
    if (kind < 4U) {
        return kind == 0U ? r0 : kind == 1U ? r1 : kind == 2U ? r2 : r3;
    }
    return kind == 4U ? f0 : kind == 5U ? f1 : kind == 6U ? f2 : f3;
}

__global__ __launch_bounds__(256) void m3_program_kernel(
    const uint32_t *__restrict__ operands, const uint32_t *__restrict__ code,
    uint32_t code_words, uint64_t count)
{
    const uint64_t groups = (count + 3U) / 4U;
    const uint64_t full_groups = count / 4U;
    const uint64_t step = (uint64_t)gridDim.x * kThreads;

    for (uint64_t g = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
         g < groups; g += step) {
        const bool full = g < full_groups;
        const m3_f32x4 zero = {0.0F, 0.0F, 0.0F, 0.0F};
        m3_f32x4 r0 = zero, r1 = zero, r2 = zero, r3 = zero;
        m3_f32x4 f0 = zero, f1 = zero, f2 = zero, f3 = zero;
        uint32_t pc = 0U;

        while (pc < code_words) {
            const uint32_t w = code[pc];
            const uint32_t opcode = w & 3U;

            if (opcode == M3_HIP_PROGRAM_FETCH) {
                const uint32_t list = code[pc + 1U];
                const uint32_t n = ((w >> 2U) & 3U) + 1U;

                f0 = m3_fetch4(m3_operand_address(operands, list & 0xffU), g,
                               full, count);
                if (n > 1U) {
                    f1 = m3_fetch4(
                        m3_operand_address(operands, (list >> 8U) & 0xffU), g,
                        full, count);
                }
                if (n > 2U) {
                    f2 = m3_fetch4(
                        m3_operand_address(operands, (list >> 16U) & 0xffU),
                        g, full, count);
                }
                if (n > 3U) {
                    f3 = m3_fetch4(m3_operand_address(operands, list >> 24U),
                                   g, full, count);
                }
            } else if (opcode == M3_HIP_PROGRAM_OP) {
                const uint32_t left_kind = (w >> 8U) & 15U;
                const uint32_t right_kind = (w >> 12U) & 15U;
                const float v =
                    left_kind == kScalarSource || right_kind == kScalarSource
                        ? *(const float *)m3_operand_address(
                              operands, (w >> 16U) & 0xffU)
                        : 0.0F;
                const m3_f32x4 scalar = {v, v, v, v};
                const m3_f32x4 left =
                    left_kind == kScalarSource
                        ? scalar
                        : m3_pick(left_kind, r0, r1, r2, r3, f0, f1, f2, f3);
                const m3_f32x4 right =
                    right_kind == kScalarSource
                        ? scalar
                        : m3_pick(right_kind, r0, r1, r2, r3, f0, f1, f2, f3);
                m3_f32x4 r;

                switch ((w >> 2U) & 3U) {
                case M3N_ADD:
                    r = m3_apply4<M3N_ADD>(left, right);
                    break;
                case M3N_MUL:
                    r = m3_apply4<M3N_MUL>(left, right);
                    break;
                case M3N_SUB:
                    r = m3_apply4<M3N_SUB>(left, right);
                    break;
                default:
                    r = m3_apply4<M3N_DIV>(left, right);
                    break;
                }
                const uint32_t dst = (w >> 4U) & 3U;

                r0 = dst == 0U ? r : r0;
                r1 = dst == 1U ? r : r1;
                r2 = dst == 2U ? r : r2;
                r3 = dst == 3U ? r : r3;
            } else {
                const uint32_t src = (w >> 4U) & 3U;

                m3_store4((uint8_t *)m3_operand_address(operands,
                                                        (w >> 8U) & 0xffU),
                          g, full, count,
                          src == 0U   ? r0
                          : src == 1U ? r1
                          : src == 2U ? r2
                                      : r3);
            }
            pc += opcode == M3_HIP_PROGRAM_FETCH ? 2U : 1U;
        }
    }
}

bool m3_operand_is_scalar(const uint32_t *operands, uint32_t index)
{
    return (operands[2U * index] & 1U) != 0U;
}

/* Structural check of the words; 0 when valid, else the word index + 1 of
 * the first offending word (for the message). */
size_t m3_program_check(const uint32_t *words, size_t word_count)
{
    const uint32_t operand_count = words[1];
    const uint32_t code_words = words[2];
    const uint32_t *operands = words + M3_HIP_PROGRAM_HEADER_WORDS;
    const uint32_t *code = operands + 2U * operand_count;
    const size_t code_base = M3_HIP_PROGRAM_HEADER_WORDS + 2U * operand_count;

    if (words[0] != M3_HIP_PROGRAM_MAGIC) {
        return 1U;
    }
    if (operand_count > M3_HIP_PROGRAM_MAX_OPERANDS ||
        code_words > M3_HIP_PROGRAM_MAX_WORDS) {
        return 2U;
    }
    if (word_count != code_base + code_words) {
        return 3U;
    }
    if (words[5] != 0U || words[6] != 0U || words[7] != 0U) {
        return 6U;
    }
    for (uint32_t p = 0U; p < operand_count; ++p) {
        const uint32_t low = operands[2U * p];
        const uint32_t high = operands[2U * p + 1U];
        const bool scalar = (low & 1U) != 0U;

        if (((low & ~1U) == 0U && high == 0U) ||
            (scalar ? (low & 2U) != 0U : (low & 15U) != 0U)) {
            return M3_HIP_PROGRAM_HEADER_WORDS + 2U * p + 1U;
        }
    }
    for (uint32_t pc = 0U; pc < code_words;) {
        const uint32_t w = code[pc];
        const size_t at = code_base + pc + 1U;

        switch (w & 3U) {
        case M3_HIP_PROGRAM_FETCH: {
            const uint32_t n = ((w >> 2U) & 3U) + 1U;

            if ((w >> 4U) != 0U || pc + 1U >= code_words) {
                return at;
            }
            for (uint32_t k = 0U; k < n; ++k) {
                const uint32_t index = (code[pc + 1U] >> (8U * k)) & 0xffU;

                if (index >= operand_count ||
                    m3_operand_is_scalar(operands, index)) {
                    return at + 1U;
                }
            }
            if (n < 4U && (code[pc + 1U] >> (8U * n)) != 0U) {
                return at + 1U;
            }
            pc += 2U;
            break;
        }
        case M3_HIP_PROGRAM_OP: {
            const uint32_t left = (w >> 8U) & 15U;
            const uint32_t right = (w >> 12U) & 15U;
            const uint32_t scalar = (w >> 16U) & 0xffU;
            const bool uses_scalar =
                left == kScalarSource || right == kScalarSource;

            if ((w & 0xc0U) != 0U || (w >> 24U) != 0U ||
                left > kScalarSource || right > kScalarSource ||
                (uses_scalar &&
                 (scalar >= operand_count ||
                  !m3_operand_is_scalar(operands, scalar))) ||
                (!uses_scalar && scalar != 0U)) {
                return at;
            }
            pc += 1U;
            break;
        }
        case M3_HIP_PROGRAM_STORE: {
            const uint32_t index = (w >> 8U) & 0xffU;

            if ((w & 0xcU) != 0U || (w & 0xc0U) != 0U || (w >> 16U) != 0U ||
                index >= operand_count ||
                m3_operand_is_scalar(operands, index)) {
                return at;
            }
            pc += 1U;
            break;
        }
        default:
            return at;
        }
    }
    return 0U;
}

} // namespace

extern "C" int m3_hip_launch_program(m3_hip_device *device,
                                     const uint32_t *words,
                                     const void *device_words,
                                     size_t word_count, char *message,
                                     size_t capacity)
{
    if (device == nullptr || words == nullptr || device_words == nullptr ||
        word_count < M3_HIP_PROGRAM_HEADER_WORDS ||
        ((uintptr_t)device_words & 3U) != 0U) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "elementwise program arguments are malformed");
    }
    size_t offending = m3_program_check(words, word_count);

    if (offending != 0U) {
        return m3_hip_fail(message, capacity, M3_HIP_INVALID,
                           "elementwise program word %zu is invalid",
                           offending - 1U);
    }
    const uint64_t count = (uint64_t)words[3] | ((uint64_t)words[4] << 32U);

    if (count == 0U || words[2] == 0U) {
        return M3_HIP_OK;
    }
    const uint32_t *operands =
        (const uint32_t *)device_words + M3_HIP_PROGRAM_HEADER_WORDS;
    const uint32_t *code = operands + 2U * words[1];
    const uint32_t code_words = words[2];
    uint32_t blocks =
        m3_grid_blocks(device, (count + 3U) / 4U, kThreads, kBlocksPerCu);

    return m3_hip_launch(
        device, "m3_program",
        [&](hipEvent_t start, hipEvent_t stop) {
            hipExtLaunchKernelGGL(m3_program_kernel, dim3(blocks),
                                  dim3(kThreads), 0, device->stream, start,
                                  stop, 0U, operands, code, code_words,
                                  count);
        },
        message, capacity);
}
