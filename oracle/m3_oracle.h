/*
 * m3_oracle.h - CPU restatement of the reference's host tensor ops.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this code, and only to check or
 * time results.
 * The product (libm3.so / libm3_hip.so) never links or calls it.
 *
 * Every function restates the reference CPU provider of
 * taconotsandwich/m3.c (its host backend, single-threaded by design) and
 * cites the lines it follows. Buffers are plain host memory described by
 * oracle_view; outputs must be contiguous, as in the reference.
 *
 * Pinning (what checks each function, besides the reference's golden
 * vectors):
 *   conversions      exhaustive vs the compiled reference (oracle/_ref):
 *                    the full F32->F16/BF16 tables (all 2^32 inputs) and
 *                    F16/BF16->F32 tables (all 2^16) hash to the values the
 *                    reference's CAST produces (tests/test_numeric_cpu.py);
 *                    closed-form IEEE RNE vs numpy for finite values
 *   binary           closed form (one IEEE op, RNE) vs numpy; strided and
 *                    broadcast layouts vs the compiled reference
 *   cast             conversions above + truncation closed form
 *   softmax          reference KATs; special rows closed form; finite rows
 *                    vs the compiled reference (bit-exact: same libm)
 *   snake1d          reference KATs (0x3e20def4, +inf); vs the compiled
 *                    reference (bit-exact: same libm)
 *   gated_silu       closed forms (silu(0) = 0, silu(+inf) = +inf,
 *                    silu(-inf) = NaN, gate rounding = the converters);
 *                    vs the compiled reference on random, special and
 *                    NaN-payload inputs of every dtype (bit-exact: same libm)
 *   tanh             closed forms (odd, +-1 beyond 22, x for tiny x);
 *                    vs the compiled reference on all special classes
 *   preflight        reference KATs (NaN / non-finite / out of range)
 */
#ifndef M3_ORACLE_H
#define M3_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#define ORACLE_MAX_RANK 8

enum { ORACLE_F32 = 0, ORACLE_F16 = 1, ORACLE_BF16 = 2, ORACLE_I32 = 3 };
enum { ORACLE_ADD = 0, ORACLE_MUL = 1, ORACLE_SUB = 2, ORACLE_DIV = 3 };

typedef struct {
    void *data;            /* host address of byte 0 of the storage */
    uint64_t byte_offset;
    uint32_t dtype;
    uint32_t rank;
    uint64_t shape[ORACLE_MAX_RANK];
    uint64_t byte_strides[ORACLE_MAX_RANK];
} oracle_view;

/* Bit-exact converters (src/m3_op_numeric.c:27-130). */
uint32_t oracle_f16_to_f32(uint16_t half);
uint16_t oracle_f32_to_f16(uint32_t bits);
uint32_t oracle_bf16_to_f32(uint16_t brain);
uint16_t oracle_f32_to_bf16(uint32_t bits);

/* Status codes mirror m3_status: 0 ok, 2 out of range. */
int oracle_binary(uint32_t op, const oracle_view *left,
                  const oracle_view *right, const oracle_view *output);
int oracle_cast(const oracle_view *input, const oracle_view *output);
int oracle_copy(const oracle_view *input, const oracle_view *output);
int oracle_softmax(const oracle_view *input, const oracle_view *output);
int oracle_snake1d(const oracle_view *input, const oracle_view *alpha,
                   const oracle_view *output);
int oracle_gated_silu(const oracle_view *gate, const oracle_view *up,
                      const oracle_view *output);
int oracle_tanh(const oracle_view *input, const oracle_view *output);

/* Data preflight (src/m3_op_data_preflight.c:8-64): 2 when the view holds
 * a NaN / a value that is non-finite or outside [-2^31, 2^31). */
int oracle_preflight_nan(const oracle_view *view);
int oracle_preflight_i32(const oracle_view *view);

/* Bulk helpers for tests: contiguous arrays. */
void oracle_f32_to_f16_array(const uint32_t *in, uint16_t *out, size_t n);
void oracle_f16_to_f32_array(const uint16_t *in, uint32_t *out, size_t n);
void oracle_f32_to_bf16_array(const uint32_t *in, uint16_t *out, size_t n);

#endif
