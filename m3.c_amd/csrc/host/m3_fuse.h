/*
 * m3_fuse.h - elementwise fusion planner of the session compiler.
 *
 * The planner sees the graph as values (role, dtype, element count) and
 * nodes in execution order, and groups consecutive ADD/SUB/MUL/DIV and
 * CAST/COPY nodes over F32, F16 and BF16 values of one element space into
 * programs for m3_hip_launch_program (word layout in m3_hip.h). It works
 * on value indices only; the session compiler resolves operands to device
 * addresses. Nothing here touches a device, so the planner is tested on
 * the host.
 *
 * Rules, in the order nodes run:
 *   - a node may join a group when it is eligible (its provider executes
 *     programs) and is either ADD/SUB/MUL/DIV whose operands and output
 *     are F32, F16 or BF16 and whose operands have the output's element
 *     count (an array read at the same flat index), one element (a
 *     scalar read by every element) or, when the node marks the operand
 *     trailing, M elements with M a multiple of 4 that divides the
 *     output's count (a periodic operand: element e reads e mod M, the
 *     right-aligned broadcast of a tensor whose shape, leading ones
 *     removed, is the output's trailing dimensions); or a CAST between
 *     two of those dtypes, or a COPY of F32, described with
 *     right == left and an input of the output's element count;
 *   - a group is a run of consecutive such nodes with the same element
 *     count; a value produced in the group lives in one of four registers
 *     from its producer to its last use, and a node joins only if a
 *     register is free for its output after its operands' last uses;
 *   - a value produced in the group is stored unless it is a TEMPORARY
 *     whose every use is inside the group (those never reach memory);
 *   - operands produced before the group are fetched in batches of up to
 *     four arrays covering the next nodes, so their loads overlap;
 *   - the lanes of a program run in no particular order, so a group may
 *     not store a value over memory that another lane may still read: a
 *     stored value's bytes may overlap an operand the group reads from
 *     memory only when both are arrays of the group's element count with
 *     the same base address and element size (each lane then reads its
 *     element before it writes the same bytes). Slots come from the
 *     unfused liveness plan, which lets a value produced late take the
 *     slot of one whose last reader ran earlier; a group that would store
 *     over a periodic or scalar operand, or over an array of another
 *     element size, is cut short before the node that makes it so.
 * Liveness counts every value a node reads (`reads`), whatever its kind,
 * so a value produced in a group and read later by a node that is not
 * fused (SOFTMAX, TANH, SNAKE1D, GATED_SILU, ...) is stored.
 * Groups of one node are not formed. The per-element order of operations,
 * the operations themselves and every stored value are the unfused ones: a
 * value of a 16-bit dtype is kept in its register as the F32 a store and a
 * load back give.
 */
#ifndef M3_FUSE_H
#define M3_FUSE_H

#include "m3_internal.h"

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

/* address/byte_count: where the value lives; byte_count 0 when it has no
 * memory of its own (it then overlaps nothing). */
typedef struct {
    m3_graph_value_role role;
    m3_dtype dtype;
    uint64_t element_count;
    uint64_t address;
    uint64_t byte_count;
} m3_fuse_value;

#define M3_FUSE_MAX_READS 5U

/* reads: every value the node reads, whatever its kind (liveness).
 * left/right/output: the operands of a node that may fuse (a unary node
 * has right == left); output is also the value the node writes.
 * left_trailing / right_trailing: the operand's shape, leading ones
 * removed, equals the output's trailing dimensions, so a smaller operand
 * is a right-aligned broadcast read at e mod its element count. */
typedef struct {
    m3_op_kind kind;
    uint32_t reads[M3_FUSE_MAX_READS];
    uint32_t read_count;
    uint32_t left;
    uint32_t right;
    uint32_t output;
    bool eligible;
    bool left_trailing;
    bool right_trailing;
} m3_fuse_node;

/* An operand of a group's program: value index, whether it is read as a
 * scalar, and its period (0 unless it is a periodic array). Operand i of
 * the group is entry operand_first + i. */
typedef struct {
    uint32_t value;
    bool scalar;
    uint64_t period;
} m3_fuse_operand;

typedef struct {
    size_t first_node;
    size_t node_count;
    uint64_t element_count;
    size_t operand_first;
    size_t operand_count;
    size_t period_count; /* operands with a period */
    size_t code_first;
    size_t code_count;
} m3_fuse_group;

typedef struct {
    m3_fuse_group *groups;
    size_t group_count;
    m3_fuse_operand *operands;
    size_t operand_count;
    uint32_t *code;
    size_t code_count;
} m3_fuse_plan;

/* Plans the groups of `nodes` (execution order). Values are referenced by
 * index; every node's reads, operands and output must be < value_count,
 * and an eligible node's left and right must be among its reads. On
 * success *plan owns its arrays (free with m3_fuse_plan_free); a plan
 * with no groups is valid. */
m3_status m3_fuse_plan_build(const m3_fuse_value *values, size_t value_count,
                             const m3_fuse_node *nodes, size_t node_count,
                             m3_fuse_plan *plan, m3_error *error);
void m3_fuse_plan_free(m3_fuse_plan *plan);

#endif
