/*
 * fuse_check.c - host check of the session compiler's elementwise fusion
 * planner (m3.c_amd/csrc/host/m3_fuse.c) and of the program format it
 * emits (m3_hip_launch_program in include/m3_hip.h).
 *
 * A graph is executed node by node with one buffer per value (the
 * expected values), and then with every group the planner forms replaced
 * by its program, interpreted per element exactly as the kernel does
 * (registers R0-R3 and F0-F3, FETCH, OP, ROUND, STORE; m3_binary_f32_bits
 * for each operation, m3_round_through_bits for the rounding dtype,
 * conversions on load and store). The fused run works on one byte memory
 * in which every value sits in the slot the session compiler's liveness
 * plan gives it (INPUT, CONSTANT and OUTPUT values own a slot; a TEMPORARY
 * takes the smallest slot free before its producer that is large enough),
 * so values whose lives do not overlap share bytes as on the device. A
 * program's lanes run in no fixed order, so the fused run is made twice,
 * once over the elements in increasing and once in decreasing order: a
 * store that lands on bytes another element still reads changes the
 * result in one of the two. Before every node or program the values it
 * reads from memory must hold their expected bits; after it, every value
 * it stored that must reach memory (OUTPUT values, values read outside
 * their producer's group) must too, and so must every OUTPUT value at the
 * end. The words are also checked structurally (the rules of the
 * launcher).
 *
 * Modes (one JSON line on stdout; exit status 1 on any mismatch):
 *   fuse_check random <graphs> <seed> [planted]
 *       Random graphs of ADD/SUB/MUL/DIV, CAST and COPY over F32, F16 and
 *       BF16 values with array, scalar and differently sized operands,
 *       OUTPUT and TEMPORARY roles, and nodes on another provider between
 *       them. An operand smaller than the output (its count divides the
 *       output's) is a trailing broadcast, read at e mod its count, or,
 *       when the node does not mark it trailing, a leading one, read at
 *       e / (output count / its count); only the first kind may fuse.
 *       Nodes of kinds that never fuse (SOFTMAX with one input,
 *       GATED_SILU with two) read values between the groups.
 *       The last argument plants a mistake, and the comparison must then
 *       fail:
 *         `planted` corrupts each plan before it runs (the first STORE is
 *         turned into a store of another register, the sources of every
 *         SUB/DIV are swapped, OPs lose their rounding dtype and periodic
 *         operands their period);
 *         `unaware` hides where values live from the planner (no address
 *         ranges), so it cannot see a store landing on an operand's bytes;
 *         `blind` hides the reads of the nodes that never fuse from the
 *         planner, so it keeps values they read in registers only.
 *   fuse_check euler <steps>
 *       The Euler CFG graph of the flow solver, 6 nodes per step; reports
 *       the plan's shape and checks its result.
 */
#include "m3_fuse.h"
#include "m3_hip.h"
#include "m3_numeric.h"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define SENTINEL 0x7fbadbadU
#define NO_GROUP SIZE_MAX

typedef struct {
    m3_fuse_value *values;
    size_t value_count;
    size_t value_capacity;
    m3_fuse_node *nodes;
    size_t node_count;
    size_t node_capacity;
    uint32_t **data; /* per value: element_count raw elements */
    uint8_t *memory; /* when set, values live here, at their address */
} graph_t;

typedef enum {
    PLANT_NONE,
    PLANT_CODE,
    PLANT_UNAWARE,
    PLANT_BLIND
} plant_t;

static uint64_t rng_state;

static uint64_t next_random(void)
{
    uint64_t z = (rng_state += 0x9e3779b97f4a7c15ULL);

    z = (z ^ (z >> 30U)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27U)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31U);
}

static uint32_t below(uint32_t n)
{
    return (uint32_t)(next_random() % n);
}

static void *grow(void *array, size_t *capacity, size_t needed, size_t size)
{
    if (needed > *capacity) {
        *capacity = needed * 2U;
        array = realloc(array, *capacity * size);
        if (array == NULL) {
            fprintf(stderr, "out of memory\n");
            exit(2);
        }
    }
    return array;
}

static uint32_t add_value(graph_t *g, m3_graph_value_role role,
                          m3_dtype dtype, uint64_t count)
{
    g->values = grow(g->values, &g->value_capacity, g->value_count + 1U,
                     sizeof(*g->values));
    g->values[g->value_count].role = role;
    g->values[g->value_count].dtype = dtype;
    g->values[g->value_count].element_count = count;
    return (uint32_t)g->value_count++;
}

static void add_node(graph_t *g, m3_op_kind kind, uint32_t left,
                     uint32_t right, uint32_t output, bool eligible)
{
    g->nodes = grow(g->nodes, &g->node_capacity, g->node_count + 1U,
                    sizeof(*g->nodes));
    memset(&g->nodes[g->node_count], 0, sizeof(*g->nodes));
    g->nodes[g->node_count].kind = kind;
    g->nodes[g->node_count].reads[0] = left;
    g->nodes[g->node_count].reads[1] = right;
    g->nodes[g->node_count].read_count = left == right ? 1U : 2U;
    g->nodes[g->node_count].left = left;
    g->nodes[g->node_count].right = right;
    g->nodes[g->node_count].output = output;
    g->nodes[g->node_count].eligible = eligible;
    g->nodes[g->node_count].left_trailing = false;
    g->nodes[g->node_count].right_trailing = false;
    g->node_count += 1U;
}

/* A node of a kind that never fuses, reading `left` and `right` (one value
 * when they are equal). */
static bool opaque(const m3_fuse_node *node)
{
    return node->kind == M3_OP_SOFTMAX || node->kind == M3_OP_GATED_SILU;
}

static uint64_t element_size(m3_dtype dtype)
{
    return dtype == M3_DTYPE_F32 ? 4U : 2U;
}

/* Raw element `index` of a value: from its buffer, or from the memory at
 * the value's address during the fused run. */
static uint32_t load_raw(const graph_t *g, uint32_t value, uint64_t index)
{
    const m3_fuse_value *v = &g->values[value];
    const uint8_t *at;

    if (g->memory == NULL) {
        return g->data[value][index];
    }
    at = g->memory + v->address + index * element_size(v->dtype);
    return element_size(v->dtype) == 4U
               ? (uint32_t)at[0] | ((uint32_t)at[1] << 8U) |
                     ((uint32_t)at[2] << 16U) | ((uint32_t)at[3] << 24U)
               : (uint32_t)at[0] | ((uint32_t)at[1] << 8U);
}

static void store_raw(graph_t *g, uint32_t value, uint64_t index,
                      uint32_t bits)
{
    const m3_fuse_value *v = &g->values[value];
    uint8_t *at;

    if (g->memory == NULL) {
        g->data[value][index] = bits;
        return;
    }
    at = g->memory + v->address + index * element_size(v->dtype);
    for (uint64_t b = 0U; b < element_size(v->dtype); ++b) {
        at[b] = (uint8_t)(bits >> (8U * b));
    }
}

/* Slots as the session compiler plans them (src/m3_graph_compile.c:
 * 260-324 of the reference): INPUT, CONSTANT and OUTPUT values own one;
 * a TEMPORARY produced by node n takes the smallest slot whose last user
 * ran before n and that is large enough, else a new one. Slots are laid
 * out 64-byte aligned from address 4096. Returns the memory size. */
static uint64_t plan_memory(graph_t *g)
{
    const size_t count = g->value_count;
    uint64_t *slot_bytes = calloc(count, sizeof(*slot_bytes));
    uint64_t *slot_at = calloc(count, sizeof(*slot_at));
    size_t *busy = calloc(count, sizeof(*busy));
    size_t *slot_of = calloc(count, sizeof(*slot_of));
    size_t *last = calloc(count, sizeof(*last));
    size_t *producer = calloc(count, sizeof(*producer));
    size_t slots = 0U;
    uint64_t end = 4096U;

    if (slot_bytes == NULL || slot_at == NULL || busy == NULL ||
        slot_of == NULL || last == NULL || producer == NULL) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    for (size_t v = 0U; v < count; ++v) {
        producer[v] = SIZE_MAX;
        last[v] = 0U;
    }
    for (size_t n = 0U; n < g->node_count; ++n) {
        for (uint32_t k = 0U; k < g->nodes[n].read_count; ++k) {
            last[g->nodes[n].reads[k]] = n;
        }
        producer[g->nodes[n].output] = n;
        last[g->nodes[n].output] = n;
    }
    for (size_t v = 0U; v < count; ++v) {
        g->values[v].byte_count = g->values[v].element_count *
                                  element_size(g->values[v].dtype);
        if (g->values[v].role != M3_GRAPH_TEMPORARY) {
            slot_bytes[slots] = g->values[v].byte_count;
            busy[slots] = SIZE_MAX;
            slot_of[v] = slots++;
        }
    }
    for (size_t n = 0U; n < g->node_count; ++n) {
        const uint32_t v = g->nodes[n].output;
        size_t best = SIZE_MAX;

        if (g->values[v].role != M3_GRAPH_TEMPORARY || producer[v] != n) {
            continue;
        }
        for (size_t s = 0U; s < slots; ++s) {
            if (busy[s] < n && slot_bytes[s] >= g->values[v].byte_count &&
                (best == SIZE_MAX || slot_bytes[s] < slot_bytes[best])) {
                best = s;
            }
        }
        if (best == SIZE_MAX) {
            slot_bytes[slots] = g->values[v].byte_count;
            best = slots++;
        }
        slot_of[v] = best;
        busy[best] = last[v];
    }
    for (size_t s = 0U; s < slots; ++s) {
        slot_at[s] = end;
        end += (slot_bytes[s] + 63U) & ~(uint64_t)63U;
    }
    for (size_t v = 0U; v < count; ++v) {
        g->values[v].address = slot_at[slot_of[v]];
    }
    free(slot_bytes);
    free(slot_at);
    free(busy);
    free(slot_of);
    free(last);
    free(producer);
    return end;
}

/* Random F32 bits: mostly normal values near 1, with zeros, infinities,
 * NaN payloads of both signs and subnormals. */
static uint32_t random_f32(void)
{
    uint32_t pick = below(100U);
    uint32_t bits = (uint32_t)next_random();

    if (pick < 4U) {
        return (bits & 0x80000000U) | 0x7f800000U | (bits & 0x7fffffU) | 1U;
    }
    if (pick < 6U) {
        return (bits & 0x80000000U) | 0x7f800000U;
    }
    if (pick < 8U) {
        return bits & 0x80000000U;
    }
    if (pick < 10U) {
        return bits & 0x807fffffU;
    }
    return (bits & 0x807fffffU) | ((120U + below(14U)) << 23U);
}

/* Element `index` of a value, as F32 bits. */
static uint32_t load_f32(const graph_t *g, uint32_t value, uint64_t index)
{
    return m3_load_as_f32_bits(load_raw(g, value, index),
                               (uint32_t)g->values[value].dtype);
}

/* Index of an operand of `count` elements read for output element e of
 * `out` elements: the same element, the one scalar, a trailing broadcast
 * (e mod count) or a leading one (e / (out / count)). */
static uint64_t broadcast_index(uint64_t count, uint64_t out, bool trailing,
                                uint64_t e)
{
    return count == out  ? e
           : count == 1U ? 0U
           : trailing    ? e % count
                         : e / (out / count);
}

static uint32_t op_of(m3_op_kind kind)
{
    return kind == M3_OP_ADD   ? M3N_ADD
           : kind == M3_OP_MUL ? M3N_MUL
           : kind == M3_OP_SUB ? M3N_SUB
                               : M3N_DIV;
}

/* One node over all its elements, as the unfused provider runs it: COPY
 * and a CAST between equal dtypes copy the raw element
 * (src/m3_op_execute_basic.c:11-36), CAST converts through F32 (:37-59),
 * ADD/SUB/MUL/DIV compute in F32 and store in the output's dtype. */
static void run_node(graph_t *g, size_t n)
{
    const m3_fuse_node *node = &g->nodes[n];
    const m3_fuse_value *out = &g->values[node->output];
    uint64_t e;

    for (e = 0U; e < out->element_count; ++e) {
        uint32_t result;

        if ((node->kind == M3_OP_COPY || node->kind == M3_OP_CAST) &&
            g->values[node->left].dtype == out->dtype) {
            store_raw(g, node->output, e, load_raw(g, node->left, e));
            continue;
        }
        if (opaque(node)) {
            /* any fixed function of the inputs: x*x, or x*x + y */
            const uint32_t a = node->reads[0];
            const uint32_t b = node->reads[node->read_count - 1U];
            const uint32_t x = load_f32(
                g, a,
                broadcast_index(g->values[a].element_count,
                                out->element_count, false, e));
            const uint32_t y = load_f32(
                g, b,
                broadcast_index(g->values[b].element_count,
                                out->element_count, false, e));

            result = m3_binary_f32_bits(M3N_MUL, x, x);
            if (node->read_count == 2U) {
                result = m3_binary_f32_bits(M3N_ADD, result, y);
            }
        } else if (node->kind == M3_OP_CAST) {
            result = load_f32(g, node->left, e);
        } else {
            const uint64_t lc = g->values[node->left].element_count;
            const uint64_t rc = g->values[node->right].element_count;

            result = m3_binary_f32_bits(
                op_of(node->kind),
                load_f32(g, node->left,
                         broadcast_index(lc, out->element_count,
                                         node->left_trailing, e)),
                load_f32(g, node->right,
                         broadcast_index(rc, out->element_count,
                                         node->right_trailing, e)));
        }
        store_raw(g, node->output, e,
                  m3_store_from_f32_bits(result, (uint32_t)out->dtype));
    }
}

/* Structural check of a group's words (the launcher's rules). Returns
 * the number of violations. */
static size_t check_words(const m3_fuse_plan *plan, const m3_fuse_group *gr,
                          const graph_t *g)
{
    const uint32_t *code = plan->code + gr->code_first;
    size_t bad = 0U;
    size_t pc = 0U;
    size_t periodic = 0U;

    if (gr->operand_count > M3_HIP_PROGRAM_MAX_OPERANDS ||
        gr->code_count > M3_HIP_PROGRAM_MAX_WORDS) {
        return 1U;
    }
    for (size_t p = 0U; p < gr->operand_count; ++p) {
        const m3_fuse_operand *o = &plan->operands[gr->operand_first + p];
        uint64_t count;

        if (o->value >= g->value_count) {
            bad += 1U;
            continue;
        }
        count = g->values[o->value].element_count;
        bad += o->scalar != (count == 1U && gr->element_count > 1U);
        /* an array smaller than the group is read with its period, a
         * multiple of 4 dividing the group's count (the launcher's rule) */
        bad += o->period != (!o->scalar && count != gr->element_count
                                 ? count
                                 : 0U);
        bad += o->period != 0U && (o->period % 4U != 0U ||
                                   gr->element_count % o->period != 0U);
        periodic += o->period != 0U;
    }
    bad += periodic != gr->period_count;
    while (pc < gr->code_count) {
        uint32_t w = code[pc];

        switch (w & 3U) {
        case M3_HIP_PROGRAM_FETCH: {
            uint32_t n = ((w >> 2U) & 3U) + 1U;

            bad += (w >> 4U) != 0U || pc + 1U >= gr->code_count;
            for (uint32_t k = 0U; k < n && pc + 1U < gr->code_count; ++k) {
                uint32_t index = (code[pc + 1U] >> (8U * k)) & 0xffU;

                bad += index >= gr->operand_count ||
                       plan->operands[gr->operand_first + index].scalar;
            }
            pc += 2U;
            break;
        }
        case M3_HIP_PROGRAM_OP: {
            uint32_t left = (w >> 8U) & 15U;
            uint32_t right = (w >> 12U) & 15U;
            uint32_t scalar = (w >> 16U) & 0xffU;

            bad += (w & 0xc0U) != 0U || (w >> 26U) != 0U ||
                   ((w >> 24U) & 3U) > M3N_BF16 || left > 8U || right > 8U;
            if (left == 8U || right == 8U) {
                bad += scalar >= gr->operand_count ||
                       !plan->operands[gr->operand_first + scalar].scalar;
            } else {
                bad += scalar != 0U;
            }
            pc += 1U;
            break;
        }
        case M3_HIP_PROGRAM_ROUND: {
            uint32_t source = (w >> 8U) & 15U;
            uint32_t scalar = (w >> 16U) & 0xffU;

            bad += (w & 0xccU) != 0U || (w & 0xf000U) != 0U ||
                   (w >> 26U) != 0U || ((w >> 24U) & 3U) > M3N_BF16 ||
                   source > 8U;
            if (source == 8U) {
                bad += scalar >= gr->operand_count ||
                       !plan->operands[gr->operand_first + scalar].scalar;
            } else {
                bad += scalar != 0U;
            }
            pc += 1U;
            break;
        }
        case M3_HIP_PROGRAM_STORE: {
            uint32_t index = (w >> 8U) & 0xffU;

            bad += (w & 0xccU) != 0U || (w >> 16U) != 0U ||
                   index >= gr->operand_count ||
                   plan->operands[gr->operand_first + index].scalar ||
                   plan->operands[gr->operand_first + index].period != 0U;
            pc += 1U;
            break;
        }
        default:
            bad += 1U;
            pc += 1U;
            break;
        }
    }
    return bad;
}

/* The group's program over every element, as the kernel runs it, the
 * elements taken in increasing or in decreasing order. */
static size_t run_program(graph_t *g, const m3_fuse_plan *plan,
                          const m3_fuse_group *gr, bool decreasing)
{
    const uint32_t *code = plan->code + gr->code_first;
    const m3_fuse_operand *operands = plan->operands + gr->operand_first;
    size_t unwritten = 0U;
    uint64_t i;

    for (i = 0U; i < gr->element_count; ++i) {
        const uint64_t e = decreasing ? gr->element_count - 1U - i : i;
        uint32_t r[4] = {SENTINEL, SENTINEL, SENTINEL, SENTINEL};
        uint32_t f[4] = {SENTINEL, SENTINEL, SENTINEL, SENTINEL};
        bool r_set[4] = {false, false, false, false};
        bool f_set[4] = {false, false, false, false};
        size_t pc = 0U;

        while (pc < gr->code_count) {
            uint32_t w = code[pc];

            if ((w & 3U) == M3_HIP_PROGRAM_FETCH) {
                uint32_t n = ((w >> 2U) & 3U) + 1U;

                for (uint32_t k = 0U; k < n; ++k) {
                    const m3_fuse_operand *o =
                        &operands[(code[pc + 1U] >> (8U * k)) & 0xffU];
                    uint64_t at = o->period != 0U ? e % o->period : e;

                    /* a read past the value (a lost period) counts as
                     * unwritten and yields the sentinel */
                    if (at < g->values[o->value].element_count) {
                        f[k] = load_f32(g, o->value, at);
                        f_set[k] = true;
                    } else {
                        f[k] = SENTINEL;
                        f_set[k] = false;
                    }
                }
                pc += 2U;
            } else if ((w & 3U) == M3_HIP_PROGRAM_OP ||
                       (w & 3U) == M3_HIP_PROGRAM_ROUND) {
                bool binary = (w & 3U) == M3_HIP_PROGRAM_OP;
                uint32_t kinds[2] = {(w >> 8U) & 15U, (w >> 12U) & 15U};
                uint32_t x[2] = {0U, 0U};

                for (int k = 0; k < (binary ? 2 : 1); ++k) {
                    if (kinds[k] < 4U) {
                        x[k] = r[kinds[k]];
                        unwritten += !r_set[kinds[k]];
                    } else if (kinds[k] < 8U) {
                        x[k] = f[kinds[k] - 4U];
                        unwritten += !f_set[kinds[k] - 4U];
                    } else {
                        x[k] = load_f32(
                            g, operands[(w >> 16U) & 0xffU].value, 0U);
                    }
                }
                r[(w >> 4U) & 3U] = m3_round_through_bits(
                    binary ? m3_binary_f32_bits((w >> 2U) & 3U, x[0], x[1])
                           : x[0],
                    (w >> 24U) & 3U);
                r_set[(w >> 4U) & 3U] = true;
                pc += 1U;
            } else {
                uint32_t src = (w >> 4U) & 3U;
                uint32_t target = operands[(w >> 8U) & 0xffU].value;

                store_raw(g, target, e,
                          m3_store_from_f32_bits(
                              r[src], (uint32_t)g->values[target].dtype));
                unwritten += !r_set[src];
                pc += 1U;
            }
        }
    }
    return unwritten;
}

/* Corrupts a plan: the first STORE stores another register, the sources
 * of every SUB and DIV are swapped, no OP rounds through its output's
 * 16-bit dtype, and periodic operands lose their period. */
static void plant_code(m3_fuse_plan *plan)
{
    bool first = true;

    for (size_t p = 0U; p < plan->operand_count; ++p) {
        plan->operands[p].period = 0U;
    }
    for (size_t gi = 0U; gi < plan->group_count; ++gi) {
        const m3_fuse_group *gr = &plan->groups[gi];
        uint32_t *code = plan->code + gr->code_first;
        size_t pc = 0U;

        while (pc < gr->code_count) {
            uint32_t w = code[pc];

            if ((w & 3U) == M3_HIP_PROGRAM_FETCH) {
                pc += 2U;
                continue;
            }
            if ((w & 3U) == M3_HIP_PROGRAM_OP &&
                ((w >> 2U) & 3U) >= M3N_SUB) {
                uint32_t left = (w >> 8U) & 15U;
                uint32_t right = (w >> 12U) & 15U;

                code[pc] = (w & ~0xff00U) | (right << 8U) | (left << 12U);
            }
            if ((w & 3U) == M3_HIP_PROGRAM_OP) {
                code[pc] &= ~(3U << 24U); /* drop the rounding dtype */
            }
            if ((w & 3U) == M3_HIP_PROGRAM_STORE && first) {
                code[pc] = w ^ (1U << 4U);
                first = false;
            }
            pc += 1U;
        }
    }
}

typedef struct {
    size_t groups;
    size_t fused_nodes;
    size_t stores;
    size_t internal;
    size_t compared;
    size_t mismatches;
    size_t stale;     /* a node or program read bytes not holding its operand */
    size_t structure;
    size_t unwritten;
    size_t rounds;         /* ROUND instructions (fused CAST/COPY) */
    size_t rounding_ops;   /* OP instructions with a 16-bit rounding */
    size_t narrow_operands; /* F16/BF16 operands of programs */
    size_t periodic_operands; /* operands read with a period */
    size_t shared_slots;   /* program operands whose slot a store reuses */
} stats_t;

static void allocate_data(graph_t *g, uint32_t **data)
{
    for (size_t v = 0U; v < g->value_count; ++v) {
        data[v] = malloc((size_t)g->values[v].element_count *
                         sizeof(uint32_t) + sizeof(uint32_t));
        if (data[v] == NULL) {
            fprintf(stderr, "out of memory\n");
            exit(2);
        }
    }
}

/* The fused run's memory holds value v's expected bits. */
static bool holds(const graph_t *g, uint32_t **expected, uint32_t v)
{
    for (uint64_t e = 0U; e < g->values[v].element_count; ++e) {
        if (load_raw(g, v, e) != expected[v][e]) {
            return false;
        }
    }
    return true;
}

static bool node_reads(const m3_fuse_node *node, uint32_t v)
{
    for (uint32_t k = 0U; k < node->read_count; ++k) {
        if (node->reads[k] == v) {
            return true;
        }
    }
    return false;
}

/* What the planner is told: the graph, or the graph with a mistake of the
 * caller planted (no address ranges; no reads for nodes that never fuse,
 * whose records are then all zero). */
static void describe(const graph_t *g, plant_t plant, m3_fuse_value *values,
                     m3_fuse_node *nodes)
{
    memcpy(values, g->values, g->value_count * sizeof(*values));
    memcpy(nodes, g->nodes, g->node_count * sizeof(*nodes));
    for (size_t v = 0U; plant == PLANT_UNAWARE && v < g->value_count; ++v) {
        values[v].address = 0U;
        values[v].byte_count = 0U;
    }
    for (size_t n = 0U; plant == PLANT_BLIND && n < g->node_count; ++n) {
        if (opaque(&nodes[n])) {
            memset(&nodes[n], 0, sizeof(nodes[n]));
            nodes[n].kind = g->nodes[n].kind;
        }
    }
}

/* Plans g, runs it node by node and fused, and compares. */
static void check_graph(graph_t *g, plant_t plant, stats_t *st)
{
    const uint64_t memory_bytes = plan_memory(g);
    uint32_t **expected = calloc(g->value_count, sizeof(*expected));
    size_t *group_of = malloc(g->node_count * sizeof(*group_of));
    size_t *producer = malloc(g->value_count * sizeof(*producer));
    m3_fuse_value *told_values = malloc(g->value_count * sizeof(*told_values));
    m3_fuse_node *told_nodes = malloc(g->node_count * sizeof(*told_nodes));
    m3_fuse_plan plan;
    m3_error error;
    size_t v;
    size_t n;

    if (expected == NULL || group_of == NULL || producer == NULL ||
        told_values == NULL || told_nodes == NULL) {
        fprintf(stderr, "out of memory\n");
        exit(2);
    }
    allocate_data(g, expected);
    for (v = 0U; v < g->value_count; ++v) {
        const m3_fuse_value *val = &g->values[v];
        bool given = val->role == M3_GRAPH_INPUT ||
                     val->role == M3_GRAPH_CONSTANT;

        producer[v] = SIZE_MAX;
        for (uint64_t e = 0U; e < val->element_count; ++e) {
            uint32_t bits = random_f32();

            if (val->dtype == M3_DTYPE_F16) {
                bits = m3_f32_to_f16_bits(bits);
            } else if (val->dtype == M3_DTYPE_BF16) {
                bits = m3_f32_to_bf16_bits(bits);
            }
            expected[v][e] = given ? bits : SENTINEL;
        }
    }
    for (n = 0U; n < g->node_count; ++n) {
        producer[g->nodes[n].output] = n;
    }
    describe(g, plant, told_values, told_nodes);
    if (m3_fuse_plan_build(told_values, g->value_count, told_nodes,
                           g->node_count, &plan, &error) != M3_STATUS_OK) {
        fprintf(stderr, "plan failed: %s\n", error.message);
        exit(2);
    }
    if (plant == PLANT_CODE) {
        plant_code(&plan);
    }
    for (n = 0U; n < g->node_count; ++n) {
        group_of[n] = NO_GROUP;
    }
    for (size_t gi = 0U; gi < plan.group_count; ++gi) {
        const m3_fuse_group *gr = &plan.groups[gi];

        st->groups += 1U;
        st->fused_nodes += gr->node_count;
        st->structure += check_words(&plan, gr, g);
        for (size_t pc = 0U; pc < gr->code_count;) {
            uint32_t w = plan.code[gr->code_first + pc];

            st->stores += (w & 3U) == M3_HIP_PROGRAM_STORE;
            st->rounds += (w & 3U) == M3_HIP_PROGRAM_ROUND;
            st->rounding_ops += (w & 3U) == M3_HIP_PROGRAM_OP &&
                                ((w >> 24U) & 3U) != 0U;
            pc += (w & 3U) == M3_HIP_PROGRAM_FETCH ? 2U : 1U;
        }
        for (size_t p = 0U; p < gr->operand_count; ++p) {
            const m3_fuse_operand *o = &plan.operands[gr->operand_first + p];

            st->narrow_operands +=
                g->values[o->value].dtype != M3_DTYPE_F32;
            st->periodic_operands += o->period != 0U;
            for (size_t q = 0U; q < gr->operand_count; ++q) {
                const m3_fuse_operand *w =
                    &plan.operands[gr->operand_first + q];

                st->shared_slots +=
                    q != p &&
                    g->values[o->value].address ==
                        g->values[w->value].address;
            }
        }
        for (n = gr->first_node; n < gr->first_node + gr->node_count; ++n) {
            group_of[n] = gi;
        }
    }
    g->data = expected;
    g->memory = NULL;
    for (n = 0U; n < g->node_count; ++n) {
        run_node(g, n);
    }
    for (int pass = 0; pass < 2; ++pass) {
        g->memory = malloc(memory_bytes);
        if (g->memory == NULL) {
            fprintf(stderr, "out of memory\n");
            exit(2);
        }
        memset(g->memory, 0xa5, memory_bytes);
        for (v = 0U; v < g->value_count; ++v) {
            if (g->values[v].role == M3_GRAPH_INPUT ||
                g->values[v].role == M3_GRAPH_CONSTANT) {
                for (uint64_t e = 0U; e < g->values[v].element_count; ++e) {
                    store_raw(g, (uint32_t)v, e, expected[v][e]);
                }
            }
        }
        n = 0U;
        while (n < g->node_count) {
            size_t first = n;
            size_t end = n + 1U;

            if (group_of[n] != NO_GROUP) {
                const m3_fuse_group *gr = &plan.groups[group_of[n]];

                end = gr->first_node + gr->node_count;
                for (size_t p = 0U; p < gr->operand_count; ++p) {
                    uint32_t o = plan.operands[gr->operand_first + p].value;

                    if ((producer[o] == SIZE_MAX || producer[o] < first ||
                         producer[o] >= end) &&
                        !holds(g, expected, o)) {
                        st->stale += 1U;
                    }
                }
                st->unwritten += run_program(g, &plan, gr, pass == 1);
            } else {
                for (uint32_t k = 0U; k < g->nodes[n].read_count; ++k) {
                    st->stale += !holds(g, expected, g->nodes[n].reads[k]);
                }
                run_node(g, n);
            }
            /* every value produced here that must reach memory */
            for (size_t m = first; m < end; ++m) {
                const uint32_t out = g->nodes[m].output;
                bool needed = g->values[out].role != M3_GRAPH_TEMPORARY;

                for (size_t r = end; r < g->node_count && !needed; ++r) {
                    needed = node_reads(&g->nodes[r], out);
                }
                if (!needed) {
                    st->internal += pass == 0 && group_of[m] != NO_GROUP;
                    continue;
                }
                st->compared += 1U;
                st->mismatches += !holds(g, expected, out);
            }
            n = end;
        }
        for (v = 0U; v < g->value_count; ++v) {
            if (g->values[v].role == M3_GRAPH_OUTPUT) {
                st->compared += 1U;
                st->mismatches += !holds(g, expected, (uint32_t)v);
            }
        }
        free(g->memory);
        g->memory = NULL;
    }
    for (v = 0U; v < g->value_count; ++v) {
        free(expected[v]);
    }
    free(expected);
    free(group_of);
    free(producer);
    free(told_values);
    free(told_nodes);
    m3_fuse_plan_free(&plan);
}

static void random_graph(graph_t *g)
{
    static const m3_op_kind kinds[] = {M3_OP_ADD, M3_OP_MUL, M3_OP_SUB,
                                       M3_OP_DIV};
    /* half of the graphs have a count that is a multiple of 4, with a
     * period (a multiple of 4 dividing it) for trailing operands; a value
     * of half the count (not always a multiple of 4) is read with either
     * broadcast */
    const uint64_t quads = 1U + below(10U);
    const uint64_t base = below(2U) ? 4U * quads : 1U + below(40U);
    uint64_t period = 4U;
    const uint64_t counts[3] = {base, 1U, 1U + below(12U)};
    size_t nodes = 2U + below(40U);

    if (base % 4U == 0U) {
        do {
            period = 4U * (1U + below((uint32_t)quads));
        } while (base % period != 0U);
    }
    memset(g, 0, sizeof(*g));
    for (int k = 0; k < 3; ++k) {
        (void)add_value(g, below(2U) ? M3_GRAPH_INPUT : M3_GRAPH_CONSTANT,
                        M3_DTYPE_F32, counts[0]);
    }
    (void)add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, 1U);
    (void)add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, 1U);
    (void)add_value(g, M3_GRAPH_INPUT, M3_DTYPE_F32, counts[2]);
    (void)add_value(g, M3_GRAPH_INPUT, M3_DTYPE_F16, counts[0]);
    (void)add_value(g, M3_GRAPH_INPUT, M3_DTYPE_BF16, counts[0]);
    (void)add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_BF16, 1U);
    (void)add_value(g, M3_GRAPH_INPUT, M3_DTYPE_F32, period);
    (void)add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_BF16, period);
    (void)add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32,
                    base % 2U == 0U ? base / 2U : base);
    for (size_t n = 0U; n < nodes; ++n) {
        static const m3_dtype floats[3] = {M3_DTYPE_F32, M3_DTYPE_F16,
                                           M3_DTYPE_BF16};
        uint32_t left = below((uint32_t)g->value_count);
        uint64_t lc = g->values[left].element_count;
        uint32_t right;
        uint64_t rc;
        m3_dtype dtype = M3_DTYPE_F32;
        uint32_t unary = below(100U);
        m3_graph_value_role role =
            n + 1U == nodes || below(100U) < 15U ? M3_GRAPH_OUTPUT
                                                 : M3_GRAPH_TEMPORARY;

        do {
            right = below((uint32_t)g->value_count);
            rc = g->values[right].element_count;
        } while (lc % rc != 0U && rc % lc != 0U);
        if (g->values[left].dtype != M3_DTYPE_F32 ||
            g->values[right].dtype != M3_DTYPE_F32 || below(100U) < 20U) {
            dtype = floats[below(3U)];
        }
        if (unary < 8U) {
            uint32_t out = add_value(g, role, g->values[left].dtype, lc);

            add_node(g, M3_OP_COPY, left, left, out, below(2U) != 0U);
            continue;
        }
        if (unary < 20U) {
            uint32_t out = add_value(g, role, floats[below(3U)], lc);

            add_node(g, M3_OP_CAST, left, left, out, below(100U) >= 5U);
            continue;
        }
        if (unary < 28U) {
            /* a node that never fuses, reading one or two values */
            const bool two = below(2U) != 0U;
            uint32_t out = add_value(g, role, floats[below(3U)],
                                     two && rc > lc ? rc : lc);

            add_node(g, two ? M3_OP_GATED_SILU : M3_OP_SOFTMAX, left,
                     two ? right : left, out, below(2U) != 0U);
            continue;
        }
        add_node(g, kinds[below(4U)], left, right,
                 add_value(g, role, dtype, lc > rc ? lc : rc),
                 below(100U) >= 5U);
        g->nodes[g->node_count - 1U].left_trailing = below(100U) < 75U;
        g->nodes[g->node_count - 1U].right_trailing = below(100U) < 75U;
    }
}

static void euler_graph(graph_t *g, size_t steps, uint64_t count)
{
    uint32_t x;
    uint32_t minus_one;
    uint32_t scale;
    uint32_t dt;

    memset(g, 0, sizeof(*g));
    x = add_value(g, M3_GRAPH_INPUT, M3_DTYPE_F32, count);
    minus_one = add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, 1U);
    scale = add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, 1U);
    dt = add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, 1U);
    for (size_t k = 0U; k < steps; ++k) {
        uint32_t vu = add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, count);
        uint32_t vc = add_value(g, M3_GRAPH_CONSTANT, M3_DTYPE_F32, count);
        uint32_t t[5];
        uint32_t next;

        for (int i = 0; i < 5; ++i) {
            t[i] = add_value(g, M3_GRAPH_TEMPORARY, M3_DTYPE_F32, count);
        }
        next = add_value(g,
                         k + 1U == steps ? M3_GRAPH_OUTPUT
                                         : M3_GRAPH_TEMPORARY,
                         M3_DTYPE_F32, count);
        add_node(g, M3_OP_MUL, vu, minus_one, t[0], true);
        add_node(g, M3_OP_ADD, vc, t[0], t[1], true);
        add_node(g, M3_OP_MUL, t[1], scale, t[2], true);
        add_node(g, M3_OP_ADD, vu, t[2], t[3], true);
        add_node(g, M3_OP_MUL, t[3], dt, t[4], true);
        add_node(g, M3_OP_ADD, x, t[4], next, true);
        x = next;
    }
}

static void free_graph(graph_t *g)
{
    free(g->values);
    free(g->nodes);
}

static void print_stats(const char *mode, size_t graphs, const stats_t *st)
{
    printf("{\"mode\": \"%s\", \"graphs\": %zu, \"groups\": %zu, "
           "\"fused_nodes\": %zu, \"stores\": %zu, \"internal_values\": %zu, "
           "\"compared_values\": %zu, \"mismatches\": %zu, "
           "\"structure_errors\": %zu, \"unwritten_reads\": %zu, "
           "\"rounds\": %zu, \"rounding_ops\": %zu, "
           "\"narrow_operands\": %zu, \"periodic_operands\": %zu, "
           "\"stale_reads\": %zu, \"shared_slots\": %zu",
           mode, graphs, st->groups, st->fused_nodes, st->stores,
           st->internal, st->compared, st->mismatches, st->structure,
           st->unwritten, st->rounds, st->rounding_ops, st->narrow_operands,
           st->periodic_operands, st->stale, st->shared_slots);
}

int main(int argc, char **argv)
{
    stats_t st;

    memset(&st, 0, sizeof(st));
    if (argc >= 4 && strcmp(argv[1], "random") == 0) {
        size_t graphs = strtoull(argv[2], NULL, 10);
        const char *mode = argc >= 5 ? argv[4] : "random";
        plant_t plant = strcmp(mode, "planted") == 0   ? PLANT_CODE
                        : strcmp(mode, "unaware") == 0 ? PLANT_UNAWARE
                        : strcmp(mode, "blind") == 0   ? PLANT_BLIND
                                                       : PLANT_NONE;

        rng_state = strtoull(argv[3], NULL, 10);
        for (size_t i = 0U; i < graphs; ++i) {
            graph_t g;

            random_graph(&g);
            check_graph(&g, plant, &st);
            free_graph(&g);
        }
        print_stats(plant == PLANT_NONE ? "random" : mode, graphs, &st);
        printf("}\n");
        return st.mismatches == 0U && st.stale == 0U &&
                       st.structure == 0U && st.unwritten == 0U
                   ? 0
                   : 1;
    }
    if (argc == 3 && strcmp(argv[1], "euler") == 0) {
        size_t steps = strtoull(argv[2], NULL, 10);
        graph_t g;
        m3_fuse_plan plan;
        m3_error error;
        size_t fetch_loads = 0U;

        rng_state = 7U;
        euler_graph(&g, steps, 37U);
        if (m3_fuse_plan_build(g.values, g.value_count, g.nodes, g.node_count,
                               &plan, &error) != M3_STATUS_OK) {
            fprintf(stderr, "plan failed: %s\n", error.message);
            return 2;
        }
        for (size_t gi = 0U; gi < plan.group_count; ++gi) {
            const m3_fuse_group *gr = &plan.groups[gi];
            size_t pc = 0U;

            while (pc < gr->code_count) {
                uint32_t w = plan.code[gr->code_first + pc];

                if ((w & 3U) == M3_HIP_PROGRAM_FETCH) {
                    fetch_loads += ((w >> 2U) & 3U) + 1U;
                    pc += 2U;
                } else {
                    pc += 1U;
                }
            }
        }
        check_graph(&g, PLANT_NONE, &st);
        print_stats("euler", 1U, &st);
        printf(", \"first_group_nodes\": %zu, \"first_group_operands\": %zu, "
               "\"first_group_words\": %zu, \"fetched_arrays\": %zu}\n",
               plan.group_count ? plan.groups[0].node_count : 0U,
               plan.group_count ? plan.groups[0].operand_count : 0U,
               plan.group_count ? plan.groups[0].code_count : 0U,
               fetch_loads);
        m3_fuse_plan_free(&plan);
        free_graph(&g);
        return st.mismatches == 0U && st.stale == 0U &&
                       st.structure == 0U && st.unwritten == 0U
                   ? 0
                   : 1;
    }
    fprintf(stderr, "usage: fuse_check random <graphs> <seed> "
                    "[planted|unaware|blind] | "
                    "euler <steps>\n");
    return 2;
}
