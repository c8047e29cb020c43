/*
 * m3_fuse.c - elementwise fusion planner (rules in m3_fuse.h).
 *
 * Two passes over the nodes. The first decides group membership: a node
 * joins while the register state admits it (m3_fuse_step). The second
 * replays the same register state over each group and emits its program:
 * FETCH batches for operands produced before the group, one OP (binary
 * nodes) or ROUND (CAST, COPY) per node, and a STORE for every value that
 * must reach memory. A unary node is described with right == left, so the
 * register and fetch logic sees its one operand twice and counts it once.
 * Between the passes, a group whose stores could land on memory another
 * lane still reads is shortened (m3_fuse_group_races).
 */
#include "m3_fuse.h"

#include "m3_hip.h"

#include <stdlib.h>
#include <string.h>

#define M3_FUSE_REGISTERS 4U
#define M3_FUSE_FETCHES 4U
#define M3_FUSE_NONE UINT32_MAX
#define M3_FUSE_NO_NODE SIZE_MAX
#define M3_FUSE_SCALAR_SOURCE 8U
/* Upper bound of the instruction words one node adds to a program: a
 * two-word FETCH, the OP and a STORE. */
#define M3_FUSE_NODE_WORDS 4U

typedef struct {
    const m3_fuse_value *values;
    size_t value_count;
    const m3_fuse_node *nodes;
    size_t node_count;
    size_t *producer; /* node producing each value, or M3_FUSE_NO_NODE */
    size_t *last_use; /* last node reading each value, or M3_FUSE_NO_NODE */
} m3_fuse_graph;

typedef struct {
    size_t first;
    uint64_t count;
    uint32_t holder[M3_FUSE_REGISTERS]; /* value in R_i, or M3_FUSE_NONE */
} m3_fuse_registers;

static bool m3_fuse_op_of(m3_op_kind kind, uint32_t *op)
{
    switch (kind) {
    case M3_OP_ADD:
        *op = M3_HIP_ADD;
        return true;
    case M3_OP_MUL:
        *op = M3_HIP_MUL;
        return true;
    case M3_OP_SUB:
        *op = M3_HIP_SUB;
        return true;
    case M3_OP_DIV:
        *op = M3_HIP_DIV;
        return true;
    default:
        return false;
    }
}

static bool m3_fuse_float(m3_dtype dtype)
{
    return dtype == M3_DTYPE_F32 || dtype == M3_DTYPE_F16 ||
           dtype == M3_DTYPE_BF16;
}

static bool m3_fuse_unary(m3_op_kind kind)
{
    return kind == M3_OP_CAST || kind == M3_OP_COPY;
}

/* An operand of `element_count` elements read periodically by a group of
 * `count`: every group of four elements lies within one period, and the
 * period fits its program word. */
static bool m3_fuse_periodic(uint64_t element_count, uint64_t count)
{
    return element_count > 1U && element_count < count &&
           element_count <= UINT32_MAX && element_count % 4U == 0U &&
           count % element_count == 0U;
}

static bool m3_fuse_candidate(const m3_fuse_graph *g, size_t n)
{
    const m3_fuse_node *node = &g->nodes[n];
    const uint32_t operands[2] = {node->left, node->right};
    const m3_fuse_value *output = &g->values[node->output];
    uint32_t op;
    size_t k;

    if (!node->eligible || output->element_count == 0U ||
        !m3_fuse_float(output->dtype)) {
        return false;
    }
    if (m3_fuse_unary(node->kind)) {
        const m3_fuse_value *input = &g->values[node->left];

        /* A 16-bit value kept in a register is F32; storing it again is
         * not a byte copy for a signalling NaN, so a copy between equal
         * dtypes fuses only for F32, whose register holds the raw bits. */
        return node->right == node->left && m3_fuse_float(input->dtype) &&
               input->element_count == output->element_count &&
               (input->dtype != output->dtype ||
                output->dtype == M3_DTYPE_F32);
    }
    if (!m3_fuse_op_of(node->kind, &op)) {
        return false;
    }
    for (k = 0U; k < 2U; ++k) {
        const m3_fuse_value *value = &g->values[operands[k]];
        const bool trailing =
            k == 0U ? node->left_trailing : node->right_trailing;

        if (!m3_fuse_float(value->dtype) ||
            (value->element_count != output->element_count &&
             value->element_count != 1U &&
             !(trailing && m3_fuse_periodic(value->element_count,
                                            output->element_count)))) {
            return false;
        }
    }
    return true;
}

static bool m3_fuse_in_group(const m3_fuse_graph *g, uint32_t value,
                             size_t first, size_t node)
{
    size_t producer = g->producer[value];

    return producer != M3_FUSE_NO_NODE && producer >= first &&
           producer < node;
}

static bool m3_fuse_scalar(const m3_fuse_graph *g, uint32_t value,
                           uint64_t count)
{
    return g->values[value].element_count == 1U && count > 1U;
}

static uint32_t m3_fuse_holder_of(const m3_fuse_registers *r, uint32_t value)
{
    uint32_t i;

    for (i = 0U; i < M3_FUSE_REGISTERS; ++i) {
        if (r->holder[i] == value) {
            return i;
        }
    }
    return M3_FUSE_NONE;
}

/* Node `n` joins the group whose register state is *r: its operands
 * produced in the group must be in registers; those whose last use is n
 * are released; the output takes the lowest free register (released again
 * at once when nothing reads it). Returns false, leaving *r unchanged,
 * when an operand is not held or no register is free. */
static bool m3_fuse_step(const m3_fuse_graph *g, m3_fuse_registers *r,
                         size_t n, uint32_t *output_register)
{
    const m3_fuse_node *node = &g->nodes[n];
    const uint32_t operands[2] = {node->left, node->right};
    m3_fuse_registers next = *r;
    uint32_t chosen = M3_FUSE_NONE;
    uint32_t i;
    size_t k;

    for (k = 0U; k < 2U; ++k) {
        if (m3_fuse_in_group(g, operands[k], r->first, n) &&
            m3_fuse_holder_of(r, operands[k]) == M3_FUSE_NONE) {
            return false;
        }
    }
    for (k = 0U; k < 2U; ++k) {
        if (m3_fuse_in_group(g, operands[k], r->first, n) &&
            g->last_use[operands[k]] == n) {
            uint32_t held = m3_fuse_holder_of(&next, operands[k]);

            if (held != M3_FUSE_NONE) {
                next.holder[held] = M3_FUSE_NONE;
            }
        }
    }
    for (i = 0U; i < M3_FUSE_REGISTERS && chosen == M3_FUSE_NONE; ++i) {
        if (next.holder[i] == M3_FUSE_NONE) {
            chosen = i;
        }
    }
    if (chosen == M3_FUSE_NONE) {
        return false;
    }
    next.holder[chosen] = node->output;
    if (g->last_use[node->output] == M3_FUSE_NO_NODE) {
        next.holder[chosen] = M3_FUSE_NONE;
    }
    *r = next;
    *output_register = chosen;
    return true;
}

static uint64_t m3_fuse_element_size(m3_dtype dtype)
{
    return dtype == M3_DTYPE_F32 ? 4U : 2U;
}

static bool m3_fuse_overlap(const m3_fuse_value *a, const m3_fuse_value *b)
{
    return a->byte_count != 0U && b->byte_count != 0U &&
           a->address < b->address + b->byte_count &&
           b->address < a->address + a->byte_count;
}

/* A value produced in [first, end) that the group's program stores. */
static bool m3_fuse_stored(const m3_fuse_graph *g, uint32_t value,
                           size_t first, size_t end)
{
    const size_t producer = g->producer[value];
    const size_t last = g->last_use[value];

    return producer != M3_FUSE_NO_NODE && producer >= first &&
           producer < end &&
           (g->values[value].role != M3_GRAPH_TEMPORARY ||
            (last != M3_FUSE_NO_NODE && last >= end));
}

/* True when the program of nodes [first, end) would store over memory
 * that a lane other than the storing one may still read: a stored value
 * overlapping an operand read from memory, unless both are arrays of the
 * group's element count at one base address with one element size. */
static bool m3_fuse_group_races(const m3_fuse_graph *g, size_t first,
                                size_t end)
{
    const uint64_t count = g->values[g->nodes[first].output].element_count;
    size_t m;
    size_t p;
    size_t k;

    for (m = first; m < end; ++m) {
        const uint32_t operands[2] = {g->nodes[m].left, g->nodes[m].right};

        for (k = 0U; k < 2U; ++k) {
            const m3_fuse_value *read = &g->values[operands[k]];

            if (m3_fuse_in_group(g, operands[k], first, m)) {
                continue;
            }
            for (p = first; p < end; ++p) {
                const uint32_t output = g->nodes[p].output;
                const m3_fuse_value *stored = &g->values[output];

                if (!m3_fuse_stored(g, output, first, end) ||
                    !m3_fuse_overlap(read, stored)) {
                    continue;
                }
                if (read->element_count == count &&
                    read->address == stored->address &&
                    m3_fuse_element_size(read->dtype) ==
                        m3_fuse_element_size(stored->dtype)) {
                    continue;
                }
                return true;
            }
        }
    }
    return false;
}

static bool m3_fuse_grow(void **array, size_t *capacity, size_t needed,
                         size_t element)
{
    size_t grown;
    void *moved;

    if (needed <= *capacity) {
        return true;
    }
    grown = *capacity == 0U ? 64U : *capacity;
    while (grown < needed) {
        grown *= 2U;
    }
    moved = realloc(*array, grown * element);
    if (moved == NULL) {
        return false;
    }
    *array = moved;
    *capacity = grown;
    return true;
}

typedef struct {
    m3_fuse_plan *plan;
    size_t group_capacity;
    size_t operand_capacity;
    size_t code_capacity;
    bool failed;
} m3_fuse_writer;

static void m3_fuse_emit(m3_fuse_writer *w, uint32_t word)
{
    m3_fuse_plan *plan = w->plan;

    if (w->failed || !m3_fuse_grow((void **)&plan->code, &w->code_capacity,
                                   plan->code_count + 1U,
                                   sizeof(*plan->code))) {
        w->failed = true;
        return;
    }
    plan->code[plan->code_count++] = word;
}

/* Index of (value, scalar) among the group's operands, added if new. An
 * array with fewer elements than the group is periodic (the candidate
 * rule admits no other). */
static uint32_t m3_fuse_operand_index(const m3_fuse_graph *g,
                                      m3_fuse_writer *w,
                                      const m3_fuse_group *group,
                                      uint32_t value, bool scalar)
{
    m3_fuse_plan *plan = w->plan;
    const uint64_t element_count = g->values[value].element_count;
    size_t i;

    for (i = group->operand_first; i < plan->operand_count; ++i) {
        if (plan->operands[i].value == value &&
            plan->operands[i].scalar == scalar) {
            return (uint32_t)(i - group->operand_first);
        }
    }
    if (w->failed ||
        !m3_fuse_grow((void **)&plan->operands, &w->operand_capacity,
                      plan->operand_count + 1U, sizeof(*plan->operands))) {
        w->failed = true;
        return 0U;
    }
    plan->operands[plan->operand_count].value = value;
    plan->operands[plan->operand_count].scalar = scalar;
    plan->operands[plan->operand_count].period =
        !scalar && element_count != group->element_count ? element_count
                                                          : 0U;
    plan->operand_count += 1U;
    return (uint32_t)(i - group->operand_first);
}

/* Operands of node n read from memory as arrays (produced before the
 * group, not scalars), distinct, in operand order. */
static size_t m3_fuse_array_operands(const m3_fuse_graph *g, size_t first,
                                     uint64_t count, size_t n,
                                     uint32_t arrays[2])
{
    const m3_fuse_node *node = &g->nodes[n];
    const uint32_t operands[2] = {node->left, node->right};
    size_t found = 0U;
    size_t k;

    for (k = 0U; k < 2U; ++k) {
        uint32_t value = operands[k];

        if (m3_fuse_in_group(g, value, first, n) ||
            m3_fuse_scalar(g, value, count) ||
            (found == 1U && arrays[0] == value)) {
            continue;
        }
        arrays[found++] = value;
    }
    return found;
}

static bool m3_fuse_batch_has(const uint32_t *batch, size_t size,
                              uint32_t value, uint32_t *slot)
{
    size_t i;

    for (i = 0U; i < size; ++i) {
        if (batch[i] == value) {
            *slot = (uint32_t)i;
            return true;
        }
    }
    return false;
}

/* Emits the program of the nodes [first, end). */
static void m3_fuse_emit_group(const m3_fuse_graph *g, m3_fuse_writer *w,
                               size_t first, size_t end)
{
    m3_fuse_plan *plan = w->plan;
    m3_fuse_group group;
    m3_fuse_registers r;
    uint32_t batch[M3_FUSE_FETCHES];
    size_t batch_size = 0U;
    size_t n;
    uint32_t i;

    (void)memset(&group, 0, sizeof(group));
    group.first_node = first;
    group.node_count = end - first;
    group.element_count = g->values[g->nodes[first].output].element_count;
    group.operand_first = plan->operand_count;
    group.code_first = plan->code_count;
    r.first = first;
    r.count = group.element_count;
    for (i = 0U; i < M3_FUSE_REGISTERS; ++i) {
        r.holder[i] = M3_FUSE_NONE;
    }
    for (n = first; n < end && !w->failed; ++n) {
        const m3_fuse_node *node = &g->nodes[n];
        const uint32_t operands[2] = {node->left, node->right};
        uint32_t sources[2];
        uint32_t scalar = 0U;
        uint32_t arrays[2];
        size_t array_count =
            m3_fuse_array_operands(g, first, group.element_count, n, arrays);
        uint32_t slot = 0U;
        uint32_t op = 0U;
        uint32_t destination = 0U;
        const m3_fuse_value *output = &g->values[node->output];
        size_t k;

        /* a new FETCH batch when an operand array is not loaded: the
         * distinct operand arrays of this node and the following ones,
         * up to four */
        for (k = 0U; k < array_count; ++k) {
            if (!m3_fuse_batch_has(batch, batch_size, arrays[k], &slot)) {
                break;
            }
        }
        if (k < array_count) {
            uint32_t list = 0U;
            size_t m;

            batch_size = 0U;
            for (m = n; m < end; ++m) {
                uint32_t more[2];
                size_t more_count =
                    m3_fuse_array_operands(g, first, group.element_count, m,
                                           more);
                size_t fresh = 0U;
                size_t q;

                for (q = 0U; q < more_count; ++q) {
                    fresh += m3_fuse_batch_has(batch, batch_size, more[q],
                                               &slot)
                                 ? 0U
                                 : 1U;
                }
                if (batch_size + fresh > M3_FUSE_FETCHES) {
                    break;
                }
                for (q = 0U; q < more_count; ++q) {
                    if (!m3_fuse_batch_has(batch, batch_size, more[q],
                                           &slot)) {
                        batch[batch_size++] = more[q];
                    }
                }
            }
            for (m = 0U; m < batch_size; ++m) {
                list |= m3_fuse_operand_index(g, w, &group, batch[m], false)
                        << (8U * m);
            }
            m3_fuse_emit(w, (uint32_t)M3_HIP_PROGRAM_FETCH |
                                ((uint32_t)(batch_size - 1U) << 2U));
            m3_fuse_emit(w, list);
        }
        for (k = 0U; k < 2U; ++k) {
            uint32_t value = operands[k];

            if (m3_fuse_in_group(g, value, first, n)) {
                sources[k] = m3_fuse_holder_of(&r, value);
            } else if (m3_fuse_scalar(g, value, group.element_count)) {
                scalar = m3_fuse_operand_index(g, w, &group, value, true);
                sources[k] = M3_FUSE_SCALAR_SOURCE;
            } else {
                (void)m3_fuse_batch_has(batch, batch_size, value, &slot);
                sources[k] = M3_FUSE_FETCHES + slot;
            }
        }
        if (!m3_fuse_step(g, &r, n, &destination)) {
            w->failed = true; /* the first pass admitted this node */
            break;
        }
        /* the register holds the value a store to the output's dtype and
         * a load back give */
        if (m3_fuse_unary(node->kind)) {
            m3_fuse_emit(w, (uint32_t)M3_HIP_PROGRAM_ROUND |
                                (destination << 4U) | (sources[0] << 8U) |
                                (scalar << 16U) |
                                ((uint32_t)output->dtype << 24U));
        } else {
            (void)m3_fuse_op_of(node->kind, &op);
            m3_fuse_emit(w, (uint32_t)M3_HIP_PROGRAM_OP | (op << 2U) |
                                (destination << 4U) | (sources[0] << 8U) |
                                (sources[1] << 12U) | (scalar << 16U) |
                                ((uint32_t)output->dtype << 24U));
        }
        if (output->role != M3_GRAPH_TEMPORARY ||
            (g->last_use[node->output] != M3_FUSE_NO_NODE &&
             g->last_use[node->output] >= end)) {
            m3_fuse_emit(w, (uint32_t)M3_HIP_PROGRAM_STORE |
                                (destination << 4U) |
                                (m3_fuse_operand_index(g, w, &group,
                                                       node->output, false)
                                 << 8U));
        }
    }
    if (w->failed) {
        return;
    }
    group.operand_count = plan->operand_count - group.operand_first;
    for (i = 0U; i < group.operand_count; ++i) {
        group.period_count +=
            plan->operands[group.operand_first + i].period != 0U ? 1U : 0U;
    }
    group.code_count = plan->code_count - group.code_first;
    if (!m3_fuse_grow((void **)&plan->groups, &w->group_capacity,
                      plan->group_count + 1U, sizeof(*plan->groups))) {
        w->failed = true;
        return;
    }
    plan->groups[plan->group_count++] = group;
}

void m3_fuse_plan_free(m3_fuse_plan *plan)
{
    if (plan == NULL) {
        return;
    }
    free(plan->groups);
    free(plan->operands);
    free(plan->code);
    (void)memset(plan, 0, sizeof(*plan));
}

m3_status m3_fuse_plan_build(const m3_fuse_value *values, size_t value_count,
                             const m3_fuse_node *nodes, size_t node_count,
                             m3_fuse_plan *plan, m3_error *error)
{
    m3_fuse_graph g;
    m3_fuse_writer w;
    size_t n;
    size_t v;

    if (plan == NULL || (value_count != 0U && values == NULL) ||
        (node_count != 0U && nodes == NULL)) {
        return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                            "fusion plan arguments are incomplete");
    }
    (void)memset(plan, 0, sizeof(*plan));
    for (n = 0U; n < node_count; ++n) {
        const m3_fuse_node *node = &nodes[n];
        bool left_read = !node->eligible;
        bool right_read = !node->eligible;
        uint32_t k;

        if (node->read_count > M3_FUSE_MAX_READS ||
            node->left >= value_count || node->right >= value_count ||
            node->output >= value_count) {
            return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                                "fusion node %zu names a value out of range",
                                n);
        }
        for (k = 0U; k < node->read_count; ++k) {
            if (node->reads[k] >= value_count) {
                return m3_error_set(error, M3_STATUS_OUT_OF_RANGE,
                                    "fusion node %zu reads a value out of "
                                    "range",
                                    n);
            }
            left_read = left_read || node->reads[k] == node->left;
            right_read = right_read || node->reads[k] == node->right;
        }
        if (!left_read || !right_read) {
            return m3_error_set(error, M3_STATUS_INVALID_ARGUMENT,
                                "fusion node %zu does not list its operands "
                                "among its reads",
                                n);
        }
    }
    (void)memset(&g, 0, sizeof(g));
    g.values = values;
    g.value_count = value_count;
    g.nodes = nodes;
    g.node_count = node_count;
    g.producer = malloc((value_count == 0U ? 1U : value_count) *
                        sizeof(*g.producer));
    g.last_use = malloc((value_count == 0U ? 1U : value_count) *
                        sizeof(*g.last_use));
    if (g.producer == NULL || g.last_use == NULL) {
        free(g.producer);
        free(g.last_use);
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate fusion planner state");
    }
    for (v = 0U; v < value_count; ++v) {
        g.producer[v] = M3_FUSE_NO_NODE;
        g.last_use[v] = M3_FUSE_NO_NODE;
    }
    for (n = 0U; n < node_count; ++n) {
        uint32_t k;

        for (k = 0U; k < nodes[n].read_count; ++k) {
            g.last_use[nodes[n].reads[k]] = n;
        }
        if (g.producer[nodes[n].output] == M3_FUSE_NO_NODE) {
            g.producer[nodes[n].output] = n;
        }
    }
    (void)memset(&w, 0, sizeof(w));
    w.plan = plan;
    n = 0U;
    while (n < node_count && !w.failed) {
        m3_fuse_registers r;
        size_t end = n;
        size_t budget_words = 0U;
        /* operand budget: distinct operands read from memory, values
         * produced in the group that are not TEMPORARY (always stored),
         * and at most one store per register for values still live when
         * the group ends */
        uint32_t externals[M3_HIP_PROGRAM_MAX_OPERANDS];
        size_t external_count = 0U;
        size_t kept = 0U;
        uint32_t i;

        if (!m3_fuse_candidate(&g, n)) {
            n += 1U;
            continue;
        }
        r.first = n;
        r.count = values[nodes[n].output].element_count;
        for (i = 0U; i < M3_FUSE_REGISTERS; ++i) {
            r.holder[i] = M3_FUSE_NONE;
        }
        while (end < node_count && m3_fuse_candidate(&g, end) &&
               values[nodes[end].output].element_count == r.count &&
               budget_words + M3_FUSE_NODE_WORDS <=
                   M3_HIP_PROGRAM_MAX_WORDS) {
            const uint32_t operands[2] = {nodes[end].left, nodes[end].right};
            size_t added = 0U;
            uint32_t fresh[2];
            uint32_t held;
            size_t k;

            for (k = 0U; k < 2U; ++k) {
                size_t e;

                if (m3_fuse_in_group(&g, operands[k], n, end) ||
                    (k == 1U && added == 1U && fresh[0] == operands[1])) {
                    continue;
                }
                for (e = 0U; e < external_count; ++e) {
                    if (externals[e] == operands[k]) {
                        break;
                    }
                }
                if (e == external_count) {
                    fresh[added++] = operands[k];
                }
            }
            if (external_count + added + kept +
                    (values[nodes[end].output].role != M3_GRAPH_TEMPORARY
                         ? 1U
                         : 0U) +
                    M3_FUSE_REGISTERS >
                M3_HIP_PROGRAM_MAX_OPERANDS) {
                break;
            }
            if (!m3_fuse_step(&g, &r, end, &held)) {
                break;
            }
            for (k = 0U; k < added; ++k) {
                externals[external_count++] = fresh[k];
            }
            kept += values[nodes[end].output].role != M3_GRAPH_TEMPORARY
                        ? 1U
                        : 0U;
            budget_words += M3_FUSE_NODE_WORDS;
            end += 1U;
        }
        while (end - n >= 2U && m3_fuse_group_races(&g, n, end)) {
            end -= 1U;
        }
        if (end - n >= 2U) {
            m3_fuse_emit_group(&g, &w, n, end);
        }
        n = end > n ? end : n + 1U;
    }
    free(g.producer);
    free(g.last_use);
    if (w.failed) {
        m3_fuse_plan_free(plan);
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate the fusion plan");
    }
    m3_error_reset(error);
    return M3_STATUS_OK;
}
