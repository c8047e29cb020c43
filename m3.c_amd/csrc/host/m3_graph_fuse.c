/*
 * m3_graph_fuse.c - the list m3_session_run executes.
 *
 * The run list is the session's commands in node order, except that each
 * group the fusion planner (m3_fuse.c) forms from consecutive ADD/SUB/
 * MUL/DIV and float CAST/COPY nodes on the HIP provider becomes one
 * elementwise-program command. The planner works on value indices; here operands become device
 * addresses of the values' slots, and all programs of the session are
 * written once, at session creation, into one backend storage next to the
 * arena. Node providers, slots and allocated_bytes are those of the
 * unfused plan: fusion changes which intermediate values are written, not
 * where values live.
 *
 * Fusion is on for HIP sessions unless the environment variable
 * M3_HIP_FUSION is "0" when the session is created; then every node runs
 * as its own command (used to compare the two paths).
 */
#include "m3_session_internal.h"

#include "m3_fuse.h"
#include "m3_hip.h"

#include <stdlib.h>
#include <string.h>

#define M3_PROGRAM_ALIGNMENT 256U

static bool m3_fusion_enabled(const m3_session *session)
{
    const char *setting = getenv("M3_HIP_FUSION");
    m3_backend_info info;

    if (setting != NULL && strcmp(setting, "0") == 0) {
        return false;
    }
    return m3_backend_get_info(session->backend, &info, NULL) ==
               M3_STATUS_OK &&
           info.kind == M3_BACKEND_HIP;
}

static void m3_runs_unfused(m3_session *session)
{
    size_t n;

    for (n = 0U; n < session->node_count; ++n) {
        session->run_commands[n] = session->commands[n];
        session->run_providers[n] = session->providers[n];
        session->run_first_node[n] = n;
    }
    session->run_count = session->node_count;
}

/* Device address and dtype of value v's view, as two program words; false
 * when the address does not have the alignment its use needs or does not
 * fit beside the dtype bits. */
static bool m3_operand_words(const m3_session *session, uint32_t value,
                             bool scalar, uint32_t *low, uint32_t *high)
{
    const m3_tensor_view *view = &session->views[value];
    const m3_dtype dtype = view->metadata.dtype;
    uint64_t address =
        (uint64_t)(uintptr_t)m3_storage_device_data(view->storage) +
        (uint64_t)view->byte_offset;
    uint64_t alignment = scalar ? (dtype == M3_DTYPE_F32 ? 4U : 2U)
                                : (dtype == M3_DTYPE_F32 ? 16U : 8U);

    if (address == 0U || (address & (alignment - 1U)) != 0U ||
        (address >> 62U) != 0U) {
        return false;
    }
    *low = (uint32_t)address | (scalar ? 1U : 0U);
    *high = (uint32_t)(address >> 32U) | ((uint32_t)dtype << 30U);
    return true;
}

/* Words of a group's program: header, operand table, period table and
 * instructions. */
static size_t m3_program_word_count(const m3_fuse_group *group)
{
    return M3_HIP_PROGRAM_HEADER_WORDS + 2U * group->operand_count +
           2U * group->period_count + group->code_count;
}

/* True when the operand's shape, leading ones removed, is the output's
 * trailing dimensions: under the right-aligned broadcast of the binary
 * operations, output element e then reads operand element e mod its
 * element count. */
static bool m3_trailing_broadcast(const m3_tensor_metadata *operand,
                                  const m3_tensor_metadata *output)
{
    size_t first = 0U;
    size_t kept;
    size_t i;

    while (first < operand->rank && operand->shape[first] == 1U) {
        first += 1U;
    }
    kept = operand->rank - first;
    if (kept > output->rank) {
        return false;
    }
    for (i = 0U; i < kept; ++i) {
        if (operand->shape[first + i] !=
            output->shape[output->rank - kept + i]) {
            return false;
        }
    }
    return true;
}

/* Writes the programs of all groups into session->program_words; false
 * when an operand address is unusable (the session then runs unfused). */
static bool m3_write_programs(m3_session *session, const m3_fuse_plan *plan,
                              size_t *offsets)
{
    size_t at = 0U;
    size_t gi;

    for (gi = 0U; gi < plan->group_count; ++gi) {
        const m3_fuse_group *group = &plan->groups[gi];
        uint32_t *words = session->program_words + at;
        uint32_t *periods = words + M3_HIP_PROGRAM_HEADER_WORDS +
                            2U * group->operand_count;
        size_t p;

        offsets[gi] = at;
        (void)memset(words, 0, M3_HIP_PROGRAM_HEADER_WORDS * sizeof(*words));
        words[0] = M3_HIP_PROGRAM_MAGIC;
        words[1] = (uint32_t)group->operand_count;
        words[2] = (uint32_t)group->code_count;
        words[3] = (uint32_t)group->element_count;
        words[4] = (uint32_t)(group->element_count >> 32U);
        words[5] = (uint32_t)group->period_count;
        for (p = 0U; p < group->operand_count; ++p) {
            const m3_fuse_operand *operand =
                &plan->operands[group->operand_first + p];

            if (!m3_operand_words(
                    session, operand->value, operand->scalar,
                    &words[M3_HIP_PROGRAM_HEADER_WORDS + 2U * p],
                    &words[M3_HIP_PROGRAM_HEADER_WORDS + 2U * p + 1U])) {
                return false;
            }
            if (operand->period != 0U) {
                periods[0] = (uint32_t)p;
                periods[1] = (uint32_t)operand->period;
                periods += 2U;
            }
        }
        (void)memcpy(periods, plan->code + group->code_first,
                     group->code_count * sizeof(*words));
        at += m3_program_word_count(group);
    }
    return true;
}

static void m3_runs_fused(m3_session *session, const m3_fuse_plan *plan,
                          const size_t *offsets)
{
    size_t n = 0U;
    size_t gi = 0U;
    size_t out = 0U;

    while (n < session->node_count) {
        if (gi < plan->group_count && plan->groups[gi].first_node == n) {
            const m3_fuse_group *group = &plan->groups[gi];
            m3_command *command = &session->run_commands[out];
            m3_op_elementwise_program *program =
                &command->descriptor.elementwise_program;

            (void)memset(command, 0, sizeof(*command));
            command->kind = M3_OP_ELEMENTWISE_PROGRAM;
            program->commands = &session->commands[n];
            program->command_count = group->node_count;
            program->words = session->program_words + offsets[gi];
            program->word_count = m3_program_word_count(group);
            program->storage = session->program_storage;
            program->byte_offset = offsets[gi] * sizeof(uint32_t);
            session->run_providers[out] = session->providers[n];
            session->run_first_node[out] = n;
            out += 1U;
            n += group->node_count;
            gi += 1U;
            continue;
        }
        session->run_commands[out] = session->commands[n];
        session->run_providers[out] = session->providers[n];
        session->run_first_node[out] = n;
        out += 1U;
        n += 1U;
    }
    session->run_count = out;
}

/* Compiles every program's kernel now, so that the session's first run
 * does not (a failure only leaves that program to the interpreter). */
static void m3_prepare_programs(m3_session *session,
                                const m3_fuse_plan *plan,
                                const size_t *offsets)
{
    m3_hip_device *device = m3_backend_hip_device(session->backend);
    size_t gi;

    for (gi = 0U; device != NULL && gi < plan->group_count; ++gi) {
        const m3_fuse_group *group = &plan->groups[gi];

        (void)m3_hip_prepare_program(device,
                                     session->program_words + offsets[gi],
                                     m3_program_word_count(group), NULL, 0U);
    }
}

m3_status m3_session_plan_runs(m3_session *session, const m3_graph *graph,
                               m3_error *error)
{
    size_t count = session->node_count == 0U ? 1U : session->node_count;
    size_t values = session->value_count == 0U ? 1U : session->value_count;
    m3_fuse_value *fuse_values = NULL;
    m3_fuse_node *fuse_nodes = NULL;
    m3_fuse_plan plan;
    size_t *offsets = NULL;
    size_t total = 0U;
    size_t n;
    size_t v;
    m3_status status;

    (void)memset(&plan, 0, sizeof(plan));
    (void)graph;
    session->run_commands = calloc(count, sizeof(*session->run_commands));
    session->run_providers = calloc(count, sizeof(*session->run_providers));
    session->run_first_node = calloc(count,
                                     sizeof(*session->run_first_node));
    if (session->run_commands == NULL || session->run_providers == NULL ||
        session->run_first_node == NULL) {
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate the session run list");
    }
    m3_runs_unfused(session);
    if (session->node_count < 2U || !m3_fusion_enabled(session)) {
        return M3_STATUS_OK;
    }
    fuse_values = calloc(values, sizeof(*fuse_values));
    fuse_nodes = calloc(count, sizeof(*fuse_nodes));
    if (fuse_values == NULL || fuse_nodes == NULL) {
        free(fuse_values);
        free(fuse_nodes);
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate fusion planner input");
    }
    for (v = 0U; v < session->value_count; ++v) {
        const m3_tensor_view *view = &session->views[v];

        fuse_values[v].role = session->values[v].desc.role;
        fuse_values[v].dtype = session->values[v].meta.dtype;
        fuse_values[v].element_count =
            (uint64_t)session->values[v].meta.element_count;
        fuse_values[v].address =
            (uint64_t)(uintptr_t)m3_storage_device_data(view->storage) +
            (uint64_t)view->byte_offset;
        fuse_values[v].byte_count =
            (uint64_t)session->values[v].meta.byte_count;
    }
    for (n = 0U; n < session->node_count; ++n) {
        const m3_graph_node_desc *node = &session->nodes[n];
        size_t i;

        fuse_nodes[n].kind = node->kind;
        /* every value the node reads counts for liveness, fused or not */
        for (i = 0U; i < M3_GRAPH_NODE_INPUT_CAPACITY &&
                     i < M3_FUSE_MAX_READS &&
                     node->inputs[i] != M3_GRAPH_VALUE_NONE;
             ++i) {
            fuse_nodes[n].reads[i] = (uint32_t)node->inputs[i];
        }
        fuse_nodes[n].read_count = (uint32_t)i;
        fuse_nodes[n].output = (uint32_t)node->outputs[0];
        fuse_nodes[n].left = fuse_nodes[n].output;
        fuse_nodes[n].right = fuse_nodes[n].output;
        if (m3_op_binary_of(&session->commands[n]) != NULL) {
            const m3_tensor_metadata *output =
                &session->values[node->outputs[0]].meta;

            fuse_nodes[n].left = (uint32_t)node->inputs[0];
            fuse_nodes[n].right = (uint32_t)node->inputs[1];
            fuse_nodes[n].output = (uint32_t)node->outputs[0];
            fuse_nodes[n].eligible =
                session->providers[n] == M3_PROVIDER_HIP;
            fuse_nodes[n].left_trailing = m3_trailing_broadcast(
                &session->values[node->inputs[0]].meta, output);
            fuse_nodes[n].right_trailing = m3_trailing_broadcast(
                &session->values[node->inputs[1]].meta, output);
        } else if (node->kind == M3_OP_CAST || node->kind == M3_OP_COPY) {
            fuse_nodes[n].left = (uint32_t)node->inputs[0];
            fuse_nodes[n].right = (uint32_t)node->inputs[0];
            fuse_nodes[n].output = (uint32_t)node->outputs[0];
            fuse_nodes[n].eligible =
                session->providers[n] == M3_PROVIDER_HIP;
        }
    }
    status = m3_fuse_plan_build(fuse_values, session->value_count,
                                fuse_nodes, session->node_count, &plan,
                                error);
    free(fuse_values);
    free(fuse_nodes);
    if (status != M3_STATUS_OK || plan.group_count == 0U) {
        m3_fuse_plan_free(&plan);
        return status;
    }
    for (n = 0U; n < plan.group_count; ++n) {
        total += m3_program_word_count(&plan.groups[n]);
    }
    session->program_words = malloc(total * sizeof(uint32_t));
    offsets = malloc(plan.group_count * sizeof(*offsets));
    if (session->program_words == NULL || offsets == NULL) {
        free(offsets);
        m3_fuse_plan_free(&plan);
        return m3_error_set(error, M3_STATUS_OUT_OF_MEMORY,
                            "cannot allocate elementwise programs");
    }
    if (!m3_write_programs(session, &plan, offsets)) {
        free(offsets);
        m3_fuse_plan_free(&plan);
        free(session->program_words);
        session->program_words = NULL;
        return M3_STATUS_OK;
    }
    status = m3_storage_allocate(session->backend, total * sizeof(uint32_t),
                                 M3_PROGRAM_ALIGNMENT,
                                 &session->program_storage, error);
    if (status == M3_STATUS_OK) {
        status = m3_storage_write(session->program_storage, 0U,
                                  session->program_words,
                                  total * sizeof(uint32_t), error);
    }
    if (status == M3_STATUS_OK) {
        m3_runs_fused(session, &plan, offsets);
        m3_prepare_programs(session, &plan, offsets);
    }
    free(offsets);
    m3_fuse_plan_free(&plan);
    return status;
}

void m3_session_free_runs(m3_session *session)
{
    m3_storage_free(session->program_storage);
    session->program_storage = NULL;
    free(session->program_words);
    free(session->run_commands);
    free(session->run_providers);
    free(session->run_first_node);
    session->program_words = NULL;
    session->run_commands = NULL;
    session->run_providers = NULL;
    session->run_first_node = NULL;
    session->run_count = 0U;
}
