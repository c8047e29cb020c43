/*
 * m3_graph_internal.h - graph and session state shared by the graph files.
 *
 * The shapes of these records follow src/m3_graph_internal.h:10-88 of the
 * reference; Core ML nodes do not exist in this library, so every node is
 * a regular node.
 */
#ifndef M3_GRAPH_INTERNAL_H
#define M3_GRAPH_INTERNAL_H

#include "m3_internal.h"

typedef struct {
    m3_graph_value_desc description;
    m3_tensor_metadata metadata;
    void *constant_data;
    size_t constant_size;
    bool constant_set;
} m3_graph_value;

struct m3_graph {
    m3_graph_value *values;
    size_t value_count;
    size_t value_capacity;
    m3_graph_node_desc *nodes;
    size_t node_count;
    size_t node_capacity;
};

typedef struct {
    m3_graph_value_desc description;
    m3_tensor_metadata metadata;
    size_t slot;
} m3_session_value;

typedef struct {
    m3_storage *storage;
    size_t byte_count;
} m3_session_slot;

struct m3_session {
    m3_backend *backend;
    m3_session_options options;
    m3_session_value *values;
    m3_tensor_view *views;
    size_t value_count;
    m3_session_slot *slots;
    size_t slot_count;
    m3_provider_kind *providers;
    m3_command *commands;
    size_t node_count;
    /* What m3_session_run executes: the commands, with each fused run of
     * ADD/SUB/MUL/DIV commands replaced by one elementwise-program command
     * whose words live in program_words (host) and program_storage. */
    m3_command *run_commands;
    m3_provider_kind *run_providers;
    size_t run_count;
    uint32_t *program_words;
    m3_storage *program_storage;
    void *scratch;
    size_t scratch_capacity;
    size_t allocated_bytes;
};

m3_status m3_graph_bind_command(const m3_graph_node_desc *description,
                                m3_tensor_view *views, size_t value_count,
                                m3_command *command, m3_error *error);
/* Builds run_commands/run_providers (m3_graph_fuse.c). */
m3_status m3_session_plan_runs(m3_session *session, const m3_graph *graph,
                               m3_error *error);
void m3_session_free_runs(m3_session *session);

#endif
