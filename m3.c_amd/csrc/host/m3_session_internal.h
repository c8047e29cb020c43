/*
 * m3_session_internal.h - private records of graphs and sessions.
 *
 * A graph is two growable lists: value specs (the caller's descriptor, the
 * metadata derived from it, and an owned copy of constant bytes) and node
 * descriptors, copied as given. A session is compiled from a graph in four
 * layers (m3_session.c):
 *   plan     topology, liveness slots and the arena (m3_plan.c)
 *   views    one contiguous view per value over its slot
 *   nodes    one command per node with the provider that runs it, and
 *            the node's lane: on the GPU, on the CPU over host storage,
 *            or on the CPU over host mirrors of device values (staged)
 *   runs     the list m3_session_run walks, with fused elementwise
 *            programs in place of the nodes they cover (m3_graph_fuse.c)
 */
#ifndef M3_SESSION_INTERNAL_H
#define M3_SESSION_INTERNAL_H

#include "m3_internal.h"

/* ---- graphs ------------------------------------------------------------- */

typedef struct {
    void *items;
    size_t count;
    size_t capacity;
} m3_list;

typedef struct {
    m3_graph_value_desc desc;
    m3_tensor_metadata meta;
    uint8_t *constant; /* owned; NULL until set (or when empty) */
    bool constant_given;
} m3_value_spec;

struct m3_graph {
    m3_list values; /* m3_value_spec */
    m3_list nodes;  /* m3_graph_node_desc */
};

static inline const m3_value_spec *m3_graph_value_at(const m3_graph *graph,
                                                     size_t index)
{
    return (const m3_value_spec *)graph->values.items + index;
}

static inline const m3_graph_node_desc *m3_graph_node_at(
    const m3_graph *graph, size_t index)
{
    return (const m3_graph_node_desc *)graph->nodes.items + index;
}

/* ---- the liveness plan (m3_plan.c) -------------------------------------- */

#define M3_NO_NODE SIZE_MAX

typedef struct {
    size_t count;
    size_t *slot_of;    /* per value */
    size_t *slot_bytes; /* per slot, the size of the value that opened it */
    size_t slot_count;
    size_t plain_bytes; /* sum of slot sizes (allocated_bytes) */
    size_t arena_bytes; /* sum of slot sizes rounded up to the granule */
} m3_plan;

/* Checks the data flow of `graph` in node order (operands present, read
 * only after they are produced, written once, never an INPUT or
 * CONSTANT), then assigns slots: INPUT, CONSTANT and OUTPUT values own one
 * each; a TEMPORARY takes the smallest slot whose last reader ran before
 * its producer and that is large enough, else opens one. */
m3_status m3_plan_build(const m3_graph *graph, m3_plan *plan,
                        m3_error *error);
void m3_plan_release(m3_plan *plan);

/* ---- sessions ----------------------------------------------------------- */

typedef enum {
    M3_LANE_GPU = 0,
    M3_LANE_CPU,    /* CPU provider, operands in host storage */
    M3_LANE_STAGED  /* CPU provider, operands mirrored from the device */
} m3_lane;

/* Host mirror of a device value, for staged nodes. `fresh` is set while
 * the mirror holds the value's current bits in this run. */
typedef struct {
    m3_storage *storage; /* NULL for values no staged node touches */
    bool fresh;
    bool keep;      /* CONSTANT: mirrored once, fresh in every run */
    bool gpu_reads; /* a node on the GPU reads the value */
} m3_mirror;

struct m3_session {
    m3_session_options options;
    m3_backend *backend;
    size_t value_count;
    size_t node_count;
    m3_value_spec *values;   /* copies of the graph's specs (no constants) */
    m3_graph_node_desc *nodes; /* copies of the graph's nodes */
    m3_plan plan;
    m3_storage **slots;      /* plan.slot_count */
    m3_tensor_view *views;   /* per value */
    m3_command *commands;    /* per node, over `views` (or mirrors) */
    m3_provider_kind *providers;
    m3_lane *lanes;
    /* staging (only when some node is staged) */
    m3_backend *mirror_backend; /* host storage for the mirrors */
    m3_mirror *mirrors;         /* per value */
    m3_tensor_view *mirror_viewset; /* per value: its mirror's view, or
                                     * its device view when unmirrored */
    /* run list (m3_graph_fuse.c) */
    m3_command *run_commands;
    m3_provider_kind *run_providers;
    size_t *run_first_node;  /* per run entry: the first node it covers */
    size_t run_count;
    uint32_t *program_words;
    m3_storage *program_storage;
};

m3_status m3_graph_bind_command(const m3_graph_node_desc *description,
                                m3_tensor_view *views, size_t value_count,
                                m3_command *command, m3_error *error);
/* Builds the run list (m3_graph_fuse.c). */
m3_status m3_session_plan_runs(m3_session *session, const m3_graph *graph,
                               m3_error *error);
void m3_session_free_runs(m3_session *session);

#endif
