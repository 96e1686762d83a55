// A declaration subset of ggml's internal header ggml-impl.h (which backends built in ggml's tree include): its log
// entry point and the macro the MI355X backend logs errors with, and the graph internals a fusing backend reads --
// the layout of ggml_cgraph, its visited-tensor hash set and the per-tensor use counts ggml_build_forward_expand
// keeps over the whole graph (a graph view, as ggml_backend_sched hands a backend one split of it, shares them).
#pragma once

#include "ggml.h"

#ifdef __cplusplus
extern "C" {
#endif

GGML_API void ggml_log_internal(enum ggml_log_level level, const char *format, ...);

// ggml's bit set: bit i of word i >> 5.
typedef uint32_t ggml_bitset_t;

static inline bool ggml_bitset_get(const ggml_bitset_t *bitset, size_t i) {
    return (bitset[i >> 5] >> (i & 31)) & 1u;
}

// Open-addressing set of tensors keyed by address: slot h(t) = (address >> 4) mod size, then the next slots in turn.
struct ggml_hash_set {
    size_t size;
    ggml_bitset_t *used;       // which slots hold a key
    struct ggml_tensor **keys;  // the key of each used slot
};

#define GGML_HASHSET_FULL ((size_t)-1)

static inline size_t ggml_hash(const struct ggml_tensor *p) { return (size_t)(uintptr_t)p >> 4; }

// The slot of key, or of the first free slot probed on the way to it (GGML_HASHSET_FULL: every slot taken by others).
static inline size_t ggml_hash_find(const struct ggml_hash_set *hash_set, const struct ggml_tensor *key) {
    const size_t h = ggml_hash(key) % hash_set->size;
    size_t i = h;
    while (ggml_bitset_get(hash_set->used, i) && hash_set->keys[i] != key) {
        i = (i + 1) % hash_set->size;
        if (i == h) return GGML_HASHSET_FULL;
    }
    return i;
}

enum ggml_cgraph_eval_order {
    GGML_CGRAPH_EVAL_ORDER_LEFT_TO_RIGHT = 0,
    GGML_CGRAPH_EVAL_ORDER_RIGHT_TO_LEFT,
    GGML_CGRAPH_EVAL_ORDER_COUNT
};

struct ggml_cgraph {
    int size;     // capacity of nodes / leafs (0 for a view)
    int n_nodes;
    int n_leafs;
    struct ggml_tensor **nodes;
    struct ggml_tensor **grads;
    struct ggml_tensor **grad_accs;
    struct ggml_tensor **leafs;
    int32_t *use_counts;  // per hash slot: how many times the whole graph's nodes name the tensor as a source
    struct ggml_hash_set visited_hash_set;
    enum ggml_cgraph_eval_order order;
};

// Nodes [i0, i1) of a graph, sharing its use counts and hash set (what ggml_backend_sched computes a split as). The
// backend does not call it (ggml-base need not export it); the test host provides it.
struct ggml_cgraph ggml_graph_view(struct ggml_cgraph *cgraph, int i0, int i1);

// How many sources, over the whole graph the node came from, name node node_idx (0 for a tensor no node reads).
static inline int ggml_node_get_use_count(const struct ggml_cgraph *cgraph, int node_idx) {
    const struct ggml_tensor *node = cgraph->nodes[node_idx];
    const size_t pos = ggml_hash_find(&cgraph->visited_hash_set, node);
    if (pos == GGML_HASHSET_FULL || !ggml_bitset_get(cgraph->visited_hash_set.used, pos)) return 0;
    return cgraph->use_counts[pos];
}

#ifdef __cplusplus
}
#endif

#define GGML_LOG_ERROR(...) ggml_log_internal(GGML_LOG_LEVEL_ERROR, __VA_ARGS__)
#define GGML_LOG_WARN(...) ggml_log_internal(GGML_LOG_LEVEL_WARN, __VA_ARGS__)
