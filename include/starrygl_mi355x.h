/*
 * starrygl_mi355x.h -- C ABI of the MI355X-native CTDG training-step library
 * (libstarrygl_mi355x.so, HIP kernels for gfx950).
 *
 * Conventions
 *   - Every pointer argument is DEVICE memory unless its comment says "host".
 *   - Every entry point returns 0 (SGL_OK) or an SGL_ERR_* code and then sets a
 *     thread-local message readable with sgl_last_error().
 *   - Work is enqueued on `stream` and returns without synchronising. Device
 *     side data errors (an id out of range) are reported through `err_flag`, a
 *     caller-owned device int32 that kernels OR bits into (SGL_DERR_*); the
 *     caller reads it whenever it synchronises. Kernels never access memory
 *     outside the declared extents, whatever the ids say.
 *   - Scratch memory is supplied by the caller as `workspace` of at least the
 *     size returned by the matching *_workspace_bytes() query.
 *   - The library allocates no device memory of its own.
 */
#ifndef STARRYGL_MI355X_H
#define STARRYGL_MI355X_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGL_ABI_VERSION 1

#define SGL_OK 0
#define SGL_ERR_INVALID 1   /* bad argument (host-checked) */
#define SGL_ERR_HIP 2       /* HIP runtime error */
#define SGL_ERR_WORKSPACE 3 /* workspace smaller than the query says */

/* bits OR-ed into err_flag by kernels */
#define SGL_DERR_NODE_RANGE 1 /* a node id outside [0, num_nodes) */
#define SGL_DERR_EID_RANGE 2  /* an edge id outside [0, 2^31) */

/* (8) version / ABI query. */
int sgl_abi_version(void);
const char *sgl_last_error(void);

/* ---------------------------------------------------------------------------
 * (1) Temporal CSR build.
 * Replaces get_neighbors(graph_name, row, col, num_nodes, is_distinct, eid,
 * dist_eid, edge_weight, time)   vendor/bts_sampler/sampler/include/neighbors.h:209-284
 * (bound at vendor/bts_sampler/sampler/export.cpp:13-15, called from
 * native/bts_sampler.py:19-40).
 *
 * Builds per-node IN-neighbour lists keyed by col (dst), in input (event)
 * order: entry j of node n's list is the j-th event with col == n. Output is
 * a CSR: indptr[N+1] (int64), and per entry nbr (=row, int32), eid (int32)
 * and ts (int64). eid == NULL means eid[i] = i.
 * Limits: num_nodes < 2^31, num_edges < 2^31.
 * ------------------------------------------------------------------------- */
size_t sgl_tcsr_workspace_bytes(int64_t num_nodes, int64_t num_edges);
int sgl_tcsr_build(int64_t num_nodes, int64_t num_edges, const int64_t *row,
                   const int64_t *col, const int64_t *eid, const int64_t *ts,
                   int64_t *indptr, int32_t *nbr, int32_t *eid_out,
                   int64_t *ts_out, void *workspace, size_t workspace_bytes,
                   int32_t *err_flag, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (2) Recent-k temporal sampling, one hop (one kernel).
 * Replaces ParallelSampler::neighbor_sample_from_nodes with policy "recent"
 * (vendor/bts_sampler/sampler/include/sampler.h:69-90 -> _with_before_layer
 * :213-391; bound at export.cpp:73-79, called from native/bts_sampler.py:77-82).
 *
 * For query i = (node n, time t): end = lower_bound(ts[n's list], t) (the
 * count of entries with ts < t for a time-sorted list; the same probe
 * sequence as std::lower_bound otherwise), start = max(0, end - fanout).
 * Output is PADDED: out_cnt[i] = end - start, and row i of the out_* arrays
 * (entries [i*fanout, i*fanout + out_cnt[i])) holds the window oldest->newest:
 * nbr (int32), eid (int32), dt = float32(t - ts) rounded to nearest even, and,
 * if out_ts != NULL, the entry's int64 timestamp (the next hop's query time,
 * sampler.h:396-397). Entries past out_cnt[i] are left untouched.
 * out_* arrays hold num_queries * fanout entries; out_cnt num_queries.
 *
 * q_node is int64 when q_node_is_i64 != 0, else int32. If q_valid_cnt is not
 * NULL, query i is sampled only when (i % q_stride) < q_valid_cnt[i / q_stride]
 * (so a padded previous hop can be the query list; q_valid_cnt then holds
 * ceil(num_queries / q_stride) entries); other queries get out_cnt = 0.
 * ------------------------------------------------------------------------- */
int sgl_recent_sample(const int64_t *indptr, const int32_t *nbr,
                      const int32_t *eid, const int64_t *ts, int64_t num_nodes,
                      const void *q_node, int q_node_is_i64,
                      const int64_t *q_ts, int64_t num_queries,
                      const int32_t *q_valid_cnt, int32_t q_stride,
                      int32_t fanout, int32_t *out_cnt, int32_t *out_nbr,
                      int32_t *out_eid, float *out_dt, int64_t *out_ts,
                      int32_t *err_flag, hipStream_t stream);

/* Padded -> the reference's concatenated layout (TemporalGraphBlock order:
 * root order, each window oldest->newest; output.h:4-30). out_ptr[Q+1] is the
 * exclusive scan of cnt, entry j of window i lands at out_ptr[i] + j. The
 * reference's src_index[j] is the i with out_ptr[i] <= j < out_ptr[i+1] and
 * its sample_weight[j] is j - out_ptr[i]. out_ts/pad_ts may be NULL. */
size_t sgl_compact_workspace_bytes(int64_t num_queries);
int sgl_recent_compact(int64_t num_queries, int32_t fanout, const int32_t *cnt,
                       const int32_t *pad_nbr, const int32_t *pad_eid,
                       const float *pad_dt, const int64_t *pad_ts,
                       int64_t *out_ptr, int32_t *out_nbr, int32_t *out_eid,
                       float *out_dt, int64_t *out_ts, void *workspace,
                       size_t workspace_bytes, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* STARRYGL_MI355X_H */
