/*
 * TEST INFRASTRUCTURE ONLY -- CPU restatement ("oracle") of the reference's
 * temporal neighbour block and recent-k sampler. Only tests/, smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as a checker.
 * The product path never links or calls it.
 *
 * Follows:
 *   get_neighbors                 vendor/bts_sampler/sampler/include/neighbors.h:209-284
 *     per-node IN-neighbour lists keyed by col (dst), in input (event) order
 *     (:243-267); deg = list length (:277-280).
 *   _with_before_layer ("recent") vendor/bts_sampler/sampler/include/sampler.h:213-261,360-384
 *     end = std::lower_bound(ts[n], t)  (:242), start = max(0, end-k) (:252),
 *     window emitted oldest->newest with src_index=i, delta_ts=t-ts,
 *     sample_weight = c-start (:253-260); output concatenated in root order.
 *   _with_before                  sampler.h:393-399 (hop l+1 queries = hop l
 *     (sample_nodes, sample_nodes_ts)) -- driven from sampler_oracle.py.
 *
 * The CSR stores the lists contiguously: indptr[N+1], and per entry the
 * neighbour id, edge id and timestamp, which is the same content as the
 * reference's vector<vector<int64>> triple.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <omp.h>

void orc_set_threads(int n) { if (n > 0) omp_set_num_threads(n); }
int orc_get_threads(void) { return omp_get_max_threads(); }

/* Stable counting sort of events by col; equivalent to the reference's
 * push_back loops in event order (neighbors.h:243-267).
 * Returns 0, or -1 when an endpoint lies outside [0, num_nodes). */
int orc_tcsr_build(int64_t num_nodes, int64_t num_edges,
                   const int64_t *row, const int64_t *col,
                   const int64_t *eid, const int64_t *ts,
                   int64_t *indptr, int64_t *nbr, int64_t *eid_out,
                   int64_t *ts_out)
{
    for (int64_t i = 0; i < num_edges; ++i) {
        if (col[i] < 0 || col[i] >= num_nodes || row[i] < 0 || row[i] >= num_nodes)
            return -1;
    }
    memset(indptr, 0, sizeof(int64_t) * (size_t)(num_nodes + 1));
    for (int64_t i = 0; i < num_edges; ++i) indptr[col[i] + 1] += 1;
    for (int64_t n = 0; n < num_nodes; ++n) indptr[n + 1] += indptr[n];
    int64_t *cursor = (int64_t *)malloc(sizeof(int64_t) * (size_t)(num_nodes > 0 ? num_nodes : 1));
    if (!cursor) return -2;
    memcpy(cursor, indptr, sizeof(int64_t) * (size_t)num_nodes);
    for (int64_t i = 0; i < num_edges; ++i) {
        int64_t p = cursor[col[i]]++;
        nbr[p] = row[i];
        eid_out[p] = eid ? eid[i] : i;
        ts_out[p] = ts[i];
    }
    free(cursor);
    return 0;
}

/* The same probe sequence as libstdc++'s std::lower_bound, so that the result
 * is identical even if a node's timestamps are not sorted. */
static int64_t lower_bound_i64(const int64_t *a, int64_t len, int64_t v)
{
    int64_t first = 0;
    while (len > 0) {
        int64_t half = len >> 1;
        int64_t mid = first + half;
        if (a[mid] < v) { first = mid + 1; len = len - half - 1; }
        else len = half;
    }
    return first;
}

/* Per query: window [begin, begin+cnt) of the CSR (absolute positions).
 * Returns 0, or -1 on an out-of-range query node. */
int orc_recent_search(const int64_t *indptr, const int64_t *ts, int64_t num_nodes,
                      int64_t nq, const int64_t *q_node, const int64_t *q_ts,
                      int fanout, int64_t *begin, int64_t *cnt)
{
    int bad = 0;
#pragma omp parallel for schedule(static) reduction(|:bad)
    for (int64_t i = 0; i < nq; ++i) {
        int64_t n = q_node[i];
        if (n < 0 || n >= num_nodes) { bad = 1; begin[i] = 0; cnt[i] = 0; continue; }
        int64_t lo = indptr[n], deg = indptr[n + 1] - lo;
        int64_t end = lower_bound_i64(ts + lo, deg, q_ts[i]);
        int64_t start = end - fanout; if (start < 0) start = 0;
        begin[i] = lo + start;
        cnt[i] = end - start;
    }
    return bad ? -1 : 0;
}

/* Fill the concatenated outputs given offsets = exclusive scan of cnt. */
void orc_recent_fill(const int64_t *nbr, const int64_t *eid, const int64_t *ts,
                     int64_t nq, const int64_t *q_ts, const int64_t *begin,
                     const int64_t *cnt, const int64_t *offsets,
                     int64_t *src_index, int64_t *out_nodes, int64_t *out_ts,
                     int64_t *out_eid, int64_t *out_dt, float *out_weight)
{
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < nq; ++i) {
        int64_t o = offsets[i], b = begin[i];
        for (int64_t j = 0; j < cnt[i]; ++j) {
            src_index[o + j] = i;
            out_nodes[o + j] = nbr[b + j];
            out_ts[o + j] = ts[b + j];
            out_eid[o + j] = eid[b + j];
            out_dt[o + j] = q_ts[i] - ts[b + j];
            out_weight[o + j] = (float)j;
        }
    }
}
