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
 *   - The library allocates no device memory of its own (one static scratch
 *     array, see sgl_recent_compact_noalloc).
 */
#ifndef STARRYGL_MI355X_H
#define STARRYGL_MI355X_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SGL_ABI_VERSION 22

#define SGL_OK 0
#define SGL_ERR_INVALID 1   /* bad argument (host-checked) */
#define SGL_ERR_HIP 2       /* HIP runtime error */
#define SGL_ERR_WORKSPACE 3 /* workspace smaller than the query says */

/* bits OR-ed into err_flag by kernels */
#define SGL_DERR_NODE_RANGE 1 /* a node id outside [0, num_nodes) */
#define SGL_DERR_EID_RANGE 2  /* an edge id outside [0, 2^31) */
#define SGL_DERR_STALE_NODE_BITS 4 /* sgl_batch_prepare found node bits set before it marked its batch
                                    * (the previous preparation's commit did not run): the batch is
                                    * given no roots and the bitmap is cleared */

/* (8) version / ABI query. */
int sgl_abi_version(void);
const char *sgl_last_error(void);
/* The device-visible address of pinned host memory (hipHostGetDevicePointer),
 * so that a kernel can read host-staged inputs in place instead of through a
 * separate copy (the negatives' draws). No reference counterpart: the
 * reference draws and looks up negatives on the host. */
int sgl_host_device_pointer(const void *host, void **device);

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
 * If num_queries_dev is not NULL (a device int64), only queries
 * i < *num_queries_dev are live: launch shapes stay at the capacity
 * num_queries while the live count is known only on the device.
 * ------------------------------------------------------------------------- */
int sgl_recent_sample(const int64_t *indptr, const int32_t *nbr,
                      const int32_t *eid, const int64_t *ts, int64_t num_nodes,
                      const void *q_node, int q_node_is_i64,
                      const int64_t *q_ts, int64_t num_queries,
                      const int64_t *num_queries_dev,
                      const int32_t *q_valid_cnt, int32_t q_stride,
                      int32_t fanout, int32_t *out_cnt, int32_t *out_nbr,
                      int32_t *out_eid, float *out_dt, int64_t *out_ts,
                      int32_t *err_flag, hipStream_t stream);
/* The same over a packed copy of the CSR that the caller makes when every
 * timestamp fits in int32: nbr_eid holds (nbr, eid) pairs ([num_edges][2],
 * 8-byte aligned) and ts the int32 timestamps. Each entry is compared with the
 * int64 query time exactly as its int64 value would be, so the results are
 * identical; a search probe reads half the bytes (32 timestamps per 128-byte
 * line) and a window's ids one contiguous run. fence (may be NULL) holds
 * ts[32 f] for f < ceil(num_edges / 32) and may be given only when every
 * node's list is sorted by time: the queries of more than 32768-query
 * launches then search the fences inside their list first (a small array
 * that stays in cache) and one 32-entry line of ts after it. */
int sgl_recent_sample_packed(const int64_t *indptr, const int32_t *nbr_eid,
                             const int32_t *ts, const int32_t *fence, int64_t num_nodes,
                             const void *q_node, int q_node_is_i64,
                             const int64_t *q_ts, int64_t num_queries,
                             const int64_t *num_queries_dev,
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
/* The same compaction without a workspace argument and without allocating:
 * its scratch (the per-tile count sums and offsets) is a static device array
 * of the library, 1 MiB per GPU, held until the process ends. No counterpart
 * in the reference: it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). Limit: num_queries <= SGL_COMPACT_NOALLOC_MAX_QUERIES (larger
 * calls return SGL_ERR_INVALID). Every call on one GPU uses that GPU's one
 * array, so calls that overlap on a GPU (other streams, other host threads)
 * race; the stream must belong to the current device. Results are identical
 * to sgl_recent_compact's. */
#define SGL_COMPACT_NOALLOC_MAX_QUERIES (1LL << 24)
int sgl_recent_compact_noalloc(int64_t num_queries, int32_t fanout,
                               const int32_t *cnt, const int32_t *pad_nbr,
                               const int32_t *pad_eid, const float *pad_dt,
                               const int64_t *pad_ts, int64_t *out_ptr,
                               int32_t *out_nbr, int32_t *out_eid,
                               float *out_dt, int64_t *out_ts, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (3) Batch preparation.
 * Replaces CTDGOnlineRuntime._prepare (backends/ctdg/runtime/runtime.py:138-144:
 * roots = sorted unique(src ∪ dst), query time int(batch.ts.max())) and the
 * duplicate handling of CTDGMemoryBank._write_slots (memory.py:237-248).
 *
 * node_bits holds W = ceil(N/32) rounded up to a multiple of 4 bitmap words
 * followed by ceil(W/32) rounded up to a multiple of 4 summary words
 * (sgl_node_bits_words(N) in all, 16-byte aligned); word_prefix holds W
 * words. node_bits must be all zero on entry and is left zero (batches of up
 * to 2048 events clear it themselves, larger ones through sgl_memory_commit).
 * Outputs, all device-resident (no host sync):
 *   num_roots / num_roots64: U;  roots[0..U) sorted ascending (int64);
 *   root_ts[0..U) = t_query = trunc(max ts) for every root; ts_max = max ts;
 *   ridx_src/ridx_dst[e] = root index of src[e]/dst[e]; ridx_neg[e] = root
 *   index of neg[e] or -1 when neg[e] is not a root (neg may be NULL);
 *   win_src/win_dst[r] = (order(ts) << 32 | e) of the LAST event in stable
 *   timestamp order in which root r is the src / dst; cnt_src/cnt_dst[r] =
 *   how many events root r is src / dst in; any_edges reset to 0.
 * Arrays indexed by root hold 2*batch entries (the capacity).
 * cursor (device int64, may be NULL): when given, src/dst/ts/neg span the
 * whole event stream and the batch is events [*cursor, *cursor + batch);
 * batch_start (device int64) then receives *cursor and *cursor advances by
 * `batch` (so one captured HIP graph replays the step for consecutive
 * batches). Without a cursor the arrays hold the batch's own events. Event
 * indices e above are relative to the batch start.
 * ------------------------------------------------------------------------- */
int64_t sgl_node_bits_words(int64_t num_nodes);
/* Negative destinations from uniform draws. Replaces the lookup and the
 * collision rule of CTDGOnlineRuntime._negative_sample
 * (backends/ctdg/runtime/runtime.py:124-136) after its torch.randint draw:
 * neg[e] = pool[draw[e]], and when that equals dst[e], pool[(draw[e] + 1)
 * mod pool_size] instead (once, as there). pool is the sorted unique dst
 * pool; draws outside [0, pool_size) set SGL_DERR_NODE_RANGE. draw and neg
 * may be the same array; draw may be pinned host memory read in place
 * (sgl_host_device_pointer). */
int sgl_negatives_from_draws(int64_t n, const int64_t *draw, const int64_t *pool,
                             int64_t pool_size, const int64_t *dst, int64_t *neg,
                             int32_t *err_flag, hipStream_t stream);
int sgl_batch_prepare(int64_t num_nodes, int64_t batch, const int64_t *src,
                      const int64_t *dst, const int64_t *neg, const float *ts,
                      int64_t *cursor, int64_t *batch_start, uint32_t *node_bits, int32_t *word_prefix,
                      int32_t *num_roots, int64_t *num_roots64, float *ts_max,
                      int64_t *t_query, int64_t *roots, int64_t *root_ts,
                      int32_t *ridx_src, int32_t *ridx_dst, int32_t *ridx_neg,
                      uint64_t *win_src, uint64_t *win_dst, int32_t *cnt_src,
                      int32_t *cnt_dst, int32_t *any_edges, int32_t *err_flag,
                      hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (4)+(6) Memory update (GRU) fused with the mailbox write.
 * Replaces, for the U roots of a batch:
 *   CTDGMemoryUpdater.forward  backends/ctdg/runtime/models.py:244-254
 *     (nn.GRU over the K mailbox slots in slot order from h0 = 0, then
 *      nn.GRUCell(agg, memory); PyTorch weight layouts, gate order r,z,n)
 *   CTDGMemoryBank.read_mailbox / gather   memory.py:135-168
 *   CTDGMemoryBank.write_mailbox / _write_slots   memory.py:183-248
 * new_mem[r] (capacity x D) receives the updated memory of roots[r]; the
 * memory table itself is not written (see sgl_memory_commit), so the mailbox
 * messages [mem(self) | mem(other) | efeat[e]] use pre-update memory as the
 * reference does (runtime.py:270-282). Mailbox slot, ts and next_mail_pos
 * (int32 here) follow memory.py:237-248: one slot per node and role per
 * batch, src role first, pointer advanced by the occurrence counts.
 * Weights: w_ih [3D][2D+F], w_hh [3D][D], wc_ih [3D][D], wc_hh [3D][D].
 * batch_start (may be NULL): sgl_batch_prepare's output when it ran with a
 * cursor; src/dst/efeat/ts then span the whole stream.
 * ------------------------------------------------------------------------- */
size_t sgl_memory_update_lds_bytes(int32_t D, int32_t F);
/* Roots per tile that sgl_memory_update_bf16 uses for these shapes when its
 * arrays are 16-byte aligned and the fragment-order weight copy is passed:
 * 64 or 16 (the wide-tile kernel, whose dynamic and static LDS must fit the
 * CU's 160 KiB), or 0 (the 16-root kernel on row-major bf16 weights). Host
 * arithmetic only (no device call). No counterpart in the reference: it
 * tells a caller which kernel shape serves a configuration. */
int32_t sgl_memory_update_bf16_tile_rows(int32_t D, int32_t F, int64_t capacity);
int sgl_memory_update(int32_t D, int32_t K, int32_t F, int64_t capacity,
                      const int32_t *num_roots, const int64_t *roots,
                      const float *memory, float *mailbox, float *mailbox_ts,
                      int32_t *next_mail_pos, const float *w_ih,
                      const float *w_hh, const float *b_ih, const float *b_hh,
                      const float *wc_ih, const float *wc_hh,
                      const float *bc_ih, const float *bc_hh,
                      const int64_t *src, const int64_t *dst,
                      const float *efeat, const float *ts,
                      const int64_t *batch_start,
                      const uint64_t *win_src, const uint64_t *win_dst,
                      const int32_t *cnt_src, const int32_t *cnt_dst,
                      float *new_mem, hipStream_t stream);
/* The same update with the GRU's four weight matrices in bf16 (raw 16-bit
 * patterns, the same layouts): its GEMMs run on bf16 MFMA with fp32
 * accumulation, the mailbox rows, hidden state and memory rounded to bf16 as
 * they enter a product; biases, gates, state and the mailbox stay fp32 (the
 * mixed-precision setting: bf16 GEMMs, fp32 memory). The updater's weights
 * never train (its output is detached, runtime.py:279), so the caller makes
 * the bf16 copies once. Mailbox contents, slots and pointers are the same as
 * sgl_memory_update's; new_mem within the bf16 tolerance (rtol 2e-2).
 * packed: the same four matrices in the wide-tile kernel's fragment order
 * (sgl_gru_pack_bf16; 16-byte aligned), remade whenever the bf16 copies
 * change. NULL runs the 16-root kernel on the row-major copies instead
 * (slower; the same tolerance). */
int sgl_memory_update_bf16(int32_t D, int32_t K, int32_t F, int64_t capacity,
                           const int32_t *num_roots, const int64_t *roots,
                           const float *memory, float *mailbox, float *mailbox_ts,
                           int32_t *next_mail_pos, const uint16_t *w_ih,
                           const uint16_t *w_hh, const float *b_ih, const float *b_hh,
                           const uint16_t *wc_ih, const uint16_t *wc_hh,
                           const float *bc_ih, const float *bc_hh,
                           const int64_t *src, const int64_t *dst,
                           const float *efeat, const float *ts,
                           const int64_t *batch_start,
                           const uint64_t *win_src, const uint64_t *win_dst,
                           const int32_t *cnt_src, const int32_t *cnt_dst,
                           float *new_mem, const uint16_t *packed, hipStream_t stream);
/* Elements (uint16) of the fragment-order copy of the four bf16 GRU weight
 * matrices for hidden width D and edge-feature width F (0 if D <= 0 or F < 0).
 * No reference counterpart: a layout of this build's bf16 copies. */
int64_t sgl_gru_packed_elems(int32_t D, int32_t F);
/* Writes that copy from the row-major bf16 matrices w_ih [3D][2D+F], w_hh,
 * wc_ih, wc_hh [3D][D] (bit copies, zero padding), on `stream`. Element
 * (((g*nc + c)*nks + s)*64 + l)*8 + t of a matrix's region (regions in that
 * order, nc = ceil(D/16), nks = ceil(kd/32)) holds
 * W[g*D + 16c + l%16][32s + 8(l/16) + t], or 0 past D or kd. */
int sgl_gru_pack_bf16(int32_t D, int32_t F, const uint16_t *w_ih, const uint16_t *w_hh,
                      const uint16_t *wc_ih, const uint16_t *wc_hh, uint16_t *packed,
                      hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (5) Memory commit.
 * Replaces CTDGMemoryBank._apply_memory_update (memory.py:254-269):
 * memory[roots[r]] = new_mem[r], memory_ts[roots[r]] = ts_max for r < U.
 * Also clears node_bits for the next batch and sets any_edges = 1 if some
 * root has sample_cnt[r] > 0 (sample_cnt may be NULL). root_dt (may be
 * NULL) receives ts_max - memory_ts[roots[r]] as it was before the write:
 * the time since the root's previous update (the time-projection
 * embedding's input).
 * ------------------------------------------------------------------------- */
int sgl_memory_commit(int32_t D, int64_t capacity, const int32_t *num_roots,
                      const int64_t *roots, const float *new_mem,
                      float *memory, float *memory_ts, const float *ts_max,
                      uint32_t *node_bits, const int32_t *sample_cnt,
                      int32_t *any_edges, float *root_dt, hipStream_t stream);
/* The same step point without a memory updater: rows[r] = memory[roots[r]]
 * for r < U (the attention's root rows), node_bits cleared and any_edges set
 * as above; memory and memory_ts are not written. Replaces the gather of
 * CTDGMemoryBank.gather (memory.py:135-151) on the path of
 * CTDGOnlineRuntime.train_step without an updater (runtime.py:283-285), which
 * scores from the memory as it is. */
int sgl_memory_gather(int32_t D, int64_t capacity, const int32_t *num_roots,
                      const int64_t *roots, const float *memory, float *rows,
                      uint32_t *node_bits, const int32_t *sample_cnt,
                      int32_t *any_edges, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (7) Time encoding + temporal attention, forward and backward.
 * Replaces TemporalTransformerConv.forward (backends/ctdg/runtime/models.py:77-137)
 * with TimeEncode (runtime/modules/time_encode.py:41-58) over the block of
 * build_dgl_block (models.py:144-197), one tile of sgl_conv_tile_rows()
 * roots per workgroup.
 * Inputs per root r < U: h_root[r] (its updated memory), its padded hop-0
 * window (cnt[r] sampled slots of fanout, the sampler's dt rows
 * [cap][fanout]) and that window's edge rows X [cap][fanout][D+F+T], whose
 * first D+F columns [memory[nbr] | efeat[eid]] come from sgl_edge_rows. The
 * forward computes the time encodings cos(te_w * dt + te_b) (argument
 * rounded as fl(fl(dt * w) + b)), writes them into the rows' last T columns
 * and their sines into S [cap][fanout][T]; the backward reads X and S.
 * Parameters use nn.Linear layouts: w_q [D][D+T], w_k/w_v [D][D+F+T],
 * w_out [D][2D], ln_g/ln_b [D], te_w/te_b [T]. capacity % 16 == 0.
 * Forward writes y [capacity][D] plus the saved state the backward needs
 * (sv_*: Q [cap][D], qt/xbar [cap][H][D+F+T], score [cap][fanout][H],
 * ml [cap][H][2], agg [cap][D], z [cap][D], stats [cap][2]); rows of y
 * >= U are zero, rows of the saved state >= U are left unwritten. If
 * any_edges == 0 the whole output and saved state are zero (models.py:88-89).
 * sv_phi0 [T] (may be NULL) receives cos(te_b), the query's time encoding.
 * Dropout (models.py:127,136; training only): p_att drops attention weights
 * after the softmax, p_out the output projection before the ReLU, both
 * inverted (kept entries scaled by 1/(1-p)); p = 0 turns either off, and
 * with both 0 the masks, seed, rng_step, pass and sv_sdrop are unused and
 * the results are those of the dropout-free kernels. The masks are drawn
 * from a counter-based generator (Philox4x32-10) at (seed, *rng_step, pass,
 * root row, edge slot / column), so the backward regenerates them; the
 * reference runs the attention three times per step with independent masks
 * (runtime.py:193-195), which the caller reproduces as passes 0, 1, 2 with
 * their own saved state. sv_sdrop [cap][H] receives, with attention dropout,
 * the sum of each row's kept and rescaled weights (agg = W_v xbar' + sdrop
 * b_v; the backward reads it).
 * Backward takes dL/dy as gy [cap][D], or (gy NULL) as W_s^T g_src + W_d^T
 * g_dst from sgl_predictor's per-root rows and the predictor's src_fc /
 * dst_fc weights w_s, w_d [D][D]: it reads the fixed-point accumulators
 * acc_src / acc_dst [cap+1][D], writes their rows as floats to g_src / g_dst
 * [cap+1][D] (for the src_fc / dst_fc weight reductions) and clears them for
 * the next step. acc_dst may be NULL (a dropout pass: dL/dy = W_s^T g_src
 * with the pass's own accumulator and weight in the src_* arguments). The
 * dropout arguments are the forward's. It writes gz, gagg [cap][D], G [cap][H][D+F+T],
 * sigma [cap][H], gQ [cap][D] (inputs of the weight-gradient GEMMs; rows
 * >= U unwritten, all zero if any_edges == 0), and per
 * tile partial sums ln_part [cap/R][2][D] (gamma, beta) and
 * te_part [cap/R][2][T] (time-encoding w, b; the b part includes the
 * query's cos(b) term through w_q), R = sgl_conv_backward_tile_rows(D, F,
 * T, H, bw != NULL).
 * ------------------------------------------------------------------------- */
/* Edge rows of the attention's neighbour windows, built once per step after
 * the memory commit: for every root r < U (device) and sampled slot e <
 * cnt[r], row r*fanout + e of X [capacity*fanout][D+F+T] gets
 * [memory[nbr] | efeat[eid]] in its first D+F columns (nbr, eid: the
 * sampler's padded rows); the last T columns are the forward's. Padding
 * slots are not written. Replaces the per-edge feature assembly of
 * TemporalTransformerConv.forward (models.py:77-137 over the block of
 * models.py:144-197). It reads no trained parameter, so it may run beside
 * the previous step's update. */
int sgl_edge_rows(int32_t D, int32_t F, int32_t T, int32_t fanout,
                  int64_t capacity, const int32_t *num_roots,
                  const float *memory, const float *efeat,
                  const int32_t *cnt, const int32_t *nbr, const int32_t *eid,
                  float *X, hipStream_t stream);
/* Roots per attention workgroup of the fp32 and dropout instances for these
 * dimensions (4, or 8 where the 4-root layouts of the 8-wave instances do
 * not fit in LDS; a divisor of 16); 0 if the dimensions are unsupported. */
int32_t sgl_conv_tile_rows(int32_t D, int32_t F, int32_t T, int32_t H);
/* Roots per workgroup of the backward instance sgl_conv_backward runs for
 * these dimensions, with bf16 weight copies (bf16 != 0) or without: the row
 * count of one ln_part / te_part tile (1, 4 or 8; a divisor of 16); 0 if the
 * dimensions are unsupported. No reference counterpart (sizes this build's
 * buffers). */
int32_t sgl_conv_backward_tile_rows(int32_t D, int32_t F, int32_t T, int32_t H, int32_t bf16);
/* bf16 copies of the attention and edge-predictor weights, for the bf16
 * GEMM variants of sgl_conv_forward, sgl_conv_backward and sgl_predictor
 * (argument bw; NULL: the fp32 products). Benchmark configurations 4 and 5 ask for
 * bf16 GEMMs with fp32 memory; the reference runs these products in fp32
 * torch (models.py:77-137, 313-324), so this has no reference counterpart.
 * Every matrix is row-major raw bf16 with rows of ld elements (ld % 8 == 0,
 * 16-byte aligned) and zero padding columns, kept equal to the rounded fp32
 * parameters by sgl_grad_adam's shadow stores (sgl_grad_shadows rebuilds
 * them). With H heads of dh = D/H rows and C = D+F+T:
 *   wq [D][ld_q] = w_q (D+T columns); wk, wv [D][ld_c] = w_k, w_v (C);
 *   wout [D][ld_o] = w_out (2D);
 *   wkt, wvt [C][ld_h] = w_k^T, w_v^T, head h's dh columns from h*hp
 *   (hp % 8 == 0, hp >= dh);
 *   wot [D][ld_d] = w_out[:, :D]^T;
 *   ws, wd [D][ld_d] = the predictor's src_fc / dst_fc weights, wst, wdt
 *   [D][ld_d] their transposes.
 * The bf16 variants take the fp32 arguments too (biases, LayerNorm, time
 * encoding, the backward's query term) and need dropout 0. Products round
 * their fp32 activations to bf16 and accumulate in fp32. */
typedef struct sgl_bf16_weights {
  const uint16_t *wq, *wk, *wv, *wout, *wkt, *wvt, *wot, *ws, *wd, *wst, *wdt;
  int32_t ld_q, ld_c, ld_o, ld_h, hp, ld_d;
} sgl_bf16_weights;
int sgl_conv_forward(int32_t D, int32_t F, int32_t T, int32_t H,
                     int32_t fanout, int64_t capacity,
                     const int32_t *num_roots, const int32_t *any_edges,
                     const float *h_root, const int32_t *cnt, float *X,
                     const float *dt, const float *w_q, const float *b_q,
                     const float *w_k, const float *b_k, const float *w_v,
                     const float *b_v, const float *w_out, const float *b_out,
                     const float *ln_g, const float *ln_b, const float *te_w,
                     const float *te_b, float *sv_Q, float *sv_qt,
                     float *sv_xbar, float *sv_score, float *sv_ml,
                     float *sv_agg, float *sv_z, float *sv_stats,
                     float *sv_phi0, float *S, float *y, float p_att, float p_out,
                     uint64_t seed, const uint64_t *rng_step, int32_t pass,
                     float *sv_sdrop, const sgl_bf16_weights *bw,
                     hipStream_t stream);
int sgl_conv_backward(int32_t D, int32_t F, int32_t T, int32_t H,
                      int32_t fanout, int64_t capacity,
                      const int32_t *num_roots, const int32_t *any_edges,
                      const int32_t *cnt, const float *X, const float *S,
                      const float *dt, const float *w_q, const float *b_q,
                      const float *w_k, const float *b_k, const float *w_v,
                      const float *b_v, const float *w_out, const float *b_out,
                      const float *ln_g, const float *ln_b, const float *te_b,
                      const float *sv_Q, const float *sv_qt,
                      const float *sv_xbar, const float *sv_score,
                      const float *sv_ml, const float *sv_agg,
                      const float *sv_z, const float *sv_stats,
                      const float *gy, int64_t *acc_src, int64_t *acc_dst,
                      const float *w_s, const float *w_d,
                      float *g_src, float *g_dst,
                      float *gz, float *gagg, float *G,
                      float *sigma, float *gQ, float *ln_part, float *te_part,
                      float p_att, float p_out, uint64_t seed,
                      const uint64_t *rng_step, int32_t pass,
                      const float *sv_sdrop, const sgl_bf16_weights *bw,
                      hipStream_t stream);
/* The attention's dropout masks for rows [0, rows) of a pass, as the
 * kernels above draw them (values 0 or 1/(1-p)): att_mask [rows][fanout][H]
 * and out_mask [rows][D] (either may be NULL). For tests and debugging; no
 * reference counterpart (torch draws its masks from its own generator). */
int sgl_dropout_masks(int64_t rows, int32_t fanout, int32_t H, int32_t D,
                      float p_att, float p_out, uint64_t seed,
                      const uint64_t *rng_step, int32_t pass, float *att_mask,
                      float *out_mask, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Time-projection embedding (config 2's JODIE model: memory + GRU + a time
 * projection, no attention). The reference builds its TGN model for family
 * "jodie" (backends/ctdg/runtime/models.py:337-338); this embedding follows
 * the JODIE paper (h(t + Delta) = (1 + W_p Delta) * h(t)) and is selected by
 * ctdg.embedding = time_projection:
 *   y[r] = h_root[r] * (1 + w * x_r + b),  x_r = (root_dt[r] - shift) * scale
 * for r < U, y rows U .. rows-1 zero (rows >= capacity + 1). w, b [D]
 * (nn.Linear(1, D) weight and bias). The backward takes dL/dy = W_s^T g_src +
 * W_d^T g_dst from sgl_predictor's fixed-point rows (consumed, cleared and
 * written as floats to g_src / g_dst [cap+1][D], as sgl_conv_backward does)
 * and writes per-tile partial sums part [cap/16][2][D] of dL/dw and dL/db
 * (reduced by sgl_grad_adam jobs). capacity % 16 == 0.
 * ------------------------------------------------------------------------- */
int sgl_time_projection_forward(int32_t D, int64_t rows, const int32_t *num_roots,
                                const float *h_root, const float *root_dt, float shift,
                                float scale, const float *w, const float *b, float *y,
                                hipStream_t stream);
int sgl_time_projection_backward(int32_t D, int64_t capacity, const int32_t *num_roots,
                                 const float *h_root, const float *root_dt, float shift,
                                 float scale, int64_t *acc_src, int64_t *acc_dst,
                                 const float *w_s, const float *w_d, float *g_src,
                                 float *g_dst, float *part, hipStream_t stream);

/* Fractional bits of the fixed-point int64 accumulators (value = v * 2^-40)
 * that sgl_predictor scatters into and sgl_conv_backward consumes: integer
 * atomics make the sums independent of the order of the additions. */
#define SGL_FIXED_SHIFT 40

/* Size in int32 words of sgl_predictor's completion counter (`done`): 16
 * group words and a top word, 64 words apart, so that the workgroups of a
 * large launch do not all count themselves on one word. */
#define SGL_DONE_WORDS 1088
/* done[SGL_DONE_RANGE_WORD] (a word the counter never uses) becomes nonzero
 * when sgl_predictor met a value outside the fixed-point range of its sums
 * (|v| >= 2^23, or NaN; the value is clamped, so the sums are wrong); the
 * caller reads and clears it. */
#define SGL_DONE_RANGE_WORD 32

/* ---------------------------------------------------------------------------
 * Edge predictor + BCE, forward and (train != 0) backward.
 * Replaces CTDGLinkPredictor.forward (backends/ctdg/runtime/models.py:313-324)
 * on the root rows selected as in runtime.py:176-183, and the loss of
 * runtime.py:290-292. y [capacity][D] are the attention outputs of the
 * roots; ridx_* (from sgl_batch_prepare) pick each event's rows, -1 meaning
 * a zero embedding. Weights in nn.Linear layout: w_s, w_d [D][D], w_o [1][D].
 * Writes pos/neg logits [batch] and loss (mean BCE, pos label 1, neg 0).
 * With train it also writes the out_fc gradients g_wo [D], g_bo [1] and adds
 * the per-root sums of the hidden-layer gradients into the fixed-point
 * accumulators acc_src / acc_dst [capacity+1][D] (SGL_FIXED_SHIFT; zero at
 * entry, e.g. allocated zeroed and cleared by sgl_conv_backward, which
 * consumes them): acc_src[r] = sum over events with root r as src of dL/dh_s,
 * acc_dst[r] = the same for dst (dL/dh_d) and negatives (dL/dh_n); negatives
 * that are not roots add into row U = *num_roots. With dropout (three
 * attention passes, runtime.py:193-195) e_d and e_n come from the rows of
 * y + y_pass_stride and y + 2 y_pass_stride (floats; 0: every role from y)
 * and, when acc_neg is not NULL, the negatives' sums (row U included) go to
 * acc_neg [capacity+1][D] instead of acc_dst. The src_fc / dst_fc
 * gradients follow as reductions over rows 0..U (sgl_grad_adam jobs) and
 * dL/dy through sgl_conv_backward. acc_out (int64 [D+2]) and done (int32
 * [SGL_DONE_WORDS]) are the launch's own accumulator and completion counter:
 * zero before the first call, left zero by every call. All sums over events are exact integer
 * sums, so results do not depend on the order of the workgroups. With bw
 * (may be NULL; sgl_bf16_weights) the src_fc / dst_fc products run on its
 * bf16 copies ws, wd (y_pass_stride 0).
 * ------------------------------------------------------------------------- */
int sgl_predictor(int64_t batch, int32_t D, int64_t capacity, int32_t train,
                  const int32_t *num_roots, const float *y,
                  const int32_t *ridx_src, const int32_t *ridx_dst,
                  const int32_t *ridx_neg, const float *w_s, const float *b_s,
                  const float *w_d, const float *b_d, const float *w_o,
                  const float *b_o, float *pos_logits, float *neg_logits,
                  float *loss, int64_t *acc_src, int64_t *acc_dst,
                  float *g_wo, float *g_bo, int64_t *acc_out, int32_t *done,
                  int64_t y_pass_stride, int64_t *acc_neg,
                  const sgl_bf16_weights *bw, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * (9) Link-prediction metrics of a step on the device.
 * Replaces CTDGOnlineRuntime._metric_dict (backends/ctdg/runtime/runtime.py:
 * 202-214; scikit-learn on the host after a device-to-host copy): from the
 * n_pos positive and n_neg negative logits, scores sigmoid(logit) in float32
 * with labels 1 / 0, "ap" = average_precision_score, "auc" = roc_auc_score,
 * "mrr" = mean over pairs of [pos score > neg score] (float32, as the
 * reference's float mean). One launch, no host synchronisation.
 * Writes (loss, ap, auc, mrr) as doubles to out[4] (may be NULL) and, with a
 * ring, to ring[4 * (*seq % ring_slots)], then increments *seq (a device
 * word the caller zeroes once): consecutive steps' metrics in stream order.
 * loss may be NULL (NaN is written). n_pos + n_neg <= SGL_LINK_METRICS_MAX_SCORES;
 * with no positive or no negative score every metric is NaN.
 * work: sgl_link_metrics_work_doubles(n_pos) doubles of per-workgroup
 * partial sums; done: a device word that is 0 before the first call (each
 * call leaves it 0). Calls sharing work / done must be stream-ordered.
 * ------------------------------------------------------------------------- */
#define SGL_LINK_METRICS_MAX_SCORES 8192
int64_t sgl_link_metrics_work_doubles(int32_t n_pos);
int sgl_link_metrics(int32_t n_pos, int32_t n_neg, const float *pos_logits,
                     const float *neg_logits, const float *loss, uint64_t *seq,
                     double *ring, int32_t ring_slots, double *out,
                     double *work, uint32_t *done, hipStream_t stream);
/* sgl_batch_prepare of a batch and sgl_link_metrics of an earlier step
 * (its logits, loss and metric outputs: arrays the preparation neither
 * reads nor writes) in one launch when the batch takes the one-workgroup
 * preparation (up to 2048 events): the metrics' workgroups run beside the
 * preparation's, after the same launch-plan gate. Larger batches make the
 * two launches in order. Arguments: sgl_batch_prepare's, then
 * sgl_link_metrics'. No counterpart in the reference (it computes the
 * metrics on the host after every step); for callers that overlap a step's
 * metrics with the next step's preparation. */
int sgl_batch_prepare_metrics(int64_t num_nodes, int64_t batch, const int64_t *src,
                              const int64_t *dst, const int64_t *neg, const float *ts,
                              int64_t *cursor, int64_t *batch_start, uint32_t *node_bits,
                              int32_t *word_prefix, int32_t *num_roots, int64_t *num_roots64,
                              float *ts_max, int64_t *t_query, int64_t *roots, int64_t *root_ts,
                              int32_t *ridx_src, int32_t *ridx_dst, int32_t *ridx_neg,
                              uint64_t *win_src, uint64_t *win_dst, int32_t *cnt_src,
                              int32_t *cnt_dst, int32_t *any_edges, int32_t *err_flag,
                              int32_t n_pos, int32_t n_neg, const float *pos_logits,
                              const float *neg_logits, const float *loss, uint64_t *seq,
                              double *ring, int32_t ring_slots, double *out, double *work,
                              uint32_t *done, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Adam over a flat parameter segment (torch.optim.Adam arithmetic), for the
 * optimizer of backends/ctdg/runtime/factory.py:122-128. `step` is a device
 * float holding the completed step count (read as t-1); sgl_adam_advance
 * adds one after the segment's update. `active` (device int32, may be NULL)
 * gates both: 0 leaves parameters, moments and step untouched, as Adam does
 * for parameters whose grad is None.
 * ------------------------------------------------------------------------- */
int sgl_adam_step(int64_t n, float *param, const float *grad, float *exp_avg,
                  float *exp_avg_sq, const float *step, const int32_t *active,
                  float lr, float beta1, float beta2, float eps,
                  float weight_decay, hipStream_t stream);
int sgl_adam_advance(float *step, const int32_t *active, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Fused weight gradients + Adam for one training step.
 * Replaces the backward weight-gradient products of TemporalTransformerConv's
 * nn.Linear / LayerNorm / TimeEncode parameters (autograd of models.py:77-137)
 * and the optimizer.step() of runtime.py:294-296 (torch.optim.Adam of
 * factory.py:122-128), for parameters kept in one flat fp32 buffer with
 * moments exp_avg / exp_avg_sq at the same offsets.
 *
 * A job (device array) is one of:
 *   kind 0: a gradient block G[a][b] = sum_{p<npass} sum_{r<R}
 *           x1[p*ps1 + r*s1 + a] * x2[p*ps2 + r*s2 + b] for a < rows,
 *           b < cols, stored at grad[off + a*ldo + b]; R is r_fixed when
 *           r_fixed >= 0, *num_roots + r_extra when r_fixed == -1, and
 *           ceil(*num_roots / -r_fixed) when r_fixed <= -2 (per-tile partial
 *           sums of tiles of -r_fixed roots: the tiles holding live roots);
 *           npass 0 counts as 1 (the passes of a dropout step). s1 >= rows
 *           (s2 may be 0: a broadcast row). Tiles: ceil(rows/16) *
 *           ceil(cols/16), tiles_b = ceil(cols/16); the job's tile l is the
 *           16x16 block (l / tiles_b, l % tiles_b).
 *   kind 1: rows*cols contiguous elements from off whose gradient is already
 *           in grad (Adam only). Tiles: ceil(rows*cols/256), tile l the
 *           elements from l*256.
 * tile_job (device, num_tiles entries, one workgroup each) holds for
 * workgroup t the job index in bits 0-7 and the tile's index l within its
 * job in bits 8-30, or -1 for no tile; every tile of every job appears
 * once. Workgroup t runs on XCD t % 8, so the table decides which XCD's L2
 * fetches a job's activation strips: starry_unigraph.native.step.xcd_tile_deal
 * gives each job's tiles to one XCD where the per-XCD share allows. The
 * jobs' tile0 field is not read then. With tile_job NULL, jobs holds
 * num_tiles entries instead, one per workgroup: a copy of the workgroup's job
 * with tile0 the tile's index l within it, or kind -1 for an empty slot
 * (starry_unigraph.native.step.per_workgroup_jobs builds it from the same
 * deal; the workgroup then loads its job in one round trip instead of two).
 * sgl_grad_shadows reads either form the same way.
 * Each gradient element is written once, then Adam-updated (torch.optim.Adam
 * arithmetic) if its segment `seg` is active: gates[seg] NULL or
 * *gates[seg] != 0, with the bias corrections coef[2*seg] = lr / (1 -
 * beta1^t) and coef[2*seg+1] = sqrt(1 - beta2^t) of the segment's step t
 * (device floats, written by sgl_adam_coef). gates is a host array of
 * nseg <= SGL_MAX_ADAM_SEGMENTS device pointers (NULL: every segment open).
 * With shadow (may be NULL; see sgl_bf16_weights) a kind-0 job also stores
 * each element's parameter, rounded to bf16 (nearest even), at
 * shadow[sh_off + a*sh_ld + b] when sh_off >= 0 and at
 * shadow[sht_off + b*sht_ld + a] (the transpose) when sht_off >= 0.
 * ------------------------------------------------------------------------- */
#define SGL_MAX_ADAM_SEGMENTS 8

typedef struct sgl_grad_job {
  const float *x1;
  const float *x2;
  int64_t s1, s2;
  int64_t off;
  int64_t ps1, ps2;
  int32_t ldo, rows, cols, kind, seg, r_fixed, r_extra, tiles_b, tile0, npass;
  int64_t sh_off, sht_off;
  int32_t sh_ld, sht_ld;
} sgl_grad_job;

int sgl_grad_adam(const sgl_grad_job *jobs, const int32_t *tile_job,
                  int32_t num_tiles, const int32_t *num_roots, float *param,
                  float *grad, float *exp_avg, float *exp_avg_sq, int32_t nseg,
                  const int32_t *const *gates, const float *coef, float beta1,
                  float beta2, float eps, float weight_decay, uint16_t *shadow,
                  hipStream_t stream);
/* The bf16 copies of sgl_grad_adam's kind-0 jobs from the current
 * parameters (no update): after the parameters are set outside the fused
 * update (initialisation, a loaded checkpoint). No reference counterpart. */
int sgl_grad_shadows(const sgl_grad_job *jobs, const int32_t *tile_job,
                     int32_t num_tiles, const float *param, uint16_t *shadow,
                     hipStream_t stream);

/* Step counts and bias corrections for one sgl_grad_adam launch. Replaces
 * torch.optim.Adam's per-step `step += 1` and bias corrections (the
 * optimizer of backends/ctdg/runtime/factory.py:122-128). For each segment
 * s < nseg whose gate is open (gates NULL, gates[s] NULL or *gates[s] != 0)
 * the completed-step count *steps[s] (device float) advances by one; coef[2s]
 * and coef[2s+1] become lr / (1 - beta1^t) and sqrt(1 - beta2^t) for t =
 * the count after the advance (a closed segment: the count plus one), in
 * double as torch computes them. One lane per segment; the steps[s] must be
 * distinct counters (SGL_ERR_INVALID otherwise). Enqueue it after the gates
 * are written and after the sgl_grad_adam launch that last read this coef;
 * steps and gates are host arrays of device pointers. With step_counter
 * (device uint64, may be NULL) it also advances the training-step counter
 * and copies the new value to step_out (the dropout masks' step, kept with
 * the step's buffers; no reference counterpart). */
int sgl_adam_coef(int32_t nseg, float *const *steps,
                  const int32_t *const *gates, float *coef, float lr,
                  float beta1, float beta2, uint64_t *step_counter,
                  uint64_t *step_out, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Launch plans: a training step's calls of the entry points above, recorded
 * once and replayed by one host call. Replaces the reference's per-step call
 * sequence in CTDGOnlineRuntime.train_step / eval_step
 * (backends/ctdg/runtime/runtime.py:225-386, the stages one after another on
 * one stream) for consecutive full batches; the overlap of steps has no
 * reference counterpart.
 * An op is one call: kind = sgl_plan_op_kind(entry point name), nargs its
 * argument count without the trailing stream, a[i] argument i (pointers and
 * integers as their value, floats as their bit pattern in the low 32 bits).
 * sgl_plan_run enqueues, without blocking the host, ops [0, n_front) (the
 * step's front part: batch preparation, sampling, GRU, memory commit, edge
 * rows, Adam step counts) on the front stream and n_back ops (attention
 * forward, predictor, backward, fused Adam) on the back stream, ordering the
 * two streams through uint32 words in device memory (64 words, zero before
 * the first run): sync[0] = back (last back part done), sync[16] = fronted
 * (last front part done), sync[48] = timeout. A write is a one-lane kernel
 * that stores the number once the stream's earlier kernels are done; a wait
 * is a one-lane kernel that polls the word and ends when it reaches the
 * value, or after about two seconds, setting timeout to 1 (the ordering is
 * then lost; the host checks that word):
 *   front stream: wait until back >= need_back, front ops, write fronted = seq
 *   back stream:  wait until fronted >= seq, back ops, write back = seq
 * With two step-buffer sets used alternately, need_back is the sequence
 * number of the step before the previous one (its back part read this
 * step's buffers): step t+1's front part overlaps step t's back part. A back
 * part must not read the memory table (the edge rows carry the neighbours'
 * memory). Sequence numbers increase (from 1, need_back < seq). Work queued
 * on the back stream between runs that the next front part depends on is
 * published by writing a fresh number v to sync[0] on the back stream after
 * it and passing need_back = v (a fence). With front NULL every op runs in
 * order on the back stream (sync, seq, need_back unused). An op's own checks
 * run when it is replayed; the first failing op's error is returned (ops
 * before it are already enqueued). timed_op >= 0 has that op's kernel record
 * t_start and t_end at its own start and end (see sgl_time_next_launch; -1:
 * no timing).
 * ------------------------------------------------------------------------- */
/* Has the next kernel that the calling host thread launches through one of
 * the step entry points (batch_prepare, recent_sample, memory_update,
 * memory_commit, conv_forward/backward, predictor, grad_adam: their main
 * kernel) record `start` and `stop` (hipEvent_t, timing enabled) at the
 * dispatch's own start and end (hipExtLaunchKernel), so the interval is the
 * kernel alone. NULL, NULL cancels. No reference counterpart (measurement). */
int sgl_time_next_launch(hipEvent_t start, hipEvent_t stop);

#define SGL_OP_MAX_ARGS 64

typedef struct sgl_op {
  int32_t kind;
  int32_t nargs;
  uint64_t a[SGL_OP_MAX_ARGS];
} sgl_op;

/* Kind of a plannable entry point ("sgl_conv_forward", ...), -1 if the name
 * is not one; *nargs (may be NULL) receives its argument count without the
 * stream. */
int32_t sgl_plan_op_kind(const char *name, int32_t *nargs);
int sgl_plan_run(const sgl_op *ops, int32_t n_front, int32_t n_back,
                 hipStream_t front, hipStream_t back, uint32_t *sync,
                 uint32_t seq, uint32_t need_back, int32_t timed_op,
                 hipEvent_t t_start, hipEvent_t t_end);

#ifdef __cplusplus
}
#endif

#endif /* STARRYGL_MI355X_H */
