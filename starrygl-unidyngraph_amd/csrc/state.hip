// Per-step node state: batch preparation, the fused GRU memory update +
// mailbox write, and the memory commit. Counterparts of
//   CTDGOnlineRuntime._prepare / train_step steps 3-5   backends/ctdg/runtime/runtime.py:138-144,268-282
//   CTDGMemoryBank.gather/read_mailbox                   backends/ctdg/runtime/memory.py:135-168
//   CTDGMemoryUpdater.forward (GRU over K slots + GRUCell)  backends/ctdg/runtime/models.py:244-254
//   CTDGMemoryBank.write_mailbox/_write_slots            memory.py:183-248
//   CTDGMemoryBank._apply_memory_update                  memory.py:254-269
//
// Roots (= sorted unique(src ∪ dst)) come from a node bitmap: mark, scan the
// word popcounts, then rank(n) = prefix[n/32] + popc(word & below(n)); the
// rank is the root index and the roots come out sorted without a sort.
// Batches of up to 2048 events do all of it in one workgroup (one launch);
// larger ones use three grid-wide launches.
// Capacity-sized arrays (2B roots) plus a device-side root count keep every
// launch shape static (HIP-graph capturable, no host sync).
#include <climits>

#include "common.h"
#include "metrics.h"
#include "mfma.h"

namespace {

constexpr int kBlock = 256;
constexpr int kScanBlock = 1024;
constexpr int kScanUnroll = 4;  // 256-word rounds per wave in flight in k_step_scan
constexpr int kTileRows = 16;

__device__ __forceinline__ uint32_t ts_order(float x) {
  // monotone map float -> uint32 (larger float -> larger key)
  const uint32_t b = __float_as_uint(x);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ int32_t node_rank(const uint32_t *__restrict__ bits,
                                             const int32_t *__restrict__ prefix, int64_t n) {
  const uint32_t w = bits[n >> 5];
  const uint32_t below = (1u << (n & 31)) - 1u;
  return prefix[n >> 5] + __popc(w & below);
}

__device__ __forceinline__ float ts_from_order(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Multi-workgroup batch preparation (batches above kPrepMaxBatch events):
// mark, scan, index. Each workgroup of the mark and index kernels takes
// kB * kPer consecutive events and combines them per node (mark) or per
// root (index) in a small LDS table before touching global memory: the hot
// nodes of a skewed stream (a Zipf-distributed one has a node in a third of
// all events) then cost one global atomic per workgroup instead of one per
// event, as same-address atomics serialise in L2. A node whose table slot is
// held by another goes to global memory directly. The running timestamp
// maximum of the mark kernel lives in the first summary word of node_bits as
// order(max ts), and the number of bits the mark kernel set in the second
// (words this path does not otherwise use); the scan reads and clears them.
// Two workgroup shapes: batches of up to kAggSmallMax events take one event
// per thread of 256-thread workgroups (config 5's 4,000 events: 16
// workgroups, every event's dependent loads in flight at once, where
// 4,096-event workgroups left the batch to one workgroup whose threads
// walked four events each); larger batches 4,096 events per 1,024-thread
// workgroup, where the per-workgroup aggregation of the hub nodes pays.
constexpr int kAggBlock = 1024;
constexpr int kAggPer = 4;
constexpr int kAggEvents = kAggBlock * kAggPer;
constexpr int kMarkLog2 = 12;  // node table of the mark kernel (4096 slots, 16 KB)
constexpr int kIdxLog2 = 10;   // per-role root table of the index kernel (1024 slots, 2 x 16 KB)
constexpr int kAggSmallBlock = 256;
constexpr int64_t kAggSmallMax = 65536;
constexpr int kMarkSmallLog2 = 10;  // at most 512 nodes per workgroup
constexpr int kIdxSmallLog2 = 9;    // at most 256 roots per role and workgroup
constexpr unsigned kFewGroups = 32;  // mark grids this small skip the read before each bit's atomic

__device__ __forceinline__ uint32_t agg_slot(uint32_t key, int log2_slots) {
  return (key * 2654435761u) >> (32 - log2_slots);
}

template <int kB, int kPer, int kL2>
__global__ __launch_bounds__(kB) void k_step_mark(
    int64_t batch, int64_t num_nodes, int64_t cap, const int64_t *__restrict__ src,
    const int64_t *__restrict__ dst, const float *__restrict__ ts, const int64_t *__restrict__ cursor,
    int64_t *__restrict__ batch_start, uint32_t *__restrict__ bits, uint32_t *__restrict__ ts_slot,
    unsigned long long *__restrict__ win_src, unsigned long long *__restrict__ win_dst,
    int32_t *__restrict__ cnt_src, int32_t *__restrict__ cnt_dst,
    int32_t *__restrict__ any_edges, int32_t *__restrict__ err) {
  __shared__ int32_t s_node[(1 << kL2)];
  __shared__ float s_m[kB / sgl::kWave];
  __shared__ int32_t s_new;  // bits this workgroup set (summed into new_count)
  const int tid = threadIdx.x;
  const bool few = gridDim.x <= kFewGroups;
  if (tid == 0) s_new = 0;
  const int64_t g = int64_t(blockIdx.x) * kB + tid;
  if (g == 0) *any_edges = 0;
  for (int64_t r = g; r < cap; r += int64_t(gridDim.x) * kB) {
    win_src[r] = 0ull;
    win_dst[r] = 0ull;
    cnt_src[r] = 0;
    cnt_dst[r] = 0;
  }
  for (int i = tid; i < (1 << kL2); i += kB) s_node[i] = -1;
  const int64_t off = cursor != nullptr ? *cursor : 0;
  if (cursor != nullptr && g == 0) *batch_start = off;
  __syncthreads();
  float m = -INFINITY;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int64_t e = int64_t(blockIdx.x) * (kB * kPer) + j * kB + tid;
    if (e >= batch) break;
    const int64_t s = src[off + e], d = dst[off + e];
    m = fmaxf(m, ts[off + e]);  // fmaxf ignores NaN
    if (s < 0 || s >= num_nodes || d < 0 || d >= num_nodes) {
      if (err != nullptr) atomicOr(err, SGL_DERR_NODE_RANGE);
      continue;
    }
#pragma unroll
    for (int role = 0; role < 2; ++role) {
      const int32_t n = int32_t(role == 0 ? s : d);
      const int32_t old = atomicCAS(&s_node[agg_slot(uint32_t(n), kL2)], -1, n);
      if (old == n) continue;  // this workgroup marks n already
      // first in this workgroup (or its slot is taken): set the bit, with no
      // atomic when another workgroup has set it already (a grid of at most
      // kFewGroups issues the atomic at once: one round trip less, and few
      // same-address atomics on a hub's word)
      const uint32_t mb = 1u << (n & 31);
      if ((few || (bits[n >> 5] & mb) == 0u) && (atomicOr(&bits[n >> 5], mb) & mb) == 0u) atomicAdd(&s_new, 1);
    }
  }
  // the block's timestamp maximum, then one atomic max per block, skipped
  // when the slot already holds as much
#pragma unroll
  for (int dd = 32; dd > 0; dd >>= 1) m = fmaxf(m, __shfl_xor(m, dd, sgl::kWave));
  if ((tid & 63) == 0) s_m[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    float mm = s_m[0];
#pragma unroll
    for (int w = 1; w < kB / sgl::kWave; ++w) mm = fmaxf(mm, s_m[w]);
    if (mm > -INFINITY) {
      const uint32_t k = ts_order(mm);
      if (few || *ts_slot < k) atomicMax(ts_slot, k);
    }
    if (s_new > 0) atomicAdd(ts_slot + 1, uint32_t(s_new));
  }
}

// One workgroup: exclusive scan of the bitmap word popcounts (-> root count)
// and the batch's max timestamp from the mark kernel's slot (-> the
// sampler's query time). Each wave takes a contiguous range of the bitmap
// (a multiple of 256 words): a first pass sums its popcounts (16-byte loads,
// kScanUnroll rounds of 64 lanes in flight, every load instruction one
// contiguous kilobyte), one barrier gives each wave the words before its
// range, and a second pass re-reads the range (now in L2) and writes the
// prefixes round by round, a wave scan per round. Threads holding many
// consecutive words instead made each load touch 64 lines (a 16-word stride
// per lane: 12-13 us for configs 4 and 5's 35,632 words, as slow as one
// workgroup-wide scan per 4,096 words). Thread 0 reads the mark kernel's
// words and the batch start first, so that their round trip overlaps the
// bitmap's.
__global__ __launch_bounds__(kScanBlock) void k_step_scan(
    int64_t nwords, int64_t all_words, uint32_t *__restrict__ bits, int32_t *__restrict__ prefix,
    int32_t *__restrict__ num_roots, int64_t *__restrict__ num_roots64, int64_t batch,
    uint32_t *__restrict__ ts_slot, int64_t *__restrict__ cursor, const int64_t *__restrict__ batch_start,
    float *__restrict__ ts_max, int64_t *__restrict__ t_query, int32_t *__restrict__ err) {
  constexpr int kWaves = kScanBlock / sgl::kWave;
  constexpr int kRound = 4 * sgl::kWave;  // words per wave and round
  __shared__ int32_t s_w[kWaves];
  __shared__ int32_t s_stale;
  uint32_t k_ts = 0u, n_set = 0u;
  int64_t b_start = 0;
  if (threadIdx.x == 0) {
    k_ts = ts_slot[0];
    n_set = ts_slot[1];
    if (cursor != nullptr) b_start = *batch_start;
  }
  const int wave = threadIdx.x / sgl::kWave, lane = threadIdx.x & (sgl::kWave - 1);
  // the wave's words [w0, w1): nwords is a multiple of 4, so every 16-byte
  // group a lane takes is whole
  const int64_t per = ((nwords + kWaves - 1) / kWaves + kRound - 1) / kRound * kRound;
  const int64_t w0 = min(nwords, int64_t(wave) * per), w1 = min(nwords, w0 + per);
  int32_t cnt = 0;
  for (int64_t r0 = w0; r0 < w1; r0 += int64_t(kScanUnroll) * kRound) {
    uint4 w[kScanUnroll];
#pragma unroll
    for (int u = 0; u < kScanUnroll; ++u) {
      const int64_t i = r0 + int64_t(u) * kRound + 4 * lane;
      w[u] = i < w1 ? *reinterpret_cast<const uint4 *>(bits + i) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kScanUnroll; ++u) cnt += __popc(w[u].x) + __popc(w[u].y) + __popc(w[u].z) + __popc(w[u].w);
  }
  const int32_t wave_total = __shfl(sgl::wave_inclusive_scan(cnt), sgl::kWave - 1, sgl::kWave);
  if (lane == 0) s_w[wave] = wave_total;
  __syncthreads();
  int32_t run = 0, carry = 0;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    const int32_t t = s_w[v];
    run += v < wave ? t : 0;
    carry += t;
  }
  for (int64_t r0 = w0; r0 < w1; r0 += int64_t(kScanUnroll) * kRound) {
    uint4 w[kScanUnroll];
#pragma unroll
    for (int u = 0; u < kScanUnroll; ++u) {
      const int64_t i = r0 + int64_t(u) * kRound + 4 * lane;
      w[u] = i < w1 ? *reinterpret_cast<const uint4 *>(bits + i) : make_uint4(0u, 0u, 0u, 0u);
    }
#pragma unroll
    for (int u = 0; u < kScanUnroll; ++u) {
      const int64_t i = r0 + int64_t(u) * kRound + 4 * lane;
      const int32_t c0 = __popc(w[u].x), c1 = __popc(w[u].y), c2 = __popc(w[u].z), c3 = __popc(w[u].w);
      const int32_t sum = c0 + c1 + c2 + c3;
      const int32_t inc = sgl::wave_inclusive_scan(sum);
      const int32_t at = run + inc - sum;
      if (i < w1) *reinterpret_cast<int4 *>(prefix + i) = make_int4(at, at + c0, at + c0 + c1, at + c0 + c1 + c2);
      run += __shfl(inc, sgl::kWave - 1, sgl::kWave);
    }
  }
  // every set bit was set by this batch's mark kernel, unless a previous
  // preparation's commit did not run: then its ranks could exceed the
  // buffers; report it, clear the bitmap and give the batch no roots
  if (threadIdx.x == 0) s_stale = carry != int32_t(n_set);
  __syncthreads();
  const bool stale = s_stale != 0;
  if (stale)
    for (int64_t w = threadIdx.x; w < all_words; w += kScanBlock) bits[w] = 0u;
  if (threadIdx.x == 0) {
    ts_slot[0] = 0u;
    ts_slot[1] = 0u;
    const float mm = k_ts != 0u ? ts_from_order(k_ts) : -INFINITY;
    if (stale && err != nullptr) atomicOr(err, SGL_DERR_STALE_NODE_BITS);
    if (stale) carry = 0;
    *num_roots = carry;
    *num_roots64 = carry;
    *ts_max = mm;
    // int(float max) truncates toward zero (runtime.py:142); the float32 round
    // trip of sampler.py:113 then bts_sampler.py:81 is exact for that value.
    *t_query = batch > 0 ? (long long)truncf(mm) : 0;
    if (cursor != nullptr) *cursor = b_start + batch;
  }
}

template <int kB, int kPer, int kL2>
__global__ __launch_bounds__(kB) void k_step_index(
    int64_t batch, int64_t num_nodes, const int32_t *__restrict__ num_roots, const int64_t *__restrict__ src,
    const int64_t *__restrict__ dst, const int64_t *__restrict__ neg,
    const float *__restrict__ ts, const int64_t *__restrict__ batch_start, const uint32_t *__restrict__ bits,
    const int32_t *__restrict__ prefix, const int64_t *__restrict__ t_query,
    int64_t *__restrict__ roots, int64_t *__restrict__ root_ts,
    int32_t *__restrict__ ridx_src, int32_t *__restrict__ ridx_dst,
    int32_t *__restrict__ ridx_neg, unsigned long long *__restrict__ win_src,
    unsigned long long *__restrict__ win_dst, int32_t *__restrict__ cnt_src,
    int32_t *__restrict__ cnt_dst) {
  // per role: root rank, count and last-writer key of the table's roots
  __shared__ int32_t s_root[2][(1 << kL2)], s_cnt[2][(1 << kL2)];
  __shared__ unsigned long long s_win[2][(1 << kL2)];
  const int tid = threadIdx.x;
  for (int i = tid; i < (1 << kL2); i += kB) {
    s_root[0][i] = s_root[1][i] = -1;
    s_cnt[0][i] = s_cnt[1][i] = 0;
    s_win[0][i] = s_win[1][i] = 0ull;
  }
  if (batch_start != nullptr) {
    const int64_t off = *batch_start;
    src += off;
    dst += off;
    ts += off;
    if (neg != nullptr) neg += off;
  }
  const int64_t tq = *t_query;
  if (*num_roots == 0) {  // no valid event, or a stale bitmap (k_step_scan): no event has a root
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int64_t e = int64_t(blockIdx.x) * (kB * kPer) + j * kB + tid;
      if (e >= batch) break;
      ridx_src[e] = -1;
      ridx_dst[e] = -1;
      if (neg != nullptr) ridx_neg[e] = -1;
    }
    return;
  }
  __syncthreads();
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int64_t e = int64_t(blockIdx.x) * (kB * kPer) + j * kB + tid;
    if (e >= batch) break;
    const int64_t s = src[e], d = dst[e];
    if (neg != nullptr) {
      const int64_t n = neg[e];
      int32_t rn = -1;
      if (n >= 0 && n < num_nodes && ((bits[n >> 5] >> (n & 31)) & 1u)) rn = node_rank(bits, prefix, n);
      ridx_neg[e] = rn;
    }
    if (s < 0 || s >= num_nodes || d < 0 || d >= num_nodes) {
      ridx_src[e] = -1;
      ridx_dst[e] = -1;
      continue;
    }
    const int32_t rs = node_rank(bits, prefix, s);
    const int32_t rd = node_rank(bits, prefix, d);
    ridx_src[e] = rs;
    ridx_dst[e] = rd;
    // last writer per root and role = the largest (order(ts), e) key (stable timestamp order)
    const unsigned long long key = (static_cast<unsigned long long>(ts_order(ts[e])) << 32) |
                                   static_cast<unsigned long long>(e);
#pragma unroll
    for (int role = 0; role < 2; ++role) {
      const int32_t r = role == 0 ? rs : rd;
      const int64_t node = role == 0 ? s : d;
      const int slot = int(agg_slot(uint32_t(r), kL2));
      const int32_t old = atomicCAS(&s_root[role][slot], -1, r);
      if (old == -1 || old == r) {
        if (old == -1) {  // the root's first event in this workgroup
          roots[r] = node;
          root_ts[r] = tq;
        }
        atomicAdd(&s_cnt[role][slot], 1);
        atomicMax(&s_win[role][slot], key);
      } else {  // the slot holds another root
        roots[r] = node;
        root_ts[r] = tq;
        atomicAdd(role == 0 ? &cnt_src[r] : &cnt_dst[r], 1);
        atomicMax(role == 0 ? &win_src[r] : &win_dst[r], key);
      }
    }
  }
  __syncthreads();
  for (int i = tid; i < 2 * (1 << kL2); i += kB) {
    const int role = i / (1 << kL2), slot = i - role * (1 << kL2);
    const int32_t r = s_root[role][slot];
    if (r < 0) continue;
    atomicAdd(role == 0 ? &cnt_src[r] : &cnt_dst[r], s_cnt[role][slot]);
    atomicMax(role == 0 ? &win_src[r] : &win_dst[r], s_win[role][slot]);
  }
}

// One-workgroup batch preparation for batches of up to kPrepMaxBatch events.
// The node bitmap gives the roots in ascending order without a sort. Marking
// also sets a summary bitmap (bit w: word w of the node bitmap is nonzero),
// so on large graphs the popcount prefix only visits the nonzero words: scan
// the summary, popcount the flagged words, block-scan, and rank(n) =
// prefix[n / 32] + popc(word & below(n)); a bitmap of at most
// kPrepDirectWords words is read whole instead, a few words per thread in
// one round (configs 1 and 2: 289 words, where the summary walk left ten
// threads each loading about 29 flagged words one after another). Per-(root, role) counts and last writers are LDS
// atomics (64-bit max of order(ts) << 32 | e: the last event in stable
// timestamp order); negatives need one bit test. The workgroup clears the
// bits it set, leaving both bitmaps zero.
constexpr int kPrepBlock = 1024;
constexpr int kPrepMaxBatch = 2048;
constexpr int kPrepPer = kPrepMaxBatch / kPrepBlock;
constexpr int kPrepDirectPer = 4;  // bitmap words per thread of the direct prefix
constexpr int64_t kPrepDirectWords = int64_t(kPrepDirectPer) * kPrepBlock;

__host__ __device__ inline int64_t bitmap_words(int64_t num_nodes) { return ((num_nodes + 31) / 32 + 3) & ~int64_t(3); }
__host__ __device__ inline int64_t summary_words(int64_t num_nodes) {
  return ((bitmap_words(num_nodes) + 31) / 32 + 3) & ~int64_t(3);
}

// A batch preparation that found bits set before it marked its own: every
// bitmap word cleared, no event mapped to a root, no counts (one workgroup
// of nthr threads; the callers then report SGL_DERR_STALE_NODE_BITS and a
// root count of 0).
__device__ void stale_batch(int tid, int nthr, int64_t batch, int64_t cap, uint32_t *bits, int64_t words,
                            int32_t *ridx_src, int32_t *ridx_dst, int32_t *ridx_neg,
                            unsigned long long *win_src, unsigned long long *win_dst, int32_t *cnt_src,
                            int32_t *cnt_dst) {
  for (int64_t w = tid; w < words; w += nthr) bits[w] = 0u;
  for (int64_t e = tid; e < batch; e += nthr) {
    ridx_src[e] = -1;
    ridx_dst[e] = -1;
    if (ridx_neg != nullptr) ridx_neg[e] = -1;
  }
  for (int64_t r = tid; r < cap; r += nthr) {
    win_src[r] = 0ull;
    win_dst[r] = 0ull;
    cnt_src[r] = 0;
    cnt_dst[r] = 0;
  }
}

__global__ __launch_bounds__(kPrepBlock) void k_step_prepare_wg(
    int64_t batch, int64_t num_nodes, int64_t cap, const int64_t *__restrict__ src,
    const int64_t *__restrict__ dst, const int64_t *__restrict__ neg, const float *__restrict__ ts,
    int64_t *__restrict__ cursor, int64_t *__restrict__ batch_start, uint32_t *__restrict__ bits,
    int32_t *__restrict__ prefix,
    int32_t *__restrict__ num_roots, int64_t *__restrict__ num_roots64, float *__restrict__ ts_max,
    int64_t *__restrict__ t_query, int64_t *__restrict__ roots, int64_t *__restrict__ root_ts,
    int32_t *__restrict__ ridx_src, int32_t *__restrict__ ridx_dst, int32_t *__restrict__ ridx_neg,
    unsigned long long *__restrict__ win_src, unsigned long long *__restrict__ win_dst,
    int32_t *__restrict__ cnt_src, int32_t *__restrict__ cnt_dst, int32_t *__restrict__ any_edges,
    int32_t *__restrict__ err, const uint32_t *gate_word, uint32_t gate_value, uint32_t *gate_timeout,
    sgl::met::Args mr) {
  if (blockIdx.x > 0) {
    // the workgroups past the first: a previous step's link metrics
    // (sgl_batch_prepare_metrics), which read only that step's logits and
    // loss, after the same gate
    if (gate_word != nullptr) {
      if (threadIdx.x == 0) sgl::gate_wait(gate_word, gate_value, gate_timeout);
      __syncthreads();
    }
    sgl::met::run(mr, blockIdx.x - 1, gridDim.x - 1);
    return;
  }
  extern __shared__ unsigned long long l_win[];                      // [2][cap]
  int32_t *l_cnt = reinterpret_cast<int32_t *>(l_win + 2 * cap);     // [2][cap]
  __shared__ int32_t s_scan[kPrepBlock / sgl::kWave];
  __shared__ float s_max[kPrepBlock / sgl::kWave];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (gate_word != nullptr) {
    // a launch plan's cross-stream gate, before anything is read or written:
    // thread 0's acquire loads invalidate this CU's L1 and the XCD's L2 for
    // the whole workgroup (one CU), which the barrier then orders after
    if (tid == 0) sgl::gate_wait(gate_word, gate_value, gate_timeout);
    __syncthreads();
  }
  uint32_t *summary = bits + bitmap_words(num_nodes);
  const int64_t off = cursor != nullptr ? *cursor : 0;
  src += off;
  dst += off;
  ts += off;
  if (neg != nullptr) neg += off;
  for (int r = tid; r < 2 * cap; r += kPrepBlock) {
    l_win[r] = 0ull;
    l_cnt[r] = 0;
  }
  // bits this batch sets itself (a bit already set belongs to a previous
  // batch whose commit did not run: checked against the root count below)
  __shared__ int32_t s_new;
  if (tid == 0) s_new = 0;
  __syncthreads();
  // endpoints, times and negatives of events e = tid + c * kPrepBlock (one
  // round of loads); mark the endpoints' bits
  int64_t es[kPrepPer], ed[kPrepPer], en[kPrepPer];
  float te[kPrepPer];
  bool ok[kPrepPer];
  float m = -INFINITY;
#pragma unroll
  for (int c = 0; c < kPrepPer; ++c) {
    const int e = tid + c * kPrepBlock;
    const bool live = e < batch;
    es[c] = live ? src[e] : 0;
    ed[c] = live ? dst[e] : 0;
    te[c] = live ? ts[e] : 0.f;
    en[c] = live && neg != nullptr ? neg[e] : -1;
  }
#pragma unroll
  for (int c = 0; c < kPrepPer; ++c) {
    const int e = tid + c * kPrepBlock;
    ok[c] = false;
    if (e < batch) {
      ok[c] = es[c] >= 0 && es[c] < num_nodes && ed[c] >= 0 && ed[c] < num_nodes;
      m = fmaxf(m, te[c]);
      if (ok[c]) {
        const uint32_t bs = 1u << (es[c] & 31), bd = 1u << (ed[c] & 31);
        int fresh = (atomicOr(&bits[es[c] >> 5], bs) & bs) ? 0 : 1;
        fresh += (atomicOr(&bits[ed[c] >> 5], bd) & bd) ? 0 : 1;
        if (fresh) atomicAdd(&s_new, fresh);
        atomicOr(&summary[es[c] >> 10], 1u << ((es[c] >> 5) & 31));
        atomicOr(&summary[ed[c] >> 10], 1u << ((ed[c] >> 5) & 31));
      } else {
        if (err != nullptr) atomicOr(err, SGL_DERR_NODE_RANGE);
        ridx_src[e] = -1;
        ridx_dst[e] = -1;
      }
    }
  }
#pragma unroll
  for (int dd = 32; dd > 0; dd >>= 1) m = fmaxf(m, __shfl_xor(m, dd, sgl::kWave));
  if (lane == 0) s_max[wave] = m;
  __syncthreads();
  float mm = -INFINITY;
#pragma unroll
  for (int w = 0; w < kPrepBlock / sgl::kWave; ++w) mm = fmaxf(mm, s_max[w]);
  // int(float max) truncates toward zero (runtime.py:142); the float32 round
  // trip of sampler.py:113 then bts_sampler.py:81 is exact for that value.
  const int64_t tq = batch > 0 ? (long long)truncf(mm) : 0;

  // popcount prefix over the nonzero words, in word order. A bitmap of at
  // most kPrepDirectWords words (graphs up to 131,072 nodes): thread t owns
  // words [t * per, t * per + per), all loaded in one round. Larger ones:
  // thread t owns summary words [s0, s0 + cs) and visits the bitmap words
  // they flag (a small graph's few summary words would leave a handful of
  // threads each loading tens of flagged words one after another).
  const int64_t nbw = bitmap_words(num_nodes);
  const bool direct = nbw <= kPrepDirectWords;
  const int per = int((nbw + kPrepBlock - 1) / kPrepBlock);  // <= kPrepDirectPer when direct
  const int64_t nsum = (nbw + 31) / 32;
  const int64_t cs = (nsum + kPrepBlock - 1) / kPrepBlock;
  const int64_t s0 = int64_t(tid) * cs;
  const int64_t s1 = s0 + cs < nsum ? s0 + cs : nsum;
  int32_t cnt_here = 0;
  uint32_t dw[kPrepDirectPer];
  if (direct) {
#pragma unroll
    for (int q = 0; q < kPrepDirectPer; ++q) {
      const int64_t w = int64_t(tid) * per + q;
      dw[q] = q < per && w < nbw ? bits[w] : 0u;
      cnt_here += __popc(dw[q]);
    }
  } else {
    for (int64_t sw = s0; sw < s1; ++sw) {
      uint32_t f = summary[sw];
      while (f != 0u) {
        const int b = __ffs(f) - 1;
        f &= f - 1u;
        cnt_here += __popc(bits[(sw << 5) + b]);
      }
    }
  }
  int32_t U;
  int32_t run = sgl::block_exclusive_scan<int32_t, kPrepBlock>(cnt_here, s_scan, U);
  if (U != s_new) {
    // the bitmap held bits before this batch (a previous preparation whose
    // commit did not run): its ranks could exceed the buffers. Report it,
    // clear both bitmaps and leave the batch without roots.
    stale_batch(tid, kPrepBlock, batch, cap, bits, bitmap_words(num_nodes) + summary_words(num_nodes), ridx_src,
                ridx_dst, neg != nullptr ? ridx_neg : nullptr, win_src, win_dst, cnt_src, cnt_dst);
    if (tid == 0) {
      if (err != nullptr) atomicOr(err, SGL_DERR_STALE_NODE_BITS);
      *num_roots = 0;
      *num_roots64 = 0;
      *ts_max = mm;
      *t_query = tq;
      *any_edges = 0;
      if (cursor != nullptr) {
        *batch_start = off;
        *cursor = off + batch;
      }
    }
    return;
  }
  if (direct) {
#pragma unroll
    for (int q = 0; q < kPrepDirectPer; ++q) {
      const int64_t w = int64_t(tid) * per + q;
      if (q < per && w < nbw) {
        prefix[w] = run;
        run += __popc(dw[q]);
      }
    }
  } else {
    for (int64_t sw = s0; sw < s1; ++sw) {
      uint32_t f = summary[sw];
      while (f != 0u) {
        const int b = __ffs(f) - 1;
        f &= f - 1u;
        const int64_t w = (sw << 5) + b;
        prefix[w] = run;
        run += __popc(bits[w]);
      }
    }
  }
  __syncthreads();

  // ranks, roots, counts and last writers; the bitmap and prefix words of
  // every endpoint and negative are loaded in one round
  uint32_t wb[kPrepPer][3];
  int32_t wp[kPrepPer][3];
#pragma unroll
  for (int c = 0; c < kPrepPer; ++c) {
    const int e = tid + c * kPrepBlock;
    const bool live = e < batch;
    const int64_t nn = en[c] >= 0 && en[c] < num_nodes ? en[c] : 0;
    const int64_t w[3] = {live && ok[c] ? es[c] >> 5 : 0, live && ok[c] ? ed[c] >> 5 : 0, live ? nn >> 5 : 0};
#pragma unroll
    for (int r = 0; r < 3; ++r) {
      wb[c][r] = bits[w[r]];
      wp[c][r] = prefix[w[r]];
    }
  }
#pragma unroll
  for (int c = 0; c < kPrepPer; ++c) {
    const int e = tid + c * kPrepBlock;
    if (e >= batch) continue;
    if (ok[c]) {
      const unsigned long long wkey =
          (static_cast<unsigned long long>(ts_order(te[c])) << 32) | static_cast<unsigned long long>(e);
#pragma unroll
      for (int role = 0; role < 2; ++role) {
        const int64_t n = role ? ed[c] : es[c];
        const int32_t rank = wp[c][role] + __popc(wb[c][role] & ((1u << (n & 31)) - 1u));
        (role ? ridx_dst : ridx_src)[e] = rank;
        roots[rank] = n;
        root_ts[rank] = tq;
        atomicAdd(&l_cnt[role * cap + rank], 1);
        atomicMax(&l_win[role * cap + rank], wkey);
      }
    }
    if (neg != nullptr) {
      const int64_t n = en[c];
      int32_t rn = -1;
      if (n >= 0 && n < num_nodes && ((wb[c][2] >> (n & 31)) & 1u))
        rn = wp[c][2] + __popc(wb[c][2] & ((1u << (n & 31)) - 1u));
      ridx_neg[e] = rn;
    }
  }
  __syncthreads();
  for (int r = tid; r < cap; r += kPrepBlock) {
    cnt_src[r] = l_cnt[r];
    cnt_dst[r] = l_cnt[cap + r];
    win_src[r] = l_win[r];
    win_dst[r] = l_win[cap + r];
  }
  // leave both bitmaps zero (every read of them is behind the barrier above)
#pragma unroll
  for (int c = 0; c < kPrepPer; ++c) {
    const int e = tid + c * kPrepBlock;
    if (e >= batch || !ok[c]) continue;
    bits[es[c] >> 5] = 0u;
    bits[ed[c] >> 5] = 0u;
    summary[es[c] >> 10] = 0u;
    summary[ed[c] >> 10] = 0u;
  }
  if (tid == 0) {
    *num_roots = U;
    *num_roots64 = U;
    *ts_max = mm;
    *t_query = tq;
    *any_edges = 0;
    if (cursor != nullptr) {  // every read of *cursor is behind the barriers above
      *batch_start = off;
      *cursor = off + batch;
    }
  }
}

// Gate nonlinearities of the bf16 wide-tile kernel from the hardware's base-2
// exponential and reciprocal (v_exp_f32, v_rcp_f32, about 1 ulp each):
//   s(x) = 1 / (1 + 2^(-x log2 e)),  tanh(x) = 1 - 2 / (1 + 2^(2x log2 e)),
// which saturate at the ends (2^+inf = inf, 1/inf = 0). Absolute error about
// 1e-7, far inside the bf16 products' tolerance; at 16 gate values per lane
// and slot the library expf / tanhf and divisions cost that kernel as much VALU
// time as its products. The fp32 kernels keep expf / tanhf.
__device__ __forceinline__ float gate_sigmoid(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-1.44269504f * x));
}
__device__ __forceinline__ float gate_tanh(float x) {
  return 1.f - 2.f * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(2.88539008f * x));
}

// GRU gate combination (PyTorch order r, z, n):
//   r = s(gi_r + gh_r), z = s(gi_z + gh_z), n = tanh(gi_n + r * gh_n),
//   h' = (1 - z) * n + z * h
__device__ __forceinline__ float gru_combine(float gir, float giz, float gin, float ghr, float ghz,
                                             float ghn, float h) {
  const float r = 1.f / (1.f + expf(-(gir + ghr)));
  const float z = 1.f / (1.f + expf(-(giz + ghz)));
  const float n = tanhf(gin + r * ghn);
  return (1.f - z) * n + z * h;
}

constexpr int kGruBlock = 1024;
constexpr int kGruWaves = kGruBlock / sgl::kWave;
constexpr int kMaxMsgSlots = 8;  // S = 2D + F <= 512
static_assert(kGruWaves == kTileRows, "the mailbox phase maps wave w to root w");

// One workgroup of 16 waves = 16 roots. LDS: x [16][S], h [16][D],
// mem [16][D], gi [16][3D], gh [16][3D] (leading dims padded by one float).
// Wave i also assembles root i's outgoing messages: their foreign parts (the
// other endpoint's memory row and the edge's features) are loaded into
// registers before the GEMMs and stored after them, so the loads overlap
// the GRU arithmetic.
// The GRU's weight matrices are fp32 (WT = float: fp32 MFMA) or bf16
// (WT = uint16_t, raw bf16 patterns: bf16 MFMA with fp32 accumulation, the
// LDS operands rounded to bf16 as they are read); biases, gates and state
// stay fp32.
// AT: the LDS operand type (fp32 tiles for fp32 weights, bf16 copies of the
// tiles for bf16 weights).
template <typename WT, typename AT>
__device__ __forceinline__ void gru_products(const AT *A0, int lda0, const WT *W0, int ldw0, const float *b0,
                                             float *O0, int kd0, int n0, const AT *A1, int lda1, const WT *W1,
                                             int ldw1, const float *b1, float *O1, int kd1, int n1, int ldo) {
  if constexpr (std::is_same_v<WT, float>) {
    sgl::GemmJob jobs[2] = {{A0, lda0, W0, ldw0, b0, O0, ldo, kd0, n0}, {A1, lda1, W1, ldw1, b1, O1, ldo, kd1, n1}};
    sgl::tile_gemm16_jobs<sgl::kNT>(jobs, kGruWaves);
  } else {
    sgl::GemmJobBf16<AT> jobs[2] = {{A0, lda0, W0, ldw0, b0, O0, ldo, kd0, n0},
                                    {A1, lda1, W1, ldw1, b1, O1, ldo, kd1, n1}};
    sgl::tile_gemm16_jobs_bf16(jobs, kGruWaves);
  }
}

// Leading dimension (elements) of a bf16 LDS tile: a multiple of 8 (16-byte
// rows) that is an odd multiple of 8, so that rows start in alternating
// 16-byte bank groups.
__host__ __device__ constexpr int lds_ld_bf16(int n) { return ((n + 7) & ~7) | 8; }

// Static LDS of the wide-tile kernel at R rows per tile (its root tables:
// three int64 and four int32 entries per row, two roles where they differ).
__host__ __device__ constexpr size_t wide_static_lds(int R) { return size_t(R) * (5 * 8 + 5 * 4); }

template <typename WT>
__global__ __launch_bounds__(kGruBlock) void k_gru_mailbox(
    int D, int K, int F, const int32_t *__restrict__ num_roots,
    const int64_t *__restrict__ roots, const float *__restrict__ memory,
    float *__restrict__ mailbox, float *__restrict__ mailbox_ts,
    int32_t *__restrict__ next_mail_pos, const WT *__restrict__ w_ih,
    const WT *__restrict__ w_hh, const float *__restrict__ b_ih,
    const float *__restrict__ b_hh, const WT *__restrict__ wc_ih,
    const WT *__restrict__ wc_hh, const float *__restrict__ bc_ih,
    const float *__restrict__ bc_hh, const int64_t *__restrict__ src,
    const int64_t *__restrict__ dst, const float *__restrict__ efeat,
    const float *__restrict__ ts, const int64_t *__restrict__ batch_start,
    const unsigned long long *__restrict__ win_src,
    const unsigned long long *__restrict__ win_dst, const int32_t *__restrict__ cnt_src,
    const int32_t *__restrict__ cnt_dst, float *__restrict__ new_mem) {
  extern __shared__ __align__(16) float lds[];
  const int S = 2 * D + F;
  const int G = 3 * D;
  const int ldx = sgl::lds_ld(S), ldh = sgl::lds_ld(D), ldg = sgl::lds_ld(G);
  float *xs = lds;
  float *hs = xs + kTileRows * ldx;
  float *ms = hs + kTileRows * ldh;
  float *gi = ms + kTileRows * ldh;
  float *gh = gi + kTileRows * ldg;
  // bf16 weights: the products read bf16 copies of the tiles, written once
  // per value (the mailbox rows go to LDS as bf16 only; h and memory keep
  // their fp32 tiles for the gate combine)
  constexpr bool kBf = !std::is_same_v<WT, float>;
  const int lbx = lds_ld_bf16(S), lbh = lds_ld_bf16(D);
  uint16_t *xb = reinterpret_cast<uint16_t *>(xs);
  uint16_t *hb = reinterpret_cast<uint16_t *>(gh + kTileRows * ldg);
  uint16_t *mb = hb + kTileRows * lbh;
  auto to_bf = [](float v) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(v)); };
  __shared__ int64_t s_root[kTileRows], s_e[2][kTileRows];
  __shared__ int32_t s_cnt[2][kTileRows];
  const int U = *num_roots;

  if (batch_start != nullptr) {  // event arrays are the whole stream
    const int64_t off = *batch_start;
    src += off;
    dst += off;
    ts += off;
    efeat += off * F;
  }
  // tiles of 16 roots, strided over a bounded grid (uniform per workgroup)
  for (int r0 = blockIdx.x * kTileRows; r0 < U; r0 += gridDim.x * kTileRows) {
    // the thread index is made opaque per tile so that the per-thread index
    // arithmetic (divisions by D and S, message column masks) is recomputed
    // in each tile rather than kept live across the loop
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    const int tid = t, wave = t >> 6, lane = t & 63;
    const int nrows = min(kTileRows, U - r0);
    if (tid < kTileRows) {
      const bool ok = tid < nrows;
      s_root[tid] = ok ? roots[r0 + tid] : 0;
      s_cnt[0][tid] = ok ? cnt_src[r0 + tid] : 0;
      s_cnt[1][tid] = ok ? cnt_dst[r0 + tid] : 0;
      s_e[0][tid] = ok ? int64_t(win_src[r0 + tid] & 0xffffffffull) : 0;
      s_e[1][tid] = ok ? int64_t(win_dst[r0 + tid] & 0xffffffffull) : 0;
    }
    __syncthreads();
    for (int idx = tid; idx < kTileRows * D; idx += kGruBlock) {
      const int i = idx / D, j = idx - i * D;
      const float mv = i < nrows ? memory[s_root[i] * D + j] : 0.f;
      ms[i * ldh + j] = mv;
      hs[i * ldh + j] = 0.f;
      if constexpr (kBf) {
        mb[i * lbh + j] = to_bf(mv);
        hb[i * lbh + j] = 0;
      }
    }
    // Mailbox messages (memory.py:218-248): the src-role message of node u is
    // [mem(u) || mem(other) || f_e] of its last src event e, the dst-role one
    // the same for its last dst event. Prefetch the foreign parts.
    const int i_msg = wave;
    const bool msg_row = i_msg < nrows;
    float part[2][kMaxMsgSlots];
    float ts_e[2] = {0.f, 0.f};
    int p_slot = 0;
    if (msg_row) {
      const int64_t u = s_root[i_msg];
      p_slot = next_mail_pos[u];
#pragma unroll
      for (int role = 0; role < 2; ++role) {
        const bool has = s_cnt[role][i_msg] > 0;
        const int64_t e = s_e[role][i_msg];
        const int64_t other = has ? (role == 0 ? dst[e] : src[e]) : 0;
        if (has) ts_e[role] = ts[e];
#pragma unroll
        for (int jj = 0; jj < kMaxMsgSlots; ++jj) {
          const int c = lane + 64 * jj;
          float v = 0.f;
          if (has && c >= D && c < 2 * D) v = memory[other * D + (c - D)];
          else if (has && c >= 2 * D && c < S) v = efeat[e * F + (c - 2 * D)];
          part[role][jj] = v;
        }
      }
    }
    // GRU layer over the K mailbox slots in slot-index order, h0 = 0
    for (int k = 0; k < K; ++k) {
      for (int idx = tid; idx < kTileRows * S; idx += kGruBlock) {
        const int i = idx / S, j = idx - (idx / S) * S;
        const float xv = i < nrows ? mailbox[(s_root[i] * K + k) * S + j] : 0.f;
        if constexpr (kBf) xb[i * lbx + j] = to_bf(xv);
        else xs[i * ldx + j] = xv;
      }
      __syncthreads();
      if constexpr (kBf)
        gru_products<WT>(xb, lbx, w_ih, S, b_ih, gi, S, G, hb, lbh, w_hh, D, b_hh, gh, D, k > 0 ? G : 0, ldg);
      else
        gru_products<WT>(xs, ldx, w_ih, S, b_ih, gi, S, G, hs, ldh, w_hh, D, b_hh, gh, D, k > 0 ? G : 0, ldg);
      __syncthreads();
      for (int idx = tid; idx < kTileRows * D; idx += kGruBlock) {
        const int i = idx / D, j = idx - (idx / D) * D;
        const float *g1 = gi + i * ldg;
        float ghr, ghz, ghn;
        if (k > 0) {
          const float *g2 = gh + i * ldg;
          ghr = g2[j]; ghz = g2[D + j]; ghn = g2[2 * D + j];
        } else {  // W_hh h0 = 0
          ghr = b_hh[j]; ghz = b_hh[D + j]; ghn = b_hh[2 * D + j];
        }
        const float hv = gru_combine(g1[j], g1[D + j], g1[2 * D + j], ghr, ghz, ghn, hs[i * ldh + j]);
        hs[i * ldh + j] = hv;
        if constexpr (kBf) hb[i * lbh + j] = to_bf(hv);
      }
      __syncthreads();
    }
    // GRUCell(agg = h, memory)
    if constexpr (kBf)
      gru_products<WT>(hb, lbh, wc_ih, D, bc_ih, gi, D, G, mb, lbh, wc_hh, D, bc_hh, gh, D, G, ldg);
    else
      gru_products<WT>(hs, ldh, wc_ih, D, bc_ih, gi, D, G, ms, ldh, wc_hh, D, bc_hh, gh, D, G, ldg);
    __syncthreads();
    for (int idx = tid; idx < nrows * D; idx += kGruBlock) {
      const int i = idx / D, j = idx - (idx / D) * D;
      const float *g1 = gi + i * ldg;
      const float *g2 = gh + i * ldg;
      new_mem[size_t(r0 + i) * D + j] =
          gru_combine(g1[j], g1[D + j], g1[2 * D + j], g2[j], g2[D + j], g2[2 * D + j], ms[i * ldh + j]);
    }

    // Mailbox write: the src-role message goes to slot p = next_mail_pos[u],
    // the dst-role one to (p + #src occurrences) % K, so with one slot the dst
    // role wins; the pointer advances by both counts. Every read of this
    // root's mailbox rows happened before the barriers above.
    if (msg_row) {
      const int64_t u = s_root[i_msg];
      const int cs = s_cnt[0][i_msg], cd = s_cnt[1][i_msg];
      const int p2 = (p_slot + cs) % K;
      const bool write_src = cs > 0 && !(cd > 0 && p2 == p_slot);
#pragma unroll
      for (int role = 0; role < 2; ++role) {
        if (role == 0 && !write_src) continue;
        if (role == 1 && cd == 0) continue;
        const int slot = role == 0 ? p_slot : p2;
        float *out = mailbox + (u * K + slot) * S;
#pragma unroll
        for (int jj = 0; jj < kMaxMsgSlots; ++jj) {
          const int c = lane + 64 * jj;
          if (c < D) out[c] = ms[i_msg * ldh + c];
          else if (c < S) out[c] = part[role][jj];
        }
        if (lane == 0) mailbox_ts[u * K + slot] = ts_e[role];
      }
      if (lane == 0) next_mail_pos[u] = int32_t((int64_t(p_slot) + cs + cd) % K);
    }
    __syncthreads();  // the next tile reuses the shared root table and LDS tiles
  }
}

// ---------------------------------------------------------------------------
// Wide-tile bf16 GRU + mailbox kernel. A workgroup takes 16*RB roots and
// one wave per 16 hidden columns (a chunk; ceil(D/16) <= 12 waves). For its
// chunk a wave computes the three gates for every row of the tile: the r and
// z pre-activations of the input and hidden products share one accumulator
// each (they are only ever summed), n keeps two (r scales the hidden part),
// so a stage holds 4*RB MFMA accumulators and combines the gates in
// registers: no gate tile goes through LDS. Each weight fragment loaded from
// L2 feeds RB MFMAs (one per 16-row block), so the weight traffic per root
// falls by RB against the 16-root kernel. A wave keeps its chunk's fp32
// hidden state in registers across the K slots and publishes the bf16 copy
// that the next hidden product reads after the barrier that ends the
// products, together with the next slot's mailbox tile. Global reads are
// issued in flat batches over the whole workgroup (the memory tile with the
// first mailbox tile; the messages' parts for every root of the tile), so a
// tile waits for few memory round trips.
constexpr int kWideMaxChunks = 12;
constexpr int kWideDepthSmall = 4;  // weight prefetch depth, 16-root tiles
constexpr int kWideDepthLarge = 2;  // weight prefetch depth, 64-root tiles

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bf16_rsrc(const uint16_t *p, uint32_t elems) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  const uint32_t bytes = __builtin_amdgcn_readfirstlane(elems * 2u);
  uint16_t *u = reinterpret_cast<uint16_t *>((uint64_t(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, int(bytes), 0x00020000);
}

// Fragment-order copy of a bf16 GRU weight matrix W [3D][kd] (row-major,
// gates r, z, n) for the wide-tile kernel: element
//   (((g * nc + c) * nks + s) * 64 + l) * 8 + t,  nc = ceil(D/16), nks = ceil(kd/32),
// holds W[g*D + 16c + l%16][32s + 8(l/16) + t] (0 past D or kd): the B
// fragment of gate g, column chunk c and k step s for lane l of
// v_mfma_f32_16x16x32_bf16. A wave's 16-byte loads of one fragment are then
// one contiguous kilobyte (eight 128-byte lines) instead of sixteen row
// segments that straddle lines; the vector-memory path (address, tag and
// data cycles per line) is what the row-major loads were bound by.
__host__ __device__ inline int64_t gru_packed_elems(int D, int kd) {
  return 3ll * ((D + 15) / 16) * ((kd + 31) / 32) * 512;
}

// A[row][k .. k+8) of a bf16 LDS row (lda % 8 == 0, lda >= kd) with the
// elements at k >= kd zeroed: the 16 bytes at min(k, lda - 8) stay inside
// the row (k > lda - 8 means k >= kd: every element is zeroed).
__device__ __forceinline__ bf16x8_t load_a8_tail(const uint16_t *arow, int k, int kd, int lda) {
  sgl::u32x4 w = *reinterpret_cast<const sgl::u32x4 *>(arow + min(k, lda - 8));
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const uint32_t keep = (k + 2 * t < kd ? 0x0000ffffu : 0u) | (k + 2 * t + 1 < kd ? 0xffff0000u : 0u);
    w[t] &= keep;
  }
  return __builtin_bit_cast(bf16x8_t, w);
}

// acc_g[rb] += A[16 rb + i][0..kd) . W[g*D + n0 + i'][0..kd) for the three
// gates g of a GRU weight matrix W (its fragment-order copy Wp, chunk
// n0 / 16 of nc) and the RB 16-row blocks of the LDS tile A (lda % 8 == 0,
// lda >= kd). The gate fragments of a k step are loaded once and multiplied
// into every row block. The loads run P-1 steps ahead of the products
// through P register sets (the loop unrolled by P, so that no set is
// copied): an L2 round trip is long against one step's products, and each
// wave's steps are a serial chain. Only the last step (k past kd) masks A.
template <int RB, int P>
__device__ __forceinline__ void wide_gates(int lane, const uint16_t *A, int lda, int kd, const uint16_t *Wp, int nc,
                                           int n0, sgl::f32x4 (&a0)[RB], sgl::f32x4 (&a1)[RB],
                                           sgl::f32x4 (&a2)[RB]) {
  const int i = lane & 15, q = lane >> 4;
  const int nks = (kd + 31) >> 5, nfull = kd >> 5;
  const __amdgpu_buffer_rsrc_t wr = bf16_rsrc(Wp, uint32_t(3 * nc * nks) * 512u);
  // byte offsets: this lane's 16 bytes of gate 0's fragment at k step 0, and
  // the strides between k steps and gates
  const uint32_t lane0 = ((uint32_t(n0 >> 4) * uint32_t(nks)) * 64u + uint32_t(lane)) * 16u;
  const uint32_t gstride = uint32_t(nc * nks) * 1024u;
  const uint16_t *arow = A + i * lda + 8 * q;
  auto load = [&](bf16x8_t (&b)[3], int ks) {
    const uint32_t o = lane0 + 1024u * uint32_t(ks);
#pragma unroll
    for (int g = 0; g < 3; ++g)
      b[g] = __builtin_bit_cast(bf16x8_t, __builtin_amdgcn_raw_buffer_load_b128(wr, int(o + g * gstride), 0, 0));
  };
  auto mma = [&](const bf16x8_t (&b)[3], const bf16x8_t (&a)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      a0[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb], b[0], a0[rb], 0, 0, 0);
      a1[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb], b[1], a1[rb], 0, 0, 0);
      a2[rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[rb], b[2], a2[rb], 0, 0, 0);
    }
  };
  auto step_full = [&](const bf16x8_t (&b)[3], int ks) {
    bf16x8_t a[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) a[rb] = *reinterpret_cast<const bf16x8_t *>(arow + 16 * rb * lda + 32 * ks);
    mma(b, a);
  };
  bf16x8_t b[P][3];
#pragma unroll
  for (int u = 0; u < P - 1; ++u) load(b[u], u);
  int ks = 0;
  // groups of P full steps; the scheduling barriers keep each load ahead of
  // the products it overlaps
  for (; ks + P <= nfull; ks += P) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      load(b[(u + P - 1) % P], ks + u + P - 1);
      __builtin_amdgcn_sched_barrier(0);
      step_full(b[u], ks + u);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // the remaining nks - ks <= P steps: sets 0 .. P-2 hold steps ks .. ks+P-2
  load(b[P - 1], ks + P - 1);
#pragma unroll
  for (int u = 0; u < P; ++u) {
    const int kk = ks + u;
    if (kk < nfull) {
      step_full(b[u], kk);
    } else if (kk < nks) {
      bf16x8_t a[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) a[rb] = load_a8_tail(A + (16 * rb + i) * lda, 32 * kk + 8 * q, kd, lda);
      mma(b[u], a);
    }
  }
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const uint32_t lo = __builtin_bit_cast(uint16_t, static_cast<__bf16>(a));
  const uint32_t hi = __builtin_bit_cast(uint16_t, static_cast<__bf16>(b));
  return lo | (hi << 16);
}

// One fp32 -> bf16 row-tile copy: rows [0, R) x columns [0, 4*n4) of the
// rows at base + row_off(i) (16-byte aligned) into an LDS tile with leading
// dimension ld; rows >= nrows read 0.
template <typename RowOff>
struct TileCopy {
  uint16_t *tile;
  int ld;
  const float *base;
  RowOff row_off;
  int n4;
};

// Up to two tile copies as one flat index space, NB loads per thread issued
// before their stores (one memory round trip per NB * blockDim.x vectors).
// Branch-free: rows past nrows and positions past the end load the last live
// row (their values land in padding rows whose outputs are discarded, or
// nowhere), so the loads issue back to back (nrows > 0).
template <int R, int NB, typename C0, typename C1>
__device__ __forceinline__ void tiles_to_bf16(const C0 &c0, const C1 *c1, int nrows) {
  const int nthr = blockDim.x;
  const int t0 = R * c0.n4;
  const int total = t0 + (c1 != nullptr ? R * c1->n4 : 0);
  for (int f0 = threadIdx.x; f0 < total; f0 += NB * nthr) {
    sgl::f32x4 v[NB];
    int at[NB];  // LDS element offset within the region's tile, -1: none
    bool second[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      const int f = min(f0 + u * nthr, total - 1);
      const bool in1 = f >= t0;
      const int g = in1 ? f - t0 : f;
      const int n4 = in1 ? c1->n4 : c0.n4;
      const int i = g / n4, c4 = g - i * n4;
      const int il = min(i, nrows - 1);
      const float *p = in1 ? c1->base + c1->row_off(il) + 4 * c4 : c0.base + c0.row_off(il) + 4 * c4;
      v[u] = *reinterpret_cast<const sgl::f32x4 *>(p);
      at[u] = f0 + u * nthr < total ? i * (in1 ? c1->ld : c0.ld) + 4 * c4 : -1;
      second[u] = in1;
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < NB; ++u) {
      if (at[u] < 0) continue;
      uint16_t *tile = second[u] ? c1->tile : c0.tile;
      *reinterpret_cast<u32x2_t *>(tile + at[u]) =
          u32x2_t{pack_bf16x2(v[u][0], v[u][1]), pack_bf16x2(v[u][2], v[u][3])};
    }
  }
}

template <typename RowOff>
__device__ __forceinline__ TileCopy<RowOff> tile_copy(uint16_t *tile, int ld, const float *base, RowOff f, int n4) {
  return TileCopy<RowOff>{tile, ld, base, f, n4};
}

// packed: the fragment-order copies of W_ih, W_hh, the cell's W_ih and W_hh
// one after another (sgl_gru_pack_bf16); P: the weight prefetch depth.
template <int RB, int P>
__global__ __launch_bounds__(kWideMaxChunks * 64) void k_gru_mailbox_wide(
    int D, int K, int F, const int32_t *__restrict__ num_roots, const int64_t *__restrict__ roots,
    const float *__restrict__ memory, float *__restrict__ mailbox, float *__restrict__ mailbox_ts,
    int32_t *__restrict__ next_mail_pos, const uint16_t *__restrict__ packed,
    const float *__restrict__ b_ih, const float *__restrict__ b_hh, const float *__restrict__ bc_ih,
    const float *__restrict__ bc_hh,
    const int64_t *__restrict__ src, const int64_t *__restrict__ dst, const float *__restrict__ efeat,
    const float *__restrict__ ts, const int64_t *__restrict__ batch_start,
    const unsigned long long *__restrict__ win_src, const unsigned long long *__restrict__ win_dst,
    const int32_t *__restrict__ cnt_src, const int32_t *__restrict__ cnt_dst, float *__restrict__ new_mem) {
  constexpr int R = 16 * RB;
  // loads in flight per thread in the tile copies and the message copy: one
  // batch per copy at these tile sizes (the last batch repeats positions).
  // With D = 172, F = 16 (11 waves): the memory and first mailbox tiles are
  // 64 x (43 + 90) float4, 12.1 per thread; the messages 64 x 2 x 90, 16.4
  // per thread. (17 tile loads per thread spill; 13 do not.)
  constexpr int NB = RB >= 4 ? 13 : 4;
  constexpr int MB = RB >= 4 ? 17 : 4;
  extern __shared__ __align__(16) float lds[];
  const int S = 2 * D + F;
  const int lbx = lds_ld_bf16(S), lbh = lds_ld_bf16(D);
  const int ldf = sgl::lds_ld(D);
  float *hf = lds;                                                     // fp32 hidden state
  uint16_t *xb = reinterpret_cast<uint16_t *>(hf + R * ldf);          // mailbox tile
  uint16_t *hb = xb + R * lbx;                                         // hidden tile (bf16)
  uint16_t *mb = hb + R * lbh;                                         // memory tile
  __shared__ int64_t s_root[R], s_e[2][R], s_other[2][R];
  __shared__ int32_t s_cnt[2][R], s_pos[R], s_slot[2][R];
  static_assert(sizeof(s_root) + sizeof(s_e) + sizeof(s_other) + sizeof(s_cnt) + sizeof(s_pos) + sizeof(s_slot) ==
                    wide_static_lds(R),
                "wide_static_lds must count the kernel's static LDS");
  const int U = *num_roots;
  const int nthr = blockDim.x;
  const int S4 = S >> 2, D4 = D >> 2;
  const int nc = (D + 15) >> 4;
  const uint16_t *pk_ih = packed, *pk_hh = pk_ih + gru_packed_elems(D, S);
  const uint16_t *pkc_ih = pk_hh + gru_packed_elems(D, D), *pkc_hh = pkc_ih + gru_packed_elems(D, D);
  // The thread index is made opaque at the start of each stage, so that the
  // stage's per-lane address arithmetic is recomputed there rather than
  // hoisted out of the tile and slot loops and kept live (in registers the
  // MFMA accumulators need) across the whole kernel.
  auto opaque_tid = [] {
    int t = int(threadIdx.x);
    asm volatile("" : "+v"(t));
    return t;
  };

  if (batch_start != nullptr) {  // event arrays are the whole stream
    const int64_t off = *batch_start;
    src += off;
    dst += off;
    ts += off;
    efeat += off * F;
  }
  for (int r0 = blockIdx.x * R; r0 < U; r0 += gridDim.x * R) {
    const int nrows = min(R, U - r0);
    for (int t = threadIdx.x; t < R; t += nthr) {
      const bool ok = t < nrows;
      s_root[t] = ok ? roots[r0 + t] : 0;
      s_cnt[0][t] = ok ? cnt_src[r0 + t] : 0;
      s_cnt[1][t] = ok ? cnt_dst[r0 + t] : 0;
      // the event of each role (0 for a role without events: a valid index)
      s_e[0][t] = ok && cnt_src[r0 + t] > 0 ? int64_t(win_src[r0 + t] & 0xffffffffull) : 0;
      s_e[1][t] = ok && cnt_dst[r0 + t] > 0 ? int64_t(win_dst[r0 + t] & 0xffffffffull) : 0;
    }
    __syncthreads();
    // the memory tile and the first mailbox tile in one batch; the roots'
    // slot pointers and the messages' other endpoints beside them
    {
      const int t = threadIdx.x;
      int pos = 0;
      int64_t oth[2] = {0, 0};
      if (t < nrows) {  // s_e is a valid event index for a role without events
        pos = next_mail_pos[s_root[t]];
        const int64_t o0 = dst[s_e[0][t]], o1 = src[s_e[1][t]];
        oth[0] = s_cnt[0][t] > 0 ? o0 : 0;
        oth[1] = s_cnt[1][t] > 0 ? o1 : 0;
      }
      const auto cm = tile_copy(mb, lbh, memory, [&](int i) { return s_root[i] * D; }, D4);
      const auto cx = tile_copy(xb, lbx, mailbox, [&](int i) { return s_root[i] * K * S; }, S4);
      tiles_to_bf16<R, NB>(cm, &cx, nrows);
      if (t < R) {
        s_pos[t] = pos;
        s_other[0][t] = oth[0];
        s_other[1][t] = oth[1];
      }
    }
    __syncthreads();
    // The fp32 hidden state lives in LDS (hf): each wave reads and writes
    // only its own chunk's columns, so it needs no barrier of its own, and
    // the registers stay with the MFMA accumulators and weight loads.
    // GRU layer over the K mailbox slots in slot-index order, h0 = 0
    for (int k = 0; k < K; ++k) {
      if (k > 0) {
        // publish the hidden state (bf16), then the slot's mailbox tile
        {
          const int t = opaque_tid(), lane = t & 63;
          const int j = 16 * (t >> 6) + (lane & 15);
          if (j < D) {
            for (int i = lane >> 4; i < R; i += 4)
              hb[i * lbh + j] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(hf[i * ldf + j]));
          }
        }
        const auto cx = tile_copy(xb, lbx, mailbox, [&](int i) { return (s_root[i] * K + k) * S; }, S4);
        tiles_to_bf16<R, NB>(cx, static_cast<const decltype(cx) *>(nullptr), nrows);
        __syncthreads();
      }
      const int t = opaque_tid(), lane = t & 63;
      const int n0 = 16 * (t >> 6);
      const int j = n0 + (lane & 15);
      const bool jok = j < D;
      const int jc = jok ? j : D - 1;
      const int rq = 4 * (lane >> 4);
      sgl::f32x4 ar[RB], az[RB], an[RB], ah[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) ar[rb] = az[rb] = an[rb] = ah[rb] = sgl::f32x4{0.f, 0.f, 0.f, 0.f};
      wide_gates<RB, P>(lane, xb, lbx, S, pk_ih, nc, n0, ar, az, an);
      if (k > 0) wide_gates<RB, P>(lane, hb, lbh, D, pk_hh, nc, n0, ar, az, ah);
      const float br = b_ih[jc] + b_hh[jc], bz = b_ih[D + jc] + b_hh[D + jc];
      const float bn = b_ih[2 * D + jc], bhn = b_hh[2 * D + jc];
      if (jok) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            float *hp = hf + (16 * rb + rq + v) * ldf + j;
            const float hold = k > 0 ? *hp : 0.f;
            const float r = gate_sigmoid(ar[rb][v] + br);
            const float z = gate_sigmoid(az[rb][v] + bz);
            const float nn = gate_tanh(an[rb][v] + bn + r * (ah[rb][v] + bhn));
            *hp = (1.f - z) * nn + z * hold;
          }
        }
      }
      __syncthreads();  // the mailbox and hidden tiles are consumed
    }
    // GRUCell(agg = h, memory)
    {
      const int t = opaque_tid(), lane = t & 63;
      const int j = 16 * (t >> 6) + (lane & 15);
      if (j < D) {
        for (int i = lane >> 4; i < R; i += 4)
          hb[i * lbh + j] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(hf[i * ldf + j]));
      }
    }
    __syncthreads();
    {
      const int t = opaque_tid(), lane = t & 63;
      const int n0 = 16 * (t >> 6);
      const int j = n0 + (lane & 15);
      const bool jok = j < D;
      const int jc = jok ? j : D - 1;
      const int rq = 4 * (lane >> 4);
      sgl::f32x4 ar[RB], az[RB], an[RB], ah[RB];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) ar[rb] = az[rb] = an[rb] = ah[rb] = sgl::f32x4{0.f, 0.f, 0.f, 0.f};
      wide_gates<RB, P>(lane, hb, lbh, D, pkc_ih, nc, n0, ar, az, an);
      wide_gates<RB, P>(lane, mb, lbh, D, pkc_hh, nc, n0, ar, az, ah);
      const float br = bc_ih[jc] + bc_hh[jc], bz = bc_ih[D + jc] + bc_hh[D + jc];
      const float bn = bc_ih[2 * D + jc], bhn = bc_hh[2 * D + jc];
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int i = 16 * rb + rq + v;
          if (!jok || i >= nrows) continue;
          const float m = memory[s_root[i] * D + j];
          const float r = gate_sigmoid(ar[rb][v] + br);
          const float z = gate_sigmoid(az[rb][v] + bz);
          const float nn = gate_tanh(an[rb][v] + bn + r * (ah[rb][v] + bhn));
          new_mem[size_t(r0 + i) * D + j] = (1.f - z) * nn + z * m;
        }
      }
    }
    // Mailbox write (memory.py:218-248), after every read of the tile's
    // mailbox rows (the barriers ending the slots): the src-role message
    // [mem(u) || mem(other) || f_e] of u's last src event goes to slot
    // p = next_mail_pos[u], the dst-role one to (p + #src occurrences) % K,
    // so with one slot the dst role wins; the pointer advances by both counts.
    // Slot -1: the role writes nothing.
    for (int t = threadIdx.x; t < nrows; t += nthr) {
      const int64_t u = s_root[t];
      const int p = s_pos[t], cs = s_cnt[0][t], cd = s_cnt[1][t];
      const int p2 = (p + cs) % K;
      const bool write_src = cs > 0 && !(cd > 0 && p2 == p);
      s_slot[0][t] = write_src ? p : -1;
      s_slot[1][t] = cd > 0 ? p2 : -1;
      if (write_src) mailbox_ts[u * K + p] = ts[s_e[0][t]];
      if (cd > 0) mailbox_ts[u * K + p2] = ts[s_e[1][t]];
      next_mail_pos[u] = int32_t((int64_t(p) + cs + cd) % K);
    }
    __syncthreads();
    {
      // the messages' parts, all loads of a batch issued before its stores
      // (a skipped role loads its root's own row and stores nothing)
      const int total = nrows * 2 * S4;
      for (int f0 = threadIdx.x; f0 < total; f0 += MB * nthr) {
        sgl::f32x4 v[MB];
        float *to[MB];
#pragma unroll
        for (int u = 0; u < MB; ++u) {
          const int f = min(f0 + u * nthr, total - 1);
          const int rt = f / S4, c4 = f - rt * S4;  // rt = 2 * root + role
          const int t = rt >> 1, role = rt & 1;
          const int slot = s_slot[role][t];
          const int64_t uu = s_root[t];
          const float *from = c4 < D4 ? memory + uu * D + 4 * c4
                                      : (c4 < 2 * D4 ? memory + s_other[role][t] * D + 4 * (c4 - D4)
                                                     : efeat + s_e[role][t] * F + 4 * (c4 - 2 * D4));
          v[u] = *reinterpret_cast<const sgl::f32x4 *>(from);
          to[u] = f0 + u * nthr < total && slot >= 0 ? mailbox + (uu * K + slot) * S + 4 * c4 : nullptr;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < MB; ++u)
          if (to[u] != nullptr) *reinterpret_cast<sgl::f32x4 *>(to[u]) = v[u];
      }
    }
    __syncthreads();  // the next tile reuses the shared root table and LDS tiles
  }
}

__global__ __launch_bounds__(kBlock) void k_memory_commit(
    int D, bool vec4, bool gather, int64_t cap, const int32_t *__restrict__ num_roots,
    const int64_t *__restrict__ roots, float *__restrict__ rows, float *__restrict__ memory,
    float *__restrict__ memory_ts, const float *__restrict__ ts_max, uint32_t *__restrict__ bits,
    const int32_t *__restrict__ sample_cnt, int32_t *__restrict__ any_edges, float *__restrict__ root_dt) {
  // grid-stride over the live roots' elements (the grid is bounded, so a
  // large capacity with few live roots costs no idle workgroups), four at a
  // time when the rows allow 16-byte accesses. Commit: memory[roots[r]] =
  // rows[r] and memory_ts = ts_max; gather (no memory updater): rows[r] =
  // memory[roots[r]]. Both clear the roots' bitmap words and set the gate.
  const int64_t nr = min(cap, int64_t(*num_roots));
  const float tmax = gather ? 0.0f : *ts_max;
  const int W = vec4 ? D >> 2 : D;
  const int64_t live = nr * W;
  for (int64_t idx = int64_t(blockIdx.x) * kBlock + threadIdx.x; idx < live; idx += int64_t(gridDim.x) * kBlock) {
    const int64_t r = idx / W;
    const int j = int(idx - r * W);
    const int64_t u = roots[r];
    if (vec4) {
      float4 *m4 = reinterpret_cast<float4 *>(memory) + u * W + j;
      float4 *r4 = reinterpret_cast<float4 *>(rows) + r * W + j;
      if (gather) *r4 = *m4; else *m4 = *r4;
    } else {
      if (gather) rows[r * D + j] = memory[u * D + j]; else memory[u * D + j] = rows[r * D + j];
    }
    if (j == 0) {
      if (!gather) {
        if (root_dt != nullptr) root_dt[r] = tmax - memory_ts[u];  // time since the root's last update
        memory_ts[u] = tmax;
      }
      bits[u >> 5] = 0u;  // leave the bitmap clear for the next step
      if (sample_cnt != nullptr && sample_cnt[r] > 0) *any_edges = 1;
    }
  }
}

// Negative destinations from uniform draws over the sorted dst pool
// (runtime.py:124-136): neg = pool[i]; when it equals the event's dst the
// draw moves to the next pool entry (once, as there). In place: draw and neg
// may be the same array (each element is read, then written by one thread).
__global__ __launch_bounds__(kBlock) void k_negatives(int64_t n, const int64_t *draw, const int64_t *__restrict__ pool,
                                                      int64_t pool_size, const int64_t *__restrict__ dst,
                                                      int64_t *neg, int32_t *__restrict__ err) {
  for (int64_t e = int64_t(blockIdx.x) * kBlock + threadIdx.x; e < n; e += int64_t(gridDim.x) * kBlock) {
    int64_t i = draw[e];
    if (i < 0 || i >= pool_size) {
      if (err != nullptr) atomicOr(err, SGL_DERR_NODE_RANGE);
      i = 0;
    }
    int64_t v = pool[i];
    if (v == dst[e]) {
      i = i + 1 == pool_size ? 0 : i + 1;
      v = pool[i];
    }
    neg[e] = v;
  }
}

}  // namespace

extern "C" int sgl_negatives_from_draws(int64_t n, const int64_t *draw, const int64_t *pool, int64_t pool_size,
                                        const int64_t *dst, int64_t *neg, int32_t *err_flag, hipStream_t stream) {
  SGL_REQUIRE(n >= 0, "negatives: n < 0");
  if (n == 0) return SGL_OK;
  SGL_REQUIRE(pool_size > 0, "negatives: empty dst pool");
  SGL_REQUIRE(draw && pool && dst && neg, "negatives: NULL array");
  const unsigned grid = unsigned(std::min<int64_t>((n + kBlock - 1) / kBlock, sgl::kMaxGrid));
  k_negatives<<<grid, kBlock, 0, stream>>>(n, draw, pool, pool_size, dst, neg, err_flag);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int64_t sgl_node_bits_words(int64_t num_nodes) {
  return num_nodes > 0 ? bitmap_words(num_nodes) + summary_words(num_nodes) : 0;
}

static int batch_prepare(int64_t num_nodes, int64_t batch, const int64_t *src, const int64_t *dst,
                         const int64_t *neg, const float *ts, int64_t *cursor, int64_t *batch_start,
                         uint32_t *node_bits, int32_t *word_prefix, int32_t *num_roots, int64_t *num_roots64,
                         float *ts_max, int64_t *t_query, int64_t *roots, int64_t *root_ts, int32_t *ridx_src,
                         int32_t *ridx_dst, int32_t *ridx_neg, uint64_t *win_src, uint64_t *win_dst,
                         int32_t *cnt_src, int32_t *cnt_dst, int32_t *any_edges, int32_t *err_flag,
                         const sgl::met::Args *metrics, hipStream_t stream) {
  SGL_REQUIRE(num_nodes > 0 && num_nodes < INT_MAX, "batch_prepare: num_nodes %lld out of range", (long long)num_nodes);
  SGL_REQUIRE(batch >= 0 && batch < (INT_MAX / 2), "batch_prepare: batch %lld out of range", (long long)batch);
  SGL_REQUIRE(node_bits && word_prefix && num_roots && num_roots64 && ts_max && t_query && any_edges,
              "batch_prepare: NULL state array");
  SGL_REQUIRE(cursor == nullptr || batch_start != nullptr, "batch_prepare: cursor without batch_start");
  SGL_REQUIRE((reinterpret_cast<uintptr_t>(node_bits) & 15u) == 0, "batch_prepare: node_bits not 16-byte aligned");
  SGL_REQUIRE(batch == 0 || (src && dst && ts && roots && root_ts && ridx_src && ridx_dst && win_src && win_dst &&
                             cnt_src && cnt_dst && (neg == nullptr || ridx_neg)),
              "batch_prepare: NULL batch array");
  const int64_t cap = 2 * batch;
  const sgl::PlanGate gate = sgl::take_gate();  // a launch plan's gate (folded, or its own kernel first)
  if (batch <= kPrepMaxBatch) {
    const sgl::met::Args none{};
    const sgl::met::Args &mr = metrics != nullptr ? *metrics : none;
    size_t lds = (2 * sizeof(unsigned long long) + 2 * sizeof(int32_t)) * size_t(cap > 0 ? cap : 1);
    if (metrics != nullptr) lds = std::max(lds, sgl::met::lds_bytes(mr.P, mr.N));
    const unsigned grid = 1u + (metrics != nullptr ? unsigned(sgl::met::blocks_for(mr.P)) : 0u);
    SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(&k_step_prepare_wg), lds));
    sgl::launch(&k_step_prepare_wg, dim3(grid), dim3(kPrepBlock), lds, stream, batch, num_nodes, cap, src, dst, neg,
                ts, cursor, batch_start, node_bits, word_prefix, num_roots, num_roots64, ts_max, t_query, roots,
                root_ts, ridx_src, ridx_dst, ridx_neg, reinterpret_cast<unsigned long long *>(win_src),
                reinterpret_cast<unsigned long long *>(win_dst), cnt_src, cnt_dst, any_edges, err_flag, gate.word,
                gate.value, gate.timeout, mr);
    SGL_CHECK_LAUNCH();
    return SGL_OK;
  }
  SGL_REQUIRE(metrics == nullptr, "batch_prepare: metrics ride only on the one-workgroup preparation");
  if (gate.word != nullptr)
    if (int rc = sgl::launch_gate(gate, stream)) return rc;
  SGL_REQUIRE((reinterpret_cast<uintptr_t>(word_prefix) & 15u) == 0, "batch_prepare: word_prefix not 16-byte aligned");
  const int64_t nwords = bitmap_words(num_nodes);  // a multiple of 4, padding words zero
  uint32_t *ts_slot = node_bits + nwords;          // the first summary word
  const bool small = batch <= kAggSmallMax;
  const int64_t per_wg = small ? kAggSmallBlock : kAggEvents;
  const unsigned grid = unsigned(std::max<int64_t>(1, (batch + per_wg - 1) / per_wg));
  auto *ws = reinterpret_cast<unsigned long long *>(win_src);
  auto *wd = reinterpret_cast<unsigned long long *>(win_dst);
  if (small)
    k_step_mark<kAggSmallBlock, 1, kMarkSmallLog2><<<grid, kAggSmallBlock, 0, stream>>>(
        batch, num_nodes, cap, src, dst, ts, cursor, batch_start, node_bits, ts_slot, ws, wd, cnt_src, cnt_dst,
        any_edges, err_flag);
  else
    k_step_mark<kAggBlock, kAggPer, kMarkLog2><<<grid, kAggBlock, 0, stream>>>(
        batch, num_nodes, cap, src, dst, ts, cursor, batch_start, node_bits, ts_slot, ws, wd, cnt_src, cnt_dst,
        any_edges, err_flag);
  SGL_CHECK_LAUNCH();
  k_step_scan<<<1, kScanBlock, 0, stream>>>(nwords, nwords + summary_words(num_nodes), node_bits, word_prefix,
                                            num_roots, num_roots64, batch, ts_slot, cursor, batch_start, ts_max,
                                            t_query, err_flag);
  SGL_CHECK_LAUNCH();
  if (batch > 0) {
    const int64_t *bs = cursor != nullptr ? batch_start : nullptr;
    if (small)
      k_step_index<kAggSmallBlock, 1, kIdxSmallLog2><<<grid, kAggSmallBlock, 0, stream>>>(
          batch, num_nodes, num_roots, src, dst, neg, ts, bs, node_bits, word_prefix, t_query, roots, root_ts,
          ridx_src, ridx_dst, ridx_neg, ws, wd, cnt_src, cnt_dst);
    else
      k_step_index<kAggBlock, kAggPer, kIdxLog2><<<grid, kAggBlock, 0, stream>>>(
          batch, num_nodes, num_roots, src, dst, neg, ts, bs, node_bits, word_prefix, t_query, roots, root_ts,
          ridx_src, ridx_dst, ridx_neg, ws, wd, cnt_src, cnt_dst);
    SGL_CHECK_LAUNCH();
  }
  return SGL_OK;
}

extern "C" int sgl_batch_prepare(int64_t num_nodes, int64_t batch, const int64_t *src, const int64_t *dst,
                                 const int64_t *neg, const float *ts, int64_t *cursor, int64_t *batch_start,
                                 uint32_t *node_bits,
                                 int32_t *word_prefix, int32_t *num_roots, int64_t *num_roots64,
                                 float *ts_max, int64_t *t_query, int64_t *roots, int64_t *root_ts,
                                 int32_t *ridx_src, int32_t *ridx_dst, int32_t *ridx_neg,
                                 uint64_t *win_src, uint64_t *win_dst, int32_t *cnt_src, int32_t *cnt_dst,
                                 int32_t *any_edges, int32_t *err_flag, hipStream_t stream) {
  return batch_prepare(num_nodes, batch, src, dst, neg, ts, cursor, batch_start, node_bits, word_prefix, num_roots,
                       num_roots64, ts_max, t_query, roots, root_ts, ridx_src, ridx_dst, ridx_neg, win_src, win_dst,
                       cnt_src, cnt_dst, any_edges, err_flag, nullptr, stream);
}

extern "C" int sgl_batch_prepare_metrics(
    int64_t num_nodes, int64_t batch, const int64_t *src, const int64_t *dst, const int64_t *neg, const float *ts,
    int64_t *cursor, int64_t *batch_start, uint32_t *node_bits, int32_t *word_prefix, int32_t *num_roots,
    int64_t *num_roots64, float *ts_max, int64_t *t_query, int64_t *roots, int64_t *root_ts, int32_t *ridx_src,
    int32_t *ridx_dst, int32_t *ridx_neg, uint64_t *win_src, uint64_t *win_dst, int32_t *cnt_src, int32_t *cnt_dst,
    int32_t *any_edges, int32_t *err_flag, int32_t n_pos, int32_t n_neg, const float *pos_logits,
    const float *neg_logits, const float *loss, uint64_t *seq, double *ring, int32_t ring_slots, double *out,
    double *work, uint32_t *done, hipStream_t stream) {
  SGL_REQUIRE(n_pos >= 0 && n_neg >= 0 && int64_t(n_pos) + n_neg <= SGL_LINK_METRICS_MAX_SCORES,
              "batch_prepare_metrics: %d positive + %d negative scores (at most %d)", n_pos, n_neg,
              SGL_LINK_METRICS_MAX_SCORES);
  SGL_REQUIRE((n_pos == 0 || pos_logits) && (n_neg == 0 || neg_logits), "batch_prepare_metrics: NULL logits");
  SGL_REQUIRE(ring == nullptr || (seq != nullptr && ring_slots > 0),
              "batch_prepare_metrics: a ring needs seq and slots");
  SGL_REQUIRE(ring != nullptr || out != nullptr, "batch_prepare_metrics: no metrics output");
  SGL_REQUIRE(work != nullptr && done != nullptr, "batch_prepare_metrics: NULL work or done word");
  if (batch > kPrepMaxBatch) {   // the multi-kernel preparation, then the metrics' own launch
    if (int rc = batch_prepare(num_nodes, batch, src, dst, neg, ts, cursor, batch_start, node_bits, word_prefix,
                               num_roots, num_roots64, ts_max, t_query, roots, root_ts, ridx_src, ridx_dst, ridx_neg,
                               win_src, win_dst, cnt_src, cnt_dst, any_edges, err_flag, nullptr, stream))
      return rc;
    return sgl_link_metrics(n_pos, n_neg, pos_logits, neg_logits, loss, seq, ring, ring_slots, out, work, done,
                            stream);
  }
  const sgl::met::Args mr{int(n_pos), int(n_neg), pos_logits, neg_logits, loss,
                          reinterpret_cast<unsigned long long *>(seq), ring, int(ring_slots), out, work,
                          reinterpret_cast<unsigned int *>(done)};
  return batch_prepare(num_nodes, batch, src, dst, neg, ts, cursor, batch_start, node_bits, word_prefix, num_roots,
                       num_roots64, ts_max, t_query, roots, root_ts, ridx_src, ridx_dst, ridx_neg, win_src, win_dst,
                       cnt_src, cnt_dst, any_edges, err_flag, &mr, stream);
}

extern "C" size_t sgl_memory_update_lds_bytes(int32_t D, int32_t F) {
  const size_t S = size_t(2 * D + F), G = size_t(3 * D);
  return sizeof(float) * kTileRows * (sgl::lds_ld(int(S)) + 2 * sgl::lds_ld(D) + 2 * sgl::lds_ld(int(G)));
}

// Dynamic LDS of the wide-tile kernel: the fp32 hidden state and the bf16
// mailbox, hidden and memory tiles
static size_t wide_lds_bytes(int D, int F, int rows) {
  return sizeof(float) * size_t(rows) * size_t(sgl::lds_ld(D)) +
         sizeof(uint16_t) * size_t(rows) * (size_t(lds_ld_bf16(2 * D + F)) + 2 * size_t(lds_ld_bf16(D)));
}

static bool host_aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rows per tile of the wide-tile kernel: 16 for batches that give fewer
// tiles than CUs, 64 once a batch has 64-root tiles for every CU; 0 when the
// shape does not fit it (float4 rows, at most 12 chunks, LDS) or the caller
// passed no fragment-order weight copy.
static int wide_rows_for_shape(int D, int F, int64_t capacity) {
  if (D <= 0 || F < 0 || D % 4 != 0 || F % 4 != 0 || (D + 15) / 16 > kWideMaxChunks) return 0;
  // dynamic plus static LDS (the kernel's root tables) within the CU's 160 KiB;
  // 64-root tiles that do not fit fall back to 16-root tiles
  const auto fits = [&](int rows) { return wide_lds_bytes(D, F, rows) + wide_static_lds(rows) <= 160 * 1024; };
  if (capacity >= 64 * 256 && fits(64)) return 64;
  return fits(16) ? 16 : 0;
}

static int wide_rows(int D, int F, int64_t capacity, const float *memory, const float *mailbox,
                     const float *new_mem, const float *efeat, const uint16_t *packed) {
  if (packed == nullptr) return 0;
  if (!host_aligned16(memory) || !host_aligned16(mailbox) || !host_aligned16(new_mem) ||
      (F > 0 && !host_aligned16(efeat)) || !host_aligned16(packed))
    return 0;
  return wide_rows_for_shape(D, F, capacity);
}

template <int RB, int P>
static int launch_wide(int32_t D, int32_t K, int32_t F, int64_t capacity, const int32_t *num_roots,
                       const int64_t *roots, const float *memory, float *mailbox, float *mailbox_ts,
                       int32_t *next_mail_pos, const uint16_t *packed, const float *b_ih, const float *b_hh,
                       const float *bc_ih, const float *bc_hh, const int64_t *src, const int64_t *dst,
                       const float *efeat, const float *ts, const int64_t *batch_start, const uint64_t *win_src,
                       const uint64_t *win_dst, const int32_t *cnt_src, const int32_t *cnt_dst, float *new_mem,
                       hipStream_t stream) {
  auto kern = &k_gru_mailbox_wide<RB, P>;
  const size_t wl = wide_lds_bytes(D, F, 16 * RB);
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(kern), wl));
  const unsigned grid = unsigned(std::min<int64_t>((capacity + 16 * RB - 1) / (16 * RB), sgl::kMaxGrid));
  sgl::launch(kern, dim3(grid), dim3(sgl::kWave * ((D + 15) / 16)), wl, stream, D, K, F, num_roots, roots, memory,
              mailbox, mailbox_ts, next_mail_pos, packed, b_ih, b_hh, bc_ih, bc_hh, src, dst,
              efeat, ts, batch_start, reinterpret_cast<const unsigned long long *>(win_src),
              reinterpret_cast<const unsigned long long *>(win_dst), cnt_src, cnt_dst, new_mem);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

template <typename WT>
static int memory_update(int32_t D, int32_t K, int32_t F, int64_t capacity, const int32_t *num_roots, const int64_t *roots,
                  const float *memory, float *mailbox, float *mailbox_ts, int32_t *next_mail_pos, const WT *w_ih,
                  const WT *w_hh, const float *b_ih, const float *b_hh, const WT *wc_ih, const WT *wc_hh,
                  const float *bc_ih, const float *bc_hh, const int64_t *src, const int64_t *dst, const float *efeat,
                  const float *ts, const int64_t *batch_start, const uint64_t *win_src, const uint64_t *win_dst,
                  const int32_t *cnt_src, const int32_t *cnt_dst, float *new_mem, const uint16_t *packed,
                  hipStream_t stream) {
  SGL_REQUIRE(D > 0 && K > 0 && F >= 0, "memory_update: bad dims D=%d K=%d F=%d", D, K, F);
  SGL_REQUIRE(capacity >= 0 && capacity < INT_MAX, "memory_update: capacity out of range");
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && roots && memory && mailbox && mailbox_ts && next_mail_pos && w_ih && w_hh && b_ih &&
                  b_hh && wc_ih && wc_hh && bc_ih && bc_hh && src && dst && ts && win_src && win_dst &&
                  cnt_src && cnt_dst && new_mem && (F == 0 || efeat),
              "memory_update: NULL array");
  // the bf16 variant adds bf16 copies of the h and memory tiles (the mailbox tile's reuses the fp32 one)
  const size_t lds = sgl_memory_update_lds_bytes(D, F) +
                     (std::is_same_v<WT, float> ? 0 : sizeof(uint16_t) * 2 * kTileRows * size_t(lds_ld_bf16(D)));
  SGL_REQUIRE(lds <= 160 * 1024, "memory_update: D=%d F=%d needs %zu bytes of LDS (> 160 KiB)", D, F, lds);
  SGL_REQUIRE(2 * D + F <= 64 * kMaxMsgSlots, "memory_update: message width 2D+F = %d exceeds %d", 2 * D + F,
              64 * kMaxMsgSlots);
  if constexpr (!std::is_same_v<WT, float>) {
    const int rows = wide_rows(D, F, capacity, memory, mailbox, new_mem, efeat, packed);
    if (rows > 0) {
      const auto fn = rows == 64 ? &launch_wide<4, kWideDepthLarge> : &launch_wide<1, kWideDepthSmall>;
      return fn(D, K, F, capacity, num_roots, roots, memory, mailbox, mailbox_ts, next_mail_pos, packed, b_ih, b_hh,
                bc_ih, bc_hh, src, dst, efeat, ts, batch_start, win_src, win_dst, cnt_src, cnt_dst, new_mem, stream);
    }
  }
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(&k_gru_mailbox<WT>), lds));
  const unsigned grid = unsigned(std::min<int64_t>((capacity + kTileRows - 1) / kTileRows, sgl::kMaxGrid));
  sgl::launch(&k_gru_mailbox<WT>, dim3(grid), dim3(kGruBlock), lds, stream, D, K, F, num_roots, roots, memory,
              mailbox, mailbox_ts, next_mail_pos, w_ih, w_hh, b_ih, b_hh, wc_ih, wc_hh, bc_ih, bc_hh, src, dst,
              efeat, ts, batch_start, reinterpret_cast<const unsigned long long *>(win_src),
              reinterpret_cast<const unsigned long long *>(win_dst), cnt_src, cnt_dst, new_mem);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int32_t sgl_memory_update_bf16_tile_rows(int32_t D, int32_t F, int64_t capacity) {
  return wide_rows_for_shape(D, F, capacity);
}

extern "C" int sgl_memory_update(int32_t D, int32_t K, int32_t F, int64_t capacity, const int32_t *num_roots,
                                 const int64_t *roots, const float *memory, float *mailbox, float *mailbox_ts,
                                 int32_t *next_mail_pos, const float *w_ih, const float *w_hh, const float *b_ih,
                                 const float *b_hh, const float *wc_ih, const float *wc_hh, const float *bc_ih,
                                 const float *bc_hh, const int64_t *src, const int64_t *dst, const float *efeat,
                                 const float *ts, const int64_t *batch_start, const uint64_t *win_src,
                                 const uint64_t *win_dst,
                                 const int32_t *cnt_src, const int32_t *cnt_dst, float *new_mem,
                                 hipStream_t stream) {
  return memory_update<float>(D, K, F, capacity, num_roots, roots, memory, mailbox, mailbox_ts, next_mail_pos, w_ih,
                              w_hh, b_ih, b_hh, wc_ih, wc_hh, bc_ih, bc_hh, src, dst, efeat, ts, batch_start,
                              win_src, win_dst, cnt_src, cnt_dst, new_mem, nullptr, stream);
}

extern "C" int sgl_memory_update_bf16(int32_t D, int32_t K, int32_t F, int64_t capacity, const int32_t *num_roots,
                                      const int64_t *roots, const float *memory, float *mailbox, float *mailbox_ts,
                                      int32_t *next_mail_pos, const uint16_t *w_ih, const uint16_t *w_hh,
                                      const float *b_ih, const float *b_hh, const uint16_t *wc_ih,
                                      const uint16_t *wc_hh, const float *bc_ih, const float *bc_hh,
                                      const int64_t *src, const int64_t *dst, const float *efeat, const float *ts,
                                      const int64_t *batch_start, const uint64_t *win_src, const uint64_t *win_dst,
                                      const int32_t *cnt_src, const int32_t *cnt_dst, float *new_mem,
                                      const uint16_t *packed, hipStream_t stream) {
  return memory_update<uint16_t>(D, K, F, capacity, num_roots, roots, memory, mailbox, mailbox_ts, next_mail_pos,
                                 w_ih, w_hh, b_ih, b_hh, wc_ih, wc_hh, bc_ih, bc_hh, src, dst, efeat, ts,
                                 batch_start, win_src, win_dst, cnt_src, cnt_dst, new_mem, packed, stream);
}

namespace {
// One thread per packed element: gather from the row-major bf16 matrix of its
// region (W_ih [3D][2D+F], then W_hh, the cell's W_ih and W_hh [3D][D]).
__global__ __launch_bounds__(kBlock) void k_gru_pack(int D, int S, const uint16_t *__restrict__ w_ih,
                                                      const uint16_t *__restrict__ w_hh,
                                                      const uint16_t *__restrict__ wc_ih,
                                                      const uint16_t *__restrict__ wc_hh, uint16_t *__restrict__ out) {
  const int64_t e_ih = gru_packed_elems(D, S), e_d = gru_packed_elems(D, D);
  const int64_t total = e_ih + 3 * e_d;
  const int nc = (D + 15) >> 4;
  for (int64_t o = int64_t(blockIdx.x) * kBlock + threadIdx.x; o < total; o += int64_t(gridDim.x) * kBlock) {
    const int m = o < e_ih ? 0 : int(1 + (o - e_ih) / e_d);
    const int64_t r = m == 0 ? o : (o - e_ih) - int64_t(m - 1) * e_d;
    const int kd = m == 0 ? S : D;
    const uint16_t *w = m == 0 ? w_ih : m == 1 ? w_hh : m == 2 ? wc_ih : wc_hh;
    const int nks = (kd + 31) >> 5;
    const int t = int(r & 7), l = int((r >> 3) & 63);
    const int64_t f = r >> 9;  // (g * nc + c) * nks + s
    const int s = int(f % nks), gc = int(f / nks);
    const int c = gc % nc, g = gc / nc;
    const int n = 16 * c + (l & 15), k = 32 * s + 8 * (l >> 4) + t;
    out[o] = n < D && k < kd ? w[(int64_t(g) * D + n) * kd + k] : uint16_t(0);
  }
}
}  // namespace

extern "C" int64_t sgl_gru_packed_elems(int32_t D, int32_t F) {
  if (D <= 0 || F < 0) return 0;
  return gru_packed_elems(D, 2 * D + F) + 3 * gru_packed_elems(D, D);
}

extern "C" int sgl_gru_pack_bf16(int32_t D, int32_t F, const uint16_t *w_ih, const uint16_t *w_hh,
                                 const uint16_t *wc_ih, const uint16_t *wc_hh, uint16_t *packed,
                                 hipStream_t stream) {
  SGL_REQUIRE(D > 0 && F >= 0, "gru_pack: bad dims D=%d F=%d", D, F);
  SGL_REQUIRE(w_ih && w_hh && wc_ih && wc_hh && packed, "gru_pack: NULL array");
  const int64_t total = sgl_gru_packed_elems(D, F);
  const unsigned grid = unsigned(std::min<int64_t>((total + kBlock - 1) / kBlock, sgl::kMaxGrid));
  k_gru_pack<<<grid, kBlock, 0, stream>>>(D, 2 * D + F, w_ih, w_hh, wc_ih, wc_hh, packed);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

static int memory_rows(const char *what, bool gather, int32_t D, int64_t capacity, const int32_t *num_roots,
                       const int64_t *roots, float *rows, float *memory, float *memory_ts, const float *ts_max,
                       uint32_t *node_bits, const int32_t *sample_cnt, int32_t *any_edges, float *root_dt,
                       hipStream_t stream) {
  SGL_REQUIRE(D > 0, "%s: D <= 0", what);
  SGL_REQUIRE(capacity >= 0, "%s: capacity < 0", what);
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && roots && rows && memory && node_bits && any_edges && (gather || (memory_ts && ts_max)),
              "%s: NULL array", what);
  const bool vec4 = D % 4 == 0 && ((reinterpret_cast<uintptr_t>(memory) | reinterpret_cast<uintptr_t>(rows)) & 15u) == 0;
  const int64_t total = capacity * (vec4 ? D / 4 : D);
  const unsigned grid = unsigned(std::min<int64_t>((total + kBlock - 1) / kBlock, sgl::kMaxGrid));
  sgl::launch(&k_memory_commit, dim3(grid), dim3(kBlock), 0, stream, D, vec4, gather, capacity,
              num_roots, roots, rows, memory, memory_ts, ts_max, node_bits, sample_cnt, any_edges, root_dt);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_memory_commit(int32_t D, int64_t capacity, const int32_t *num_roots, const int64_t *roots,
                                 const float *new_mem, float *memory, float *memory_ts, const float *ts_max,
                                 uint32_t *node_bits, const int32_t *sample_cnt, int32_t *any_edges,
                                 float *root_dt, hipStream_t stream) {
  return memory_rows("memory_commit", false, D, capacity, num_roots, roots, const_cast<float *>(new_mem), memory,
                     memory_ts, ts_max, node_bits, sample_cnt, any_edges, root_dt, stream);
}

extern "C" int sgl_memory_gather(int32_t D, int64_t capacity, const int32_t *num_roots, const int64_t *roots,
                                 const float *memory, float *rows, uint32_t *node_bits, const int32_t *sample_cnt,
                                 int32_t *any_edges, hipStream_t stream) {
  return memory_rows("memory_gather", true, D, capacity, num_roots, roots, rows, const_cast<float *>(memory),
                     nullptr, nullptr, node_bits, sample_cnt, any_edges, nullptr, stream);
}
