// Recent-k temporal neighbour sampling over the device CSR (the GPU
// counterpart of ParallelSampler::neighbor_sample_from_nodes_with_before_layer
// with policy "recent", vendor/bts_sampler/sampler/include/sampler.h:213-261).
//
// Hot path: ONE kernel per hop, HBM/latency bound integer work. Up to 32768
// queries (a training step) take k_recent_wave, one wavefront per query;
// more take k_recent_padded:
//   phase 1: one lane per query -- lower_bound over the node's int64
//            timestamps (the same probe sequence as std::lower_bound) gives
//            the window [end-k, end) of the node's list;
//   phase 2: the wavefront copies its 64 windows cooperatively: the wave's
//            padded output rows [q*k, q*k+k) are contiguous, so lane l of
//            iteration it owns slot s = it*64 + l, i.e. (query s/k, entry
//            s%k). Stores are fully contiguous and loads are contiguous
//            inside each window.
// The padded layout (row q holds cnt[q] <= k valid entries, oldest first) is
// what the attention kernels consume. sgl_recent_compact() turns it into the
// reference's concatenated layout (a block scan of the counts, tile offsets
// scanned by one workgroup, then a copy).
#include <climits>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace {

constexpr int kBlock = 256;
constexpr int kTile = 256;      // queries per compaction tile
constexpr int kScanBlock = 1024;
constexpr int64_t kWaveModeMaxQueries = 1 << 15;  // below: one wavefront per query
constexpr int64_t kFence = 32;  // CSR entries per fence (one 128-byte line of int32 times)
constexpr int kCopyBatch = 10;  // window-copy iterations per batch of loads (k = 10: one batch)

// TsT: the CSR's timestamps as stored, int64 or (when every timestamp fits)
// int32, compared with the int64 query times exactly. With int32 times the
// ids come interleaved: nbr points at (nbr, eid) pairs and eid is unused.
template <typename NodeT, typename TsT>
__global__ __launch_bounds__(kBlock) void k_recent_padded(
    int64_t nq, const int64_t *__restrict__ nq_live_dev, const NodeT *__restrict__ q_node,
    const int64_t *__restrict__ q_ts, const int32_t *__restrict__ q_valid_cnt, int q_stride,
    const int64_t *__restrict__ indptr, const int32_t *__restrict__ nbr,
    const int32_t *__restrict__ eid, const TsT *__restrict__ ts, const TsT *__restrict__ fence,
    int64_t num_nodes, int k, int32_t *__restrict__ out_cnt,
    int32_t *__restrict__ out_nbr, int32_t *__restrict__ out_eid,
    float *__restrict__ out_dt, int64_t *__restrict__ out_ts,
    int32_t *__restrict__ err) {
  const int lane = threadIdx.x & (sgl::kWave - 1);
  const int64_t q0 = int64_t(blockIdx.x) * kBlock + (threadIdx.x & ~(sgl::kWave - 1));
  const int64_t i = q0 + lane;
  int c = 0;
  int64_t b = 0, t = 0;
  const int64_t nq_live = nq_live_dev != nullptr ? min(nq, *nq_live_dev) : nq;
  if (i < nq) {
    bool valid = i < nq_live;
    if (valid && q_valid_cnt != nullptr) valid = int(i % q_stride) < q_valid_cnt[i / q_stride];
    if (valid) {
      const int64_t n = int64_t(q_node[i]);
      t = q_ts[i];
      if (n < 0 || n >= num_nodes) {
        if (err != nullptr) atomicOr(err, SGL_DERR_NODE_RANGE);
      } else {
        const int64_t lo = indptr[n], hi = indptr[n + 1];
        int64_t first = lo, len = hi - lo;
        if (fence != nullptr && len > 2 * kFence) {
          // every list time-sorted: lower_bound over the fences (ts[kFence * f],
          // a small array that stays in cache) inside [lo, hi) first; the
          // answer then lies in the one line (kFence * (f - 1), kFence * f]
          const int64_t a = (lo + kFence - 1) / kFence, bf = (hi - 1) / kFence;
          int64_t f = a, fl = bf - a + 1;
          while (fl > 0) {
            const int64_t half = fl >> 1;
            if (int64_t(fence[f + half]) < t) {
              f += half + 1;
              fl -= half + 1;
            } else {
              fl = half;
            }
          }
          first = f == a ? lo : kFence * (f - 1) + 1;
          len = (f > bf ? hi : kFence * f) - first;
        }
        while (len > 0) {  // std::lower_bound
          const int64_t half = len >> 1;
          const int64_t mid = first + half;
          if (int64_t(ts[mid]) < t) {
            first = mid + 1;
            len -= half + 1;
          } else {
            len = half;
          }
        }
        const int64_t end = first - lo;
        int64_t start = end - k;
        if (start < 0) start = 0;
        b = lo + start;
        c = int(end - start);
      }
    }
    out_cnt[i] = c;
  }
  // Cooperative copy of the wave's 64 windows into its contiguous padded rows,
  // kCopyBatch iterations at a time: every load of a batch is issued before
  // its first store, so a batch costs one memory round trip (one per
  // iteration when each load waited for the previous iteration's stores).
  const int64_t obase = q0 * k;
  for (int it0 = 0; it0 < k; it0 += kCopyBatch) {
    TsT tv[kCopyBatch];
    int32_t vn[kCopyBatch], ve[kCopyBatch];
    bool ok[kCopyBatch];
#pragma unroll
    for (int u = 0; u < kCopyBatch; ++u) {
      const int s = (it0 + u) * sgl::kWave + lane;
      const int ql = s / k;  // < 64 while it0 + u < k
      const int j = s - ql * k;
      const int cq = __shfl(c, ql & (sgl::kWave - 1), sgl::kWave);
      const int64_t bq = __shfl(b, ql & (sgl::kWave - 1), sgl::kWave);
      ok[u] = it0 + u < k && j < cq;
      tv[u] = 0;
      vn[u] = ve[u] = 0;
      if (ok[u]) {
        const int64_t src = bq + j;
        tv[u] = ts[src];
        if constexpr (std::is_same_v<TsT, int32_t>) {  // ids interleaved (nbr, eid) with int32 times
          const int2 v = reinterpret_cast<const int2 *>(nbr)[src];
          vn[u] = v.x;
          ve[u] = v.y;
        } else {
          vn[u] = nbr[src];
          ve[u] = eid[src];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kCopyBatch; ++u) {
      const int s = (it0 + u) * sgl::kWave + lane;
      const int ql = s / k;
      const int64_t tq = __shfl(t, ql & (sgl::kWave - 1), sgl::kWave);
      if (ok[u]) {
        const int64_t o = obase + s;
        out_nbr[o] = vn[u];
        out_eid[o] = ve[u];
        out_dt[o] = float(tq - int64_t(tv[u]));  // int64 -> f32, round to nearest even
        if (out_ts != nullptr) out_ts[o] = int64_t(tv[u]);
      }
    }
  }
}

// Latency variant for small query counts (a training step's few hundred
// roots): one wavefront per query, following std::lower_bound's decision
// tree exactly (so unsorted timestamp lists give the reference's result
// too), six levels per memory round trip: lane h-1 evaluates node h of the
// next six levels' complete binary subtree (its (first, len) follows from
// the path bits of h), a ballot collects the 63 comparisons, and the wave
// then walks the six levels. A 100k-entry list takes 3 round trips instead
// of 17 dependent probes. The window is then copied by the wave's lanes.
constexpr int kWaveQueriesPerBlock = kBlock / sgl::kWave;

template <typename NodeT, typename TsT>
__global__ __launch_bounds__(kBlock) void k_recent_wave(
    int64_t nq, const int64_t *__restrict__ nq_live_dev, const NodeT *__restrict__ q_node,
    const int64_t *__restrict__ q_ts, const int32_t *__restrict__ q_valid_cnt, int q_stride,
    const int64_t *__restrict__ indptr, const int32_t *__restrict__ nbr,
    const int32_t *__restrict__ eid, const TsT *__restrict__ ts,
    int64_t num_nodes, int k, int32_t *__restrict__ out_cnt,
    int32_t *__restrict__ out_nbr, int32_t *__restrict__ out_eid,
    float *__restrict__ out_dt, int64_t *__restrict__ out_ts,
    int32_t *__restrict__ err) {
  const int lane = threadIdx.x & (sgl::kWave - 1);
  const int64_t i = int64_t(blockIdx.x) * kWaveQueriesPerBlock + (threadIdx.x >> 6);
  if (i >= nq) return;  // uniform per wave
  const int64_t nq_live = nq_live_dev != nullptr ? min(nq, *nq_live_dev) : nq;
  bool valid = i < nq_live;
  if (valid && q_valid_cnt != nullptr) valid = int(i % q_stride) < q_valid_cnt[i / q_stride];
  int c = 0;
  int64_t b = 0, t = 0;
  if (valid) {
    const int64_t n = int64_t(q_node[i]);
    t = q_ts[i];
    if (n < 0 || n >= num_nodes) {
      if (err != nullptr && lane == 0) atomicOr(err, SGL_DERR_NODE_RANGE);
    } else {
      const int64_t lo = indptr[n];
      int64_t first = lo, len = indptr[n + 1] - lo;
      const int h = lane + 1;  // heap index of this lane's node (1..63; lane 63 idle)
      const int depth = 31 - __clz(h);
      while (len > 0) {
        int64_t fh = first, lh = len;
        for (int d = depth - 1; d >= 0; --d) {
          const int64_t half = lh >> 1;
          if ((h >> d) & 1) {
            fh += half + 1;
            lh -= half + 1;
          } else {
            lh = half;
          }
        }
        const bool below = h < sgl::kWave && lh > 0 && int64_t(ts[fh + (lh >> 1)]) < t;
        const unsigned long long res = __ballot(below);
        int node = 1;
#pragma unroll
        for (int lev = 0; lev < 6; ++lev) {
          if (len == 0) break;
          const int64_t half = len >> 1;
          const bool r = (res >> (node - 1)) & 1ull;
          if (r) {
            first += half + 1;
            len -= half + 1;
          } else {
            len = half;
          }
          node = 2 * node + (r ? 1 : 0);
        }
      }
      const int64_t end = first - lo;
      int64_t start = end - k;
      if (start < 0) start = 0;
      b = lo + start;
      c = int(end - start);
    }
  }
  if (lane == 0) out_cnt[i] = c;
  const int64_t obase = i * k;
  for (int j = lane; j < c; j += sgl::kWave) {
    const int64_t src = b + j;
    const int64_t tv = int64_t(ts[src]);
    if constexpr (std::is_same_v<TsT, int32_t>) {
      const int2 v = reinterpret_cast<const int2 *>(nbr)[src];
      out_nbr[obase + j] = v.x;
      out_eid[obase + j] = v.y;
    } else {
      out_nbr[obase + j] = nbr[src];
      out_eid[obase + j] = eid[src];
    }
    out_dt[obase + j] = float(t - tv);  // int64 -> f32, round to nearest even
    if (out_ts != nullptr) out_ts[obase + j] = tv;
  }
}

__global__ __launch_bounds__(kTile) void k_tile_sums(int64_t nq, const int32_t *__restrict__ cnt,
                                                     int64_t *__restrict__ tile_sum) {
  const int64_t i = int64_t(blockIdx.x) * kTile + threadIdx.x;
  const int64_t c = i < nq ? cnt[i] : 0;
  __shared__ int64_t s_w[kTile / sgl::kWave];
  const int64_t s = sgl::wave_reduce_sum(c);
  if ((threadIdx.x & (sgl::kWave - 1)) == 0) s_w[threadIdx.x / sgl::kWave] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t tot = 0;
#pragma unroll
    for (int w = 0; w < kTile / sgl::kWave; ++w) tot += s_w[w];
    tile_sum[blockIdx.x] = tot;
  }
}

// Exclusive scan of n tile totals by one workgroup: each thread owns a
// contiguous chunk, chunk sums are block-scanned, then chunks are rewritten.
__global__ __launch_bounds__(kScanBlock) void k_scan_tiles(
    int64_t n, const int64_t *__restrict__ in, int64_t *__restrict__ out_excl) {
  __shared__ int64_t s_w[kScanBlock / sgl::kWave];
  const int64_t per = (n + kScanBlock - 1) / kScanBlock;
  const int64_t b = int64_t(threadIdx.x) * per;
  const int64_t e = b + per < n ? b + per : n;
  int64_t sum = 0;
  for (int64_t i = b; i < e; ++i) sum += in[i];
  int64_t total;
  int64_t run = sgl::block_exclusive_scan<int64_t, kScanBlock>(sum, s_w, total);
  for (int64_t i = b; i < e; ++i) {
    const int64_t v = in[i];
    out_excl[i] = run;
    run += v;
  }
}

__global__ __launch_bounds__(kTile) void k_compact_fill(
    int64_t nq, int k, const int32_t *__restrict__ cnt,
    const int64_t *__restrict__ tile_off, const int32_t *__restrict__ pnbr,
    const int32_t *__restrict__ peid, const float *__restrict__ pdt,
    const int64_t *__restrict__ pts, int64_t *__restrict__ out_ptr,
    int32_t *__restrict__ out_nbr, int32_t *__restrict__ out_eid,
    float *__restrict__ out_dt, int64_t *__restrict__ out_ts) {
  __shared__ int32_t s_off[kTile + 1];
  __shared__ int32_t s_w[kTile / sgl::kWave];
  const int tid = threadIdx.x;
  const int64_t q0 = int64_t(blockIdx.x) * kTile;
  const int64_t i = q0 + tid;
  const int c = i < nq ? cnt[i] : 0;
  int32_t total;
  const int32_t off = sgl::block_exclusive_scan<int32_t, kTile>(c, s_w, total);
  s_off[tid] = off;
  if (tid == 0) s_off[kTile] = total;
  const int64_t base = tile_off[blockIdx.x];
  if (i < nq) out_ptr[i] = base + off;
  if (i == nq - 1) out_ptr[nq] = base + off + c;
  __syncthreads();
  for (int j = tid; j < total; j += kTile) {
    int lo = 0, hi = kTile;  // owner: the largest q with s_off[q] <= j
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (s_off[mid] <= j) lo = mid; else hi = mid;
    }
    const int64_t src = (q0 + lo) * k + (j - s_off[lo]);
    const int64_t o = base + j;
    out_nbr[o] = pnbr[src];
    out_eid[o] = peid[src];
    out_dt[o] = pdt[src];
    if (out_ts != nullptr) out_ts[o] = pts[src];
  }
}

__global__ void k_write_zero_ptr(int64_t *out_ptr) { out_ptr[0] = 0; }

}  // namespace

template <typename TsT>
static int recent_sample(const int64_t *indptr, const int32_t *nbr, const int32_t *eid, const TsT *ts,
                         const TsT *fence, int64_t num_nodes, const void *q_node, int q_node_is_i64, const int64_t *q_ts,
                         int64_t num_queries, const int64_t *num_queries_dev, const int32_t *q_valid_cnt,
                         int32_t q_stride, int32_t fanout, int32_t *out_cnt, int32_t *out_nbr, int32_t *out_eid,
                         float *out_dt, int64_t *out_ts, int32_t *err_flag, hipStream_t stream) {
  SGL_REQUIRE(num_queries >= 0, "recent: num_queries < 0");
  SGL_REQUIRE(fanout >= 0 && fanout <= 4096, "recent: fanout %d outside [0, 4096]", fanout);
  SGL_REQUIRE(num_nodes >= 0, "recent: num_nodes < 0");
  if (num_queries == 0) return SGL_OK;
  SGL_REQUIRE(indptr && q_node && q_ts && out_cnt, "recent: NULL graph, query or count array");
  constexpr bool kPacked = std::is_same_v<TsT, int32_t>;
  SGL_REQUIRE(fanout == 0 || (nbr && (kPacked || eid) && ts && out_nbr && out_eid && out_dt),
              "recent: NULL graph or output array");
  SGL_REQUIRE(!kPacked || (reinterpret_cast<uintptr_t>(nbr) & 7u) == 0, "recent: nbr_eid not 8-byte aligned");
  SGL_REQUIRE(q_valid_cnt == nullptr || q_stride > 0, "recent: q_stride must be > 0 with q_valid_cnt");
  const int64_t blocks = (num_queries + kBlock - 1) / kBlock;
  SGL_REQUIRE(blocks < INT_MAX, "recent: too many queries");
  if (num_queries <= kWaveModeMaxQueries) {  // latency: one wavefront per query
    const unsigned wblocks = unsigned((num_queries + kWaveQueriesPerBlock - 1) / kWaveQueriesPerBlock);
    if (q_node_is_i64)
      sgl::launch(&k_recent_wave<int64_t, TsT>, dim3(wblocks), dim3(kBlock), 0, stream, num_queries,
                  num_queries_dev, static_cast<const int64_t *>(q_node), q_ts, q_valid_cnt, q_stride, indptr, nbr,
                  eid, ts, num_nodes, fanout, out_cnt, out_nbr, out_eid, out_dt, out_ts, err_flag);
    else
      sgl::launch(&k_recent_wave<int32_t, TsT>, dim3(wblocks), dim3(kBlock), 0, stream, num_queries,
                  num_queries_dev, static_cast<const int32_t *>(q_node), q_ts, q_valid_cnt, q_stride, indptr, nbr,
                  eid, ts, num_nodes, fanout, out_cnt, out_nbr, out_eid, out_dt, out_ts, err_flag);
    SGL_CHECK_LAUNCH();
    return SGL_OK;
  }
  if (q_node_is_i64) {
    k_recent_padded<int64_t, TsT><<<unsigned(blocks), kBlock, 0, stream>>>(
        num_queries, num_queries_dev, static_cast<const int64_t *>(q_node), q_ts, q_valid_cnt, q_stride, indptr,
        nbr, eid, ts, fence, num_nodes, fanout, out_cnt, out_nbr, out_eid, out_dt, out_ts, err_flag);
  } else {
    k_recent_padded<int32_t, TsT><<<unsigned(blocks), kBlock, 0, stream>>>(
        num_queries, num_queries_dev, static_cast<const int32_t *>(q_node), q_ts, q_valid_cnt, q_stride, indptr,
        nbr, eid, ts, fence, num_nodes, fanout, out_cnt, out_nbr, out_eid, out_dt, out_ts, err_flag);
  }
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_recent_sample(
    const int64_t *indptr, const int32_t *nbr, const int32_t *eid,
    const int64_t *ts, int64_t num_nodes, const void *q_node, int q_node_is_i64,
    const int64_t *q_ts, int64_t num_queries, const int64_t *num_queries_dev, const int32_t *q_valid_cnt,
    int32_t q_stride, int32_t fanout, int32_t *out_cnt, int32_t *out_nbr,
    int32_t *out_eid, float *out_dt, int64_t *out_ts, int32_t *err_flag,
    hipStream_t stream) {
  return recent_sample<int64_t>(indptr, nbr, eid, ts, nullptr, num_nodes, q_node, q_node_is_i64, q_ts, num_queries,
                                num_queries_dev, q_valid_cnt, q_stride, fanout, out_cnt, out_nbr, out_eid, out_dt,
                                out_ts, err_flag, stream);
}

extern "C" int sgl_recent_sample_packed(
    const int64_t *indptr, const int32_t *nbr_eid, const int32_t *ts, const int32_t *fence, int64_t num_nodes,
    const void *q_node,
    int q_node_is_i64, const int64_t *q_ts, int64_t num_queries, const int64_t *num_queries_dev,
    const int32_t *q_valid_cnt, int32_t q_stride, int32_t fanout, int32_t *out_cnt, int32_t *out_nbr,
    int32_t *out_eid, float *out_dt, int64_t *out_ts, int32_t *err_flag, hipStream_t stream) {
  return recent_sample<int32_t>(indptr, nbr_eid, nullptr, ts, fence, num_nodes, q_node, q_node_is_i64, q_ts,
                                num_queries,
                                num_queries_dev, q_valid_cnt, q_stride, fanout, out_cnt, out_nbr, out_eid, out_dt,
                                out_ts, err_flag, stream);
}

extern "C" size_t sgl_compact_workspace_bytes(int64_t num_queries) {
  if (num_queries < 0) return 0;
  const size_t tiles = (size_t(num_queries) + kTile - 1) / kTile;
  return 2 * sgl::align_up(tiles * 8) + 256;
}

namespace {

// The checks and launches shared by both compaction entry points; tile_sum
// and tile_off hold ceil(num_queries / kTile) entries each. Every entry is
// written before it is read, so the scratch needs no clearing.
int compact_checks(int64_t num_queries, int32_t fanout, const int32_t *cnt, const int32_t *pad_nbr,
                   const int32_t *pad_eid, const float *pad_dt, const int64_t *pad_ts, const int64_t *out_ptr,
                   const int32_t *out_nbr, const int32_t *out_eid, const float *out_dt, const int64_t *out_ts) {
  SGL_REQUIRE(num_queries >= 0, "compact: num_queries < 0");
  SGL_REQUIRE(fanout >= 0 && fanout <= 4096, "compact: fanout %d outside [0, 4096]", fanout);
  SGL_REQUIRE(out_ptr != nullptr, "compact: out_ptr is NULL");
  if (num_queries == 0) return SGL_OK;
  SGL_REQUIRE(cnt != nullptr, "compact: cnt is NULL");
  SGL_REQUIRE(fanout == 0 || (pad_nbr && pad_eid && pad_dt && out_nbr && out_eid && out_dt), "compact: NULL array");
  SGL_REQUIRE(out_ts == nullptr || pad_ts != nullptr, "compact: out_ts needs pad_ts");
  const size_t tiles = (size_t(num_queries) + kTile - 1) / kTile;
  SGL_REQUIRE(tiles < size_t(INT_MAX), "compact: too many queries");
  return SGL_OK;
}

int compact_run(int64_t num_queries, int32_t fanout, const int32_t *cnt, const int32_t *pad_nbr,
                const int32_t *pad_eid, const float *pad_dt, const int64_t *pad_ts, int64_t *out_ptr,
                int32_t *out_nbr, int32_t *out_eid, float *out_dt, int64_t *out_ts, int64_t *tile_sum,
                int64_t *tile_off, hipStream_t stream) {
  if (num_queries == 0) {
    k_write_zero_ptr<<<1, 1, 0, stream>>>(out_ptr);
    SGL_CHECK_LAUNCH();
    return SGL_OK;
  }
  const size_t tiles = (size_t(num_queries) + kTile - 1) / kTile;
  k_tile_sums<<<unsigned(tiles), kTile, 0, stream>>>(num_queries, cnt, tile_sum);
  SGL_CHECK_LAUNCH();
  k_scan_tiles<<<1, kScanBlock, 0, stream>>>(int64_t(tiles), tile_sum, tile_off);
  SGL_CHECK_LAUNCH();
  k_compact_fill<<<unsigned(tiles), kTile, 0, stream>>>(num_queries, fanout, cnt, tile_off, pad_nbr, pad_eid,
                                                        pad_dt, pad_ts, out_ptr, out_nbr, out_eid, out_dt, out_ts);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

}  // namespace

extern "C" int sgl_recent_compact(int64_t num_queries, int32_t fanout,
                                  const int32_t *cnt, const int32_t *pad_nbr,
                                  const int32_t *pad_eid, const float *pad_dt,
                                  const int64_t *pad_ts, int64_t *out_ptr,
                                  int32_t *out_nbr, int32_t *out_eid,
                                  float *out_dt, int64_t *out_ts,
                                  void *workspace, size_t workspace_bytes,
                                  hipStream_t stream) {
  int rc = compact_checks(num_queries, fanout, cnt, pad_nbr, pad_eid, pad_dt, pad_ts, out_ptr, out_nbr, out_eid,
                          out_dt, out_ts);
  if (rc != SGL_OK) return rc;
  int64_t *tile_sum = nullptr, *tile_off = nullptr;
  if (num_queries > 0) {
    const size_t need = sgl_compact_workspace_bytes(num_queries);
    if (workspace_bytes < need || workspace == nullptr) {
      sgl::set_error("compact: workspace %zu bytes < required %zu", workspace_bytes, need);
      return SGL_ERR_WORKSPACE;
    }
    const size_t tiles = (size_t(num_queries) + kTile - 1) / kTile;
    sgl::Carver c(workspace);
    tile_sum = c.take<int64_t>(tiles);
    tile_off = c.take<int64_t>(tiles);
  }
  return compact_run(num_queries, fanout, cnt, pad_nbr, pad_eid, pad_dt, pad_ts, out_ptr, out_nbr, out_eid, out_dt,
                     out_ts, tile_sum, tile_off, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free compaction: the tile sums and offsets live in `scratch`, a
// static device array (each GPU holds its own copy for the life of the
// process), so a caller that cannot allocate (HIP graph capture, a serving
// loop) passes only its inputs and outputs. Calls that overlap on one GPU
// share the array and race.
static constexpr int64_t kNoAllocTiles = SGL_COMPACT_NOALLOC_MAX_QUERIES / kTile;
static __device__ __align__(256) int64_t scratch[2 * kNoAllocTiles];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
int64_t *g_scratch_dev[kMaxDevices] = {};

// The current device's copy of `scratch`, looked up once per device (the
// host-side name is a stand-in, not a device address).
int scratch_of_current_device(int64_t **out) {
  int dev = -1;
  SGL_CHECK_HIP(hipGetDevice(&dev));
  SGL_REQUIRE(dev >= 0 && dev < kMaxDevices, "compact_noalloc: device %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void *p = nullptr;
    SGL_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    SGL_REQUIRE(p != nullptr, "compact_noalloc: no device address for the scratch array on device %d", dev);
    g_scratch_dev[dev] = static_cast<int64_t *>(p);
  }
  *out = g_scratch_dev[dev];
  return SGL_OK;
}

}  // namespace

extern "C" int sgl_recent_compact_noalloc(int64_t num_queries, int32_t fanout, const int32_t *cnt,
                                          const int32_t *pad_nbr, const int32_t *pad_eid, const float *pad_dt,
                                          const int64_t *pad_ts, int64_t *out_ptr, int32_t *out_nbr,
                                          int32_t *out_eid, float *out_dt, int64_t *out_ts, hipStream_t stream) {
  SGL_REQUIRE(num_queries <= SGL_COMPACT_NOALLOC_MAX_QUERIES,
              "compact_noalloc: %lld queries exceed the static scratch limit of %lld (use sgl_recent_compact)",
              (long long)num_queries, (long long)SGL_COMPACT_NOALLOC_MAX_QUERIES);
  int rc = compact_checks(num_queries, fanout, cnt, pad_nbr, pad_eid, pad_dt, pad_ts, out_ptr, out_nbr, out_eid,
                          out_dt, out_ts);
  if (rc != SGL_OK) return rc;
  int64_t *sc = nullptr;
  if (num_queries > 0) {
    rc = scratch_of_current_device(&sc);
    if (rc != SGL_OK) return rc;
  }
  return compact_run(num_queries, fanout, cnt, pad_nbr, pad_eid, pad_dt, pad_ts, out_ptr, out_nbr, out_eid, out_dt,
                     out_ts, sc, sc == nullptr ? nullptr : sc + kNoAllocTiles, stream);
}
