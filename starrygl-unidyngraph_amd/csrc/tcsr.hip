// Temporal CSR build on the device (the GPU counterpart of the reference's
// get_neighbors, vendor/bts_sampler/sampler/include/neighbors.h:209-284).
//
// The reference appends every event to vector<>s of its dst node in event
// order. Here the same lists are laid out contiguously in HBM:
//   1. key[i] = col[i] (range-checked), val[i] = i
//   2. stable LSD radix sort of (key, val) over ceil(log2(N+1)) bits -- a
//      stable sort keyed by dst keeps event order inside each node's list
//   3. gather row/eid/ts through the sorted event index (int32 / int64 SoA)
//   4. indptr from the boundaries of the sorted keys (no atomics)
#include <rocprim/device/device_radix_sort.hpp>

#include <climits>

#include "common.h"

namespace {

constexpr int kBlock = 256;

unsigned key_bits(int64_t num_nodes) {
  unsigned b = 1;
  while (b < 32 && (int64_t(1) << b) <= num_nodes) ++b;  // keys lie in [0, N]
  return b;
}

size_t sort_temp_bytes(int64_t num_edges, unsigned bits) {
  size_t temp = 0;
  if (num_edges <= 0) return 0;
  hipError_t e = rocprim::radix_sort_pairs(
      nullptr, temp, static_cast<uint32_t *>(nullptr),
      static_cast<uint32_t *>(nullptr), static_cast<int32_t *>(nullptr),
      static_cast<int32_t *>(nullptr), static_cast<size_t>(num_edges), 0u,
      bits, hipStream_t(0));
  return e == hipSuccess ? temp : 0;
}

__global__ __launch_bounds__(kBlock) void k_tcsr_keys(
    int64_t num_edges, int64_t num_nodes, const int64_t *__restrict__ row,
    const int64_t *__restrict__ col, const int64_t *__restrict__ eid,
    uint32_t *__restrict__ keys, int32_t *__restrict__ vals,
    int32_t *__restrict__ err) {
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= num_edges) return;
  const int64_t d = col[i];
  const int64_t s = row[i];
  int bad = 0;
  if (d < 0 || d >= num_nodes || s < 0 || s >= num_nodes) bad |= SGL_DERR_NODE_RANGE;
  if (eid != nullptr) {
    const int64_t e = eid[i];
    if (e < 0 || e > INT_MAX) bad |= SGL_DERR_EID_RANGE;
  }
  if (bad && err != nullptr) atomicOr(err, bad);
  // Invalid dst ids sort past every valid node and never reach indptr.
  keys[i] = (d >= 0 && d < num_nodes) ? uint32_t(d) : uint32_t(num_nodes);
  vals[i] = int32_t(i);
}

__global__ __launch_bounds__(kBlock) void k_tcsr_gather(
    int64_t num_edges, const int32_t *__restrict__ order,
    const int64_t *__restrict__ row, const int64_t *__restrict__ eid,
    const int64_t *__restrict__ ts, int32_t *__restrict__ nbr,
    int32_t *__restrict__ eid_out, int64_t *__restrict__ ts_out) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (j >= num_edges) return;
  const int32_t e = order[j];  // a permutation of [0, num_edges)
  nbr[j] = int32_t(row[e]);
  eid_out[j] = eid != nullptr ? int32_t(eid[e]) : e;
  ts_out[j] = ts[e];
}

// Thread j in [0, E] writes indptr[n] = j for every node n in (key[j-1], key[j]].
__global__ __launch_bounds__(kBlock) void k_tcsr_indptr(
    int64_t num_edges, int64_t num_nodes, const uint32_t *__restrict__ skeys,
    int64_t *__restrict__ indptr) {
  const int64_t j = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (j > num_edges) return;
  const int64_t prev = j == 0 ? -1 : int64_t(skeys[j - 1]);
  const int64_t cur = j == num_edges ? num_nodes : int64_t(skeys[j]);
  for (int64_t n = prev + 1; n <= cur && n <= num_nodes; ++n) indptr[n] = j;
}

}  // namespace

extern "C" size_t sgl_tcsr_workspace_bytes(int64_t num_nodes, int64_t num_edges) {
  if (num_nodes < 0 || num_edges < 0) return 0;
  const size_t e = size_t(num_edges);
  return 4 * sgl::align_up(e * 4) + sgl::align_up(sort_temp_bytes(num_edges, key_bits(num_nodes))) + 256;
}

extern "C" int sgl_tcsr_build(int64_t num_nodes, int64_t num_edges,
                              const int64_t *row, const int64_t *col,
                              const int64_t *eid, const int64_t *ts,
                              int64_t *indptr, int32_t *nbr, int32_t *eid_out,
                              int64_t *ts_out, void *workspace,
                              size_t workspace_bytes, int32_t *err_flag,
                              hipStream_t stream) {
  SGL_REQUIRE(num_nodes >= 0 && num_nodes < INT_MAX, "tcsr: num_nodes %lld out of range [0, 2^31-1)", (long long)num_nodes);
  SGL_REQUIRE(num_edges >= 0 && num_edges < INT_MAX, "tcsr: num_edges %lld out of range [0, 2^31-1)", (long long)num_edges);
  SGL_REQUIRE(indptr != nullptr, "tcsr: indptr is NULL");
  SGL_REQUIRE(num_edges == 0 || (row && col && ts && nbr && eid_out && ts_out), "tcsr: NULL input/output array");
  const size_t need = sgl_tcsr_workspace_bytes(num_nodes, num_edges);
  if (workspace_bytes < need || (num_edges > 0 && workspace == nullptr)) {
    sgl::set_error("tcsr: workspace %zu bytes < required %zu", workspace_bytes, need);
    return SGL_ERR_WORKSPACE;
  }
  const unsigned bits = key_bits(num_nodes);
  if (num_edges > 0) {
    const size_t e = size_t(num_edges);
    sgl::Carver c(workspace);
    uint32_t *keys_in = c.take<uint32_t>(e);
    uint32_t *keys_out = c.take<uint32_t>(e);
    int32_t *vals_in = c.take<int32_t>(e);
    int32_t *vals_out = c.take<int32_t>(e);
    size_t temp = sort_temp_bytes(num_edges, bits);
    void *temp_ptr = c.take<char>(temp);
    const unsigned grid = unsigned((e + kBlock - 1) / kBlock);
    k_tcsr_keys<<<grid, kBlock, 0, stream>>>(num_edges, num_nodes, row, col, eid, keys_in, vals_in, err_flag);
    SGL_CHECK_LAUNCH();
    SGL_CHECK_HIP(rocprim::radix_sort_pairs(temp_ptr, temp, keys_in, keys_out, vals_in, vals_out, e, 0u, bits, stream));
    k_tcsr_gather<<<grid, kBlock, 0, stream>>>(num_edges, vals_out, row, eid, ts, nbr, eid_out, ts_out);
    SGL_CHECK_LAUNCH();
    const unsigned grid1 = unsigned((e + 1 + kBlock - 1) / kBlock);
    k_tcsr_indptr<<<grid1, kBlock, 0, stream>>>(num_edges, num_nodes, keys_out, indptr);
    SGL_CHECK_LAUNCH();
  } else {
    k_tcsr_indptr<<<1, kBlock, 0, stream>>>(0, num_nodes, nullptr, indptr);
    SGL_CHECK_LAUNCH();
  }
  return SGL_OK;
}
