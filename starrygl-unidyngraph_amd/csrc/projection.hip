// JODIE-style time-projection embedding (config 2: memory + GRU + a time
// projection instead of the temporal attention), forward and backward.
//
// The reference registers "jodie" but builds its TGN model for it
// (backends/ctdg/runtime/models.py:337-338); this embedding follows the JODIE
// paper (Kumar, Zhang, Leskovec, KDD 2019, eq. 3: h(t + Delta) = (1 + w) * h(t),
// w = W_p Delta):
//   y_r = h_r * (1 + w * x_r + b),  x_r = (dt_r - shift) * scale
// for root r with updated memory h_r, where dt_r = t_batch - memory_ts[r]
// before the step's update (sgl_memory_commit writes it) and shift / scale
// normalise the time since a node's last update. The memory is detached
// (runtime.py:279), so the backward produces only the projection's weight
// and bias gradients:
//   dL/dw = sum_r (dL/dy_r * h_r) x_r,  dL/db = sum_r dL/dy_r * h_r
// with dL/dy_r = W_s^T g_src[r] + W_d^T g_dst[r] from the edge predictor's
// per-root rows (the attention backward's first product, on MFMA).
#include <climits>

#include "common.h"
#include "mfma.h"

namespace {

constexpr int kRows = 16;    // roots per backward workgroup (one MFMA row tile)
constexpr int kWaves = 8;
constexpr int kBlock = kWaves * 64;
constexpr int kFwdBlock = 256;

__device__ __forceinline__ float proj_x(float dt, float shift, float scale) {
#pragma clang fp contract(off)
  return (dt - shift) * scale;
}

__global__ __launch_bounds__(kFwdBlock) void k_proj_fwd(int D, int64_t rows, const int32_t *__restrict__ num_roots,
                                                        const float *__restrict__ h, const float *__restrict__ dt,
                                                        float shift, float scale, const float *__restrict__ w,
                                                        const float *__restrict__ b, float *__restrict__ y) {
  const int64_t U = *num_roots;
  for (int64_t i = int64_t(blockIdx.x) * kFwdBlock + threadIdx.x; i < rows * D;
       i += int64_t(gridDim.x) * kFwdBlock) {
    const int64_t r = i / D;
    const int d = int(i - r * D);
    float v = 0.f;  // rows >= U: zero (row U is the predictor's null embedding)
    if (r < U) {
      const float x = proj_x(dt[r], shift, scale);
      const float lin = x * w[d] + b[d];
      v = h[i] * (1.f + lin);
    }
    y[i] = v;
  }
}

__global__ __launch_bounds__(kBlock) void k_proj_bwd(int D, const int32_t *__restrict__ num_roots,
                                                     const float *__restrict__ h, const float *__restrict__ dt,
                                                     float shift, float scale, long long *__restrict__ acc_src,
                                                     long long *__restrict__ acc_dst, const float *__restrict__ w_s,
                                                     const float *__restrict__ w_d, float *__restrict__ g_src,
                                                     float *__restrict__ g_dst, float *__restrict__ part) {
  extern __shared__ __align__(16) float lds[];
  const int ld = sgl::lds_ld(D);
  float *GA = lds, *GB = GA + kRows * ld, *Y1 = GB + kRows * ld, *Y2 = Y1 + kRows * ld;
  const int tid = threadIdx.x;
  const int U = *num_roots;
  const int r0 = blockIdx.x * kRows;
  const int nrows = max(0, min(kRows, U - r0));
  // row U (the negatives that are not roots; row capacity when every row is
  // a root) belongs to the tile holding it, or to the last tile
  if ((U >= r0 && U < r0 + kRows) || (U == int(gridDim.x) * kRows && blockIdx.x == gridDim.x - 1)) {
    for (int j = tid; j < D; j += kBlock) {
      const size_t o = size_t(U) * D + j;
      g_src[o] = sgl::from_fixed(acc_src[o]);
      g_dst[o] = sgl::from_fixed(acc_dst[o]);
      acc_src[o] = 0;
      acc_dst[o] = 0;
    }
  }
  if (nrows == 0) {
    for (int j = tid; j < 2 * D; j += kBlock) part[size_t(blockIdx.x) * 2 * D + j] = 0.f;
    return;
  }
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    float vs = 0.f, vd = 0.f;
    if (i < nrows) {
      const size_t o = size_t(r0 + i) * D + j;
      vs = sgl::from_fixed(acc_src[o]);
      vd = sgl::from_fixed(acc_dst[o]);
      acc_src[o] = 0;
      acc_dst[o] = 0;
      g_src[o] = vs;
      g_dst[o] = vd;
    }
    GA[i * ld + j] = vs;
    GB[i * ld + j] = vd;
  }
  __syncthreads();
  // dL/dy = W_s^T g_src + W_d^T g_dst (rows of W are the reduction index)
  const sgl::GemmJob jobs[2] = {{GA, ld, w_s, D, nullptr, Y1, ld, D, D}, {GB, ld, w_d, D, nullptr, Y2, ld, D, D}};
  sgl::tile_gemm16_jobs<sgl::kNN>(jobs, kWaves);
  __syncthreads();
  // this tile's weight / bias gradient partials, in row order
  for (int j = tid; j < D; j += kBlock) {
    float pw = 0.f, pb = 0.f;
    for (int i = 0; i < nrows; ++i) {
      const float g = (Y1[i * ld + j] + Y2[i * ld + j]) * h[size_t(r0 + i) * D + j];
      pw += g * proj_x(dt[r0 + i], shift, scale);
      pb += g;
    }
    part[size_t(blockIdx.x) * 2 * D + j] = pw;
    part[size_t(blockIdx.x) * 2 * D + D + j] = pb;
  }
}

}  // namespace

extern "C" int sgl_time_projection_forward(int32_t D, int64_t rows, const int32_t *num_roots, const float *h_root,
                                           const float *root_dt, float shift, float scale, const float *w,
                                           const float *b, float *y, hipStream_t stream) {
  SGL_REQUIRE(D > 0 && rows >= 0 && rows < INT_MAX, "time_projection: bad sizes");
  if (rows == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && h_root && root_dt && w && b && y, "time_projection: NULL array");
  const unsigned grid = unsigned(std::min<int64_t>((rows * D + kFwdBlock - 1) / kFwdBlock, sgl::kMaxGrid));
  sgl::launch(&k_proj_fwd, dim3(grid), dim3(kFwdBlock), 0, stream, int(D), rows, num_roots, h_root, root_dt, shift,
              scale, w, b, y);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_time_projection_backward(int32_t D, int64_t capacity, const int32_t *num_roots,
                                            const float *h_root, const float *root_dt, float shift, float scale,
                                            int64_t *acc_src, int64_t *acc_dst, const float *w_s, const float *w_d,
                                            float *g_src, float *g_dst, float *part, hipStream_t stream) {
  SGL_REQUIRE(D > 0 && capacity >= 0 && capacity < INT_MAX && capacity % kRows == 0,
              "time_projection_backward: capacity %lld must be a multiple of %d", (long long)capacity, kRows);
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && h_root && root_dt && acc_src && acc_dst && w_s && w_d && g_src && g_dst && part,
              "time_projection_backward: NULL array");
  const size_t lds = sizeof(float) * 4 * kRows * size_t(sgl::lds_ld(D));
  SGL_REQUIRE(lds <= 160 * 1024, "time_projection_backward: D=%d needs %zu bytes of LDS", D, lds);
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(&k_proj_bwd), lds));
  sgl::launch(&k_proj_bwd, dim3(unsigned(capacity / kRows)), dim3(kBlock), lds, stream, int(D), num_roots, h_root,
              root_dt, shift, scale, reinterpret_cast<long long *>(acc_src), reinterpret_cast<long long *>(acc_dst),
              w_s, w_d, g_src, g_dst, part);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
