// Edge predictor + BCE loss, forward and backward, one workgroup (16 waves)
// per 16 events. Reference: CTDGLinkPredictor.forward (backends/ctdg/runtime/models.py:313-324),
// the root-row selection of _conv_output (runtime.py:176-183) and the loss of
// train_step (runtime.py:290-292):
//   e_s = y[rs], e_d = y[rd], e_n = y[rn] (0 when the negative is not a root)
//   h_s = W_s e_s + b_s, h_d = W_d e_d + b_d, h_n = W_d e_n + b_d
//   pos = w_o . relu(h_s + h_d) + b_o,  neg = w_o . relu(h_s + h_n) + b_o
//   loss = mean softplus(-pos) + mean softplus(neg)  (BCE with logits, labels 1 / 0)
// In training mode the same launch produces the predictor's parameter
// gradients (accumulated with atomics into caller-zeroed buffers) and the
// gradient w.r.t. the attention output y (scattered with atomics into gy).
#include <climits>

#include "common.h"
#include "mfma.h"

namespace {

constexpr int kBlock = 1024;
constexpr int kRows = 16;
constexpr int kWaves = kBlock / 64;  // one event per wave for the logits

__device__ __forceinline__ float softplus(float x) {
  // log(1 + exp(x)), stable: max(x, 0) + log1p(exp(-|x|))
  return fmaxf(x, 0.f) + log1pf(expf(-fabsf(x)));
}

__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

__global__ __launch_bounds__(256) void k_zero(float *__restrict__ a, int64_t n, float *__restrict__ b,
                                                 int64_t m) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) a[i] = 0.f;
  if (i < m) b[i] = 0.f;
}

__global__ __launch_bounds__(kBlock) void k_predictor(
    int64_t batch, int D, int train, const float *__restrict__ y, const int32_t *__restrict__ rs,
    const int32_t *__restrict__ rd, const int32_t *__restrict__ rn, const float *__restrict__ w_s,
    const float *__restrict__ b_s, const float *__restrict__ w_d, const float *__restrict__ b_d,
    const float *__restrict__ w_o, const float *__restrict__ b_o, float *__restrict__ pos_out,
    float *__restrict__ neg_out, float *__restrict__ loss, float *__restrict__ gy,
    float *__restrict__ g_ws, float *__restrict__ g_bs, float *__restrict__ g_wd, float *__restrict__ g_bd,
    float *__restrict__ g_wo, float *__restrict__ g_bo) {
  extern __shared__ float lds[];
  const int ld = D + 1;
  float *Es = lds;
  float *Ed = Es + kRows * ld;
  float *En = Ed + kRows * ld;
  float *Hs = En + kRows * ld;  // h_s, then g_h_s
  float *Hd = Hs + kRows * ld;  // h_d -> a_p -> g_h_d
  float *Hn = Hd + kRows * ld;  // h_n -> a_n -> g_h_n
  float *Gx = Hn + kRows * ld;  // backward rows to scatter
  __shared__ float s_gp[kRows], s_gn[kRows];
  __shared__ int s_idx[3][kRows];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t e0 = int64_t(blockIdx.x) * kRows;
  const int nrows = int(min<int64_t>(kRows, batch - e0));
  if (tid < kRows) {
    const bool ok = tid < nrows;
    s_idx[0][tid] = ok ? rs[e0 + tid] : -1;
    s_idx[1][tid] = ok ? rd[e0 + tid] : -1;
    s_idx[2][tid] = ok ? rn[e0 + tid] : -1;
  }
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    const int a = s_idx[0][i], b = s_idx[1][i], c = s_idx[2][i];
    Es[i * ld + j] = a >= 0 ? y[size_t(a) * D + j] : 0.f;
    Ed[i * ld + j] = b >= 0 ? y[size_t(b) * D + j] : 0.f;
    En[i * ld + j] = c >= 0 ? y[size_t(c) * D + j] : 0.f;
  }
  __syncthreads();
  {
    sgl::GemmJob jobs[3] = {{Es, ld, w_s, D, b_s, Hs, ld, D, D}, {Ed, ld, w_d, D, b_d, Hd, ld, D, D},
                            {En, ld, w_d, D, b_d, Hn, ld, D, D}};
    sgl::tile_gemm16_jobs<sgl::kNT>(jobs, kWaves);
  }
  __syncthreads();
  // logits, loss, logit gradients: one wave per event
  for (int i = wave; i < kRows; i += kWaves) {
    float pp = 0.f, pn = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float hs = Hs[i * ld + j];
      const float ap = fmaxf(hs + Hd[i * ld + j], 0.f);
      const float an = fmaxf(hs + Hn[i * ld + j], 0.f);
      Hd[i * ld + j] = ap;
      Hn[i * ld + j] = an;
      pp += w_o[j] * ap;
      pn += w_o[j] * an;
    }
#pragma unroll
    for (int dd = 32; dd > 0; dd >>= 1) {
      pp += __shfl_xor(pp, dd, 64);
      pn += __shfl_xor(pn, dd, 64);
    }
    if (lane == 0) {
      float gp = 0.f, gn = 0.f;
      if (i < nrows) {
        const float p = pp + b_o[0], n = pn + b_o[0];
        pos_out[e0 + i] = p;
        neg_out[e0 + i] = n;
        atomicAdd(loss, (softplus(-p) + softplus(n)) / float(batch));
        gp = (sigmoid(p) - 1.f) / float(batch);
        gn = sigmoid(n) / float(batch);
      }
      s_gp[i] = gp;
      s_gn[i] = gn;
    }
  }
  if (!train) return;  // uniform
  __syncthreads();
  // out_fc grads and the hidden-layer gradients
  for (int j = tid; j < D; j += kBlock) {
    float gw = 0.f;
    for (int i = 0; i < kRows; ++i) gw += s_gp[i] * Hd[i * ld + j] + s_gn[i] * Hn[i * ld + j];
    atomicAdd(&g_wo[j], gw);
  }
  if (tid == 0) {
    float gb = 0.f;
    for (int i = 0; i < kRows; ++i) gb += s_gp[i] + s_gn[i];
    atomicAdd(g_bo, gb);
  }
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    const float ghp = Hd[i * ld + j] > 0.f ? s_gp[i] * w_o[j] : 0.f;
    const float ghn = Hn[i * ld + j] > 0.f ? s_gn[i] * w_o[j] : 0.f;
    Hs[i * ld + j] = ghp + ghn;  // g_h_s
    Hd[i * ld + j] = ghp;        // g_h_d
    Hn[i * ld + j] = ghn;        // g_h_n
  }
  __syncthreads();
  // weight / bias gradients: sums over the tile's events
  for (int idx = tid; idx < D * D; idx += kBlock) {
    const int a = idx / D, b = idx - (idx / D) * D;
    float s = 0.f, d = 0.f;
#pragma unroll 4
    for (int i = 0; i < kRows; ++i) {
      s += Hs[i * ld + a] * Es[i * ld + b];
      d += Hd[i * ld + a] * Ed[i * ld + b] + Hn[i * ld + a] * En[i * ld + b];
    }
    atomicAdd(&g_ws[idx], s);
    atomicAdd(&g_wd[idx], d);
  }
  for (int j = tid; j < D; j += kBlock) {
    float s = 0.f, d = 0.f;
    for (int i = 0; i < kRows; ++i) {
      s += Hs[i * ld + j];
      d += Hd[i * ld + j] + Hn[i * ld + j];
    }
    atomicAdd(&g_bs[j], s);
    atomicAdd(&g_bd[j], d);
  }
  // embedding gradients scattered to the roots: g_e = W^T g_h
  for (int role = 0; role < 3; ++role) {
    const float *GH = role == 0 ? Hs : (role == 1 ? Hd : Hn);
    sgl::tile_gemm16<sgl::kNN>(GH, ld, role == 0 ? w_s : w_d, D, nullptr, Gx, ld, D, D, kWaves);
    __syncthreads();
    for (int idx = tid; idx < kRows * D; idx += kBlock) {
      const int i = idx / D, j = idx - i * D;
      const int r = s_idx[role][i];
      if (r >= 0) atomicAdd(&gy[size_t(r) * D + j], Gx[i * ld + j]);
    }
    __syncthreads();
  }
}

}  // namespace

extern "C" int sgl_predictor(int64_t batch, int32_t D, int64_t capacity, int32_t train, const float *y,
                             const int32_t *ridx_src, const int32_t *ridx_dst, const int32_t *ridx_neg,
                             const float *w_s, const float *b_s, const float *w_d, const float *b_d,
                             const float *w_o, const float *b_o, float *pos_logits, float *neg_logits,
                             float *loss, float *gy, float *g_ws, float *g_bs, float *g_wd, float *g_bd,
                             float *g_wo, float *g_bo, hipStream_t stream) {
  SGL_REQUIRE(batch >= 0 && batch < INT_MAX && D > 0 && capacity >= 0, "predictor: bad sizes");
  SGL_REQUIRE(y && ridx_src && ridx_dst && ridx_neg && w_s && b_s && w_d && b_d && w_o && b_o && pos_logits &&
                  neg_logits && loss,
              "predictor: NULL array");
  SGL_REQUIRE(!train || (gy && g_ws && g_bs && g_wd && g_bd && g_wo && g_bo), "predictor: NULL gradient array");
  const int64_t nz = train ? capacity * D : 0;
  const int64_t zb = ((nz > 1 ? nz : 1) + 255) / 256;
  k_zero<<<unsigned(zb), 256, 0, stream>>>(gy, nz, loss, 1);
  SGL_CHECK_LAUNCH();
  if (batch == 0) return SGL_OK;
  const size_t lds = sizeof(float) * size_t(kRows) * 7 * (D + 1);
  SGL_REQUIRE(lds <= 160 * 1024, "predictor: D=%d needs %zu bytes of LDS", D, lds);
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(&k_predictor), lds));
  k_predictor<<<unsigned((batch + kRows - 1) / kRows), kBlock, lds, stream>>>(
      batch, D, train, y, ridx_src, ridx_dst, ridx_neg, w_s, b_s, w_d, b_d, w_o, b_o, pos_logits, neg_logits, loss,
      gy, g_ws, g_bs, g_wd, g_bd, g_wo, g_bo);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
