// TGN temporal attention (TimeEncode + TemporalTransformerConv), forward and
// backward, one workgroup per tile of 16 roots.
//
// Reference: TemporalTransformerConv.forward  backends/ctdg/runtime/models.py:77-137,
//            build_dgl_block                  models.py:144-197,
//            TimeEncode                       runtime/modules/time_encode.py:41-58.
//
// Per root r with neighbour window e = 1..cnt (padded sampler rows):
//   X_e  = [ memory[nbr_e] (D) | efeat[eid_e] (F) | cos(w*dt_e + b) (T) ]   (C = D+F+T)
//   Q_r  = W_q [h_r | cos(b)] + b_q                 (h_r = the root's updated memory)
//   s_eh = <Q_rh, W_kh X_e + b_kh> = <qt_rh, X_e> + <Q_rh, b_kh>,  qt_rh = W_kh^T Q_rh
//   a_eh = LeakyReLU_0.2(s_eh);  alpha = softmax over the root's edges
//   agg_rh = sum_e alpha_eh (W_vh X_e + b_vh) = W_vh xbar_rh + b_vh,  xbar_rh = sum_e alpha_eh X_e
//   agg_r = 0 for a root without edges (DGL copy_e/sum over no edges)
//   y_r  = LayerNorm(ReLU(W_out [agg_r | h_r] + b_out)), all zero if the whole
//          block has no edges (models.py:88-89, runtime.py:168-169)
// The re-association moves the K/V projections from per-edge to per-root
// GEMMs (qt and the W_v product), so per edge only a gather, T cosines and
// 2H dot/axpy passes over C floats remain. The edge loop is one wavefront per
// root with an online (running max / running sum) softmax.
//
// No 1/sqrt(d) scaling (models.py:125). The time-encoding argument is
// fl(fl(dt * w) + b), then cos.
#include <climits>

#include "common.h"
#include "mfma.h"

namespace {

constexpr int kBlock = 256;
constexpr int kRows = 16;
constexpr int kWaves = kBlock / 64;
constexpr int kMaxH = 4;
constexpr int kMaxJ = 8;  // C <= 512

struct Dims {
  int D, F, T, H, C, dh, k;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Argument of the time encoding: the product rounded, then the bias added
// (a GEMM with a bias epilogue, as nn.Linear(1, T) runs on the GPU). The
// rounding matters: cos() of arguments in the 1e5-1e8 range turns one ulp of
// difference into a different value.
// (HIP's __fmul_rn/__fadd_rn are plain operators that -ffp-contract=fast fuses
// into v_fmac; the pragma keeps v_mul_f32 + v_add_f32.)
__device__ __forceinline__ float te_arg(float dt, float w, float b) {
#pragma clang fp contract(off)
  const float prod = dt * w;
  return prod + b;
}

// lane's slice of X_e: c = lane + 64*j
__device__ __forceinline__ void load_x(const Dims &d, const float *__restrict__ memory,
                                       const float *__restrict__ efeat,
                                       const float *__restrict__ te_w,
                                       const float *__restrict__ te_b, int64_t nb, int64_t ei,
                                       float dtv, int lane, float (&x)[kMaxJ]) {
#pragma unroll
  for (int j = 0; j < kMaxJ; ++j) {
    const int c = lane + 64 * j;
    float v = 0.f;
    if (c < d.D) {
      v = memory[nb * d.D + c];
    } else if (c < d.D + d.F) {
      v = efeat[ei * d.F + (c - d.D)];
    } else if (c < d.C) {
      const int t = c - d.D - d.F;
      v = cosf(te_arg(dtv, te_w[t], te_b[t]));
    }
    x[j] = v;
  }
}

struct ConvParams {
  const float *w_q, *b_q, *w_k, *b_k, *w_v, *b_v, *w_out, *b_out, *ln_g, *ln_b, *te_w, *te_b;
};

struct ConvSaved {
  float *Q;      // [cap][D]
  float *qt;     // [cap][H][C]
  float *xbar;   // [cap][H][C]
  float *score;  // [cap][k][H]  LeakyReLU'd scores
  float *ml;     // [cap][H][2]  softmax max and sum
  float *agg;    // [cap][D]
  float *z;      // [cap][D]     pre-ReLU output projection
  float *stats;  // [cap][2]     LayerNorm mean, rstd
};

__global__ __launch_bounds__(kBlock) void k_conv_fwd(
    Dims d, const int32_t *__restrict__ num_roots, const int32_t *__restrict__ any_edges,
    const float *__restrict__ h_root, const float *__restrict__ memory,
    const float *__restrict__ efeat, const int32_t *__restrict__ cnt,
    const int32_t *__restrict__ nbr, const int32_t *__restrict__ eid,
    const float *__restrict__ dt, ConvParams p, ConvSaved sv, float *__restrict__ y) {
  extern __shared__ float lds[];
  const int D = d.D, T = d.T, H = d.H, C = d.C, dh = d.dh, K = d.k;
  const int ldr = D + 1, ldq = H * C + 1;
  float *Hd = lds;
  float *Qs = Hd + kRows * ldr;
  float *Ag = Qs + kRows * ldr;
  float *Zs = Ag + kRows * ldr;
  float *QT = Zs + kRows * ldr;
  float *cq = QT + kRows * ldq;
  float *phi0 = cq + D;
  float *qb = phi0 + T;
  __shared__ int s_cnt[kRows];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int U = *num_roots;
  const int r0 = blockIdx.x * kRows;
  const int nrows = max(0, min(kRows, U - r0));
  const bool live = *any_edges != 0;
  if (nrows == 0 || !live) {
    // rows outside the live set, or a block without edges: zero output and
    // zero saved state (the backward then produces zero gradients)
    for (int idx = tid; idx < kRows * D; idx += kBlock) {
      const size_t o = size_t(r0) * D + idx;
      y[o] = 0.f; sv.Q[o] = 0.f; sv.agg[o] = 0.f; sv.z[o] = 0.f;
    }
    for (int idx = tid; idx < kRows * H * C; idx += kBlock) {
      sv.qt[size_t(r0) * H * C + idx] = 0.f;
      sv.xbar[size_t(r0) * H * C + idx] = 0.f;
    }
    for (int idx = tid; idx < kRows * 2; idx += kBlock) sv.stats[size_t(r0) * 2 + idx] = 0.f;
    return;
  }
  if (tid < kRows) s_cnt[tid] = tid < nrows ? cnt[r0 + tid] : 0;
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    Hd[i * ldr + j] = i < nrows ? h_root[size_t(r0 + i) * D + j] : 0.f;
  }
  for (int t = tid; t < T; t += kBlock) phi0[t] = cosf(p.te_b[t]);  // TimeEncode(0) = cos(0*w + b)
  __syncthreads();
  for (int n = tid; n < D; n += kBlock) {
    float acc = p.b_q[n];
    const float *wr = p.w_q + size_t(n) * (D + T) + D;
    for (int t = 0; t < T; ++t) acc += wr[t] * phi0[t];
    cq[n] = acc;
  }
  __syncthreads();
  // Q = W_q[:, :D] h + (W_q[:, D:] cos(b) + b_q)
  sgl::tile_gemm16<sgl::kNT>(Hd, ldr, p.w_q, D + T, cq, Qs, ldr, D, D, kWaves);
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    sv.Q[size_t(r0 + i) * D + j] = Qs[i * ldr + j];
  }
  if (tid < kRows * H) {
    const int i = tid / H, h = tid - (tid / H) * H;
    float acc = 0.f;
    for (int j = 0; j < dh; ++j) acc += Qs[i * ldr + h * dh + j] * p.b_k[h * dh + j];
    qb[i * H + h] = acc;
  }
  // qt_h = Q_h W_k[h rows, :]  (kNN: rows of W_k are the reduction index)
  for (int h = 0; h < H; ++h)
    sgl::tile_gemm16<sgl::kNN>(Qs + h * dh, ldr, p.w_k + size_t(h) * dh * C, C, nullptr, QT + h * C, ldq, dh,
                               C, kWaves);
  __syncthreads();
  for (int idx = tid; idx < kRows * H * C; idx += kBlock) {
    const int i = idx / (H * C), hc = idx - i * (H * C);
    sv.qt[size_t(r0 + i) * H * C + hc] = QT[i * ldq + hc];
  }

  // edge pass: one wave per root, online softmax, xbar overwrites qt in LDS
  for (int i = wave; i < kRows; i += kWaves) {
    const int r = r0 + i;
    const int ne = s_cnt[i];
    float q[kMaxH][kMaxJ], acc[kMaxH][kMaxJ], m[kMaxH], l[kMaxH];
#pragma unroll
    for (int h = 0; h < kMaxH; ++h) {
      m[h] = -INFINITY;
      l[h] = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j) {
        const int c = lane + 64 * j;
        q[h][j] = (h < H && c < C) ? QT[i * ldq + h * C + c] : 0.f;
        acc[h][j] = 0.f;
      }
    }
    for (int e = 0; e < ne; ++e) {
      const size_t idx = size_t(r) * K + e;
      float x[kMaxJ];
      load_x(d, memory, efeat, p.te_w, p.te_b, nbr[idx], eid[idx], dt[idx], lane, x);
#pragma unroll
      for (int h = 0; h < kMaxH; ++h) {
        if (h >= H) continue;
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j) part += q[h][j] * x[j];
        const float s = wave_sum(part) + qb[i * H + h];
        const float a = s > 0.f ? s : 0.2f * s;
        const float mn = fmaxf(m[h], a);
        const float sc = __expf(m[h] - mn);
        const float pe = __expf(a - mn);
        l[h] = l[h] * sc + pe;
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j) acc[h][j] = acc[h][j] * sc + pe * x[j];
        m[h] = mn;
        if (lane == 0) sv.score[idx * H + h] = a;
      }
    }
#pragma unroll
    for (int h = 0; h < kMaxH; ++h) {
      if (h >= H) continue;
      const float inv = ne > 0 ? 1.f / l[h] : 0.f;
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j) {
        const int c = lane + 64 * j;
        if (c < C) {
          const float v = acc[h][j] * inv;
          QT[i * ldq + h * C + c] = v;
          sv.xbar[size_t(r) * H * C + h * C + c] = v;
        }
      }
      if (lane == 0) {
        sv.ml[(size_t(r) * H + h) * 2 + 0] = ne > 0 ? m[h] : 0.f;
        sv.ml[(size_t(r) * H + h) * 2 + 1] = ne > 0 ? l[h] : 1.f;
      }
    }
  }
  __syncthreads();
  // agg_h = W_v[h rows] xbar_h + b_v[h]
  for (int h = 0; h < H; ++h)
    sgl::tile_gemm16<sgl::kNT>(QT + h * C, ldq, p.w_v + size_t(h) * dh * C, C, p.b_v + h * dh, Ag + h * dh,
                               ldr, C, dh, kWaves);
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    if (s_cnt[i] == 0) Ag[i * ldr + j] = 0.f;  // no in-edges: the sum aggregator gives 0
    sv.agg[size_t(r0 + i) * D + j] = Ag[i * ldr + j];
  }
  __syncthreads();
  // z = W_out[:, :D] agg + W_out[:, D:] h + b_out
  sgl::tile_gemm16<sgl::kNT>(Ag, ldr, p.w_out, 2 * D, p.b_out, Zs, ldr, D, D, kWaves);
  sgl::tile_gemm16<sgl::kNT, true>(Hd, ldr, p.w_out + D, 2 * D, nullptr, Zs, ldr, D, D, kWaves);
  __syncthreads();
  // y = LayerNorm(ReLU(z)), eps 1e-5, biased variance
  for (int i = wave; i < kRows; i += kWaves) {
    const size_t ro = size_t(r0 + i) * D;
    float s1 = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float zz = Zs[i * ldr + j];
      sv.z[ro + j] = i < nrows ? zz : 0.f;
      s1 += fmaxf(zz, 0.f);
    }
    const float mean = wave_sum(s1) / D;
    float s2 = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float dv = fmaxf(Zs[i * ldr + j], 0.f) - mean;
      s2 += dv * dv;
    }
    const float rstd = 1.f / sqrtf(wave_sum(s2) / D + 1e-5f);
    for (int j = lane; j < D; j += 64) {
      const float xh = (fmaxf(Zs[i * ldr + j], 0.f) - mean) * rstd;
      y[ro + j] = i < nrows ? xh * p.ln_g[j] + p.ln_b[j] : 0.f;
    }
    if (lane == 0) {
      sv.stats[size_t(r0 + i) * 2 + 0] = mean;
      sv.stats[size_t(r0 + i) * 2 + 1] = rstd;
    }
  }
}

struct ConvGrads {
  float *gz;       // [cap][D]
  float *gagg;     // [cap][D]
  float *G;        // [cap][H][C]  sum_e gs_eh X_e
  float *sigma;    // [cap][H]     sum_e gs_eh
  float *gQ;       // [cap][D]
  float *ln_part;  // [tiles][2][D]  per-tile sums of gy*xhat and gy
  float *te_part;  // [tiles][2][T]  per-tile time-encoding weight / bias grads
};

__global__ __launch_bounds__(kBlock) void k_conv_bwd(
    Dims d, const int32_t *__restrict__ num_roots, const int32_t *__restrict__ any_edges,
    const float *__restrict__ memory, const float *__restrict__ efeat,
    const int32_t *__restrict__ cnt, const int32_t *__restrict__ nbr,
    const int32_t *__restrict__ eid, const float *__restrict__ dt, ConvParams p,
    ConvSaved sv, const float *__restrict__ gy, ConvGrads g) {
  extern __shared__ float lds[];
  const int D = d.D, T = d.T, H = d.H, C = d.C, dh = d.dh, K = d.k;
  const int ldr = D + 1, ldq = H * C + 1;
  float *GZ = lds;
  float *GA = GZ + kRows * ldr;
  float *GQ = GA + kRows * ldr;
  float *GX = GQ + kRows * ldr;      // g_xbar, then G
  float *tep = GX + kRows * ldq;     // [kWaves][2][T]
  __shared__ int s_cnt[kRows];
  __shared__ float s_sig[kRows][kMaxH];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int U = *num_roots;
  const int r0 = blockIdx.x * kRows;
  const int nrows = max(0, min(kRows, U - r0));
  const bool live = *any_edges != 0;
  if (nrows == 0 || !live) {
    for (int idx = tid; idx < kRows * D; idx += kBlock) {
      const size_t o = size_t(r0) * D + idx;
      g.gz[o] = 0.f; g.gagg[o] = 0.f; g.gQ[o] = 0.f;
    }
    for (int idx = tid; idx < kRows * H * C; idx += kBlock) g.G[size_t(r0) * H * C + idx] = 0.f;
    for (int idx = tid; idx < kRows * H; idx += kBlock) g.sigma[size_t(r0) * H + idx] = 0.f;
    for (int idx = tid; idx < 2 * D; idx += kBlock) g.ln_part[size_t(blockIdx.x) * 2 * D + idx] = 0.f;
    for (int idx = tid; idx < 2 * T; idx += kBlock) g.te_part[size_t(blockIdx.x) * 2 * T + idx] = 0.f;
    return;
  }
  if (tid < kRows) s_cnt[tid] = tid < nrows ? cnt[r0 + tid] : 0;
  __syncthreads();
  // LayerNorm + ReLU backward, one wave per row
  for (int i = wave; i < kRows; i += kWaves) {
    const size_t ro = size_t(r0 + i) * D;
    if (i >= nrows) {
      for (int j = lane; j < D; j += 64) GZ[i * ldr + j] = 0.f;
      continue;
    }
    const float mean = sv.stats[size_t(r0 + i) * 2], rstd = sv.stats[size_t(r0 + i) * 2 + 1];
    float a1 = 0.f, a2 = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float xh = (fmaxf(sv.z[ro + j], 0.f) - mean) * rstd;
      const float gxh = gy[ro + j] * p.ln_g[j];
      a1 += gxh;
      a2 += gxh * xh;
    }
    a1 = wave_sum(a1) / D;
    a2 = wave_sum(a2) / D;
    for (int j = lane; j < D; j += 64) {
      const float zz = sv.z[ro + j];
      const float xh = (fmaxf(zz, 0.f) - mean) * rstd;
      const float gx = rstd * (gy[ro + j] * p.ln_g[j] - a1 - xh * a2);
      GZ[i * ldr + j] = zz > 0.f ? gx : 0.f;
    }
  }
  // per-tile LayerNorm parameter grads
  for (int j = tid; j < D; j += kBlock) {
    float sg = 0.f, sb = 0.f;
    for (int i = 0; i < nrows; ++i) {
      const size_t ro = size_t(r0 + i) * D;
      const float mean = sv.stats[size_t(r0 + i) * 2], rstd = sv.stats[size_t(r0 + i) * 2 + 1];
      const float xh = (fmaxf(sv.z[ro + j], 0.f) - mean) * rstd;
      sg += gy[ro + j] * xh;
      sb += gy[ro + j];
    }
    g.ln_part[size_t(blockIdx.x) * 2 * D + j] = sg;
    g.ln_part[size_t(blockIdx.x) * 2 * D + D + j] = sb;
  }
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    g.gz[size_t(r0 + i) * D + j] = GZ[i * ldr + j];
  }
  // g_agg = gz W_out[:, :D]
  sgl::tile_gemm16<sgl::kNN>(GZ, ldr, p.w_out, 2 * D, nullptr, GA, ldr, D, D, kWaves);
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    if (s_cnt[i] == 0) GA[i * ldr + j] = 0.f;  // agg was the constant 0
    g.gagg[size_t(r0 + i) * D + j] = GA[i * ldr + j];
  }
  __syncthreads();
  // g_xbar_h = g_agg_h W_v[h rows, :]
  for (int h = 0; h < H; ++h)
    sgl::tile_gemm16<sgl::kNN>(GA + h * dh, ldr, p.w_v + size_t(h) * dh * C, C, nullptr, GX + h * C, ldq, dh, C,
                               kWaves);
  __syncthreads();

  // edge backward pass: one wave per root
  float tw[kMaxJ], tb[kMaxJ];
#pragma unroll
  for (int j = 0; j < kMaxJ; ++j) { tw[j] = 0.f; tb[j] = 0.f; }
  for (int i = wave; i < kRows; i += kWaves) {
    const int r = r0 + i;
    const int ne = s_cnt[i];
    float q[kMaxH][kMaxJ], xb[kMaxH][kMaxJ], gx[kMaxH][kMaxJ], G[kMaxH][kMaxJ];
    float dot[kMaxH], sig[kMaxH], mh[kMaxH], lh[kMaxH];
#pragma unroll
    for (int h = 0; h < kMaxH; ++h) {
      float pd = 0.f;
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j) {
        const int c = lane + 64 * j;
        const bool ok = h < H && c < C;
        q[h][j] = ok ? sv.qt[size_t(r) * H * C + h * C + c] : 0.f;
        xb[h][j] = ok ? sv.xbar[size_t(r) * H * C + h * C + c] : 0.f;
        gx[h][j] = ok ? GX[i * ldq + h * C + c] : 0.f;
        G[h][j] = 0.f;
        pd += gx[h][j] * xb[h][j];
      }
      dot[h] = wave_sum(pd);
      sig[h] = 0.f;
      mh[h] = h < H ? sv.ml[(size_t(r) * H + h) * 2] : 0.f;
      lh[h] = h < H ? sv.ml[(size_t(r) * H + h) * 2 + 1] : 1.f;
    }
    for (int e = 0; e < ne; ++e) {
      const size_t idx = size_t(r) * K + e;
      const float dtv = dt[idx];
      float x[kMaxJ];
      load_x(d, memory, efeat, p.te_w, p.te_b, nbr[idx], eid[idx], dtv, lane, x);
      float gsv[kMaxH], al[kMaxH];
#pragma unroll
      for (int h = 0; h < kMaxH; ++h) {
        gsv[h] = 0.f;
        al[h] = 0.f;
        if (h >= H) continue;
        float part = 0.f;
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j) part += gx[h][j] * x[j];
        const float t = wave_sum(part);
        const float a = sv.score[idx * H + h];
        const float alpha = __expf(a - mh[h]) / lh[h];
        const float ga = alpha * (t - dot[h]);  // softmax backward
        const float gs = ga * (a > 0.f ? 1.f : 0.2f);
        gsv[h] = gs;
        al[h] = alpha;
        sig[h] += gs;
#pragma unroll
        for (int j = 0; j < kMaxJ; ++j) G[h][j] += gs * x[j];
      }
      // time-encoding gradients for this edge's T columns
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j) {
        const int c = lane + 64 * j;
        if (c >= d.D + d.F && c < C) {
          float gphi = 0.f;
#pragma unroll
          for (int h = 0; h < kMaxH; ++h)
            if (h < H) gphi += gsv[h] * q[h][j] + al[h] * gx[h][j];
          const int t = c - d.D - d.F;
          const float ds = -sinf(te_arg(dtv, p.te_w[t], p.te_b[t])) * gphi;
          tw[j] += ds * dtv;
          tb[j] += ds;
        }
      }
    }
#pragma unroll
    for (int h = 0; h < kMaxH; ++h) {
      if (h >= H) continue;
#pragma unroll
      for (int j = 0; j < kMaxJ; ++j) {
        const int c = lane + 64 * j;
        if (c < C) {
          GX[i * ldq + h * C + c] = G[h][j];
          g.G[size_t(r) * H * C + h * C + c] = G[h][j];
        }
      }
      if (lane == 0) {
        g.sigma[size_t(r) * H + h] = sig[h];
        s_sig[i][h] = sig[h];
      }
    }
  }
  // reduce the waves' time-encoding partials
#pragma unroll
  for (int j = 0; j < kMaxJ; ++j) {
    const int c = lane + 64 * j;
    if (c >= d.D + d.F && c < C) {
      const int t = c - d.D - d.F;
      tep[(wave * 2 + 0) * T + t] = tw[j];
      tep[(wave * 2 + 1) * T + t] = tb[j];
    }
  }
  __syncthreads();
  for (int t = tid; t < T; t += kBlock) {
    float a = 0.f, b = 0.f;
    for (int w = 0; w < kWaves; ++w) { a += tep[(w * 2) * T + t]; b += tep[(w * 2 + 1) * T + t]; }
    g.te_part[size_t(blockIdx.x) * 2 * T + t] = a;
    g.te_part[size_t(blockIdx.x) * 2 * T + T + t] = b;
  }
  // gQ_h = W_k[h rows] G_h + b_k[h] sigma_h
  for (int h = 0; h < H; ++h)
    sgl::tile_gemm16<sgl::kNT>(GX + h * C, ldq, p.w_k + size_t(h) * dh * C, C, nullptr, GQ + h * dh, ldr, C, dh,
                               kWaves);
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    const int h = j / dh;
    const float v = i < nrows ? GQ[i * ldr + j] + p.b_k[j] * s_sig[i][h] : 0.f;
    g.gQ[size_t(r0 + i) * D + j] = v;
  }
}

size_t fwd_lds_bytes(const Dims &d) {
  return sizeof(float) * (size_t(kRows) * (4 * (d.D + 1) + d.H * d.C + 1) + d.D + d.T + kRows * d.H);
}

size_t bwd_lds_bytes(const Dims &d) {
  return sizeof(float) * (size_t(kRows) * (3 * (d.D + 1) + d.H * d.C + 1) + size_t(kWaves) * 2 * d.T);
}

int check_dims(const Dims &d) {
  SGL_REQUIRE(d.D > 0 && d.H > 0 && d.H <= kMaxH && d.D % d.H == 0, "conv: need 0 < H <= %d and D %% H == 0 (D=%d H=%d)",
              kMaxH, d.D, d.H);
  SGL_REQUIRE(d.F >= 0 && d.T >= 0 && d.C <= 64 * kMaxJ, "conv: C = D+F+T = %d exceeds %d", d.C, 64 * kMaxJ);
  SGL_REQUIRE(d.k >= 0 && d.k <= 4096, "conv: fanout %d out of range", d.k);
  return SGL_OK;
}

}  // namespace

extern "C" int sgl_conv_forward(int32_t D, int32_t F, int32_t T, int32_t H, int32_t fanout, int64_t capacity,
                                const int32_t *num_roots, const int32_t *any_edges, const float *h_root,
                                const float *memory, const float *efeat, const int32_t *cnt, const int32_t *nbr,
                                const int32_t *eid, const float *dt, const float *w_q, const float *b_q,
                                const float *w_k, const float *b_k, const float *w_v, const float *b_v,
                                const float *w_out, const float *b_out, const float *ln_g, const float *ln_b,
                                const float *te_w, const float *te_b, float *sv_Q, float *sv_qt, float *sv_xbar,
                                float *sv_score, float *sv_ml, float *sv_agg, float *sv_z, float *sv_stats,
                                float *y, hipStream_t stream) {
  Dims d{D, F, T, H, D + F + T, H > 0 ? D / H : 0, fanout};
  if (int rc = check_dims(d)) return rc;
  SGL_REQUIRE(capacity >= 0 && capacity < INT_MAX && capacity % kRows == 0,
              "conv: capacity %lld must be a multiple of %d", (long long)capacity, kRows);
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && any_edges && h_root && memory && cnt && w_q && b_q && w_k && b_k && w_v && b_v && w_out &&
                  b_out && ln_g && ln_b && te_w && te_b && sv_Q && sv_qt && sv_xbar && sv_ml && sv_agg && sv_z &&
                  sv_stats && y && (F == 0 || efeat) && (fanout == 0 || (nbr && eid && dt && sv_score)),
              "conv_forward: NULL array");
  const size_t lds = fwd_lds_bytes(d);
  SGL_REQUIRE(lds <= 160 * 1024, "conv_forward: %zu bytes of LDS needed (> 160 KiB)", lds);
  SGL_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_conv_fwd),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
  ConvParams p{w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b, te_w, te_b};
  ConvSaved sv{sv_Q, sv_qt, sv_xbar, sv_score, sv_ml, sv_agg, sv_z, sv_stats};
  k_conv_fwd<<<unsigned(capacity / kRows), kBlock, lds, stream>>>(d, num_roots, any_edges, h_root, memory, efeat,
                                                                   cnt, nbr, eid, dt, p, sv, y);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_conv_backward(int32_t D, int32_t F, int32_t T, int32_t H, int32_t fanout, int64_t capacity,
                                 const int32_t *num_roots, const int32_t *any_edges, const float *memory,
                                 const float *efeat, const int32_t *cnt, const int32_t *nbr, const int32_t *eid,
                                 const float *dt, const float *w_q, const float *b_q, const float *w_k,
                                 const float *b_k, const float *w_v, const float *b_v, const float *w_out,
                                 const float *b_out, const float *ln_g, const float *ln_b, const float *te_w,
                                 const float *te_b, const float *sv_Q, const float *sv_qt, const float *sv_xbar,
                                 const float *sv_score, const float *sv_ml, const float *sv_agg, const float *sv_z,
                                 const float *sv_stats, const float *gy, float *gz, float *gagg, float *G,
                                 float *sigma, float *gQ, float *ln_part, float *te_part, hipStream_t stream) {
  Dims d{D, F, T, H, D + F + T, H > 0 ? D / H : 0, fanout};
  if (int rc = check_dims(d)) return rc;
  SGL_REQUIRE(capacity >= 0 && capacity < INT_MAX && capacity % kRows == 0,
              "conv: capacity %lld must be a multiple of %d", (long long)capacity, kRows);
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && any_edges && memory && cnt && w_q && w_k && b_k && w_v && w_out && ln_g && te_w && te_b &&
                  sv_qt && sv_xbar && sv_ml && sv_z && sv_stats && gy && gz && gagg && G && sigma && gQ && ln_part &&
                  te_part && (F == 0 || efeat) && (fanout == 0 || (nbr && eid && dt && sv_score)),
              "conv_backward: NULL array");
  const size_t lds = bwd_lds_bytes(d);
  SGL_REQUIRE(lds <= 160 * 1024, "conv_backward: %zu bytes of LDS needed (> 160 KiB)", lds);
  SGL_CHECK_HIP(hipFuncSetAttribute(reinterpret_cast<const void *>(&k_conv_bwd),
                                    hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
  ConvParams p{w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b, te_w, te_b};
  ConvSaved sv{const_cast<float *>(sv_Q), const_cast<float *>(sv_qt), const_cast<float *>(sv_xbar),
               const_cast<float *>(sv_score), const_cast<float *>(sv_ml), const_cast<float *>(sv_agg),
               const_cast<float *>(sv_z), const_cast<float *>(sv_stats)};
  ConvGrads g{gz, gagg, G, sigma, gQ, ln_part, te_part};
  k_conv_bwd<<<unsigned(capacity / kRows), kBlock, lds, stream>>>(d, num_roots, any_edges, memory, efeat, cnt, nbr,
                                                                  eid, dt, p, sv, gy, g);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
