// Row-tile GEMM primitives on CDNA MFMA for the fused per-root kernels.
//
// A workgroup owns a tile of 16 rows (roots / nodes) whose activations sit in
// LDS; weights stream from global memory (L2-resident: every weight matrix on
// this path is < 1 MB). A wave computes 16x16 output blocks with
// v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate).
//
// Lane layout of v_mfma_f32_16x16x4_f32 (one block, K = 4):
//   A[i][k] comes from lane i + 16*k, B[k][j] from lane j + 16*k,
//   D[i][j] lands in lane j + 16*(i/4), accumulator element i%4.
#pragma once

#include <hip/hip_runtime.h>

namespace sgl {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Weight operand layouts for OUT = A * op(W):
//   kNT: W is [N][ldw] row-major and OUT[i][n] = sum_k A[i][k] * W[n][k]   (nn.Linear weight)
//   kNN: W is [K][ldw] row-major and OUT[i][n] = sum_k A[i][k] * W[k][n]
enum WLayout { kNT = 0, kNN = 1 };

// One 16x16 output block: rows 0..15 of A (LDS, leading dim lda), columns
// n0..n0+15 of op(W), reduction over k in [0, kd). Out-of-range k or n read
// as 0. Returns this lane's four accumulators (rows 4*(lane/16)+v, column
// n0 + lane%16).
template <int LAYOUT>
__device__ __forceinline__ f32x4 mfma_block16(const float *__restrict__ A, int lda,
                                              const float *__restrict__ W, int ldw,
                                              int n0, int kd, int n_total) {
  const int lane = threadIdx.x & 63;
  const int i = lane & 15;
  const int kq = lane >> 4;
  const int n = n0 + i;
  const bool n_ok = n < n_total;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int k0 = 0;
  // main loop: 4 k-steps (16 values) per iteration, loads issued before MFMAs
  for (; k0 + 16 <= kd; k0 += 16) {
    float a[4], b[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const int k = k0 + 4 * s + kq;
      a[s] = A[i * lda + k];
      if (LAYOUT == kNT)
        b[s] = n_ok ? W[size_t(n) * ldw + k] : 0.f;
      else
        b[s] = n_ok ? W[size_t(k) * ldw + n] : 0.f;
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], acc, 0, 0, 0);
  }
  for (; k0 < kd; k0 += 4) {
    const int k = k0 + kq;
    const bool k_ok = k < kd;
    const float a = k_ok ? A[i * lda + k] : 0.f;
    float b = 0.f;
    if (k_ok && n_ok) b = (LAYOUT == kNT) ? W[size_t(n) * ldw + k] : W[size_t(k) * ldw + n];
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  }
  return acc;
}

// OUT (LDS, 16 x n_total, leading dim ldo) = A * op(W) + bias (bias may be
// NULL), the n-blocks split over the workgroup's waves. No barrier inside;
// the caller synchronises before reading OUT. If ACC, adds to OUT.
template <int LAYOUT, bool ACC = false>
__device__ __forceinline__ void tile_gemm16(const float *__restrict__ A, int lda,
                                            const float *__restrict__ W, int ldw,
                                            const float *__restrict__ bias,
                                            float *__restrict__ OUT, int ldo,
                                            int kd, int n_total, int nwaves) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int nblocks = (n_total + 15) >> 4;
  for (int nb = wave; nb < nblocks; nb += nwaves) {
    const int n0 = nb * 16;
    f32x4 acc = mfma_block16<LAYOUT>(A, lda, W, ldw, n0, kd, n_total);
    const int col = n0 + (lane & 15);
    if (col < n_total) {
      const float bv = bias != nullptr ? bias[col] : 0.f;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = 4 * (lane >> 4) + v;
        float o = acc[v] + bv;
        if (ACC) o += OUT[row * ldo + col];
        OUT[row * ldo + col] = o;
      }
    }
  }
}

}  // namespace sgl
