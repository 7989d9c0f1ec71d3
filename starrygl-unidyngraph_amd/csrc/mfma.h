// Row-tile GEMM primitives on CDNA MFMA for the fused per-root kernels.
//
// A workgroup owns a tile of 16 rows (roots / events) whose activations sit in
// LDS; weights stream from global memory (L2-resident: every weight matrix on
// this path is < 1 MB). A wave computes 16x16 output blocks with
// v_mfma_f32_16x16x4_f32 (fp32 in, fp32 accumulate).
//
// Lane layout of v_mfma_f32_16x16x4_f32 (one block, K = 4 per instruction):
//   A[i][k] comes from lane i + 16*q, B[k][j] from lane j + 16*q (q = 0..3
//   picks which of the instruction's 4 k values the lane supplies),
//   D[i][j] lands in lane j + 16*(i/4), accumulator element i%4.
// Which actual k a (lane, instruction) pair supplies is free as long as A and
// B agree. Here lane q supplies k = 16g + 4q + s in instruction s of group g,
// so each lane reads four consecutive k values of its row: one 16-byte load
// from global memory (weights) and one from LDS (activations).
//
// The blocks are latency-bound (16 rows, a few hundred k), so the weight loads
// of a whole 64-k chunk are issued before its MFMAs, and the next chunk's
// loads before the current chunk's MFMAs (two register buffers). Weight
// matrices are < 4 GiB, so element offsets are 32-bit.
#pragma once

#include <type_traits>

#include <hip/hip_runtime.h>

#include <cstdint>

namespace sgl {

typedef float f32x4 __attribute__((ext_vector_type(4)));

// Leading dimension (floats) of an LDS row tile of x columns: a multiple of 4
// with ld / 4 odd. 16-byte aligned rows let the MFMA blocks read A with one
// 16-byte LDS read per k group, and the rows of a 16-row tile start in 16
// distinct 4-bank groups, so those reads, column walks (one row per lane)
// and the blocks' output stores are free of bank conflicts.
__host__ __device__ constexpr int lds_ld(int x) { return ((x + 3) & ~3) | 4; }

// Weight operand layouts for OUT = A * op(W):
//   kNT: W is [N][ldw] row-major and OUT[i][n] = sum_k A[i][k] * W[n][k]   (nn.Linear weight)
//   kNN: W is [K][ldw] row-major and OUT[i][n] = sum_k A[i][k] * W[k][n]
enum WLayout { kNT = 0, kNN = 1 };

constexpr int kChunkGroups = 4;  // 4 groups of 16 k = 64 k per chunk

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Weight reads go through a raw buffer resource whose range is exactly the
// operand's span: elements past it read as 0 without a branch or a fault, so
// the loads of a chunk issue back to back. The whole byte offset is in the
// VGPR operand (the range check does not cover the scalar offset).
// The operand pointer and span are wave-uniform; readfirstlane states it, so
// the descriptor lives in scalar registers (a descriptor the compiler has to
// treat as per-lane turns every load into a waterfall loop).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t weight_rsrc(const float *p, uint32_t nfloats) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  const uint32_t bytes = __builtin_amdgcn_readfirstlane(nfloats * 4u);
  float *u = reinterpret_cast<float *>((uint64_t(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, int(bytes), 0x00020000);
}


__device__ __forceinline__ float buf_load(__amdgpu_buffer_rsrc_t r, uint32_t elem) {
  return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, int(elem * 4u), 0, 0));
}

__device__ __forceinline__ f32x4 buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t elem) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, int(elem * 4u), 0, 0);
  f32x4 f;
  f[0] = __uint_as_float(v[0]); f[1] = __uint_as_float(v[1]);
  f[2] = __uint_as_float(v[2]); f[3] = __uint_as_float(v[3]);
  return f;
}

__device__ __forceinline__ bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// b[g][s] = op(W)[k][n] for k = kb + 16g + 4q + s. Positions past the
// operand's span read 0; positions inside it but outside k < kd or
// n < n_total read neighbouring (finite) weights, which meet a zero A element
// (k) or land in a discarded output column (n).
template <int LAYOUT>
__device__ __forceinline__ void load_w_chunk(float (&b)[kChunkGroups][4], __amdgpu_buffer_rsrc_t W, int ldw, int n,
                                             int kb, int q, bool vec) {
  if (LAYOUT == kNT && vec) {
    // ldw % 4 == 0, kd % 4 == 0, 16-byte aligned base: one 16-byte load per group
    const uint32_t row = uint32_t(n) * uint32_t(ldw) + uint32_t(kb + 4 * q);
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g) {
      const f32x4 v = buf_load4(W, row + 16u * g);
      b[g][0] = v[0]; b[g][1] = v[1]; b[g][2] = v[2]; b[g][3] = v[3];
    }
  } else if (LAYOUT == kNT) {
    const uint32_t row = uint32_t(n) * uint32_t(ldw) + uint32_t(kb + 4 * q);
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g)
#pragma unroll
      for (int s = 0; s < 4; ++s) b[g][s] = buf_load(W, row + uint32_t(16 * g + s));
  } else {
    const uint32_t col = uint32_t(kb + 4 * q) * uint32_t(ldw) + uint32_t(n);
#pragma unroll
    for (int g = 0; g < kChunkGroups; ++g)
#pragma unroll
      for (int s = 0; s < 4; ++s) b[g][s] = buf_load(W, col + uint32_t(16 * g + s) * uint32_t(ldw));
  }
}

// acc += A[rows][kb .. kb+64) * b, A read from LDS. A chunk that lies
// wholly inside k < kd (FULL) reads A without bounds logic: 16-byte reads
// when AVEC (lda % 4 == 0, 16-byte aligned A), else 4-byte reads. The last,
// partial chunk clamps its reads in bounds, zeroes k >= kd and skips the
// groups past kd. Group g+1's reads are issued before group g's MFMAs, and the
// MFMAs alternate between two accumulators: a single dependent MFMA chain
// issues at about half the rate of two interleaved ones.
template <bool FULL, bool AVEC>
__device__ __forceinline__ void load_a_group(float (&a)[4], const float *__restrict__ arow, int k, int kd) {
  if (FULL && AVEC) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(arow + k);
    a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
  } else if (FULL) {
#pragma unroll
    for (int s = 0; s < 4; ++s) a[s] = arow[k + s];
  } else {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const float v = arow[min(k + s, kd - 1)];
      a[s] = (k + s < kd) ? v : 0.f;
    }
  }
}

template <bool FULL, bool AVEC>
__device__ __forceinline__ void mfma_chunk(f32x4 &acc0, f32x4 &acc1, const float (&b)[kChunkGroups][4],
                                           const float *__restrict__ arow, int kb, int kd, int q) {
  float a0[4], a1[4];
  load_a_group<FULL, AVEC>(a0, arow, kb + 4 * q, kd);
#pragma unroll
  for (int g = 0; g < kChunkGroups; ++g) {
    if (!FULL && kb + 16 * g >= kd) break;  // uniform across the wave
    float (&cur)[4] = (g & 1) ? a1 : a0;
    float (&nxt)[4] = (g & 1) ? a0 : a1;
    if (g + 1 < kChunkGroups) load_a_group<FULL, AVEC>(nxt, arow, kb + 16 * (g + 1) + 4 * q, kd);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[0], b[g][0], acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[1], b[g][1], acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[2], b[g][2], acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(cur[3], b[g][3], acc1, 0, 0, 0);
  }
}

__device__ __forceinline__ void mfma_chunk_any(f32x4 &acc0, f32x4 &acc1, const float (&b)[kChunkGroups][4],
                                               const float *__restrict__ arow, int kb, int kd, int q, bool avec) {
  if (kb + 16 * kChunkGroups <= kd) {  // uniform
    if (avec) mfma_chunk<true, true>(acc0, acc1, b, arow, kb, kd, q);
    else mfma_chunk<true, false>(acc0, acc1, b, arow, kb, kd, q);
  } else {
    mfma_chunk<false, false>(acc0, acc1, b, arow, kb, kd, q);
  }
}

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
  const int q = lane >> 4;
  const int n = n0 + i;
  // the operand's span: rows of op(W)^T up to the last used element
  const uint32_t span = LAYOUT == kNT ? uint32_t(n_total - 1) * uint32_t(ldw) + uint32_t(kd)
                                      : uint32_t(kd - 1) * uint32_t(ldw) + uint32_t(n_total);
  const __amdgpu_buffer_rsrc_t wr = weight_rsrc(W, span);
  // 16-byte loads: aligned, and never straddling the span end (kd % 4 == 0)
  const bool wvec = LAYOUT == kNT && (kd & 3) == 0 && (ldw & 3) == 0 && aligned16(W);
  const bool avec = (lda & 3) == 0 && aligned16(A);
  const float *arow = A + i * lda;
  constexpr int kc = 16 * kChunkGroups;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  float b0[kChunkGroups][4], b1[kChunkGroups][4];
  load_w_chunk<LAYOUT>(b0, wr, ldw, n, 0, q, wvec);
  for (int kb = 0; kb < kd; kb += 2 * kc) {
    const bool more = kb + kc < kd;
    if (more) load_w_chunk<LAYOUT>(b1, wr, ldw, n, kb + kc, q, wvec);
    mfma_chunk_any(acc0, acc1, b0, arow, kb, kd, q, avec);
    if (!more) break;
    if (kb + 2 * kc < kd) load_w_chunk<LAYOUT>(b0, wr, ldw, n, kb + 2 * kc, q, wvec);
    mfma_chunk_any(acc0, acc1, b1, arow, kb + kc, kd, q, avec);
  }
  return acc0 + acc1;
}

// Two 16-row tiles A0, A1 against the same op(W) block: the weight loads are
// shared and the two tiles' MFMA chains are independent.
template <int LAYOUT>
__device__ __forceinline__ void mfma_block16_pair(const float *__restrict__ A0, const float *__restrict__ A1,
                                                  int lda, const float *__restrict__ W, int ldw, int n0, int kd,
                                                  int n_total, f32x4 &out0, f32x4 &out1) {
  const int lane = threadIdx.x & 63;
  const int i = lane & 15;
  const int q = lane >> 4;
  const int n = n0 + i;
  const uint32_t span = LAYOUT == kNT ? uint32_t(n_total - 1) * uint32_t(ldw) + uint32_t(kd)
                                      : uint32_t(kd - 1) * uint32_t(ldw) + uint32_t(n_total);
  const __amdgpu_buffer_rsrc_t wr = weight_rsrc(W, span);
  const bool wvec = LAYOUT == kNT && (kd & 3) == 0 && (ldw & 3) == 0 && aligned16(W);
  const bool avec = (lda & 3) == 0 && aligned16(A0) && aligned16(A1);
  const float *arow0 = A0 + i * lda, *arow1 = A1 + i * lda;
  constexpr int kc = 16 * kChunkGroups;
  f32x4 p0 = {0.f, 0.f, 0.f, 0.f}, p1 = p0, r0 = p0, r1 = p0;
  float b0[kChunkGroups][4], b1[kChunkGroups][4];
  load_w_chunk<LAYOUT>(b0, wr, ldw, n, 0, q, wvec);
  for (int kb = 0; kb < kd; kb += 2 * kc) {
    const bool more = kb + kc < kd;
    if (more) load_w_chunk<LAYOUT>(b1, wr, ldw, n, kb + kc, q, wvec);
    mfma_chunk_any(p0, p1, b0, arow0, kb, kd, q, avec);
    mfma_chunk_any(r0, r1, b0, arow1, kb, kd, q, avec);
    if (!more) break;
    if (kb + 2 * kc < kd) load_w_chunk<LAYOUT>(b0, wr, ldw, n, kb + 2 * kc, q, wvec);
    mfma_chunk_any(p0, p1, b1, arow0, kb + kc, kd, q, avec);
    mfma_chunk_any(r0, r1, b1, arow1, kb + kc, kd, q, avec);
  }
  out0 = p0 + p1;
  out1 = r0 + r1;
}

// OUT (LDS, 16 x n_total, leading dim ldo) = A * op(W) + bias (bias may be
// NULL), the n-blocks split over the workgroup's waves. No barrier inside;
// the caller synchronises before reading OUT. If ACC, adds to OUT.
// Waves [wave0, wave0 + nwaves) take part (two products can run side by
// side on disjoint wave ranges).
template <int LAYOUT, bool ACC = false>
__device__ __forceinline__ void tile_gemm16(const float *__restrict__ A, int lda,
                                            const float *__restrict__ W, int ldw,
                                            const float *__restrict__ bias,
                                            float *__restrict__ OUT, int ldo,
                                            int kd, int n_total, int nwaves, int wave0 = 0) {
  const int wave = int(threadIdx.x >> 6) - wave0;
  if (wave < 0) return;
  const int lane = threadIdx.x & 63;
  const int nblocks = (n_total + 15) >> 4;
  for (int nb = wave; nb < nblocks; nb += nwaves) {
    const int n0 = nb * 16;
    const int col = n0 + (lane & 15);
    // the bias is loaded before the block's k loop (one round trip less)
    const float bv = bias != nullptr && col < n_total ? bias[col] : 0.f;
    f32x4 acc = mfma_block16<LAYOUT>(A, lda, W, ldw, n0, kd, n_total);
    if (col < n_total) {
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

// Several independent OUT = A * op(W) + bias products of one layout, their
// 16x16 blocks dealt over the workgroup's waves together (so a wave is not
// idle in one product while another has blocks left). No barrier inside.
struct GemmJob {
  const float *A;
  int lda;
  const float *W;
  int ldw;
  const float *bias;  // may be NULL
  float *OUT;
  int ldo;
  int kd, n_total;
};

template <int LAYOUT, int NJOBS>
__device__ __forceinline__ void tile_gemm16_jobs(const GemmJob (&jobs)[NJOBS], int nwaves) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int total = 0;
#pragma unroll
  for (int j = 0; j < NJOBS; ++j) total += (jobs[j].n_total + 15) >> 4;
  for (int blk = wave; blk < total; blk += nwaves) {
    // find the job of this block with unrolled selects (no dynamic indexing
    // of the local array, which would go through scratch memory)
    GemmJob jb = jobs[0];
    int nb = blk, first = 0;
#pragma unroll
    for (int j = 0; j < NJOBS; ++j) {
      const int nbj = (jobs[j].n_total + 15) >> 4;
      if (blk >= first && blk < first + nbj) {
        jb = jobs[j];
        nb = blk - first;
      }
      first += nbj;
    }
    const int n0 = nb * 16;
    const int col = n0 + (lane & 15);
    const float bv = jb.bias != nullptr && col < jb.n_total ? jb.bias[col] : 0.f;
    f32x4 acc = mfma_block16<LAYOUT>(jb.A, jb.lda, jb.W, jb.ldw, n0, jb.kd, jb.n_total);
    if (col < jb.n_total) {
#pragma unroll
      for (int v = 0; v < 4; ++v) jb.OUT[(4 * (lane >> 4) + v) * jb.ldo + col] = acc[v] + bv;
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 products with fp32 accumulation: v_mfma_f32_16x16x32_bf16. Lane l
// supplies eight k values of A row l % 16 and of op(W) column n0 + l % 16,
// k = kb + 8 (l / 16) + j for j < 8; the hardware pairs A's and W's elements
// by (lane group, element), so the product is the full sum over k whatever
// order it assigns them. The result layout is the 16x16 f32 one above. A is
// fp32 in LDS and rounded to bf16 (nearest even) as it is read; W is a bf16
// weight matrix (raw 16-bit patterns) in global memory, row n holding op(W)
// column n (kNT). k past kd and columns past n_total read 0.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ bf16x8 bf16x8_from_f32(const f32x4 &x0, const f32x4 &x1) {
  bf16x8 r;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    r[j] = static_cast<__bf16>(x0[j]);
    r[4 + j] = static_cast<__bf16>(x1[j]);
  }
  return r;
}

// AT = float: A is fp32 in LDS, rounded as it is read; AT = uint16_t: A is
// already bf16 in LDS (rows 16-byte aligned when lda % 8 == 0).
template <typename AT>
__device__ __forceinline__ f32x4 mfma_block16_bf16(const AT *__restrict__ A, int lda,
                                                   const uint16_t *__restrict__ W, int ldw, int n0, int kd,
                                                   int n_total) {
  const int lane = threadIdx.x & 63;
  const int i = lane & 15;
  const int q = lane >> 4;
  const int n = n0 + i;
  const bool nok = n < n_total;
  const uint16_t *wrow = W + size_t(nok ? n : 0) * size_t(ldw);
  const AT *arow = A + i * lda;
  // 16-byte weight loads when row starts and k offsets are multiples of 8
  // elements, else two 8-byte loads when they are multiples of 4 (D = 172)
  const bool wvec = (ldw & 7) == 0 && (kd & 7) == 0 && aligned16(W);
  const bool wvec4 = !wvec && (ldw & 3) == 0 && (kd & 3) == 0 && (reinterpret_cast<uintptr_t>(W) & 7u) == 0;
  const bool avec = std::is_same_v<AT, float> ? (lda & 3) == 0 && aligned16(A) : (lda & 7) == 0 && aligned16(A);
  constexpr int kU = 8;  // k steps of 32 whose weights are loaded together
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  for (int kb = 0; kb < kd; kb += 32 * kU) {
    bf16x8 b[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = kb + 32 * u + 8 * q;
      if (wvec && nok && k + 8 <= kd) {
        b[u] = *reinterpret_cast<const bf16x8 *>(wrow + k);
      } else if (wvec4 && nok && k + 4 <= kd) {
        typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
        const bf16x4 lo = *reinterpret_cast<const bf16x4 *>(wrow + k);
        const bf16x4 hi = k + 8 <= kd ? *reinterpret_cast<const bf16x4 *>(wrow + k + 4)
                                      : bf16x4{static_cast<__bf16>(0.f), static_cast<__bf16>(0.f),
                                               static_cast<__bf16>(0.f), static_cast<__bf16>(0.f)};
        b[u] = bf16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      } else {
#pragma unroll
        for (int j = 0; j < 8; ++j)
          b[u][j] = (nok && k + j < kd) ? __builtin_bit_cast(__bf16, wrow[k + j]) : static_cast<__bf16>(0.f);
      }
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      const int k = kb + 32 * u + 8 * q;
      if (kb + 32 * u >= kd) break;  // uniform
      bf16x8 a;
      if constexpr (std::is_same_v<AT, float>) {
        if (avec && k + 8 <= kd) {
          a = bf16x8_from_f32(*reinterpret_cast<const f32x4 *>(arow + k),
                              *reinterpret_cast<const f32x4 *>(arow + k + 4));
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) a[j] = static_cast<__bf16>(k + j < kd ? arow[min(k + j, kd - 1)] : 0.f);
        }
      } else {
        if (avec && k + 8 <= kd) {
          a = *reinterpret_cast<const bf16x8 *>(arow + k);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j)
            a[j] = k + j < kd ? __builtin_bit_cast(__bf16, arow[min(k + j, kd - 1)]) : static_cast<__bf16>(0.f);
        }
      }
      if (u & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[u], acc1, 0, 0, 0);
      else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[u], acc0, 0, 0, 0);
    }
  }
  return acc0 + acc1;
}

// The bf16 counterpart of GemmJob / tile_gemm16_jobs (kNT weights only); A
// fp32 (rounded on read) or bf16 (AT = uint16_t).
template <typename AT>
struct GemmJobBf16 {
  const AT *A;
  int lda;
  const uint16_t *W;
  int ldw;
  const float *bias;  // fp32, may be NULL
  float *OUT;
  int ldo;
  int kd, n_total;
};

template <typename AT, int NJOBS>
__device__ __forceinline__ void tile_gemm16_jobs_bf16(const GemmJobBf16<AT> (&jobs)[NJOBS], int nwaves) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int total = 0;
#pragma unroll
  for (int j = 0; j < NJOBS; ++j) total += (jobs[j].n_total + 15) >> 4;
  for (int blk = wave; blk < total; blk += nwaves) {
    GemmJobBf16<AT> jb = jobs[0];
    int nb = blk, first = 0;
#pragma unroll
    for (int j = 0; j < NJOBS; ++j) {
      const int nbj = (jobs[j].n_total + 15) >> 4;
      if (blk >= first && blk < first + nbj) {
        jb = jobs[j];
        nb = blk - first;
      }
      first += nbj;
    }
    const int n0 = nb * 16;
    const int col = n0 + (lane & 15);
    const float bv = jb.bias != nullptr && col < jb.n_total ? jb.bias[col] : 0.f;
    f32x4 acc = mfma_block16_bf16<AT>(jb.A, jb.lda, jb.W, jb.ldw, n0, jb.kd, jb.n_total);
    if (col < jb.n_total) {
#pragma unroll
      for (int v = 0; v < 4; ++v) jb.OUT[(4 * (lane >> 4) + v) * jb.ldo + col] = acc[v] + bv;
    }
  }
}

// ---------------------------------------------------------------------------
// 16-row products against padded bf16 weight copies (v_mfma_f32_16x16x32_bf16,
// fp32 accumulation). W is [n_total][ldw] row-major bf16 with ldw % 8 == 0 and
// 16-byte aligned rows, so every lane's eight weights of a k step are one
// 16-byte buffer load at row n, k = 32 s + 8 q, with no bounds logic: reads
// past the copy's span return 0 (the descriptor's range) and k >= kd meets a
// zeroed A element, so the weights there only need to be finite. A is an
// fp32 LDS tile (16 rows, leading dim lda) rounded to bf16 (nearest even) as
// it is read. Each block issues all of its weight loads (up to 8 k steps)
// before the first MFMA: the products are short and latency-bound.
struct GemmJobBw {
  const float *A;
  int lda;
  const uint16_t *W;
  int ldw;
  const float *bias;  // fp32 [n_total] or NULL
  float *OUT;
  int ldo;
  int kd, n_total;
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t bf16_weight_rsrc(const uint16_t *p, uint32_t elems) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  const uint32_t bytes = __builtin_amdgcn_readfirstlane(elems * 2u);
  uint16_t *u = reinterpret_cast<uint16_t *>((uint64_t(hi) << 32) | lo);
  return __builtin_amdgcn_make_buffer_rsrc(u, (short)0, int(bytes), 0x00020000);
}

// A[row][k .. k+8) as bf16, elements at k >= kd zero. CLS: 2 = 16-byte
// aligned rows (two 16-byte LDS reads), 1 = 8-byte aligned (four 8-byte
// reads), 0 = 4-byte reads; the last, partial step clamps and masks.
template <int CLS>
__device__ __forceinline__ bf16x8 load_a_bf16(const float *__restrict__ arow, int k, int kd) {
  bf16x8 a;
  if (k + 8 <= kd) {
    if constexpr (CLS == 2) {
      return bf16x8_from_f32(*reinterpret_cast<const f32x4 *>(arow + k), *reinterpret_cast<const f32x4 *>(arow + k + 4));
    } else if constexpr (CLS == 1) {
      typedef float f32x2 __attribute__((ext_vector_type(2)));
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const f32x2 v = *reinterpret_cast<const f32x2 *>(arow + k + 2 * t);
        a[2 * t] = static_cast<__bf16>(v[0]);
        a[2 * t + 1] = static_cast<__bf16>(v[1]);
      }
      return a;
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float v = arow[min(k + j, kd - 1)];
    a[j] = static_cast<__bf16>(k + j < kd ? v : 0.f);
  }
  return a;
}

template <int CLS>
__device__ __forceinline__ f32x4 mfma_block16_bw_cls(const float *__restrict__ A, int lda, __amdgpu_buffer_rsrc_t wr,
                                                     uint32_t wrow, int kd) {
  const int lane = threadIdx.x & 63;
  const float *arow = A + (lane & 15) * lda;
  const int q = lane >> 4;
  const int nks = (kd + 31) >> 5;
  constexpr int kU = 8;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
  for (int ks0 = 0; ks0 < nks; ks0 += kU) {
    bf16x8 b[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (ks0 + u >= nks) break;  // uniform
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, int((wrow + 32u * uint32_t(ks0 + u)) * 2u), 0, 0);
      b[u] = __builtin_bit_cast(bf16x8, v);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (ks0 + u >= nks) break;
      const bf16x8 a = load_a_bf16<CLS>(arow, 32 * (ks0 + u) + 8 * q, kd);
      if (u & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[u], acc1, 0, 0, 0);
      else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[u], acc0, 0, 0, 0);
    }
  }
  return acc0 + acc1;
}

// mfma_block16_bw_cls for two A tiles against the same weight block: each
// weight fragment is loaded once and feeds both tiles' products, which keep
// the single-tile order (bit-identical to two separate calls).
template <int CLS>
__device__ __forceinline__ void mfma_block16_bw_pair_cls(const float *__restrict__ A0, const float *__restrict__ A1,
                                                         int lda, __amdgpu_buffer_rsrc_t wr, uint32_t wrow, int kd,
                                                         f32x4 &out0, f32x4 &out1) {
  const int lane = threadIdx.x & 63;
  const float *arow0 = A0 + (lane & 15) * lda;
  const float *arow1 = A1 + (lane & 15) * lda;
  const int q = lane >> 4;
  const int nks = (kd + 31) >> 5;
  constexpr int kU = 8;
  f32x4 a00 = {0.f, 0.f, 0.f, 0.f}, a01 = a00, a10 = a00, a11 = a00;
  for (int ks0 = 0; ks0 < nks; ks0 += kU) {
    bf16x8 b[kU];
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (ks0 + u >= nks) break;  // uniform
      const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(wr, int((wrow + 32u * uint32_t(ks0 + u)) * 2u), 0, 0);
      b[u] = __builtin_bit_cast(bf16x8, v);
    }
#pragma unroll
    for (int u = 0; u < kU; ++u) {
      if (ks0 + u >= nks) break;
      const bf16x8 x0 = load_a_bf16<CLS>(arow0, 32 * (ks0 + u) + 8 * q, kd);
      const bf16x8 x1 = load_a_bf16<CLS>(arow1, 32 * (ks0 + u) + 8 * q, kd);
      if (u & 1) {
        a01 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, b[u], a01, 0, 0, 0);
        a11 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, b[u], a11, 0, 0, 0);
      } else {
        a00 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x0, b[u], a00, 0, 0, 0);
        a10 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x1, b[u], a10, 0, 0, 0);
      }
    }
  }
  out0 = a00 + a01;
  out1 = a10 + a11;
}

// The pair product of mfma_block16_bw's block (A0, A1 aligned as CLS 2: rows
// 16-byte aligned, lda % 4 == 0).
__device__ __forceinline__ void mfma_block16_bw_pair(const float *__restrict__ A0, const float *__restrict__ A1,
                                                     int lda, const uint16_t *__restrict__ W, int ldw, int n0, int kd,
                                                     int n_total, f32x4 &out0, f32x4 &out1) {
  const int lane = threadIdx.x & 63;
  const int n = min(n0 + (lane & 15), n_total - 1);
  const __amdgpu_buffer_rsrc_t wr = bf16_weight_rsrc(W, uint32_t(n_total) * uint32_t(ldw));
  const uint32_t wrow = uint32_t(n) * uint32_t(ldw) + 8u * uint32_t(lane >> 4);
  mfma_block16_bw_pair_cls<2>(A0, A1, lda, wr, wrow, kd, out0, out1);
}

// One 16x16 output block (rows 0..15 of A, columns n0..n0+15 of W^T); this
// lane's accumulators are rows 4*(lane/16)+v, column n0 + lane%16. Columns
// past n_total read row n_total-1 (their outputs are discarded). CLS >= 0
// fixes the A read width for tiles known to be aligned (less code); -1
// picks it from A and lda.
template <int CLS = -1>
__device__ __forceinline__ f32x4 mfma_block16_bw(const float *__restrict__ A, int lda, const uint16_t *__restrict__ W,
                                                 int ldw, int n0, int kd, int n_total) {
  const int lane = threadIdx.x & 63;
  const int n = min(n0 + (lane & 15), n_total - 1);
  const __amdgpu_buffer_rsrc_t wr = bf16_weight_rsrc(W, uint32_t(n_total) * uint32_t(ldw));
  const uint32_t wrow = uint32_t(n) * uint32_t(ldw) + 8u * uint32_t(lane >> 4);
  if constexpr (CLS >= 0) {
    return mfma_block16_bw_cls<CLS>(A, lda, wr, wrow, kd);
  } else {
    const uintptr_t ab = reinterpret_cast<uintptr_t>(A);
    if ((ab & 15) == 0 && (lda & 3) == 0) return mfma_block16_bw_cls<2>(A, lda, wr, wrow, kd);
    if ((ab & 7) == 0 && (lda & 1) == 0) return mfma_block16_bw_cls<1>(A, lda, wr, wrow, kd);
    return mfma_block16_bw_cls<0>(A, lda, wr, wrow, kd);
  }
}

// The weight fragments of one 16-column block of a bf16 W^T product (k steps
// 0 .. ceil(kd/32)-1 <= KP; the rest zero), loaded ahead of the block's
// products, e.g. before its A rows are gathered; lane layout and bounds as in
// mfma_block16_bw.
template <int KP>
__device__ __forceinline__ void load_wfrag_bw(bf16x8 (&b)[KP], const uint16_t *__restrict__ W, int ldw, int n0, int kd,
                                              int n_total) {
  const int lane = threadIdx.x & 63;
  const int n = min(n0 + (lane & 15), n_total - 1);
  const __amdgpu_buffer_rsrc_t wr = bf16_weight_rsrc(W, uint32_t(n_total) * uint32_t(ldw));
  const uint32_t wrow = uint32_t(n) * uint32_t(ldw) + 8u * uint32_t(lane >> 4);
  const int nks = (kd + 31) >> 5;
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    b[u] = bf16x8{};
    if (u < nks)
      b[u] = __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(wr, int((wrow + 32u * uint32_t(u)) * 2u), 0, 0));
  }
}

// mfma_block16_bw with the weight fragments already in registers
// (load_wfrag_bw): the same products in the same order (kd <= 32 KP).
template <int CLS, int KP>
__device__ __forceinline__ f32x4 mfma_block16_bw_pre(const float *__restrict__ A, int lda, const bf16x8 (&b)[KP],
                                                     int kd) {
  const int lane = threadIdx.x & 63;
  const float *arow = A + (lane & 15) * lda;
  const int q = lane >> 4;
  const int nks = (kd + 31) >> 5;
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = acc0;
#pragma unroll
  for (int u = 0; u < KP; ++u) {
    if (u >= nks) break;  // uniform
    const bf16x8 a = load_a_bf16<CLS>(arow, 32 * u + 8 * q, kd);
    if (u & 1) acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[u], acc1, 0, 0, 0);
    else acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b[u], acc0, 0, 0, 0);
  }
  return acc0 + acc1;
}

// OUT (LDS, 16 x n_total) = A * W^T + bias for every job, the 16-column
// blocks of all jobs dealt over the workgroup's waves. No barrier inside.
template <int NJOBS>
__device__ __forceinline__ void tile_gemm16_bw_jobs(const GemmJobBw (&jobs)[NJOBS], int nwaves) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int total = 0;
#pragma unroll
  for (int j = 0; j < NJOBS; ++j) total += (jobs[j].n_total + 15) >> 4;
  for (int blk = wave; blk < total; blk += nwaves) {
    GemmJobBw jb = jobs[0];
    int nb = blk, first = 0;
#pragma unroll
    for (int j = 0; j < NJOBS; ++j) {
      const int nbj = (jobs[j].n_total + 15) >> 4;
      if (blk >= first && blk < first + nbj) {
        jb = jobs[j];
        nb = blk - first;
      }
      first += nbj;
    }
    const int n0 = nb * 16;
    const int col = n0 + (lane & 15);
    const float bv = jb.bias != nullptr && col < jb.n_total ? jb.bias[col] : 0.f;
    const f32x4 acc = mfma_block16_bw(jb.A, jb.lda, jb.W, jb.ldw, n0, jb.kd, jb.n_total);
    if (col < jb.n_total) {
#pragma unroll
      for (int v = 0; v < 4; ++v) jb.OUT[(4 * (lane >> 4) + v) * jb.ldo + col] = acc[v] + bv;
    }
  }
}

// ---------------------------------------------------------------------------
// Four-row tiles (a workgroup's 4 live roots): v_mfma_f32_4x4x1_16b_f32 runs
// 16 independent 4x4x1 blocks. With every block fed the same four A rows and
// block b taking columns 4b..4b+3 of a 64-column strip, one instruction adds
// a rank-1 update to 4 rows x 64 columns, so no MFMA work goes to padding
// rows. Lane layout (16 blocks, K = 1): A[i][k] of block b comes from lane
// 4b + i, B[k][j] from lane 4b + j, D[i][j] lands in lane 4b + j, element i.
// So lane l supplies A[l % 4][k] and B[k][n0 + l], and holds column n0 + l of
// the four output rows. Per 4 k a lane reads 16 bytes of A from LDS (four
// distinct addresses per wave) and 16 bytes of its weight row (kNT) or four
// values strided by ldw (kNN; 64 consecutive floats per k across the wave).
// A strip's k range is split over several waves and the partial sums are
// added through LDS, so each wave's MFMA chain is a fraction of the depth.

// acc += A[0..3][k0 .. k1) * op(W)[k][n], k0 % 4 == 0; A rows past k1 read 0.
template <int LAYOUT>
__device__ __forceinline__ f32x4 mfma_strip4(const float *__restrict__ A, int lda, __amdgpu_buffer_rsrc_t wr,
                                             int ldw, int n, int k0, int k1, bool wvec, bool avec) {
  const int lane = threadIdx.x & 63;
  const float *arow = A + (lane & 3) * lda;
  constexpr int kG = 8;  // groups of 4 k per load batch
  // A for the group at k (LDS; k past k1 reads 0)
  auto load_a = [&](float (&a)[4], int k) {
    if (avec && k + 4 <= k1) {
      const f32x4 v = *reinterpret_cast<const f32x4 *>(arow + k);
      a[0] = v[0]; a[1] = v[1]; a[2] = v[2]; a[3] = v[3];
    } else {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const float v = arow[min(k + t, k1 - 1)];
        a[t] = k + t < k1 ? v : 0.f;
      }
    }
  };
  f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
  for (int kb = k0; kb < k1; kb += 4 * kG) {
    // the batch's weights are loaded together, A one group ahead of its MFMAs
    float w[kG][4];
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      const int k = kb + 4 * g;
      if (k >= k1) break;  // uniform
      if (LAYOUT == kNT && wvec) {
        const f32x4 v = buf_load4(wr, uint32_t(n) * uint32_t(ldw) + uint32_t(k));
        w[g][0] = v[0]; w[g][1] = v[1]; w[g][2] = v[2]; w[g][3] = v[3];
      } else if (LAYOUT == kNT) {
#pragma unroll
        for (int t = 0; t < 4; ++t) w[g][t] = buf_load(wr, uint32_t(n) * uint32_t(ldw) + uint32_t(k + t));
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) w[g][t] = buf_load(wr, uint32_t(k + t) * uint32_t(ldw) + uint32_t(n));
      }
    }
    float a0[4], a1[4];
    load_a(a0, kb);
#pragma unroll
    for (int g = 0; g < kG; ++g) {
      if (kb + 4 * g >= k1) break;
      float (&cur)[4] = (g & 1) ? a1 : a0;
      float (&nxt)[4] = (g & 1) ? a0 : a1;
      if (g + 1 < kG && kb + 4 * (g + 1) < k1) load_a(nxt, kb + 4 * (g + 1));
      acc0 = __builtin_amdgcn_mfma_f32_4x4x1f32(cur[0], w[g][0], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_4x4x1f32(cur[1], w[g][1], acc1, 0, 0, 0);
      acc0 = __builtin_amdgcn_mfma_f32_4x4x1f32(cur[2], w[g][2], acc0, 0, 0, 0);
      acc1 = __builtin_amdgcn_mfma_f32_4x4x1f32(cur[3], w[g][3], acc1, 0, 0, 0);
    }
  }
  return acc0 + acc1;
}

// OUT[0..3][n] (LDS, ldo) = A[0..3] * op(W) + bias for every job (GemmJob;
// only rows 0..3 of A and OUT are touched). The jobs' 64-column strips are
// dealt over the waves, each strip's k range split into `parts` slices of a
// multiple of 4 (parts = nwaves / strips, at least 1); with parts > 1 the
// slices' sums go through scratch (LDS, nwaves * 256 floats) and a barrier,
// so all threads of the workgroup must call this. Without a barrier at the
// end: the caller synchronises before reading OUT.
template <int LAYOUT, int NJOBS>
__device__ __forceinline__ void tile_gemm4_jobs(const GemmJob (&jobs)[NJOBS], int nwaves,
                                                float *__restrict__ scratch) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  int strips = 0;
#pragma unroll
  for (int j = 0; j < NJOBS; ++j) strips += (jobs[j].n_total + 63) >> 6;
  const int parts = max(1, nwaves / max(strips, 1));
  // Items (strip, part) are numbered job by job; wave w takes items w,
  // w + nwaves, ... Each job is handled by its own unrolled code (constant
  // indices into jobs[]: a dynamically indexed job table would live in
  // scratch memory).
  int first = 0;  // the job's first item
#pragma unroll
  for (int j = 0; j < NJOBS; ++j) {
    const GemmJob &jb = jobs[j];
    const int nitems = ((jb.n_total + 63) >> 6) * parts;
    int it = wave;
    if (it < first) it += ((first - it + nwaves - 1) / nwaves) * nwaves;
    for (; it < first + nitems; it += nwaves) {
      const int local = it - first, sl = local / parts, p = local - sl * parts;
      const int n = sl * 64 + lane;
      const int per = ((jb.kd + parts - 1) / parts + 3) & ~3;
      const int k0 = min(jb.kd, p * per), k1 = min(jb.kd, k0 + per);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      if (k0 < k1) {
        const uint32_t span = LAYOUT == kNT ? uint32_t(jb.n_total - 1) * uint32_t(jb.ldw) + uint32_t(jb.kd)
                                            : uint32_t(jb.kd - 1) * uint32_t(jb.ldw) + uint32_t(jb.n_total);
        const __amdgpu_buffer_rsrc_t wr = weight_rsrc(jb.W, span);
        const bool wvec = LAYOUT == kNT && (jb.kd & 3) == 0 && (jb.ldw & 3) == 0 && aligned16(jb.W);
        const bool avec = (jb.lda & 3) == 0 && aligned16(jb.A);
        acc = mfma_strip4<LAYOUT>(jb.A, jb.lda, wr, jb.ldw, n, k0, k1, wvec, avec);
      }
      if (parts == 1) {
        if (n < jb.n_total) {
          const float bv = jb.bias != nullptr ? jb.bias[n] : 0.f;
#pragma unroll
          for (int i = 0; i < 4; ++i) jb.OUT[i * jb.ldo + n] = acc[i] + bv;
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) scratch[(it * 4 + i) * 64 + lane] = acc[i];
      }
    }
    first += nitems;
  }
  if (parts > 1) {
    __syncthreads();
    int sfirst = 0;  // the job's first strip
#pragma unroll
    for (int j = 0; j < NJOBS; ++j) {
      const GemmJob &jb = jobs[j];
      const int sj = (jb.n_total + 63) >> 6;
      for (int idx = threadIdx.x; idx < sj * 256; idx += nwaves * 64) {
        const int sl = idx >> 8, i = (idx >> 6) & 3, l = idx & 63;
        const int n = sl * 64 + l;
        if (n < jb.n_total) {
          float v = jb.bias != nullptr ? jb.bias[n] : 0.f;
          for (int p = 0; p < parts; ++p) v += scratch[(((sfirst + sl) * parts + p) * 4 + i) * 64 + l];
          jb.OUT[i * jb.ldo + n] = v;
        }
      }
      sfirst += sj;
    }
  }
}

}  // namespace sgl
