// Link-prediction metrics of one step on the device: average precision,
// ROC AUC and the pairwise statistic the reference calls "mrr", from the
// step's positive and negative logits, with no host synchronisation.
//
// Reference: CTDGOnlineRuntime._metric_dict  backends/ctdg/runtime/runtime.py:202-214
//   scores = sigmoid(logits) (float32), labels 1 for positives, 0 for negatives;
//   ap  = sklearn average_precision_score(labels, scores)
//   auc = sklearn roc_auc_score(labels, scores)
//   mrr = mean over (i, j) of [pos_score_i > neg_score_j]
//
// Per positive i with score s_i, counted over all scores:
//   lt_i = negatives below s_i, eq_i = negatives equal to s_i,
//   gp_i = positives >= s_i,    gn_i = negatives >= s_i = N - lt_i;
//   mrr = sum_i lt_i / (P N)
//   auc = sum_i (lt_i + eq_i / 2) / (P N)   (the Mann-Whitney statistic with
//         ties at one half: the trapezoidal area scikit-learn computes)
//   ap  = sum_i gp_i / (gp_i + gn_i) / P    (scikit-learn sums, over the
//         distinct scores in descending order, the recall step times the
//         precision at that score with every tied score counted: each
//         positive of a tie group adds 1/P times the group's precision)
// Scores are compared as float32 values, so ties are exact.
//
// The counts are direct comparisons, P (P + N) of them, spread so that a
// step's few thousand scores take one short launch: kSlices threads per
// positive each count a contiguous slice of the scores (staged in LDS by
// every workgroup, read four at a time), the slices' counts are summed with
// lane shuffles, the
// positives' terms summed in a fixed order per workgroup, and the last
// workgroup to finish (a device counter) adds the workgroups' partial sums in
// a fixed order: the result does not depend on the order workgroups finish.
// mrr is rounded to float32 as the reference's float mean of 0/1 values is
// (an exact count divided once).
//
// The workgroup body is shared by sgl_link_metrics (metrics.hip) and the
// batch preparation that carries a previous step's metrics in the same
// launch (state.hip): both call sgl::met::run from their own kernels.
#pragma once

#include "common.h"

namespace sgl {
namespace met {

constexpr int kBlock = 1024;
constexpr int kSlices = 16;                    // threads per positive
constexpr int kPosPerBlock = kBlock / kSlices; // 64
constexpr int kStage = 4;                      // staged scores per thread and round trip

// The metrics of one call: n_pos positive and n_neg negative logits, the
// loss to copy through (may be NULL), the ring and its counter (ring may be
// NULL), out[4] (may be NULL), per-workgroup partials [3 * blocks] and the
// completion word (0 between calls; the last workgroup resets it).
struct Args {
  int P, N;
  const float *pos, *neg, *loss;
  unsigned long long *seq;
  double *ring;
  int slots;
  double *out, *partials;
  unsigned int *done;
};

inline int64_t blocks_for(int64_t n_pos) { return n_pos > kPosPerBlock ? (n_pos + kPosPerBlock - 1) / kPosPerBlock : 1; }
inline size_t region(int m) { return size_t(kSlices) * size_t(((m + kSlices - 1) / kSlices + 3) & ~3); }
// dynamic LDS of a workgroup (the staged scores)
inline size_t lds_bytes(int n_pos, int n_neg) { return sizeof(float) * std::max<size_t>(4, region(n_pos) + region(n_neg)); }

__device__ __forceinline__ float sigmoid_f32(float x) { return 1.f / (1.f + expf(-x)); }

template <typename T>
__device__ __forceinline__ T block_sum(T v, T *s_part) {
  v = sgl::wave_reduce_sum(v);
  const int lane = threadIdx.x & (sgl::kWave - 1), w = threadIdx.x / sgl::kWave;
  if (lane == 0) s_part[w] = v;
  __syncthreads();
  T t = 0;
#pragma unroll
  for (int i = 0; i < kBlock / sgl::kWave; ++i) t += s_part[i];
  __syncthreads();
  return t;
}

// Workgroup b of nb (every thread of a kBlock-thread workgroup calls it;
// blocks_for(P) workgroups in all).
__device__ __forceinline__ void run(const Args &a, unsigned b, unsigned nb) {
  const int P = a.P, N = a.N;
  // LDS: the positives' scores in kSlices chunks of cp (padded with -inf,
  // which no score is >= of), then the negatives' in chunks of cn (padded
  // with +inf, neither below nor equal to a score); cp, cn multiples of 4
  extern __shared__ float4 s_score4[];
  float *s_score = reinterpret_cast<float *>(s_score4);
  __shared__ double s_part[kBlock / sgl::kWave];
  __shared__ bool s_last;
  const int tid = threadIdx.x;
  const int cp = ((P + kSlices - 1) / kSlices + 3) & ~3, cn = ((N + kSlices - 1) / kSlices + 3) & ~3;
  const int rp = kSlices * cp, rn = kSlices * cn;
  // every load of the staging issued before the first use (one memory round
  // trip for the common sizes: kStage values per thread)
  for (int i0 = tid; i0 < rp + rn; i0 += kStage * kBlock) {
    float x[kStage];
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = i0 + u * kBlock;
      x[u] = 0.f;
      if (i < rp) {
        if (i < P) x[u] = a.pos[i];
      } else if (i < rp + rn && i - rp < N) {
        x[u] = a.neg[i - rp];
      }
    }
#pragma unroll
    for (int u = 0; u < kStage; ++u) {
      const int i = i0 + u * kBlock;
      if (i < rp + rn)
        s_score[i] = i < rp ? (i < P ? sigmoid_f32(x[u]) : -INFINITY) : (i - rp < N ? sigmoid_f32(x[u]) : INFINITY);
    }
  }
  __syncthreads();
  const int slice = tid % kSlices;
  const int ip = int(b) * kPosPerBlock + tid / kSlices;
  int lt = 0, eq = 0, gp = 0;
  if (ip < P) {
    const float s = s_score[ip];
    // this slice's chunks, four scores per load, four loads in flight
    const float4 *pa = s_score4 + slice * (cp / 4);
#pragma unroll 4
    for (int m = 0; m < cp / 4; ++m) {
      const float4 v = pa[m];
      gp += (v.x >= s) + (v.y >= s) + (v.z >= s) + (v.w >= s);
    }
    const float4 *pb = s_score4 + rp / 4 + slice * (cn / 4);
#pragma unroll 4
    for (int m = 0; m < cn / 4; ++m) {
      const float4 v = pb[m];
      lt += (v.x < s) + (v.y < s) + (v.z < s) + (v.w < s);
      eq += (v.x == s) + (v.y == s) + (v.z == s) + (v.w == s);
    }
  }
  // the slices of one positive are consecutive lanes
#pragma unroll
  for (int d = kSlices / 2; d > 0; d >>= 1) {
    lt += __shfl_xor(lt, d, sgl::kWave);
    eq += __shfl_xor(eq, d, sgl::kWave);
    gp += __shfl_xor(gp, d, sgl::kWave);
  }
  const bool lead = ip < P && slice == 0;
  const double t_mrr = lead ? double(lt) : 0.0;
  const double t_auc = lead ? double(lt) + 0.5 * double(eq) : 0.0;
  const double t_ap = lead ? double(gp) / double(gp + N - lt) : 0.0;
  const double b_mrr = block_sum(t_mrr, s_part);
  const double b_auc = block_sum(t_auc, s_part);
  const double b_ap = block_sum(t_ap, s_part);
  if (tid == 0) {
    double *pp = a.partials + 3 * b;
    pp[0] = b_mrr;
    pp[1] = b_auc;
    pp[2] = b_ap;
    __threadfence();   // the partials before the count (release)
    s_last = atomicAdd(a.done, 1u) == nb - 1u;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();     // every workgroup's partials after its count (acquire)
  // the partials in a fixed order: thread t sums workgroups t, t + 1024, ...,
  // then a fixed tree over the threads
  double p_mrr = 0.0, p_auc = 0.0, p_ap = 0.0;
  for (unsigned w = tid; w < nb; w += kBlock) {
    const double *pp = a.partials + 3 * w;
    p_mrr += pp[0];
    p_auc += pp[1];
    p_ap += pp[2];
  }
  const double s_mrr = block_sum(p_mrr, s_part);
  const double s_auc = block_sum(p_auc, s_part);
  const double s_ap = block_sum(p_ap, s_part);
  if (tid != 0) return;
  *a.done = 0u;
  const double nan = __longlong_as_double(0x7ff8000000000000ll);
  const double pn = double(P) * double(N);
  const bool ok = P > 0 && N > 0;
  const double ap = ok ? s_ap / double(P) : nan;
  const double auc = ok ? s_auc / pn : nan;
  const double mrr = ok ? double(float(s_mrr) / float(pn)) : nan;
  // (the loss may come from another stream's work, ordered by a gate folded
  // into the kernel: an atomic load, never a scalar load issued before the
  // wait or served from the scalar cache)
  const double l =
      a.loss != nullptr ? double(__hip_atomic_load(const_cast<float *>(a.loss), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT))
                        : nan;
  if (a.out != nullptr) {
    a.out[0] = l;
    a.out[1] = ap;
    a.out[2] = auc;
    a.out[3] = mrr;
  }
  if (a.ring != nullptr) {
    const unsigned long long i = atomicAdd(a.seq, 1ull);   // stream-ordered calls: a plain increment
    double *r = a.ring + 4 * (i % static_cast<unsigned long long>(a.slots));
    r[0] = l;
    r[1] = ap;
    r[2] = auc;
    r[3] = mrr;
  }
}

}  // namespace met
}  // namespace sgl
