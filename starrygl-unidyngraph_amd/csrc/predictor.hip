// Edge predictor + BCE loss, forward and backward, one workgroup (16 waves)
// per 16 events. Reference: CTDGLinkPredictor.forward
// (backends/ctdg/runtime/models.py:313-324), the root-row selection of
// _conv_output (runtime.py:176-183) and the loss of train_step
// (runtime.py:290-292):
//   e_s = y[rs], e_d = y[rd], e_n = y[rn] (0 when the negative is not a root)
//   h_s = W_s e_s + b_s, h_d = W_d e_d + b_d, h_n = W_d e_n + b_d
//   pos = w_o . relu(h_s + h_d) + b_o,  neg = w_o . relu(h_s + h_n) + b_o
//   loss = mean softplus(-pos) + mean softplus(neg)  (BCE with logits, labels 1 / 0)
// In training mode the launch also produces the out_fc gradients and, per
// root r, the summed hidden-layer gradients
//   g_src[r] = sum_{e: rs[e] = r} dL/dh_s[e]
//   g_dst[r] = sum_{e: rd[e] = r} dL/dh_d[e] + sum_{e: rn[e] = r} dL/dh_n[e]
// with the negatives that are not roots summed into row U of g_dst. From
// these rows the attention backward gets dL/dy = W_s^T g_src + W_d^T g_dst,
// and the src_fc / dst_fc gradients are reductions over the roots
// (dW_s = sum_r g_src[r] y[r]^T, db_d = sum_{r <= U} g_dst[r], ...).
// With dropout the reference runs the attention once per role with its own
// masks (runtime.py:193-195): e_s, e_d and e_n then come from three passes'
// outputs (y, y + y_pass_stride, y + 2 y_pass_stride) and the negatives'
// gradients go to their own accumulator acc_neg (row U for non-roots).
// Every sum over events is accumulated in fixed point with integer atomics
// (exact, so independent of the workgroups' order): the per-root rows in the
// caller's accumulators (consumed and cleared by the attention backward), the
// loss and out_fc gradients in a small accumulator that the last workgroup to
// finish converts into the float outputs and clears.
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

struct ZeroSpans {
  float *p[4];
  int64_t n[4];
};

__global__ __launch_bounds__(256) void k_zero(ZeroSpans z) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (i < z.n[k]) z.p[k][i] = 0.f;
}

// PRE (bf16 products with every 16-column block of W_s and W_d on a wave of
// its own, D <= 32 kPreSteps): each wave loads its block's weight fragments
// and bias first, so that their round trip overlaps the index loads and row
// gathers, and holds them in registers for the products.
constexpr int kPreSteps = 4;
template <bool BF, bool PRE = false>
__global__ __launch_bounds__(kBlock) void k_predictor(
    int64_t batch, int D, int train, const int32_t *__restrict__ num_roots, const float *__restrict__ y,
    const int32_t *__restrict__ rs, const int32_t *__restrict__ rd, const int32_t *__restrict__ rn,
    const float *__restrict__ w_s, const float *__restrict__ b_s, const float *__restrict__ w_d,
    const float *__restrict__ b_d, const float *__restrict__ w_o, const float *__restrict__ b_o,
    float *__restrict__ pos_out, float *__restrict__ neg_out, float *__restrict__ loss,
    long long *__restrict__ acc_src, long long *__restrict__ acc_dst, float *__restrict__ g_wo,
    float *__restrict__ g_bo, long long *__restrict__ acc_out, int32_t *__restrict__ done, int agg,
    int64_t ystride, long long *__restrict__ acc_neg, sgl_bf16_weights bw) {
  const bool sep = acc_neg != nullptr;  // the negatives' rows apart from the dst rows
  int32_t *range_flag = done + SGL_DONE_RANGE_WORD;  // a value outside the fixed-point range
  long long *acc_n = sep ? acc_neg : acc_dst;
  extern __shared__ __align__(16) float lds[];
  const int ld = sgl::lds_ld(D);
  long long *Nul = reinterpret_cast<long long *>(lds);  // [D] dL/dh_n of the tile's non-root negatives
  float *Es = lds + 2 * ((D + 1) & ~1);
  float *Ed = Es + kRows * ld;
  float *En = Ed + kRows * ld;
  float *Hs = En + kRows * ld;   // h_s
  float *Hd = Hs + kRows * ld;   // h_d -> a_p
  float *Hn = Hd + kRows * ld;   // h_n -> a_n
  float *Wo = Hn + kRows * ld;   // [D] out_fc weight
  // with agg: per-root sums of the tile's hidden-layer gradients (fixed
  // point) before the global atomics, rows indexed by the root's first entry
  // in the src list (16) and the dst list (32: (i, dst), (i, neg) of event i)
  long long *Gs = reinterpret_cast<long long *>(Wo + ((D + 3) & ~3));
  long long *Gd = Gs + kRows * D;
  __shared__ float s_gp[kRows], s_gn[kRows], s_sp[kRows], s_pp[kRows], s_pn[kRows];
  __shared__ int s_idx[3][kRows];
  __shared__ int s_lead[3 * kRows];  // leader entry of src entry i, dst entries 2i / 2i+1
  __shared__ int s_last;
  __shared__ float s_bo;  // out_fc bias, staged with the first loads

  static_assert(!PRE || BF, "held weights are the bf16 copies");
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int64_t e0 = int64_t(blockIdx.x) * kRows;
  const int nrows = int(min<int64_t>(kRows, batch - e0));
  const int nblk = (D + 15) >> 4;
  sgl::bf16x8 wf[PRE ? kPreSteps : 1];
  float bv0 = 0.f;
  if constexpr (PRE) {
    if (wave < 2 * nblk) {
      const int nb = wave < nblk ? wave : wave - nblk, col = nb * 16 + (lane & 15);
      sgl::load_wfrag_bw<kPreSteps>(wf, wave < nblk ? bw.ws : bw.wd, bw.ld_d, nb * 16, D, D);
      bv0 = col < D ? (wave < nblk ? b_s[col] : b_d[col]) : 0.f;
    }
  }
  if (tid < kRows) {
    const bool ok = tid < nrows;
    s_idx[0][tid] = ok ? rs[e0 + tid] : -1;
    s_idx[1][tid] = ok ? rd[e0 + tid] : -1;
    s_idx[2][tid] = ok ? rn[e0 + tid] : -1;
  }
  for (int j = tid; j < D; j += kBlock) {
    Nul[j] = 0;
    Wo[j] = w_o[j];
  }
  if (tid == kRows) s_bo = b_o[0];
  if (agg && train)
    for (int k = tid; k < 3 * kRows * D; k += kBlock) Gs[k] = 0;
  __syncthreads();
  if (agg && train && tid < 3 * kRows) {
    // the first entry of the same list with the same root (-1: no root);
    // unrolled over the whole list, so its LDS reads issue together
    if (tid < kRows) {
      const int a = s_idx[0][tid];
      int l = -1;
#pragma unroll
      for (int t = kRows - 1; t >= 0; --t)
        if (t <= tid && a >= 0 && s_idx[0][t] == a) l = t;
      s_lead[tid] = l;
    } else {
      const int e = tid - kRows;
      const int r = s_idx[1 + (e & 1)][e >> 1];
      int l = -1;
#pragma unroll
      for (int t = 2 * kRows - 1; t >= 0; --t)
        if (t <= e && r >= 0 && s_idx[1 + (t & 1)][t >> 1] == r && (!sep || ((t ^ e) & 1) == 0)) l = t;
      s_lead[tid] = l;
    }
  }
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    const int a = s_idx[0][i], b = s_idx[1][i], c = s_idx[2][i];
    Es[i * ld + j] = a >= 0 ? y[size_t(a) * D + j] : 0.f;
    Ed[i * ld + j] = b >= 0 ? y[ystride + size_t(b) * D + j] : 0.f;
    En[i * ld + j] = c >= 0 ? y[2 * ystride + size_t(c) * D + j] : 0.f;
  }
  __syncthreads();
  if constexpr (PRE) {
    // the same products from the held fragments (one block per wave)
    if (wave < 2 * nblk) {
      const int nb = wave < nblk ? wave : wave - nblk, col = nb * 16 + (lane & 15);
      if (wave < nblk) {
        const sgl::f32x4 acc = sgl::mfma_block16_bw_pre<2, kPreSteps>(Es, ld, wf, D);
        if (col < D) {
#pragma unroll
          for (int v = 0; v < 4; ++v) Hs[(4 * (lane >> 4) + v) * ld + col] = acc[v] + bv0;
        }
      } else {
        const sgl::f32x4 ad = sgl::mfma_block16_bw_pre<2, kPreSteps>(Ed, ld, wf, D);
        const sgl::f32x4 an = sgl::mfma_block16_bw_pre<2, kPreSteps>(En, ld, wf, D);
        if (col < D) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            Hd[(4 * (lane >> 4) + v) * ld + col] = ad[v] + bv0;
            Hn[(4 * (lane >> 4) + v) * ld + col] = an[v] + bv0;
          }
        }
      }
    }
  } else {
    // h_s = W_s e_s + b_s on one set of waves; h_d and h_n (both W_d) on
    // another, each block's W_d loads shared by the two tiles
    for (int u = wave; u < 2 * nblk; u += kWaves) {
      const int nb = u < nblk ? u : u - nblk, n0 = nb * 16, col = n0 + (lane & 15);
      // the bias is loaded before the block's k loop (one round trip less)
      const float bv = col < D ? (u < nblk ? b_s[col] : b_d[col]) : 0.f;
      if (u < nblk) {
        // (the tiles are 16-byte aligned with ld % 4 == 0: two 16-byte reads per k step)
        const sgl::f32x4 acc = BF ? sgl::mfma_block16_bw<2>(Es, ld, bw.ws, bw.ld_d, n0, D, D)
                                  : sgl::mfma_block16<sgl::kNT>(Es, ld, w_s, D, n0, D, D);
        if (col < D) {
#pragma unroll
          for (int v = 0; v < 4; ++v) Hs[(4 * (lane >> 4) + v) * ld + col] = acc[v] + bv;
        }
      } else {
        sgl::f32x4 ad, an;
        if constexpr (BF) {
          // the block's W_d fragments loaded once for both tiles
          sgl::mfma_block16_bw_pair(Ed, En, ld, bw.wd, bw.ld_d, n0, D, D, ad, an);
        } else {
          sgl::mfma_block16_pair<sgl::kNT>(Ed, En, ld, w_d, D, n0, D, D, ad, an);
        }
        if (col < D) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            Hd[(4 * (lane >> 4) + v) * ld + col] = ad[v] + bv;
            Hn[(4 * (lane >> 4) + v) * ld + col] = an[v] + bv;
          }
        }
      }
    }
  }
  __syncthreads();
  // the two hidden-layer dot products: one wave per event
  for (int i = wave; i < kRows; i += kWaves) {
    float pp = 0.f, pn = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float hs = Hs[i * ld + j];
      const float ap = fmaxf(hs + Hd[i * ld + j], 0.f);
      const float an = fmaxf(hs + Hn[i * ld + j], 0.f);
      Hd[i * ld + j] = ap;
      Hn[i * ld + j] = an;
      pp += Wo[j] * ap;
      pn += Wo[j] * an;
    }
    pp = sgl::wave_sum_dpp(pp);
    pn = sgl::wave_sum_dpp(pn);
    if (lane == 0) {
      s_pp[i] = pp;
      s_pn[i] = pn;
    }
  }
  __syncthreads();
  // logits, loss terms and logit gradients of the tile's events on 16 lanes
  // of one wave (the waves sharing a SIMD would run the branchy scalar tail
  // one after another)
  if (tid < kRows) {
    const int i = tid;
    float gp = 0.f, gn = 0.f, sp = 0.f;
    if (i < nrows) {
      const float p = s_pp[i] + s_bo, n = s_pn[i] + s_bo;
      pos_out[e0 + i] = p;
      neg_out[e0 + i] = n;
      sp = softplus(-p) + softplus(n);
      gp = (sigmoid(p) - 1.f) / float(batch);
      gn = sigmoid(n) / float(batch);
    }
    s_gp[i] = gp;
    s_gn[i] = gn;
    s_sp[i] = sp;
  }
  __syncthreads();
  if (tid == 0) {
    float sp = 0.f;
    for (int i = 0; i < kRows; ++i) sp += s_sp[i];
    sgl::atomic_add_fixed(&acc_out[D + 1], sgl::to_fixed_checked(sp, range_flag));
  }
  if (train) {  // uniform
    // out_fc gradients: this tile's sums
    for (int j = tid; j < D; j += kBlock) {
      float gw = 0.f;
      for (int i = 0; i < kRows; ++i) gw += s_gp[i] * Hd[i * ld + j] + s_gn[i] * Hn[i * ld + j];
      sgl::atomic_add_fixed(&acc_out[j], sgl::to_fixed_checked(gw, range_flag));
    }
    if (tid == 64) {
      float gb = 0.f;
      for (int i = 0; i < kRows; ++i) gb += s_gp[i] + s_gn[i];
      sgl::atomic_add_fixed(&acc_out[D], sgl::to_fixed_checked(gb, range_flag));
    }
    // hidden-layer gradients, summed into their roots' rows
    for (int idx = tid; idx < kRows * D; idx += kBlock) {
      const int i = idx / D, j = idx - i * D;
      if (i >= nrows) continue;
      const float ghp = Hd[i * ld + j] > 0.f ? s_gp[i] * Wo[j] : 0.f;
      const float ghn = Hn[i * ld + j] > 0.f ? s_gn[i] * Wo[j] : 0.f;
      const int a = s_idx[0][i], b = s_idx[1][i], c = s_idx[2][i];
      const long long fp = sgl::to_fixed_checked(ghp, range_flag), fn = sgl::to_fixed_checked(ghn, range_flag);
      if (agg) {  // LDS atomics into the roots' leader rows
        auto add = [](long long *q, long long v) {
          atomicAdd(reinterpret_cast<unsigned long long *>(q), static_cast<unsigned long long>(v));
        };
        if (a >= 0) add(&Gs[s_lead[i] * D + j], fp + fn);
        if (b >= 0) add(&Gd[s_lead[kRows + 2 * i] * D + j], fp);
        if (c >= 0) add(&Gd[s_lead[kRows + 2 * i + 1] * D + j], fn);
        else if (fn != 0) add(&Nul[j], fn);
        continue;
      }
      if (a >= 0) sgl::atomic_add_fixed(&acc_src[size_t(a) * D + j], fp + fn);
      if (b >= 0) sgl::atomic_add_fixed(&acc_dst[size_t(b) * D + j], fp);
      if (c >= 0) sgl::atomic_add_fixed(&acc_n[size_t(c) * D + j], fn);
      else if (fn != 0) atomicAdd(reinterpret_cast<unsigned long long *>(&Nul[j]), static_cast<unsigned long long>(fn));
    }
  }
  // The last workgroup to finish its loss and out_fc sums turns them into the
  // outputs and clears the accumulator and the counter for the next launch.
  // The sums only ever change by atomics, which are performed at the
  // device's coherence point: a workgroup waits for its own atomics to
  // complete before it counts itself done, and the last one reads the sums
  // with atomics too, so no cache writeback is needed. With the per-root
  // sums aggregated in LDS (agg), the wait comes before their global atomics
  // (the attention backward, the next kernel, is their only reader), so the
  // count and the conversion overlap them.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) s_last = sgl::last_block(done);
  __syncthreads();
  if (s_last) {
    auto take = [&](int k) {
      return sgl::from_fixed(static_cast<long long>(atomicExch(reinterpret_cast<unsigned long long *>(&acc_out[k]), 0ull)));
    };
    if (train) {
      for (int j = tid; j < D; j += kBlock) g_wo[j] = take(j);
      if (tid == 64) g_bo[0] = take(D);
    }
    if (tid == 0) *loss = float(double(take(D + 1)) / double(batch));
  }
  if (!train) return;  // uniform
  if (agg) {  // one global atomic per (root in the tile, column)
    for (int k = tid; k < 3 * kRows * D; k += kBlock) {
      const int e = k / D, j = k - e * D;
      if (s_lead[e] != (e < kRows ? e : e - kRows)) continue;  // not a leader, or no root
      const long long v = Gs[k];
      if (v == 0) continue;
      if (e < kRows) {
        sgl::atomic_add_fixed(&acc_src[size_t(s_idx[0][e]) * D + j], v);
      } else {
        const int t = e - kRows;
        sgl::atomic_add_fixed(&((t & 1) ? acc_n : acc_dst)[size_t(s_idx[1 + (t & 1)][t >> 1]) * D + j], v);
      }
    }
  }
  const int U = *num_roots;
  for (int j = tid; j < D; j += kBlock)
    if (Nul[j] != 0) sgl::atomic_add_fixed(&acc_n[size_t(U) * D + j], Nul[j]);
}

}  // namespace

extern "C" int sgl_predictor(int64_t batch, int32_t D, int64_t capacity, int32_t train, const int32_t *num_roots,
                             const float *y, const int32_t *ridx_src, const int32_t *ridx_dst, const int32_t *ridx_neg,
                             const float *w_s, const float *b_s, const float *w_d, const float *b_d,
                             const float *w_o, const float *b_o, float *pos_logits, float *neg_logits, float *loss,
                             int64_t *acc_src, int64_t *acc_dst, float *g_wo, float *g_bo, int64_t *acc_out,
                             int32_t *done, int64_t y_pass_stride, int64_t *acc_neg, const sgl_bf16_weights *bw,
                             hipStream_t stream) {
  SGL_REQUIRE(batch >= 0 && batch < INT_MAX && D > 0 && capacity >= 0, "predictor: bad sizes");
  SGL_REQUIRE(num_roots && y && ridx_src && ridx_dst && ridx_neg && w_s && b_s && w_d && b_d && w_o && b_o &&
                  pos_logits && neg_logits && loss && acc_out && done,
              "predictor: NULL array");
  SGL_REQUIRE(!train || (acc_src && acc_dst && g_wo && g_bo), "predictor: NULL gradient array");
  SGL_REQUIRE(y_pass_stride >= 0, "predictor: negative y_pass_stride");
  SGL_REQUIRE(bw == nullptr || (bw->ws && bw->wd && bw->ld_d >= D && bw->ld_d % 8 == 0 && y_pass_stride == 0 &&
                                (reinterpret_cast<uintptr_t>(bw->ws) & 15u) == 0 &&
                                (reinterpret_cast<uintptr_t>(bw->wd) & 15u) == 0),
              "predictor: bad bf16 weight copies (or a dropout pass stride with them)");
  if (batch == 0) {  // no events: zero loss and out_fc gradients
    const ZeroSpans z{{loss, train ? g_wo : nullptr, train ? g_bo : nullptr, nullptr}, {1, train ? D : 0, train, 0}};
    k_zero<<<unsigned((D + 255) / 256), 256, 0, stream>>>(z);
    SGL_CHECK_LAUNCH();
    return SGL_OK;
  }
  const size_t lds0 = sizeof(float) * (size_t(kRows) * 6 * sgl::lds_ld(D) + 2 * ((D + 1) & ~1) + ((D + 3) & ~3));
  SGL_REQUIRE(lds0 <= 160 * 1024, "predictor: D=%d needs %zu bytes of LDS", D, lds0);
  // the per-root gradient sums in LDS when they fit (otherwise one global atomic per event)
  const size_t lds_agg = lds0 + sizeof(long long) * 3 * kRows * size_t(D);
  const int agg = train && lds_agg <= 160 * 1024 ? 1 : 0;
  const size_t lds = agg ? lds_agg : lds0;
  const bool pre = bw != nullptr && 2 * ((D + 15) / 16) <= kWaves && D <= 32 * kPreSteps;
  auto kern = bw == nullptr ? &k_predictor<false> : pre ? &k_predictor<true, true> : &k_predictor<true>;
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(kern), lds));
  sgl::launch(kern, dim3(unsigned((batch + kRows - 1) / kRows)), dim3(kBlock), lds, stream, batch, D, train,
              num_roots, y, ridx_src, ridx_dst, ridx_neg, w_s, b_s, w_d, b_d, w_o, b_o, pos_logits, neg_logits, loss,
              reinterpret_cast<long long *>(acc_src), reinterpret_cast<long long *>(acc_dst), g_wo, g_bo,
              reinterpret_cast<long long *>(acc_out), done, agg, y_pass_stride,
              train ? reinterpret_cast<long long *>(acc_neg) : nullptr, bw != nullptr ? *bw : sgl_bf16_weights{});
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
