// TGN temporal attention (TimeEncode + TemporalTransformerConv), forward and
// backward, one workgroup (8 or 16 waves) per tile of 4 or 8 roots (the
// 16-wave bf16 forward: one root).
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
// 2H dot/axpy passes over C floats remain.
//
// Latency structure: a step has a few hundred roots, and every phase is a
// chain of L2 round trips. The edge rows' gathered columns [memory[nbr] |
// efeat[eid]] are copied beforehand by k_edge_rows, one wave per sampled
// edge, in the padded sampler layout [root][slot], so the attention kernels
// read each edge's row contiguously instead of chasing (nbr, eid) to the
// memory table. The forward fills in the rows' time-encoding columns (they
// depend on trained parameters) and saves the sines for the backward. A
// workgroup takes few roots (RPW = 1, 4 or 8; the MFMA tiles keep 16 rows,
// zero-padded), so a launch spreads over U/RPW workgroups. The GEMMs issue all weight loads of a block at once (mfma.h).
// In the edge phase WPR = waves / RPW waves share a root: each takes a
// contiguous slice of the window and reads the rows of 4 edges per round
// trip, with its own online softmax (running max, running sum); the slices
// are merged through LDS (global max, rescaled sums). The backward splits the
// window the same way and sums the slices' gradient partials.
//
// No 1/sqrt(d) scaling (models.py:125). The time-encoding argument is
// fl(fl(dt * w) + b), then cos.
#include <climits>

#include "common.h"
#include "mfma.h"

namespace {

constexpr int kRows = 16;   // MFMA tile rows
constexpr int kEC = 4;      // edges gathered per round trip
constexpr int kMaxH = 4;
constexpr int kMaxJ = 8;    // C <= 512
constexpr int kMaxWaves = 16;

// Waves per workgroup for a (heads, column slots) instance: 16 (128 VGPRs
// each) while the edge loop's per-lane [H][J] arrays fit, else 8 (256 VGPRs).
constexpr int waves_for(int hm, int jm) { return hm * jm <= 6 || (hm == 2 && jm == 4) ? 16 : 8; }
// Roots per workgroup: 16 waves share 4 roots (4 waves a root, merged
// through LDS); 8 waves take 8 roots (one wave each, no merge).
constexpr int rows_for(int nw) { return nw == 16 ? 4 : 8; }
// The fp32 and dropout instances take 4 roots with either wave count (the
// 8-wave ones two waves a root, merged through LDS) where both 4-root
// layouts fit in LDS (fp32_four_fits): a 16-row product tile of 4 roots costs
// about what one of 8 does, and twice the workgroups share the step's roots
// (config 1, 8 waves: forward 44.0 -> 37.8 us, backward 41.3 -> 33.9 us;
// 2 roots 37.4 / 35.4). Wider shapes (config 5's 4 heads of 288 columns:
// the merge partials need 184 KB) keep 8 roots, one wave each.
constexpr int kFp32Rows = 4;

struct Dims {
  int D, F, T, H, C, dh, k;
};

__device__ __forceinline__ float wave_sum(float v) { return sgl::wave_sum_dpp(v); }

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

// sin and cos of an fp32 time-encoding argument. Cody-Waite reduction by
// pi/2 in double precision with a three-part split of pi/2 (26-, 23- and
// 53-bit pieces, so k*P1 and k*P2 are exact for |k| < 2^27), then fp32
// polynomials on |r| <= pi/4 with the Cephes sinf/cosf coefficients
// (S. Moshier, Cephes Math Library); about 1.3 ulp against a float64 libm.
// Arguments beyond 1.5e8 (k near 2^27) take the library sincosf.
__device__ __forceinline__ void te_sincos(float x, float &sn, float &cs) {
  if (fabsf(x) > 1.5e8f) {
    sincosf(x, &sn, &cs);
    return;
  }
  const double xd = x;
  const double k = rint(xd * 0.63661977236758134308);
  double r = fma(-k, 1.5707963407039642, xd);
  r = fma(-k, -1.3909067675399456e-08, r);
  r = fma(-k, 6.123233995736766e-17, r);
  const float rf = float(r), z = rf * rf;
  const float sp = fmaf(fmaf(fmaf(-1.9515295891e-4f, z, 8.3321608736e-3f), z, -1.6666654611e-1f), z * rf, rf);
  const float cp =
      fmaf(fmaf(fmaf(2.443315711809948e-5f, z, -1.388731625493765e-3f), z, 4.166664568298827e-2f), z * z,
           fmaf(-0.5f, z, 1.f));
  const int q = int(k) & 3;  // quadrant (two's complement keeps it right for k < 0)
  sn = q == 0 ? sp : q == 1 ? cp : q == 2 ? -sp : -cp;
  cs = q == 0 ? cp : q == 1 ? -sp : q == 2 ? -cp : sp;
}

// Edge rows: X[r*K + e][0, D+F) = [memory[nbr] | efeat[eid]] for every live
// root r < U and sampled slot e < cnt[r] (rows of C = D+F+T floats; padding
// slots are not written). The time-encoding columns depend on trained
// parameters and are filled in by the attention forward. A wave takes RW
// consecutive roots (a bounded grid strides over the live roots) and copies
// their live rows as one list, 64/L rows per pass, so padding slots cost
// nothing and a pass is full whatever the per-root counts (RW = kEdgeGroup
// when the roots outnumber one pass of the grid; one root per wave below that, for
// the shortest chain of dependent loads). Rows are copied in V-float vectors
// by L lanes each, up to JM vectors per lane: V = 4 when D, F and C are
// multiples of four and the arrays 16-byte aligned, with the fewest lanes per
// row that keep JM <= 12 (4 lanes for D+F <= 192); otherwise a float per lane
// and the whole wave per row. Each lane's loads are issued together.
constexpr int kEdgeBlock = 256;
constexpr int kEdgeWaves = kEdgeBlock / sgl::kWave;
constexpr int kEdgeGroup = 4;  // roots per wave when the roots outnumber one pass of the grid

template <int V> struct EdgeVec;
template <> struct EdgeVec<1> { using type = float; };
template <> struct EdgeVec<4> { using type = float4; };

template <int V, int L, int JM, int RW>
__global__ __launch_bounds__(kEdgeBlock) void k_edge_rows(
    Dims d, int64_t capacity, const int32_t *__restrict__ num_roots, const float *__restrict__ memory,
    const float *__restrict__ efeat, const int32_t *__restrict__ cnt, const int32_t *__restrict__ nbr,
    const int32_t *__restrict__ eid, float *__restrict__ X) {
  static_assert(RW == 1 || RW == 2 || RW == 4 || RW == 8 || RW == 16, "RW: a power of two up to 16");
  using vec = typename EdgeVec<V>::type;
  constexpr int kPass = sgl::kWave / L;  // rows per pass
  const int lane = threadIdx.x & 63;
  const int q = lane & (L - 1), sub = lane / L;
  const int Dv = d.D / V, Fv = d.F / V, Wv = Dv + Fv, Cv = d.C / V;
  const int64_t live = min(capacity, int64_t(*num_roots));
  for (int64_t r0 = (int64_t(blockIdx.x) * kEdgeWaves + (threadIdx.x >> 6)) * RW; r0 < live;
       r0 += int64_t(gridDim.x) * kEdgeWaves * RW) {
    // lanes 0..RW-1: the group's counts and their inclusive prefix
    const int c = (lane < RW && r0 + lane < live) ? cnt[r0 + lane] : 0;
    int incl = c;
#pragma unroll
    for (int dd = 1; dd < RW; dd <<= 1) {
      const int t = __shfl_up(incl, dd, sgl::kWave);
      if (lane >= dd) incl += t;
    }
    const int total = __shfl(incl, RW - 1, sgl::kWave);
    for (int f0 = 0; f0 < total; f0 += kPass) {  // uniform trip count: every lane takes the shuffles
      const int f = f0 + sub;
      // the group's root j holding list entry f: the number of prefixes <= f
      int j = 0;
#pragma unroll
      for (int st = RW / 2; st > 0; st >>= 1) {
        const int p = __shfl(incl, j + st - 1, sgl::kWave);
        if (p <= f) j += st;
      }
      const int e = f - __shfl(incl - c, j, sgl::kWave);
      if (f >= total) continue;
      const int64_t row = (r0 + j) * d.k + e;
      const int nb = nbr[row], ei = eid[row];
      const vec *mrow = reinterpret_cast<const vec *>(memory) + size_t(nb) * Dv;
      const vec *frow = reinterpret_cast<const vec *>(efeat) + size_t(ei) * Fv;
      vec *xrow = reinterpret_cast<vec *>(X) + size_t(row) * Cv;
      vec v[JM];
#pragma unroll
      for (int jj = 0; jj < JM; ++jj) {
        const int cc = q + L * jj;
        const vec *src = cc < Dv ? mrow + cc : frow + (cc - Dv);
        v[jj] = cc < Wv ? *src : vec{};
      }
#pragma unroll
      for (int jj = 0; jj < JM; ++jj) {
        const int cc = q + L * jj;
        if (cc < Wv) xrow[cc] = v[jj];
      }
    }
  }
}

// This lane's slice of edge row `row` (c = lane + 64*j; zero past C) with
// its time-encoding columns computed from dt and the time encoding's
// parameters (te_w / te_b, staged in LDS): cos into x and into the row,
// sin into S's row.
template <int JM>
__device__ __forceinline__ void fill_row(const Dims &d, float *__restrict__ X, float *__restrict__ S, size_t row,
                                         const float *__restrict__ te_w, const float *__restrict__ te_b, float dtv,
                                         int lane, float (&x)[JM]) {
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int c = lane + 64 * j;
    float v = 0.f;
    if (c < d.D + d.F) {
      v = X[row * d.C + c];
    } else if (c < d.C) {
      const int t = c - d.D - d.F;
      float sn;
      te_sincos(te_arg(dtv, te_w[t], te_b[t]), sn, v);
      X[row * d.C + c] = v;
      S[row * d.T + t] = sn;
    }
    x[j] = v;
  }
}

// This lane's slice of edge row `row` of X (c = lane + 64*j; zero past C).
template <int JM>
__device__ __forceinline__ void load_row(const Dims &d, const float *__restrict__ X, size_t row, int lane,
                                         float (&x)[JM]) {
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int c = lane + 64 * j;
    x[j] = c < d.C ? X[row * d.C + c] : 0.f;
  }
}

// A tile's products OUT = A * op(W) + bias: four-row MFMA strips for tiles
// of 4 roots with k-major weights (sgl::tile_gemm4_jobs, partial sums in
// `scratch`; a wave's weight loads are 64 consecutive floats per k), 16x16
// blocks otherwise (for row-major weights a four-row strip would read 64
// weight rows per load instruction). Called by every thread of the
// workgroup.
template <int LAYOUT, int RPW, int NJOBS>
__device__ __forceinline__ void tile_products(const sgl::GemmJob (&jobs)[NJOBS], int nwaves, float *scratch) {
  if constexpr (RPW == 4 && LAYOUT == sgl::kNN) {
    sgl::tile_gemm4_jobs<LAYOUT>(jobs, nwaves, scratch);
  } else {
    (void)scratch;
    sgl::tile_gemm16_jobs<LAYOUT>(jobs, nwaves);
  }
}

// The slice [lo, hi) of a window of ne edges that slice `sub` of `nsub` takes.
__device__ __forceinline__ void window_slice(int ne, int sub, int nsub, int &lo, int &hi) {
  const int per = (ne + nsub - 1) / nsub;
  lo = min(ne, sub * per);
  hi = min(ne, lo + per);
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
  float *phi0;   // [T]          cos(b): the query's time encoding (may be NULL)
  float *sdrop;  // [cap][H]     with attention dropout: sum of the kept, rescaled weights
};

struct FwdLds {
  int ldh, ldr, lda, ldq;
  float *HT;    // [16][ldh]  [h | cos(b)]
  float *Qs;    // [16][ldr]
  float *AH;    // [16][lda]  [agg | h]
  float *Zs;    // [16][ldr]
  float *QT;    // [16][ldq]  qt, then xbar
  float *qb;    // [16][H]
  float *TW, *TB;  // [T] time-encoding weight / bias
  float *BK, *LG, *LB;  // [D] key bias, LayerNorm weight and bias (staged with the first loads)
  float *part;  // [NW][H*C]  a slice's unnormalised sums (slices only)
  float *pml;   // [NW][H][3] a slice's running max, sum and kept sum (slices only)
  float *scr;   // [NW][4][64] partial sums of the four-row products (4-root tiles only)
  float *DT;    // [rows][k] the tile's edges' dt (16-wave instances: stage_dt)
  float *Ts;    // [ts_rows][T] the tile's edges' time encodings (cos), when staged
};

// 16-wave instances encode the tile's edges' times beside the Q product, on
// the waves Q leaves idle, one edge slot per wave at a time (lanes over the T
// columns: the slot's index arithmetic is scalar, no per-element division).
// The tile's dt rows are staged in LDS with the setup loads, so the loop
// waits on no global load (each such wait would also wait for the loop's
// earlier stores: loads and stores share one in-order counter).
__host__ __device__ constexpr bool stage_dt(int nw, int rows) { return nw == 16 && rows > 0; }

__host__ __device__ inline FwdLds fwd_lds(const Dims &d, float *base, int nw, int rows, bool slices) {
  FwdLds L;
  L.ldh = sgl::lds_ld(d.D + d.T);
  L.ldr = sgl::lds_ld(d.D);
  L.lda = sgl::lds_ld(2 * d.D);
  L.ldq = sgl::lds_ld(d.H * d.C);
  L.HT = base;
  L.Qs = L.HT + kRows * L.ldh;
  L.AH = L.Qs + kRows * L.ldr;
  L.Zs = L.AH + kRows * L.lda;
  L.QT = L.Zs + kRows * L.ldr;
  L.qb = L.QT + kRows * L.ldq;
  L.TW = L.qb + kRows * d.H;
  L.TB = L.TW + d.T;
  L.BK = L.TB + d.T;
  L.LG = L.BK + d.D;
  L.LB = L.LG + d.D;
  L.part = L.LB + d.D;
  L.pml = L.part + (slices ? nw * d.H * d.C : 0);
  L.scr = L.pml + (slices ? ((nw * d.H * 3 + 3) & ~3) : 0);
  L.DT = L.scr + (rows == 4 ? nw * 256 : 0);
  L.Ts = L.DT + (stage_dt(nw, rows) ? ((rows * d.k + 3) & ~3) : 0);
  return L;
}

// ts_rows: edges whose time encodings are staged in LDS (roots per tile *
// fanout), 0 = computed in the edge loop instead.
inline size_t fwd_lds_floats(const Dims &d, int nw, int rows, bool slices, int ts_rows) {
  float *base = reinterpret_cast<float *>(uintptr_t(4096));
  const FwdLds L = fwd_lds(d, base, nw, rows, slices);
  return size_t(L.Ts + size_t(ts_rows) * d.T - base);
}

// HG: head groups per root in the edge phase. With HG = 2 the two waves of a
// root each take half of its heads over the whole window (heads are
// independent there: no merge), halving the per-lane [head][column] arrays,
// so that wide rows with several heads fit 16-wave workgroups.
template <int HM, int JM, bool DROP, bool BF = false, int NW = waves_for(HM, JM), int RPW = rows_for(NW), int HG = 1>
__global__ __launch_bounds__(NW * 64) void k_conv_fwd(
    Dims d, const int32_t *__restrict__ num_roots, const int32_t *__restrict__ any_edges,
    const float *__restrict__ h_root, const int32_t *__restrict__ cnt, float *__restrict__ X,
    const float *__restrict__ dt, float *__restrict__ S, ConvParams p, ConvSaved sv, float *__restrict__ y,
    int ts_rows, sgl::DropCfg dc, sgl_bf16_weights bw) {
  constexpr int kWaves = NW, kBlock = NW * 64;
  constexpr int WPR = NW / RPW;  // waves per root in the edge phase
  constexpr int NS = WPR / HG;   // window slices per root (merged through LDS when > 1)
  constexpr int HL = HM / HG;    // heads per wave in the edge phase
  static_assert(RPW <= kRows && NW % RPW == 0, "tile shape");
  static_assert(WPR % HG == 0 && HM % HG == 0 && (HG == 1 || NS == 1), "head groups");
  static_assert(!(BF && DROP), "the bf16 products run without dropout");
  extern __shared__ __align__(16) float lds[];
  const int D = d.D, T = d.T, H = d.H, C = d.C, dh = d.dh, K = d.k;
  const FwdLds L = fwd_lds(d, lds, NW, RPW, NS > 1);
  __shared__ int s_cnt[kRows];
  __shared__ float s_sd[kRows][kMaxH];  // with attention dropout: the rows' kept-weight sums

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int U = *num_roots;
  const int r0 = blockIdx.x * RPW;
  const int nrows = max(0, min(RPW, U - r0));
  const bool live = *any_edges != 0;
  const unsigned long long dstep = DROP ? *dc.step : 0ull;
  const float sa = sgl::drop_scale(dc.p_att), so = sgl::drop_scale(dc.p_out);
  if (nrows == 0 || !live) {
    // rows outside the live set: zero output (y's row U is the null
    // embedding the predictor's reductions read); a block without edges:
    // zero output and zero saved state (the backward then produces zero
    // gradients). Saved state of rows past the live set is never read.
    for (int idx = tid; idx < RPW * D; idx += kBlock) y[size_t(r0) * D + idx] = 0.f;
    if (live) return;
    for (int idx = tid; idx < RPW * D; idx += kBlock) {
      const size_t o = size_t(r0) * D + idx;
      sv.Q[o] = 0.f; sv.agg[o] = 0.f; sv.z[o] = 0.f;
    }
    for (int idx = tid; idx < RPW * H * C; idx += kBlock) {
      sv.qt[size_t(r0) * H * C + idx] = 0.f;
      sv.xbar[size_t(r0) * H * C + idx] = 0.f;
    }
    for (int idx = tid; idx < RPW * 2; idx += kBlock) sv.stats[size_t(r0) * 2 + idx] = 0.f;
    if (DROP)
      for (int idx = tid; idx < RPW * H; idx += kBlock) sv.sdrop[size_t(r0) * H + idx] = 0.f;
    return;
  }
  if (tid < kRows) s_cnt[tid] = tid < nrows ? cnt[r0 + tid] : 0;
  for (int t = tid; t < T; t += kBlock) {
    L.TW[t] = p.te_w[t];
    L.TB[t] = p.te_b[t];
  }
  // the tile's dt rows (padding slots included: only live slots are encoded)
  if constexpr (stage_dt(NW, RPW))
    if (T > 0)
      for (int idx = tid; idx < RPW * K; idx += kBlock) L.DT[idx] = dt[size_t(r0) * K + idx];
  // the small parameter vectors of later phases, staged now so that no later
  // phase waits on a global load for them
  for (int j = tid; j < D; j += kBlock) {
    L.BK[j] = p.b_k[j];
    L.LG[j] = p.ln_g[j];
    L.LB[j] = p.ln_b[j];
  }
  // HT = [h | cos(b)] (TimeEncode(0) = cos(0*w + b)); AH[:, D:] = h
  for (int idx = tid; idx < kRows * (D + T); idx += kBlock) {
    const int i = idx / (D + T), j = idx - i * (D + T);
    float v;
    if (j < D) {
      v = i < nrows ? h_root[size_t(r0 + i) * D + j] : 0.f;
      L.AH[i * L.lda + D + j] = v;
    } else {
      v = cosf(p.te_b[j - D]);
      if (i == 0 && blockIdx.x == 0 && sv.phi0 != nullptr) sv.phi0[j - D] = v;
    }
    L.HT[i * L.ldh + j] = v;
  }
  __syncthreads();
  // Q = W_q [h | cos(b)] + b_q on the first (D+15)/16 waves (one 16x16
  // block each). In 16-wave instances the other waves compute the tile's
  // edges' cos / sin meanwhile: cos into the rows' time columns (and into
  // LDS when staged, ts_rows == RPW * K), sin into S (the backward); the
  // edge loop reads them after the barrier. 8-wave instances compute them
  // in the edge loop.
  constexpr bool kPre = NW == 16;
  const bool staged = kPre && ts_rows > 0;
  if constexpr (BF) {
    const sgl::GemmJobBw jobs[1] = {{L.HT, L.ldh, bw.wq, bw.ld_q, p.b_q, L.Qs, L.ldr, D + T, D}};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    const sgl::GemmJob jobs[1] = {{L.HT, L.ldh, p.w_q, D + T, p.b_q, L.Qs, L.ldr, D + T, D}};
    tile_products<sgl::kNT, RPW>(jobs, kWaves, L.scr);
  }
  if (kPre) {
    const int qwaves = min(kWaves - 1, (D + 15) / 16);
    // wave tw takes edge slots el = tw, tw + ntw, ... (el = i * K + e)
    const int ntw = kWaves - qwaves, tw = wave - qwaves;
    if (tw >= 0 && K > 0) {
      int i = tw / K, e = tw - (tw / K) * K;
      for (int el = tw; el < RPW * K; el += ntw) {
        if (e < s_cnt[i]) {
          const size_t row = size_t(r0 + i) * K + e;
          const float dtv = stage_dt(NW, RPW) ? L.DT[el] : dt[row];
          for (int t = lane; t < T; t += 64) {
            float sn, cs;
            te_sincos(te_arg(dtv, L.TW[t], L.TB[t]), sn, cs);
            if (staged) L.Ts[el * T + t] = cs;
            X[row * C + D + d.F + t] = cs;
            S[row * T + t] = sn;
          }
        }
        e += ntw;
        while (e >= K) { e -= K; ++i; }
      }
    }
  }
  __syncthreads();
  for (int idx = tid; idx < RPW * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    sv.Q[size_t(r0 + i) * D + j] = i < nrows ? L.Qs[i * L.ldr + j] : 0.f;
  }
  // qb[i][h] = <Q_ih, b_k,h> for the live rows: one wave per (row, head)
  for (int pr = wave; pr < RPW * H; pr += kWaves) {
    const int i = pr / H, h = pr - (pr / H) * H;
    float acc = 0.f;
    for (int j = lane; j < dh; j += 64) acc += L.Qs[i * L.ldr + h * dh + j] * L.BK[h * dh + j];
    acc = wave_sum(acc);
    if (lane == 0) L.qb[i * H + h] = acc;
  }
  // qt_h = Q_h W_k[h rows, :]  (kNN: rows of W_k are the reduction index;
  // the bf16 products read W_k^T)
  if constexpr (BF) {
    sgl::GemmJobBw jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.Qs + h * dh, L.ldr, bw.wkt + h * bw.hp, bw.ld_h, nullptr, L.QT + h * C, L.ldq, dh,
                 h < H ? C : 0};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    sgl::GemmJob jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.Qs + h * dh, L.ldr, p.w_k + size_t(h) * dh * C, C, nullptr, L.QT + h * C, L.ldq, dh,
                 h < H ? C : 0};
    tile_products<sgl::kNN, RPW>(jobs, kWaves, L.scr);
  }
  __syncthreads();

  // edge phase: wave w takes window slice sl of root w / WPR's window for
  // the heads of its head group hg (sub = w % WPR = hg * NS + sl)
  {
    const int i = wave / WPR, sub = wave % WPR;
    const int hg = sub / NS, sl = sub - hg * NS;
    const int r = r0 + i;
    const int ne = s_cnt[i];
    int elo, ehi;
    window_slice(ne, sl, NS, elo, ehi);
    float q[HL][JM], acc[HL][JM], m[HL], l[HL], qbh[HL];
    float ls[HL];  // with attention dropout: the running sum of the kept, rescaled weights
#pragma unroll
    for (int h = 0; h < HL; ++h) {
      const int hh = hg * HL + h;
      m[h] = -INFINITY;
      l[h] = 0.f;
      ls[h] = 0.f;
      qbh[h] = hh < H ? L.qb[i * H + hh] : 0.f;
#pragma unroll
      for (int j = 0; j < JM; ++j) {
        const int c = lane + 64 * j;
        const bool ok = hh < H && c < C;
        q[h][j] = ok ? L.QT[i * L.ldq + hh * C + c] : 0.f;
        if (ok && sl == 0) sv.qt[size_t(r) * H * C + hh * C + c] = i < nrows ? q[h][j] : 0.f;
        acc[h][j] = 0.f;
      }
    }
    const size_t base = size_t(r) * K;
    // one chunk of nv <= kEC edges from window position e: the scores first
    // (independent reductions), then the online-softmax updates in edge order
    auto consume = [&](const float (&x)[kEC][JM], int e, int nv) {
      float sc[kEC][HL];
#pragma unroll
      for (int u = 0; u < kEC; ++u)
#pragma unroll
        for (int h = 0; h < HL; ++h) {
          float part = 0.f;
#pragma unroll
          for (int j = 0; j < JM; ++j) part += q[h][j] * x[u][j];
          sc[u][h] = u < nv ? wave_sum(part) + qbh[h] : 0.f;
        }
#pragma unroll
      for (int u = 0; u < kEC; ++u) {
        if (u >= nv) break;
        const size_t idx = base + e + u;
        sgl::U32x4 bits{};
        if constexpr (DROP)
          if (dc.p_att > 0.f) bits = sgl::drop_bits(dc, dstep, uint32_t(r), uint32_t(e + u), 0);
#pragma unroll
        for (int h = 0; h < HL; ++h) {
          const int hh = hg * HL + h;
          if (hh >= H) continue;
          const float sh = sc[u][h];
          const float a = sh > 0.f ? sh : 0.2f * sh;
          const float mn = fmaxf(m[h], a);
          const float scale = __expf(m[h] - mn);
          const float pe = __expf(a - mn);
          l[h] = l[h] * scale + pe;
          if constexpr (DROP) {
            // softmax over every edge (l), the kept weights rescaled (pk)
            const float pk = pe * sgl::drop_keep(bits.v[hh], dc.p_att, sa);
            ls[h] = ls[h] * scale + pk;
#pragma unroll
            for (int j = 0; j < JM; ++j) acc[h][j] = acc[h][j] * scale + pk * x[u][j];
          } else {
#pragma unroll
            for (int j = 0; j < JM; ++j) acc[h][j] = acc[h][j] * scale + pe * x[u][j];
          }
          m[h] = mn;
          if (lane == 0) sv.score[idx * H + hh] = a;
        }
      }
    };
    if (kPre) {
      // gathered columns from the rows, time encodings from LDS (staged) or
      // from the rows (written before the last barrier)
      for (int c0 = elo; c0 < ehi; c0 += kEC) {
        const int nv = min(kEC, ehi - c0);
        float x[kEC][JM];
#pragma unroll
        for (int u = 0; u < kEC; ++u) {
          const int e = c0 + min(u, nv - 1);
          const size_t row = base + e;
          if (staged) {
            const float *ts = L.Ts + (i * K + e) * T - (D + d.F);
#pragma unroll
            for (int j = 0; j < JM; ++j) {
              const int c = lane + 64 * j;
              x[u][j] = u < nv ? (c < D + d.F ? X[row * C + c] : c < C ? ts[c] : 0.f) : 0.f;
            }
          } else {
            load_row<JM>(d, X, row, lane, x[u]);
            if (u >= nv) {
#pragma unroll
              for (int j = 0; j < JM; ++j) x[u][j] = 0.f;
            }
          }
        }
        consume(x, c0, nv);
      }
    } else {
      for (int e0 = elo; e0 < ehi; e0 += 64) {
        const int wend = min(ehi, e0 + 64);
        const float my_dt = e0 + lane < wend ? dt[base + e0 + lane] : 0.f;
        for (int c0 = e0; c0 < wend; c0 += kEC) {
          const int nv = min(kEC, wend - c0);
          float x[kEC][JM];
#pragma unroll
          for (int u = 0; u < kEC; ++u) {
            if (u < nv) {
              fill_row<JM>(d, X, S, base + c0 + u, L.TW, L.TB, __shfl(my_dt, c0 + u - e0, 64), lane, x[u]);
            } else {
#pragma unroll
              for (int j = 0; j < JM; ++j) x[u][j] = 0.f;
            }
          }
          consume(x, c0, nv);
        }
      }
    }
    if constexpr (NS == 1) {
      // the wave owns its root's heads of group hg: xbar overwrites their qt
      // columns in the root's LDS row (only this wave reads them)
#pragma unroll
      for (int h = 0; h < HL; ++h) {
        const int hh = hg * HL + h;
        if (hh >= H) continue;
        const float inv = ne > 0 ? 1.f / l[h] : 0.f;
#pragma unroll
        for (int j = 0; j < JM; ++j) {
          const int c = lane + 64 * j;
          if (c < C) {
            const float v = acc[h][j] * inv;
            L.QT[i * L.ldq + hh * C + c] = v;
            sv.xbar[size_t(r) * H * C + hh * C + c] = v;
          }
        }
        if (lane == 0) {
          sv.ml[(size_t(r) * H + hh) * 2 + 0] = ne > 0 ? m[h] : 0.f;
          sv.ml[(size_t(r) * H + hh) * 2 + 1] = ne > 0 ? l[h] : 1.f;
          if (DROP) {
            const float sd = ne > 0 ? ls[h] * inv : 0.f;
            s_sd[i][hh] = sd;
            sv.sdrop[size_t(r) * H + hh] = sd;
          }
        }
      }
    } else {
      // publish this slice's state for the merge (an empty slice has
      // m = -inf, l = 0, acc = 0 and drops out with weight e^-inf = 0)
#pragma unroll
      for (int h = 0; h < HM; ++h) {
        if (h >= H) continue;
#pragma unroll
        for (int j = 0; j < JM; ++j) {
          const int c = lane + 64 * j;
          if (c < C) L.part[(wave * H + h) * C + c] = acc[h][j];
        }
        if (lane == 0) {
          L.pml[(wave * H + h) * 3 + 0] = m[h];
          L.pml[(wave * H + h) * 3 + 1] = l[h];
          L.pml[(wave * H + h) * 3 + 2] = ls[h];
        }
      }
    }
  }
  __syncthreads();
  if constexpr (NS > 1) {
    // merge the slices: M = max_s m_s, Lsum = sum_s l_s e^(m_s - M),
    // xbar = sum_s acc_s e^(m_s - M) / Lsum (the whole window's softmax)
    for (int idx = tid; idx < RPW * H * C; idx += kBlock) {
      const int i = idx / (H * C), hc = idx - i * (H * C), h = hc / C, c = hc - h * C;
      const int r = r0 + i;
      float v = 0.f, M = -INFINITY, Ls = 0.f, Lk = 0.f;
      if (s_cnt[i] > 0) {
#pragma unroll
        for (int s = 0; s < WPR; ++s) M = fmaxf(M, L.pml[((i * WPR + s) * H + h) * 3]);
#pragma unroll
        for (int s = 0; s < WPR; ++s) {
          const int w = i * WPR + s;
          const float f = __expf(L.pml[(w * H + h) * 3] - M);
          Ls += L.pml[(w * H + h) * 3 + 1] * f;
          if (DROP) Lk += L.pml[(w * H + h) * 3 + 2] * f;
          v += L.part[(w * H + h) * C + c] * f;
        }
        v /= Ls;
      }
      L.QT[i * L.ldq + hc] = v;
      sv.xbar[size_t(r) * H * C + hc] = v;
      if (c == 0) {
        sv.ml[(size_t(r) * H + h) * 2 + 0] = s_cnt[i] > 0 ? M : 0.f;
        sv.ml[(size_t(r) * H + h) * 2 + 1] = s_cnt[i] > 0 ? Ls : 1.f;
        if (DROP) {
          const float sd = s_cnt[i] > 0 ? Lk / Ls : 0.f;
          s_sd[i][h] = sd;
          sv.sdrop[size_t(r) * H + h] = sd;
        }
      }
    }
    __syncthreads();
  }
  // agg_h = W_v[h rows] xbar_h + b_v[h]  -> AH[:, :D]; with attention
  // dropout the kept weights sum to s_h, not 1: agg_h = W_v xbar'_h + s_h b_v[h]
  if constexpr (BF) {
    sgl::GemmJobBw jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.QT + h * C, L.ldq, bw.wv + size_t(h) * dh * bw.ld_c, bw.ld_c, p.b_v + h * dh, L.AH + h * dh,
                 L.lda, C, h < H ? dh : 0};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    sgl::GemmJob jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.QT + h * C, L.ldq, p.w_v + size_t(h) * dh * C, C, DROP ? nullptr : p.b_v + h * dh,
                 L.AH + h * dh, L.lda, C, h < H ? dh : 0};
    tile_products<sgl::kNT, RPW>(jobs, kWaves, L.scr);
  }
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    if (DROP && i < RPW && s_cnt[i] > 0) L.AH[i * L.lda + j] += s_sd[i][j / dh] * p.b_v[j];
    if (s_cnt[i] == 0) L.AH[i * L.lda + j] = 0.f;  // no in-edges: the sum aggregator gives 0
    if (i < RPW) sv.agg[size_t(r0 + i) * D + j] = L.AH[i * L.lda + j];
  }
  __syncthreads();
  // z = W_out [agg | h] + b_out
  if constexpr (BF) {
    const sgl::GemmJobBw jobs[1] = {{L.AH, L.lda, bw.wout, bw.ld_o, p.b_out, L.Zs, L.ldr, 2 * D, D}};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    const sgl::GemmJob jobs[1] = {{L.AH, L.lda, p.w_out, 2 * D, p.b_out, L.Zs, L.ldr, 2 * D, D}};
    tile_products<sgl::kNT, RPW>(jobs, kWaves, L.scr);
  }
  __syncthreads();
  // y = LayerNorm(ReLU(z)), eps 1e-5, biased variance; one wave per row;
  // with output dropout z is masked first (models.py:136: dropout, then
  // ReLU) and saved masked
  for (int i = wave; i < RPW; i += kWaves) {
    const size_t ro = size_t(r0 + i) * D;
    float s1 = 0.f;
    for (int j = lane; j < D; j += 64) {
      float zz = L.Zs[i * L.ldr + j];
      if (DROP && dc.p_out > 0.f) {
        zz *= sgl::drop_keep(sgl::drop_bits(dc, dstep, uint32_t(r0 + i), uint32_t(j >> 2), 1).v[j & 3],
                             dc.p_out, so);
        L.Zs[i * L.ldr + j] = zz;
      }
      sv.z[ro + j] = i < nrows ? zz : 0.f;
      s1 += fmaxf(zz, 0.f);
    }
    const float mean = wave_sum(s1) / D;
    float s2 = 0.f;
    for (int j = lane; j < D; j += 64) {
      const float dv = fmaxf(L.Zs[i * L.ldr + j], 0.f) - mean;
      s2 += dv * dv;
    }
    const float rstd = 1.f / sqrtf(wave_sum(s2) / D + 1e-5f);
    for (int j = lane; j < D; j += 64) {
      const float xh = (fmaxf(L.Zs[i * L.ldr + j], 0.f) - mean) * rstd;
      y[ro + j] = i < nrows ? xh * L.LG[j] + L.LB[j] : 0.f;
    }
    if (lane == 0) {
      sv.stats[size_t(r0 + i) * 2 + 0] = i < nrows ? mean : 0.f;
      sv.stats[size_t(r0 + i) * 2 + 1] = i < nrows ? rstd : 0.f;
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

struct BwdLds {
  int ldr, ldq;
  float *GZ, *GA, *GQ, *XH, *GY;  // [16][ldr]
  float *GX;                      // [16][ldq]  g_xbar, then G
  float *tep;                     // [waves][2][T]
  float *TB;                      // [T] time-encoding bias
  float *LG, *BK;                 // [D] LayerNorm weight, key bias (staged with the first loads)
  float *part;                    // [NW][H*C]  a slice's G partial (slices only)
  float *psig;                    // [NW][H]    a slice's sigma partial (slices only)
  float *scr;                     // [NW][4][64] four-row product partials (4-root tiles only)
};

__host__ __device__ inline BwdLds bwd_lds(const Dims &d, float *base, int nw, bool slices) {
  BwdLds L;
  L.ldr = sgl::lds_ld(d.D);
  L.ldq = sgl::lds_ld(d.H * d.C);
  L.GZ = base;
  L.GA = L.GZ + kRows * L.ldr;
  L.GQ = L.GA + kRows * L.ldr;
  L.XH = L.GQ + kRows * L.ldr;
  L.GY = L.XH + kRows * L.ldr;
  L.GX = L.GY + kRows * L.ldr;
  L.tep = L.GX + kRows * L.ldq;
  L.TB = L.tep + nw * 2 * d.T;
  L.LG = L.TB + d.T;
  L.BK = L.LG + d.D;
  L.part = L.BK + d.D;
  L.psig = L.part + (slices ? nw * d.H * d.C : 0);
  // 16-byte aligned for the product partials
  L.scr = L.psig + (((slices ? nw * d.H : 0) + 3) & ~3);
  return L;
}

inline size_t bwd_lds_floats(const Dims &d, int nw, int rows, bool slices) {
  float *base = reinterpret_cast<float *>(uintptr_t(4096));
  const BwdLds L = bwd_lds(d, base, nw, slices);
  return size_t(L.scr + (rows == 4 ? nw * 256 : 0) - base);
}

// The edge predictor's per-root gradient rows r0 .. r0+nrows-1 (fixed-point
// accumulators): returned as floats in g_src / g_dst and cleared for the
// next step (acc_dst may be NULL: one accumulator).
__device__ __forceinline__ void consume_rows(long long *__restrict__ acc_src, long long *__restrict__ acc_dst,
                                             float *__restrict__ g_src, float *__restrict__ g_dst, int r0,
                                             int nrows, int D, int tid, int nthreads) {
  for (int idx = tid; idx < nrows * D; idx += nthreads) {
    const size_t o = size_t(r0) * D + idx;
    g_src[o] = sgl::from_fixed(acc_src[o]);
    acc_src[o] = 0;
    if (acc_dst != nullptr) {
      g_dst[o] = sgl::from_fixed(acc_dst[o]);
      acc_dst[o] = 0;
    }
  }
}

// HG: head groups per root in the edge phase, as in k_conv_fwd.
template <int HM, int JM, bool DROP, bool BF = false, int NW = waves_for(HM, JM), int RPW = rows_for(NW), int HG = 1>
__global__ __launch_bounds__(NW * 64) void k_conv_bwd(
    Dims d, const int32_t *__restrict__ num_roots, const int32_t *__restrict__ any_edges,
    const int32_t *__restrict__ cnt, const float *__restrict__ X, const float *__restrict__ S,
    const float *__restrict__ dt, ConvParams p,
    ConvSaved sv, const float *__restrict__ gy, long long *__restrict__ acc_src,
    long long *__restrict__ acc_dst, const float *__restrict__ w_s, const float *__restrict__ w_d,
    float *__restrict__ g_src, float *__restrict__ g_dst, ConvGrads g, sgl::DropCfg dc, sgl_bf16_weights bw) {
  constexpr int kWaves = NW, kBlock = NW * 64;
  constexpr int WPR = NW / RPW;
  constexpr int NS = WPR / HG;  // window slices per root (summed through LDS when > 1)
  constexpr int HL = HM / HG;   // heads per wave in the edge phase
  constexpr int EC = HG > 1 ? 2 : kEC;  // edges per round trip (fewer under the 1024-thread register cap)
  static_assert(RPW <= kRows && NW % RPW == 0 && NW <= kMaxWaves, "tile shape");
  static_assert(WPR % HG == 0 && HM % HG == 0 && (HG == 1 || NS == 1), "head groups");
  static_assert(!(BF && DROP), "the bf16 products run without dropout");
  extern __shared__ __align__(16) float lds[];
  const int D = d.D, T = d.T, H = d.H, C = d.C, dh = d.dh, K = d.k;
  const BwdLds L = bwd_lds(d, lds, NW, NS > 1);
  __shared__ int s_cnt[kRows];
  __shared__ float s_sig[kRows][kMaxH];

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int U = *num_roots;
  const int r0 = blockIdx.x * RPW;
  const int nrows = max(0, min(RPW, U - r0));
  const bool live = *any_edges != 0;
  const unsigned long long dstep = DROP ? *dc.step : 0ull;
  const float sa = sgl::drop_scale(dc.p_att), so = sgl::drop_scale(dc.p_out);
  // row U of the accumulators (the non-root negatives; row capacity when
  // every row is a root) belongs to the workgroup whose tile holds it, or
  // to the last one; the rows past U are never written by the predictor
  if (gy == nullptr && ((U >= r0 && U < r0 + RPW) || (U == int(gridDim.x) * RPW && blockIdx.x == gridDim.x - 1)))
    consume_rows(acc_src, acc_dst, g_src, g_dst, U, 1, D, tid, kBlock);
  if (nrows == 0 || !live) {
    // rows outside the live set are never read; a block without edges has
    // zero gradients in its live rows
    if (gy == nullptr) consume_rows(acc_src, acc_dst, g_src, g_dst, r0, nrows, D, tid, kBlock);
    if (!live) {
      for (int idx = tid; idx < RPW * D; idx += kBlock) {
        const size_t o = size_t(r0) * D + idx;
        g.gz[o] = 0.f; g.gagg[o] = 0.f; g.gQ[o] = 0.f;
      }
      for (int idx = tid; idx < RPW * H * C; idx += kBlock) g.G[size_t(r0) * H * C + idx] = 0.f;
      for (int idx = tid; idx < RPW * H; idx += kBlock) g.sigma[size_t(r0) * H + idx] = 0.f;
    }
    // rows past the live set: zero gradient rows (the weight reductions of
    // dropout passes stop at U, but their products never read stale rows)
    for (int idx = tid; idx < 2 * D; idx += kBlock) g.ln_part[size_t(blockIdx.x) * 2 * D + idx] = 0.f;
    for (int idx = tid; idx < 2 * T; idx += kBlock) g.te_part[size_t(blockIdx.x) * 2 * T + idx] = 0.f;
    return;
  }
  if (tid < kRows) s_cnt[tid] = tid < nrows ? cnt[r0 + tid] : 0;
  for (int t = tid; t < T; t += kBlock) L.TB[t] = p.te_b[t];
  for (int j = tid; j < D; j += kBlock) {
    L.LG[j] = p.ln_g[j];
    L.BK[j] = p.b_k[j];
  }
  // dL/dy of the tile: given, or W_s^T g_src + W_d^T g_dst from the edge
  // predictor's per-root rows (GA / GQ are free until later phases)
  // (the two products land in GY and XH in parallel; the LayerNorm pass
  // adds them)
  if (gy != nullptr) {
    for (int idx = tid; idx < kRows * D; idx += kBlock) {
      const int i = idx / D, j = idx - i * D;
      L.GY[i * L.ldr + j] = i < nrows ? gy[size_t(r0 + i) * D + j] : 0.f;
      L.XH[i * L.ldr + j] = 0.f;
    }
    __syncthreads();
  } else {
    const bool two = acc_dst != nullptr;  // one accumulator: the pass of a dropout step
    for (int idx = tid; idx < kRows * D; idx += kBlock) {
      const int i = idx / D, j = idx - i * D;
      float vs = 0.f, vd = 0.f;
      if (i < nrows) {  // the tile's live rows (row U is consumed above)
        const size_t o = size_t(r0 + i) * D + j;
        vs = sgl::from_fixed(acc_src[o]);
        acc_src[o] = 0;
        g_src[o] = vs;
        if (two) {
          vd = sgl::from_fixed(acc_dst[o]);
          acc_dst[o] = 0;
          g_dst[o] = vd;
        }
      }
      L.GA[i * L.ldr + j] = vs;
      L.GQ[i * L.ldr + j] = vd;
      if (!two) L.XH[i * L.ldr + j] = 0.f;
    }
    __syncthreads();
    if constexpr (BF) {
      const sgl::GemmJobBw jobs[2] = {{L.GA, L.ldr, bw.wst, bw.ld_d, nullptr, L.GY, L.ldr, D, D},
                                      {L.GQ, L.ldr, bw.wdt, bw.ld_d, nullptr, L.XH, L.ldr, D, two ? D : 0}};
      sgl::tile_gemm16_bw_jobs(jobs, kWaves);
    } else {
      const sgl::GemmJob jobs[2] = {{L.GA, L.ldr, w_s, D, nullptr, L.GY, L.ldr, D, D},
                                    {L.GQ, L.ldr, two ? w_d : w_s, D, nullptr, L.XH, L.ldr, D, two ? D : 0}};
      tile_products<sgl::kNN, RPW>(jobs, kWaves, L.scr);
    }
    __syncthreads();
  }
  // LayerNorm + ReLU backward; one wave per row (rows past the tile zeroed)
  for (int i = wave; i < kRows; i += kWaves) {
    const size_t ro = size_t(r0 + i) * D;
    if (i >= nrows) {
      for (int j = lane; j < D; j += 64) {
        L.GZ[i * L.ldr + j] = 0.f;
        L.XH[i * L.ldr + j] = 0.f;
        L.GY[i * L.ldr + j] = 0.f;
      }
    } else {
      const float mean = sv.stats[size_t(r0 + i) * 2], rstd = sv.stats[size_t(r0 + i) * 2 + 1];
      float a1 = 0.f, a2 = 0.f;
      for (int j = lane; j < D; j += 64) {
        const float zz = sv.z[ro + j], gv = L.GY[i * L.ldr + j] + L.XH[i * L.ldr + j];
        const float xh = (fmaxf(zz, 0.f) - mean) * rstd;
        const float gxh = gv * L.LG[j];
        L.GY[i * L.ldr + j] = gv;
        L.XH[i * L.ldr + j] = xh;
        L.GZ[i * L.ldr + j] = zz;
        a1 += gxh;
        a2 += gxh * xh;
      }
      a1 = wave_sum(a1) / D;
      a2 = wave_sum(a2) / D;
      for (int j = lane; j < D; j += 64) {
        const float zz = L.GZ[i * L.ldr + j];
        const float xh = L.XH[i * L.ldr + j];
        const float gx = rstd * (L.GY[i * L.ldr + j] * L.LG[j] - a1 - xh * a2);
        float gzv = zz > 0.f ? gx : 0.f;
        if (DROP && dc.p_out > 0.f)  // through the output mask (z was saved masked)
          gzv *= sgl::drop_keep(sgl::drop_bits(dc, dstep, uint32_t(r0 + i), uint32_t(j >> 2), 1).v[j & 3],
                                dc.p_out, so);
        L.GZ[i * L.ldr + j] = gzv;
      }
    }
  }
  __syncthreads();
  // per-tile LayerNorm parameter grads; gz out
  for (int j = tid; j < D; j += kBlock) {
    float sg = 0.f, sb = 0.f;
#pragma unroll
    for (int i = 0; i < RPW; ++i) {
      sg += L.GY[i * L.ldr + j] * L.XH[i * L.ldr + j];
      sb += L.GY[i * L.ldr + j];
    }
    g.ln_part[size_t(blockIdx.x) * 2 * D + j] = sg;
    g.ln_part[size_t(blockIdx.x) * 2 * D + D + j] = sb;
  }
  for (int idx = tid; idx < RPW * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    g.gz[size_t(r0 + i) * D + j] = L.GZ[i * L.ldr + j];
  }
  // g_agg = gz W_out[:, :D]
  if constexpr (BF) {
    const sgl::GemmJobBw jobs[1] = {{L.GZ, L.ldr, bw.wot, bw.ld_d, nullptr, L.GA, L.ldr, D, D}};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    const sgl::GemmJob jobs[1] = {{L.GZ, L.ldr, p.w_out, 2 * D, nullptr, L.GA, L.ldr, D, D}};
    tile_products<sgl::kNN, RPW>(jobs, kWaves, L.scr);
  }
  __syncthreads();
  for (int idx = tid; idx < kRows * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    if (s_cnt[i] == 0) L.GA[i * L.ldr + j] = 0.f;  // agg was the constant 0
    if (i < RPW) g.gagg[size_t(r0 + i) * D + j] = L.GA[i * L.ldr + j];
  }
  __syncthreads();
  // g_xbar_h = g_agg_h W_v[h rows, :]
  if constexpr (BF) {
    sgl::GemmJobBw jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.GA + h * dh, L.ldr, bw.wvt + h * bw.hp, bw.ld_h, nullptr, L.GX + h * C, L.ldq, dh,
                 h < H ? C : 0};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    sgl::GemmJob jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.GA + h * dh, L.ldr, p.w_v + size_t(h) * dh * C, C, nullptr, L.GX + h * C, L.ldq, dh,
                 h < H ? C : 0};
    tile_products<sgl::kNN, RPW>(jobs, kWaves, L.scr);
  }
  __syncthreads();

  // edge backward phase: wave w takes window slice sl of root w / WPR's
  // window for the heads of its head group hg (sub = w % WPR = hg * NS + sl)
  float twp[JM], tbp[JM];  // this lane's time-encoding weight / bias partials
#pragma unroll
  for (int j = 0; j < JM; ++j) { twp[j] = 0.f; tbp[j] = 0.f; }
  {
    const int i = wave / WPR, sub = wave % WPR;
    const int hg = sub / NS, sl = sub - hg * NS;
    const int r = r0 + i;
    const int ne = s_cnt[i];
    int elo, ehi;
    window_slice(ne, sl, NS, elo, ehi);
    float q[HL][JM], gx[HL][JM], G[HL][JM];
    float dot[HL], sig[HL], mh[HL], lh[HL], cb[HL];
#pragma unroll
    for (int h = 0; h < HL; ++h) {
      const int hh = hg * HL + h;
      float pd = 0.f;
#pragma unroll
      for (int j = 0; j < JM; ++j) {
        const int c = lane + 64 * j;
        const bool ok = hh < H && c < C;
        q[h][j] = ok ? sv.qt[size_t(r) * H * C + hh * C + c] : 0.f;
        const float xb = ok ? sv.xbar[size_t(r) * H * C + hh * C + c] : 0.f;
        gx[h][j] = ok ? L.GX[i * L.ldq + hh * C + c] : 0.f;
        G[h][j] = 0.f;
        pd += gx[h][j] * xb;
      }
      dot[h] = wave_sum(pd);
      cb[h] = 0.f;
      if constexpr (DROP) {
        // with attention dropout the weights no longer sum to 1, so the
        // value bias stays in: dL/dalpha'_e = <g_xbar_h, X_e> + c_h with
        // c_h = <g_agg_h, b_v[h]>, and sum_e alpha_e dL/dalpha_e = dot + c_h s_h
        if (hh < H) {
          float pc = 0.f;
          for (int j = lane; j < dh; j += 64) pc += L.GA[i * L.ldr + hh * dh + j] * p.b_v[hh * dh + j];
          cb[h] = wave_sum(pc);
          dot[h] += cb[h] * sv.sdrop[size_t(r) * H + hh];
        }
      }
      sig[h] = 0.f;
      mh[h] = hh < H ? sv.ml[(size_t(r) * H + hh) * 2] : 0.f;
      lh[h] = hh < H ? sv.ml[(size_t(r) * H + hh) * 2 + 1] : 1.f;
    }
    const size_t base = size_t(r) * K;
    for (int e0 = elo; e0 < ehi; e0 += 64) {
      const int mwin = min(64, ehi - e0);
      float my_dt = 0.f, my_sc[HL];
#pragma unroll
      for (int h = 0; h < HL; ++h) my_sc[h] = 0.f;
      if (lane < mwin) {
        my_dt = dt[base + e0 + lane];
#pragma unroll
        for (int h = 0; h < HL; ++h)
          if (hg * HL + h < H) my_sc[h] = sv.score[(base + e0 + lane) * H + hg * HL + h];
      }
      for (int c0 = 0; c0 < mwin; c0 += EC) {
        float x[EC][JM], sn[EC][JM];
#pragma unroll
        for (int u = 0; u < EC; ++u) {
          const size_t row = base + e0 + min(c0 + u, mwin - 1);
          load_row<JM>(d, X, row, lane, x[u]);
#pragma unroll
          for (int j = 0; j < JM; ++j) {
            const int t = lane + 64 * j - d.D - d.F;
            sn[u][j] = t >= 0 && t < d.T ? S[row * d.T + t] : 0.f;
          }
        }
        float tg[EC][HL];  // <g_xbar_h, X_e> for the chunk's edges
#pragma unroll
        for (int u = 0; u < EC; ++u)
#pragma unroll
          for (int h = 0; h < HL; ++h) {
            float part = 0.f;
#pragma unroll
            for (int j = 0; j < JM; ++j) part += gx[h][j] * x[u][j];
            tg[u][h] = wave_sum(part);
          }
#pragma unroll
        for (int u = 0; u < EC; ++u) {
          if (c0 + u >= mwin) break;
          const int e = c0 + u;
          const float dtv = __shfl(my_dt, e, 64);
          float gsv[HL], al[HL];
          sgl::U32x4 bits{};
          if constexpr (DROP)
            if (dc.p_att > 0.f) bits = sgl::drop_bits(dc, dstep, uint32_t(r), uint32_t(e0 + e), 0);
#pragma unroll
          for (int h = 0; h < HL; ++h) {
            const int hh = hg * HL + h;
            gsv[h] = 0.f;
            al[h] = 0.f;
            if (hh >= H) continue;
            const float t = tg[u][h];
            const float a = __shfl(my_sc[h], e, 64);
            const float alpha = __expf(a - mh[h]) / lh[h];
            float ga, aw = alpha;
            if constexpr (DROP) {
              const float mk = sgl::drop_keep(bits.v[hh], dc.p_att, sa);
              ga = alpha * (mk * (t + cb[h]) - dot[h]);  // softmax backward through the mask
              aw = alpha * mk;                           // the edge's weight in xbar'
            } else {
              ga = alpha * (t - dot[h]);  // softmax backward
            }
            const float gs = ga * (a > 0.f ? 1.f : 0.2f);
            gsv[h] = gs;
            al[h] = aw;
            sig[h] += gs;
#pragma unroll
            for (int j = 0; j < JM; ++j) G[h][j] += gs * x[u][j];
          }
          // time-encoding gradients for this edge's T columns
#pragma unroll
          for (int j = 0; j < JM; ++j) {
            const int c = lane + 64 * j;
            if (c >= D + d.F && c < C) {
              float gphi = 0.f;  // this wave's heads (the waves' partials are summed below)
#pragma unroll
              for (int h = 0; h < HL; ++h)
                if (hg * HL + h < H) gphi += gsv[h] * q[h][j] + al[h] * gx[h][j];
              const float ds = -sn[u][j] * gphi;
              twp[j] += ds * dtv;
              tbp[j] += ds;
            }
          }
        }
      }
    }
    if constexpr (NS == 1) {
      // the wave owns its root's heads of group hg: G overwrites their
      // g_xbar columns in the root's LDS row (only this wave reads them)
#pragma unroll
      for (int h = 0; h < HL; ++h) {
        const int hh = hg * HL + h;
        if (hh >= H) continue;
#pragma unroll
        for (int j = 0; j < JM; ++j) {
          const int c = lane + 64 * j;
          if (c < C) {
            L.GX[i * L.ldq + hh * C + c] = G[h][j];
            g.G[size_t(r) * H * C + hh * C + c] = G[h][j];
          }
        }
        if (lane == 0) {
          g.sigma[size_t(r) * H + hh] = sig[h];
          s_sig[i][hh] = sig[h];
        }
      }
    } else {  // one head group (HL == HM): the slice's partials of every head
#pragma unroll
      for (int h = 0; h < HL; ++h) {
        if (h >= H) continue;
#pragma unroll
        for (int j = 0; j < JM; ++j) {
          const int c = lane + 64 * j;
          if (c < C) L.part[(wave * H + h) * C + c] = G[h][j];
        }
        if (lane == 0) L.psig[wave * H + h] = sig[h];
      }
    }
  }
  // the waves' time-encoding partials (reduced at the end)
#pragma unroll
  for (int j = 0; j < JM; ++j) {
    const int c = lane + 64 * j;
    if (c >= D + d.F && c < C) {
      const int t = c - D - d.F;
      L.tep[(wave * 2 + 0) * T + t] = twp[j];
      L.tep[(wave * 2 + 1) * T + t] = tbp[j];
    }
  }
  __syncthreads();
  if constexpr (NS > 1) {
    // sum the slices' partials into the root's row (every read of g_xbar is
    // behind the barrier above)
    for (int idx = tid; idx < RPW * H * C; idx += kBlock) {
      const int i = idx / (H * C), hc = idx - i * (H * C), h = hc / C, c = hc - h * C;
      float v = 0.f;
#pragma unroll
      for (int s = 0; s < WPR; ++s) v += L.part[((i * WPR + s) * H + h) * C + c];
      L.GX[i * L.ldq + hc] = v;
      g.G[size_t(r0 + i) * H * C + hc] = v;
    }
    for (int idx = tid; idx < RPW * H; idx += kBlock) {
      const int i = idx / H, h = idx - (idx / H) * H;
      float v = 0.f;
#pragma unroll
      for (int s = 0; s < WPR; ++s) v += L.psig[(i * WPR + s) * H + h];
      g.sigma[size_t(r0 + i) * H + h] = v;
      s_sig[i][h] = v;
    }
    __syncthreads();
  }
  // gQ_h = W_k[h rows] G_h + b_k[h] sigma_h
  if constexpr (BF) {
    sgl::GemmJobBw jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.GX + h * C, L.ldq, bw.wk + size_t(h) * dh * bw.ld_c, bw.ld_c, nullptr, L.GQ + h * dh, L.ldr, C,
                 h < H ? dh : 0};
    sgl::tile_gemm16_bw_jobs(jobs, kWaves);
  } else {
    sgl::GemmJob jobs[HM];
#pragma unroll
    for (int h = 0; h < HM; ++h)
      jobs[h] = {L.GX + h * C, L.ldq, p.w_k + size_t(h) * dh * C, C, nullptr, L.GQ + h * dh, L.ldr, C,
                 h < H ? dh : 0};
    tile_products<sgl::kNT, RPW>(jobs, kWaves, L.scr);
  }
  __syncthreads();
  for (int idx = tid; idx < RPW * D; idx += kBlock) {
    const int i = idx / D, j = idx - i * D;
    const int h = j / dh;
    const float v = i < nrows ? L.GQ[i * L.ldr + j] + L.BK[j] * s_sig[i][h] : 0.f;
    L.GQ[i * L.ldr + j] = v;
    g.gQ[size_t(r0 + i) * D + j] = v;
  }
  __syncthreads();
  // column sums of this tile's gQ (GA row 0 is free by now)
  for (int j = tid; j < D; j += kBlock) {
    float sq = 0.f;
#pragma unroll
    for (int i = 0; i < RPW; ++i) sq += L.GQ[i * L.ldr + j];
    L.GA[j] = sq;
  }
  __syncthreads();
  // the query's cos(b) term of the time-encoding bias gradient,
  // -sin(b_t) * sum_j W_q[j][D+t] * colsum[j]: the j range split over the
  // waves, partial sums in GX (free by now), added in wave order
  // (the weights of a batch of kQJ rows and two t columns are loaded
  // together: one memory round trip per batch)
  {
    constexpr int kQJ = 12;
    const int per = (D + kWaves - 1) / kWaves;
    const int j0 = wave * per, j1 = min(D, j0 + per);
    for (int t0 = lane; t0 < T; t0 += 128) {
      const int t1 = t0 + 64;
      float acc0 = 0.f, acc1 = 0.f;
      for (int jb = j0; jb < j1; jb += kQJ) {
        float w0[kQJ], w1[kQJ];
#pragma unroll
        for (int u = 0; u < kQJ; ++u) {
          const size_t row = size_t(min(jb + u, j1 - 1)) * (D + T) + D;
          w0[u] = p.w_q[row + t0];
          w1[u] = t1 < T ? p.w_q[row + t1] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kQJ; ++u) {
          if (jb + u >= j1) break;
          acc0 += w0[u] * L.GA[jb + u];
          acc1 += w1[u] * L.GA[jb + u];
        }
      }
      L.GX[wave * T + t0] = acc0;
      if (t1 < T) L.GX[wave * T + t1] = acc1;
    }
  }
  __syncthreads();
  // per-tile time-encoding gradients: the edges' terms and the query's term
  for (int t = tid; t < T; t += kBlock) {
    float a = 0.f, b = 0.f, qterm = 0.f;
    for (int w = 0; w < kWaves; ++w) {
      a += L.tep[(w * 2) * T + t];
      b += L.tep[(w * 2 + 1) * T + t];
      qterm += L.GX[w * T + t];
    }
    b += -sinf(L.TB[t]) * qterm;
    g.te_part[size_t(blockIdx.x) * 2 * T + t] = a;
    g.te_part[size_t(blockIdx.x) * 2 * T + T + t] = b;
  }
}

int check_dims(const Dims &d) {
  SGL_REQUIRE(d.D > 0 && d.H > 0 && d.H <= kMaxH && d.D % d.H == 0, "conv: need 0 < H <= %d and D %% H == 0 (D=%d H=%d)",
              kMaxH, d.D, d.H);
  SGL_REQUIRE(d.F >= 0 && d.T >= 0 && d.C <= 64 * kMaxJ, "conv: C = D+F+T = %d exceeds %d", d.C, 64 * kMaxJ);
  SGL_REQUIRE(d.k >= 0 && d.k <= 4096, "conv: fanout %d out of range", d.k);
  return SGL_OK;
}

// Kernel instance for (H, C): register arrays sized to the next supported
// head count (1, 2, 4) and column-slot count (2, 4, 6, 8 slots of 64).
template <typename Fn>
struct Instance {
  Fn fn;
  int waves;
  int rows;    // roots per workgroup
  int hg = 1;  // head groups per root in the edge phase
};

inline void instance_shape(const Dims &d, int &hm, int &jm) {
  const int j = (d.C + 63) / 64;
  jm = j <= 2 ? 2 : j <= 4 ? 4 : j <= 6 ? 6 : 8;
  hm = d.H <= 1 ? 1 : d.H <= 2 ? 2 : 4;
}

template <template <int, int> class Pick>
auto pick_instance(const Dims &d) -> decltype(Pick<1, 2>::get()) {
  int hm, jm;
  instance_shape(d, hm, jm);
#define SGL_PICK(HH, JJ) \
  if (hm == HH && jm == JJ) return Pick<HH, JJ>::get();
  SGL_PICK(1, 2) SGL_PICK(1, 4) SGL_PICK(1, 6) SGL_PICK(1, 8)
  SGL_PICK(2, 2) SGL_PICK(2, 4) SGL_PICK(2, 6) SGL_PICK(2, 8)
  SGL_PICK(4, 2) SGL_PICK(4, 4) SGL_PICK(4, 6) SGL_PICK(4, 8)
#undef SGL_PICK
  return {nullptr, 0, 0};
}

using FwdFn = decltype(&k_conv_fwd<1, 2, false>);
using BwdFn = decltype(&k_conv_bwd<1, 2, false>);
// bf16 instances whose whole-head arrays need the 8-wave instances'
// registers split each root's heads over two waves of a 16-wave workgroup,
// keeping the 8 roots per workgroup of the 8-wave shape.
// The fp32 products' registers do not leave room for it; the backward's
// widest shape (4 heads, 8 column blocks) would spill over 200 bytes a lane
// under the 16-wave register cap and keeps the 8-wave instance.
constexpr bool split_heads(int hm, int jm) { return waves_for(hm, jm) == 8 && hm >= 2; }
constexpr bool split_heads_bwd(int hm, int jm) { return split_heads(hm, jm) && hm * jm <= 24; }
// fp32 and dropout instances: FwdPick / BwdPick (/ ...Drop) with kFp32Rows
// roots, the ...Wide twins with the wave count's own rows (rows_for), taken
// where fp32_four_fits says the 4-root layouts do not fit.
template <int HM, int JM>
struct FwdPick {
  static Instance<FwdFn> get() {
    return {&k_conv_fwd<HM, JM, false, false, waves_for(HM, JM), kFp32Rows>, waves_for(HM, JM), kFp32Rows};
  }
};
template <int HM, int JM>
struct BwdPick {
  static Instance<BwdFn> get() {
    return {&k_conv_bwd<HM, JM, false, false, waves_for(HM, JM), kFp32Rows>, waves_for(HM, JM), kFp32Rows};
  }
};
template <int HM, int JM>
struct FwdPickWide {
  static Instance<FwdFn> get() { return {&k_conv_fwd<HM, JM, false>, waves_for(HM, JM), rows_for(waves_for(HM, JM))}; }
};
template <int HM, int JM>
struct BwdPickWide {
  static Instance<BwdFn> get() { return {&k_conv_bwd<HM, JM, false>, waves_for(HM, JM), rows_for(waves_for(HM, JM))}; }
};
// the bf16-product instances (no dropout). The 16-wave forward takes one
// root per workgroup (its 16 waves split the root's window): the products'
// 16-row tiles cost the same for 1 root as for 4, and the per-root phases
// (time encodings, edge windows, LayerNorm) shrink with the roots a
// workgroup holds (config 4: 22.4 -> 20.2 us; 2 roots: 20.9). The forward
// writes no per-tile partials, so its rows need not match the backward's.
template <int HM, int JM>
struct FwdPickBf {
  static Instance<FwdFn> get() {
    if constexpr (split_heads(HM, JM)) return {&k_conv_fwd<HM, JM, false, true, 16, 8, 2>, 16, 8, 2};
    else if constexpr (waves_for(HM, JM) == 16) return {&k_conv_fwd<HM, JM, false, true, 16, 1, 1>, 16, 1};
    else return {&k_conv_fwd<HM, JM, false, true>, waves_for(HM, JM), rows_for(waves_for(HM, JM))};
  }
};
template <int HM, int JM>
struct BwdPickBf {
  // the backward's ln_part / te_part tiles are sized by the rows per
  // workgroup of the instance it runs (sgl_conv_backward_tile_rows, which
  // asks this picker). The 16-wave instance takes one root per workgroup, as
  // the forward does (config 4: 22.0 -> 20.9 us); the fp32 and dropout
  // instances keep 4 (their four-row products; one root would make config 4
  // with dropout 30 % slower).
  static_assert(!split_heads_bwd(HM, JM) || rows_for(waves_for(HM, JM)) == 8,
                "a split-head backward instance keeps the 8 rows of its 8-wave shape");
  static Instance<BwdFn> get() {
    if constexpr (split_heads_bwd(HM, JM)) return {&k_conv_bwd<HM, JM, false, true, 16, 8, 2>, 16, 8, 2};
    else if constexpr (waves_for(HM, JM) == 16) return {&k_conv_bwd<HM, JM, false, true, 16, 1, 1>, 16, 1};
    else return {&k_conv_bwd<HM, JM, false, true>, waves_for(HM, JM), rows_for(waves_for(HM, JM))};
  }
};
// the dropout instances (masks, kept-weight sums)
template <int HM, int JM>
struct FwdPickDrop {
  static Instance<FwdFn> get() {
    return {&k_conv_fwd<HM, JM, true, false, waves_for(HM, JM), kFp32Rows>, waves_for(HM, JM), kFp32Rows};
  }
};
template <int HM, int JM>
struct BwdPickDrop {
  static Instance<BwdFn> get() {
    return {&k_conv_bwd<HM, JM, true, false, waves_for(HM, JM), kFp32Rows>, waves_for(HM, JM), kFp32Rows};
  }
};
template <int HM, int JM>
struct FwdPickDropWide {
  static Instance<FwdFn> get() { return {&k_conv_fwd<HM, JM, true>, waves_for(HM, JM), rows_for(waves_for(HM, JM))}; }
};
template <int HM, int JM>
struct BwdPickDropWide {
  static Instance<BwdFn> get() { return {&k_conv_bwd<HM, JM, true>, waves_for(HM, JM), rows_for(waves_for(HM, JM))}; }
};

// Whether the fp32 / dropout instances of these dimensions take kFp32Rows
// roots: always with 16 waves (their own rows), with 8 waves when the
// forward's (time encodings not staged) and the backward's 4-root layouts,
// two waves a root, fit in the CU's LDS. A function of (D, F, T, H) alone, so
// the forward, the backward and sgl_conv_backward_tile_rows agree.
bool fp32_four_fits(const Dims &d, int nw) {
  if (nw == 16) return true;
  const bool slices = nw / kFp32Rows > 1;
  return sizeof(float) * fwd_lds_floats(d, nw, kFp32Rows, slices, 0) <= 160 * 1024 &&
         sizeof(float) * bwd_lds_floats(d, nw, kFp32Rows, slices) <= 160 * 1024;
}
template <class Fn>
Instance<Fn> fp32_or_wide(const Dims &d, Instance<Fn> four, Instance<Fn> (*wide)(const Dims &)) {
  return four.fn == nullptr || fp32_four_fits(d, four.waves) ? four : wide(d);
}

// The bf16 weight copies' shapes (sgl_bf16_weights): every pointer set,
// leading dimensions multiples of 8 and wide enough, rows 16-byte aligned.
int check_bf16_weights(const Dims &d, const sgl_bf16_weights &w, bool drop) {
  SGL_REQUIRE(!drop, "conv: the bf16 products run without dropout");
  SGL_REQUIRE(w.wq && w.wk && w.wv && w.wout && w.wkt && w.wvt && w.wot && w.ws && w.wd && w.wst && w.wdt,
              "conv: NULL bf16 weight copy");
  const uint16_t *ptrs[] = {w.wq, w.wk, w.wv, w.wout, w.wkt, w.wvt, w.wot, w.ws, w.wd, w.wst, w.wdt};
  for (const uint16_t *q : ptrs)
    SGL_REQUIRE((reinterpret_cast<uintptr_t>(q) & 15u) == 0, "conv: bf16 weight copy not 16-byte aligned");
  const int32_t lds[] = {w.ld_q, w.ld_c, w.ld_o, w.ld_h, w.hp, w.ld_d};
  for (int32_t v : lds) SGL_REQUIRE(v > 0 && v % 8 == 0, "conv: bf16 leading dimension %d not a positive multiple of 8", v);
  SGL_REQUIRE(w.ld_q >= d.D + d.T && w.ld_c >= d.C && w.ld_o >= 2 * d.D && w.hp >= d.dh && w.ld_h >= d.H * w.hp &&
                  w.ld_d >= d.D,
              "conv: bf16 weight copies narrower than the dimensions");
  return SGL_OK;
}

int drop_cfg(float p_att, float p_out, uint64_t seed, const uint64_t *rng_step, int32_t pass, const float *sdrop,
             sgl::DropCfg &dc, bool &drop) {
  SGL_REQUIRE(p_att >= 0.f && p_att < 1.f && p_out >= 0.f && p_out < 1.f,
              "conv: dropout probabilities must lie in [0, 1) (att %g, out %g)", p_att, p_out);
  drop = p_att > 0.f || p_out > 0.f;
  SGL_REQUIRE(!drop || (rng_step != nullptr && (p_att == 0.f || sdrop != nullptr)),
              "conv: dropout needs the step counter and (attention dropout) the kept-weight sums");
  SGL_REQUIRE(pass >= 0 && pass < (1 << 20), "conv: pass %d out of range", pass);
  dc = sgl::DropCfg{p_att, p_out, uint32_t(seed), uint32_t(seed >> 32),
                    reinterpret_cast<const unsigned long long *>(rng_step), pass};
  return SGL_OK;
}

}  // namespace

namespace {

__global__ __launch_bounds__(256) void k_dropout_masks(sgl::DropCfg dc, int64_t rows, int fanout, int H, int D,
                                                       float *__restrict__ att, float *__restrict__ out) {
  const unsigned long long step = *dc.step;
  const float sa = sgl::drop_scale(dc.p_att), so = sgl::drop_scale(dc.p_out);
  const int64_t na = att != nullptr ? rows * fanout : 0, no = out != nullptr ? rows * ((D + 3) / 4) : 0;
  for (int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x; i < na + no; i += int64_t(gridDim.x) * 256) {
    if (i < na) {
      const int64_t r = i / fanout;
      const int e = int(i - r * fanout);
      const sgl::U32x4 b = sgl::drop_bits(dc, step, uint32_t(r), uint32_t(e), 0);
      for (int h = 0; h < H; ++h) att[i * H + h] = sgl::drop_keep(b.v[h], dc.p_att, sa);
    } else {
      const int64_t k = i - na, g4 = (D + 3) / 4;
      const int64_t r = k / g4;
      const int c4 = int(k - r * g4);
      const sgl::U32x4 b = sgl::drop_bits(dc, step, uint32_t(r), uint32_t(c4), 1);
      for (int q = 0; q < 4 && 4 * c4 + q < D; ++q) out[r * D + 4 * c4 + q] = sgl::drop_keep(b.v[q], dc.p_out, so);
    }
  }
}

}  // namespace

extern "C" int sgl_dropout_masks(int64_t rows, int32_t fanout, int32_t H, int32_t D, float p_att, float p_out,
                                 uint64_t seed, const uint64_t *rng_step, int32_t pass, float *att_mask,
                                 float *out_mask, hipStream_t stream) {
  SGL_REQUIRE(rows >= 0 && rows < INT_MAX && fanout >= 0 && fanout <= 4096 && H > 0 && H <= kMaxH && D > 0,
              "dropout_masks: bad sizes");
  SGL_REQUIRE(rng_step != nullptr, "dropout_masks: NULL step counter");
  sgl::DropCfg dc;
  bool drop;
  if (int rc = drop_cfg(p_att, p_out, seed, rng_step, pass, reinterpret_cast<const float *>(rng_step), dc, drop))
    return rc;
  const int64_t n = (att_mask ? rows * fanout : 0) + (out_mask ? rows * ((D + 3) / 4) : 0);
  if (n == 0) return SGL_OK;
  const unsigned grid = unsigned(std::min<int64_t>((n + 255) / 256, sgl::kMaxGrid));
  k_dropout_masks<<<grid, 256, 0, stream>>>(dc, rows, fanout, H, D, att_mask, out_mask);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int32_t sgl_conv_tile_rows(int32_t D, int32_t F, int32_t T, int32_t H) {
  const Dims d{D, F, T, H, D + F + T, H > 0 ? D / H : 0, 0};
  if (check_dims(d) != SGL_OK) return 0;
  const auto inst = fp32_or_wide(d, pick_instance<BwdPick>(d), &pick_instance<BwdPickWide>);
  return inst.fn != nullptr ? inst.rows : 0;
}

extern "C" int32_t sgl_conv_backward_tile_rows(int32_t D, int32_t F, int32_t T, int32_t H, int32_t bf16) {
  const Dims d{D, F, T, H, D + F + T, H > 0 ? D / H : 0, 0};
  if (check_dims(d) != SGL_OK) return 0;
  const auto inst = bf16 ? pick_instance<BwdPickBf>(d)
                         : fp32_or_wide(d, pick_instance<BwdPick>(d), &pick_instance<BwdPickWide>);
  return inst.fn != nullptr ? inst.rows : 0;
}

extern "C" int sgl_edge_rows(int32_t D, int32_t F, int32_t T, int32_t fanout, int64_t capacity,
                             const int32_t *num_roots, const float *memory, const float *efeat, const int32_t *cnt,
                             const int32_t *nbr, const int32_t *eid, float *X, hipStream_t stream) {
  const Dims d{D, F, T, 1, D + F + T, D, fanout};
  SGL_REQUIRE(D > 0 && F >= 0 && T >= 0 && d.C <= 64 * kMaxJ, "edge_rows: C = D+F+T = %d out of (0, %d]", d.C,
              64 * kMaxJ);
  SGL_REQUIRE(fanout >= 0 && fanout <= 4096, "edge_rows: fanout %d out of range", fanout);
  SGL_REQUIRE(capacity >= 0 && capacity < INT_MAX, "edge_rows: capacity %lld out of range", (long long)capacity);
  const int64_t rows = capacity * fanout;
  if (rows == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && memory && cnt && nbr && eid && X && (F == 0 || efeat), "edge_rows: NULL array");
  const auto a16 = [](const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; };
  const bool v4 = D % 4 == 0 && F % 4 == 0 && d.C % 4 == 0 && a16(memory) && a16(X) && (F == 0 || a16(efeat));
  const unsigned grid = unsigned(std::min<int64_t>((capacity + kEdgeWaves - 1) / kEdgeWaves, sgl::kMaxGrid));
  const int wv = (D + F) / 4;  // vectors per row of the V = 4 kernels (C <= 512: at most 128)
  const bool group = capacity > sgl::kMaxGrid * kEdgeWaves;  // more roots than one pass of the grid
  auto kern = group ? &k_edge_rows<1, 64, kMaxJ, kEdgeGroup> : &k_edge_rows<1, 64, kMaxJ, 1>;
  if (v4 && wv <= 4 * 12) kern = group ? &k_edge_rows<4, 4, 12, kEdgeGroup> : &k_edge_rows<4, 4, 12, 1>;
  else if (v4 && wv <= 8 * 12) kern = group ? &k_edge_rows<4, 8, 12, kEdgeGroup> : &k_edge_rows<4, 8, 12, 1>;
  else if (v4) kern = group ? &k_edge_rows<4, 16, 8, kEdgeGroup> : &k_edge_rows<4, 16, 8, 1>;
  sgl::launch(kern, dim3(grid), dim3(kEdgeBlock), 0, stream, d, capacity, num_roots, memory, efeat, cnt, nbr, eid, X);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_conv_forward(int32_t D, int32_t F, int32_t T, int32_t H, int32_t fanout, int64_t capacity,
                                const int32_t *num_roots, const int32_t *any_edges, const float *h_root,
                                const int32_t *cnt, float *X, const float *dt, const float *w_q, const float *b_q,
                                const float *w_k, const float *b_k, const float *w_v, const float *b_v,
                                const float *w_out, const float *b_out, const float *ln_g, const float *ln_b,
                                const float *te_w, const float *te_b, float *sv_Q, float *sv_qt, float *sv_xbar,
                                float *sv_score, float *sv_ml, float *sv_agg, float *sv_z, float *sv_stats,
                                float *sv_phi0, float *S, float *y, float p_att, float p_out, uint64_t seed,
                                const uint64_t *rng_step, int32_t pass, float *sv_sdrop, const sgl_bf16_weights *bw,
                                hipStream_t stream) {
  Dims d{D, F, T, H, D + F + T, H > 0 ? D / H : 0, fanout};
  if (int rc = check_dims(d)) return rc;
  sgl::DropCfg dc;
  bool drop;
  if (int rc = drop_cfg(p_att, p_out, seed, rng_step, pass, sv_sdrop, dc, drop)) return rc;
  if (bw != nullptr)
    if (int rc = check_bf16_weights(d, *bw, drop)) return rc;
  SGL_REQUIRE(capacity >= 0 && capacity < INT_MAX && capacity % kRows == 0,
              "conv: capacity %lld must be a multiple of %d", (long long)capacity, kRows);
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && any_edges && h_root && cnt && w_q && b_q && w_k && b_k && w_v && b_v && w_out && b_out &&
                  ln_g && ln_b && te_w && te_b && sv_Q && sv_qt && sv_xbar && sv_ml && sv_agg && sv_z && sv_stats &&
                  y && (fanout == 0 || (X && dt && sv_score && (T == 0 || S))),
              "conv_forward: NULL array");
  const auto inst = bw != nullptr ? pick_instance<FwdPickBf>(d)
                    : drop ? fp32_or_wide(d, pick_instance<FwdPickDrop>(d), &pick_instance<FwdPickDropWide>)
                           : fp32_or_wide(d, pick_instance<FwdPick>(d), &pick_instance<FwdPickWide>);
  SGL_REQUIRE(inst.fn != nullptr, "conv_forward: no kernel instance for H=%d C=%d", H, d.C);
  // stage the tile's time encodings in LDS when they fit
  const bool slices = inst.waves / inst.rows / inst.hg > 1;
  int ts_rows = fanout > 0 && T > 0 ? inst.rows * fanout : 0;
  if (sizeof(float) * fwd_lds_floats(d, inst.waves, inst.rows, slices, ts_rows) > 160 * 1024) ts_rows = 0;
  const size_t lds = sizeof(float) * fwd_lds_floats(d, inst.waves, inst.rows, slices, ts_rows);
  SGL_REQUIRE(lds <= 160 * 1024, "conv_forward: %zu bytes of LDS needed (> 160 KiB)", lds);
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(inst.fn), lds));
  ConvParams p{w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b, te_w, te_b};
  ConvSaved sv{sv_Q, sv_qt, sv_xbar, sv_score, sv_ml, sv_agg, sv_z, sv_stats, sv_phi0, sv_sdrop};
  sgl::launch(inst.fn, dim3(unsigned(capacity / inst.rows)), dim3(unsigned(inst.waves * 64)), lds, stream, d,
              num_roots, any_edges, h_root, cnt, X, dt, S, p, sv, y, ts_rows, dc,
              bw != nullptr ? *bw : sgl_bf16_weights{});
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_conv_backward(int32_t D, int32_t F, int32_t T, int32_t H, int32_t fanout, int64_t capacity,
                                 const int32_t *num_roots, const int32_t *any_edges, const int32_t *cnt,
                                 const float *X, const float *S, const float *dt, const float *w_q,
                                 const float *b_q, const float *w_k, const float *b_k, const float *w_v,
                                 const float *b_v, const float *w_out, const float *b_out, const float *ln_g,
                                 const float *ln_b, const float *te_b, const float *sv_Q, const float *sv_qt,
                                 const float *sv_xbar, const float *sv_score, const float *sv_ml,
                                 const float *sv_agg, const float *sv_z, const float *sv_stats, const float *gy,
                                 int64_t *acc_src,
                                 int64_t *acc_dst, const float *w_s, const float *w_d, float *g_src, float *g_dst,
                                 float *gz, float *gagg, float *G, float *sigma, float *gQ, float *ln_part,
                                 float *te_part, float p_att, float p_out, uint64_t seed, const uint64_t *rng_step,
                                 int32_t pass, const float *sv_sdrop, const sgl_bf16_weights *bw,
                                 hipStream_t stream) {
  Dims d{D, F, T, H, D + F + T, H > 0 ? D / H : 0, fanout};
  if (int rc = check_dims(d)) return rc;
  sgl::DropCfg dc;
  bool drop;
  if (int rc = drop_cfg(p_att, p_out, seed, rng_step, pass, sv_sdrop, dc, drop)) return rc;
  if (bw != nullptr) {
    if (int rc = check_bf16_weights(d, *bw, drop)) return rc;
    SGL_REQUIRE(gy != nullptr || acc_dst != nullptr, "conv_backward: the bf16 products need both accumulators");
  }
  SGL_REQUIRE(capacity >= 0 && capacity < INT_MAX && capacity % kRows == 0,
              "conv: capacity %lld must be a multiple of %d", (long long)capacity, kRows);
  if (capacity == 0) return SGL_OK;
  SGL_REQUIRE(num_roots && any_edges && cnt && w_q && w_k && b_k && w_v && w_out && ln_g && te_b && sv_qt &&
                  sv_xbar && sv_ml && sv_z && sv_stats && (gy || (acc_src && w_s && g_src)) &&
                  (acc_dst == nullptr || (w_d && g_dst)) && (!drop || b_v) &&
                  gz && gagg && G && sigma && gQ && ln_part && te_part &&
                  (fanout == 0 || (X && dt && sv_score && (T == 0 || S))),
              "conv_backward: NULL array");
  const auto inst = bw != nullptr ? pick_instance<BwdPickBf>(d)
                    : drop ? fp32_or_wide(d, pick_instance<BwdPickDrop>(d), &pick_instance<BwdPickDropWide>)
                           : fp32_or_wide(d, pick_instance<BwdPick>(d), &pick_instance<BwdPickWide>);
  SGL_REQUIRE(inst.fn != nullptr, "conv_backward: no kernel instance for H=%d C=%d", H, d.C);
  // one ln_part / te_part tile per workgroup: the caller sized them by
  // sgl_conv_backward_tile_rows (the dropout instances' rows are the fp32 ones)
  const int32_t tile_rows = sgl_conv_backward_tile_rows(D, F, T, H, bw != nullptr ? 1 : 0);
  SGL_REQUIRE(inst.rows == tile_rows, "conv_backward: %d roots per workgroup, %d per tile", inst.rows, tile_rows);
  const size_t lds = sizeof(float) * bwd_lds_floats(d, inst.waves, inst.rows, inst.waves / inst.rows / inst.hg > 1);
  SGL_REQUIRE(lds <= 160 * 1024, "conv_backward: %zu bytes of LDS needed (> 160 KiB)", lds);
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(inst.fn), lds));
  ConvParams p{w_q, b_q, w_k, b_k, w_v, b_v, w_out, b_out, ln_g, ln_b, nullptr, te_b};
  ConvSaved sv{const_cast<float *>(sv_Q),     const_cast<float *>(sv_qt),   const_cast<float *>(sv_xbar),
               const_cast<float *>(sv_score), const_cast<float *>(sv_ml),   const_cast<float *>(sv_agg),
               const_cast<float *>(sv_z),     const_cast<float *>(sv_stats), nullptr,
               const_cast<float *>(sv_sdrop)};
  ConvGrads g{gz, gagg, G, sigma, gQ, ln_part, te_part};
  sgl::launch(inst.fn, dim3(unsigned(capacity / inst.rows)), dim3(unsigned(inst.waves * 64)), lds, stream, d,
              num_roots, any_edges, cnt, X, S, dt, p, sv, gy,
              reinterpret_cast<long long *>(acc_src), reinterpret_cast<long long *>(acc_dst), w_s, w_d, g_src, g_dst,
              g, dc, bw != nullptr ? *bw : sgl_bf16_weights{});
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
