// Adam over a flat parameter segment, gated by a device flag.
//
// The reference optimises model + updater parameters with torch.optim.Adam
// (backends/ctdg/runtime/factory.py:122-128). A parameter whose .grad is None
// in a step is skipped by Adam: no moment update, no step count. That happens
// to the whole temporal-attention module when a batch's sampled block has no
// edges (its output is a constant zero, models.py:88-89 / runtime.py:168-169).
// The gate `active` (device int32, NULL = always) reproduces that skip without
// a host round trip. Arithmetic follows torch's single-tensor Adam:
//   m = lerp(m, g, 1-b1); v = b2*v + (1-b2)*g*g;
//   p -= (lr / (1-b1^t)) * m / (sqrt(v) / sqrt(1-b2^t) + eps)
#include <cmath>

#include "common.h"
#include "mfma.h"

namespace {

constexpr int kBlock = 256;

__global__ __launch_bounds__(kBlock) void k_adam(int64_t n, float *__restrict__ p,
                                                 const float *__restrict__ g, float *__restrict__ m,
                                                 float *__restrict__ v, const float *__restrict__ step,
                                                 const int32_t *__restrict__ active, float lr, float b1,
                                                 float b2, float eps, float wd) {
  if (active != nullptr && *active == 0) return;
  const int64_t i = int64_t(blockIdx.x) * kBlock + threadIdx.x;
  if (i >= n) return;
  const double t = double(*step) + 1.0;
  const double bc1 = 1.0 - pow(double(b1), t);
  const double bc2 = 1.0 - pow(double(b2), t);
  const float step_size = float(double(lr) / bc1);
  const float bc2_sqrt = float(sqrt(bc2));
  float gi = g[i];
  if (wd != 0.f) gi = gi + wd * p[i];
  const float w = 1.f - b1;
  float mi = m[i];
  mi = mi + w * (gi - mi);
  const float vi = v[i] * b2 + (1.f - b2) * gi * gi;
  m[i] = mi;
  v[i] = vi;
  const float denom = sqrtf(vi) / bc2_sqrt + eps;
  p[i] = p[i] - step_size * (mi / denom);
}

__global__ void k_adam_advance(float *step, const int32_t *active) {
  if (active == nullptr || *active != 0) *step += 1.f;
}

}  // namespace

extern "C" int sgl_adam_step(int64_t n, float *param, const float *grad, float *exp_avg, float *exp_avg_sq,
                             const float *step, const int32_t *active, float lr, float beta1, float beta2,
                             float eps, float weight_decay, hipStream_t stream) {
  SGL_REQUIRE(n >= 0, "adam: n < 0");
  if (n == 0) return SGL_OK;
  SGL_REQUIRE(param && grad && exp_avg && exp_avg_sq && step, "adam: NULL array");
  k_adam<<<unsigned((n + kBlock - 1) / kBlock), kBlock, 0, stream>>>(n, param, grad, exp_avg, exp_avg_sq, step,
                                                                     active, lr, beta1, beta2, eps, weight_decay);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_adam_advance(float *step, const int32_t *active, hipStream_t stream) {
  SGL_REQUIRE(step != nullptr, "adam_advance: NULL step");
  k_adam_advance<<<1, 1, 0, stream>>>(step, active);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

// ---------------------------------------------------------------------------
// Fused weight gradients + Adam.
//
// Each workgroup owns one tile of one job (sgl_grad_job). A kind-0 job is a
// gradient block G[a][b] = sum_{r < R} X1[r][a] * X2[r][b] (a reduction over
// the step's roots or tiles); its 16x16 tile is computed with
// v_mfma_f32_16x16x4_f32, the four waves taking every fourth group of 4 rows,
// then summed through LDS. A kind-1 job covers 256 contiguous elements whose
// gradient is already in place. Either way each thread then owns one
// gradient element: it stores the gradient and, if its segment is active
// this step, applies the Adam update to the parameter and moments with the
// bias corrections in coef (k_adam_coef, enqueued earlier). No workgroup
// reads a value another one of this launch writes, and none counts
// completions: the step counts advance in k_adam_coef. A kind-0 job may
// also keep bf16 copies of its parameter block (as is and transposed, at
// the job's shadow offsets) for the bf16 products of the attention and the
// edge predictor; they are written from the parameter after the update.
namespace {

constexpr int kGaBlock = 256;
constexpr int kGaChunk = 16;  // MFMA row groups per wave per load batch

struct AdamSegs {
  float *step[SGL_MAX_ADAM_SEGMENTS];
  const int32_t *gate[SGL_MAX_ADAM_SEGMENTS];
};

// A tile's entry of tile_job: its job in the low 8 bits and its index among
// the job's tiles above them (-1: no tile). The host deals each job's tiles
// to one XCD where it can (workgroup w runs on XCD w % 8) and splits the
// larger ones into ranges of consecutive tiles, so that the activation
// strips a job reads are fetched into few XCDs' L2s. A kind-0 job's tile l
// computes the 16x16 block (l / tiles_b, l % tiles_b): a range of them is a
// band of block rows, which shares the x1 strips of its rows.
__device__ __forceinline__ int tile_entry_job(int32_t e) { return e & 0xFF; }
__device__ __forceinline__ int tile_entry_local(int32_t e) { return e >> 8; }

// Workgroup blockIdx.x's job and tile (false: a padding slot, nothing to do;
// uniform). With tile_job, its entry names the job and the tile; without,
// jobs holds one copy per workgroup with the tile's index in tile0 (kind < 0
// marks padding), which takes the entry's load off the front of the chain.
__device__ __forceinline__ bool workgroup_tile(const sgl_grad_job *__restrict__ jobs,
                                               const int32_t *__restrict__ tile_job, sgl_grad_job &jb, int &local) {
  if (tile_job != nullptr) {
    const int32_t entry = tile_job[blockIdx.x];
    if (entry < 0) return false;
    jb = jobs[tile_entry_job(entry)];
    local = tile_entry_local(entry);
    return true;
  }
  jb = jobs[blockIdx.x];
  local = jb.tile0;
  return jb.kind >= 0;
}

// The reduction length of a kind-0 job: r_fixed; *num_roots + r_extra when
// r_fixed == -1; the tiles of -r_fixed rows that hold live rows when
// r_fixed <= -2 (per-tile partial sums; the rest are zero).
__device__ __forceinline__ int job_rows(const sgl_grad_job &jb, const int32_t *num_roots) {
  if (jb.r_fixed >= 0) return jb.r_fixed;
  if (jb.r_fixed == -1) return *num_roots + jb.r_extra;
  return (*num_roots - jb.r_fixed - 1) / (-jb.r_fixed);
}

__global__ __launch_bounds__(kGaBlock) void k_grad_adam(const sgl_grad_job *__restrict__ jobs,
                                                       const int32_t *__restrict__ tile_job,
                                                       const int32_t *__restrict__ num_roots, float *__restrict__ p,
                                                       float *__restrict__ g, float *__restrict__ m,
                                                       float *__restrict__ v, AdamSegs segs,
                                                       const float *__restrict__ coef, float b1, float b2, float eps,
                                                       float wd, uint16_t *__restrict__ shadow) {
  __shared__ float red[4][16][17];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  sgl_grad_job jb;
  int local;
  if (!workgroup_tile(jobs, tile_job, jb, local)) return;  // uniform: a padding slot of the XCD deal
  const bool active = segs.gate[jb.seg] == nullptr || *segs.gate[jb.seg] != 0;
  const float step_size = coef[2 * jb.seg], bc2_sqrt = coef[2 * jb.seg + 1];

  int64_t idx = 0;
  bool valid = false;
  float gv = 0.f, pv = 0.f, mv = 0.f, vv = 0.f;
  int ea = 0, eb = 0;  // a kind-0 element's position in its block
  if (jb.kind == 0) {
    const int ta = local / jb.tiles_b, tb = local - ta * jb.tiles_b;
    const int a0 = 16 * ta, b0 = 16 * tb;
    const int oa = tid >> 4, ob = tid & 15;
    ea = a0 + oa;
    eb = b0 + ob;
    valid = a0 + oa < jb.rows && b0 + ob < jb.cols;
    idx = jb.off + int64_t(a0 + oa) * jb.ldo + (b0 + ob);
    // this thread's Adam operands, loaded while the tile is reduced
    if (valid) {
      pv = p[idx];
      mv = m[idx];
      vv = v[idx];
    }
    const int R = job_rows(jb, num_roots);
    const int i16 = lane & 15, q = lane >> 4;
    sgl::f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const int npass = jb.npass > 0 ? jb.npass : 1;
    for (int ps = 0; R > 0 && ps < npass; ++ps) {
      // rows >= R read 0 through the buffer ranges (X1 rows are at least
      // `rows` wide, so row R starts past X1's span)
      const uint32_t span1 = uint32_t(R - 1) * uint32_t(jb.s1) + uint32_t(jb.rows);
      const uint32_t span2 = uint32_t(R - 1) * uint32_t(jb.s2) + uint32_t(jb.cols);
      const __amdgpu_buffer_rsrc_t r1 = sgl::weight_rsrc(jb.x1 + ps * jb.ps1, span1);
      const __amdgpu_buffer_rsrc_t r2 = sgl::weight_rsrc(jb.x2 + ps * jb.ps2, span2);
      const int ngroups = (R + 3) >> 2;
      for (int gb = wave; gb < ngroups; gb += 4 * kGaChunk) {
        float xa[kGaChunk], xb[kGaChunk];
#pragma unroll
        for (int c = 0; c < kGaChunk; ++c) {
          const uint32_t r = uint32_t(4 * (gb + 4 * c) + q);
          xa[c] = sgl::buf_load(r1, r * uint32_t(jb.s1) + uint32_t(a0 + i16));
          xb[c] = sgl::buf_load(r2, r * uint32_t(jb.s2) + uint32_t(b0 + i16));
        }
#pragma unroll
        for (int c = 0; c < kGaChunk; ++c) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[c], xb[c], acc, 0, 0, 0);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) red[wave][4 * (lane >> 4) + e][lane & 15] = acc[e];
    __syncthreads();
    gv = red[0][oa][ob] + red[1][oa][ob] + red[2][oa][ob] + red[3][oa][ob];
    if (valid) g[idx] = gv;
  } else {
    // kind 1: Adam over contiguous elements whose gradient is in place
    const int64_t e = int64_t(local) * kGaBlock + tid;
    valid = e < int64_t(jb.rows) * jb.cols;
    idx = jb.off + e;
    if (valid) {
      gv = g[idx];
      pv = p[idx];
      mv = m[idx];
      vv = v[idx];
    }
  }
  if (valid && active) {
    float gi = gv;
    if (wd != 0.f) gi = gi + wd * pv;
    mv = mv + (1.f - b1) * (gi - mv);
    vv = vv * b2 + (1.f - b2) * gi * gi;
    m[idx] = mv;
    v[idx] = vv;
    const float denom = sqrtf(vv) / bc2_sqrt + eps;
    pv = pv - step_size * (mv / denom);
    p[idx] = pv;
  }
  if (shadow != nullptr && valid && jb.kind == 0) {
    const uint16_t hv = __builtin_bit_cast(uint16_t, static_cast<__bf16>(pv));
    if (jb.sh_off >= 0) shadow[jb.sh_off + int64_t(ea) * jb.sh_ld + eb] = hv;
    if (jb.sht_off >= 0) shadow[jb.sht_off + int64_t(eb) * jb.sht_ld + ea] = hv;
  }
}

// The bf16 copies of every kind-0 job's block from the parameters as they
// are (one 16x16 tile per workgroup, as k_grad_adam deals them).
__global__ __launch_bounds__(kGaBlock) void k_grad_shadows(const sgl_grad_job *__restrict__ jobs,
                                                          const int32_t *__restrict__ tile_job,
                                                          const float *__restrict__ p,
                                                          uint16_t *__restrict__ shadow) {
  sgl_grad_job jb;
  int local;
  if (!workgroup_tile(jobs, tile_job, jb, local)) return;
  if (jb.kind != 0 || (jb.sh_off < 0 && jb.sht_off < 0)) return;
  const int ta = local / jb.tiles_b, tb = local - (local / jb.tiles_b) * jb.tiles_b;
  const int ea = 16 * ta + (threadIdx.x >> 4), eb = 16 * tb + (threadIdx.x & 15);
  if (ea >= jb.rows || eb >= jb.cols) return;
  const uint16_t hv = __builtin_bit_cast(uint16_t, static_cast<__bf16>(p[jb.off + int64_t(ea) * jb.ldo + eb]));
  if (jb.sh_off >= 0) shadow[jb.sh_off + int64_t(ea) * jb.sh_ld + eb] = hv;
  if (jb.sht_off >= 0) shadow[jb.sht_off + int64_t(eb) * jb.sht_ld + ea] = hv;
}

// One lane per segment: advance the open segments' step counts and write
// the bias corrections of the step they are now at (torch.optim.Adam: the
// count is incremented first, then lr / (1 - b1^t) and sqrt(1 - b2^t) in
// double). A closed segment keeps its count; its coef (for the next count) is
// unused. Every load is issued before the first store (one round trip; the
// step counters are distinct words, sgl_adam_coef checks it).
__global__ void k_adam_coef(int nseg, AdamSegs segs, float *__restrict__ coef, float lr, float b1, float b2,
                            unsigned long long *step_counter, unsigned long long *step_out, uint32_t *sig_word,
                            uint32_t sig_value) {
  const int lane = threadIdx.x;
  float *sp = nullptr;
  const int32_t *gp = nullptr;
#pragma unroll
  for (int s = 0; s < SGL_MAX_ADAM_SEGMENTS; ++s)
    if (lane == s) {
      sp = segs.step[s];
      gp = segs.gate[s];
    }
  const bool mine = lane < nseg;
  const bool counts = lane == 0 && step_counter != nullptr;
  unsigned long long n = 0ull;
  if (counts) n = *step_counter;
  float st = 0.f;
  int32_t g = 1;
  if (mine) {
    st = *sp;
    if (gp != nullptr) g = *gp;
  }
  if (counts) {
    *step_counter = n + 1ull;
    *step_out = n + 1ull;
  }
  if (mine) {
    if (g != 0) *sp = st + 1.f;
    const double t = double(st) + 1.0;
    coef[2 * lane] = float(double(lr) / (1.0 - pow(double(b1), t)));
    coef[2 * lane + 1] = float(sqrt(1.0 - pow(double(b2), t)));
  }
  // a launch plan's signal: the earlier kernels of the stream are done
  // (stream order); every lane's writes are released before lane 0's store
  if (sig_word != nullptr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    __syncthreads();
    if (lane == 0) __hip_atomic_store(sig_word, sig_value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
  }
}

AdamSegs make_segs(int nseg, float *const *steps, const int32_t *const *gates) {
  AdamSegs segs{};
  for (int s = 0; s < nseg; ++s) {
    segs.step[s] = steps != nullptr ? steps[s] : nullptr;
    segs.gate[s] = gates != nullptr ? gates[s] : nullptr;
  }
  return segs;
}

}  // namespace

extern "C" int sgl_grad_adam(const sgl_grad_job *jobs, const int32_t *tile_job, int32_t num_tiles,
                             const int32_t *num_roots, float *param, float *grad, float *exp_avg, float *exp_avg_sq,
                             int32_t nseg, const int32_t *const *gates, const float *coef, float beta1, float beta2,
                             float eps, float weight_decay, uint16_t *shadow, hipStream_t stream) {
  SGL_REQUIRE(num_tiles >= 0, "grad_adam: num_tiles < 0");
  SGL_REQUIRE(nseg > 0 && nseg <= SGL_MAX_ADAM_SEGMENTS, "grad_adam: nseg %d out of range", nseg);
  if (num_tiles == 0) return SGL_OK;
  SGL_REQUIRE(jobs && param && grad && exp_avg && exp_avg_sq && coef, "grad_adam: NULL array");
  sgl::launch(&k_grad_adam, dim3(unsigned(num_tiles)), dim3(kGaBlock), 0, stream, jobs, tile_job, num_roots, param,
              grad, exp_avg, exp_avg_sq, make_segs(nseg, nullptr, gates), coef, beta1, beta2, eps, weight_decay,
              shadow);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_grad_shadows(const sgl_grad_job *jobs, const int32_t *tile_job, int32_t num_tiles,
                                const float *param, uint16_t *shadow, hipStream_t stream) {
  SGL_REQUIRE(num_tiles >= 0, "grad_shadows: num_tiles < 0");
  if (num_tiles == 0) return SGL_OK;
  SGL_REQUIRE(jobs && param && shadow, "grad_shadows: NULL array");
  sgl::launch(&k_grad_shadows, dim3(unsigned(num_tiles)), dim3(kGaBlock), 0, stream, jobs, tile_job, param, shadow);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

extern "C" int sgl_adam_coef(int32_t nseg, float *const *steps, const int32_t *const *gates, float *coef, float lr,
                             float beta1, float beta2, uint64_t *step_counter, uint64_t *step_out,
                             hipStream_t stream) {
  SGL_REQUIRE(nseg > 0 && nseg <= SGL_MAX_ADAM_SEGMENTS, "adam_coef: nseg %d out of range", nseg);
  SGL_REQUIRE(steps != nullptr && coef != nullptr, "adam_coef: NULL array");
  SGL_REQUIRE(step_counter == nullptr || step_out != nullptr, "adam_coef: step_counter without step_out");
  for (int s = 0; s < nseg; ++s) {
    SGL_REQUIRE(steps[s] != nullptr, "adam_coef: NULL step counter %d", s);
    for (int r = 0; r < s; ++r) SGL_REQUIRE(steps[r] != steps[s], "adam_coef: segments %d and %d share a step counter", r, s);
  }
  const sgl::PlanSignal sig = sgl::take_signal();  // a launch plan's signal, folded
  sgl::launch(&k_adam_coef, dim3(1), dim3(64), 0, stream, int(nseg), make_segs(nseg, steps, gates), coef, lr, beta1,
              beta2, reinterpret_cast<unsigned long long *>(step_counter),
              reinterpret_cast<unsigned long long *>(step_out), sig.word, sig.value);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
