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
