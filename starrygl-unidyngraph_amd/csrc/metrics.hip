// sgl_link_metrics: one step's link-prediction metrics on the device (the
// computation and its reference citations are in metrics.h).
#include <climits>

#include "metrics.h"

namespace {

__global__ __launch_bounds__(sgl::met::kBlock) void k_link_metrics(sgl::met::Args a) {
  sgl::met::run(a, blockIdx.x, gridDim.x);
}

}  // namespace

extern "C" int64_t sgl_link_metrics_work_doubles(int32_t n_pos) {
  return n_pos >= 0 ? 3 * sgl::met::blocks_for(n_pos) : 0;
}

extern "C" int sgl_link_metrics(int32_t n_pos, int32_t n_neg, const float *pos_logits, const float *neg_logits,
                                const float *loss, uint64_t *seq, double *ring, int32_t ring_slots, double *out,
                                double *work, uint32_t *done, hipStream_t stream) {
  SGL_REQUIRE(n_pos >= 0 && n_neg >= 0 && int64_t(n_pos) + n_neg <= SGL_LINK_METRICS_MAX_SCORES,
              "link_metrics: %d positive + %d negative scores (at most %d)", n_pos, n_neg,
              SGL_LINK_METRICS_MAX_SCORES);
  SGL_REQUIRE((n_pos == 0 || pos_logits) && (n_neg == 0 || neg_logits), "link_metrics: NULL logits");
  SGL_REQUIRE(ring == nullptr || (seq != nullptr && ring_slots > 0), "link_metrics: a ring needs seq and slots");
  SGL_REQUIRE(ring != nullptr || out != nullptr, "link_metrics: no output");
  SGL_REQUIRE(work != nullptr && done != nullptr, "link_metrics: NULL work or done word");
  const size_t lds = sgl::met::lds_bytes(n_pos, n_neg);
  SGL_CHECK_HIP(sgl::ensure_dynamic_lds(reinterpret_cast<const void *>(&k_link_metrics), lds));
  const sgl::met::Args a{int(n_pos), int(n_neg), pos_logits, neg_logits, loss,
                         reinterpret_cast<unsigned long long *>(seq), ring, int(ring_slots), out, work,
                         reinterpret_cast<unsigned int *>(done)};
  sgl::launch(&k_link_metrics, dim3(unsigned(sgl::met::blocks_for(n_pos))), dim3(sgl::met::kBlock), lds, stream, a);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}
