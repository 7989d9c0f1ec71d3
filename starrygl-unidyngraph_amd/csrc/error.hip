// C-ABI error state, version query and the once-per-kernel LDS attribute.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <unordered_map>

#include "common.h"

namespace sgl {

static thread_local char g_last_error[1024] = {0};

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
}

void clear_error() { g_last_error[0] = 0; }

hipError_t ensure_dynamic_lds(const void *kernel, size_t bytes) {
  static std::mutex mu;
  static std::unordered_map<const void *, size_t> done;
  std::lock_guard<std::mutex> lock(mu);
  auto it = done.find(kernel);
  if (it != done.end() && it->second >= bytes) return hipSuccess;
  const hipError_t e = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, int(bytes));
  if (e == hipSuccess) done[kernel] = bytes;
  return e;
}

LaunchTimer &pending_timer() {
  static thread_local LaunchTimer t{nullptr, nullptr};
  return t;
}

PlanGate &pending_gate() {
  static thread_local PlanGate g{nullptr, 0u, nullptr};
  return g;
}

PlanSignal &pending_signal() {
  static thread_local PlanSignal s{nullptr, 0u, nullptr};
  return s;
}

}  // namespace sgl

extern "C" int sgl_abi_version(void) { return SGL_ABI_VERSION; }

extern "C" int sgl_time_next_launch(hipEvent_t start, hipEvent_t stop) {
  SGL_REQUIRE((start == nullptr) == (stop == nullptr), "time_next_launch: give both events or neither");
  sgl::pending_timer() = sgl::LaunchTimer{start, stop};
  return SGL_OK;
}

extern "C" const char *sgl_last_error(void) { return sgl::g_last_error; }

extern "C" int sgl_host_device_pointer(const void *host, void **device) {
  SGL_REQUIRE(host != nullptr && device != nullptr, "host_device_pointer: NULL argument");
  SGL_CHECK_HIP(hipHostGetDevicePointer(device, const_cast<void *>(host), 0));
  return SGL_OK;
}
