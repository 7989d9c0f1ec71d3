// Shared helpers for the MI355X (gfx950) CTDG kernels: C-ABI error state,
// launch checks and wave64 scan primitives.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <type_traits>

#include "../../include/starrygl_mi355x.h"

namespace sgl {

// Upper bound on the grids of the grid-stride kernels whose work is the live
// part of a capacity-sized range (8 workgroups of 256 threads per CU): a
// batch far below capacity then costs no idle workgroups.
constexpr int64_t kMaxGrid = 2048;

// Thread-local last error (read through sgl_last_error()).
void set_error(const char *fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

constexpr int kWave = 64;

// Raises a kernel's dynamic-LDS limit to at least `bytes` (the first call per
// kernel and size only; thread-safe). Keeps hipFuncSetAttribute out of the
// steady state, and so out of captured HIP graphs once a step has run.
hipError_t ensure_dynamic_lds(const void *kernel, size_t bytes);

// Timing of the next kernel launch on this host thread (sgl_time_next_launch,
// a plan's timed op): the launch records the two events itself, from the
// dispatch's own start and end (hipExtLaunchKernel), so nothing else is
// queued between them.
struct LaunchTimer {
  hipEvent_t start, stop;
};
LaunchTimer &pending_timer();

// A launch plan's cross-stream ordering handed to the first or last kernel
// of one of its parts (sgl_plan_run, this host thread): the gate holds the
// kernel's work until *word >= value (giving up after ~2 s and setting
// *timeout); the signal stores value to *word once all of the launch's work
// is done (release; counter is unused by the one-lane kernels that take
// signals). An entry point that takes one either folds it into its kernel or
// launches the one-lane gate / signal kernel itself (launch_gate /
// launch_signal), so that each is issued exactly once and in order.
struct PlanGate {
  const uint32_t *word;
  uint32_t value;
  uint32_t *timeout;
};
struct PlanSignal {
  uint32_t *word;
  uint32_t value;
  uint32_t *counter;
};
PlanGate &pending_gate();
PlanSignal &pending_signal();
inline PlanGate take_gate() {
  const PlanGate g = pending_gate();
  pending_gate() = PlanGate{nullptr, 0u, nullptr};
  return g;
}
inline PlanSignal take_signal() {
  const PlanSignal s = pending_signal();
  pending_signal() = PlanSignal{nullptr, 0u, nullptr};
  return s;
}
int launch_gate(const PlanGate &g, hipStream_t stream);
int launch_signal(const PlanSignal &s, hipStream_t stream);

// One thread: poll the gate word (acquire, agent scope) with s_sleep between
// reads; after ~2 s (100 MHz clock) set the timeout word and give up.
__device__ __forceinline__ void gate_wait(const uint32_t *word, uint32_t value, uint32_t *timeout) {
  const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
  while (__hip_atomic_load(word, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < value) {
    if (__builtin_amdgcn_s_memrealtime() - t0 > 200000000ull) {
      __hip_atomic_store(timeout, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      return;
    }
    __builtin_amdgcn_s_sleep(1);
  }
}

template <typename F, typename... Args>
inline void launch(F kernel, dim3 grid, dim3 block, size_t lds, hipStream_t stream, Args... args) {
  LaunchTimer &t = pending_timer();
  if (t.start != nullptr) {
    const LaunchTimer u = t;
    t = LaunchTimer{nullptr, nullptr};
    hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(lds), stream, u.start, u.stop, 0u, args...);
  } else {
    kernel<<<grid, block, lds, stream>>>(args...);
  }
}

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }

// Carves aligned sub-buffers out of a caller-provided workspace.
struct Carver {
  char *base;
  size_t used = 0;
  explicit Carver(void *p) : base(static_cast<char *>(p)) {}
  template <typename T>
  T *take(size_t count) {
    T *p = reinterpret_cast<T *>(base ? base + used : nullptr);
    used = align_up(used + count * sizeof(T));
    return p;
  }
};

// Inclusive scan across one 64-lane wavefront.
template <typename T>
__device__ __forceinline__ T wave_inclusive_scan(T v) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int d = 1; d < kWave; d <<= 1) {
    T n = __shfl_up(v, d, kWave);
    if (lane >= d) v += n;
  }
  return v;
}

// Sum over the 64 lanes of a wavefront, returned to every lane, through lane
// permutes that stay in the VALU: DPP quad_perm (xor 1, xor 2), DPP row_ror
// 4 and 8 (a 16-lane row sums to every lane of the row), ds_swizzle xor 16
// (32-lane halves), then the two halves' sums read from lanes 0 and 32.
__device__ __forceinline__ float wave_sum_dpp(float v) {
  auto mov = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, true));
  };
  v += mov(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  v += mov(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  v += mov(v, std::integral_constant<int, 0x124>{});  // row_ror:4
  v += mov(v, std::integral_constant<int, 0x128>{});  // row_ror:8
  v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16 within 32 lanes
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0)) +
         __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
}

// Fixed-point accumulation (SGL_FIXED_SHIFT fractional bits in an int64):
// integer atomics are exact, so sums scattered by many workgroups do not
// depend on the order the additions happen in. Values are clamped to the
// int64 range (|x| < 2^23 fits); to_fixed_checked reports a value outside it.
__device__ __forceinline__ long long to_fixed(float x) {
  const float s = x * 0x1p40f;
  return static_cast<long long>(rintf(fminf(fmaxf(s, -9.0e18f), 9.0e18f)));
}
// to_fixed, and *flag |= 1 when x lies outside the range (|x| >= 2^23, or
// NaN): the clamped value no longer adds up to the sum the caller wanted.
__device__ __forceinline__ long long to_fixed_checked(float x, int32_t *flag) {
  if (!(fabsf(x) < 0x1p23f)) atomicOr(flag, 1);
  return to_fixed(x);
}
__device__ __forceinline__ float from_fixed(long long v) { return float(double(v) * 0x1p-40); }
__device__ __forceinline__ void atomic_add_fixed(long long *p, long long v) {
  atomicAdd(reinterpret_cast<unsigned long long *>(p), static_cast<unsigned long long>(v));
}
static_assert(SGL_FIXED_SHIFT == 40, "to_fixed / from_fixed scale");

// "The last workgroup of a launch does X". Same-word atomics serialize
// (~20 ns each) and every atomic is a round trip (~1.5 us), so a small grid
// counts on one word and a large one on two levels: block b counts itself
// into group b % kDoneGroups's word, the last of a group into the top word,
// the last of those is the launch's last block. done holds SGL_DONE_WORDS
// int32 (the group words kDoneStride apart, the top word after them), zero
// between launches; each word is cleared by the block that completes it.
// Call from one thread per block, after the block's own global writes and
// atomics have completed; one-dimensional grids.
constexpr int kDoneGroups = 16, kDoneStride = 64, kDoneFlat = 64;
static_assert((kDoneGroups + 1) * kDoneStride == SGL_DONE_WORDS, "completion counter size");
__device__ inline bool last_block(int32_t *done) {
  const unsigned g = gridDim.x, b = blockIdx.x;
  int32_t *top = done + kDoneGroups * kDoneStride;
  int arrivals = int(g);
  if (g > unsigned(kDoneFlat)) {
    const unsigned grp = b % kDoneGroups;
    int32_t *w = done + grp * kDoneStride;
    if (atomicAdd(w, 1) != int((g - grp + kDoneGroups - 1) / kDoneGroups) - 1) return false;
    __hip_atomic_store(w, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    arrivals = kDoneGroups;
  }
  if (atomicAdd(top, 1) != arrivals - 1) return false;
  __hip_atomic_store(top, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// Counter-based random numbers: Philox4x32-10 (Salmon, Moraes, Dror, Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC 2011): ten rounds of two
// 32x32->64 multiplies with the published multipliers and Weyl key
// increments. Four independent uint32 per (counter, key); no state.
struct U32x4 {
  uint32_t v[4];
};
__device__ __forceinline__ U32x4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                               uint32_t k1) {
  constexpr uint32_t kM0 = 0xD2511F53u, kM1 = 0xCD9E8D57u, kW0 = 0x9E3779B9u, kW1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = uint64_t(kM0) * c0, p1 = uint64_t(kM1) * c2;
    const uint32_t n0 = uint32_t(p1 >> 32) ^ c1 ^ k0, n2 = uint32_t(p0 >> 32) ^ c3 ^ k1;
    c0 = n0;
    c1 = uint32_t(p1);
    c2 = n2;
    c3 = uint32_t(p0);
    k0 += kW0;
    k1 += kW1;
  }
  return U32x4{{c0, c1, c2, c3}};
}

// Dropout masks of the attention (inverted dropout: kept entries scale by
// 1 / (1 - p)). A mask value is keep(u) ? scale : 0 for the uint32 u at the
// element's place in the stream of (seed, step): attention weights draw
// counter (row, slot, 2 * pass, step) and take lane h (head h < 4); output
// entries draw (row, col / 4, 2 * pass + 1, step) and take lane col % 4.
// Key = (seed low word, seed high word ^ step high word). u / 2^32 >= p keeps.
struct DropCfg {
  float p_att, p_out;          // drop probabilities (0: that dropout is off)
  uint32_t seed_lo, seed_hi;
  const unsigned long long *step;  // the step's counter (device)
  int pass;
};
__device__ __forceinline__ float drop_scale(float p) { return p > 0.f ? 1.f / (1.f - p) : 1.f; }
__device__ __forceinline__ float drop_keep(uint32_t u, float p, float scale) {
  return float(u >> 8) * 0x1p-24f >= p ? scale : 0.f;
}
__device__ __forceinline__ U32x4 drop_bits(const DropCfg &c, unsigned long long step, uint32_t row, uint32_t col,
                                           int out) {
  return philox4x32_10(row, col, uint32_t(2 * c.pass + out), uint32_t(step), c.seed_lo,
                       c.seed_hi ^ uint32_t(step >> 32));
}

template <typename T>
__device__ __forceinline__ T wave_reduce_sum(T v) {
#pragma unroll
  for (int d = kWave / 2; d > 0; d >>= 1) v += __shfl_xor(v, d, kWave);
  return v;
}

// Exclusive scan across a block of BLOCK threads (BLOCK a multiple of 64).
// s_wave must hold BLOCK/64 elements. Returns the exclusive prefix and the
// block total. Contains two __syncthreads(): call from uniform control flow.
template <typename T, int BLOCK>
__device__ __forceinline__ T block_exclusive_scan(T v, T *s_wave, T &total) {
  static_assert(BLOCK % kWave == 0, "block must be whole waves");
  constexpr int W = BLOCK / kWave;
  const T inc = wave_inclusive_scan(v);
  const int lane = threadIdx.x & (kWave - 1);
  const int w = threadIdx.x / kWave;
  if (lane == kWave - 1) s_wave[w] = inc;
  __syncthreads();
  T before = 0, tot = 0;
#pragma unroll
  for (int i = 0; i < W; ++i) {
    const T s = s_wave[i];
    before += (i < w) ? s : T(0);
    tot += s;
  }
  total = tot;
  __syncthreads();
  return before + inc - v;
}

}  // namespace sgl

#define SGL_CHECK_HIP(expr)                                                    \
  do {                                                                         \
    hipError_t e_ = (expr);                                                    \
    if (e_ != hipSuccess) {                                                    \
      sgl::set_error("%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                     __FILE__, __LINE__);                                      \
      return SGL_ERR_HIP;                                                      \
    }                                                                          \
  } while (0)

#define SGL_CHECK_LAUNCH() SGL_CHECK_HIP(hipGetLastError())

#define SGL_REQUIRE(cond, ...)                                                 \
  do {                                                                         \
    if (!(cond)) {                                                             \
      sgl::set_error(__VA_ARGS__);                                             \
      return SGL_ERR_INVALID;                                                  \
    }                                                                          \
  } while (0)
