// Launch plans: a training step's library calls recorded once (their
// arguments are fixed device pointers and sizes: events are read at a device
// cursor) and replayed with plain kernel launches by one host call.
//
// A plan is two runs of ops: the front part of a step (batch preparation,
// sampling, GRU memory update, memory commit, the edge rows, the Adam step
// counts) and the back part (attention forward, edge predictor, backward,
// fused Adam). Consecutive steps use different step buffers, and nothing in
// a back part reads the memory table (the edge rows hold the neighbours'
// memory), so step t's front part only needs the back part of step t-2
// (the last reader of its buffers) to be done, and runs beside step t-1's
// back part. The streams order themselves through two device words (a
// one-lane signal kernel stores a number once the stream's earlier kernels
// are done; a one-lane wait kernel holds the stream until the word reaches
// a value):
//
//   front:  wait(back >= need_back) -> front ops -> signal(fronted = seq)
//   back:   signal(back = seq - 1), wait(fronted >= seq) -> back ops
//
// (a back part's number is stored by the next back part's first kernel, once
// every earlier kernel of the back stream is done)
//
// A gate is folded only into a kernel of few workgroups (the batch
// preparation): the workgroups of a large kernel waiting at a gate can hold
// every CU, so that the other stream's work they wait for cannot run (a
// folded gate in the attention forward timed out that way).
//
// Plain launches cost the GPU well under a microsecond between kernels; the
// same kernels replayed as graphs cost several, and more at graph
// boundaries; the signal / wait kernels cost less than ROCm's stream memory
// operations or events between streams.
#include <cstring>
#include <type_traits>
#include <utility>

#include "common.h"

namespace {

template <typename T>
T from_slot(uint64_t v) {
  if constexpr (std::is_pointer_v<T>) {
    return reinterpret_cast<T>(static_cast<uintptr_t>(v));
  } else if constexpr (std::is_same_v<T, float>) {
    const uint32_t u = static_cast<uint32_t>(v);
    float f;
    std::memcpy(&f, &u, sizeof f);
    return f;
  } else {
    static_assert(std::is_integral_v<T>, "plan slots hold pointers, integers and floats");
    return static_cast<T>(v);
  }
}

template <typename T, size_t I, size_t N>
T arg_at(const uint64_t *a, hipStream_t s) {
  if constexpr (I + 1 == N) {
    static_assert(std::is_same_v<T, hipStream_t>, "a planned entry point takes the stream last");
    return s;
  } else {
    return from_slot<T>(a[I]);
  }
}

template <typename... Args, size_t... I>
int invoke(int (*fn)(Args...), const uint64_t *a, hipStream_t s, std::index_sequence<I...>) {
  return fn(arg_at<Args, I, sizeof...(Args)>(a, s)...);
}

template <typename... Args>
constexpr int slots_of(int (*)(Args...)) {
  return int(sizeof...(Args)) - 1;
}

template <auto Fn>
int run_op(const uint64_t *a, hipStream_t s) {
  return invoke(Fn, a, s, std::make_index_sequence<size_t(slots_of(Fn) + 1)>{});
}

struct OpEntry {
  const char *name;
  int (*run)(const uint64_t *, hipStream_t);
  int slots;
  bool takes_gate;    // as a part's first op it takes the part's gate (sgl::take_gate)
  bool takes_signal;  // as a part's last op it takes the part's signal (sgl::take_signal)
};

#define SGL_OP(fn) {#fn, &run_op<&fn>, slots_of(&fn), false, false}
#define SGL_OP_GS(fn, g, s) {#fn, &run_op<&fn>, slots_of(&fn), g, s}
const OpEntry kOps[] = {
    SGL_OP_GS(sgl_batch_prepare, true, false), SGL_OP(sgl_recent_sample), SGL_OP(sgl_memory_update),
    SGL_OP(sgl_memory_commit), SGL_OP(sgl_conv_forward), SGL_OP(sgl_predictor), SGL_OP(sgl_conv_backward),
    SGL_OP(sgl_grad_adam), SGL_OP_GS(sgl_adam_coef, false, true), SGL_OP(sgl_edge_rows),
    SGL_OP(sgl_memory_update_bf16), SGL_OP(sgl_recent_sample_packed), SGL_OP(sgl_memory_gather),
    SGL_OP(sgl_negatives_from_draws), SGL_OP(sgl_time_projection_forward), SGL_OP(sgl_time_projection_backward),
    SGL_OP(sgl_link_metrics), SGL_OP_GS(sgl_batch_prepare_metrics, true, false),
};
#undef SGL_OP
#undef SGL_OP_GS
constexpr int kNumOps = int(sizeof(kOps) / sizeof(kOps[0]));
static_assert(kNumOps > 0, "op table");

// Optional timing of one op: its kernel's dispatch records the two events.
struct OpTimer {
  int op;
  hipEvent_t start, end;
};

// The ops of one part in order. `gate` (word NULL: none) is handed to the
// first op, `sig` to the last; both must take theirs (their kinds say so).
int run_ops(const sgl_op *ops, int n, hipStream_t s, int base, const OpTimer &t, const sgl::PlanGate &gate,
            const sgl::PlanSignal &sig) {
  for (int i = 0; i < n; ++i) {
    const sgl_op &op = ops[i];
    SGL_REQUIRE(op.kind >= 0 && op.kind < kNumOps, "plan op %d: unknown kind %d", base + i, op.kind);
    const OpEntry &e = kOps[op.kind];
    SGL_REQUIRE(op.nargs == e.slots, "plan op %d (%s): %d arguments recorded, %d expected", base + i, e.name,
                op.nargs, e.slots);
    const bool timed = base + i == t.op;
    if (timed) sgl::pending_timer() = sgl::LaunchTimer{t.start, t.end};  // the op's (first) kernel records them
    if (i == 0 && gate.word != nullptr) sgl::pending_gate() = gate;
    if (i == n - 1 && sig.word != nullptr) sgl::pending_signal() = sig;
    const int rc = e.run(op.a, s);
    if (timed) sgl::pending_timer() = sgl::LaunchTimer{nullptr, nullptr};
    // an op that failed before taking them leaves nothing pending
    const bool left = sgl::take_gate().word != nullptr || sgl::take_signal().word != nullptr;
    if (rc) return rc;
    SGL_REQUIRE(!left, "plan op %d (%s): the part's gate or signal was not taken", base + i, e.name);
  }
  return SGL_OK;
}

// Cross-stream ordering: a one-lane kernel that stores a sequence number
// (release: the stream's earlier kernels have completed, their writes are
// visible to the device) and one that waits until a word reaches a value
// (acquire), polling with s_sleep and giving up after about two seconds
// (then it sets the timeout word, which the host checks).
__global__ void k_signal(uint32_t *word, uint32_t value) {
  if (threadIdx.x == 0) __hip_atomic_store(word, value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void k_gate(const uint32_t *word, uint32_t value, uint32_t *timeout) {
  if (threadIdx.x == 0) sgl::gate_wait(word, value, timeout);
}

// The back part's first kernel: the previous step's back part is done (it
// precedes this kernel on the back stream), so its number is stored here
// (release), then the kernel waits for this step's front part. One launch
// where a signal at the end of each back part and a wait at the start of the
// next took two on the critical stream.
__global__ void k_signal_gate(uint32_t *sig_word, uint32_t sig_value, const uint32_t *word, uint32_t value,
                              uint32_t *timeout) {
  if (threadIdx.x == 0) {
    if (sig_word != nullptr) __hip_atomic_store(sig_word, sig_value, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
    sgl::gate_wait(word, value, timeout);
  }
}

int signal(uint32_t *word, uint32_t value, hipStream_t s) {
  k_signal<<<1, 64, 0, s>>>(word, value);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

int gate(const uint32_t *word, uint32_t value, uint32_t *timeout, hipStream_t s) {
  k_gate<<<1, 64, 0, s>>>(word, value, timeout);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

int signal_gate(uint32_t *sig_word, uint32_t sig_value, const uint32_t *word, uint32_t value, uint32_t *timeout,
                hipStream_t s) {
  k_signal_gate<<<1, 64, 0, s>>>(sig_word, sig_value, word, value, timeout);
  SGL_CHECK_LAUNCH();
  return SGL_OK;
}

}  // namespace

int sgl::launch_gate(const PlanGate &g, hipStream_t s) { return gate(g.word, g.value, g.timeout, s); }
int sgl::launch_signal(const PlanSignal &sg, hipStream_t s) { return signal(sg.word, sg.value, s); }

extern "C" int32_t sgl_plan_op_kind(const char *name, int32_t *nargs) {
  if (name == nullptr) return -1;
  for (int k = 0; k < kNumOps; ++k)
    if (std::strcmp(kOps[k].name, name) == 0) {
      if (nargs != nullptr) *nargs = kOps[k].slots;
      return k;
    }
  return -1;
}

extern "C" int sgl_plan_run(const sgl_op *ops, int32_t n_front, int32_t n_back, hipStream_t front,
                            hipStream_t back, uint32_t *sync, uint32_t seq, uint32_t need_back, int32_t timed_op,
                            hipEvent_t t_start, hipEvent_t t_end) {
  SGL_REQUIRE(ops != nullptr || n_front + n_back == 0, "plan_run: NULL ops");
  SGL_REQUIRE(n_front >= 0 && n_back >= 0, "plan_run: negative op count");
  SGL_REQUIRE(timed_op < 0 || (t_start && t_end), "plan_run: NULL timing event");
  const OpTimer t{timed_op, t_start, t_end};
  const sgl::PlanGate no_gate{nullptr, 0u, nullptr};
  const sgl::PlanSignal no_signal{nullptr, 0u, nullptr};
  if (front == nullptr) {  // one stream: everything in order on the back stream
    return run_ops(ops, n_front + n_back, back, 0, t, no_gate, no_signal);
  }
  SGL_REQUIRE(sync != nullptr && seq > 0 && need_back < seq,
              "plan_run: NULL sync words or inconsistent sequence numbers");
  SGL_REQUIRE(front != back, "plan_run: the front and back streams must differ");
  // separate 64-byte lines; sync[48] is the waits' timeout word
  uint32_t *w_back = sync, *w_front = sync + 16, *timeout = sync + 48;
  // the gates and signals go into the parts' first and last kernels where
  // those can take them (fewer launches), else into one-lane kernels
  auto first_takes = [&](const sgl_op *p, int n) { return n > 0 && p[0].kind >= 0 && p[0].kind < kNumOps &&
                                                          kOps[p[0].kind].takes_gate; };
  auto last_takes = [&](const sgl_op *p, int n) { return n > 0 && p[n - 1].kind >= 0 && p[n - 1].kind < kNumOps &&
                                                         kOps[p[n - 1].kind].takes_signal; };
  const sgl::PlanGate g_front{w_back, need_back, timeout};
  // (a signal is folded only into a one-workgroup kernel: a multi-workgroup
  // one would need every workgroup to write back its XCD's L2 first)
  const sgl::PlanSignal s_front{w_front, seq, nullptr};
  const bool fg = first_takes(ops, n_front), fs = last_takes(ops, n_front);
  if (!fg)
    if (int rc = gate(w_back, need_back, timeout, front)) return rc;
  if (int rc = run_ops(ops, n_front, front, 0, t, fg ? g_front : no_gate, fs ? s_front : no_signal)) return rc;
  if (!fs)
    if (int rc = signal(w_front, seq, front)) return rc;
  // The back part's number is stored when the next back part starts (every
  // earlier back-stream kernel is done then): a front part waits for the back
  // part two steps before it, whose number the back part one step before it
  // (submitted earlier) stores. The number stored, seq - 1, is the last one
  // issued before this step (a planned step's or a fence's; a fence stores its
  // own as well).
  if (int rc = signal_gate(seq > 1 ? w_back : nullptr, seq - 1, w_front, seq, timeout, back)) return rc;
  return run_ops(ops + n_front, n_back, back, n_front, t, no_gate, no_signal);
}
