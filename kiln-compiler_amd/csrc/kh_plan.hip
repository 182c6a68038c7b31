// kh_plan.hip - the C ABI (include/kiln_hip.h): device setup, plan creation,
// binding, execution, and hipGraph capture/replay.
//
// Replaces the reference's GPUExecutable (kiln/gpu/runtime.py:135-217):
// instead of one Python launch per Triton kernel, a whole compiled graph is
// one plan; kh_plan_run launches every kernel from C++ in one ctypes call,
// and kh_plan_capture records the launches once into a hipGraph that
// kh_plan_replay submits with a single call.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

#include "kh_common.hpp"
#include "kh_internal.hpp"
#include "kiln_hip.h"

// Split-K partials of kh_plan_run_noalloc. Each GPU the library runs on holds
// its own copy of this array, at its own address, until the process ends. In
// host code `scratch` names a host-side stand-in, not device memory: kernels
// and copies get the device address that hipGetSymbolAddress returns for the
// current device, kept in kh::g_scratch (resolved once per device).
static __device__ __align__(256) unsigned char scratch[KH_NOALLOC_WORKSPACE_BYTES];

namespace kh {
namespace {

thread_local std::string g_error;
Device g_device;
bool g_device_ready = false;

int fail(int code, const std::string &msg) {
  g_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(KH_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch[kMaxDevices] = {};

// Device address of `scratch` on `device`, which must be the current device.
int scratch_address(int device, void **out) {
  if (device < 0 || device >= kMaxDevices) return fail(KH_ERR_INVALID, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (p == nullptr) return fail(KH_ERR_HIP, "hipGetSymbolAddress(scratch) returned a null address");
    g_scratch[device] = p;
  }
  *out = g_scratch[device];
  return KH_OK;
}

}  // namespace

const Device &current_device() {
  if (!g_device_ready) {
    int id = 0;
    hipDeviceProp_t prop;
    if (hipGetDevice(&id) == hipSuccess && hipGetDeviceProperties(&prop, id) == hipSuccess) {
      g_device.id = id;
      g_device.cus = prop.multiProcessorCount;
      g_device.lds_bytes = (int)prop.maxSharedMemoryPerMultiProcessor;
      std::snprintf(g_device.arch, sizeof(g_device.arch), "%s", prop.gcnArchName);
      g_device_ready = true;
    }
    (void)hipGetLastError();  // no device (host-only validation): keep MI355X defaults
  }
  return g_device;
}

bool check_tape(const kh_launch &L, int begin, int end, bool allow_row_ops, TapeInfo &info, std::string &err,
                int first_ref) {
  if (L.n_insns < 0 || L.n_insns > KH_MAX_INSNS || begin < 0 || end > L.n_insns || begin > end) {
    err = "tape range outside KH_MAX_INSNS";
    return false;
  }
  auto slot_ok = [](int s) { return s < KH_NREGS || s == KH_SRC_IMM; };
  bool leading = true;
  for (int i = begin; i < end; ++i) {
    const kh_insn &in = L.insns[i];
    if (in.op >= KH_OP_COUNT) {
      err = "tape: unknown opcode " + std::to_string(in.op);
      return false;
    }
    if (!allow_row_ops && (in.op == KH_OP_RSUM || in.op == KH_OP_RMAX)) {
      err = "tape: row reduction outside a row kernel";
      return false;
    }
    if (in.op == KH_OP_LOAD) {
      if (in.a < first_ref || in.a >= L.n_refs || in.dst >= KH_NREGS) {
        err = "tape: LOAD of a missing operand at instruction " + std::to_string(i);
        return false;
      }
      info.loaded |= 1u << in.a;
      info.slots = std::max(info.slots, in.dst + 1);
      if (leading && info.leading_loads < kFastSlots) ++info.leading_loads;
      else leading = false;
      continue;
    }
    leading = false;
    if (in.op == KH_OP_STORE) {
      if (in.dst < first_ref || in.dst >= L.n_refs || in.a >= KH_NREGS) {
        err = "tape: STORE to a missing operand at instruction " + std::to_string(i);
        return false;
      }
      info.stored |= 1u << in.dst;
      info.slots = std::max(info.slots, in.a + 1);
      continue;
    }
    if (in.dst >= KH_NREGS || !slot_ok(in.a) || !slot_ok(in.b)) {
      err = "tape: slot out of range at instruction " + std::to_string(i);
      return false;
    }
    info.slots = std::max(info.slots, in.dst + 1);
    if (in.a < KH_NREGS) info.slots = std::max(info.slots, in.a + 1);
    if (in.b < KH_NREGS) info.slots = std::max(info.slots, in.b + 1);
  }
  if (info.loaded & info.stored) {
    err = "tape: an operand is both loaded and stored";
    return false;
  }
  return true;
}

}  // namespace kh

// The workspace holds the split-K partials, shared by every launch of the
// plan in turn (launches run one after another on one stream).
struct kh_plan {
  std::vector<kh_launch> desc;
  std::vector<std::unique_ptr<kh::Op>> ops;
  std::vector<std::unique_ptr<kh::Chain>> chains;  // persistent GEMV chains over runs of launches
  std::vector<int> chain_start;                    // launch index -> chain starting there, or -1
  size_t ws_needed = 0;
  std::vector<void *> consts;
  void *arena = nullptr;
  void *workspace = nullptr;
  size_t ws_size = 0;
  bool bound = false;
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipStream_t capture_stream = nullptr;
  ~kh_plan() {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    if (capture_stream) (void)hipStreamDestroy(capture_stream);
  }
};

namespace {

using kh::fail;

// Resolve the refs of launch `i` to device pointers.
int resolve(const kh_plan *p, int i, void *const *inputs, int n_in, void *const *outputs, int n_out,
            float **ptrs) {
  const kh_launch &L = p->desc[i];
  for (int j = 0; j < L.n_refs; ++j) {
    const kh_ref &r = L.refs[j];
    void *base = nullptr;
    switch (r.base) {
      case KH_BASE_INPUT:
        if (r.index < 0 || r.index >= n_in) return fail(KH_ERR_INVALID, "launch refers to a missing input");
        base = inputs[r.index];
        break;
      case KH_BASE_OUTPUT:
        if (r.index < 0 || r.index >= n_out) return fail(KH_ERR_INVALID, "launch refers to a missing output");
        base = outputs[r.index];
        break;
      case KH_BASE_CONST:
        if (r.index < 0 || r.index >= (int)p->consts.size())
          return fail(KH_ERR_INVALID, "launch refers to a missing constant");
        base = p->consts[r.index];
        break;
      case KH_BASE_ARENA: base = p->arena; break;
      case KH_BASE_WORKSPACE: base = p->workspace; break;
      default: return fail(KH_ERR_INVALID, "bad operand base");
    }
    if (base == nullptr) return fail(KH_ERR_INVALID, std::string("null device pointer for an operand of ") + L.name);
    ptrs[j] = (kh::bf16_refs(L) >> j & 1) ? reinterpret_cast<float *>(static_cast<uint16_t *>(base) + r.offset)
                                         : static_cast<float *>(base) + r.offset;
  }
  return KH_OK;
}

// Run launches [begin, end) with `workspace` (at least p->ws_needed bytes)
// holding the split-K partials.
int run_range(kh_plan *p, int begin, int end, void *const *inputs, int n_in, void *const *outputs, int n_out,
              hipStream_t stream, void *workspace) {
  if (!p->bound) return fail(KH_ERR_INVALID, "plan is not bound (call kh_plan_bind)");
  if (p->ws_needed && !workspace)
    return fail(KH_ERR_CAPACITY, "plan needs a workspace of " + std::to_string(p->ws_needed) +
                                     " bytes: bind one (kh_plan_bind) or run it with kh_plan_run_noalloc");
  float *ptrs[KH_MAX_REFS];
  for (int i = begin; i < end;) {
    // a chain the range covers whole runs as its one launch
    const int c = p->chain_start[i];
    if (c >= 0 && p->chains[c]->active() && p->chains[c]->end() <= end) {
      const hipError_t e = p->chains[c]->launch(inputs, n_in, outputs, n_out, stream);
      if (e != hipSuccess) return kh::hip_fail(e, "GEMV chain");
      i = p->chains[c]->end();
      continue;
    }
    const int rc = resolve(p, i, inputs, n_in, outputs, n_out, ptrs);
    if (rc != KH_OK) return rc;
    float *partials = p->ops[i]->partial_floats() ? static_cast<float *>(workspace) : nullptr;
    const hipError_t e = p->ops[i]->launch(ptrs, partials, stream);
    if (e != hipSuccess) return kh::hip_fail(e, p->desc[i].name);
    ++i;
  }
  return KH_OK;
}

}  // namespace

extern "C" {

int kh_version(void) { return KH_ABI_VERSION; }

#ifndef KH_BUILD_ID
#define KH_BUILD_ID "unversioned"
#endif
const char *kh_build_id(void) { return KH_BUILD_ID; }

int kh_abi_sizes(size_t *sizes4) {
  if (!sizes4) return fail(KH_ERR_INVALID, "null argument");
  sizes4[0] = sizeof(kh_launch);
  sizes4[1] = sizeof(kh_ref);
  sizes4[2] = sizeof(kh_insn);
  sizes4[3] = sizeof(kh_pass);
  return KH_OK;
}

const char *kh_last_error(void) { return kh::g_error.c_str(); }

int kh_init(int device) {
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(KH_ERR_NO_DEVICE, "no HIP device is visible");
  }
  if (device < 0 || device >= n) return fail(KH_ERR_INVALID, "device index out of range");
  if ((e = hipSetDevice(device)) != hipSuccess) return kh::hip_fail(e, "hipSetDevice");
  hipDeviceProp_t prop;
  if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return kh::hip_fail(e, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(KH_ERR_NO_DEVICE, std::string("libkiln_hip is built for gfx950, device is ") + prop.gcnArchName);
  kh::g_device.id = device;
  kh::g_device.cus = prop.multiProcessorCount;
  kh::g_device.lds_bytes = (int)prop.maxSharedMemoryPerMultiProcessor;
  std::snprintf(kh::g_device.arch, sizeof(kh::g_device.arch), "%s", prop.gcnArchName);
  kh::g_device_ready = true;
  void *ws = nullptr;
  return kh::scratch_address(device, &ws);  // once per device, with that device current
}

int kh_device_info(int *cus, int *lds_bytes, char *arch, int arch_len) {
  const kh::Device &d = kh::current_device();
  if (cus) *cus = d.cus;
  if (lds_bytes) *lds_bytes = d.lds_bytes;
  if (arch && arch_len > 0) std::snprintf(arch, arch_len, "%s", d.arch[0] ? d.arch : "gfx950");
  return KH_OK;
}

int kh_gemm_config_count(void) { return kh::gemm_config_count(); }

int kh_gemm_config(int id, int32_t *out8) {
  if (!out8 || !kh::gemm_config(id, out8)) return fail(KH_ERR_INVALID, "unknown GEMM configuration");
  return KH_OK;
}

int kh_plan_create(const kh_launch *launches, int n_launches, kh_plan **out) {
  if (!out || n_launches < 0 || (n_launches > 0 && !launches)) return fail(KH_ERR_INVALID, "bad arguments");
  *out = nullptr;
  auto p = std::make_unique<kh_plan>();
  p->desc.assign(launches, launches + n_launches);
  for (int i = 0; i < n_launches; ++i) {
    const kh_launch &L = p->desc[i];
    std::string err;
    bool unsupported = false;
    std::unique_ptr<kh::Op> op;
    if (L.n_refs < 0 || L.n_refs > KH_MAX_REFS) {
      err = "bad operand count";
    } else {
      switch (L.family) {
        case KH_FAM_EW: op = kh::make_ew(L, err, unsupported); break;
        case KH_FAM_ROW: op = kh::make_row(L, err, unsupported); break;
        case KH_FAM_GEMM: op = kh::make_gemm(L, err, unsupported); break;
        case KH_FAM_GEMV: op = kh::make_gemv(L, err, unsupported); break;
        case KH_FAM_RED: op = kh::make_red(L, err, unsupported); break;
        case KH_FAM_ATTN: op = kh::make_attn(L, err, unsupported); break;
        default: err = "unknown kernel family " + std::to_string(L.family);
      }
    }
    if (!op) {
      char name[40];
      std::snprintf(name, sizeof(name), "%.32s", L.name);
      return fail(unsupported ? KH_ERR_UNSUPPORTED : KH_ERR_INVALID,
                  std::string("launch ") + std::to_string(i) + " (" + name + "): " + err);
    }
    p->ops.push_back(std::move(op));
  }
  size_t partials = 0;
  for (auto &op : p->ops) partials = std::max(partials, op->partial_floats());
  p->ws_needed = partials * sizeof(float);
  p->chains = kh::find_chains(p->desc, p->ops);
  p->chain_start.assign(p->desc.size(), -1);
  for (int c = 0; c < (int)p->chains.size(); ++c) p->chain_start[p->chains[c]->first()] = c;
  *out = p.release();
  return KH_OK;
}

int kh_plan_workspace_bytes(const kh_plan *plan, size_t *bytes) {
  if (!plan || !bytes) return fail(KH_ERR_INVALID, "bad arguments");
  *bytes = plan->ws_needed;
  return KH_OK;
}

int kh_plan_bind(kh_plan *plan, void *const *consts, int n_consts, void *arena, void *workspace,
                 size_t workspace_bytes) {
  if (!plan || n_consts < 0 || (n_consts > 0 && !consts)) return fail(KH_ERR_INVALID, "bad arguments");
  const bool none = workspace == nullptr && workspace_bytes == 0;  // kh_plan_run_noalloc callers
  if (!none && workspace_bytes < plan->ws_needed)
    return fail(KH_ERR_CAPACITY, "workspace of " + std::to_string(workspace_bytes) + " bytes, plan needs " +
                                     std::to_string(plan->ws_needed));
  if (!none && plan->ws_needed && !workspace) return fail(KH_ERR_INVALID, "plan needs a workspace");
  plan->consts.assign(consts, consts + n_consts);
  plan->arena = arena;
  plan->workspace = workspace;
  plan->ws_size = workspace_bytes;
  plan->bound = true;
  // chains bind their device state here; one that cannot (no GPU: a plan
  // bound for kh_plan_run_host) stays inactive and its launches run one by one
  for (auto &c : plan->chains) {
    std::string err;
    (void)c->bind(consts, n_consts, arena, err);
  }
  return KH_OK;
}

int kh_plan_chains(const kh_plan *plan, int32_t *ranges, int max_chains, int *n_chains) {
  if (!plan || !n_chains || max_chains < 0 || (max_chains > 0 && !ranges)) return fail(KH_ERR_INVALID, "bad arguments");
  *n_chains = (int)plan->chains.size();
  for (int c = 0; c < std::min(max_chains, *n_chains); ++c) {
    const kh::Chain &ch = *plan->chains[c];
    ranges[3 * c] = ch.first();
    ranges[3 * c + 1] = ch.end() - ch.first();
    ranges[3 * c + 2] = ch.active() ? 1 : 0;
  }
  return KH_OK;
}

int kh_plan_chain_timeouts(kh_plan *plan, uint64_t *timeouts) {
  if (!plan || !timeouts) return fail(KH_ERR_INVALID, "bad arguments");
  *timeouts = 0;
  for (auto &c : plan->chains) {
    unsigned long long n = 0;
    if (c->timeouts(&n) != KH_OK) return fail(KH_ERR_HIP, "reading a chain's state");
    *timeouts += n;
  }
  return KH_OK;
}

int kh_plan_chain_spin(kh_plan *plan, int64_t ticks) {
  if (!plan) return fail(KH_ERR_INVALID, "null plan");
  for (auto &c : plan->chains)
    if (c->set_spin(ticks) != KH_OK) return fail(KH_ERR_HIP, "writing a chain's state");
  return KH_OK;
}

int kh_plan_run(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs,
                void *stream) {
  if (!plan) return fail(KH_ERR_INVALID, "null plan");
  return run_range(plan, 0, (int)plan->ops.size(), inputs, n_inputs, outputs, n_outputs,
                   static_cast<hipStream_t>(stream), plan->workspace);
}

int kh_plan_run_noalloc(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs,
                        void *stream) {
  if (!plan) return fail(KH_ERR_INVALID, "null plan");
  if (plan->ws_needed > KH_NOALLOC_WORKSPACE_BYTES)
    return fail(KH_ERR_CAPACITY, "plan needs a workspace of " + std::to_string(plan->ws_needed) +
                                     " bytes, more than kh_plan_run_noalloc's " +
                                     std::to_string((size_t)KH_NOALLOC_WORKSPACE_BYTES));
  int device = 0;
  const hipError_t e = hipGetDevice(&device);
  if (e != hipSuccess) return kh::hip_fail(e, "hipGetDevice");
  void *ws = nullptr;
  const int rc = kh::scratch_address(device, &ws);
  if (rc != KH_OK) return rc;
  return run_range(plan, 0, (int)plan->ops.size(), inputs, n_inputs, outputs, n_outputs,
                   static_cast<hipStream_t>(stream), ws);
}

int kh_plan_run_host(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs) {
  if (!plan) return fail(KH_ERR_INVALID, "null plan");
  if (!plan->bound) return fail(KH_ERR_INVALID, "plan is not bound (call kh_plan_bind)");
  float *ptrs[KH_MAX_REFS];
  for (int i = 0; i < (int)plan->desc.size(); ++i) {
    const int rc = resolve(plan, i, inputs, n_inputs, outputs, n_outputs, ptrs);
    if (rc != KH_OK) return rc;
    std::string err;
    if (!kh::run_launch_host(plan->desc[i], ptrs, err)) return fail(KH_ERR_UNSUPPORTED, err);
  }
  return KH_OK;
}

int kh_plan_run_one(kh_plan *plan, int index, void *const *inputs, int n_inputs, void *const *outputs,
                    int n_outputs, void *stream) {
  if (!plan || index < 0 || index >= (int)plan->ops.size()) return fail(KH_ERR_INVALID, "bad launch index");
  return run_range(plan, index, index + 1, inputs, n_inputs, outputs, n_outputs, static_cast<hipStream_t>(stream),
                   plan->workspace);
}

int kh_plan_capture(kh_plan *plan, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs) {
  if (!plan) return fail(KH_ERR_INVALID, "null plan");
  hipError_t e;
  if (plan->exec) {
    (void)hipGraphExecDestroy(plan->exec);
    plan->exec = nullptr;
  }
  if (plan->graph) {
    (void)hipGraphDestroy(plan->graph);
    plan->graph = nullptr;
  }
  if (!plan->capture_stream && (e = hipStreamCreateWithFlags(&plan->capture_stream, hipStreamNonBlocking)) != hipSuccess)
    return kh::hip_fail(e, "hipStreamCreateWithFlags");
  if ((e = hipStreamBeginCapture(plan->capture_stream, hipStreamCaptureModeThreadLocal)) != hipSuccess)
    return kh::hip_fail(e, "hipStreamBeginCapture");
  const int rc = run_range(plan, 0, (int)plan->ops.size(), inputs, n_inputs, outputs, n_outputs, plan->capture_stream,
                           plan->workspace);
  hipGraph_t g = nullptr;
  e = hipStreamEndCapture(plan->capture_stream, &g);
  if (rc != KH_OK) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (e != hipSuccess) return kh::hip_fail(e, "hipStreamEndCapture");
  plan->graph = g;
  if ((e = hipGraphInstantiate(&plan->exec, g, nullptr, nullptr, 0)) != hipSuccess)
    return kh::hip_fail(e, "hipGraphInstantiate");
  return KH_OK;
}

namespace {

// Owns the graph, executable and events of one kh_plan_time call.
struct TimingGraph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  hipEvent_t start = nullptr, stop = nullptr;
  ~TimingGraph() {
    if (start) (void)hipEventDestroy(start);
    if (stop) (void)hipEventDestroy(stop);
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
  }
};

}  // namespace

int kh_plan_time(kh_plan *plan, int index, void *const *inputs, int n_inputs, void *const *outputs, int n_outputs,
                 int repeats, int rounds, void *stream, double *seconds) {
  if (!plan || !seconds) return fail(KH_ERR_INVALID, "null argument");
  const int n = (int)plan->ops.size();
  if (index < -1 || index >= n) return fail(KH_ERR_INVALID, "bad launch index");
  if (repeats < 1 || repeats > 4096 || rounds < 1 || rounds > 64)
    return fail(KH_ERR_INVALID, "repeats must be 1..4096 and rounds 1..64");
  const int begin = index < 0 ? 0 : index, end = index < 0 ? n : index + 1;
  hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  // two launches outside the graph first (first-launch costs, caches)
  for (int w = 0; w < 2; ++w) {
    const int rc = run_range(plan, begin, end, inputs, n_inputs, outputs, n_outputs, s, plan->workspace);
    if (rc != KH_OK) return rc;
  }
  if (!plan->capture_stream && (e = hipStreamCreateWithFlags(&plan->capture_stream, hipStreamNonBlocking)) != hipSuccess)
    return kh::hip_fail(e, "hipStreamCreateWithFlags");
  TimingGraph t;
  if ((e = hipStreamBeginCapture(plan->capture_stream, hipStreamCaptureModeThreadLocal)) != hipSuccess)
    return kh::hip_fail(e, "hipStreamBeginCapture");
  int rc = KH_OK;
  for (int r = 0; r < repeats && rc == KH_OK; ++r)
    rc = run_range(plan, begin, end, inputs, n_inputs, outputs, n_outputs, plan->capture_stream, plan->workspace);
  e = hipStreamEndCapture(plan->capture_stream, &t.graph);
  if (rc != KH_OK) return rc;
  if (e != hipSuccess) return kh::hip_fail(e, "hipStreamEndCapture");
  if ((e = hipGraphInstantiate(&t.exec, t.graph, nullptr, nullptr, 0)) != hipSuccess)
    return kh::hip_fail(e, "hipGraphInstantiate");
  if ((e = hipEventCreate(&t.start)) != hipSuccess || (e = hipEventCreate(&t.stop)) != hipSuccess)
    return kh::hip_fail(e, "hipEventCreate");
  if ((e = hipGraphLaunch(t.exec, s)) != hipSuccess) return kh::hip_fail(e, "hipGraphLaunch");  // warm-up replay
  float best = 0.0f;
  for (int r = 0; r < rounds; ++r) {
    float ms = 0.0f;
    if ((e = hipEventRecord(t.start, s)) != hipSuccess || (e = hipGraphLaunch(t.exec, s)) != hipSuccess ||
        (e = hipEventRecord(t.stop, s)) != hipSuccess || (e = hipEventSynchronize(t.stop)) != hipSuccess ||
        (e = hipEventElapsedTime(&ms, t.start, t.stop)) != hipSuccess)
      return kh::hip_fail(e, "timing replay");
    if (r == 0 || ms < best) best = ms;
  }
  *seconds = (double)best * 1e-3 / repeats;
  return KH_OK;
}

int kh_plan_replay(kh_plan *plan, void *stream) {
  if (!plan || !plan->exec) return fail(KH_ERR_INVALID, "plan has no captured graph");
  const hipError_t e = hipGraphLaunch(plan->exec, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return kh::hip_fail(e, "hipGraphLaunch");
  return KH_OK;
}

int kh_plan_destroy(kh_plan *plan) {
  delete plan;
  return KH_OK;
}

int kh_probe_attn_timeline(const float *q, const float *k, const float *v, float *out, int batch, int tq, int tk,
                           const int64_t *strides8, int waves, float scale, uint64_t *rec, void *stream) {
  std::string err;
  const hipError_t e = kh::probe_attn_timeline(q, k, v, out, batch, tq, tk, strides8, waves, scale, rec,
                                               (hipStream_t)stream, err);
  if (e == hipErrorInvalidValue && !err.empty()) return fail(KH_ERR_INVALID, err);
  if (e != hipSuccess) return kh::hip_fail(e, "kh_probe_attn_timeline");
  return KH_OK;
}

int kh_probe_mfma_valu(int chains, int group, int valu, int waves_per_simd, double *out2) {
  std::string err;
  const hipError_t e = kh::probe_mfma_valu(chains, group, valu, waves_per_simd, out2, err);
  if (e == hipErrorInvalidValue && !err.empty()) return fail(KH_ERR_INVALID, err);
  if (e != hipSuccess) return fail(KH_ERR_HIP, err.empty() ? std::string("kh_probe_mfma_valu") : err);
  return KH_OK;
}

}  // extern "C"
