// kh_internal.hpp - host-side interface between the plan executor and the
// kernel families. Each family validates a kh_launch once, at plan creation,
// into an Op that keeps its precomputed kernel arguments; running the op only
// patches the resolved device pointers and launches.
#pragma once

#include <hip/hip_runtime.h>

#include <memory>
#include <string>
#include <vector>

#include "kiln_hip.h"

namespace kh {

struct GemmArgs;

struct Device {
  int id = -1;
  int cus = 256;
  int lds_bytes = 160 * 1024;
  char arch[64] = {0};
};
const Device &current_device();

class Op {
 public:
  virtual ~Op() = default;
  // ptrs[j] = device address of element 0 of ref j (slot pointer + offset).
  // partials: scratch of at least partial_floats() floats shared by every op
  // of the plan (ops run one after another on one stream); null when the op
  // asks for none. Every op writes all the partials it reads back.
  virtual hipError_t launch(float *const *ptrs, float *partials, hipStream_t stream) = 0;
  virtual size_t partial_floats() const { return 0; }
  // GEMV ops: the parsed arguments and kernel choice (for chaining); false
  // for every other family.
  virtual bool gemv_facts(struct GemvFacts &) const { return false; }
};

struct GemvFacts {
  const GemmArgs *args = nullptr;
  int nk_r = 0;       // > 0: the K-contiguous kernel ([N][K] weights) runs it
  bool bf16 = false;  // bf16 weights
};

// Consecutive GEMV launches [first(), end()) of a plan that run as one
// persistent launch (kh_chain.hip). bind() resolves the operands and sets up
// the chain's device state (it allocates); launch() resolves the plan's
// inputs and outputs and launches.
class Chain {
 public:
  virtual ~Chain() = default;
  virtual int first() const = 0;
  virtual int end() const = 0;
  virtual bool active() const = 0;  // bound on a GPU
  virtual int bind(void *const *consts, int n_consts, void *arena, std::string &err) = 0;
  virtual hipError_t launch(void *const *inputs, int n_in, void *const *outputs, int n_out, hipStream_t stream) = 0;
  virtual int timeouts(unsigned long long *out) = 0;
  // Wall-clock ticks (100 MHz) each wait may take; < 0: every wait gives up.
  virtual int set_spin(int64_t ticks) = 0;
};

// The chains of a plan's launches (only GEMV launches marked KH_GEMV_CHAIN
// whose operands allow it; at least two launches each).
std::vector<std::unique_ptr<Chain>> find_chains(const std::vector<kh_launch> &desc,
                                                const std::vector<std::unique_ptr<Op>> &ops);

// bf16 storage (cfg[7] of a ROW, ATTN or GEMM launch): bit j set means ref j
// holds bf16 values, its offset and strides counted in bf16 elements. Each
// family's factory accepts it only where its kernel reads or writes bf16.
inline uint32_t bf16_refs(const kh_launch &L) {
  const bool fam = L.family == KH_FAM_ROW || L.family == KH_FAM_ATTN || L.family == KH_FAM_GEMM;
  return fam ? (uint32_t)L.cfg[7] & ((1u << KH_MAX_REFS) - 1) : 0u;
}

// Pair storage (cfg[7] bit 16 + j of a ROW, ATTN or GEMM launch): ref j holds
// each fp32 value x of a three-pass operand as one 32-bit word, bf16(x) in the
// low half and bf16(x - bf16(x)) in the high half (0 for a non-finite
// bf16(x)): the two halves a three-pass product splits x into, made once by
// the producer. Offsets and strides count words, as for fp32.
inline uint32_t pair_refs(const kh_launch &L) {
  const bool fam = L.family == KH_FAM_ROW || L.family == KH_FAM_ATTN || L.family == KH_FAM_GEMM;
  return fam ? ((uint32_t)L.cfg[7] >> 16) & ((1u << KH_MAX_REFS) - 1) : 0u;
}

// Each factory returns nullptr and sets `err` when the descriptor is invalid or
// unsupported; `unsupported` distinguishes the two for the status code.
std::unique_ptr<Op> make_ew(const kh_launch &L, std::string &err, bool &unsupported);
std::unique_ptr<Op> make_row(const kh_launch &L, std::string &err, bool &unsupported);
std::unique_ptr<Op> make_gemm(const kh_launch &L, std::string &err, bool &unsupported);
std::unique_ptr<Op> make_gemv(const kh_launch &L, std::string &err, bool &unsupported);
std::unique_ptr<Op> make_red(const kh_launch &L, std::string &err, bool &unsupported);
std::unique_ptr<Op> make_attn(const kh_launch &L, std::string &err, bool &unsupported);

// The meaning of launch L, executed on the CPU over host pointers
// (kh_host.hip); false with `err` set for a family it cannot run.
bool run_launch_host(const kh_launch &L, float *const *ptrs, std::string &err);

int gemm_config_count();
bool gemm_config(int id, int32_t out8[8]);

// Measurement probes (kh_probe_attn_timeline, kh_probe_mfma_valu).
hipError_t probe_attn_timeline(const float *q, const float *k, const float *v, float *o, int batch, int tq, int tk,
                               const int64_t *strides8, int nw, float scale, uint64_t *rec, hipStream_t stream,
                               std::string &err);
hipError_t probe_mfma_valu(int chains, int group, int valu, int waves_per_simd, double out2[2], std::string &err);

// Shared descriptor checks.
// Facts about a validated tape range.
struct TapeInfo {
  int slots = 0;          // highest slot used + 1
  int leading_loads = 0;  // LOADs at the start of the range (at most 8)
  uint32_t loaded = 0;    // refs read by LOAD
  uint32_t stored = 0;    // refs written by STORE
};

// Validate tape[begin, end): opcodes, slot numbers, and that LOAD/STORE name
// refs in [first_ref, n_refs) (GEMM epilogues start at ref 2).
bool check_tape(const kh_launch &L, int begin, int end, bool allow_row_ops, TapeInfo &info, std::string &err,
                int first_ref = 0);

}  // namespace kh
