// kh_ew.hip - the elementwise family (K-EW): one fused elementwise DAG (or a
// strided copy) evaluated over one output shape.
//
// Replaces the reference's flat 1-D Triton loop (kiln/gpu/codegen.py:284-310).
// MI355X design:
//   * the host coalesces the iteration space into (outer dims..., inner) and
//     marks every operand whose inner stride is 1 and whose addresses stay
//     16-byte aligned; those move as 128-bit loads/stores (global_load_dwordx4),
//     inner-stride-0 operands (a bias along rows) are one broadcast load;
//   * each thread owns groups of 4 adjacent inner elements, grid-stride over
//     groups; outer indices come from multiply-high division (no int division);
//   * all loads of a group are issued before the tape runs, so a wave keeps
//     every operand's request in flight at once;
//   * the register file size is a template parameter: the host picks the
//     smallest variant that holds the tape, which keeps VGPR use (and so the
//     number of resident waves hiding HBM latency) as high as possible.
#include <algorithm>
#include <cstring>

#include "kh_common.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

constexpr int kEwThreads = 256;

struct EwArgs {
  int32_t n_refs, n_insns, n_pre, outer_rank;
  uint32_t vec_mask, bcast_mask;
  uint32_t inner, groups_per_row, total_groups;
  FastDiv gdiv;
  FastDiv odiv[KH_MAX_RANK];
  float *ptr[KH_MAX_REFS];
  int64_t ostride[KH_MAX_REFS][KH_MAX_RANK];
  int64_t istride[KH_MAX_REFS];
  kh_insn insns[KH_MAX_INSNS];
};

template <int NS>
__global__ __launch_bounds__(kEwThreads) void ew_kernel(const EwArgs a) {
  const uint32_t stride = gridDim.x * kEwThreads;
  for (uint32_t g = blockIdx.x * kEwThreads + threadIdx.x; g < a.total_groups; g += stride) {
    const uint32_t row = fdiv(g, a.gdiv);
    const uint32_t col0 = (g - row * a.groups_per_row) * 4;
    const uint32_t valid = min(4u, a.inner - col0);
    uint32_t idx[KH_MAX_RANK];
    uint32_t rem = row;
#pragma unroll
    for (int d = KH_MAX_RANK - 1; d >= 0; --d) {
      if (d < a.outer_rank) {
        const uint32_t q = fdiv(rem, a.odiv[d]);
        idx[d] = rem - q * a.odiv[d].d;
        rem = q;
      } else {
        idx[d] = 0;
      }
    }
    auto base = [&](int j) {
      int64_t off = 0;
#pragma unroll
      for (int d = 0; d < KH_MAX_RANK; ++d)
        if (d < a.outer_rank) off += (int64_t)idx[d] * a.ostride[j][d];
      return a.ptr[j] + off;
    };
    auto load = [&](int j) -> Vec<4> {
      const float *p = base(j);
      if (a.bcast_mask >> j & 1) return splat4(p[0]);
      Vec<4> out;
      if ((a.vec_mask >> j & 1) && valid == 4) {
        const float4 q = *reinterpret_cast<const float4 *>(p + col0);
        out.v[0] = q.x, out.v[1] = q.y, out.v[2] = q.z, out.v[3] = q.w;
      } else {
        const int64_t st = a.istride[j];
#pragma unroll
        for (int i = 0; i < 4; ++i) out.v[i] = i < (int)valid ? p[(int64_t)(col0 + i) * st] : 0.0f;
      }
      return out;
    };
    auto store = [&](int j, const Vec<4> &v) {
      float *p = base(j);
      if ((a.vec_mask >> j & 1) && valid == 4) {
        *reinterpret_cast<float4 *>(p + col0) = make_float4(v.v[0], v.v[1], v.v[2], v.v[3]);
      } else {
        const int64_t st = a.istride[j];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (i < (int)valid) p[(int64_t)(col0 + i) * st] = v.v[i];
      }
    };
    float f[NS * 4];
    exec_tape<NS>(a.insns, 0, a.n_insns, a.n_pre, f, load, store, [](const kh_insn &, const Vec<4> &) {});
  }
}

class EwOp final : public Op {
 public:
  EwArgs args{};
  int slots = kFastSlots;
  uint32_t vec_candidates = 0;  // refs whose layout allows 128-bit access
  int grid = 1;

  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    EwArgs a = args;
    a.vec_mask = 0;
    for (int j = 0; j < a.n_refs; ++j) {
      a.ptr[j] = ptrs[j];
      if ((vec_candidates >> j & 1) && (reinterpret_cast<uintptr_t>(ptrs[j]) & 15) == 0) a.vec_mask |= 1u << j;
    }
    if (a.total_groups == 0) return hipSuccess;
    if (slots <= kFastSlots) hipLaunchKernelGGL((ew_kernel<kFastSlots>), dim3(grid), dim3(kEwThreads), 0, stream, a);
    else hipLaunchKernelGGL((ew_kernel<KH_NREGS>), dim3(grid), dim3(kEwThreads), 0, stream, a);
    return hipGetLastError();
  }
};

// ---------------------------------------------------------------------------
// Fast path: out = act(a op b) (or act(a)) on a rows x inner space whose
// operands are contiguous along inner, per-row broadcast or a bias row. No
// tape: the op pair is a template, each thread keeps 4 groups of 4 in flight
// (all loads issued first), and registers stay low so waves stay resident.
enum { kFastAdd = 0, kFastSub, kFastMul, kFastNone };
enum { kActNone = 0, kActGeluTanh, kActGeluErf, kActRelu };

struct EwFastArgs {
  const float *a, *b;
  float *out;
  int64_t a_os, b_os, out_os;  // row strides (elements)
  int32_t a_bc, b_bc;          // 1: one value per row (inner stride 0)
  int32_t b_imm, imm_left;     // b is the immediate; the immediate is the left operand
  float imm;
  uint32_t inner4, total4;
  FastDiv div;
};

constexpr int kFastUnroll = 2;

template <int OP, int ACT>
__global__ __launch_bounds__(kEwThreads) void ew_fast_kernel(const EwFastArgs a) {
  const uint32_t stride = gridDim.x * kEwThreads;
  for (uint32_t g0 = blockIdx.x * kEwThreads + threadIdx.x; g0 < a.total4; g0 += stride * kFastUnroll) {
    float4 xa[kFastUnroll], xb[kFastUnroll];
    uint32_t row[kFastUnroll], col[kFastUnroll];
#pragma unroll
    for (int u = 0; u < kFastUnroll; ++u) {
      const uint32_t g = g0 + u * stride;
      row[u] = fdiv(g, a.div);
      col[u] = (g - row[u] * a.inner4) * 4;
      if (g < a.total4) {
        const float *pa = a.a + (int64_t)row[u] * a.a_os;
        if (a.a_bc) {
          const float s = pa[0];
          xa[u] = make_float4(s, s, s, s);
        } else {
          xa[u] = *reinterpret_cast<const float4 *>(pa + col[u]);
        }
        if (OP != kFastNone && !a.b_imm) {
          const float *pb = a.b + (int64_t)row[u] * a.b_os;
          if (a.b_bc) {
            const float s = pb[0];
            xb[u] = make_float4(s, s, s, s);
          } else {
            xb[u] = *reinterpret_cast<const float4 *>(pb + col[u]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kFastUnroll; ++u) {
      const uint32_t g = g0 + u * stride;
      if (g >= a.total4) break;
      float v[4] = {xa[u].x, xa[u].y, xa[u].z, xa[u].w};
      const float w[4] = {xb[u].x, xb[u].y, xb[u].z, xb[u].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float l = v[i], r = a.b_imm ? a.imm : w[i];
        if (a.b_imm && a.imm_left) r = v[i], l = a.imm;
        float x = OP == kFastAdd ? l + r : OP == kFastSub ? l - r : OP == kFastMul ? l * r : v[i];
        if (ACT == kActGeluTanh) x = op_gelu_tanh(x);
        if (ACT == kActGeluErf) x = op_gelu_erf(x);
        if (ACT == kActRelu) x = x != x ? x : fmaxf(x, 0.0f);
        v[i] = x;
      }
      store_stream(a.out + (int64_t)row[u] * a.out_os + col[u], v[0], v[1], v[2], v[3]);
    }
  }
}

class EwFastOp final : public Op {
 public:
  EwFastArgs args{};
  int op = kFastAdd, act = kActNone, ra = 0, rb = -1, ro = 0, grid = 1;
  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    EwFastArgs x = args;
    x.a = ptrs[ra];
    x.b = rb >= 0 ? ptrs[rb] : nullptr;
    x.out = ptrs[ro];
    for (int j : {ra, rb, ro})
      if (j >= 0 && (reinterpret_cast<uintptr_t>(ptrs[j]) & 15) != 0 &&
          !(j == ra && x.a_bc) && !(j == rb && x.b_bc))
        return fallback->launch(ptrs, nullptr, stream);  // unaligned buffer: tape path
    if (x.total4 == 0) return hipSuccess;
#define KH_FAST_CASE(O, A) \
  if (op == O && act == A) hipLaunchKernelGGL((ew_fast_kernel<O, A>), dim3(grid), dim3(kEwThreads), 0, stream, x);
#define KH_FAST_ACTS(O) KH_FAST_CASE(O, kActNone) KH_FAST_CASE(O, kActGeluTanh) KH_FAST_CASE(O, kActGeluErf) \
  KH_FAST_CASE(O, kActRelu)
    KH_FAST_ACTS(kFastAdd)
    KH_FAST_ACTS(kFastSub)
    KH_FAST_ACTS(kFastMul)
    KH_FAST_ACTS(kFastNone)
#undef KH_FAST_ACTS
#undef KH_FAST_CASE
    return hipGetLastError();
  }
  std::unique_ptr<Op> fallback;
};

// Recognise LOAD a; [LOAD b]; [add|sub|mul]; [gelu|relu]; STORE over a space
// that coalesces to (rows, inner) with inner % 4 == 0 and vector-friendly
// operands. Returns nullptr when the descriptor does not qualify.
std::unique_ptr<Op> try_fast_ew(const kh_launch &L, EwOp &generic, int rank, int outer_rank) {
  const EwArgs &g = generic.args;
  if (rank < 1 || outer_rank > 1 || g.inner % 4 != 0 || g.total_groups == 0) return nullptr;
  const kh_insn *t = L.insns;
  int n = L.n_insns, pc = 0;
  int slot_a = -1, slot_b = -1, ra = -1, rb = -1;
  if (pc < n && t[pc].op == KH_OP_LOAD) slot_a = t[pc].dst, ra = t[pc].a, ++pc;
  if (pc < n && t[pc].op == KH_OP_LOAD) slot_b = t[pc].dst, rb = t[pc].a, ++pc;
  if (ra < 0) return nullptr;
  int op = kFastNone, act = kActNone, cur = slot_a;
  bool b_imm = false, imm_left = false;
  float imm = 0.0f;
  if (pc < n && (t[pc].op == KH_OP_ADD || t[pc].op == KH_OP_SUB || t[pc].op == KH_OP_MUL)) {
    const kh_insn &in = t[pc++];
    op = in.op == KH_OP_ADD ? kFastAdd : in.op == KH_OP_SUB ? kFastSub : kFastMul;
    if (slot_b >= 0 && in.a == slot_a && in.b == slot_b) {
    } else if (slot_b >= 0 && in.a == slot_b && in.b == slot_a) {
      std::swap(ra, rb);
      std::swap(slot_a, slot_b);
    } else if (slot_b < 0 && in.a == slot_a && in.b == KH_SRC_IMM) {
      b_imm = true, imm = in.imm;
    } else if (slot_b < 0 && in.b == slot_a && in.a == KH_SRC_IMM) {
      b_imm = true, imm_left = true, imm = in.imm;
    } else {
      return nullptr;
    }
    cur = in.dst;
  } else if (slot_b >= 0) {
    return nullptr;
  }
  if (pc < n && (t[pc].op == KH_OP_GELU_TANH || t[pc].op == KH_OP_GELU_ERF || t[pc].op == KH_OP_RELU ||
                 t[pc].op == KH_OP_MOV)) {
    const kh_insn &in = t[pc++];
    if (in.a != cur) return nullptr;
    act = in.op == KH_OP_GELU_TANH ? kActGeluTanh : in.op == KH_OP_GELU_ERF ? kActGeluErf
                                                    : in.op == KH_OP_RELU ? kActRelu : kActNone;
    cur = in.dst;
  }
  if (pc != n - 1 || t[pc].op != KH_OP_STORE || t[pc].a != cur) return nullptr;
  const int ro = t[pc].dst;
  auto vec = [&](int j) { return (generic.vec_candidates >> j & 1) != 0; };
  auto bc = [&](int j) { return g.istride[j] == 0; };
  if (!vec(ro) || (!vec(ra) && !bc(ra)) || (rb >= 0 && !vec(rb) && !bc(rb))) return nullptr;
  auto fast = std::make_unique<EwFastOp>();
  EwFastArgs &f = fast->args;
  fast->op = op, fast->act = act, fast->ra = ra, fast->rb = rb, fast->ro = ro;
  f.a_os = outer_rank ? g.ostride[ra][0] : 0;
  f.b_os = (rb >= 0 && outer_rank) ? g.ostride[rb][0] : 0;
  f.out_os = outer_rank ? g.ostride[ro][0] : 0;
  f.a_bc = bc(ra);
  f.b_bc = rb >= 0 && bc(rb);
  f.b_imm = b_imm, f.imm_left = imm_left, f.imm = imm;
  f.inner4 = g.inner / 4;
  f.total4 = g.total_groups;
  f.div = make_fastdiv(f.inner4);
  const int64_t blocks = ((int64_t)f.total4 + kEwThreads * kFastUnroll - 1) / (kEwThreads * kFastUnroll);
  // one pass over the data, no grid-stride loop: workgroups start and retire
  // at different times, so reads, arithmetic and writes of different waves
  // overlap (a capped grid moves every phase in lockstep)
  fast->grid = (int)std::max<int64_t>(1, std::min<int64_t>(blocks, (int64_t)1 << 30));
  auto copy = std::make_unique<EwOp>(generic);
  fast->fallback = std::move(copy);
  return fast;
}

}  // namespace

std::unique_ptr<Op> make_ew(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  if (L.rank < 0 || L.rank > KH_MAX_RANK || L.n_refs < 1 || L.n_refs > KH_MAX_REFS) {
    err = "elementwise: bad rank or operand count";
    return nullptr;
  }
  TapeInfo info;
  if (!check_tape(L, 0, L.n_insns, false, info, err)) return nullptr;

  // Coalesce: drop size-1 dims, merge neighbours that are contiguous for every operand.
  int64_t shape[KH_MAX_RANK];
  int64_t strides[KH_MAX_REFS][KH_MAX_RANK];
  int rank = 0;
  for (int d = 0; d < L.rank; ++d) {
    if (L.shape[d] < 0) {
      err = "elementwise: negative extent";
      return nullptr;
    }
    if (L.shape[d] == 1) continue;
    shape[rank] = L.shape[d];
    for (int j = 0; j < L.n_refs; ++j) strides[j][rank] = L.refs[j].strides[d];
    ++rank;
  }
  int64_t numel = 1;
  for (int d = 0; d < rank; ++d) numel *= shape[d];
  if (L.rank > 0 && numel == 0) rank = 0;
  int w = 0;
  for (int d = 0; d < rank; ++d) {
    bool merge = w > 0;
    for (int j = 0; merge && j < L.n_refs; ++j) merge = strides[j][w - 1] == strides[j][d] * shape[d];
    if (merge) {
      shape[w - 1] *= shape[d];
      for (int j = 0; j < L.n_refs; ++j) strides[j][w - 1] = strides[j][d];
    } else {
      shape[w] = shape[d];
      for (int j = 0; j < L.n_refs; ++j) strides[j][w] = strides[j][d];
      ++w;
    }
  }
  rank = w;
  const bool empty = numel == 0;

  auto op = std::make_unique<EwOp>();
  EwArgs &a = op->args;
  a.n_refs = L.n_refs;
  a.n_pre = info.leading_loads;
  a.n_insns = L.n_insns;
  std::memcpy(a.insns, L.insns, sizeof(kh_insn) * L.n_insns);
  const int64_t inner = rank ? shape[rank - 1] : 1;
  const int outer_rank = rank ? rank - 1 : 0;
  const int64_t gpr = (inner + 3) / 4;
  int64_t outer = 1;
  for (int d = 0; d < outer_rank; ++d) outer *= shape[d];
  const int64_t total = empty ? 0 : outer * gpr;
  if (total >= (1ll << 31) || inner >= (1ll << 31)) {
    unsupported = true;
    err = "elementwise: more than 2^31 element groups in one launch";
    return nullptr;
  }
  a.outer_rank = outer_rank;
  a.inner = (uint32_t)inner;
  a.groups_per_row = (uint32_t)gpr;
  a.total_groups = (uint32_t)total;
  a.gdiv = make_fastdiv((uint32_t)std::max<int64_t>(gpr, 1));
  for (int d = 0; d < outer_rank; ++d) a.odiv[d] = make_fastdiv((uint32_t)shape[d]);
  for (int j = 0; j < L.n_refs; ++j) {
    for (int d = 0; d < outer_rank; ++d) a.ostride[j][d] = strides[j][d];
    a.istride[j] = rank ? strides[j][rank - 1] : 0;
    if (a.istride[j] == 0 && info.loaded >> j & 1) a.bcast_mask |= 1u << j;
    bool vec = a.istride[j] == 1 && inner % 4 == 0 && L.refs[j].offset % 4 == 0;
    for (int d = 0; vec && d < outer_rank; ++d) vec = a.ostride[j][d] % 4 == 0;
    if (vec) op->vec_candidates |= 1u << j;
  }
  op->slots = info.slots;
  const int64_t blocks = (total + kEwThreads - 1) / kEwThreads;
  op->grid = (int)std::max<int64_t>(1, std::min<int64_t>(blocks, (int64_t)current_device().cus * 16));
  if (auto fast = try_fast_ew(L, *op, rank, outer_rank)) return fast;
  return op;
}

}  // namespace kh
