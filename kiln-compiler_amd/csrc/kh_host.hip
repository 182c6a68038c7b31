// kh_host.hip - the meaning of every kernel family, executed on the CPU.
//
// kh_plan_run_host runs a plan's launches one after another over host memory,
// element by element, straight from the kh_launch descriptors: operand
// addressing (element offset + sum of index x stride, stride 0 = broadcast),
// instruction tapes (the same op_scalar the GPU kernels use,
// kh_semantics.hpp), row passes with their reductions, K-RED, GEMM / GEMV
// with their prologues and epilogue tapes (bf16 inputs rounded as the MFMA
// variants round them), and attention. It is the counterpart of the
// reference's interpreter switch (kiln/gpu/runtime.py:39-50, Triton's
// TRITON_INTERPRET), there for the CPU test suite: it checks the lowering's
// descriptors and tapes against the oracle without a GPU. It is a test
// instrument, never a fallback: nothing on the GPU path calls it.
//
// Products and attention accumulate in double; results are rounded to float
// once. The GPU kernels accumulate in fp32 in their own order, so the two
// agree to rounding, not bit for bit.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <string>
#include <vector>

#include "kh_internal.hpp"
#include "kh_semantics.hpp"
#include "kiln_hip.h"

namespace kh {
namespace {

constexpr float kNaN = std::numeric_limits<float>::quiet_NaN();

// Odometer over an index space of up to KH_MAX_RANK dims.
struct Odometer {
  int rank;
  int64_t shape[KH_MAX_RANK];
  int64_t idx[KH_MAX_RANK];
  bool done;

  Odometer(int r, const int64_t *s) : rank(r), done(false) {
    for (int d = 0; d < KH_MAX_RANK; ++d) shape[d] = d < r ? s[d] : 1, idx[d] = 0;
    for (int d = 0; d < r; ++d)
      if (shape[d] <= 0) done = true;
  }
  void next() {
    for (int d = rank - 1; d >= 0; --d) {
      if (++idx[d] < shape[d]) return;
      idx[d] = 0;
    }
    done = true;
  }
};

inline int64_t offset_of(const kh_ref &r, const int64_t *idx, int rank) {
  int64_t off = 0;
  for (int d = 0; d < rank; ++d) off += idx[d] * r.strides[d];
  return off;
}

// float -> bf16 -> float, round to nearest even; NaN stays NaN.
inline float bf16_round(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return x;
  u = (u + (((u >> 16) & 1u) + 0x7FFFu)) & 0xFFFF0000u;
  float y;
  std::memcpy(&y, &u, 4);
  return y;
}

inline float bf16_value(uint16_t bits) {
  const uint32_t u = (uint32_t)bits << 16;
  float y;
  std::memcpy(&y, &u, 4);
  return y;
}

inline uint16_t bf16_bits(float x) {
  uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);   // NaN stays (quiet) NaN
  return (uint16_t)((u + (((u >> 16) & 1u) + 0x7FFFu)) >> 16);
}

// Operand j at element `off`: fp32, or bf16 when the launch stores it as
// bf16 (kh_launch.cfg[7]), read widened and written rounded to nearest even
// as the kernels do.
struct Operands {
  float *const *p;
  uint32_t m16;
  Operands(const kh_launch &L, float *const *ptrs) : p(ptrs), m16(bf16_refs(L)) {}
  float ld(int j, int64_t off) const {
    return (m16 >> j & 1) ? bf16_value(reinterpret_cast<const uint16_t *>(p[j])[off]) : p[j][off];
  }
  void st(int j, int64_t off, float v) const {
    if (m16 >> j & 1) reinterpret_cast<uint16_t *>(p[j])[off] = bf16_bits(v);
    else p[j][off] = v;
  }
};

// Runs tape[begin, end) on `slot` at one element. load(j) / store(j, v) read
// and write operand j at that element; reduce(insn, v) handles RSUM / RMAX.
// Returns the mask of slots the range wrote.
template <class Load, class Store, class Reduce>
uint32_t run_tape(const kh_launch &L, int begin, int end, float *slot, Load &&load, Store &&store,
                  Reduce &&reduce) {
  uint32_t written = 0;
  auto value = [&](int s, float imm) { return s == KH_SRC_IMM ? imm : slot[s]; };
  for (int pc = begin; pc < end; ++pc) {
    const kh_insn &in = L.insns[pc];
    switch (in.op) {
      case KH_OP_LOAD:
        slot[in.dst] = load(in.a);
        written |= 1u << in.dst;
        break;
      case KH_OP_STORE: store(in.dst, value(in.a, in.imm)); break;
      case KH_OP_RSUM:
      case KH_OP_RMAX: reduce(in, value(in.a, in.imm)); break;
      default:
        slot[in.dst] = op_scalar(in.op, value(in.a, in.imm), value(in.b, in.imm));
        written |= 1u << in.dst;
    }
  }
  return written;
}

// -- elementwise ------------------------------------------------------------------

void host_ew(const kh_launch &L, float *const *p) {
  float slot[KH_NREGS] = {0};
  for (Odometer o(L.rank, L.shape); !o.done; o.next()) {
    run_tape(
        L, 0, L.n_insns, slot, [&](int j) { return p[j][offset_of(L.refs[j], o.idx, L.rank)]; },
        [&](int j, float v) { p[j][offset_of(L.refs[j], o.idx, L.rank)] = v; }, [](const kh_insn &, float) {});
  }
}

// -- rows -----------------------------------------------------------------------------

void host_row(const kh_launch &L, float *const *p) {
  const Operands mem(L, p);
  const int rank = L.rank;
  const int64_t inner = rank > 0 ? L.shape[rank - 1] : 1;
  int64_t row_shape[KH_MAX_RANK];
  for (int d = 0; d < rank - 1; ++d) row_shape[d] = L.shape[d];
  std::vector<float> cols((size_t)std::max<int64_t>(inner, 1) * KH_NREGS);
  for (Odometer o(rank - 1, row_shape); !o.done; o.next()) {
    int64_t idx[KH_MAX_RANK] = {0};
    for (int d = 0; d < rank - 1; ++d) idx[d] = o.idx[d];
    std::fill(cols.begin(), cols.end(), 0.0f);
    for (int pi = 0; pi < L.n_passes; ++pi) {
      const kh_pass &P = L.passes[pi];
      float acc[KH_NREGS] = {0};
      for (int s = 0; s < KH_NREGS; ++s)
        if (P.acc_mask >> s & 1) acc[s] = (P.max_mask >> s & 1) ? -INFINITY : 0.0f;
      uint32_t vec_written = 0;
      for (int64_t c = 0; c < inner; ++c) {
        idx[rank - 1] = c;
        float *slot = &cols[(size_t)c * KH_NREGS];
        vec_written |= run_tape(
            L, P.vec_begin, P.vec_end, slot, [&](int j) { return mem.ld(j, offset_of(L.refs[j], idx, rank)); },
            [&](int j, float v) { mem.st(j, offset_of(L.refs[j], idx, rank), v); },
            [&](const kh_insn &in, float x) {
              acc[in.dst] = in.op == KH_OP_RSUM ? acc[in.dst] + x : nan_max(acc[in.dst], x);
            });
      }
      // a chunked row recomputes per-column values in every pass: poison
      // what this pass computed per column so that a later read of it shows
      if (!P.single_chunk)
        for (int64_t c = 0; c < inner; ++c)
          for (int s = 0; s < KH_NREGS; ++s)
            if ((vec_written >> s & 1) && !(P.acc_mask >> s & 1)) cols[(size_t)c * KH_NREGS + s] = kNaN;
      // the row's reductions and its per-row scalar work, then every column sees them
      float row[KH_NREGS];
      std::memcpy(row, inner > 0 ? &cols[0] : cols.data(), sizeof(row));
      uint32_t uniform = 0;
      for (int s = 0; s < KH_NREGS; ++s)
        if (P.acc_mask >> s & 1) row[s] = acc[s], uniform |= 1u << s;
      idx[rank - 1] = 0;
      uniform |= run_tape(
          L, P.post_begin, P.post_end, row, [&](int j) { return mem.ld(j, offset_of(L.refs[j], idx, rank - 1)); },
          [&](int j, float v) { mem.st(j, offset_of(L.refs[j], idx, rank - 1), v); }, [](const kh_insn &, float) {});
      for (int64_t c = 0; c < std::max<int64_t>(inner, 1); ++c)
        for (int s = 0; s < KH_NREGS; ++s)
          if (uniform >> s & 1) cols[(size_t)c * KH_NREGS + s] = row[s];
    }
  }
}

// -- reductions over other dims ---------------------------------------------------------

void host_red(const kh_launch &L, float *const *p) {
  const uint32_t mask = (uint32_t)L.cfg[0];
  const bool is_max = L.cfg[1] != 0;
  int64_t kept[KH_MAX_RANK];
  for (int d = 0; d < L.rank; ++d) kept[d] = (mask >> d & 1) ? 1 : L.shape[d];
  for (Odometer o(L.rank, kept); !o.done; o.next())
    p[1][offset_of(L.refs[1], o.idx, L.rank)] = is_max ? -INFINITY : 0.0f;
  for (Odometer o(L.rank, L.shape); !o.done; o.next()) {
    float &out = p[1][offset_of(L.refs[1], o.idx, L.rank)];
    const float v = p[0][offset_of(L.refs[0], o.idx, L.rank)];
    out = is_max ? nan_max(out, v) : out + v;
  }
}

// -- attention ---------------------------------------------------------------------------

// out[d] = sum_j softmax_j(s_j) v_j[d] for one query; s_j from q . k_j, the
// scale mode and the mask mode. Fully masked rows give NaN, as eager does.
// bf16 products (bf): q and k rounded to bf16 for the scores, the softmax
// weights and v rounded to bf16 for the weighted sum (the two products of an
// unfused attention whose matmuls take bf16 inputs).
void attend(int64_t tk, int64_t dh, int scale_mode, float scale, int mask_mode, int64_t query,
            const float *q, int64_t q_sd, const float *k, int64_t k_sj, int64_t k_sd, const float *v, int64_t v_sj,
            int64_t v_sd, const float *mask, int64_t mask_sj, double *out, int prec = 0) {
  // one product of the two matmuls: fp32 inputs, bf16-rounded inputs, or the
  // three-pass sum lo.hi + hi.lo + hi.hi of the bf16 halves (a non-finite hi
  // keeps lo 0)
  auto prod = [prec](float x, float y) -> double {
    if (prec == 0) return (double)x * (double)y;
    const float xh = bf16_round(x), yh = bf16_round(y);
    if (prec == 1) return (double)xh * (double)yh;
    const float xl = std::isfinite(xh) ? bf16_round(x - xh) : 0.0f, yl = std::isfinite(yh) ? bf16_round(y - yh) : 0.0f;
    return (double)xl * yh + (double)xh * yl + (double)xh * yh;
  };
  std::vector<double> s((size_t)tk);
  double m = -INFINITY;
  for (int64_t j = 0; j < tk; ++j) {
    float dot = 0.0f;
    double acc = 0.0;
    for (int64_t d = 0; d < dh; ++d) acc += prod(q[d * q_sd], k[j * k_sj + d * k_sd]);
    dot = (float)acc;
    if (scale_mode == KH_ATTN_SCALE_MUL) dot *= scale;
    if (scale_mode == KH_ATTN_SCALE_DIV) dot /= scale;
    if (mask_mode == KH_ATTN_MASK_CAUSAL && j > query) dot = -INFINITY;
    if (mask_mode == KH_ATTN_MASK_ADD) dot += mask[j * mask_sj];
    s[j] = dot;
    m = (dot != dot || m != m) ? NAN : std::max(m, (double)dot);
  }
  double l = 0.0;
  for (int64_t j = 0; j < tk; ++j) l += (s[j] = std::exp(s[j] - m));
  // bf16 and three-pass products take the normalised weights in fp32, as the
  // unfused softmax hands them to its matmul
  for (int64_t d = 0; d < dh; ++d) {
    double acc = 0.0;
    for (int64_t j = 0; j < tk; ++j)
      acc += prec ? prod((float)(s[j] / l), v[j * v_sj + d * v_sd]) : s[j] * (double)v[j * v_sj + d * v_sd];
    out[d] = prec ? acc : acc / l;
  }
}

void host_attn(const kh_launch &L, float *const *p0) {
  const int64_t batch = L.gemm[0], tq = L.gemm[1], tk = L.gemm[2], dh = L.gemm[3];
  const kh_ref &Q = L.refs[0], &K = L.refs[1], &V = L.refs[2], &O = L.refs[3];
  std::vector<double> out((size_t)dh);
  // q, k, v stored as bf16: widened copies of the elements the refs reach
  std::vector<float> wide[3];
  float *p[KH_MAX_REFS];
  for (int j = 0; j < KH_MAX_REFS; ++j) p[j] = p0[j];
  const uint32_t m16 = bf16_refs(L);
  for (int j = 0; j < 3; ++j) {
    if (!(m16 >> j & 1)) continue;
    const kh_ref &r = L.refs[j];
    const int64_t rows = j == 0 ? tq : tk;
    const int64_t span = (batch - 1) * r.strides[0] + (rows - 1) * r.strides[1] + (dh - 1) * r.strides[2] + 1;
    wide[j].resize((size_t)std::max<int64_t>(span, 0));
    const uint16_t *src = reinterpret_cast<const uint16_t *>(p0[j]);
    for (int64_t i = 0; i < span; ++i) wide[j][(size_t)i] = bf16_value(src[i]);
    p[j] = wide[j].data();
  }
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t i = 0; i < tq; ++i) {
      const float *mask = L.cfg[0] == KH_ATTN_MASK_ADD ? p[4] + b * L.refs[4].strides[0] + i * L.refs[4].strides[1]
                                                       : nullptr;
      attend(tk, dh, L.cfg[1], L.fparams[0], L.cfg[0], i, p[0] + b * Q.strides[0] + i * Q.strides[1], Q.strides[2],
             p[1] + b * K.strides[0], K.strides[1], K.strides[2], p[2] + b * V.strides[0], V.strides[1], V.strides[2],
             mask, mask ? L.refs[4].strides[2] : 0, out.data(), L.cfg[5]);
      for (int64_t d = 0; d < dh; ++d)
        Operands(L, p).st(3, b * O.strides[0] + i * O.strides[1] + d * O.strides[2], (float)out[d]);
    }
}

// -- matrix products ----------------------------------------------------------------------

// The A row (b, m, 0..K) the product reads: A itself, or what a prologue
// makes of it (a GEMV's LayerNorm of the row, or one query's head-merged
// attention; a GEMM's LayerNorm prologue only normalises, (x - mean) * rstd:
// its gamma and beta are folded into B and a per-column constant).
void a_row(const kh_launch &L, float *const *p, int64_t b, int64_t m, std::vector<float> &row) {
  const int64_t K = L.gemm[3];
  const kh_ref &A = L.refs[0];
  const bool gemv = L.family == KH_FAM_GEMV;
  if (gemv && L.cfg[4] == KH_GEMV_PRO_ATTN) {
    const int64_t dh = L.cfg[0], heads = K / dh, tk = L.cfg[7];
    const int j = L.cfg[5];
    const kh_ref &Q = L.refs[j], &Kr = L.refs[j + 1], &V = L.refs[j + 2];
    const int mask_mode = L.cfg[6] & 3, scale_mode = L.cfg[6] >> 2;
    std::vector<double> out((size_t)dh);
    for (int64_t h = 0; h < heads; ++h) {
      const float *mask = mask_mode == KH_ATTN_MASK_ADD ? p[j + 3] + h * L.refs[j + 3].strides[0] : nullptr;
      attend(tk, dh, scale_mode, L.fparams[0], mask_mode, 0, p[j] + h * Q.strides[0], Q.strides[2],
             p[j + 1] + h * Kr.strides[0], Kr.strides[1], Kr.strides[2], p[j + 2] + h * V.strides[0], V.strides[1],
             V.strides[2], mask, mask ? L.refs[j + 3].strides[2] : 0, out.data());
      for (int64_t d = 0; d < dh; ++d) row[(size_t)(h * dh + d)] = (float)out[d];
    }
    return;
  }
  const Operands mem(L, p);
  for (int64_t k = 0; k < K; ++k) row[(size_t)k] = mem.ld(0, b * A.strides[0] + m * A.strides[1] + k * A.strides[2]);
  if (L.cfg[4] == KH_GEMV_PRO_LAYERNORM) {
    double sum = 0.0;
    for (int64_t k = 0; k < K; ++k) sum += row[(size_t)k];
    const double mean = sum * L.fparams[0];
    double sq = 0.0;
    for (int64_t k = 0; k < K; ++k) sq += (row[(size_t)k] - mean) * (row[(size_t)k] - mean);
    const double rstd = 1.0 / std::sqrt(sq * L.fparams[1] + L.fparams[2]);
    for (int64_t k = 0; k < K; ++k) {
      double y = (row[(size_t)k] - mean) * rstd;
      if (gemv && L.cfg[5] >= 0) y *= p[L.cfg[5]][b * L.refs[L.cfg[5]].strides[0] + k * L.refs[L.cfg[5]].strides[2]];
      if (gemv && L.cfg[6] >= 0) y += p[L.cfg[6]][b * L.refs[L.cfg[6]].strides[0] + k * L.refs[L.cfg[6]].strides[2]];
      row[(size_t)k] = (float)y;
    }
  }
}

void host_matmul(const kh_launch &L, float *const *p) {
  const int64_t batch = L.gemm[0], M = L.gemm[1], N = L.gemm[2], K = L.gemm[3];
  const int prec = L.cfg[3];
  const kh_ref &B = L.refs[1];
  const int64_t k_pad = (K + 7) / 8 * 8;   // the bf16 copies' padded row: [N][K'] or [N][2K']
  const uint16_t *b16 = reinterpret_cast<const uint16_t *>(p[1]);
  std::vector<float> row((size_t)K);
  float slot[KH_NREGS] = {0};
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t m = 0; m < M; ++m) {
      a_row(L, p, b, m, row);
      for (int64_t n = 0; n < N; ++n) {
        double acc = 0.0;
        for (int64_t k = 0; k < K; ++k) {
          const int64_t at = b * B.strides[0] + k * B.strides[1] + n * B.strides[2];
          const float a = row[(size_t)k];
          if (prec == KH_PREC_FP32) {
            acc += (double)a * (double)p[1][at];
          } else if (prec == KH_PREC_BF16) {
            acc += (double)bf16_round(a) * (double)bf16_value(b16[at]);
          } else {   // three products of bf16 halves: lo*hi + hi*lo + hi*hi
            const float a_hi = bf16_round(a);
            const float a_lo = std::isfinite(a_hi) ? bf16_round(a - a_hi) : 0.0f;
            const double w_hi = bf16_value(b16[at]), w_lo = bf16_value(b16[at + k_pad]);
            acc += (double)a_lo * w_hi + (double)a_hi * w_lo + (double)a_hi * w_hi;
          }
        }
        const int64_t idx[3] = {b, m, n};
        // a GEMM's LayerNorm prologue: the folded beta . W, per column
        const int c_ref = L.family == KH_FAM_GEMM && L.cfg[4] == KH_GEMV_PRO_LAYERNORM ? L.cfg[6] : -1;
        if (c_ref >= 0) acc += (double)p[c_ref][offset_of(L.refs[c_ref], idx, 3)];
        slot[0] = (float)acc;
        const Operands mem(L, p);
        run_tape(
            L, 0, L.n_insns, slot, [&](int j) { return mem.ld(j, offset_of(L.refs[j], idx, 3)); },
            [&](int j, float v) { mem.st(j, offset_of(L.refs[j], idx, 3), v); }, [](const kh_insn &, float) {});
      }
    }
}

}  // namespace

// Executes one validated launch over host pointers (ptrs[j] = operand j's
// element 0). Returns false with `err` set for a family it cannot run.
bool run_launch_host(const kh_launch &L, float *const *ptrs, std::string &err) {
  switch (L.family) {
    case KH_FAM_EW: host_ew(L, ptrs); return true;
    case KH_FAM_ROW: host_row(L, ptrs); return true;
    case KH_FAM_RED: host_red(L, ptrs); return true;
    case KH_FAM_GEMM:
    case KH_FAM_GEMV: host_matmul(L, ptrs); return true;
    case KH_FAM_ATTN: host_attn(L, ptrs); return true;
    default: err = "no host semantics for kernel family " + std::to_string(L.family); return false;
  }
}

}  // namespace kh
