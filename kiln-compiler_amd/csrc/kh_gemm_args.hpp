// kh_gemm_args.hpp - kernel arguments and the epilogue tape shared by the
// GEMM and GEMV kernels (both end in epilogue(acc) over (batch, m, n)).
#pragma once

#include <string>

#include "kh_common.hpp"

namespace kh {

struct GemmArgs {
  int32_t batch, M, N, K;
  const float *A;
  int64_t sa_b, sa_m, sa_k;
  const float *B;
  int64_t sb_b, sb_k, sb_n;
  int32_t a_vec, b_vec;
  int32_t tiles_m, tiles_n, splitk, k_per_split;
  int32_t n_refs, n_insns, n_pre;
  uint32_t e_vec_mask, e_bcast_mask;
  float *eptr[KH_MAX_REFS];           // epilogue operand j = descriptor ref j + 2
  int64_t estride[KH_MAX_REFS][3];
  kh_insn insns[KH_MAX_INSNS];        // LOAD/STORE operands renumbered to epilogue slots
  float *ws_partial;
  uint32_t *ws_count;
};

// Run the epilogue tape for columns [n, n + valid) of output row (b, m);
// slot 0 starts as the accumulator values. Epilogue tapes use at most 8 slots.
__device__ __forceinline__ void run_epilogue(const GemmArgs &a, int64_t b, int64_t m, int64_t n, int valid,
                                             const Vec<4> &acc) {
  auto base = [&](int j) { return a.eptr[j] + b * a.estride[j][0] + m * a.estride[j][1]; };
  auto load = [&](int j) -> Vec<4> {
    const float *p = base(j);
    if (a.e_bcast_mask >> j & 1) return splat4(p[0]);
    Vec<4> out;
    if ((a.e_vec_mask >> j & 1) && valid == 4) {
      const float4 q = *reinterpret_cast<const float4 *>(p + n);
      out.v[0] = q.x, out.v[1] = q.y, out.v[2] = q.z, out.v[3] = q.w;
      return out;
    }
    const int64_t sn = a.estride[j][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) out.v[i] = i < valid ? p[(n + i) * sn] : 0.0f;
    return out;
  };
  auto store = [&](int j, const Vec<4> &v) {
    float *p = base(j);
    if ((a.e_vec_mask >> j & 1) && valid == 4) {
      *reinterpret_cast<float4 *>(p + n) = make_float4(v.v[0], v.v[1], v.v[2], v.v[3]);
      return;
    }
    const int64_t sn = a.estride[j][2];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < valid) p[(n + i) * sn] = v.v[i];
  };
  float f[kFastSlots * 4];
  bank_set(f, 0, acc);
  exec_tape<kFastSlots>(a.insns, 0, a.n_insns, a.n_pre, f, load, store, [](const kh_insn &, const Vec<4> &) {});
}

// Host: validate the epilogue refs/tape of a matmul descriptor into `a`.
bool fill_epilogue(const kh_launch &L, GemmArgs &a, uint32_t &vec_candidates, std::string &err);

}  // namespace kh
