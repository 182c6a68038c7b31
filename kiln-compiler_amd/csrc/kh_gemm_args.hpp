// kh_gemm_args.hpp - kernel arguments and the epilogue tape shared by the
// GEMM and GEMV kernels (both end in epilogue(acc) over (batch, m, n)).
#pragma once

#include <algorithm>
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
  int32_t tiles_m, tiles_n, splitk, k_per_split, group_m;
  int32_t n_refs, n_insns, n_pre;
  uint32_t e_vec_mask, e_bcast_mask;
  float *eptr[KH_MAX_REFS];           // epilogue operand j = descriptor ref j + 2
  int64_t estride[KH_MAX_REFS][3];
  kh_insn insns[KH_MAX_INSNS];        // LOAD/STORE operands renumbered to epilogue slots
  float *ws_partial;
  // direct epilogue (the host recognised the tape as out = act((acc [+ bias])
  // [+ res])): epilogue operand indices, -1 when absent, and the activation
  int32_t direct, d_bias, d_res, d_out, d_act;
  // GEMV LayerNorm prologue: A is the raw row x and the kernel multiplies
  // ((x - mean) * rstd [* gamma] [+ beta]); gamma / beta are epilogue operand
  // indices (-1 when absent), c1 / c2 the 1/C factors of mean and variance
  int32_t pro, pro_g, pro_b;
  float pro_c1, pro_c2, pro_eps;
  // GEMV attention prologue (pro == 2): epilogue operand index of Q (K and V
  // follow), of the additive mask (-1: none), keys, head dim, mask and scale
  // modes, scale
  int32_t att_q, att_mask, att_tk, att_dh, att_mask_mode, att_scale_mode;
  float att_scale;
  // bf16 storage (kind 7 only): A holds bf16 values (its strides count bf16
  // elements); the direct epilogue's output is written as bf16
  int32_t a16, o16;
  // pair storage (three-pass configurations): A holds pair words; the direct
  // epilogue writes its output as pair words
  int32_t a_pair, o_pair;
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

// Split-K, second kernel: partials are dense [split][batch][M][N] fp32 in the
// workspace (written by the first kernel without any cross-workgroup
// synchronisation; the kernel boundary makes them visible to every XCD).
// Each thread sums the splits of 4 adjacent columns in split order (the
// result does not depend on scheduling) and runs the epilogue.
namespace {
constexpr int kReduceThreads = 256;
constexpr int kReduceGroup = 8;
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const GemmArgs a) {
  const uint32_t n4 = (uint32_t)(a.N + 3) / 4;
  const uint64_t rows = (uint64_t)a.batch * a.M;
  const uint64_t total = rows * n4;
  const uint64_t plane = rows * (uint64_t)a.N;
  const bool vec = (a.N & 3) == 0;
  for (uint64_t q = (uint64_t)blockIdx.x * 256 + threadIdx.x; q < total; q += (uint64_t)gridDim.x * 256) {
    const uint64_t row = q / n4;
    const int n = (int)(q - row * n4) * 4;
    const int valid = min(4, a.N - n);
    const float *p = a.ws_partial + row * a.N + n;
    Vec<4> s = splat4(0.0f);
    // issue a group of split loads before the first add (one memory latency
    // per group, not per split); the adds stay in split order
    for (int sp0 = 0; sp0 < a.splitk; sp0 += kReduceGroup) {
      float4 v[kReduceGroup];
#pragma unroll
      for (int j = 0; j < kReduceGroup; ++j) {
        v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (sp0 + j >= a.splitk) continue;
        const float *src = p + (uint64_t)(sp0 + j) * plane;
        if (vec) {
          v[j] = *reinterpret_cast<const float4 *>(src);
        } else {
          if (0 < valid) v[j].x = src[0];
          if (1 < valid) v[j].y = src[1];
          if (2 < valid) v[j].z = src[2];
          if (3 < valid) v[j].w = src[3];
        }
      }
#pragma unroll
      for (int j = 0; j < kReduceGroup; ++j)
        if (sp0 + j < a.splitk) s.v[0] += v[j].x, s.v[1] += v[j].y, s.v[2] += v[j].z, s.v[3] += v[j].w;
    }
    run_epilogue(a, (int64_t)(row / a.M), (int64_t)(row % a.M), n, valid, s);
  }
}

inline hipError_t launch_splitk_reduce(const GemmArgs &a, int cus, hipStream_t stream) {
  const uint64_t total = (uint64_t)a.batch * a.M * (uint64_t)((a.N + 3) / 4);
  const uint64_t blocks = (total + kReduceThreads - 1) / kReduceThreads;
  const unsigned grid = (unsigned)std::max<uint64_t>(1, std::min<uint64_t>(blocks, (uint64_t)cus * 8));
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(grid), dim3(kReduceThreads), 0, stream, a);
  return hipGetLastError();
}
}  // namespace

// Configurations of the K-contiguous fp32 kernel (kind 5, kh_gemm_nt.hip):
// id, macro tile BM x BN (K step 32), waves WM x WN (one or two per SIMD;
// persistent, at most one workgroup per CU), LDS stages NS.
#define KH_GEMM_NT_CONFIGS(X) \
  X(55, 128, 192, 2, 2, 3)    \
  X(56, 64, 288, 2, 2, 2)     \
  X(57, 64, 96, 2, 2, 3)      \
  X(58, 128, 96, 2, 2, 3)     \
  X(59, 128, 128, 2, 4, 3)    \
  X(60, 64, 192, 2, 4, 3)     \
  X(61, 128, 192, 2, 4, 3)    \
  X(62, 64, 128, 2, 4, 3)     \
  X(63, 32, 96, 2, 2, 3)      \
  X(64, 64, 64, 2, 2, 3)

// The same kernel over the bf16 (prec 1) and three-pass bf16 (prec 2) weight
// copies: id, BM x BN, waves WM x WN, stages NS, prec.
#define KH_GEMM_NT_BF16_CONFIGS(X) \
  X(87, 128, 256, 2, 4, 3, 1)      \
  X(88, 128, 192, 2, 2, 4, 1)      \
  X(89, 256, 128, 4, 2, 3, 1)      \
  X(90, 128, 128, 2, 4, 4, 1)      \
  X(91, 64, 192, 2, 2, 4, 1)       \
  X(92, 128, 256, 2, 4, 2, 2)      \
  X(93, 128, 192, 2, 2, 3, 2)      \
  X(94, 128, 128, 2, 4, 3, 2)

// Configurations of the bf16 kernel with 64-deep K steps (kind 7,
// kh_gemm_bf.hip; K a multiple of 64, one tile per workgroup): id, BM x BN,
// waves WM x WN, stages NS.
#define KH_GEMM_BF_CONFIGS(X) \
  X(95, 128, 192, 2, 4, 2)             \
  X(96, 64, 192, 2, 4, 3)              \
  X(97, 64, 128, 2, 4, 3)              \
  X(98, 64, 96, 2, 2, 3)               \
  X(99, 64, 64, 2, 2, 3)               \
  X(100, 128, 96, 2, 2, 3)

// Launch configuration `id` of kind 5 (hipErrorInvalidValue for another id).
hipError_t launch_gemm_nt(int id, const GemmArgs &a, dim3 grid, hipStream_t stream);
// Launch configuration `id` of kind 7 (hipErrorInvalidValue for another id).
hipError_t launch_gemm_bf(int id, const GemmArgs &a, dim3 grid, hipStream_t stream);

// Longest row a small-M GEMM's LayerNorm prologue takes.
constexpr int kLnMaxK = 1024;

// Configurations of the small-M kernel (kind 6, kh_gemm_small.hip): id, tile
// BM x BN, WK waves splitting K (each with a private LDS ring), NS stages,
// precision (0 fp32, 1 bf16, 2 three-pass bf16).
#define KH_GEMM_SMALL_CONFIGS(X) \
  X(65, 16, 32, 4, 3, 0)         \
  X(66, 16, 32, 4, 2, 0)         \
  X(67, 16, 16, 4, 3, 0)         \
  X(68, 16, 64, 4, 2, 0)         \
  X(69, 32, 32, 4, 2, 0)         \
  X(70, 16, 32, 8, 2, 0)         \
  X(71, 16, 16, 8, 2, 0)         \
  X(72, 32, 64, 4, 2, 0)         \
  X(73, 32, 32, 8, 2, 0)         \
  X(74, 16, 16, 4, 2, 0)         \
  X(75, 16, 32, 4, 2, 1)         \
  X(76, 16, 32, 8, 2, 1)         \
  X(77, 32, 32, 4, 2, 1)         \
  X(78, 16, 64, 4, 2, 1)         \
  X(79, 16, 16, 4, 2, 1)         \
  X(80, 16, 32, 4, 2, 2)         \
  X(81, 16, 32, 8, 2, 2)         \
  X(82, 32, 32, 4, 2, 2)         \
  X(83, 16, 16, 4, 2, 2)         \
  X(84, 16, 16, 8, 2, 1)         \
  X(85, 32, 32, 8, 2, 1)         \
  X(86, 16, 16, 8, 2, 2)

// Launch configuration `id` of kind 6 (hipErrorInvalidValue for another id).
hipError_t launch_gemm_small(int id, const GemmArgs &a, dim3 grid, hipStream_t stream);

// Host: validate the epilogue refs/tape of a matmul descriptor into `a`.
bool fill_epilogue(const kh_launch &L, GemmArgs &a, uint32_t &vec_candidates, std::string &err);
// Recognise the tape out = act((acc [+ bias]) [+ res]) and fill the direct
// epilogue fields (a.direct = 1); false (fields untouched) for any other tape.
bool match_direct_epilogue(const kh_launch &L, GemmArgs &a);

}  // namespace kh
