// kh_gemv.hip - the M = 1 matmul path (decode): out[b, n] = epilogue(sum_k
// x[b, k] * W[b, k, n]).
//
// A GEMV moves every weight byte once and does 2 flops per 4 bytes, so it is
// HBM-bound; at decode sizes (a few MB per launch) a launch lasts about one
// memory latency plus the streaming time of the busiest CU, so the kernel is
// shaped for memory-level parallelism and spread:
//   * a workgroup of 256 or 1024 threads covers CQ column quads (4 * CQ
//     columns, CQ = 8, 4 or 2, so a row segment is 128, 64 or 32 contiguous
//     bytes) and threads / CQ k-lanes; each thread issues kRows 128-bit row
//     loads (and the matching x values) before its first FMA;
//   * CQ is the widest that still gives about half the CUs a workgroup, so
//     the weight stream is spread over the chip rather than queued behind a
//     few CUs; narrower segments than 64 bytes were measured slower (a wave's
//     load then touches 64 cache lines). When even CQ = 4 leaves few column
//     blocks (N small, K large) the workgroup grows to 1024 threads so each
//     CU still has its whole share of rows in flight in one or two passes;
//   * the k-lanes are reduced in a fixed tree (shuffles inside a wave, then the
//     four waves through LDS) and the same workgroup runs the epilogue;
//   * a LayerNorm whose only consumer is the GEMV runs as its prologue (decode:
//     the normalised row never goes through memory, one launch instead of
//     two): every workgroup recomputes the row's mean and variance in one
//     pass (sums shifted by the row's first value, one workgroup reduction)
//     and normalises x as it loads it;
//   * only when even CQ = 1 leaves too few workgroups for the rows (tiny N, huge
//     K) is K split across workgroups; the splits' partials are then summed in
//     split order by the split-K reduce kernel (shared with the GEMM family),
//     which runs the epilogue. Cross-workgroup combining inside one launch was
//     measured slower at these sizes (agent-scope fences across 8 XCDs).
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

constexpr int kRows = 8;           // row loads in flight per thread
constexpr int kTargetBlocks = 128;  // workgroups wanted before narrowing stops

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float4 shfl_xor4(float4 v, int m) {
  return make_float4(__shfl_xor(v.x, m, 64), __shfl_xor(v.y, m, 64), __shfl_xor(v.z, m, 64),
                     __shfl_xor(v.w, m, 64));
}

// Sum of v over the workgroup, in a fixed order (wave tree, then the waves in
// order); every thread gets the total. `red` holds NW entries.
template <int NW>
__device__ __forceinline__ float2 block_sum2(float2 v, float2 *red) {
#pragma unroll
  for (int m = 32; m >= 1; m /= 2) v.x += __shfl_xor(v.x, m, 64), v.y += __shfl_xor(v.y, m, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float2 s = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) s.x += red[w].x, s.y += red[w].y;
  return s;
}

constexpr int kProCache = 4;  // x values per thread kept in registers by the prologue

template <int CQ, int THREADS, bool PRO>
__global__ __launch_bounds__(THREADS) void gemv_kernel(const GemmArgs a) {
  constexpr int KL = THREADS / CQ;  // k-lanes: rows one load instruction covers
  constexpr int NW = THREADS / 64;
  __shared__ float4 wave_part[NW][CQ];
  __shared__ float2 red[NW];
  const int tid = threadIdx.x;
  const int cq = tid % CQ, kl = tid / CQ;
  const int nb = blockIdx.x, b = blockIdx.y, split = blockIdx.z;
  const int n = nb * 4 * CQ + cq * 4;
  const int k_begin = split * a.k_per_split;
  const int k_end = min(a.K, k_begin + a.k_per_split);
  const float *x = a.A + (int64_t)b * a.sa_b;
  const float *W = a.B + (int64_t)b * a.sb_b;
  // LayerNorm prologue: statistics of the whole row (every split needs them);
  // an absent gamma / beta reads x[0] (stride 0) and is deselected
  float mean = 0.0f, rstd = 1.0f;
  const float *gam = x, *bet = x;
  int g_st = 0, b_st = 0;
  if constexpr (PRO) {
    // one pass over the row, sums shifted by its first value c (so the
    // variance does not cancel for rows far from zero):
    //   mean = c + S1 / C,  var = (S2 - S1^2 / C) * c2,  S_p = sum (x - c)^p
    const float c = x[0];
    float xs[kProCache];
#pragma unroll
    for (int i = 0; i < kProCache; ++i) {
      const int k = tid + i * THREADS;
      xs[i] = k < a.K ? x[(int64_t)k * a.sa_k] - c : 0.0f;
    }
    float2 s = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < kProCache; ++i) s.x += xs[i], s.y = fmaf(xs[i], xs[i], s.y);
    for (int k = tid + kProCache * THREADS; k < a.K; k += THREADS) {
      const float d = x[(int64_t)k * a.sa_k] - c;
      s.x += d, s.y = fmaf(d, d, s.y);
    }
    s = block_sum2<NW>(s, red);
    const float m1 = s.x * a.pro_c1;
    mean = c + m1;
    rstd = rsqrtf(fmaxf(fmaf(-s.x, m1, s.y), 0.0f) * a.pro_c2 + a.pro_eps);
    if (a.pro_g >= 0) gam = a.eptr[a.pro_g] + b * a.estride[a.pro_g][0], g_st = 1;
    if (a.pro_b >= 0) bet = a.eptr[a.pro_b] + b * a.estride[a.pro_b][0], b_st = 1;
  }
  auto walk = [&](auto vec_tag) {
    constexpr bool vec = decltype(vec_tag)::value;
    auto row = [&](int k) -> float4 {
      const float *p = W + (int64_t)k * a.sb_k;
      if constexpr (vec) {
        return *reinterpret_cast<const float4 *>(p + n);
      } else {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (n + 0 < a.N) v.x = p[(int64_t)(n + 0) * a.sb_n];
        if (n + 1 < a.N) v.y = p[(int64_t)(n + 1) * a.sb_n];
        if (n + 2 < a.N) v.z = p[(int64_t)(n + 2) * a.sb_n];
        if (n + 3 < a.N) v.w = p[(int64_t)(n + 3) * a.sb_n];
        return v;
      }
    };
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = k_begin + kl; k0 < k_end; k0 += KL * kRows) {
      float4 w[kRows];
      float xv[kRows], gv[kRows], bv[kRows];
      // Rows past the end are clamped to the last row (an in-bounds load,
      // issued with the others) and their products dropped by a select. All
      // loads of the batch are issued before the first use of any of them.
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const int k = min(k0 + j * KL, k_end - 1);
        w[j] = row(k);
        xv[j] = x[(int64_t)k * a.sa_k];
        if constexpr (PRO) gv[j] = gam[k * g_st], bv[j] = bet[k * b_st];
      }
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const bool in = k0 + j * KL < k_end;
        float xn = xv[j];
        if constexpr (PRO) {
          xn = (xn - mean) * rstd;
          xn = g_st ? xn * gv[j] : xn;
          xn = b_st ? xn + bv[j] : xn;
        }
        const float xs = in ? xn : 0.0f;
        const float4 ws = in ? w[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        acc.x = fmaf(xs, ws.x, acc.x), acc.y = fmaf(xs, ws.y, acc.y);
        acc.z = fmaf(xs, ws.z, acc.z), acc.w = fmaf(xs, ws.w, acc.w);
      }
    }
    return acc;
  };
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < a.N) acc = (a.b_vec && n + 3 < a.N) ? walk(std::true_type{}) : walk(std::false_type{});
  // fixed-order tree over the k-lanes of a wave (lane = CQ * k-lane + quad),
  // then the waves in order
#pragma unroll
  for (int m = CQ; m < 64; m *= 2) acc = add4(acc, shfl_xor4(acc, m));
  if ((tid & 63) < CQ) wave_part[tid >> 6][cq] = acc;
  __syncthreads();
  if (tid >= CQ || n >= a.N) return;
  float4 s = wave_part[0][cq];
#pragma unroll
  for (int w = 1; w < NW; ++w) s = add4(s, wave_part[w][cq]);
  const int valid = min(4, a.N - n);
  if (a.splitk > 1) {
    // dense partial row [split][batch][N]; splitk_reduce_kernel finishes it
    float *dst = a.ws_partial + ((int64_t)split * a.batch + b) * a.N + n;
    if (valid > 0) dst[0] = s.x;
    if (valid > 1) dst[1] = s.y;
    if (valid > 2) dst[2] = s.z;
    if (valid > 3) dst[3] = s.w;
    return;
  }
  Vec<4> out;
  out.v[0] = s.x, out.v[1] = s.y, out.v[2] = s.z, out.v[3] = s.w;
  run_epilogue(a, b, 0, n, valid, out);
}

// (column quads, threads) per workgroup by variant id (1..5); 0 = chosen
// from the shape.
constexpr int kVariants[][2] = {{0, 0}, {8, 256}, {4, 256}, {2, 256}, {8, 1024}, {4, 1024}};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

class GemvOp final : public Op {
 public:
  GemmArgs args{};
  dim3 grid;
  size_t n_partials = 0;
  int quads = 8, threads = 256;
  bool b_vec_layout = false;
  uint32_t e_vec_candidates = 0;

  hipError_t launch(float *const *ptrs, uint32_t *counters, float *partials, hipStream_t stream) override {
    GemmArgs a = args;
    a.A = ptrs[0];
    a.B = ptrs[1];
    a.b_vec = b_vec_layout && (reinterpret_cast<uintptr_t>(ptrs[1]) & 15) == 0;
    a.e_vec_mask = 0;
    for (int j = 0; j < a.n_refs; ++j) {
      a.eptr[j] = ptrs[2 + j];
      if ((e_vec_candidates >> j & 1) && (reinterpret_cast<uintptr_t>(ptrs[2 + j]) & 15) == 0)
        a.e_vec_mask |= 1u << j;
    }
    a.ws_partial = partials;
    if (a.N == 0 || a.batch == 0) return hipSuccess;
    if (a.splitk > 1 && !partials) return hipErrorInvalidValue;
    if (a.pro) launch_variant(a, grid, stream, std::true_type{});
    else launch_variant(a, grid, stream, std::false_type{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splitk == 1) return e;
    return launch_splitk_reduce(a, current_device().cus, stream);
  }
  size_t partial_floats() const override { return n_partials; }

  template <class P>
  void launch_variant(const GemmArgs &a, dim3 g, hipStream_t stream, P) const {
    constexpr bool pro = P::value;
    if (threads == 1024) {
      if (quads == 8) hipLaunchKernelGGL((gemv_kernel<8, 1024, pro>), g, dim3(1024), 0, stream, a);
      else hipLaunchKernelGGL((gemv_kernel<4, 1024, pro>), g, dim3(1024), 0, stream, a);
    } else {
      if (quads == 8) hipLaunchKernelGGL((gemv_kernel<8, 256, pro>), g, dim3(256), 0, stream, a);
      else if (quads == 4) hipLaunchKernelGGL((gemv_kernel<4, 256, pro>), g, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((gemv_kernel<2, 256, pro>), g, dim3(256), 0, stream, a);
    }
  }
};

}  // namespace

std::unique_ptr<Op> make_gemv(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  if (L.n_refs < 3 || L.n_refs > KH_MAX_REFS) {
    err = "gemv: bad operand count";
    return nullptr;
  }
  const int64_t batch = L.gemm[0], M = L.gemm[1], N = L.gemm[2], K = L.gemm[3];
  if (M != 1) {
    err = "gemv: M must be 1";
    return nullptr;
  }
  if (batch < 0 || N < 0 || K < 0 || batch >= (1 << 16) || N >= (1ll << 30) || K >= (1ll << 30)) {
    unsupported = true;
    err = "gemv: sizes out of range";
    return nullptr;
  }
  auto op = std::make_unique<GemvOp>();
  GemmArgs &a = op->args;
  a.batch = (int)batch, a.M = 1, a.N = (int)N, a.K = (int)K;
  a.sa_b = L.refs[0].strides[0], a.sa_m = L.refs[0].strides[1], a.sa_k = L.refs[0].strides[2];
  a.sb_b = L.refs[1].strides[0], a.sb_k = L.refs[1].strides[1], a.sb_n = L.refs[1].strides[2];
  op->b_vec_layout = a.sb_n == 1 && L.refs[1].offset % 4 == 0 && a.sb_k % 4 == 0 && a.sb_b % 4 == 0;
  if (!fill_epilogue(L, a, op->e_vec_candidates, err)) return nullptr;
  // LayerNorm prologue: cfg[4] = 1, cfg[5] / cfg[6] = ref index of gamma /
  // beta (-1: none), fparams = {1/C, 1/C, eps}; gamma and beta are [K] rows
  a.pro = L.cfg[4], a.pro_g = -1, a.pro_b = -1;
  if (a.pro != 0 && a.pro != 1) {
    err = "gemv: unknown prologue " + std::to_string(a.pro);
    return nullptr;
  }
  if (a.pro) {
    for (int w = 0; w < 2; ++w) {
      const int r = L.cfg[5 + w];
      if (r == -1) continue;
      if (r < 2 || r >= L.n_refs) {
        err = "gemv: prologue operand index out of range";
        return nullptr;
      }
      const kh_ref &g = L.refs[r];
      if (g.strides[1] != 0 || g.strides[2] != 1) {
        err = "gemv: LayerNorm gamma / beta must be unit-stride rows over K";
        return nullptr;
      }
      (w == 0 ? a.pro_g : a.pro_b) = r - 2;
    }
    a.pro_c1 = L.fparams[0], a.pro_c2 = L.fparams[1], a.pro_eps = L.fparams[2];
  }
  // column quads per workgroup: the widest giving kTargetBlocks workgroups;
  // if none does, 64-byte segments with 1024-thread workgroups
  const int64_t b1 = std::max<int64_t>(1, batch);
  const int variant = L.cfg[1];
  if (variant < 0 || variant >= kNumVariants) {
    err = "gemv: unknown variant " + std::to_string(variant);
    return nullptr;
  }
  int quads = kVariants[variant][0], threads = kVariants[variant][1];
  if (quads == 0) {
    quads = 4, threads = 1024;
    for (int q : {8, 4}) {
      if ((N + 4 * q - 1) / (4 * q) * b1 >= kTargetBlocks) {
        quads = q, threads = 256;
        break;
      }
    }
  }
  const int64_t n_blocks = std::max<int64_t>(1, (N + 4 * quads - 1) / (4 * quads));
  const int64_t k_lanes = threads / quads;
  // split K (two kernels) only when the blocks are few and each thread would
  // walk more than four passes of kRows rows
  int64_t splitk = L.cfg[2];
  if (splitk <= 0) {
    splitk = 1;
    const int64_t rows_per_thread = (K + k_lanes - 1) / k_lanes;
    if (n_blocks * b1 < kTargetBlocks / 2 && rows_per_thread > 4 * kRows)
      splitk = std::min<int64_t>((kTargetBlocks + n_blocks * b1 - 1) / (n_blocks * b1),
                                 (rows_per_thread + 4 * kRows - 1) / (4 * kRows));
  }
  splitk = std::max<int64_t>(1, std::min<int64_t>(splitk, std::max<int64_t>(1, K / k_lanes)));
  const int64_t kper = std::max<int64_t>(k_lanes, ((K + splitk - 1) / splitk + k_lanes - 1) / k_lanes * k_lanes);
  splitk = std::max<int64_t>(1, (K + kper - 1) / kper);
  if (n_blocks * b1 >= (1ll << 31) || b1 >= 65536) {
    unsupported = true;
    err = "gemv: too many column blocks";
    return nullptr;
  }
  op->quads = quads;
  op->threads = threads;
  a.k_per_split = (int)kper;
  a.splitk = (int)splitk;
  op->grid = dim3((unsigned)n_blocks, (unsigned)b1, (unsigned)splitk);
  if (splitk > 1) {
    op->n_partials = (size_t)splitk * batch * N;
  }
  return op;
}

}  // namespace kh
