// kh_gemv.hip - the M = 1 matmul path (decode): out[b, n] = epilogue(sum_k
// x[b, k] * W[b, k, n]).
//
// A GEMV moves every weight byte once and does 2 flops per 4 bytes, so it is
// HBM-bound; MFMA tiles would waste 31/32 of their rows. Instead a workgroup
// of 256 threads covers 64 columns: 16 lanes read 16 consecutive 128-bit
// column quads of one weight row (1 KiB contiguous per k), 16 k-lanes walk
// the K range four rows at a time so each thread has four loads in flight.
// The 16 partial sums per column are combined through LDS in a fixed order.
// When the column blocks cannot fill the GPU, K is split across workgroups:
// each writes a dense partial row and splitk_reduce_kernel (shared with the
// GEMM family) sums them in split order and applies the epilogue.
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

constexpr int kCols = 64;  // columns per workgroup

__global__ __launch_bounds__(256) void gemv_kernel(const GemmArgs a) {
  __shared__ float4 part[16][16];
  const int cq = threadIdx.x & 15, kl = threadIdx.x >> 4;
  const int nb = blockIdx.x, b = blockIdx.y, split = blockIdx.z;
  const int n = nb * kCols + cq * 4;
  const int k_begin = split * a.k_per_split;
  const int k_end = min(a.K, k_begin + a.k_per_split);
  const float *x = a.A + (int64_t)b * a.sa_b;
  const float *W = a.B + (int64_t)b * a.sb_b;
  // The vector/scalar choice is made once, outside the K loop, so the four
  // row loads of an iteration carry no control flow between them and are all
  // in flight together.
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
    int k = k_begin + kl;
    for (; k + 48 < k_end; k += 64) {
      const float4 w0 = row(k), w1 = row(k + 16), w2 = row(k + 32), w3 = row(k + 48);
      const float x0 = x[(int64_t)k * a.sa_k], x1 = x[(int64_t)(k + 16) * a.sa_k];
      const float x2 = x[(int64_t)(k + 32) * a.sa_k], x3 = x[(int64_t)(k + 48) * a.sa_k];
      acc.x = fmaf(x0, w0.x, acc.x), acc.y = fmaf(x0, w0.y, acc.y), acc.z = fmaf(x0, w0.z, acc.z), acc.w = fmaf(x0, w0.w, acc.w);
      acc.x = fmaf(x1, w1.x, acc.x), acc.y = fmaf(x1, w1.y, acc.y), acc.z = fmaf(x1, w1.z, acc.z), acc.w = fmaf(x1, w1.w, acc.w);
      acc.x = fmaf(x2, w2.x, acc.x), acc.y = fmaf(x2, w2.y, acc.y), acc.z = fmaf(x2, w2.z, acc.z), acc.w = fmaf(x2, w2.w, acc.w);
      acc.x = fmaf(x3, w3.x, acc.x), acc.y = fmaf(x3, w3.y, acc.y), acc.z = fmaf(x3, w3.z, acc.z), acc.w = fmaf(x3, w3.w, acc.w);
    }
    for (; k < k_end; k += 16) {
      const float4 w = row(k);
      const float xv = x[(int64_t)k * a.sa_k];
      acc.x = fmaf(xv, w.x, acc.x), acc.y = fmaf(xv, w.y, acc.y), acc.z = fmaf(xv, w.z, acc.z), acc.w = fmaf(xv, w.w, acc.w);
    }
    return acc;
  };
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < a.N) acc = (a.b_vec && n + 3 < a.N) ? walk(std::true_type{}) : walk(std::false_type{});
  part[kl][cq] = acc;
  __syncthreads();
  Vec<4> v = splat4(0.0f);
  if (kl == 0) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float4 p = part[i][cq];
      v.v[0] += p.x, v.v[1] += p.y, v.v[2] += p.z, v.v[3] += p.w;
    }
  }
  if (kl != 0 || n >= a.N) return;
  if (a.splitk > 1) {
    // dense partial row [split][batch][N]; splitk_reduce_kernel finishes it
    float *dst = a.ws_partial + ((int64_t)split * a.batch + b) * a.N + n;
    for (int i = 0; i < 4 && n + i < a.N; ++i) dst[i] = v.v[i];
    return;
  }
  run_epilogue(a, b, 0, n, min(4, a.N - n), v);
}

class GemvOp final : public Op {
 public:
  GemmArgs args{};
  dim3 grid;
  size_t n_partials = 0;
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
    hipLaunchKernelGGL(gemv_kernel, grid, dim3(256), 0, stream, a);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splitk == 1) return e;
    return launch_splitk_reduce(a, current_device().cus, stream);
  }
  size_t partial_floats() const override { return n_partials; }
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
  const int n_blocks = (int)std::max<int64_t>(1, (N + kCols - 1) / kCols);
  int splitk = L.cfg[2];
  if (splitk <= 0) {
    const int64_t want = 2ll * current_device().cus;
    splitk = (int)std::max<int64_t>(1, std::min<int64_t>(want / std::max<int64_t>(1, n_blocks * batch), K / 64));
  }
  const int64_t kper = std::max<int64_t>(16, ((K + splitk - 1) / splitk + 15) / 16 * 16);
  splitk = (int)std::max<int64_t>(1, (K + kper - 1) / kper);
  a.k_per_split = (int)kper;
  a.splitk = splitk;
  op->grid = dim3((unsigned)n_blocks, (unsigned)std::max<int64_t>(batch, 1), (unsigned)splitk);
  if (splitk > 1) {
    op->n_partials = (size_t)splitk * batch * N;
  }
  return op;
}

}  // namespace kh
