// kh_reduce.hip - reductions over dims other than the innermost (K-RED):
// column sums, reductions over several leading dims, full reductions.
//
// Replaces the reference's [64 outputs x <= 64 reduced] Triton program
// (kiln/gpu/codegen.py:432-482). With many outputs, one thread per output
// walks the reduced extent (adjacent threads read adjacent addresses when the
// kept innermost dim is contiguous, the column-sum case). With few outputs,
// one workgroup per output splits the reduced extent over 256 threads and
// combines the partials in a fixed order, so results are deterministic.
#include <algorithm>
#include <cmath>

#include "kh_common.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

struct RedArgs {
  const float *x;
  float *out;
  int32_t kept_rank, red_rank, is_max;
  uint32_t n_out, n_red;
  FastDiv kdiv[KH_MAX_RANK], rdiv[KH_MAX_RANK];
  int64_t xk[KH_MAX_RANK], xr[KH_MAX_RANK], ok[KH_MAX_RANK];
};

__device__ __forceinline__ void split_index(uint32_t v, int rank, const FastDiv *div, const int64_t *s1,
                                            const int64_t *s2, int64_t &o1, int64_t &o2) {
  o1 = 0, o2 = 0;
#pragma unroll
  for (int d = KH_MAX_RANK - 1; d >= 0; --d) {
    if (d < rank) {
      const uint32_t q = fdiv(v, div[d]);
      const uint32_t i = v - q * div[d].d;
      o1 += (int64_t)i * s1[d];
      if (s2) o2 += (int64_t)i * s2[d];
      v = q;
    }
  }
}

__global__ __launch_bounds__(256) void reduce_thread_kernel(const RedArgs a) {
  for (uint32_t o = blockIdx.x * 256 + threadIdx.x; o < a.n_out; o += gridDim.x * 256) {
    int64_t xo, oo;
    split_index(o, a.kept_rank, a.kdiv, a.xk, a.ok, xo, oo);
    float acc = a.is_max ? -INFINITY : 0.0f;
    for (uint32_t r = 0; r < a.n_red; ++r) {
      int64_t xr, unused;
      split_index(r, a.red_rank, a.rdiv, a.xr, nullptr, xr, unused);
      const float v = a.x[xo + xr];
      acc = a.is_max ? nan_max(acc, v) : acc + v;
    }
    a.out[oo] = acc;
  }
}

__global__ __launch_bounds__(256) void reduce_block_kernel(const RedArgs a) {
  __shared__ float part[4];
  for (uint32_t o = blockIdx.x; o < a.n_out; o += gridDim.x) {
    int64_t xo, oo;
    split_index(o, a.kept_rank, a.kdiv, a.xk, a.ok, xo, oo);
    float acc = a.is_max ? -INFINITY : 0.0f;
    for (uint32_t r = threadIdx.x; r < a.n_red; r += 256) {
      int64_t xr, unused;
      split_index(r, a.red_rank, a.rdiv, a.xr, nullptr, xr, unused);
      const float v = a.x[xo + xr];
      acc = a.is_max ? nan_max(acc, v) : acc + v;
    }
    acc = a.is_max ? wave_max(acc) : wave_sum(acc);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
      float r = part[0];
      for (int w = 1; w < 4; ++w) r = a.is_max ? nan_max(r, part[w]) : r + part[w];
      a.out[oo] = r;
    }
  }
}

class RedOp final : public Op {
 public:
  RedArgs args{};
  bool per_block = false;
  int grid = 1;
  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    RedArgs a = args;
    a.x = ptrs[0];
    a.out = ptrs[1];
    if (a.n_out == 0) return hipSuccess;
    if (per_block) hipLaunchKernelGGL(reduce_block_kernel, dim3(grid), dim3(256), 0, stream, a);
    else hipLaunchKernelGGL(reduce_thread_kernel, dim3(grid), dim3(256), 0, stream, a);
    return hipGetLastError();
  }
};

}  // namespace

std::unique_ptr<Op> make_red(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  if (L.n_refs != 2 || L.rank < 0 || L.rank > KH_MAX_RANK) {
    err = "reduce: expects one input and one output operand";
    return nullptr;
  }
  auto op = std::make_unique<RedOp>();
  RedArgs &a = op->args;
  const uint32_t mask = (uint32_t)L.cfg[0];
  a.is_max = L.cfg[1] != 0;
  int64_t n_out = 1, n_red = 1;
  bool empty_out = false, empty_red = false;
  for (int d = 0; d < L.rank; ++d) {
    if (L.shape[d] < 0) {
      err = "reduce: negative extent";
      return nullptr;
    }
    if (L.shape[d] == 0) ((mask >> d & 1) ? empty_red : empty_out) = true;
  }
  for (int d = 0; d < L.rank; ++d) {
    const int64_t s = L.shape[d];
    if (s <= 1) continue;
    if (mask >> d & 1) {
      a.rdiv[a.red_rank] = make_fastdiv((uint32_t)s);
      a.xr[a.red_rank] = L.refs[0].strides[d];
      ++a.red_rank;
      n_red *= s;
    } else {
      a.kdiv[a.kept_rank] = make_fastdiv((uint32_t)s);
      a.xk[a.kept_rank] = L.refs[0].strides[d];
      a.ok[a.kept_rank] = L.refs[1].strides[d];
      ++a.kept_rank;
      n_out *= s;
    }
  }
  if (empty_out) n_out = 0;
  if (empty_red) n_red = 0;
  if (n_out >= (1ll << 31) || n_red >= (1ll << 31)) {
    unsupported = true;
    err = "reduce: extent beyond 2^31";
    return nullptr;
  }
  a.n_out = (uint32_t)n_out;
  a.n_red = (uint32_t)n_red;
  const int cus = current_device().cus;
  op->per_block = n_out < (int64_t)cus * 64 && n_red >= 256;
  op->grid = op->per_block ? (int)std::max<int64_t>(1, std::min<int64_t>(n_out, cus * 16))
                           : (int)std::max<int64_t>(1, std::min<int64_t>((n_out + 255) / 256, cus * 16));
  return op;
}

}  // namespace kh
