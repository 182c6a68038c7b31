// kh_probe.hip - a measurement probe of the matrix cores: how many shader
// cycles a 32x32x2 fp32 MFMA costs a SIMD when the same wave also issues
// vector ALU work, and how that depends on the number of independent
// accumulator chains and on how MFMAs and VALU instructions are grouped.
//
// This is the question behind the fused attention kernel's schedule (its
// score and P.V MFMAs run next to the softmax arithmetic in the same waves);
// kh_probe_attn_timeline (kh_attn.hip) measures the kernel itself. No
// counterpart in the reference, which has no hand-written kernels.
//
// The probe kernel: one workgroup per CU, 64 * 4 * waves_per_simd threads, so
// every SIMD runs waves_per_simd waves. Each iteration issues 32 MFMAs in
// groups of G back-to-back instructions over C independent accumulators
// (round-robin), each group followed by V independent fp32 FMAs on values of
// the wave's own. Every wave of workgroup 0 reads the shader clock
// (s_memtime) and the 100 MHz wall clock (s_memrealtime) around its loop; the
// probe's time is the span from the first start to the last end on that CU.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <string>

#include "kh_internal.hpp"

namespace kh {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kIters = 200;

template <int C, int G, int V>
__global__ __launch_bounds__(512) void mfma_valu_kernel(float *out, uint64_t *clk, float a0) {
  const float a = a0 + threadIdx.x * 1e-7f, b = a0 * 0.5f;
  float x[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) x[i] = a0 * (i + 1) * 1e-3f + threadIdx.x * 1e-9f;
  f32x16 acc[C];
#pragma unroll
  for (int i = 0; i < C; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int g = 0; g < 32 / G; ++g) {
#pragma unroll
      for (int i = 0; i < G; ++i)
        acc[(g * G + i) % C] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc[(g * G + i) % C], 0, 0, 0);
#pragma unroll
      for (int v = 0; v < V; ++v) x[v % 16] = fmaf(x[v % 16], 0.999f, 1e-4f);
      __builtin_amdgcn_sched_group_barrier(0x008, G, 0);  // MFMA
      if (V) __builtin_amdgcn_sched_group_barrier(0x002, V, 0);  // VALU
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < C; ++i) s += acc[i][0] + acc[i][15];
#pragma unroll
  for (int i = 0; i < 16; ++i) s += x[i];
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  if (blockIdx.x == 0 && (threadIdx.x & 63) == 0) {
    uint64_t *c = clk + 4 * (threadIdx.x >> 6);
    c[0] = t0, c[1] = t1, c[2] = r0, c[3] = r1;
  }
}

// (chains, group, valu) combinations the probe offers
#define KH_PROBE_MFMA_CASES(X) \
  X(1, 1, 0)                   \
  X(2, 1, 0)                   \
  X(1, 1, 1)                   \
  X(1, 1, 2)                   \
  X(1, 1, 4)                   \
  X(2, 1, 2)                   \
  X(4, 1, 2)                   \
  X(8, 1, 2)                   \
  X(1, 4, 8)                   \
  X(1, 8, 16)                  \
  X(2, 8, 16)                  \
  X(1, 32, 64)

}  // namespace

hipError_t probe_mfma_valu(int chains, int group, int valu, int waves_per_simd, double out2[2], std::string &err) {
  if (!out2 || (waves_per_simd != 1 && waves_per_simd != 2)) {
    err = "MFMA probe: waves per SIMD must be 1 or 2";
    return hipErrorInvalidValue;
  }
  const int blocks = current_device().cus, threads = 256 * waves_per_simd;
  float *out = nullptr;
  uint64_t *clk = nullptr;
  hipError_t e = hipMalloc(&out, (size_t)blocks * threads * sizeof(float));
  const int waves = threads / 64;
  if (e == hipSuccess) e = hipMalloc(&clk, 4 * waves * sizeof(uint64_t));
  bool known = false;
  auto run = [&](auto kernel) {
    known = true;
    for (int rep = 0; rep < 2 && e == hipSuccess; ++rep) {  // the first run warms clocks and caches
      hipLaunchKernelGGL(kernel, dim3(blocks), dim3(threads), 0, 0, out, clk, 1.0f);
      e = hipGetLastError();
      if (e == hipSuccess) e = hipDeviceSynchronize();
    }
  };
#define KH_PROBE_MFMA_RUN(c, g, v) \
  if (e == hipSuccess && !known && chains == c && group == g && valu == v) run(mfma_valu_kernel<c, g, v>);
  KH_PROBE_MFMA_CASES(KH_PROBE_MFMA_RUN)
#undef KH_PROBE_MFMA_RUN
  uint64_t h[4 * 8] = {};
  if (e == hipSuccess && known) e = hipMemcpy(h, clk, 4 * waves * sizeof(uint64_t), hipMemcpyDeviceToHost);
  if (out) (void)hipFree(out);
  if (clk) (void)hipFree(clk);
  if (e != hipSuccess) {
    err = std::string("MFMA probe: ") + hipGetErrorString(e);
    return e;
  }
  if (!known) {
    err = "MFMA probe: no kernel for this (chains, group, valu) combination";
    return hipErrorInvalidValue;
  }
  // shader cycles per MFMA per SIMD (every SIMD issues kIters * 32 per wave)
  uint64_t c0 = h[0], c1 = h[1], r0 = h[2], r1 = h[3];
  for (int w = 1; w < waves; ++w) {
    c0 = std::min(c0, h[4 * w]), c1 = std::max(c1, h[4 * w + 1]);
    r0 = std::min(r0, h[4 * w + 2]), r1 = std::max(r1, h[4 * w + 3]);
  }
  out2[0] = (double)(c1 - c0) / ((double)kIters * 32 * waves_per_simd);
  out2[1] = r1 > r0 ? (double)(c1 - c0) / ((double)(r1 - r0) / 100e6) / 1e9 : 0.0;
  return hipSuccess;
}

}  // namespace kh
