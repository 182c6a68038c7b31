// kh_semantics.hpp - scalar meaning of the fused op set, compiled for the GPU
// kernels and for the host interpreter of plans (kh_host.hip) alike, so the
// CPU test suite checks the same formulas the kernels run.
//
// The op semantics follow the reference's op table (kiln/ir/ops.py:48-97) and
// its GPU forms (kiln/gpu/codegen.py:53-88, 223-248). Where this file uses a
// different but more accurate formula it says so.
#pragma once

#include <hip/hip_runtime.h>

#include <cmath>

#include "kiln_hip.h"

namespace kh {

// max / min that return NaN when either operand is NaN (fmaxf alone returns
// the other operand), as torch.maximum and np.max do.
__host__ __device__ __forceinline__ float nan_max(float a, float b) {
  return (a != a) ? a : ((b != b) ? b : fmaxf(a, b));
}
__host__ __device__ __forceinline__ float nan_min(float a, float b) {
  return (a != a) ? a : ((b != b) ? b : fminf(a, b));
}

__host__ __device__ __forceinline__ float op_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

// GELU(tanh) evaluated as x * sigmoid(2u) = x / (1 + exp(-2u)),
// u = sqrt(2/pi) (x + 0.044715 x^3): algebraically equal to
// 0.5 x (1 + tanh(u)) but free of the 1 - e cancellation of the tanh form.
// On the GPU the exponential is the hardware base-2 one (v_exp_f32 of
// -2u * log2(e), relative error ~1e-6 for |2u| < 88, exact overflow to inf /
// underflow to 0) and the quotient a hardware reciprocal (v_rcp_f32, 1 ulp):
// GELU is the elementwise hot op of the MLP, and the error stays far inside
// the 1e-4 tolerance its results are checked at. The host uses exp2f and a
// division.
__host__ __device__ __forceinline__ float op_gelu_tanh(float x) {
  const float u = 0.7978845608028654f * fmaf(0.044715f * x, x * x, x);
#if defined(__HIP_DEVICE_COMPILE__)
  const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * u);  // exp(-2u) = 2^(-2u log2 e)
  return x * __builtin_amdgcn_rcpf(1.0f + e);
#else
  return x / (1.0f + exp2f(-2.8853900817779268f * u));
#endif
}

__host__ __device__ __forceinline__ float op_gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f));
}

__host__ __device__ __forceinline__ float op_rsqrt(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return rsqrtf(x);
#else
  return 1.0f / sqrtf(x);
#endif
}

// One tape instruction other than LOAD / STORE / RSUM / RMAX on one element.
__host__ __device__ __forceinline__ float op_scalar(int op, float u, float w) {
  switch (op) {
    case KH_OP_ADD: return u + w;
    case KH_OP_SUB: return u - w;
    case KH_OP_MUL: return u * w;
    case KH_OP_DIV: return u / w;
    case KH_OP_MAX: return nan_max(u, w);
    case KH_OP_MIN: return nan_min(u, w);
    case KH_OP_NEG: return -u;
    case KH_OP_RELU: return u != u ? u : fmaxf(u, 0.0f);
    case KH_OP_EXP: return expf(u);
    case KH_OP_TANH: return tanhf(u);
    case KH_OP_SIGMOID: return op_sigmoid(u);
    case KH_OP_ERF: return erff(u);
    case KH_OP_GELU_TANH: return op_gelu_tanh(u);
    case KH_OP_GELU_ERF: return op_gelu_erf(u);
    case KH_OP_RSQRT: return op_rsqrt(u);
    case KH_OP_SQRT: return sqrtf(u);
    default: return u;   // MOV
  }
}

}  // namespace kh
