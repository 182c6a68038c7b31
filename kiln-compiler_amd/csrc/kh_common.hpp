// kh_common.hpp - device helpers shared by Kiln's gfx950 kernel families:
// scalar math of the fused op set, the instruction-tape interpreter, wave64
// reductions and fast integer division for index decomposition.
//
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kiln_hip.h"
#include "kh_semantics.hpp"

namespace kh {

constexpr int kWave = 64;

// ---------------------------------------------------------------------------
// Fast unsigned division by a runtime constant (n, d < 2^31), the round-up
// multiply-high method (Granlund & Montgomery 1994): q = (umulhi(n, m) + n) >> s.
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  FastDiv f;
  f.d = d;
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  f.s = s;
  f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
  return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
  return (__umulhi(n, f.m) + n) >> f.s;
}

// Scalar math of the op set (op_scalar, nan_max, GELU forms ...) lives in
// kh_semantics.hpp, shared with the host interpreter of plans.

// 128-bit load marked non-temporal
__device__ __forceinline__ float4 load_stream4(const float *p) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const f32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t *>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}

// 128-bit store marked non-temporal (streamed past the caches): for
// outputs of memory-bound kernels
__device__ __forceinline__ void store_stream(float *p, float x, float y, float z, float w) {
  typedef float f32x4_t __attribute__((ext_vector_type(4)));
  const f32x4_t v = {x, y, z, w};
  __builtin_nontemporal_store(v, reinterpret_cast<f32x4_t *>(p));
}

// Four values rounded to bf16 (nearest even, as every bf16 input of the
// matmul family is rounded) and stored as one 64-bit write at element `i` of
// the bf16 array `p`: the output of a producer whose only consumer is a bf16
// matmul.
__device__ __forceinline__ void store_bf16x4(void *p, int64_t i, float x, float y, float z, float w) {
  typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
  const bf16x4_t v = {(__bf16)x, (__bf16)y, (__bf16)z, (__bf16)w};
  *reinterpret_cast<bf16x4_t *>(static_cast<__bf16 *>(p) + i) = v;
}

// ---------------------------------------------------------------------------
// wave64 all-reductions: DPP within rows of 16 lanes, then cross-row swizzles.
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// The two cross-row steps exchange register values between rows with
// v_permlane16_swap (rows 2k and 2k + 1) and v_permlane32_swap (lane halves)
// instead of LDS permutes: each returns the pair (value of the even row or
// low half, value of the odd row or high half) in every lane of the pair, so
// combining the two gives every lane the same value, and the result is the
// one the xor butterfly over lanes l ^ 16, l ^ 32 gives (the same two
// operands per step; fp addition and max are commutative).
__device__ __forceinline__ float2 row_pair(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float2 half_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp<0x141>(v);  // row_half_mirror
  v += dpp<0x140>(v);  // row_mirror
  float2 p = row_pair(v);
  v = p.x + p.y;
  p = half_pair(v);
  return p.x + p.y;
}

// NaN-propagating at every step (v_max_f32 alone returns the non-NaN operand),
// so a NaN held by any lane reaches all lanes, like max over the row.
__device__ __forceinline__ float wave_max(float v) {
  v = nan_max(v, dpp<0xB1>(v));
  v = nan_max(v, dpp<0x4E>(v));
  v = nan_max(v, dpp<0x141>(v));
  v = nan_max(v, dpp<0x140>(v));
  float2 p = row_pair(v);
  v = nan_max(p.x, p.y);
  p = half_pair(v);
  return nan_max(p.x, p.y);
}

// ---------------------------------------------------------------------------
// Instruction-tape interpreter pieces. A thread evaluates a tape on a group of
// 4 adjacent elements, so each (wave-uniform) instruction is decoded once per
// 4 elements. Kernels keep registers and prefetched operands in small arrays
// indexed by wave-uniform numbers.
template <int V>
struct Vec {
  float v[V];
};

__device__ __forceinline__ Vec<4> splat4(float s) {
  Vec<4> o;
  o.v[0] = o.v[1] = o.v[2] = o.v[3] = s;
  return o;
}

// Slot bank: NS slots of 4 floats in one flat array. With NS = 8 LLVM keeps
// the array in VGPRs and indexes it with s_set_gpr_idx for a wave-uniform slot
// number; a larger bank (or two banks) is placed in scratch memory, so tapes
// that fit 8 slots use the VGPR variant.
constexpr int kFastSlots = 8;

template <int N>
__device__ __forceinline__ Vec<4> bank_get(const float (&b)[N], int s) {
  Vec<4> o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o.v[i] = b[(s & (N / 4 - 1)) * 4 + i];
  return o;
}

template <int N>
__device__ __forceinline__ void bank_set(float (&b)[N], int s, const Vec<4> &v) {
#pragma unroll
  for (int i = 0; i < 4; ++i) b[(s & (N / 4 - 1)) * 4 + i] = v.v[i];
}

// One tape instruction (not STORE/RSUM/RMAX) on 4 lanes of data. The switch
// on the (wave-uniform) opcode is outside the element loop; each case calls
// op_scalar with a constant opcode, which folds to that op's expression.
__device__ __forceinline__ Vec<4> apply4(int op, const Vec<4> &x, const Vec<4> &y) {
  Vec<4> r;
#define KH_OP_CASE(OP)                                                    \
  case OP:                                                                \
    _Pragma("unroll") for (int i = 0; i < 4; ++i) r.v[i] = op_scalar(OP, x.v[i], y.v[i]); \
    break;
  switch (op) {
    KH_OP_CASE(KH_OP_ADD) KH_OP_CASE(KH_OP_SUB) KH_OP_CASE(KH_OP_MUL) KH_OP_CASE(KH_OP_DIV)
    KH_OP_CASE(KH_OP_MAX) KH_OP_CASE(KH_OP_MIN) KH_OP_CASE(KH_OP_NEG) KH_OP_CASE(KH_OP_RELU)
    KH_OP_CASE(KH_OP_EXP) KH_OP_CASE(KH_OP_TANH) KH_OP_CASE(KH_OP_SIGMOID) KH_OP_CASE(KH_OP_ERF)
    KH_OP_CASE(KH_OP_GELU_TANH) KH_OP_CASE(KH_OP_GELU_ERF) KH_OP_CASE(KH_OP_RSQRT) KH_OP_CASE(KH_OP_SQRT)
    default: r = x;
  }
#undef KH_OP_CASE
  return r;
}

// Execute tape[begin, end) on slot bank `f` (NS slots). The first `n_pre`
// instructions are LOADs: they are issued together before any result is
// needed. `load(ref)` returns the 4 values of operand ref at the current
// elements, `store(ref, v)` writes them, `reduce(insn, v)` handles RSUM/RMAX.
template <int NS, class Load, class Store, class Reduce>
__device__ __forceinline__ void exec_tape(const kh_insn *tape, int begin, int end, int n_pre, float (&f)[NS * 4],
                                          Load &&load, Store &&store, Reduce &&reduce) {
  Vec<4> pre[kFastSlots];
#pragma unroll
  for (int i = 0; i < kFastSlots; ++i)
    if (i < n_pre) pre[i] = load(tape[begin + i].a);
#pragma unroll
  for (int i = 0; i < kFastSlots; ++i)
    if (i < n_pre) bank_set(f, tape[begin + i].dst, pre[i]);
  for (int pc = begin + n_pre; pc < end; ++pc) {
    const kh_insn in = tape[pc];
    if (in.op == KH_OP_LOAD) {
      bank_set(f, in.dst, load(in.a));
      continue;
    }
    const Vec<4> x = in.a == KH_SRC_IMM ? splat4(in.imm) : bank_get(f, in.a);
    if (in.op == KH_OP_STORE) {
      store(in.dst, x);
    } else if (in.op == KH_OP_RSUM || in.op == KH_OP_RMAX) {
      reduce(in, x);
    } else {
      const Vec<4> y = in.b == KH_SRC_IMM ? splat4(in.imm) : bank_get(f, in.b);
      bank_set(f, in.dst, apply4(in.op, x, y));
    }
  }
}

// ---------------------------------------------------------------------------
// bf16 operands of the matrix cores (round to nearest, ties to even).
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));

// Two fp32 values as bf16 in one word, a's bits low (one v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t r;
  r[0] = (__bf16)a, r[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, r);
}

// Eight fp32 values as one bf16 operand, one conversion per pair (element-wise
// assignments into the vector can cost the compiler a second conversion and a
// permute per pair).
__device__ __forceinline__ bf16x8_t pack_bf16x8(const float4 &x, const float4 &y) {
  return __builtin_bit_cast(bf16x8_t, make_uint4(pack_bf16x2(x.x, x.y), pack_bf16x2(x.z, x.w),
                                                 pack_bf16x2(y.x, y.y), pack_bf16x2(y.z, y.w)));
}

// x as its pair word (see split_bf16x8): bf16(x) low, bf16(x - bf16(x)) high
// (0 for a non-finite bf16(x)), returned as a float's bits for an fp32 store.
__device__ __forceinline__ float pair_word(float x) {
  const float hv = __uint_as_float(pack_bf16x2(x, x) & 0xffff0000u);
  const float lo = __builtin_isfinite(hv) ? x - hv : 0.0f;
  return __uint_as_float(pack_bf16x2(x, lo));
}

// Eight pair words (as stored by a pair-storing producer) as the hi and lo
// operands split_bf16x8 would make of the values they hold.
__device__ __forceinline__ void unpair_bf16x8(const float4 &x, const float4 &y, bf16x8_t &hi, bf16x8_t &lo) {
  const uint32_t w[8] = {__float_as_uint(x.x), __float_as_uint(x.y), __float_as_uint(x.z), __float_as_uint(x.w),
                         __float_as_uint(y.x), __float_as_uint(y.y), __float_as_uint(y.z), __float_as_uint(y.w)};
  uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = __builtin_amdgcn_perm(w[2 * e + 1], w[2 * e], 0x05040100u);
    l[e] = __builtin_amdgcn_perm(w[2 * e + 1], w[2 * e], 0x07060302u);
  }
  hi = __builtin_bit_cast(bf16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8_t, make_uint4(l[0], l[1], l[2], l[3]));
}

// Eight fp32 values as the two bf16 halves of a three-pass product:
// hi = bf16(x), lo = bf16(x - hi) (the difference is exact in fp32; a
// non-finite hi keeps lo 0), so x.y ~ x_lo y_hi + x_hi y_lo + x_hi y_hi with
// the dropped x_lo y_lo ~2^-16 of the product. CHECK = false for values that
// are finite or NaN (softmax probabilities), where the hi part alone already
// makes a NaN result. Per pair of values: two conversions, a byte permute and
// a mask to widen the hi halves back to fp32, two subtractions.
template <bool CHECK>
__device__ __forceinline__ void split_bf16x8(const float4 &x, const float4 &y, bf16x8_t &hi, bf16x8_t &lo) {
  const float v[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = pack_bf16x2(v[2 * e], v[2 * e + 1]);
    // (the low half through a byte permute: the compiler would otherwise
    // recompute it with a second conversion)
    const float h0 = __uint_as_float(__builtin_amdgcn_perm(h[e], h[e], 0x01000c0cu));
    const float h1 = __uint_as_float(h[e] & 0xffff0000u);
    float l0 = v[2 * e] - h0, l1 = v[2 * e + 1] - h1;
    if constexpr (CHECK) {
      l0 = __builtin_isfinite(h0) ? l0 : 0.0f;
      l1 = __builtin_isfinite(h1) ? l1 : 0.0f;
    }
    l[e] = pack_bf16x2(l0, l1);
  }
  hi = __builtin_bit_cast(bf16x8_t, make_uint4(h[0], h[1], h[2], h[3]));
  lo = __builtin_bit_cast(bf16x8_t, make_uint4(l[0], l[1], l[2], l[3]));
}

}  // namespace kh
