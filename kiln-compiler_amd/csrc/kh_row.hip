// kh_row.hip - the row family (K-ROW): reductions over the innermost dim plus
// the elementwise work around them (LayerNorm, softmax, any row program the
// fusion pass forms).
//
// Replaces the reference's one-program-per-row Triton kernel
// (kiln/gpu/codegen.py:312-430). MI355X design:
//   * LayerNorm and softmax, recognised by the host from the exact op
//     sequences the frontend emits (kiln/frontend/fx_import.py:212-230), run
//     one wave64 per row with the whole row in VGPRs (up to 4096 floats):
//     every lane moves 128-bit vectors of a contiguous 1 KiB span per step,
//     and the reductions are DPP row ops plus two cross-row swizzles;
//   * every other row program runs on the generic row kernel: one workgroup
//     per row, the instruction tape split into passes (one per reduction
//     level). A row that fits one chunk (workgroup x 4 floats) is read once
//     and stays in registers across passes; longer rows are processed in
//     chunks, each pass recomputing its elementwise values from the inputs,
//     so registers and memory stay constant for any row length (the
//     reference's chunked scheme, codegen.py:371-428).
#include <algorithm>
#include <cmath>
#include <cstring>

#include "kh_common.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

// ------------------------------------------------------------------------------
// Fast paths: one wave per row, NV float4 per lane.

struct LnArgs {
  const float *x;
  const float *gamma;   // may be null
  const float *beta;    // may be null
  float *out;           // (a bf16 array when out16)
  int64_t x_rs, out_rs; // row strides (elements)
  uint32_t rows, inner;
  float inv_n1, inv_n2, eps;
  int32_t out16;        // the output is bf16 (its consumer is a bf16 matmul)
  int32_t out_pair;     // the output is pair words (its consumer is a three-pass matmul)
};

// One row per wave and no grid-stride loop: the grid covers every row, so
// workgroups start and retire at different times and one wave's reductions
// overlap other waves' loads and stores.
// NTL: non-temporal input loads, for inputs larger than the Infinity Cache
// (as in softmax_kernel).
template <int NV, bool NTL>
__global__ __launch_bounds__(256) void layernorm_kernel(const LnArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row < a.rows) {
    const float *x = a.x + (int64_t)row * a.x_rs;
    float4 v[NV];
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t c = (i * 64 + lane) * 4;
      v[i] = c >= a.inner ? make_float4(0.f, 0.f, 0.f, 0.f)
             : NTL        ? load_stream4(x + c)
                          : *reinterpret_cast<const float4 *>(x + c);
      s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
    }
    const float mean = wave_sum(s) * a.inv_n1;
    float s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t c = (i * 64 + lane) * 4;
      if (c < a.inner) {
        v[i].x -= mean, v[i].y -= mean, v[i].z -= mean, v[i].w -= mean;
        s2 += (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
      }
    }
    const float rstd = rsqrtf(wave_sum(s2) * a.inv_n2 + a.eps);
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t c = (i * 64 + lane) * 4;
      if (c < a.inner) {
        float4 y = make_float4(v[i].x * rstd, v[i].y * rstd, v[i].z * rstd, v[i].w * rstd);
        if (a.gamma) {
          const float4 g = *reinterpret_cast<const float4 *>(a.gamma + c);
          y.x *= g.x, y.y *= g.y, y.z *= g.z, y.w *= g.w;
        }
        if (a.beta) {
          const float4 b = *reinterpret_cast<const float4 *>(a.beta + c);
          y.x += b.x, y.y += b.y, y.z += b.z, y.w += b.w;
        }
        if (a.out_pair) y = make_float4(pair_word(y.x), pair_word(y.y), pair_word(y.z), pair_word(y.w));
        if (a.out16) store_bf16x4(a.out, (int64_t)row * a.out_rs + c, y.x, y.y, y.z, y.w);
        else store_stream(a.out + (int64_t)row * a.out_rs + c, y.x, y.y, y.z, y.w);
      }
    }
  }
}

// exp(v - m) for the softmax row kernel; v - m is NaN for an infinite or NaN
// input, so the row turns NaN as in the reference
__device__ __forceinline__ float exp_shifted(float v, float m) {
  return __builtin_amdgcn_exp2f((v - m) * 1.4426950408889634f);
}

struct SmxArgs {
  const float *x;
  float *out;
  int64_t x_rs, out_rs;
  uint32_t rows, inner;
  int pre;        // 0 none, 1 multiply by `scale`, 2 divide by `scale`
  float scale;
};

// exp(v - m) as one v_exp_f32 of (v - m) log2(e): the two roundings of the
// argument give a relative error of about |v - m| * 1.2e-7 (below 1.1e-5 over
// the whole range |v - m| < 88 of normal results, below 1e-6 where
// |v - m| < 8); the quotient is a product with the row's reciprocal sum (one
// IEEE division per row).
// NTL: the input is read with non-temporal loads, for inputs larger than the
// 256 MB Infinity Cache (streamed once: 303 -> 292 us at 1.5 GiB per call);
// smaller inputs keep cached loads (a re-read input stays in the cache).
template <int NV, bool NTL>
__global__ __launch_bounds__(256) void softmax_kernel(const SmxArgs a) {
  const int lane = threadIdx.x & 63;
  const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row < a.rows) {
    const float *x = a.x + (int64_t)row * a.x_rs;
    float4 v[NV];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t c = (i * 64 + lane) * 4;
      if (c < a.inner) {
        v[i] = NTL ? load_stream4(x + c) : *reinterpret_cast<const float4 *>(x + c);
        if (a.pre == 1) v[i].x *= a.scale, v[i].y *= a.scale, v[i].z *= a.scale, v[i].w *= a.scale;
        if (a.pre == 2) v[i].x /= a.scale, v[i].y /= a.scale, v[i].z /= a.scale, v[i].w /= a.scale;
        m = nan_max(m, nan_max(nan_max(v[i].x, v[i].y), nan_max(v[i].z, v[i].w)));
      }
    }
    m = wave_max(m);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t c = (i * 64 + lane) * 4;
      if (c < a.inner) {
        v[i].x = exp_shifted(v[i].x, m), v[i].y = exp_shifted(v[i].y, m);
        v[i].z = exp_shifted(v[i].z, m), v[i].w = exp_shifted(v[i].w, m);
        s += (v[i].x + v[i].y) + (v[i].z + v[i].w);
      }
    }
    const float r = 1.0f / wave_sum(s);
    float *o = a.out + (int64_t)row * a.out_rs;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const uint32_t c = (i * 64 + lane) * 4;
      if (c < a.inner)
        store_stream(o + c, v[i].x * r, v[i].y * r, v[i].z * r, v[i].w * r);
    }
  }
}

// ------------------------------------------------------------------------------
// Generic row program.

struct RowArgs {
  int32_t n_refs, n_insns, n_passes, row_rank;
  uint32_t vec_mask, bcast_mask;
  uint32_t rows, inner;
  int8_t n_pre[KH_MAX_PASSES];
  FastDiv rdiv[KH_MAX_RANK];
  float *ptr[KH_MAX_REFS];
  int64_t rstride[KH_MAX_REFS][KH_MAX_RANK];
  int64_t istride[KH_MAX_REFS];
  kh_insn insns[KH_MAX_INSNS];
  kh_pass passes[KH_MAX_PASSES];
};

template <int T>
__device__ __forceinline__ float block_reduce(float v, bool is_max, float *smem) {
  v = is_max ? wave_max(v) : wave_sum(v);
  if (T == 64) return v;
  constexpr int W = T / 64;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) smem[threadIdx.x >> 6] = v;
  __syncthreads();
  float r = smem[0];
#pragma unroll
  for (int w = 1; w < W; ++w) r = is_max ? nan_max(r, smem[w]) : r + smem[w];
  return r;
}

template <int T, int NS>
__global__ __launch_bounds__(T) void row_kernel(const RowArgs a) {
  __shared__ float smem[T / 64];
  constexpr int kChunk = T * 4;
  for (uint32_t row = blockIdx.x; row < a.rows; row += gridDim.x) {
    uint32_t idx[KH_MAX_RANK];
    uint32_t rem = row;
#pragma unroll
    for (int d = KH_MAX_RANK - 1; d >= 0; --d) {
      if (d < a.row_rank) {
        const uint32_t q = fdiv(rem, a.rdiv[d]);
        idx[d] = rem - q * a.rdiv[d].d;
        rem = q;
      } else {
        idx[d] = 0;
      }
    }
    auto base = [&](int j) {
      int64_t off = 0;
#pragma unroll
      for (int d = 0; d < KH_MAX_RANK; ++d)
        if (d < a.row_rank) off += (int64_t)idx[d] * a.rstride[j][d];
      return a.ptr[j] + off;
    };
    float f[NS * 4];
#pragma unroll
    for (int i = 0; i < NS * 4; ++i) f[i] = 0.0f;
    for (int p = 0; p < a.n_passes; ++p) {
      const kh_pass P = a.passes[p];
#pragma unroll
      for (int s = 0; s < NS; ++s)
        if (P.acc_mask >> s & 1) bank_set(f, s, splat4((P.max_mask >> s & 1) ? -INFINITY : 0.0f));
      const int n_chunks = P.single_chunk ? 1 : (int)((a.inner + kChunk - 1) / kChunk);
      for (int c = 0; c < n_chunks; ++c) {
        const int32_t col0 = c * kChunk + threadIdx.x * 4;
        const int32_t valid = max(0, min(4, (int32_t)a.inner - col0));
        auto load = [&](int j) -> Vec<4> {
          const float *q = base(j);
          if (a.bcast_mask >> j & 1) return splat4(q[0]);
          Vec<4> out;
          if ((a.vec_mask >> j & 1) && valid == 4) {
            const float4 v = *reinterpret_cast<const float4 *>(q + col0);
            out.v[0] = v.x, out.v[1] = v.y, out.v[2] = v.z, out.v[3] = v.w;
          } else {
            const int64_t st = a.istride[j];
#pragma unroll
            for (int i = 0; i < 4; ++i) out.v[i] = i < valid ? q[(int64_t)(col0 + i) * st] : 0.0f;
          }
          return out;
        };
        auto store = [&](int j, const Vec<4> &v) {
          float *q = base(j);
          if ((a.vec_mask >> j & 1) && valid == 4) {
            *reinterpret_cast<float4 *>(q + col0) = make_float4(v.v[0], v.v[1], v.v[2], v.v[3]);
          } else {
            const int64_t st = a.istride[j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
              if (i < valid) q[(int64_t)(col0 + i) * st] = v.v[i];
          }
        };
        auto reduce = [&](const kh_insn &in, const Vec<4> &x) {
          Vec<4> acc = bank_get(f, in.dst);
          float r = acc.v[0];
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (i < valid) r = in.op == KH_OP_RSUM ? r + x.v[i] : nan_max(r, x.v[i]);
          acc.v[0] = r;
          bank_set(f, in.dst, acc);
        };
        exec_tape<NS>(a.insns, P.vec_begin, P.vec_end, a.n_pre[p], f, load, store, reduce);
      }
      // Combine the per-thread partials of this pass's reductions.
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        if (P.acc_mask >> s & 1) {
          const float v = block_reduce<T>(bank_get(f, s).v[0], P.max_mask >> s & 1, smem);
          bank_set(f, s, splat4(v));
        }
      }
      // Per-row scalar work (uniform across the workgroup).
      auto load_scalar = [&](int j) -> Vec<4> { return splat4(base(j)[0]); };
      auto store_scalar = [&](int j, const Vec<4> &v) {
        if (threadIdx.x == 0) base(j)[0] = v.v[0];
      };
      exec_tape<NS>(a.insns, P.post_begin, P.post_end, 0, f, load_scalar, store_scalar,
                    [](const kh_insn &, const Vec<4> &) {});
    }
  }
}

// ------------------------------------------------------------------------------
// Host side.

int pick_nv(int64_t inner) {
  static const int kNv[] = {1, 2, 3, 4, 6, 8, 12, 16};
  for (int nv : kNv)
    if (inner <= (int64_t)nv * 256) return nv;
  return 0;
}

#define KH_NV_SWITCH(NV, ...)                                   \
  switch (NV) {                                                 \
    case 1: { constexpr int kNV = 1; __VA_ARGS__; } break;      \
    case 2: { constexpr int kNV = 2; __VA_ARGS__; } break;      \
    case 3: { constexpr int kNV = 3; __VA_ARGS__; } break;      \
    case 4: { constexpr int kNV = 4; __VA_ARGS__; } break;      \
    case 6: { constexpr int kNV = 6; __VA_ARGS__; } break;      \
    case 8: { constexpr int kNV = 8; __VA_ARGS__; } break;      \
    case 12: { constexpr int kNV = 12; __VA_ARGS__; } break;    \
    default: { constexpr int kNV = 16; __VA_ARGS__; } break;    \
  }

constexpr int64_t kStreamBytes = 256ll << 20;  // the Infinity Cache

class LayerNormOp final : public Op {
 public:
  LnArgs args{};
  int x_ref = 0, g_ref = -1, b_ref = -1, out_ref = 0;
  int nv = 1, grid = 1;
  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    LnArgs a = args;
    a.x = ptrs[x_ref];
    a.gamma = g_ref >= 0 ? ptrs[g_ref] : nullptr;
    a.beta = b_ref >= 0 ? ptrs[b_ref] : nullptr;
    a.out = ptrs[out_ref];
    if (a.rows == 0) return hipSuccess;
    if ((int64_t)a.rows * a.inner * 4 >= kStreamBytes) {
      KH_NV_SWITCH(nv, hipLaunchKernelGGL((layernorm_kernel<kNV, true>), dim3(grid), dim3(256), 0, stream, a));
    } else {
      KH_NV_SWITCH(nv, hipLaunchKernelGGL((layernorm_kernel<kNV, false>), dim3(grid), dim3(256), 0, stream, a));
    }
    return hipGetLastError();
  }
};

class SoftmaxOp final : public Op {
 public:
  SmxArgs args{};
  int x_ref = 0, out_ref = 1;
  int nv = 1, grid = 1;
  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    SmxArgs a = args;
    a.x = ptrs[x_ref];
    a.out = ptrs[out_ref];
    if (a.rows == 0) return hipSuccess;
    if ((int64_t)a.rows * a.inner * 4 >= kStreamBytes) {
      KH_NV_SWITCH(nv, hipLaunchKernelGGL((softmax_kernel<kNV, true>), dim3(grid), dim3(256), 0, stream, a));
    } else {
      KH_NV_SWITCH(nv, hipLaunchKernelGGL((softmax_kernel<kNV, false>), dim3(grid), dim3(256), 0, stream, a));
    }
    return hipGetLastError();
  }
};

class RowOp final : public Op {
 public:
  RowArgs args{};
  uint32_t vec_candidates = 0;
  int threads = 256, grid = 1, slots = kFastSlots;
  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    RowArgs a = args;
    a.vec_mask = 0;
    for (int j = 0; j < a.n_refs; ++j) {
      a.ptr[j] = ptrs[j];
      if ((vec_candidates >> j & 1) && (reinterpret_cast<uintptr_t>(ptrs[j]) & 15) == 0) a.vec_mask |= 1u << j;
    }
    if (a.rows == 0 || a.inner == 0) return hipSuccess;
    if (slots <= kFastSlots) {
      if (threads == 64) hipLaunchKernelGGL((row_kernel<64, kFastSlots>), dim3(grid), dim3(64), 0, stream, a);
      else if (threads == 128) hipLaunchKernelGGL((row_kernel<128, kFastSlots>), dim3(grid), dim3(128), 0, stream, a);
      else hipLaunchKernelGGL((row_kernel<256, kFastSlots>), dim3(grid), dim3(256), 0, stream, a);
    } else {
      if (threads == 64) hipLaunchKernelGGL((row_kernel<64, KH_NREGS>), dim3(grid), dim3(64), 0, stream, a);
      else if (threads == 128) hipLaunchKernelGGL((row_kernel<128, KH_NREGS>), dim3(grid), dim3(128), 0, stream, a);
      else hipLaunchKernelGGL((row_kernel<256, KH_NREGS>), dim3(grid), dim3(256), 0, stream, a);
    }
    return hipGetLastError();
  }
};

// Row dims of ref j coalesced into one stride, or false if they do not collapse.
bool single_row_stride(const kh_launch &L, int j, int64_t &stride) {
  const int r = L.rank - 1;
  stride = 0;
  int64_t expect = -1;  // stride the next-outer dim must have
  bool first = true;
  for (int d = r - 1; d >= 0; --d) {
    if (L.shape[d] == 1) continue;
    const int64_t s = L.refs[j].strides[d];
    if (first) {
      stride = s;
      first = false;
    } else if (s != expect) {
      return false;
    }
    expect = s * L.shape[d];
  }
  return true;
}

bool vec_ok(const kh_launch &L, int j, int64_t rs) {
  const int r = L.rank - 1;
  return L.refs[j].strides[r] == 1 && L.shape[r] % 4 == 0 && L.refs[j].offset % 4 == 0 && rs % 4 == 0;
}

}  // namespace

std::unique_ptr<Op> make_row(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  if (L.rank < 1 || L.rank > KH_MAX_RANK || L.n_refs < 1 || L.n_refs > KH_MAX_REFS || L.n_passes < 1 ||
      L.n_passes > KH_MAX_PASSES) {
    err = "row: bad rank, operand or pass count";
    return nullptr;
  }
  TapeInfo info;
  if (!check_tape(L, 0, L.n_insns, true, info, err)) return nullptr;
  const int64_t inner = L.shape[L.rank - 1];
  int64_t rows = 1;
  for (int d = 0; d < L.rank; ++d)
    if (L.shape[d] < 0) {
      err = "row: negative extent";
      return nullptr;
    }
  for (int d = 0; d < L.rank - 1; ++d) rows *= L.shape[d];
  if (rows >= (1ll << 31) || inner >= (1ll << 31)) {
    unsupported = true;
    err = "row: more than 2^31 rows or columns";
    return nullptr;
  }
  const Device &dev = current_device();
  const int nv = pick_nv(inner);
  const uint32_t m16 = bf16_refs(L), mp = pair_refs(L);

  if (L.variant == KH_ROW_LAYERNORM || L.variant == KH_ROW_SOFTMAX) {
    // refs: [x, (gamma), (beta)] loads, then the output; cfg[4] = 1 if gamma, cfg[5] = 1 if beta.
    bool ok = nv > 0;
    int64_t rs[KH_MAX_REFS];
    for (int j = 0; ok && j < L.n_refs; ++j) ok = single_row_stride(L, j, rs[j]);
    if (ok && L.variant == KH_ROW_LAYERNORM) {
      const int has_g = L.cfg[4], has_b = L.cfg[5];
      const int x = 0, g = has_g ? 1 : -1, b = has_b ? 1 + has_g : -1, out = 1 + has_g + has_b;
      ok = L.n_refs == out + 1 && vec_ok(L, x, rs[x]) && vec_ok(L, out, rs[out]);
      if (ok && g >= 0) ok = vec_ok(L, g, 0) && rs[g] == 0;
      if (ok && b >= 0) ok = vec_ok(L, b, 0) && rs[b] == 0;
      if (ok) {
        auto op = std::make_unique<LayerNormOp>();
        op->x_ref = x, op->g_ref = g, op->b_ref = b, op->out_ref = out, op->nv = nv;
        op->args.x_rs = rs[x], op->args.out_rs = rs[out];
        op->args.rows = (uint32_t)rows, op->args.inner = (uint32_t)inner;
        op->args.inv_n1 = L.fparams[0], op->args.inv_n2 = L.fparams[1], op->args.eps = L.fparams[2];
        op->grid = (int)std::max<int64_t>(1, std::min<int64_t>((rows + 3) / 4, (int64_t)1 << 30));
        // a bf16 output: only the output, 8-byte aligned rows of 4-value groups
        if (m16 && (m16 != 1u << out || L.refs[out].offset % 4 || rs[out] % 4)) {
          unsupported = true;
          err = "row: bf16 storage only for a LayerNorm's output with 4-aligned rows";
          return nullptr;
        }
        op->args.out16 = m16 ? 1 : 0;
        // pair words: only the output
        if (mp && (mp != 1u << out || m16)) {
          unsupported = true;
          err = "row: pair storage only for a LayerNorm's output";
          return nullptr;
        }
        op->args.out_pair = mp ? 1 : 0;
        return op;
      }
    }
    if (m16 || mp) {
      unsupported = true;
      err = "row: bf16 or pair storage only for the one-wave LayerNorm kernel";
      return nullptr;
    }
    if (ok && L.variant == KH_ROW_SOFTMAX) {
      ok = L.n_refs == 2 && vec_ok(L, 0, rs[0]) && vec_ok(L, 1, rs[1]);
      if (ok) {
        auto op = std::make_unique<SoftmaxOp>();
        op->nv = nv;
        op->args.x_rs = rs[0], op->args.out_rs = rs[1];
        op->args.rows = (uint32_t)rows, op->args.inner = (uint32_t)inner;
        op->args.pre = L.cfg[4], op->args.scale = L.fparams[0];
        op->grid = (int)std::max<int64_t>(1, std::min<int64_t>((rows + 3) / 4, (int64_t)1 << 30));
        return op;
      }
    }
    // Not eligible for the fast path: the tape in the descriptor is complete, run it generically.
  }

  if (m16 || mp) {
    unsupported = true;
    err = "row: bf16 or pair storage only for the one-wave LayerNorm kernel";
    return nullptr;
  }
  auto op = std::make_unique<RowOp>();
  RowArgs &a = op->args;
  a.n_refs = L.n_refs;
  a.n_insns = L.n_insns;
  a.n_passes = L.n_passes;
  op->slots = info.slots;
  a.rows = (uint32_t)rows;
  a.inner = (uint32_t)inner;
  std::memcpy(a.insns, L.insns, sizeof(kh_insn) * L.n_insns);
  std::memcpy(a.passes, L.passes, sizeof(kh_pass) * L.n_passes);
  int rr = 0;
  for (int d = 0; d < L.rank - 1; ++d) {
    if (L.shape[d] <= 1 || rows == 0) continue;
    a.rdiv[rr] = make_fastdiv((uint32_t)L.shape[d]);
    for (int j = 0; j < L.n_refs; ++j) a.rstride[j][rr] = L.refs[j].strides[d];
    ++rr;
  }
  a.row_rank = rr;
  for (int j = 0; j < L.n_refs; ++j) {
    a.istride[j] = L.refs[j].strides[L.rank - 1];
    if ((a.istride[j] == 0 || inner == 1) && (info.loaded >> j & 1)) a.bcast_mask |= 1u << j;
    bool vec = a.istride[j] == 1 && inner % 4 == 0 && L.refs[j].offset % 4 == 0;
    for (int d = 0; vec && d < rr; ++d) vec = a.rstride[j][d] % 4 == 0;
    if (vec) op->vec_candidates |= 1u << j;
  }
  for (int p = 0; p < L.n_passes; ++p) {
    const kh_pass &P = L.passes[p];
    TapeInfo vi, pi;
    if (!check_tape(L, P.vec_begin, P.vec_end, true, vi, err) ||
        !check_tape(L, P.post_begin, P.post_end, false, pi, err)) {
      err = "row pass " + std::to_string(p) + ": " + err;
      return nullptr;
    }
    if ((P.acc_mask >> (op->slots > kFastSlots ? KH_NREGS : kFastSlots)) != 0 && op->slots <= kFastSlots) {
      err = "row: accumulator slot outside the tape's slots";
      return nullptr;
    }
    a.n_pre[p] = (int8_t)vi.leading_loads;
  }
  op->threads = inner <= 256 ? 64 : inner <= 512 ? 128 : 256;
  for (int p = 0; p < L.n_passes; ++p)
    if (L.passes[p].single_chunk && inner > (int64_t)op->threads * 4) {
      err = "row: single-chunk pass on a row longer than one chunk";
      return nullptr;
    }
  op->grid = (int)std::max<int64_t>(1, std::min<int64_t>(rows, (int64_t)dev.cus * 64));
  return op;
}

}  // namespace kh
