// kh_gemm.hip - the matmul family (K-MM): C[b] = epilogue(A[b] @ B[b]) on the
// CDNA4 matrix cores.
//
// Replaces the reference's tl.dot kernel with fused epilogue
// (kiln/gpu/codegen.py:484-530) and its tile heuristic (552-598). MI355X design:
//   * fp32 operands on v_mfma_f32_32x32x2_f32 / v_mfma_f32_16x16x4_f32 (full
//     fp32 products, fp32 accumulation). Tiles are sized for wave64: a
//     workgroup of WM x WN x WK waves computes a BM x BN tile; each wave owns a
//     (BM/WM) x (BN/WN) sub-tile and, with WK > 1, a 1/WK share of every K
//     step (the partial tiles are summed in LDS in a fixed order);
//   * K advances in BK steps through two LDS buffers: the next step's global
//     loads (128-bit along K for A, along N for B) are in flight while the
//     matrix cores work on the current one;
//   * the reduction order over K inside a step is permuted so each lane reads
//     its A operand as 128-bit LDS vectors (a dot product is order-free; the
//     same permutation is applied to A and B);
//   * the epilogue stages the accumulator tile through LDS and runs the same
//     instruction tape as the elementwise family on row-contiguous groups of
//     4, so bias, GELU, residual, scale and mask operands are read with
//     coalesced 128-bit loads and the output is written with 128-bit stores;
//   * split-K (for M = 128 shapes that cannot fill 256 CUs): each split writes
//     its raw partial tile, dense [split][batch][M][N], to the workspace and
//     a second kernel sums them in split order and runs the epilogue. The
//     kernel boundary is the only synchronisation (a per-tile device-scope
//     counter would need an L2 write-back per workgroup across 8 XCDs), and
//     the fixed summation order keeps the result independent of scheduling;
//   * workgroup ids are remapped so each XCD (own L2) receives a contiguous
//     block of tiles.
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

template <int MT>
struct Mfma;

template <>
struct Mfma<32> {
  typedef f32x16 acc_t;
  static constexpr int kRegs = 16;
  __device__ static acc_t mma(float a, float b, acc_t c) { return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0); }
  // Row within the 32x32 block held by accumulator register i of `lane`
  // (the column is lane % 32).
  __device__ static int row(int i, int lane) { return (i >> 2) * 8 + (lane >> 5) * 4 + (i & 3); }
};

template <>
struct Mfma<16> {
  typedef f32x4 acc_t;
  static constexpr int kRegs = 4;
  __device__ static acc_t mma(float a, float b, acc_t c) { return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0); }
  __device__ static int row(int i, int lane) { return (lane >> 4) * 4 + i; }
};

// XCD-aware tile order: hardware hands consecutive workgroup ids to the 8 XCDs
// round-robin; remap so XCD x sees a contiguous range of tiles.
__device__ __forceinline__ int xcd_remap(int id, int n) {
  constexpr int kXcd = 8;
  if (n % kXcd) return id;
  return (id % kXcd) * (n / kXcd) + id / kXcd;
}

template <int BM, int BN, int BK, int WM, int WN, int WK, int MT>
__global__ __launch_bounds__(64 * WM * WN * WK) void gemm_f32_kernel(const GemmArgs a) {
  constexpr int kThreads = 64 * WM * WN * WK;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / MT, FN = TN / MT;
  constexpr int G = 64 / MT;   // lane groups = K values one MFMA consumes
  constexpr int KW = BK / WK;  // K per wave per step
  constexpr int KG = KW / G;   // K per lane group per step
  // LDS: A as [m][k] (row stride BK + 4: 16-byte aligned rows, conflict-free
  // 128-bit reads), B transposed to [n][k] (row stride BK + 2: conflict-free
  // 64-bit reads and conflict-free transposing writes), both double-buffered.
  constexpr int A_STRIDE = BK + 4, B_STRIDE = BK + 2, C_STRIDE = BN + 4;
  constexpr int A_FLOATS = BM * A_STRIDE, B_FLOATS = BN * B_STRIDE;
  constexpr int AB_FLOATS = 2 * (A_FLOATS + B_FLOATS);
  constexpr int C_FLOATS = BM * C_STRIDE;
  constexpr int LDS_FLOATS = AB_FLOATS > C_FLOATS ? AB_FLOATS : C_FLOATS;
  constexpr int A_VECS = BM * BK / 4, B_VECS = BK * BN / 4;
  constexpr int A_LOADS = (A_VECS + kThreads - 1) / kThreads;
  constexpr int B_LOADS = (B_VECS + kThreads - 1) / kThreads;
  static_assert(TM % MT == 0 && TN % MT == 0, "wave tile must be a multiple of the MFMA tile");
  static_assert(KG % 4 == 0, "each lane group needs a multiple of 4 K values per step");
  static_assert(BK % 8 == 0 && BN % 32 == 0 && B_VECS % 64 == 0, "B load mapping");
  static_assert(LDS_FLOATS * 4 <= 160 * 1024, "LDS");
  using M = Mfma<MT>;
  typedef typename M::acc_t acc_t;

  __shared__ __attribute__((aligned(16))) float lds[LDS_FLOATS];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wk = wave / (WM * WN);
  const int wm = (wave % (WM * WN)) / WN;
  const int wn = wave % WN;
  const int n_tiles = a.tiles_m * a.tiles_n;
  const int tile = xcd_remap(blockIdx.x, n_tiles);
  const int tm = tile / a.tiles_n, tn = tile % a.tiles_n;
  const int bidx = blockIdx.y, split = blockIdx.z;
  const int m0 = tm * BM, n0 = tn * BN;
  const int k_begin = split * a.k_per_split;
  const int k_end = min(a.K, k_begin + a.k_per_split);
  const float *Ab = a.A + (int64_t)bidx * a.sa_b;
  const float *Bb = a.B + (int64_t)bidx * a.sb_b;
  // A float4 i of a step: row idx / (BK/4), k quad idx % (BK/4) (rows of BK
  // contiguous floats). B float4 i: each wave covers 8 k-rows x 8 n-quads
  // (128 contiguous bytes per row), so the transposing LDS writes hit 32
  // distinct banks.
  auto a_pos = [&](int i, int &r, int &kq) {
    const int idx = tid + i * kThreads;
    r = idx / (BK / 4), kq = idx % (BK / 4);
  };
  auto b_pos = [&](int i, int &kr, int &nq) {
    const int idx = tid + i * kThreads;
    const int c = idx >> 6;
    kr = (c % (BK / 8)) * 8 + ((idx & 63) >> 3);
    nq = (c / (BK / 8)) * 8 + (idx & 7);
  };
  const bool interior = m0 + BM <= a.M && n0 + BN <= a.N && a.a_vec && a.b_vec &&
                        (k_end - k_begin) % BK == 0;

  float4 ra[A_LOADS], rb[B_LOADS];
  // `fast_tag` is std::true_type for interior tiles: unconditional 128-bit
  // loads, no control flow between them, so every load of a step is in flight
  // at once. Edge tiles use the guarded path.
  auto load_step = [&](int k0, auto fast_tag) {
    constexpr bool fast = decltype(fast_tag)::value;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int r, kq;
      a_pos(i, r, kq);
      const int m = m0 + r, k = k0 + kq * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      const bool in_tile = A_VECS % kThreads == 0 || tid + i * kThreads < A_VECS;
      if constexpr (fast) {
        if (in_tile) v = *reinterpret_cast<const float4 *>(Ab + (int64_t)m * a.sa_m + k);
      } else if (in_tile && m < a.M) {
        const float *p = Ab + (int64_t)m * a.sa_m;
        if (a.a_vec && k + 3 < k_end) {
          v = *reinterpret_cast<const float4 *>(p + k);
        } else {
          if (k + 0 < k_end) v.x = p[(int64_t)(k + 0) * a.sa_k];
          if (k + 1 < k_end) v.y = p[(int64_t)(k + 1) * a.sa_k];
          if (k + 2 < k_end) v.z = p[(int64_t)(k + 2) * a.sa_k];
          if (k + 3 < k_end) v.w = p[(int64_t)(k + 3) * a.sa_k];
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      int kr, nq;
      b_pos(i, kr, nq);
      const int k = k0 + kr, n = n0 + nq * 4;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      const bool in_tile = B_VECS % kThreads == 0 || tid + i * kThreads < B_VECS;
      if constexpr (fast) {
        if (in_tile) v = *reinterpret_cast<const float4 *>(Bb + (int64_t)k * a.sb_k + n);
      } else if (in_tile && k < k_end) {
        const float *p = Bb + (int64_t)k * a.sb_k;
        if (a.b_vec && n + 3 < a.N) {
          v = *reinterpret_cast<const float4 *>(p + n);
        } else {
          if (n + 0 < a.N) v.x = p[(int64_t)(n + 0) * a.sb_n];
          if (n + 1 < a.N) v.y = p[(int64_t)(n + 1) * a.sb_n];
          if (n + 2 < a.N) v.z = p[(int64_t)(n + 2) * a.sb_n];
          if (n + 3 < a.N) v.w = p[(int64_t)(n + 3) * a.sb_n];
        }
      }
      rb[i] = v;
    }
  };
  auto store_step = [&](int buf) {
    float *As = lds + buf * (A_FLOATS + B_FLOATS);
    float *Bs = As + A_FLOATS;
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      int r, kq;
      a_pos(i, r, kq);
      if (A_VECS % kThreads == 0 || tid + i * kThreads < A_VECS)
        *reinterpret_cast<float4 *>(As + r * A_STRIDE + kq * 4) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      int kr, nq;
      b_pos(i, kr, nq);
      if (B_VECS % kThreads == 0 || tid + i * kThreads < B_VECS) {
        float *b = Bs + (nq * 4) * B_STRIDE + kr;
        b[0] = rb[i].x;
        b[B_STRIDE] = rb[i].y;
        b[2 * B_STRIDE] = rb[i].z;
        b[3 * B_STRIDE] = rb[i].w;
      }
    }
  };

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < M::kRegs; ++r) acc[i][j][r] = 0.0f;

  const int g = lane / MT, li = lane % MT;
  const int kb = wk * KW + g * KG;
  const int n_steps = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;
  auto main_loop = [&](auto fast_tag) {
  if (n_steps > 0) {
    load_step(k_begin, fast_tag);
    store_step(0);
  }
  __syncthreads();
  for (int s = 0; s < n_steps; ++s) {
    const int buf = s & 1;
    if (s + 1 < n_steps) load_step(k_begin + (s + 1) * BK, fast_tag);
    const float *As = lds + buf * (A_FLOATS + B_FLOATS) + (wm * TM + li) * A_STRIDE + kb;
    const float *Bs = lds + buf * (A_FLOATS + B_FLOATS) + A_FLOATS + (wn * TN + li) * B_STRIDE + kb;
    // fragments of 4 K values, double-buffered in registers
    float4 av[2][FM];
    float2 bv[2][FN][2];
    auto read_frag = [&](int set, int j4) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
        av[set][fm] = *reinterpret_cast<const float4 *>(As + fm * MT * A_STRIDE + j4);
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        bv[set][fn][0] = *reinterpret_cast<const float2 *>(Bs + fn * MT * B_STRIDE + j4);
        bv[set][fn][1] = *reinterpret_cast<const float2 *>(Bs + fn * MT * B_STRIDE + j4 + 2);
      }
    };
    read_frag(0, 0);
#pragma unroll
    for (int j4 = 0; j4 < KG; j4 += 4) {
      const int cur = (j4 / 4) & 1;
      if (j4 + 4 < KG) read_frag(cur ^ 1, j4 + 4);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          const float4 A4 = av[cur][fm];
          const float x = jj == 0 ? A4.x : jj == 1 ? A4.y : jj == 2 ? A4.z : A4.w;
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            const float2 B2 = bv[cur][fn][jj >> 1];
            acc[fm][fn] = M::mma(x, (jj & 1) ? B2.y : B2.x, acc[fm][fn]);
          }
        }
      }
    }
    if (s + 1 < n_steps) store_step(buf ^ 1);
    __syncthreads();
  }
  };
  if (interior) main_loop(std::true_type{});
  else main_loop(std::false_type{});

  // Stage the tile in LDS (the K-split wave groups add in a fixed order).
  float *Cs = lds;
#pragma unroll
  for (int w = 0; w < WK; ++w) {
    if (wk == w) {
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int r = 0; r < M::kRegs; ++r) {
            float *c = Cs + (wm * TM + fm * MT + M::row(r, lane)) * C_STRIDE + wn * TN + fn * MT + li;
            *c = w == 0 ? acc[fm][fn][r] : *c + acc[fm][fn][r];
          }
    }
    __syncthreads();
  }

  constexpr int GROUPS = BM * BN / 4;
  if (a.splitk > 1) {
    // raw partial tile -> dense [split][batch][M][N]; the reduce kernel adds
    // the splits and runs the epilogue
    float *part = a.ws_partial + ((int64_t)split * a.batch + bidx) * (int64_t)a.M * a.N;
    const bool vec = (a.N & 3) == 0;
    for (int q = tid; q < GROUPS; q += kThreads) {
      const int r = q / (BN / 4), c = (q % (BN / 4)) * 4;
      const int m = m0 + r, n = n0 + c;
      if (m >= a.M || n >= a.N) continue;
      const float *src = Cs + r * C_STRIDE + c;
      float *dst = part + (int64_t)m * a.N + n;
      if (vec) {
        *reinterpret_cast<float4 *>(dst) = *reinterpret_cast<const float4 *>(src);
      } else {
        for (int i = 0; i < 4 && n + i < a.N; ++i) dst[i] = src[i];
      }
    }
    return;
  }
  for (int q = tid; q < GROUPS; q += kThreads) {
    const int r = q / (BN / 4), c = (q % (BN / 4)) * 4;
    const int m = m0 + r, n = n0 + c;
    if (m >= a.M || n >= a.N) continue;
    Vec<4> v;
    const float4 p = *reinterpret_cast<const float4 *>(Cs + r * C_STRIDE + c);
    v.v[0] = p.x, v.v[1] = p.y, v.v[2] = p.z, v.v[3] = p.w;
    run_epilogue(a, bidx, m, n, min(4, a.N - n), v);
  }
}

// ---------------------------------------------------------------------------
// Host side.

struct TileCfg {
  int bm, bn, bk, wm, wn, wk, mt;
};

#define KH_GEMM_CONFIGS(X)        \
  X(0, 128, 128, 32, 2, 2, 1, 32) \
  X(1, 128, 192, 32, 2, 2, 1, 32) \
  X(2, 256, 128, 32, 2, 2, 1, 32) \
  X(3, 64, 64, 32, 2, 2, 1, 32)   \
  X(4, 64, 128, 32, 2, 2, 1, 32)  \
  X(5, 128, 64, 32, 2, 2, 1, 32)  \
  X(6, 32, 64, 32, 1, 2, 2, 32)   \
  X(7, 32, 32, 32, 1, 1, 4, 32)   \
  X(8, 64, 64, 32, 1, 1, 4, 32)   \
  X(9, 32, 32, 32, 2, 2, 1, 16)   \
  X(10, 16, 64, 32, 1, 4, 1, 16)  \
  X(11, 64, 32, 32, 2, 2, 1, 16)  \
  X(12, 128, 128, 32, 4, 2, 1, 32) \
  X(13, 128, 192, 32, 4, 2, 1, 32) \
  X(14, 256, 128, 32, 4, 2, 1, 32) \
  X(15, 64, 128, 64, 2, 2, 1, 32)  \
  X(16, 128, 64, 64, 2, 2, 1, 32)  \
  X(17, 64, 64, 64, 2, 2, 1, 32)

constexpr TileCfg kConfigs[] = {
#define KH_CFG_ROW(id, bm, bn, bk, wm, wn, wk, mt) {bm, bn, bk, wm, wn, wk, mt},
    KH_GEMM_CONFIGS(KH_CFG_ROW)
#undef KH_CFG_ROW
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

hipError_t launch_config(int id, const GemmArgs &a, dim3 grid, hipStream_t stream) {
  switch (id) {
#define KH_CFG_CASE(cid, bm, bn, bk, wm, wn, wk, mt)                                                          \
  case cid:                                                                                                  \
    hipLaunchKernelGGL((gemm_f32_kernel<bm, bn, bk, wm, wn, wk, mt>), grid, dim3(64 * wm * wn * wk), 0, stream, \
                       a);                                                                                   \
    break;
    KH_GEMM_CONFIGS(KH_CFG_CASE)
#undef KH_CFG_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

class GemmOp final : public Op {
 public:
  GemmArgs args{};
  int cfg = 0;
  dim3 grid;
  size_t n_partials = 0;
  bool a_vec_layout = false, b_vec_layout = false;
  uint32_t e_vec_candidates = 0;

  hipError_t launch(float *const *ptrs, uint32_t *counters, float *partials, hipStream_t stream) override {
    GemmArgs a = args;
    a.A = ptrs[0];
    a.B = ptrs[1];
    a.a_vec = a_vec_layout && (reinterpret_cast<uintptr_t>(ptrs[0]) & 15) == 0;
    a.b_vec = b_vec_layout && (reinterpret_cast<uintptr_t>(ptrs[1]) & 15) == 0;
    a.e_vec_mask = 0;
    for (int j = 0; j < a.n_refs; ++j) {
      a.eptr[j] = ptrs[2 + j];
      if ((e_vec_candidates >> j & 1) && (reinterpret_cast<uintptr_t>(ptrs[2 + j]) & 15) == 0)
        a.e_vec_mask |= 1u << j;
    }
    a.ws_partial = partials;
    if (a.M == 0 || a.N == 0 || a.batch == 0) return hipSuccess;
    if (a.splitk > 1 && !partials) return hipErrorInvalidValue;
    const hipError_t e = launch_config(cfg, a, grid, stream);
    if (e != hipSuccess || a.splitk == 1) return e;
    return launch_splitk_reduce(a, current_device().cus, stream);
  }
  size_t partial_floats() const override { return n_partials; }
};

}  // namespace

int gemm_config_count() { return kNumConfigs; }

bool gemm_config(int id, int32_t out8[8]) {
  if (id < 0 || id >= kNumConfigs) return false;
  const TileCfg &t = kConfigs[id];
  const int32_t v[8] = {t.bm, t.bn, t.bk, t.wm, t.wn, t.wk, t.mt, KH_PREC_FP32};
  std::memcpy(out8, v, sizeof(v));
  return true;
}

// Shared with the GEMV factory: validate and fill the epilogue part of GemmArgs.
bool fill_epilogue(const kh_launch &L, GemmArgs &a, uint32_t &vec_candidates, std::string &err) {
  a.n_refs = L.n_refs - 2;
  a.n_insns = L.n_insns;
  if (a.n_refs < 1) {
    err = "matmul: no epilogue operand (the output)";
    return false;
  }
  TapeInfo info;
  if (!check_tape(L, 0, L.n_insns, false, info, err, 2)) return false;
  if (info.slots > kFastSlots) {
    err = "matmul: epilogue needs more than 8 slots";
    return false;
  }
  if (!info.stored) {
    err = "matmul: epilogue stores nothing";
    return false;
  }
  a.n_pre = info.leading_loads;
  std::memcpy(a.insns, L.insns, sizeof(kh_insn) * L.n_insns);
  for (int i = 0; i < L.n_insns; ++i) {
    if (a.insns[i].op == KH_OP_LOAD) a.insns[i].a -= 2;
    if (a.insns[i].op == KH_OP_STORE) a.insns[i].dst -= 2;
  }
  vec_candidates = 0;
  a.e_bcast_mask = 0;
  for (int j = 0; j < a.n_refs; ++j) {
    const kh_ref &r = L.refs[2 + j];
    for (int d = 0; d < 3; ++d) a.estride[j][d] = r.strides[d];
    if (r.strides[2] == 0 && (info.loaded >> (j + 2) & 1)) a.e_bcast_mask |= 1u << j;
    if (r.strides[2] == 1 && r.offset % 4 == 0 && r.strides[0] % 4 == 0 && r.strides[1] % 4 == 0)
      vec_candidates |= 1u << j;
  }
  return true;
}

std::unique_ptr<Op> make_gemm(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  auto op = std::make_unique<GemmOp>();
  GemmArgs &a = op->args;
  if (L.n_refs < 3 || L.n_refs > KH_MAX_REFS) {
    err = "matmul: bad operand count";
    return nullptr;
  }
  const int64_t batch = L.gemm[0], M = L.gemm[1], N = L.gemm[2], K = L.gemm[3];
  if (batch < 0 || M < 0 || N < 0 || K < 0 || batch >= (1 << 16) || M >= (1ll << 30) || N >= (1ll << 30) ||
      K >= (1ll << 30)) {
    unsupported = true;
    err = "matmul: sizes out of range for the GEMM family";
    return nullptr;
  }
  const int cfg = L.cfg[1];
  if (cfg < 0 || cfg >= kNumConfigs) {
    err = "matmul: unknown tile configuration " + std::to_string(cfg);
    return nullptr;
  }
  if (L.cfg[3] != KH_PREC_FP32) {
    unsupported = true;
    err = "matmul: precision not compiled into this library";
    return nullptr;
  }
  const TileCfg &t = kConfigs[cfg];
  a.batch = (int)batch, a.M = (int)M, a.N = (int)N, a.K = (int)K;
  a.sa_b = L.refs[0].strides[0], a.sa_m = L.refs[0].strides[1], a.sa_k = L.refs[0].strides[2];
  a.sb_b = L.refs[1].strides[0], a.sb_k = L.refs[1].strides[1], a.sb_n = L.refs[1].strides[2];
  op->a_vec_layout = a.sa_k == 1 && L.refs[0].offset % 4 == 0 && a.sa_m % 4 == 0 && a.sa_b % 4 == 0;
  op->b_vec_layout = a.sb_n == 1 && L.refs[1].offset % 4 == 0 && a.sb_k % 4 == 0 && a.sb_b % 4 == 0;
  if (!fill_epilogue(L, a, op->e_vec_candidates, err)) return nullptr;
  a.tiles_m = (int)((M + t.bm - 1) / t.bm);
  a.tiles_n = (int)((N + t.bn - 1) / t.bn);
  int splitk = std::max(1, L.cfg[2]);
  const int k_steps = (int)std::max<int64_t>(1, (K + t.bk - 1) / t.bk);
  splitk = std::min(splitk, k_steps);
  a.k_per_split = ((k_steps + splitk - 1) / splitk) * t.bk;
  splitk = (int)std::max<int64_t>(1, (K + a.k_per_split - 1) / std::max(1, a.k_per_split));
  if (K == 0) splitk = 1, a.k_per_split = 0;
  a.splitk = splitk;
  const int64_t n_tiles = (int64_t)a.tiles_m * a.tiles_n;
  if (n_tiles >= (1ll << 31)) {
    unsupported = true;
    err = "matmul: too many tiles";
    return nullptr;
  }
  op->cfg = cfg;
  op->grid = dim3((unsigned)n_tiles, (unsigned)batch, (unsigned)splitk);
  if (splitk > 1) {
    op->n_partials = (size_t)splitk * batch * M * N;
  }
  return op;
}

}  // namespace kh
