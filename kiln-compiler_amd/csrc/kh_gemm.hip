// kh_gemm.hip - the matmul family (K-MM): C[b] = epilogue(A[b] @ B[b]) on the
// CDNA4 matrix cores.
//
// Replaces the reference's tl.dot kernel with fused epilogue
// (kiln/gpu/codegen.py:484-530) and its tile heuristic (552-598). Two kernels
// share the argument block, the epilogue tape and the split-K scheme:
//   * gemm3_f32_kernel (configurations 0-7), the main path: fp32 operands on
//     v_mfma_f32_16x16x4_f32, global memory copied straight into LDS
//     (global_load_lds) through a ring of LDS stages, two K steps ahead of the
//     matrix cores, XOR/rotation-swizzled LDS chunks, four or eight waves per
//     workgroup sized so that one to four workgroups share a CU; its design
//     notes are at the kernel;
//   * gemm_f32_kernel (configurations 8-14): register-staged loads into two
//     LDS buffers, v_mfma_f32_32x32x2_f32 or 16x16x4, and optionally K split
//     across the waves of a workgroup (WK > 1, summed in LDS in a fixed
//     order) for skinny tiles; it also serves operands too large for the
//     pipeline's 32-bit copy offsets.
// Both:
//   * permute the reduction order over K inside a step so each lane reads its
//     A operand as 128-bit LDS vectors (a dot product is order-free; the same
//     permutation is applied to A and B);
//   * stage the accumulator tile through LDS for the epilogue and run the same
//     instruction tape as the elementwise family on row-contiguous groups of
//     4, so bias, GELU, residual, scale and mask operands are read with
//     coalesced 128-bit loads and the output is written with 128-bit stores;
//   * split-K (for M = 128 shapes that cannot fill 256 CUs): each split writes
//     its raw partial tile, dense [split][batch][M][N], to the workspace and
//     a second kernel sums them in split order and runs the epilogue. The
//     kernel boundary is the only synchronisation (a per-tile device-scope
//     counter would need an L2 write-back per workgroup across 8 XCDs), and
//     the fixed summation order keeps the result independent of scheduling;
//   * remap workgroup ids so each XCD (own L2) receives a contiguous block of
//     tiles.
#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_gemm_dev.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

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
  int tm, tn;
  tile_coords(blockIdx.x, a, tm, tn);
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
// Pipelined variant: global memory is copied straight into LDS
// (global_load_lds, 128-bit per lane for aligned row-major operands, 32-bit
// for any other strides) through a ring of NS LDS stages, NS - 1 steps ahead
// of the matrix cores, so no VGPRs hold data in flight and a load has NS - 1
// MFMA phases to arrive. (Rings deeper than 3 were measured on the benchmark
// shapes and won nowhere, so every configuration uses NS = 3.)
//   * K advances in steps of 32. Within a step, lane group g of an MFMA
//     (lanes l / 16) owns K values 8g .. 8g+7 and MFMA j consumes value 8g + j
//     in every group: each lane reads its A values as two 128-bit LDS vectors
//     and its B values as one 32-bit read per MFMA, and B keeps its global
//     [k][n] layout in LDS (no transpose);
//   * LDS holds 16-byte chunks. A row r (32 floats = 8 chunks) puts chunk c at
//     c ^ ((r ^ r/8) % 8); B row k of lane group g puts chunk c at
//     (c + 4g) mod (BN/4). The 128-bit A reads and the per-group 32-bit B
//     reads then hit distinct banks. A copy instruction writes 64 consecutive
//     chunks, so each lane fetches the global chunk its LDS position holds;
//   * each stage is its own LDS array and the loop is unrolled over the three
//     stages, so the compiler sees which copies a read depends on; before a
//     stage is read every wave waits for its own copies into it (vmcnt), then
//     a barrier publishes them;
//   * ragged edges: rows past M and columns past N are fetched from clamped,
//     valid addresses (their results are never stored); K values past the
//     end of the step range are fetched clamped and overwritten with zeros in
//     LDS before the barrier;
//   * the epilogue stages the accumulators through LDS per 16-row block and
//     runs the tape on row-contiguous groups of 4 (coalesced 128-bit operand
//     loads and stores).

// BF16B: B is a bf16 copy of a constant in [batch][N][K'] layout (K' = K
// rounded up to 8, zero padded) and the products run on
// v_mfma_f32_16x16x32_bf16 with A rounded to bf16 (round to nearest even) as
// its fragments are read; accumulation stays fp32. In a K step lane group g
// holds K values KG.g .. KG.g + KG-1 of A and of B (KG = BK / 4) - the same
// ownership as the fp32 path - and the step's BK / 32 MFMAs of one output
// block take them 8 at a time.
// X3 (with BF16B): three-pass bf16. B is [batch][N][2K'], row n holding
// bf16(w) in [0, K') and bf16(w - bf16(w)) in [K', 2K'); A splits the same
// way as its fragments are read, and a.b = a_lo.b_hi + a_hi.b_lo + a_hi.b_hi
// (the a_lo.b_lo term, ~2^-16 of the product, is dropped). A stage holds the
// B hi rows, then the B lo rows.
template <int BM, int BN, int BK, int WM, int WN, int NS, int VW, bool BF16B, bool X3 = false>
__global__ __launch_bounds__(64 * WM * WN, 2) void gemm3_f32_kernel(const GemmArgs a) {
  constexpr int MT = 16;
  constexpr int kWaves = WM * WN, kThreads = 64 * kWaves;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / MT, FN = TN / MT;
  constexpr int KG = BK / 4;            // K values per lane group per step
  constexpr int ACH = BK / 4;           // 16-byte chunks per A row
  static_assert(BK == 32 || BK == 64 || BK == 128, "K step");
  constexpr int CB = BK / 8;            // 16-byte chunks per bf16 B row
  constexpr int KB = BF16B ? BK / 32 : 1;  // bf16 MFMAs per output block per step
  constexpr int B_CH = BN / 4;          // chunks per fp32 B row
  // stage sizes in 4-byte words (a bf16 B stage is BN rows of 64 bytes)
  static_assert(BF16B || !X3, "three-pass bf16 needs the bf16 B layout");
  constexpr int B_HALF = BN * BK / 2;   // words of one bf16 copy of a B stage
  constexpr int A_FLOATS = BM * BK, B_FLOATS = BF16B ? B_HALF * (X3 ? 2 : 1) : BK * BN,
                STAGE = A_FLOATS + B_FLOATS;
  // B copy width in 4-byte words per lane
  constexpr int VB = BF16B ? 4 : VW;
  // copy instructions per wave per step: each covers 64 lanes x VW floats
  constexpr int A_INSN = A_FLOATS / (64 * VW), B_INSN = B_FLOATS / (64 * VB);
  constexpr int A_PER_WAVE = A_INSN / kWaves, B_PER_WAVE = B_INSN / kWaves;
  constexpr int COPIES = A_PER_WAVE + B_PER_WAVE;
  static_assert(VW == 4 || VW == 1, "copy width");
  static_assert(TM % MT == 0 && TN % MT == 0, "wave tile must be a multiple of the MFMA tile");
  static_assert(A_INSN % kWaves == 0 && B_INSN % kWaves == 0, "copy mapping");
  static_assert(BF16B || (BN % 16 == 0 && B_CH >= 16), "B chunk rotation");
  static_assert(NS >= 2 && (NS - 2) * COPIES < 64, "vmcnt");
  using M = Mfma<MT>;
  typedef typename M::acc_t acc_t;

  __shared__ float4 ring[NS * STAGE / 4];

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int wm = wave / WN, wn = wave % WN;
  int tm, tn;
  tile_coords(blockIdx.x, a, tm, tn);
  const int bidx = blockIdx.y, split = blockIdx.z;
  const int m0 = tm * BM, n0 = tn * BN;
  const int k_begin = split * a.k_per_split;
  const int k_end = min(a.K, k_begin + a.k_per_split);
  const float *Ab = a.A + (int64_t)bidx * a.sa_b;
  const float *Bb = a.B + (int64_t)bidx * a.sb_b;
  const int n_steps = k_end > k_begin ? (k_end - k_begin + BK - 1) / BK : 0;

  // Per-lane copy sources: byte offsets from the step's K origin (rows and
  // columns clamped to valid ones), plus the K index each copy covers; the
  // LDS destinations are wave-uniform.
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  uint32_t a_off0[A_PER_WAVE], b_off0[B_PER_WAVE];
  int a_kk[A_PER_WAVE], b_kk[B_PER_WAVE], a_mn[A_PER_WAVE], b_mn[B_PER_WAVE];
#pragma unroll
  for (int i = 0; i < A_PER_WAVE; ++i) {
    const int p = (wave * A_PER_WAVE + i) * 64 + lane;  // LDS position (units of VW floats)
    int r, kk;
    if constexpr (VW == 4) {
      r = p / ACH;
      kk = ((p % ACH) ^ swz_rows<ACH>(r)) * 4;
    } else {
      r = p / BK;
      const int pc = (p % BK) / 4;
      kk = ((pc ^ swz_rows<ACH>(r)) * 4) + (p & 3);
    }
    a_mn[i] = min(m0 + r, a.M - 1) * (int)a.sa_m;
    a_kk[i] = kk;
    a_off0[i] = (uint32_t)(a_mn[i] + kk * (int)a.sa_k) * 4u;
  }
#pragma unroll
  for (int i = 0; i < B_PER_WAVE; ++i) {
    const int p = (wave * B_PER_WAVE + i) * 64 + lane;
    if constexpr (BF16B) {
      // byte offsets into the bf16 copy: row n, chunk of 8 K values (three
      // pass: positions past the hi rows read the row's lo half, K' further)
      const int half = X3 ? p / (BN * CB) : 0;
      const int pp = p - half * BN * CB;
      const int n = pp / CB;
      const int kk = ((pp % CB) ^ swz_b16<CB>(n)) * 8;
      b_mn[i] = min(n0 + n, a.N - 1) * (int)a.sb_n + half * (int)(a.sb_n / 2);
      b_kk[i] = kk;
      b_off0[i] = (uint32_t)(b_mn[i] + kk) * 2u;
    } else {
      int k, nn;
      if constexpr (VW == 4) {
        k = p / B_CH;
        const int g = k / KG;
        nn = (((p % B_CH) - 4 * g + 4 * B_CH) % B_CH) * 4;
      } else {
        k = p / BN;
        const int g = k / KG;
        const int pc = (p % BN) / 4;
        nn = (((pc - 4 * g + 4 * B_CH) % B_CH) * 4) + (p & 3);
      }
      b_mn[i] = min(n0 + nn, a.N - VW) * (int)a.sb_n;
      b_kk[i] = k;
      b_off0[i] = (uint32_t)(b_mn[i] + k * (int)a.sb_k) * 4u;
    }
  }
  // issue the copies of step `step` into `stage`
  auto issue = [&](int step, float4 *stage) {
    const int k0 = k_begin + step * BK;
    const float *abase = uniform_ptr(Ab + (int64_t)k0 * a.sa_k);
    const float *bbase = BF16B ? uniform_ptr(reinterpret_cast<const float *>(
                                     reinterpret_cast<const __bf16 *>(a.B) + (int64_t)bidx * a.sb_b + k0))
                               : uniform_ptr(Bb + (int64_t)k0 * a.sb_k);
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_void_t *)stage;
    if (k0 + BK <= k_end) {
#pragma unroll
      for (int i = 0; i < A_PER_WAVE; ++i)
        copy_to_lds<VW>(abase, a_off0[i], lds + ((wave_u * A_PER_WAVE + i) * 64 * VW) * 4);
#pragma unroll
      for (int i = 0; i < B_PER_WAVE; ++i)
        copy_to_lds<VB>(bbase, b_off0[i], lds + (A_FLOATS + (wave_u * B_PER_WAVE + i) * 64 * VB) * 4);
    } else {
      // last, partial step: K indices clamped into the range (zeroed later)
      const int kmax = k_end - k0;
#pragma unroll
      for (int i = 0; i < A_PER_WAVE; ++i)
        copy_to_lds<VW>(abase, (uint32_t)(a_mn[i] + min(a_kk[i], kmax - VW) * (int)a.sa_k) * 4u,
                        lds + ((wave_u * A_PER_WAVE + i) * 64 * VW) * 4);
#pragma unroll
      for (int i = 0; i < B_PER_WAVE; ++i) {
        uint32_t off;
        if constexpr (BF16B)
          off = (uint32_t)(b_mn[i] + min(b_kk[i], ((kmax - 1) / 8) * 8)) * 2u;
        else
          off = (uint32_t)(b_mn[i] + min(b_kk[i], kmax - 1) * (int)a.sb_k) * 4u;
        copy_to_lds<VB>(bbase, off, lds + (A_FLOATS + (wave_u * B_PER_WAVE + i) * 64 * VB) * 4);
      }
    }
  };
  // after this thread's copies of `step` landed: zero what lies past k_end
  // (a bf16 chunk straddling k_end holds the copy's zero padding past K)
  auto zero_tail = [&](int step, float4 *stage) {
    const int k0 = k_begin + step * BK;
    if (k0 + BK <= k_end) return;
    float *st = reinterpret_cast<float *>(stage);
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
      float *d = st + ((wave * A_PER_WAVE + i) * 64 + lane) * VW;
#pragma unroll
      for (int e = 0; e < VW; ++e)
        if (k0 + a_kk[i] + e >= k_end) d[e] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < B_PER_WAVE; ++i) {
      float *d = st + A_FLOATS + ((wave * B_PER_WAVE + i) * 64 + lane) * VB;
      if (k0 + b_kk[i] >= k_end)
#pragma unroll
        for (int e = 0; e < VB; ++e) d[e] = 0.0f;
    }
  };

  // per-lane LDS offsets of the MFMA fragments (loop invariant)
  const int g = lane / MT, li = lane % MT;
  constexpr int AH = KG / 4;             // 128-bit A reads per fragment
  int a_off[FM][AH], b_off[FN][KB];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int r = wm * TM + fm * MT + li;
#pragma unroll
    for (int h = 0; h < AH; ++h) a_off[fm][h] = r * BK + (((AH * g + h) ^ swz_rows<ACH>(r)) * 4);
  }
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int n = wn * TN + fn * MT + li;
    if constexpr (BF16B) {
#pragma unroll
      for (int j = 0; j < KB; ++j)  // word offset of the 8 bf16 K values KG.g + 8j ..
        b_off[fn][j] = A_FLOATS + n * (BK / 2) + (((KB * g + j) ^ swz_b16<CB>(n)) * 4);
    } else {
      b_off[fn][0] = A_FLOATS + g * KG * BN + ((((n / 4) + 4 * g) % B_CH) * 4) + (n & 3);
    }
  }

  acc_t acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < M::kRegs; ++r) acc[i][j][r] = 0.0f;

  auto compute = [&](const float4 *stage) {
    const float *st = reinterpret_cast<const float *>(stage);
    float af[FM][KG];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int h = 0; h < AH; ++h) {
        const float4 v = *reinterpret_cast<const float4 *>(st + a_off[fm][h]);
        af[fm][4 * h + 0] = v.x, af[fm][4 * h + 1] = v.y, af[fm][4 * h + 2] = v.z, af[fm][4 * h + 3] = v.w;
      }
    if constexpr (BF16B && X3) {
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        bf16x8 ah[FM], al[FM], bh[FN], bl[FN];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          const float4 x0 = make_float4(af[fm][8 * j], af[fm][8 * j + 1], af[fm][8 * j + 2], af[fm][8 * j + 3]);
          const float4 x1 = make_float4(af[fm][8 * j + 4], af[fm][8 * j + 5], af[fm][8 * j + 6], af[fm][8 * j + 7]);
          if (a.a_pair) unpair_bf16x8(x0, x1, ah[fm], al[fm]);
          else split_bf16x8<true>(x0, x1, ah[fm], al[fm]);
        }
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) {
          bh[fn] = *reinterpret_cast<const bf16x8 *>(st + b_off[fn][j]);
          bl[fn] = *reinterpret_cast<const bf16x8 *>(st + b_off[fn][j] + B_HALF);
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[fm], bh[fn], acc[fm][fn], 0, 0, 0);
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[fm], bl[fn], acc[fm][fn], 0, 0, 0);
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[fm], bh[fn], acc[fm][fn], 0, 0, 0);
          }
      }
    } else if constexpr (BF16B) {
#pragma unroll
      for (int j = 0; j < KB; ++j) {
        bf16x8 a8[FM], b8[FN];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
          a8[fm] = pack_bf16x8(make_float4(af[fm][8 * j], af[fm][8 * j + 1], af[fm][8 * j + 2], af[fm][8 * j + 3]),
                               make_float4(af[fm][8 * j + 4], af[fm][8 * j + 5], af[fm][8 * j + 6], af[fm][8 * j + 7]));
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) b8[fn] = *reinterpret_cast<const bf16x8 *>(st + b_off[fn][j]);
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a8[fm], b8[fn], acc[fm][fn], 0, 0, 0);
      }
    } else {
      float bf[FN][KG];
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int j = 0; j < KG; ++j) bf[fn][j] = st[b_off[fn][0] + j * BN];
#pragma unroll
      for (int j = 0; j < KG; ++j)
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = M::mma(af[fm][j], bf[fn][j], acc[fm][fn]);
    }
  };
  // wait until this wave's copies of step `s` have landed, knowing that the
  // copies of `later` further steps were issued after them
  auto wait_step = [&](int later) {
    if constexpr (NS == 2) {
      wait_vmcnt<0>();
      return;
    }
    switch (later) {
      case 0: wait_vmcnt<0>(); break;
      case 1: wait_vmcnt<COPIES>(); break;
      case 2: wait_vmcnt<(NS > 3 ? 2 : 1) * COPIES>(); break;
      case 3: wait_vmcnt<(NS > 4 ? 3 : 1) * COPIES>(); break;
      default: wait_vmcnt<(NS > 5 ? 4 : 1) * COPIES>(); break;
    }
  };
  static_assert(NS <= 6, "wait_step covers up to 4 later steps");

  if (n_steps > 0) {
    for (int p = 0; p < NS - 1 && p < n_steps; ++p) issue(p, ring + p * (STAGE / 4));
    wait_step(min(NS - 2, n_steps - 1));
    zero_tail(0, ring);
    stage_barrier();
    int cur = 0, nxt = NS - 1;  // ring slots of step s and of step s + NS - 1
    for (int s = 0; s < n_steps; ++s) {
      if (s + NS - 1 < n_steps) issue(s + NS - 1, ring + nxt * (STAGE / 4));
      compute(ring + cur * (STAGE / 4));
      cur = cur + 1 == NS ? 0 : cur + 1;
      nxt = nxt + 1 == NS ? 0 : nxt + 1;
      if (s + 1 < n_steps) {
        wait_step(min(NS - 2, n_steps - 2 - s));
        zero_tail(s + 1, ring + cur * (STAGE / 4));
      }
      stage_barrier();
    }
  }

  // Direct epilogue (bias / activation / residual recognised on the host):
  // each wave stages its accumulators through its own LDS slice one 16-row
  // block at a time (every wave passed the last stage barrier, so the ring
  // is free) and reads them back as row-contiguous groups of 4 columns, so
  // the operands are read and the output written with 128-bit accesses. LDS
  // operations of one wave complete in order: no workgroup barrier.
  if (a.direct && a.splitk == 1) {
    constexpr int DS = TN + 4;
    static_assert(kWaves * MT * DS <= NS * STAGE, "epilogue staging");
    float *Cw = reinterpret_cast<float *>(ring) + wave * MT * DS;
    const int row0 = m0 + wm * TM, col0 = n0 + wn * TN;
    auto load4 = [&](int j, int m, int n, int valid) {
      const float *p = a.eptr[j] + (int64_t)bidx * a.estride[j][0] + (int64_t)m * a.estride[j][1];
      if ((a.e_vec_mask >> j & 1) && valid == 4) return *reinterpret_cast<const float4 *>(p + n);
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      for (int i = 0; i < valid; ++i) v[i] = p[(int64_t)(n + i) * a.estride[j][2]];
      return make_float4(v[0], v[1], v[2], v[3]);
    };
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int r = 0; r < M::kRegs; ++r) Cw[M::row(r, lane) * DS + fn * MT + li] = acc[fm][fn][r];
      __builtin_amdgcn_wave_barrier();
#pragma unroll
      for (int q = lane; q < MT * TN / 4; q += 64) {
        const int r = q / (TN / 4), c = (q % (TN / 4)) * 4;
        const int m = row0 + fm * MT + r, n = col0 + c;
        if (m >= a.M || n >= a.N) continue;
        const float4 p = *reinterpret_cast<const float4 *>(Cw + r * DS + c);
        const int valid = min(4, a.N - n);
        // out = act((acc [+ bias]) [+ res]), in the tape's order
        float v[4] = {p.x, p.y, p.z, p.w};
        if (a.d_bias >= 0) {
          const float4 bv = load4(a.d_bias, m, n, valid);
          v[0] += bv.x, v[1] += bv.y, v[2] += bv.z, v[3] += bv.w;
        }
        if (a.d_res >= 0) {
          const float4 rv = load4(a.d_res, m, n, valid);
          v[0] = rv.x + v[0], v[1] = rv.y + v[1], v[2] = rv.z + v[2], v[3] = rv.w + v[3];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if (a.d_act == KH_OP_GELU_TANH) v[i] = op_gelu_tanh(v[i]);
          else if (a.d_act == KH_OP_GELU_ERF) v[i] = op_gelu_erf(v[i]);
          else if (a.d_act == KH_OP_RELU) v[i] = v[i] != v[i] ? v[i] : fmaxf(v[i], 0.0f);
        }
        if (a.o_pair) {
#pragma unroll
          for (int i = 0; i < 4; ++i) v[i] = pair_word(v[i]);
        }
        float *o = a.eptr[a.d_out] + (int64_t)bidx * a.estride[a.d_out][0] + (int64_t)m * a.estride[a.d_out][1];
        if ((a.e_vec_mask >> a.d_out & 1) && valid == 4) {
          *reinterpret_cast<float4 *>(o + n) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
          for (int i = 0; i < valid; ++i) o[(int64_t)(n + i) * a.estride[a.d_out][2]] = v[i];
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    return;
  }

  // Epilogue: the waves stage their accumulators through LDS one 16-row
  // block (16 x TN per wave) at a time and read them back as row-contiguous
  // groups of 4.
  constexpr int CS = TN + 4;
  static_assert(kWaves * MT * CS <= NS * STAGE, "epilogue staging");
  float *Cw = reinterpret_cast<float *>(ring) + wave * MT * CS;
  const int row0 = m0 + wm * TM, col0 = n0 + wn * TN;
  float *part = a.splitk > 1 ? a.ws_partial + ((int64_t)split * a.batch + bidx) * (int64_t)a.M * a.N : nullptr;
  const bool vec = (a.N & 3) == 0;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int r = 0; r < M::kRegs; ++r) Cw[M::row(r, lane) * CS + fn * MT + li] = acc[fm][fn][r];
    __syncthreads();
#pragma unroll 1
    for (int q = lane; q < MT * TN / 4; q += 64) {
      const int r = q / (TN / 4), c = (q % (TN / 4)) * 4;
      const int m = row0 + fm * MT + r, n = col0 + c;
      if (m >= a.M || n >= a.N) continue;
      const float4 p = *reinterpret_cast<const float4 *>(Cw + r * CS + c);
      if (part) {
        float *dst = part + (int64_t)m * a.N + n;
        if (vec) {
          *reinterpret_cast<float4 *>(dst) = p;
        } else {
          const float pv[4] = {p.x, p.y, p.z, p.w};
          for (int i = 0; i < 4 && n + i < a.N; ++i) dst[i] = pv[i];
        }
      } else {
        Vec<4> v;
        v.v[0] = p.x, v.v[1] = p.y, v.v[2] = p.z, v.v[3] = p.w;
        run_epilogue(a, bidx, m, n, min(4, a.N - n), v);
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Skinny-M GEMM (kind 4), for products with few rows (M up to a few hundred)
// where tiles that fill 256 CUs are too small to keep the LDS pipeline busy
// and splitting K across workgroups needs a second kernel. One workgroup owns
// one BM x BN output tile and its WK waves split K between them. Operands go
// straight from global memory into registers, no LDS staging: A is row-major
// [M][K] and B the [batch][N][K] copy of a constant weight (the nn.Linear
// layout, K contiguous), so lane (row li, group g) loads the 16-byte pieces
// A[m][k + 4g .. + 3] and B[n][k + 4g .. + 3], and the four MFMA steps of a
// 16-deep chunk take its four values in turn (K is permuted the same way for
// A and B; a dot product does not depend on the order of its terms).
//
// Loads are buffer loads: a piece outside the wave's share of K (or past the
// end of K) gets an offset beyond the resource's extent and reads as zeros,
// so no load is conditional and the compiler can count the loads in flight
// exactly. Rows and columns past M and N are clamped to the last one (their
// results are never stored). Each wave runs a ring of DEPTH chunks: the MFMAs
// of a chunk, then the loads of the chunk DEPTH later into the same slot;
// the ring is unrolled over at most kSkinnyIters turns (the host checks that a
// wave's share of K fits), so the code is straight-line and every wait is
// for exactly the chunk it needs.
// The waves' partial tiles are then summed through LDS in wave order (the
// result does not depend on scheduling) and the epilogue runs on
// row-contiguous groups of 4 columns: directly for bias / residual /
// activation, else through the epilogue tape.
constexpr int kSkinnyIters = 4;              // turns of a wave's ring

template <int BM, int BN, int WK, int DEPTH>
__global__ __launch_bounds__(64 * WK) void gemm_skinny_kernel(const GemmArgs a) {
  constexpr int FM = BM / 16, FN = BN / 16;
  constexpr int CS = BN + 4;   // LDS row stride: 16-byte aligned rows
  static_assert(BM % 16 == 0 && BN % 16 == 0, "tile of whole MFMA blocks");
  static_assert(WK * BM * CS * 4 <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(16))) float red[WK * BM * CS];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int li = lane & 15, g = lane >> 4;
  int tm, tn;
  tile_coords(blockIdx.x, a, tm, tn);
  const int bidx = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const int chunks = (a.K + 15) / 16;
  const int per_wave = (chunks + WK - 1) / WK;
  const int c_begin = wave * per_wave;
  const int c_end = min(chunks, c_begin + per_wave);
  const int n_iter = (max(0, c_end - c_begin) + DEPTH - 1) / DEPTH;

  // extents in bytes (the host checks both spans are below 2^29 elements)
  const __amdgpu_buffer_rsrc_t ares = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.A + (int64_t)bidx * a.sa_b), (short)0, (int)(((uint32_t)(a.M - 1) * (uint32_t)a.sa_m + a.K) * 4),
      kBufferRaw);
  const __amdgpu_buffer_rsrc_t bres = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.B + (int64_t)bidx * a.sb_b), (short)0, (int)(((uint32_t)(a.N - 1) * (uint32_t)a.sb_n + a.K) * 4),
      kBufferRaw);
  uint32_t row_a[FM], row_b[FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) row_a[fm] = (uint32_t)min(m0 + fm * 16 + li, a.M - 1) * (uint32_t)a.sa_m * 4;
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) row_b[fn] = (uint32_t)min(n0 + fn * 16 + li, a.N - 1) * (uint32_t)a.sb_n * 4;

  float4 ra[DEPTH][FM], rb[DEPTH][FN];
  auto load = [&](int c, int s) {   // chunk c_begin + c into ring slot s
    const int k = (c_begin + c) * 16 + 4 * g;
    const uint32_t kb = (c_begin + c < c_end && k < a.K) ? (uint32_t)k * 4 : kOutside;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(ares, kb == kOutside ? kOutside : row_a[fm] + kb, 0, 0);
      ra[s][fm] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                              __uint_as_float(x[3]));
    }
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(bres, kb == kOutside ? kOutside : row_b[fn] + kb, 0, 0);
      rb[s][fn] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                              __uint_as_float(x[3]));
    }
  };
  auto part = [](const float4 &v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < DEPTH; ++s) load(s, s);
  __builtin_amdgcn_sched_barrier(0);   // every first-turn load is issued before the first MFMA
  const int n_chunks = max(0, c_end - c_begin);
#pragma unroll
  for (int it = 0; it < kSkinnyIters; ++it) {
    if (it >= n_iter) break;
#pragma unroll
    for (int s = 0; s < DEPTH; ++s) {
      // slots past the wave's share hold zeros: no MFMAs for them
      if (it * DEPTH + s < n_chunks) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
              acc[fm][fn] = Mfma<16>::mma(part(ra[s][fm], j), part(rb[s][fn], j), acc[fm][fn]);
      }
      // refill the slot right away (past the share: zeros, never used); the
      // scheduling barrier keeps the compiler from sinking the loads to the
      // end of the iteration, so DEPTH - 1 chunks stay in flight
      __builtin_amdgcn_sched_barrier(0);
      load((it + 1) * DEPTH + s, s);
      __builtin_amdgcn_sched_barrier(0);
    }
  }

  float *mine = red + wave * BM * CS;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[(fm * 16 + Mfma<16>::row(i, lane)) * CS + fn * 16 + li] = acc[fm][fn][i];
  __syncthreads();
  for (int q = threadIdx.x; q < BM * BN / 4; q += 64 * WK) {
    const int r = q / (BN / 4), c = (q % (BN / 4)) * 4;
    const int m = m0 + r, n = n0 + c;
    if (m >= a.M || n >= a.N) continue;
    float4 sum = *reinterpret_cast<const float4 *>(red + r * CS + c);
#pragma unroll
    for (int w = 1; w < WK; ++w) {
      const float4 p = *reinterpret_cast<const float4 *>(red + w * BM * CS + r * CS + c);
      sum.x += p.x, sum.y += p.y, sum.z += p.z, sum.w += p.w;
    }
    const int valid = min(4, a.N - n);
    Vec<4> v;
    v.v[0] = sum.x, v.v[1] = sum.y, v.v[2] = sum.z, v.v[3] = sum.w;
    if (!a.direct) {
      run_epilogue(a, bidx, m, n, valid, v);
      continue;
    }
    // out = act((acc [+ bias]) [+ res]), as the tape computes it
    auto operand = [&](int j) -> Vec<4> {
      const float *p = a.eptr[j] + (int64_t)bidx * a.estride[j][0] + (int64_t)m * a.estride[j][1];
      Vec<4> o;
      if ((a.e_vec_mask >> j & 1) && valid == 4) {
        const float4 t = *reinterpret_cast<const float4 *>(p + n);
        o.v[0] = t.x, o.v[1] = t.y, o.v[2] = t.z, o.v[3] = t.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) o.v[i] = i < valid ? p[(int64_t)(n + i) * a.estride[j][2]] : 0.0f;
      }
      return o;
    };
    if (a.d_bias >= 0) {
      const Vec<4> bv = operand(a.d_bias);
#pragma unroll
      for (int i = 0; i < 4; ++i) v.v[i] += bv.v[i];
    }
    if (a.d_res >= 0) {
      const Vec<4> rv = operand(a.d_res);
#pragma unroll
      for (int i = 0; i < 4; ++i) v.v[i] = rv.v[i] + v.v[i];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (a.d_act == KH_OP_GELU_TANH) v.v[i] = op_gelu_tanh(v.v[i]);
      else if (a.d_act == KH_OP_GELU_ERF) v.v[i] = op_gelu_erf(v.v[i]);
      else if (a.d_act == KH_OP_RELU) v.v[i] = v.v[i] != v.v[i] ? v.v[i] : fmaxf(v.v[i], 0.0f);
    }
    float *o = a.eptr[a.d_out] + (int64_t)bidx * a.estride[a.d_out][0] + (int64_t)m * a.estride[a.d_out][1];
    if ((a.e_vec_mask >> a.d_out & 1) && valid == 4) {
      *reinterpret_cast<float4 *>(o + n) = make_float4(v.v[0], v.v[1], v.v[2], v.v[3]);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < valid) o[(int64_t)(n + i) * a.estride[a.d_out][2]] = v.v[i];
    }
  }
}

// ---------------------------------------------------------------------------
// Host side.

struct TileCfg {
  int bm, bn, bk, wm, wn, wk, mt, kind, stages, prec;  // kind 1: register-staged loads; 3: LDS-copy pipeline;
                                                       // 4: skinny-M direct loads ([N][K] B); 5: one
                                                       // workgroup per CU, A and B K-contiguous ([N][K] B);
                                                       // 6: small tiles, waves split K ([N][K] B); 7: bf16,
                                                       // 64-deep steps, one tile per workgroup ([N][K] B)
};

// Configurations by id. Ids 0-7: the copy pipeline (BK = 32, MFMA
// 16x16x4, NS LDS stages; each has a 128-bit and a 32-bit copy variant,
// chosen at launch from the operand layouts). Ids 8-14: register-staged
// loads, for skinny tiles and K split across the waves of a workgroup.
#define KH_GEMM3_CONFIGS(X)  \
  X(0, 64, 128, 32, 2, 2, 3) \
  X(1, 128, 64, 32, 2, 2, 3) \
  X(2, 64, 64, 32, 2, 2, 3)  \
  X(3, 32, 128, 32, 1, 4, 3) \
  X(4, 32, 64, 32, 2, 2, 3)  \
  X(5, 64, 96, 32, 2, 2, 3)  \
  X(6, 128, 192, 32, 2, 4, 3) \
  X(7, 128, 128, 32, 2, 4, 3)

#define KH_GEMM_CONFIGS(X)        \
  X(8, 64, 64, 32, 2, 2, 1, 32)  \
  X(9, 32, 64, 32, 1, 2, 2, 32)  \
  X(10, 32, 32, 32, 1, 1, 4, 32)  \
  X(11, 32, 32, 32, 2, 2, 1, 16)  \
  X(12, 16, 64, 32, 1, 4, 1, 16)  \
  X(13, 64, 32, 32, 2, 2, 1, 16)  \
  X(14, 64, 64, 64, 2, 2, 1, 32)

// bf16-input configurations of the copy pipeline (B is a bf16 copy of a
// constant, A fp32 rounded to bf16 in the kernel)
#define KH_GEMM3_BF16_CONFIGS(X) \
  X(15, 128, 128, 2, 2, 3)       \
  X(16, 64, 128, 2, 2, 4)        \
  X(17, 128, 64, 2, 2, 4)        \
  X(18, 64, 64, 2, 2, 4)         \
  X(19, 32, 64, 2, 2, 4)         \
  X(20, 128, 256, 2, 4, 3)

// 128-deep K steps for the smallest pipelined tile (M = 128 blocks: a quarter
// of the 32-deep tile's barriers per K)
#define KH_GEMM3_K128_CONFIGS(X) \
  X(32, 32, 64, 128, 2, 2, 2)    \
  X(33, 32, 64, 128, 2, 2, 3)

// bf16-input configurations with 64- and 128-deep K steps (two or four bf16
// MFMAs per output block between barriers instead of one)
#define KH_GEMM3_BF16_DEEP_CONFIGS(X) \
  X(34, 128, 128, 64, 2, 2, 2)        \
  X(35, 64, 128, 64, 2, 2, 2)         \
  X(36, 128, 64, 64, 2, 2, 2)         \
  X(37, 64, 64, 64, 2, 2, 3)          \
  X(38, 32, 64, 64, 2, 2, 3)          \
  X(39, 128, 256, 64, 2, 4, 2)        \
  X(40, 32, 64, 128, 2, 2, 2)         \
  X(41, 64, 64, 128, 2, 2, 2)

// 32x96 tiles: N = 2304 splits into 24 column tiles, so 1024 x 2304 is 768
// tiles, one round of three per CU (10% faster than the 32x64 tile there)
#define KH_GEMM3_W96_CONFIGS(X) \
  X(46, 32, 96, 32, 2, 2, 3)

// three-pass bf16 with 64-deep K steps
#define KH_GEMM3_BF16X3_DEEP_CONFIGS(X) \
  X(42, 128, 128, 64, 2, 2, 2)          \
  X(43, 64, 128, 64, 2, 2, 2)           \
  X(44, 64, 64, 64, 2, 2, 2)            \
  X(45, 32, 64, 64, 2, 2, 3)

// three-pass bf16 (allow_tf32): the bf16 shapes with hi and lo B rows per stage
#define KH_GEMM3_BF16X3_CONFIGS(X) \
  X(26, 128, 128, 2, 2, 3)         \
  X(27, 64, 128, 2, 2, 3)          \
  X(28, 128, 64, 2, 2, 3)          \
  X(29, 64, 64, 2, 2, 3)           \
  X(30, 32, 64, 2, 2, 3)           \
  X(31, 128, 256, 2, 4, 2)

// copy pipeline with 64 K values per stage (half the barriers and fragment
// reads per flop; two stages to stay within LDS)
#define KH_GEMM3_DEEP_CONFIGS(X) \
  X(21, 64, 64, 64, 2, 2, 2)     \
  X(22, 64, 128, 64, 2, 2, 2)    \
  X(23, 32, 64, 64, 2, 2, 3)     \
  X(24, 128, 192, 64, 2, 4, 2)   \
  X(25, 64, 96, 64, 2, 2, 2)

// skinny-M direct-load tiles (kind 4): BM x BN, WK waves splitting K
#define KH_GEMM_SKINNY_CONFIGS(X) \
  X(47, 16, 32, 8, 8)             \
  X(48, 16, 32, 16, 4)            \
  X(49, 32, 32, 8, 8)             \
  X(50, 16, 64, 8, 4)             \
  X(51, 32, 32, 16, 4)            \
  X(52, 16, 16, 8, 8)             \
  X(53, 32, 64, 8, 4)             \
  X(54, 16, 32, 4, 8)

// the register-staged configuration a pipelined tile falls back to for
// operands too large for 32-bit copy offsets
constexpr int kFallbackConfig = 8;

constexpr TileCfg kConfigs[] = {
#define KH_CFG3_ROW(id, bm, bn, bk, wm, wn, ns) {bm, bn, bk, wm, wn, 1, 16, 3, ns, KH_PREC_FP32},
    KH_GEMM3_CONFIGS(KH_CFG3_ROW)
#undef KH_CFG3_ROW
#define KH_CFG_ROW(id, bm, bn, bk, wm, wn, wk, mt) {bm, bn, bk, wm, wn, wk, mt, 1, 2, KH_PREC_FP32},
    KH_GEMM_CONFIGS(KH_CFG_ROW)
#undef KH_CFG_ROW
#define KH_CFGB_ROW(id, bm, bn, wm, wn, ns) {bm, bn, 32, wm, wn, 1, 16, 3, ns, KH_PREC_BF16},
    KH_GEMM3_BF16_CONFIGS(KH_CFGB_ROW)
#undef KH_CFGB_ROW
#define KH_CFG3_ROW(id, bm, bn, bk, wm, wn, ns) {bm, bn, bk, wm, wn, 1, 16, 3, ns, KH_PREC_FP32},
    KH_GEMM3_DEEP_CONFIGS(KH_CFG3_ROW)
#undef KH_CFG3_ROW
#define KH_CFGX_ROW(id, bm, bn, wm, wn, ns) {bm, bn, 32, wm, wn, 1, 16, 3, ns, KH_PREC_BF16X3},
    KH_GEMM3_BF16X3_CONFIGS(KH_CFGX_ROW)
#undef KH_CFGX_ROW
#define KH_CFG3_ROW(id, bm, bn, bk, wm, wn, ns) {bm, bn, bk, wm, wn, 1, 16, 3, ns, KH_PREC_FP32},
    KH_GEMM3_K128_CONFIGS(KH_CFG3_ROW)
#undef KH_CFG3_ROW
#define KH_CFGBD_ROW(id, bm, bn, bk, wm, wn, ns) {bm, bn, bk, wm, wn, 1, 16, 3, ns, KH_PREC_BF16},
    KH_GEMM3_BF16_DEEP_CONFIGS(KH_CFGBD_ROW)
#undef KH_CFGBD_ROW
#define KH_CFGXD_ROW(id, bm, bn, bk, wm, wn, ns) {bm, bn, bk, wm, wn, 1, 16, 3, ns, KH_PREC_BF16X3},
    KH_GEMM3_BF16X3_DEEP_CONFIGS(KH_CFGXD_ROW)
#undef KH_CFGXD_ROW
#define KH_CFG3_ROW(id, bm, bn, bk, wm, wn, ns) {bm, bn, bk, wm, wn, 1, 16, 3, ns, KH_PREC_FP32},
    KH_GEMM3_W96_CONFIGS(KH_CFG3_ROW)
#undef KH_CFG3_ROW
#define KH_CFGS_ROW(id, bm, bn, wk, depth) {bm, bn, 16, 1, 1, wk, 16, 4, depth, KH_PREC_FP32},
    KH_GEMM_SKINNY_CONFIGS(KH_CFGS_ROW)
#undef KH_CFGS_ROW
#define KH_CFGNT_ROW(id, bm, bn, wm, wn, ns) {bm, bn, 32, wm, wn, 1, 16, 5, ns, KH_PREC_FP32},
    KH_GEMM_NT_CONFIGS(KH_CFGNT_ROW)
#undef KH_CFGNT_ROW
#define KH_CFGSM_ROW(id, bm, bn, wk, ns, prec) \
  {bm, bn, 32, 1, 1, wk, 16, 6, ns, prec == 0 ? KH_PREC_FP32 : prec == 1 ? KH_PREC_BF16 : KH_PREC_BF16X3},
    KH_GEMM_SMALL_CONFIGS(KH_CFGSM_ROW)
#undef KH_CFGSM_ROW
#define KH_CFGNTB_ROW(id, bm, bn, wm, wn, ns, prec) \
  {bm, bn, 32, wm, wn, 1, 16, 5, ns, prec == 1 ? KH_PREC_BF16 : KH_PREC_BF16X3},
    KH_GEMM_NT_BF16_CONFIGS(KH_CFGNTB_ROW)
#undef KH_CFGNTB_ROW
#define KH_CFGBF_ROW(id, bm, bn, wm, wn, ns) {bm, bn, 64, wm, wn, 1, 16, 7, ns, KH_PREC_BF16},
    KH_GEMM_BF_CONFIGS(KH_CFGBF_ROW)
#undef KH_CFGBF_ROW
};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

// Tile rows per group of the tile order (tile_coords). An XCD (32 CUs) holds
// about R = 32 x (workgroups per CU) tiles at once; walking g tile rows
// column-major, they cover g x BM rows of A and R / g x BN columns of B, whose
// panels sum to the least L2 footprint at g = sqrt(R x BN / BM). Workgroups
// per CU are estimated from the LDS a workgroup holds (at most 4). Measured
// on the GPT-2 block's shapes against row-major order (interleaved, warm
// GPU): 2048x3072x768 on the 32x64 tile 5% faster, the others within 1%.
int tile_group(const TileCfg &t, int tiles_m) {
  const int lds = t.kind == 6   ? 4 * t.stages * t.bk * (t.bm + t.bn) * t.wk   // (fp32 bound)
                  : t.kind == 5 ? 4 * t.stages * t.bk * (t.bm + t.bn)   // (fp32 bound)
                  : t.kind == 7 ? t.stages * t.bk * (4 * t.bm + 2 * t.bn)
                  : t.kind == 3 ? 4 * t.stages * (t.bm * t.bk + (t.prec == KH_PREC_FP32 ? t.bk * t.bn
                                                                 : t.bn * t.bk / 2 * (t.prec == KH_PREC_BF16X3 ? 2 : 1)))
                              : 8 * (t.bm * (t.bk + 4) + t.bn * (t.bk + 2));
  const int per_cu = std::max(1, std::min(4, 163840 / std::max(1, lds)));
  const double ideal = std::sqrt(32.0 * per_cu * t.bn / t.bm);
  int g = 1;
  while (g * 2 <= tiles_m && g * 2 <= 64 && std::abs(std::log2(g * 2.0) - std::log2(ideal)) <
                                                 std::abs(std::log2((double)g) - std::log2(ideal)))
    g *= 2;
  return g;
}

hipError_t launch_config(int id, const GemmArgs &a, dim3 grid, hipStream_t stream) {
  if (kConfigs[id].kind == 5) return launch_gemm_nt(id, a, grid, stream);
  if (kConfigs[id].kind == 7) return launch_gemm_bf(id, a, grid, stream);
  if (kConfigs[id].kind == 6) return launch_gemm_small(id, a, grid, stream);
  switch (id) {
#define KH_CFGS_CASE(cid, bm, bn, wk, depth)                                                            \
  case cid:                                                                                            \
    hipLaunchKernelGGL((gemm_skinny_kernel<bm, bn, wk, depth>), grid, dim3(64 * wk), 0, stream, a);       \
    break;
    KH_GEMM_SKINNY_CONFIGS(KH_CFGS_CASE)
#undef KH_CFGS_CASE
#define KH_CFG_CASE(cid, bm, bn, bk, wm, wn, wk, mt)                                                          \
  case cid:                                                                                                  \
    hipLaunchKernelGGL((gemm_f32_kernel<bm, bn, bk, wm, wn, wk, mt>), grid, dim3(64 * wm * wn * wk), 0, stream, \
                       a);                                                                                   \
    break;
    KH_GEMM_CONFIGS(KH_CFG_CASE)
#undef KH_CFG_CASE
#define KH_CFG3_CASE(cid, bm, bn, bk, wm, wn, ns)                                                         \
  case cid:                                                                                              \
    if (a.a_vec && a.b_vec)                                                                              \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, bk, wm, wn, ns, 4, false>), grid, dim3(64 * wm * wn), 0, \
                         stream, a);                                                                     \
    else                                                                                                 \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, bk, wm, wn, ns, 1, false>), grid, dim3(64 * wm * wn), 0, \
                         stream, a);                                                                     \
    break;
    KH_GEMM3_CONFIGS(KH_CFG3_CASE)
    KH_GEMM3_DEEP_CONFIGS(KH_CFG3_CASE)
    KH_GEMM3_K128_CONFIGS(KH_CFG3_CASE)
    KH_GEMM3_W96_CONFIGS(KH_CFG3_CASE)
#undef KH_CFG3_CASE
#define KH_CFGB_CASE(cid, bm, bn, wm, wn, ns)                                                                      \
  case cid:                                                                                                       \
    if (a.a_vec)                                                                                                  \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, 32, wm, wn, ns, 4, true>), grid, dim3(64 * wm * wn), 0, stream, a); \
    else                                                                                                          \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, 32, wm, wn, ns, 1, true>), grid, dim3(64 * wm * wn), 0, stream, a); \
    break;
    KH_GEMM3_BF16_CONFIGS(KH_CFGB_CASE)
#undef KH_CFGB_CASE
#define KH_CFGX_CASE(cid, bm, bn, wm, wn, ns)                                                                        \
  case cid:                                                                                                         \
    if (a.a_vec)                                                                                                    \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, 32, wm, wn, ns, 4, true, true>), grid, dim3(64 * wm * wn), 0,    \
                         stream, a);                                                                                \
    else                                                                                                            \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, 32, wm, wn, ns, 1, true, true>), grid, dim3(64 * wm * wn), 0,    \
                         stream, a);                                                                                \
    break;
    KH_GEMM3_BF16X3_CONFIGS(KH_CFGX_CASE)
#undef KH_CFGX_CASE
#define KH_CFGD_CASE(cid, bm, bn, bk, wm, wn, ns, x3)                                                          \
  case cid:                                                                                                  \
    if (a.a_vec)                                                                                             \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, bk, wm, wn, ns, 4, true, x3>), grid, dim3(64 * wm * wn), 0, \
                         stream, a);                                                                         \
    else                                                                                                     \
      hipLaunchKernelGGL((gemm3_f32_kernel<bm, bn, bk, wm, wn, ns, 1, true, x3>), grid, dim3(64 * wm * wn), 0, \
                         stream, a);                                                                         \
    break;
#define KH_CFGBD_CASE(cid, bm, bn, bk, wm, wn, ns) KH_CFGD_CASE(cid, bm, bn, bk, wm, wn, ns, false)
#define KH_CFGXD_CASE(cid, bm, bn, bk, wm, wn, ns) KH_CFGD_CASE(cid, bm, bn, bk, wm, wn, ns, true)
    KH_GEMM3_BF16_DEEP_CONFIGS(KH_CFGBD_CASE)
    KH_GEMM3_BF16X3_DEEP_CONFIGS(KH_CFGXD_CASE)
#undef KH_CFGBD_CASE
#undef KH_CFGXD_CASE
#undef KH_CFGD_CASE
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
  bool k_major = false;   // kinds 4, 5 and 6: A and B both K-contiguous
  uint32_t e_vec_candidates = 0;

  hipError_t launch(float *const *ptrs, float *partials, hipStream_t stream) override {
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
    // the skinny and K-contiguous kernels read A and B only as 16-byte pieces
    if (k_major && !(a.a_vec && a.b_vec)) return hipErrorInvalidValue;
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
  const int32_t v[8] = {t.bm, t.bn, t.bk, t.wm, t.wn, t.wk, t.mt, t.prec};
  std::memcpy(out8, v, sizeof(v));
  return true;
}

// Recognise an epilogue tape of the form out = act((acc [+ bias]) [+ res])
// (bias broadcast along M, act one of GELU tanh / GELU erf / ReLU, applied
// last and only without a residual) and fill the direct-epilogue fields. The
// tape is evaluated symbolically; additions match in either operand order
// (IEEE addition is commutative), so the direct path computes bit for bit
// what the tape computes. Returns false for any other tape.
bool match_direct_epilogue(const kh_launch &L, GemmArgs &a) {
  enum { kAcc = 1, kBias = 2, kRes = 4, kAct = 8 };
  int slot[KH_NREGS];     // expression per slot: bitmask of kAcc/kBias/kRes/kAct, or -1 for a raw load
  int loaded[KH_NREGS];   // ref a slot holds when it is a raw load
  for (int i = 0; i < KH_NREGS; ++i) slot[i] = -2, loaded[i] = -1;
  slot[0] = kAcc;
  int bias = -1, res = -1, out = -1, act = -1, stores = 0;
  auto full = [&](int j) {  // an [M, N] operand (not broadcast along M or N)
    return a.estride[j][1] != 0 && a.estride[j][2] != 0;
  };
  for (int pc = 0; pc < L.n_insns; ++pc) {
    const kh_insn &in = a.insns[pc];
    if (in.op == KH_OP_LOAD) {
      if (in.dst >= KH_NREGS) return false;
      slot[in.dst] = -1, loaded[in.dst] = in.a;
      continue;
    }
    if (in.op == KH_OP_STORE) {
      if (in.a >= KH_NREGS || ++stores > 1 || slot[in.a] < 0 || !full(in.dst)) return false;
      out = in.dst;
      const int e = slot[in.a];
      if (!(e & kAcc)) return false;
      continue;
    }
    if (in.dst >= KH_NREGS || in.a >= KH_NREGS) return false;
    if (in.op == KH_OP_ADD) {
      if (in.b >= KH_NREGS) return false;
      int x = in.a, y = in.b;
      if (slot[x] == -1) std::swap(x, y);         // x: the accumulator expression, y: a raw load
      if (slot[x] < 0 || slot[y] != -1) return false;
      const int j = loaded[y], e = slot[x];
      if (e & kAct) return false;
      if (e == kAcc && a.estride[j][1] == 0 && a.estride[j][2] != 0) {
        if (bias >= 0) return false;
        bias = j, slot[in.dst] = e | kBias;
      } else if (!(e & kRes) && full(j)) {
        res = j, slot[in.dst] = e | kRes;
      } else {
        return false;
      }
      continue;
    }
    if (in.op == KH_OP_GELU_TANH || in.op == KH_OP_GELU_ERF || in.op == KH_OP_RELU) {
      const int e = slot[in.a];
      if (e < 0 || (e & (kAct | kRes))) return false;
      act = in.op, slot[in.dst] = e | kAct;
      continue;
    }
    return false;
  }
  if (stores != 1) return false;
  a.direct = 1, a.d_bias = bias, a.d_res = res, a.d_out = out, a.d_act = act;
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
  if (L.cfg[3] != KH_PREC_FP32 && L.cfg[3] != KH_PREC_BF16 && L.cfg[3] != KH_PREC_BF16X3) {
    unsupported = true;
    err = "matmul: precision not compiled into this library";
    return nullptr;
  }
  const TileCfg &t = kConfigs[cfg];
  if (L.cfg[3] != t.prec) {
    err = "matmul: tile configuration " + std::to_string(cfg) + " is for another precision";
    return nullptr;
  }
  a.batch = (int)batch, a.M = (int)M, a.N = (int)N, a.K = (int)K;
  a.sa_b = L.refs[0].strides[0], a.sa_m = L.refs[0].strides[1], a.sa_k = L.refs[0].strides[2];
  a.sb_b = L.refs[1].strides[0], a.sb_k = L.refs[1].strides[1], a.sb_n = L.refs[1].strides[2];
  op->a_vec_layout = a.sa_k == 1 && L.refs[0].offset % 4 == 0 && a.sa_m % 4 == 0 && a.sa_b % 4 == 0;
  op->b_vec_layout = a.sb_n == 1 && L.refs[1].offset % 4 == 0 && a.sb_k % 4 == 0 && a.sb_b % 4 == 0;
  if (!fill_epilogue(L, a, op->e_vec_candidates, err)) return nullptr;
  a.direct = 0, a.d_bias = a.d_res = a.d_out = a.d_act = -1;
  match_direct_epilogue(L, a);
  // LayerNorm prologue (cfg[4] = 1; fp32 small-M configurations holding at
  // most 4 rows per wave, K <= kLnMaxK): A is the LayerNorm's input x and
  // the product is rstd * ((x - s) . B - (mean - s) * g) + c per row (s the
  // mean of the row's first 32 values, mean = sum(x) * fparams[0], rstd = rsqrt(sum((x -
  // mean)^2) * fparams[1] + fparams[2])), i.e. LayerNorm(x) . B with the
  // LayerNorm's gamma folded into B: g = refs[cfg[5]] (column sums of B) and
  // c = refs[cfg[6]] (beta . B before the folding; -1: none), both with
  // strides 0 over M and 1 over N, added before the epilogue
  a.pro = L.cfg[4], a.pro_g = -1, a.pro_b = -1;
  if (a.pro != KH_GEMV_PRO_NONE) {
    if (a.pro != KH_GEMV_PRO_LAYERNORM || t.kind != 6 || t.prec != KH_PREC_FP32 || t.bm > 4 * t.wk ||
        t.bm % t.wk) {
      err = "matmul: a LayerNorm prologue needs an fp32 small-M configuration with at most 4 rows per wave";
      return nullptr;
    }
    if (K > kLnMaxK) {
      unsupported = true;
      err = "matmul: LayerNorm prologue rows longer than " + std::to_string(kLnMaxK);
      return nullptr;
    }
    for (int w = 0; w < 2; ++w) {
      const int r = L.cfg[5 + w];
      if (r == -1 && w == 1) continue;
      if (r < 2 || r >= L.n_refs || L.refs[r].strides[1] != 0 || L.refs[r].strides[2] != 1) {
        err = "matmul: the LayerNorm prologue's column vectors must be operands with strides 0 over M, 1 over N";
        return nullptr;
      }
      (w == 0 ? a.pro_g : a.pro_b) = r - 2;
    }
    a.pro_c1 = L.fparams[0], a.pro_c2 = L.fparams[1], a.pro_eps = L.fparams[2];
  }
  int cfg_run = cfg;
  if (t.prec == KH_PREC_BF16) {
    // B must be the library-layout bf16 copy: [batch][N][K'] with K' a
    // multiple of 8 (16-byte rows), unit K stride
    const kh_ref &rb = L.refs[1];
    if (a.sb_k != 1 || a.sb_n % 8 || a.sb_b % 8 || rb.offset % 8 || a.sb_n < K) {
      err = "matmul: bf16 B operand must be [batch][N][K'] with K' a multiple of 8 and >= K";
      return nullptr;
    }
    op->b_vec_layout = true;
  }
  if (t.prec == KH_PREC_BF16X3) {
    // B must be the three-pass copy: [batch][N][2K'], hi then lo halves of K'
    const kh_ref &rb = L.refs[1];
    if (a.sb_k != 1 || a.sb_n % 16 || a.sb_b % 8 || rb.offset % 8 || a.sb_n / 2 < K) {
      err = "matmul: bf16x3 B operand must be [batch][N][2K'] with K' a multiple of 8 and >= K";
      return nullptr;
    }
    op->b_vec_layout = true;
  }
  if (t.kind == 4 || t.kind == 5 || t.kind == 6 || t.kind == 7) {
    // skinny-M direct loads / K-contiguous pipelines: A row-major with unit K
    // stride, B the [batch][N][K] copy, both read as whole 16-byte pieces; K
    // is not split across workgroups (and is a positive whole number of
    // steps, 32 or 64 deep, for kinds 5 and 6)
    const kh_ref &ra = L.refs[0], &rb = L.refs[1];
    const bool steps = t.kind == 5 || t.kind == 6 || t.kind == 7;
    const int step = steps ? t.bk : 4;
    op->b_vec_layout = a.sb_k == 1 && rb.offset % 4 == 0 && a.sb_n % 4 == 0 && a.sb_b % 4 == 0 && a.sb_n >= K;
    if (!op->a_vec_layout || !op->b_vec_layout || K % step || (steps && K == 0) || ra.offset % 4) {
      err = "matmul: configuration " + std::to_string(cfg) +
            " needs A [.., M, K] and B [batch][N][K] with unit K stride, 16-byte aligned rows and K a " +
            (steps ? "positive multiple of " + std::to_string(step) : std::string("multiple of 4"));
      return nullptr;
    }
    // buffer-load byte offsets are 32-bit (and must stay below the
    // out-of-range marker)
    const int64_t span_a = std::max<int64_t>(0, M - 1) * a.sa_m + K, span_b = std::max<int64_t>(0, N - 1) * a.sb_n + K;
    if (span_a >= (1ll << 29) || span_b >= (1ll << 29)) {
      unsupported = true;
      err = "matmul: K-contiguous configuration with an operand spanning 2^29 elements or more";
      return nullptr;
    }
    // a skinny wave's share of K must fit the unrolled ring
    const int64_t share = ((K + 15) / 16 + t.wk - 1) / t.wk;
    if (t.kind == 4 && share > (int64_t)t.stages * kSkinnyIters) {
      unsupported = true;
      err = "matmul: K = " + std::to_string(K) + " is too deep for skinny configuration " + std::to_string(cfg);
      return nullptr;
    }
  }
  if (t.kind == 3) {
    // 128-bit copies never straddle the end of a row or of K
    op->a_vec_layout = op->a_vec_layout && K % 4 == 0;
    op->b_vec_layout = op->b_vec_layout && N % 4 == 0;
    // per-lane copy offsets are 32-bit byte offsets: fall back to a general
    // kernel for operands spanning 2^29 elements or more
    const int64_t span_a = std::max<int64_t>(0, M - 1) * std::abs(a.sa_m) + std::max<int64_t>(0, K - 1) * std::abs(a.sa_k);
    const int64_t span_b = std::max<int64_t>(0, K - 1) * std::abs(a.sb_k) + std::max<int64_t>(0, N - 1) * std::abs(a.sb_n);
    if (span_a >= (1ll << 29) || span_b >= (1ll << 29) || a.sa_m < 0 || a.sa_k < 0 || a.sb_k < 0 || a.sb_n < 0) {
      if (t.prec != KH_PREC_FP32) {
        unsupported = true;
        err = "matmul: bf16 operands spanning 2^29 elements or more";
        return nullptr;
      }
      cfg_run = kFallbackConfig;
    }
  }
  // bf16 storage (cfg[7]): A and / or the direct epilogue's output, on the
  // bf16 kernel with 64-deep steps only
  const uint32_t m16 = bf16_refs(L);
  if (m16) {
    const bool a16 = m16 & 1u, o16 = a.direct && (m16 >> (2 + a.d_out) & 1u);
    const uint32_t known = (a16 ? 1u : 0u) | (o16 ? 1u << (2 + a.d_out) : 0u);
    if (t.kind != 7 || m16 != known || a.pro != KH_GEMV_PRO_NONE) {
      unsupported = true;
      err = "matmul: bf16 storage only for A and a direct epilogue's output on a 64-deep bf16 configuration";
      return nullptr;
    }
    if (a16 && (a.sa_k != 1 || a.sa_m % 8 || a.sa_b % 8 || L.refs[0].offset % 8)) {
      err = "matmul: a bf16 A operand needs unit K stride and 16-byte aligned rows";
      return nullptr;
    }
    if (o16 && (a.estride[a.d_out][2] != 1 || a.estride[a.d_out][1] % 4 || a.estride[a.d_out][0] % 4 ||
                L.refs[2 + a.d_out].offset % 4)) {
      err = "matmul: a bf16 output needs unit N stride and 8-byte aligned rows";
      return nullptr;
    }
    a.a16 = a16 ? 1 : 0, a.o16 = o16 ? 1 : 0;
  }
  const TileCfg &tr = kConfigs[cfg_run];
  a.tiles_m = (int)((M + tr.bm - 1) / tr.bm);
  a.tiles_n = (int)((N + tr.bn - 1) / tr.bn);
  int splitk = tr.kind >= 4 ? 1 : std::max(1, L.cfg[2]);
  const int k_steps = (int)std::max<int64_t>(1, (K + tr.bk - 1) / tr.bk);
  splitk = std::min(splitk, k_steps);
  a.k_per_split = ((k_steps + splitk - 1) / splitk) * tr.bk;
  splitk = (int)std::max<int64_t>(1, (K + a.k_per_split - 1) / std::max(1, a.k_per_split));
  if (K == 0) splitk = 1, a.k_per_split = 0;
  a.splitk = splitk;
  // pair storage (cfg[7] bits 16 + j): A and / or the direct epilogue's
  // output, on the three-pass configurations (the kernels of kinds 3, 5 and
  // 6, which split A fragments and write a direct epilogue's output)
  const uint32_t mp = pair_refs(L);
  if (mp) {
    const bool ap = mp & 1u, op_ = a.direct && (mp >> (2 + a.d_out) & 1u);
    const uint32_t known = (ap ? 1u : 0u) | (op_ ? 1u << (2 + a.d_out) : 0u);
    const bool kind_ok = tr.kind == 3 || tr.kind == 5 || tr.kind == 6;
    if (mp != known || m16 || cfg_run != cfg || t.prec != KH_PREC_BF16X3 || !kind_ok || a.pro != KH_GEMV_PRO_NONE ||
        (op_ && a.splitk != 1)) {
      unsupported = true;
      err = "matmul: pair storage only for A and a direct epilogue's output of a three-pass configuration "
            "(the output without split-K)";
      return nullptr;
    }
    a.a_pair = ap ? 1 : 0, a.o_pair = op_ ? 1 : 0;
  }
  const int64_t n_tiles = (int64_t)a.tiles_m * a.tiles_n;
  if (n_tiles >= (1ll << 31)) {
    unsupported = true;
    err = "matmul: too many tiles";
    return nullptr;
  }
  a.group_m = tile_group(tr, a.tiles_m);
  op->k_major = tr.kind >= 4;
  op->cfg = cfg_run;
  // the K-contiguous kernel with a direct epilogue is persistent: at most
  // one workgroup per CU, each walking its tiles
  const int64_t grid_x = tr.kind == 5 && a.direct ? std::min<int64_t>(n_tiles, current_device().cus) : n_tiles;
  op->grid = dim3((unsigned)std::max<int64_t>(1, grid_x), (unsigned)batch, (unsigned)splitk);
  if (splitk > 1) {
    op->n_partials = (size_t)splitk * batch * M * N;
  }
  return op;
}

}  // namespace kh
