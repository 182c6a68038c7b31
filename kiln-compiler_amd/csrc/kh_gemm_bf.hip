// kh_gemm_bf.hip - bf16-input matmul with 64-deep K steps (configuration
// kind 7): C[b] = epilogue(A[b] @ B[b]) with A [.., M, K] fp32 K-contiguous,
// rounded to bf16 as its fragments are read, and B the bf16 [batch][N][K']
// copy of a constant (the arithmetic of the other bf16 GEMMs: bf16 inputs,
// fp32 accumulation).
//
// Same contract as the rest of the matmul family (the reference's tl.dot
// kernel with fused epilogue, kiln/gpu/codegen.py:484-530). A bf16 MFMA step
// is 16x shorter than an fp32 one, so at one K step per stage of 32 values
// (kinds 3 and 5) a step's copy wait and barrier cost more than its matrix
// work. Here:
//   * a stage holds 64 K values: A rows of 64 floats (16 chunks of 16 bytes,
//     chunk c of row r at c ^ swz_rows<16>(r)) and bf16 B rows of 64 values
//     (8 chunks, chunk c of row n at c ^ swz_h64(n)), copied with 128-bit
//     global_load_lds (no VGPRs, no VALU); NS stages in a ring, the copies
//     of step s + NS - 1 issued right after the barrier of step s;
//   * a step is two 32-deep halves; in half k2 lane (row li, group g) reads
//     K values 32 k2 + 8g .. 32 k2 + 8g + 7 of its A rows (two 128-bit
//     reads, rounded to bf16) and of its B rows (one 128-bit read), and each
//     16 x 16 output block takes one v_mfma_f32_16x16x32_bf16;
//   * one tile per workgroup and no persistence: the hardware runs two
//     workgroups of the smaller tiles per CU, so one's copy latency hides
//     under the other's MFMAs;
//   * the epilogue stages the accumulators of 16 rows at a time through the
//     ring (free once the main loop is done) and reads, computes and writes
//     row-contiguous groups of 4 columns with 128-bit accesses: bias /
//     residual / activation directly, other tapes through the tape
//     interpreter.
// Measured against the 32-deep K-contiguous kernel on 2048x3072x768 (bf16
// weights, fp32 activations): 27.5 -> 23.1 us per product; 18.6 us with bf16
// A. Where its time goes (the same product at K = 64 .. 3072): a one-step
// product takes ~10 us, half of it the epilogue's output stores, and each
// further 64-deep step ~0.74 us, bound by the copies into LDS (~15 TB/s over
// all CUs from L2); without its MFMAs or its fragment reads a step is barely
// shorter, and a deeper ring or a barrier in the middle of the step does not
// shorten it.
// bf16 storage (ABF; a.a16): when the producer of A wrote it as bf16 (a
// LayerNorm, attention or another product whose only consumer is this one),
// A rows are 64 bf16 values per stage (8 chunks, like B's), half the bytes
// copied and one 128-bit fragment read per half step with no rounding (the
// same bits: the producer rounded to nearest even as the fragment read
// does). a.o16: the direct epilogue writes its output as bf16 for a
// consumer that reads it that way.
// K must be a positive multiple of 64 and the operands' spans below 2^29
// elements (the host checks both).
#include <algorithm>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_gemm_dev.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {


template <int BM, int BN, int WM, int WN, int NS, bool TAPE, bool ABF>
__global__ __launch_bounds__(64 * WM * WN) void gemm_bf_kernel(const GemmArgs a) {
  constexpr int BK = 64, MT = 16, kWaves = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / MT, FN = TN / MT;
  constexpr int ACH = ABF ? 8 : 16;                                      // 16-byte chunks per A row and stage
  constexpr int A_BYTES = BM * ACH * 16, STAGE = A_BYTES + BN * BK * 2;  // bytes
  constexpr int A_PW = BM * ACH / 64 / kWaves, B_PW = BN * 8 / 64 / kWaves, COPIES = A_PW + B_PW;
  constexpr int CS = TN + 4;   // epilogue staging row stride (floats, 16-byte aligned rows)
  constexpr int QJ = MT * TN / 4 / 64;   // epilogue column groups per lane and 16-row block
  static_assert(TM % MT == 0 && TN % MT == 0, "wave tile of whole MFMA blocks");
  static_assert((MT * TN / 4) % 64 == 0, "16-row blocks of whole 64-lane column-group rounds");
  static_assert((BM * ACH) % (64 * kWaves) == 0 && (BN * 8) % (64 * kWaves) == 0, "copy mapping");
  static_assert(NS >= 2 && NS <= 4 && (NS - 2) * COPIES < 64, "ring depth / vmcnt range");
  static_assert(NS * STAGE <= 160 * 1024 && kWaves * MT * CS * 4 <= NS * STAGE, "LDS: ring, staging inside it");
  __shared__ float4 ring4[NS * STAGE / 16];
  char *ring = reinterpret_cast<char *>(ring4);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave / WN, wn = wave % WN, li = lane & 15, g = lane >> 4;
  const int bidx = blockIdx.y;
  int tm, tn;
  tile_coords(blockIdx.x, a, tm, tn);
  const int m0 = tm * BM, n0 = tn * BN;
  // A in its element type: fp32, or bf16 (ABF)
  const char *Ab = reinterpret_cast<const char *>(a.A) + (int64_t)bidx * a.sa_b * (ABF ? 2 : 4);
  const __bf16 *Bb = reinterpret_cast<const __bf16 *>(a.B) + (int64_t)bidx * a.sb_b;

  // per-lane copy sources: byte offsets from the step's first K column (rows
  // past M / N clamped to the last one; their results are never stored)
  uint32_t a_off[A_PW], b_off[B_PW];
#pragma unroll
  for (int i = 0; i < A_PW; ++i) {
    const int p = (wave * A_PW + i) * 64 + lane, r = p / ACH;
    a_off[i] = ABF ? (uint32_t)(min(m0 + r, a.M - 1) * (int)a.sa_m + ((p % 8) ^ swz_h64(r)) * 8) * 2u
                   : (uint32_t)(min(m0 + r, a.M - 1) * (int)a.sa_m + ((p % 16) ^ swz_rows<16>(r)) * 4) * 4u;
  }
#pragma unroll
  for (int i = 0; i < B_PW; ++i) {
    const int p = (wave * B_PW + i) * 64 + lane, r = p / 8;
    b_off[i] = (uint32_t)(min(n0 + r, a.N - 1) * (int)a.sb_n + ((p % 8) ^ swz_h64(r)) * 8) * 2u;
  }
  const int n_steps = a.K / BK;   // the host checks K % 64 == 0 and K > 0
  auto issue = [&](int step) {
    const float *ab = uniform_ptr(reinterpret_cast<const float *>(Ab + step * BK * (ABF ? 2 : 4)));
    const float *bb = uniform_ptr(reinterpret_cast<const float *>(Bb + step * BK));
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_void_t *)(ring + (step % NS) * STAGE);
#pragma unroll
    for (int i = 0; i < A_PW; ++i) copy_to_lds<4>(ab, a_off[i], lds + (wave_u * A_PW + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_PW; ++i) copy_to_lds<4>(bb, b_off[i], lds + A_BYTES + (wave_u * B_PW + i) * 1024);
  };
  // fragment byte offsets within a stage, per 32-deep half k2
  int fa[FM][2][2], fb[FN][2];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int r = wm * TM + fm * MT + li;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2)
#pragma unroll
      for (int q = 0; q < 2; ++q)
        fa[fm][k2][q] = ABF ? r * 128 + ((4 * k2 + g) ^ swz_h64(r)) * 16
                            : r * 256 + ((8 * k2 + 2 * g + q) ^ swz_rows<16>(r)) * 16;
  }
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int r = wn * TN + fn * MT + li;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) fb[fn][k2] = A_BYTES + r * 128 + ((4 * k2 + g) ^ swz_h64(r)) * 16;
  }
  f32x4 acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};

  // direct epilogue: operand pointers, strides and layouts, read from the
  // kernel arguments here (scalar loads whose indices are themselves loaded:
  // issued at the end of the tile they would be two dependent memory round
  // trips in front of the first store, ~2 us per tile). Lane l handles the
  // column groups (l + 64 j) % (TN / 4), j < QJ, of every 16-row block: its
  // bias values are loaded here, before the first copies (so the copies'
  // vmcnt waits never count them), and its residual values at the start of
  // the last K step (one memory latency under that step's MFMAs instead of
  // one per 16-row block in the epilogue: ~2 us per tile each).
  const bool has_b = a.d_bias >= 0, has_r = a.d_res >= 0;
  const int jb = has_b ? a.d_bias : 0, jr = has_r ? a.d_res : 0, jo = TAPE ? 0 : a.d_out;
  const float *pb = a.eptr[jb] + (int64_t)bidx * a.estride[jb][0];
  const float *pr = a.eptr[jr] + (int64_t)bidx * a.estride[jr][0];
  float *po = a.eptr[jo] + (int64_t)bidx * a.estride[jo][0];
  const int64_t sbn = a.estride[jb][2], srm = a.estride[jr][1], srn = a.estride[jr][2];
  const int64_t som = a.estride[jo][1], son = a.estride[jo][2];
  const bool vb = a.e_vec_mask >> jb & 1, vr = a.e_vec_mask >> jr & 1, vo = a.e_vec_mask >> jo & 1;
  const int act = a.d_act, M = a.M, N = a.N, o16 = a.o16;
  __bf16 *po16 = reinterpret_cast<__bf16 *>(a.eptr[jo]) + (int64_t)bidx * a.estride[jo][0];
  const int row0 = m0 + wm * TM, col0 = n0 + wn * TN;
  float4 bias_v[QJ];
#pragma unroll
  for (int j = 0; j < QJ; ++j) {
    const int n = col0 + ((lane + 64 * j) % (TN / 4)) * 4;
    bias_v[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!TAPE && has_b && vb && n + 4 <= N) bias_v[j] = *reinterpret_cast<const float4 *>(pb + n);
  }
  float4 res_v[FM][QJ];
  auto load_residual = [&]() {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int j = 0; j < QJ; ++j) {
        const int q = lane + 64 * j, m = row0 + fm * MT + q / (TN / 4), n = col0 + (q % (TN / 4)) * 4;
        res_v[fm][j] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (!TAPE && has_r && vr && m < M && n + 4 <= N)
          res_v[fm][j] = *reinterpret_cast<const float4 *>(pr + (int64_t)m * srm + n);
      }
  };

  for (int p = 0; p < NS - 1 && p < n_steps; ++p) issue(p);

  for (int s = 0; s < n_steps; ++s) {
    // this wave's copies of step s landed (the copies of `later` steps were
    // issued after them), then every wave's: the barrier also says that every
    // wave is done reading stage s - 1, whose slot the next copies refill
    const int later = min(NS - 2, n_steps - 1 - s);
    if (later <= 0) wait_vmcnt<0>();
    else if (later == 1) wait_vmcnt<COPIES>();
    else wait_vmcnt<2 * COPIES>();
    stage_barrier();
    if (s + NS - 1 < n_steps) issue(s + NS - 1);
    if (s == n_steps - 1) load_residual();   // no copy wait follows
    const char *st = ring + (s % NS) * STAGE;
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      bf16x8 xa[FM], xb[FN];
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        if constexpr (ABF) {
          xa[fm] = *reinterpret_cast<const bf16x8 *>(st + fa[fm][k2][0]);
        } else {
          const float4 lo = *reinterpret_cast<const float4 *>(st + fa[fm][k2][0]);
          const float4 hi = *reinterpret_cast<const float4 *>(st + fa[fm][k2][1]);
          xa[fm] = pack_bf16x8(lo, hi);
        }
      }
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) xb[fn] = *reinterpret_cast<const bf16x8 *>(st + fb[fn][k2]);
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[fm], xb[fn], acc[fm][fn], 0, 0, 0);
    }
  }


  // epilogue: 16-row blocks of the wave tile through the wave's slice of the
  // ring (its own, and LDS operations of one wave complete in order)
  __syncthreads();   // every wave's fragment reads of the ring are done
  float *Cw = reinterpret_cast<float *>(ring) + wave * MT * CS;
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int i = 0; i < 4; ++i) Cw[(4 * g + i) * CS + fn * MT + li] = acc[fm][fn][i];
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
      const int q = lane + 64 * j, r = q / (TN / 4), c = (q % (TN / 4)) * 4;
      const int m = row0 + fm * MT + r, n = col0 + c;
      if (m < M && n < N) {
        const float4 p = *reinterpret_cast<const float4 *>(Cw + r * CS + c);
        const int valid = min(4, N - n);
        if constexpr (TAPE) {
          Vec<4> v;
          v.v[0] = p.x, v.v[1] = p.y, v.v[2] = p.z, v.v[3] = p.w;
          run_epilogue(a, bidx, m, n, valid, v);
        } else {
          // out = act((acc [+ bias]) [+ res]), in the tape's order
          float v[4] = {p.x, p.y, p.z, p.w};
          if (has_b) {
            if (vb && valid == 4) {
              const float4 t = bias_v[j];
              v[0] += t.x, v[1] += t.y, v[2] += t.z, v[3] += t.w;
            } else {
              for (int i = 0; i < valid; ++i) v[i] += pb[(int64_t)(n + i) * sbn];
            }
          }
          if (has_r) {
            const float *rr = pr + (int64_t)m * srm;
            if (vr && valid == 4) {
              const float4 t = res_v[fm][j];
              v[0] = t.x + v[0], v[1] = t.y + v[1], v[2] = t.z + v[2], v[3] = t.w + v[3];
            } else {
              for (int i = 0; i < valid; ++i) v[i] = rr[(int64_t)(n + i) * srn] + v[i];
            }
          }
          if (act == KH_OP_GELU_TANH) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = op_gelu_tanh(v[i]);
          } else if (act == KH_OP_GELU_ERF) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = op_gelu_erf(v[i]);
          } else if (act == KH_OP_RELU) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = v[i] != v[i] ? v[i] : fmaxf(v[i], 0.0f);
          }
          if (o16) {
            if (valid == 4) {
              store_bf16x4(po16, (int64_t)m * som + n, v[0], v[1], v[2], v[3]);
            } else {
              for (int i = 0; i < valid; ++i) po16[(int64_t)m * som + n + i] = (__bf16)v[i];
            }
          } else {
            float *o = po + (int64_t)m * som;
            if (vo && valid == 4) {
              *reinterpret_cast<float4 *>(o + n) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
              for (int i = 0; i < valid; ++i) o[(int64_t)(n + i) * son] = v[i];
            }
          }
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

hipError_t launch_gemm_bf(int id, const GemmArgs &a, dim3 grid, hipStream_t stream) {
  switch (id) {
#define KH_CFGBF_CASE(cid, bm, bn, wm, wn, ns)                                                                     \
  case cid:                                                                                                        \
    if (a.direct && a.a16)                                                                                         \
      hipLaunchKernelGGL((gemm_bf_kernel<bm, bn, wm, wn, ns, false, true>), grid, dim3(64 * wm * wn), 0, stream, a); \
    else if (a.direct)                                                                                             \
      hipLaunchKernelGGL((gemm_bf_kernel<bm, bn, wm, wn, ns, false, false>), grid, dim3(64 * wm * wn), 0, stream, a); \
    else if (a.a16)                                                                                                \
      hipLaunchKernelGGL((gemm_bf_kernel<bm, bn, wm, wn, ns, true, true>), grid, dim3(64 * wm * wn), 0, stream, a);  \
    else                                                                                                           \
      hipLaunchKernelGGL((gemm_bf_kernel<bm, bn, wm, wn, ns, true, false>), grid, dim3(64 * wm * wn), 0, stream, a); \
    break;
    KH_GEMM_BF_CONFIGS(KH_CFGBF_CASE)
#undef KH_CFGBF_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kh
