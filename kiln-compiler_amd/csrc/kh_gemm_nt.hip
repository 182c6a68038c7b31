// kh_gemm_nt.hip - matmul over a constant weight read through its
// [batch][N][K] copy (configuration kind 5; fp32, or the bf16 / three-pass
// bf16 copies), for the large products of a transformer block:
// C[b] = epilogue(A[b] @ B[b]) with both operands K-contiguous in memory.
//
// Same contract as the other members of the matmul family (the reference's
// tl.dot kernel with fused epilogue, kiln/gpu/codegen.py:484-530); what
// differs is the shape of the work on a CU:
//   * one workgroup per CU, its waves one per SIMD (or two), each owning a
//     large wave tile (up to 64 x 96: 24 MFMA blocks of 16 x 16), so a K step
//     of 32 is 8 x FM x FN v_mfma_f32_16x16x4_f32 per wave between barriers
//     (192 for the largest tile, ~6000 matrix cycles);
//   * A and B rows both hold K contiguously, so both are copied into LDS with
//     the same 128-bit global_load_lds pattern (rows of 32 floats = 8 chunks
//     of 16 bytes, chunk c of row r at c ^ swz_a(r)) and both fragments are
//     read as two 128-bit LDS vectors per row: lane (row li, group g) takes K
//     values 8g .. 8g+7 of its A row and of its B row, and MFMA j of a step
//     consumes value 8g + j in every group (the K order is permuted the same
//     way for A and B; a dot product does not depend on it);
//   * a ring of NS LDS stages, copies issued NS - 1 steps ahead; the barrier
//     that publishes stage s + 1 sits in the middle of step s's MFMAs, and
//     the fragment reads of stage s + 1 follow it, so they run under the
//     second half of step s's MFMAs and the next step starts with its
//     operands in registers (two register sets of fragments, one per half
//     step, each loaded while the other feeds the MFMAs);
//   * persistent (for bias / residual / activation epilogues): the grid is at
//     most one workgroup per CU and each workgroup walks its tiles, issuing
//     the next tile's first stages before the current tile's epilogue, so the
//     loads are in flight while the epilogue runs and the stores drain under
//     the next main loop (other epilogue tapes: one tile per workgroup);
//   * the epilogue stages 16-row blocks of the accumulators through a per-wave
//     LDS slice and reads, computes and writes row-contiguous groups of 4
//     columns with 128-bit accesses (bias / residual / activation directly,
//     other tapes through the tape interpreter).
// bf16 inputs (PREC 1, the arithmetic of the other bf16 GEMMs): B is the
// bf16 [batch][N][K'] copy (rows of 32 K values = 4 chunks of 16 bytes in a
// stage, chunk c of row n at c ^ swz_b16<4>(n)), A is read as fp32 like the
// fp32 kernel and rounded to bf16 as its fragments are read; each step is one
// v_mfma_f32_16x16x32_bf16 per output block (lane (li, g) supplies K values
// 8g .. 8g+7 of its A row and its B row), fp32 accumulation. Three-pass bf16
// (PREC 2): B the [batch][N][2K'] copy, hi then lo rows in a stage, A split
// the same way, a.b = a_lo.b_hi + a_hi.b_lo + a_hi.b_hi. With an MFMA step
// this short the fp32 kernel's mid-step barrier does not pay: a bf16 step
// waits for its stage, passes the barrier, refills the slot the previous step
// read and then reads and multiplies (two workgroup waves per SIMD, or one
// wave with the next copies NS - 1 steps ahead).
// K must be a positive multiple of 32 and the operands' spans below 2^29
// elements (the host checks both; other shapes use the other kernels of the
// family).
#include <algorithm>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_gemm_dev.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

// TAPE = false: persistent over tiles, direct epilogue (bias / residual /
// activation, recognised on the host); TAPE = true: one tile per workgroup
// and the general epilogue tape after the main loop (kept out of the tile
// loop so the tape interpreter is not replicated into it).
template <int BM, int BN, int WM, int WN, int NS, bool TAPE, int PREC>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(WM * WN / 4, WM * WN / 4)))
void gemm_nt_kernel(const GemmArgs a) {
  constexpr int BK = 32, MT = 16, ACH = BK / 4;
  constexpr bool BF = PREC != 0;
  constexpr int NB = PREC == 2 ? 2 : 1;                      // bf16 copies of B rows per stage (hi, lo)
  constexpr int kWaves = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / MT, FN = TN / MT;
  constexpr int A_FLOATS = BM * BK;
  constexpr int B_HALF = BN * BK / 2;                        // words of one bf16 copy of a stage's B rows
  constexpr int STAGE = A_FLOATS + (BF ? B_HALF * NB : BN * BK);
  constexpr int B_CHUNKS = BF ? BN * 4 * NB : BN * ACH;      // 16-byte chunks of B per stage
  constexpr int A_PER_WAVE = BM * ACH / 64 / kWaves, B_PER_WAVE = B_CHUNKS / 64 / kWaves;
  constexpr int COPIES = A_PER_WAVE + B_PER_WAVE;
  static_assert(TM % MT == 0 && TN % MT == 0, "wave tile of whole MFMA blocks");
  static_assert((BM * ACH) % (64 * kWaves) == 0 && B_CHUNKS % (64 * kWaves) == 0, "copy mapping");
  static_assert(NS >= 2 && NS <= 4 && (NS - 2) * COPIES < 64, "ring depth / vmcnt range");
  static_assert(kWaves % 4 == 0, "whole SIMDs");

  constexpr int CS = TN + 4;   // epilogue staging row stride (floats, 16-byte aligned rows)
  static_assert(NS * STAGE * 4 + kWaves * MT * CS * 4 <= 160 * 1024, "LDS: ring and epilogue staging");

  __shared__ float4 ring[NS * STAGE / 4];
  __shared__ float4 staging[kWaves * MT * CS / 4];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int wm = wave / WN, wn = wave % WN;
  const int li = lane & 15, g = lane >> 4;
  const int bidx = blockIdx.y;
  const float *Ab = a.A + (int64_t)bidx * a.sa_b;
  // (B in its element type: fp32, or the bf16 copy)
  const char *Bb = reinterpret_cast<const char *>(a.B) + (int64_t)bidx * a.sb_b * (BF ? 2 : 4);
  const int n_steps = a.K / BK;   // the host checks K % 32 == 0 and K > 0
  const int n_tiles = a.tiles_m * a.tiles_n;

  // per-lane copy sources of the current tile: byte offsets from the step's
  // first K column (rows past M / N clamped to the last one; their results
  // are never stored)
  uint32_t a_off[A_PER_WAVE], b_off[B_PER_WAVE];
  int m0 = 0, n0 = 0;
  auto set_tile = [&](int t) {
    int tm, tn;
    tile_coords(t, a, tm, tn);
    m0 = tm * BM, n0 = tn * BN;
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) {
      const int p = (wave * A_PER_WAVE + i) * 64 + lane;
      const int r = p / ACH;
      a_off[i] = (uint32_t)(min(m0 + r, a.M - 1) * (int)a.sa_m + ((p % ACH) ^ swz_a(r)) * 4) * 4u;
    }
#pragma unroll
    for (int i = 0; i < B_PER_WAVE; ++i) {
      const int p = (wave * B_PER_WAVE + i) * 64 + lane;
      if constexpr (BF) {
        // bf16 row r: 4 chunks of 8 K values; three-pass: the lo rows (K'
        // further along the copy's row) follow the hi rows
        const int half = p / (BN * 4), pp = p % (BN * 4), r = pp / 4;
        const int row = min(n0 + r, a.N - 1) * (int)a.sb_n + half * ((int)a.sb_n / 2);
        b_off[i] = (uint32_t)(row + ((pp % 4) ^ swz_b16<4>(r)) * 8) * 2u;
      } else {
        const int r = p / ACH;
        b_off[i] = (uint32_t)(min(n0 + r, a.N - 1) * (int)a.sb_n + ((p % ACH) ^ swz_a(r)) * 4) * 4u;
      }
    }
  };
  auto slot_ptr = [&](int step) { return ring + (step % NS) * (STAGE / 4); };
  auto issue = [&](int step) {
    const float *abase = uniform_ptr(Ab + step * BK);
    const float *bbase = uniform_ptr(reinterpret_cast<const float *>(Bb + step * BK * (BF ? 2 : 4)));
    const uint32_t lds = (uint32_t)(uintptr_t)(lds_void_t *)slot_ptr(step);
#pragma unroll
    for (int i = 0; i < A_PER_WAVE; ++i) copy_to_lds<4>(abase, a_off[i], lds + (wave_u * A_PER_WAVE + i) * 1024);
#pragma unroll
    for (int i = 0; i < B_PER_WAVE; ++i)
      copy_to_lds<4>(bbase, b_off[i], lds + A_FLOATS * 4 + (wave_u * B_PER_WAVE + i) * 1024);
  };
  // this wave's copies of a step have landed, `later` steps' copies being
  // issued after them (and no other vector memory operation after those)
  auto wait_landed = [&](int later) {
    if (later <= 0) wait_vmcnt<0>();
    else if (later == 1 || NS < 4) wait_vmcnt<COPIES>();
    else wait_vmcnt<2 * COPIES>();
  };

  // fragment offsets (floats, within a stage): two 128-bit reads per row
  int fa_off[FM][2], fb_off[FN][2];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int r = wm * TM + fm * MT + li;
#pragma unroll
    for (int h = 0; h < 2; ++h) fa_off[fm][h] = r * BK + ((2 * g + h) ^ swz_a(r)) * 4;
  }
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int r = wn * TN + fn * MT + li;
    if constexpr (BF) {
      // one 16-byte bf16 chunk per row (and the lo row's for three-pass)
      fb_off[fn][0] = A_FLOATS + r * (BK / 2) + ((g ^ swz_b16<4>(r)) * 4);
      fb_off[fn][1] = fb_off[fn][0] + B_HALF;
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) fb_off[fn][h] = A_FLOATS + r * BK + ((2 * g + h) ^ swz_a(r)) * 4;
    }
  }

  f32x4 acc[FM][FN];
  // Fragments in two register sets, one per half step: set h holds K values
  // 8g + 4h .. 8g + 4h + 3 of the lane's A rows and B rows (one 128-bit LDS
  // read per row).
  float4 f0a[FM], f0b[FN], f1a[FM], f1b[FN];
  // (the scheduling barrier keeps the compiler from sinking the reads towards
  // their first use at the start of the next half, where the wave would then
  // wait for them)
  auto read_half = [&](int step, int h, float4 (&xa)[FM], float4 (&xb)[FN]) {
    const float *st = reinterpret_cast<const float *>(slot_ptr(step));
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) xa[fm] = *reinterpret_cast<const float4 *>(st + fa_off[fm][h]);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) xb[fn] = *reinterpret_cast<const float4 *>(st + fb_off[fn][h]);
    __builtin_amdgcn_sched_barrier(0);
  };
  auto part = [](const float4 &v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; };
  auto mfmas = [&](const float4 (&xa)[FM], const float4 (&xb)[FN]) {
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x4f32(part(xa[fm], j), part(xb[fn], j), acc[fm][fn], 0, 0, 0);
  };

  // Epilogue of the tile at (tm0, tn0): each wave stages its accumulators
  // through its own LDS slice one 16-row block (16 x TN) at a time and reads
  // them back as row-contiguous groups of 4 columns, so operands are read and
  // the output written with 128-bit accesses. The slice is the wave's own and
  // LDS operations of one wave complete in order, so no barrier is needed.
  float *Cw = reinterpret_cast<float *>(staging) + wave * MT * CS;
  auto load4 = [&](int j, int m, int n, int valid) {
    const float *p = a.eptr[j] + (int64_t)bidx * a.estride[j][0] + (int64_t)m * a.estride[j][1];
    if ((a.e_vec_mask >> j & 1) && valid == 4) return *reinterpret_cast<const float4 *>(p + n);
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < valid; ++i) v[i] = p[(int64_t)(n + i) * a.estride[j][2]];
    return make_float4(v[0], v[1], v[2], v[3]);
  };
  auto act = [&](float v) {
    if (a.d_act == KH_OP_GELU_TANH) return op_gelu_tanh(v);
    if (a.d_act == KH_OP_GELU_ERF) return op_gelu_erf(v);
    if (a.d_act == KH_OP_RELU) return v != v ? v : fmaxf(v, 0.0f);
    return v;
  };
  auto epilogue = [&](int tm0, int tn0) {
    const int row0 = tm0 + wm * TM, col0 = tn0 + wn * TN;
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
#pragma unroll
        for (int i = 0; i < 4; ++i) Cw[(4 * g + i) * CS + fn * MT + li] = acc[fm][fn][i];
      __builtin_amdgcn_wave_barrier();
      auto emit = [&](int q) {
        const int r = q / (TN / 4), c = (q % (TN / 4)) * 4;
        const int m = row0 + fm * MT + r, n = col0 + c;
        if (m >= a.M || n >= a.N) return;
        const float4 p = *reinterpret_cast<const float4 *>(Cw + r * CS + c);
        const int valid = min(4, a.N - n);
        if constexpr (TAPE) {
          Vec<4> v;
          v.v[0] = p.x, v.v[1] = p.y, v.v[2] = p.z, v.v[3] = p.w;
          run_epilogue(a, bidx, m, n, valid, v);
        } else {
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
          for (int i = 0; i < 4; ++i) v[i] = act(v[i]);
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
      };
      // the tape interpreter once, in a loop; the direct form unrolled
      if constexpr (TAPE) {
#pragma unroll 1
        for (int q = lane; q < MT * TN / 4; q += 64) emit(q);
      } else {
#pragma unroll
        for (int q = lane; q < MT * TN / 4; q += 64) emit(q);
      }
      __builtin_amdgcn_wave_barrier();
    }
  };

  // Persistent loop: workgroup w takes tiles w, w + grid, ... The next tile's
  // first NS - 1 stages are issued as soon as every wave is done with the
  // ring, before this tile's epilogue, so its loads are in flight while the
  // epilogue runs and the output stores drain under the next main loop.
  int t = blockIdx.x;
  if (t >= n_tiles) return;
  set_tile(t);
  for (int p = 0; p < NS - 1 && p < n_steps; ++p) issue(p);
  bool first = true;
  while (true) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (BF) {
      for (int s = 0; s < n_steps; ++s) {
        // stage s landed everywhere (after a previous tile, whose epilogue
        // issued memory operations behind the first copies, wait for all),
        // and every wave is done reading stage s - 1, whose slot the copies
        // of step s + NS - 1 refill
        if (s == 0 && !first) wait_vmcnt<0>();
        else wait_landed(min(NS - 2, n_steps - 1 - s));
        stage_barrier();
        if (s + NS - 1 < n_steps) issue(s + NS - 1);
        const float *st = reinterpret_cast<const float *>(slot_ptr(s));
        float4 xa[FM][2], xb[FN][NB];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int h = 0; h < 2; ++h) xa[fm][h] = *reinterpret_cast<const float4 *>(st + fa_off[fm][h]);
#pragma unroll
        for (int fn = 0; fn < FN; ++fn)
#pragma unroll
          for (int h = 0; h < NB; ++h) xb[fn][h] = *reinterpret_cast<const float4 *>(st + fb_off[fn][h]);
        bf16x8 ah[FM], al[FM];
#pragma unroll
        for (int fm = 0; fm < FM; ++fm) {
          if constexpr (PREC == 2) {
            if (a.a_pair) unpair_bf16x8(xa[fm][0], xa[fm][1], ah[fm], al[fm]);
            else split_bf16x8<true>(xa[fm][0], xa[fm][1], ah[fm], al[fm]);
          } else {
            ah[fm] = pack_bf16x8(xa[fm][0], xa[fm][1]);
          }
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn) {
            const bf16x8 bh = *reinterpret_cast<const bf16x8 *>(&xb[fn][0]);
            if constexpr (PREC == 2) {
              const bf16x8 bl = *reinterpret_cast<const bf16x8 *>(&xb[fn][NB - 1]);
              acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[fm], bh, acc[fm][fn], 0, 0, 0);
              acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[fm], bl, acc[fm][fn], 0, 0, 0);
            }
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[fm], bh, acc[fm][fn], 0, 0, 0);
          }
      }
    } else {
      // stage 0 of this tile landed everywhere (after a previous tile, whose
      // epilogue issued memory operations behind these copies, wait for all)
      if (first) wait_landed(min(NS - 2, n_steps - 1));
      else wait_vmcnt<0>();
      stage_barrier();
      read_half(0, 0, f0a, f0b);
      // every step but the last (the loop body has no conditional LDS reads, so
      // the compiler's counter waits before the second half stay exact)
      for (int s = 0; s + 1 < n_steps; ++s) {
        // first half of step s (set 0) under the reads of its second half
        if (s + NS - 1 < n_steps) issue(s + NS - 1);
        read_half(s, 1, f1a, f1b);
        mfmas(f0a, f0b);
        // stage s + 1 landed everywhere: its first half is read under the
        // second half of step s (set 1)
        wait_landed(min(NS - 2, n_steps - 2 - s));
        stage_barrier();
        read_half(s + 1, 0, f0a, f0b);
        mfmas(f1a, f1b);
      }
      read_half(n_steps - 1, 1, f1a, f1b);
      mfmas(f0a, f0b);
      mfmas(f1a, f1b);
    }

    const int tm0 = m0, tn0 = n0;
    const int t_next = TAPE ? n_tiles : t + (int)gridDim.x;
    if (t_next < n_tiles) {
      __syncthreads();   // every wave's fragment reads of the ring have completed
      set_tile(t_next);
      for (int p = 0; p < NS - 1 && p < n_steps; ++p) issue(p);
    }
    epilogue(tm0, tn0);
    if (t_next >= n_tiles) break;
    t = t_next;
    first = false;
  }
}

}  // namespace

hipError_t launch_gemm_nt(int id, const GemmArgs &a, dim3 grid, hipStream_t stream) {
  switch (id) {
#define KH_CFGNTP_CASE(cid, bm, bn, wm, wn, ns, prec)                                                                  \
  case cid:                                                                                                          \
    if (a.direct)                                                                                                    \
      hipLaunchKernelGGL((gemm_nt_kernel<bm, bn, wm, wn, ns, false, prec>), grid, dim3(64 * wm * wn), 0, stream, a); \
    else                                                                                                             \
      hipLaunchKernelGGL((gemm_nt_kernel<bm, bn, wm, wn, ns, true, prec>), grid, dim3(64 * wm * wn), 0, stream, a);  \
    break;
#define KH_CFGNT_CASE(cid, bm, bn, wm, wn, ns) KH_CFGNTP_CASE(cid, bm, bn, wm, wn, ns, 0)
    KH_GEMM_NT_CONFIGS(KH_CFGNT_CASE)
    KH_GEMM_NT_BF16_CONFIGS(KH_CFGNTP_CASE)
#undef KH_CFGNT_CASE
#undef KH_CFGNTP_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kh
