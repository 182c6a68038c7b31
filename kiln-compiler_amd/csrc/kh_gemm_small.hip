// kh_gemm_small.hip - matmul for products with few rows (configuration kind
// 6): C[b] = epilogue(A[b] @ B[b]) with A [.., M, K] row-major fp32 and B the
// [batch][N][K] copy of a constant weight (fp32, or the bf16 / three-pass
// bf16 copies), both K-contiguous.
//
// Same contract as the rest of the matmul family (the reference's tl.dot
// kernel with fused epilogue, kiln/gpu/codegen.py:484-530). A product with a
// few hundred rows has too little work per output tile to keep a CU's four
// SIMDs busy when each tile goes to one wave, and tiles large enough to do so
// leave most of the 256 CUs idle; splitting K across workgroups needs a
// second kernel. Here a workgroup owns one small BM x BN tile and its WK
// waves split K between them, so a product is many small workgroups and every
// SIMD of every CU gets a wave:
//   * each wave streams its own K range through a private ring of NS LDS
//     stages with 128-bit global_load_lds copies (rows of 32 floats = 8
//     chunks, chunk c of row r at c ^ swz_a(r); A rows then B rows in a
//     stage), NS - 1 steps ahead of its MFMAs; a wave waits only for its own
//     copies (vmcnt) and no other wave reads its ring, so the main loop has no
//     workgroup barrier;
//   * fragments are two 128-bit LDS reads per row: lane (row li, group g)
//     takes K values 8g .. 8g+7 of its A row and its B row, and MFMA j of a
//     step (v_mfma_f32_16x16x4_f32) consumes value 8g + j in every group (the
//     K order is permuted the same way for A and B);
//   * the waves' partial tiles are then summed through LDS in wave order (the
//     result does not depend on scheduling) and the epilogue runs on
//     row-contiguous groups of 4 columns with 128-bit accesses: bias /
//     residual / activation directly, other tapes through the tape
//     interpreter; the direct operands are loaded before the partial sums so
//     their latency overlaps the reduction.
// LayerNorm prologue (LN, fp32; a LayerNorm whose only consumer is this
// product's A operand): A is the LayerNorm's input x; the lowering folds
// gamma into B (B' = gamma * B) and provides g = column sums of B' and
// c = beta . B. With s a shift near the row's mean,
//     LayerNorm(x) . B = rstd * ((x - s) . B' - (mean - s) * g) + c,
// so A fragments enter the MFMAs as x - s and the row statistics come from the
// same fragments as the K loop streams them: each lane merges the mean and
// the sum of squared deviations of its 8-value chunks (Chan's pairwise
// update), lanes and then waves merge theirs in a fixed order, and the
// epilogue applies the formula before the tape. The rounding error of the
// accumulated (x - s) . B' and of the correction grows with |mean - s| /
// std, so s is the mean of the row's first 32 values (every wave of the
// workgroup computes it in the same order, so they all use the same s): a
// row whose first value is an outlier (x[0] = 200 over N(0, 1) values)
// would make the row's first value a shift about 27 standard deviations
// from the mean, the sample mean about one. The LayerNorm's launch and its
// output's round trip through memory go away; A is read once (plus the 128
// bytes of the shift, an L2 hit).
// K must be a positive multiple of 32 and the operands' spans below 2^29
// elements (the host checks both).
#include <algorithm>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_gemm_dev.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

// PREC: 0 fp32 (v_mfma_f32_16x16x4_f32, eight per output block and step);
// 1 bf16 - B the bf16 [batch][N][K'] copy, A rounded to bf16 as its
// fragments are read, one v_mfma_f32_16x16x32_bf16 per block and step, fp32
// accumulation (the arithmetic of the other bf16 GEMMs); 2 three-pass bf16 -
// B the [batch][N][2K'] copy holding bf16(w) then bf16(w - bf16(w)) per row,
// A split the same way, a.b = a_lo.b_hi + a_hi.b_lo + a_hi.b_hi.
template <int BM, int BN, int WK, int NS, int PREC, bool LN>
__global__ __launch_bounds__(64 * WK) void gemm_small_kernel(const GemmArgs a) {
  constexpr int BK = 32, MT = 16, ACH = BK / 4;
  constexpr int FM = BM / MT, FN = BN / MT;
  constexpr bool BF = PREC != 0;
  static_assert(!LN || (!BF && BM % WK == 0 && BM / WK <= 4), "LayerNorm prologue: fp32, at most 4 rows per wave");
  constexpr int B_HALF = BN * BK / 2;           // words of one bf16 copy of a stage's B rows
  constexpr int A_FLOATS = BM * BK;
  constexpr int STAGE = A_FLOATS + (BF ? B_HALF * (PREC == 2 ? 2 : 1) : BN * BK);   // words: A rows, then B rows
  constexpr int B_CHUNKS = BF ? BN * 4 * (PREC == 2 ? 2 : 1) : BN * ACH;   // 16-byte chunks of B per stage
  constexpr int A_COPIES = BM * ACH / 64, B_COPIES = B_CHUNKS / 64;
  constexpr int COPIES = A_COPIES + B_COPIES;   // copy instructions per stage and wave
  constexpr int CS = BN + 4;                    // partial-tile row stride (16-byte aligned rows)
  static_assert(BM % MT == 0 && BN % MT == 0, "tile of whole MFMA blocks");
  static_assert((BM * ACH) % 64 == 0 && B_CHUNKS % 64 == 0, "whole copy instructions");
  static_assert(NS >= 2 && NS <= 4 && (NS - 2) * COPIES < 64, "ring depth / vmcnt range");
  static_assert(BM * CS <= NS * STAGE, "partial tile fits the wave's ring");
  static_assert(WK * NS * STAGE * 4 <= 160 * 1024, "LDS");

  __shared__ float4 rings[WK * NS * STAGE / 4];
  __shared__ float4 ln_part[LN ? WK : 1][LN ? BM : 1];   // LN: (count, mean, M2) per wave and tile row

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wave_u = __builtin_amdgcn_readfirstlane(wave);
  const int li = lane & 15, g = lane >> 4;
  int tm, tn;
  tile_coords(blockIdx.x, a, tm, tn);
  const int bidx = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const float *Ab = a.A + (int64_t)bidx * a.sa_b;
  // this wave's K steps (the host checks K % 32 == 0 and K > 0)
  const int steps = a.K / BK;
  const int per_wave = (steps + WK - 1) / WK;
  const int s_begin = wave_u * per_wave;
  const int n_steps = max(0, min(steps, s_begin + per_wave) - s_begin);

  float4 *ring = rings + wave_u * (NS * STAGE / 4);
  const uint32_t ring_lds = (uint32_t)(uintptr_t)(lds_void_t *)ring;
  // per-lane copy sources: byte offsets from the step's first K column (rows
  // past M / N clamped to the last one; their results are never stored)
  uint32_t a_off[A_COPIES], b_off[B_COPIES];
#pragma unroll
  for (int i = 0; i < A_COPIES; ++i) {
    const int p = i * 64 + lane, r = p / ACH;
    a_off[i] = (uint32_t)(min(m0 + r, a.M - 1) * (int)a.sa_m + ((p % ACH) ^ swz_a(r)) * 4) * 4u;
  }
#pragma unroll
  for (int i = 0; i < B_COPIES; ++i) {
    const int p = i * 64 + lane;
    if constexpr (BF) {
      // bf16 row n: 4 chunks of 8 K values, chunk c at c ^ swz_b16<4>(n);
      // three-pass: the lo rows (K' further along the copy's row) follow
      const int half = p / (BN * 4), pp = p % (BN * 4), r = pp / 4;
      const int64_t row = (int64_t)min(n0 + r, a.N - 1) * a.sb_n + half * (a.sb_n / 2);
      b_off[i] = (uint32_t)(row + ((pp % 4) ^ swz_b16<4>(r)) * 8) * 2u;
    } else {
      const int r = p / ACH;   // B row r of the tile sits at stage row BM + r
      b_off[i] = (uint32_t)(min(n0 + r, a.N - 1) * (int)a.sb_n + ((p % ACH) ^ swz_a(BM + r)) * 4) * 4u;
    }
  }
  auto issue = [&](int s) {   // this wave's step s (0-based within its range)
    const int k0 = (s_begin + s) * BK;
    const float *abase = uniform_ptr(Ab + k0);
    const float *bbase =
        BF ? uniform_ptr(reinterpret_cast<const float *>(reinterpret_cast<const __bf16 *>(a.B) +
                                                          (int64_t)bidx * a.sb_b + k0))
           : uniform_ptr(a.B + (int64_t)bidx * a.sb_b + k0);
    const uint32_t lds = ring_lds + (uint32_t)((s % NS) * STAGE * 4);
#pragma unroll
    for (int i = 0; i < A_COPIES; ++i) copy_to_lds<4>(abase, a_off[i], lds + i * 1024);
#pragma unroll
    for (int i = 0; i < B_COPIES; ++i) copy_to_lds<4>(bbase, b_off[i], lds + A_FLOATS * 4 + i * 1024);
  };
  // this wave's copies of a step have landed, `later` steps' copies being
  // issued after them
  auto wait_landed = [&](int later) {
    if (later <= 0) wait_vmcnt<0>();
    else if (later == 1 || NS < 4) wait_vmcnt<COPIES>();
    else wait_vmcnt<2 * COPIES>();
  };

  // fragment offsets (words, within a stage): lane (li, g) reads K values
  // 8g .. 8g+7 of its A row (two 128-bit reads) and of its B row (two fp32
  // reads, or one 16-byte bf16 chunk)
  int fa_off[FM][2], fb_off[FN][2];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int r = fm * MT + li;
#pragma unroll
    for (int h = 0; h < 2; ++h) fa_off[fm][h] = r * BK + ((2 * g + h) ^ swz_a(r)) * 4;
  }
#pragma unroll
  for (int fn = 0; fn < FN; ++fn) {
    const int r = fn * MT + li;
    if constexpr (BF) {
      fb_off[fn][0] = A_FLOATS + r * (BK / 2) + ((g ^ swz_b16<4>(r)) * 4);
      fb_off[fn][1] = fb_off[fn][0] + B_HALF;   // three-pass: the lo row
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h) fb_off[fn][h] = (BM + r) * BK + ((2 * g + h) ^ swz_a(BM + r)) * 4;
    }
  }

  f32x4 acc[FM][FN];
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = f32x4{0.f, 0.f, 0.f, 0.f};
  auto part = [](const float4 &v, int j) { return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w; };

  for (int p = 0; p < NS - 1 && p < n_steps; ++p) issue(p);
  // LN: the shift s (the mean of the row's first 32 values: lane group g
  // sums values 8g .. 8g+7, the four groups' sums are added by two xor
  // shuffles, which gives every lane of the row the same bits) and this
  // lane's running (count, mean, M2) of x - s per row of the tile
  float ln_x0[FM], ln_n[FM], ln_mean[FM], ln_m2[FM];
  if constexpr (LN) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const float *row = Ab + (int64_t)min(m0 + fm * MT + li, a.M - 1) * a.sa_m + 8 * g;
      float v[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = row[e];
      float t = ((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]));
      t += __shfl_xor(t, 16, 64);
      t += __shfl_xor(t, 32, 64);
      ln_x0[fm] = t * 0.03125f;
      ln_n[fm] = 0.0f, ln_mean[fm] = 0.0f, ln_m2[fm] = 0.0f;
    }
  }
  // Chan's update: (n, mean, m2) += the statistics (nb, mb, m2b) of more values
  auto merge = [](float &n, float &mean, float &m2, float nb, float mb, float m2b) {
    const float nt = n + nb;
    if (nt > 0.0f) {
      const float d = mb - mean;
      mean = fmaf(d, nb / nt, mean);
      m2 = m2 + m2b + d * d * (n * nb / nt);
      n = nt;
    }
  };
  for (int s = 0; s < n_steps; ++s) {
    wait_landed(min(NS - 2, n_steps - 1 - s));
    // the wave's own LDS: its copies landed (vmcnt), nothing else writes it
    __builtin_amdgcn_wave_barrier();
    const float *st = reinterpret_cast<const float *>(ring + (s % NS) * (STAGE / 4));
    float4 xa[FM][2], xb[FN][2];
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int h = 0; h < 2; ++h) xa[fm][h] = *reinterpret_cast<const float4 *>(st + fa_off[fm][h]);
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int h = 0; h < (PREC == 1 ? 1 : 2); ++h) xb[fn][h] = *reinterpret_cast<const float4 *>(st + fb_off[fn][h]);
    // the slot read now is refilled NS steps later: its fragment reads must
    // have completed before this wave issues that copy (next iterations)
    __builtin_amdgcn_s_waitcnt((3 << 14) | (7 << 4) | 15);  // lgkmcnt(0); vmcnt, expcnt unconstrained
    if (s + NS - 1 < n_steps) issue(s + NS - 1);
    if constexpr (LN) {
      // chunk s + 1 of 8 values joins s chunks: Chan's update with weight
      // 8 / (8 (s + 1)) (one reciprocal per step for every row)
      const float w1 = __builtin_amdgcn_rcpf((float)(s + 1)), w2 = 8.0f * (float)s * w1;
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = part(xa[fm][e / 4], e % 4) - ln_x0[fm];
        xa[fm][0] = make_float4(v[0], v[1], v[2], v[3]);
        xa[fm][1] = make_float4(v[4], v[5], v[6], v[7]);
        const float cm = (((v[0] + v[1]) + (v[2] + v[3])) + ((v[4] + v[5]) + (v[6] + v[7]))) * 0.125f;
        float cm2 = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) cm2 = fmaf(v[e] - cm, v[e] - cm, cm2);
        const float d = cm - ln_mean[fm];
        ln_mean[fm] = fmaf(d, w1, ln_mean[fm]);
        ln_m2[fm] = fmaf(d * d, w2, ln_m2[fm] + cm2);
      }
    }
    if constexpr (BF) {
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
            const bf16x8 bl = *reinterpret_cast<const bf16x8 *>(&xb[fn][1]);
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[fm], bh, acc[fm][fn], 0, 0, 0);
            acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[fm], bl, acc[fm][fn], 0, 0, 0);
          }
          acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[fm], bh, acc[fm][fn], 0, 0, 0);
        }
    } else {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
              acc[fm][fn] = __builtin_amdgcn_mfma_f32_16x16x4f32(part(xa[fm][h], j), part(xb[fn][h], j),
                                                                 acc[fm][fn], 0, 0, 0);
    }
  }
  wait_vmcnt<0>();   // (no copy of this wave is outstanding past here)

  // this thread's first output group's operands (the direct epilogue's bias
  // and residual, the LN prologue's g and c), loaded before the partial
  // tiles are summed so their latency overlaps the reduction
  constexpr int GROUPS = BM * BN / 4;
  const int q0 = threadIdx.x;
  auto group_mn = [&](int q, int &m, int &n) {
    m = m0 + q / (BN / 4);
    n = n0 + (q % (BN / 4)) * 4;
  };
  auto load4 = [&](int j, int m, int n, int valid) {
    const float *p = a.eptr[j] + (int64_t)bidx * a.estride[j][0] + (int64_t)m * a.estride[j][1];
    if ((a.e_vec_mask >> j & 1) && valid == 4) return *reinterpret_cast<const float4 *>(p + n);
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < valid; ++i) v[i] = p[(int64_t)(n + i) * a.estride[j][2]];
    return make_float4(v[0], v[1], v[2], v[3]);
  };
  float4 pre_b = make_float4(0.f, 0.f, 0.f, 0.f), pre_r = pre_b, pre_g = pre_b, pre_c = pre_b;
  if ((a.direct || LN) && q0 < GROUPS) {
    int m, n;
    group_mn(q0, m, n);
    if (m < a.M && n < a.N) {
      const int valid = min(4, a.N - n);
      if constexpr (LN) {   // the prologue's column vectors g and c
        pre_g = load4(a.pro_g, m, n, valid);
        if (a.pro_b >= 0) pre_c = load4(a.pro_b, m, n, valid);
      }
      if (a.direct && a.d_bias >= 0) pre_b = load4(a.d_bias, m, n, valid);
      if (a.direct && a.d_res >= 0) pre_r = load4(a.d_res, m, n, valid);
    }
  }

  // partial tiles through LDS (each wave into its own ring), summed in wave
  // order
  float *mine = reinterpret_cast<float *>(ring);
#pragma unroll
  for (int fm = 0; fm < FM; ++fm)
#pragma unroll
    for (int fn = 0; fn < FN; ++fn)
#pragma unroll
      for (int i = 0; i < 4; ++i) mine[(fm * MT + 4 * g + i) * CS + fn * MT + li] = acc[fm][fn][i];
  if constexpr (LN) {
    // the row's statistics over this wave's K range: lanes li, li + 16,
    // li + 32, li + 48 merged (lane group 0's result kept)
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      ln_n[fm] = 8.0f * (float)n_steps;
#pragma unroll
      for (int off = 16; off <= 32; off <<= 1) {
        const float nb = __shfl_xor(ln_n[fm], off, 64), mb = __shfl_xor(ln_mean[fm], off, 64);
        const float m2b = __shfl_xor(ln_m2[fm], off, 64);
        merge(ln_n[fm], ln_mean[fm], ln_m2[fm], nb, mb, m2b);
      }
      if (g == 0) ln_part[wave_u][fm * MT + li] = make_float4(ln_n[fm], ln_mean[fm], ln_m2[fm], 0.0f);
    }
  }
  __syncthreads();
  const float *parts = reinterpret_cast<const float *>(rings);
  for (int q = q0; q < GROUPS; q += 64 * WK) {
    int m, n;
    group_mn(q, m, n);
    if (m >= a.M || n >= a.N) continue;
    const int off = (m - m0) * CS + (n - n0);
    float4 sum = *reinterpret_cast<const float4 *>(parts + off);
#pragma unroll
    for (int w = 1; w < WK; ++w) {
      const float4 p = *reinterpret_cast<const float4 *>(parts + w * NS * STAGE + off);
      sum.x += p.x, sum.y += p.y, sum.z += p.z, sum.w += p.w;
    }
    const int valid = min(4, a.N - n);
    if constexpr (LN) {
      // the row's statistics over all of K (waves merged in order), then
      // rstd * (sum - (mean - s) * g) + c
      float4 st = ln_part[0][m - m0];
#pragma unroll
      for (int w = 1; w < WK; ++w) {
        const float4 o = ln_part[w][m - m0];
        merge(st.x, st.y, st.z, o.x, o.y, o.z);
      }
      const float rstd = rsqrtf(st.z * a.pro_c2 + a.pro_eps), mu = st.y;
      const float4 gs = q == q0 ? pre_g : load4(a.pro_g, m, n, valid);
      sum.x = rstd * fmaf(-mu, gs.x, sum.x), sum.y = rstd * fmaf(-mu, gs.y, sum.y);
      sum.z = rstd * fmaf(-mu, gs.z, sum.z), sum.w = rstd * fmaf(-mu, gs.w, sum.w);
      if (a.pro_b >= 0) {   // the folded beta . B
        const float4 c = q == q0 ? pre_c : load4(a.pro_b, m, n, valid);
        sum.x += c.x, sum.y += c.y, sum.z += c.z, sum.w += c.w;
      }
    }
    if (!a.direct) {
      Vec<4> v;
      v.v[0] = sum.x, v.v[1] = sum.y, v.v[2] = sum.z, v.v[3] = sum.w;
      run_epilogue(a, bidx, m, n, valid, v);
      continue;
    }
    // out = act((acc [+ bias]) [+ res]), in the tape's order
    const float4 bv = q == q0 ? pre_b : (a.d_bias >= 0 ? load4(a.d_bias, m, n, valid) : pre_b);
    const float4 rv = q == q0 ? pre_r : (a.d_res >= 0 ? load4(a.d_res, m, n, valid) : pre_r);
    float v[4] = {sum.x, sum.y, sum.z, sum.w};
    if (a.d_bias >= 0) v[0] += bv.x, v[1] += bv.y, v[2] += bv.z, v[3] += bv.w;
    if (a.d_res >= 0) v[0] = rv.x + v[0], v[1] = rv.y + v[1], v[2] = rv.z + v[2], v[3] = rv.w + v[3];
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
}

}  // namespace

hipError_t launch_gemm_small(int id, const GemmArgs &a, dim3 grid, hipStream_t stream) {
  switch (id) {
#define KH_CFGSM_CASE(cid, bm, bn, wk, ns, prec)                                                             \
  case cid:                                                                                                 \
    if (a.pro == KH_GEMV_PRO_LAYERNORM) {                                                                   \
      if constexpr (prec == 0 && bm <= 4 * wk && bm % wk == 0)                                              \
        hipLaunchKernelGGL((gemm_small_kernel<bm, bn, wk, ns, prec, true>), grid, dim3(64 * wk), 0, stream, a); \
      else                                                                                                  \
        return hipErrorInvalidValue;                                                                        \
    } else {                                                                                                \
      hipLaunchKernelGGL((gemm_small_kernel<bm, bn, wk, ns, prec, false>), grid, dim3(64 * wk), 0, stream, a); \
    }                                                                                                       \
    break;
    KH_GEMM_SMALL_CONFIGS(KH_CFGSM_CASE)
#undef KH_CFGSM_CASE
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kh
