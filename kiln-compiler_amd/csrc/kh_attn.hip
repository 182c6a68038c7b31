// kh_attn.hip - the fused attention family: for every batch/head b and query
// row i,
//     s[j]  = (q[b,i,:] . k[b,j,:]) (* or / scale) (+ mask[b,i,j])
//     o[b,i,:] = sum_j softmax(s)[j] * v[b,j,:]
// in one kernel, with the scores never leaving the chip.
//
// This is the kernel the reference lists as its missing piece (README.md:185):
// its backend runs the same computation as five launches (a K^T copy, the
// scores matmul with scale and mask epilogue, a softmax row kernel, the
// probabilities x V matmul and a head-merging copy; kiln/gpu/codegen.py
// 484-530 and 312-430), moving the [B, Tq, Tk] scores through HBM three times.
// The lowering recognises that five-kernel pattern and emits this family
// instead; results agree with the unfused path within fp32 rounding (the
// softmax is evaluated online, FlashAttention-2 style, so the exponentials are
// taken against a running maximum and rescaled).
//
// gfx950 design (fp32 operands on v_mfma_f32_32x32x2_f32, wave64):
//   * a workgroup owns 32 query rows of one head; its NW waves split the key
//     blocks (32 keys each) round-robin and merge their partial results
//     through LDS at the end, so short sequences still put NW waves per
//     query block on the GPU;
//   * the scores are computed transposed, S^T = K Q^T: an accumulator column
//     is one query (lane % 32) and its 16 registers are 16 keys, so the
//     softmax max/sum over keys is a per-lane loop plus one v_permlane32_swap
//     between the lane halves. Each lane keeps its query's Q half-row (DH/2
//     floats, pre-multiplied by scale * log2(e)) in registers for the whole
//     kernel and reads K rows with 128-bit buffer loads; the head dimension
//     is split between the two lane halves (a dot product is order-free);
//   * O^T += V^T P^T consumes the probabilities straight from the score
//     registers: MFMA step r takes, from each lane half, the key held in
//     accumulator register r, so the V^T operand is read with the same key
//     permutation and P never moves through LDS or across lanes;
//   * software pipeline per wave: the score MFMAs of block j+1 are issued
//     interleaved with the softmax VALU work of block j, then the P.V MFMAs of
//     block j interleaved with the loads of later blocks (K two blocks ahead,
//     V one), so the matrix cores keep working through the exponentials;
//   * causal masks (the frozen upper-triangular -inf constant) are applied
//     from indices: key blocks wholly above the diagonal are skipped and only
//     the diagonal block is compared. Other additive masks are read from
//     memory;
//   * workgroups are issued longest-first (causal rows near the end of the
//     sequence have the most key blocks);
//   * grids that 32-query blocks leave short of work (under 1.5 workgroups
//     per CU: the GPT-2 block up to T = 512) run attn16_kernel, 16 queries
//     per workgroup on 16 x 16 MFMAs;
//   * decode shapes (at most 4 queries over at most 64 keys) run a separate
//     kernel with one wave per query row (attn_rows_kernel).
#include <algorithm>
#include <cmath>
#include <cstring>
#include <type_traits>

#include "kh_common.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int kQB = 32;  // queries per workgroup
constexpr int kKB = 32;  // keys per block
// buffer resource word 3 for gfx9-family raw buffers: 32-bit data format
constexpr int kBufferFlags = 0x00020000;

struct AttnArgs {
  const float *q, *k, *v;
  float *o;                // (a bf16 array when o16)
  const float *mask;
  int64_t q_b, q_t, k_b, k_t, v_b, v_t, o_b, o_t, m_b, m_q, m_k;
  int32_t batch, tq, tk, n_qblocks;
  int32_t mask_mode, scale_mode;
  float scale;
  int32_t o16;             // the output is bf16 (its consumer is a bf16 matmul)
  int32_t o_pair;          // the output is pair words (its consumer is a three-pass matmul)
  uint64_t *rec;           // timeline probe only: 8 words per wave (kh_probe_attn_timeline)
};

// Exchange between the two lane halves (lanes l and l ^ 32): returns
// (x[l & 31], x[32 + (l & 31)]), the low half's value first in every lane,
// so a combine of the two is the same in both halves. One v_permlane32_swap.
__device__ __forceinline__ float2 halves(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return make_float2(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// BF: bf16 products (plans whose matrix products take bf16 inputs): Q and K
// rounded to bf16 (round to nearest even) for the scores, the probabilities
// and V for P.V, on v_mfma_f32_32x32x16_bf16; the scale, mask, softmax and
// accumulation stay fp32. The accumulator layouts are those of the fp32
// MFMAs, so everything but the operands is shared:
//   * S^T: MFMA c (16-wide chunk c of the head dimension) takes from lane
//     (col, half) K[key col] and Q[query col] elements 16 c + 8 half .. + 7;
//   * O^T += V^T P^T: MFMA (c, t) covers keys 16 c .. 16 c + 15 of the
//     block, K slot j of lane half h being key 16 c + 8 (j / 4) + 4 h + j % 4
//     - the keys of the lane's score registers 8 c .. 8 c + 7 - so a lane's B
//     operand is its own probabilities and its A operand the V values the
//     fp32 path loads for those registers;
//   * K and V are loaded as fp32 and rounded when an MFMA operand is formed.
// IN16 (with BF): q, k and v are stored as bf16 by their producer, so the
// operands are loaded as bf16 (K as one 16-byte load per chunk, V as 16-bit
// loads paired into MFMA operand words) and rounded by no one here.
// X3 (with BF, fp32 storage): three-pass bf16 products (plans with
// allow_tf32): each of q, k, the probabilities and v splits into bf16 hi and
// lo parts (split_bf16x8) and a product is lo.hi + hi.lo + hi.hi, three MFMAs
// where BF issues one. P3 (with X3): q, k and v are stored as pair words by
// their producer (the two halves already made), so only the probabilities
// are split here.
// REC (the timeline probe only): each wave also records its start, loop-end
// and end times, the shader clock and the CU it ran on.
template <int DH, int NW, bool ADD, bool BF = false, bool REC = false, bool IN16 = false, bool X3 = false,
          bool P3 = false>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void attn_kernel(const AttnArgs a) {
  uint64_t rec_t0 = 0, rec_c0 = 0;
  if constexpr (REC) rec_t0 = __builtin_amdgcn_s_memrealtime(), rec_c0 = __builtin_amdgcn_s_memtime();
  constexpr int NT = DH / 32;  // 32-wide tiles of the head dimension in O^T
  constexpr int QS = DH / 2;   // head-dim elements per lane half (= MFMA steps of S^T)
  __shared__ float o_part[NW][kQB][DH + 4];
  __shared__ float m_part[NW][kQB], l_part[NW][kQB];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave-uniform: scalar loop control
  const int col = lane & 31, half = lane >> 5;
  const int b = blockIdx.x % a.batch;
  const int qb = a.n_qblocks - 1 - (int)(blockIdx.x / a.batch);
  const int q0 = qb * kQB;
  const int qi = q0 + col;
  const bool q_ok = qi < a.tq;

  // Scores are kept in the base-2 domain: u = (s * scale + mask) * log2(e), so
  // each exponential is one v_exp_f32 (exp2) and softmax(s) = 2^(u - max u) / sum.
  // The scale and log2(e) are folded into this lane's Q half-row, which is
  // kept in registers for the whole kernel.
  constexpr float kLog2e = 1.4426950408889634f;
  const float c_scale = a.scale_mode == KH_ATTN_SCALE_MUL   ? a.scale * kLog2e
                        : a.scale_mode == KH_ATTN_SCALE_DIV ? kLog2e / a.scale
                                                            : kLog2e;
  float qf[BF ? 1 : QS];
  bf16x8 qh[BF ? DH / 16 : 1];   // (bf16 products: Q as it is, the scale applied to the scores)
  bf16x8 ql[X3 ? DH / 16 : 1];   // (three-pass products: Q's lo part)
  static_assert(BF || !IN16, "bf16 storage of q, k, v comes with bf16 products");
  static_assert(!X3 || (BF && !IN16), "three-pass products split fp32 q, k, v");
  static_assert(!P3 || X3, "pair-stored q, k, v come with three-pass products");
  if constexpr (IN16) {
    const uint16_t *qp = reinterpret_cast<const uint16_t *>(a.q) + b * a.q_b + (int64_t)min(qi, a.tq - 1) * a.q_t + 8 * half;
#pragma unroll
    for (int c = 0; c < DH / 16; ++c) {
      qh[c] = *reinterpret_cast<const bf16x8 *>(qp + 16 * c);
      if (!q_ok) qh[c] = bf16x8{};
    }
  } else if constexpr (BF) {
    const float *qp = a.q + b * a.q_b + (int64_t)min(qi, a.tq - 1) * a.q_t + 8 * half;
#pragma unroll
    for (int c = 0; c < DH / 16; ++c) {
      float4 x = *reinterpret_cast<const float4 *>(qp + 16 * c), y = *reinterpret_cast<const float4 *>(qp + 16 * c + 4);
      if (!q_ok) x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
      if constexpr (P3) unpair_bf16x8(x, y, qh[c], ql[c]);
      else if constexpr (X3) split_bf16x8<true>(x, y, qh[c], ql[c]);
      else qh[c] = pack_bf16x8(x, y);
    }
  } else {
    const float *qp = a.q + b * a.q_b + (int64_t)min(qi, a.tq - 1) * a.q_t + half * QS;
#pragma unroll
    for (int j = 0; j < QS / 4; ++j) {
      float4 t = *reinterpret_cast<const float4 *>(qp + 4 * j);
      if (!q_ok) t = make_float4(0.f, 0.f, 0.f, 0.f);
      qf[4 * j] = t.x * c_scale, qf[4 * j + 1] = t.y * c_scale;
      qf[4 * j + 2] = t.z * c_scale, qf[4 * j + 3] = t.w * c_scale;
    }
  }

  const bool causal = a.mask_mode == KH_ATTN_MASK_CAUSAL;
  const int kend = causal ? min(a.tk, q0 + kQB) : a.tk;
  const int nkb = (kend + kKB - 1) / kKB;
  // keys below `lim` are visible to this lane's query
  const int lim = causal ? min(a.tk, qi + 1) : a.tk;

  // K and V are read with buffer loads: a per-head resource (base in SGPRs)
  // plus a 32-bit byte offset per lane (the host checks that every operand
  // spans < 2^30 elements) and the column step as an immediate. Key indices
  // are clamped to the last key, so every load of a partial block stays
  // inside the operand (and the resource's extent bounds it as well).
  constexpr uint32_t ES = IN16 ? 2 : 4;   // bytes per q, k, v element
  const uint32_t k_t4 = (uint32_t)a.k_t * ES, v_t4 = (uint32_t)a.v_t * ES;
  const __amdgpu_buffer_rsrc_t k_res = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(reinterpret_cast<const char *>(a.k) + b * a.k_b * ES), (short)0,
      (int)(((uint32_t)(a.tk - 1) * (uint32_t)a.k_t + DH) * ES), kBufferFlags);
  const __amdgpu_buffer_rsrc_t v_res = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(reinterpret_cast<const char *>(a.v) + b * a.v_b * ES), (short)0,
      (int)(((uint32_t)(a.tk - 1) * (uint32_t)a.v_t + DH) * ES), kBufferFlags);
  // a lane's K elements: fp32 products half * QS .. + QS - 1; bf16 products
  // 16 c + 8 half .. + 7 of every chunk c (kf[2 c], kf[2 c + 1]; bf16
  // storage: kf[c], eight bf16)
  const uint32_t k_lane = BF ? half * 8 * ES : half * QS * 4;
  const uint32_t k_last = (uint32_t)(a.tk - 1) * k_t4 + k_lane;
  const uint32_t v_last = (uint32_t)(a.tk - 1) * v_t4 + col * ES;
  auto load_k = [&](int kb, float4 (&kf)[QS / 4]) {
    const uint32_t off = min((uint32_t)(kb * kKB + col) * k_t4 + k_lane, k_last);
#pragma unroll
    for (int j = 0; j < (IN16 ? DH / 16 : QS / 4); ++j) {
      const auto x = __builtin_amdgcn_raw_buffer_load_b128(
          k_res, off + (IN16 ? 32 * j : BF ? 64 * (j / 2) + 16 * (j % 2) : 16 * j), 0, 0);
      kf[j] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3]));
    }
  };
  // V^T operand of MFMA step r, tile t: V[key(r)][t*32 + col], key(r) =
  // key0 + (r/4)*8 + half*4 + r%4, the key held in accumulator register r of
  // this lane half.
  auto load_v = [&](int kb, float (&vf)[16 * NT]) {
    const uint32_t base = (uint32_t)(kb * kKB + half * 4) * v_t4 + col * ES;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const uint32_t off = min(base + (uint32_t)((r >> 2) * 8 + (r & 3)) * v_t4, v_last);
#pragma unroll
      for (int t = 0; t < NT; ++t) {
        if constexpr (IN16)   // (the bf16 bits in the low half)
          vf[r * NT + t] = __uint_as_float((uint32_t)__builtin_amdgcn_raw_buffer_load_b16(v_res, off + 64 * t, 0, 0));
        else
          vf[r * NT + t] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(v_res, off + 128 * t, 0, 0));
      }
    }
  };
  // S^T block: register r of lane (col, half) = score of query col, key(r)
  auto scores = [&](const float4 (&kc)[QS / 4]) {
    f32x16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
    if constexpr (BF) {
#pragma unroll
      for (int c = 0; c < DH / 16; ++c) {
        if constexpr (X3) {
          bf16x8 kh, kl;
          if constexpr (P3) unpair_bf16x8(kc[2 * c], kc[2 * c + 1], kh, kl);
          else split_bf16x8<true>(kc[2 * c], kc[2 * c + 1], kh, kl);
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kl, qh[c], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, ql[c], s, 0, 0, 0);
          s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kh, qh[c], s, 0, 0, 0);
          continue;
        }
        const bf16x8 k8 = IN16 ? __builtin_bit_cast(bf16x8, kc[c]) : pack_bf16x8(kc[2 * c], kc[2 * c + 1]);
        s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k8, qh[c], s, 0, 0, 0);
      }
      return s;
    }
#pragma unroll
    for (int j = 0; j < QS / 4; ++j) {
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[j].x, qf[4 * j + 0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[j].y, qf[4 * j + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[j].z, qf[4 * j + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kc[j].w, qf[4 * j + 3], s, 0, 0, 0);
    }
    return s;
  };

  f32x16 oacc[NT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) oacc[t][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;

  // Online softmax of one score block, in place (scores become the
  // unnormalised probabilities), with the running (max, sum) and O^T rescaled.
  // Only a wave's last block can hold keys past the causal diagonal or past
  // the last key (every earlier block lies wholly below both), so the mask
  // is applied there alone.
  auto softmax = [&](f32x16 &s, int kb, auto masked) {
    const int room = lim - kb * kKB - half * 4;  // key(r) < lim  <=>  (r/4)*8 + r%4 < room
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float u = BF ? s[r] * c_scale : s[r];
      if (ADD) {
        const int key = min(kb * kKB + half * 4 + (r >> 2) * 8 + (r & 3), a.tk - 1);
        u = fmaf(a.mask[b * a.m_b + (int64_t)min(qi, a.tq - 1) * a.m_q + (int64_t)key * a.m_k], kLog2e, u);
      }
      if (decltype(masked)::value) u = (r >> 2) * 8 + (r & 3) < room ? u : -INFINITY;
      s[r] = u;
      mx = fmaxf(mx, u);
    }
    const float2 mh = halves(mx);
    const float m_new = fmaxf(m_run, fmaxf(mh.x, mh.y));
    // a row with no finite score so far keeps m = -inf; exponentials are then
    // taken against 0 so they stay 0 instead of becoming NaN
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float sum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[r] = __builtin_amdgcn_exp2f(s[r] - m_use);
      sum += s[r];
    }
    const float2 sh = halves(sum);
    l_run = fmaf(l_run, alpha, sh.x + sh.y);
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < NT; ++t) oacc[t] *= alpha;
  };
  // O^T += V^T P^T, key order permuted to match the score registers
  auto pv = [&](const float (&vf)[16 * NT], const f32x16 &p) {
    if constexpr (BF) {
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        const float4 p0 = make_float4(p[8 * c], p[8 * c + 1], p[8 * c + 2], p[8 * c + 3]);
        const float4 p1 = make_float4(p[8 * c + 4], p[8 * c + 5], p[8 * c + 6], p[8 * c + 7]);
        bf16x8 pb, pl;
        if constexpr (X3) split_bf16x8<false>(p0, p1, pb, pl);
        else pb = pack_bf16x8(p0, p1);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
          const float *v8 = vf + 8 * c * NT + t;
          bf16x8 va;
          if constexpr (X3) {
            bf16x8 vl;
            const float4 v0 = make_float4(v8[0], v8[NT], v8[2 * NT], v8[3 * NT]);
            const float4 v1 = make_float4(v8[4 * NT], v8[5 * NT], v8[6 * NT], v8[7 * NT]);
            if constexpr (P3) unpair_bf16x8(v0, v1, va, vl);
            else split_bf16x8<true>(v0, v1, va, vl);
            oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vl, pb, oacc[t], 0, 0, 0);
            oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pl, oacc[t], 0, 0, 0);
          } else if constexpr (IN16) {
            uint4 w;
            w.x = __float_as_uint(v8[0]) | (__float_as_uint(v8[NT]) << 16);
            w.y = __float_as_uint(v8[2 * NT]) | (__float_as_uint(v8[3 * NT]) << 16);
            w.z = __float_as_uint(v8[4 * NT]) | (__float_as_uint(v8[5 * NT]) << 16);
            w.w = __float_as_uint(v8[6 * NT]) | (__float_as_uint(v8[7 * NT]) << 16);
            va = __builtin_bit_cast(bf16x8, w);
          } else {
            va = pack_bf16x8(make_float4(v8[0], v8[NT], v8[2 * NT], v8[3 * NT]),
                             make_float4(v8[4 * NT], v8[5 * NT], v8[6 * NT], v8[7 * NT]));
          }
          oacc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(va, pb, oacc[t], 0, 0, 0);
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int t = 0; t < NT; ++t)
        oacc[t] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[r * NT + t], p[r], oacc[t], 0, 0, 0);
  };

  // Software pipeline over this wave's key blocks (w, w + NW, ...): the score
  // MFMAs of the next block are issued before the softmax of the current one,
  // so the matrix cores work through the exponentials; K runs two blocks and
  // V one block ahead of their use.
  int kb = w;
  if (kb < nkb) {
    float4 kf[QS / 4];
    float vf[16 * NT];
    load_k(kb, kf);
    load_v(kb, vf);
    f32x16 s_cur = scores(kf);
    load_k(min(kb + NW, nkb - 1), kf);
    for (; kb + NW < nkb; kb += NW) {
      const f32x16 s_nxt = scores(kf);
      softmax(s_cur, kb, std::false_type{});
      load_k(min(kb + 2 * NW, nkb - 1), kf);
      pv(vf, s_cur);
      load_v(kb + NW, vf);
      s_cur = s_nxt;
      // issue order (fp32 products): each score MFMA of the next block
      // followed by softmax VALU work, then each P.V MFMA followed by a load
      // and its addressing
      if constexpr (!BF) {
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
          __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
        }
      }
    }
    softmax(s_cur, kb, std::true_type{});
    pv(vf, s_cur);
  }

  uint64_t rec_t1 = 0;
  if constexpr (REC) rec_t1 = __builtin_amdgcn_s_memrealtime();
  // merge the NW key-split partials: o = sum_w 2^(m_w - M) o_w / sum_w 2^(m_w - M) l_w
  if (half == 0) m_part[w][col] = m_run, l_part[w][col] = l_run;
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o_part[w][col][t * 32 + (r >> 2) * 8 + half * 4 + (r & 3)] = oacc[t][r];
  __syncthreads();
  constexpr int kChunks = kQB * DH / 4;
  for (int c = threadIdx.x; c < kChunks; c += 64 * NW) {
    const int qr = c / (DH / 4), d = (c % (DH / 4)) * 4;
    if (q0 + qr >= a.tq) continue;
    float mm = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) mm = fmaxf(mm, m_part[u][qr]);
    const float mu = mm == -INFINITY ? 0.0f : mm;
    float l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float e = __builtin_amdgcn_exp2f(m_part[u][qr] - mu);   // m is in the base-2 domain
      l += l_part[u][qr] * e;
      acc.x += o_part[u][qr][d] * e, acc.y += o_part[u][qr][d + 1] * e;
      acc.z += o_part[u][qr][d + 2] * e, acc.w += o_part[u][qr][d + 3] * e;
    }
    acc.x /= l, acc.y /= l, acc.z /= l, acc.w /= l;
    const int64_t at = b * a.o_b + (int64_t)(q0 + qr) * a.o_t + d;
    if (a.o_pair) acc = make_float4(pair_word(acc.x), pair_word(acc.y), pair_word(acc.z), pair_word(acc.w));
    if (a.o16) store_bf16x4(a.o, at, acc.x, acc.y, acc.z, acc.w);
    else *reinterpret_cast<float4 *>(a.o + at) = acc;
  }
  if constexpr (REC) {
    const uint64_t t2 = __builtin_amdgcn_s_memrealtime(), c2 = __builtin_amdgcn_s_memtime();
    uint32_t hw, xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    if (lane == 0) {
      uint64_t *r = a.rec + ((int64_t)blockIdx.x * NW + w) * 8;
      r[0] = rec_t0, r[1] = rec_t1, r[2] = t2, r[3] = rec_c0, r[4] = c2;
      r[5] = hw, r[6] = xcc, r[7] = w < nkb ? (uint64_t)((nkb - w + NW - 1) / NW) : 0;
    }
  }
}

// The same computation with 16 queries per workgroup on
// v_mfma_f32_16x16x4_f32, for grids that 32-query blocks leave short of work
// (a 32-key block costs a wave half the matrix-core time it costs above, and
// a causal row's key blocks spread over twice the workgroups). Lane (li =
// lane % 16, g = lane / 16):
//   * S^T = K Q^T as two 16 x 16 tiles per 32-key block: lane (li, g) holds
//     the scores of query li with keys 16 t + 4 g + r (tile t, register r);
//     MFMA step j of a tile sums head-dimension element g * DH/4 + j of the
//     four lane groups (the dot product is order-free), so each lane reads
//     its Q and K row pieces as contiguous 128-bit loads;
//   * the softmax max and sum over a query's 32 keys: 8 registers per lane,
//     then the four lane groups (two xor shuffles, the same bits in all four);
//   * O^T += V^T P^T: MFMA step (t, r) takes key 16 t + 4 g + r from lane
//     group g, which is where that key's probability already is; lane (li,
//     g) ends with head-dimension elements 16 d + 4 g .. + 3 of query li,
//     written as one 128-bit store per 16-wide tile d.
template <int DH, int NW, bool ADD>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void attn16_kernel(const AttnArgs a) {
  constexpr int QB = 16;       // queries per workgroup
  constexpr int QS = DH / 4;   // head-dimension elements per lane group (MFMA steps of a score tile)
  constexpr int DT = DH / 16;  // 16-wide tiles of the head dimension in O^T
  __shared__ __attribute__((aligned(16))) float o_part[NW][QB][DH + 4];   // (128-bit stores: 16-byte rows)
  __shared__ float m_part[NW][QB], l_part[NW][QB];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int b = blockIdx.x % a.batch;
  const int qb = a.n_qblocks - 1 - (int)(blockIdx.x / a.batch);
  const int q0 = qb * QB;
  const int qi = q0 + li;
  const bool q_ok = qi < a.tq;

  constexpr float kLog2e = 1.4426950408889634f;
  const float c_scale = a.scale_mode == KH_ATTN_SCALE_MUL   ? a.scale * kLog2e
                        : a.scale_mode == KH_ATTN_SCALE_DIV ? kLog2e / a.scale
                                                            : kLog2e;
  float qf[QS];
  {
    const float *qp = a.q + b * a.q_b + (int64_t)min(qi, a.tq - 1) * a.q_t + g * QS;
#pragma unroll
    for (int j = 0; j < QS / 4; ++j) {
      float4 t = *reinterpret_cast<const float4 *>(qp + 4 * j);
      if (!q_ok) t = make_float4(0.f, 0.f, 0.f, 0.f);
      qf[4 * j] = t.x * c_scale, qf[4 * j + 1] = t.y * c_scale;
      qf[4 * j + 2] = t.z * c_scale, qf[4 * j + 3] = t.w * c_scale;
    }
  }

  const bool causal = a.mask_mode == KH_ATTN_MASK_CAUSAL;
  const int kend = causal ? min(a.tk, q0 + QB) : a.tk;
  const int nkb = (kend + kKB - 1) / kKB;
  const int lim = causal ? min(a.tk, qi + 1) : a.tk;

  // buffer loads as in attn_kernel: key indices clamped to the last key
  const uint32_t k_t4 = (uint32_t)a.k_t * 4, v_t4 = (uint32_t)a.v_t * 4;
  const __amdgpu_buffer_rsrc_t k_res = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.k + b * a.k_b), (short)0, (int)(((uint32_t)(a.tk - 1) * (uint32_t)a.k_t + DH) * 4), kBufferFlags);
  const __amdgpu_buffer_rsrc_t v_res = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.v + b * a.v_b), (short)0, (int)(((uint32_t)(a.tk - 1) * (uint32_t)a.v_t + DH) * 4), kBufferFlags);
  const uint32_t k_last = (uint32_t)(a.tk - 1) * k_t4 + g * QS * 4;
  const uint32_t v_last = (uint32_t)(a.tk - 1) * v_t4 + li * 4;
  // K[16 t + li][g * QS ..] of key block kb, tile t
  auto load_k = [&](int kb, float4 (&kf)[2][QS / 4]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t off = min((uint32_t)(kb * kKB + t * 16 + li) * k_t4 + g * QS * 4, k_last);
#pragma unroll
      for (int j = 0; j < QS / 4; ++j) {
        const auto x = __builtin_amdgcn_raw_buffer_load_b128(k_res, off + 16 * j, 0, 0);
        kf[t][j] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]), __uint_as_float(x[3]));
      }
    }
  };
  // V^T operand of MFMA step (t, r), tile d: V[16 t + 4 g + r][16 d + li]
  auto load_v = [&](int kb, float (&vf)[8 * DT]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t off = min((uint32_t)(kb * kKB + t * 16 + 4 * g + r) * v_t4 + li * 4, v_last);
#pragma unroll
        for (int d = 0; d < DT; ++d)
          vf[(t * 4 + r) * DT + d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(v_res, off + 64 * d, 0, 0));
      }
  };
  auto scores = [&](const float4 (&kc)[2][QS / 4], f32x4 (&s)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < QS / 4; ++j) {
        s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[t][j].x, qf[4 * j + 0], s[t], 0, 0, 0);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[t][j].y, qf[4 * j + 1], s[t], 0, 0, 0);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[t][j].z, qf[4 * j + 2], s[t], 0, 0, 0);
        s[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(kc[t][j].w, qf[4 * j + 3], s[t], 0, 0, 0);
      }
    }
  };

  f32x4 oacc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  // online softmax of one score block, as in attn_kernel (base-2 domain, a
  // row with no finite score so far takes its exponentials against 0)
  auto softmax = [&](f32x4 (&s)[2], int kb, auto masked) {
    const int room = lim - kb * kKB - 4 * g;   // key(t, r) < lim  <=>  16 t + r < room
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float u = s[t][r];
        if (ADD) {
          const int key = min(kb * kKB + t * 16 + 4 * g + r, a.tk - 1);
          u = fmaf(a.mask[b * a.m_b + (int64_t)min(qi, a.tq - 1) * a.m_q + (int64_t)key * a.m_k], kLog2e, u);
        }
        if (decltype(masked)::value) u = 16 * t + r < room ? u : -INFINITY;
        s[t][r] = u;
        mx = fmaxf(mx, u);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[t][r] = __builtin_amdgcn_exp2f(s[t][r] - m_use);
        sum += s[t][r];
      }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    l_run = fmaf(l_run, alpha, sum);
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < DT; ++d) oacc[d] *= alpha;
  };
  auto pv = [&](const float (&vf)[8 * DT], const f32x4 (&p)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int d = 0; d < DT; ++d)
          oacc[d] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[(t * 4 + r) * DT + d], p[t][r], oacc[d], 0, 0, 0);
  };

  // the software pipeline of attn_kernel: K two blocks and V one block ahead
  int kb = w;
  if (kb < nkb) {
    float4 kf[2][QS / 4];
    float vf[8 * DT];
    f32x4 s_cur[2], s_nxt[2];
    load_k(kb, kf);
    load_v(kb, vf);
    scores(kf, s_cur);
    load_k(min(kb + NW, nkb - 1), kf);
    for (; kb + NW < nkb; kb += NW) {
      scores(kf, s_nxt);
      softmax(s_cur, kb, std::false_type{});
      load_k(min(kb + 2 * NW, nkb - 1), kf);
      pv(vf, s_cur);
      load_v(kb + NW, vf);
      s_cur[0] = s_nxt[0], s_cur[1] = s_nxt[1];
#pragma unroll
      for (int i = 0; i < 2 * QS; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // VALU
      }
#pragma unroll
      for (int i = 0; i < 8 * DT; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // VMEM read
        __builtin_amdgcn_sched_group_barrier(0x002, 1, 0);  // VALU
      }
    }
    softmax(s_cur, kb, std::true_type{});
    pv(vf, s_cur);
  }

  // merge the NW key-split partials as in attn_kernel
  if (g == 0) m_part[w][li] = m_run, l_part[w][li] = l_run;
#pragma unroll
  for (int d = 0; d < DT; ++d)
    *reinterpret_cast<float4 *>(&o_part[w][li][d * 16 + 4 * g]) = make_float4(oacc[d][0], oacc[d][1], oacc[d][2], oacc[d][3]);
  __syncthreads();
  constexpr int kChunks = QB * DH / 4;
  for (int c = threadIdx.x; c < kChunks; c += 64 * NW) {
    const int qr = c / (DH / 4), d = (c % (DH / 4)) * 4;
    if (q0 + qr >= a.tq) continue;
    float mm = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) mm = fmaxf(mm, m_part[u][qr]);
    const float mu = mm == -INFINITY ? 0.0f : mm;
    float l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float e = __builtin_amdgcn_exp2f(m_part[u][qr] - mu);
      l += l_part[u][qr] * e;
      acc.x += o_part[u][qr][d] * e, acc.y += o_part[u][qr][d + 1] * e;
      acc.z += o_part[u][qr][d + 2] * e, acc.w += o_part[u][qr][d + 3] * e;
    }
    acc.x /= l, acc.y /= l, acc.z /= l, acc.w /= l;
    const int64_t at = b * a.o_b + (int64_t)(q0 + qr) * a.o_t + d;
    if (a.o_pair) acc = make_float4(pair_word(acc.x), pair_word(acc.y), pair_word(acc.z), pair_word(acc.w));
    if (a.o16) store_bf16x4(a.o, at, acc.x, acc.y, acc.z, acc.w);
    else *reinterpret_cast<float4 *>(a.o + at) = acc;
  }
}

// The 16-query computation with bf16 products (plans whose matrix products
// run bf16 inputs with fp32 accumulation): Q and K rounded to bf16 (round to
// nearest even) for the scores, the probabilities and V rounded to bf16 for
// P.V, on v_mfma_f32_16x16x32_bf16; the scale, the mask, the softmax and the
// accumulation stay fp32. Lane (li, g) layout as in attn16_kernel:
//   * S^T tile t (16 keys) is one MFMA per 32-wide chunk c of the head
//     dimension: lane (li, g) gives K[16 t + li] and Q[li] elements
//     32 c + 8 g .. + 7, and holds the scores of query li with keys
//     16 t + 4 g + r (register r), the layout the softmax of attn16_kernel
//     works on;
//   * O^T += V^T P^T is one MFMA per 16-wide head-dimension tile d over all
//     32 keys of a block: K slot j of lane group g is key 16 (j / 4) + 4 g +
//     j % 4, so a lane's B operand is its own 8 probabilities and its A
//     operand V[that key][16 d + li];
//   * K and V are loaded as fp32 (the operands of the launch are fp32) and
//     converted when the MFMA operands are formed, so a load is not waited
//     for before its block is reached.
template <int DH, int NW, bool ADD>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(2))) void attnbf_kernel(const AttnArgs a) {
  constexpr int QB = 16;       // queries per workgroup
  constexpr int QC = DH / 32;  // 32-wide chunks of the head dimension (K steps of a score MFMA)
  constexpr int DT = DH / 16;  // 16-wide tiles of the head dimension in O^T
  __shared__ __attribute__((aligned(16))) float o_part[NW][QB][DH + 4];
  __shared__ float m_part[NW][QB], l_part[NW][QB];

  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, g = lane >> 4;
  const int b = blockIdx.x % a.batch;
  const int qb = a.n_qblocks - 1 - (int)(blockIdx.x / a.batch);
  const int q0 = qb * QB;
  const int qi = q0 + li;
  const bool q_ok = qi < a.tq;

  constexpr float kLog2e = 1.4426950408889634f;
  // applied to the fp32 scores (the products see Q as it is)
  const float c_scale = a.scale_mode == KH_ATTN_SCALE_MUL   ? a.scale * kLog2e
                        : a.scale_mode == KH_ATTN_SCALE_DIV ? kLog2e / a.scale
                                                            : kLog2e;
  auto pack8 = [](const float4 &x, const float4 &y) { return pack_bf16x8(x, y); };
  bf16x8 qh[QC];
  {
    const float *qp = a.q + b * a.q_b + (int64_t)min(qi, a.tq - 1) * a.q_t + 8 * g;
#pragma unroll
    for (int c = 0; c < QC; ++c) {
      float4 x = *reinterpret_cast<const float4 *>(qp + 32 * c), y = *reinterpret_cast<const float4 *>(qp + 32 * c + 4);
      if (!q_ok) x = make_float4(0.f, 0.f, 0.f, 0.f), y = x;
      qh[c] = pack8(x, y);
    }
  }

  const bool causal = a.mask_mode == KH_ATTN_MASK_CAUSAL;
  const int kend = causal ? min(a.tk, q0 + QB) : a.tk;
  const int nkb = (kend + kKB - 1) / kKB;
  const int lim = causal ? min(a.tk, qi + 1) : a.tk;

  // buffer loads as in attn_kernel: key indices clamped to the last key
  const uint32_t k_t4 = (uint32_t)a.k_t * 4, v_t4 = (uint32_t)a.v_t * 4;
  const __amdgpu_buffer_rsrc_t k_res = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.k + b * a.k_b), (short)0, (int)(((uint32_t)(a.tk - 1) * (uint32_t)a.k_t + DH) * 4), kBufferFlags);
  const __amdgpu_buffer_rsrc_t v_res = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(a.v + b * a.v_b), (short)0, (int)(((uint32_t)(a.tk - 1) * (uint32_t)a.v_t + DH) * 4), kBufferFlags);
  const uint32_t k_last = (uint32_t)(a.tk - 1) * k_t4 + g * 32;
  const uint32_t v_last = (uint32_t)(a.tk - 1) * v_t4 + li * 4;
  // K[16 t + li][32 c + 8 g .. + 7] of key block kb: kf[t][c][0..1]
  auto load_k = [&](int kb, float4 (&kf)[2][QC][2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const uint32_t off = min((uint32_t)(kb * kKB + t * 16 + li) * k_t4 + g * 32, k_last);
#pragma unroll
      for (int c = 0; c < QC; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const auto x = __builtin_amdgcn_raw_buffer_load_b128(k_res, off + 128 * c + 16 * h, 0, 0);
          kf[t][c][h] = make_float4(__uint_as_float(x[0]), __uint_as_float(x[1]), __uint_as_float(x[2]),
                                    __uint_as_float(x[3]));
        }
    }
  };
  // V^T operand of tile d, K slot j = 4 t + r: V[16 t + 4 g + r][16 d + li]
  auto load_v = [&](int kb, float (&vf)[8 * DT]) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t off = min((uint32_t)(kb * kKB + t * 16 + 4 * g + r) * v_t4 + li * 4, v_last);
#pragma unroll
        for (int d = 0; d < DT; ++d)
          vf[(t * 4 + r) * DT + d] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(v_res, off + 64 * d, 0, 0));
      }
  };
  auto scores = [&](const float4 (&kf)[2][QC][2], f32x4 (&s)[2]) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      s[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < QC; ++c)
        s[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pack8(kf[t][c][0], kf[t][c][1]), qh[c], s[t], 0, 0, 0);
    }
  };

  f32x4 oacc[DT];
#pragma unroll
  for (int d = 0; d < DT; ++d) oacc[d] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.0f;

  // online softmax of one score block as in attn16_kernel, the scale applied
  // here; the probabilities' fp32 sum is the normaliser
  auto softmax = [&](f32x4 (&s)[2], int kb, auto masked) {
    const int room = lim - kb * kKB - 4 * g;   // key(t, r) < lim  <=>  16 t + r < room
    float mx = -INFINITY;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        float u = s[t][r] * c_scale;
        if (ADD) {
          const int key = min(kb * kKB + t * 16 + 4 * g + r, a.tk - 1);
          u = fmaf(a.mask[b * a.m_b + (int64_t)min(qi, a.tq - 1) * a.m_q + (int64_t)key * a.m_k], kLog2e, u);
        }
        if (decltype(masked)::value) u = 16 * t + r < room ? u : -INFINITY;
        s[t][r] = u;
        mx = fmaxf(mx, u);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    float sum = 0.0f;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s[t][r] = __builtin_amdgcn_exp2f(s[t][r] - m_use);
        sum += s[t][r];
      }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    l_run = fmaf(l_run, alpha, sum);
    m_run = m_new;
#pragma unroll
    for (int d = 0; d < DT; ++d) oacc[d] *= alpha;
  };
  auto pv = [&](const float (&vf)[8 * DT], const f32x4 (&p)[2]) {
    const bf16x8 pb = pack8(make_float4(p[0][0], p[0][1], p[0][2], p[0][3]), make_float4(p[1][0], p[1][1], p[1][2], p[1][3]));
#pragma unroll
    for (int d = 0; d < DT; ++d) {
      const bf16x8 va = pack_bf16x8(make_float4(vf[d], vf[DT + d], vf[2 * DT + d], vf[3 * DT + d]),
                                    make_float4(vf[4 * DT + d], vf[5 * DT + d], vf[6 * DT + d], vf[7 * DT + d]));
      oacc[d] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb, oacc[d], 0, 0, 0);
    }
  };

  // the software pipeline of attn16_kernel: K two blocks and V one block ahead
  int kb = w;
  if (kb < nkb) {
    float4 kf[2][QC][2];
    float vf[8 * DT];
    f32x4 s_cur[2], s_nxt[2];
    load_k(kb, kf);
    load_v(kb, vf);
    scores(kf, s_cur);
    load_k(min(kb + NW, nkb - 1), kf);
    for (; kb + NW < nkb; kb += NW) {
      scores(kf, s_nxt);
      softmax(s_cur, kb, std::false_type{});
      load_k(min(kb + 2 * NW, nkb - 1), kf);
      pv(vf, s_cur);
      load_v(kb + NW, vf);
      s_cur[0] = s_nxt[0], s_cur[1] = s_nxt[1];
    }
    softmax(s_cur, kb, std::true_type{});
    pv(vf, s_cur);
  }

  // merge the NW key-split partials as in attn_kernel
  if (g == 0) m_part[w][li] = m_run, l_part[w][li] = l_run;
#pragma unroll
  for (int d = 0; d < DT; ++d)
    *reinterpret_cast<float4 *>(&o_part[w][li][d * 16 + 4 * g]) = make_float4(oacc[d][0], oacc[d][1], oacc[d][2], oacc[d][3]);
  __syncthreads();
  constexpr int kChunks = QB * DH / 4;
  for (int c = threadIdx.x; c < kChunks; c += 64 * NW) {
    const int qr = c / (DH / 4), d = (c % (DH / 4)) * 4;
    if (q0 + qr >= a.tq) continue;
    float mm = -INFINITY;
#pragma unroll
    for (int u = 0; u < NW; ++u) mm = fmaxf(mm, m_part[u][qr]);
    const float mu = mm == -INFINITY ? 0.0f : mm;
    float l = 0.0f;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int u = 0; u < NW; ++u) {
      const float e = __builtin_amdgcn_exp2f(m_part[u][qr] - mu);
      l += l_part[u][qr] * e;
      acc.x += o_part[u][qr][d] * e, acc.y += o_part[u][qr][d + 1] * e;
      acc.z += o_part[u][qr][d + 2] * e, acc.w += o_part[u][qr][d + 3] * e;
    }
    acc.x /= l, acc.y /= l, acc.z /= l, acc.w /= l;
    const int64_t at = b * a.o_b + (int64_t)(q0 + qr) * a.o_t + d;
    if (a.o_pair) acc = make_float4(pair_word(acc.x), pair_word(acc.y), pair_word(acc.z), pair_word(acc.w));
    if (a.o16) store_bf16x4(a.o, at, acc.x, acc.y, acc.z, acc.w);
    else *reinterpret_cast<float4 *>(a.o + at) = acc;
  }
}

// Few-query attention (decode shapes: Tq <= kRowsMaxQ queries over at most
// kRowsMaxK keys): one wave per (head, query), lane d holding head dimension
// d (lanes DH.. idle for DH = 32). Each chunk of kRowKeys keys has its K and
// V rows (and mask values) loaded before the first dot product; a score is
// one wave sum. The online softmax is the one of attn_kernel: base-2 domain,
// u = (s * scale + mask) * log2(e), and a row with no finite score so far
// takes its exponentials against 0, so a fully masked row ends as 0 / 0 =
// NaN (as in eager) and a NaN or +inf score turns the row NaN.
constexpr int kRowsMaxQ = 4;
constexpr int kRowsMaxK = 64;
constexpr int kRowKeys = 8;

template <int DH, bool ADD>
__global__ __launch_bounds__(256) void attn_rows_kernel(const AttnArgs a) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= a.batch * a.tq) return;  // whole waves; the kernel has no barrier
  const int b = row / a.tq, qi = row % a.tq;
  const bool on = lane < DH;
  const int d = on ? lane : 0;
  constexpr float kLog2e = 1.4426950408889634f;
  const float c_scale = a.scale_mode == KH_ATTN_SCALE_MUL   ? a.scale * kLog2e
                        : a.scale_mode == KH_ATTN_SCALE_DIV ? kLog2e / a.scale
                                                            : kLog2e;
  const float qv = on ? a.q[b * a.q_b + (int64_t)qi * a.q_t + d] * c_scale : 0.0f;
  const int lim = a.mask_mode == KH_ATTN_MASK_CAUSAL ? min(a.tk, qi + 1) : a.tk;
  const float *kp = a.k + b * a.k_b + d, *vp = a.v + b * a.v_b + d;
  float m = -INFINITY, l = 0.0f, acc = 0.0f;
  for (int j0 = 0; j0 < lim; j0 += kRowKeys) {
    float kv[kRowKeys], vv[kRowKeys], mv[kRowKeys];
#pragma unroll
    for (int c = 0; c < kRowKeys; ++c) {
      const int j = min(j0 + c, lim - 1);  // clamped: an in-bounds load, the key is dropped below
      kv[c] = kp[(int64_t)j * a.k_t];
      vv[c] = vp[(int64_t)j * a.v_t];
      if (ADD) mv[c] = a.mask[b * a.m_b + (int64_t)qi * a.m_q + (int64_t)j * a.m_k];
    }
#pragma unroll
    for (int c = 0; c < kRowKeys; ++c) {
      if (j0 + c >= lim) break;
      float u = wave_sum(qv * kv[c]);
      if (ADD) u = fmaf(mv[c], kLog2e, u);
      const float m_new = fmaxf(m, u);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m - m_use);
      const float p = __builtin_amdgcn_exp2f(u - m_use);
      l = fmaf(l, alpha, p);
      acc = fmaf(acc, alpha, p * vv[c]);
      m = m_new;
    }
  }
  if (on) a.o[b * a.o_b + (int64_t)qi * a.o_t + d] = acc / l;
}

class AttnOp final : public Op {
 public:
  AttnArgs args{};
  int dh = 64, nw = 4;
  bool rows = false;  // few-query kernel
  bool q16 = false;   // 16 queries per workgroup (attn16_kernel)
  bool bf = false;    // bf16 products (attn_kernel<..., BF> / attnbf_kernel)
  bool in16 = false;  // q, k, v stored as bf16 (attn_kernel<..., BF, ..., IN16>)
  bool x3 = false;    // three-pass bf16 products (attn_kernel<..., BF, ..., X3>)
  bool p3 = false;    // q, k, v stored as pair words (attn_kernel<..., X3, P3>)
  dim3 grid;

  hipError_t launch(float *const *ptrs, float *, hipStream_t stream) override {
    AttnArgs a = args;
    a.q = ptrs[0], a.k = ptrs[1], a.v = ptrs[2], a.o = ptrs[3];
    a.mask = a.mask_mode == KH_ATTN_MASK_ADD ? ptrs[4] : nullptr;
    for (int j = 0; j < 4; ++j)
      if (reinterpret_cast<uintptr_t>(ptrs[j]) & (j == 3 && a.o16 ? 7 : 15)) return hipErrorInvalidValue;
    if (a.batch == 0 || a.tq == 0) return hipSuccess;
    if (rows) {
      const dim3 g((unsigned)((a.batch * a.tq + 3) / 4));
      const bool add = a.mask_mode == KH_ATTN_MASK_ADD;
      if (dh == 64 && add) hipLaunchKernelGGL((attn_rows_kernel<64, true>), g, dim3(256), 0, stream, a);
      else if (dh == 64) hipLaunchKernelGGL((attn_rows_kernel<64, false>), g, dim3(256), 0, stream, a);
      else if (add) hipLaunchKernelGGL((attn_rows_kernel<32, true>), g, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((attn_rows_kernel<32, false>), g, dim3(256), 0, stream, a);
      return hipGetLastError();
    }
#define KH_ATTNBF_LAUNCH(D, W)                                                                       \
  if (bf && q16 && dh == D && nw == W) {                                                             \
    if (a.mask_mode == KH_ATTN_MASK_ADD)                                                             \
      hipLaunchKernelGGL((attnbf_kernel<D, W, true>), grid, dim3(64 * W), 0, stream, a);            \
    else                                                                                             \
      hipLaunchKernelGGL((attnbf_kernel<D, W, false>), grid, dim3(64 * W), 0, stream, a);           \
    return hipGetLastError();                                                                        \
  }
    KH_ATTNBF_LAUNCH(64, 8)
    KH_ATTNBF_LAUNCH(64, 4)
    KH_ATTNBF_LAUNCH(64, 2)
    KH_ATTNBF_LAUNCH(64, 1)
    KH_ATTNBF_LAUNCH(32, 4)
    KH_ATTNBF_LAUNCH(32, 2)
    KH_ATTNBF_LAUNCH(32, 1)
#undef KH_ATTNBF_LAUNCH
#define KH_ATTN16_LAUNCH(D, W)                                                                       \
  if (q16 && dh == D && nw == W) {                                                                   \
    if (a.mask_mode == KH_ATTN_MASK_ADD)                                                             \
      hipLaunchKernelGGL((attn16_kernel<D, W, true>), grid, dim3(64 * W), 0, stream, a);            \
    else                                                                                             \
      hipLaunchKernelGGL((attn16_kernel<D, W, false>), grid, dim3(64 * W), 0, stream, a);           \
    return hipGetLastError();                                                                        \
  }
    KH_ATTN16_LAUNCH(64, 8)
    KH_ATTN16_LAUNCH(64, 4)
    KH_ATTN16_LAUNCH(64, 2)
    KH_ATTN16_LAUNCH(64, 1)
    KH_ATTN16_LAUNCH(32, 4)
    KH_ATTN16_LAUNCH(32, 2)
    KH_ATTN16_LAUNCH(32, 1)
#undef KH_ATTN16_LAUNCH
#define KH_ATTN_LAUNCH(D, W)                                                                         \
  if (dh == D && nw == W) {                                                                          \
    const bool add = a.mask_mode == KH_ATTN_MASK_ADD;                                                \
    if (p3 && add) hipLaunchKernelGGL((attn_kernel<D, W, true, true, false, false, true, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (p3) hipLaunchKernelGGL((attn_kernel<D, W, false, true, false, false, true, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (x3 && add) hipLaunchKernelGGL((attn_kernel<D, W, true, true, false, false, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (x3) hipLaunchKernelGGL((attn_kernel<D, W, false, true, false, false, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (in16 && add) hipLaunchKernelGGL((attn_kernel<D, W, true, true, false, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (in16) hipLaunchKernelGGL((attn_kernel<D, W, false, true, false, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (bf && add) hipLaunchKernelGGL((attn_kernel<D, W, true, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (bf) hipLaunchKernelGGL((attn_kernel<D, W, false, true>), grid, dim3(64 * W), 0, stream, a); \
    else if (add) hipLaunchKernelGGL((attn_kernel<D, W, true>), grid, dim3(64 * W), 0, stream, a);  \
    else hipLaunchKernelGGL((attn_kernel<D, W, false>), grid, dim3(64 * W), 0, stream, a);         \
    return hipGetLastError();                                                                        \
  }
    KH_ATTN_LAUNCH(64, 8)
    KH_ATTN_LAUNCH(64, 4)
    KH_ATTN_LAUNCH(64, 2)
    KH_ATTN_LAUNCH(64, 1)
    KH_ATTN_LAUNCH(32, 4)
    KH_ATTN_LAUNCH(32, 2)
    KH_ATTN_LAUNCH(32, 1)
#undef KH_ATTN_LAUNCH
    return hipErrorInvalidValue;
  }
};

bool aligned4(int64_t v) { return v % 4 == 0; }

}  // namespace

std::unique_ptr<Op> make_attn(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  const int mask_mode = L.cfg[0], scale_mode = L.cfg[1];
  if (mask_mode < KH_ATTN_MASK_NONE || mask_mode > KH_ATTN_MASK_ADD || scale_mode < KH_ATTN_SCALE_NONE ||
      scale_mode > KH_ATTN_SCALE_DIV) {
    err = "attention: bad mask or scale mode";
    return nullptr;
  }
  const int want_refs = mask_mode == KH_ATTN_MASK_ADD ? 5 : 4;
  if (L.n_refs != want_refs) {
    err = "attention: expected q, k, v, out" + std::string(want_refs == 5 ? ", mask" : "") + " operands";
    return nullptr;
  }
  const int64_t batch = L.gemm[0], tq = L.gemm[1], tk = L.gemm[2], dh = L.gemm[3];
  if (batch < 0 || tq < 0 || tk < 0 || batch >= (1 << 20) || tq >= (1 << 24) || tk >= (1 << 24)) {
    unsupported = true;
    err = "attention: sizes out of range";
    return nullptr;
  }
  if (tq > 0 && tk == 0) {
    err = "attention: no keys";
    return nullptr;
  }
  if (dh != 32 && dh != 64) {
    unsupported = true;
    err = "attention: head dimension must be 32 or 64";
    return nullptr;
  }
  const uint32_t m16 = bf16_refs(L);
  for (int j = 0; j < 4; ++j) {
    const kh_ref &r = L.refs[j];
    // 16-byte aligned rows: 4 fp32 or (bf16 storage of q, k, v) 8 bf16 elements
    const int64_t al = j < 3 && (m16 >> j & 1) ? 8 : 4;
    if (r.strides[2] != 1 || r.offset % al || r.strides[0] % al || r.strides[1] % al) {
      unsupported = true;
      err = "attention: q, k, v and out need unit head-dim stride and 16-byte aligned rows";
      return nullptr;
    }
  }
  for (int j = 0; j < 4; ++j) {
    const kh_ref &r = L.refs[j];
    const int64_t rows = j == 0 || j == 3 ? tq : tk;
    const int64_t span = std::max<int64_t>(0, batch - 1) * r.strides[0] + std::max<int64_t>(0, rows - 1) * r.strides[1] + dh;
    if (r.strides[0] < 0 || r.strides[1] < 0 || span >= (1ll << 30)) {
      unsupported = true;
      err = "attention: operands must span fewer than 2^30 elements with non-negative strides";
      return nullptr;
    }
  }
  if (scale_mode == KH_ATTN_SCALE_DIV && L.fparams[0] == 0.0f) {
    err = "attention: division by a zero scale";
    return nullptr;
  }
  auto op = std::make_unique<AttnOp>();
  AttnArgs &a = op->args;
  a.batch = (int)batch, a.tq = (int)tq, a.tk = (int)tk;
  a.q_b = L.refs[0].strides[0], a.q_t = L.refs[0].strides[1];
  a.k_b = L.refs[1].strides[0], a.k_t = L.refs[1].strides[1];
  a.v_b = L.refs[2].strides[0], a.v_t = L.refs[2].strides[1];
  a.o_b = L.refs[3].strides[0], a.o_t = L.refs[3].strides[1];
  if (mask_mode == KH_ATTN_MASK_ADD)
    a.m_b = L.refs[4].strides[0], a.m_q = L.refs[4].strides[1], a.m_k = L.refs[4].strides[2];
  a.mask_mode = mask_mode, a.scale_mode = scale_mode, a.scale = L.fparams[0];
  // queries per workgroup (cfg[3]: 0 = library picks, 16 or 32)
  const int qpw = L.cfg[3];
  if (qpw != 0 && qpw != 16 && qpw != 32) {
    err = "attention: queries per workgroup must be 0, 16 or 32";
    return nullptr;
  }
  // products precision (cfg[5]): 0 fp32, 1 bf16 inputs with fp32 accumulation
  // (attn_kernel<..., BF> or, for 16 queries per workgroup, attnbf_kernel),
  // 2 three-pass bf16 (attn_kernel<..., BF, ..., X3>, 32 queries per workgroup)
  const int prec = L.cfg[5];
  if (prec < 0 || prec > 2) {
    err = "attention: products precision must be 0 (fp32), 1 (bf16) or 2 (three-pass bf16)";
    return nullptr;
  }
  op->bf = prec >= 1;
  op->x3 = prec == 2;
  // 16 when 32-query blocks would give under 1.5 workgroups per CU (measured
  // on the GPT-2 block, 12 heads causal: T = 128 6.2 -> 4.7 us, 512 13.5 ->
  // 11.4 us; from T = 1024 on the 32-query kernel is faster); with bf16
  // products under half a workgroup per CU (T = 128 5.0 -> 4.1 us, 256 6.4 ->
  // 5.9; T = 384 7.4 against 7.7-8.1, 512 8.5 against 9.5-10.6)
  const int64_t groups32 = batch * ((tq + kQB - 1) / kQB);
  // q, k, v stored as bf16 (all three, with bf16 products): the 32-query kernel
  op->in16 = (m16 & 7u) != 0;
  if ((m16 & ~0xFu) || (op->in16 && ((m16 & 7u) != 7u || !op->bf || qpw == 16))) {
    unsupported = true;
    err = "attention: bf16 storage of q, k, v needs all three, bf16 products and 32 queries per workgroup";
    return nullptr;
  }
  if (op->x3 && ((m16 & 7u) || qpw == 16)) {
    unsupported = true;
    err = "attention: three-pass products split fp32 q, k, v on 32 queries per workgroup";
    return nullptr;
  }
  // pair words (cfg[7] bits 16 + j): q, k, v together (three-pass products)
  // and / or the output of a blocked kernel
  const uint32_t mp = pair_refs(L);
  op->p3 = (mp & 7u) != 0;
  if ((mp & ~0xFu) || (op->p3 && ((mp & 7u) != 7u || !op->x3)) || (mp & m16)) {
    unsupported = true;
    err = "attention: pair storage of q, k, v needs all three and three-pass products; of the output, fp32 storage";
    return nullptr;
  }
  op->q16 = !op->in16 && !op->x3 && (qpw == 16 || (qpw == 0 && (op->bf ? 2 * groups32 < current_device().cus
                                                              : 2 * groups32 < 3ll * current_device().cus)));
  a.n_qblocks = (int)((tq + (op->q16 ? 16 : kQB) - 1) / (op->q16 ? 16 : kQB));
  op->dh = (int)dh;
  // key-split waves per workgroup: enough workgroups x waves to cover the GPU
  int nw = L.cfg[2];
  if (nw <= 0) {
    const int64_t groups = batch * a.n_qblocks;
    const int64_t kblocks = (tk + kKB - 1) / kKB;
    // key blocks an average query block visits (half of them under a causal mask)
    const int64_t visited = mask_mode == KH_ATTN_MASK_CAUSAL ? (kblocks + 1) / 2 : kblocks;
    // measured on the GPT-2 shapes (12 heads, T = 128 .. 2048): four waves per
    // query block, eight once each wave still gets two or more key blocks and
    // the grid is under three workgroups per CU (T = 1024 .. 1536: 20% faster)
    nw = groups >= 16ll * current_device().cus ? 2 : 4;
    if (nw == 4 && visited >= 16 && groups < 3ll * current_device().cus && dh == 64) nw = 8;
    // 16-query blocks: four waves, eight from 8 visited key blocks (T = 512:
    // 12.3 -> 11.4 us)
    if (op->q16) nw = visited >= 8 && dh == 64 ? 8 : 4;
    // three-pass products: eight waves for grids of one to one and a half
    // workgroups per CU, four otherwise (GPT-2 block: T = 768 15.8 / 16.9
    // us with 8 / 4, T = 1024 20.9 / 22.8; T = 512 11.2 / 12.2 with 4 / 8,
    // T = 1536 34.7 / 37.2, T = 2048 52.8 / 56.5; two waves 28-41% slower)
    else if (op->x3) nw = groups >= current_device().cus && 2 * groups <= 3ll * current_device().cus && dh == 64 ? 8 : 4;
    // bf16 products, 32-query blocks: two waves up to 16 visited key blocks,
    // four beyond (GPT-2 block: T = 512 8.5 against 8.9 / 10.7 us with 4 / 8,
    // T = 1024 17.1 against 18.5 / 17.2, T = 1536 26.9 against 29.2 / 29.7 with
    // 2 / 8, T = 2048 37.8 against 43.4 / 46.1)
    else if (op->bf && groups < 16ll * current_device().cus) nw = visited <= 16 ? 2 : 4;
    if (kblocks < nw) nw = kblocks >= 2 ? 2 : 1;
  }
  if (nw != 1 && nw != 2 && nw != 4 && !(nw == 8 && dh == 64)) {
    err = "attention: waves per workgroup must be 1, 2, 4 (or 8 for head dim 64)";
    return nullptr;
  }
  op->nw = nw;
  // decode shapes (a few queries, a few keys): one wave per query row
  op->rows = !op->bf && !op->in16 && tq <= kRowsMaxQ && tk <= kRowsMaxK && L.cfg[2] <= 0 && batch * tq < (1ll << 31);
  const int64_t n_groups = batch * (int64_t)a.n_qblocks;
  if (n_groups >= (1ll << 31)) {
    unsupported = true;
    err = "attention: grid too large";
    return nullptr;
  }
  op->grid = dim3((unsigned)std::max<int64_t>(1, n_groups));
  // a bf16 output (the head-merged result read only by a bf16 matmul): not
  // on the few-query kernel
  if ((m16 >> 3 & 1) && op->rows) {
    unsupported = true;
    err = "attention: bf16 storage only for the output of the blocked kernel";
    return nullptr;
  }
  a.o16 = m16 >> 3 & 1;
  if ((mp >> 3 & 1) && op->rows) {
    unsupported = true;
    err = "attention: pair storage only for the output of the blocked kernels";
    return nullptr;
  }
  a.o_pair = mp >> 3 & 1;
  return op;
}

hipError_t probe_attn_timeline(const float *q, const float *k, const float *v, float *o, int batch, int tq, int tk,
                               const int64_t *st, int nw, float scale, uint64_t *rec, hipStream_t stream,
                               std::string &err) {
  if (!q || !k || !v || !o || !st || !rec || batch <= 0 || tq <= 0 || tk <= 0 || (nw != 4 && nw != 8)) {
    err = "attention timeline: null operand, empty shape or waves not 4 or 8";
    return hipErrorInvalidValue;
  }
  if (tq >= (1 << 24) || tk >= (1 << 24) || (int64_t)batch * ((tq + kQB - 1) / kQB) >= (1ll << 31)) {
    err = "attention timeline: sizes out of range";
    return hipErrorInvalidValue;
  }
  const float *base[4] = {q, k, v, o};
  for (int j = 0; j < 4; ++j) {
    const int64_t rows = j == 0 || j == 3 ? tq : tk;
    const int64_t span = (int64_t)(batch - 1) * st[2 * j] + (rows - 1) * st[2 * j + 1] + 64;
    if ((reinterpret_cast<uintptr_t>(base[j]) & 15) || st[2 * j] < 0 || st[2 * j + 1] < 0 || st[2 * j] % 4 ||
        st[2 * j + 1] % 4 || span >= (1ll << 30)) {
      err = "attention timeline: operands need 16-byte aligned rows and spans under 2^30 elements";
      return hipErrorInvalidValue;
    }
  }
  AttnArgs a{};
  a.q = q, a.k = k, a.v = v, a.o = o, a.mask = nullptr, a.rec = rec;
  a.q_b = st[0], a.q_t = st[1], a.k_b = st[2], a.k_t = st[3], a.v_b = st[4], a.v_t = st[5], a.o_b = st[6], a.o_t = st[7];
  a.batch = batch, a.tq = tq, a.tk = tk, a.n_qblocks = (tq + kQB - 1) / kQB;
  a.mask_mode = KH_ATTN_MASK_CAUSAL, a.scale_mode = KH_ATTN_SCALE_MUL, a.scale = scale;
  const dim3 grid((unsigned)(batch * a.n_qblocks));
  if (nw == 4) hipLaunchKernelGGL((attn_kernel<64, 4, false, false, true>), grid, dim3(256), 0, stream, a);
  else hipLaunchKernelGGL((attn_kernel<64, 8, false, false, true>), grid, dim3(512), 0, stream, a);
  return hipGetLastError();
}

}  // namespace kh
