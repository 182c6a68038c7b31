// kh_gemv.hip - the M = 1 matmul path (decode): out[b, n] = epilogue(sum_k
// x[b, k] * W[b, k, n]).
//
// A GEMV moves every weight byte once and does 2 flops per 4 bytes, so it is
// HBM-bound; at decode sizes (a few MB per launch) a launch lasts about one
// memory latency plus the streaming time of the busiest CU, so the kernel is
// shaped for memory-level parallelism and spread:
//   * a workgroup of 256 or 1024 threads covers CQ column quads (4 * CQ
//     columns, CQ = 8, 4 or 2, so a row segment is 128, 64 or 32 contiguous
//     bytes) and threads / CQ k-lanes; each thread issues kRows 128-bit row
//     loads (and the matching x values) before its first FMA;
//   * CQ is the widest that still gives about half the CUs a workgroup, so
//     the weight stream is spread over the chip rather than queued behind a
//     few CUs; narrower segments than 64 bytes were measured slower (a wave's
//     load then touches 64 cache lines). When even CQ = 4 leaves few column
//     blocks (N small, K large) the workgroup grows to 1024 threads so each
//     CU still has its whole share of rows in flight in one or two passes;
//   * the k-lanes are reduced in a fixed tree (shuffles inside a wave, then the
//     four waves through LDS) and the same workgroup runs the epilogue;
//   * a LayerNorm whose only consumer is the GEMV runs as its prologue (decode:
//     the normalised row never goes through memory, one launch instead of
//     two): every workgroup recomputes the row's mean and variance in one
//     pass (sums shifted by the row's first value, one workgroup reduction)
//     and normalises x as it loads it;
//   * only when even CQ = 1 leaves too few workgroups for the rows (tiny N, huge
//     K) is K split across workgroups; the splits' partials are then summed in
//     split order by the split-K reduce kernel (shared with the GEMM family),
//     which runs the epilogue. Cross-workgroup combining inside one launch was
//     measured slower at these sizes (agent-scope fences across 8 XCDs).
#include <algorithm>
#include <cstring>
#include <type_traits>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

constexpr int kRows = 8;           // row loads in flight per thread
constexpr int kTargetBlocks = 128;  // workgroups wanted before narrowing stops

__device__ __forceinline__ float4 add4(float4 a, float4 b) {
  return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}

__device__ __forceinline__ float4 shfl_xor4(float4 v, int m) {
  return make_float4(__shfl_xor(v.x, m, 64), __shfl_xor(v.y, m, 64), __shfl_xor(v.z, m, 64),
                     __shfl_xor(v.w, m, 64));
}

// Sum of v over the workgroup, in a fixed order (wave tree, then the waves in
// order); every thread gets the total. `red` holds NW entries.
template <int NW>
__device__ __forceinline__ float2 block_sum2(float2 v, float2 *red) {
#pragma unroll
  for (int m = 32; m >= 1; m /= 2) v.x += __shfl_xor(v.x, m, 64), v.y += __shfl_xor(v.y, m, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float2 s = red[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) s.x += red[w].x, s.y += red[w].y;
  return s;
}

constexpr int kProCache = 4;  // x values per thread kept in registers by the prologue

template <int CQ, int THREADS, bool PRO>
__global__ __launch_bounds__(THREADS) void gemv_kernel(const GemmArgs a) {
  constexpr int KL = THREADS / CQ;  // k-lanes: rows one load instruction covers
  constexpr int NW = THREADS / 64;
  __shared__ float4 wave_part[NW][CQ];
  __shared__ float2 red[NW];
  const int tid = threadIdx.x;
  const int cq = tid % CQ, kl = tid / CQ;
  const int nb = blockIdx.x, b = blockIdx.y, split = blockIdx.z;
  const int n = nb * 4 * CQ + cq * 4;
  const int k_begin = split * a.k_per_split;
  const int k_end = min(a.K, k_begin + a.k_per_split);
  const float *x = a.A + (int64_t)b * a.sa_b;
  const float *W = a.B + (int64_t)b * a.sb_b;
  // LayerNorm prologue: statistics of the whole row (every split needs them);
  // an absent gamma / beta reads x[0] (stride 0) and is deselected
  float mean = 0.0f, rstd = 1.0f;
  const float *gam = x, *bet = x;
  int g_st = 0, b_st = 0;
  if constexpr (PRO) {
    // one pass over the row, sums shifted by its first value c (so the
    // variance does not cancel for rows far from zero):
    //   mean = c + S1 / C,  var = (S2 - S1^2 / C) * c2,  S_p = sum (x - c)^p
    const float c = x[0];
    float xs[kProCache];
#pragma unroll
    for (int i = 0; i < kProCache; ++i) {
      const int k = tid + i * THREADS;
      xs[i] = k < a.K ? x[(int64_t)k * a.sa_k] - c : 0.0f;
    }
    float2 s = make_float2(0.0f, 0.0f);
#pragma unroll
    for (int i = 0; i < kProCache; ++i) s.x += xs[i], s.y = fmaf(xs[i], xs[i], s.y);
    for (int k = tid + kProCache * THREADS; k < a.K; k += THREADS) {
      const float d = x[(int64_t)k * a.sa_k] - c;
      s.x += d, s.y = fmaf(d, d, s.y);
    }
    s = block_sum2<NW>(s, red);
    const float m1 = s.x * a.pro_c1;
    mean = c + m1;
    rstd = rsqrtf(fmaxf(fmaf(-s.x, m1, s.y), 0.0f) * a.pro_c2 + a.pro_eps);
    if (a.pro_g >= 0) gam = a.eptr[a.pro_g] + b * a.estride[a.pro_g][0], g_st = 1;
    if (a.pro_b >= 0) bet = a.eptr[a.pro_b] + b * a.estride[a.pro_b][0], b_st = 1;
  }
  auto walk = [&](auto vec_tag) {
    constexpr bool vec = decltype(vec_tag)::value;
    auto row = [&](int k) -> float4 {
      const float *p = W + (int64_t)k * a.sb_k;
      if constexpr (vec) {
        return *reinterpret_cast<const float4 *>(p + n);
      } else {
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (n + 0 < a.N) v.x = p[(int64_t)(n + 0) * a.sb_n];
        if (n + 1 < a.N) v.y = p[(int64_t)(n + 1) * a.sb_n];
        if (n + 2 < a.N) v.z = p[(int64_t)(n + 2) * a.sb_n];
        if (n + 3 < a.N) v.w = p[(int64_t)(n + 3) * a.sb_n];
        return v;
      }
    };
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int k0 = k_begin + kl; k0 < k_end; k0 += KL * kRows) {
      float4 w[kRows];
      float xv[kRows], gv[kRows], bv[kRows];
      // Rows past the end are clamped to the last row (an in-bounds load,
      // issued with the others) and their products dropped by a select. All
      // loads of the batch are issued before the first use of any of them.
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const int k = min(k0 + j * KL, k_end - 1);
        w[j] = row(k);
        xv[j] = x[(int64_t)k * a.sa_k];
        if constexpr (PRO) gv[j] = gam[k * g_st], bv[j] = bet[k * b_st];
      }
#pragma unroll
      for (int j = 0; j < kRows; ++j) {
        const bool in = k0 + j * KL < k_end;
        float xn = xv[j];
        if constexpr (PRO) {
          xn = (xn - mean) * rstd;
          xn = g_st ? xn * gv[j] : xn;
          xn = b_st ? xn + bv[j] : xn;
        }
        const float xs = in ? xn : 0.0f;
        const float4 ws = in ? w[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        acc.x = fmaf(xs, ws.x, acc.x), acc.y = fmaf(xs, ws.y, acc.y);
        acc.z = fmaf(xs, ws.z, acc.z), acc.w = fmaf(xs, ws.w, acc.w);
      }
    }
    return acc;
  };
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
  if (n < a.N) acc = (a.b_vec && n + 3 < a.N) ? walk(std::true_type{}) : walk(std::false_type{});
  // fixed-order tree over the k-lanes of a wave (lane = CQ * k-lane + quad),
  // then the waves in order
#pragma unroll
  for (int m = CQ; m < 64; m *= 2) acc = add4(acc, shfl_xor4(acc, m));
  if ((tid & 63) < CQ) wave_part[tid >> 6][cq] = acc;
  __syncthreads();
  if (tid >= CQ || n >= a.N) return;
  float4 s = wave_part[0][cq];
#pragma unroll
  for (int w = 1; w < NW; ++w) s = add4(s, wave_part[w][cq]);
  const int valid = min(4, a.N - n);
  if (a.splitk > 1) {
    // dense partial row [split][batch][N]; splitk_reduce_kernel finishes it
    float *dst = a.ws_partial + ((int64_t)split * a.batch + b) * a.N + n;
    if (valid > 0) dst[0] = s.x;
    if (valid > 1) dst[1] = s.y;
    if (valid > 2) dst[2] = s.z;
    if (valid > 3) dst[3] = s.w;
    return;
  }
  Vec<4> out;
  out.v[0] = s.x, out.v[1] = s.y, out.v[2] = s.z, out.v[3] = s.w;
  run_epilogue(a, b, 0, n, valid, out);
}

// K-contiguous GEMV: W is [batch][N][K] (each output column's weights are one
// contiguous row, the nn.Linear layout, kept as a copy of the frozen constant
// for M = 1 plans). A workgroup owns 4 adjacent output columns and its NW
// waves split K: lane l of wave w reads float4 q = w*64 + l + i*64*NW (i < R)
// of x and of the 4 weight rows, so one wave load is 1 KiB of one row. Every
// load of a pass - 4R weight vectors and R of x (and gamma / beta) - is
// issued before the first FMA, and with the LayerNorm prologue before the row
// statistics are computed, so a launch costs about one memory latency plus
// the streaming time of its bytes. Partial dot products are summed in a
// fixed order: lanes by the DPP tree, then the waves in index order.
constexpr int kNkCols = 4;
constexpr int kNkMaxWaves = 8;

// Sum over the workgroup's nw waves in wave order; every thread gets it.
__device__ __forceinline__ float nk_block_sum(float v, float *red, int wave, int nw) {
  v = wave_sum(v);
  __syncthreads();  // `red` may still be read from a previous reduction
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  float s = red[0];
  for (int w = 1; w < nw; ++w) s += red[w];
  return s;
}

// 128-bit load marked non-temporal: each weight byte is read once per call,
// so the weights should not displace the activations in the caches.
__device__ __forceinline__ uint4 load_stream(const uint4 *p) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// One K value of a weight chunk (4 fp32 or 8 bf16 values in a uint4).
template <bool BF16>
__device__ __forceinline__ float nk_weight(const uint4 &w, int e) {
  const uint32_t word = e / (BF16 ? 2 : 1) == 0 ? w.x : e / (BF16 ? 2 : 1) == 1 ? w.y
                        : e / (BF16 ? 2 : 1) == 2 ? w.z : w.w;
  if constexpr (BF16) return __uint_as_float(e & 1 ? word & 0xffff0000u : word << 16);
  else return __uint_as_float(word);
}

// Attention prologue: x values k0 .. k0 + KV - 1 (k0 = u * KV) of the
// head-merged attention output of one query, x[h * dh + d] = softmax_j(s_j) .
// v_jh[d] with s_j = q_h . k_jh scaled (+ mask). The dh / KV lanes that share
// a head hold its dims k0 % dh .. + KV - 1 and sum their partial dot products
// by xor shuffles, so every lane of the group has s_j; the online softmax is
// attn_kernel's (base 2, exponentials against 0 while no score is finite).
template <int KV, int R>
__device__ __forceinline__ void nk_attention(const GemmArgs &a, const int (&u)[R], float (&x)[R][KV]) {
  constexpr float kLog2e = 1.4426950408889634f;
  constexpr int kChunk = 2;  // keys per round of loads (all R units' rows issued together)
  const int group = a.att_dh / KV;  // lanes per head
  const float c_scale = a.att_scale_mode == KH_ATTN_SCALE_MUL   ? a.att_scale * kLog2e
                        : a.att_scale_mode == KH_ATTN_SCALE_DIV ? kLog2e / a.att_scale
                                                                : kLog2e;
  const int qi = a.att_q, ki = a.att_q + 1, vi = a.att_q + 2;
  int h[R], d0[R];
#pragma unroll
  for (int i = 0; i < R; ++i) h[i] = u[i] * KV / a.att_dh, d0[i] = u[i] * KV - h[i] * a.att_dh;
  auto row = [&](int j, int i, int t) {  // operand j's (head h[i], token t) row at dim d0[i]
    return a.eptr[j] + (int64_t)h[i] * a.estride[j][0] + (int64_t)t * a.estride[j][1] + d0[i];
  };
  auto load = [&](const float *p, float (&dst)[KV]) {
    if (a.a_vec) {
#pragma unroll
      for (int e = 0; e < KV; e += 4) {
        const float4 t = *reinterpret_cast<const float4 *>(p + e);
        dst[e] = t.x, dst[e + 1] = t.y, dst[e + 2] = t.z, dst[e + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < KV; ++e) dst[e] = p[e];
    }
  };
  const int lim = a.att_mask_mode == KH_ATTN_MASK_CAUSAL ? 1 : a.att_tk;  // the query is token 0
  float q[R][KV], m[R], l[R];
#pragma unroll
  for (int i = 0; i < R; ++i) {
    load(row(qi, i, 0), q[i]);
    m[i] = -INFINITY, l[i] = 0.0f;
#pragma unroll
    for (int e = 0; e < KV; ++e) x[i][e] = 0.0f;  // the running sum of p v
  }
  for (int j0 = 0; j0 < lim; j0 += kChunk) {
    float kv[R][kChunk][KV], vv[R][kChunk][KV], mk[R][kChunk];
#pragma unroll
    for (int i = 0; i < R; ++i)
#pragma unroll
      for (int c = 0; c < kChunk; ++c) {
        const int j = min(j0 + c, lim - 1);  // clamped: an in-bounds load, the key is dropped below
        load(row(ki, i, j), kv[i][c]);
        load(row(vi, i, j), vv[i][c]);
        mk[i][c] = a.att_mask >= 0 ? a.eptr[a.att_mask][(int64_t)h[i] * a.estride[a.att_mask][0] +
                                                         (int64_t)j * a.estride[a.att_mask][2]]
                                   : 0.0f;
      }
#pragma unroll
    for (int c = 0; c < kChunk; ++c) {
      if (j0 + c >= lim) break;
#pragma unroll
      for (int i = 0; i < R; ++i) {
        float t = 0.0f;
#pragma unroll
        for (int e = 0; e < KV; ++e) t = fmaf(q[i][e] * c_scale, kv[i][c][e], t);
        for (int s = 1; s < group; s <<= 1) t += __shfl_xor(t, s, 64);
        if (a.att_mask >= 0) t = fmaf(mk[i][c], kLog2e, t);
        const float m_new = fmaxf(m[i], t);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m[i] - m_use);
        const float p = __builtin_amdgcn_exp2f(t - m_use);
        l[i] = fmaf(l[i], alpha, p);
#pragma unroll
        for (int e = 0; e < KV; ++e) x[i][e] = fmaf(x[i][e], alpha, p * vv[i][c][e]);
        m[i] = m_new;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < R; ++i)
#pragma unroll
    for (int e = 0; e < KV; ++e) x[i][e] /= l[i];
}

// BF16: the weights are the bf16 [batch][N][K] copy, a unit is 8 K values
// (one 16-byte chunk), x is rounded to bf16 (round to nearest even) at the
// product - the arithmetic of the bf16 GEMM (exact products, fp32 sums).
// PRO: 0 none, 1 LayerNorm prologue, 2 attention prologue.
template <int R, int PRO, bool BF16>
__global__ __launch_bounds__(64 * kNkMaxWaves) void gemv_nk_kernel(const GemmArgs a) {
  constexpr int KV = BF16 ? 8 : 4;  // K values per lane and unit
  __shared__ float red[kNkMaxWaves];
  __shared__ float part[kNkMaxWaves][kNkCols];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  const int n0 = blockIdx.x * kNkCols, b = blockIdx.y;
  const int U = a.K / KV, step = 64 * nw;  // the host checks K % KV == 0
  const float *xrow = a.A + (int64_t)b * a.sa_b;
  const float *grow = PRO == 1 && a.pro_g >= 0 ? a.eptr[a.pro_g] + (int64_t)b * a.estride[a.pro_g][0] : nullptr;
  const float *brow = PRO == 1 && a.pro_b >= 0 ? a.eptr[a.pro_b] + (int64_t)b * a.estride[a.pro_b][0] : nullptr;
  const uint4 *w16[kNkCols];
#pragma unroll
  for (int c = 0; c < kNkCols; ++c) {
    const int64_t off = (int64_t)b * a.sb_b + (int64_t)min(n0 + c, a.N - 1) * a.sb_n;
    w16[c] = BF16 ? reinterpret_cast<const uint4 *>(reinterpret_cast<const __bf16 *>(a.B) + off)
                  : reinterpret_cast<const uint4 *>(a.B + off);
  }
  // KV consecutive floats of a row at unit u: 128-bit loads when the rows
  // are 16-byte aligned (a_vec, set at launch), else scalar loads
  auto load_row = [&](const float *row, int u, float (&dst)[KV]) {
    if (a.a_vec) {
#pragma unroll
      for (int h = 0; h < KV / 4; ++h) {
        const float4 t = reinterpret_cast<const float4 *>(row)[u * (KV / 4) + h];
        dst[4 * h] = t.x, dst[4 * h + 1] = t.y, dst[4 * h + 2] = t.z, dst[4 * h + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < KV; ++e) dst[e] = row[u * KV + e];
    }
  };
  // direct epilogue (bias / residual / activation recognised on the host):
  // the thread that finishes the 4 columns loads their operands up front, so
  // they arrive with the weights rather than after the reduction
  float pre_b[kNkCols] = {0.0f, 0.0f, 0.0f, 0.0f}, pre_r[kNkCols] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (a.direct && threadIdx.x == 0) {
#pragma unroll
    for (int c = 0; c < kNkCols; ++c) {
      const int64_t n = min(n0 + c, a.N - 1);
      if (a.d_bias >= 0) pre_b[c] = a.eptr[a.d_bias][b * a.estride[a.d_bias][0] + n * a.estride[a.d_bias][2]];
      if (a.d_res >= 0) pre_r[c] = a.eptr[a.d_res][b * a.estride[a.d_res][0] + n * a.estride[a.d_res][2]];
    }
  }
  float p[kNkCols] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int base = wave * 64 + lane; base - lane < U; base += R * step) {
    uint4 wv[kNkCols][R];
    float xv[R][KV], gv[R][KV], bv[R][KV];
    bool in[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const int u = base + i * step;
      in[i] = u < U;
      const int uc = in[i] ? u : U - 1;  // clamped: an in-bounds load, product dropped
#pragma unroll
      for (int c = 0; c < kNkCols; ++c) wv[c][i] = load_stream(w16[c] + uc);
      if constexpr (PRO != 2) load_row(xrow, uc, xv[i]);
      if constexpr (PRO == 1) {
        if (grow) load_row(grow, uc, gv[i]);
        if (brow) load_row(brow, uc, bv[i]);
      }
    }
    if constexpr (PRO == 2) {
      int us[R];
#pragma unroll
      for (int i = 0; i < R; ++i) us[i] = min(base + i * step, U - 1);
      nk_attention<KV, R>(a, us, xv);
    }
    if constexpr (PRO == 1) {
      // the whole row is in this pass (the host guarantees U <= R * 64 * NW):
      // mean, then the variance of the centred values
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < R; ++i)
        if (in[i])
#pragma unroll
          for (int e = 0; e < KV; ++e) s += xv[i][e];
      const float mean = nk_block_sum(s, red, wave, nw) * a.pro_c1;
      float s2 = 0.0f;
#pragma unroll
      for (int i = 0; i < R; ++i)
#pragma unroll
        for (int e = 0; e < KV; ++e) {
          xv[i][e] -= mean;
          if (in[i]) s2 = fmaf(xv[i][e], xv[i][e], s2);
        }
      const float rstd = rsqrtf(nk_block_sum(s2, red, wave, nw) * a.pro_c2 + a.pro_eps);
#pragma unroll
      for (int i = 0; i < R; ++i)
#pragma unroll
        for (int e = 0; e < KV; ++e) {
          float y = xv[i][e] * rstd;
          if (grow) y *= gv[i][e];
          if (brow) y += bv[i][e];
          xv[i][e] = y;
        }
    }
#pragma unroll
    for (int i = 0; i < R; ++i) {
      if (!in[i]) continue;
#pragma unroll
      for (int c = 0; c < kNkCols; ++c) {
        float t = p[c];
#pragma unroll
        for (int e = 0; e < KV; ++e) {
          const float xe = BF16 ? (float)(__bf16)xv[i][e] : xv[i][e];
          t = fmaf(xe, nk_weight<BF16>(wv[c][i], e), t);
        }
        p[c] = t;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < kNkCols; ++c) p[c] = wave_sum(p[c]);
  if (lane == 0)
#pragma unroll
    for (int c = 0; c < kNkCols; ++c) part[wave][c] = p[c];
  __syncthreads();
  if (threadIdx.x != 0 || n0 >= a.N) return;
  Vec<4> out;
#pragma unroll
  for (int c = 0; c < kNkCols; ++c) {
    float v = part[0][c];
    for (int w = 1; w < nw; ++w) v += part[w][c];
    out.v[c] = v;
  }
  const int valid = min(kNkCols, a.N - n0);
  if (a.direct) {
    // the tape's operations in its order: (acc + bias), then res + that, then act
    float *o = a.eptr[a.d_out] + b * a.estride[a.d_out][0];
#pragma unroll
    for (int c = 0; c < kNkCols; ++c) {
      if (c >= valid) break;
      float v = out.v[c];
      if (a.d_bias >= 0) v += pre_b[c];
      if (a.d_res >= 0) v = pre_r[c] + v;
      if (a.d_act == KH_OP_GELU_TANH) v = op_gelu_tanh(v);
      else if (a.d_act == KH_OP_GELU_ERF) v = op_gelu_erf(v);
      else if (a.d_act == KH_OP_RELU) v = v != v ? v : fmaxf(v, 0.0f);
      o[(int64_t)(n0 + c) * a.estride[a.d_out][2]] = v;
    }
    return;
  }
  run_epilogue(a, b, 0, n0, valid, out);
}

// (column quads, threads) per workgroup by variant id (1..5); 0 = chosen
// from the shape.
constexpr int kVariants[][2] = {{0, 0}, {8, 256}, {4, 256}, {2, 256}, {8, 1024}, {4, 1024}};
constexpr int kNumVariants = sizeof(kVariants) / sizeof(kVariants[0]);

class GemvOp final : public Op {
 public:
  GemmArgs args{};
  dim3 grid;
  size_t n_partials = 0;
  int quads = 8, threads = 256;
  bool b_vec_layout = false;
  uint32_t e_vec_candidates = 0;
  // K-contiguous kernel: chosen at plan creation (nk_r > 0), taken at launch
  // when the operands it reads as float4 are 16-byte aligned
  int nk_r = 0, nk_waves = 1;
  bool bf16 = false;  // weights are the bf16 [batch][N][K] copy (K-contiguous kernel only)
  bool att_vec = false;  // attention prologue rows keep 16-byte alignment (strides and offsets)
  dim3 nk_grid;

  hipError_t launch(float *const *ptrs, float *partials, hipStream_t stream) override {
    GemmArgs a = args;
    a.A = ptrs[0];
    a.B = ptrs[1];
    a.b_vec = b_vec_layout && (reinterpret_cast<uintptr_t>(ptrs[1]) & 15) == 0;
    a.e_vec_mask = 0;
    for (int j = 0; j < a.n_refs; ++j) {
      a.eptr[j] = ptrs[2 + j];
      if ((e_vec_candidates >> j & 1) && (reinterpret_cast<uintptr_t>(ptrs[2 + j]) & 15) == 0)
        a.e_vec_mask |= 1u << j;
    }
    a.ws_partial = partials;
    if (a.N == 0 || a.batch == 0) return hipSuccess;
    // bf16 weights and the attention prologue exist only on the K-contiguous kernel
    if (nk_r > 0 && (bf16 || a.pro == 2 || aligned16(ptrs[1]))) {
      a.splitk = 1;
      if (a.pro == 2)
        a.a_vec = att_vec && aligned16(a.eptr[a.att_q]) && aligned16(a.eptr[a.att_q + 1]) &&
                  aligned16(a.eptr[a.att_q + 2]);
      else
        a.a_vec = aligned16(ptrs[0]) && (a.pro_g < 0 || aligned16(a.eptr[a.pro_g])) &&
                  (a.pro_b < 0 || aligned16(a.eptr[a.pro_b]));
      if ((bf16 || a.pro == 2) && !aligned16(ptrs[1])) return hipErrorInvalidValue;
      launch_nk(a, stream);
      return hipGetLastError();
    }
    if (a.splitk > 1 && !partials) return hipErrorInvalidValue;
    if (a.pro == KH_GEMV_PRO_LAYERNORM) launch_variant(a, grid, stream, std::true_type{});
    else launch_variant(a, grid, stream, std::false_type{});
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splitk == 1) return e;
    return launch_splitk_reduce(a, current_device().cus, stream);
  }
  size_t partial_floats() const override { return n_partials; }
  bool gemv_facts(GemvFacts &f) const override {
    f.args = &args, f.nk_r = nk_r, f.bf16 = bf16;
    return true;
  }

  static bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

  void launch_nk(const GemmArgs &a, hipStream_t stream) const {
    const dim3 block(64 * nk_waves);
#define KH_NK_PRO(R, P)                                                                             \
  if (a.pro == P) {                                                                                 \
    if (bf16) hipLaunchKernelGGL((gemv_nk_kernel<R, P, true>), nk_grid, block, 0, stream, a);        \
    else hipLaunchKernelGGL((gemv_nk_kernel<R, P, false>), nk_grid, block, 0, stream, a);            \
  }
#define KH_NK_CASE(R) \
  case R:             \
    KH_NK_PRO(R, 0)   \
    KH_NK_PRO(R, 1)   \
    KH_NK_PRO(R, 2)   \
    break;
    // R = 4 has no attention-prologue variant (its registers would spill)
    switch (nk_r) {
      KH_NK_CASE(1)
      KH_NK_CASE(2)
      KH_NK_CASE(3)
      case 4:
        KH_NK_PRO(4, 0)
        KH_NK_PRO(4, 1)
        break;
    }
#undef KH_NK_CASE
#undef KH_NK_PRO
  }

  template <class P>
  void launch_variant(const GemmArgs &a, dim3 g, hipStream_t stream, P) const {
    constexpr bool pro = P::value;
    if (threads == 1024) {
      if (quads == 8) hipLaunchKernelGGL((gemv_kernel<8, 1024, pro>), g, dim3(1024), 0, stream, a);
      else hipLaunchKernelGGL((gemv_kernel<4, 1024, pro>), g, dim3(1024), 0, stream, a);
    } else {
      if (quads == 8) hipLaunchKernelGGL((gemv_kernel<8, 256, pro>), g, dim3(256), 0, stream, a);
      else if (quads == 4) hipLaunchKernelGGL((gemv_kernel<4, 256, pro>), g, dim3(256), 0, stream, a);
      else hipLaunchKernelGGL((gemv_kernel<2, 256, pro>), g, dim3(256), 0, stream, a);
    }
  }
};

}  // namespace

std::unique_ptr<Op> make_gemv(const kh_launch &L, std::string &err, bool &unsupported) {
  unsupported = false;
  if (L.n_refs < 3 || L.n_refs > KH_MAX_REFS) {
    err = "gemv: bad operand count";
    return nullptr;
  }
  const int64_t batch = L.gemm[0], M = L.gemm[1], N = L.gemm[2], K = L.gemm[3];
  if (L.variant != 0 && L.variant != KH_GEMV_CHAIN) {
    err = "gemv: unknown launch flags " + std::to_string(L.variant);
    return nullptr;
  }
  if (M != 1) {
    err = "gemv: M must be 1";
    return nullptr;
  }
  if (batch < 0 || N < 0 || K < 0 || batch >= (1 << 16) || N >= (1ll << 30) || K >= (1ll << 30)) {
    unsupported = true;
    err = "gemv: sizes out of range";
    return nullptr;
  }
  auto op = std::make_unique<GemvOp>();
  GemmArgs &a = op->args;
  a.batch = (int)batch, a.M = 1, a.N = (int)N, a.K = (int)K;
  a.sa_b = L.refs[0].strides[0], a.sa_m = L.refs[0].strides[1], a.sa_k = L.refs[0].strides[2];
  a.sb_b = L.refs[1].strides[0], a.sb_k = L.refs[1].strides[1], a.sb_n = L.refs[1].strides[2];
  op->b_vec_layout = a.sb_n == 1 && L.refs[1].offset % 4 == 0 && a.sb_k % 4 == 0 && a.sb_b % 4 == 0;
  if (!fill_epilogue(L, a, op->e_vec_candidates, err)) return nullptr;
  a.direct = 0, a.d_bias = a.d_res = a.d_out = a.d_act = -1;
  match_direct_epilogue(L, a);
  if (L.cfg[3] != KH_PREC_FP32 && L.cfg[3] != KH_PREC_BF16) {
    unsupported = true;
    err = "gemv: precision must be fp32 or bf16";
    return nullptr;
  }
  op->bf16 = L.cfg[3] == KH_PREC_BF16;
  // LayerNorm prologue: cfg[4] = 1, cfg[5] / cfg[6] = ref index of gamma /
  // beta (-1: none), fparams = {1/C, 1/C, eps}; gamma and beta are [K] rows
  a.pro = L.cfg[4], a.pro_g = -1, a.pro_b = -1, a.att_q = -1, a.att_mask = -1;
  if (a.pro != KH_GEMV_PRO_NONE && a.pro != KH_GEMV_PRO_LAYERNORM && a.pro != KH_GEMV_PRO_ATTN) {
    err = "gemv: unknown prologue " + std::to_string(a.pro);
    return nullptr;
  }
  if (a.pro == KH_GEMV_PRO_ATTN) {
    // attention prologue: Q, K, V (+ mask) refs from cfg[5]; one query
    const int r = L.cfg[5], mask_mode = L.cfg[6] & 3, scale_mode = L.cfg[6] >> 2, dh = L.cfg[0], tk = L.cfg[7];
    const int n_att = mask_mode == KH_ATTN_MASK_ADD ? 4 : 3;
    if (r < 2 || r + n_att > L.n_refs) {
      err = "gemv: attention prologue operand index out of range";
      return nullptr;
    }
    if (mask_mode > KH_ATTN_MASK_ADD || scale_mode > KH_ATTN_SCALE_DIV || (dh != 32 && dh != 64) || K % dh ||
        tk < 1 || tk > 64 || batch != 1 || (scale_mode == KH_ATTN_SCALE_DIV && L.fparams[0] == 0.0f)) {
      err = "gemv: attention prologue needs one query, 1..64 keys, head dim 32 or 64 dividing K, batch 1";
      return nullptr;
    }
    op->att_vec = true;
    for (int j = 0; j < 3; ++j) {
      const kh_ref &q = L.refs[r + j];
      if (q.strides[2] != 1 || q.strides[0] < 0 || q.strides[1] < 0) {
        err = "gemv: attention prologue Q / K / V need unit head-dim stride";
        return nullptr;
      }
      op->att_vec = op->att_vec && q.offset % 4 == 0 && q.strides[0] % 4 == 0 && q.strides[1] % 4 == 0;
    }
    a.att_q = r - 2, a.att_mask = mask_mode == KH_ATTN_MASK_ADD ? r + 1 : -1;
    a.att_tk = tk, a.att_dh = dh, a.att_mask_mode = mask_mode, a.att_scale_mode = scale_mode;
    a.att_scale = L.fparams[0];
  }
  if (a.pro == KH_GEMV_PRO_LAYERNORM) {
    for (int w = 0; w < 2; ++w) {
      const int r = L.cfg[5 + w];
      if (r == -1) continue;
      if (r < 2 || r >= L.n_refs) {
        err = "gemv: prologue operand index out of range";
        return nullptr;
      }
      const kh_ref &g = L.refs[r];
      if (g.strides[1] != 0 || g.strides[2] != 1) {
        err = "gemv: LayerNorm gamma / beta must be unit-stride rows over K";
        return nullptr;
      }
      (w == 0 ? a.pro_g : a.pro_b) = r - 2;
    }
    a.pro_c1 = L.fparams[0], a.pro_c2 = L.fparams[1], a.pro_eps = L.fparams[2];
  }
  // column quads per workgroup: the widest giving kTargetBlocks workgroups;
  // if none does, 64-byte segments with 1024-thread workgroups
  const int64_t b1 = std::max<int64_t>(1, batch);
  const int variant = L.cfg[1];
  if (variant < 0 || variant >= kNumVariants) {
    err = "gemv: unknown variant " + std::to_string(variant);
    return nullptr;
  }
  int quads = kVariants[variant][0], threads = kVariants[variant][1];
  if (quads == 0) {
    quads = 4, threads = 1024;
    for (int q : {8, 4}) {
      if ((N + 4 * q - 1) / (4 * q) * b1 >= kTargetBlocks) {
        quads = q, threads = 256;
        break;
      }
    }
  }
  const int64_t n_blocks = std::max<int64_t>(1, (N + 4 * quads - 1) / (4 * quads));
  const int64_t k_lanes = threads / quads;
  // split K (two kernels) only when the blocks are few and each thread would
  // walk more than four passes of kRows rows
  int64_t splitk = L.cfg[2];
  if (splitk <= 0) {
    splitk = 1;
    const int64_t rows_per_thread = (K + k_lanes - 1) / k_lanes;
    if (n_blocks * b1 < kTargetBlocks / 2 && rows_per_thread > 4 * kRows)
      splitk = std::min<int64_t>((kTargetBlocks + n_blocks * b1 - 1) / (n_blocks * b1),
                                 (rows_per_thread + 4 * kRows - 1) / (4 * kRows));
  }
  splitk = std::max<int64_t>(1, std::min<int64_t>(splitk, std::max<int64_t>(1, K / k_lanes)));
  const int64_t kper = std::max<int64_t>(k_lanes, ((K + splitk - 1) / splitk + k_lanes - 1) / k_lanes * k_lanes);
  splitk = std::max<int64_t>(1, (K + kper - 1) / kper);
  if (n_blocks * b1 >= (1ll << 31) || b1 >= 65536) {
    unsupported = true;
    err = "gemv: too many column blocks";
    return nullptr;
  }
  // K-contiguous layout ([batch][N][K] weights, unit-stride x, K a multiple
  // of 4, gamma / beta unit-stride): float4 loads per lane; R float4 per lane
  // and wave, NW = ceil(K/4 / 64R) waves, the (R, NW) with the fewest idle
  // lanes. A LayerNorm prologue needs the whole row in one pass.
  const int kv = op->bf16 ? 8 : 4;  // K values per 16-byte weight chunk
  const bool nk_layout = a.sb_k == 1 && a.sb_n >= K && a.sb_n % kv == 0 && a.sb_b % kv == 0 &&
                         L.refs[1].offset % kv == 0 && a.sa_k == 1 && a.sa_b % 4 == 0 &&
                         L.refs[0].offset % 4 == 0 && K % kv == 0 && K > 0 &&
                         (N + kNkCols - 1) / kNkCols < (1ll << 31);
  bool nk_pro_ok = true;
  if (a.pro == KH_GEMV_PRO_LAYERNORM)
    for (int r : {L.cfg[5], L.cfg[6]})
      if (r >= 0 && (L.refs[r].offset % 4 != 0 || L.refs[r].strides[0] % 4 != 0)) nk_pro_ok = false;
  if (a.pro == KH_GEMV_PRO_ATTN && !nk_layout) {
    err = "gemv: an attention prologue needs the K-contiguous weight layout";
    return nullptr;
  }
  if (op->bf16 && !(nk_layout && nk_pro_ok)) {
    err = "gemv: bf16 weights must be a [batch][N][K] copy with K a multiple of 8 and unit-stride, "
          "16-byte aligned x (and LayerNorm gamma / beta) rows";
    return nullptr;
  }
  if (nk_layout && nk_pro_ok) {
    const int64_t k4 = K / kv;
    int best_r = 0, best_w = 0;
    int64_t best_waste = -1;
    for (int r : {3, 4, 2, 1}) {
      if (r == 4 && a.pro == KH_GEMV_PRO_ATTN) continue;
      const int64_t w = (k4 + 64 * r - 1) / (64 * r);
      if (w > kNkMaxWaves) continue;
      const int64_t waste = 64 * r * w - k4;
      if (best_waste < 0 || waste < best_waste) best_r = r, best_w = (int)w, best_waste = waste;
    }
    if (best_r == 0 && a.pro != KH_GEMV_PRO_LAYERNORM)  // several passes over K
      best_r = a.pro == KH_GEMV_PRO_ATTN ? 3 : 4, best_w = kNkMaxWaves;
    if (best_r == 0 && op->bf16) {
      unsupported = true;
      err = "gemv: a bf16 LayerNorm prologue needs the row in one pass (K <= 16384)";
      return nullptr;
    }
    if (best_r > 0) {
      op->nk_r = best_r, op->nk_waves = best_w;
      op->nk_grid = dim3((unsigned)((N + kNkCols - 1) / kNkCols), (unsigned)b1, 1);
    }
  }
  op->quads = quads;
  op->threads = threads;
  a.k_per_split = (int)kper;
  a.splitk = (int)splitk;
  op->grid = dim3((unsigned)n_blocks, (unsigned)b1, (unsigned)splitk);
  if (splitk > 1) {
    op->n_partials = (size_t)splitk * batch * N;
  }
  return op;
}

}  // namespace kh
