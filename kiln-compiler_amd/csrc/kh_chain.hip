// kh_chain.hip - persistent GEMV chains: consecutive one-row matmuls, each
// reading the previous one's output (decode: ln_1 + qkv, attention + c_proj
// + residual, ln_2 + fc + GELU, proj + residual, layer after layer), run as
// ONE launch instead of one launch each.
//
// A decode GEMV streams a few MB of weights; as its own launch it costs the
// launch itself (~1.8 us in a hipGraph), one memory latency for its first
// loads and the streaming time, all in series. Here one workgroup per CU
// walks every stage of the chain:
//   * before waiting for stage s's input, each wave has already issued the
//     loads of its weight slice of stage s (and the bias / residual / gamma /
//     beta it needs), so the weight stream of a stage overlaps the hand-over
//     of the previous one;
//   * stage outputs are handed over as 64-bit words (value, epoch) written
//     with device-scope stores by a fifth wave of the workgroup that only
//     stores (below); a consumer polls the words of its input
//     with device-scope loads until every epoch is the current call's, so a
//     value and the proof that it is ready arrive in one load - no counter,
//     no fence, no atomics on shared addresses (a shared arrival counter was
//     measured at 2.8-20 us per stage with 64-256 workgroups, serialised on
//     its one address);
//   * the epoch is a per-plan word read by every workgroup at kernel start
//     (+1 = this call's tag); workgroup 0 stores the new value as its last
//     act, after every workgroup has reported (a `started` word each) that it
//     read the old one, so the next call's tags never match a stale word;
//   * every wait is bounded (wall clock, `spin` ticks of the plan's state);
//     a wait that gives up counts a timeout in the plan's state, and its
//     workgroup stores NaN, under the current epoch, as every output it
//     still owed (its columns of the stage that gave up and of every later
//     stage) and leaves the kernel: the grid always drains, the workgroups
//     that wait for those columns get them at once, and every value
//     downstream of the give-up is NaN (kh_plan_chain_timeouts reports the
//     count; the Python runtime raises on it);
//   * the four compute waves never store: one counter (vmcnt) tracks a
//     wave's loads and stores together and in issue order, so a wave that
//     stored its outputs would wait for the stores' device-scope
//     acknowledgement (a memory round trip) at its next wait for a load -
//     before the next stage's weights or hand-over words could be used. They
//     leave their outputs in LDS and pass a barrier; the store wave, which
//     issues no loads, stores them.
// Stage t's in-chain operands (x, q / k / v of the attention prologue, the
// residual) are read from the hand-over words of the stage that produced
// them; operands from outside the chain are read from memory. A stage also
// stores its output in the plan's buffers only where a launch after the
// chain reads it and no later stage of the chain overwrites it, so no two
// workgroups of the chain store to one address.
//
// The host side finds the chains at plan creation (find_chains) from the
// GEMV descriptors marked KH_GEMV_CHAIN, proves from the operands' element
// ranges which stage produced each operand and that nothing else overlaps,
// and binds device state (descriptors, hand-over words, epoch) in
// kh_plan_bind.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "kh_common.hpp"
#include "kh_gemm_args.hpp"
#include "kh_internal.hpp"

namespace kh {
namespace {

constexpr int kSlots = 12;                    // 16-byte weight chunks per lane and pass
constexpr int kThreads = 256;                 // 4 compute waves per workgroup
constexpr int kWaves = kThreads / 64;
constexpr int kBlock = kThreads + 64;         // and the store wave
constexpr int kMaxK = 4096;                   // x row staged in LDS
constexpr int kPerThread = kMaxK / kThreads;  // x words per thread
constexpr int kAttRounds = 4;                 // attention prologue: head rounds per wave
constexpr int kMaxDyn = 8;                    // distinct input / output slots a chain reads or writes
constexpr int kMaxGroups = 1024;              // workgroups (one per CU)
constexpr int kMaxStages = 96;                // stages of one chain (their descriptors sit in LDS)
constexpr int64_t kSpinTicks = 2000000;     // default bound per wait: 20 ms of the 100 MHz wall clock

// An operand address: the absolute address (constants, arena) resolved at
// bind, or dynamic slot `slot` (a plan input or output) + `off` floats.
struct CPtr {
  const void *abs;
  int64_t off;
  int32_t slot;
  int32_t pad;
};

struct ChainDyn {
  float *p[kMaxDyn];
};

struct ChainState {
  uint32_t epoch;
  uint32_t pad;
  unsigned long long timeouts;
  int64_t spin;                  // wall-clock ticks a wait may take; < 0: every wait gives up (test hook)
  uint64_t started[kMaxGroups];  // (epoch, group) words: group g has read the epoch
};

struct alignas(16) CStage {
  CPtr w, x, gamma, beta, bias, res, out, q, k, v, mask;
  const uint64_t *x_ll;    // non-null: x word i = x_ll[i]
  const uint64_t *res_ll;  // non-null: residual of column n = res_ll[n * res_sn]
  const uint64_t *att_ll;  // non-null: q / k / v element e (offset from its pointer) = att_ll[e + shift]
  int64_t q_shift, k_shift, v_shift, att_n;
  uint64_t *out_ll;        // this stage's hand-over words, one per column
  int64_t w_sn, bias_sn, res_sn, out_sn;
  int64_t q_s0, k_s0, k_s1, v_s0, v_s1, m_s0, m_s2;
  int32_t N, K, bf16, pro, act, plain_out, has_bias, has_res, has_gamma, has_beta;
  float c1, c2, eps, att_cscale;
  int32_t att_dh, att_lim, att_heads, att_mask;
  int32_t kind;  // index into kKinds: the (chunks per lane and column, bf16) variant of the stage code
};

// Stage code variants: P 16-byte weight chunks per lane and column (P >=
// ceil(K / (4 or 8) / 64)), up to kSlots / P columns per wave, fp32 or bf16
// weights. Fixed shapes let the compiler keep the weights in registers with
// static indices and issue each stage's loads as one burst.
constexpr int kKindP[] = {1, 2, 3, 4, 6, 12};
constexpr int kNumP = sizeof(kKindP) / sizeof(kKindP[0]);

// Every address the kernel reads or writes comes out of a descriptor in
// memory, where the compiler cannot see that it is global memory; a generic
// (flat) access would also count against the LDS / scalar-load wait counter,
// so each wait for an LDS read would wait for every weight load in flight.
// All accesses therefore go through global address-space pointers.
template <class T>
using global_ptr = __attribute__((address_space(1))) T *;
template <class T>
__device__ __forceinline__ global_ptr<const T> gbl(const T *p) {
  return (global_ptr<const T>)p;
}
template <class T>
__device__ __forceinline__ global_ptr<T> gbl_w(T *p) {
  return (global_ptr<T>)p;
}

__device__ __forceinline__ uint64_t ll_get(const uint64_t *p) {
  return __hip_atomic_load(gbl(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ll_put(uint64_t *p, uint64_t w) {
  __hip_atomic_store(gbl_w(p), w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t ll_word(float v, uint32_t e) {
  return (uint64_t)e << 32 | __float_as_uint(v);
}
__device__ __forceinline__ bool ll_ok(uint64_t w, uint32_t e) { return (uint32_t)(w >> 32) == e; }
__device__ __forceinline__ float ll_val(uint64_t w) { return __uint_as_float((uint32_t)w); }

__device__ __forceinline__ const float *cptr(const CPtr &p, const ChainDyn &d) {
  if (p.slot < 0) return static_cast<const float *>(p.abs);
  const float *b = d.p[0];
#pragma unroll
  for (int i = 1; i < kMaxDyn; ++i)
    if (p.slot == i) b = d.p[i];
  return b + p.off;
}

// 128-bit weight load marked non-temporal (each weight byte is read once per
// call).
__device__ __forceinline__ uint4 load_weights(const uint4 *p) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t v = __builtin_nontemporal_load(gbl(reinterpret_cast<const u32x4_t *>(p)));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float ld(const float *p, int64_t i) { return gbl(p)[i]; }

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float round_bf16(float x) { return (float)(__bf16)x; }

// Sum over the compute waves in a fixed order (wave tree, then waves 0..3).
// Two barriers; the LayerNorm prologue takes two sums, and the store wave
// passes the same kLnBarriers barriers.
constexpr int kLnBarriers = 4;
__device__ __forceinline__ float group_sum(float v, float *red) {
  v = wave_sum(v);
  __syncthreads();  // `red` may still be read from a previous sum
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// The fields of a stage that its prefetch and compute use, read from the
// descriptor once, in one burst, into wave-uniform registers (addresses
// resolved): reading them where they are used would put a dependent LDS or
// scalar load in front of most instructions of the stage.
struct Hot {
  const char *w;
  const float *bias, *res, *gamma, *beta;
  float *out;
  const uint64_t *res_ll;
  uint64_t *out_ll;
  int64_t w_sn, bias_sn, res_sn, out_sn;
  int N, K, kind, act, pro, plain_out, has_bias, has_res, has_gamma, has_beta;
};

__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint64_t u = (uint64_t)v;
  return (int64_t)((uint64_t)(uint32_t)uni((int)(uint32_t)(u >> 32)) << 32 | (uint32_t)uni((int)(uint32_t)u));
}
template <class T>
__device__ __forceinline__ T *unip(T *p) {
  return reinterpret_cast<T *>(uni64(reinterpret_cast<int64_t>(p)));
}

__device__ __forceinline__ Hot hot_of(const CStage &S, const ChainDyn &dyn) {
  Hot h;
  h.w = unip(reinterpret_cast<const char *>(cptr(S.w, dyn)));
  h.bias = unip(S.has_bias ? cptr(S.bias, dyn) : reinterpret_cast<const float *>(h.w));
  h.res = unip(S.has_res && !S.res_ll ? cptr(S.res, dyn) : reinterpret_cast<const float *>(h.w));
  h.gamma = unip(S.has_gamma ? cptr(S.gamma, dyn) : reinterpret_cast<const float *>(h.w));
  h.beta = unip(S.has_beta ? cptr(S.beta, dyn) : reinterpret_cast<const float *>(h.w));
  h.out = unip(const_cast<float *>(cptr(S.out, dyn)));
  h.res_ll = unip(S.res_ll);
  h.out_ll = unip(S.out_ll);
  h.w_sn = uni64(S.w_sn), h.bias_sn = uni64(S.bias_sn), h.res_sn = uni64(S.res_sn), h.out_sn = uni64(S.out_sn);
  h.N = uni(S.N), h.K = uni(S.K), h.kind = uni(S.kind), h.act = uni(S.act), h.pro = uni(S.pro);
  h.plain_out = uni(S.plain_out), h.has_bias = uni(S.has_bias), h.has_res = uni(S.has_res);
  h.has_gamma = uni(S.has_gamma), h.has_beta = uni(S.has_beta);
  return h;
}

// What one thread keeps from the prefetch of a stage to its compute: the
// weight chunks of its wave's columns, and in lane c the bias and residual
// word of column c.
struct Carry {
  uint4 w[kSlots];
  float pb, prp;   // bias; residual read from memory
  uint64_t pr;     // residual hand-over word
};

// Columns of stage S that wave gw owns: gw, gw + nwaves, ...
__device__ __forceinline__ int wave_columns(const Hot &S, int gw, int nwaves) {
  return gw < S.N ? (S.N - 1 - gw) / nwaves + 1 : 0;
}

template <int P, bool BF16>
__device__ __forceinline__ void prefetch_t(const Hot &S, int gw, int nwaves, int lane, Carry &cr) {
  constexpr int CMAX = kSlots / P;
  const int U = S.K / (BF16 ? 8 : 4);
  const int nc = wave_columns(S, gw, nwaves);
  if (nc == 0) return;
  const int64_t row_bytes = S.w_sn * (BF16 ? 2 : 4);
#pragma unroll
  for (int c = 0; c < CMAX; ++c) {
    if (c < nc) {
      const uint4 *row = reinterpret_cast<const uint4 *>(S.w + (gw + (int64_t)c * nwaves) * row_bytes);
#pragma unroll
      for (int j = 0; j < P; ++j)  // chunks past the row end re-read its last chunk (dropped at use)
        cr.w[c * P + j] = load_weights(row + min(lane + 64 * j, U - 1));
    }
  }
  // lane c: the bias and residual of column c (other lanes re-read column 0).
  // Every load here is unconditional, into the register its use reads (an
  // absent operand reads a valid stand-in address and is ignored at use): a
  // load merged with a default value would make the compiler wait for it on
  // the spot, and that wait also covers every weight load and store before it.
  const int64_t col = gw + (int64_t)(lane < min(nc, CMAX) ? lane : 0) * nwaves;
  cr.pb = ld(S.bias, S.has_bias ? col * S.bias_sn : 0);
  cr.prp = ld(S.res, S.has_res && !S.res_ll ? col * S.res_sn : 0);
  cr.pr = ll_get(S.res_ll ? S.res_ll + col * S.res_sn : S.out_ll);
}

// The wave's dot products from the weight chunks in registers and x in LDS,
// then in lane c the epilogue of column c, left in outs[64 * wave + c] for
// the store wave.
template <int P, bool BF16>
__device__ __forceinline__ void compute_t(const Hot &S, int gw, int nwaves, int lane, uint32_t epoch, Carry &cr,
                                          const float *xs, float *outs, ChainState *state, int64_t spin) {
  constexpr int CMAX = kSlots / P;
  const int U = S.K / (BF16 ? 8 : 4);
  const int nc = wave_columns(S, gw, nwaves);
  if (nc == 0) return;
  const float4 *x4 = reinterpret_cast<const float4 *>(xs);
  float outv = 0.0f;
#pragma unroll
  for (int c = 0; c < CMAX; ++c) {
    if (c >= nc) continue;
    float part = 0.0f;
#pragma unroll
    for (int j = 0; j < P; ++j) {
      const int u = lane + 64 * j;
      const bool in = 64 * (j + 1) <= U || u < U;
      const int ua = min(u, U - 1);
      const uint4 q = cr.w[c * P + j];
      if constexpr (BF16) {
        const float4 a = x4[2 * ua], b = x4[2 * ua + 1];
        float t = 0.0f;
        t = fmaf(round_bf16(a.x), bf16_lo(q.x), t);
        t = fmaf(round_bf16(a.y), bf16_hi(q.x), t);
        t = fmaf(round_bf16(a.z), bf16_lo(q.y), t);
        t = fmaf(round_bf16(a.w), bf16_hi(q.y), t);
        t = fmaf(round_bf16(b.x), bf16_lo(q.z), t);
        t = fmaf(round_bf16(b.y), bf16_hi(q.z), t);
        t = fmaf(round_bf16(b.z), bf16_lo(q.w), t);
        t = fmaf(round_bf16(b.w), bf16_hi(q.w), t);
        part += in ? t : 0.0f;
      } else {
        const float4 a = x4[ua];
        float t = a.x * __uint_as_float(q.x);
        t = fmaf(a.y, __uint_as_float(q.y), t);
        t = fmaf(a.z, __uint_as_float(q.z), t);
        t = fmaf(a.w, __uint_as_float(q.w), t);
        part += in ? t : 0.0f;
      }
    }
    const float tot = wave_sum(part);
    if (lane == c) outv = tot;
  }
  if (lane >= min(nc, CMAX)) return;
  const int64_t col = gw + (int64_t)lane * nwaves;
  uint64_t pr = S.res_ll ? cr.pr : ll_word(cr.prp, epoch);
  if (S.has_res && S.res_ll && !ll_ok(pr, epoch)) {
    const long long t0 = wall_clock64();
    while (!ll_ok(pr = ll_get(S.res_ll + col * S.res_sn), epoch)) {
      if (spin < 0 || wall_clock64() - t0 > spin) {
        atomicAdd(&state->timeouts, 1ull);
        pr = ll_word(__builtin_nanf(""), epoch);   // the column's output becomes NaN
        break;
      }
    }
  }
  // the tape's operations in its order: (acc + bias), then res + that, then act
  float v = outv;
  if (S.has_bias) v += cr.pb;
  if (S.has_res) v = ll_val(pr) + v;
  if (S.act == KH_OP_GELU_TANH) v = op_gelu_tanh(v);
  else if (S.act == KH_OP_GELU_ERF) v = op_gelu_erf(v);
  else if (S.act == KH_OP_RELU) v = v != v ? v : fmaxf(v, 0.0f);
  outs[threadIdx.x] = v;   // (threadIdx.x = 64 * wave + lane: an address the compiler need not keep)
}

#define KH_CHAIN_KINDS(X) \
  X(0, 1, false) X(1, 2, false) X(2, 3, false) X(3, 4, false) X(4, 6, false) X(5, 12, false) \
  X(6, 1, true) X(7, 2, true) X(8, 3, true) X(9, 4, true) X(10, 6, true) X(11, 12, true)

__device__ __forceinline__ void prefetch(const Hot &S, int gw, int nwaves, int lane, Carry &cr) {
  switch (S.kind) {
#define KH_X(k, P, B) \
  case k: prefetch_t<P, B>(S, gw, nwaves, lane, cr); break;
    KH_CHAIN_KINDS(KH_X)
#undef KH_X
  }
}

__device__ __forceinline__ void compute(const Hot &S, int gw, int nwaves, int lane, uint32_t epoch, Carry &cr,
                                        const float *xs, float *outs, ChainState *state, int64_t spin) {
  switch (S.kind) {
#define KH_X(k, P, B) \
  case k: compute_t<P, B>(S, gw, nwaves, lane, epoch, cr, xs, outs, state, spin); break;
    KH_CHAIN_KINDS(KH_X)
#undef KH_X
  }
}

// The store wave: lane 16w + c stores column c of compute wave w's outputs
// (its memory copy when the stage's output is read after the chain, and its
// hand-over word).
// `poison`: NaN instead of the computed value (a stage this workgroup gave up).
__device__ __forceinline__ void store_outputs(const Hot &S, int nwaves, int lane, uint32_t epoch,
                                              const float *outs, bool poison = false) {
  const int w = lane >> 4, c = lane & 15;
  const int gw = (int)blockIdx.x * kWaves + w;
  const int nc = min(wave_columns(S, gw, nwaves), kSlots / kKindP[S.kind % kNumP]);
  if (w >= kWaves || c >= nc) return;
  const int64_t col = gw + (int64_t)c * nwaves;
  const float v = poison ? __builtin_nanf("") : outs[w * 64 + c];
  if (S.plain_out) gbl_w(S.out)[col * S.out_sn] = v;
  ll_put(S.out_ll + col, ll_word(v, epoch));
}

// Poll n words until each carries `epoch` or the wait's time runs out;
// `reload(i)` re-reads word i.
// The wall clock (a scalar-memory read) is checked every 64 rounds only, so
// a round costs one memory round trip.
template <int N, class Need, class Reload>
__device__ __forceinline__ bool poll(uint64_t (&v)[N], uint32_t epoch, int64_t spin, Need need, Reload reload) {
  if (spin < 0) return false;
  long long t0 = 0;
  for (unsigned round = 0;; ++round) {
    bool all = true;
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (need(i) && !ll_ok(v[i], epoch)) all = false;
    if (all) return true;
    if ((round & 63) == 0) {
      const long long now = wall_clock64();
      if (round == 0) t0 = now;
      else if (now - t0 > spin) return false;
    }
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (need(i) && !ll_ok(v[i], epoch)) v[i] = reload(i);
  }
}

// The stage's row x into LDS: from the producer's hand-over words (or
// memory), with the LayerNorm prologue applied. false: a wait gave up.
__device__ __forceinline__ bool acquire_x(const CStage &S, const Hot &hot, const ChainDyn &dyn, uint32_t epoch,
                                          int64_t spin, float *xs, float *red) {
  uint64_t v[kPerThread];
  const float *xp = S.x_ll ? nullptr : cptr(S.x, dyn);
  const int tid = threadIdx.x;
  // the LayerNorm's gamma / beta, issued with the first polls (unconditional
  // loads: clamped indices, an absent gamma / beta reads a stand-in and is
  // ignored at use)
  float pg[kPerThread], pbe[kPerThread];
  if (S.pro == KH_GEMV_PRO_LAYERNORM) {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int k = min(tid + i * kThreads, S.K - 1);
      if (tid + i * kThreads < S.K) pg[i] = ld(hot.gamma, k), pbe[i] = ld(hot.beta, k);
    }
  }
#pragma unroll
  for (int i = 0; i < kPerThread; ++i) {
    const int k = tid + i * kThreads;
    if (k < S.K) v[i] = S.x_ll ? ll_get(S.x_ll + k) : ll_word(ld(xp, k), epoch);
  }
  const bool good = poll(
      v, epoch, spin, [&](int i) { return tid + i * kThreads < S.K; },
      [&](int i) { return ll_get(S.x_ll + tid + i * kThreads); });
  if (S.pro == KH_GEMV_PRO_LAYERNORM) {
    // mean, then the variance of the centred values (every thread takes part
    // in both sums, also after a failed wait, so the barriers stay uniform)
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      if (tid + i * kThreads < S.K) s += ll_val(v[i]);
    const float mean = group_sum(s, red) * S.c1;
    float s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kPerThread; ++i)
      if (tid + i * kThreads < S.K) {
        const float d = ll_val(v[i]) - mean;
        s2 = fmaf(d, d, s2);
      }
    const float rstd = rsqrtf(group_sum(s2, red) * S.c2 + S.eps);
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int k = tid + i * kThreads;
      if (k < S.K) {
        float y = (ll_val(v[i]) - mean) * rstd;
        if (S.has_gamma) y *= pg[i];
        if (S.has_beta) y += pbe[i];
        xs[k] = y;
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) {
      const int k = tid + i * kThreads;
      if (k < S.K) xs[k] = ll_val(v[i]);
    }
  }
  return good;
}

// Attention prologue: x[h * dh + d] = softmax_j(scaled q_h . k_jh [+ mask])
// . v_jh[d] for the one query, into LDS. Wave w takes heads (w + 4r) * HPI +
// lane / dh (HPI = 64 / dh heads per round), lane % dh = d; the base-2
// online softmax of the attention kernels (exponentials against 0 while no
// score is finite; a fully masked row gives NaN as in eager).
__device__ __forceinline__ bool attend(const CStage &S, const ChainDyn &dyn, uint32_t epoch, int64_t spin,
                                       float *xs) {
  constexpr float kLog2e = 1.4426950408889634f;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int dh = S.att_dh, hpi = 64 / dh, sub = lane / dh, d = lane % dh;
  const float *qp = cptr(S.q, dyn), *kp = cptr(S.k, dyn), *vp = cptr(S.v, dyn);
  const float *mp = S.att_mask ? cptr(S.mask, dyn) : nullptr;
  auto word = [&](const float *plain, int64_t e, int64_t shift) -> uint64_t {
    const int64_t idx = e + shift;
    if (S.att_ll && idx >= 0 && idx < S.att_n) return ll_get(S.att_ll + idx);
    return ll_word(ld(plain, e), epoch);
  };
  int h[kAttRounds];
  bool on[kAttRounds];
#pragma unroll
  for (int r = 0; r < kAttRounds; ++r) {
    h[r] = (wave + kWaves * r) * hpi + sub;
    on[r] = h[r] < S.att_heads;
  }
  uint64_t wq[kAttRounds];
#pragma unroll
  for (int r = 0; r < kAttRounds; ++r)
    if (on[r]) wq[r] = word(qp, (int64_t)h[r] * S.q_s0 + d, S.q_shift);
  float m[kAttRounds], l[kAttRounds], acc[kAttRounds];
#pragma unroll
  for (int r = 0; r < kAttRounds; ++r) m[r] = -INFINITY, l[r] = 0.0f, acc[r] = 0.0f;
  bool good = true;
  for (int j = 0; j < S.att_lim; ++j) {
    // the key and value words of every round, and the query words, polled together
    uint64_t kv[3 * kAttRounds];
#pragma unroll
    for (int r = 0; r < kAttRounds; ++r) {
      if (!on[r]) continue;
      kv[3 * r] = word(kp, (int64_t)h[r] * S.k_s0 + (int64_t)j * S.k_s1 + d, S.k_shift);
      kv[3 * r + 1] = word(vp, (int64_t)h[r] * S.v_s0 + (int64_t)j * S.v_s1 + d, S.v_shift);
      kv[3 * r + 2] = wq[r];
    }
    good = poll(
               kv, epoch, spin, [&](int i) { return on[i / 3]; },
               [&](int i) {
                 const int r = i / 3;
                 if (i % 3 == 0) return word(kp, (int64_t)h[r] * S.k_s0 + (int64_t)j * S.k_s1 + d, S.k_shift);
                 if (i % 3 == 1) return word(vp, (int64_t)h[r] * S.v_s0 + (int64_t)j * S.v_s1 + d, S.v_shift);
                 return word(qp, (int64_t)h[r] * S.q_s0 + d, S.q_shift);
               }) &&
           good;
#pragma unroll
    for (int r = 0; r < kAttRounds; ++r) {
      if ((wave + kWaves * r) * hpi >= S.att_heads) continue;  // wave-uniform: no lane of the round is on
      wq[r] = kv[3 * r + 2];
      float t = on[r] ? ll_val(wq[r]) * S.att_cscale * ll_val(kv[3 * r]) : 0.0f;
      for (int o = 1; o < dh; o <<= 1) t += __shfl_xor(t, o, 64);
      if (!on[r]) continue;
      if (mp) t = fmaf(ld(mp, (int64_t)h[r] * S.m_s0 + (int64_t)j * S.m_s2), kLog2e, t);
      const float m_new = fmaxf(m[r], t);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m[r] - m_use);
      const float p = __builtin_amdgcn_exp2f(t - m_use);
      l[r] = fmaf(l[r], alpha, p);
      acc[r] = fmaf(acc[r], alpha, p * ll_val(kv[3 * r + 1]));
      m[r] = m_new;
    }
  }
#pragma unroll
  for (int r = 0; r < kAttRounds; ++r)
    if (on[r]) xs[h[r] * dh + d] = acc[r] / l[r];
  return good;
}

__global__ __launch_bounds__(kBlock) void gemv_chain_kernel(const CStage *st, int n_stages,
                                                              ChainDyn dyn, ChainState *state) {
  __shared__ float4 xs4[kMaxK / 4];
  __shared__ float red[kWaves];
  __shared__ float outs[kWaves * 64];   // the compute waves' stage outputs, for the store wave
  __shared__ int alive;
  // the stage descriptors, copied once: a stage's fields are then LDS reads
  // instead of scalar loads that miss the scalar cache stage after stage
  __shared__ CStage st_lds[kMaxStages];
  float *xs = reinterpret_cast<float *>(xs4);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int nwaves = gridDim.x * kWaves, gw = blockIdx.x * kWaves + wave;
  {
    static_assert(sizeof(CStage) % 16 == 0, "descriptors copy as 16-byte pieces");
    typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
    const u32x4_t *from = reinterpret_cast<const u32x4_t *>(st);
    u32x4_t *to = reinterpret_cast<u32x4_t *>(st_lds);
    const int pieces = n_stages * (int)(sizeof(CStage) / 16);
    for (int i = tid; i < pieces; i += kBlock) to[i] = gbl(from)[i];
    __syncthreads();
    st = st_lds;
  }
  const uint32_t epoch = __hip_atomic_load(&state->epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
  const int64_t spin = __hip_atomic_load(&state->spin, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const bool storer = wave == kWaves;
  if (tid == 0) alive = 1;
  if (storer && lane == 0) ll_put(&state->started[blockIdx.x], (uint64_t)epoch << 32 | blockIdx.x);
  // Every wave passes the same barriers per stage: B1 at the start, the
  // LayerNorm prologue's, B2 once x is in LDS, B3 once the outputs are in
  // `outs`. The store wave has a loop of its own (values of the compute
  // loop merged into it would be copied between registers, and each copy
  // would wait for the stores before it).
  if (storer) {
    for (int s = 0; s < n_stages; ++s) {
      const CStage &S = st[s];
      if ((int)blockIdx.x * kWaves >= S.N) continue;
      __syncthreads();                                 // B1
      if (S.pro == KH_GEMV_PRO_LAYERNORM)
        for (int i = 0; i < kLnBarriers; ++i) __syncthreads();
      __syncthreads();                                 // B2
      if (!alive) {
        // a wait of this workgroup gave up at stage s: NaN for every column
        // it owes from stage s on, so no other workgroup waits for them and
        // everything computed from them is NaN
        for (int s2 = s; s2 < n_stages; ++s2)
          if ((int)blockIdx.x * kWaves < st[s2].N) store_outputs(hot_of(st[s2], dyn), nwaves, lane, epoch, outs, true);
        break;
      }
      __syncthreads();                                 // B3
      store_outputs(hot_of(S, dyn), nwaves, lane, epoch, outs);   // `outs` is rewritten only after the next B2
    }
    return;
  }
  for (int s = 0; s < n_stages; ++s) {
    const CStage &S = st[s];
    if ((int)blockIdx.x * kWaves >= S.N) continue;  // this workgroup owns no columns of stage s
    const Hot hot = hot_of(S, dyn);
    // The stage's weights and epilogue operands are loaded before its input
    // is awaited. They live in registers of this iteration only: a value
    // carried to the next stage would be copied between registers at the end
    // of the stage, and the copy's wait for the load would also wait for
    // every memory operation issued before it.
    Carry cr;
    prefetch(hot, gw, nwaves, lane, cr);
    __syncthreads();                                   // B1: the previous stage's reads of xs are done
    const bool good =
        S.pro == KH_GEMV_PRO_ATTN ? attend(S, dyn, epoch, spin, xs) : acquire_x(S, hot, dyn, epoch, spin, xs, red);
    if (!good) alive = 0;
    __syncthreads();                                   // B2
    if (!alive) {
      if (tid == 0) atomicAdd(&state->timeouts, 1ull);
      break;
    }
    compute(hot, gw, nwaves, lane, epoch, cr, xs, outs, state, spin);
    __syncthreads();                                   // B3
  }
  if (blockIdx.x == 0 && wave == 0) {
    // every workgroup has read the old epoch before the new one is stored
    const long long t0 = wall_clock64();
    for (int g = lane; g < (int)gridDim.x; g += 64) {
      while (!ll_ok(ll_get(&state->started[g]), epoch)) {
        if (wall_clock64() - t0 > kSpinTicks) {
          atomicAdd(&state->timeouts, 1ull);
          break;
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
    if (lane == 0) __hip_atomic_store(&state->epoch, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ---------------------------------------------------------------------------
// host side

struct Range {
  int base = -1, index = 0;
  int64_t lo = 0, hi = 0;  // element offsets [lo, hi)
  bool overlaps(const Range &o) const { return base == o.base && index == o.index && lo < o.hi && o.lo < hi; }
  bool inside(const Range &o) const { return base == o.base && index == o.index && lo >= o.lo && hi <= o.hi; }
};

Range range_of(const kh_ref &r, int64_t extent) {  // extent: highest element offset from r.offset + 1
  Range g;
  g.base = r.base, g.index = r.index, g.lo = r.offset, g.hi = r.offset + extent;
  return g;
}

struct HostOperand {
  bool present = false;
  kh_ref ref{};
};

struct HostStage {
  int launch = -1;
  CStage d{};
  HostOperand w, x, gamma, beta, bias, res, out, q, k, v, mask;
  Range out_range;
  bool out_unit = false;  // output columns are adjacent elements (hand-over word n = element n)
  int x_from = -1, res_from = -1, att_from = -1;
  int64_t x_ll_off = 0, res_ll_off = 0;
};

class GemvChain final : public Chain {
 public:
  std::vector<HostStage> st;
  std::vector<std::pair<int, int>> dyn_slots;  // (base, index) of dynamic slot i
  int groups = 1;
  CStage *d_stages = nullptr;
  uint64_t *d_ll = nullptr;
  ChainState *d_state = nullptr;
  std::vector<int64_t> ll_at;  // word offset of stage i's hand-over words
  bool bound_ok = false;

  ~GemvChain() override {
    if (d_stages) (void)hipFree(d_stages);
    if (d_ll) (void)hipFree(d_ll);
    if (d_state) (void)hipFree(d_state);
  }
  int first() const override { return st.front().launch; }
  int end() const override { return st.back().launch + 1; }
  bool active() const override { return bound_ok; }

  int dyn_slot(int base, int index) {
    for (int i = 0; i < (int)dyn_slots.size(); ++i)
      if (dyn_slots[i].first == base && dyn_slots[i].second == index) return i;
    dyn_slots.emplace_back(base, index);
    return (int)dyn_slots.size() - 1;
  }

  // Static address of an operand (constants, arena) or its dynamic slot.
  bool resolve(const HostOperand &o, void *const *consts, int n_consts, void *arena, CPtr &p, std::string &err) {
    p = CPtr{};
    p.slot = -1;
    if (!o.present) return true;
    const kh_ref &r = o.ref;
    switch (r.base) {
      case KH_BASE_CONST:
        if (r.index < 0 || r.index >= n_consts || !consts[r.index]) {
          err = "chain: missing constant";
          return false;
        }
        p.abs = static_cast<const float *>(consts[r.index]) + r.offset;
        return true;
      case KH_BASE_ARENA:
        if (!arena) {
          err = "chain: no arena bound";
          return false;
        }
        p.abs = static_cast<const float *>(arena) + r.offset;
        return true;
      case KH_BASE_INPUT:
      case KH_BASE_OUTPUT:
        p.slot = dyn_slot(r.base, r.index);
        p.off = r.offset;
        return true;
      default: err = "chain: unsupported operand base"; return false;
    }
  }

  int bind(void *const *consts, int n_consts, void *arena, std::string &err) override {
    bound_ok = false;
    dyn_slots.clear();
    std::vector<CStage> dev(st.size());
    int64_t words = 0;
    ll_at.assign(st.size(), 0);
    for (size_t i = 0; i < st.size(); ++i) ll_at[i] = words, words += st[i].d.N;
    if (!d_ll) {
      hipError_t e;
      if ((e = hipMalloc(&d_ll, std::max<int64_t>(1, words) * sizeof(uint64_t))) != hipSuccess ||
          (e = hipMalloc(&d_state, sizeof(ChainState))) != hipSuccess ||
          (e = hipMalloc(&d_stages, st.size() * sizeof(CStage))) != hipSuccess ||
          (e = hipMemset(d_ll, 0, std::max<int64_t>(1, words) * sizeof(uint64_t))) != hipSuccess ||
          (e = hipMemset(d_state, 0, sizeof(ChainState))) != hipSuccess ||
          (e = hipMemcpy(&d_state->spin, &kSpinTicks, sizeof(int64_t), hipMemcpyHostToDevice)) != hipSuccess) {
        (void)hipGetLastError();
        err = std::string("chain state: ") + hipGetErrorString(e);
        return KH_ERR_HIP;
      }
    }
    for (size_t i = 0; i < st.size(); ++i) {
      const HostStage &h = st[i];
      CStage d = h.d;
      if (!resolve(h.w, consts, n_consts, arena, d.w, err) || !resolve(h.x, consts, n_consts, arena, d.x, err) ||
          !resolve(h.gamma, consts, n_consts, arena, d.gamma, err) ||
          !resolve(h.beta, consts, n_consts, arena, d.beta, err) ||
          !resolve(h.bias, consts, n_consts, arena, d.bias, err) ||
          !resolve(h.res, consts, n_consts, arena, d.res, err) ||
          !resolve(h.out, consts, n_consts, arena, d.out, err) || !resolve(h.q, consts, n_consts, arena, d.q, err) ||
          !resolve(h.k, consts, n_consts, arena, d.k, err) || !resolve(h.v, consts, n_consts, arena, d.v, err) ||
          !resolve(h.mask, consts, n_consts, arena, d.mask, err))
        return KH_ERR_INVALID;
      if (d.w.slot >= 0 || (reinterpret_cast<uintptr_t>(d.w.abs) & 15)) {
        err = "chain: weights must be a 16-byte aligned constant";
        return KH_ERR_INVALID;
      }
      d.out_ll = d_ll + ll_at[i];
      d.x_ll = h.x_from >= 0 ? d_ll + ll_at[h.x_from] + h.x_ll_off : nullptr;
      d.res_ll = h.res_from >= 0 ? d_ll + ll_at[h.res_from] + h.res_ll_off : nullptr;
      d.att_ll = h.att_from >= 0 ? d_ll + ll_at[h.att_from] : nullptr;
      dev[i] = d;
    }
    if ((int)dyn_slots.size() > kMaxDyn) {
      err = "chain: too many input / output slots";
      return KH_ERR_UNSUPPORTED;
    }
    const hipError_t e = hipMemcpy(d_stages, dev.data(), dev.size() * sizeof(CStage), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      err = std::string("chain descriptors: ") + hipGetErrorString(e);
      return KH_ERR_HIP;
    }
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_chain_kernel, kBlock, 0) != hipSuccess ||
        per_cu < 1) {
      (void)hipGetLastError();
      err = "chain: the kernel does not fit a CU";
      return KH_ERR_UNSUPPORTED;
    }
    int64_t max_n = 1;
    for (const HostStage &h : st) max_n = std::max<int64_t>(max_n, h.d.N);
    groups = (int)std::min<int64_t>({(int64_t)current_device().cus, (max_n + kWaves - 1) / kWaves, kMaxGroups});
    for (const HostStage &h : st) {
      const int64_t waves = (int64_t)groups * kWaves;
      if ((h.d.N + waves - 1) / waves > kSlots / kKindP[h.d.kind % kNumP]) {
        err = "chain: a stage has more columns per wave than its code variant holds";
        return KH_ERR_UNSUPPORTED;
      }
    }
    bound_ok = true;
    return KH_OK;
  }

  hipError_t launch(void *const *inputs, int n_in, void *const *outputs, int n_out, hipStream_t stream) override {
    if (!bound_ok) return hipErrorNotReady;
    ChainDyn dyn{};
    for (int i = 0; i < (int)dyn_slots.size(); ++i) {
      const int base = dyn_slots[i].first, index = dyn_slots[i].second;
      void *p = nullptr;
      if (base == KH_BASE_INPUT && index >= 0 && index < n_in) p = inputs[index];
      if (base == KH_BASE_OUTPUT && index >= 0 && index < n_out) p = outputs[index];
      if (!p) return hipErrorInvalidValue;
      dyn.p[i] = static_cast<float *>(p);
    }
    hipLaunchKernelGGL(gemv_chain_kernel, dim3(groups), dim3(kBlock), 0, stream, d_stages, (int)st.size(), dyn,
                       d_state);
    return hipGetLastError();
  }

  int set_spin(int64_t ticks) override {
    if (!d_state) return KH_OK;
    return hipMemcpy(&d_state->spin, &ticks, sizeof(ticks), hipMemcpyHostToDevice) == hipSuccess ? KH_OK
                                                                                                 : KH_ERR_HIP;
  }

  int timeouts(unsigned long long *out) override {
    *out = 0;
    if (!d_state) return KH_OK;
    ChainState h;
    const hipError_t e = hipMemcpy(&h, d_state, sizeof(h), hipMemcpyDeviceToHost);
    if (e != hipSuccess) return KH_ERR_HIP;
    *out = h.timeouts;
    return KH_OK;
  }
};

// Stage facts of launch L (a GEMV the chain kernel can run), or false.
bool stage_of(const kh_launch &L, const Op &op, HostStage &h) {
  GemvFacts f;
  if (L.family != KH_FAM_GEMV || !(L.variant & KH_GEMV_CHAIN) || !op.gemv_facts(f)) return false;
  const GemmArgs &a = *f.args;
  if (f.nk_r <= 0 || !a.direct || a.batch != 1 || a.M != 1 || a.N < 1 || a.K < 1 || a.K > kMaxK) return false;
  const int kv = f.bf16 ? 8 : 4;
  if (a.K % kv || a.sa_k != 1 || a.sb_k != 1 || a.sb_n % kv) return false;
  // the stage code variant: the fewest chunks per lane and column that cover
  // a weight row, and every wave's columns in its registers at one workgroup
  // per CU
  const int chunks = (a.K / kv + 63) / 64;
  int pk = -1;
  for (int i = 0; i < kNumP && pk < 0; ++i)
    if (kKindP[i] >= chunks) pk = i;
  if (pk < 0) return false;
  const int64_t waves = (int64_t)std::min(current_device().cus, kMaxGroups) * kWaves;
  if ((a.N + waves - 1) / waves > kSlots / kKindP[pk]) return false;
  CStage &d = h.d;
  d.kind = pk + (f.bf16 ? kNumP : 0);
  d.N = a.N, d.K = a.K, d.bf16 = f.bf16, d.pro = a.pro, d.act = a.d_act;
  d.w_sn = a.sb_n;
  h.w.present = true, h.w.ref = L.refs[1];
  auto epi = [&](int j, HostOperand &o) {
    if (j < 0) return false;
    o.present = true, o.ref = L.refs[2 + j];
    return true;
  };
  if (!epi(a.d_out, h.out)) return false;
  d.out_sn = a.estride[a.d_out][2];
  if (d.out_sn < 0) return false;
  d.has_bias = epi(a.d_bias, h.bias);
  d.bias_sn = d.has_bias ? a.estride[a.d_bias][2] : 0;
  d.has_res = epi(a.d_res, h.res);
  d.res_sn = d.has_res ? a.estride[a.d_res][2] : 0;
  if (d.bias_sn < 0 || d.res_sn < 0) return false;
  if (a.pro == KH_GEMV_PRO_ATTN) {
    constexpr float kLog2e = 1.4426950408889634f;
    const int dh = a.att_dh, heads = a.K / dh;
    if (heads > kAttRounds * kWaves * (64 / dh)) return false;
    epi(a.att_q, h.q), epi(a.att_q + 1, h.k), epi(a.att_q + 2, h.v);
    d.att_mask = epi(a.att_mask, h.mask);
    d.q_s0 = a.estride[a.att_q][0];
    d.k_s0 = a.estride[a.att_q + 1][0], d.k_s1 = a.estride[a.att_q + 1][1];
    d.v_s0 = a.estride[a.att_q + 2][0], d.v_s1 = a.estride[a.att_q + 2][1];
    if (d.att_mask) d.m_s0 = a.estride[a.att_mask][0], d.m_s2 = a.estride[a.att_mask][2];
    d.att_dh = dh, d.att_heads = heads;
    d.att_lim = a.att_mask_mode == KH_ATTN_MASK_CAUSAL ? 1 : a.att_tk;
    d.att_cscale = a.att_scale_mode == KH_ATTN_SCALE_MUL   ? a.att_scale * kLog2e
                   : a.att_scale_mode == KH_ATTN_SCALE_DIV ? kLog2e / a.att_scale
                                                           : kLog2e;
  } else {
    h.x.present = true, h.x.ref = L.refs[0];
    if (a.pro == KH_GEMV_PRO_LAYERNORM) {
      d.has_gamma = epi(a.pro_g, h.gamma);
      d.has_beta = epi(a.pro_b, h.beta);
      d.c1 = a.pro_c1, d.c2 = a.pro_c2, d.eps = a.pro_eps;
    }
  }
  h.out_range = range_of(h.out.ref, (int64_t)(a.N - 1) * d.out_sn + 1);
  h.out_unit = d.out_sn == 1;
  return true;
}

// Element ranges of a stage's operands read from memory or hand-over words.
struct Reads {
  Range r;
  HostOperand *op;
  int kind;  // 0 x, 1 residual, 2 q, 3 k, 4 v, 5 other (read from memory only)
};

std::vector<Reads> reads_of(HostStage &h) {
  std::vector<Reads> out;
  const CStage &d = h.d;
  auto add = [&](HostOperand &o, int64_t extent, int kind) {
    if (o.present) out.push_back({range_of(o.ref, std::max<int64_t>(1, extent)), &o, kind});
  };
  add(h.w, (int64_t)(d.N - 1) * d.w_sn + d.K, 5);
  add(h.x, d.K, 0);
  add(h.gamma, d.K, 5);
  add(h.beta, d.K, 5);
  add(h.bias, (int64_t)(d.N - 1) * d.bias_sn + 1, 5);
  add(h.res, (int64_t)(d.N - 1) * d.res_sn + 1, 1);
  if (d.pro == KH_GEMV_PRO_ATTN) {
    add(h.q, (int64_t)(d.att_heads - 1) * d.q_s0 + d.att_dh, 2);
    add(h.k, (int64_t)(d.att_heads - 1) * d.k_s0 + (int64_t)(d.att_lim - 1) * d.k_s1 + d.att_dh, 3);
    add(h.v, (int64_t)(d.att_heads - 1) * d.v_s0 + (int64_t)(d.att_lim - 1) * d.v_s1 + d.att_dh, 4);
    add(h.mask, (int64_t)(d.att_heads - 1) * d.m_s0 + (int64_t)(d.att_lim - 1) * d.m_s2 + 1, 5);
  }
  return out;
}

// Try to append stage h (index t in the chain) to `chain`; false leaves
// the chain unchanged.
//
// Why the rules below make the one-launch execution equal to the launches
// in order: stage t's operands produced inside the chain are read from the
// hand-over words of their latest producer (so they see exactly the value
// the launch order gives them), and stage t reads ALL of stage t - 1's
// outputs (x is the whole output row; or q, k and v of the attention
// prologue tile it). A wave working on stage t has therefore seen every
// output of stage t - 1, each stored after its wave read that stage's
// operands; by induction every read of every earlier stage has completed.
// So a plain store of stage t cannot overtake a read of an earlier stage
// (write after read), stage t's own reads from memory never touch a range an
// earlier stage of the chain wrote (they would have had a producer), and
// they are only overwritten by later stages, which wait for them.
bool append(std::vector<HostStage> &chain, HostStage h) {
  const int t = (int)chain.size();
  if (t >= kMaxStages) return false;
  for (Reads &rd : reads_of(h)) {
    if (rd.r.base == KH_BASE_WORKSPACE) return false;
    int latest = -1;
    for (int s = t - 1; s >= 0 && latest < 0; --s)
      if (rd.r.overlaps(chain[s].out_range)) latest = s;
    if (latest < 0) continue;  // produced outside the chain: read from memory
    const HostStage &p = chain[latest];
    // an in-chain producer: the operand must lie inside its output, read
    // through its hand-over words (kinds 0..4 only)
    if (rd.kind == 5 || !p.out_unit || !rd.r.inside(p.out_range)) return false;
    const int64_t shift = rd.r.lo - p.out_range.lo;
    if (rd.kind == 0) {
      h.x_from = latest, h.x_ll_off = shift;
    } else if (rd.kind == 1) {
      h.res_from = latest, h.res_ll_off = shift;
    } else {
      if (h.att_from >= 0 && h.att_from != latest) return false;
      h.att_from = latest;
      int64_t &sh = rd.kind == 2 ? h.d.q_shift : rd.kind == 3 ? h.d.k_shift : h.d.v_shift;
      sh = shift;
      h.d.att_n = p.d.N;
    }
  }
  if (t > 0) {
    // stage t reads the whole output of stage t - 1
    const HostStage &p = chain[t - 1];
    if (h.d.pro != KH_GEMV_PRO_ATTN) {
      if (h.x_from != t - 1 || h.x_ll_off != 0 || h.d.K != p.d.N) return false;
    } else {
      const CStage &d = h.d;
      int64_t s[3] = {d.q_shift, d.k_shift, d.v_shift};
      std::sort(s, s + 3);
      if (h.att_from != t - 1 || d.att_lim != 1 || d.q_s0 != d.att_dh || d.k_s0 != d.att_dh ||
          d.v_s0 != d.att_dh || s[0] != 0 || s[1] != d.K || s[2] != 2 * (int64_t)d.K || p.d.N != 3 * d.K)
        return false;
    }
  }
  // the output must not overlap any operand this stage reads from memory,
  // except an in-place residual (read and then written by the same lane)
  for (Reads &rd : reads_of(h)) {
    const bool from_ll = (rd.kind == 0 && h.x_from >= 0) || (rd.kind == 1 && h.res_from >= 0) ||
                         (rd.kind >= 2 && rd.kind <= 4 && h.att_from >= 0);
    if (from_ll || !rd.r.overlaps(h.out_range)) continue;
    const bool in_place = rd.kind == 1 && rd.r.lo == h.out_range.lo && rd.op->ref.strides[2] == h.d.out_sn;
    if (!in_place) return false;
  }
  chain.push_back(h);
  return true;
}

// Bounding element range of operand j of launch L over the launch's
// iteration space (kiln_hip.h: what each family's refs stride over).
Range ref_range(const kh_launch &L, int j) {
  const kh_ref &r = L.refs[j];
  int64_t ext[KH_MAX_RANK] = {0, 0, 0, 0, 0, 0};
  int rank = 3;
  const int64_t *g = L.gemm;
  switch (L.family) {
    case KH_FAM_EW:
    case KH_FAM_ROW:
    case KH_FAM_RED:
      rank = std::min(std::max(L.rank, 0), KH_MAX_RANK);
      for (int d = 0; d < rank; ++d) ext[d] = L.shape[d];
      break;
    case KH_FAM_GEMM:
    case KH_FAM_GEMV: {
      if (j == 0) ext[0] = g[0], ext[1] = g[1], ext[2] = g[3];
      else if (j == 1) ext[0] = g[0], ext[1] = g[3], ext[2] = g[2];
      else ext[0] = g[0], ext[1] = g[1], ext[2] = g[2];
      if (L.family == KH_FAM_GEMV && L.cfg[4] == KH_GEMV_PRO_ATTN && j >= L.cfg[5] && L.cfg[0] > 0) {
        const int64_t heads = g[3] / L.cfg[0], tk = L.cfg[7];
        if (j < L.cfg[5] + 3) ext[0] = heads, ext[1] = tk, ext[2] = L.cfg[0];
        else if (j == L.cfg[5] + 3) ext[0] = heads, ext[1] = 1, ext[2] = tk;  // additive mask
      }
      break;
    }
    case KH_FAM_ATTN:
      if (j == 1 || j == 2) ext[0] = g[0], ext[1] = g[2], ext[2] = g[3];
      else if (j == 4) ext[0] = g[0], ext[1] = g[1], ext[2] = g[2];
      else ext[0] = g[0], ext[1] = g[1], ext[2] = g[3];
      break;
    default:
      // unknown iteration space: the whole slot
      return Range{r.base, r.index, INT64_MIN / 4, INT64_MAX / 4};
  }
  int64_t lo = r.offset, hi = r.offset;
  for (int d = 0; d < rank; ++d) {
    if (ext[d] <= 0) return Range{r.base, r.index, r.offset, r.offset};  // empty
    const int64_t span = (ext[d] - 1) * r.strides[d];
    if (span < 0) lo += span;
    else hi += span;
  }
  return Range{r.base, r.index, lo, hi + 1};
}

// Parts of `r` outside every range in `cover` (same slot).
std::vector<Range> subtract(const Range &r, std::vector<Range> cover) {
  std::sort(cover.begin(), cover.end(), [](const Range &a, const Range &b) { return a.lo < b.lo; });
  std::vector<Range> out;
  int64_t at = r.lo;
  for (const Range &c : cover) {
    if (!c.overlaps(r)) continue;
    if (c.lo > at) out.push_back(Range{r.base, r.index, at, c.lo});
    at = std::max(at, c.hi);
  }
  if (at < r.hi) out.push_back(Range{r.base, r.index, at, r.hi});
  return out;
}

// Which stages store their output in memory: the part of a stage's output
// that no later stage of the chain overwrites, when a launch after the chain
// reads it (or it is a plan output). false: two stages would both store to
// one address (their relative order is not guaranteed), so no chain.
bool plan_plain_stores(std::vector<HostStage> &chain, const std::vector<kh_launch> &desc, int end) {
  for (size_t s = 0; s < chain.size(); ++s) {
    std::vector<Range> later;
    for (size_t t = s + 1; t < chain.size(); ++t) later.push_back(chain[t].out_range);
    const Range &o = chain[s].out_range;
    bool needed = false;
    for (const Range &u : subtract(o, later)) {
      if (o.base != KH_BASE_ARENA) needed = true;
      for (int i = end; i < (int)desc.size() && !needed; ++i)
        for (int j = 0; j < desc[i].n_refs && !needed; ++j) needed = ref_range(desc[i], j).overlaps(u);
    }
    chain[s].d.plain_out = needed;
    if (needed)
      for (const Range &l : later)
        if (l.overlaps(o)) return false;
  }
  return true;
}

}  // namespace

std::vector<std::unique_ptr<Chain>> find_chains(const std::vector<kh_launch> &desc,
                                                const std::vector<std::unique_ptr<Op>> &ops) {
  std::vector<std::unique_ptr<Chain>> out;
  std::vector<HostStage> cur;
  auto flush = [&]() {
    if (cur.size() >= 2 && plan_plain_stores(cur, desc, cur.back().launch + 1)) {
      auto c = std::make_unique<GemvChain>();
      c->st = cur;
      out.push_back(std::move(c));
    }
    cur.clear();
  };
  for (size_t i = 0; i < desc.size(); ++i) {
    HostStage h;
    h.launch = (int)i;
    if (!stage_of(desc[i], *ops[i], h)) {
      flush();
      continue;
    }
    if (!append(cur, h)) {
      flush();
      append(cur, h);  // a chain may start here
    }
  }
  flush();
  return out;
}

}  // namespace kh
