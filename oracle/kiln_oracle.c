/*
 * kiln_oracle.c - CPU restatement of the computations on Kiln's GPU hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load this library, and only as the checker
 * (or the timed CPU baseline); the HIP product path never calls it.
 *
 * Every function computes in double precision from float inputs and writes
 * float outputs. Each follows the reference's definition of the operation:
 *   - op semantics: kiln/ir/ops.py:48-109 (gelu in float64, ops.py:41-45);
 *   - the decompositions the GPU kernels receive: kiln/frontend/fx_import.py
 *     (linear/addmm 140-153, softmax 212-216, layer_norm 217-230);
 *   - the GPT-2 block: tests/models/transformer.py:4-28.
 * How each function is pinned (library routines, closed forms, brute force)
 * is listed in tests/test_oracle.py.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define KO_API __attribute__((visibility("default")))

/* gelu, kiln/ir/ops.py:41-45: tanh form if approximate != 0, else the erf form. */
static double gelu(double x, int approximate) {
  if (approximate) return 0.5 * x * (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x)));
  return 0.5 * x * (1.0 + erf(x / sqrt(2.0)));
}

KO_API void ko_gelu(const float *x, int64_t n, int approximate, float *out) {
  for (int64_t i = 0; i < n; ++i) out[i] = (float)gelu(x[i], approximate);
}

/* Round to the nearest bfloat16 value, ties to even, computed arithmetically
 * (not from the float's bits): the value is scaled by its bf16 quantum - 2^(e-7)
 * for a normal value in [2^e, 2^(e+1)), 2^-133 below 2^-126 - and rint()
 * (the default rounding mode, half to even) picks the neighbour. Results
 * beyond the largest finite bf16 (0x7F7F, (2 - 2^-7) * 2^127) become inf.
 * Follows the bf16 rounding of the GEMM variant the north star states
 * (bf16 inputs, fp32 accumulation). */
KO_API void ko_bf16_round(const float *x, int64_t n, float *out) {
  const double max_bf16 = (2.0 - ldexp(1.0, -7)) * ldexp(1.0, 127);
  for (int64_t i = 0; i < n; ++i) {
    const double v = x[i];
    if (isnan(v) || isinf(v) || v == 0.0) {
      out[i] = x[i];
      continue;
    }
    int e;
    frexp(fabs(v), &e); /* |v| = f * 2^e, f in [0.5, 1): leading bit 2^(e-1) */
    int qexp = (e - 1) - 7;
    if (qexp < -133) qexp = -133;
    const double q = ldexp(1.0, qexp);
    double r = rint(v / q) * q;
    if (fabs(r) > max_bf16) r = r > 0 ? INFINITY : -INFINITY;
    out[i] = (float)r;
  }
}

/* bias + GELU over rows: out[r][c] = gelu(x[r][c] + b[c]) (bench_gpu.py:149). */
KO_API void ko_bias_gelu(const float *x, const float *b, int64_t rows, int64_t cols, int approximate, float *out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = (float)gelu((double)x[r * cols + c] + (double)b[c], approximate);
}

/*
 * Row LayerNorm as the frontend decomposes it (fx_import.py:217-230):
 * mean = sum(x) * (1/n); xc = x - mean; var = sum(xc*xc) * (1/n);
 * y = xc * rsqrt(var + eps); y = y * gamma; y = y + beta (gamma/beta optional).
 */
KO_API void ko_layernorm(const float *x, const float *gamma, const float *beta, double eps, int64_t rows,
                         int64_t inner, float *out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * inner;
    double s = 0.0;
    for (int64_t c = 0; c < inner; ++c) s += xr[c];
    const double mean = s * (1.0 / (double)inner);
    double s2 = 0.0;
    for (int64_t c = 0; c < inner; ++c) {
      const double d = xr[c] - mean;
      s2 += d * d;
    }
    const double rstd = 1.0 / sqrt(s2 * (1.0 / (double)inner) + eps);
    for (int64_t c = 0; c < inner; ++c) {
      double y = (xr[c] - mean) * rstd;
      if (gamma) y *= gamma[c];
      if (beta) y += beta[c];
      out[r * inner + c] = (float)y;
    }
  }
}

/*
 * Row softmax as decomposed (fx_import.py:212-216): m = max(x); e = exp(x - m);
 * out = e / sum(e). `scale` multiplies x first (softmax(x * scale)).
 */
KO_API void ko_softmax(const float *x, double scale, int64_t rows, int64_t inner, float *out) {
  double *e = (double *)malloc(sizeof(double) * (size_t)(inner > 0 ? inner : 1));
  for (int64_t r = 0; r < rows; ++r) {
    const float *xr = x + r * inner;
    double m = -INFINITY;
    for (int64_t c = 0; c < inner; ++c) m = fmax(m, xr[c] * scale);
    double s = 0.0;
    for (int64_t c = 0; c < inner; ++c) {
      e[c] = (m == -INFINITY) ? NAN : exp(xr[c] * scale - m);
      s += e[c];
    }
    for (int64_t c = 0; c < inner; ++c) out[r * inner + c] = (float)(e[c] / s);
  }
  free(e);
}

/*
 * Batched matmul with strided operands (ops.py:102-109):
 * C[b][m][n] = sum_k A[b][m][k] * B[b][k][n], accumulated in double.
 * Strides are in elements; C is written contiguous [batch][M][N].
 */
KO_API void ko_matmul(const float *A, int64_t sab, int64_t sam, int64_t sak, const float *B, int64_t sbb,
                      int64_t sbk, int64_t sbn, int64_t batch, int64_t M, int64_t N, int64_t K, float *C) {
  double *row = (double *)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t m = 0; m < M; ++m) {
      for (int64_t n = 0; n < N; ++n) row[n] = 0.0;
      for (int64_t k = 0; k < K; ++k) {
        const double a = A[b * sab + m * sam + k * sak];
        const float *br = B + b * sbb + k * sbk;
        for (int64_t n = 0; n < N; ++n) row[n] += a * (double)br[n * sbn];
      }
      for (int64_t n = 0; n < N; ++n) C[(b * M + m) * N + n] = (float)row[n];
    }
  free(row);
}

/*
 * nn.Linear as Kiln compiles it (fx_import.py:140-153 + the frozen, folded
 * W^T of kiln/passes/freeze.py:45-75): out = act(x @ wt + bias) [+ residual],
 * x [M,K], wt [K,N] (N contiguous), bias [N] or NULL, residual [M,N] or NULL,
 * act: 0 none, 1 gelu(tanh), 2 gelu(erf).
 */
KO_API void ko_linear(const float *x, const float *wt, const float *bias, const float *residual, int act, int64_t M,
                      int64_t N, int64_t K, float *out) {
  double *row = (double *)malloc(sizeof(double) * (size_t)(N > 0 ? N : 1));
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t n = 0; n < N; ++n) row[n] = bias ? (double)bias[n] : 0.0;
    for (int64_t k = 0; k < K; ++k) {
      const double a = x[m * K + k];
      const float *w = wt + k * N;
      for (int64_t n = 0; n < N; ++n) row[n] += a * (double)w[n];
    }
    for (int64_t n = 0; n < N; ++n) {
      double v = row[n];
      if (act == 1) v = gelu(v, 1);
      if (act == 2) v = gelu(v, 0);
      if (residual) v += residual[m * N + n];
      out[m * N + n] = (float)v;
    }
  }
  free(row);
}

/*
 * GPT-2 pre-LN block (tests/models/transformer.py:4-28), d = nh * hd:
 *   h = LN1(x); qkv = h @ w_attn + b_attn; per head: att = softmax(q k^T / sqrt(hd)
 *   + mask) with mask[i][j] = -inf for j > i; y = att v; x1 = x + (y @ w_cproj +
 *   b_cproj); out = x1 + (gelu_tanh(LN2(x1) @ w_fc + b_fc) @ w_proj + b_proj).
 * Weights are given transposed ([in, out], as freezing stores them).
 */
KO_API void ko_block(const float *x, int64_t T, int64_t d, int64_t nh, const float *ln1_g, const float *ln1_b,
                     const float *w_attn, const float *b_attn, const float *w_cproj, const float *b_cproj,
                     const float *ln2_g, const float *ln2_b, const float *w_fc, const float *b_fc,
                     const float *w_proj, const float *b_proj, float *out) {
  const int64_t hd = d / nh;
  float *h = (float *)malloc(sizeof(float) * T * d);
  float *qkv = (float *)malloc(sizeof(float) * T * 3 * d);
  float *y = (float *)malloc(sizeof(float) * T * d);
  float *x1 = (float *)malloc(sizeof(float) * T * d);
  float *f = (float *)malloc(sizeof(float) * T * 4 * d);
  double *sc = (double *)malloc(sizeof(double) * T);
  const double scale = 1.0 / sqrt((double)hd);

  ko_layernorm(x, ln1_g, ln1_b, 1e-5, T, d, h);
  ko_linear(h, w_attn, b_attn, NULL, 0, T, 3 * d, d, qkv);
  for (int64_t hh = 0; hh < nh; ++hh) {
    for (int64_t i = 0; i < T; ++i) {
      const float *q = qkv + i * 3 * d + hh * hd;
      double m = -INFINITY;
      for (int64_t j = 0; j <= i; ++j) {
        const float *k = qkv + j * 3 * d + d + hh * hd;
        double s = 0.0;
        for (int64_t c = 0; c < hd; ++c) s += (double)q[c] * (double)k[c];
        sc[j] = s * scale;
        m = fmax(m, sc[j]);
      }
      double z = 0.0;
      for (int64_t j = 0; j <= i; ++j) {
        sc[j] = exp(sc[j] - m);
        z += sc[j];
      }
      for (int64_t c = 0; c < hd; ++c) {
        double acc = 0.0;
        for (int64_t j = 0; j <= i; ++j) acc += sc[j] * (double)qkv[j * 3 * d + 2 * d + hh * hd + c];
        y[i * d + hh * hd + c] = (float)(acc / z);
      }
    }
  }
  ko_linear(y, w_cproj, b_cproj, x, 0, T, d, d, x1);
  ko_layernorm(x1, ln2_g, ln2_b, 1e-5, T, d, h);
  ko_linear(h, w_fc, b_fc, NULL, 1, T, 4 * d, d, f);
  ko_linear(f, w_proj, b_proj, x1, 0, T, d, 4 * d, out);
  free(h), free(qkv), free(y), free(x1), free(f), free(sc);
}
