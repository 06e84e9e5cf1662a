/*
 * bwpp_oracle.c -- CPU parity oracle (test infrastructure only; see
 * bwpp_oracle.h).  Build: oracle/Makefile, -std=c11 -O2 -ffp-contract=off.
 *
 * The restated functions keep, for every output element, the exact sequence
 * of fp32 operations of runtime/cpu/bwpp_cpu_ref.c.  Loop nests are reordered
 * only where that leaves each output's operation sequence unchanged (e.g. the
 * matmul runs i-k-j with one fp32 accumulator per output column, which adds
 * the same products in the same k order as the reference's i-j-k loop).
 */
#include "bwpp_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* bwpp_cpu_ref.c:4-6 */
static float oracle_silu(float x) { return x / (1.0f + expf(-x)); }

static int oracle_matmul_core(const float *a, const float *b, float *c,
                              uint32_t M, uint32_t N, uint32_t K,
                              uint32_t lda, uint32_t ldb, uint32_t ldc,
                              int trans_a, int trans_b, const float *bias,
                              int apply_silu, int apply_bias) {
  if (!a || !b || !c) return -1;
  if (N == 0 || M == 0) return 0;
  /* Rows are processed in groups of up to 4 sharing each B row (or, with
   * trans_b, each column run); every output still starts from 0.0f and adds
   * av * b for k = 0, 1, ..., K-1 in that order. */
  enum { RB = 4 };
  float *acc = (float *)malloc(sizeof(float) * (size_t)N * RB);
  if (!acc) return -1;
  for (uint32_t row0 = 0; row0 < M; row0 += RB) {
    const uint32_t nr = M - row0 < RB ? M - row0 : RB;
    for (size_t i = 0; i < (size_t)N * nr; ++i) acc[i] = 0.0f;
    if (!trans_b) {
      for (uint32_t k = 0; k < K; ++k) {
        const float *brow = b + (size_t)k * ldb;
        for (uint32_t r = 0; r < nr; ++r) {
          const uint32_t row = row0 + r;
          const float av = trans_a ? a[(size_t)k * lda + row] : a[(size_t)row * lda + k];
          float *ar = acc + (size_t)r * N;
          for (uint32_t col = 0; col < N; ++col) ar[col] += av * brow[col];
        }
      }
    } else {
      /* B stored [N x K]: a dot product per output over contiguous k. */
      for (uint32_t r = 0; r < nr; ++r) {
        const uint32_t row = row0 + r;
        for (uint32_t col = 0; col < N; ++col) {
          const float *bcol = b + (size_t)col * ldb;
          float s = 0.0f;
          for (uint32_t k = 0; k < K; ++k) {
            const float av = trans_a ? a[(size_t)k * lda + row] : a[(size_t)row * lda + k];
            s += av * bcol[k];
          }
          acc[(size_t)r * N + col] = s;
        }
      }
    }
    for (uint32_t r = 0; r < nr; ++r) {
      float *crow = c + (size_t)(row0 + r) * ldc;
      const float *ar = acc + (size_t)r * N;
      for (uint32_t col = 0; col < N; ++col) {
        float v = ar[col];
        if (apply_bias && bias) v += bias[col]; /* bwpp_cpu_ref.c:26-28 */
        if (apply_silu) v = oracle_silu(v);     /* bwpp_cpu_ref.c:29-31 */
        crow[col] = v;
      }
    }
  }
  free(acc);
  return 0;
}

int oracle_matmul_f32(const float *a, const float *b, float *c, uint32_t M,
                      uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                      uint32_t ldc, const float *bias, int apply_silu,
                      int apply_bias) {
  return oracle_matmul_core(a, b, c, M, N, K, lda, ldb, ldc, 0, 0, bias,
                            apply_silu, apply_bias);
}

int oracle_matmul_ex_f32(const float *a, const float *b, float *c, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                         uint32_t ldc, int trans_a, int trans_b,
                         const float *bias, int apply_silu, int apply_bias) {
  return oracle_matmul_core(a, b, c, M, N, K, lda, ldb, ldc, trans_a, trans_b,
                            bias, apply_silu, apply_bias);
}

/* bwpp_cpu_ref.c:37-61: max pass, exp+sum pass (unnormalised exp stored in
 * y), scale pass with inv = sum > 0 ? 1/sum : 0. */
int oracle_softmax_f32(const float *x, float *y, uint32_t rows, uint32_t cols,
                       uint32_t ld) {
  if (!x || !y) return -1;
  for (uint32_t r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * ld;
    float *yr = y + (size_t)r * ld;
    float maxv = -INFINITY;
    for (uint32_t c = 0; c < cols; ++c) {
      if (xr[c] > maxv) maxv = xr[c];
    }
    float sum = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) {
      float e = expf(xr[c] - maxv);
      yr[c] = e;
      sum += e;
    }
    float inv = sum > 0.0f ? (1.0f / sum) : 0.0f;
    for (uint32_t c = 0; c < cols; ++c) yr[c] *= inv;
  }
  return 0;
}

/* bwpp_cpu_ref.c:63-90 */
int oracle_rmsnorm_f32(const float *x, float *y, const float *gamma,
                       const float *beta, uint32_t rows, uint32_t cols,
                       uint32_t ld, float eps) {
  if (!x || !y) return -1;
  for (uint32_t r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * ld;
    float *yr = y + (size_t)r * ld;
    float sumsq = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) sumsq += xr[c] * xr[c];
    float mean = sumsq / (float)cols;
    float inv = 1.0f / sqrtf(mean + eps);
    for (uint32_t c = 0; c < cols; ++c) {
      float v = xr[c] * inv;
      if (gamma) v *= gamma[c];
      if (beta) v += beta[c];
      yr[c] = v;
    }
  }
  return 0;
}

int oracle_layernorm_f32(const float *x, float *y, const float *gamma,
                         const float *beta, uint32_t rows, uint32_t cols,
                         uint32_t ld, float eps) {
  if (!x || !y) return -1;
  for (uint32_t r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * ld;
    float *yr = y + (size_t)r * ld;
    float sum = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) sum += xr[c];
    float mean = sum / (float)cols;
    float sumsq = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) {
      float d = xr[c] - mean;
      sumsq += d * d;
    }
    float var = sumsq / (float)cols;
    float inv = 1.0f / sqrtf(var + eps);
    for (uint32_t c = 0; c < cols; ++c) {
      float v = (xr[c] - mean) * inv;
      if (gamma) v *= gamma[c];
      if (beta) v += beta[c];
      yr[c] = v;
    }
  }
  return 0;
}

/* One attention slice.  Scores s_n = (sum_kk q*k in kk order) * scale are
 * computed once; the reference recomputes the identical value 2+D times
 * (bwpp_cpu_ref.c:110-140), so caching it changes no bit.  Then
 * max (strictly greater from -INF), sum of expf(s-max) in n order,
 * inv = sum > 0 ? 1/sum : 0, w_n = expf(s_n-max)*inv, out_d = sum_n w_n*v[n,d]
 * in n order. */
static void oracle_attention_slice(const float *q, const float *k,
                                   const float *v, float *o, uint32_t M,
                                   uint32_t N, uint32_t K, uint32_t D,
                                   uint32_t ldq, uint32_t ldk, uint32_t ldv,
                                   uint32_t ldo, float scale, int causal,
                                   float *s, float *out) {
  for (uint32_t m = 0; m < M; ++m) {
    const float *qm = q + (size_t)m * ldq;
    /* visible keys: n <= m + (N - M) when causal */
    int64_t last = causal ? (int64_t)m + (int64_t)N - (int64_t)M : (int64_t)N - 1;
    if (last > (int64_t)N - 1) last = (int64_t)N - 1;
    uint32_t nvis = last < 0 ? 0u : (uint32_t)(last + 1);
    float maxv = -INFINITY;
    for (uint32_t n = 0; n < nvis; ++n) {
      const float *kn = k + (size_t)n * ldk;
      float acc = 0.0f;
      for (uint32_t kk = 0; kk < K; ++kk) acc += qm[kk] * kn[kk];
      acc = acc * scale;
      s[n] = acc;
      if (acc > maxv) maxv = acc;
    }
    float sum = 0.0f;
    for (uint32_t n = 0; n < nvis; ++n) sum += expf(s[n] - maxv);
    float inv = sum > 0.0f ? (1.0f / sum) : 0.0f;
    for (uint32_t d = 0; d < D; ++d) out[d] = 0.0f;
    for (uint32_t n = 0; n < nvis; ++n) {
      float w = expf(s[n] - maxv) * inv;
      const float *vn = v + (size_t)n * ldv;
      for (uint32_t d = 0; d < D; ++d) out[d] += w * vn[d];
    }
    float *om = o + (size_t)m * ldo;
    for (uint32_t d = 0; d < D; ++d) om[d] = out[d];
  }
}

int oracle_attention_f32(const float *q, const float *k, const float *v,
                         float *o, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t D, uint32_t ldq, uint32_t ldk, uint32_t ldv,
                         uint32_t ldo) {
  return oracle_attention_bh_f32(q, k, v, o, 1, 1, M, N, K, D, ldq, ldk, ldv,
                                 ldo, 0, 0, 0, 0, 0, 0, 0, 0, 1.0f, 0);
}

int oracle_attention_bh_f32(const float *q, const float *k, const float *v,
                            float *o, uint32_t B, uint32_t H, uint32_t M,
                            uint32_t N, uint32_t K, uint32_t D, uint32_t ldq,
                            uint32_t ldk, uint32_t ldv, uint32_t ldo,
                            uint64_t q_bs, uint64_t q_hs, uint64_t k_bs,
                            uint64_t k_hs, uint64_t v_bs, uint64_t v_hs,
                            uint64_t o_bs, uint64_t o_hs, float scale,
                            int causal) {
  if (!q || !k || !v || !o) return -1;
  float *s = (float *)malloc(sizeof(float) * ((size_t)N + 1));
  float *out = (float *)malloc(sizeof(float) * ((size_t)D + 1));
  if (!s || !out) {
    free(s);
    free(out);
    return -1;
  }
  for (uint32_t b = 0; b < B; ++b) {
    for (uint32_t h = 0; h < H; ++h) {
      oracle_attention_slice(q + b * q_bs + h * q_hs, k + b * k_bs + h * k_hs,
                             v + b * v_bs + h * v_hs, o + b * o_bs + h * o_hs,
                             M, N, K, D, ldq, ldk, ldv, ldo, scale, causal, s,
                             out);
    }
  }
  free(s);
  free(out);
  return 0;
}

/* Log-sum-exp of each query's scaled, masked scores (natural log):
 * lse[m] = max + logf(sum_n expf(s_n - max)), -INFINITY when no key is
 * visible.  Contiguous [B,H,M,K] / [B,H,N,K] layouts.  Extension (no
 * reference counterpart): the saved statistic of the attention backward. */
int oracle_attention_lse_f32(const float *q, const float *k, float *lse,
                             uint32_t B, uint32_t H, uint32_t M, uint32_t N,
                             uint32_t K, float scale, int causal) {
  if (!q || !k || !lse) return -1;
  float *s = (float *)malloc(sizeof(float) * ((size_t)N + 1));
  if (!s) return -1;
  for (uint32_t bh = 0; bh < B * H; ++bh) {
    const float *qs = q + (size_t)bh * M * K, *ks = k + (size_t)bh * N * K;
    for (uint32_t m = 0; m < M; ++m) {
      int64_t last = causal ? (int64_t)m + (int64_t)N - (int64_t)M : (int64_t)N - 1;
      if (last > (int64_t)N - 1) last = (int64_t)N - 1;
      uint32_t nvis = last < 0 ? 0u : (uint32_t)(last + 1);
      float maxv = -INFINITY;
      for (uint32_t n = 0; n < nvis; ++n) {
        float acc = 0.0f;
        for (uint32_t kk = 0; kk < K; ++kk) acc += qs[(size_t)m * K + kk] * ks[(size_t)n * K + kk];
        s[n] = acc * scale;
        if (s[n] > maxv) maxv = s[n];
      }
      float sum = 0.0f;
      for (uint32_t n = 0; n < nvis; ++n) sum += expf(s[n] - maxv);
      lse[(size_t)bh * M + m] = nvis ? maxv + logf(sum) : -INFINITY;
    }
  }
  free(s);
  return 0;
}

/* Attention backward for O = softmax(scale Q K^T [causal]) V, closed form
 * per (b, h) slice with P the softmax probabilities (masked keys 0):
 *   dV = P^T dO,  dP = dO V^T,  dS = P * (dP - rowsum(dP * P)),
 *   dQ = scale dS K,  dK = scale dS^T Q.
 * Contiguous [B,H,M,K] q / dq, [B,H,N,K] k / dk, [B,H,N,D] v / dv,
 * [B,H,M,D] dout.  fp32, loops in index order.  Extension: the reference
 * differentiates attention only through its decomposed graph ops
 * (graph_ir.c:1722-1733, 1529-1583). */
int oracle_attention_grad_f32(const float *q, const float *k, const float *v,
                              const float *dout, float *dq, float *dk, float *dv,
                              uint32_t B, uint32_t H, uint32_t M, uint32_t N,
                              uint32_t K, uint32_t D, float scale, int causal) {
  if (!q || !k || !v || !dout || !dq || !dk || !dv) return -1;
  float *p = (float *)malloc(sizeof(float) * ((size_t)N + 1));
  float *ds = (float *)malloc(sizeof(float) * ((size_t)N + 1));
  if (!p || !ds) {
    free(p);
    free(ds);
    return -1;
  }
  for (uint32_t bh = 0; bh < B * H; ++bh) {
    const float *qs = q + (size_t)bh * M * K, *ks = k + (size_t)bh * N * K;
    const float *vs = v + (size_t)bh * N * D, *dos = dout + (size_t)bh * M * D;
    float *dqs = dq + (size_t)bh * M * K, *dks = dk + (size_t)bh * N * K, *dvs = dv + (size_t)bh * N * D;
    for (size_t i = 0; i < (size_t)N * K; ++i) dks[i] = 0.0f;
    for (size_t i = 0; i < (size_t)N * D; ++i) dvs[i] = 0.0f;
    for (uint32_t m = 0; m < M; ++m) {
      int64_t last = causal ? (int64_t)m + (int64_t)N - (int64_t)M : (int64_t)N - 1;
      if (last > (int64_t)N - 1) last = (int64_t)N - 1;
      uint32_t nvis = last < 0 ? 0u : (uint32_t)(last + 1);
      const float *qm = qs + (size_t)m * K, *dom = dos + (size_t)m * D;
      float maxv = -INFINITY;
      for (uint32_t n = 0; n < nvis; ++n) {
        float acc = 0.0f;
        for (uint32_t kk = 0; kk < K; ++kk) acc += qm[kk] * ks[(size_t)n * K + kk];
        p[n] = acc * scale;
        if (p[n] > maxv) maxv = p[n];
      }
      float sum = 0.0f;
      for (uint32_t n = 0; n < nvis; ++n) sum += expf(p[n] - maxv);
      float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
      float rowdot = 0.0f; /* rowsum(dP * P) */
      for (uint32_t n = 0; n < nvis; ++n) {
        p[n] = expf(p[n] - maxv) * inv;
        float dp = 0.0f;
        for (uint32_t d = 0; d < D; ++d) dp += dom[d] * vs[(size_t)n * D + d];
        ds[n] = dp;
        rowdot += dp * p[n];
      }
      for (uint32_t kk = 0; kk < K; ++kk) dqs[(size_t)m * K + kk] = 0.0f;
      for (uint32_t n = 0; n < nvis; ++n) {
        const float dsn = p[n] * (ds[n] - rowdot);
        for (uint32_t kk = 0; kk < K; ++kk) {
          dqs[(size_t)m * K + kk] += scale * dsn * ks[(size_t)n * K + kk];
          dks[(size_t)n * K + kk] += scale * dsn * qm[kk];
        }
        for (uint32_t d = 0; d < D; ++d) dvs[(size_t)n * D + d] += p[n] * dom[d];
      }
    }
  }
  free(p);
  free(ds);
  return 0;
}

/* bwpp_cpu_ref.c:146-190 */
int oracle_reduce_max_mask_f32(const float *x, float *mask, uint32_t rows,
                               uint32_t cols, int axis) {
  if (!x || !mask) return -1;
  const size_t total = (size_t)rows * cols;
  for (size_t i = 0; i < total; ++i) mask[i] = 0.0f;
  if (axis == 0) {
    for (uint32_t c = 0; c < cols; ++c) {
      float maxv = -INFINITY;
      for (uint32_t r = 0; r < rows; ++r) {
        float v = x[(size_t)r * cols + c];
        if (v > maxv) maxv = v;
      }
      for (uint32_t r = 0; r < rows; ++r) {
        if (x[(size_t)r * cols + c] == maxv) mask[(size_t)r * cols + c] = 1.0f;
      }
    }
  } else {
    for (uint32_t r = 0; r < rows; ++r) {
      float maxv = -INFINITY;
      for (uint32_t c = 0; c < cols; ++c) {
        float v = x[(size_t)r * cols + c];
        if (v > maxv) maxv = v;
      }
      for (uint32_t c = 0; c < cols; ++c) {
        if (x[(size_t)r * cols + c] == maxv) mask[(size_t)r * cols + c] = 1.0f;
      }
    }
  }
  return 0;
}

/* bwpp_cpu_ref.c:192-219 */
int oracle_reduce_max_grad_mask_f32(const float *mask, const float *dy,
                                    float *dx, uint32_t rows, uint32_t cols,
                                    int axis) {
  if (!mask || !dy || !dx) return -1;
  if (axis == 0) {
    for (uint32_t r = 0; r < rows; ++r)
      for (uint32_t c = 0; c < cols; ++c)
        dx[(size_t)r * cols + c] = mask[(size_t)r * cols + c] * dy[c];
  } else {
    for (uint32_t r = 0; r < rows; ++r) {
      float g = dy[r];
      for (uint32_t c = 0; c < cols; ++c)
        dx[(size_t)r * cols + c] = mask[(size_t)r * cols + c] * g;
    }
  }
  return 0;
}

/* Fold of bwpp_cpu_ref.c:159-165 over one line of n elements at stride st,
 * plus the lowest index equal to the result. */
static void oracle_max_line(const float *x, uint32_t n, size_t st, float *out_max,
                            int32_t *out_idx) {
  float maxv = -INFINITY;
  for (uint32_t i = 0; i < n; ++i) {
    float v = x[(size_t)i * st];
    if (v > maxv) maxv = v;
  }
  int32_t idx = -1;
  for (uint32_t i = 0; i < n; ++i) {
    if (x[(size_t)i * st] == maxv) {
      idx = (int32_t)i;
      break;
    }
  }
  *out_max = maxv;
  *out_idx = idx;
}

int oracle_reduce_max_f32(const float *x, float *maxv, int32_t *argmax,
                          uint32_t rows, uint32_t cols, uint32_t ld, int axis) {
  if (!x) return -1;
  if (axis == 0) {
    for (uint32_t c = 0; c < cols; ++c) {
      float m;
      int32_t i;
      oracle_max_line(x + c, rows, ld, &m, &i);
      if (maxv) maxv[c] = m;
      if (argmax) argmax[c] = i;
    }
  } else {
    for (uint32_t r = 0; r < rows; ++r) {
      float m;
      int32_t i;
      oracle_max_line(x + (size_t)r * ld, cols, 1, &m, &i);
      if (maxv) maxv[r] = m;
      if (argmax) argmax[r] = i;
    }
  }
  return 0;
}

int oracle_reduce_max_grad_f32(const float *x, const int32_t *argmax,
                               const float *dy, float *dx, uint32_t rows,
                               uint32_t cols, uint32_t ld, int axis) {
  if ((!x && !argmax) || !dy || !dx) return -1;
  for (uint32_t r = 0; r < rows; ++r)
    for (uint32_t c = 0; c < cols; ++c) dx[(size_t)r * ld + c] = 0.0f;
  const uint32_t lines = axis == 0 ? cols : rows;
  for (uint32_t l = 0; l < lines; ++l) {
    int32_t idx;
    if (argmax) {
      idx = argmax[l];
    } else {
      float m;
      if (axis == 0)
        oracle_max_line(x + l, rows, ld, &m, &idx);
      else
        oracle_max_line(x + (size_t)l * ld, cols, 1, &m, &idx);
    }
    if (idx < 0) continue;
    if (axis == 0) {
      if ((uint32_t)idx < rows) dx[(size_t)idx * ld + l] = dy[l];
    } else {
      if ((uint32_t)idx < cols) dx[(size_t)l * ld + (uint32_t)idx] = dy[l];
    }
  }
  return 0;
}

int oracle_silu_grad_f32(const float *x, const float *dy, float *dx,
                         uint64_t n) {
  if (!x || !dy || !dx) return -1;
  for (uint64_t i = 0; i < n; ++i) {
    float s = 1.0f / (1.0f + expf(-x[i]));
    dx[i] = dy[i] * (s * (1.0f + x[i] * (1.0f - s)));
  }
  return 0;
}

int oracle_softmax_grad_f32(const float *y, const float *dy, float *dx,
                            uint32_t rows, uint32_t cols, uint32_t ld) {
  if (!y || !dy || !dx) return -1;
  for (uint32_t r = 0; r < rows; ++r) {
    const float *yr = y + (size_t)r * ld;
    const float *gr = dy + (size_t)r * ld;
    float *dr = dx + (size_t)r * ld;
    float dot = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) dot += gr[c] * yr[c];
    for (uint32_t c = 0; c < cols; ++c) dr[c] = yr[c] * (gr[c] - dot);
  }
  return 0;
}

int oracle_rmsnorm_grad_f32(const float *x, const float *gamma,
                            const float *dy, float *dx, float *dgamma,
                            float *dbeta, uint32_t rows, uint32_t cols,
                            uint32_t ld, float eps) {
  if (!x || !dy || !dx) return -1;
  if (dgamma)
    for (uint32_t c = 0; c < cols; ++c) dgamma[c] = 0.0f;
  if (dbeta)
    for (uint32_t c = 0; c < cols; ++c) dbeta[c] = 0.0f;
  for (uint32_t r = 0; r < rows; ++r) {
    const float *xr = x + (size_t)r * ld;
    const float *gr = dy + (size_t)r * ld;
    float *dr = dx + (size_t)r * ld;
    float sumsq = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) sumsq += xr[c] * xr[c];
    float inv = 1.0f / sqrtf(sumsq / (float)cols + eps);
    float dot = 0.0f;
    for (uint32_t c = 0; c < cols; ++c) {
      float g = gamma ? gamma[c] * gr[c] : gr[c];
      dot += (xr[c] * inv) * g;
    }
    float mdot = dot / (float)cols;
    for (uint32_t c = 0; c < cols; ++c) {
      float xh = xr[c] * inv;
      float g = gamma ? gamma[c] * gr[c] : gr[c];
      dr[c] = inv * (g - xh * mdot);
      if (dgamma) dgamma[c] += gr[c] * xh;
      if (dbeta) dbeta[c] += gr[c];
    }
  }
  return 0;
}

int oracle_reduce_sum_f32(const float *x, float *out, uint32_t rows,
                          uint32_t cols, uint32_t ld, int axis) {
  if (!x || !out) return -1;
  if (axis == 0) {
    for (uint32_t c = 0; c < cols; ++c) out[c] = 0.0f;
    for (uint32_t r = 0; r < rows; ++r)
      for (uint32_t c = 0; c < cols; ++c) out[c] += x[(size_t)r * ld + c];
  } else {
    for (uint32_t r = 0; r < rows; ++r) {
      float s = 0.0f;
      for (uint32_t c = 0; c < cols; ++c) s += x[(size_t)r * ld + c];
      out[r] = s;
    }
  }
  return 0;
}

uint16_t oracle_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, sizeof u);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float oracle_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, sizeof f);
  return f;
}

void oracle_round_bf16_f32(const float *x, float *y, uint64_t n) {
  for (uint64_t i = 0; i < n; ++i) y[i] = oracle_bf16_to_f32(oracle_f32_to_bf16(x[i]));
}
