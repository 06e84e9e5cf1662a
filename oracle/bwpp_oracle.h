/*
 * bwpp_oracle.h -- CPU parity oracle for the libbwpp_hip hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links or calls
 * this code.  Only tests/, __graft_entry__.smoke() and the cpu_baseline leg
 * of bench.py may load it, and only as the checker or the timed CPU
 * baseline -- never as a fallback for the GPU path.
 *
 * Two kinds of functions live here:
 *
 *  1. Restatements of the reference's fp32 CPU kernels
 *     (runtime/cpu/bwpp_cpu_ref.c:4-219).  They keep the reference's per-output
 *     arithmetic order (fp32 accumulators, same summation order, expf/sqrtf,
 *     built with -ffp-contract=off), so their outputs are bit-identical to the
 *     reference's.  Pinned against oracle/_ref (the reference C compiled from
 *     /root/reference by oracle/Makefile) and the committed golden vectors in
 *     tests/golden/.
 *
 *  2. Closed-form extensions the build needs but the reference does not
 *     implement numerically: LayerNorm, scaled/causal batched attention,
 *     reduce_max forward with int32 argmax, one-hot reduce_max grad, and the
 *     autodiff grad ops the reference's graph emits (graph_ir.c:1709-1821).
 *     Each one follows the same fp32 conventions and is pinned by
 *     mathematics (fp64 brute force, finite differences, invariants,
 *     reduction to the reference at the special cases) in tests/.
 *
 * Every function returns 0 on success and -1 on a NULL required pointer or an
 * invalid size, where the reference silently returns
 * (bwpp_cpu_ref.c:104-106, 151-153, 198-200).
 */
#ifndef BWPP_ORACLE_H
#define BWPP_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- restatements of runtime/cpu/bwpp_cpu_ref.c (bit-identical) ---- */

/* bwpp_cpu_ref.c:8-35 (+ SiLU at :4-6) */
int oracle_matmul_f32(const float *a, const float *b, float *c, uint32_t M,
                      uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                      uint32_t ldc, const float *bias, int apply_silu,
                      int apply_bias);

/* bwpp_cpu_ref.c:37-61 */
int oracle_softmax_f32(const float *x, float *y, uint32_t rows, uint32_t cols,
                       uint32_t ld);

/* bwpp_cpu_ref.c:63-90 */
int oracle_rmsnorm_f32(const float *x, float *y, const float *gamma,
                       const float *beta, uint32_t rows, uint32_t cols,
                       uint32_t ld, float eps);

/* bwpp_cpu_ref.c:92-144 (O(M*N*(K+D)) restatement with identical arithmetic) */
int oracle_attention_f32(const float *q, const float *k, const float *v,
                         float *o, uint32_t M, uint32_t N, uint32_t K,
                         uint32_t D, uint32_t ldq, uint32_t ldk, uint32_t ldv,
                         uint32_t ldo);

/* bwpp_cpu_ref.c:146-190 (all tied maxima marked; axis 0 = columns) */
int oracle_reduce_max_mask_f32(const float *x, float *mask, uint32_t rows,
                               uint32_t cols, int axis);

/* bwpp_cpu_ref.c:192-219 (dx = mask * dy broadcast along axis) */
int oracle_reduce_max_grad_mask_f32(const float *mask, const float *dy,
                                    float *dx, uint32_t rows, uint32_t cols,
                                    int axis);

/* ---- closed-form extensions ---- */

/* C = op(A)·op(B) (+bias[col]) (→SiLU), fp32 accumulators in k order.
 * trans_a: A is stored [K x M] (row stride lda); trans_b: B is stored [N x K].
 * With trans_a = trans_b = 0 this is exactly oracle_matmul_f32.  The
 * transposed forms are the GEMMs autodiff emits for matmul
 * (graph_ir.c:1529-1583: dA = dY·B^T, dB = A^T·dY). */
int oracle_matmul_ex_f32(const float *a, const float *b, float *c, uint32_t M,
                         uint32_t N, uint32_t K, uint32_t lda, uint32_t ldb,
                         uint32_t ldc, int trans_a, int trans_b,
                         const float *bias, int apply_silu, int apply_bias);

/* LayerNorm (absent from the reference; ROADMAP.md:14).  Population variance,
 * y = (x - mean) * (1/sqrtf(var + eps)), then *gamma[c], then +beta[c]: the
 * RMSNorm conventions of bwpp_cpu_ref.c:63-90. */
int oracle_layernorm_f32(const float *x, float *y, const float *gamma,
                         const float *beta, uint32_t rows, uint32_t cols,
                         uint32_t ld, float eps);

/* Batched multi-head attention.  For each (b, h) slice this is
 * bwpp_cpu_ref.c:92-144 with the score multiplied by `scale` after the dot
 * product and, when `causal`, keys n > m + (N - M) excluded (bottom-right
 * aligned mask; rows with no visible key produce zeros).  With scale = 1,
 * causal = 0, B = H = 1 it is bit-identical to oracle_attention_f32.
 * Strides are in elements. */
int oracle_attention_bh_f32(const float *q, const float *k, const float *v,
                            float *o, uint32_t B, uint32_t H, uint32_t M,
                            uint32_t N, uint32_t K, uint32_t D, uint32_t ldq,
                            uint32_t ldk, uint32_t ldv, uint32_t ldo,
                            uint64_t q_bs, uint64_t q_hs, uint64_t k_bs,
                            uint64_t k_hs, uint64_t v_bs, uint64_t v_hs,
                            uint64_t o_bs, uint64_t o_hs, float scale,
                            int causal);

/* Per-query log-sum-exp of the scaled, masked scores (natural log; -INF
 * for a query with no visible key).  Contiguous layouts. */
int oracle_attention_lse_f32(const float *q, const float *k, float *lse,
                             uint32_t B, uint32_t H, uint32_t M, uint32_t N,
                             uint32_t K, float scale, int causal);

/* Attention backward (closed form, see the .c): dq, dk, dv from q, k, v
 * and the upstream gradient dout.  Contiguous layouts. */
int oracle_attention_grad_f32(const float *q, const float *k, const float *v,
                              const float *dout, float *dq, float *dk, float *dv,
                              uint32_t B, uint32_t H, uint32_t M, uint32_t N,
                              uint32_t K, uint32_t D, float scale, int causal);

/* reduce_max forward.  axis 1: one value per row; axis 0: one per column.
 * maxv follows the reference's fold (start at -INF, take strictly greater,
 * bwpp_cpu_ref.c:159-165); argmax is the lowest index whose value equals
 * maxv, or -1 when no element does (all NaN, or an empty reduction).
 * Either output may be NULL. */
int oracle_reduce_max_f32(const float *x, float *maxv, int32_t *argmax,
                          uint32_t rows, uint32_t cols, uint32_t ld, int axis);

/* reduce_max grad routed one-hot to the lowest-index maximum.  Pass either x
 * (argmax recomputed) or argmax (saved indices); dy has one value per
 * reduced row (axis 1) or column (axis 0).  dx has leading dimension ld. */
int oracle_reduce_max_grad_f32(const float *x, const int32_t *argmax,
                               const float *dy, float *dx, uint32_t rows,
                               uint32_t cols, uint32_t ld, int axis);

/* silu_grad (graph_ir.c:1709-1720, inputs (x, dY)):
 * s = 1/(1+expf(-x)); dx = dy * (s * (1 + x * (1 - s))). */
int oracle_silu_grad_f32(const float *x, const float *dy, float *dx,
                         uint64_t n);

/* softmax_grad along the last axis (graph_ir.c:1722-1733, inputs (Y, dY)):
 * dot = sum_c dy*y (c order); dx = y * (dy - dot). */
int oracle_softmax_grad_f32(const float *y, const float *dy, float *dx,
                            uint32_t rows, uint32_t cols, uint32_t ld);

/* rmsnorm_grad (graph_ir.c:1735-1789, inputs (X, gamma, dY)):
 * inv = 1/sqrtf(sum x^2/cols + eps); xh = x*inv; g = gamma*dy;
 * m = (sum_c xh*g)/cols; dx = inv * (g - xh*m).
 * dgamma[c] = sum_r dy*xh, dbeta[c] = sum_r dy (r order); either may be NULL.
 * gamma NULL means 1. */
int oracle_rmsnorm_grad_f32(const float *x, const float *gamma,
                            const float *dy, float *dx, float *dgamma,
                            float *dbeta, uint32_t rows, uint32_t cols,
                            uint32_t ld, float eps);

/* reduce_sum over rows (axis 0, out[cols]) or along rows (axis 1, out[rows]),
 * fp32 accumulation in index order (graph_ir.c:1410-1455 reduce_to_shape). */
int oracle_reduce_sum_f32(const float *x, float *out, uint32_t rows,
                          uint32_t cols, uint32_t ld, int axis);

/* f32 -> bf16 round to nearest even (NaN stays a quiet NaN) and back. */
uint16_t oracle_f32_to_bf16(float x);
float oracle_bf16_to_f32(uint16_t h);
void oracle_round_bf16_f32(const float *x, float *y, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* BWPP_ORACLE_H */
