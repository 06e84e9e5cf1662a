/* Kernel argument blocks shared by the host runtime (g++) and the gfx950
 * kernels (hipcc).  Each kernel takes exactly one of these by value, so a
 * launch passes a single kernelParams entry to hipModuleLaunchKernel.
 * Plain C layout only: no HIP or C++ types. */
#ifndef BWPP_KARGS_H
#define BWPP_KARGS_H

#include <stdint.h>

/* Row-wise and column-wise reductions and their grads. */
typedef struct {
  const float *x;
  float *y; /* output rows (softmax/norm output, mask, dx) */
  const float *gamma;
  const float *beta;
  const float *dy; /* upstream grad: per line (reduce_max) or per element */
  const int32_t *idx_in;
  float *maxv;
  int32_t *argmax;
  float *dgamma; /* rmsnorm_grad partials */
  float *dbeta;
  uint32_t rows;
  uint32_t cols;
  uint32_t ld;
  float eps;
} BwppRowArgs;

/* GEMM: C = op(A)·op(B) (+bias) (->SiLU); see gemm.hip. */
typedef struct {
  const void *a;
  const void *b;
  const void *bias; /* NULL: no bias even if the epilogue asks for one */
  void *c;
  uint32_t M;
  uint32_t N;
  uint32_t K;
  uint32_t lda;
  uint32_t ldb;
  uint32_t ldc;
  uint32_t epilogue; /* BWPP_HIP_EPILOGUE_* values */
  uint32_t tiles_m;  /* ceil(M / BM) */
  uint32_t tiles_n;  /* ceil(N / BN) */
  uint32_t group_m;  /* tile-order group height (in tiles) */
  uint32_t vec_ok;   /* 1: rows are 16-byte aligned (edge kernels only) */
  /* Split-K (fp32 full tiles): block b computes K range [s * kchunk, ..)
   * of tile b % tiles for s = b / tiles into part[s] ([M][N] raw sums);
   * bwpp_gemm_f32_splitk_reduce then applies the epilogue. */
  uint32_t ksplit;
  uint32_t kchunk;
  float *part;
  /* fp32 fusions after the epilogue (BWPP_HIP_FUSE_*): residual C += aux,
   * dual output c2 = SiLU(C), SiLU gradient C *= silu'(aux) */
  uint32_t fuse;
  uint32_t ldaux;
  const float *aux;
  float *c2;
  uint32_t ldc2;
} BwppGemmArgs;

/* Attention: O = softmax(scale * Q K^T [causal]) V per (batch, head). */
typedef struct {
  const void *q;
  const void *k;
  const void *v;
  void *o;
  uint32_t M; /* queries */
  uint32_t N; /* keys */
  uint32_t ldq, ldk, ldv, ldo;
  uint32_t heads;
  uint32_t q_tiles; /* ceil(M / queries per block) */
  uint64_t q_bs, q_hs, k_bs, k_hs, v_bs, v_hs, o_bs, o_hs;
  float scale_log2; /* scale * log2(e) (flash path); the plain scale (generic path) */
  uint32_t causal;
  uint32_t kdim; /* Q/K head dim (generic path) */
  uint32_t vdim; /* V/O head dim (generic path) */
  /* Forward: optional per-query log-sum-exp out ([B*H][M] fp32).
   * Backward: lse in, dout (O's strides), dq / dk / dv (Q / K / V strides),
   * dsum = rowsum(dout * o) scratch ([B*H][M] fp32). */
  float *lse;
  const void *dout;
  void *dq;
  void *dk;
  void *dv;
  float *dsum;
  float scale; /* the plain score scale (fp32 MFMA path, which gets scale * log2(e) in scale_log2) */
  uint32_t zigzag; /* fp32 MFMA causal kernels: tile order heavy ranks first, then the light ones
                      lightest first (a one-wave grid then pairs heavy with light on each CU) */
  /* Backward with a stored dS: dS^T written by the dK/dV pass and read by
   * the dQ pass, in blocks of 32 keys x 32 queries (bf16: DsBlk in
   * attention_bwd.hip, fp32: DsBlk32 in attention_f32.hip); ld_dst = the
   * query count rounded up to 128. */
  void *dst;
  uint32_t ld_dst;
  uint32_t items; /* persistent flash forward: (slice, query tile) items */
} BwppAttnArgs;

/* Attention operand copies between the caller's strided bf16 layout
 * ([batch][head] slices of rows x cols, leading dimension ld) and
 * contiguous fp32 [batch * heads][rows][cols] (attention_f32.hip). */
typedef struct {
  const void *src;
  void *dst;
  uint64_t bs, hs;   /* batch / head strides of the bf16 side (elements) */
  uint32_t rows, cols, ld, heads;
  uint32_t slices;   /* batch * heads */
  uint32_t vec;      /* 1: bf16 rows are 16-byte aligned (8-element loads / stores) */
} BwppConvArgs;

/* Grad ops and elementwise glue (grad.hip). */
typedef struct {
  const float *a;   /* x, y or the left operand */
  const float *b;   /* dy or the right operand */
  const float *gamma;
  float *out;       /* dx or the result */
  float *out2;      /* dbeta (bwpp_col_partials_sum) */
  float *part_g;    /* [nblocks][cols] dgamma partials (rmsnorm_grad) */
  float *part_b;    /* [nblocks][cols] dbeta partials */
  uint64_t n;       /* element count (flat ops) */
  uint32_t rows;
  uint32_t cols;
  uint32_t ld;
  float eps;
  uint32_t op;      /* elementwise op */
  uint32_t bmode;   /* broadcast of b: 0 full, 1 row vector [cols], 2 column vector [rows], 3 scalar */
  uint32_t nparts;  /* partial rows to reduce */
  uint32_t vec;     /* 1: a, b, out are 16-byte aligned (flat ops); 16-byte
                       rows (elementwise) */
  uint32_t ldb;     /* elementwise, full broadcast: row stride of b */
  const float *acc; /* rmsnorm_grad: added to dx (row stride ld; may equal out) */
  const float *s_loss, *s_grad; /* mean_square: device scalars (NULL = 1) */
} BwppGradArgs;

/* Up to four strided copies in one launch (bwpp_copy_multi): segment s
 * copies rows row0[s] .. row0[s+1]-1 of the launch's row space. */
#define BWPP_COPY_MULTI_MAX 4
typedef struct {
  const float *src[BWPP_COPY_MULTI_MAX];
  float *dst[BWPP_COPY_MULTI_MAX];
  uint32_t ld_src[BWPP_COPY_MULTI_MAX], ld_dst[BWPP_COPY_MULTI_MAX], cols[BWPP_COPY_MULTI_MAX];
  uint32_t row0[BWPP_COPY_MULTI_MAX + 1];
  uint32_t n;   /* segments */
  uint32_t vec; /* 1: every segment has 16-byte rows (cols, strides, pointers) */
} BwppCopyArgs;

#endif /* BWPP_KARGS_H */
