/*
 * bwpp_hip.h -- C ABI of libbwpp_hip, the MI355X (gfx950) execution backend
 * for BW++'s hot ops.
 *
 * It replaces the reference's Metal operator seam
 * (runtime/metal/dispatch_stub.h:42-74, implemented in dispatch_stub.m) and
 * gives runtime/core's arena (runtime/core/arena.h:6-15) a device-memory
 * twin.  Kernels are hand-written gfx950 HIP, prebuilt into code objects
 * (*.hsaco) that bwpp_hip_create() loads with hipModuleLoad; every operator
 * launches with hipModuleLaunchKernel on the handle's stream.
 *
 * Conventions (kept from the reference):
 *  - the caller owns every buffer; pointers are device pointers unless a
 *    function says otherwise;
 *  - row-major with explicit leading dimensions (in elements); softmax and
 *    the norms run along the last axis;
 *  - a NULL gamma / beta / bias means 1 / 0 / 0 (dispatch_stub.m:103-110,
 *    215-234);
 *  - the params structs keep the reference's type names and leading fields,
 *    in the reference's order (dispatch_stub.h:9-40); fields added after them
 *    take their documented default when zero, so a reference-style
 *    initialiser `{M, N, K, lda, ldb, ldc}` keeps its meaning.
 * Differences:
 *  - every call returns a status instead of returning silently on bad
 *    arguments (dispatch_stub.m:66-79); a failed call launches nothing;
 *  - launches are asynchronous on the handle's stream; bwpp_hip_sync() waits
 *    (the reference waits inside every dispatch, dispatch_stub.m:139-140);
 *  - the function cache is filled once in bwpp_hip_create() and read-only
 *    afterwards (the reference's function-static PSO caches are not
 *    thread-safe, dispatch_stub.m:81), but a handle also holds its stream,
 *    its last-error text and the grad ops' workspace: use one handle per
 *    host thread, or serialise calls on a shared one.
 */
#ifndef BWPP_HIP_H
#define BWPP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 0 and 1 coincide with the reference's BwppStatus {BWPP_OK, BWPP_ERR}
 * (compiler/include/bwpp.h:8-11); the rest refine BWPP_ERR. */
typedef enum {
  BWPP_HIP_OK = 0,
  BWPP_HIP_ERR = 1,
  BWPP_HIP_ERR_INVALID_ARG = 2,   /* NULL pointer, bad size, ld < cols, ... */
  BWPP_HIP_ERR_HIP = 3,           /* a HIP runtime call failed */
  BWPP_HIP_ERR_NO_KERNEL = 4,     /* code object or kernel symbol missing */
  BWPP_HIP_ERR_ALIAS = 5,         /* GEMM/attention output overlaps an input */
  BWPP_HIP_ERR_OUT_OF_MEMORY = 6, /* device allocation or arena exhausted */
  BWPP_HIP_ERR_UNSUPPORTED = 7,   /* valid request this build does not run */
  BWPP_HIP_ERR_NO_DEVICE = 8      /* no usable HIP device */
} BwppHipStatus;

typedef enum { BWPP_HIP_F32 = 0, BWPP_HIP_BF16 = 1 } BwppHipDType;

/* Same values as BwppTileEpilogue (compiler/include/tile_ir.h:35-40). */
typedef enum {
  BWPP_HIP_EPILOGUE_NONE = 0,
  BWPP_HIP_EPILOGUE_ADD = 1,
  BWPP_HIP_EPILOGUE_SILU = 2,
  BWPP_HIP_EPILOGUE_ADD_SILU = 3
} BwppHipEpilogue;

/* dispatch_stub.h:9-16 + extensions.
 * C = op(A)·op(B) (+bias[col]) (→SiLU).  A is [M x K] (trans_a: stored
 * [K x M]), B is [K x N] (trans_b: stored [N x K]); lda/ldb/ldc are the row
 * strides of the stored matrices.  dtype F32: fp32 in/out on FP32 MFMA;
 * BF16: bf16 A, B, bias and C with fp32 accumulation and epilogue, C rounded
 * to nearest even.  bias is read only when the epilogue includes ADD. */
typedef struct {
  uint32_t M;
  uint32_t N;
  uint32_t K;
  uint32_t lda;
  uint32_t ldb;
  uint32_t ldc;
  uint32_t dtype;    /* BwppHipDType, 0 = F32 */
  uint32_t epilogue; /* BwppHipEpilogue, 0 = none */
  uint32_t trans_a;  /* 0 = A row-major [M x K] */
  uint32_t trans_b;  /* 0 = B row-major [K x N] */
} BwppMatmulParams;

/* dispatch_stub.h:18-22.  ld is the row stride of x and y (0 = cols). */
typedef struct {
  uint32_t rows;
  uint32_t cols;
  uint32_t ld;
} BwppSoftmaxParams;

/* dispatch_stub.h:24-29; also used by LayerNorm and the norm grads.
 * ld is the row stride of x, y and dy (0 = cols). */
typedef struct {
  uint32_t rows;
  uint32_t cols;
  uint32_t ld;
  float eps;
} BwppRmsnormParams;

/* dispatch_stub.h:31-40 + extensions.  One (batch, head) slice is the
 * reference's single-head problem: Q [M x K], K [N x K], V [N x D],
 * O [M x D] with row strides ldq/ldk/ldv/ldo; slices are placed by the
 * batch/head strides (elements).  O = softmax(scale * Q·K^T [masked]) · V.
 * causal masks keys n > m + (N - M) (bottom-right aligned; rows that see no
 * key produce zeros).  dtype BF16: bf16 Q/K/V/O, fp32 softmax and
 * accumulation; F32: fp32 throughout. */
typedef struct {
  uint32_t M;
  uint32_t N;
  uint32_t K;
  uint32_t D;
  uint32_t ldq;
  uint32_t ldk;
  uint32_t ldv;
  uint32_t ldo;
  uint32_t batch; /* 0 = 1 */
  uint32_t heads; /* 0 = 1 */
  uint64_t q_batch_stride, q_head_stride;
  uint64_t k_batch_stride, k_head_stride;
  uint64_t v_batch_stride, v_head_stride;
  uint64_t o_batch_stride, o_head_stride;
  float scale;     /* 0 = 1.0: the reference applies no scale */
  uint32_t causal; /* 0 = unmasked, as the reference */
  uint32_t dtype;  /* BwppHipDType, 0 = F32 */
} BwppAttentionParams;

/* reduce_max family.  axis follows bwpp_cpu_ref.c:156,172: axis == 0 reduces
 * over rows (one result per column), any other value reduces along each row
 * (one result per row). */
typedef struct {
  uint32_t rows;
  uint32_t cols;
  uint32_t ld; /* row stride of x / mask / dx; 0 = cols */
  int32_t axis;
} BwppReduceParams;

/* Elementwise glue of the autodiff graph (graph_ir.c:697-770, 1457-1470,
 * 1585-1654): out = a (op) b with b broadcast as selected; op COPY writes
 * the broadcast b and op SILU its SiLU b / (1 + expf(-b)) (graph op
 * BWPP_GOP_SILU, bwpp_cpu_ref.c:4-6; a unused for both).  rows x cols with
 * leading dimension ld (0 = cols) for a, out and a full b. */
typedef enum {
  BWPP_HIP_OP_ADD = 0,
  BWPP_HIP_OP_SUB = 1,
  BWPP_HIP_OP_MUL = 2,
  BWPP_HIP_OP_DIV = 3,
  BWPP_HIP_OP_COPY = 4,
  BWPP_HIP_OP_SILU = 5
} BwppHipElementwiseOp;
typedef enum {
  BWPP_HIP_BCAST_FULL = 0,   /* b is rows x cols */
  BWPP_HIP_BCAST_ROW = 1,    /* b[cols], repeated for every row */
  BWPP_HIP_BCAST_COL = 2,    /* b[rows], repeated along each row */
  BWPP_HIP_BCAST_SCALAR = 3  /* b[0] */
} BwppHipBroadcast;
typedef struct {
  uint32_t rows;
  uint32_t cols;
  uint32_t ld;
  uint32_t op;    /* BwppHipElementwiseOp */
  uint32_t bmode; /* BwppHipBroadcast */
} BwppElementwiseParams;

typedef struct BwppHip BwppHip;

/* ---- handle ---- */

/* Selects `device`, loads every code object from code_object_dir (NULL: the
 * directory holding libbwpp_hip.so) and resolves every kernel.  Fails with
 * NO_DEVICE / NO_KERNEL / HIP rather than returning a half-built handle.
 * Replaces the per-op PSO cache (dispatch_stub.m:6-56). */
BwppHipStatus bwpp_hip_create(BwppHip **out, int device,
                              const char *code_object_dir);
void bwpp_hip_destroy(BwppHip *h);
/* Stream for subsequent launches (a hipStream_t); NULL = the null stream.
 * The handle's workspace (split-K partials, attention-backward row sums,
 * column partials) is ordered on the handle's stream: when the stream
 * changes, the new stream first waits for the work queued on the old one. */
BwppHipStatus bwpp_hip_set_stream(BwppHip *h, void *hip_stream);
void *bwpp_hip_get_stream(const BwppHip *h);
/* Waits for all work on the handle's stream. */
BwppHipStatus bwpp_hip_sync(BwppHip *h);
/* Text of the last failure on this handle ("" if none). */
const char *bwpp_hip_last_error(const BwppHip *h);
const char *bwpp_hip_status_string(BwppHipStatus s);
/* Number of compute units of the handle's device (for launch heuristics). */
int bwpp_hip_device_cus(const BwppHip *h);
/* Symbol of the last kernel this handle launched ("" if none): which
 * variant a dispatch chose.  No reference counterpart (diagnostics). */
const char *bwpp_hip_last_kernel(const BwppHip *h);
/* Symbol of the launch `back` launches before the last (0 = the last, at
 * most 3; "" if none): the kernels of a dispatch that launches several,
 * e.g. a split-K GEMM and its reduce.  No reference counterpart
 * (diagnostics). */
const char *bwpp_hip_recent_kernel(const BwppHip *h, int back);

/* ---- device memory ---- */

/* Device twin of runtime/core/arena.h:6-15 / arena.c:4-38: one hipMalloc of
 * `capacity` bytes, bump allocation with power-of-two alignment, NULL on
 * exhaustion, reset rewinds, destroy frees. */
typedef struct {
  unsigned char *buffer; /* device address */
  size_t capacity;
  size_t offset;
  int device;
} BwppHipArena;

BwppHipStatus bwpp_hip_arena_init(BwppHip *h, BwppHipArena *arena,
                                  size_t capacity);
void bwpp_hip_arena_reset(BwppHipArena *arena);
void *bwpp_hip_arena_alloc(BwppHipArena *arena, size_t size, size_t align);
void bwpp_hip_arena_destroy(BwppHipArena *arena);

/* ---- tensor metadata (device twin of runtime/core/tensor.h) ---- */

/* The three dtype numberings met on the path:
 *   runtime/core BwppDType (runtime/core/tensor.h:7-11): F16 0, BF16 1, F32 2
 *   compiler BwppDType (compiler/include/graph_ir.h:18-23):
 *                                            UNKNOWN 0, F16 1, BF16 2, F32 3
 *   BwppHipDType (above):                    F32 0, BF16 1
 * BwppHipTensor carries runtime/core's numbering, as BwppTensor does; the
 * mappers below convert between them and return -1 for a dtype with no
 * counterpart (compiler UNKNOWN; F16, for which this build has no
 * kernels). */
typedef enum {
  BWPP_HIP_CORE_F16 = 0,
  BWPP_HIP_CORE_BF16 = 1,
  BWPP_HIP_CORE_F32 = 2
} BwppHipCoreDType;
typedef enum {
  BWPP_HIP_LAYOUT_ROW_MAJOR = 0, /* runtime/core/tensor.h:13-16 */
  BWPP_HIP_LAYOUT_COL_MAJOR = 1
} BwppHipLayout;

/* runtime/core/tensor.h:18-25 with a device buffer: same fields, order and
 * widths (the enums are int-sized), so a BwppTensor that describes device
 * memory has this layout.  stride[i] is in elements; a contiguous
 * row-major tensor has stride[rank-1] = 1.  COL_MAJOR marks a rank-2
 * tensor stored transposed (stride[0] = 1, stride[1] = leading dim). */
typedef struct {
  int32_t dtype;  /* BwppHipCoreDType */
  int32_t layout; /* BwppHipLayout */
  uint32_t rank;  /* 1..4 */
  uint64_t shape[4];
  uint64_t stride[4];
  void *buffer;   /* device address */
} BwppHipTensor;

int32_t bwpp_hip_dtype_from_core(int32_t core_dtype);   /* -> BwppHipDType */
int32_t bwpp_hip_dtype_from_graph(int32_t graph_dtype); /* -> BwppHipDType */
int32_t bwpp_hip_dtype_to_core(int32_t hip_dtype);      /* -> runtime/core */
int32_t bwpp_hip_dtype_to_graph(int32_t hip_dtype);     /* -> compiler */
/* Bytes per element of a runtime/core dtype (0 if unknown). */
size_t bwpp_hip_core_dtype_size(int32_t core_dtype);

/* Describes `buffer` as a contiguous tensor of `rank` dims in the given
 * layout (COL_MAJOR needs rank 2).  buffer may be NULL (shape only). */
BwppHipStatus bwpp_hip_tensor_init(BwppHipTensor *t, int32_t core_dtype,
                                   int32_t layout, uint32_t rank,
                                   const uint64_t *shape, void *buffer);
/* Bytes spanned by the tensor's elements (its strides included). */
size_t bwpp_hip_tensor_bytes(const BwppHipTensor *t);
/* bwpp_hip_tensor_init over memory taken from a device arena (256-byte
 * aligned); OUT_OF_MEMORY when the arena is exhausted. */
BwppHipStatus bwpp_hip_tensor_alloc(BwppHipArena *arena, BwppHipTensor *t,
                                    int32_t core_dtype, int32_t layout,
                                    uint32_t rank, const uint64_t *shape);
/* The [rows x cols] matrix with row stride ld (elements) that a row-major
 * tensor is to the row operators: cols = last dim, rows = product of the
 * others, which must be stacked at one stride.  UNSUPPORTED otherwise. */
BwppHipStatus bwpp_hip_tensor_matrix(const BwppHipTensor *t, uint32_t *rows,
                                     uint32_t *cols, uint32_t *ld);

/* Tensor-level forms of the operators below: parameters come from the
 * metadata (dtype, shape, strides, layout).  C = A·B (+bias) (→SiLU) with A
 * [M,K], B [K,N], C [M,N] rank 2 (a COL_MAJOR A or B runs transposed);
 * softmax / rmsnorm / layernorm along the last dim of any rank; attention
 * over rank-4 [batch, heads, seq, dim] q, k, v, o (slice strides from the
 * tensors).  dtypes must agree (f32, or bf16 for matmul / attention). */
BwppHipStatus bwpp_hip_tensor_matmul(BwppHip *h, const BwppHipTensor *a,
                                     const BwppHipTensor *b,
                                     const BwppHipTensor *bias,
                                     BwppHipTensor *c, uint32_t epilogue);
BwppHipStatus bwpp_hip_tensor_softmax(BwppHip *h, const BwppHipTensor *x,
                                      BwppHipTensor *y);
BwppHipStatus bwpp_hip_tensor_rmsnorm(BwppHip *h, const BwppHipTensor *x,
                                      const BwppHipTensor *gamma,
                                      const BwppHipTensor *beta,
                                      BwppHipTensor *y, float eps);
BwppHipStatus bwpp_hip_tensor_layernorm(BwppHip *h, const BwppHipTensor *x,
                                        const BwppHipTensor *gamma,
                                        const BwppHipTensor *beta,
                                        BwppHipTensor *y, float eps);
BwppHipStatus bwpp_hip_tensor_attention(BwppHip *h, const BwppHipTensor *q,
                                        const BwppHipTensor *k,
                                        const BwppHipTensor *v,
                                        BwppHipTensor *o, float scale,
                                        uint32_t causal);

/* Stream-ordered copies, complete on return. */
BwppHipStatus bwpp_hip_copy_to_device(BwppHip *h, void *dst, const void *src,
                                      size_t bytes);
BwppHipStatus bwpp_hip_copy_to_host(BwppHip *h, void *dst, const void *src,
                                    size_t bytes);

/* ---- operators (device pointers; asynchronous on the handle's stream) ---- */

/* bwpp_metal_dispatch_matmul (dispatch_stub.h:42-49); CPU twin
 * bwpp_cpu_matmul_f32 (bwpp_cpu_ref.c:8-35).  C must not overlap A, B or
 * bias (ALIAS). */
BwppHipStatus bwpp_hip_dispatch_matmul(BwppHip *h, const void *a,
                                       const void *b, void *c,
                                       const void *bias,
                                       BwppMatmulParams params);

/* Matmul with a fused elementwise tail (no reference counterpart: the
 * HIP lowering's fusions of the graph's add / silu / silu_grad nodes into
 * the GEMM that feeds them).  fp32 only (dtype F32, else UNSUPPORTED).
 * After the params' bias / SiLU epilogue, with Y = that result:
 *   RESIDUAL   C = Y + aux        (aux [M x N], row stride ld_aux; aux may
 *                                  be C itself, with ld_aux = ldc)
 *   DUAL_SILU  C = Y, c2 = SiLU(Y) (c2 [M x N], row stride ld_c2; the
 *                                  params' epilogue may not include SiLU)
 *   SILU_GRAD  C = Y * s (1 + x (1 - s)), x = aux, s = 1 / (1 + e^-x)
 *                                 (the graph's silu_grad with Y as dY;
 *                                  epilogue must be NONE)
 * NONE is bwpp_hip_dispatch_matmul. */
typedef enum {
  BWPP_HIP_FUSE_NONE = 0,
  BWPP_HIP_FUSE_RESIDUAL = 1,
  BWPP_HIP_FUSE_DUAL_SILU = 2,
  BWPP_HIP_FUSE_SILU_GRAD = 3
} BwppHipFusion;

typedef struct {
  uint32_t kind;   /* BwppHipFusion */
  uint32_t ld_aux; /* 0 = N */
  uint32_t ld_c2;  /* 0 = N */
} BwppHipFusionParams;

BwppHipStatus bwpp_hip_dispatch_matmul_fused(BwppHip *h, const void *a,
                                             const void *b, void *c,
                                             const void *bias,
                                             const float *aux, float *c2,
                                             BwppMatmulParams params,
                                             BwppHipFusionParams fusion);

/* bwpp_metal_dispatch_softmax (dispatch_stub.h:51-56); CPU twin
 * bwpp_cpu_softmax_f32 (bwpp_cpu_ref.c:37-61).  y may equal x. */
BwppHipStatus bwpp_hip_dispatch_softmax(BwppHip *h, const float *x, float *y,
                                        BwppSoftmaxParams params);

/* bwpp_metal_dispatch_rmsnorm (dispatch_stub.h:58-65); CPU twin
 * bwpp_cpu_rmsnorm_f32 (bwpp_cpu_ref.c:63-90).  y may equal x. */
BwppHipStatus bwpp_hip_dispatch_rmsnorm(BwppHip *h, const float *x,
                                        const float *gamma, const float *beta,
                                        float *y, BwppRmsnormParams params);

/* LayerNorm: no reference kernel (ROADMAP.md:14); same argument order as
 * rmsnorm.  y = (x-mean)/sqrt(var+eps)*gamma+beta, population variance. */
BwppHipStatus bwpp_hip_dispatch_layernorm(BwppHip *h, const float *x,
                                          const float *gamma,
                                          const float *beta, float *y,
                                          BwppRmsnormParams params);

/* bwpp_metal_dispatch_attention (dispatch_stub.h:67-74); CPU twin
 * bwpp_cpu_attention_f32 (bwpp_cpu_ref.c:92-144).  O must not overlap Q, K
 * or V (ALIAS). */
BwppHipStatus bwpp_hip_dispatch_attention(BwppHip *h, const void *q,
                                          const void *k, const void *v,
                                          void *o, BwppAttentionParams params);

/* Forward attention that also writes lse[(b*H + h)*M + m], the natural-log
 * log-sum-exp of query m's scaled, masked scores (-inf when it sees no key),
 * for the backward below.  No reference counterpart (the reference
 * differentiates attention through its decomposed graph ops,
 * graph_ir.c:1722-1733, 1529-1583).  The same kernels as the plain forward
 * run: bf16 with K = D = 128 and 16-byte rows (pointers, leading dims and
 * slice strides in multiples of 8 elements) takes the bf16 flash kernel;
 * fp32 with K = D = 64 or 128 and 16-byte rows takes the fp32 matrix-core
 * kernel; anything else the generic kernel. */
BwppHipStatus bwpp_hip_dispatch_attention_lse(BwppHip *h, const void *q,
                                              const void *k, const void *v,
                                              void *o, float *lse,
                                              BwppAttentionParams params);

/* Attention backward: dq, dk, dv of O = softmax(scale Q K^T [causal]) V
 * for the upstream gradient dout, from q, k, v, o and the forward's lse.
 * dout / dq / dk / dv use the strides of o / q / k / v.  Outputs must not
 * overlap inputs or each other.  Uses the handle's workspace for
 * rowsum(dout * o) and, for bf16 with K = D = 128 and for the fp32
 * matrix-core shapes, for dS (2 or 4 bytes x batch * heads *
 * ceil(N / 32) * 32 * ceil(M / 128) * 128, up to BWPP_ATTN_BWD_DS_MB MiB,
 * default 8192; beyond that, with 0, or when the device cannot allocate
 * it, S and dP are recomputed instead, with the same results).  Replaces the decomposed path of
 * graph_ir.c:1722-1733 (softmax_grad over materialised probabilities). */
BwppHipStatus bwpp_hip_dispatch_attention_grad(BwppHip *h, const void *q,
                                               const void *k, const void *v,
                                               const void *o, const void *dout,
                                               const float *lse, void *dq,
                                               void *dk, void *dv,
                                               BwppAttentionParams params);

/* bwpp_hip_dispatch_attention_grad that allocates nothing: no reference
 * counterpart; for callers that cannot call hipMalloc (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  The
 * per-query row sums rowsum(dout * o) live in a device-resident scratch
 * array of the library (8 MiB per GPU, held until the process ends)
 * instead of the handle's workspace, so batch * heads * M may be at most
 * 2,097,151 query rows (UNSUPPORTED beyond, nothing launched).  bf16 rows
 * that are not 16-byte aligned (which need fp32 copies in the workspace)
 * are UNSUPPORTED too.  Every call on one GPU shares that GPU's scratch:
 * calls that overlap on one GPU (several streams, handles or threads) race
 * on it; calls ordered on one stream do not.  Results are bit-identical to
 * bwpp_hip_dispatch_attention_grad's (but for the sign of a zero that is
 * an all-zero sum: this entry recomputes S and dP in the dQ pass rather
 * than storing dS). */
BwppHipStatus bwpp_hip_dispatch_attention_grad_noalloc(
    BwppHip *h, const void *q, const void *k, const void *v, const void *o,
    const void *dout, const float *lse, void *dq, void *dk, void *dv,
    BwppAttentionParams params);

/* reduce_max forward (graph op BWPP_GOP_REDUCE_MAX, graph_ir.h:48; no
 * reference kernel): maxv as the reference's fold, argmax = lowest index
 * holding it (-1 if none).  Either output may be NULL, not both. */
BwppHipStatus bwpp_hip_dispatch_reduce_max(BwppHip *h, const float *x,
                                           float *maxv, int32_t *argmax,
                                           BwppReduceParams params);

/* bwpp_cpu_reduce_max_mask_f32 (bwpp_cpu_ref.c:146-190): 1.0 at every
 * element equal to its line's maximum, else 0.0. */
BwppHipStatus bwpp_hip_dispatch_reduce_max_mask(BwppHip *h, const float *x,
                                                float *mask,
                                                BwppReduceParams params);

/* bwpp_cpu_reduce_max_grad_f32 (bwpp_cpu_ref.c:192-219): dx = mask * dy,
 * dy broadcast along the reduced axis. */
BwppHipStatus bwpp_hip_dispatch_reduce_max_grad(BwppHip *h, const float *mask,
                                                const float *dy, float *dx,
                                                BwppReduceParams params);

/* reduce_max grad routed one-hot to the lowest-index maximum: pass x (the
 * argmax is recomputed in the same pass) or argmax (saved indices), not
 * both NULL; dx is fully written. */
BwppHipStatus bwpp_hip_dispatch_reduce_max_grad_argmax(
    BwppHip *h, const float *x, const int32_t *argmax, const float *dy,
    float *dx, BwppReduceParams params);

/* ---- autodiff grad ops (graph_ir.c:1485-1839 emits them; the reference
 * has no numeric kernels, the closed forms are in oracle/bwpp_oracle.h) ---- */

/* BWPP_GOP_SILU_GRAD (graph_ir.c:1709-1720), n contiguous elements:
 * s = 1/(1+e^-x); dx = dy * s * (1 + x (1 - s)). */
BwppHipStatus bwpp_hip_dispatch_silu_grad(BwppHip *h, const float *x, const float *dy, float *dx,
                                          uint64_t n);

/* BWPP_GOP_SOFTMAX_GRAD (graph_ir.c:1722-1733), along rows:
 * dx = y * (dy - sum_c dy*y). */
BwppHipStatus bwpp_hip_dispatch_softmax_grad(BwppHip *h, const float *y, const float *dy, float *dx,
                                             BwppSoftmaxParams params);

/* BWPP_GOP_RMSNORM_GRAD (graph_ir.c:1735-1789): dx for every row, and the
 * column sums dgamma = sum_r dy * xhat, dbeta = sum_r dy when those
 * pointers are non-NULL (needs cols <= 8192).  gamma NULL means 1. */
BwppHipStatus bwpp_hip_dispatch_rmsnorm_grad(BwppHip *h, const float *x, const float *gamma,
                                             const float *dy, float *dx, float *dgamma,
                                             float *dbeta, BwppRmsnormParams params);

/* bwpp_hip_dispatch_rmsnorm_grad with dx = acc + the gradient: the
 * autodiff graph's add of the residual branch's gradient
 * (graph_ir.c:1529-1545, ADD of the two gradient contributions to x) folded
 * into the same pass, with one fp32 rounding like the separate add.  acc has
 * dx's layout (row stride params.ld) and may be dx itself; NULL acc is
 * bwpp_hip_dispatch_rmsnorm_grad. */
BwppHipStatus bwpp_hip_dispatch_rmsnorm_grad_acc(BwppHip *h, const float *x, const float *gamma,
                                                 const float *dy, const float *acc, float *dx,
                                                 float *dgamma, float *dbeta,
                                                 BwppRmsnormParams params);

/* Mean-square training loss and its gradient, the loss the HIP target's
 * `--train mean_square` appends (no reference counterpart: the reference
 * compiler has no loss; the C5 configuration names loss = mean(out^2)):
 * loss[0] = loss_scale * sum of x^2 over rows x cols, and dx = grad_scale * x
 * when dx is non-NULL (dx may be x).  The scales are device scalars (NULL
 * = 1), e.g. 1/n and 2/n.  One pass over x plus a one-block finish; the sum
 * is taken in a fixed order (deterministic for a given device).  Either
 * output may be NULL, not both. */
typedef struct {
  uint32_t rows;
  uint32_t cols;
  uint32_t ld; /* row stride of x and dx; 0 = cols */
} BwppMeanSquareParams;

BwppHipStatus bwpp_hip_dispatch_mean_square(BwppHip *h, const float *x, const float *loss_scale,
                                            const float *grad_scale, float *loss, float *dx,
                                            BwppMeanSquareParams params);

/* BWPP_GOP_REDUCE_SUM / reduce_to_shape (graph_ir.c:1410-1455): axis 0 sums
 * over rows (out[cols]), any other axis along each row (out[rows]). */
BwppHipStatus bwpp_hip_dispatch_reduce_sum(BwppHip *h, const float *x, float *out,
                                           BwppReduceParams params);

/* add / sub / mul / div with broadcasting, and broadcast (op COPY). */
BwppHipStatus bwpp_hip_dispatch_elementwise(BwppHip *h, const float *a, const float *b, float *out,
                                            BwppElementwiseParams params);

/* ---- launch plans (compiled graphs) ----
 *
 * The executor for a lowered BW++ graph: `bwppc` hands its graph to the
 * Metal codegen today (main.c:186, codegen_metal.h:7); a HIP target emits
 * this text instead (format in csrc/runtime/bwpp_plan.cpp: dims, named
 * values, strided views, ordered operator launches over the dispatch calls
 * above).  Creation parses and builds the memory plan: liveness-based
 * buffer reuse as compiler/mem_plan.c:43-146, with byte sizes from the
 * bound dims and no operator ever given the buffer of one of its own
 * inputs.  h may be NULL to parse and plan only (report, arena size).
 * On failure *out still receives a plan whose last_error says why; destroy
 * it. */
typedef struct BwppHipPlan BwppHipPlan;
BwppHipStatus bwpp_hip_plan_create(BwppHip *h, const char *text, BwppHipPlan **out);
void bwpp_hip_plan_destroy(BwppHipPlan *plan);
const char *bwpp_hip_plan_last_error(const BwppHipPlan *plan);
/* Device bytes of all planned buffers (temps, outputs, consts). */
size_t bwpp_hip_plan_arena_bytes(const BwppHipPlan *plan);
/* One device arena (bwpp_hip_arena_init) holding every planned buffer;
 * const values are filled. */
BwppHipStatus bwpp_hip_plan_allocate(BwppHipPlan *plan);
/* Caller memory for an input or param value. */
BwppHipStatus bwpp_hip_plan_bind(BwppHipPlan *plan, const char *name, void *device_ptr);
/* Device address of any value (NULL if unknown or not yet placed). */
void *bwpp_hip_plan_value_ptr(const BwppHipPlan *plan, const char *name);
/* Runs every launch in order on the handle's stream. */
BwppHipStatus bwpp_hip_plan_run(BwppHipPlan *plan);
/* Records the plan's launches as a HIP graph (no reference counterpart: for
 * loops that replay one plan and should not pay the host cost of each
 * launch).  Runs the plan once eagerly first, so every workspace reaches its
 * final size, then captures one run on the handle's stream, which must not
 * be the default (null) stream (UNSUPPORTED).  Binding a different address
 * afterwards drops the graph; capture again. */
BwppHipStatus bwpp_hip_plan_capture(BwppHipPlan *plan);
/* Launches the captured graph on the handle's current stream (INVALID_ARG
 * when there is none).  Results equal bwpp_hip_plan_run's. */
BwppHipStatus bwpp_hip_plan_replay(BwppHipPlan *plan);
/* Memory-plan report in mem_plan.c:176-193's layout plus byte sizes, arena
 * offsets and the total; returns the bytes needed including the NUL. */
size_t bwpp_hip_plan_report(const BwppHipPlan *plan, char *buf, size_t cap);

/* ---- synthetic inputs (host memory, no device needed) ----
 * Counter-based: element i of (seed, stream) is a pure function of
 * (seed, stream, i), so subsets and threads agree with a full fill.
 * SplitMix64 -> 24-bit uniform; normal by Box-Muller in double. */
void bwpp_synth_uniform_f32(float *dst, uint64_t n, uint64_t seed,
                            uint64_t stream, float lo, float hi);
void bwpp_synth_normal_f32(float *dst, uint64_t n, uint64_t seed,
                           uint64_t stream, float mean, float stddev);
/* The reference's test fixture x[i][j] = (i*cols + j + 1) * scale
 * (runtime/cpu/test_matmul.c:7-13). */
void bwpp_synth_ramp_f32(float *dst, uint32_t rows, uint32_t cols,
                         float scale);
/* fp32 -> bf16 round to nearest even (NaN kept quiet), and back (exact). */
void bwpp_f32_to_bf16(const float *src, uint16_t *dst, uint64_t n);
void bwpp_bf16_to_f32(const uint16_t *src, float *dst, uint64_t n);

#ifdef __cplusplus
}
#endif

#endif /* BWPP_HIP_H */
