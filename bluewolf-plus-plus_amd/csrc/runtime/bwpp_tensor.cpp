// Tensor metadata layer of libbwpp_hip: the device twin of runtime/core's
// BwppTensor (runtime/core/tensor.h:18-25), the mapping between the three
// dtype numberings on the path (runtime/core/tensor.h:7-11,
// compiler/include/graph_ir.h:18-23 and BwppHipDType), and tensor-level
// forms of the operators that derive each dispatch's params struct from the
// metadata.  Nothing here launches work itself: every operator goes through
// the bwpp_hip_dispatch_* entry point it names.
#include "bwpp_hip.h"
#include "internal.h"

#include <cstddef>
#include <cstdint>
#include <initializer_list>

static_assert(sizeof(BwppHipTensor) == 88 && offsetof(BwppHipTensor, shape) == 16 &&
                  offsetof(BwppHipTensor, stride) == 48 && offsetof(BwppHipTensor, buffer) == 80,
              "BwppHipTensor must keep runtime/core/tensor.h's BwppTensor layout");

namespace {

// compiler/include/graph_ir.h:18-23
constexpr int32_t kGraphUnknown = 0, kGraphF16 = 1, kGraphBF16 = 2, kGraphF32 = 3;

bool valid_rank(const BwppHipTensor *t) { return t && t->rank >= 1 && t->rank <= 4; }

int32_t hip_dtype(const BwppHipTensor *t) { return bwpp_hip_dtype_from_core(t->dtype); }

// Leading dims of a row-major tensor stacked at one stride?
bool stacked(const BwppHipTensor *t) {
  for (uint32_t i = 0; i + 2 < t->rank; ++i)
    if (t->shape[i + 1] > 1 && t->stride[i] != t->stride[i + 1] * t->shape[i + 1]) return false;
  return true;
}

bool fits_u32(uint64_t v) { return v <= 0xffffffffull; }

BwppHipStatus bad(BwppHip *h, const char *what) {
  return bwpp_hip_set_error(h, BWPP_HIP_ERR_INVALID_ARG, "tensor: %s", what);
}

}  // namespace

extern "C" {

int32_t bwpp_hip_dtype_from_core(int32_t core_dtype) {
  switch (core_dtype) {
    case BWPP_HIP_CORE_F32: return BWPP_HIP_F32;
    case BWPP_HIP_CORE_BF16: return BWPP_HIP_BF16;
    default: return -1;  // F16: no kernels in this build
  }
}

int32_t bwpp_hip_dtype_from_graph(int32_t graph_dtype) {
  switch (graph_dtype) {
    case kGraphF32: return BWPP_HIP_F32;
    case kGraphBF16: return BWPP_HIP_BF16;
    case kGraphF16:
    case kGraphUnknown:
    default: return -1;
  }
}

int32_t bwpp_hip_dtype_to_core(int32_t hip_dtype) {
  switch (hip_dtype) {
    case BWPP_HIP_F32: return BWPP_HIP_CORE_F32;
    case BWPP_HIP_BF16: return BWPP_HIP_CORE_BF16;
    default: return -1;
  }
}

int32_t bwpp_hip_dtype_to_graph(int32_t hip_dtype) {
  switch (hip_dtype) {
    case BWPP_HIP_F32: return kGraphF32;
    case BWPP_HIP_BF16: return kGraphBF16;
    default: return -1;
  }
}

size_t bwpp_hip_core_dtype_size(int32_t core_dtype) {
  switch (core_dtype) {
    case BWPP_HIP_CORE_F16:
    case BWPP_HIP_CORE_BF16: return 2;
    case BWPP_HIP_CORE_F32: return 4;
    default: return 0;
  }
}

BwppHipStatus bwpp_hip_tensor_init(BwppHipTensor *t, int32_t core_dtype, int32_t layout, uint32_t rank,
                                   const uint64_t *shape, void *buffer) {
  if (!t || !shape || rank < 1 || rank > 4 || bwpp_hip_core_dtype_size(core_dtype) == 0)
    return BWPP_HIP_ERR_INVALID_ARG;
  if (layout != BWPP_HIP_LAYOUT_ROW_MAJOR && !(layout == BWPP_HIP_LAYOUT_COL_MAJOR && rank == 2))
    return BWPP_HIP_ERR_INVALID_ARG;
  BwppHipTensor r = {};
  r.dtype = core_dtype;
  r.layout = layout;
  r.rank = rank;
  for (uint32_t i = 0; i < rank; ++i) r.shape[i] = shape[i];
  if (layout == BWPP_HIP_LAYOUT_COL_MAJOR) {
    r.stride[0] = 1;
    r.stride[1] = shape[0];
  } else {
    uint64_t s = 1;
    for (uint32_t i = rank; i-- > 0;) {
      r.stride[i] = s;
      s *= shape[i];
    }
  }
  r.buffer = buffer;
  *t = r;
  return BWPP_HIP_OK;
}

size_t bwpp_hip_tensor_bytes(const BwppHipTensor *t) {
  if (!valid_rank(t)) return 0;
  uint64_t last = 0;
  for (uint32_t i = 0; i < t->rank; ++i) {
    if (t->shape[i] == 0) return 0;
    last += (t->shape[i] - 1) * t->stride[i];
  }
  return (size_t)((last + 1) * bwpp_hip_core_dtype_size(t->dtype));
}

BwppHipStatus bwpp_hip_tensor_alloc(BwppHipArena *arena, BwppHipTensor *t, int32_t core_dtype, int32_t layout,
                                    uint32_t rank, const uint64_t *shape) {
  if (!arena) return BWPP_HIP_ERR_INVALID_ARG;
  BwppHipTensor r;
  BwppHipStatus s = bwpp_hip_tensor_init(&r, core_dtype, layout, rank, shape, nullptr);
  if (s != BWPP_HIP_OK) return s;
  const size_t bytes = bwpp_hip_tensor_bytes(&r);
  if (bytes > 0) {
    r.buffer = bwpp_hip_arena_alloc(arena, bytes, 256);
    if (!r.buffer) return BWPP_HIP_ERR_OUT_OF_MEMORY;
  }
  *t = r;
  return BWPP_HIP_OK;
}

BwppHipStatus bwpp_hip_tensor_matrix(const BwppHipTensor *t, uint32_t *rows, uint32_t *cols, uint32_t *ld) {
  if (!valid_rank(t) || !rows || !cols || !ld) return BWPP_HIP_ERR_INVALID_ARG;
  if (t->layout != BWPP_HIP_LAYOUT_ROW_MAJOR || t->stride[t->rank - 1] != 1 || !stacked(t))
    return BWPP_HIP_ERR_UNSUPPORTED;
  uint64_t r = 1;
  for (uint32_t i = 0; i + 1 < t->rank; ++i) r *= t->shape[i];
  const uint64_t c = t->shape[t->rank - 1];
  const uint64_t l = t->rank >= 2 ? t->stride[t->rank - 2] : c;
  if (!fits_u32(r) || !fits_u32(c) || !fits_u32(l) || (r > 1 && l < c)) return BWPP_HIP_ERR_UNSUPPORTED;
  *rows = (uint32_t)r;
  *cols = (uint32_t)c;
  *ld = (uint32_t)(r > 1 ? l : (l < c ? c : l));
  return BWPP_HIP_OK;
}

BwppHipStatus bwpp_hip_tensor_matmul(BwppHip *h, const BwppHipTensor *a, const BwppHipTensor *b,
                                     const BwppHipTensor *bias, BwppHipTensor *c, uint32_t epilogue) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  if (!a || !b || !c || a->rank != 2 || b->rank != 2 || c->rank != 2) return bad(h, "matmul takes rank-2 a, b, c");
  const int32_t dt = hip_dtype(a);
  if (dt < 0 || hip_dtype(b) != dt || hip_dtype(c) != dt || (bias && hip_dtype(bias) != dt))
    return bad(h, "matmul operands need one dtype, f32 or bf16");
  const uint64_t M = a->shape[0], K = a->shape[1], N = b->shape[1];
  if (b->shape[0] != K || c->shape[0] != M || c->shape[1] != N) return bad(h, "matmul shapes do not chain");
  // A [M,K] and B [K,N]: row-major (unit last stride) or column-major
  // (stored transposed, unit first stride).
  auto orient = [](const BwppHipTensor *t, uint32_t &trans, uint64_t &ld) {
    if (t->stride[1] == 1 && t->layout == BWPP_HIP_LAYOUT_ROW_MAJOR) {
      trans = 0;
      ld = t->stride[0];
      return true;
    }
    if (t->stride[0] == 1 && t->layout == BWPP_HIP_LAYOUT_COL_MAJOR) {
      trans = 1;
      ld = t->stride[1];
      return true;
    }
    return false;
  };
  uint32_t ta = 0, tb = 0, tc = 0;
  uint64_t lda = 0, ldb = 0, ldc = 0;
  if (!orient(a, ta, lda) || !orient(b, tb, ldb) || !orient(c, tc, ldc) || tc)
    return bad(h, "matmul: a and b row- or column-major, c row-major, unit inner stride");
  if (bias && (bias->rank != 1 || bias->shape[0] != N || bias->stride[0] != 1))
    return bad(h, "matmul: bias must be a contiguous [N] vector");
  if (!fits_u32(M) || !fits_u32(N) || !fits_u32(K) || !fits_u32(lda) || !fits_u32(ldb) || !fits_u32(ldc))
    return bwpp_hip_set_error(h, BWPP_HIP_ERR_UNSUPPORTED, "tensor: matmul sizes above 2^32");
  BwppMatmulParams p = {(uint32_t)M, (uint32_t)N, (uint32_t)K, (uint32_t)lda, (uint32_t)ldb, (uint32_t)ldc,
                        (uint32_t)dt, epilogue, ta, tb};
  return bwpp_hip_dispatch_matmul(h, a->buffer, b->buffer, c->buffer, bias ? bias->buffer : nullptr, p);
}

namespace {

// x and y as matrices of one shape and one row stride, f32.
BwppHipStatus row_pair(BwppHip *h, const BwppHipTensor *x, const BwppHipTensor *y, uint32_t &rows,
                       uint32_t &cols, uint32_t &ld) {
  if (!x || !y) return bad(h, "NULL x or y");
  if (hip_dtype(x) != BWPP_HIP_F32 || hip_dtype(y) != BWPP_HIP_F32) return bad(h, "row operators take f32");
  uint32_t yr = 0, yc = 0, yl = 0;
  if (bwpp_hip_tensor_matrix(x, &rows, &cols, &ld) != BWPP_HIP_OK ||
      bwpp_hip_tensor_matrix(y, &yr, &yc, &yl) != BWPP_HIP_OK)
    return bwpp_hip_set_error(h, BWPP_HIP_ERR_UNSUPPORTED, "tensor: x / y are not stacked row-major rows");
  if (yr != rows || yc != cols || (rows > 1 && yl != ld)) return bad(h, "x and y need one shape and row stride");
  return BWPP_HIP_OK;
}

const float *vec(const BwppHipTensor *t) { return t ? static_cast<const float *>(t->buffer) : nullptr; }

BwppHipStatus norm(BwppHip *h, const BwppHipTensor *x, const BwppHipTensor *gamma, const BwppHipTensor *beta,
                   BwppHipTensor *y, float eps, bool layer) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  uint32_t rows, cols, ld;
  BwppHipStatus s = row_pair(h, x, y, rows, cols, ld);
  if (s != BWPP_HIP_OK) return s;
  for (const BwppHipTensor *v : {gamma, beta})
    if (v && (v->rank != 1 || v->shape[0] != cols || v->stride[0] != 1 || hip_dtype(v) != BWPP_HIP_F32))
      return bad(h, "gamma / beta must be contiguous f32 [cols]");
  BwppRmsnormParams p = {rows, cols, ld, eps};
  float *yp = static_cast<float *>(y->buffer);
  const float *xp = static_cast<const float *>(x->buffer);
  return layer ? bwpp_hip_dispatch_layernorm(h, xp, vec(gamma), vec(beta), yp, p)
               : bwpp_hip_dispatch_rmsnorm(h, xp, vec(gamma), vec(beta), yp, p);
}

}  // namespace

BwppHipStatus bwpp_hip_tensor_softmax(BwppHip *h, const BwppHipTensor *x, BwppHipTensor *y) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  uint32_t rows, cols, ld;
  BwppHipStatus s = row_pair(h, x, y, rows, cols, ld);
  if (s != BWPP_HIP_OK) return s;
  BwppSoftmaxParams p = {rows, cols, ld};
  return bwpp_hip_dispatch_softmax(h, static_cast<const float *>(x->buffer), static_cast<float *>(y->buffer), p);
}

BwppHipStatus bwpp_hip_tensor_rmsnorm(BwppHip *h, const BwppHipTensor *x, const BwppHipTensor *gamma,
                                      const BwppHipTensor *beta, BwppHipTensor *y, float eps) {
  return norm(h, x, gamma, beta, y, eps, false);
}

BwppHipStatus bwpp_hip_tensor_layernorm(BwppHip *h, const BwppHipTensor *x, const BwppHipTensor *gamma,
                                        const BwppHipTensor *beta, BwppHipTensor *y, float eps) {
  return norm(h, x, gamma, beta, y, eps, true);
}

BwppHipStatus bwpp_hip_tensor_attention(BwppHip *h, const BwppHipTensor *q, const BwppHipTensor *k,
                                        const BwppHipTensor *v, BwppHipTensor *o, float scale, uint32_t causal) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  if (!q || !k || !v || !o || q->rank != 4 || k->rank != 4 || v->rank != 4 || o->rank != 4)
    return bad(h, "attention takes rank-4 [batch, heads, seq, dim] q, k, v, o");
  const int32_t dt = hip_dtype(q);
  if (dt < 0 || hip_dtype(k) != dt || hip_dtype(v) != dt || hip_dtype(o) != dt)
    return bad(h, "attention operands need one dtype, f32 or bf16");
  for (const BwppHipTensor *t : {q, k, v, static_cast<const BwppHipTensor *>(o)})
    if (t->layout != BWPP_HIP_LAYOUT_ROW_MAJOR || t->stride[3] != 1)
      return bad(h, "attention: row-major tensors with unit inner stride");
  const uint64_t B = q->shape[0], H = q->shape[1], M = q->shape[2], Kd = q->shape[3];
  const uint64_t N = k->shape[2], D = v->shape[3];
  if (k->shape[0] != B || k->shape[1] != H || k->shape[3] != Kd || v->shape[0] != B || v->shape[1] != H ||
      v->shape[2] != N || o->shape[0] != B || o->shape[1] != H || o->shape[2] != M || o->shape[3] != D)
    return bad(h, "attention shapes do not agree");
  for (uint64_t x : {B, H, M, N, Kd, D, q->stride[2], k->stride[2], v->stride[2], o->stride[2]})
    if (!fits_u32(x)) return bwpp_hip_set_error(h, BWPP_HIP_ERR_UNSUPPORTED, "tensor: attention sizes above 2^32");
  BwppAttentionParams p = {};
  p.M = (uint32_t)M;
  p.N = (uint32_t)N;
  p.K = (uint32_t)Kd;
  p.D = (uint32_t)D;
  p.ldq = (uint32_t)q->stride[2];
  p.ldk = (uint32_t)k->stride[2];
  p.ldv = (uint32_t)v->stride[2];
  p.ldo = (uint32_t)o->stride[2];
  p.batch = (uint32_t)B;
  p.heads = (uint32_t)H;
  p.q_batch_stride = q->stride[0];
  p.q_head_stride = q->stride[1];
  p.k_batch_stride = k->stride[0];
  p.k_head_stride = k->stride[1];
  p.v_batch_stride = v->stride[0];
  p.v_head_stride = v->stride[1];
  p.o_batch_stride = o->stride[0];
  p.o_head_stride = o->stride[1];
  p.scale = scale;
  p.causal = causal;
  p.dtype = (uint32_t)dt;
  return bwpp_hip_dispatch_attention(h, q->buffer, k->buffer, v->buffer, o->buffer, p);
}

}  // extern "C"
