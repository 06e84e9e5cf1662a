/*
 * lower_hip.c -- BwppGraph -> libbwpp_hip launch plan (see lower_hip.h).
 *
 * The pass keeps, for every graph value, where its data lives in the plan:
 * a plan value, possibly seen transposed (a transpose is never
 * materialised: it becomes a GEMM operand flag) or broadcast (folded into
 * the consuming elementwise op's broadcast mode).  Nodes are lowered in
 * graph order, which is a topological order (graph_ir.c adds a node after
 * its inputs).  Fused regions are found first and their nodes skipped.
 *
 * Training plans lower the forward graph, the loss, then the autodiff
 * graph.  That graph refers to forward activations through clones
 * (graph_ir.c:1375-1386, bwpp_graph_import_activation) whose link to the
 * forward value is not kept; this pass rebuilds it by walking the forward
 * graph in the autodiff pass's order (graph_ir.c:1520-1822) and pairing its
 * imports with the clones in creation order, checking names and shapes.
 */
#include "lower_hip.h"

#include <math.h>
#include <stdarg.h>
#include <stdlib.h>
#include <string.h>

#define MAX_PV 4096
#define NAME_LEN 64
#define DIM_LEN 96

enum { BC_FULL = 0, BC_ROW, BC_COL, BC_SCALAR, BC_BAD };

typedef struct {
  uint32_t rank;
  char d[BWPP_GRAPH_MAX_DIMS][DIM_LEN]; /* symbolic dim text (unbatched) */
  uint64_t n[BWPP_GRAPH_MAX_DIMS];      /* bound value (unbatched) */
} Shape;

typedef struct {
  char name[NAME_LEN];
  int bf16;
  uint32_t rank;
  char d[BWPP_GRAPH_MAX_DIMS][DIM_LEN + 8]; /* plan dims (batched) */
  char kind[64];
  /* a 2-D strided window into plan value view_of (kind "view") */
  int view_of;
  char off[DIM_LEN + 8], ld[DIM_LEN + 8];
} PVal;

typedef struct {
  int pv;       /* plan value holding the data, -1 = none yet */
  int trans;    /* the data is pv transposed (rank 2) */
  int bcast;    /* the value is pv broadcast to `shape` */
  int fused;    /* computed inside a fused region, no plan value of its own */
  int batched;  /* leading dim stacked `batch` times in the plan */
  int bf16;
  int known;    /* shape inferred */
  int preset;   /* pv chosen before the producer is lowered (a view) */
  Shape shape;  /* logical shape (unbatched) */
  Shape src;    /* bcast: shape of pv's data */
} LVal;

typedef struct {
  int mm1, tk, sm, mm2;  /* forward nodes: q @ kT, kT = transpose(k), softmax, probs @ v */
  uint32_t q, k, v, kt, s, o;
  int lse_pv;
  uint32_t heads, batch;
  int bhsd;
  char bdim[DIM_LEN], hdim[DIM_LEN]; /* bhsd: q's batch and head dims */
  float scale;
} AttnRegion;

/* Sibling GEMMs: matmuls that share their left operand and take weights
 * (params) of one shape, Y_m = A @ W_m.  They run as one GEMM against the
 * column concatenation [W_0 | W_1 | ...] into [Y_0 | Y_1 | ...], each Y_m a
 * column view.  In the autodiff graph (matmul rule, graph_ir.c:1529-1583)
 * each member has dW_m = transpose(A') @ dY_m and dA_m = dY_m @
 * transpose(W_m'), and the dA_m are summed by adds; with the dY_m written
 * as column views of one [dY_0 | dY_1 | ...] these become two GEMMs:
 * [dW_0 | dW_1 | ...] = transpose(A) @ dYcat and sum_m dA_m = dYcat @
 * transpose(Wcat). */
#define MM_GROUP_MAX 8
typedef struct {
  uint32_t a;
  int n;
  int node[MM_GROUP_MAX];
  uint32_t w[MM_GROUP_MAX], y[MM_GROUP_MAX];
  int wcat_pv;
  /* autodiff graph */
  int bwd;                      /* dW / dY grouping applies */
  int da;                       /* the dA sum is grouped too */
  int dw_node[MM_GROUP_MAX], da_node[MM_GROUP_MAX];
  uint32_t dy[MM_GROUP_MAX];
  uint32_t da_sum;              /* value holding sum_m dA_m */
  int first_bwd;                /* node that emits the backward GEMMs */
} MMGroup;

typedef struct {
  const BwppLowerOptions *opt;
  char *err;
  size_t err_cap;
  int failed;
  PVal *pv;
  int npv;
  char *ops;
  size_t ops_len, ops_cap;
  const char *batch_dim;
  uint32_t const_used;
  AttnRegion *regions;
  int nregions;
  MMGroup *groups;
  int ngroups;
} Ctx;

typedef struct {
  const BwppGraph *g;
  LVal *lv;
  uint32_t **cons; /* consumer node ids per value */
  uint32_t *ncons;
  uint8_t *skip;   /* node lowered as part of a fused region */
  int is_grad;
} GCtx;

/* ------------------------------------------------------------ utilities */

static void fail(Ctx *c, const char *fmt, ...) {
  if (c->failed) return;
  c->failed = 1;
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(c->err, c->err_cap, fmt, ap);
  va_end(ap);
}

static void emit(Ctx *c, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  int n = vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (n < 0) return;
  if ((size_t)n >= sizeof buf) n = (int)sizeof buf - 1;
  if (c->ops_len + (size_t)n + 1 > c->ops_cap) {
    size_t cap = c->ops_cap ? c->ops_cap * 2 : 8192;
    while (cap < c->ops_len + (size_t)n + 1) cap *= 2;
    char *p = (char *)realloc(c->ops, cap);
    if (!p) {
      fail(c, "out of memory");
      return;
    }
    c->ops = p;
    c->ops_cap = cap;
  }
  memcpy(c->ops + c->ops_len, buf, (size_t)n);
  c->ops_len += (size_t)n;
  c->ops[c->ops_len] = '\0';
}

static void str_copy(char *dst, size_t cap, const char *p, size_t len) {
  if (len >= cap) len = cap - 1;
  memcpy(dst, p, len);
  dst[len] = '\0';
}

/* Value of a dim: an integer literal, a bound name, or a product. */
static int dim_eval(const Ctx *c, const char *e, uint64_t *out) {
  uint64_t v = 1;
  const char *p = e;
  while (*p) {
    const char *q = strchr(p, '*');
    size_t len = q ? (size_t)(q - p) : strlen(p);
    char tok[DIM_LEN];
    str_copy(tok, sizeof tok, p, len);
    char *end = NULL;
    unsigned long long lit = strtoull(tok, &end, 10);
    if (tok[0] && end && *end == '\0') {
      v *= lit;
    } else {
      uint32_t i = 0;
      for (; i < c->opt->dim_count; ++i)
        if (strcmp(c->opt->dim_names[i], tok) == 0) break;
      if (i == c->opt->dim_count) return 0;
      v *= c->opt->dim_values[i];
    }
    if (!q) break;
    p = q + 1;
  }
  *out = v;
  return 1;
}

static uint64_t shape_elems(const Shape *s) {
  uint64_t n = 1;
  for (uint32_t i = 0; i < s->rank; ++i) n *= s->n[i];
  return n;
}

static int shape_from_graph(Ctx *c, const BwppShape *gs, Shape *out) {
  memset(out, 0, sizeof *out);
  out->rank = gs->rank;
  for (uint32_t i = 0; i < gs->rank; ++i) {
    if (!gs->dims[i].ptr) {
      fail(c, "a graph shape has an empty dim");
      return 0;
    }
    str_copy(out->d[i], DIM_LEN, gs->dims[i].ptr, gs->dims[i].len);
    if (!dim_eval(c, out->d[i], &out->n[i])) {
      fail(c, "dim '%s' is not bound (pass --dim %s=N)", out->d[i], out->d[i]);
      return 0;
    }
  }
  return 1;
}

static void shape_set_dim(Shape *s, uint32_t i, const char *text, uint64_t n) {
  str_copy(s->d[i], DIM_LEN, text, strlen(text));
  s->n[i] = n;
}

static void shape_swap_last(Shape *s) {
  if (s->rank < 2) return;
  Shape t = *s;
  memcpy(s->d[s->rank - 1], t.d[s->rank - 2], DIM_LEN);
  memcpy(s->d[s->rank - 2], t.d[s->rank - 1], DIM_LEN);
  s->n[s->rank - 1] = t.n[s->rank - 2];
  s->n[s->rank - 2] = t.n[s->rank - 1];
}

static int dtype_bf16(Ctx *c, BwppDType dt) {
  if (dt == BWPP_DTYPE_BF16) return 1;
  if (dt == BWPP_DTYPE_F16) return c->opt->f16_as == BWPP_DTYPE_BF16;
  return 0;
}

/* ------------------------------------------------------------ plan values */

/* A plan identifier from a graph name (final uniqueness is settled when
 * the plan is written: inlined functions repeat their local names). */
static void sanitize(const char *base, char *out) {
  size_t j = 0;
  for (const char *p = base; *p && j + 1 < NAME_LEN - 12; ++p) {
    const char ch = *p;
    out[j++] = (ch == '_' || (ch >= '0' && ch <= '9') || (ch >= 'a' && ch <= 'z') || (ch >= 'A' && ch <= 'Z'))
                   ? ch : '_';
  }
  out[j] = '\0';
  if (j == 0) strcpy(out, "t");
}

/* A plan value for logical shape `s`; batched: the leading dim is stacked. */
static int new_pv(Ctx *c, const char *base, const Shape *s, int batched, int bf16, const char *kind) {
  if (c->npv >= MAX_PV) {
    fail(c, "too many plan values");
    return -1;
  }
  PVal *p = &c->pv[c->npv];
  memset(p, 0, sizeof *p);
  p->view_of = -1;
  sanitize(base, p->name);
  p->bf16 = bf16;
  p->rank = s->rank ? s->rank : 1;
  if (s->rank == 0) {
    strcpy(p->d[0], "1");
  } else {
    for (uint32_t i = 0; i < s->rank; ++i) {
      if (i == 0 && batched && c->opt->batch > 1)
        snprintf(p->d[0], sizeof p->d[0], "BATCH*%s", s->d[0]);
      else
        strcpy(p->d[i], s->d[i]);
    }
  }
  snprintf(p->kind, sizeof p->kind, "%s", kind);
  return c->npv++;
}

/* A view of plan value `base`: shape `s` (rank 2), columns from `off`, row
 * stride `ld` (dim expressions, in elements). */
static int new_view(Ctx *c, int base, const char *name, const Shape *s, int batched, const char *off,
                    const char *ld) {
  const int pv = new_pv(c, name, s, batched, base >= 0 ? c->pv[base].bf16 : 0, "view");
  if (pv < 0) return pv;
  c->pv[pv].view_of = base;
  snprintf(c->pv[pv].off, sizeof c->pv[pv].off, "%s", off);
  snprintf(c->pv[pv].ld, sizeof c->pv[pv].ld, "%s", ld);
  return pv;
}

static void value_name(const BwppGraph *g, uint32_t v, const char *dflt, char *out) {
  const BwppStr n = g->values[v].name;
  if (n.ptr && n.len && n.len < NAME_LEN && !(n.ptr[0] == '-' || (n.ptr[0] >= '0' && n.ptr[0] <= '9')))
    str_copy(out, NAME_LEN, n.ptr, n.len);
  else
    snprintf(out, NAME_LEN, "%s%u", dflt, v);
}

/* ------------------------------------------------------------ graph walk */

static int gctx_init(Ctx *c, GCtx *gc, const BwppGraph *g, int is_grad) {
  memset(gc, 0, sizeof *gc);
  gc->g = g;
  gc->is_grad = is_grad;
  gc->lv = (LVal *)calloc(g->value_count ? g->value_count : 1, sizeof(LVal));
  gc->cons = (uint32_t **)calloc(g->value_count ? g->value_count : 1, sizeof(uint32_t *));
  gc->ncons = (uint32_t *)calloc(g->value_count ? g->value_count : 1, sizeof(uint32_t));
  gc->skip = (uint8_t *)calloc(g->node_count ? g->node_count : 1, 1);
  if (!gc->lv || !gc->cons || !gc->ncons || !gc->skip) {
    fail(c, "out of memory");
    return 0;
  }
  for (uint32_t v = 0; v < g->value_count; ++v) gc->lv[v].pv = -1;
  for (uint32_t i = 0; i < g->node_count; ++i) {
    const BwppGraphNode *n = &g->nodes[i];
    for (uint32_t j = 0; j < n->input_count && j < BWPP_GRAPH_MAX_INPUTS; ++j) {
      const uint32_t v = n->inputs[j];
      if (v >= g->value_count) continue;
      uint32_t *p = (uint32_t *)realloc(gc->cons[v], (gc->ncons[v] + 1) * sizeof(uint32_t));
      if (!p) {
        fail(c, "out of memory");
        return 0;
      }
      gc->cons[v] = p;
      gc->cons[v][gc->ncons[v]++] = i;
    }
  }
  return 1;
}

static void gctx_free(GCtx *gc) {
  if (gc->cons)
    for (uint32_t v = 0; v < gc->g->value_count; ++v) free(gc->cons[v]);
  free(gc->cons);
  free(gc->ncons);
  free(gc->lv);
  free(gc->skip);
}

static int is_output(const BwppGraph *g, uint32_t v) {
  for (uint32_t i = 0; i < g->output_count; ++i)
    if (g->outputs[i] == v) return 1;
  return 0;
}

static int producer_op(const BwppGraph *g, uint32_t v, BwppGraphOpKind op) {
  if (v >= g->value_count) return -1;
  const uint32_t p = g->values[v].producer;
  if (p == BWPP_GRAPH_NO_NODE || p >= g->node_count || g->nodes[p].op != op) return -1;
  return (int)p;
}

/* Forward activations the autodiff pass imports, in import order: the same
 * walk as graph_ir.c:1520-1822 (which inputs get a gradient, which values
 * each rule imports).  Forward inputs are imported up front
 * (graph_ir.c:1507-1511) and are not part of the list. */
static int replay_imports(const BwppGraph *f, uint32_t *order, uint32_t *count, uint8_t *imported, uint8_t *has) {
  *count = 0;
  for (uint32_t v = 0; v < f->value_count; ++v)
    imported[v] = (f->values[v].flags & BWPP_GRAPH_VALUE_INPUT) ? 1 : 0;
  for (uint32_t i = 0; i < f->output_count; ++i) has[f->outputs[i]] = 1;
#define IMPORT(x)                  \
  do {                             \
    const uint32_t x_ = (x);       \
    if (!imported[x_]) {           \
      imported[x_] = 2;            \
      order[(*count)++] = x_;      \
    }                              \
  } while (0)
  for (int32_t i = (int32_t)f->node_count - 1; i >= 0; --i) {
    const BwppGraphNode *n = &f->nodes[i];
    if (!has[n->output]) continue;
    const uint32_t ic = n->input_count;
    switch (n->op) {
      case BWPP_GOP_MATMUL:
      case BWPP_GOP_MUL:
      case BWPP_GOP_DIV:
        if (ic < 2) break;
        IMPORT(n->inputs[0]);
        IMPORT(n->inputs[1]);
        has[n->inputs[0]] = has[n->inputs[1]] = 1;
        break;
      case BWPP_GOP_ADD:
      case BWPP_GOP_SUB:
        if (ic < 2) break;
        has[n->inputs[0]] = has[n->inputs[1]] = 1;
        break;
      case BWPP_GOP_TRANSPOSE:
      case BWPP_GOP_PERMUTE:
      case BWPP_GOP_RESHAPE:
      case BWPP_GOP_REDUCE_SUM:
        if (ic < 1) break;
        has[n->inputs[0]] = 1;
        break;
      case BWPP_GOP_SILU:
      case BWPP_GOP_REDUCE_MAX:
        if (ic < 1) break;
        IMPORT(n->inputs[0]);
        has[n->inputs[0]] = 1;
        break;
      case BWPP_GOP_SOFTMAX:
        if (ic < 1) break;
        IMPORT(n->output);
        has[n->inputs[0]] = 1;
        break;
      case BWPP_GOP_RMSNORM:
        if (ic < 2) break;
        IMPORT(n->inputs[0]);
        IMPORT(n->inputs[1]);
        IMPORT(n->output);
        if (ic >= 3) IMPORT(n->inputs[2]);
        has[n->inputs[0]] = has[n->inputs[1]] = 1;
        if (ic >= 3) has[n->inputs[2]] = 1;
        break;
      default:
        break;
    }
  }
#undef IMPORT
  return 1;
}

/* ------------------------------------------------------------ operands */

/* Ops refer to plan values as $index$; names are final only when the plan
 * is written (outputs are renamed last). */
typedef struct {
  char s[24];
} Ref;

static Ref ref(int pv) {
  Ref r;
  snprintf(r.s, sizeof r.s, "$%d$", pv);
  return r;
}

/* Reference to a value used as a plain (untransposed, unbroadcast) operand. */
static Ref operand(Ctx *c, const GCtx *gc, uint32_t v) {
  const LVal *l = &gc->lv[v];
  if (l->pv < 0) {
    fail(c, "value v%u is used before it is computed (or only inside a fused region)", v);
    return ref(0);
  }
  if (l->trans || l->bcast) {
    fail(c, "value v%u is a transposed or broadcast view where a plain tensor is needed", v);
    return ref(0);
  }
  return ref(l->pv);
}

/* How value `v` enters an elementwise op whose result has shape `o`. */
static int classify(const GCtx *gc, uint32_t v, const Shape *o) {
  const LVal *l = &gc->lv[v];
  if (l->trans) return BC_BAD;
  const uint64_t cols = o->rank ? o->n[o->rank - 1] : 1;
  const uint64_t rows = o->rank ? shape_elems(o) / (cols ? cols : 1) : 1;
  const Shape *s = l->bcast ? &l->src : &l->shape;
  const uint64_t e = shape_elems(s);
  if (!l->bcast && e == rows * cols && (s->rank == 0 || s->n[s->rank - 1] == cols)) return BC_FULL;
  if (e == 1) return BC_SCALAR;
  int lead_ones = 1;
  for (uint32_t i = 0; i + 1 < s->rank; ++i)
    if (s->n[i] != 1) lead_ones = 0;
  if (e == cols && lead_ones) return BC_ROW;
  if (e == rows && s->rank >= 1 && s->n[s->rank - 1] == 1) return BC_COL;
  if (e == rows && s->rank == 1 && rows != cols) return BC_COL;
  return BC_BAD;
}

static const char *bc_name(int b) {
  return b == BC_ROW ? "row" : b == BC_COL ? "col" : b == BC_SCALAR ? "scalar" : "full";
}

/* Broadcast result shape of two shapes (numpy rules on bound values). */
static int broadcast_shape(Ctx *c, const Shape *a, const Shape *b, Shape *o) {
  memset(o, 0, sizeof *o);
  o->rank = a->rank > b->rank ? a->rank : b->rank;
  for (uint32_t i = 0; i < o->rank; ++i) {
    const int ai = (int)a->rank - 1 - (int)i, bi = (int)b->rank - 1 - (int)i;
    const uint64_t an = ai >= 0 ? a->n[ai] : 1, bn = bi >= 0 ? b->n[bi] : 1;
    const char *ad = ai >= 0 ? a->d[ai] : "1", *bd = bi >= 0 ? b->d[bi] : "1";
    const uint32_t oi = o->rank - 1 - i;
    if (an == bn || bn == 1)
      shape_set_dim(o, oi, ad, an);
    else if (an == 1)
      shape_set_dim(o, oi, bd, bn);
    else {
      fail(c, "shapes do not broadcast (%s vs %s)", ad, bd);
      return 0;
    }
  }
  return 1;
}

static int lval_batched(const Ctx *c, const Shape *s) {
  return c->opt->batch > 1 && s->rank >= 1 && strcmp(s->d[0], c->batch_dim) == 0;
}

/* Gives graph value `v` a fresh plan value (temp) for its shape. */
static int assign_pv(Ctx *c, GCtx *gc, uint32_t v, const char *prefix) {
  LVal *l = &gc->lv[v];
  if (l->preset) return l->pv;
  char base[NAME_LEN];
  value_name(gc->g, v, prefix, base);
  l->batched = lval_batched(c, &l->shape);
  l->pv = new_pv(c, base, &l->shape, l->batched, l->bf16, "temp");
  l->trans = l->bcast = 0;
  return l->pv;
}

/* ------------------------------------------------------------ fused regions */

/* q @ transpose(k) -> softmax -> @ v, with nothing else reading the scores,
 * the probabilities or transpose(k) in the forward graph. */
static void find_attention(Ctx *c, GCtx *gc) {
  const BwppGraph *g = gc->g;
  for (uint32_t i = 0; i < g->node_count; ++i) {
    const BwppGraphNode *sm = &g->nodes[i];
    if (sm->op != BWPP_GOP_SOFTMAX || sm->input_count < 1) continue;
    const int mm1 = producer_op(g, sm->inputs[0], BWPP_GOP_MATMUL);
    if (mm1 < 0 || g->nodes[mm1].input_count < 2) continue;
    const uint32_t q = g->nodes[mm1].inputs[0], kt = g->nodes[mm1].inputs[1];
    const int tk = producer_op(g, kt, BWPP_GOP_TRANSPOSE);
    if (tk < 0 || g->nodes[tk].input_count < 1) continue;
    const uint32_t s = sm->output;
    if (gc->ncons[s] != 1 || gc->ncons[sm->inputs[0]] != 1 || gc->ncons[kt] != 1) continue;
    const BwppGraphNode *mm2 = &g->nodes[gc->cons[s][0]];
    if (mm2->op != BWPP_GOP_MATMUL || mm2->input_count < 2 || mm2->inputs[0] != s) continue;
    if (is_output(g, s) || is_output(g, sm->inputs[0]) || is_output(g, kt)) continue;
    if (sm->attr.has_axis && sm->attr.axis != (int)g->values[q].shape.rank - 1 &&
        g->values[q].shape.rank != 0)
      continue;
    AttnRegion r;
    memset(&r, 0, sizeof r);
    r.mm1 = mm1;
    r.tk = tk;
    r.sm = (int)i;
    r.mm2 = (int)gc->cons[s][0];
    r.q = q;
    r.k = g->nodes[tk].inputs[0];
    r.v = mm2->inputs[1];
    r.kt = kt;
    r.s = s;
    r.o = mm2->output;
    r.lse_pv = -1;
    AttnRegion *p = (AttnRegion *)realloc(c->regions, (size_t)(c->nregions + 1) * sizeof(AttnRegion));
    if (!p) {
      fail(c, "out of memory");
      return;
    }
    c->regions = p;
    c->regions[c->nregions++] = r;
    gc->skip[mm1] = gc->skip[tk] = gc->skip[i] = gc->skip[r.mm2] = 1;
  }
}

/* Shortest decimal that reads back as the same float. */
static void fmt_float(char *buf, size_t cap, double v) {
  for (int prec = 6; prec <= 9; ++prec) {
    snprintf(buf, cap, "%.*g", prec, v);
    if ((float)strtod(buf, NULL) == (float)v) return;
  }
}

static void attn_attrs(Ctx *c, const AttnRegion *r, char *buf, size_t cap) {
  char scale[32];
  if (c->opt->attn_scale_auto)
    strcpy(scale, "auto");
  else
    fmt_float(scale, sizeof scale, (double)r->scale);
  /* rank-2 regions take batch / heads from the plan's BATCH / HEADS dims,
   * so a plan's sizes can be rebound without lowering it again */
  if (r->bhsd)  /* batch / heads: the dims of q's [B, H, T, d] shape */
    snprintf(buf, cap, "batch=%s heads=%s causal=%d scale=%s layout=bhsd", r->bdim, r->hdim,
             c->opt->causal ? 1 : 0, scale);
  else
    snprintf(buf, cap, "batch=%s heads=HEADS causal=%d scale=%s", c->opt->batch > 1 ? "BATCH" : "1",
             c->opt->causal ? 1 : 0, scale);
}

static void lower_attention(Ctx *c, GCtx *gc, AttnRegion *r, int with_lse) {
  LVal *q = &gc->lv[r->q], *k = &gc->lv[r->k], *v = &gc->lv[r->v];
  if (!q->known || !k->known || !v->known) {
    fail(c, "attention operands without shapes");
    return;
  }
  const Shape *qs = &q->shape;
  uint32_t dk;
  if (qs->rank == 4) {
    if (c->opt->batch > 1) {
      fail(c, "--batch applies to rank-2 graphs; a rank-4 attention carries its own batch dim");
      return;
    }
    r->bhsd = 1;
    r->batch = (uint32_t)qs->n[0];
    r->heads = (uint32_t)qs->n[1];
    strcpy(r->bdim, qs->d[0]);
    strcpy(r->hdim, qs->d[1]);
    dk = (uint32_t)qs->n[3];
    if (k->shape.rank != 4 || v->shape.rank != 4 || k->shape.n[0] != qs->n[0] || k->shape.n[1] != qs->n[1] ||
        k->shape.n[3] != qs->n[3] || v->shape.n[2] != k->shape.n[2]) {
      fail(c, "rank-4 attention operands disagree");
      return;
    }
  } else if (qs->rank == 2) {
    r->bhsd = 0;
    r->batch = c->opt->batch > 1 ? c->opt->batch : 1;
    r->heads = c->opt->heads ? c->opt->heads : 1;
    if (qs->n[1] % r->heads || v->shape.n[1] % r->heads || k->shape.n[1] != qs->n[1]) {
      fail(c, "attention: %u heads do not divide the q/k/v widths", r->heads);
      return;
    }
    if (c->opt->batch > 1 && (!q->batched || !k->batched || !v->batched)) {
      fail(c, "attention over a batch needs q, k and v stacked along the batch dim");
      return;
    }
    dk = (uint32_t)(qs->n[1] / r->heads);
  } else {
    fail(c, "attention needs rank-2 [T, D] or rank-4 [B, H, T, d] operands");
    return;
  }
  {
    const BwppGraphNode *sm = &gc->g->nodes[r->sm];
    if (sm->attr.has_axis && sm->attr.axis != (int)qs->rank - 1) {
      fail(c, "attention softmax over axis %d (only the key axis, the last, is supported)", sm->attr.axis);
      return;
    }
  }
  r->scale = c->opt->attn_scale_auto ? (float)(1.0 / sqrt((double)dk))
                                     : (c->opt->attn_scale != 0.0f ? c->opt->attn_scale : 1.0f);
  LVal *o = &gc->lv[r->o];
  o->shape = *qs;
  shape_set_dim(&o->shape, o->shape.rank - 1, v->shape.d[v->shape.rank - 1], v->shape.n[v->shape.rank - 1]);
  o->known = 1;
  o->bf16 = q->bf16;
  assign_pv(c, gc, r->o, "att");
  const Ref qn = operand(c, gc, r->q), kn = operand(c, gc, r->k), vn = operand(c, gc, r->v);
  char attrs[320];
  attn_attrs(c, r, attrs, sizeof attrs);
  if (with_lse) {
    Shape ls;
    memset(&ls, 0, sizeof ls);
    ls.rank = 3;
    if (r->bhsd) {
      shape_set_dim(&ls, 0, qs->d[0], qs->n[0]);
      shape_set_dim(&ls, 1, qs->d[1], qs->n[1]);
      shape_set_dim(&ls, 2, qs->d[2], qs->n[2]);
    } else {
      if (c->opt->batch > 1)
        shape_set_dim(&ls, 0, "BATCH", c->opt->batch);
      else
        shape_set_dim(&ls, 0, "1", 1);
      shape_set_dim(&ls, 1, "HEADS", r->heads);
      shape_set_dim(&ls, 2, qs->d[0], qs->n[0]);
    }
    r->lse_pv = new_pv(c, "lse", &ls, 0, 0, "temp");
    emit(c, "op attention out=%s,%s in=%s,%s,%s %s\n", ref(o->pv).s, ref(r->lse_pv).s, qn.s, kn.s, vn.s, attrs);
  } else {
    emit(c, "op attention out=%s in=%s,%s,%s %s\n", ref(o->pv).s, qn.s, kn.s, vn.s, attrs);
  }
  gc->lv[r->s].fused = gc->lv[r->kt].fused = gc->lv[gc->g->nodes[r->mm1].output].fused = 1;
}

/* The autodiff chain of one attention region in the autodiff graph
 * (matmul rule graph_ir.c:1529-1583, softmax rule 1722-1733, transpose
 * rule 1656-1670), x' being the clone of forward value x:
 *   dP  = dO @ transpose(v')           dV  = transpose(S') @ dO
 *   dS  = softmax_grad(S', dP)
 *   dQ  = dS @ transpose(kT')          dKT = transpose(q') @ dS
 *   dK  = transpose(dKT)
 * It becomes one attention_grad launch, emitted where dP is. */
typedef struct {
  int region;
  int first;            /* node that emits the fused op */
  uint32_t dout, dq, dk, dv;
} AttnGrad;

typedef struct {
  int rg;               /* rmsnorm_grad node (emits the fused op) */
  int div, mul, rsum;   /* the dGamma chain */
} NormGrad;

typedef struct {
  const BwppGraph *f;
  GCtx *fc;
  int32_t *g2f;         /* autodiff-graph clone -> forward value, -1 none */
  AttnGrad *ag;
  int nag;
  NormGrad *ng;
  int nng;
} Bwd;

static int clone_of(const Bwd *b, uint32_t gv, uint32_t fv) { return b->g2f[gv] == (int32_t)fv; }

/* Node `m`: MATMUL whose operand `side` is TRANSPOSE(clone of fv). */
static int mm_with_tclone(const Bwd *b, const GCtx *gc, int m, int side, uint32_t fv) {
  if (m < 0) return 0;
  const BwppGraphNode *n = &gc->g->nodes[m];
  if (n->op != BWPP_GOP_MATMUL || n->input_count < 2) return 0;
  const int t = producer_op(gc->g, n->inputs[side], BWPP_GOP_TRANSPOSE);
  if (t < 0 || gc->ncons[n->inputs[side]] != 1) return 0;
  return clone_of(b, gc->g->nodes[t].inputs[0], fv);
}

static void find_attention_grads(Ctx *c, GCtx *gc, Bwd *b) {
  const BwppGraph *g = gc->g;
  for (int r = 0; r < c->nregions; ++r) {
    const AttnRegion *R = &c->regions[r];
    int sg = -1;
    for (uint32_t i = 0; i < g->node_count && sg < 0; ++i)
      if (g->nodes[i].op == BWPP_GOP_SOFTMAX_GRAD && g->nodes[i].input_count >= 2 &&
          clone_of(b, g->nodes[i].inputs[0], R->s))
        sg = (int)i;
    if (sg < 0) {
      fail(c, "attention region %d: no softmax_grad over its probabilities in the autodiff graph", r);
      return;
    }
    const uint32_t dp = g->nodes[sg].inputs[1], ds = g->nodes[sg].output;
    const int b1 = producer_op(g, dp, BWPP_GOP_MATMUL);
    if (!mm_with_tclone(b, gc, b1, 1, R->v) || gc->ncons[dp] != 1) {
      fail(c, "attention region %d: dP is not dO @ transpose(v)", r);
      return;
    }
    const uint32_t dout = g->nodes[b1].inputs[0];
    int b2 = -1, b4 = -1, b5 = -1;
    for (uint32_t j = 0; j < gc->ncons[dout]; ++j) {
      const int m = (int)gc->cons[dout][j];
      if (g->nodes[m].inputs[1] == dout && mm_with_tclone(b, gc, m, 0, R->s)) b2 = m;
    }
    for (uint32_t j = 0; j < gc->ncons[ds]; ++j) {
      const int m = (int)gc->cons[ds][j];
      if (g->nodes[m].inputs[0] == ds && mm_with_tclone(b, gc, m, 1, R->kt)) b4 = m;
      if (g->nodes[m].inputs[1] == ds && mm_with_tclone(b, gc, m, 0, R->q)) b5 = m;
    }
    if (b2 < 0 || b4 < 0 || b5 < 0 || gc->ncons[ds] != 2) {
      fail(c, "attention region %d: the autodiff chain of the attention does not have its expected form", r);
      return;
    }
    const uint32_t dkt = g->nodes[b5].output;
    if (gc->ncons[dkt] != 1 || g->nodes[gc->cons[dkt][0]].op != BWPP_GOP_TRANSPOSE) {
      fail(c, "attention region %d: dK^T is not transposed back", r);
      return;
    }
    const int b6 = (int)gc->cons[dkt][0];
    const int nodes[] = {b1, b2, sg, b4, b5, b6};
    int first = b1;
    for (int k = 0; k < 6; ++k) {
      gc->skip[nodes[k]] = 1;
      if (nodes[k] < first) first = nodes[k];
      if (k != 2 && k != 5)  /* the matmuls' transpose operands */
        for (int side = 0; side < 2; ++side) {
          const int t = producer_op(g, g->nodes[nodes[k]].inputs[side], BWPP_GOP_TRANSPOSE);
          if (t >= 0 && gc->ncons[g->nodes[nodes[k]].inputs[side]] == 1) gc->skip[t] = 1;
        }
    }
    AttnGrad *p = (AttnGrad *)realloc(b->ag, (size_t)(b->nag + 1) * sizeof(AttnGrad));
    if (!p) {
      fail(c, "out of memory");
      return;
    }
    b->ag = p;
    AttnGrad *a = &b->ag[b->nag++];
    a->region = r;
    a->first = first;
    a->dout = dout;
    a->dq = g->nodes[b4].output;
    a->dk = g->nodes[b6].output;
    a->dv = g->nodes[b2].output;
  }
}

/* rmsnorm_grad(x', g', dY) with the dGamma chain of graph_ir.c:1747-1781
 * (no beta): reduce_sum(dY * (Y' / g'), axis 0). */
static void find_norm_grads(Ctx *c, GCtx *gc, Bwd *b) {
  const BwppGraph *g = gc->g;
  for (uint32_t i = 0; i < g->node_count; ++i) {
    const BwppGraphNode *rg = &g->nodes[i];
    if (rg->op != BWPP_GOP_RMSNORM_GRAD || rg->input_count < 3) continue;
    const int32_t fx = b->g2f[rg->inputs[0]], fg = b->g2f[rg->inputs[1]];
    if (fx < 0 || fg < 0) continue;
    int fy = -1;  /* the forward rmsnorm's output */
    for (uint32_t k = 0; k < b->f->node_count; ++k) {
      const BwppGraphNode *fn = &b->f->nodes[k];
      if (fn->op == BWPP_GOP_RMSNORM && fn->input_count == 2 && fn->inputs[0] == (uint32_t)fx &&
          fn->inputs[1] == (uint32_t)fg)
        fy = (int)fn->output;
    }
    if (fy < 0) continue;
    for (uint32_t j = i + 1; j < g->node_count; ++j) {
      const BwppGraphNode *dv = &g->nodes[j];
      if (dv->op != BWPP_GOP_DIV || dv->input_count < 2 || dv->inputs[1] != rg->inputs[1] ||
          !clone_of(b, dv->inputs[0], (uint32_t)fy) || gc->ncons[dv->output] != 1)
        continue;
      const int mu = (int)gc->cons[dv->output][0];
      const BwppGraphNode *mn = &g->nodes[mu];
      if (mn->op != BWPP_GOP_MUL || mn->input_count < 2 || mn->inputs[0] != rg->inputs[2] ||
          mn->inputs[1] != dv->output || gc->ncons[mn->output] != 1)
        continue;
      const int rs = (int)gc->cons[mn->output][0];
      const BwppGraphNode *rn = &g->nodes[rs];
      if (rn->op != BWPP_GOP_REDUCE_SUM || !rn->attr.has_axis || rn->attr.axis != 0) continue;
      if (gc->lv[rg->inputs[0]].shape.rank != 2) continue;
      NormGrad *p = (NormGrad *)realloc(b->ng, (size_t)(b->nng + 1) * sizeof(NormGrad));
      if (!p) {
        fail(c, "out of memory");
        return;
      }
      b->ng = p;
      b->ng[b->nng++] = (NormGrad){(int)i, (int)j, mu, rs};
      gc->skip[j] = gc->skip[mu] = gc->skip[rs] = 1;
      break;
    }
  }
}

/* ------------------------------------------------------------ sibling GEMMs */

static void need_known(Ctx *c, const GCtx *gc, uint32_t v);

/* A forward matmul whose result lower_matmul would not fuse into an
 * epilogue or emit transposed: the candidates for grouping. */
static int mm_groupable(const GCtx *gc, uint32_t node) {
  const BwppGraph *g = gc->g;
  const BwppGraphNode *n = &g->nodes[node];
  if (n->op != BWPP_GOP_MATMUL || n->input_count < 2 || gc->skip[node]) return 0;
  const uint32_t w = n->inputs[1], y = n->output;
  if (!(g->values[w].flags & BWPP_GRAPH_VALUE_INPUT) || g->values[w].shape.rank != 2) return 0;
  if (is_output(g, y)) return 0;
  /* the result becomes a strided column view: only readers that take a row
   * stride (a fused attention region, another matmul) */
  for (uint32_t j = 0; j < gc->ncons[y]; ++j) {
    const uint32_t k = gc->cons[y][j];
    if (!gc->skip[k] && g->nodes[k].op != BWPP_GOP_MATMUL) return 0;
  }
  return 1;
}

static int same_shape_text(const BwppShape *a, const BwppShape *b) {
  if (a->rank != b->rank) return 0;
  for (uint32_t i = 0; i < a->rank; ++i)
    if (a->dims[i].len != b->dims[i].len || memcmp(a->dims[i].ptr, b->dims[i].ptr, a->dims[i].len)) return 0;
  return 1;
}

static void find_mm_groups(Ctx *c, GCtx *gc) {
  const BwppGraph *g = gc->g;
  uint8_t *taken = (uint8_t *)calloc(g->node_count ? g->node_count : 1, 1);
  if (!taken) {
    fail(c, "out of memory");
    return;
  }
  for (uint32_t i = 0; i < g->node_count; ++i) {
    if (taken[i] || !mm_groupable(gc, i)) continue;
    const BwppGraphNode *ni = &g->nodes[i];
    MMGroup G;
    memset(&G, 0, sizeof G);
    G.a = ni->inputs[0];
    G.node[0] = (int)i;
    G.w[0] = ni->inputs[1];
    G.y[0] = ni->output;
    G.n = 1;
    for (uint32_t j = i + 1; j < g->node_count && G.n < MM_GROUP_MAX; ++j) {
      const BwppGraphNode *nj = &g->nodes[j];
      if (taken[j] || !mm_groupable(gc, j) || nj->inputs[0] != G.a) continue;
      const BwppGraphValue *wi = &g->values[G.w[0]], *wj = &g->values[nj->inputs[1]];
      if (wi->dtype != wj->dtype || !same_shape_text(&wi->shape, &wj->shape) || nj->inputs[1] == G.w[0]) continue;
      G.node[G.n] = (int)j;
      G.w[G.n] = nj->inputs[1];
      G.y[G.n] = nj->output;
      ++G.n;
    }
    if (G.n < 2) continue;
    for (int m = 0; m < G.n; ++m) {
      taken[G.node[m]] = 1;
      if (m) gc->skip[G.node[m]] = 1;
    }
    G.wcat_pv = -1;
    G.first_bwd = -1;
    MMGroup *p = (MMGroup *)realloc(c->groups, (size_t)(c->ngroups + 1) * sizeof(MMGroup));
    if (!p) {
      fail(c, "out of memory");
      break;
    }
    c->groups = p;
    c->groups[c->ngroups++] = G;
  }
  free(taken);
}

/* "m*N" for column block m of width N (dim text). */
static void block_expr(char *buf, size_t cap, int m, const char *n) {
  if (m == 0)
    snprintf(buf, cap, "0");
  else if (m == 1)
    snprintf(buf, cap, "%s", n);
  else
    snprintf(buf, cap, "%d*%s", m, n);
}

/* Emits a forward group at its first node: the weight concatenation, one
 * GEMM, and the members' results as column views. */
static void lower_mm_group(Ctx *c, GCtx *gc, MMGroup *G) {
  const LVal *A = &gc->lv[G->a];
  need_known(c, gc, G->a);
  if (c->failed) return;
  if (A->shape.rank != 2 || A->trans || A->bcast || A->pv < 0) {
    fail(c, "grouped matmul: left operand v%u is not a plain matrix", G->a);
    return;
  }
  const LVal *W0 = &gc->lv[G->w[0]];
  if (W0->shape.rank != 2 || W0->shape.n[0] != A->shape.n[1] || W0->bf16 != A->bf16) {
    fail(c, "grouped matmul: weight shape or dtype does not match the left operand");
    return;
  }
  char ncat[DIM_LEN + 8], off[DIM_LEN + 8], nm[NAME_LEN];
  snprintf(ncat, sizeof ncat, "%d*%s", G->n, W0->shape.d[1]);
  Shape ws = W0->shape;
  shape_set_dim(&ws, 1, ncat, W0->shape.n[1] * (uint64_t)G->n);
  G->wcat_pv = new_pv(c, "wcat", &ws, 0, A->bf16, "temp");
  for (int m = 0; m < G->n; ++m) {
    block_expr(off, sizeof off, m, W0->shape.d[1]);
    value_name(gc->g, G->w[m], "w", nm);
    char vn[NAME_LEN + 8];
    snprintf(vn, sizeof vn, "%s_in_cat", nm);
    const int view = new_view(c, G->wcat_pv, vn, &W0->shape, 0, off, ncat);
    emit(c, "op copy out=%s in=%s bcast=full\n", ref(view).s, operand(c, gc, G->w[m]).s);
  }
  Shape ys;
  memset(&ys, 0, sizeof ys);
  ys.rank = 2;
  shape_set_dim(&ys, 0, A->shape.d[0], A->shape.n[0]);
  shape_set_dim(&ys, 1, ncat, W0->shape.n[1] * (uint64_t)G->n);
  const int ycat = new_pv(c, "ycat", &ys, A->batched, A->bf16, "temp");
  emit(c, "op matmul out=%s in=%s,%s\n", ref(ycat).s, ref(A->pv).s, ref(G->wcat_pv).s);
  for (int m = 0; m < G->n; ++m) {
    LVal *Y = &gc->lv[G->y[m]];
    memset(&Y->shape, 0, sizeof Y->shape);
    Y->shape.rank = 2;
    shape_set_dim(&Y->shape, 0, A->shape.d[0], A->shape.n[0]);
    shape_set_dim(&Y->shape, 1, W0->shape.d[1], W0->shape.n[1]);
    Y->known = 1;
    Y->bf16 = A->bf16;
    Y->batched = A->batched;
    Y->trans = Y->bcast = 0;
    block_expr(off, sizeof off, m, W0->shape.d[1]);
    value_name(gc->g, G->y[m], "y", nm);
    Y->pv = new_view(c, ycat, nm, &Y->shape, Y->batched, off, ncat);
  }
}

/* The members' autodiff terms (see MMGroup).  Applies when every dY_m is
 * an output of a fused attention_grad (which writes strided blocks) and is
 * read only by its dW_m and dA_m. */
static void find_mm_group_grads(Ctx *c, GCtx *gc, Bwd *b) {
  const BwppGraph *g = gc->g;
  uint8_t *mask = (uint8_t *)calloc(g->value_count ? g->value_count : 1, 1);
  if (!mask) {
    fail(c, "out of memory");
    return;
  }
  for (int gi = 0; gi < c->ngroups; ++gi) {
    MMGroup *G = &c->groups[gi];
    G->bwd = G->da = 0;
    if (G->wcat_pv < 0) continue;
    int ok = 1;
    for (int m = 0; m < G->n && ok; ++m) {
      int da = -1, dw = -1;
      for (uint32_t i = 0; i < g->node_count && da < 0; ++i)
        if (!gc->skip[i] && mm_with_tclone(b, gc, (int)i, 1, G->w[m])) da = (int)i;
      if (da < 0) {
        ok = 0;
        break;
      }
      const uint32_t dy = g->nodes[da].inputs[0];
      for (uint32_t j = 0; j < gc->ncons[dy]; ++j) {
        const int k = (int)gc->cons[dy][j];
        if (k != da && g->nodes[k].input_count >= 2 && g->nodes[k].inputs[1] == dy &&
            mm_with_tclone(b, gc, k, 0, G->a))
          dw = k;
      }
      int from_attn = 0;
      for (int a = 0; a < b->nag; ++a)
        from_attn |= b->ag[a].dq == dy || b->ag[a].dk == dy || b->ag[a].dv == dy;
      /* dW_m becomes a view too: it must be read by nothing (a grad output) */
      if (dw < 0 || gc->ncons[dy] != 2 || !from_attn || is_output(g, dy) ||
          gc->ncons[g->nodes[dw].output] != 0)
        ok = 0;
      G->da_node[m] = da;
      G->dw_node[m] = dw;
      G->dy[m] = dy;
    }
    if (!ok) continue;
    G->bwd = 1;
    /* the adds that sum the dA_m */
    memset(mask, 0, g->value_count);
    const uint8_t full = (uint8_t)((1u << G->n) - 1u);
    int da_ok = 1;
    for (int m = 0; m < G->n; ++m) {
      const uint32_t o = g->nodes[G->da_node[m]].output;
      if (gc->ncons[o] != 1 || is_output(g, o)) da_ok = 0;
      mask[o] = (uint8_t)(1u << m);
    }
    int adds[MM_GROUP_MAX], nadds = 0;
    int32_t sum = -1;
    for (uint32_t i = 0; i < g->node_count && da_ok && sum < 0; ++i) {
      const BwppGraphNode *n = &g->nodes[i];
      if (n->op != BWPP_GOP_ADD || n->input_count < 2 || gc->skip[i]) continue;
      const uint8_t ma = mask[n->inputs[0]], mb = mask[n->inputs[1]];
      if (!ma || !mb) continue;
      if ((ma & mb) || gc->ncons[n->inputs[0]] != 1 || gc->ncons[n->inputs[1]] != 1 || nadds >= MM_GROUP_MAX) {
        da_ok = 0;
        break;
      }
      adds[nadds++] = (int)i;
      mask[n->output] = (uint8_t)(ma | mb);
      if (mask[n->output] == full) sum = (int32_t)n->output;
    }
    G->da = da_ok && sum >= 0;
    G->first_bwd = G->dw_node[0];
    for (int m = 0; m < G->n; ++m) {
      if (G->dw_node[m] < G->first_bwd) G->first_bwd = G->dw_node[m];
      gc->skip[G->dw_node[m]] = 1;
      if (G->da) {
        if (G->da_node[m] < G->first_bwd) G->first_bwd = G->da_node[m];
        gc->skip[G->da_node[m]] = 1;
      }
    }
    if (G->da) {
      G->da_sum = (uint32_t)sum;
      for (int k = 0; k < nadds; ++k) gc->skip[adds[k]] = 1;
    }
    /* dY_m: column views of one [rows, n*N] buffer, filled by attention_grad */
    const LVal *Y0 = &b->fc->lv[G->y[0]];
    char ncat[DIM_LEN + 8], off[DIM_LEN + 8], nm[NAME_LEN];
    snprintf(ncat, sizeof ncat, "%d*%s", G->n, Y0->shape.d[1]);
    Shape ys = Y0->shape;
    shape_set_dim(&ys, 1, ncat, Y0->shape.n[1] * (uint64_t)G->n);
    const int dycat = new_pv(c, "dycat", &ys, Y0->batched, Y0->bf16, "temp");
    for (int m = 0; m < G->n; ++m) {
      LVal *l = &gc->lv[G->dy[m]];
      l->shape = Y0->shape;
      l->known = 1;
      l->bf16 = Y0->bf16;
      l->batched = Y0->batched;
      l->trans = l->bcast = 0;
      block_expr(off, sizeof off, m, Y0->shape.d[1]);
      value_name(b->f, G->y[m], "y", nm);
      char vn[NAME_LEN + 8];
      snprintf(vn, sizeof vn, "d%s", nm);
      l->pv = new_view(c, dycat, vn, &Y0->shape, Y0->batched, off, ncat);
      l->preset = 1;
    }
  }
  free(mask);
}

/* The backward GEMMs of a group, at its first autodiff node. */
static void lower_mm_group_grad(Ctx *c, GCtx *gc, const Bwd *b, const MMGroup *G) {
  const GCtx *fc = b->fc;
  const LVal *A = &fc->lv[G->a], *W0 = &fc->lv[G->w[0]];
  const int dycat = c->pv[gc->lv[G->dy[0]].pv].view_of;
  char ncat[DIM_LEN + 8], off[DIM_LEN + 8];
  snprintf(ncat, sizeof ncat, "%d*%s", G->n, W0->shape.d[1]);
  Shape ws = W0->shape;
  shape_set_dim(&ws, 1, ncat, W0->shape.n[1] * (uint64_t)G->n);
  const int dwcat = new_pv(c, "dwcat", &ws, 0, A->bf16, "temp");
  emit(c, "op matmul out=%s in=%s,%s ta=1\n", ref(dwcat).s, ref(A->pv).s, ref(dycat).s);
  for (int m = 0; m < G->n; ++m) {
    LVal *l = &gc->lv[gc->g->nodes[G->dw_node[m]].output];
    l->shape = W0->shape;
    l->known = 1;
    l->bf16 = A->bf16;
    l->batched = 0;
    l->trans = l->bcast = 0;
    block_expr(off, sizeof off, m, W0->shape.d[1]);
    char nm[NAME_LEN], vn[NAME_LEN + 8];
    value_name(b->f, G->w[m], "w", nm);
    snprintf(vn, sizeof vn, "d%s_in_cat", nm);
    l->pv = new_view(c, dwcat, vn, &W0->shape, 0, off, ncat);
  }
  if (G->da) {
    LVal *l = &gc->lv[G->da_sum];
    l->shape = A->shape;
    l->known = 1;
    l->bf16 = A->bf16;
    assign_pv(c, gc, G->da_sum, "t");
    emit(c, "op matmul out=%s in=%s,%s tb=1\n", ref(l->pv).s, ref(dycat).s, ref(G->wcat_pv).s);
  }
}

/* ------------------------------------------------------------ node rules */

static void need_known(Ctx *c, const GCtx *gc, uint32_t v) {
  if (!gc->lv[v].known) fail(c, "value v%u has no inferred shape (unsupported producer?)", v);
}

static void lower_elementwise(Ctx *c, GCtx *gc, uint32_t node, const char *opname) {
  const BwppGraphNode *n = &gc->g->nodes[node];
  uint32_t a = n->inputs[0], b = n->inputs[1];
  need_known(c, gc, a);
  need_known(c, gc, b);
  if (c->failed) return;
  LVal *out = &gc->lv[n->output];
  Shape o;
  if (!broadcast_shape(c, &gc->lv[a].shape, &gc->lv[b].shape, &o)) return;
  int ca = classify(gc, a, &o), cb = classify(gc, b, &o);
  const int commutes = !strcmp(opname, "add") || !strcmp(opname, "mul");
  Ref ar;
  if (ca != BC_FULL && cb == BC_FULL && commutes) {
    uint32_t t = a;
    a = b;
    b = t;
    int tc = ca;
    ca = cb;
    cb = tc;
  }
  if (cb == BC_BAD || ca == BC_BAD) {
    fail(c, "%s: operand shapes do not map to a broadcast mode (row, column, scalar)", opname);
    return;
  }
  out->shape = o;
  out->known = 1;
  out->bf16 = gc->lv[a].bf16;
  if (ca != BC_FULL) {  /* broadcast the first operand into a full temp */
    LVal tmp = *out;
    const int pv = new_pv(c, "bcast", &o, lval_batched(c, &o), tmp.bf16, "temp");
    emit(c, "op copy out=%s in=%s bcast=%s\n", ref(pv).s, ref(gc->lv[a].pv).s, bc_name(ca));
    ar = ref(pv);
  } else {
    ar = operand(c, gc, a);
  }
  if (gc->lv[b].pv < 0 || gc->lv[b].trans) {
    fail(c, "%s: second operand v%u is not materialised", opname, b);
    return;
  }
  assign_pv(c, gc, n->output, "t");
  emit(c, "op %s out=%s in=%s,%s bcast=%s\n", opname, ref(out->pv).s, ar.s, ref(gc->lv[b].pv).s, bc_name(cb));
}

static void lower_unary(Ctx *c, GCtx *gc, uint32_t node, const char *opname, const char *attrs) {
  const BwppGraphNode *n = &gc->g->nodes[node];
  need_known(c, gc, n->inputs[0]);
  if (c->failed) return;
  LVal *out = &gc->lv[n->output];
  out->shape = gc->lv[n->inputs[0]].shape;
  out->known = 1;
  out->bf16 = gc->lv[n->inputs[0]].bf16;
  char ins[256] = "";
  for (uint32_t j = 0; j < n->input_count; ++j) {
    need_known(c, gc, n->inputs[j]);
    const Ref r = operand(c, gc, n->inputs[j]);
    strncat(ins, j ? "," : "", sizeof ins - strlen(ins) - 1);
    strncat(ins, r.s, sizeof ins - strlen(ins) - 1);
  }
  assign_pv(c, gc, n->output, "t");
  emit(c, "op %s out=%s in=%s%s%s\n", opname, ref(out->pv).s, ins, attrs[0] ? " " : "", attrs);
}

static int is_needed(const uint8_t *needed, const GCtx *gc, uint32_t v) {
  return is_output(gc->g, v) || (needed && needed[v]);
}

static void lower_matmul(Ctx *c, GCtx *gc, uint32_t node, const uint8_t *needed) {
  const BwppGraph *g = gc->g;
  const BwppGraphNode *n = &g->nodes[node];
  const uint32_t a = n->inputs[0], b = n->inputs[1];
  need_known(c, gc, a);
  need_known(c, gc, b);
  if (c->failed) return;
  const LVal *A = &gc->lv[a], *B = &gc->lv[b];
  if (A->shape.rank != 2 || B->shape.rank != 2) {
    fail(c, "matmul of rank %u x %u outside a fused attention region (only rank-2 GEMMs run unfused)",
         A->shape.rank, B->shape.rank);
    return;
  }
  if (A->bcast || B->bcast || A->pv < 0 || B->pv < 0) {
    fail(c, "matmul operand not materialised");
    return;
  }
  if (A->shape.n[1] != B->shape.n[0]) {
    fail(c, "matmul contraction dims differ (%s = %llu vs %s = %llu)", A->shape.d[1],
         (unsigned long long)A->shape.n[1], B->shape.d[0], (unsigned long long)B->shape.n[0]);
    return;
  }
  if (A->bf16 != B->bf16) {
    fail(c, "matmul operands of different dtypes");
    return;
  }
  if (c->opt->batch > 1 && strcmp(B->shape.d[1], c->batch_dim) == 0) {
    fail(c, "matmul result has the batch dim as columns (it would mix samples): fuse it into an attention "
            "region or lower with --batch 1");
    return;
  }
  Shape o;
  memset(&o, 0, sizeof o);
  o.rank = 2;
  shape_set_dim(&o, 0, A->shape.d[0], A->shape.n[0]);
  shape_set_dim(&o, 1, B->shape.d[1], B->shape.n[1]);
  uint32_t last = n->output;
  const char *epi = "none";
  int bias = -1;
  if (!gc->is_grad && gc->ncons[last] == 1 && !is_needed(needed, gc, last) && !gc->skip[gc->cons[last][0]]) {
    const BwppGraphNode *c1 = &g->nodes[gc->cons[last][0]];
    if (c1->op == BWPP_GOP_ADD && c1->input_count == 2) {
      uint32_t w = c1->inputs[0] == last ? c1->inputs[1] : c1->inputs[0];
      /* a reshape of the bias may come after the matmul in graph order:
       * look through it to data that exists already */
      for (int r = producer_op(g, w, BWPP_GOP_RESHAPE); r >= 0 && gc->lv[w].pv < 0;
           r = producer_op(g, w, BWPP_GOP_RESHAPE))
        w = g->nodes[r].inputs[0];
      const LVal *W = &gc->lv[w];
      if (W->known && !W->trans && !W->bcast && W->pv >= 0 && shape_elems(&W->shape) == o.n[1] &&
          W->shape.n[W->shape.rank ? W->shape.rank - 1 : 0] == o.n[1] && W->bf16 == A->bf16) {
        bias = (int)w;
        epi = "add";
        gc->skip[gc->cons[last][0]] = 1;
        gc->lv[last].fused = 1;
        last = c1->output;
        if (gc->ncons[last] == 1 && !is_needed(needed, gc, last) &&
            g->nodes[gc->cons[last][0]].op == BWPP_GOP_SILU) {
          epi = "add_silu";
          gc->skip[gc->cons[last][0]] = 1;
          gc->lv[last].fused = 1;
          last = g->nodes[gc->cons[last][0]].output;
        }
      }
    } else if (c1->op == BWPP_GOP_SILU) {
      epi = "silu";
      gc->skip[gc->cons[last][0]] = 1;
      gc->lv[last].fused = 1;
      last = c1->output;
    }
  }
  /* fp32 tails fused after the epilogue (BWPP_HIP_FUSE_*):
   *   residual   the result's only reader adds a full matrix already computed
   *   dual_silu  SiLU of the result where the result itself is also needed
   *              (the backward's silu_grad reads it)
   *   silu_grad  the result is the dY of silu_grad(x, dY) (autodiff graph) */
  const char *fuse = "none";
  int aux = -1, c2v = -1;
  if (!A->bf16 && gc->ncons[last] == 1 && !gc->skip[gc->cons[last][0]] && c->opt->fuse_tails) {
    const uint32_t cn = gc->cons[last][0];
    const BwppGraphNode *c1 = &g->nodes[cn];
    if (c1->op == BWPP_GOP_ADD && c1->input_count == 2 && !is_needed(needed, gc, last)) {
      const uint32_t r = c1->inputs[0] == last ? c1->inputs[1] : c1->inputs[0];
      const LVal *R = &gc->lv[r];
      if (r != last && R->known && R->pv >= 0 && !R->trans && !R->bcast && !R->bf16 && R->shape.rank >= 1 &&
          shape_elems(&R->shape) == o.n[0] * o.n[1] && R->shape.n[R->shape.rank - 1] == o.n[1]) {
        fuse = "residual";
        aux = (int)r;
        gc->skip[cn] = 1;
        gc->lv[last].fused = 1;
        last = c1->output;
      }
    } else if (c1->op == BWPP_GOP_SILU && !gc->is_grad && strcmp(epi, "silu") && strcmp(epi, "add_silu")) {
      fuse = "dual_silu";
      c2v = (int)c1->output;
      gc->skip[cn] = 1;
    } else if (c1->op == BWPP_GOP_SILU_GRAD && c1->input_count >= 2 && c1->inputs[1] == last &&
               c1->inputs[0] != last && !strcmp(epi, "none") && !is_needed(needed, gc, last)) {
      const LVal *X = &gc->lv[c1->inputs[0]];
      if (X->known && X->pv >= 0 && !X->trans && !X->bcast && !X->bf16 &&
          shape_elems(&X->shape) == o.n[0] * o.n[1] && X->shape.n[X->shape.rank - 1] == o.n[1]) {
        fuse = "silu_grad";
        aux = (int)c1->inputs[0];
        gc->skip[cn] = 1;
        gc->lv[last].fused = 1;
        last = c1->output;
      }
    }
  }
  const Ref ar = ref(A->pv), br = ref(B->pv);
  char extra[64] = "";
  if (strcmp(fuse, "none")) {
    LVal *out = &gc->lv[last];
    out->shape = o;
    out->known = 1;
    out->bf16 = 0;
    assign_pv(c, gc, last, "t");
    char ins[160], outs[96];
    snprintf(ins, sizeof ins, "%s,%s", ar.s, br.s);
    if (bias >= 0) {
      strcat(ins, ",");
      strcat(ins, ref(gc->lv[bias].pv).s);
    }
    if (aux >= 0) {
      strcat(ins, ",");
      strcat(ins, ref(gc->lv[aux].pv).s);
    }
    snprintf(outs, sizeof outs, "%s", ref(out->pv).s);
    if (c2v >= 0) {
      LVal *o2 = &gc->lv[c2v];
      o2->shape = o;
      o2->known = 1;
      o2->bf16 = 0;
      assign_pv(c, gc, (uint32_t)c2v, "t");
      strcat(outs, ",");
      strcat(outs, ref(o2->pv).s);
    }
    if (A->trans) strcat(extra, " ta=1");
    if (B->trans) strcat(extra, " tb=1");
    if (strcmp(epi, "none")) {
      strcat(extra, " epi=");
      strcat(extra, epi);
    }
    emit(c, "op matmul out=%s in=%s%s fuse=%s\n", outs, ins, extra, fuse);
    return;
  }
  if (!strcmp(epi, "none") && gc->ncons[last] == 1 && !is_needed(needed, gc, last) &&
      !gc->skip[gc->cons[last][0]] && g->nodes[gc->cons[last][0]].op == BWPP_GOP_TRANSPOSE) {
    /* Only read transposed: compute C^T = B^T A^T, so the transpose that
     * follows is free. */
    LVal *out = &gc->lv[last];
    Shape t = o;
    shape_swap_last(&t);
    out->shape = t;
    out->known = 1;
    out->bf16 = A->bf16;
    assign_pv(c, gc, last, "t");
    out->shape = o;
    out->trans = 1;
    if (!B->trans) strcat(extra, " ta=1");
    if (!A->trans) strcat(extra, " tb=1");
    emit(c, "op matmul out=%s in=%s,%s%s\n", ref(out->pv).s, br.s, ar.s, extra);
    return;
  }
  LVal *out = &gc->lv[last];
  out->shape = o;
  out->known = 1;
  out->bf16 = A->bf16;
  assign_pv(c, gc, last, "t");
  if (A->trans) strcat(extra, " ta=1");
  if (B->trans) strcat(extra, " tb=1");
  if (strcmp(epi, "none")) {
    strcat(extra, " epi=");
    strcat(extra, epi);
  }
  if (bias >= 0)
    emit(c, "op matmul out=%s in=%s,%s,%s%s\n", ref(out->pv).s, ar.s, br.s, ref(gc->lv[bias].pv).s, extra);
  else
    emit(c, "op matmul out=%s in=%s,%s%s\n", ref(out->pv).s, ar.s, br.s, extra);
}

static void lower_reduce(Ctx *c, GCtx *gc, uint32_t node, const char *opname) {
  const BwppGraphNode *n = &gc->g->nodes[node];
  const uint32_t x = n->inputs[0];
  need_known(c, gc, x);
  if (c->failed) return;
  const Shape *s = &gc->lv[x].shape;
  const int rank = (int)s->rank;
  const int axis = n->attr.has_axis ? n->attr.axis : rank - 1;
  int plan_axis;
  if (rank >= 1 && axis == rank - 1)
    plan_axis = 1;  /* along each row */
  else if (rank == 2 && axis == 0)
    plan_axis = 0;  /* over the rows */
  else {
    fail(c, "%s over axis %d of a rank-%d value", opname, axis, rank);
    return;
  }
  LVal *out = &gc->lv[n->output];
  out->shape = *s;
  if (rank == 0) out->shape.rank = 0;
  else shape_set_dim(&out->shape, (uint32_t)axis, "1", 1);
  out->known = 1;
  out->bf16 = 0;
  const Ref xr = operand(c, gc, x);
  assign_pv(c, gc, n->output, "t");
  emit(c, "op %s out=%s in=%s axis=%d\n", opname, ref(out->pv).s, xr.s, plan_axis);
}

static void lower_node(Ctx *c, GCtx *gc, uint32_t i, const uint8_t *needed) {
  const BwppGraph *g = gc->g;
  const BwppGraphNode *n = &g->nodes[i];
  LVal *out = &gc->lv[n->output];
  char attrs[96];
  switch (n->op) {
    case BWPP_GOP_TRANSPOSE: {
      const LVal *x = &gc->lv[n->inputs[0]];
      need_known(c, gc, n->inputs[0]);
      if (c->failed) return;
      if (x->shape.rank != 2 || x->bcast) {
        fail(c, "transpose of a rank-%u value outside a fused attention region", x->shape.rank);
        return;
      }
      *out = *x;
      out->trans = !x->trans;
      shape_swap_last(&out->shape);
      return;
    }
    case BWPP_GOP_RESHAPE:
    case BWPP_GOP_BROADCAST: {
      const LVal *x = &gc->lv[n->inputs[0]];
      need_known(c, gc, n->inputs[0]);
      if (c->failed) return;
      Shape t;
      if (!shape_from_graph(c, &n->attr.shape, &t)) return;
      if (x->trans) {
        fail(c, "%s of a transposed value", n->op == BWPP_GOP_RESHAPE ? "reshape" : "broadcast");
        return;
      }
      *out = *x;
      if (n->op == BWPP_GOP_RESHAPE) {
        if (x->bcast || shape_elems(&t) != shape_elems(&x->shape)) {
          fail(c, "reshape changes the element count");
          return;
        }
      } else if (!x->bcast) {
        out->src = x->shape;
        out->bcast = 1;
      }
      out->shape = t;
      return;
    }
    case BWPP_GOP_PERMUTE: {
      for (uint32_t k = 0; k < n->attr.perm_rank; ++k)
        if (n->attr.perm[k] != k) {
          fail(c, "permute other than the identity (no transposing copy kernel in this backend)");
          return;
        }
      *out = gc->lv[n->inputs[0]];
      return;
    }
    case BWPP_GOP_MATMUL:
    case BWPP_GOP_BATCH_MATMUL:
      lower_matmul(c, gc, i, needed);
      return;
    case BWPP_GOP_ADD: lower_elementwise(c, gc, i, "add"); return;
    case BWPP_GOP_SUB: lower_elementwise(c, gc, i, "sub"); return;
    case BWPP_GOP_MUL: lower_elementwise(c, gc, i, "mul"); return;
    case BWPP_GOP_DIV: lower_elementwise(c, gc, i, "div"); return;
    case BWPP_GOP_REDUCE_MAX_GRAD: lower_elementwise(c, gc, i, "mul"); return;  /* mask * broadcast dY */
    case BWPP_GOP_REDUCE_SUM: lower_reduce(c, gc, i, "reduce_sum"); return;
    case BWPP_GOP_REDUCE_MAX: lower_reduce(c, gc, i, "reduce_max"); return;
    case BWPP_GOP_REDUCE_MAX_MASK: {
      const int rank = (int)gc->lv[n->inputs[0]].shape.rank;
      const int axis = n->attr.has_axis ? n->attr.axis : rank - 1;
      snprintf(attrs, sizeof attrs, "axis=%d", (rank == 2 && axis == 0) ? 0 : 1);
      lower_unary(c, gc, i, "reduce_max_mask", attrs);
      return;
    }
    case BWPP_GOP_SOFTMAX: {
      const int rank = (int)gc->lv[n->inputs[0]].shape.rank;
      if (n->attr.has_axis && n->attr.axis != rank - 1) {
        fail(c, "softmax over axis %d (only the last axis is supported)", n->attr.axis);
        return;
      }
      lower_unary(c, gc, i, "softmax", "");
      return;
    }
    case BWPP_GOP_SILU: lower_unary(c, gc, i, "silu", ""); return;
    case BWPP_GOP_SILU_GRAD: lower_unary(c, gc, i, "silu_grad", ""); return;
    case BWPP_GOP_SOFTMAX_GRAD: lower_unary(c, gc, i, "softmax_grad", ""); return;
    case BWPP_GOP_RMSNORM:
    case BWPP_GOP_RMSNORM_GRAD:
      {
        char e[32];
        fmt_float(e, sizeof e, n->attr.has_epsilon ? (double)n->attr.epsilon : 1e-5);
        snprintf(attrs, sizeof attrs, "eps=%s", e);
      }
      lower_unary(c, gc, i, n->op == BWPP_GOP_RMSNORM ? "rmsnorm" : "rmsnorm_grad", attrs);
      return;
  }
  fail(c, "graph op %d has no HIP lowering", (int)n->op);
}

/* ------------------------------------------------------------ graph passes */

static void lower_consts(Ctx *c, GCtx *gc) {
  const BwppGraph *g = gc->g;
  for (uint32_t v = 0; v < g->value_count; ++v) {
    const BwppGraphValue *gv = &g->values[v];
    if (!(gv->flags & BWPP_GRAPH_VALUE_CONST) || gv->producer != BWPP_GRAPH_NO_NODE) continue;
    double val = 0.0;
    char *end = NULL;
    char txt[NAME_LEN] = "";
    if (gv->name.ptr) str_copy(txt, sizeof txt, gv->name.ptr, gv->name.len);
    if (txt[0] && (val = strtod(txt, &end), end && *end == '\0')) {
      /* the autodiff pass's named constants, e.g. "-1" (graph_ir.c:1387-1408) */
    } else if (c->const_used < c->opt->const_count) {
      val = c->opt->const_values[c->const_used++];
    } else {
      fail(c, "numeric literal v%u reaches the graph without its value (graph_ir.c:817-824); pass the "
              "literals in graph order with --const", v);
      return;
    }
    LVal *l = &gc->lv[v];
    memset(&l->shape, 0, sizeof l->shape);
    l->known = 1;
    char kind[64], base[NAME_LEN];
    char num[32];
    fmt_float(num, sizeof num, val);
    snprintf(kind, sizeof kind, "const=%s", num);
    snprintf(base, sizeof base, "c%u", v);
    l->pv = new_pv(c, base, &l->shape, 0, 0, kind);
  }
}

static void lower_inputs(Ctx *c, GCtx *gc) {
  const BwppGraph *g = gc->g;
  for (uint32_t v = 0; v < g->value_count && !c->failed; ++v) {
    const BwppGraphValue *gv = &g->values[v];
    if (!(gv->flags & BWPP_GRAPH_VALUE_INPUT)) continue;
    LVal *l = &gc->lv[v];
    char nm[NAME_LEN];
    value_name(g, v, "in", nm);
    if (gv->shape.rank == 0 || gv->dtype == BWPP_DTYPE_UNKNOWN) {
      fail(c, "input '%s' has no declared type (undeclared identifier?)", nm);
      return;
    }
    if (!shape_from_graph(c, &gv->shape, &l->shape)) return;
    l->known = 1;
    l->bf16 = dtype_bf16(c, gv->dtype);
    l->batched = lval_batched(c, &l->shape);
    const int activation = l->shape.rank >= 1 && !strcmp(l->shape.d[0], c->batch_dim);
    l->pv = new_pv(c, nm, &l->shape, l->batched, l->bf16, activation ? "input" : "param");
  }
}

static void lower_nodes(Ctx *c, GCtx *gc, const uint8_t *needed, Bwd *bwd, int with_lse) {
  const BwppGraph *g = gc->g;
  for (uint32_t i = 0; i < g->node_count && !c->failed; ++i) {
    if (!gc->is_grad) {
      for (int r = 0; r < c->nregions; ++r)
        if (c->regions[r].mm2 == (int)i) lower_attention(c, gc, &c->regions[r], with_lse);
      for (int k = 0; k < c->ngroups; ++k)
        if (c->groups[k].node[0] == (int)i) {
          lower_mm_group(c, gc, &c->groups[k]);
          gc->skip[i] = 2;  /* emitted */
        }
    } else if (bwd) {
      for (int k = 0; k < c->ngroups; ++k)
        if (c->groups[k].bwd && c->groups[k].first_bwd == (int)i) lower_mm_group_grad(c, gc, bwd, &c->groups[k]);
      for (int a = 0; a < bwd->nag; ++a) {
        const AttnGrad *ag = &bwd->ag[a];
        if (ag->first != (int)i) continue;
        const AttnRegion *R = &c->regions[ag->region];
        const GCtx *fc = bwd->fc;
        const Ref dor = operand(c, gc, ag->dout);
        char attrs[320];
        attn_attrs(c, R, attrs, sizeof attrs);
        const uint32_t outs[3] = {ag->dq, ag->dk, ag->dv};
        const uint32_t srcs[3] = {R->q, R->k, R->v};
        for (int k = 0; k < 3; ++k) {
          LVal *l = &gc->lv[outs[k]];
          l->shape = fc->lv[srcs[k]].shape;
          l->known = 1;
          l->bf16 = fc->lv[srcs[k]].bf16;
          assign_pv(c, gc, outs[k], k == 0 ? "dq" : k == 1 ? "dk" : "dv");
        }
        emit(c, "op attention_grad out=%s,%s,%s in=%s,%s,%s,%s,%s,%s %s\n", ref(gc->lv[ag->dq].pv).s,
             ref(gc->lv[ag->dk].pv).s, ref(gc->lv[ag->dv].pv).s, ref(fc->lv[R->q].pv).s, ref(fc->lv[R->k].pv).s,
             ref(fc->lv[R->v].pv).s, ref(fc->lv[R->o].pv).s, dor.s, ref(R->lse_pv).s, attrs);
      }
      for (int k = 0; k < bwd->nng; ++k) {
        const NormGrad *ng = &bwd->ng[k];
        if (ng->rg != (int)i) continue;
        const BwppGraphNode *rg = &g->nodes[i];
        LVal *dx = &gc->lv[rg->output];
        const uint32_t rs = g->nodes[ng->rsum].output;
        LVal *dgam = &gc->lv[rs];
        for (uint32_t j = 0; j < 3; ++j) need_known(c, gc, rg->inputs[j]);
        if (c->failed) return;
        dx->shape = gc->lv[rg->inputs[0]].shape;
        dx->known = 1;
        dgam->shape = dx->shape;
        shape_set_dim(&dgam->shape, 0, "1", 1);
        dgam->known = 1;
        const Ref xr = operand(c, gc, rg->inputs[0]), gr = operand(c, gc, rg->inputs[1]),
                  dyr = operand(c, gc, rg->inputs[2]);
        /* The residual branch's gradient: when dX's only reader adds a
         * matrix of dX's shape that is already computed (autodiff's sum of
         * the two gradient contributions to a residual input), the add
         * runs inside rmsnorm_grad as its fourth input. */
        uint32_t dxv = rg->output;
        int acc = -1;
        if (c->opt->fuse_tails && gc->ncons[rg->output] == 1 && !is_needed(needed, gc, rg->output)) {
          const uint32_t an = gc->cons[rg->output][0];
          const BwppGraphNode *ad = &g->nodes[an];
          if (!gc->skip[an] && ad->op == BWPP_GOP_ADD && ad->input_count == 2) {
            const uint32_t r = ad->inputs[0] == rg->output ? ad->inputs[1] : ad->inputs[0];
            const LVal *R = &gc->lv[r];
            if (r != rg->output && R->known && R->pv >= 0 && !R->trans && !R->bcast && !R->bf16 &&
                R->shape.rank >= 1 && shape_elems(&R->shape) == shape_elems(&dx->shape) &&
                R->shape.n[R->shape.rank - 1] == dx->shape.n[dx->shape.rank - 1]) {
              acc = (int)r;
              gc->skip[an] = 1;
              dx->fused = 1;
              dxv = ad->output;
              LVal *o = &gc->lv[dxv];
              o->shape = dx->shape;
              o->known = 1;
              o->bf16 = 0;
            }
          }
        }
        assign_pv(c, gc, dxv, "dx");
        assign_pv(c, gc, rs, "dgamma");
        char e[32], accs[80] = "";
        fmt_float(e, sizeof e, rg->attr.has_epsilon ? (double)rg->attr.epsilon : 1e-5);
        if (acc >= 0) snprintf(accs, sizeof accs, ",%s", ref(gc->lv[acc].pv).s);
        emit(c, "op rmsnorm_grad out=%s,%s in=%s,%s,%s%s eps=%s\n", ref(gc->lv[dxv].pv).s, ref(dgam->pv).s, xr.s,
             gr.s, dyr.s, accs, e);
        gc->skip[i] = 2;  /* emitted */
      }
    }
    if (gc->skip[i]) continue;
    lower_node(c, gc, i, needed);
  }
}

/* Makes graph value v a plan output named `name` (a copy when its data is
 * an input, a shared plan value or a view). */
static void make_output(Ctx *c, GCtx *gc, uint32_t v, const char *name, uint8_t *pv_is_out) {
  LVal *l = &gc->lv[v];
  if (l->pv < 0) {
    fail(c, "output '%s' is not computed by any lowered op", name);
    return;
  }
  const char *kind = c->pv[l->pv].kind;
  const int plain = !l->trans && !l->bcast && !strcmp(kind, "temp") && !pv_is_out[l->pv];
  if (plain) {
    sanitize(name, c->pv[l->pv].name);
    snprintf(c->pv[l->pv].kind, sizeof c->pv[l->pv].kind, "output");
    pv_is_out[l->pv] = 1;
    return;
  }
  if (l->trans) {
    fail(c, "output '%s' is only available transposed", name);
    return;
  }
  const Shape *s = &l->shape;
  const int pv = new_pv(c, name, s, lval_batched(c, s), l->bf16, "output");
  const int src = l->bcast ? classify(gc, v, s) : BC_FULL;
  emit(c, "op copy out=%s in=%s bcast=%s\n", ref(pv).s, ref(l->pv).s, bc_name(src));
  l->pv = pv;
  l->bcast = 0;
  pv_is_out[pv] = 1;
}

/* ------------------------------------------------------------ entry */

void bwpp_lower_options_init(BwppLowerOptions *opt) {
  memset(opt, 0, sizeof *opt);
  opt->batch = 1;
  opt->heads = 1;
  opt->f16_as = BWPP_DTYPE_F32;
  opt->fuse_attention = 1;
  opt->group_gemms = 1;
  opt->fuse_tails = 1;
}

/* Plan value a copy touches: the value, or the base a view looks into. */
static int pv_base(const Ctx *c, int pv) { return c->pv[pv].view_of >= 0 ? c->pv[pv].view_of : pv; }

/* Runs of consecutive single-pair full copies (`op copy out=$A$ in=$B$
 * bcast=full`) become one multi-pair copy of up to 4 pairs, one launch
 * instead of one per pair (the weights into their concatenation, the
 * concatenated gradient out to its blocks), as long as no pair writes a
 * value (or the base of a view) that another pair of the run reads or
 * writes. */
static void merge_copies(Ctx *c) {
  if (!c->ops) return;
  char *outbuf = (char *)malloc(c->ops_len + 1);
  if (!outbuf) {
    fail(c, "out of memory");
    return;
  }
  size_t olen = 0;
  const char *s = c->ops;
  int run_o[4], run_i[4], nrun = 0;
  while (*s || nrun) {
    const char *e = *s ? strchr(s, '\n') : NULL;
    const size_t len = e ? (size_t)(e - s) + 1 : strlen(s);
    int o = -1, i = -1, end = 0;
    const int is_copy = *s && sscanf(s, "op copy out=$%d$ in=$%d$ bcast=full%n", &o, &i, &end) == 2 &&
                        (s[end] == '\n' || s[end] == '\0');
    int ok = is_copy && nrun < 4;
    for (int k = 0; ok && k < nrun; ++k) {
      const int bo = pv_base(c, o), bi = pv_base(c, i);
      if (pv_base(c, run_o[k]) == bi || pv_base(c, run_i[k]) == bo || run_o[k] == o) ok = 0;
    }
    if (ok) {
      run_o[nrun] = o;
      run_i[nrun] = i;
      ++nrun;
      s += len;
      continue;
    }
    if (nrun) {  /* flush the run */
      olen += (size_t)sprintf(outbuf + olen, "op copy out=");
      for (int k = 0; k < nrun; ++k) olen += (size_t)sprintf(outbuf + olen, "%s$%d$", k ? "," : "", run_o[k]);
      olen += (size_t)sprintf(outbuf + olen, " in=");
      for (int k = 0; k < nrun; ++k) olen += (size_t)sprintf(outbuf + olen, "%s$%d$", k ? "," : "", run_i[k]);
      olen += (size_t)sprintf(outbuf + olen, " bcast=full\n");
      nrun = 0;
      continue;  /* the current line is looked at again */
    }
    memcpy(outbuf + olen, s, len);
    olen += len;
    s += len;
  }
  outbuf[olen] = '\0';
  free(c->ops);
  c->ops = outbuf;
  c->ops_len = olen;
  c->ops_cap = c->ops_len + 1;
}

static void render(Ctx *c, FILE *out) {
  /* final names: outputs, inputs, params and consts keep theirs (made
   * unique in that order), temps take what is left */
  char (*names)[NAME_LEN + 16] = (char (*)[NAME_LEN + 16])calloc((size_t)c->npv + 1, NAME_LEN + 16);
  if (!names) {
    fail(c, "out of memory");
    return;
  }
  for (int pass = 0; pass < 2; ++pass)
    for (int i = 0; i < c->npv; ++i) {
      const int temp = !strcmp(c->pv[i].kind, "temp");
      if (temp != pass) continue;
      const char *base = c->pv[i].name;
      strcpy(names[i], base);
      for (int k = 1;; ++k) {
        int clash = 0;
        for (int j = 0; j < c->npv && !clash; ++j)
          if (j != i && names[j][0] && !strcmp(names[j], names[i])) clash = 1;
        if (!clash) break;
        snprintf(names[i], sizeof names[i], "%s_%d", base, k);
      }
    }
  fprintf(out, "bwpp.plan 1\n");
  if (c->opt->header) fprintf(out, "%s", c->opt->header);
  for (uint32_t i = 0; i < c->opt->dim_count; ++i)
    fprintf(out, "dim %s %llu\n", c->opt->dim_names[i], (unsigned long long)c->opt->dim_values[i]);
  if (c->opt->batch > 1) fprintf(out, "dim BATCH %u\n", c->opt->batch);
  int rank2_attention = 0;
  for (int r = 0; r < c->nregions; ++r) rank2_attention |= !c->regions[r].bhsd;
  if (rank2_attention) fprintf(out, "dim HEADS %u\n", c->opt->heads ? c->opt->heads : 1);
  fprintf(out, "\n");
  for (int i = 0; i < c->npv; ++i) {
    const PVal *p = &c->pv[i];
    if (p->view_of >= 0) continue;
    fprintf(out, "value %s %s [", names[i], p->bf16 ? "bf16" : "f32");
    for (uint32_t d = 0; d < p->rank; ++d) fprintf(out, "%s%s", d ? "," : "", p->d[d]);
    fprintf(out, "] %s\n", p->kind);
  }
  for (int i = 0; i < c->npv; ++i) {
    const PVal *p = &c->pv[i];
    if (p->view_of < 0) continue;
    fprintf(out, "view %s of=%s offset=%s ld=%s shape=[%s,%s]\n", names[i], names[p->view_of], p->off, p->ld,
            p->d[0], p->d[1]);
  }
  fprintf(out, "\n");
  for (const char *s = c->ops; s && *s; ++s) {
    if (*s == '$') {
      const int idx = atoi(s + 1);
      fputs(idx >= 0 && idx < c->npv ? names[idx] : "?", out);
      s = strchr(s + 1, '$');
      if (!s) break;
      continue;
    }
    fputc(*s, out);
  }
  free(names);
}

BwppStatus bwpp_codegen_hip(const BwppGraph *graph, const BwppGraph *grad, const BwppLowerOptions *opt, FILE *out,
                            char *err, size_t err_cap) {
  Ctx c;
  memset(&c, 0, sizeof c);
  c.opt = opt;
  c.err = err;
  c.err_cap = err_cap;
  if (err && err_cap) err[0] = '\0';
  if (!graph || !opt || !out) return BWPP_ERR;
  if (opt->train != BWPP_LOWER_TRAIN_NONE && !grad) {
    fail(&c, "training needs the autodiff graph");
    return BWPP_ERR;
  }
  c.pv = (PVal *)calloc(MAX_PV, sizeof(PVal));
  GCtx fc, gcx;
  memset(&gcx, 0, sizeof gcx);
  uint8_t *needed = (uint8_t *)calloc(graph->value_count + 1, 1);
  uint32_t *order = (uint32_t *)calloc(graph->value_count + 1, sizeof(uint32_t));
  uint8_t *pv_is_out = (uint8_t *)calloc(MAX_PV, 1);
  uint8_t *has = (uint8_t *)calloc(graph->value_count + 1, 1);
  Bwd bwd;
  memset(&bwd, 0, sizeof bwd);
  uint32_t norder = 0;
  if (!c.pv || !needed || !order || !pv_is_out || !has || !gctx_init(&c, &fc, graph, 0)) {
    fail(&c, "out of memory");
    goto done;
  }
  /* the batched dim: leading dim of the entry's first parameter */
  c.batch_dim = opt->batch_dim;
  for (uint32_t v = 0; v < graph->value_count && !c.batch_dim; ++v)
    if ((graph->values[v].flags & BWPP_GRAPH_VALUE_INPUT) && graph->values[v].shape.rank >= 1) {
      static char bd[DIM_LEN];
      str_copy(bd, sizeof bd, graph->values[v].shape.dims[0].ptr, graph->values[v].shape.dims[0].len);
      c.batch_dim = bd;
    }
  if (!c.batch_dim) c.batch_dim = "";
  if (opt->train != BWPP_LOWER_TRAIN_NONE) {
    replay_imports(graph, order, &norder, needed, has);
    for (uint32_t v = 0; v < graph->value_count; ++v) needed[v] = needed[v] == 2;
  } else {
    memset(needed, 0, graph->value_count + 1);
  }

  /* ---- forward */
  lower_inputs(&c, &fc);
  lower_consts(&c, &fc);
  if (opt->fuse_attention && !c.failed) {
    /* attention operands need shapes before the region is recognised:
     * lower the nodes ahead of each region first (cheap: one pass) */
    find_attention(&c, &fc);
  }
  if (opt->group_gemms && !c.failed) find_mm_groups(&c, &fc);
  lower_nodes(&c, &fc, needed, NULL, opt->train != BWPP_LOWER_TRAIN_NONE);
  if (c.failed) goto done;
  if (graph->output_count != 1) {
    fail(&c, "the entry must return one value (it returns %u)", graph->output_count);
    goto done;
  }
  const uint32_t fo = graph->outputs[0];
  char oname[NAME_LEN];
  if (graph->values[fo].name.ptr && graph->values[fo].name.len)
    value_name(graph, fo, "out", oname);
  else
    strcpy(oname, "out");  /* `return <expression>` */
  make_output(&c, &fc, fo, oname, pv_is_out);
  if (c.failed) goto done;

  if (opt->train != BWPP_LOWER_TRAIN_NONE) {
    /* ---- loss and seed */
    const LVal *O = &fc.lv[fo];
    int seed_pv;
    if (opt->train == BWPP_LOWER_TRAIN_MEAN_SQUARE) {
      const PVal *P = &c.pv[O->pv];
      char nexpr[4 * DIM_LEN] = "";
      for (uint32_t d = 0; d < P->rank; ++d) {
        if (d) strcat(nexpr, "*");
        strncat(nexpr, P->d[d], sizeof nexpr - strlen(nexpr) - 1);
      }
      Shape one;
      memset(&one, 0, sizeof one);
      char kind[4 * DIM_LEN + 16];
      char dn[NAME_LEN + 8];
      snprintf(dn, sizeof dn, "d%s", oname);
      if (opt->fuse_tails) {
        /* one pass over the output: loss = (1/n) sum out^2 and the seed
         * d<out> = (2/n) out (the graph ops below, fused) */
        snprintf(kind, sizeof kind, "const=1/%s", nexpr);
        const int inv = new_pv(&c, "inv_n", &one, 0, 0, kind);
        snprintf(kind, sizeof kind, "const=2/%s", nexpr);
        const int two = new_pv(&c, "two_n", &one, 0, 0, kind);
        const int loss = new_pv(&c, "loss", &one, 0, 0, "output");
        pv_is_out[loss] = 1;
        seed_pv = new_pv(&c, dn, &O->shape, O->batched, 0, "temp");
        emit(&c, "op mean_square out=%s,%s in=%s,%s,%s\n", ref(loss).s, ref(seed_pv).s, ref(O->pv).s, ref(inv).s,
             ref(two).s);
      } else {
        const int sq = new_pv(&c, "sq", &O->shape, O->batched, 0, "temp");
        emit(&c, "op mul out=%s in=%s,%s bcast=full\n", ref(sq).s, ref(O->pv).s, ref(O->pv).s);
        int sum_in = sq;
        if (O->shape.rank >= 2) {
          Shape rows = O->shape;
          rows.rank = O->shape.rank - 1;
          const int rs = new_pv(&c, "rowsum", &rows, O->batched, 0, "temp");
          emit(&c, "op reduce_sum out=%s in=%s axis=1\n", ref(rs).s, ref(sq).s);
          sum_in = rs;
        }
        const int total = new_pv(&c, "total", &one, 0, 0, "temp");
        emit(&c, "op reduce_sum out=%s in=%s axis=1\n", ref(total).s, ref(sum_in).s);
        snprintf(kind, sizeof kind, "const=1/%s", nexpr);
        const int inv = new_pv(&c, "inv_n", &one, 0, 0, kind);
        const int loss = new_pv(&c, "loss", &one, 0, 0, "output");
        pv_is_out[loss] = 1;
        emit(&c, "op mul out=%s in=%s,%s bcast=scalar\n", ref(loss).s, ref(total).s, ref(inv).s);
        snprintf(kind, sizeof kind, "const=2/%s", nexpr);
        const int two = new_pv(&c, "two_n", &one, 0, 0, kind);
        seed_pv = new_pv(&c, dn, &O->shape, O->batched, 0, "temp");
        emit(&c, "op mul out=%s in=%s,%s bcast=scalar\n", ref(seed_pv).s, ref(O->pv).s, ref(two).s);
      }
    } else {
      char dn[NAME_LEN + 8];
      snprintf(dn, sizeof dn, "d%s", oname);
      seed_pv = new_pv(&c, dn, &O->shape, O->batched, O->bf16, "input");
    }

    /* ---- autodiff graph */
    if (!gctx_init(&c, &gcx, grad, 1)) goto done;
    bwd.f = graph;
    bwd.fc = &fc;
    bwd.g2f = (int32_t *)malloc((grad->value_count + 1) * sizeof(int32_t));
    if (!bwd.g2f) {
      fail(&c, "out of memory");
      goto done;
    }
    for (uint32_t v = 0; v < grad->value_count; ++v) bwd.g2f[v] = -1;
    /* clones, in creation order: forward inputs (graph_ir.c:1507-1511),
     * the output's seed (1513-1519), then imported activations */
    uint32_t fin = 0, next_act = 0, gin = 0;
    for (uint32_t v = 0; v < graph->value_count; ++v)
      if (graph->values[v].flags & BWPP_GRAPH_VALUE_INPUT) ++fin;
    for (uint32_t v = 0; v < grad->value_count && !c.failed; ++v) {
      const BwppGraphValue *gv = &grad->values[v];
      if (!(gv->flags & BWPP_GRAPH_VALUE_INPUT) || gv->producer != BWPP_GRAPH_NO_NODE) continue;
      uint32_t f;
      if (gin < fin) {
        uint32_t k = 0;
        for (f = 0; f < graph->value_count; ++f)
          if ((graph->values[f].flags & BWPP_GRAPH_VALUE_INPUT) && k++ == gin) break;
      } else if (gin == fin) {
        f = fo;  /* the seed */
      } else {
        if (next_act >= norder) {
          fail(&c, "autodiff graph has more activation clones than the replay predicts");
          break;
        }
        f = order[next_act++];
      }
      const BwppGraphValue *fv = &graph->values[f];
      if (fv->name.ptr != gv->name.ptr || fv->name.len != gv->name.len || fv->shape.rank != gv->shape.rank) {
        fail(&c, "autodiff clone v%u does not match forward value v%u", v, f);
        break;
      }
      if (gin == fin) {
        LVal *l = &gcx.lv[v];
        l->shape = fc.lv[fo].shape;
        l->known = 1;
        l->batched = fc.lv[fo].batched;
        l->pv = seed_pv;
      } else {
        gcx.lv[v] = fc.lv[f];
        bwd.g2f[v] = (int32_t)f;
      }
      ++gin;
    }
    if (!c.failed && next_act != norder)
      fail(&c, "autodiff graph imports %u activations, the replay predicts %u", next_act, norder);
    if (c.failed) goto done;
    lower_consts(&c, &gcx);
    if (opt->fuse_attention) find_attention_grads(&c, &gcx, &bwd);
    if (!c.failed) find_mm_group_grads(&c, &gcx, &bwd);
    find_norm_grads(&c, &gcx, &bwd);
    lower_nodes(&c, &gcx, NULL, &bwd, 0);
    if (c.failed) goto done;
    /* the autodiff graph's outputs are the gradients of the forward inputs
     * that received one, in forward value order (graph_ir.c:1824-1832) */
    uint32_t k = 0;
    for (uint32_t v = 0; v < graph->value_count && !c.failed; ++v) {
      if (!(graph->values[v].flags & BWPP_GRAPH_VALUE_INPUT) || !has[v]) continue;
      if (k >= grad->output_count) {
        fail(&c, "autodiff graph has fewer outputs than inputs with gradients");
        break;
      }
      char in_name[NAME_LEN], dn[NAME_LEN + 8];
      value_name(graph, v, "in", in_name);
      snprintf(dn, sizeof dn, "d%s", in_name);
      make_output(&c, &gcx, grad->outputs[k], dn, pv_is_out);
      ++k;
    }
    if (!c.failed && k != grad->output_count) fail(&c, "autodiff graph has outputs the replay does not predict");
  }

done:
  if (!c.failed) merge_copies(&c);
  if (!c.failed) render(&c, out);
  gctx_free(&fc);
  if (gcx.g) gctx_free(&gcx);
  free(bwd.g2f);
  free(bwd.ag);
  free(bwd.ng);
  free(needed);
  free(order);
  free(pv_is_out);
  free(has);
  free(c.pv);
  free(c.ops);
  free(c.regions);
  free(c.groups);
  return c.failed ? BWPP_ERR : BWPP_OK;
}
