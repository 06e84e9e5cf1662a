/*
 * lower_hip.h -- the HIP target of BW++'s compiler: lowers a BwppGraph
 * (compiler/include/graph_ir.h:96-109) and, for training, the graph
 * bwpp_graph_autodiff builds from it (graph_ir.c:1485-1839) to a libbwpp_hip
 * launch plan (the text bwpp_hip_plan_create runs; grammar in
 * bluewolf-plus-plus_amd/csrc/runtime/bwpp_plan.cpp).
 *
 * It takes the place of bwpp_codegen_metal (compiler/include/
 * codegen_metal.h:7, called at compiler/main.c:186).  Where codegen_metal
 * emits one main kernel per program (attention or matmul,
 * codegen_metal.c:233) plus aux kernels, this target emits one launch per
 * graph node or fused region, in graph order:
 *   - q @ transpose(k) -> softmax -> @ v (the pattern of
 *     bwpp_graph_detect_attention, graph_ir.c:1852-1899) becomes one fused
 *     `attention` launch, and its autodiff chain (matmul / transpose /
 *     softmax_grad, graph_ir.c:1529-1583, 1722-1733) one `attention_grad`;
 *   - a transpose feeding a matmul becomes that matmul's ta / tb flag;
 *   - add of a [N] vector to a matmul result, and silu of it, fuse into
 *     the GEMM epilogue by pattern (the graph marks bias by the name
 *     `bias` only, graph_ir.c:760-768), when nothing else reads the
 *     intermediate (the backward's activations included);
 *   - rmsnorm_grad plus the graph's dGamma chain (div / mul / reduce_sum,
 *     graph_ir.c:1747-1781) become one rmsnorm_grad launch with two
 *     outputs;
 *   - in fp32, the add of a full matrix to a matmul result, SiLU of a
 *     result the backward also reads (both written), and silu_grad whose
 *     dY is a matmul result fuse into that GEMM's tail;
 *   - matmuls that share their left operand and take weights of one shape
 *     (q, k, v projections) run as one GEMM against the weights' column
 *     concatenation, their results column views; in training their weight
 *     gradients and the sum of their input gradients are one GEMM each.
 * Shapes are inferred here rather than read from the graph where the graph
 * leaves them unset: `@` and transpose of rank 3/4 (graph_ir.c:557-562,
 * 848-863).  Symbolic dims are bound by the caller (--dim).  Numeric
 * literals reach the graph without their value (graph_ir.c:817-824); the
 * caller supplies them in graph order (const_values) or lowering fails.
 */
#ifndef BWPP_LOWER_HIP_H
#define BWPP_LOWER_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#include "graph_ir.h"

#define BWPP_LOWER_MAX_DIMS 16
#define BWPP_LOWER_MAX_CONSTS 16

typedef enum {
  BWPP_LOWER_TRAIN_NONE = 0,        /* forward graph only */
  BWPP_LOWER_TRAIN_SEED = 1,        /* forward + backward; the output's
                                       gradient is a plan input d<out> */
  BWPP_LOWER_TRAIN_MEAN_SQUARE = 2  /* forward, loss = mean(out^2) (a plan
                                       output `loss`), its gradient as the
                                       seed, then the backward */
} BwppLowerTrain;

typedef struct {
  /* --dim NAME=VALUE bindings of the graph's symbolic dims */
  const char *dim_names[BWPP_LOWER_MAX_DIMS];
  uint64_t dim_values[BWPP_LOWER_MAX_DIMS];
  uint32_t dim_count;
  /* batch > 1: the entry runs on `batch` independent samples with shared
   * weights.  Every value whose leading dim is `batch_dim` (default: the
   * leading dim of the entry's first parameter) is stacked batch times
   * along that dim; attention runs per sample; reductions over that dim
   * (weight gradients, dGamma) sum over the samples. */
  uint32_t batch;
  const char *batch_dim;
  /* rank-2 attention regions: heads > 1 splits q, k, v's columns into
   * `heads` heads of width cols / heads (rank-4 regions take heads from
   * their [B, H, T, d] shape). */
  uint32_t heads;
  int causal;          /* mask keys after the query (the graph has no mask op) */
  float attn_scale;    /* score scale; 0 = 1 (the graph has no scale op) */
  int attn_scale_auto; /* scale = 1 / sqrt(head dim) */
  /* storage dtype of f16 graph values (this backend has no f16 kernels):
   * BWPP_DTYPE_F32 or BWPP_DTYPE_BF16 */
  BwppDType f16_as;
  BwppLowerTrain train;
  int fuse_attention; /* 0: lower the attention pattern op by op */
  int group_gemms;    /* matmuls sharing their left operand, with weights of
                         one shape, run as one GEMM against the weights'
                         column concatenation (and so do their dW and dA
                         terms in training); 0: one GEMM each */
  int fuse_tails;     /* fp32 GEMM tails: a residual add of the result, SiLU
                         of a result the backward also reads (both written),
                         silu_grad whose dY is the result; 0: separate ops */
  /* payloads of the graph's valueless numeric literals, in value order */
  float const_values[BWPP_LOWER_MAX_CONSTS];
  uint32_t const_count;
  /* written at the top of the plan as comments (e.g. the command line) */
  const char *header;
} BwppLowerOptions;

void bwpp_lower_options_init(BwppLowerOptions *opt);

/* Lowers `graph` (the entry's forward graph) to plan text on `out`.  For
 * training, `grad` is bwpp_graph_autodiff(graph).  Returns BWPP_OK, or
 * BWPP_ERR with a message in err. */
BwppStatus bwpp_codegen_hip(const BwppGraph *graph, const BwppGraph *grad, const BwppLowerOptions *opt,
                            FILE *out, char *err, size_t err_cap);

#endif
