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

#endif /* BWPP_KARGS_H */
