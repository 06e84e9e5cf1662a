// Library-internal entry points of libbwpp_hip (not part of the C ABI).
#pragma once

#include "bwpp_hip.h"

// Attention backward without the hull-based aliasing test of
// bwpp_hip_dispatch_attention_grad: for callers that place dq / dk / dv
// themselves (the plan executor writes them as disjoint column blocks of
// one buffer, which the hull test would reject).
BwppHipStatus bwpp_hip_attention_grad_planned(BwppHip *h, const void *q, const void *k, const void *v,
                                              const void *o, const void *dout, const float *lse, void *dq,
                                              void *dk, void *dv, const BwppAttentionParams &p);

// Records `fmt` as the handle's last-error text (the thread's create error
// when h is NULL) and returns s.
BwppHipStatus bwpp_hip_set_error(BwppHip *h, BwppHipStatus s, const char *fmt, ...)
    __attribute__((format(printf, 3, 4)));

// Device address of the handle's grad / split-K workspace (NULL before its
// first use).  It moves when an op needs more than its current size, so a
// HIP graph recorded with the old address must not be replayed after that.
const void *bwpp_hip_workspace(const BwppHip *h);

// Size of the device-resident scratch array of bwpp_scratch.hip, which the
// allocation-free attention backward uses for its per-query row sums.
#define BWPP_HIP_NOALLOC_SCRATCH_BYTES (8u << 20)

// Device address of `device`'s scratch array, looked up once per device
// (hipGetSymbolAddress) with that device current.  On failure *ptr is NULL,
// *why names the HIP error and the status is BWPP_HIP_ERR_HIP.
BwppHipStatus bwpp_hip_scratch_setup(int device, void **ptr, const char **why);

// dst[r][c] = src[r][c] for rows x cols with independent row strides (in
// elements), on the handle's stream: the plan executor's copy between a
// tensor and a strided view of another.
BwppHipStatus bwpp_hip_copy_strided(BwppHip *h, const float *src, uint32_t ld_src, float *dst, uint32_t ld_dst,
                                    uint32_t rows, uint32_t cols);

// n <= 4 such copies (segment i: src[i] -> dst[i], rows[i] x cols[i]) in
// one launch.  The segments must not overlap one another's destinations.
#ifndef BWPP_COPY_MULTI_MAX
#define BWPP_COPY_MULTI_MAX 4
#endif
BwppHipStatus bwpp_hip_copy_strided_multi(BwppHip *h, uint32_t n, const float *const *src, const uint32_t *ld_src,
                                          float *const *dst, const uint32_t *ld_dst, const uint32_t *rows,
                                          const uint32_t *cols);
