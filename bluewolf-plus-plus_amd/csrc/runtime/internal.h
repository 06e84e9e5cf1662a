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

