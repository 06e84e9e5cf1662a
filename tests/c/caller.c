/*
 * A plain C11 caller of libbwpp_hip, written the way INTEGRATION.md shows a
 * maintainer binding it in place of runtime/metal/dispatch_stub.m: one
 * handle, one device arena, reference-style params initialisers, status
 * checks, and the tensor-metadata forms of the operators.  Each result is
 * checked against a naive C computation on the host.
 *
 * Exit status: 0 all checks passed, 1 a check or call failed, 2 no usable
 * GPU (bwpp_hip_create returned BWPP_HIP_ERR_NO_DEVICE).
 */
#include "bwpp_hip.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define M 64
#define N 80
#define K 48
#define ROWS 16
#define COLS 96

static int fails = 0;

static void check(const char *what, const float *got, const float *want, size_t n, float tol) {
  float maxerr = 0.0f, maxref = 0.0f;
  for (size_t i = 0; i < n; ++i) {
    float e = fabsf(got[i] - want[i]);
    if (e > maxerr || e != e) maxerr = e;
    if (fabsf(want[i]) > maxref) maxref = fabsf(want[i]);
  }
  float rel = maxerr / (maxref > 0.0f ? maxref : 1.0f);
  printf("%-28s rel max err %.3e\n", what, (double)rel);
  if (!(rel <= tol)) ++fails;
}

static int ok(BwppHip *h, BwppHipStatus s, const char *what) {
  if (s == BWPP_HIP_OK) return 1;
  fprintf(stderr, "%s: %s (%s)\n", what, bwpp_hip_status_string(s), bwpp_hip_last_error(h));
  ++fails;
  return 0;
}

int main(void) {
  BwppHip *h = NULL;
  BwppHipStatus s = bwpp_hip_create(&h, 0, NULL);
  if (s == BWPP_HIP_ERR_NO_DEVICE) {
    printf("no device: %s\n", bwpp_hip_last_error(NULL));
    return 2;
  }
  if (s != BWPP_HIP_OK) {
    fprintf(stderr, "create: %s\n", bwpp_hip_last_error(NULL));
    return 1;
  }

  static float a[M * K], b[K * N], bias[N], c[M * N], want[M * N];
  static float x[ROWS * COLS], y[ROWS * COLS], ywant[ROWS * COLS], gamma[COLS];
  for (int i = 0; i < M * K; ++i) a[i] = (float)((i * 37) % 17 - 8) / 8.0f;
  for (int i = 0; i < K * N; ++i) b[i] = (float)((i * 11) % 13 - 6) / 6.0f;
  for (int i = 0; i < N; ++i) bias[i] = (float)(i % 7) / 7.0f - 0.5f;
  for (int i = 0; i < ROWS * COLS; ++i) x[i] = (float)((i * 29) % 23 - 11) / 4.0f;
  for (int i = 0; i < COLS; ++i) gamma[i] = 0.5f + (float)(i % 5) / 5.0f;

  BwppHipArena arena;
  if (!ok(h, bwpp_hip_arena_init(h, &arena, 1u << 20), "arena_init")) return 1;
  float *da = bwpp_hip_arena_alloc(&arena, sizeof a, 256);
  float *db = bwpp_hip_arena_alloc(&arena, sizeof b, 256);
  float *dbias = bwpp_hip_arena_alloc(&arena, sizeof bias, 256);
  float *dc = bwpp_hip_arena_alloc(&arena, sizeof c, 256);
  float *dx = bwpp_hip_arena_alloc(&arena, sizeof x, 256);
  float *dy = bwpp_hip_arena_alloc(&arena, sizeof y, 256);
  float *dg = bwpp_hip_arena_alloc(&arena, sizeof gamma, 256);
  if (!da || !db || !dbias || !dc || !dx || !dy || !dg) {
    fprintf(stderr, "arena exhausted\n");
    return 1;
  }
  ok(h, bwpp_hip_copy_to_device(h, da, a, sizeof a), "copy a");
  ok(h, bwpp_hip_copy_to_device(h, db, b, sizeof b), "copy b");
  ok(h, bwpp_hip_copy_to_device(h, dbias, bias, sizeof bias), "copy bias");
  ok(h, bwpp_hip_copy_to_device(h, dx, x, sizeof x), "copy x");
  ok(h, bwpp_hip_copy_to_device(h, dg, gamma, sizeof gamma), "copy gamma");

  /* 1. matmul, reference-style initialiser (dispatch_stub.h:9-16 fields). */
  BwppMatmulParams mp = {M, N, K, K, N, N, BWPP_HIP_F32, BWPP_HIP_EPILOGUE_NONE, 0, 0};
  if (ok(h, bwpp_hip_dispatch_matmul(h, da, db, dc, NULL, mp), "matmul") &&
      ok(h, bwpp_hip_copy_to_host(h, c, dc, sizeof c), "copy c")) {
    for (int i = 0; i < M; ++i)
      for (int j = 0; j < N; ++j) {
        float acc = 0.0f;
        for (int k = 0; k < K; ++k) acc += a[i * K + k] * b[k * N + j];
        want[i * N + j] = acc;
      }
    check("matmul f32", c, want, M * N, 1e-5f);
  }

  /* 2. the same product with bias + SiLU through tensor metadata. */
  BwppHipTensor ta, tb, tbias, tc;
  const uint64_t sa[2] = {M, K}, sb[2] = {K, N}, sbias[1] = {N}, sc[2] = {M, N};
  ok(h, bwpp_hip_tensor_init(&ta, BWPP_HIP_CORE_F32, BWPP_HIP_LAYOUT_ROW_MAJOR, 2, sa, da), "tensor a");
  ok(h, bwpp_hip_tensor_init(&tb, BWPP_HIP_CORE_F32, BWPP_HIP_LAYOUT_ROW_MAJOR, 2, sb, db), "tensor b");
  ok(h, bwpp_hip_tensor_init(&tbias, BWPP_HIP_CORE_F32, BWPP_HIP_LAYOUT_ROW_MAJOR, 1, sbias, dbias), "tensor bias");
  ok(h, bwpp_hip_tensor_init(&tc, BWPP_HIP_CORE_F32, BWPP_HIP_LAYOUT_ROW_MAJOR, 2, sc, dc), "tensor c");
  if (ok(h, bwpp_hip_tensor_matmul(h, &ta, &tb, &tbias, &tc, BWPP_HIP_EPILOGUE_ADD_SILU), "tensor_matmul") &&
      ok(h, bwpp_hip_copy_to_host(h, c, dc, sizeof c), "copy c")) {
    for (int i = 0; i < M * N; ++i) {
      float v = want[i] + bias[i % N];
      want[i] = v / (1.0f + expf(-v));
    }
    check("tensor matmul+bias+SiLU", c, want, M * N, 1e-5f);
  }

  /* 3. RMSNorm, reference-style initialiser (dispatch_stub.h:24-29). */
  BwppRmsnormParams rp = {ROWS, COLS, COLS, 1e-5f};
  if (ok(h, bwpp_hip_dispatch_rmsnorm(h, dx, dg, NULL, dy, rp), "rmsnorm") &&
      ok(h, bwpp_hip_copy_to_host(h, y, dy, sizeof y), "copy y")) {
    for (int r = 0; r < ROWS; ++r) {
      float ss = 0.0f;
      for (int j = 0; j < COLS; ++j) ss += x[r * COLS + j] * x[r * COLS + j];
      float inv = 1.0f / sqrtf(ss / COLS + 1e-5f);
      for (int j = 0; j < COLS; ++j) ywant[r * COLS + j] = x[r * COLS + j] * inv * gamma[j];
    }
    check("rmsnorm", y, ywant, ROWS * COLS, 1e-5f);
  }

  /* 4. softmax over a rank-3 tensor [2, ROWS/2, COLS]. */
  BwppHipTensor tx, ty;
  const uint64_t s3[3] = {2, ROWS / 2, COLS};
  ok(h, bwpp_hip_tensor_init(&tx, BWPP_HIP_CORE_F32, BWPP_HIP_LAYOUT_ROW_MAJOR, 3, s3, dx), "tensor x");
  ok(h, bwpp_hip_tensor_init(&ty, BWPP_HIP_CORE_F32, BWPP_HIP_LAYOUT_ROW_MAJOR, 3, s3, dy), "tensor y");
  if (ok(h, bwpp_hip_tensor_softmax(h, &tx, &ty), "tensor_softmax") &&
      ok(h, bwpp_hip_copy_to_host(h, y, dy, sizeof y), "copy y")) {
    for (int r = 0; r < ROWS; ++r) {
      float mx = -INFINITY, sum = 0.0f;
      for (int j = 0; j < COLS; ++j) mx = x[r * COLS + j] > mx ? x[r * COLS + j] : mx;
      for (int j = 0; j < COLS; ++j) sum += (ywant[r * COLS + j] = expf(x[r * COLS + j] - mx));
      for (int j = 0; j < COLS; ++j) ywant[r * COLS + j] /= sum;
    }
    check("tensor softmax (rank 3)", y, ywant, ROWS * COLS, 1e-5f);
  }

  /* 5. errors come back as statuses, nothing is launched. */
  BwppSoftmaxParams bad = {ROWS, COLS, COLS - 1};
  if (bwpp_hip_dispatch_softmax(h, dx, dy, bad) != BWPP_HIP_ERR_INVALID_ARG) {
    fprintf(stderr, "ld < cols was not rejected\n");
    ++fails;
  }
  if (bwpp_hip_dtype_from_graph(3) != BWPP_HIP_F32 || bwpp_hip_dtype_to_core(BWPP_HIP_BF16) != BWPP_HIP_CORE_BF16) {
    fprintf(stderr, "dtype mapping\n");
    ++fails;
  }

  ok(h, bwpp_hip_sync(h), "sync");
  bwpp_hip_arena_destroy(&arena);
  bwpp_hip_destroy(h);
  printf("%s\n", fails ? "FAILED" : "OK");
  return fails ? 1 : 0;
}
