// Lane-layout probes for the gfx950 MFMA builtins the GEMM and attention
// kernels use.  Each kernel is one 64-lane wave: lane l feeds its operand
// registers from a[l*NA ..], b[l*NB ..] and writes its accumulator registers
// to c[l*NC ..].  tests/test_gpu_mfma_layout.py checks the results against a
// CPU model of the operand/accumulator layouts the kernels assume.
// Not loaded by the runtime.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct ProbeArgs {
  const void *a;
  const void *b;
  float *c;
};

extern "C" __global__ __launch_bounds__(64) void probe_mfma_32x32x16_bf16(ProbeArgs p) {
  const int l = threadIdx.x;
  const bf16x8 a = reinterpret_cast<const bf16x8 *>(p.a)[l];
  const bf16x8 b = reinterpret_cast<const bf16x8 *>(p.b)[l];
  f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
  for (int r = 0; r < 16; ++r) p.c[l * 16 + r] = acc[r];
}

extern "C" __global__ __launch_bounds__(64) void probe_mfma_16x16x32_bf16(ProbeArgs p) {
  const int l = threadIdx.x;
  const bf16x8 a = reinterpret_cast<const bf16x8 *>(p.a)[l];
  const bf16x8 b = reinterpret_cast<const bf16x8 *>(p.b)[l];
  f32x4 acc = {};
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
  for (int r = 0; r < 4; ++r) p.c[l * 4 + r] = acc[r];
}

extern "C" __global__ __launch_bounds__(64) void probe_mfma_32x32x2_f32(ProbeArgs p) {
  const int l = threadIdx.x;
  const float a = reinterpret_cast<const float *>(p.a)[l];
  const float b = reinterpret_cast<const float *>(p.b)[l];
  f32x16 acc = {};
  acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
  for (int r = 0; r < 16; ++r) p.c[l * 16 + r] = acc[r];
}

extern "C" __global__ __launch_bounds__(64) void probe_mfma_16x16x4_f32(ProbeArgs p) {
  const int l = threadIdx.x;
  const float a = reinterpret_cast<const float *>(p.a)[l];
  const float b = reinterpret_cast<const float *>(p.b)[l];
  f32x4 acc = {};
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
  for (int r = 0; r < 4; ++r) p.c[l * 4 + r] = acc[r];
}
