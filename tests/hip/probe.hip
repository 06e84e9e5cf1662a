// Lane-layout probes for the gfx950 MFMA builtins the GEMM and attention
// kernels use.  Each kernel is one 64-lane wave: lane l feeds its operand
// registers from a[l*NA ..], b[l*NB ..] and writes its accumulator registers
// to c[l*NC ..].  tests/test_gpu_mfma_layout.py checks the results against a
// CPU model of the operand/accumulator layouts the kernels assume.
// Test code: built by tests/hip/Makefile, never loaded by the runtime.
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

// ds_read_b64_tr_b16: LDS holds s[i] = i (4096 shorts).  Lane l reads at
// element offset addr(l) = (mode == 0) ? 4 * l : 64 * l; out[l*4 .. l*4+3]
// receives the four 16-bit results.
typedef short v4s __attribute__((ext_vector_type(4)));
struct TrArgs {
  int *out;
  int mode;
};
extern "C" __global__ __launch_bounds__(64) void probe_ds_read_tr16_b64(TrArgs p) {
  __shared__ short s[4096];
  const int l = threadIdx.x;
  for (int i = l; i < 4096; i += 64) s[i] = (short)i;
  __syncthreads();
  const int off = p.mode == 0 ? 4 * l : 64 * l;
  const v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4s *)(s + off));
  for (int e = 0; e < 4; ++e) p.out[l * 4 + e] = r[e];
}

// global_load_lds (16 bytes per lane): lane l loads ints src[4*(63-l) ..
// 4*(63-l)+3] into LDS; the 1 KiB of LDS is then copied out in order, so
// dst shows where each lane's 16 bytes landed.
struct LdsArgs {
  const int *src;
  int *dst;
};
extern "C" __global__ __launch_bounds__(64) void probe_global_load_lds16(LdsArgs p) {
  __shared__ int s[512];
  const int l = threadIdx.x;
  for (int i = l; i < 512; i += 64) s[i] = -1;
  __syncthreads();
  __builtin_amdgcn_global_load_lds(p.src + 4 * (63 - l), (__attribute__((address_space(3))) void *)s, 16, 0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int i = l; i < 512; i += 64) p.dst[i] = s[i];
}
