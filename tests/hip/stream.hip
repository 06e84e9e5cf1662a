// Stream kernels for measuring this box's HBM copy and read ceilings (the
// rooflines the row operators are held against).  Test/measurement code:
// built by tests/hip/Makefile, never loaded by the runtime.
//
// bwpp_stream_copy_v<V>: y[i] = x[i] over n float4, each thread moving V
// float4 per trip of a grid-stride loop (non-temporal 128-bit loads and
// stores, the access the row kernels use), all V loads issued before the
// stores; bwpp_stream_read_v<V>: the same loads, no stores.  Every index is
// checked against n.
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct StreamArgs {
  const f32x4 *x;
  f32x4 *y;
  uint64_t n;  // 16-byte elements
};

template <int V>
__device__ __forceinline__ void stream_copy(const StreamArgs &a) {
  const uint64_t nt = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t step = nt * V;
  for (uint64_t base = (uint64_t)blockIdx.x * blockDim.x * V + threadIdx.x; base < a.n; base += step) {
    f32x4 v[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint64_t i = base + (uint64_t)j * blockDim.x;
      if (i < a.n) v[j] = __builtin_nontemporal_load(a.x + i);
    }
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint64_t i = base + (uint64_t)j * blockDim.x;
      if (i < a.n) __builtin_nontemporal_store(v[j], a.y + i);
    }
  }
}

// Read-only stream (the ceiling of reduce_max, which reads X and writes a
// few KB): the loads are summed per thread, and the sum is stored only if
// it equals a value N(0,1) data never sums to, so nothing is written in
// practice while the loads stay live.  The store index is below n.
template <int V>
__device__ __forceinline__ void stream_read(const StreamArgs &a) {
  const uint64_t nt = (uint64_t)gridDim.x * blockDim.x;
  const uint64_t step = nt * V;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint64_t base = (uint64_t)blockIdx.x * blockDim.x * V + threadIdx.x; base < a.n; base += step) {
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const uint64_t i = base + (uint64_t)j * blockDim.x;
      if (i < a.n) acc += __builtin_nontemporal_load(a.x + i);
    }
  }
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (acc.x == 1.0e30f && t < a.n) a.y[t] = acc;
}

#define STREAM(V)                                                                         \
  extern "C" __global__ __launch_bounds__(1024) void bwpp_stream_copy_v##V(StreamArgs a) { \
    stream_copy<V>(a);                                                                    \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(1024) void bwpp_stream_read_v##V(StreamArgs a) { \
    stream_read<V>(a);                                                                    \
  }
STREAM(1)
STREAM(2)
STREAM(4)
STREAM(8)
