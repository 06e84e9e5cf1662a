// Device helpers shared by the gfx950 kernels of libbwpp_hip.
// Wavefronts are 64 lanes.  Reductions stay inside a row of 16 lanes with DPP
// moves (quad_perm / row_half_mirror / row_mirror) and cross rows with
// two lane-exchange steps (xor 16, xor 32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define BWPP_WAVE 64

namespace bwpp {

// DPP control words (GCN/CDNA DPP encoding).
constexpr int kDppQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;

template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float xor_f32(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ uint32_t xor_u32(uint32_t v, int m) {
  return (uint32_t)__shfl_xor((int)v, m, 64);
}

// All-reduce over the 64 lanes of a wave; every lane returns the result.
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<kDppQuadXor1>(v);
  v += dpp_f32<kDppQuadXor2>(v);
  v += dpp_f32<kDppRowHalfMirror>(v);
  v += dpp_f32<kDppRowMirror>(v);
  v += xor_f32(v, 16);
  v += xor_f32(v, 32);
  return v;
}

// Max that ignores NaN operands (v_max_f32 returns the non-NaN operand),
// which matches a strictly-greater fold started at -INF.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<kDppQuadXor1>(v));
  v = fmaxf(v, dpp_f32<kDppQuadXor2>(v));
  v = fmaxf(v, dpp_f32<kDppRowHalfMirror>(v));
  v = fmaxf(v, dpp_f32<kDppRowMirror>(v));
  v = fmaxf(v, xor_f32(v, 16));
  v = fmaxf(v, xor_f32(v, 32));
  return v;
}

// (count, mean, M2) triples of Chan, Golub & LeVeque's pairwise variance
// update: merging two partial row statistics costs one exchange step.
__device__ __forceinline__ void chan_merge(float &n, float &mu, float &m2, float n2,
                                           float mu2, float m22) {
  const float nt = n + n2;
  if (nt > 0.0f) {
    const float d = mu2 - mu;
    const float w = n2 / nt;
    mu = mu + d * w;
    m2 = m2 + m22 + d * d * n * w;
  }
  n = nt;
}

__device__ __forceinline__ void wave_chan(float &n, float &mu, float &m2) {
  chan_merge(n, mu, m2, dpp_f32<kDppQuadXor1>(n), dpp_f32<kDppQuadXor1>(mu), dpp_f32<kDppQuadXor1>(m2));
  chan_merge(n, mu, m2, dpp_f32<kDppQuadXor2>(n), dpp_f32<kDppQuadXor2>(mu), dpp_f32<kDppQuadXor2>(m2));
  chan_merge(n, mu, m2, dpp_f32<kDppRowHalfMirror>(n), dpp_f32<kDppRowHalfMirror>(mu),
             dpp_f32<kDppRowHalfMirror>(m2));
  chan_merge(n, mu, m2, dpp_f32<kDppRowMirror>(n), dpp_f32<kDppRowMirror>(mu), dpp_f32<kDppRowMirror>(m2));
  chan_merge(n, mu, m2, xor_f32(n, 16), xor_f32(mu, 16), xor_f32(m2, 16));
  chan_merge(n, mu, m2, xor_f32(n, 32), xor_f32(mu, 32), xor_f32(m2, 32));
}

// (value, index) pairs: larger value wins, equal values keep the lower
// index.  "No element" is (-INF, 0xFFFFFFFF), which loses to any real pair.
__device__ __forceinline__ void argmax_merge(float &v, uint32_t &i, float v2,
                                             uint32_t i2) {
  if (v2 > v || (v2 == v && i2 < i)) {
    v = v2;
    i = i2;
  }
}

// Wave-wide (max, first index of the max) for lane pairs whose v is never
// NaN: the max first, then the smallest index among the lanes holding it
// (the pairwise argmax_merge result, with one plain max and one unsigned
// min per step instead of a compare-and-swap of both).
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
  v = min(v, dpp_u32<kDppQuadXor1>(v));
  v = min(v, dpp_u32<kDppQuadXor2>(v));
  v = min(v, dpp_u32<kDppRowHalfMirror>(v));
  v = min(v, dpp_u32<kDppRowMirror>(v));
  v = min(v, xor_u32(v, 16));
  v = min(v, xor_u32(v, 32));
  return v;
}
// The value returned is the winning lane's own element, not the max of the
// max reduction: when the maximum is a zero, -0 and +0 compare equal and the
// max picks either sign, while the strict fold keeps the first one's.
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i) {
  const float m = wave_max(v);
  const uint32_t w = wave_min_u32(v == m ? i : 0xffffffffu);
  const uint64_t won = __ballot(v == m && i == w);
  v = won ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), (int)__builtin_ctzll(won))) : m;
  i = w;
}

// 128-bit non-temporal global accesses for data streamed exactly once.
typedef float f32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 load_nt4(const float *p) {
  const f32x4 t = __builtin_nontemporal_load(reinterpret_cast<const f32x4 *>(p));
  return make_float4(t.x, t.y, t.z, t.w);
}
__device__ __forceinline__ void store_nt4(float *p, const float4 &o) {
  const f32x4 t = {o.x, o.y, o.z, o.w};
  __builtin_nontemporal_store(t, reinterpret_cast<f32x4 *>(p));
}

// bf16 <-> fp32.  fp32 -> bf16 uses the gfx950 conversion instruction
// (v_cvt_pk_bf16_f32: round to nearest even, NaN stays NaN), two values per
// instruction when packed.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  const bf16x2_t v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float((uint32_t)h << 16);
}

}  // namespace bwpp
