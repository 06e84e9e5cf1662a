// Synthetic inputs for tests and benchmarks (host memory only).
//
// Element i of the (seed, stream) sequence is a pure function of
// (seed, stream, i): a SplitMix64 finaliser (Steele, Lea & Flood, "Fast
// splittable pseudorandom number generators", OOPSLA 2014) applied to a
// Weyl sequence keyed by seed and stream.  Fills are split over OpenMP
// threads; the values do not depend on the thread count.
#include "bwpp_hip.h"

#include <cmath>
#include <cstring>

namespace {

constexpr uint64_t kGolden = 0x9E3779B97F4A7C15ull;

inline uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t stream_key(uint64_t seed, uint64_t stream) {
  return mix64(seed * kGolden + mix64(stream + 0x632BE59BD9B4E019ull));
}

inline uint64_t draw(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGolden); }

inline uint16_t to_bf16(float x) {
  uint32_t u;
  std::memcpy(&u, &x, sizeof u);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

}  // namespace

extern "C" {

void bwpp_synth_uniform_f32(float *dst, uint64_t n, uint64_t seed, uint64_t stream,
                            float lo, float hi) {
  if (!dst) return;
  const uint64_t key = stream_key(seed, stream);
  const float span = hi - lo;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) {
    const float u = (float)(draw(key, (uint64_t)i) >> 40) * (1.0f / 16777216.0f);
    dst[i] = lo + span * u;
  }
}

void bwpp_synth_normal_f32(float *dst, uint64_t n, uint64_t seed, uint64_t stream,
                           float mean, float stddev) {
  if (!dst) return;
  const uint64_t key = stream_key(seed, stream);
  const double two_pi = 6.283185307179586476925286766559;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) {
    const uint64_t r1 = draw(key, 2 * (uint64_t)i);
    const uint64_t r2 = draw(key, 2 * (uint64_t)i + 1);
    const double u1 = ((double)(r1 >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(r2 >> 11) * (1.0 / 9007199254740992.0);
    const double z = std::sqrt(-2.0 * std::log(u1)) * std::cos(two_pi * u2);
    dst[i] = (float)((double)mean + (double)stddev * z);
  }
}

void bwpp_synth_ramp_f32(float *dst, uint32_t rows, uint32_t cols, float scale) {
  if (!dst) return;
  for (uint32_t i = 0; i < rows; ++i)
    for (uint32_t j = 0; j < cols; ++j)
      dst[(size_t)i * cols + j] = (float)(i * cols + j + 1) * scale;
}

void bwpp_f32_to_bf16(const float *src, uint16_t *dst, uint64_t n) {
  if (!src || !dst) return;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) dst[i] = to_bf16(src[i]);
}

void bwpp_bf16_to_f32(const uint16_t *src, float *dst, uint64_t n) {
  if (!src || !dst) return;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < (int64_t)n; ++i) {
    const uint32_t u = (uint32_t)src[i] << 16;
    std::memcpy(&dst[i], &u, sizeof u);
  }
}

}  // extern "C"
