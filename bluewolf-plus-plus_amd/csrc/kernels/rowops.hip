// Bandwidth-bound row operators for gfx950: softmax, RMSNorm, LayerNorm,
// reduce_max (value + argmax), reduce_max mask, and the reduce_max grads.
//
// Semantics follow runtime/cpu/bwpp_cpu_ref.c (softmax :37-61, rmsnorm
// :63-90, reduce_max mask :146-190, grad :192-219); LayerNorm and the
// argmax forms are the closed forms documented in include/bwpp_hip.h.
//
// Main path ("reg"): the row is read from HBM once with 128-bit
// non-temporal loads into registers, reduced with DPP + lane exchanges,
// transformed and written once with 128-bit non-temporal stores (the data is
// streamed exactly once, so it is kept out of the caches' way).  WPR waves
// share a row: WPR < 4 packs 4/WPR rows into a 256-thread block; WPR >= 4
// gives each row a block of 64*WPR threads with a cross-wave step through
// LDS.  Thread g of the row group owns float4 chunks g, g + 64*WPR, ...,
// so each load instruction of the group covers 1 KiB * WPR of contiguous
// memory.  VPT chunks per thread (<= 16) keep the row in registers.
// Blocks loop over row groups with stride gridDim.x (the host may cap the
// grid); the next group's loads are issued before the current group's
// reductions, and gamma/beta chunks are loaded once per block.
//
// Fallback path ("gen"): one 256-thread block per row, scalar loads, several
// passes; any cols, ld and alignment.
#include "common.h"
#include "../kargs.h"

using namespace bwpp;

namespace {

enum RowOp : int {
  OP_SOFTMAX = 0,
  OP_RMSNORM = 1,
  OP_LAYERNORM = 2,
  OP_MAX = 3,      // maxv + argmax
  OP_MAX_GRAD = 4, // dx one-hot from x
  OP_MASK = 5,     // reference mask (all ties)
};

constexpr uint32_t kNoIndex = 0xFFFFFFFFu;

// Cross-wave steps of the row reductions.  A block holds 4/WPR rows
// (WPR < 4) or one row of WPR waves; waves w0 .. w0+WPR-1 share a row.
template <int WPR>
__device__ __forceinline__ float row_sum(float v, float *red) {
  v = wave_sum(v);
  if constexpr (WPR > 1) {
    const int w = threadIdx.x >> 6, w0 = (w / WPR) * WPR;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = red[w0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) v += red[w0 + i];
  }
  return v;
}

template <int WPR>
__device__ __forceinline__ float row_max(float v, float *red) {
  v = wave_max(v);
  if constexpr (WPR > 1) {
    const int w = threadIdx.x >> 6, w0 = (w / WPR) * WPR;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    v = red[w0];
#pragma unroll
    for (int i = 1; i < WPR; ++i) v = fmaxf(v, red[w0 + i]);
  }
  return v;
}

template <int WPR>
__device__ __forceinline__ void row_argmax(float &v, uint32_t &i, float *redf,
                                           uint32_t *redu) {
  wave_argmax(v, i);
  if constexpr (WPR > 1) {
    const int w = threadIdx.x >> 6, w0 = (w / WPR) * WPR;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      redf[w] = v;
      redu[w] = i;
    }
    __syncthreads();
    v = redf[w0];
    i = redu[w0];
#pragma unroll
    for (int k = 1; k < WPR; ++k) argmax_merge(v, i, redf[w0 + k], redu[w0 + k]);
  }
}

// Row mean and M2 = sum (x - mean)^2 from per-thread partial statistics.
template <int WPR>
__device__ __forceinline__ void row_chan(float &n, float &mu, float &m2, float *red) {
  wave_chan(n, mu, m2);
  if constexpr (WPR > 1) {
    const int w = threadIdx.x >> 6, w0 = (w / WPR) * WPR;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      red[3 * w] = n;
      red[3 * w + 1] = mu;
      red[3 * w + 2] = m2;
    }
    __syncthreads();
    n = red[3 * w0];
    mu = red[3 * w0 + 1];
    m2 = red[3 * w0 + 2];
#pragma unroll
    for (int i = 1; i < WPR; ++i)
      chan_merge(n, mu, m2, red[3 * (w0 + i)], red[3 * (w0 + i) + 1], red[3 * (w0 + i) + 2]);
  }
}

// row_chan for equal per-thread counts n (full rows): the same statistics
// with the equal-weight form of the merge; WPR waves' (mean, M2) combine as
// mean = average of the means, M2 = sum of M2 + n_wave * sum (mean_i - mean)^2.
template <int WPR>
__device__ __forceinline__ void row_chan_equal(float &n, float &mu, float &m2, float *red) {
  auto merge = [&](float mu2, float m22) {
    const float d = mu2 - mu;
    mu = mu + 0.5f * d;
    m2 = m2 + m22 + d * d * (0.5f * n);
    n = 2.0f * n;
  };
  merge(dpp_f32<kDppQuadXor1>(mu), dpp_f32<kDppQuadXor1>(m2));
  merge(dpp_f32<kDppQuadXor2>(mu), dpp_f32<kDppQuadXor2>(m2));
  merge(dpp_f32<kDppRowHalfMirror>(mu), dpp_f32<kDppRowHalfMirror>(m2));
  merge(dpp_f32<kDppRowMirror>(mu), dpp_f32<kDppRowMirror>(m2));
  merge(xor_f32(mu, 16), xor_f32(m2, 16));
  merge(xor_f32(mu, 32), xor_f32(m2, 32));
  if constexpr (WPR > 1) {
    const int w = threadIdx.x >> 6, w0 = (w / WPR) * WPR;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) {
      red[2 * w] = mu;
      red[2 * w + 1] = m2;
    }
    __syncthreads();
    float smu = 0.0f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) smu += red[2 * (w0 + i)];
    const float gmu = smu * (1.0f / (float)WPR);
    float sm2 = 0.0f;
#pragma unroll
    for (int i = 0; i < WPR; ++i) {
      const float d = red[2 * (w0 + i)] - gmu;
      sm2 += red[2 * (w0 + i) + 1] + d * d * n;
    }
    mu = gmu;
    m2 = sm2;
    n = n * (float)WPR;
  }
}

template <int WPR>
struct RowGeom {
  static constexpr int kBlock = WPR >= 4 ? 64 * WPR : 256;  // threads per block
  static constexpr int kGroup = 64 * WPR;                    // threads per row
  static constexpr int kRows = kBlock / kGroup;              // rows per block
};

__device__ __forceinline__ float get(const float4 &v, int e) {
  return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}
__device__ __forceinline__ void set(float4 &v, int e, float t) {
  if (e == 0) v.x = t;
  else if (e == 1) v.y = t;
  else if (e == 2) v.z = t;
  else v.w = t;
}

template <int OP, int VPT, int WPR, bool FULL>
__device__ __forceinline__ void row_reg(const BwppRowArgs &a) {
  using G = RowGeom<WPR>;
  constexpr int GT = G::kGroup;
  constexpr bool kNorm = (OP == OP_RMSNORM || OP == OP_LAYERNORM);
  // 16 chunks per thread already fill half the register file: no prefetch
  // buffer and no hoisted gamma/beta there (they would spill).
  constexpr bool kPrefetch = VPT <= 8;
  constexpr bool kHoist = kNorm && VPT <= 8;
  __shared__ float redf[3 * 16];
  __shared__ uint32_t redu[16];
  const int tid = threadIdx.x;
  const int g = tid % GT;
  const uint32_t sub = (uint32_t)(tid / GT);  // row slot in the block
  const uint32_t cols = a.cols;
  const uint32_t ngroups = (a.rows + G::kRows - 1) / G::kRows;
  const float fill = kNorm ? 0.0f : -INFINITY;

  auto chunk_col = [&](int j) { return (uint32_t)(j * GT + g) * 4u; };
  auto in_full = [&](uint32_t c) { return FULL || c + 4u <= cols; };

  // Loads the row of group `grp` (rows past the end re-read the last row;
  // their results are never stored), and for the max grad its dy with it.
  auto load_row = [&](uint32_t grp, float4 *v, float &dyv) {
    // The row is wave-uniform (a row is owned by whole waves): through
    // readfirstlane its base stays in SGPRs and the loads take the
    // SGPR-base + 32-bit lane offset form, with no 64-bit address VGPRs
    // (which the compiler otherwise recycled into the prefetch buffer,
    // waiting for all memory operations at the loop head).
    const uint32_t row = __builtin_amdgcn_readfirstlane(grp * G::kRows + sub);
    const uint32_t rr = row < a.rows ? row : a.rows - 1;
    const float *xr = a.x + (size_t)rr * a.ld;
    if constexpr (OP == OP_MAX_GRAD) dyv = a.dy[rr];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const uint32_t c = chunk_col(j);
      if (in_full(c)) {
        v[j] = load_nt4(xr + c);
      } else {
        v[j] = make_float4(fill, fill, fill, fill);
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < cols) set(v[j], e, xr[c + e]);
      }
    }
  };

  // gamma / beta chunk j (1 / 0 where absent or past the row end).
  auto affine_chunk = [&](int j, float4 &gj, float4 &bj) {
    const uint32_t c = chunk_col(j);
    gj = make_float4(1.0f, 1.0f, 1.0f, 1.0f);
    bj = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (in_full(c)) {
      if (a.gamma) gj = *reinterpret_cast<const float4 *>(a.gamma + c);
      if (a.beta) bj = *reinterpret_cast<const float4 *>(a.beta + c);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (c + e < cols) {
          if (a.gamma) set(gj, e, a.gamma[c + e]);
          if (a.beta) set(bj, e, a.beta[c + e]);
        }
    }
  };
  // Hoisted copies, reused for every row the block normalises.
  float4 gm[kHoist ? VPT : 1], bt[kHoist ? VPT : 1];
  if constexpr (kHoist) {
#pragma unroll
    for (int j = 0; j < VPT; ++j) affine_chunk(j, gm[j], bt[j]);
  }

  // Processes the row group `grp` held in v[] (reductions + stores).
  auto process = [&](float4(&v)[VPT], uint32_t grp, float dyv) {
    const uint32_t row = __builtin_amdgcn_readfirstlane(grp * G::kRows + sub);  // wave-uniform
    const bool valid = row < a.rows;
    float *yr = a.y ? a.y + (size_t)(valid ? row : 0) * a.ld : nullptr;
    auto store = [&](int j, const float4 &o) {
      const uint32_t c = chunk_col(j);
      if (!valid) return;
      if (in_full(c)) {
        store_nt4(yr + c, o);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (c + e < cols) yr[c + e] = get(o, e);
      }
    };

    if constexpr (OP == OP_SOFTMAX) {
      float m = -INFINITY;
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        m = fmaxf(fmaxf(m, fmaxf(v[j].x, v[j].y)), fmaxf(v[j].z, v[j].w));
      m = row_max<WPR>(m, redf);
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        v[j].x = __expf(v[j].x - m);
        v[j].y = __expf(v[j].y - m);
        v[j].z = __expf(v[j].z - m);
        v[j].w = __expf(v[j].w - m);
        const uint32_t c = chunk_col(j);
        if (in_full(c)) {
          s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (c + e < cols) s += get(v[j], e);
        }
      }
      s = row_sum<WPR>(s, redf);
      const float inv = s > 0.0f ? 1.0f / s : 0.0f;
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        store(j, make_float4(v[j].x * inv, v[j].y * inv, v[j].z * inv, v[j].w * inv));
    } else if constexpr (kNorm) {
      float mean = 0.0f, ss = 0.0f;
      if constexpr (OP == OP_LAYERNORM) {
        // Thread-local mean and M2 from registers (two passes, exact), then
        // one merged reduction of (count, mean, M2) across the row.
        float n = 0.0f, s = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          const uint32_t c = chunk_col(j);
          if (in_full(c)) {
            s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
            n += 4.0f;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (c + e < cols) {
                s += get(v[j], e);
                n += 1.0f;
              }
          }
        }
        float mu = n > 0.0f ? s / n : 0.0f;
        float m2 = 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          const uint32_t c = chunk_col(j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            if (FULL || c + e < cols) {
              const float d = get(v[j], e) - mu;
              m2 += d * d;
            }
          }
        }
        if constexpr (FULL) {
          // Full rows: every thread holds 4 VPT values, so every merge step
          // joins equal counts n and Chan's update needs no division:
          // mu = (mu_a + mu_b) / 2, M2 = M2_a + M2_b + (mu_b - mu_a)^2 n / 2.
          row_chan_equal<WPR>(n, mu, m2, redf);
        } else {
          row_chan<WPR>(n, mu, m2, redf);
        }
        mean = mu;
        ss = m2;
      } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j)
          ss += (v[j].x * v[j].x + v[j].y * v[j].y) + (v[j].z * v[j].z + v[j].w * v[j].w);
        ss = row_sum<WPR>(ss, redf);
      }
      const float inv = 1.0f / sqrtf(ss / (float)cols + a.eps);
#pragma unroll
      for (int j = 0; j < VPT; ++j) {
        float4 o, gj, bj;
        if constexpr (kHoist) {
          gj = gm[j];
          bj = bt[j];
        } else {
          affine_chunk(j, gj, bj);
        }
        o.x = (v[j].x - mean) * inv * gj.x + bj.x;
        o.y = (v[j].y - mean) * inv * gj.y + bj.y;
        o.z = (v[j].z - mean) * inv * gj.z + bj.z;
        o.w = (v[j].w - mean) * inv * gj.w + bj.w;
        store(j, o);
      }
    } else if constexpr (OP == OP_MAX || OP == OP_MAX_GRAD) {
      float m = -INFINITY;
      uint32_t mi = kNoIndex;
      if constexpr (FULL) {
        // Two passes over the registers: the lane's max (fmaxf skips NaN,
        // -inf when the lane holds no number), then its first column
        // holding that value and the element there (a backward scan, the
        // last hit wins), which is the first strict-or-equal maximum of the
        // one-pass rule below (the element, not fmaxf's result, carries the
        // sign of a zero maximum).
#pragma unroll
        for (int j = 0; j < VPT; ++j) m = fmaxf(fmaxf(m, fmaxf(v[j].x, v[j].y)), fmaxf(v[j].z, v[j].w));
        float mv = m;
#pragma unroll
        for (int j = VPT - 1; j >= 0; --j) {
          const uint32_t c = chunk_col(j);
          mi = v[j].w == m ? c + 3u : mi;
          mv = v[j].w == m ? v[j].w : mv;
          mi = v[j].z == m ? c + 2u : mi;
          mv = v[j].z == m ? v[j].z : mv;
          mi = v[j].y == m ? c + 1u : mi;
          mv = v[j].y == m ? v[j].y : mv;
          mi = v[j].x == m ? c : mi;
          mv = v[j].x == m ? v[j].x : mv;
        }
        m = mv;
      } else {
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          const uint32_t c = chunk_col(j);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float t = get(v[j], e);
            if (c + e < cols) {
              if (t > m || (mi == kNoIndex && t == m)) {
                m = t;
                mi = c + e;
              }
            }
          }
        }
      }
      row_argmax<WPR>(m, mi, redf, redu);
      if constexpr (OP == OP_MAX) {
        if (g == 0 && valid) {
          if (a.maxv) a.maxv[row] = m;
          if (a.argmax) a.argmax[row] = (mi == kNoIndex) ? -1 : (int32_t)mi;
        }
      } else {
        const float gv = valid ? dyv : 0.0f;
#pragma unroll
        for (int j = 0; j < VPT; ++j) {
          const uint32_t c = chunk_col(j);
          float4 o;
          o.x = (c + 0 == mi) ? gv : 0.0f;
          o.y = (c + 1 == mi) ? gv : 0.0f;
          o.z = (c + 2 == mi) ? gv : 0.0f;
          o.w = (c + 3 == mi) ? gv : 0.0f;
          store(j, o);
        }
      }
    } else if constexpr (OP == OP_MASK) {
      float m = -INFINITY;
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        m = fmaxf(fmaxf(m, fmaxf(v[j].x, v[j].y)), fmaxf(v[j].z, v[j].w));
      m = row_max<WPR>(m, redf);
#pragma unroll
      for (int j = 0; j < VPT; ++j)
        store(j, make_float4(v[j].x == m ? 1.0f : 0.0f, v[j].y == m ? 1.0f : 0.0f,
                             v[j].z == m ? 1.0f : 0.0f, v[j].w == m ? 1.0f : 0.0f));
    }

  };

  // Group loop, two groups per trip so the prefetch buffers alternate
  // without copies; every trip count is block-uniform.  The last group of a
  // block is processed on a path of its own, so inside the loop the
  // next-group loads are issued unconditionally: the compiler's vmcnt
  // waits then count them as younger than the current group's loads (with
  // a conditional prefetch it merges both paths and waits for the prefetch
  // too, which serialises the rows).
  uint32_t grp = blockIdx.x;
  if (grp >= ngroups) return;  // block-uniform
  float4 va[VPT], vb[VPT];
  float da = 0.0f, db = 0.0f;
  load_row(grp, va, da);
  for (;;) {
    uint32_t next = grp + gridDim.x;
    if (next >= ngroups) {
      process(va, grp, da);
      break;
    }
    if (kPrefetch) load_row(next, vb, db);
    process(va, grp, da);
    if (!kPrefetch) load_row(next, vb, db);
    grp = next;
    next = grp + gridDim.x;
    if (next >= ngroups) {
      process(vb, grp, db);
      break;
    }
    if (kPrefetch) load_row(next, va, da);
    process(vb, grp, db);
    if (!kPrefetch) load_row(next, va, da);
    grp = next;
  }
}

// ---------------------------------------------------------------- fallback

__device__ __forceinline__ float block_sum(float v, float *red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}
__device__ __forceinline__ float block_max(float v, float *red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <int OP>
__device__ __forceinline__ void row_gen(const BwppRowArgs &a) {
  __shared__ float redf[4];
  __shared__ uint32_t redu[4];
  const uint32_t row = blockIdx.x;
  if (row >= a.rows) return;  // block-uniform
  const uint32_t cols = a.cols;
  const uint32_t t = threadIdx.x;
  const float *xr = a.x + (size_t)row * a.ld;
  float *yr = a.y ? a.y + (size_t)row * a.ld : nullptr;

  if constexpr (OP == OP_SOFTMAX) {
    float m = -INFINITY;
    for (uint32_t c = t; c < cols; c += 256) m = fmaxf(m, xr[c]);
    m = block_max(m, redf);
    float s = 0.0f;
    for (uint32_t c = t; c < cols; c += 256) s += __expf(xr[c] - m);
    s = block_sum(s, redf);
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    for (uint32_t c = t; c < cols; c += 256) yr[c] = __expf(xr[c] - m) * inv;
  } else if constexpr (OP == OP_RMSNORM || OP == OP_LAYERNORM) {
    float mean = 0.0f;
    if constexpr (OP == OP_LAYERNORM) {
      float s = 0.0f;
      for (uint32_t c = t; c < cols; c += 256) s += xr[c];
      mean = block_sum(s, redf) / (float)cols;
    }
    float ss = 0.0f;
    for (uint32_t c = t; c < cols; c += 256) {
      const float d = xr[c] - mean;
      ss += d * d;
    }
    ss = block_sum(ss, redf);
    const float inv = 1.0f / sqrtf(ss / (float)cols + a.eps);
    for (uint32_t c = t; c < cols; c += 256) {
      float o = (xr[c] - mean) * inv;
      if (a.gamma) o *= a.gamma[c];
      if (a.beta) o += a.beta[c];
      yr[c] = o;
    }
  } else if constexpr (OP == OP_MAX || OP == OP_MAX_GRAD) {
    float m = -INFINITY;
    uint32_t mi = kNoIndex;
    for (uint32_t c = t; c < cols; c += 256) {
      const float v = xr[c];
      if (v > m || (mi == kNoIndex && v == m)) {
        m = v;
        mi = c;
      }
    }
    row_argmax<4>(m, mi, redf, redu);
    if constexpr (OP == OP_MAX) {
      if (t == 0) {
        if (a.maxv) a.maxv[row] = m;
        if (a.argmax) a.argmax[row] = (mi == kNoIndex) ? -1 : (int32_t)mi;
      }
    } else {
      const float gv = a.dy[row];
      for (uint32_t c = t; c < cols; c += 256) yr[c] = (c == mi) ? gv : 0.0f;
    }
  } else if constexpr (OP == OP_MASK) {
    float m = -INFINITY;
    for (uint32_t c = t; c < cols; c += 256) m = fmaxf(m, xr[c]);
    m = block_max(m, redf);
    for (uint32_t c = t; c < cols; c += 256) yr[c] = (xr[c] == m) ? 1.0f : 0.0f;
  }
}

}  // namespace

// ------------------------------------------------------------ entry points
// Register path: bwpp_row_<op>_v<VPT>_w<WPR>_<f|p>  (f: cols == 256*WPR*VPT)
#define BWPP_ROW_REG(NAME, OP, VPT, WPR)                                      \
  extern "C" __global__ __launch_bounds__(RowGeom<WPR>::kBlock) void          \
      bwpp_row_##NAME##_v##VPT##_w##WPR##_f(const BwppRowArgs a) {            \
    row_reg<OP, VPT, WPR, true>(a);                                           \
  }                                                                           \
  extern "C" __global__ __launch_bounds__(RowGeom<WPR>::kBlock) void          \
      bwpp_row_##NAME##_v##VPT##_w##WPR##_p(const BwppRowArgs a) {            \
    row_reg<OP, VPT, WPR, false>(a);                                          \
  }

// Keep this list in sync with kRowCfgs in runtime/bwpp_hip.cpp.
#define BWPP_ROW_ALL_CFG(NAME, OP)                                            \
  BWPP_ROW_REG(NAME, OP, 1, 1)                                                \
  BWPP_ROW_REG(NAME, OP, 2, 1)                                                \
  BWPP_ROW_REG(NAME, OP, 4, 1)                                                \
  BWPP_ROW_REG(NAME, OP, 8, 1)                                                \
  BWPP_ROW_REG(NAME, OP, 16, 1)                                               \
  BWPP_ROW_REG(NAME, OP, 2, 2)                                                \
  BWPP_ROW_REG(NAME, OP, 4, 2)                                                \
  BWPP_ROW_REG(NAME, OP, 8, 2)                                                \
  BWPP_ROW_REG(NAME, OP, 1, 4)                                                \
  BWPP_ROW_REG(NAME, OP, 2, 4)                                                \
  BWPP_ROW_REG(NAME, OP, 4, 4)                                                \
  BWPP_ROW_REG(NAME, OP, 8, 4)                                                \
  BWPP_ROW_REG(NAME, OP, 16, 4)                                               \
  BWPP_ROW_REG(NAME, OP, 2, 8)                                                \
  BWPP_ROW_REG(NAME, OP, 4, 8)                                                \
  BWPP_ROW_REG(NAME, OP, 8, 8)                                                \
  BWPP_ROW_REG(NAME, OP, 16, 8)                                               \
  extern "C" __global__ __launch_bounds__(256) void bwpp_row_##NAME##_gen(const BwppRowArgs a) { \
    row_gen<OP>(a);                                                           \
  }

BWPP_ROW_ALL_CFG(softmax, OP_SOFTMAX)
BWPP_ROW_ALL_CFG(rmsnorm, OP_RMSNORM)
BWPP_ROW_ALL_CFG(layernorm, OP_LAYERNORM)
BWPP_ROW_ALL_CFG(max, OP_MAX)
BWPP_ROW_ALL_CFG(maxgrad, OP_MAX_GRAD)
BWPP_ROW_ALL_CFG(mask, OP_MASK)

// ------------------------------------------------------- streaming kernels

// reduce_max grad from saved indices, axis 1: dx[r, c] = (c == idx[r]) ? dy[r] : 0.
// Block per row (grid-stride), each thread writes columns t, t+256, ...
extern "C" __global__ __launch_bounds__(256) void bwpp_row_maxgrad_idx(const BwppRowArgs a) {
  for (uint32_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
    const int32_t idx = a.idx_in[r];
    const float gv = a.dy[r];
    float *yr = a.y + (size_t)r * a.ld;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256)
      yr[c] = ((int32_t)c == idx) ? gv : 0.0f;
  }
}

// Same, 128-bit stores (host checks dx alignment and ld % 4 == 0).
extern "C" __global__ __launch_bounds__(256) void bwpp_row_maxgrad_idx_v4(const BwppRowArgs a) {
  for (uint32_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
    const int32_t idx = a.idx_in[r];
    const float gv = a.dy[r];
    float *yr = a.y + (size_t)r * a.ld;
    const uint32_t c4 = a.cols & ~3u;
    for (uint32_t c = threadIdx.x * 4u; c < c4; c += 1024u) {
      float4 o;
      o.x = ((int32_t)c == idx) ? gv : 0.0f;
      o.y = ((int32_t)c + 1 == idx) ? gv : 0.0f;
      o.z = ((int32_t)c + 2 == idx) ? gv : 0.0f;
      o.w = ((int32_t)c + 3 == idx) ? gv : 0.0f;
      *reinterpret_cast<float4 *>(yr + c) = o;
    }
    for (uint32_t c = c4 + threadIdx.x; c < a.cols; c += 256)
      yr[c] = ((int32_t)c == idx) ? gv : 0.0f;
  }
}

// Reference grad (bwpp_cpu_ref.c:192-219): dx = mask * dy[line].
// axis 1: dy per row; axis 0 variant below: dy per column.
extern "C" __global__ __launch_bounds__(256) void bwpp_row_maskgrad(const BwppRowArgs a) {
  for (uint32_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
    const float gv = a.dy[r];
    const float *mr = a.x + (size_t)r * a.ld;
    float *yr = a.y + (size_t)r * a.ld;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) yr[c] = mr[c] * gv;
  }
}
extern "C" __global__ __launch_bounds__(256) void bwpp_col_maskgrad(const BwppRowArgs a) {
  for (uint32_t r = blockIdx.x; r < a.rows; r += gridDim.x) {
    const float *mr = a.x + (size_t)r * a.ld;
    float *yr = a.y + (size_t)r * a.ld;
    for (uint32_t c = threadIdx.x; c < a.cols; c += 256) yr[c] = mr[c] * a.dy[c];
  }
}

// ---------------------------------------------------------- axis 0 (columns)
// One thread per column; rows are walked in order, so the fold is the
// reference's (bwpp_cpu_ref.c:156-171) and the first equal row is the lowest.

__device__ __forceinline__ void col_argmax(const BwppRowArgs &a, uint32_t c,
                                           float &m, int32_t &mi) {
  m = -INFINITY;
  for (uint32_t r = 0; r < a.rows; ++r) {
    const float v = a.x[(size_t)r * a.ld + c];
    if (v > m) m = v;
  }
  mi = -1;
  for (uint32_t r = 0; r < a.rows; ++r) {
    if (a.x[(size_t)r * a.ld + c] == m) {
      mi = (int32_t)r;
      break;
    }
  }
}

extern "C" __global__ __launch_bounds__(256) void bwpp_col_max(const BwppRowArgs a) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.cols) return;
  float m;
  int32_t mi;
  col_argmax(a, c, m, mi);
  if (a.maxv) a.maxv[c] = m;
  if (a.argmax) a.argmax[c] = mi;
}

extern "C" __global__ __launch_bounds__(256) void bwpp_col_maxgrad(const BwppRowArgs a) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.cols) return;
  int32_t mi;
  if (a.idx_in) {
    mi = a.idx_in[c];
  } else {
    float m;
    col_argmax(a, c, m, mi);
  }
  const float gv = a.dy[c];
  for (uint32_t r = 0; r < a.rows; ++r) a.y[(size_t)r * a.ld + c] = ((int32_t)r == mi) ? gv : 0.0f;
}

extern "C" __global__ __launch_bounds__(256) void bwpp_col_mask(const BwppRowArgs a) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.cols) return;
  float m = -INFINITY;
  for (uint32_t r = 0; r < a.rows; ++r) m = fmaxf(m, a.x[(size_t)r * a.ld + c]);
  for (uint32_t r = 0; r < a.rows; ++r) {
    const size_t o = (size_t)r * a.ld + c;
    a.y[o] = (a.x[o] == m) ? 1.0f : 0.0f;
  }
}
