// Autodiff grad ops and elementwise glue for gfx950 (fp32).
//
// The reference's autodiff (compiler/graph_ir.c:1485-1839) emits these
// internal ops; the reference has no numeric kernels for them, so the
// semantics are the closed forms restated in oracle/bwpp_oracle.c:
//   silu_grad      (graph_ir.c:1709-1720)  dx = dy * s * (1 + x (1 - s))
//   softmax_grad   (graph_ir.c:1722-1733)  dx = y * (dy - sum(dy * y))
//   rmsnorm_grad   (graph_ir.c:1735-1789)  dx, dgamma = sum_r dy * xhat,
//                                          dbeta = sum_r dy
//   reduce_sum     (graph_ir.c:1410-1455)  along rows or over rows
//   add/sub/mul/div with broadcasting, broadcast (graph_ir.c:697-770,
//   1457-1470, 1585-1654)
// All are HBM-bound: one read of each input, one write of each output,
// 128-bit accesses where rows are 16-byte aligned.
#include "common.h"
#include "../kargs.h"

using namespace bwpp;

namespace {

__device__ __forceinline__ float block_sum256(float v, float *red) {
  v = wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __forceinline__ float silu_grad1(float x, float dy) {
  const float s = 1.0f / (1.0f + __expf(-x));
  return dy * (s * (1.0f + x * (1.0f - s)));
}

}  // namespace

// Flat elementwise silu_grad over n elements; vec: 16-byte aligned buffers.
extern "C" __global__ __launch_bounds__(256) void bwpp_silu_grad(const BwppGradArgs g) {
  const uint64_t stride = (uint64_t)gridDim.x * 256u;
  const uint64_t n4 = g.vec ? g.n / 4 : 0;
  const float4 *x4 = reinterpret_cast<const float4 *>(g.a);
  const float4 *d4 = reinterpret_cast<const float4 *>(g.b);
  float4 *o4 = reinterpret_cast<float4 *>(g.out);
  for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n4; i += stride) {
    const float4 x = load_nt4(reinterpret_cast<const float *>(x4 + i));
    const float4 d = load_nt4(reinterpret_cast<const float *>(d4 + i));
    store_nt4(reinterpret_cast<float *>(o4 + i),
              make_float4(silu_grad1(x.x, d.x), silu_grad1(x.y, d.y), silu_grad1(x.z, d.z), silu_grad1(x.w, d.w)));
  }
  for (uint64_t i = n4 * 4 + (uint64_t)blockIdx.x * 256u + threadIdx.x; i < g.n; i += stride)
    g.out[i] = silu_grad1(g.a[i], g.b[i]);
}

// Row-wise softmax_grad: one block per row (grid-stride); the dot product is
// reduced in fp32 across the block, the second pass re-reads the row (L2).
extern "C" __global__ __launch_bounds__(256) void bwpp_softmax_grad(const BwppGradArgs g) {
  __shared__ float red[4];
  for (uint32_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
    const float *y = g.a + (size_t)r * g.ld;
    const float *dy = g.b + (size_t)r * g.ld;
    float *dx = g.out + (size_t)r * g.ld;
    float dot = 0.0f;
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) dot += dy[c] * y[c];
    dot = block_sum256(dot, red);
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) dx[c] = y[c] * (dy[c] - dot);
  }
}

// Mean-square loss and its gradient in one pass over x: block b adds x^2
// over its rows (rows b, b + grid, ...; thread order fixed) into partial
// part_g[b] and, with out, writes dx = x * s_grad; bwpp_mean_square_final
// then sums the partials in index order.  Deterministic for a given grid.
extern "C" __global__ __launch_bounds__(256) void bwpp_mean_square_part(const BwppGradArgs g) {
  __shared__ float red[4];
  const float gs = g.s_grad ? *g.s_grad : 1.0f;
  float acc = 0.0f;
  for (uint32_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
    const float *x = g.a + (size_t)r * g.ld;
    float *dx = g.out ? g.out + (size_t)r * g.ld : nullptr;
    if (g.vec) {  // 16-byte rows
      for (uint32_t c = 4u * threadIdx.x; c < g.cols; c += 1024u) {
        const float4 v = *reinterpret_cast<const float4 *>(x + c);
        acc += (v.x * v.x + v.y * v.y) + (v.z * v.z + v.w * v.w);
        if (dx) *reinterpret_cast<float4 *>(dx + c) = make_float4(v.x * gs, v.y * gs, v.z * gs, v.w * gs);
      }
    } else {
      for (uint32_t c = threadIdx.x; c < g.cols; c += 256u) {
        const float v = x[c];
        acc += v * v;
        if (dx) dx[c] = v * gs;
      }
    }
  }
  acc = block_sum256(acc, red);
  if (threadIdx.x == 0) g.part_g[blockIdx.x] = acc;
}

// out2[0] = s_loss * (sum of the nparts partials), one block.
extern "C" __global__ __launch_bounds__(256) void bwpp_mean_square_final(const BwppGradArgs g) {
  __shared__ float red[4];
  float acc = 0.0f;
  for (uint32_t i = threadIdx.x; i < g.nparts; i += 256u) acc += g.part_g[i];
  acc = block_sum256(acc, red);
  if (threadIdx.x == 0) g.out2[0] = acc * (g.s_loss ? *g.s_loss : 1.0f);
}

// Row-wise rmsnorm_grad with per-block column partials of dgamma / dbeta
// (summed by bwpp_col_partials_sum).  gamma NULL means 1; with g.acc,
// dx = acc + the gradient (the residual branch's gradient added in the same
// pass; acc may be dx itself, each element being read before it is written
// by the same thread).
extern "C" __global__ __launch_bounds__(256) void bwpp_rmsnorm_grad(const BwppGradArgs g) {
  __shared__ float red[4];
  extern __shared__ float colacc[];  // [2][cols] when partials are requested
  const bool parts = g.part_g != nullptr;
  if (parts)
    for (uint32_t c = threadIdx.x; c < 2 * g.cols; c += 256) colacc[c] = 0.0f;
  __syncthreads();
  for (uint32_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
    const float *x = g.a + (size_t)r * g.ld;
    const float *dy = g.b + (size_t)r * g.ld;
    float *dx = g.out + (size_t)r * g.ld;
    const float *ac = g.acc ? g.acc + (size_t)r * g.ld : nullptr;
    float ss = 0.0f, t = 0.0f;
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) {
      const float xv = x[c];
      const float gd = g.gamma ? g.gamma[c] * dy[c] : dy[c];
      ss += xv * xv;
      t += xv * gd;
    }
    ss = block_sum256(ss, red);
    t = block_sum256(t, red);
    const float inv = 1.0f / sqrtf(ss / (float)g.cols + g.eps);
    const float mdot = inv * t / (float)g.cols;  // mean(xhat * gamma * dy)
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) {
      const float xh = x[c] * inv;
      const float d = dy[c];
      const float gd = g.gamma ? g.gamma[c] * d : d;
      const float v = inv * (gd - xh * mdot);
      if (ac) {
#pragma clang fp contract(off)
        dx[c] = ac[c] + v;  // never contracted into the product
      } else {
        dx[c] = v;
      }
      if (parts) {
        colacc[c] += d * xh;
        colacc[g.cols + c] += d;
      }
    }
  }
  if (parts) {
    __syncthreads();
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) {
      g.part_g[(size_t)blockIdx.x * g.cols + c] = colacc[c];
      g.part_b[(size_t)blockIdx.x * g.cols + c] = colacc[g.cols + c];
    }
  }
}

// rmsnorm_grad for 16-byte rows of at most 256 * VPT columns: one wave per
// row (lane l owns float4 chunks l, l + 64, ...), so the two row sums are
// wave reductions with no block barrier inside the row loop; the block's 4
// waves stride over rows, each keeping its dgamma / dbeta column sums in
// registers, and combine them once through LDS at the end into the block's
// partial row (summed by bwpp_col_partials_sum).  Same arithmetic as
// bwpp_rmsnorm_grad.  A row's loads (x, dy and acc) are all issued before
// its first use; chunks past the row end re-read the row's last chunk and
// are zeroed where they are used.
template <int VPT>
__device__ __forceinline__ void rmsnorm_grad_wave(const BwppGradArgs &g) {
  extern __shared__ float colacc[];  // [4 waves][2][cols] when partials are requested
  // wave is uniform: through readfirstlane the row pointers stay in SGPRs.
  const int lane = (int)threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const uint32_t cols = g.cols;
  const bool parts = g.part_g != nullptr;
  float4 gm[VPT], ag[VPT], ab[VPT];
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint32_t c = 4u * (uint32_t)(lane + 64 * j);
    gm[j] = make_float4(1.f, 1.f, 1.f, 1.f);
    if (g.gamma && c < cols) gm[j] = *reinterpret_cast<const float4 *>(g.gamma + c);
    ag[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    ab[j] = ag[j];
  }
  // One row's operands: x, dy and (when accumulating) acc.  acc is either
  // dx itself or disjoint from it, so reading it ahead of the row's stores
  // is exact: a lane reads each acc element before it writes that element.
  struct Row {
    float4 x[VPT], d[VPT], a[VPT];
  };
  const bool has_acc = g.acc != nullptr;
  auto load = [&](uint32_t r, Row &v) {
    const float *x = g.a + (size_t)r * g.ld;
    const float *dy = g.b + (size_t)r * g.ld;
    const float *ac = g.acc + (size_t)r * g.ld;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const uint32_t c = 4u * (uint32_t)(lane + 64 * j);
      const uint32_t cc = c < cols ? c : cols - 4u;
      v.x[j] = *reinterpret_cast<const float4 *>(x + cc);
      v.d[j] = *reinterpret_cast<const float4 *>(dy + cc);
      if (has_acc) v.a[j] = *reinterpret_cast<const float4 *>(ac + cc);
    }
  };
  auto process = [&](uint32_t r, Row &v) {
    // No contraction anywhere in the row's arithmetic: the compiler may
    // duplicate this body (with / without acc) and would be free to fuse
    // different products in each copy; with plain roundings every copy
    // gives the same bits, and dx = acc + gradient is exactly the two ops.
#pragma clang fp contract(off)
    float *dx = g.out + (size_t)r * g.ld;
    float ss = 0.0f, t = 0.0f;
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      // Zero the re-read chunks past the row end (component-wise selects:
      // a float4-valued ?: can go through memory).
      const bool in = 4u * (uint32_t)(lane + 64 * j) < cols;
      auto keep = [in](float4 q) {
        return make_float4(in ? q.x : 0.f, in ? q.y : 0.f, in ? q.z : 0.f, in ? q.w : 0.f);
      };
      v.x[j] = keep(v.x[j]);
      v.d[j] = keep(v.d[j]);
      ss += (v.x[j].x * v.x[j].x + v.x[j].y * v.x[j].y) + (v.x[j].z * v.x[j].z + v.x[j].w * v.x[j].w);
      t += (v.x[j].x * gm[j].x * v.d[j].x + v.x[j].y * gm[j].y * v.d[j].y) +
           (v.x[j].z * gm[j].z * v.d[j].z + v.x[j].w * gm[j].w * v.d[j].w);
    }
    ss = wave_sum(ss);
    t = wave_sum(t);
    const float inv = 1.0f / sqrtf(ss / (float)cols + g.eps);
    const float mdot = inv * t / (float)cols;  // mean(xhat * gamma * dy)
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const uint32_t c = 4u * (uint32_t)(lane + 64 * j);
      if (c >= cols) continue;
      float4 h, o;
      h.x = v.x[j].x * inv;
      h.y = v.x[j].y * inv;
      h.z = v.x[j].z * inv;
      h.w = v.x[j].w * inv;
      o.x = inv * (gm[j].x * v.d[j].x - h.x * mdot);
      o.y = inv * (gm[j].y * v.d[j].y - h.y * mdot);
      o.z = inv * (gm[j].z * v.d[j].z - h.z * mdot);
      o.w = inv * (gm[j].w * v.d[j].w - h.w * mdot);
      o.x = has_acc ? v.a[j].x + o.x : o.x;  // acc: a separate rounded add
      o.y = has_acc ? v.a[j].y + o.y : o.y;
      o.z = has_acc ? v.a[j].z + o.z : o.z;
      o.w = has_acc ? v.a[j].w + o.w : o.w;
      *reinterpret_cast<float4 *>(dx + c) = o;
      ag[j].x += v.d[j].x * h.x;
      ag[j].y += v.d[j].y * h.y;
      ag[j].z += v.d[j].z * h.z;
      ag[j].w += v.d[j].w * h.w;
      ab[j].x += v.d[j].x;
      ab[j].y += v.d[j].y;
      ab[j].z += v.d[j].z;
      ab[j].w += v.d[j].w;
    }
  };
  Row ra;
  for (uint32_t r = blockIdx.x * 4u + (uint32_t)wave; r < g.rows; r += gridDim.x * 4u) {
    load(r, ra);
    process(r, ra);
  }
  if (!parts) return;  // block-uniform
  float *mine = colacc + (size_t)wave * 2 * cols;
#pragma unroll
  for (int j = 0; j < VPT; ++j) {
    const uint32_t c = 4u * (uint32_t)(lane + 64 * j);
    if (c < cols) {
      *reinterpret_cast<float4 *>(mine + c) = ag[j];
      *reinterpret_cast<float4 *>(mine + cols + c) = ab[j];
    }
  }
  __syncthreads();
  for (uint32_t c = threadIdx.x; c < cols; c += 256) {
    float sg = 0.0f, sb = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      sg += colacc[(size_t)w * 2 * cols + c];
      sb += colacc[(size_t)w * 2 * cols + cols + c];
    }
    g.part_g[(size_t)blockIdx.x * cols + c] = sg;
    g.part_b[(size_t)blockIdx.x * cols + c] = sb;
  }
}

#define BWPP_RMSNORM_GRAD_WAVE(VPT)                                                                 \
  extern "C" __global__ __launch_bounds__(256) void bwpp_rmsnorm_grad_w##VPT(const BwppGradArgs g) { \
    rmsnorm_grad_wave<VPT>(g);                                                                      \
  }
BWPP_RMSNORM_GRAD_WAVE(1)
BWPP_RMSNORM_GRAD_WAVE(2)
BWPP_RMSNORM_GRAD_WAVE(4)
BWPP_RMSNORM_GRAD_WAVE(8)

// out[c] = sum_p part[p][c] for the two partial arrays (dgamma, dbeta); the
// outputs may be NULL.  A block owns 16 columns: thread (g, c) of 16 x 16
// sums parts g, g + 16, ... of column c (16 consecutive columns = 64-byte
// rows per part), then the 16 partial sums of each column are added in LDS
// in a fixed order.
extern "C" __global__ __launch_bounds__(256) void bwpp_col_partials_sum(const BwppGradArgs g) {
  __shared__ float red[2][16][17];
  const uint32_t cl = threadIdx.x & 15u, grp = threadIdx.x >> 4;
  const uint32_t c = blockIdx.x * 16u + cl;
  float sg = 0.0f, sb = 0.0f;
  if (c < g.cols) {
    // Eight parts' loads issued before their adds (same order of addition
    // as one at a time): the loop is bound by the L2 round trip, not by
    // bandwidth, and a load-add-wait per part took 32 round trips at 512
    // parts.
    uint32_t p = grp;
    for (; p + 16u * 7u < g.nparts; p += 16u * 8u) {
      float a[8], b[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        a[i] = g.part_g[(size_t)(p + 16u * i) * g.cols + c];
        b[i] = g.part_b[(size_t)(p + 16u * i) * g.cols + c];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        sg += a[i];
        sb += b[i];
      }
    }
    for (; p < g.nparts; p += 16u) {
      sg += g.part_g[(size_t)p * g.cols + c];
      sb += g.part_b[(size_t)p * g.cols + c];
    }
  }
  red[0][grp][cl] = sg;
  red[1][grp][cl] = sb;
  __syncthreads();
  if (threadIdx.x < 32) {
    const uint32_t which = threadIdx.x >> 4, col = blockIdx.x * 16u + cl;
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) t += red[which][i][cl];
    float *out = which ? g.out2 : g.out;
    if (col < g.cols && out) out[col] = t;
  }
}

// reduce_sum along each row (axis 1): one block per row.
extern "C" __global__ __launch_bounds__(256) void bwpp_reduce_sum_rows(const BwppGradArgs g) {
  __shared__ float red[4];
  for (uint32_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
    const float *x = g.a + (size_t)r * g.ld;
    float s = 0.0f;
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) s += x[c];
    s = block_sum256(s, red);
    if (threadIdx.x == 0) g.out[r] = s;
  }
}

// reduce_sum over rows (axis 0): column partials over row bands (blockIdx.y)
// into part_g, then bwpp_col_partials_sum.
extern "C" __global__ __launch_bounds__(256) void bwpp_reduce_sum_cols(const BwppGradArgs g) {
  const uint32_t c = blockIdx.x * 256u + threadIdx.x;
  if (c >= g.cols) return;
  const uint32_t band = (g.rows + gridDim.y - 1) / gridDim.y;
  const uint32_t r0 = blockIdx.y * band, r1 = min(g.rows, r0 + band);
  float s = 0.0f;
  for (uint32_t r = r0; r < r1; ++r) s += g.a[(size_t)r * g.ld + c];
  g.part_g[(size_t)blockIdx.y * g.cols + c] = s;
}

// Binary elementwise with broadcasting of b, and broadcast itself (op 4:
// out = b broadcast).  rows x cols, leading dimension ld for a / out, ldb
// for b when full.  vec (cols, ld, ldb multiples of 4, 16-byte aligned
// pointers): one float4 per thread per step, 128-bit loads and stores.
namespace {
__device__ __forceinline__ float ew1(uint32_t op, float a, float b) {
  switch (op) {
    case 0: return a + b;
    case 1: return a - b;
    case 2: return a * b;
    case 3: return a / b;
    case 5: return b / (1.0f + expf(-b));  // SiLU of b (bwpp_cpu_ref.c:4-6)
    default: return b;
  }
}
}  // namespace

extern "C" __global__ __launch_bounds__(256) void bwpp_elementwise(const BwppGradArgs g) {
  if (g.vec) {
    const uint32_t c4n = g.cols / 4;
    for (uint32_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
      const float4 *ar = g.a ? reinterpret_cast<const float4 *>(g.a + (size_t)r * g.ld) : nullptr;
      float4 *orow = reinterpret_cast<float4 *>(g.out + (size_t)r * g.ld);
      const float4 *brow = g.bmode == 0 ? reinterpret_cast<const float4 *>(g.b + (size_t)r * g.ldb)
                                        : reinterpret_cast<const float4 *>(g.b);
      const float bs = g.bmode == 2 ? g.b[r] : g.b[0];
      for (uint32_t c = threadIdx.x; c < c4n; c += 256) {
        const float4 bv = g.bmode <= 1 ? brow[c] : make_float4(bs, bs, bs, bs);
        const float4 av = ar ? ar[c] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        orow[c] = make_float4(ew1(g.op, av.x, bv.x), ew1(g.op, av.y, bv.y), ew1(g.op, av.z, bv.z),
                              ew1(g.op, av.w, bv.w));
      }
    }
    return;
  }
  for (uint32_t r = blockIdx.x; r < g.rows; r += gridDim.x) {
    const float *ar = g.a ? g.a + (size_t)r * g.ld : nullptr;
    float *orow = g.out + (size_t)r * g.ld;
    for (uint32_t c = threadIdx.x; c < g.cols; c += 256) {
      float bv;
      switch (g.bmode) {
        case 0: bv = g.b[(size_t)r * g.ldb + c]; break;
        case 1: bv = g.b[c]; break;
        case 2: bv = g.b[r]; break;
        default: bv = g.b[0]; break;
      }
      orow[c] = ew1(g.op, ar ? ar[c] : 0.0f, bv);
    }
  }
}

// Several row-strided copies in one launch (the plan's multi-pair copy:
// weights into their column blocks of a concatenation, or the blocks of a
// concatenated gradient out to the separate outputs).  Block rows stride
// over the segments' rows laid end to end.
extern "C" __global__ __launch_bounds__(256) void bwpp_copy_multi(const BwppCopyArgs a) {
  const uint32_t total = a.row0[a.n];
  for (uint32_t r = blockIdx.x; r < total; r += gridDim.x) {
    uint32_t sg = 0;
    while (sg + 1 < a.n && r >= a.row0[sg + 1]) ++sg;
    const uint32_t rr = r - a.row0[sg], cols = a.cols[sg];
    const float *src = a.src[sg] + (size_t)rr * a.ld_src[sg];
    float *dst = a.dst[sg] + (size_t)rr * a.ld_dst[sg];
    if (a.vec) {
      for (uint32_t c = threadIdx.x; c < cols / 4; c += 256)
        reinterpret_cast<float4 *>(dst)[c] = reinterpret_cast<const float4 *>(src)[c];
    } else {
      for (uint32_t c = threadIdx.x; c < cols; c += 256) dst[c] = src[c];
    }
  }
}
