// Attention forward and backward on the fp32 matrix cores of gfx950
// (v_mfma_f32_32x32x2_f32), fp32 storage, head dims K = D in {64, 128}:
//   forward   O = softmax(scale Q K^T [causal]) V, plus the per-query
//             natural-log log-sum-exp (lse) when requested;
//   backward  with p = exp(scale q.k - lse) and D_m = rowsum(dO * O)[m]:
//             dS = p (dO.v - D_m), dQ = scale dS K, dK = scale dS^T Q,
//             dV = P^T dO.
// Semantics: runtime/cpu/bwpp_cpu_ref.c:92-144 (row max, sum of exp,
// inv = sum > 0 ? 1/sum : 0) generalised with a score scale and a
// bottom-right aligned causal mask (key n visible to query m iff
// n <= m + N - M); the backward is the closed form of the graph's
// softmax_grad chain (compiler/graph_ir.c:1722-1733) fused per tile, either
// in two passes that each form S and dP (recompute) or with the dK/dV pass
// storing dS for a dQ = dS K pass (stored dS, after a D_m pass).
//
// Work layout.  A block is kW waves; each wave owns 32 rows (queries for
// the forward and dQ kernels, keys for the dK/dV kernel) and the block
// streams 32-row tiles of the other side through a two-stage LDS ring
// (register prefetch of tile t+1 during tile t, one barrier per tile).
// LDS rows are padded to D + 4 floats, so the 16-byte reads of eight
// consecutive rows hit distinct banks.
//
// MFMA operand layout (32x32x2 fp32, pinned by tests/test_gpu_mfma_layout):
// lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32]; accumulator
// register r of lane l is C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
// A dot product over the head dim runs in D/2 steps; step s pairs d = s
// (lanes 0-31) with d = D/2 + s (lanes 32-63), so each lane's operand is
// a contiguous half row (16-byte LDS reads, 16-byte global loads).
// A product over 32 rows of scores runs in 16 steps; step j pairs row
// 8 (j / 4) + j % 4 (lanes 0-31) with that row + 4 (lanes 32-63), which is
// exactly the row held by accumulator register j: probabilities and dS go
// from the accumulator into the "B" operand without data movement.
//
// Softmax runs in base 2 on scores multiplied by scale * log2(e) (passed
// as scale_log2; the plain scale is in scale).  A query's 32 scores of a
// tile are split between lanes l and l ^ 32: one permlane32 swap combines
// row maxima and the final row sums.
#include "common.h"
#include "../kargs.h"

using namespace bwpp;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kW = 4;   // waves per block (each streamed tile feeds 128 rows)
constexpr int kR = 32;  // rows per wave and per streamed tile
constexpr float kLn2 = 0.69314718055994531f;
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16 mfma(float a, float b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// Symmetric combines of lane l with lane l ^ 32.
__device__ __forceinline__ float max32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Row of accumulator register r (and of score-pair step r) for lane half hi.
__device__ __forceinline__ int acc_row(int r, int hi) { return 8 * (r >> 2) + 4 * hi + (r & 3); }

// Block-wide copy of two [kR x D] fp32 tiles (rows r0.., zero past `rows`)
// from global memory into registers, then into a padded LDS stage.
template <int D>
struct TilePair {
  static constexpr int C4 = D / 4;                   // float4 per row
  static constexpr int PER = kR * C4 / (64 * kW);    // float4 per thread per tile
  static constexpr int ST = D + 4;                   // LDS row stride (floats)
  f32x4 x[PER], y[PER];

  __device__ __forceinline__ void fetch(const float *X, uint32_t ldx, const float *Y, uint32_t ldy, uint32_t r0,
                                        uint32_t rows) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = (int)threadIdx.x + i * 64 * kW;
      const int r = idx / C4, c = idx % C4;
      const uint32_t row = r0 + (uint32_t)r;
      if (row < rows) {
        x[i] = *reinterpret_cast<const f32x4 *>(X + (size_t)row * ldx + 4 * c);
        y[i] = *reinterpret_cast<const f32x4 *>(Y + (size_t)row * ldy + 4 * c);
      } else {
        x[i] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        y[i] = x[i];
      }
    }
  }
  __device__ __forceinline__ void stash(float *lx, float *ly) const {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int idx = (int)threadIdx.x + i * 64 * kW;
      const int r = idx / C4, c = idx % C4;
      *reinterpret_cast<f32x4 *>(lx + r * ST + 4 * c) = x[i];
      *reinterpret_cast<f32x4 *>(ly + r * ST + 4 * c) = y[i];
    }
  }
};

// Half row (D/2 floats at column hi * D/2) of a [rows x ld] matrix into
// registers; zeros for rows past the end.
template <int D>
__device__ __forceinline__ void load_half_row(float (&dst)[D / 2], const float *X, uint32_t ld, uint32_t row,
                                              uint32_t rows, int hi) {
  if (row < rows) {
    const f32x4 *src = reinterpret_cast<const f32x4 *>(X + (size_t)row * ld + hi * (D / 2));
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      const f32x4 v = src[i];
      dst[4 * i] = v[0];
      dst[4 * i + 1] = v[1];
      dst[4 * i + 2] = v[2];
      dst[4 * i + 3] = v[3];
    }
  } else {
#pragma unroll
    for (int i = 0; i < D / 2; ++i) dst[i] = 0.0f;
  }
}

// acc += X_tile(rows li, half hi) . reg over the head dim: X_tile is an LDS
// tile [kR][D + 4], reg the lane's half row of the other operand.
template <int D>
__device__ __forceinline__ f32x16 dot_tile(const float *tile, const float (&reg)[D / 2], int li, int hi) {
  f32x16 acc = {};
  const float *row = tile + li * (D + 4) + hi * (D / 2);
#pragma unroll
  for (int j = 0; j < D / 2; j += 4) {
    const f32x4 v = *reinterpret_cast<const f32x4 *>(row + j);
    acc = mfma(v[0], reg[j], acc);
    acc = mfma(v[1], reg[j + 1], acc);
    acc = mfma(v[2], reg[j + 2], acc);
    acc = mfma(v[3], reg[j + 3], acc);
  }
  return acc;
}

// out[blk] (transposed [d][row-of-other-side]) += tile^T . w over the 32
// tile rows: tile [kR][D + 4] in LDS, w the 16 accumulator-layout weights.
template <int D>
__device__ __forceinline__ void acc_tile_t(f32x16 (&out)[D / 32], const float *tile, const f32x16 &w, int li,
                                           int hi) {
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const float *row = tile + acc_row(j, hi) * (D + 4) + li;
#pragma unroll
    for (int blk = 0; blk < D / 32; ++blk) out[blk] = mfma(row[32 * blk], w[j], out[blk]);
  }
}

// Stores a transposed accumulator block set (out[blk] register r = element
// [d = 32 blk + acc_row(r, hi)] of row `row`) as 16-byte pieces, times f.
template <int D>
__device__ __forceinline__ void store_t(float *X, uint32_t ld, uint32_t row, const f32x16 (&acc)[D / 32], float f,
                                        int hi) {
  float *dst = X + (size_t)row * ld + 4 * hi;
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4)
      *reinterpret_cast<f32x4 *>(dst + 32 * blk + 8 * r4) =
          f32x4{acc[blk][4 * r4] * f, acc[blk][4 * r4 + 1] * f, acc[blk][4 * r4 + 2] * f, acc[blk][4 * r4 + 3] * f};
}

struct Slice {
  uint32_t bh, b, h;
};

// Rank (0 = heaviest causal work) of this block's tile among the q_tiles
// tiles of its slice.  Blocks go out tile rank by tile rank; with zigzag
// the second half of the ranks goes out in reverse, so when the whole grid
// is resident at once (two blocks per CU, block b sharing a CU with block
// b + grid / 2) each CU holds one heavy and one light tile.
__device__ __forceinline__ uint32_t tile_rank(const BwppAttnArgs &a, uint32_t nbh) {
  const uint32_t r = blockIdx.x / nbh;
  if (!a.zigzag) return r;
  const uint32_t half = (a.q_tiles + 1) / 2;
  return r < half ? r : a.q_tiles - 1 - (r - half);
}

__device__ __forceinline__ Slice slice_of(const BwppAttnArgs &a, uint32_t nbh) {
  Slice s;
  s.bh = blockIdx.x % nbh;
  s.b = s.bh / a.heads;
  s.h = s.bh % a.heads;
  return s;
}

// ----------------------------------------------------------------- forward
template <int D, bool CAUSAL>
__device__ __forceinline__ void attn_fwd(const BwppAttnArgs &a) {
  using Tiles = TilePair<D>;
  constexpr int ST = Tiles::ST;
  __shared__ __attribute__((aligned(16))) float lds[2][2][kR * ST];  // [stage][K, V]
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const uint32_t nbh = gridDim.x / a.q_tiles;
  const uint32_t qt = a.q_tiles - 1 - tile_rank(a, nbh);  // heaviest (causal) first
  const Slice sl = slice_of(a, nbh);
  const float *Q = static_cast<const float *>(a.q) + sl.b * a.q_bs + sl.h * a.q_hs;
  const float *K = static_cast<const float *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  const float *V = static_cast<const float *>(a.v) + sl.b * a.v_bs + sl.h * a.v_hs;
  float *O = static_cast<float *>(a.o) + sl.b * a.o_bs + sl.h * a.o_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const uint32_t qb = qt * (kW * kR), q0 = qb + (uint32_t)wave * kR, qi = q0 + (uint32_t)li;

  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last = (int64_t)min(a.M, qb + kW * kR) - 1 + diag;
    kend = last < 0 ? 0u : (uint32_t)min<int64_t>(last + 1, (int64_t)a.N);
  }
  const uint32_t nt = (kend + kR - 1) / kR;
  const int64_t wlast = (int64_t)q0 + kR - 1 + diag;  // last key any query of the wave sees (causal)

  float qreg[D / 2];
  load_half_row<D>(qreg, Q, a.ldq, qi, a.M, hi);
  f32x16 o[D / 32];
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk) o[blk] = f32x16{};
  float mrun = -INFINITY, lsum = 0.0f;
  const float c = a.scale_log2;

  Tiles pf;
  if (nt > 0) {
    pf.fetch(K, a.ldk, V, a.ldv, 0, a.N);
    pf.stash(lds[0][0], lds[0][1]);
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    const int st = (int)(t & 1);
    const uint32_t k0 = t * kR;
    if (t + 1 < nt) pf.fetch(K, a.ldk, V, a.ldv, k0 + kR, a.N);
    if (!CAUSAL || (int64_t)k0 <= wlast) {  // wave-uniform
      f32x16 s = dot_tile<D>(lds[st][0], qreg, li, hi);
      const bool edge = k0 + kR > a.N || (CAUSAL && (int64_t)k0 + kR - 1 > (int64_t)q0 + diag);
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] *= c;
      // Keys past N or above the diagonal: -inf, under one block-uniform
      // branch (per element the test became compares and selects on every
      // tile).
      if (edge) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t key = k0 + (uint32_t)acc_row(r, hi);
          if (key >= a.N || (CAUSAL && (int64_t)key > (int64_t)qi + diag)) s[r] = -INFINITY;
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[r]);
      mx = max32(mx);
      const float mnew = fmaxf(mrun, mx);
      const float mu = mnew == -INFINITY ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(mrun - mu);
      float ps = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - mu);
        ps += s[r];
      }
      lsum = lsum * alpha + ps;
      mrun = mnew;
#pragma unroll
      for (int blk = 0; blk < D / 32; ++blk) o[blk] *= alpha;
      acc_tile_t<D>(o, lds[st][1], s, li, hi);
    }
    if (t + 1 < nt) pf.stash(lds[st ^ 1][0], lds[st ^ 1][1]);
    __syncthreads();
  }
  const float ltot = sum32(lsum);
  if (qi < a.M) {
    store_t<D>(O, a.ldo, qi, o, ltot > 0.0f ? 1.0f / ltot : 0.0f, hi);
    if (a.lse && hi == 0) a.lse[(size_t)sl.bh * a.M + qi] = ltot > 0.0f ? (mrun + log2f(ltot)) * kLn2 : -INFINITY;
  }
}

// ---------------------------------------------------------------- backward
// D_m = rowsum(dO * O) of query row qi (greg: the lane's half of dO's row):
// each lane half sums its D / 2 products in order, then the halves add.
// The dQ pass and the D_m pass both use it, so both give the same bits.
template <int D>
__device__ __forceinline__ float row_dsum(const float (&greg)[D / 2], const float *O, uint32_t ldo, uint32_t qi,
                                          uint32_t M, int hi) {
  float orow[D / 2];
  load_half_row<D>(orow, O, ldo, qi, M, hi);
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < D / 2; ++i) part += greg[i] * orow[i];
  return sum32(part);
}

// D_m pass of the stored-dS scheme: a wave per 32 query rows, q_tiles
// blocks of kW waves per slice.
template <int D>
__device__ __forceinline__ void attn_bwd_dsum(const BwppAttnArgs &a) {
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const uint32_t bh = blockIdx.x / a.q_tiles, tile = blockIdx.x % a.q_tiles;
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const float *O = static_cast<const float *>(a.o) + b * a.o_bs + h * a.o_hs;
  const float *dO = static_cast<const float *>(a.dout) + b * a.o_bs + h * a.o_hs;
  const uint32_t qi = (tile * kW + (uint32_t)wave) * kR + (uint32_t)li;
  float greg[D / 2];
  load_half_row<D>(greg, dO, a.ldo, qi, a.M, hi);
  const float dsum = row_dsum<D>(greg, O, a.ldo, qi, a.M, hi);
  if (qi < a.M && hi == 0) a.dsum[(size_t)bh * a.M + qi] = dsum;
}

// Stored fp32 dS^T (the stored-dS scheme): per slice, 4 KiB blocks of 32
// keys x 32 queries, [key block][query block] (query blocks padded to
// ld_dst / 32, a multiple of 4; the order of the bf16 blocks in
// attention_bwd.hip).  Inside a block the 16-byte piece holding queries
// 4 qd .. +3 of key k sits at
//   1024 (qd / 2) + 32 (k ^ (qd / 2)) + 16 (qd % 2):
// a wave of the dK / dV pass (lane = key, with quads 2 r4 + hi in its
// accumulator registers 4 r4 .. +3) writes 1 KiB per store, and the dQ
// pass's 4-byte reads (lanes = 32 queries of a wave at keys k and k + 4)
// hit 64 distinct banks (the XOR spreads the four quad pairs, 1 KiB apart,
// over the eight 32-byte bank groups with the + 4 key).
struct DsBlk32 {
  static constexpr uint32_t kBytes = 4096;
  __device__ __forceinline__ static size_t at(uint32_t bh, uint32_t kb, uint32_t qb, uint32_t n32, uint32_t m32) {
    return (((size_t)bh * n32 + kb) * m32 + qb) * kBytes;
  }
  // Byte offset of (key k, query q) inside a block.
  __device__ __forceinline__ static uint32_t elem(uint32_t k, uint32_t q) {
    return 1024u * (q >> 3) + 32u * (k ^ (q >> 3)) + 4u * (q & 7u);
  }
};

// dQ pass of the stored-dS scheme: dQ = scale dS K with dS^T read from
// a.dst (written by the dK / dV pass) instead of recomputed from S and dP.
// A wave owns 32 queries; the block streams K tiles and the matching 16 KiB
// of dS^T blocks (its 4 query blocks of a key block) through the two-stage
// ring.  The same 32 x 32 blocks as in
// attn_bwd_dq are visited (the dK / dV pass stores exactly those) and
// every MFMA gets the same operands in the same order, so dQ is
// bit-identical to attn_bwd_dq's but for the sign of all-zero sums.
template <int D, bool CAUSAL>
__device__ __forceinline__ void attn_bwd_dq_ds(const BwppAttnArgs &a) {
  constexpr int ST = D + 4, SB = kW * (int)DsBlk32::kBytes;  // dS^T bytes per tile
  constexpr int SPT = SB / 16 / (64 * kW);                      // float4 per thread per dS^T tile
  constexpr int KPT = kR * (D / 4) / (64 * kW);                 // float4 per thread per K tile
  __shared__ __attribute__((aligned(16))) float kt[2][kR * ST];
  __shared__ __attribute__((aligned(16))) unsigned char dst[2][SB];
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const uint32_t nbh = gridDim.x / a.q_tiles;
  const uint32_t qt = a.q_tiles - 1 - tile_rank(a, nbh);
  const Slice sl = slice_of(a, nbh);
  const float *K = static_cast<const float *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  float *dQ = static_cast<float *>(a.dq) + sl.b * a.q_bs + sl.h * a.q_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const uint32_t qb = qt * (kW * kR), q0 = qb + (uint32_t)wave * kR, qi = q0 + (uint32_t)li;
  const uint32_t n32 = (a.N + 31u) / 32u, m32 = a.ld_dst / 32u;
  const unsigned char *S = static_cast<const unsigned char *>(a.dst) + DsBlk32::at(sl.bh, 0, qb / 32u, n32, m32);

  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last = (int64_t)min(a.M, qb + kW * kR) - 1 + diag;
    kend = last < 0 ? 0u : (uint32_t)min<int64_t>(last + 1, (int64_t)a.N);
  }
  const uint32_t nt = (kend + kR - 1) / kR;
  const int64_t wlast = (int64_t)q0 + kR - 1 + diag;
  // This lane's dS^T element offsets (query li, key acc_row(j, hi)).
  uint32_t eoff[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) eoff[j] = (uint32_t)wave * DsBlk32::kBytes + DsBlk32::elem((uint32_t)acc_row(j, hi), (uint32_t)li);

  f32x16 dq[D / 32];
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk) dq[blk] = f32x16{};

  f32x4 kx[KPT], sx[SPT];
  auto fetch = [&](uint32_t t) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int idx = (int)threadIdx.x + i * 64 * kW, r = idx / (D / 4), c = idx % (D / 4);
      const uint32_t row = t * kR + (uint32_t)r;
      kx[i] = row < a.N ? *reinterpret_cast<const f32x4 *>(K + (size_t)row * a.ldk + 4 * c)
                        : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const f32x4 *src = reinterpret_cast<const f32x4 *>(S + (size_t)t * m32 * DsBlk32::kBytes);
#pragma unroll
    for (int i = 0; i < SPT; ++i) sx[i] = src[(int)threadIdx.x + i * 64 * kW];
  };
  auto stash = [&](int st) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int idx = (int)threadIdx.x + i * 64 * kW, r = idx / (D / 4), c = idx % (D / 4);
      *reinterpret_cast<f32x4 *>(&kt[st][r * ST + 4 * c]) = kx[i];
    }
#pragma unroll
    for (int i = 0; i < SPT; ++i) reinterpret_cast<f32x4 *>(dst[st])[(int)threadIdx.x + i * 64 * kW] = sx[i];
  };
  if (nt > 0) {
    fetch(0);
    stash(0);
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    const int st = (int)(t & 1);
    const uint32_t k0 = t * kR;
    if (t + 1 < nt) fetch(t + 1);
    if (!CAUSAL || (int64_t)k0 <= wlast) {
      f32x16 w;
#pragma unroll
      for (int j = 0; j < 16; ++j) w[j] = *reinterpret_cast<const float *>(dst[st] + eoff[j]);
      if (k0 + kR > a.N) {  // keys past N: dS = 0 (their K rows are zero)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (k0 + (uint32_t)acc_row(j, hi) >= a.N) w[j] = 0.0f;
      }
      acc_tile_t<D>(dq, kt[st], w, li, hi);  // dQ^T += K^T dS^T
    }
    if (t + 1 < nt) stash(st ^ 1);
    __syncthreads();
  }
  if (qi < a.M) store_t<D>(dQ, a.ldq, qi, dq, a.scale, hi);
}

// dQ pass: a wave owns 32 queries and streams K / V tiles; it also writes
// D_m = rowsum(dO * O) for the dK / dV pass.
template <int D, bool CAUSAL>
__device__ __forceinline__ void attn_bwd_dq(const BwppAttnArgs &a) {
  using Tiles = TilePair<D>;
  constexpr int ST = Tiles::ST;
  __shared__ __attribute__((aligned(16))) float lds[2][2][kR * ST];  // [stage][K, V]
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const uint32_t nbh = gridDim.x / a.q_tiles;
  const uint32_t qt = a.q_tiles - 1 - tile_rank(a, nbh);
  const Slice sl = slice_of(a, nbh);
  const float *Q = static_cast<const float *>(a.q) + sl.b * a.q_bs + sl.h * a.q_hs;
  const float *K = static_cast<const float *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  const float *V = static_cast<const float *>(a.v) + sl.b * a.v_bs + sl.h * a.v_hs;
  const float *O = static_cast<const float *>(a.o) + sl.b * a.o_bs + sl.h * a.o_hs;
  const float *dO = static_cast<const float *>(a.dout) + sl.b * a.o_bs + sl.h * a.o_hs;
  float *dQ = static_cast<float *>(a.dq) + sl.b * a.q_bs + sl.h * a.q_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const uint32_t qb = qt * (kW * kR), q0 = qb + (uint32_t)wave * kR, qi = q0 + (uint32_t)li;

  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last = (int64_t)min(a.M, qb + kW * kR) - 1 + diag;
    kend = last < 0 ? 0u : (uint32_t)min<int64_t>(last + 1, (int64_t)a.N);
  }
  const uint32_t nt = (kend + kR - 1) / kR;
  const int64_t wlast = (int64_t)q0 + kR - 1 + diag;

  float qreg[D / 2], greg[D / 2];
  load_half_row<D>(qreg, Q, a.ldq, qi, a.M, hi);
  load_half_row<D>(greg, dO, a.ldo, qi, a.M, hi);
  const float dsum = row_dsum<D>(greg, O, a.ldo, qi, a.M, hi);
  if (qi < a.M && hi == 0) a.dsum[(size_t)sl.bh * a.M + qi] = dsum;
  // Queries past M: +inf makes every probability exp2(-inf) = 0.
  const float lse2 = qi < a.M ? a.lse[(size_t)sl.bh * a.M + qi] * kLog2e : INFINITY;
  const float c = a.scale_log2;

  f32x16 dq[D / 32];
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk) dq[blk] = f32x16{};

  Tiles pf;
  if (nt > 0) {
    pf.fetch(K, a.ldk, V, a.ldv, 0, a.N);
    pf.stash(lds[0][0], lds[0][1]);
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    const int st = (int)(t & 1);
    const uint32_t k0 = t * kR;
    if (t + 1 < nt) pf.fetch(K, a.ldk, V, a.ldv, k0 + kR, a.N);
    if (!CAUSAL || (int64_t)k0 <= wlast) {
      f32x16 s = dot_tile<D>(lds[st][0], qreg, li, hi);   // S^T [key][query]
      const f32x16 dp = dot_tile<D>(lds[st][1], greg, li, hi);  // dP^T = V dO^T
      const bool edge = k0 + kR > a.N || (CAUSAL && (int64_t)k0 + kR - 1 > (int64_t)q0 + diag);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(s[r] * c - lse2);
        s[r] = p * (dp[r] - dsum);  // dS^T
      }
      if (edge) {  // masked keys: p = 0 (one block-uniform branch)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const uint32_t key = k0 + (uint32_t)acc_row(r, hi);
          if (key >= a.N || (CAUSAL && (int64_t)key > (int64_t)qi + diag)) s[r] = 0.0f * (dp[r] - dsum);
        }
      }
      acc_tile_t<D>(dq, lds[st][0], s, li, hi);  // dQ^T += K^T dS^T
    }
    if (t + 1 < nt) pf.stash(lds[st ^ 1][0], lds[st ^ 1][1]);
    __syncthreads();
  }
  if (qi < a.M) store_t<D>(dQ, a.ldq, qi, dq, a.scale, hi);
}

// dK / dV pass: a wave owns 32 keys and streams Q / dO tiles with their
// lse and D_m.  WS: also stores dS^T to a.dst for attn_bwd_dq_ds.
template <int D, bool CAUSAL, bool WS = false>
__device__ __forceinline__ void attn_bwd_dkdv(const BwppAttnArgs &a) {
  using Tiles = TilePair<D>;
  constexpr int ST = Tiles::ST;
  __shared__ __attribute__((aligned(16))) float lds[2][2][kR * ST];  // [stage][Q, dO]
  __shared__ __attribute__((aligned(16))) float rowv[2][2][kR];      // [stage][lse2, D_m]
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const uint32_t nbh = gridDim.x / a.q_tiles;  // q_tiles holds the key tiles here
  const uint32_t kt = tile_rank(a, nbh);         // heaviest (causal) first
  const Slice sl = slice_of(a, nbh);
  const float *Q = static_cast<const float *>(a.q) + sl.b * a.q_bs + sl.h * a.q_hs;
  const float *K = static_cast<const float *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  const float *V = static_cast<const float *>(a.v) + sl.b * a.v_bs + sl.h * a.v_hs;
  const float *dO = static_cast<const float *>(a.dout) + sl.b * a.o_bs + sl.h * a.o_hs;
  float *dK = static_cast<float *>(a.dk) + sl.b * a.k_bs + sl.h * a.k_hs;
  float *dV = static_cast<float *>(a.dv) + sl.b * a.v_bs + sl.h * a.v_hs;
  const float *lse = a.lse + (size_t)sl.bh * a.M;
  const float *dsum = a.dsum + (size_t)sl.bh * a.M;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const uint32_t kb = kt * (kW * kR), k0w = kb + (uint32_t)wave * kR, ni = k0w + (uint32_t)li;

  // Queries that see a key n: m >= n - diag (causal).
  uint32_t mbeg = 0;
  if (CAUSAL) {
    const int64_t first = (int64_t)kb - diag;
    mbeg = first <= 0 ? 0u : (first >= (int64_t)a.M ? a.M : (uint32_t)first);
    mbeg -= mbeg % kR;
  }
  const uint32_t nt = a.M > mbeg ? (a.M - mbeg + kR - 1) / kR : 0u;
  const int64_t wfirst = (int64_t)k0w - diag;  // first query that sees any key of the wave

  float kreg[D / 2], vreg[D / 2];
  load_half_row<D>(kreg, K, a.ldk, ni, a.N, hi);
  load_half_row<D>(vreg, V, a.ldv, ni, a.N, hi);
  f32x16 dk[D / 32], dv[D / 32];
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk) dk[blk] = dv[blk] = f32x16{};
  const float c = a.scale_log2;

  Tiles pf;
  float rl = INFINITY, rd = 0.0f;  // lse2 / D_m of row threadIdx.x (< kR)
  auto fetch_rows = [&](uint32_t m0) {
    if (threadIdx.x < (uint32_t)kR) {
      const uint32_t m = m0 + threadIdx.x;
      rl = m < a.M ? lse[m] * kLog2e : INFINITY;
      rd = m < a.M ? dsum[m] : 0.0f;
    }
  };
  auto stash_rows = [&](int st) {
    if (threadIdx.x < (uint32_t)kR) {
      rowv[st][0][threadIdx.x] = rl;
      rowv[st][1][threadIdx.x] = rd;
    }
  };
  if (nt > 0) {
    pf.fetch(Q, a.ldq, dO, a.ldo, mbeg, a.M);
    fetch_rows(mbeg);
    pf.stash(lds[0][0], lds[0][1]);
    stash_rows(0);
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    const int st = (int)(t & 1);
    const uint32_t m0 = mbeg + t * kR;
    if (t + 1 < nt) {
      pf.fetch(Q, a.ldq, dO, a.ldo, m0 + kR, a.M);
      fetch_rows(m0 + kR);
    }
    if (!CAUSAL || (int64_t)m0 + kR - 1 >= wfirst) {
      f32x16 s = dot_tile<D>(lds[st][0], kreg, li, hi);          // S [query][key]
      const f32x16 dp = dot_tile<D>(lds[st][1], vreg, li, hi);   // dP = dO V^T
      const bool edge = CAUSAL && (int64_t)m0 < wfirst + kR - 1;
      f32x16 ds;
#pragma unroll
      for (int r4 = 0; r4 < 4; ++r4) {
        const int row = 8 * r4 + 4 * hi;
        const f32x4 l4 = *reinterpret_cast<const f32x4 *>(&rowv[st][0][row]);
        const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&rowv[st][1][row]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = 4 * r4 + e;
          const float p = __builtin_amdgcn_exp2f(s[r] * c - l4[e]);
          s[r] = p;
          ds[r] = p * (dp[r] - d4[e]);
        }
      }
      if (edge) {  // queries before this key's diagonal: p = 0 (one block-uniform branch)
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int row = 8 * r4 + 4 * hi;
          const f32x4 d4 = *reinterpret_cast<const f32x4 *>(&rowv[st][1][row]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * r4 + e;
            if ((int64_t)ni > (int64_t)(m0 + (uint32_t)(row + e)) + diag) {
              s[r] = 0.0f;
              ds[r] = 0.0f * (dp[r] - d4[e]);
            }
          }
        }
      }
      if constexpr (WS) {
        // Registers 4 r4 .. +3: queries of quad 2 r4 + hi (1 KiB per store;
        // a wave past N has no block).
        if (k0w < a.N) {
          unsigned char *blk = static_cast<unsigned char *>(a.dst) +
                               DsBlk32::at(sl.bh, k0w / 32u, m0 / 32u, (a.N + 31u) / 32u, a.ld_dst / 32u);
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4)
            __builtin_nontemporal_store(f32x4{ds[4 * r4], ds[4 * r4 + 1], ds[4 * r4 + 2], ds[4 * r4 + 3]},
                                        reinterpret_cast<f32x4 *>(blk + 1024u * r4 + 32u * ((uint32_t)li ^ r4) +
                                                                  16u * (uint32_t)hi));
        }
      }
      acc_tile_t<D>(dv, lds[st][1], s, li, hi);   // dV^T += dO^T P
      acc_tile_t<D>(dk, lds[st][0], ds, li, hi);  // dK^T += Q^T dS
    }
    if (t + 1 < nt) {
      pf.stash(lds[st ^ 1][0], lds[st ^ 1][1]);
      stash_rows(st ^ 1);
    }
    __syncthreads();
  }
  if (ni < a.N) {
    store_t<D>(dK, a.ldk, ni, dk, a.scale, hi);
    store_t<D>(dV, a.ldv, ni, dv, 1.0f, hi);
  }
}

}  // namespace

#define BWPP_ATTN_F32(D, CAUSAL, SUFFIX)                                                                    \
  extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_f32_mfma_d##D##SUFFIX(const BwppAttnArgs a) { \
    attn_fwd<D, CAUSAL>(a);                                                                                 \
  }                                                                                                         \
  extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_bwd_f32_mfma_d##D##SUFFIX##_dq(           \
      const BwppAttnArgs a) {                                                                               \
    attn_bwd_dq<D, CAUSAL>(a);                                                                              \
  }                                                                                                         \
  extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_bwd_f32_mfma_d##D##SUFFIX##_dkdv(         \
      const BwppAttnArgs a) {                                                                               \
    attn_bwd_dkdv<D, CAUSAL>(a);                                                                            \
  }

BWPP_ATTN_F32(64, false, )
BWPP_ATTN_F32(64, true, _causal)
BWPP_ATTN_F32(128, false, )
BWPP_ATTN_F32(128, true, _causal)

// The stored-dS scheme: D_m pass, dK / dV pass that also stores dS^T, and
// the dQ = dS K pass.
#define BWPP_ATTN_F32_DS(D, CAUSAL, SUFFIX)                                                                 \
  extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_bwd_f32_mfma_d##D##SUFFIX##_dkdv_ds(      \
      const BwppAttnArgs a) {                                                                               \
    attn_bwd_dkdv<D, CAUSAL, true>(a);                                                                      \
  }                                                                                                         \
  extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_bwd_f32_mfma_d##D##SUFFIX##_dq_ds(        \
      const BwppAttnArgs a) {                                                                               \
    attn_bwd_dq_ds<D, CAUSAL>(a);                                                                           \
  }
BWPP_ATTN_F32_DS(64, false, )
BWPP_ATTN_F32_DS(64, true, _causal)
BWPP_ATTN_F32_DS(128, false, )
BWPP_ATTN_F32_DS(128, true, _causal)
extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_bwd_f32_d64_dsum(const BwppAttnArgs a) {
  attn_bwd_dsum<64>(a);
}
extern "C" __global__ __launch_bounds__(64 * kW) void bwpp_attn_bwd_f32_d128_dsum(const BwppAttnArgs a) {
  attn_bwd_dsum<128>(a);
}

// bf16 <-> fp32 operand copies for running bf16 attention backward on the
// fp32 kernels above: element (slice, r, c) of the strided bf16 tensor <->
// element [(slice * rows + r) * cols + c] of the fp32 buffer.  Eight columns
// per thread (cols is a multiple of 8 here); fp32 -> bf16 rounds to nearest
// even.
__device__ __forceinline__ size_t conv_src(const BwppConvArgs &a, uint32_t sl, uint32_t r, uint32_t c) {
  return (size_t)(sl / a.heads) * a.bs + (size_t)(sl % a.heads) * a.hs + (size_t)r * a.ld + c;
}

extern "C" __global__ __launch_bounds__(256) void bwpp_attn_conv_bf16_to_f32(const BwppConvArgs a) {
  const uint32_t c8 = a.cols / 8;
  const size_t total = (size_t)a.slices * a.rows * c8;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const uint32_t c = (uint32_t)(i % c8) * 8;
    const size_t sr = i / c8;
    const uint32_t r = (uint32_t)(sr % a.rows), sl = (uint32_t)(sr / a.rows);
    const uint16_t *src = static_cast<const uint16_t *>(a.src) + conv_src(a, sl, r, c);
    float4 lo, hi;
    if (a.vec) {
      const uint4 v = *reinterpret_cast<const uint4 *>(src);
      lo = make_float4(__uint_as_float(v.x << 16), __uint_as_float(v.x & 0xffff0000u), __uint_as_float(v.y << 16),
                       __uint_as_float(v.y & 0xffff0000u));
      hi = make_float4(__uint_as_float(v.z << 16), __uint_as_float(v.z & 0xffff0000u), __uint_as_float(v.w << 16),
                       __uint_as_float(v.w & 0xffff0000u));
    } else {
      lo = make_float4(bf16_bits_to_f32(src[0]), bf16_bits_to_f32(src[1]), bf16_bits_to_f32(src[2]),
                       bf16_bits_to_f32(src[3]));
      hi = make_float4(bf16_bits_to_f32(src[4]), bf16_bits_to_f32(src[5]), bf16_bits_to_f32(src[6]),
                       bf16_bits_to_f32(src[7]));
    }
    float *dst = static_cast<float *>(a.dst) + sr * a.cols + c;
    *reinterpret_cast<float4 *>(dst) = lo;
    *reinterpret_cast<float4 *>(dst + 4) = hi;
  }
}

extern "C" __global__ __launch_bounds__(256) void bwpp_attn_conv_f32_to_bf16(const BwppConvArgs a) {
  const uint32_t c8 = a.cols / 8;
  const size_t total = (size_t)a.slices * a.rows * c8;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const uint32_t c = (uint32_t)(i % c8) * 8;
    const size_t sr = i / c8;
    const uint32_t r = (uint32_t)(sr % a.rows), sl = (uint32_t)(sr / a.rows);
    const float *src = static_cast<const float *>(a.src) + sr * a.cols + c;
    const float4 lo = *reinterpret_cast<const float4 *>(src);
    const float4 hi = *reinterpret_cast<const float4 *>(src + 4);
    const uint4 w = make_uint4(pack_bf16x2(lo.x, lo.y), pack_bf16x2(lo.z, lo.w), pack_bf16x2(hi.x, hi.y),
                               pack_bf16x2(hi.z, hi.w));
    uint16_t *dst = static_cast<uint16_t *>(a.dst) + conv_src(a, sl, r, c);
    if (a.vec) {
      *reinterpret_cast<uint4 *>(dst) = w;
    } else {
      const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        dst[2 * e] = (uint16_t)(ws[e] & 0xffffu);
        dst[2 * e + 1] = (uint16_t)(ws[e] >> 16);
      }
    }
  }
}
