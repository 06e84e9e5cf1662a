// MFMA GEMMs for gfx950:  C = op(A) · op(B) (+ bias[col]) (-> SiLU).
//
// Semantics: runtime/cpu/bwpp_cpu_ref.c:8-35 (fp32 accumulation, bias added
// to the accumulator, then SiLU x / (1 + e^-x)); the MSL kernel it replaces
// is codegen_metal.c:357-434.  op(A) is A [M x K] or, with TA, the transpose
// of a stored [K x M]; op(B) is B [K x N] or, with TB, the transpose of a
// stored [N x K].
//
// Both kernels compute C^T tiles: the MFMA "A" operand is a tile of op(B)^T
// (rows = output columns n) and the "B" operand a tile of op(A)^T (columns =
// output rows m).  The accumulator of v_mfma_f32_32x32x{16_bf16,2f32} then
// gives each lane one output row m and runs of 4 consecutive columns n, so
// the epilogue stores 8-byte (bf16) or 16-byte (fp32) runs.
//
// bf16 kernel (v_mfma_f32_32x32x16_bf16, 8 bf16 per lane per operand):
//   block tile BM x BN x BK = 256 x 256 x 64, 4 waves in 2 x 2, each wave
//   128 x 128 (4 x 4 MFMA tiles of 32 x 32).  Both operands sit in LDS
//   K-contiguous ([row][k], 128-byte rows of eight 16-byte chunks, chunk c of
//   row r stored at c ^ (r & 7)), double-buffered: 2 x 64 KiB.  An operand
//   whose rows are K-contiguous in memory is copied with 16-byte loads; one
//   that is MN-contiguous (row-major B, or A with TA) is loaded as 8 x 8
//   blocks and transposed in registers on the way to LDS.
// fp32 kernel (v_mfma_f32_32x32x2f32, 1 float per lane per operand):
//   128 x 128 x 32 tile, 4 waves in 2 x 2 (64 x 64 each); an operand keeps its
//   memory orientation in LDS (MN-contiguous rows padded to R+32 floats,
//   K-contiguous rows padded to BK+2), which makes the per-lane 4-byte MFMA
//   operand reads bank-conflict free without any transpose.
//
// Tile order: workgroups are dispatched round-robin over the 8 XCDs, so
// block b is remapped to tile (b % 8) * (T / 8) + b / 8 (when 8 | T), giving
// each XCD a contiguous run of tiles; runs are walked group_m tile-rows at a
// time so tiles that share A rows and B columns meet in the same L2.
#include <type_traits>

#include "common.h"
#include "../kargs.h"

using namespace bwpp;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

namespace {

constexpr uint32_t kEpiAdd = 1u, kEpiSilu = 2u;

__device__ __forceinline__ void tile_coords(const BwppGemmArgs &a, uint32_t &tm, uint32_t &tn,
                                            uint32_t b = blockIdx.x) {
  const uint32_t T = a.tiles_m * a.tiles_n;
  if ((T & 7u) == 0) b = (b & 7u) * (T >> 3) + (b >> 3);
  const uint32_t gm = a.group_m;
  const uint32_t per_group = gm * a.tiles_n;
  const uint32_t g = b / per_group;
  const uint32_t first = g * gm;
  const uint32_t rows = min(gm, a.tiles_m - first);
  const uint32_t idx = b - g * per_group;
  tm = first + idx % rows;
  tn = idx / rows;
}

// x / (1 + e^-x) with the hardware exp2 and reciprocal (about 2 ulp):
// e^-x overflows to +inf for x < -88 and the result is then -0, as the
// reference's x / (1 + expf(-x)).
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x * -1.44269504088896341f));
}

// Fused tails of the fp32 kernels (BWPP_HIP_FUSE_*), applied to the
// epilogue's result y of element (m, n): residual y + aux, SiLU gradient
// y * s (1 + x (1 - s)) with x = aux (the form of grad.hip's silu_grad),
// dual output c2 = SiLU(y) (written by the caller of this function).
constexpr uint32_t kFuseResidual = 1u, kFuseDualSilu = 2u, kFuseSiluGrad = 3u;
__device__ __forceinline__ float fuse1(uint32_t fuse, float y, float x) {
  if (fuse == kFuseResidual) return y + x;
  if (fuse == kFuseSiluGrad) {
    const float s = 1.0f / (1.0f + __expf(-x));
    return y * (s * (1.0f + x * (1.0f - s)));
  }
  return y;
}
__device__ __forceinline__ float4 fuse4(uint32_t fuse, float4 y, float4 x) {
  return make_float4(fuse1(fuse, y.x, x.x), fuse1(fuse, y.y, x.y), fuse1(fuse, y.z, x.z), fuse1(fuse, y.w, x.w));
}
__device__ __forceinline__ bool fuse_reads_aux(uint32_t fuse) { return fuse == kFuseResidual || fuse == kFuseSiluGrad; }

// ---------------------------------------------------------------- bf16

__device__ __forceinline__ uint32_t dword(const uint4 &v, int d) {
  return d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
}
// bf16 i (0..7) of x0's row and the same of x1's row, packed as one dword.
__device__ __forceinline__ uint32_t pair_b16(int i, const uint4 &r0, const uint4 &r1) {
  const uint32_t x0 = dword(r0, i >> 1), x1 = dword(r1, i >> 1);
  return (i & 1) ? ((x0 >> 16) | (x1 & 0xFFFF0000u)) : ((x0 & 0xFFFFu) | (x1 << 16));
}
// 8 x 8 transpose of bf16: in[r] holds row r (8 values; dword d holds
// elements 2d and 2d+1 in its low and high halves); out[i] = column i.
__device__ __forceinline__ void transpose8x8_b16(const uint4 (&in)[8], uint4 (&out)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
    out[i] = make_uint4(pair_b16(i, in[0], in[1]), pair_b16(i, in[2], in[3]),
                        pair_b16(i, in[4], in[5]), pair_b16(i, in[6], in[7]));
}

// Gathers up to 8 bf16 from p[0..7] (element e kept only if ok(e)) into a
// 16-byte chunk, zero elsewhere.
template <class Ok>
__device__ __forceinline__ uint4 gather8_b16(const uint16_t *p, Ok ok) {
  uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (ok(e)) w[e >> 1] |= (uint32_t)p[e] << ((e & 1) * 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// One 16-byte chunk (8 bf16) of a K-contiguous row, guarded for edges.
template <bool EDGE>
__device__ __forceinline__ uint4 load_chunk_b16(const uint16_t *base, uint32_t ld, uint32_t row,
                                               uint32_t rows, uint32_t k, uint32_t K, bool vec) {
  if (!EDGE) return *reinterpret_cast<const uint4 *>(base + (size_t)row * ld + k);
  if (row >= rows) return make_uint4(0, 0, 0, 0);
  const uint16_t *p = base + (size_t)row * ld + k;
  if (vec && k + 8 <= K) return *reinterpret_cast<const uint4 *>(p);
  return gather8_b16(p, [&](int e) { return k + e < K; });
}

// 8 consecutive MN elements of one K row of an MN-contiguous operand.
template <bool EDGE>
__device__ __forceinline__ uint4 load_mnrow_b16(const uint16_t *base, uint32_t ld, uint32_t k,
                                               uint32_t K, uint32_t mn, uint32_t MN, bool vec) {
  if (!EDGE) return *reinterpret_cast<const uint4 *>(base + (size_t)k * ld + mn);
  if (k >= K) return make_uint4(0, 0, 0, 0);
  const uint16_t *p = base + (size_t)k * ld + mn;
  if (vec && mn + 8 <= MN) return *reinterpret_cast<const uint4 *>(p);
  return gather8_b16(p, [&](int e) { return mn + e < MN; });
}

// Staging of one operand tile (R rows of the LDS tile, BK = 64) through
// registers.  MNC: the operand is MN-contiguous in memory (needs transpose).
template <int R, int NT, bool MNC, bool EDGE>
struct StageB16 {
  static constexpr int kChunks = MNC ? (64 / 8) * (R / 8) / NT : R * 8 / NT;
  static constexpr int kRegs = MNC ? 8 * kChunks : kChunks;
  uint4 r[kRegs];

  // r0: first tile row (m or n); k0: first k; rows: M or N; ld: row stride.
  __device__ __forceinline__ void load(const uint16_t *g, uint32_t ld, uint32_t r0, uint32_t rows,
                                       uint32_t k0, uint32_t K, bool vec, int tid) {
    if constexpr (!MNC) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int q = tid + i * NT;
        const int row = q >> 3, c = q & 7;
        r[i] = load_chunk_b16<EDGE>(g, ld, r0 + row, rows, k0 + c * 8, K, vec);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int q = tid + i * NT;
        const int kb = q / (R / 8), nb = q % (R / 8);
#pragma unroll
        for (int e = 0; e < 8; ++e)
          r[i * 8 + e] = load_mnrow_b16<EDGE>(g, ld, k0 + kb * 8 + e, K, r0 + nb * 8, rows, vec);
      }
    }
  }

  __device__ __forceinline__ void store(uint16_t *s, int tid) const {
    uint4 *s4 = reinterpret_cast<uint4 *>(s);  // [R][8] chunks
    if constexpr (!MNC) {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int q = tid + i * NT;
        const int row = q >> 3, c = q & 7;
        s4[row * 8 + (c ^ (row & 7))] = r[i];
      }
    } else {
#pragma unroll
      for (int i = 0; i < kChunks; ++i) {
        const int q = tid + i * NT;
        const int kb = q / (R / 8), nb = q % (R / 8);
        uint4 in[8], out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) in[e] = r[i * 8 + e];
        transpose8x8_b16(in, out);
#pragma unroll
        for (int e = 0; e < 8; ++e) s4[(nb * 8 + e) * 8 + (kb ^ e)] = out[e];
      }
    }
  }
};

template <bool TA, bool TB, bool EDGE>
__device__ __forceinline__ void gemm_bf16(const BwppGemmArgs &a) {
  constexpr int BM = 256, BN = 256, BK = 64, WM = 2, WN = 2;
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  constexpr int kBuf = (BM + BN) * BK;
  constexpr int kCld = BN + 8;  // epilogue tile row stride (bf16)
  constexpr int kSmem = 2 * kBuf > BM * kCld ? 2 * kBuf : BM * kCld;
  __shared__ __attribute__((aligned(16))) uint16_t smem[kSmem];  // 132 KiB

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  uint32_t tm, tn;
  tile_coords(a, tm, tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint16_t *A = static_cast<const uint16_t *>(a.a);
  const uint16_t *B = static_cast<const uint16_t *>(a.b);
  const bool vec = a.vec_ok != 0;

  StageB16<BM, NT, TA, EDGE> sa;  // rows m
  StageB16<BN, NT, !TB, EDGE> sb; // rows n

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t nk = (a.K + BK - 1) / BK;
  if (nk > 0) {
    sa.load(A, a.lda, m0, a.M, 0, a.K, vec, tid);
    sb.load(B, a.ldb, n0, a.N, 0, a.K, vec, tid);
    sa.store(smem, tid);
    sb.store(smem + BM * BK, tid);
  }
  __syncthreads();

  // MFMA operand reads: lane row = lane % 32 within a 32-row fragment,
  // chunk (2 * ks + lane / 32) of the row, swizzled by (row & 7) = lane & 7.
  const int lrow = lane & 31, lhalf = lane >> 5;
  for (uint32_t kt = 0; kt < nk; ++kt) {
    // Prefetch the next K tile (the last tile again on the final trip, so
    // the staging registers are written on every path).
    const uint32_t kn = (kt + 1 < nk ? kt + 1 : kt) * BK;
    sa.load(A, a.lda, m0, a.M, kn, a.K, vec, tid);
    sb.load(B, a.ldb, n0, a.N, kn, a.K, vec, tid);
    const uint16_t *As = smem + (kt & 1) * kBuf;
    const uint16_t *Bs = As + BM * BK;
    const uint4 *As4 = reinterpret_cast<const uint4 *>(As);
    const uint4 *Bs4 = reinterpret_cast<const uint4 *>(Bs);
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      const int chunk = (2 * ks + lhalf) ^ (lane & 7);
      bf16x8_t af[FM], bf[FN];
#pragma unroll
      for (int j = 0; j < FM; ++j) {
        const uint4 v = As4[(wm * TM + j * 32 + lrow) * 8 + chunk];
        af[j] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i) {
        const uint4 v = Bs4[(wn * TN + i * 32 + lrow) * 8 + chunk];
        bf[i] = __builtin_bit_cast(bf16x8_t, v);
      }
#pragma unroll
      for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[i], af[j], acc[i][j], 0, 0, 0);
    }
    uint16_t *nxt = smem + ((kt + 1) & 1) * kBuf;
    sa.store(nxt, tid);
    sb.store(nxt + BM * BK, tid);
    __syncthreads();
  }

  // Epilogue, through LDS: each lane owns output row m and, per q, columns
  // n .. n+3 of the tile; bias + SiLU in fp32, rounded to bf16 and written to
  // an LDS C tile [BM][BN + 8], then stored row-contiguously in 16-byte
  // chunks.  The loop's final barrier has freed both operand buffers.
  const uint16_t *bias = static_cast<const uint16_t *>(a.bias);
  const bool add = (a.epilogue & kEpiAdd) && bias;
  const bool act = (a.epilogue & kEpiSilu) != 0;
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int ml = wm * TM + j * 32 + lrow;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = wn * TN + i * 32 + q * 8 + lhalf * 4;
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = acc[i][j][q * 4 + e];
          if (add) t += bf16_bits_to_f32(bias[min(n0 + nl + e, a.N - 1)]);
          if (act) t = silu(t);
          v[e] = t;
        }
        uint2 o;
        o.x = pack_bf16x2(v[0], v[1]);
        o.y = pack_bf16x2(v[2], v[3]);
        *reinterpret_cast<uint2 *>(smem + ml * kCld + nl) = o;
      }
    }
  }
  __syncthreads();
  uint16_t *C = static_cast<uint16_t *>(a.c);
  constexpr int kRowChunks = BN / 8;
#pragma unroll 4
  for (int it = 0; it < BM * kRowChunks / NT; ++it) {
    const int q = tid + it * NT;
    const int row = q / kRowChunks, c = q % kRowChunks;
    const uint32_t m = m0 + row, n = n0 + c * 8;
    const uint4 v = *reinterpret_cast<const uint4 *>(smem + row * kCld + c * 8);
    if (!EDGE || (m < a.M && n + 8 <= a.N && vec)) {
      *reinterpret_cast<uint4 *>(C + (size_t)m * a.ldc + n) = v;
    } else if (m < a.M) {
      const uint16_t *h = smem + row * kCld + c * 8;
      for (int e = 0; e < 8; ++e)
        if (n + e < a.N) C[(size_t)m * a.ldc + n + e] = h[e];
    }
  }
}

// ------------------------------------------------- bf16, pipelined (full tiles)
//
// Register-free staging: every operand byte goes global -> LDS with
// global_load_lds (16 bytes per lane; the lanes of one instruction fill
// 1 KiB of LDS in lane order, each lane from its own global address), into
// a ring of STAGES stages of BK = 32 (the 8-wave kernels: three, two K
// tiles in flight while the third is multiplied).
//   K-contiguous operand ("KC": A, or B with TB): LDS [rows][32 k],
//     64-byte rows of four 16-byte chunks, chunk c of row r at
//     c ^ ((r >> 2) & 3), so the 16 rows read by 16 lanes of a ds_read_b128
//     hit 16 distinct 16-byte bank groups.
//   MN-contiguous operand ("MNC": row-major B, or A with TA): LDS
//     [32 k][W], 2 W-byte rows, chunk c of row k at c ^ (4 * (k & 3)); the
//     MFMA operand (8 consecutive k of one row/column per lane) is read with
//     two ds_read_b64_tr_b16: in each 16-lane group, lane L fetches 4
//     elements of k-row kb + L/4 at column c0 + 4 * (L % 4), and the
//     hardware returns to lane j the 4 k-values of column c0 + j.
// Needs M a multiple of 256, N of 256 (of 8 for the 384-wide tiles), K of
// 32, and 16-byte aligned rows.

typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt with expcnt / lgkmcnt at their maxima (gfx9 encoding).
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

constexpr int kPipeBK = 32;

__device__ __forceinline__ uint32_t kc_off(uint32_t row, uint32_t c) {
  return row * 64u + 16u * (c ^ ((row >> 2) & 3u));
}
// MN-contiguous tile W elements wide: 2 W-byte k-rows of W / 8 chunks (a
// multiple of 16, so the XOR stays inside the row).
template <int W>
__device__ __forceinline__ uint32_t mnc_off(uint32_t k, uint32_t c) {
  static_assert(W % 128 == 0, "k-rows of a multiple of 16 chunks");
  return k * (2u * W) + 16u * (c ^ (4u * (k & 3u)));
}

// 16 bytes per lane, global -> LDS (M0 holds the wave's LDS destination;
// lane l lands at M0 + 16 * l).  Issued as inline asm so that the
// compiler's conservative LDS-DMA tracking (an s_waitcnt vmcnt(0) before
// every later LDS read) does not flatten the stage ring: completion is
// awaited explicitly with wait_vmcnt() + a barrier before a stage is read.
__device__ __forceinline__ void g2lds16(const void *gptr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(gptr)
               : "memory");
}
// The same from a wave-uniform base (SGPRs) plus a 32-bit byte offset per
// lane: one VGPR per lane instead of a 64-bit address.
__device__ __forceinline__ void g2lds16_so(const void *sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr), "v"(voff), "s"(sbase)
               : "memory");
}

// Source of this lane's 16-byte chunk in 1 KiB block `blk` of an operand
// tile of W rows (KC) or W columns (MNC) whose first K index is 0 (the
// caller adds the K advance).  CLAMP: rows (KC) or columns (MNC) from
// `lim` on re-read the last ones (a tile that overhangs N; those results
// are never stored).
template <bool MNC, int W, bool CLAMP = false>
__device__ __forceinline__ const uint16_t *tile_src(const uint16_t *g, uint32_t ld, uint32_t r0, uint32_t blk,
                                                    int lane, uint32_t lim = 0) {
  const uint32_t q = blk * 64u + (uint32_t)lane;
  if constexpr (!MNC) {
    const uint32_t row = q >> 2, c = (q & 3u) ^ ((row >> 2) & 3u);
    uint32_t r = r0 + row;
    if constexpr (CLAMP) r = min(r, lim - 1u);
    return g + (size_t)r * ld + 8u * c;
  } else {
    constexpr uint32_t kChunks = W / 8;
    const uint32_t k = q / kChunks, c = (q % kChunks) ^ (4u * (k & 3u));
    uint32_t col = r0 + 8u * c;
    if constexpr (CLAMP) col = min(col, lim - 8u);
    return g + (size_t)k * ld + col;
  }
}

// The same chunk as a byte offset from the tile's origin (row or column
// r0 at K = 0), in 32-bit arithmetic: ld * 2 * (rows of a KC tile) must
// stay below 2^32.
template <bool MNC, int W, bool CLAMP = false>
__device__ __forceinline__ uint32_t tile_off(uint32_t ld, uint32_t r0, uint32_t blk, int lane, uint32_t lim = 0) {
  const uint32_t q = blk * 64u + (uint32_t)lane;
  if constexpr (!MNC) {
    const uint32_t row = q >> 2, c = (q & 3u) ^ ((row >> 2) & 3u);
    uint32_t r = row;
    if constexpr (CLAMP) r = min(r, lim - 1u - r0);
    return 2u * (r * ld + 8u * c);
  } else {
    constexpr uint32_t kChunks = W / 8;
    const uint32_t k = q / kChunks, c = (q % kChunks) ^ (4u * (k & 3u));
    uint32_t col = 8u * c;
    if constexpr (CLAMP) col = min(col, lim - 8u - r0);
    return 2u * (k * ld + col);
  }
}

// MFMA operand (8 bf16: rows rb + lane%32, k = 16*ks + 8*(lane/32) .. +7)
// of a tile W rows (KC) or W columns (MNC) wide.
template <bool MNC, int W>
__device__ __forceinline__ bf16x8_t read_operand(const unsigned char *tile, uint32_t rb, int ks, int lane) {
  if constexpr (!MNC) {
    const uint32_t row = rb + (uint32_t)(lane & 31);
    const uint32_t c = (uint32_t)(2 * ks + (lane >> 5));
    return __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(tile + kc_off(row, c)));
  } else {
    const uint32_t g = (uint32_t)((lane >> 4) & 3), L = (uint32_t)(lane & 15);
    const uint32_t col = rb + 16u * (g & 1u) + 4u * (L & 3u);
    const uint32_t c = col >> 3;
    const uint32_t sub = (col & 7u) * 2u;
    const uint32_t k0 = (uint32_t)(16 * ks) + 8u * (g >> 1) + (L >> 2);
    const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4s_t *)(tile + mnc_off<W>(k0, c) + sub));
    const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_v4s_t *)(tile + mnc_off<W>(k0 + 4u, c) + sub));
    typedef short v8s_t __attribute__((ext_vector_type(8)));
    const v8s_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    return __builtin_bit_cast(bf16x8_t, v);
  }
}

template <bool V>
using bool_tag = std::integral_constant<bool, V>;

// 256 x BN output tile (BN 256 or 384), WM x WN waves (4 or 8); each wave
// owns a (256/WM) x (BN/WN) sub-tile.  STAGES K tiles of 32 in the LDS
// ring (STAGES - 1 in flight while one is multiplied).
//
// Schedule of one K tile (two 16-deep MFMA k-steps), per wave:
//   phase A: the k-step-0 MFMAs, interleaved with the LDS reads of k-step 1
//            and the DMA of K tile kt + STAGES - 1 into the stage freed by
//            kt - 1;
//   then:    lgkmcnt(0) (this wave is done reading tile kt), vmcnt down to
//            the tiles younger than kt + 1, barrier (tile kt + 1 is in LDS
//            for every wave, and nobody reads tile kt any more);
//   phase B: the k-step-1 MFMAs, interleaved with the LDS reads of k-step 0
//            of tile kt + 1.
// The MFMA pipe thus always has work queued while LDS reads and DMA issue,
// and there is one barrier per K tile.  sched_barrier(0) pins the order the
// source gives (the DMA is inline asm, which the scheduler cannot classify).
//
// BN = 384 (a 384-wide B tile: a sixth fewer L2 -> LDS bytes per FLOP than
// 256 x 256, and fewer LDS operand bytes per MFMA): the ring's 40 KiB
// stages fit three deep, the epilogue stages C through LDS in two halves
// of 128 rows, and N need only be a multiple of 8 -- a tile column that
// overhangs N re-reads B's last columns (or rows) and stores only n < N.
template <bool TA, bool TB, int WM, int WN, int BN = 256, int STAGES = 4>
__device__ __forceinline__ void gemm_bf16_pipe(const BwppGemmArgs &a) {
  constexpr int BM = 256;
  constexpr int NW = WM * WN, NT = 64 * NW;
  constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
  constexpr int kTileA = BM * kPipeBK * 2, kTileB = BN * kPipeBK * 2;  // bytes per operand tile
  constexpr int LPA = kTileA / 1024 / NW, LPB = kTileB / 1024 / NW;     // 1 KiB DMA blocks per wave
  static_assert(LPA * NW * 1024 == kTileA && LPB * NW * 1024 == kTileB, "DMA blocks split evenly over the waves");
  static_assert(TN % 32 == 0 && TM % 32 == 0 && STAGES >= 2 && STAGES <= 4, "tile shape");
  constexpr bool kEdgeN = BN != 256;
  // Lean register use (the 8-wave 384-wide tile holds 192 accumulator
  // VGPRs): DMA sources as 32-bit offsets from wave-uniform tile origins,
  // and one set of A operands, each re-read for the next k-step as soon as
  // its last MFMA of the current one has issued (MFMAs in A-operand order).
  constexpr bool kLean = BN != 256;
  constexpr int kStage = kTileA + kTileB;
  constexpr int kCld = BN + 8;
  constexpr int kRing = STAGES * kStage;
  constexpr int kHalves = BM * kCld * 2 + BN * 2 > 163840 ? 2 : 1;  // epilogue passes over the rows
  static_assert(kHalves == 1 || WM == kHalves, "one wave row per epilogue half");
  constexpr int kHR = BM / kHalves;  // rows per epilogue half
  constexpr int kEpi = kHR * kCld * 2;
  constexpr int kBiasOff = kRing > kEpi ? kRing : kEpi;  // bias row (bf16) after both
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kBiasOff + BN * 2];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  uint32_t tm, tn;
  tile_coords(a, tm, tn);
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint16_t *A = static_cast<const uint16_t *>(a.a);
  const uint16_t *B = static_cast<const uint16_t *>(a.b);
  const uint32_t nk = a.K / kPipeBK;
  const uint16_t *bias = static_cast<const uint16_t *>(a.bias);
  const bool add = (a.epilogue & kEpiAdd) && bias;
  const bool act = (a.epilogue & kEpiSilu) != 0;

  const uint16_t *bias_s = reinterpret_cast<const uint16_t *>(smem + kBiasOff);

  // Per-lane DMA sources at K = 0, advanced by a fixed step per K tile.
  const uint16_t *srcA[kLean ? 1 : LPA], *srcB[kLean ? 1 : LPB];
  uint32_t offA[kLean ? LPA : 1], offB[kLean ? LPB : 1];  // lean: bytes from baseA / baseB
  const uint16_t *baseA = A + (TA ? (size_t)m0 : (size_t)m0 * a.lda);
  const uint16_t *baseB = B + (TB ? (size_t)n0 * a.ldb : (size_t)n0);
#pragma unroll
  for (int i = 0; i < LPA; ++i) {
    if constexpr (kLean) offA[i] = tile_off<TA, BM>(a.lda, m0, (uint32_t)(wave * LPA + i), lane);
    else srcA[i] = tile_src<TA, BM>(A, a.lda, m0, (uint32_t)(wave * LPA + i), lane);
  }
#pragma unroll
  for (int i = 0; i < LPB; ++i) {
    if constexpr (kLean) offB[i] = tile_off<!TB, BN, kEdgeN>(a.ldb, n0, (uint32_t)(wave * LPB + i), lane, a.N);
    else srcB[i] = tile_src<!TB, BN>(B, a.ldb, n0, (uint32_t)(wave * LPB + i), lane);
  }
  const size_t stepA = TA ? (size_t)kPipeBK * a.lda : (size_t)kPipeBK;
  const size_t stepB = TB ? (size_t)kPipeBK : (size_t)kPipeBK * a.ldb;
  const uint32_t lds_base = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)smem;
  const uint32_t ldsA = lds_base + (uint32_t)(wave * LPA) * 1024u;
  const uint32_t ldsB = lds_base + (uint32_t)kTileA + (uint32_t)(wave * LPB) * 1024u;

  // DMA instruction d (0 .. LPA+LPB-1) of K tile kt.
  auto dma = [&](int d, uint32_t kt) {
    const uint32_t st = (kt % STAGES) * kStage;
    if constexpr (kLean) {
      if (d < LPA)
        g2lds16_so(baseA + kt * stepA, offA[d], ldsA + st + (uint32_t)d * 1024u);
      else
        g2lds16_so(baseB + kt * stepB, offB[d - LPA], ldsB + st + (uint32_t)(d - LPA) * 1024u);
    } else {
      if (d < LPA)
        g2lds16(srcA[d] + kt * stepA, ldsA + st + (uint32_t)d * 1024u);
      else
        g2lds16(srcB[d - LPA] + kt * stepB, ldsB + st + (uint32_t)(d - LPA) * 1024u);
    }
  };

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // fa/fb[0]: operands of k-step 0, [1]: of k-step 1 (lean: one fa set).
  bf16x8_t fa[kLean ? 1 : 2][FM], fb[2][FN];
  constexpr int kReads = FM + FN, kMfma = FM * FN, kDma = LPA + LPB;
  static_assert(kReads <= kMfma && kDma <= kMfma, "interleave needs an MFMA slot per read and DMA");
  // Wait until at most the y youngest K tiles' DMA are still in flight.
  auto wait_younger = [&](uint32_t y) {
    if constexpr (STAGES >= 4) {
      if (y >= 2) {
        wait_vmcnt<2 * kDma>();
        return;
      }
    }
    if (STAGES >= 3 && y >= 1) wait_vmcnt<kDma>();
    else wait_vmcnt<0>();
  };

  auto stage_ptr = [&](uint32_t kt) { return smem + (kt % STAGES) * kStage; };
  auto read = [&](auto buf, int r, const unsigned char *As, int ks) {
    constexpr int b = decltype(buf)::value ? 1 : 0;
    if (r < FM)
      fa[kLean ? 0 : b][r] = read_operand<TA, BM>(As, (uint32_t)(wm * TM + r * 32), ks, lane);
    else
      fb[b][r - FM] = read_operand<!TB, BN>(As + kTileA, (uint32_t)(wn * TN + (r - FM) * 32), ks, lane);
  };
  auto mfma = [&](auto buf, int s) {
    constexpr int b = decltype(buf)::value ? 1 : 0;
    const int i = kLean ? s % FN : s / FM, j = kLean ? s / FN : s % FM;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fb[b][i], fa[kLean ? 0 : b][j], acc[i][j], 0, 0, 0);
  };

  // The tile's BN bias values (16-byte aligned) are copied to LDS by the
  // first lanes of wave 0, ahead of its first K tile, so the prologue wait
  // and barrier publish them and the epilogue never waits on a global load.
  if (add && wave == 0 && lane < BN / 8) {
    uint32_t nb = n0 + 8u * (uint32_t)lane;
    if constexpr (kEdgeN) nb = min(nb, a.N - 8u);
    g2lds16(bias + nb, lds_base + (uint32_t)kBiasOff);
  }
#pragma unroll
  for (int st = 0; st < STAGES - 1; ++st)
    if ((uint32_t)st < nk) {
#pragma unroll
      for (int d = 0; d < kDma; ++d) dma(d, (uint32_t)st);
    }
  wait_younger(nk >= (uint32_t)(STAGES - 1) ? (uint32_t)(STAGES - 2) : (nk > 0 ? nk - 1 : 0u));
  __syncthreads();
  if (nk > 0) {
#pragma unroll
    for (int r = 0; r < kReads; ++r) read(bool_tag<false>{}, r, stage_ptr(0), 0);
  }

  // One K tile; DMA: issue tile kt + STAGES - 1, NEXT: a tile kt + 1 exists.
  auto ktile = [&](uint32_t kt, auto dma_tag, auto next_tag) {
    constexpr bool kDmaOn = decltype(dma_tag)::value, kNext = decltype(next_tag)::value;
    const unsigned char *cur = stage_ptr(kt);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kMfma; ++s) {
      mfma(bool_tag<false>{}, s);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kLean) {
        if (s < FN) {
          read(bool_tag<true>{}, FM + s, cur, 1);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (s % FN == FN - 1) {  // the last MFMA of fa[s / FN] has issued
          read(bool_tag<true>{}, s / FN, cur, 1);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if (s < kReads) {
        read(bool_tag<true>{}, s, cur, 1);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kDmaOn) {
        if (s < kDma) {
          dma(s, kt + STAGES - 1);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    if constexpr (kNext) {
      // Tiles issued after kt + 1 may stay in flight.
      const uint32_t younger = min(nk - 2 - kt, (uint32_t)(STAGES - 2));
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): done reading tile kt
      wait_younger(younger);
      __syncthreads();
    }
    const unsigned char *nxt = stage_ptr(kt + 1);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int s = 0; s < kMfma; ++s) {
      mfma(bool_tag<true>{}, s);
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (kNext && kLean) {
        if (s < FN) {
          read(bool_tag<false>{}, FM + s, nxt, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (s % FN == FN - 1) {
          read(bool_tag<false>{}, s / FN, nxt, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if constexpr (kNext) {
        if (s < kReads) {
          read(bool_tag<false>{}, s, nxt, 0);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
  };

  uint32_t kt = 0;
  for (; kt + STAGES - 1 < nk; ++kt) ktile(kt, bool_tag<true>{}, bool_tag<true>{});
  for (; kt + 1 < nk; ++kt) ktile(kt, bool_tag<false>{}, bool_tag<true>{});
  if (kt < nk) ktile(kt, bool_tag<false>{}, bool_tag<false>{});
  __syncthreads();

  // Epilogue through LDS (see gemm_bf16), in kHalves passes of kHR rows.
  uint16_t *cs = reinterpret_cast<uint16_t *>(smem);
  uint16_t *C = static_cast<uint16_t *>(a.c);
  const int lrow = lane & 31, lhalf = lane >> 5;
  constexpr int kRowChunks = BN / 8;
#pragma unroll
  for (int hv = 0; hv < kHalves; ++hv) {
    if (hv > 0) __syncthreads();  // the previous half has left LDS
    if (kHalves == 1 || wm == hv) {
#pragma unroll
      for (int i = 0; i < FN; ++i) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int nl = wn * TN + i * 32 + q * 8 + lhalf * 4;
          float bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
          if (add) {
            const uint2 raw = *reinterpret_cast<const uint2 *>(bias_s + nl);
            bv[0] = __uint_as_float(raw.x << 16);
            bv[1] = __uint_as_float(raw.x & 0xffff0000u);
            bv[2] = __uint_as_float(raw.y << 16);
            bv[3] = __uint_as_float(raw.y & 0xffff0000u);
          }
#pragma unroll
          for (int j = 0; j < FM; ++j) {
            const int ml = wm * TM - hv * kHR + j * 32 + lrow;
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float t = acc[i][j][q * 4 + e] + bv[e];
              if (act) t = silu(t);
              v[e] = t;
            }
            uint2 o;
            o.x = pack_bf16x2(v[0], v[1]);
            o.y = pack_bf16x2(v[2], v[3]);
            *reinterpret_cast<uint2 *>(cs + ml * kCld + nl) = o;
          }
        }
      }
    }
    __syncthreads();
#pragma unroll 4
    for (int it = 0; it < kHR * kRowChunks / NT; ++it) {
      const int q = tid + it * NT;
      const int row = q / kRowChunks, c = q % kRowChunks;
      if (!kEdgeN || n0 + (uint32_t)c * 8u < a.N)
        *reinterpret_cast<uint4 *>(C + (size_t)(m0 + hv * kHR + row) * a.ldc + n0 + c * 8) =
            *reinterpret_cast<const uint4 *>(cs + row * kCld + c * 8);
    }
  }
}

// ---------------------------------------------------------------- fp32

// LDS tiles hold both operands K-contiguous: [R rows][32 k] fp32, 128-byte
// rows of eight 16-byte chunks, chunk q of row r stored at chunk
// q ^ swz(r), swz(r) = (r & 7) ^ ((r >> 3) & 3).  Eight consecutive rows at
// one chunk (the MFMA operand reads) and rows 4t + c, t = 0..7, at one
// chunk (the transposing stores below) both map to eight distinct chunk
// positions, i.e. distinct bank groups.
__device__ __forceinline__ uint32_t f32_swz(uint32_t r) { return (r & 7u) ^ ((r >> 3) & 3u); }
__device__ __forceinline__ uint32_t f32_off(uint32_t r, uint32_t q) { return r * 32u + ((q ^ f32_swz(r)) << 2); }

// Register staging of one operand tile (R rows x 32 k) for NT threads.
// K-contiguous in memory (KC): thread t copies chunk t % 8 of rows
// t / 8 + (NT / 8) i.  MN-contiguous (the transpose of what LDS holds):
// thread t loads a 4 (k) x 4 (mn) block with four 16-byte loads along mn
// and writes its four columns as 16-byte k-runs (the 4 x 4 transpose is a
// register renaming).
template <int R, int NT, bool KC, bool EDGE>
struct TileF32 {
  static constexpr int kVecs = R * 32 / 4 / NT;
  static_assert(KC ? (NT % 8 == 0 && R % (NT / 8) == 0) : (R % 4 == 0 && NT % (R / 4) == 0), "tile shape");
  float4 v[kVecs];

  // g: operand base, ld its leading dimension; r0 the first tile row (m or
  // n), rows the operand's extent there; k0 the first k, K the k extent.
  __device__ __forceinline__ void load(const float *g, uint32_t ld, uint32_t r0, uint32_t rows, uint32_t k0,
                                       uint32_t K, bool vec, int tid) {
    if constexpr (KC) {
#pragma unroll
      for (int i = 0; i < kVecs; ++i) {
        const uint32_t row = (uint32_t)(tid / 8 + (NT / 8) * i), gk = k0 + 4u * (uint32_t)(tid % 8);
        v[i] = ld4<EDGE>(g, ld, r0 + row, rows, gk, K, vec);
      }
    } else {
      constexpr int kPer = R / 4;  // threads across one k row
      const uint32_t mn = 4u * (uint32_t)(tid % kPer);
#pragma unroll
      for (int b = 0; b < kVecs / 4; ++b) {
        const uint32_t kk = k0 + 4u * (uint32_t)(tid / kPer + (NT / kPer) * b);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[4 * b + e] = ld4<EDGE>(g, ld, kk + e, K, r0 + mn, rows, vec);
      }
    }
  }

  __device__ __forceinline__ void store(float *s, int tid) const {
    if constexpr (KC) {
#pragma unroll
      for (int i = 0; i < kVecs; ++i) {
        const uint32_t row = (uint32_t)(tid / 8 + (NT / 8) * i);
        *reinterpret_cast<float4 *>(s + f32_off(row, (uint32_t)(tid % 8))) = v[i];
      }
    } else {
      constexpr int kPer = R / 4;
      const uint32_t mn = 4u * (uint32_t)(tid % kPer);
#pragma unroll
      for (int b = 0; b < kVecs / 4; ++b) {
        const uint32_t q = (uint32_t)(tid / kPer + (NT / kPer) * b);  // k chunk
        const float4 &x0 = v[4 * b], &x1 = v[4 * b + 1], &x2 = v[4 * b + 2], &x3 = v[4 * b + 3];
        *reinterpret_cast<float4 *>(s + f32_off(mn + 0, q)) = make_float4(x0.x, x1.x, x2.x, x3.x);
        *reinterpret_cast<float4 *>(s + f32_off(mn + 1, q)) = make_float4(x0.y, x1.y, x2.y, x3.y);
        *reinterpret_cast<float4 *>(s + f32_off(mn + 2, q)) = make_float4(x0.z, x1.z, x2.z, x3.z);
        *reinterpret_cast<float4 *>(s + f32_off(mn + 3, q)) = make_float4(x0.w, x1.w, x2.w, x3.w);
      }
    }
  }

  // 16 bytes at (row, col..col+3) of a [rows x cols] matrix with leading
  // dimension ld; zeros outside (EDGE), element-wise when not 16-byte rows.
  template <bool E>
  __device__ __forceinline__ static float4 ld4(const float *g, uint32_t ld, uint32_t row, uint32_t nrows,
                                               uint32_t col, uint32_t ncols, bool vec) {
    const float *p = g + (size_t)row * ld + col;
    if (!E) return *reinterpret_cast<const float4 *>(p);
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (row < nrows) {
      if (vec && col + 4 <= ncols) {
        x = *reinterpret_cast<const float4 *>(p);
      } else {
        if (col + 0 < ncols) x.x = p[0];
        if (col + 1 < ncols) x.y = p[1];
        if (col + 2 < ncols) x.z = p[2];
        if (col + 3 < ncols) x.w = p[3];
      }
    }
    return x;
  }
};

#ifndef BWPP_F32_STORE_AFTER
#define BWPP_F32_STORE_AFTER 0
#endif

template <bool TA, bool TB, bool EDGE, bool SPLIT = false>
__device__ __forceinline__ void gemm_f32(const BwppGemmArgs &a) {
  constexpr int BM = 128, BN = 128, BK = 32, WM = 2, WN = 2;
  constexpr int NT = 64 * WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 32, FN = TN / 32;
  using SA = TileF32<BM, NT, !TA, EDGE>;  // A K-contiguous unless transposed
  using SB = TileF32<BN, NT, TB, EDGE>;   // B K-contiguous only when transposed
  constexpr int kTileA = BM * BK, kTileB = BN * BK;
  constexpr int kBuf = kTileA + kTileB;
  constexpr int kCld = BN + 4;  // epilogue C tile [BM][BN + 4], reusing the operand buffers
  constexpr int kSmem = 2 * kBuf > BM * kCld ? 2 * kBuf : BM * kCld;
  __shared__ __attribute__((aligned(16))) float smemf[kSmem];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;
  uint32_t tm, tn;
  const float *A = static_cast<const float *>(a.a);
  const float *B = static_cast<const float *>(a.b);
  uint32_t Klen = a.K, split = 0;
  if constexpr (SPLIT) {
    const uint32_t T = a.tiles_m * a.tiles_n;
    split = blockIdx.x / T;
    tile_coords(a, tm, tn, blockIdx.x - split * T);
    const uint32_t kb = split * a.kchunk;
    Klen = min(a.kchunk, a.K - kb);
    A += TA ? (size_t)kb * a.lda : kb;
    B += TB ? kb : (size_t)kb * a.ldb;
  } else {
    tile_coords(a, tm, tn);
  }
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const bool vec = a.vec_ok != 0;
  SA sa;
  SB sb;

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const uint32_t nk = (Klen + BK - 1) / BK;
  if (nk > 0) {
    sa.load(A, a.lda, m0, a.M, 0, Klen, vec, tid);
    sb.load(B, a.ldb, n0, a.N, 0, Klen, vec, tid);
    sa.store(smemf, tid);
    sb.store(smemf + kTileA, tid);
  }
  __syncthreads();

  // Operand reads: lane l takes row l % 32 of its 32-row block and, for the
  // 8-k chunk j, the 16-byte k-run 8j + 4 (l / 32) .. +3; MFMA step s of
  // the chunk pairs k = 8j + s (lanes 0-31) with 8j + 4 + s (lanes 32-63).
  const uint32_t lrow = (uint32_t)(lane & 31), lhi = (uint32_t)(lane >> 5);
  constexpr uint32_t kStoreAfter = BWPP_F32_STORE_AFTER;
  for (uint32_t kt = 0; kt < nk; ++kt) {
    const uint32_t kn = (kt + 1 < nk ? kt + 1 : kt) * BK;
    sa.load(A, a.lda, m0, a.M, kn, Klen, vec, tid);
    sb.load(B, a.ldb, n0, a.N, kn, Klen, vec, tid);
    // Keep the next tile's loads here, ahead of the MFMAs: left alone, the
    // scheduler sinks them to the LDS stores at the end of the iteration
    // and the full memory latency is exposed once per K tile.
    __builtin_amdgcn_sched_barrier(0);
    const float *As = smemf + (kt & 1) * kBuf;
    const float *Bs = As + kTileA;
    // Operands of chunk j + 1 are read while chunk j's MFMAs issue.
    float4 af[2][FM], bf[2][FN];
    auto read_chunk = [&](uint32_t j, float4(&ar)[FM], float4(&br)[FN]) {
#pragma unroll
      for (int f = 0; f < FM; ++f)
        ar[f] = *reinterpret_cast<const float4 *>(As + f32_off((uint32_t)(wm * TM + f * 32) + lrow, 2 * j + lhi));
#pragma unroll
      for (int f = 0; f < FN; ++f)
        br[f] = *reinterpret_cast<const float4 *>(Bs + f32_off((uint32_t)(wn * TN + f * 32) + lrow, 2 * j + lhi));
    };
    read_chunk(0, af[0], bf[0]);
#pragma unroll
    for (uint32_t j = 0; j < BK / 8; ++j) {
      if (j + 1 < BK / 8) read_chunk(j + 1, af[(j + 1) & 1], bf[(j + 1) & 1]);
      const float4(&ac)[FM] = af[j & 1];
      const float4(&bc)[FN] = bf[j & 1];
#pragma unroll
      for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
          for (int jj = 0; jj < FM; ++jj) {
            const float x = st == 0 ? bc[i].x : st == 1 ? bc[i].y : st == 2 ? bc[i].z : bc[i].w;
            const float y = st == 0 ? ac[jj].x : st == 1 ? ac[jj].y : st == 2 ? ac[jj].z : ac[jj].w;
            acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[i][jj], 0, 0, 0);
          }
      if (j == kStoreAfter) {
        // The next tile goes into the other buffer part way through the
        // MFMAs (nobody reads that buffer during this tile), so the wait for
        // its loads and the LDS writes overlap the remaining MFMAs.
        __builtin_amdgcn_sched_barrier(0);
        float *nxt = smemf + ((kt + 1) & 1) * kBuf;
        sa.store(nxt, tid);
        sb.store(nxt + kTileA, tid);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __syncthreads();
  }

  // Epilogue through LDS as in the bf16 kernel: C tile [BM][BN + 4] fp32.
  // Split-K blocks store raw sums; the reduce kernel applies the epilogue.
  const float *bias = static_cast<const float *>(a.bias);
  const bool add = !SPLIT && (a.epilogue & kEpiAdd) && bias;
  const bool act = !SPLIT && (a.epilogue & kEpiSilu) != 0;
  const int lhalf = lane >> 5;
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int ml = wm * TM + j * 32 + lrow;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = wn * TN + i * 32 + q * 8 + lhalf * 4;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = acc[i][j][q * 4 + e];
          if (add) t += bias[min(n0 + nl + e, a.N - 1)];
          if (act) t = silu(t);
          vv[e] = t;
        }
        *reinterpret_cast<float4 *>(smemf + ml * kCld + nl) = make_float4(vv[0], vv[1], vv[2], vv[3]);
      }
    }
  }
  __syncthreads();
  float *C = SPLIT ? a.part + (size_t)split * a.M * a.N : static_cast<float *>(a.c);
  const uint32_t ldc = SPLIT ? a.N : a.ldc;
  const uint32_t fuse = SPLIT ? 0u : a.fuse;  // split-K: the reduce kernel fuses
  constexpr int kRowVecs = BN / 4;
#pragma unroll 4
  for (int it = 0; it < BM * kRowVecs / NT; ++it) {
    const int q = tid + it * NT;
    const int row = q / kRowVecs, c = q % kRowVecs;
    const uint32_t m = m0 + row, n = n0 + c * 4;
    float4 v = *reinterpret_cast<const float4 *>(smemf + row * kCld + c * 4);
    if (!EDGE || (m < a.M && n + 4 <= a.N && vec)) {
      if (fuse_reads_aux(fuse)) v = fuse4(fuse, v, *reinterpret_cast<const float4 *>(a.aux + (size_t)m * a.ldaux + n));
      *reinterpret_cast<float4 *>(C + (size_t)m * ldc + n) = v;
      if (fuse == kFuseDualSilu)
        *reinterpret_cast<float4 *>(a.c2 + (size_t)m * a.ldc2 + n) =
            make_float4(silu(v.x), silu(v.y), silu(v.z), silu(v.w));
    } else if (m < a.M) {
      const float *h = smemf + row * kCld + c * 4;
      for (int e = 0; e < 4; ++e)
        if (n + e < a.N) {
          float y = h[e];
          if (fuse_reads_aux(fuse)) y = fuse1(fuse, y, a.aux[(size_t)m * a.ldaux + n + e]);
          C[(size_t)m * ldc + n + e] = y;
          if (fuse == kFuseDualSilu) a.c2[(size_t)m * a.ldc2 + n + e] = silu(y);
        }
    }
  }
}

// ------------------------------------------------------- fp32, DMA ring
//
// Full tiles (M, N multiples of 128, K of 32, 16-byte rows): 128 x 128
// blocks of 4 waves in 2 x 2 (64 x 64 each), K in 32-deep tiles through an
// S-stage LDS ring filled by global_load_lds_dwordx4, one barrier per tile.
// S = 2 runs two blocks per CU (two waves per SIMD); S = 4 one block with
// three tiles in flight ahead of the MFMAs.  Operand tiles keep their memory
// orientation in LDS, so the DMA copies rows as they are:
//   K-contiguous (A, or B with TB): [128 rows][32 k], 128-byte rows of
//     eight 16-byte chunks, logical chunk q of row r at q ^ (r & 7) ^
//     ((r >> 3) & 1); the MFMA reads (lane l: row l % 32, chunk 2j + l / 32
//     of the 8-k chunk j) then hit distinct bank groups in every 16-lane
//     pass of a ds_read_b128 (16 rows over 64 banks: r and r + 8 differ);
//   MN-contiguous (B, or A with TA): [32 k][128], 16-byte column chunk c of
//     k row k at c ^ (8 ((k >> 2) & 1)): lanes 32-63 read k + 4, which
//     would otherwise sit on the banks of lanes 0-31.
// MFMA step s of 8-k chunk j pairs k = 8j + s (lanes 0-31) with 8j + 4 + s
// (lanes 32-63), as in the register-staged kernel above.
// Schedule of tile kt, per wave: chunks 0-2 each after the reads of the
// next chunk; then wait for tile kt + 1's DMA, barrier (every wave has read
// tile kt), and chunk 3's MFMAs with the refill of tile kt's stage (tile
// kt + S) and the reads of chunk 0 of tile kt + 1 issued between them.  The
// last S tiles run a drain loop without refills.
constexpr int kF32Tile = 128 * 32 * 4;  // bytes of one operand tile
constexpr int kF32Stage = 2 * kF32Tile;
constexpr int kF32Cld = 128 + 4;        // epilogue C tile [128][132] fp32 in the ring

__device__ __forceinline__ uint32_t f32_mnc_pos(uint32_t k, uint32_t c) { return c ^ (((k >> 2) & 1u) << 3); }
__device__ __forceinline__ uint32_t f32_kc_swz(uint32_t row) { return (row & 7u) ^ ((row >> 3) & 1u); }

// Global source of lane `lane`'s 16 bytes in 1-KiB DMA block `blk` of an
// operand tile whose first k is 0 (the caller adds the k advance).
template <bool KC>
__device__ __forceinline__ const float *f32_dma_src(const float *g, uint32_t ld, uint32_t r0, uint32_t blk,
                                                    int lane) {
  if constexpr (KC) {
    const uint32_t row = blk * 8u + (uint32_t)lane / 8u, pc = (uint32_t)lane & 7u;
    return g + (size_t)(r0 + row) * ld + 4u * (pc ^ f32_kc_swz(row));
  } else {
    const uint32_t k = blk * 2u + (uint32_t)lane / 32u, pc = (uint32_t)lane & 31u;
    return g + (size_t)k * ld + r0 + 4u * f32_mnc_pos(k, pc);
  }
}

// The lane's operand values for the four MFMA steps of 8-k chunk j of the
// 32-row (or 32-column) block starting at rb.
template <bool KC>
__device__ __forceinline__ float4 f32_operand(const unsigned char *tile, uint32_t rb, uint32_t j, int lane) {
  const uint32_t l = (uint32_t)lane & 31u, h = (uint32_t)lane >> 5;
  if constexpr (KC) {
    const uint32_t row = rb + l, q = 2u * j + h;
    return *reinterpret_cast<const float4 *>(tile + row * 128u + 16u * (q ^ f32_kc_swz(row)));
  } else {
    const uint32_t k = 8u * j + 4u * h, col = rb + l;
    const float *t = reinterpret_cast<const float *>(tile) + k * 128u + 4u * f32_mnc_pos(k, col >> 2) + (col & 3u);
    return make_float4(t[0], t[128], t[256], t[384]);
  }
}

template <bool TA, bool TB, bool SPLIT, int S>
__device__ __forceinline__ void gemm_f32_pipe(const BwppGemmArgs &a) {
  constexpr int BM = 128, BN = 128, BK = 32, WN = 2, NT = 256;
  constexpr int TM = 64, TN = 64, FM = TM / 32, FN = TN / 32;
  constexpr int LPW = 16 / 4;         // 1 KiB DMA blocks per wave per operand tile
  constexpr int kDma = 2 * LPW;       // DMA instructions per wave per K tile
  constexpr int kSmem = S * kF32Stage > BM * kF32Cld * 4 ? S * kF32Stage : BM * kF32Cld * 4;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kSmem];
  float *smemf = reinterpret_cast<float *>(smem);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  uint32_t tm, tn;
  const float *A = static_cast<const float *>(a.a);
  const float *B = static_cast<const float *>(a.b);
  uint32_t Klen = a.K, split = 0;
  if constexpr (SPLIT) {
    const uint32_t T = a.tiles_m * a.tiles_n;
    split = blockIdx.x / T;
    tile_coords(a, tm, tn, blockIdx.x - split * T);
    const uint32_t kb = split * a.kchunk;
    Klen = min(a.kchunk, a.K - kb);
    A += TA ? (size_t)kb * a.lda : kb;
    B += TB ? kb : (size_t)kb * a.ldb;
  } else {
    tile_coords(a, tm, tn);
  }
  const uint32_t m0 = tm * BM, n0 = tn * BN;
  const uint32_t nk = Klen / BK;

  // Per-lane DMA sources at k = 0 and their advance per K tile.
  const float *srcA[LPW], *srcB[LPW];
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    srcA[i] = f32_dma_src<!TA>(A, a.lda, m0, (uint32_t)(wave * LPW + i), lane);
    srcB[i] = f32_dma_src<TB>(B, a.ldb, n0, (uint32_t)(wave * LPW + i), lane);
  }
  const size_t stepA = TA ? (size_t)BK * a.lda : (size_t)BK;
  const size_t stepB = TB ? (size_t)BK : (size_t)BK * a.ldb;
  const uint32_t lds0 =
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)smem + (uint32_t)(wave * LPW) * 1024u;
  auto dma_one = [&](uint32_t kt, int d) {  // DMA instruction d (A blocks, then B) of tile kt
    const uint32_t st = lds0 + (kt % S) * kF32Stage;
    if (d < LPW) g2lds16(srcA[d] + kt * stepA, st + (uint32_t)d * 1024u);
    else g2lds16(srcB[d - LPW] + kt * stepB, st + kF32Tile + (uint32_t)(d - LPW) * 1024u);
  };
  auto dma_tile = [&](uint32_t kt) {
#pragma unroll
    for (int d = 0; d < kDma; ++d) dma_one(kt, d);
  };
  auto stage_ptr = [&](uint32_t kt) {
    return smem + __builtin_amdgcn_readfirstlane((kt % S) * kF32Stage);
  };

  f32x16_t acc[FN][FM];
#pragma unroll
  for (int i = 0; i < FN; ++i)
#pragma unroll
    for (int j = 0; j < FM; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  float4 af[2][FM], bf[2][FN];
  auto read_chunk = [&](const unsigned char *st, uint32_t j, float4(&ar)[FM], float4(&br)[FN]) {
#pragma unroll
    for (int f = 0; f < FM; ++f) ar[f] = f32_operand<!TA>(st, (uint32_t)(wm * TM + f * 32), j, lane);
#pragma unroll
    for (int f = 0; f < FN; ++f) br[f] = f32_operand<TB>(st + kF32Tile, (uint32_t)(wn * TN + f * 32), j, lane);
  };
  // MFMA idx of a chunk: step idx / (FN FM), accumulator (idx / FM) % FN, idx % FM.
  auto mfma_one = [&](const float4(&ac)[FM], const float4(&bc)[FN], int idx) {
    const int st = idx / (FN * FM), i = (idx / FM) % FN, jj = idx % FM;
    const float x = st == 0 ? bc[i].x : st == 1 ? bc[i].y : st == 2 ? bc[i].z : bc[i].w;
    const float y = st == 0 ? ac[jj].x : st == 1 ? ac[jj].y : st == 2 ? ac[jj].z : ac[jj].w;
    acc[i][jj] = __builtin_amdgcn_mfma_f32_32x32x2f32(x, y, acc[i][jj], 0, 0, 0);
  };
  auto mfma_chunk = [&](const float4(&ac)[FM], const float4(&bc)[FN]) {
#pragma unroll
    for (int idx = 0; idx < 4 * FN * FM; ++idx) mfma_one(ac, bc, idx);
  };
  // Operand f (A fragments, then B) of chunk j into af/bf[b].
  auto read_op = [&](const unsigned char *st, uint32_t j, int f, int b) {
    if (f < FM) af[b][f] = f32_operand<!TA>(st, (uint32_t)(wm * TM + f * 32), j, lane);
    else bf[b][f - FM] = f32_operand<TB>(st + kF32Tile, (uint32_t)(wn * TN + (f - FM) * 32), j, lane);
  };
  auto read_one = [&](const unsigned char *st, int f) { read_op(st, 0, f, 0); };
  // Chunk 3 of a tile after the barrier, with tile kt + S's refill DMAs and
  // the reads of chunk 0 of tile kt + 1 issued between its MFMAs, so the
  // matrix pipe restarts right after the barrier.
  auto tail_chunk = [&](uint32_t kt) {
    const unsigned char *nxt = stage_ptr(kt + 1);
#pragma unroll
    for (int idx = 0; idx < 4 * FN * FM; ++idx) {
      __builtin_amdgcn_sched_barrier(0);
      mfma_one(af[1], bf[1], idx);
      __builtin_amdgcn_sched_barrier(0);
      if (idx < kDma) dma_one(kt + S, idx);
      if (idx >= kDma && idx < kDma + FM + FN) read_one(nxt, idx - kDma);
    }
  };

  // Prologue: the first min(S, nk) tiles in flight, wait for tile 0.
#pragma unroll
  for (int st = 0; st < S; ++st)
    if ((uint32_t)st < nk) dma_tile((uint32_t)st);
  if constexpr (S >= 4) {
    if (nk >= 4) wait_vmcnt<3 * kDma>();
    else if (nk == 3) wait_vmcnt<2 * kDma>();
    else if (nk == 2) wait_vmcnt<kDma>();
    else wait_vmcnt<0>();
  } else {
    if (nk >= 2) wait_vmcnt<kDma>();
    else wait_vmcnt<0>();
  }
  __syncthreads();
  if (nk > 0) read_chunk(stage_ptr(0), 0, af[0], bf[0]);

  // Chunks 0-2, the reads of chunk j + 1 issued one per MFMA slot among
  // chunk j's MFMAs (a burst of reads from four waves in step queues at the
  // LDS and holds up the in-order MFMA issue behind it).
  auto head_chunks = [&](uint32_t kt) {
    const unsigned char *cur = stage_ptr(kt);
#pragma unroll
    for (uint32_t j = 0; j < 3; ++j) {
#pragma unroll
      for (int idx = 0; idx < 4 * FN * FM; ++idx) {
        __builtin_amdgcn_sched_barrier(0);
        mfma_one(af[j & 1], bf[j & 1], idx);
        __builtin_amdgcn_sched_barrier(0);
        if (idx < FM + FN) read_op(cur, j + 1, idx, (int)((j + 1) & 1));
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // Steady state: tile kt + S exists, so every tile refills its stage and
  // tiles kt + 2 .. kt + S - 1 stay in flight across the barrier.
  uint32_t kt = 0;
  for (; kt + S < nk; ++kt) {
    head_chunks(kt);
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): done reading tile kt
    wait_vmcnt<(S - 2) * kDma>();
    __syncthreads();
    tail_chunk(kt);
  }
  // Drain: the last (up to) S tiles, no refills.
  for (; kt < nk; ++kt) {
    head_chunks(kt);
    if (kt + 1 < nk) {
      __builtin_amdgcn_s_waitcnt(0xc07f);
      const uint32_t younger = nk - 2 - kt;  // tiles still in flight behind kt + 1
      if (S >= 4 && younger >= 2) wait_vmcnt<2 * kDma>();
      else if (S >= 3 && younger == 1) wait_vmcnt<kDma>();
      else wait_vmcnt<0>();
      __syncthreads();
      read_chunk(stage_ptr(kt + 1), 0, af[0], bf[0]);
      __builtin_amdgcn_sched_barrier(0);
    }
    mfma_chunk(af[1], bf[1]);
  }
  __syncthreads();  // the epilogue reuses the ring

  // Epilogue through LDS (split-K blocks store raw sums; the reduce kernel
  // applies the epilogue and the fused tail).
  const float *bias = static_cast<const float *>(a.bias);
  const bool add = !SPLIT && (a.epilogue & kEpiAdd) && bias;
  const bool act = !SPLIT && (a.epilogue & kEpiSilu) != 0;
  const int lrow = lane & 31, lhalf = lane >> 5;
#pragma unroll
  for (int i = 0; i < FN; ++i) {
#pragma unroll
    for (int j = 0; j < FM; ++j) {
      const int ml = wm * TM + j * 32 + lrow;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int nl = wn * TN + i * 32 + q * 8 + lhalf * 4;
        float vv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float t = acc[i][j][q * 4 + e];
          if (add) t += bias[n0 + nl + e];
          if (act) t = silu(t);
          vv[e] = t;
        }
        *reinterpret_cast<float4 *>(smemf + ml * kF32Cld + nl) = make_float4(vv[0], vv[1], vv[2], vv[3]);
      }
    }
  }
  __syncthreads();
  float *C = SPLIT ? a.part + (size_t)split * a.M * a.N : static_cast<float *>(a.c);
  const uint32_t ldc = SPLIT ? a.N : a.ldc;
  const uint32_t fuse = SPLIT ? 0u : a.fuse;
  constexpr int kRowVecs = BN / 4;
#pragma unroll 4
  for (int it = 0; it < BM * kRowVecs / NT; ++it) {
    const int q = tid + it * NT;
    const int row = q / kRowVecs, c = q % kRowVecs;
    const uint32_t m = m0 + row, n = n0 + c * 4;
    float4 v = *reinterpret_cast<const float4 *>(smemf + row * kF32Cld + c * 4);
    if (fuse_reads_aux(fuse)) v = fuse4(fuse, v, *reinterpret_cast<const float4 *>(a.aux + (size_t)m * a.ldaux + n));
    *reinterpret_cast<float4 *>(C + (size_t)m * ldc + n) = v;
    if (fuse == kFuseDualSilu)
      *reinterpret_cast<float4 *>(a.c2 + (size_t)m * a.ldc2 + n) =
          make_float4(silu(v.x), silu(v.y), silu(v.z), silu(v.w));
  }
}

}  // namespace

// Split-K reduction: C[m][n..n+3] = epilogue(sum_s part[s][m][n..n+3]) in
// split order, then bias and SiLU as the single-pass epilogue, then the
// fused tail.  Needs N a multiple of 4 and 16-byte aligned C (and aux, c2)
// rows (the full-tile conditions).
extern "C" __global__ __launch_bounds__(256) void bwpp_gemm_f32_splitk_reduce(const BwppGemmArgs a) {
  const uint32_t nv = a.N / 4;
  const size_t total = (size_t)a.M * nv, plane = (size_t)a.M * a.N;
  const float *bias = static_cast<const float *>(a.bias);
  const bool add = (a.epilogue & kEpiAdd) && bias;
  const bool act = (a.epilogue & kEpiSilu) != 0;
  float *C = static_cast<float *>(a.c);
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
    const uint32_t m = (uint32_t)(i / nv), n = (uint32_t)(i % nv) * 4;
    const float *p = a.part + (size_t)m * a.N + n;
    float4 t = *reinterpret_cast<const float4 *>(p);
    for (uint32_t s = 1; s < a.ksplit; ++s) {
      const float4 u = *reinterpret_cast<const float4 *>(p + s * plane);
      t.x += u.x;
      t.y += u.y;
      t.z += u.z;
      t.w += u.w;
    }
    if (add) {
      t.x += bias[n];
      t.y += bias[n + 1];
      t.z += bias[n + 2];
      t.w += bias[n + 3];
    }
    if (act) {
      t.x = silu(t.x);
      t.y = silu(t.y);
      t.z = silu(t.z);
      t.w = silu(t.w);
    }
    if (fuse_reads_aux(a.fuse)) t = fuse4(a.fuse, t, *reinterpret_cast<const float4 *>(a.aux + (size_t)m * a.ldaux + n));
    *reinterpret_cast<float4 *>(C + (size_t)m * a.ldc + n) = t;
    if (a.fuse == kFuseDualSilu)
      *reinterpret_cast<float4 *>(a.c2 + (size_t)m * a.ldc2 + n) = make_float4(silu(t.x), silu(t.y), silu(t.z), silu(t.w));
  }
}

// Entry points: bwpp_gemm_<bf16|f32>_t<TA><TB>_<f|e|s>  (f: no edges,
// aligned; s: f with split-K partials)
#define BWPP_GEMM_BF16(TA, TB, EDGE, SUF)                                                  \
  extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(256, 256),            \
                                       amdgpu_waves_per_eu(1, 1))) void                  \
      bwpp_gemm_bf16_t##TA##TB##_##SUF(const BwppGemmArgs a) {                            \
    if constexpr (EDGE)                                                                   \
      gemm_bf16<TA, TB, true>(a);                                                         \
    else                                                                                  \
      gemm_bf16_pipe<TA, TB, 2, 2>(a);                                                    \
  }
// 8-wave (2 per SIMD) variant of the pipelined full-tile kernel, with a
// three-stage ring: 1-1.5 % faster than four stages on C3 (same bits; one
// tile fewer in flight), two stages 20 % slower.
#define BWPP_GEMM_BF16_W8(TA, TB)                                                          \
  extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(512, 512),            \
                                       amdgpu_waves_per_eu(2, 2))) void                  \
      bwpp_gemm_bf16w8_t##TA##TB##_f(const BwppGemmArgs a) {                              \
    gemm_bf16_pipe<TA, TB, 2, 4, 256, 3>(a);                                              \
  }
// 256 x 384 tiles: 8 waves of 128 x 96 (two per SIMD), three-stage ring.
// Row-major A only: with a transposed A the compiler spills (40 / 311
// VGPRs for t10 / t11), so those stay on the 256 x 256 kernels.
#define BWPP_GEMM_BF16_X384(TA, TB)                                                        \
  extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(512, 512),            \
                                       amdgpu_waves_per_eu(2, 2))) void                  \
      bwpp_gemm_bf16x384w8_t##TA##TB##_f(const BwppGemmArgs a) {                          \
    gemm_bf16_pipe<TA, TB, 2, 4, 384, 3>(a);                                              \
  }
#define BWPP_GEMM_F32(TA, TB, EDGE, SUF)                                                   \
  extern "C" __global__ __launch_bounds__(256) void bwpp_gemm_f32_t##TA##TB##_##SUF(     \
      const BwppGemmArgs a) {                                                             \
    gemm_f32<TA, TB, EDGE>(a);                                                            \
  }
#define BWPP_GEMM_ALL(MAC) \
  MAC(0, 0, false, f)      \
  MAC(0, 1, false, f)      \
  MAC(1, 0, false, f)      \
  MAC(1, 1, false, f)      \
  MAC(0, 0, true, e)       \
  MAC(0, 1, true, e)       \
  MAC(1, 0, true, e)       \
  MAC(1, 1, true, e)

BWPP_GEMM_ALL(BWPP_GEMM_BF16)
BWPP_GEMM_BF16_W8(0, 0)
BWPP_GEMM_BF16_W8(0, 1)
BWPP_GEMM_BF16_W8(1, 0)
BWPP_GEMM_BF16_W8(1, 1)
BWPP_GEMM_BF16_X384(0, 0)
BWPP_GEMM_BF16_X384(0, 1)
BWPP_GEMM_ALL(BWPP_GEMM_F32)
#define BWPP_GEMM_F32_SPLIT(TA, TB)                                                        \
  extern "C" __global__ __launch_bounds__(256) void bwpp_gemm_f32_t##TA##TB##_s(         \
      const BwppGemmArgs a) {                                                             \
    gemm_f32<TA, TB, false, true>(a);                                                     \
  }
BWPP_GEMM_F32_SPLIT(0, 0)
BWPP_GEMM_F32_SPLIT(0, 1)
BWPP_GEMM_F32_SPLIT(1, 0)
BWPP_GEMM_F32_SPLIT(1, 1)
// DMA-ring full-tile kernels: bwpp_gemm_f32p_t<TA><TB>_<f|s> (two blocks
// per CU, 2-stage ring) and bwpp_gemm_f32q_t<TA><TB>_<f|s> (one block per
// CU, 4-stage ring).
#define BWPP_GEMM_F32_PIPE(TA, TB)                                                         \
  extern "C" __global__ __launch_bounds__(256, 2) void bwpp_gemm_f32p_t##TA##TB##_f(     \
      const BwppGemmArgs a) {                                                             \
    gemm_f32_pipe<TA, TB, false, 2>(a);                                                   \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(256, 2) void bwpp_gemm_f32p_t##TA##TB##_s(     \
      const BwppGemmArgs a) {                                                             \
    gemm_f32_pipe<TA, TB, true, 2>(a);                                                    \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(256) void bwpp_gemm_f32q_t##TA##TB##_f(        \
      const BwppGemmArgs a) {                                                             \
    gemm_f32_pipe<TA, TB, false, 4>(a);                                                   \
  }                                                                                       \
  extern "C" __global__ __launch_bounds__(256) void bwpp_gemm_f32q_t##TA##TB##_s(        \
      const BwppGemmArgs a) {                                                             \
    gemm_f32_pipe<TA, TB, true, 4>(a);                                                    \
  }
BWPP_GEMM_F32_PIPE(0, 0)
BWPP_GEMM_F32_PIPE(0, 1)
BWPP_GEMM_F32_PIPE(1, 0)
BWPP_GEMM_F32_PIPE(1, 1)
