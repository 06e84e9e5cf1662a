// Attention backward on the bf16 matrix cores of gfx950
// (v_mfma_f32_32x32x16_bf16): bf16 Q, K, V, O, dO and dQ, dK, dV; fp32
// lse, D_m, softmax and accumulation; head dims K = D in {64, 128}.
//   p = exp(scale q.k - lse),  D_m = rowsum(dO * O)[m],
//   dS = p (dO.v - D_m),  dQ = scale dS K,  dK = scale dS^T Q,  dV = P^T dO,
// with P and dS rounded to bf16 where they enter an MFMA as an operand.
// Semantics: the closed form of the graph's softmax_grad chain
// (compiler/graph_ir.c:1722-1733) applied to the attention of
// runtime/cpu/bwpp_cpu_ref.c:92-144, generalised with a score scale and a
// bottom-right aligned causal mask (key n visible to query m iff
// n <= m + N - M).
//
// Work layout as in the fp32 kernels, with 4 waves per block: each wave
// owns 32 rows (queries in the dQ pass, keys in the dK/dV pass) and the
// block streams 64-row tiles of the other side through a two-stage LDS
// ring (tile t+1 goes straight from global memory into LDS with
// global_load_lds while tile t is used, one barrier per tile) and works
// through each tile in 32-row blocks.
//
// Two schemes.  Recompute: the dQ pass (which also writes D_m) forms S, dP
// and dS itself, then the dK/dV pass forms them again (7 products for the
// 5 the FLOP count has).  Stored dS (d = 128; the runtime's default when
// the workspace allows): a D_m pass, the dK/dV pass storing the dS it forms
// (DsBlk layout), and a dQ pass that only multiplies it by K.  Both visit
// the same 32 x 32 blocks with the same operands: the same results.
//
// MFMA operands (32x32x16 bf16): lane l supplies A[l % 32][8 (l / 32) ..
// +7] and B[8 (l / 32) .. +7][l % 32]; accumulator register r of lane l is
// C[8 (r / 4) + 4 (l / 32) + r % 4][l % 32].
//  - Products over the head dim (S, dP) take the streamed tile's rows as A
//    (one 16-byte LDS read per lane per k-step) and the wave's own rows as
//    B, held in registers (query or key l % 32, d = 16 ks + 8 (l / 32)).
//    The accumulator then gives lane l one row of the wave (l % 32) and 16
//    rows of the tile: row-wise softmax terms are lane-local.
//  - Products over the tile's rows (dQ, dK, dV) are computed transposed,
//    X^T W: W (the probabilities or dS) goes from the accumulator straight
//    into the B operand, lane half h taking tile rows 4h..4h+3 and
//    8+4h..8+4h+3 of each 16, and X^T is read from the row-major tile with
//    ds_read_b64_tr_b16 at exactly those rows.
// LDS tiles are [rows][D] bf16 with 16-byte chunk c of row r stored at
// chunk c ^ swz(r); swz is a permutation on any 16 consecutive rows (the
// row reads) and keeps the two chunks of the four rows that a 16-lane
// group of a transposing read touches apart.
#include "common.h"
#include "../kargs.h"

using namespace bwpp;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef short v8s_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

namespace {

constexpr int kR = 32;  // rows per wave and per block of a streamed tile
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f32x16_t mfma16(bf16x8_t a, bf16x8_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ float sum32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// Tile row of accumulator register r for lane half hi.
__device__ __forceinline__ int acc_row(int r, int hi) { return 8 * (r >> 2) + 4 * hi + (r & 3); }

// Two readers share every tile: 16-byte row reads (16 consecutive rows at
// one logical chunk per 16-lane quarter) and the transposing reads (32 lanes
// of 8 bytes: four consecutive rows x logical chunks q..q+3 of one
// 64-byte quartet, q a multiple of 4).  With 64 four-byte banks both are
// conflict-free when swz is a permutation on any 16 consecutive rows (row
// reads) and, for D = 128, the four rows of a transposing read land in four
// different quartets (bits 2-3 of swz take r & 3); for D = 64 (two rows per
// 256 bank bytes) rows of equal parity do (bit 2 takes (r >> 1) & 1).
template <int D>
__device__ __forceinline__ uint32_t swz(uint32_t r) {
  if constexpr (D == 128)
    return ((r & 3u) << 2) | ((r >> 2) & 3u);  // 16 chunks per 256-byte row
  else
    return (((r >> 1) & 1u) << 2) | (((r >> 2) & 1u) << 1) | ((r >> 3) & 1u);  // 8 chunks per 128-byte row
}
template <int D>
__device__ __forceinline__ uint32_t toff(uint32_t r, uint32_t c) {
  return r * (uint32_t)(D * 2) + 16u * (c ^ swz<D>(r));
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  // s_waitcnt with expcnt / lgkmcnt at their maxima (gfx9 encoding).
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane, global -> LDS (M0 holds the wave's LDS destination;
// lane l lands at M0 + 16 l).  Inline asm, so that the compiler does not
// put an s_waitcnt vmcnt(0) before every later LDS read; completion is
// awaited with wait_vmcnt<0>() and a barrier before the stage is read.
// M0 is written only here in these kernels.
__device__ __forceinline__ void g2lds16(const void *gptr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(gptr) : "memory");
}


// Two [TR x D] bf16 tiles (rows r0..; a row past `rows` re-reads row
// rows - 1, which the callers mask) loaded straight into an LDS stage in
// 1 KiB blocks: lane l of block b fills physical chunk l % (D / 8) of tile
// row b (1024 / 2D) + l / (D / 8), i.e. logical chunk pc ^ swz(row).
template <int D, int W, int TR>
struct TileDmaB {
  static constexpr int CH = D / 8;               // 16-byte chunks per row
  static constexpr int RPB = 64 / CH;            // rows per 1 KiB block
  static constexpr int BPW = TR * D * 2 / 1024 / W;  // blocks per wave per tile
  static_assert(BPW >= 1 && BPW * W * 1024 == TR * D * 2, "tile must split into whole blocks per wave");
  uint32_t row[BPW], col[BPW];
  __device__ __forceinline__ TileDmaB(int wave, int lane) {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const uint32_t r = (uint32_t)((wave * BPW + i) * RPB + lane / CH), pc = (uint32_t)(lane % CH);
      row[i] = r;
      col[i] = 8u * (pc ^ swz<D>(r));
    }
  }
  // lx, ly: LDS byte addresses of the two destination tiles; wv: the wave
  // index (uniform).
  // One tile only.
  __device__ __forceinline__ void issue1(const uint16_t *X, uint32_t ldx, uint32_t r0, uint32_t rows, uint32_t lx,
                                         uint32_t wv) const {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const uint32_t r = r0 + row[i], rr = r < rows ? r : rows - 1;
      g2lds16(X + (size_t)rr * ldx + col[i], lx + (wv * BPW + (uint32_t)i) * 1024u);
    }
  }
  __device__ __forceinline__ void issue(const uint16_t *X, uint32_t ldx, const uint16_t *Y, uint32_t ldy,
                                        uint32_t r0, uint32_t rows, uint32_t lx, uint32_t ly, uint32_t wv) const {
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
      const uint32_t r = r0 + row[i], rr = r < rows ? r : rows - 1;
      const uint32_t dst = (wv * BPW + (uint32_t)i) * 1024u;
      g2lds16(X + (size_t)rr * ldx + col[i], lx + dst);
      g2lds16(Y + (size_t)rr * ldy + col[i], ly + dst);
    }
  }
};

// The lane's 16-byte pieces of a row: d = 16 ks + 8 hi .. +7, ks < D / 16
// (zeros past the end; a row past the end loads row rows - 1, when there
// is one, and discards it).
template <int D>
__device__ __forceinline__ void load_row(bf16x8_t (&dst)[D / 16], const uint16_t *X, uint32_t ld, uint32_t row,
                                         uint32_t rows, int hi) {
  const uint32_t rr = row < rows ? row : (rows > 0 ? rows - 1 : 0);
  const bool in = row < rows;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
    if (rows > 0) v = *reinterpret_cast<const u32x4_t *>(X + (size_t)rr * ld + 16 * ks + 8 * hi);
    if (!in) v = u32x4_t{0u, 0u, 0u, 0u};
    dst[ks] = __builtin_bit_cast(bf16x8_t, v);
  }
}

// load_row for rows > 0 without the zeroing of rows past the end, and that
// zeroing as a separate step, so that a caller can issue several loads
// before the first wait (the select needs the loaded data).
template <int D>
__device__ __forceinline__ void load_row_raw(bf16x8_t (&dst)[D / 16], const uint16_t *X, uint32_t ld, uint32_t row,
                                             uint32_t rows, int hi) {
  const uint32_t rr = row < rows ? row : rows - 1;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    dst[ks] = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const u32x4_t *>(X + (size_t)rr * ld + 16 * ks + 8 * hi));
}
template <int D>
__device__ __forceinline__ void zero_past(bf16x8_t (&x)[D / 16], uint32_t row, uint32_t rows) {
  if (row >= rows) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) x[ks] = __builtin_bit_cast(bf16x8_t, u32x4_t{0u, 0u, 0u, 0u});
  }
}

// Per-lane LDS offsets: row reads (tile row li, k-step ks) and the two
// transposing reads (tile rows 0-7 / 8-15 of a 16-row step) of d block blk.
// Only the k-step 0 / d block 0 offsets are kept: the others differ in the
// chunk bits that ks (2 ks) and blk (4 blk) occupy, which the swizzle XORs
// and never carries into, so they are one XOR away.
template <int D>
struct Offsets {
  uint32_t row0, tlo0, thi0;
  __device__ __forceinline__ Offsets(int lane) {
    const uint32_t li = (uint32_t)(lane & 31), hi = (uint32_t)(lane >> 5);
    row0 = toff<D>(li, hi);
    const uint32_t grp = (uint32_t)((lane >> 4) & 3), L = (uint32_t)(lane & 15);
    const uint32_t rb = 4u * (grp >> 1) + (L >> 2);
    const uint32_t col = 16u * (grp & 1u) + 4u * (L & 3u);
    tlo0 = toff<D>(rb, col >> 3) + (col & 7u) * 2u;
    thi0 = toff<D>(rb + 8u, col >> 3) + (col & 7u) * 2u;
  }
  // A copy the compiler cannot hoist out of a loop over `salt` (an empty
  // asm that depends on it): the XORs then stay in the loop body instead of
  // occupying 16 registers across it.
  __device__ __forceinline__ Offsets fresh(uint32_t salt) const {
    Offsets o = *this;
    asm("" : "+v"(o.row0), "+v"(o.tlo0), "+v"(o.thi0) : "s"(salt));
    return o;
  }
  __device__ __forceinline__ uint32_t row(int ks) const { return row0 ^ (32u * (uint32_t)ks); }
  __device__ __forceinline__ uint32_t tlo(int blk) const { return tlo0 ^ (64u * (uint32_t)blk); }
  __device__ __forceinline__ uint32_t thi(int blk) const { return thi0 ^ (64u * (uint32_t)blk); }
};

// A operand X^T (d block blk, tile rows 16 kq .. +15 in the accumulator's
// row order) from a row-major LDS tile.  16 rows keep swz (it depends on
// the row's low four bits only).
template <int D>
__device__ __forceinline__ bf16x8_t tr_operand(const unsigned char *tile, const Offsets<D> &o, int blk, int kq) {
  const uint32_t step = (uint32_t)kq * 16u * (uint32_t)(D * 2);
  const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(tile + o.tlo(blk) + step));
  const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(tile + o.thi(blk) + step));
  const v8s_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(bf16x8_t, v);
}

// B operand from accumulator registers 8 kq .. 8 kq + 7 (rounded to bf16).
__device__ __forceinline__ bf16x8_t acc_operand(const f32x16_t &w, int kq) {
  const int r0 = 8 * kq;
  uint4 u;
  u.x = pack_bf16x2(w[r0 + 0], w[r0 + 1]);
  u.y = pack_bf16x2(w[r0 + 2], w[r0 + 3]);
  u.z = pack_bf16x2(w[r0 + 4], w[r0 + 5]);
  u.w = pack_bf16x2(w[r0 + 6], w[r0 + 7]);
  return __builtin_bit_cast(bf16x8_t, u);
}

// acc = X_tile(rows) . W^T over the head dim: X_tile rows from LDS, W the
// lane's register pieces.
template <int D>
__device__ __forceinline__ f32x16_t dot_rows(const unsigned char *tile, const Offsets<D> &o,
                                             const bf16x8_t (&w)[D / 16]) {
  f32x16_t acc = {};
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    acc = mfma16(__builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(tile + o.row(ks))), w[ks], acc);
  return acc;
}

// The same product with W's rows also in LDS (rows li, same swizzle), read
// at the same offsets as the tile's.
template <int D>
__device__ __forceinline__ f32x16_t dot_rows_lds(const unsigned char *tile, const Offsets<D> &o,
                                                 const unsigned char *wrows) {
  f32x16_t acc = {};
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
    acc = mfma16(__builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(tile + o.row(ks))),
                 __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(wrows + o.row(ks))), acc);
  return acc;
}

// Stores a wave's transposed accumulator set (lane li's register r of
// acc[blk] = element d = 32 blk + acc_row(r, hi) of row row0 + li) as bf16,
// times f, for the rows below `rows`.  The pieces go through the wave's own
// 32 x 2D-byte LDS region `stage` (16-byte chunk c of row j at chunk
// c ^ (j mod D/8): both the 8-byte writes and the 16-byte row reads are
// bank-conflict-free) and leave as whole rows, 1 KiB of consecutive rows
// per store instruction.  Stored straight from the accumulators, each
// instruction wrote 16 bytes into each of 32 rows, and at C4 the dK / dV
// pass's blocks spent 4.1 of their 144 us issuing them.  A wave's LDS
// operations run in order, so the row reads see the writes without a wait
// and the next call may reuse the region.  The stores are non-temporal:
// with plain stores the outputs sat dirty in the caches and were written
// back while the next pass streamed dS (the dQ pass 473 -> 414 us at C4).
template <int D>
__device__ __forceinline__ void store_rows(uint16_t *X, uint32_t ld, uint32_t row0, uint32_t rows,
                                           const f32x16_t (&acc)[D / 32], float f, int lane, unsigned char *stage) {
  constexpr int CH = D / 8, RB = 2 * D, RPI = 64 / CH;  // chunks per row, row bytes, rows per store
  const int li = lane & 31, hi = lane >> 5;
#pragma unroll
  for (int blk = 0; blk < D / 32; ++blk)
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
      const int c = 4 * blk + r4;
      uint2 u;
      u.x = pack_bf16x2(acc[blk][4 * r4] * f, acc[blk][4 * r4 + 1] * f);
      u.y = pack_bf16x2(acc[blk][4 * r4 + 2] * f, acc[blk][4 * r4 + 3] * f);
      *reinterpret_cast<uint2 *>(stage + li * RB + 16 * (c ^ (li & (CH - 1))) + 8 * hi) = u;
    }
  const int ch = lane % CH;
  // All row reads first: the empty asm that takes them all keeps each read
  // out of its store's branch, where it would wait for its own round trip.
  u32x4_t u[32 / RPI];
#pragma unroll
  for (int j = 0; j < 32 / RPI; ++j) {
    const int r = j * RPI + lane / CH;
    u[j] = *reinterpret_cast<const u32x4_t *>(stage + r * RB + 16 * (ch ^ (r & (CH - 1))));
  }
  static_assert(32 / RPI == 8 || 32 / RPI == 4, "4 or 8 row reads");
  if constexpr (32 / RPI == 8)
    asm volatile("" : "+v"(u[0]), "+v"(u[1]), "+v"(u[2]), "+v"(u[3]), "+v"(u[4]), "+v"(u[5]), "+v"(u[6]), "+v"(u[7]));
  else
    asm volatile("" : "+v"(u[0]), "+v"(u[1]), "+v"(u[2]), "+v"(u[3]));
#pragma unroll
  for (int j = 0; j < 32 / RPI; ++j) {
    const int r = j * RPI + lane / CH;
    if (row0 + (uint32_t)r < rows)
      __builtin_nontemporal_store(u[j], reinterpret_cast<u32x4_t *>(X + (size_t)(row0 + (uint32_t)r) * ld + 8 * ch));
  }
}

// The (batch, head) slice and the tile rank (0 .. a.q_tiles - 1, 0 the
// heaviest when causal) of this block.
//  - Unmasked: blocks are dispatched round-robin over the 8 XCDs; the
//    renumbering gives each XCD a contiguous run of slices with all of
//    their tiles, so the blocks that stream one slice's K / V (or Q / dO)
//    tiles run together and share one L2.  Numbered slice-fastest, the
//    blocks of a slice landed on one XCD but in different generations (the
//    ~512 resident blocks spanned every slice, each re-reading its slice's
//    tiles from HBM): C4's backward 2.10 -> 1.90 ms, bit-identical.
//  - Causal: tile rank first, so the heaviest tiles go first and the
//    light ones fill the end of the grid (the XCD order above lost 6 % at
//    C4 and 28 % at B2 H16 S4096 to the imbalance it leaves there).  With
//    slices a multiple of 64, each XCD works through chunks of 8 of its
//    slices, rank-major inside a chunk: the resident blocks of an XCD then
//    share 8 slices' tiles instead of 32 (C4 causal 1.18 -> 1.13 ms,
//    bit-identical); otherwise slice-fastest over the whole grid.
template <bool CAUSAL>
struct SliceB {
  uint32_t bh, b, h, tile;
  __device__ __forceinline__ explicit SliceB(const BwppAttnArgs &a) {
    const uint32_t G = gridDim.x, T = a.q_tiles;
    constexpr uint32_t kChunk = 8;  // slices per XCD per chunk
    if (CAUSAL) {
      const uint32_t nbh = G / T;
      if (nbh % (8u * kChunk) == 0) {
        const uint32_t x = blockIdx.x % 8u, i = blockIdx.x / 8u;
        bh = ((i / (kChunk * T)) * kChunk + i % kChunk) * 8u + x;
        tile = (i % (kChunk * T)) / kChunk;
      } else {
        bh = blockIdx.x % nbh;
        tile = blockIdx.x / nbh;
      }
    } else {
      const uint32_t lb = G % 8u == 0 ? (blockIdx.x % 8u) * (G / 8u) + blockIdx.x / 8u : blockIdx.x;
      bh = lb / T;
      tile = lb % T;
    }
    b = bh / a.heads;
    h = bh % a.heads;
  }
};

// D_m = rowsum(dO * O) of query row qi (gf: the lane's half of dO's row):
// lane halves 0 / 1 sum d = 16 ks + 8 hi .. +7 in order, then add.  The dQ
// pass and the D_m pass both use it, so both give the same bits.
template <int D>
__device__ __forceinline__ float row_dsum(const bf16x8_t (&gf)[D / 16], const uint16_t *O, uint32_t ldo,
                                          uint32_t qi, uint32_t M, int hi) {
  bf16x8_t of[D / 16];
  load_row<D>(of, O, ldo, qi, M, hi);
  float part = 0.0f;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) part += (float)gf[ks][e] * (float)of[ks][e];
  return sum32(part);
}

// D_m pass of the stored-dS scheme (which has no dQ pass before the dK / dV
// pass): a wave per 32 query rows, kW waves per block, q_tiles blocks per
// slice.  The block's dO and O rows come into LDS with the coalesced DMA
// (1 KiB per instruction; loading them per lane, 32 bytes of 32 rows per
// instruction, ran at 4.5 TB/s) and each lane sums its half rows from
// there in row_dsum's order, so D_m has the same bits as the dQ pass's.
template <int D, int kW>
__device__ __forceinline__ void bwd_dsum(const BwppAttnArgs &a) {
  constexpr int RB = D * 2, TB = kW * kR * RB;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][TB];  // [dO, O] rows of the block
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int hi = lane >> 5;
  const uint32_t bh = blockIdx.x / a.q_tiles, tile = blockIdx.x % a.q_tiles;
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const uint16_t *O = static_cast<const uint16_t *>(a.o) + b * a.o_bs + h * a.o_hs;
  const uint16_t *dO = static_cast<const uint16_t *>(a.dout) + b * a.o_bs + h * a.o_hs;
  const uint32_t r0 = tile * (kW * kR), qi = r0 + (uint32_t)wave * kR + (uint32_t)(lane & 31);
  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)&lds[0][0];
  const TileDmaB<D, kW, kW * kR> dma(wave, lane);
  dma.issue(dO, a.ldo, O, a.ldo, r0, a.M, lds0, lds0 + (uint32_t)TB, wv);  // rows past M re-read row M - 1
  wait_vmcnt<0>();
  __syncthreads();
  const Offsets<D> off(lane);
  const unsigned char *gt = lds[0] + wave * kR * RB, *ot = lds[1] + wave * kR * RB;
  float part = 0.0f;
#pragma unroll
  for (int ks = 0; ks < D / 16; ++ks) {
    const bf16x8_t g = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(gt + off.row(ks)));
    const bf16x8_t o = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(ot + off.row(ks)));
#pragma unroll
    for (int e = 0; e < 8; ++e) part += (float)g[e] * (float)o[e];
  }
  const float dsum = sum32(part);
  if (qi < a.M && hi == 0) a.dsum[(size_t)bh * a.M + qi] = dsum;
}

// dQ pass: a wave owns 32 queries and streams K / V tiles; also writes
// D_m = rowsum(dO * O) for the dK / dV pass.
template <int D, bool CAUSAL, int kW, int TR>
__device__ __forceinline__ void bwd_dq(const BwppAttnArgs &a) {
  constexpr int DB = D / 32, TB = TR * D * 2, RB = D * 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][2][TB];  // [stage][K, V]
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const SliceB<CAUSAL> sl(a);
  const uint32_t qt = a.q_tiles - 1 - sl.tile;  // heaviest (causal) first
  const uint16_t *Q = static_cast<const uint16_t *>(a.q) + sl.b * a.q_bs + sl.h * a.q_hs;
  const uint16_t *K = static_cast<const uint16_t *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  const uint16_t *V = static_cast<const uint16_t *>(a.v) + sl.b * a.v_bs + sl.h * a.v_hs;
  const uint16_t *O = static_cast<const uint16_t *>(a.o) + sl.b * a.o_bs + sl.h * a.o_hs;
  const uint16_t *dO = static_cast<const uint16_t *>(a.dout) + sl.b * a.o_bs + sl.h * a.o_hs;
  uint16_t *dQ = static_cast<uint16_t *>(a.dq) + sl.b * a.q_bs + sl.h * a.q_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const uint32_t qb = qt * (kW * kR), q0 = qb + (uint32_t)wave * kR, qi = q0 + (uint32_t)li;

  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last = (int64_t)min(a.M, qb + kW * kR) - 1 + diag;
    kend = last < 0 ? 0u : (uint32_t)min<int64_t>(last + 1, (int64_t)a.N);
  }
  const uint32_t nt = (kend + TR - 1) / TR;
  const int64_t wlast = (int64_t)q0 + kR - 1 + diag;

  bf16x8_t qf[D / 16], gf[D / 16];
  load_row<D>(qf, Q, a.ldq, qi, a.M, hi);
  load_row<D>(gf, dO, a.ldo, qi, a.M, hi);
  const float dsum = row_dsum<D>(gf, O, a.ldo, qi, a.M, hi);
  if (qi < a.M && hi == 0) a.dsum[(size_t)sl.bh * a.M + qi] = dsum;
  // Queries past M: +inf makes every probability exp2(-inf) = 0.
  const float lse2 = qi < a.M ? a.lse[(size_t)sl.bh * a.M + qi] * kLog2e : INFINITY;
  const float c = a.scale_log2;
  // Here the 16 per-lane offsets stay in registers (hoisted): this pass
  // has room below 256 VGPRs, and recomputing them was 1.5 % slower.
  const Offsets<D> off(lane);

  f32x16_t dq[DB];
#pragma unroll
  for (int blk = 0; blk < DB; ++blk) dq[blk] = f32x16_t{};

  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)&lds[0][0][0];
  const TileDmaB<D, kW, TR> dma(wave, lane);
  auto issue = [&](uint32_t t) {  // K / V tile t into stage t % 2
    const uint32_t sb = lds0 + (t & 1u) * (uint32_t)(2 * TB);
    dma.issue(K, a.ldk, V, a.ldv, t * TR, a.N, sb, sb + (uint32_t)TB, wv);
  };
  if (nt > 0) {
    issue(0);
    wait_vmcnt<0>();
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    const int st = (int)(t & 1);
    if (t + 1 < nt) issue(t + 1);
    // The tile in 32-key blocks (the swizzle repeats every 16 rows).
#pragma unroll
    for (int sb = 0; sb < TR / kR; ++sb) {
      const uint32_t k0 = t * TR + sb * kR;
      const unsigned char *Kt = lds[st][0] + sb * kR * RB, *Vt = lds[st][1] + sb * kR * RB;
      if ((TR == kR || k0 < kend) && (!CAUSAL || (int64_t)k0 <= wlast)) {
        f32x16_t s = dot_rows<D>(Kt, off, qf);         // S^T [key][query]
        const f32x16_t dp = dot_rows<D>(Vt, off, gf);  // dP^T = V dO^T
        const bool edge = k0 + kR > a.N || (CAUSAL && (int64_t)k0 + kR - 1 > (int64_t)q0 + diag);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(s[r] * c - lse2);
          s[r] = p * (dp[r] - dsum);  // dS^T
        }
        // Keys past N or above the diagonal: p = 0.  One block-uniform
        // branch around all 16 (per element the optimiser turned each test
        // into a compare and two selects on every tile, a third of the
        // tile's VALU work).
        if (edge) {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const uint32_t key = k0 + (uint32_t)acc_row(r, hi);
            if (key >= a.N || (CAUSAL && (int64_t)key > (int64_t)qi + diag)) s[r] = 0.0f * (dp[r] - dsum);
          }
        }
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
          const bf16x8_t w = acc_operand(s, kq);
#pragma unroll
          for (int blk = 0; blk < DB; ++blk) dq[blk] = mfma16(tr_operand<D>(Kt, off, blk, kq), w, dq[blk]);
        }
      }
    }
    wait_vmcnt<0>();  // tile t + 1 is in LDS (this wave's part; the barrier does the rest)
    __syncthreads();
  }
  // The ring is free: every wave has passed the last tile's barrier.
  static_assert(4 * TB >= kW * kR * RB, "one 32-row staging region per wave fits the ring");
  store_rows<D>(dQ, a.ldq, qb + wv * (uint32_t)kR, a.M, dq, a.scale, (int)__lane_id(),
                &lds[0][0][0] + wv * (uint32_t)(kR * RB));
}

// Stored dS^T layout: per slice, 2 KiB blocks of 32 keys x 32 queries,
// [key block][query block] (query blocks padded to ld_dst / 32, a multiple
// of 4): the dQ pass's blocks of one slice, which step through the key
// blocks together, read neighbouring 8 KiB pieces of one key block's row
// (4-7 % faster than giving each block a contiguous stream of its own).
// Inside a block the 8-byte piece holding queries 4 qd .. +3 of key k sits
// at
//   512 (qd / 2) + 16 (k ^ 4 (qd / 2)) + 8 (qd % 2),
// so a wave of the dK / dV pass (lane = key, holding quads 2 x + hi of one
// quad pair x per store) writes 512 contiguous bytes per store, the dQ
// pass's DMA copies whole blocks, and its transposing reads (four keys x
// eight quads per 32 lanes) hit 64 distinct banks: the XOR moves the four
// quad pairs, which are 512 bytes apart, onto different 16-byte slots.
struct DsBlk {
  static constexpr uint32_t kBytes = 2048;
  // Byte offset of block (key block kb, query block qb) of slice bh; n32
  // key blocks, m32 query blocks per slice.
  __device__ __forceinline__ static size_t at(uint32_t bh, uint32_t kb, uint32_t qb, uint32_t n32, uint32_t m32) {
    return (((size_t)bh * n32 + kb) * m32 + qb) * kBytes;
  }
  // Offset of key k's piece of quad hi (quad pair 0).
  __device__ __forceinline__ static uint32_t piece(uint32_t k, uint32_t hi) { return 16u * k + 8u * hi; }
  // The same piece in quad pair x: key bits 2-3 are offset bits 6-7.
  __device__ __forceinline__ static uint32_t pair(uint32_t off, uint32_t x) { return 512u * x + (off ^ (64u * x)); }
};

// dQ pass of the stored-dS scheme: dQ = scale dS K with dS^T read from
// a.dst (written by the dK / dV pass) instead of recomputed from S and dP.
// A wave owns 32 queries (one query block); the block streams TR-key tiles
// of K and the matching dS^T blocks through the two-stage ring.  The pass
// is bound by reading dS^T (a copy without its MFMAs takes as long); more
// stages (32-key tiles in 3-5, or a third dS^T stage) or staging dS^T
// through registers were slower.
// The same 32 x 32 blocks as in bwd_dq are visited (the dK / dV pass
// stores exactly those), and each MFMA gets the same operands in the same
// slots, so dQ is bit-identical to bwd_dq's but for the sign of all-zero
// sums.
template <bool CAUSAL, int TR>
__device__ __forceinline__ void bwd_dq_ds(const BwppAttnArgs &a) {
  constexpr int D = 128, DB = D / 32, kW = 4, TB = TR * D * 2, RB = D * 2;
  constexpr int KB = TR / kR;                                           // key blocks per tile
  constexpr uint32_t SB = (uint32_t)(KB * kW) * DsBlk::kBytes;          // dS^T bytes per tile
  static_assert(SB == (uint32_t)TB, "a dS^T tile (TR keys x 128 queries) is as large as a K tile");
  constexpr int SPW = (int)(SB / 1024u) / kW;                           // 1 KiB DMA pieces per wave
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][2][TB];  // [stage][K, dS^T]
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const SliceB<CAUSAL> sl(a);
  const uint32_t qt = a.q_tiles - 1 - sl.tile;  // heaviest (causal) first
  const uint32_t qb = qt * (kW * kR), q0 = qb + (uint32_t)wave * kR, qi = q0 + (uint32_t)li;
  const uint32_t n32 = (a.N + 31u) / 32u, m32 = a.ld_dst / 32u;
  const uint16_t *K = static_cast<const uint16_t *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  // The block's 4 query blocks (8 KiB, contiguous) of key block 0.
  const unsigned char *S = static_cast<const unsigned char *>(a.dst) + DsBlk::at(sl.bh, 0, qb / 32u, n32, m32);
  uint16_t *dQ = static_cast<uint16_t *>(a.dq) + sl.b * a.q_bs + sl.h * a.q_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;

  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last = (int64_t)min(a.M, qb + kW * kR) - 1 + diag;
    kend = last < 0 ? 0u : (uint32_t)min<int64_t>(last + 1, (int64_t)a.N);
  }
  const uint32_t nt = (kend + TR - 1) / TR;
  const int64_t wlast = (int64_t)q0 + kR - 1 + diag;
  const Offsets<D> off(lane);
  // Transposing reads of a dS^T block: 16-lane group g reads keys
  // 4 (g / 2) + L / 4 (+ 8 for the high half) x quad 4 (g % 2) + L % 4, as
  // tr_operand does on a row-major tile.
  uint32_t slo, shi;
  {
    const uint32_t grp = (uint32_t)((lane >> 4) & 3), L = (uint32_t)(lane & 15);
    const uint32_t rb = 4u * (grp >> 1) + (L >> 2), qd = 4u * (grp & 1u) + (L & 3u);
    slo = DsBlk::pair(DsBlk::piece(rb, qd & 1u), qd >> 1);
    shi = DsBlk::pair(DsBlk::piece(rb + 8u, qd & 1u), qd >> 1);
  }
  f32x16_t dq[DB];
#pragma unroll
  for (int blk = 0; blk < DB; ++blk) dq[blk] = f32x16_t{};

  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)&lds[0][0][0];
  const TileDmaB<D, kW, TR> dma(wave, lane);
  auto issue = [&](uint32_t t) {  // K tile t / its dS^T blocks into stage t % 2
    const uint32_t sb = lds0 + (t & 1u) * (uint32_t)(2 * TB);
    dma.issue1(K, a.ldk, t * TR, a.N, sb, wv);
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      const uint32_t j = wv * (uint32_t)SPW + (uint32_t)i;  // 1 KiB piece of the tile
      const uint32_t kb = min(t * (uint32_t)KB + j / 8u, n32 - 1u);  // past N: re-read the last block (masked)
      g2lds16(S + (size_t)kb * m32 * DsBlk::kBytes + (j % 8u) * 1024u + 16u * (uint32_t)lane,
              sb + (uint32_t)TB + j * 1024u);
    }
  };
  if (nt > 0) {
    issue(0);
    wait_vmcnt<0>();
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    if (t + 1 < nt) issue(t + 1);
    const uint32_t st = t & 1u;
#pragma unroll
    for (int sb = 0; sb < KB; ++sb) {
      const uint32_t k0 = t * TR + sb * kR;
      const unsigned char *Kt = lds[st][0] + sb * kR * RB;
      const unsigned char *Sb = lds[st][1] + (sb * kW + wave) * DsBlk::kBytes;
      if ((TR == kR || k0 < kend) && (!CAUSAL || (int64_t)k0 <= wlast)) {
        // Keys past N (their rows re-read row N - 1): dS = 0.
        const bool edge = k0 + kR > a.N;
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
          const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Sb + slo + 256u * kq));
          const v4s_t hv = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Sb + shi + 256u * kq));
          v8s_t x = {lo[0], lo[1], lo[2], lo[3], hv[0], hv[1], hv[2], hv[3]};
          if (edge) {
#pragma unroll
            for (int j = 0; j < 8; ++j)
              if (k0 + 16u * kq + (uint32_t)acc_row(j, hi) >= a.N) x[j] = 0;
          }
          const bf16x8_t w = __builtin_bit_cast(bf16x8_t, x);
#pragma unroll
          for (int blk = 0; blk < DB; ++blk) dq[blk] = mfma16(tr_operand<D>(Kt, off, blk, kq), w, dq[blk]);
        }
      }
    }
    wait_vmcnt<0>();  // tile t + 1 is in LDS (this wave's part; the barrier does the rest)
    __syncthreads();
  }
  // The ring is free: every wave has passed the last tile's barrier.
  static_assert(4 * TB >= kW * kR * RB, "one 32-row staging region per wave fits the ring");
  store_rows<D>(dQ, a.ldq, qb + wv * (uint32_t)kR, a.M, dq, a.scale, (int)__lane_id(),
                &lds[0][0][0] + wv * (uint32_t)(kR * RB));
}

// dK / dV pass: a wave owns 32 keys and streams Q / dO tiles with their
// lse and D_m.  WS: also stores dS^T (bf16, as it enters the dK product) to
// a.dst for bwd_dq_ds.
template <int D, bool CAUSAL, int kW, int TR, bool VL = false, bool WS = false>
__device__ __forceinline__ void bwd_dkdv(const BwppAttnArgs &a) {
  constexpr int DB = D / 32, TB = TR * D * 2, RB = D * 2;
  __shared__ __attribute__((aligned(16))) unsigned char lds[2][2][TB];  // [stage][Q, dO]
  __shared__ __attribute__((aligned(16))) float rowv[2][2][TR];          // [stage][lse2, D_m]
  // VL: each wave's V rows in LDS instead of 32 registers per lane.
  __shared__ __attribute__((aligned(16))) unsigned char vrows[VL ? kW : 1][VL ? kR * RB : 16];
  const int lane = (int)threadIdx.x & 63, wave = (int)threadIdx.x >> 6;
  const int li = lane & 31, hi = lane >> 5;
  const SliceB<CAUSAL> sl(a);  // q_tiles holds the key tiles here
  const uint32_t kt = sl.tile;   // heaviest (causal) first
  const uint16_t *Q = static_cast<const uint16_t *>(a.q) + sl.b * a.q_bs + sl.h * a.q_hs;
  const uint16_t *K = static_cast<const uint16_t *>(a.k) + sl.b * a.k_bs + sl.h * a.k_hs;
  const uint16_t *V = static_cast<const uint16_t *>(a.v) + sl.b * a.v_bs + sl.h * a.v_hs;
  const uint16_t *dO = static_cast<const uint16_t *>(a.dout) + sl.b * a.o_bs + sl.h * a.o_hs;
  uint16_t *dK = static_cast<uint16_t *>(a.dk) + sl.b * a.k_bs + sl.h * a.k_hs;
  uint16_t *dV = static_cast<uint16_t *>(a.dv) + sl.b * a.v_bs + sl.h * a.v_hs;
  const float *lse = a.lse + (size_t)sl.bh * a.M;
  const float *dsum = a.dsum + (size_t)sl.bh * a.M;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const uint32_t kb = kt * (kW * kR), k0w = kb + (uint32_t)wave * kR, ni = k0w + (uint32_t)li;

  // Queries that see a key n: m >= n - diag (causal).
  uint32_t mbeg = 0;
  if (CAUSAL) {
    const int64_t first = (int64_t)kb - diag;
    mbeg = first <= 0 ? 0u : (first >= (int64_t)a.M ? a.M : (uint32_t)first);
    mbeg -= mbeg % TR;
  }
  const uint32_t nt = a.M > mbeg ? (a.M - mbeg + TR - 1) / TR : 0u;
  const int64_t wfirst = (int64_t)k0w - diag;  // first query that sees any key of the wave

  // The wave's dS^T blocks (DsBlk): key block k0w / 32 of the slice, query
  // block m0 / 32; dso: this lane's piece offset for query quads 0 / 1
  // (quad pair x: + 512 x, key bits 2-3 ^ x).
  unsigned char *dsblk = nullptr;
  uint32_t dso = 0, n32 = 0, m32 = 0;
  if constexpr (WS) {
    dsblk = static_cast<unsigned char *>(a.dst);
    n32 = (a.N + 31u) / 32u;
    m32 = a.ld_dst / 32u;
    dso = DsBlk::piece(li, hi);
  }
  const uint32_t wv = (uint32_t)__builtin_amdgcn_readfirstlane(wave);
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)&lds[0][0][0];
  const TileDmaB<D, kW, TR> dma(wave, lane);
  auto issue = [&](uint32_t t) {  // Q / dO tile t into stage t % 2
    const uint32_t sb = lds0 + (t & 1u) * (uint32_t)(2 * TB);
    dma.issue(Q, a.ldq, dO, a.ldo, mbeg + t * TR, a.M, sb, sb + (uint32_t)TB, wv);
  };
  float rl = INFINITY, rd = 0.0f;  // lse2 / D_m of row threadIdx.x (< TR)
  // The loads are issued with the tile's and used only when the tile is
  // stashed: the compiler's wait for them (which also waits for the LDS
  // DMA issued before them) then falls where the DMA is awaited anyway.
  auto fetch_rows = [&](uint32_t m0) {
    if (threadIdx.x < (uint32_t)TR) {
      const uint32_t m = min(m0 + threadIdx.x, a.M - 1);
      rl = lse[m];
      rd = dsum[m];
    }
  };
  auto stash_rows = [&](int st, uint32_t m0) {
    if (threadIdx.x < (uint32_t)TR) {
      const bool in = m0 + threadIdx.x < a.M;
      rowv[st][0][threadIdx.x] = in ? rl * kLog2e : INFINITY;
      rowv[st][1][threadIdx.x] = in ? rd : 0.0f;
    }
  };
  // Prologue: the first Q / dO tile, its rows' lse / D_m and this wave's
  // K and V rows are all requested before any of them is waited for, and
  // the rows past N are zeroed only after that -- one memory round trip
  // (a block exists only for N > 0).
  // (Loaded one after the other, with load_row's zeroing select waiting
  // for each, the prologue took 8.2 of a 144 us block at C4.)
  if (nt > 0) {
    issue(0);
    fetch_rows(mbeg);
  }
  bf16x8_t kf[D / 16], vf[D / 16];
  load_row_raw<D>(kf, K, a.ldk, ni, a.N, hi);
  load_row_raw<D>(vf, V, a.ldv, ni, a.N, hi);
  zero_past<D>(kf, ni, a.N);
  zero_past<D>(vf, ni, a.N);
  f32x16_t dk[DB], dv[DB];
#pragma unroll
  for (int blk = 0; blk < DB; ++blk) dk[blk] = dv[blk] = f32x16_t{};
  const float c = a.scale_log2;
  const Offsets<D> offs(lane);
  if constexpr (VL) {
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) *reinterpret_cast<bf16x8_t *>(vrows[wave] + offs.row(ks)) = vf[ks];
  }
  if (nt > 0) {
    stash_rows(0, mbeg);
    wait_vmcnt<0>();
  }
  __syncthreads();
  for (uint32_t t = 0; t < nt; ++t) {
    const int st = (int)(t & 1);
    if (t + 1 < nt) {
      issue(t + 1);
      fetch_rows(mbeg + (t + 1) * TR);
    }
    // Offsets recomputed per tile: 13 fewer live registers (the 8-wave pass
    // spills 36 instead of 48; 7 % faster, the causal 4-wave pass 3 %).
    const Offsets<D> off = offs.fresh(t);
    // The tile in 32-query blocks (the swizzle repeats every 16 rows).
#pragma unroll
    for (int sb = 0; sb < TR / kR; ++sb) {
      const uint32_t m0 = mbeg + t * TR + sb * kR;
      const unsigned char *Qt = lds[st][0] + sb * kR * RB, *Gt = lds[st][1] + sb * kR * RB;
      if ((TR == kR || m0 < a.M) && (!CAUSAL || (int64_t)m0 + kR - 1 >= wfirst)) {
        f32x16_t s = dot_rows<D>(Qt, off, kf);         // S [query][key]
        f32x16_t dp;  // dP = dO V^T
        if constexpr (VL) dp = dot_rows_lds<D>(Gt, off, vrows[wave]);
        else dp = dot_rows<D>(Gt, off, vf);
        const bool edge = CAUSAL && (int64_t)m0 < wfirst + kR - 1;
        f32x16_t ds;
#pragma unroll
        for (int r4 = 0; r4 < 4; ++r4) {
          const int row = 8 * r4 + 4 * hi;
          const f32x4_t l4 = *reinterpret_cast<const f32x4_t *>(&rowv[st][0][sb * kR + row]);
          const f32x4_t d4 = *reinterpret_cast<const f32x4_t *>(&rowv[st][1][sb * kR + row]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int r = 4 * r4 + e;
            const float p = __builtin_amdgcn_exp2f(s[r] * c - l4[e]);
            s[r] = p;
            ds[r] = p * (dp[r] - d4[e]);
          }
        }
        // Queries before this key's diagonal: p = 0, under one block-uniform
        // branch (per element the test became compares and selects on
        // every tile).
        if (edge) {
#pragma unroll
          for (int r4 = 0; r4 < 4; ++r4) {
            const int row = 8 * r4 + 4 * hi;
            const f32x4_t d4 = *reinterpret_cast<const f32x4_t *>(&rowv[st][1][sb * kR + row]);
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
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
          const bf16x8_t wp = acc_operand(s, kq), wd = acc_operand(ds, kq);
          if constexpr (WS) {
            // Elements 0-3 / 4-7 of wd: query quads 4 kq + hi / 4 kq + 2 + hi
            // of key ni, i.e. quad pairs x = 2 kq / 2 kq + 1: two 512-byte
            // stores per wave (streaming: read once, by the dQ pass, and
            // kept out of the way of the Q / dO tiles in L2; the dQ pass
            // 4 % faster).  A wave past N has no block to write.  (Holding
            // them to the start of the next tile, out of the wait for that
            // tile's DMA, changed nothing.)
            if (k0w < a.N) {
              const uint4 u = __builtin_bit_cast(uint4, wd);
              unsigned char *blk = dsblk + DsBlk::at(sl.bh, k0w / 32u, m0 / 32u, n32, m32);
              __builtin_nontemporal_store(u32x2_t{u.x, u.y}, reinterpret_cast<u32x2_t *>(blk + DsBlk::pair(dso, 2 * kq)));
              __builtin_nontemporal_store(u32x2_t{u.z, u.w},
                                          reinterpret_cast<u32x2_t *>(blk + DsBlk::pair(dso, 2 * kq + 1)));
            }
          }
#pragma unroll
          for (int blk = 0; blk < DB; ++blk) {
            dv[blk] = mfma16(tr_operand<D>(Gt, off, blk, kq), wp, dv[blk]);  // dV^T += dO^T P
            dk[blk] = mfma16(tr_operand<D>(Qt, off, blk, kq), wd, dk[blk]);  // dK^T += Q^T dS
          }
        }
      }
    }
    if (t + 1 < nt) stash_rows(st ^ 1, mbeg + (t + 1) * TR);
    wait_vmcnt<0>();
    __syncthreads();
  }
  // Staging: the wave's own V rows (VL), or its part of the ring, which is
  // free once every wave has passed the last tile's barrier.
  static_assert(VL || 4 * TB >= kW * kR * RB, "one 32-row staging region per wave fits the ring");
  // Wave-uniform values and the lane id are formed afresh here (SGPRs and
  // mbcnt), so that nothing extra stays live in VGPRs across the tile loop.
  unsigned char *stage = VL ? &vrows[0][0] + wv * (uint32_t)(kR * RB) : &lds[0][0][0] + wv * (uint32_t)(kR * RB);
  const uint32_t r0 = kb + wv * (uint32_t)kR;
  store_rows<D>(dK, a.ldk, r0, a.N, dk, a.scale, (int)__lane_id(), stage);
  store_rows<D>(dV, a.ldv, r0, a.N, dv, 1.0f, (int)__lane_id(), stage);
}

}  // namespace

// 4 waves (128 rows) per block: each streamed tile feeds twice the rows of
// a 2-wave block (measured 5-16 % faster at the C4 / C5-like shapes).  The
// d = 128 dK/dV pass also comes with 8 waves (256 keys per block, two
// waves per SIMD), its V rows in LDS rather than registers (no spills;
// 14 % faster than with them in registers): at the C4 shape 1.35 ms
// unmasked against 1.8 for the 4-wave pass, 0.83 ms causal against 1.17.
// The runtime launches 64 * waves threads and 32 * waves rows per block.
// 64-row streamed tiles halve the barriers and load rounds per row (dQ
// and the causal dK/dV pass 8-9 % faster at the C4 shape, measured with
// register staging); the 8-wave pass keeps 32-row tiles.  Loading the
// tiles with global_load_lds instead of through registers made the dQ
// pass 18-20 % and the 8-wave dK/dV pass 16-17 % faster (fewer VGPRs, no
// LDS write instructions).
constexpr int kWQ = 4, kWK = 4;
constexpr int kTR = 64;  // rows per streamed K/V or Q/dO tile
#define BWPP_ATTN_BWD_BF16(D, CAUSAL, SUFFIX)                                                   \
  extern "C" __global__ __launch_bounds__(64 * kWQ) void bwpp_attn_bwd_bf16_mfma_d##D##SUFFIX##_dq( \
      const BwppAttnArgs a) {                                                                   \
    bwd_dq<D, CAUSAL, kWQ, kTR>(a);                                                             \
  }                                                                                             \
  extern "C" __global__ __launch_bounds__(64 * kWK) void bwpp_attn_bwd_bf16_mfma_d##D##SUFFIX##_dkdv( \
      const BwppAttnArgs a) {                                                                   \
    bwd_dkdv<D, CAUSAL, kWK, kTR>(a);                                                           \
  }

BWPP_ATTN_BWD_BF16(64, false, )
BWPP_ATTN_BWD_BF16(64, true, _causal)
BWPP_ATTN_BWD_BF16(128, false, )
BWPP_ATTN_BWD_BF16(128, true, _causal)
extern "C" __global__ __launch_bounds__(512) void bwpp_attn_bwd_bf16_mfma_d128_dkdv_w8(const BwppAttnArgs a) {
  bwd_dkdv<128, false, 8, kR, true>(a);
}
extern "C" __global__ __launch_bounds__(512) void bwpp_attn_bwd_bf16_mfma_d128_causal_dkdv_w8(const BwppAttnArgs a) {
  bwd_dkdv<128, true, 8, kR, true>(a);
}

// The stored-dS scheme (d = 128): D_m pass, dK / dV passes that also store
// dS^T (4 and 8 waves), and the dQ = dS K pass.
extern "C" __global__ __launch_bounds__(256) void bwpp_attn_bwd_bf16_d128_dsum(const BwppAttnArgs a) {
  bwd_dsum<128, 4>(a);
}
#define BWPP_ATTN_BWD_BF16_DS(CAUSAL, SUFFIX)                                                        \
  extern "C" __global__ __launch_bounds__(256) void bwpp_attn_bwd_bf16_mfma_d128##SUFFIX##_dkdv_ds(   \
      const BwppAttnArgs a) {                                                                       \
    bwd_dkdv<128, CAUSAL, kWK, kTR, false, true>(a);                                                \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(512) void bwpp_attn_bwd_bf16_mfma_d128##SUFFIX##_dkdv_w8_ds( \
      const BwppAttnArgs a) {                                                                       \
    bwd_dkdv<128, CAUSAL, 8, kR, true, true>(a);                                                    \
  }                                                                                                 \
  extern "C" __global__ __launch_bounds__(256) void bwpp_attn_bwd_bf16_mfma_d128##SUFFIX##_dq_ds(     \
      const BwppAttnArgs a) {                                                                       \
    bwd_dq_ds<CAUSAL, kTR>(a);                                                                   \
  }
BWPP_ATTN_BWD_BF16_DS(false, )
BWPP_ATTN_BWD_BF16_DS(true, _causal)
