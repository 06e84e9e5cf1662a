// Flash-style attention forward for gfx950, bf16 Q/K/V/O, fp32 softmax and
// accumulation:  O = softmax(scale * Q K^T [causal mask]) V  per (batch, head).
//
// Semantics: runtime/cpu/bwpp_cpu_ref.c:92-144 (row max, sum of exp, inv =
// sum > 0 ? 1/sum : 0, weighted sum of V) generalised with a score scale and
// a bottom-right aligned causal mask (keys n > m + N - M excluded); the MSL
// kernel it replaces is codegen_metal.c:435-556.
//
// Layout of the work: a block of 8 waves (two per SIMD) owns a tile of 256
// queries of one (batch, head) (causal: two such tiles, one after the
// other); each wave owns 32 queries of the tile.  Keys stream through LDS in
// tiles of 128 (K and V, 32 KiB each for d = 128) in a 2-stage ring, filled
// by global -> LDS DMA.  Two waves per SIMD let one wave's softmax (VALU)
// run while the other's MFMAs issue; 32 queries per wave keep the
// registers (Q^T operands, S^T tile, O^T accumulators) under 256 per wave.
//
// Why S^T: the wave computes S^T = K Q^T with v_mfma_f32_32x32x16_bf16
// (MFMA "A" = a 32-key block of K, "B" = Q^T held in registers).  The
// accumulator then gives lane l the scores of ONE query (l % 32) for 16 of
// the 32 keys; the other 16 are in lane l ^ 32.  Running max, exp, sum and
// the rescale of the output accumulator are therefore lane-local plus one
// lane exchange.  The P V product is computed as O^T += V^T P^T: the
// probabilities go into the MFMA "B" operand straight from the accumulator
// registers, because the key order implied by the accumulator layout
// (lane half h holds keys 4h..4h+3, 8+4h..8+4h+3 of each 16) is applied to
// V^T as well: V^T is read from the [key][d] LDS tile with
// ds_read_b64_tr_b16 at exactly those key rows.
//
// Softmax runs in base 2: scores are multiplied by scale * log2(e) and
// exponentiated with v_exp_f32.  The exponent offset (running maximum) is
// only raised when a tile's maximum exceeds it by more than kLazy (log2
// units): probabilities then stay below 2^kLazy, the common factor cancels
// in O = (sum p v) / (sum p), and the O rescale is skipped on most tiles.
#include <type_traits>

#include "common.h"
#include "../kargs.h"

using namespace bwpp;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef short v8s_t __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

namespace {

constexpr int kWaves = 4;               // generic path
constexpr int kFW = 8;                  // flash path: waves per block
constexpr int kQW = 32;                 // queries per wave
constexpr int kBQ = kFW * kQW;          // queries per block
constexpr float kLazy = 8.0f;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane global -> LDS (M0 = destination of lane 0, lane l at
// +16 l), from a wave-uniform 64-bit base in SGPRs plus a 32-bit per-lane
// byte offset; inline asm keeps the compiler from adding vmcnt(0) before every
// LDS read (completion is awaited with wait_vmcnt + a barrier).  M0 cannot
// be declared clobbered (it is reserved); these kernels use M0 for nothing
// else, which the generated code confirms (only these s_mov_b32 m0 write it).
__device__ __forceinline__ void g2lds16_so(const void *sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds_addr), "v"(voff), "s"(sbase)
               : "memory");
}

// K tile [64 keys][D] (256-byte rows for D = 128): chunk c of row r at
// c ^ (r & 15), so the 16 rows read by a ds_read_b128 quarter-wave hit 16
// distinct bank groups.  V tile [64 keys][D]: chunk c of row r at
// c ^ (4 * (r & 3)), conflict-free for the transposing reads (4 rows x 2
// chunks per 16-lane group, two groups per half-wave).
__device__ __forceinline__ uint32_t k_off(uint32_t r, uint32_t c) { return r * 256u + 16u * (c ^ (r & 15u)); }
__device__ __forceinline__ uint32_t v_off(uint32_t r, uint32_t c) { return r * 256u + 16u * (c ^ (4u * (r & 3u))); }

// One query tile (256 queries) of one (batch, head) slice.
template <bool CAUSAL>
__device__ __forceinline__ void attn_bf16_d128_tile(const BwppAttnArgs &a, const uint32_t bh, const uint32_t qt) {
  // Key tiles: 128 keys in a 2-stage ring (half the barriers and DMA issues
  // per key of 64-key tiles: 4 % faster at C4 unmasked, 5 % causal, where a
  // masked tile skips the 32-key blocks its wave sees none of).
  constexpr int kBKV = 128;
  constexpr int kStages = 2;
  constexpr int D = 128;
  constexpr int KS = D / 16;  // k-steps of S over d
  constexpr int DB = D / 32;  // 32-wide d blocks of O^T
  constexpr int kTile = kBKV * D * 2;
  constexpr int kStage = 2 * kTile;
  constexpr int kRing = kStages * kStage;
  constexpr int kOut = kBQ * D * 2;
  constexpr int kBlkPW = (kBKV / 4) / kFW;  // 1 KiB DMA blocks per wave per K (or V) tile
  constexpr int KB = kBKV / 32;             // 32-key blocks per tile
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kRing > kOut ? kRing : kOut];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const uint16_t *Q = static_cast<const uint16_t *>(a.q) + b * a.q_bs + h * a.q_hs;
  const uint16_t *K = static_cast<const uint16_t *>(a.k) + b * a.k_bs + h * a.k_hs;
  const uint16_t *V = static_cast<const uint16_t *>(a.v) + b * a.v_bs + h * a.v_hs;
  uint16_t *O = static_cast<uint16_t *>(a.o) + b * a.o_bs + h * a.o_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;  // key n visible to query m iff n <= m + diag

  const uint32_t qb0 = qt * kBQ;                    // block's first query
  const uint32_t q0 = qb0 + (uint32_t)wave * kQW;   // wave's first query
  const uint32_t lq = (uint32_t)(lane & 31), lh = (uint32_t)(lane >> 5);
  const uint32_t qi = q0 + lq;                      // this lane's query

  // Key tiles this block needs.
  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last_q = (int64_t)min(qb0 + kBQ, a.M) - 1;
    const int64_t lim = last_q + diag + 1;
    kend = lim <= 0 ? 0u : (uint32_t)min<int64_t>(lim, a.N);
  }
  const uint32_t nkt = (kend + kBKV - 1) / kBKV;

  // Q^T operands: lane holds query qi, d = 16 ks + 8 lh .. +7.
  bf16x8_t qf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    uint4 v = make_uint4(0, 0, 0, 0);
    if (qi < a.M) v = *reinterpret_cast<const uint4 *>(Q + (size_t)qi * a.ldq + 16 * ks + 8 * lh);
    qf[ks] = __builtin_bit_cast(bf16x8_t, v);
  }
  // Let the Q loads land before any DMA is issued: the compiler cannot see
  // the DMA, and an outstanding Q load at the loop head would make it wait
  // for vmcnt(0) -- every tile in flight -- on each iteration.
  wait_vmcnt<0>();

  // DMA: each wave loads kBlkPW of the kBKV / 4 1-KiB blocks of the K tile
  // and of the V tile.  Rows past N re-read row N - 1 (finite data; masked to -inf).
  // Lane l of block i fills 16-byte slot l of it: key row r = 4 i' + l / 16
  // of the tile (i' the block index), physical chunk l % 16, which holds the
  // logical chunk given by the K / V swizzles below.
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)smem;
  uint32_t dma_row[kBlkPW], dma_kcol[kBlkPW], dma_vcol[kBlkPW];
#pragma unroll
  for (int i = 0; i < kBlkPW; ++i) {
    const uint32_t q = (uint32_t)(wave * kBlkPW + i) * 64u + (uint32_t)lane;
    const uint32_t r = q >> 4, pc = q & 15u;
    dma_row[i] = r;
    dma_kcol[i] = 8u * (pc ^ (r & 15u));
    dma_vcol[i] = 8u * (pc ^ (4u * (r & 3u)));
  }
  auto issue = [&](uint32_t t) {
    const uint32_t st = lds0 + (t % kStages) * kStage + (uint32_t)(wave * kBlkPW) * 1024u;
#pragma unroll
    for (int i = 0; i < kBlkPW; ++i) {
      uint32_t key = t * kBKV + dma_row[i];
      key = key < a.N ? key : a.N - 1;
      // Byte offsets inside the (batch, head) slice fit 32 bits (the runtime
      // checks (N - 1) * ld + D < 2^31 before choosing this kernel).
      g2lds16_so(K, 2u * (key * a.ldk + dma_kcol[i]), st + (uint32_t)i * 1024u);
      g2lds16_so(V, 2u * (key * a.ldv + dma_vcol[i]), st + kTile + (uint32_t)i * 1024u);
    }
  };
  constexpr int kDmaPerTile = 2 * kBlkPW;

  f32x16_t o[DB];
#pragma unroll
  for (int d = 0; d < DB; ++d)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
  float mrow = -INFINITY, lrow = 0.0f;
  const float c = a.scale_log2;

  // Per-lane LDS read offsets inside a stage.  K operand of k-step ks, key
  // block kb: koff[ks] + kb * 32 rows.  V^T operand of d block d, keys
  // 32 kb + 16 kq (+8 for the upper four): voff[d] + (32 kb + 16 kq (+8))
  // rows; the V swizzle depends on the row only through r & 3, which those
  // row steps keep.
  const uint32_t grp = (uint32_t)((lane >> 4) & 3), L = (uint32_t)(lane & 15);
  uint32_t koff[KS], voff[DB];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) koff[ks] = k_off(lq, 2u * ks + lh);
  {
    const uint32_t kbase = 4u * (grp >> 1) + (L >> 2);
#pragma unroll
    for (int d = 0; d < DB; ++d) {
      const uint32_t col = 32u * d + 16u * (grp & 1u) + 4u * (L & 3u);
      voff[d] = kTile + v_off(kbase, col >> 3) + (col & 7u) * 2u;
    }
  }

  // One key tile.  MASK: some (key, query) pair of the tile is masked out.
  auto tile = [&](auto mask_tag, const unsigned char *Ks, uint32_t k0) {
    constexpr bool MASK = decltype(mask_tag)::value;
    // Masked tiles: 32-key blocks past every key this wave's queries see
    // are skipped (their scores are masked to -inf below, p = 0).
    int kbmax = KB - 1;
    if constexpr (MASK) {
      int64_t kv = (int64_t)a.N - 1 - (int64_t)k0;
      if (CAUSAL) {
        const int64_t kc = (int64_t)(q0 + kQW - 1) + diag - (int64_t)k0;
        kv = kc < kv ? kc : kv;
      }
      kbmax = kv < 0 ? -1 : (int)(kv / 32 < KB - 1 ? kv / 32 : KB - 1);
      kbmax = __builtin_amdgcn_readfirstlane(kbmax);
    }
    // S^T blocks: s[kb] = K[32 kb .. 32 kb + 31] . Q^T.
    f32x16_t s[KB];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
      if (MASK && kb > kbmax) continue;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const bf16x8_t kf =
            __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(Ks + koff[ks] + 32u * 256u * kb));
        s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb], 0, 0, 0);
      }
    }
    // Keep two K reads ahead of the MFMAs instead of hoisting all sixteen
    // (which would not fit the 256 registers of a two-wave-per-SIMD wave).
    if constexpr (!MASK) {
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int i = 0; i < KB * KS - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }

    // Online softmax for this lane's query (plus partner lane ^ 32).
    float mx = -INFINITY;
    if constexpr (MASK) {
      // Key of register r in block kb is k0 + 4 lh + (32 kb + 8 (r >> 2) +
      // (r & 3)); visible iff that offset is below `lim` (key < N and, when
      // causal, key <= query + diag).  Wave-uniform per block: blocks past
      // kbmax are all masked (their scores stay out of the max, and their
      // probabilities are 0 below), and a block whose last key every query
      // of the wave sees needs no per-element test.
      int64_t lim64 = (int64_t)a.N - (int64_t)(k0 + 4u * lh);
      if (CAUSAL) {
        const int64_t c64 = (int64_t)qi + diag + 1 - (int64_t)(k0 + 4u * lh);
        lim64 = c64 < lim64 ? c64 : lim64;
      }
      const int lim = (int)(lim64 < -1 ? -1 : (lim64 > kBKV ? kBKV : lim64));
      int64_t vis = (int64_t)a.N - 1 - (int64_t)k0;  // last key offset every query of the wave sees
      if (CAUSAL) {
        const int64_t vc = (int64_t)q0 + diag - (int64_t)k0;
        vis = vc < vis ? vc : vis;
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (kb > kbmax) continue;
        if ((int64_t)(32 * kb + 31) <= vis) {
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
        } else {
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float x = (32 * kb + 8 * (r >> 2) + (r & 3)) < lim ? s[kb][r] : -INFINITY;
            s[kb][r] = x;
            mx = fmaxf(mx, x);
          }
        }
      }
    } else {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
    }
    {
      // Lanes l and l ^ 32 hold the two halves of one query's keys.
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) * c;
    }
    // Raise the offset only past the lazy margin (or from -inf).
    float alpha = 1.0f;
    if (mx > mrow + kLazy) {
      alpha = __builtin_amdgcn_exp2f(mrow - mx);  // 0 when mrow is -inf
      mrow = mx;
    }
    const float muse = mrow == -INFINITY ? 0.0f : mrow;
    float sum = 0.0f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (MASK && kb > kbmax) continue;  // p = 0: adds nothing, and its P.V is skipped
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], c, -muse));
        s[kb][r] = p;
        sum += p;
      }
    }
    {
      const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(sum), false, false);
      sum = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    lrow = lrow * alpha + sum;
    if (__ballot(alpha != 1.0f)) {
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
    }

    // O^T += V^T P^T over the blocks of 16 keys.
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      if (MASK && kb > kbmax) continue;
#pragma unroll
      for (int kq = 0; kq < 2; ++kq) {
        const int r0 = 8 * kq;
        uint4 w;
        w.x = pack_bf16x2(s[kb][r0 + 0], s[kb][r0 + 1]);
        w.y = pack_bf16x2(s[kb][r0 + 2], s[kb][r0 + 3]);
        w.z = pack_bf16x2(s[kb][r0 + 4], s[kb][r0 + 5]);
        w.w = pack_bf16x2(s[kb][r0 + 6], s[kb][r0 + 7]);
        const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, w);
        // Key rows of this lane's operand: 32 kb + 16 kq + 4 h (+8).
        constexpr uint32_t kRowB = 256u;
        const uint32_t rstep = (32u * kb + 16u * kq) * kRowB;
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Ks + voff[d] + rstep));
          const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Ks + voff[d] + rstep + 8u * kRowB));
          const v8s_t vv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vv), pf, o[d], 0, 0, 0);
        }
      }
    }
    // Two V^T operands (four transposing reads) ahead of the MFMAs.
    if constexpr (!MASK) {
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int i = 0; i < 2 * KB * DB - 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
    }
  };

#pragma unroll
  for (int st = 0; st < kStages - 1; ++st)
    if ((uint32_t)st < nkt) issue((uint32_t)st);

  // Tiles before t_mask need no mask for any query of the block; the rest
  // go through the masked variant.  Two loops (not one with a branch, which
  // made the compiler keep a second copy of the O accumulators and spill)
  // with a block-uniform boundary: every wave passes every tile's barrier
  // from the same loop.  Inside the masked loop the waves differ only in
  // wave-uniform branches around MFMA work (the 32-key blocks and tiles
  // their queries see none of).
  uint32_t t_mask = a.N / kBKV;  // first tile with keys past N
  if (CAUSAL) {
    // First tile holding a key past the block's first query's limit.
    const int64_t first_hidden = (int64_t)qb0 + diag + 1;
    const uint32_t tc = first_hidden <= 0 ? 0u : (uint32_t)min<int64_t>(first_hidden / kBKV, (int64_t)nkt);
    t_mask = min(t_mask, tc);
  }
  t_mask = min(t_mask, nkt);

  auto step = [&](uint32_t t) {
    // Tiles t + 1 .. t + kStages - 2 may still be in flight.
    const uint32_t younger = min(nkt - 1 - t, (uint32_t)(kStages - 2));
    if (younger >= 2) wait_vmcnt<2 * kDmaPerTile>();
    else if (younger == 1) wait_vmcnt<kDmaPerTile>();
    else wait_vmcnt<0>();
    __syncthreads();
    if (t + kStages - 1 < nkt) issue(t + kStages - 1);
    // The stage base goes through readfirstlane so that loop strength
    // reduction does not turn every LDS address into its own induction
    // variable (it would need ~50 registers); the per-read offsets are then
    // base + lane offset + an immediate.
    return smem + __builtin_amdgcn_readfirstlane((t % kStages) * kStage);
  };
  for (uint32_t t = 0; t < t_mask; ++t) {
    const unsigned char *Ks = step(t);
    tile(std::integral_constant<bool, false>{}, Ks, t * kBKV);
  }
  for (uint32_t t = t_mask; t < nkt; ++t) {
    const unsigned char *Ks = step(t);
    const uint32_t k0 = t * kBKV;
    // Whole tile masked for this wave's queries: nothing to do.
    if (CAUSAL && (int64_t)k0 > (int64_t)(q0 + kQW - 1) + diag) continue;
    tile(std::integral_constant<bool, true>{}, Ks, k0);
  }
  __syncthreads();

  // O = O^T / l, staged through LDS ([query][d] bf16 per wave, 256-byte
  // rows, 16-byte chunk c of row q at c ^ (q & 15)), then stored with
  // 16-byte row chunks.  Without the swizzle the 32 rows a staging write
  // touches at one column all fall on the same banks.  The row stores are
  // non-temporal: O is not read again by this kernel, and written back
  // from the caches later it took bandwidth from the next launch (C4
  // 542 -> 530 us unmasked, 318 -> 301 causal, back to back).
  uint16_t *os = reinterpret_cast<uint16_t *>(smem) + (size_t)wave * kQW * D;
  // Natural-log log-sum-exp of the scaled scores when asked for: the sum of
  // exp(scale s) is 2^mrow * lrow (mrow in log2 units).
  if (a.lse && lh == 0 && qi < a.M)
    a.lse[(size_t)bh * a.M + qi] =
        lrow > 0.0f ? ((mrow == -INFINITY ? 0.0f : mrow) + log2f(lrow)) * 0.69314718055994531f : -INFINITY;
  {
    const float inv = lrow > 0.0f ? 1.0f / lrow : 0.0f;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const uint32_t chunk = (4u * d + q4) ^ (lq & 15u);
        uint2 w;
        w.x = pack_bf16x2(o[d][4 * q4 + 0] * inv, o[d][4 * q4 + 1] * inv);
        w.y = pack_bf16x2(o[d][4 * q4 + 2] * inv, o[d][4 * q4 + 3] * inv);
        *reinterpret_cast<uint2 *>(os + lq * D + 8u * chunk + 4u * lh) = w;
      }
  }
  __syncthreads();
  constexpr int kRowChunks = D / 8;
#pragma unroll 4
  for (int it = 0; it < kQW * kRowChunks / 64; ++it) {
    const int q = lane + it * 64;
    const uint32_t ql = (uint32_t)(q / kRowChunks), cc = (uint32_t)(q % kRowChunks);
    const uint32_t qo = q0 + ql;
    if (qo < a.M)
      __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t *>(os + ql * D + 8u * (cc ^ (ql & 15u))),
                                  reinterpret_cast<u32x4_t *>(O + (size_t)qo * a.ldo + 8u * cc));
  }
  __syncthreads();  // the block's next tile reuses smem
}

// Persistent form of the kernel: a block (one per CU) works through its
// items -- unmasked: (slice, query tile) items, item k of block b being
// k * G + b' (b' the XCD renumbering of b below, so each XCD's blocks take
// the query tiles of a few slices together in every round); causal: the
// same over pairs of query tiles, as attn_bf16_d128 pairs them.  Per item the
// work is attn_bf16_d128_tile's; what differs is the item boundary: the
// next item's first K / V stage is requested at the start of the current
// item's last key tile (into the stage that tile does not use), its Q rows
// as soon as the last tile's S products have read the current ones, and O
// is staged through the last tile's stage -- so the next item's loads are
// in flight during the last tile and the O epilogue instead of after them
// (with one item per block they cost 2.7 us for Q, 1.3 us for the first
// stage and 1.5 us for O of each 62 us item at C4).
template <bool CAUSAL>
__device__ __forceinline__ void attn_bf16_d128_persist(const BwppAttnArgs &a) {
  constexpr int kBKV = 128;
  constexpr int D = 128;
  constexpr int KS = D / 16;
  constexpr int DB = D / 32;
  constexpr int kTile = kBKV * D * 2;
  constexpr int kStage = 2 * kTile;
  constexpr int kOut = kBQ * D * 2;
  static_assert(kOut <= kStage, "O is staged through one ring stage");
  constexpr int kBlkPW = (kBKV / 4) / kFW;
  constexpr int KB = kBKV / 32;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[2 * kStage];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t lq = (uint32_t)(lane & 31), lh = (uint32_t)(lane >> 5);
  const uint32_t G = gridDim.x, QT = a.q_tiles;
  const uint32_t bp = G % 8u == 0 ? (blockIdx.x % 8u) * (G / 8u) + blockIdx.x / 8u : blockIdx.x;
  // Unmasked: a.items (slice, query tile) items.  Causal: a.items pairs of
  // query tiles QT - 1 - p and p of one slice, as attn_bf16_d128 pairs them
  // (one item when they coincide); block b' takes pairs j G + b'.
  const uint32_t P = (QT + 1) / 2;
  const uint32_t nunits = bp < a.items ? (a.items - bp + G - 1) / G : 0u;
  const uint32_t nitems = CAUSAL ? 2u * nunits : nunits;  // slots; a causal pair's second may be empty
  if (nitems == 0) return;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;  // key n visible to query m iff n <= m + diag

  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)smem;
  uint32_t dma_row[kBlkPW], dma_kcol[kBlkPW], dma_vcol[kBlkPW];
#pragma unroll
  for (int i = 0; i < kBlkPW; ++i) {
    const uint32_t q = (uint32_t)(wave * kBlkPW + i) * 64u + (uint32_t)lane;
    const uint32_t r = q >> 4, pc = q & 15u;
    dma_row[i] = r;
    dma_kcol[i] = 8u * (pc ^ (r & 15u));
    dma_vcol[i] = 8u * (pc ^ (4u * (r & 3u)));
  }
  struct Item {
    const uint16_t *Q, *K, *V;
    uint16_t *O;
    uint32_t bh, q0, qb0;
  };
  // Slot k: its slice and query tile; valid(k) is false only for the empty
  // second slot of a causal pair whose two tiles coincide.
  auto slot_tile = [&](uint32_t k, uint32_t &bh) {
    if (!CAUSAL) {
      const uint32_t li = k * G + bp;
      bh = li / QT;
      return QT - 1 - li % QT;
    }
    const uint32_t pi = (k >> 1) * G + bp, p = pi % P;
    bh = pi / P;
    return (k & 1u) ? p : QT - 1 - p;
  };
  auto valid = [&](uint32_t k) {
    if (!CAUSAL || !(k & 1u)) return k < nitems;
    const uint32_t p = ((k >> 1) * G + bp) % P;
    return k < nitems && p != QT - 1 - p;
  };
  auto item = [&](uint32_t k) {
    uint32_t bh;
    const uint32_t qt = slot_tile(k, bh);
    const uint32_t b = bh / a.heads, h = bh % a.heads;
    Item it;
    it.Q = static_cast<const uint16_t *>(a.q) + b * a.q_bs + h * a.q_hs;
    it.K = static_cast<const uint16_t *>(a.k) + b * a.k_bs + h * a.k_hs;
    it.V = static_cast<const uint16_t *>(a.v) + b * a.v_bs + h * a.v_hs;
    it.O = static_cast<uint16_t *>(a.o) + b * a.o_bs + h * a.o_hs;
    it.bh = bh;
    it.qb0 = qt * kBQ;
    it.q0 = it.qb0 + (uint32_t)wave * kQW;
    return it;
  };
  // Key tiles an item needs, and its first tile with a masked (key, query).
  auto key_tiles = [&](const Item &it) {
    uint32_t kend = a.N;
    if (CAUSAL) {
      const int64_t lim = (int64_t)min(it.qb0 + kBQ, a.M) - 1 + diag + 1;
      kend = lim <= 0 ? 0u : (uint32_t)min<int64_t>(lim, a.N);
    }
    return (kend + kBKV - 1) / kBKV;
  };
  auto first_masked = [&](const Item &it, uint32_t nkt) {
    uint32_t tm = a.N / kBKV;
    if (CAUSAL) {
      const int64_t first_hidden = (int64_t)it.qb0 + diag + 1;
      tm = min(tm, first_hidden <= 0 ? 0u : (uint32_t)min<int64_t>(first_hidden / kBKV, (int64_t)nkt));
    }
    return min(tm, nkt);
  };
  auto issue = [&](const Item &it, uint32_t t, uint32_t stage) {
    const uint32_t st = lds0 + stage * kStage + (uint32_t)(wave * kBlkPW) * 1024u;
#pragma unroll
    for (int i = 0; i < kBlkPW; ++i) {
      uint32_t key = t * kBKV + dma_row[i];
      key = key < a.N ? key : a.N - 1;
      g2lds16_so(it.K, 2u * (key * a.ldk + dma_kcol[i]), st + (uint32_t)i * 1024u);
      g2lds16_so(it.V, 2u * (key * a.ldv + dma_vcol[i]), st + kTile + (uint32_t)i * 1024u);
    }
  };
  bf16x8_t qf[KS];
  auto load_q = [&](const Item &it) {
    const uint32_t qi = it.q0 + lq;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qi < a.M) v = *reinterpret_cast<const uint4 *>(it.Q + (size_t)qi * a.ldq + 16 * ks + 8 * lh);
      qf[ks] = __builtin_bit_cast(bf16x8_t, v);
    }
  };

  // Per-lane LDS read offsets of k-step 0 / d block 0 (as in
  // attn_bf16_d128_tile); the others differ in chunk bits the swizzles XOR
  // and never carry into: K operand of k-step ks at koff0 ^ 32 ks, V^T of d
  // block d at voff0 ^ 64 d.  The tile recomputes them (see below).
  const uint32_t grp = (uint32_t)((lane >> 4) & 3), L = (uint32_t)(lane & 15);
  const uint32_t koff0 = k_off(lq, lh);
  const uint32_t voff0 = kTile + v_off(4u * (grp >> 1) + (L >> 2), 2u * (grp & 1u) + ((L & 3u) >> 1)) + (4u * (L & 1u)) * 2u;
  const float c = a.scale_log2;

  // First item: Q, then its first stage (the Q loads land first, as in
  // attn_bf16_d128_tile).
  Item cur = item(0);
  load_q(cur);
  wait_vmcnt<0>();
  issue(cur, 0, 0);
  uint32_t s0 = 0;  // ring stage of the current item's key tile 0

  for (uint32_t k = 0; k < nitems; ++k) {
    if (!valid(k)) continue;
    const uint32_t kn = valid(k + 1) ? k + 1 : k + 2;  // the next item's slot
    const bool has_next = kn < nitems;
    const Item nxt = item(has_next ? kn : k);
    const uint32_t qi = cur.q0 + lq;
    const uint32_t nkt = key_tiles(cur), t_mask = first_masked(cur, nkt);
    f32x16_t o[DB];
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[d][r] = 0.0f;
    float mrow = -INFINITY, lrow = 0.0f;

    auto tile = [&](auto mask_tag, const unsigned char *Ks, uint32_t k0, bool last) {
      constexpr bool MASK = decltype(mask_tag)::value;
      // The offsets through an empty asm tied to the tile, so that their
      // XORed forms stay inside the tile instead of occupying twelve
      // registers across the whole item loop (the causal kernel spilled).
      uint32_t ko = koff0, vo = voff0;
      asm("" : "+v"(ko), "+v"(vo) : "s"(k0));
      int kbmax = KB - 1;
      if constexpr (MASK) {
        int64_t kv = (int64_t)a.N - 1 - (int64_t)k0;
        if (CAUSAL) {
          const int64_t kc = (int64_t)(cur.q0 + kQW - 1) + diag - (int64_t)k0;
          kv = kc < kv ? kc : kv;
        }
        kbmax = kv < 0 ? -1 : (int)(kv / 32 < KB - 1 ? kv / 32 : KB - 1);
        kbmax = __builtin_amdgcn_readfirstlane(kbmax);
      }
      f32x16_t s[KB];
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][r] = 0.0f;
        if (MASK && kb > kbmax) continue;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8_t kf =
              __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(Ks + (ko ^ (32u * ks)) + 32u * 256u * kb));
          s[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb], 0, 0, 0);
        }
      }
      if constexpr (!MASK) {
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 0; i < KB * KS - 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      }
      // The current Q rows are no longer needed: request the next item's.
      if (last && has_next) load_q(nxt);

      float mx = -INFINITY;
      if constexpr (MASK) {
        // As in attn_bf16_d128_tile: blocks past kbmax are left out, and a
        // block every query of the wave sees whole needs no element test.
        int64_t lim64 = (int64_t)a.N - (int64_t)(k0 + 4u * lh);
        if (CAUSAL) {
          const int64_t c64 = (int64_t)qi + diag + 1 - (int64_t)(k0 + 4u * lh);
          lim64 = c64 < lim64 ? c64 : lim64;
        }
        const int lim = (int)(lim64 < -1 ? -1 : (lim64 > kBKV ? kBKV : lim64));
        int64_t vis = (int64_t)a.N - 1 - (int64_t)k0;
        if (CAUSAL) {
          const int64_t vc = (int64_t)cur.q0 + diag - (int64_t)k0;
          vis = vc < vis ? vc : vis;
        }
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
          if (kb > kbmax) continue;
          if ((int64_t)(32 * kb + 31) <= vis) {
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
          } else {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const float x = (32 * kb + 8 * (r >> 2) + (r & 3)) < lim ? s[kb][r] : -INFINITY;
              s[kb][r] = x;
              mx = fmaxf(mx, x);
            }
          }
        }
      } else {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[kb][r]);
      }
      {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
        mx = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1])) * c;
      }
      float alpha = 1.0f;
      if (mx > mrow + kLazy) {
        alpha = __builtin_amdgcn_exp2f(mrow - mx);
        mrow = mx;
      }
      const float muse = mrow == -INFINITY ? 0.0f : mrow;
      float sum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (MASK && kb > kbmax) continue;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][r], c, -muse));
          s[kb][r] = p;
          sum += p;
        }
      }
      {
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(sum), false, false);
        sum = __uint_as_float(r[0]) + __uint_as_float(r[1]);
      }
      lrow = lrow * alpha + sum;
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[d][r] *= alpha;
      }
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        if (MASK && kb > kbmax) continue;
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
          const int r0 = 8 * kq;
          uint4 w;
          w.x = pack_bf16x2(s[kb][r0 + 0], s[kb][r0 + 1]);
          w.y = pack_bf16x2(s[kb][r0 + 2], s[kb][r0 + 3]);
          w.z = pack_bf16x2(s[kb][r0 + 4], s[kb][r0 + 5]);
          w.w = pack_bf16x2(s[kb][r0 + 6], s[kb][r0 + 7]);
          const bf16x8_t pf = __builtin_bit_cast(bf16x8_t, w);
          constexpr uint32_t kRowB = 256u;
          const uint32_t rstep = (32u * kb + 16u * kq) * kRowB;
#pragma unroll
          for (int d = 0; d < DB; ++d) {
            const uint32_t vd = vo ^ (64u * d);
            const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Ks + vd + rstep));
            const v4s_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Ks + vd + rstep + 8u * kRowB));
            const v8s_t vv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
            o[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vv), pf, o[d], 0, 0, 0);
          }
        }
      }
      if constexpr (!MASK) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
        for (int i = 0; i < 2 * KB * DB - 2; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
      }
    };

    // Tile t lives in stage (s0 + t) % 2.  At tile t's barrier every wave is
    // done with tile t - 1, whose stage then takes tile t + 1 -- or, at the
    // last tile, the next item's tile 0.
    auto step = [&](uint32_t t) {
      wait_vmcnt<0>();
      __syncthreads();
      const uint32_t nst = (s0 + t + 1) & 1u;
      if (t + 1 < nkt) issue(cur, t + 1, nst);
      else if (has_next) issue(nxt, 0, nst);
      return smem + __builtin_amdgcn_readfirstlane(((s0 + t) & 1u) * kStage);
    };
    for (uint32_t t = 0; t < t_mask; ++t) {
      const unsigned char *Ks = step(t);
      tile(std::integral_constant<bool, false>{}, Ks, t * kBKV, t + 1 == nkt);
    }
    // A tile whose keys this wave's queries see none of goes through tile()
    // too: no MFMA runs (kbmax = -1), the all -inf scores leave the running
    // max, the sum and O exactly as they were, and the next item's Q rows
    // are requested at one place (a second one, in a skip branch, made the
    // compiler keep two versions of them and spill).
    for (uint32_t t = t_mask; t < nkt; ++t) {
      const unsigned char *Ks = step(t);
      tile(std::integral_constant<bool, true>{}, Ks, t * kBKV, t + 1 == nkt);
    }
    __syncthreads();
    if (nkt == 0 && has_next) {
      // No key tile: the next item's loads start here (after this item's
      // own, unused, first-stage DMA into the same stage has landed).
      wait_vmcnt<0>();
      load_q(nxt);
      issue(nxt, 0, s0);
    }

    // O through the last tile's stage (the other one holds the next item's
    // tile 0); the next item's tile 1 goes into this stage after its first
    // barrier, which comes after these reads.
    uint16_t *os = reinterpret_cast<uint16_t *>(smem + ((s0 + nkt + 1) & 1u) * kStage) + (size_t)wave * kQW * D;
    if (a.lse && lh == 0 && qi < a.M)
      a.lse[(size_t)cur.bh * a.M + qi] =
          lrow > 0.0f ? ((mrow == -INFINITY ? 0.0f : mrow) + log2f(lrow)) * 0.69314718055994531f : -INFINITY;
    {
      const float inv = lrow > 0.0f ? 1.0f / lrow : 0.0f;
#pragma unroll
      for (int d = 0; d < DB; ++d)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          const uint32_t chunk = (4u * d + q4) ^ (lq & 15u);
          uint2 w;
          w.x = pack_bf16x2(o[d][4 * q4 + 0] * inv, o[d][4 * q4 + 1] * inv);
          w.y = pack_bf16x2(o[d][4 * q4 + 2] * inv, o[d][4 * q4 + 3] * inv);
          *reinterpret_cast<uint2 *>(os + lq * D + 8u * chunk + 4u * lh) = w;
        }
    }
    __syncthreads();
    constexpr int kRowChunks = D / 8;
#pragma unroll 4
    for (int it = 0; it < kQW * kRowChunks / 64; ++it) {
      const int q = lane + it * 64;
      const uint32_t ql = (uint32_t)(q / kRowChunks), cc = (uint32_t)(q % kRowChunks);
      const uint32_t qo = cur.q0 + ql;
      if (qo < a.M)
        __builtin_nontemporal_store(*reinterpret_cast<const u32x4_t *>(os + ql * D + 8u * (cc ^ (ql & 15u))),
                                    reinterpret_cast<u32x4_t *>(cur.O + (size_t)qo * a.ldo + 8u * cc));
    }
    s0 = (s0 + nkt) & 1u;
    cur = nxt;
  }
}

// Work per block.  Blocks are dispatched round-robin over the 8 XCDs; the
// renumbering below gives each XCD a contiguous run of (batch, head) slices
// with all of their query tiles, so the blocks that stream the same K / V
// run together on one L2.  Unmasked: one query tile per block.  Causal: a
// block takes query tiles QT - 1 - p and p of one slice, whose visible key
// counts add up to the same total for every p (up to the clamping at 0 and
// N when M != N), so the blocks carry equal work (the runtime launches
// slices * ceil(QT / 2) blocks).
template <bool CAUSAL>
__device__ __forceinline__ void attn_bf16_d128(const BwppAttnArgs &a) {
  const uint32_t G = gridDim.x, QT = a.q_tiles;
  const uint32_t lb = G % 8u == 0 ? (blockIdx.x % 8u) * (G / 8u) + blockIdx.x / 8u : blockIdx.x;
  if (!CAUSAL) {
    attn_bf16_d128_tile<CAUSAL>(a, lb / QT, QT - 1 - lb % QT);
    return;
  }
  const uint32_t P = (QT + 1) / 2, bh = lb / P, pi = lb % P;
  for (uint32_t i = 0; i < 2; ++i) {
    if (i == 1 && QT - 1 - pi == pi) break;
    attn_bf16_d128_tile<CAUSAL>(a, bh, i == 0 ? QT - 1 - pi : pi);
  }
}

// ------------------------------------------------------------- generic path
// Any head dims K, D <= 512, fp32 or bf16 storage, fp32 arithmetic with
// expf: the reference's accumulation conventions (dot products in k order,
// bwpp_cpu_ref.c:110-113) with an online max/sum over chunks of 64 keys.
// A wave processes one query at a time: lanes split the keys for the
// scores (one key per lane per chunk), the probabilities go through LDS,
// and lanes split d for the weighted sum of V.  4 waves per block, 16
// queries per block.
constexpr int kGenQ = 16;
constexpr int kGenMaxDim = 512;

template <class T>
__device__ __forceinline__ float ld_elem(const T *p) {
  if constexpr (sizeof(T) == 2)
    return bf16_bits_to_f32(*reinterpret_cast<const uint16_t *>(p));
  else
    return *p;
}
template <class T>
__device__ __forceinline__ void st_elem(T *p, float v) {
  if constexpr (sizeof(T) == 2)
    *reinterpret_cast<uint16_t *>(p) = f32_to_bf16_bits(v);
  else
    *p = v;
}

template <class T, bool CAUSAL>
__device__ __forceinline__ void attn_generic(const BwppAttnArgs &a) {
  const uint32_t Kd = a.kdim, Dv = a.vdim;
  __shared__ float qs[kWaves][kGenMaxDim];
  __shared__ float ps[kWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t nbh = gridDim.x / a.q_tiles;
  const uint32_t qt = a.q_tiles - 1 - blockIdx.x / nbh;
  const uint32_t bh = blockIdx.x % nbh;
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const T *Q = static_cast<const T *>(a.q) + b * a.q_bs + h * a.q_hs;
  const T *K = static_cast<const T *>(a.k) + b * a.k_bs + h * a.k_hs;
  const T *V = static_cast<const T *>(a.v) + b * a.v_bs + h * a.v_hs;
  T *O = static_cast<T *>(a.o) + b * a.o_bs + h * a.o_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const float scale = a.scale_log2;  // the plain scale on this path
  constexpr int DPL = kGenMaxDim / 64;

  for (uint32_t qq = (uint32_t)wave; qq < kGenQ; qq += kWaves) {
    const uint32_t qi = qt * kGenQ + qq;
    if (qi >= a.M) break;  // wave-uniform
    for (uint32_t k = (uint32_t)lane; k < Kd; k += 64) qs[wave][k] = ld_elem(Q + (size_t)qi * a.ldq + k);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    int64_t lim = CAUSAL ? (int64_t)qi + diag + 1 : (int64_t)a.N;
    lim = lim < 0 ? 0 : (lim > (int64_t)a.N ? (int64_t)a.N : lim);
    const uint32_t kend = (uint32_t)lim;
    float m = -INFINITY, l = 0.0f;
    float o[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) o[j] = 0.0f;
    for (uint32_t n0 = 0; n0 < kend; n0 += 64) {
      const uint32_t n = n0 + (uint32_t)lane;
      float s = -INFINITY;
      if (n < kend) {
        const T *kr = K + (size_t)n * a.ldk;
        float acc = 0.0f;
        for (uint32_t k = 0; k < Kd; ++k) acc += qs[wave][k] * ld_elem(kr + k);
        s = acc * scale;
      }
      const float cm = wave_max(s);
      const float mnew = fmaxf(m, cm);
      const float muse = mnew == -INFINITY ? 0.0f : mnew;
      const float alpha = expf(m - muse);
      const float p = n < kend ? expf(s - muse) : 0.0f;
      l = l * alpha + wave_sum(p);
      m = mnew;
      __builtin_amdgcn_wave_barrier();
      ps[wave][lane] = p;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t cnt = min(64u, kend - n0);
#pragma unroll
      for (int j = 0; j < DPL; ++j) o[j] *= alpha;
      for (uint32_t t = 0; t < cnt; ++t) {
        const float pn = ps[wave][t];
        const T *vr = V + (size_t)(n0 + t) * a.ldv;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const uint32_t d = (uint32_t)lane + 64u * j;
          if (d < Dv) o[j] += pn * ld_elem(vr + d);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
    const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const uint32_t d = (uint32_t)lane + 64u * j;
      if (d < Dv) st_elem(O + (size_t)qi * a.ldo + d, o[j] * inv);
    }
    if (a.lse && lane == 0) a.lse[(size_t)bh * a.M + qi] = l > 0.0f ? m + logf(l) : -INFINITY;
    __builtin_amdgcn_wave_barrier();
  }
}

// ------------------------------------------------------- backward (generic)
// O = softmax(scale Q K^T [mask]) V.  With the saved lse (natural-log
// log-sum-exp per query) the probabilities are recomputed as
// p = exp(scale q.k - lse) and, with D_m = rowsum(dO * O)[m],
//   dS = p (dO.v - D_m),  dQ = scale dS K,  dK = scale dS^T Q,  dV = P^T dO.
// Two passes, both one wave per row with fp32 arithmetic and any head dims
// up to 512: attn_bwd_dq (one query per wave; also writes D_m) and then
// attn_bwd_dkdv (one key per wave, looping over the queries that see it).

template <class T, bool CAUSAL>
__device__ __forceinline__ void attn_bwd_dq(const BwppAttnArgs &a) {
  const uint32_t Kd = a.kdim, Dv = a.vdim;
  __shared__ float qs[kWaves][kGenMaxDim];
  __shared__ float gs[kWaves][kGenMaxDim];
  __shared__ float ps[kWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t nbh = gridDim.x / a.q_tiles;
  const uint32_t qt = a.q_tiles - 1 - blockIdx.x / nbh;
  const uint32_t bh = blockIdx.x % nbh;
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const T *Q = static_cast<const T *>(a.q) + b * a.q_bs + h * a.q_hs;
  const T *K = static_cast<const T *>(a.k) + b * a.k_bs + h * a.k_hs;
  const T *V = static_cast<const T *>(a.v) + b * a.v_bs + h * a.v_hs;
  const T *O = static_cast<const T *>(a.o) + b * a.o_bs + h * a.o_hs;
  const T *dO = static_cast<const T *>(a.dout) + b * a.o_bs + h * a.o_hs;
  T *dQ = static_cast<T *>(a.dq) + b * a.q_bs + h * a.q_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const float scale = a.scale_log2;  // the plain scale on this path
  constexpr int DPL = kGenMaxDim / 64;

  for (uint32_t qq = (uint32_t)wave; qq < kGenQ; qq += kWaves) {
    const uint32_t qi = qt * kGenQ + qq;
    if (qi >= a.M) break;  // wave-uniform
    for (uint32_t k = (uint32_t)lane; k < Kd; k += 64) qs[wave][k] = ld_elem(Q + (size_t)qi * a.ldq + k);
    float dsum = 0.0f;
    for (uint32_t d = (uint32_t)lane; d < Dv; d += 64) {
      const float g = ld_elem(dO + (size_t)qi * a.ldo + d);
      gs[wave][d] = g;
      dsum += g * ld_elem(O + (size_t)qi * a.ldo + d);
    }
    dsum = wave_sum(dsum);
    if (lane == 0) a.dsum[(size_t)bh * a.M + qi] = dsum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    const float lse = a.lse[(size_t)bh * a.M + qi];
    int64_t lim = CAUSAL ? (int64_t)qi + diag + 1 : (int64_t)a.N;
    lim = lim < 0 ? 0 : (lim > (int64_t)a.N ? (int64_t)a.N : lim);
    const uint32_t kend = (uint32_t)lim;
    float acc[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] = 0.0f;
    for (uint32_t n0 = 0; n0 < kend; n0 += 64) {
      const uint32_t n = n0 + (uint32_t)lane;
      float ds = 0.0f;
      if (n < kend) {
        const T *kr = K + (size_t)n * a.ldk;
        const T *vr = V + (size_t)n * a.ldv;
        float s = 0.0f, dp = 0.0f;
        for (uint32_t k = 0; k < Kd; ++k) s += qs[wave][k] * ld_elem(kr + k);
        for (uint32_t d = 0; d < Dv; ++d) dp += gs[wave][d] * ld_elem(vr + d);
        const float p = expf(s * scale - lse);
        ds = p * (dp - dsum);
      }
      __builtin_amdgcn_wave_barrier();
      ps[wave][lane] = ds;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t cnt = min(64u, kend - n0);
      for (uint32_t t = 0; t < cnt; ++t) {
        const float dsn = ps[wave][t];
        const T *kr = K + (size_t)(n0 + t) * a.ldk;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const uint32_t k = (uint32_t)lane + 64u * j;
          if (k < Kd) acc[j] += dsn * ld_elem(kr + k);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const uint32_t k = (uint32_t)lane + 64u * j;
      if (k < Kd) st_elem(dQ + (size_t)qi * a.ldq + k, acc[j] * scale);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

template <class T, bool CAUSAL>
__device__ __forceinline__ void attn_bwd_dkdv(const BwppAttnArgs &a) {
  const uint32_t Kd = a.kdim, Dv = a.vdim;
  __shared__ float ks[kWaves][kGenMaxDim];
  __shared__ float vs[kWaves][kGenMaxDim];
  __shared__ float pp[kWaves][64];
  __shared__ float dd[kWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t nbh = gridDim.x / a.q_tiles;  // q_tiles holds the key tiles here
  const uint32_t kt = a.q_tiles - 1 - blockIdx.x / nbh;
  const uint32_t bh = blockIdx.x % nbh;
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const T *Q = static_cast<const T *>(a.q) + b * a.q_bs + h * a.q_hs;
  const T *K = static_cast<const T *>(a.k) + b * a.k_bs + h * a.k_hs;
  const T *V = static_cast<const T *>(a.v) + b * a.v_bs + h * a.v_hs;
  const T *dO = static_cast<const T *>(a.dout) + b * a.o_bs + h * a.o_hs;
  T *dK = static_cast<T *>(a.dk) + b * a.k_bs + h * a.k_hs;
  T *dV = static_cast<T *>(a.dv) + b * a.v_bs + h * a.v_hs;
  const float *lse = a.lse + (size_t)bh * a.M;
  const float *dsum = a.dsum + (size_t)bh * a.M;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;
  const float scale = a.scale_log2;
  constexpr int DPL = kGenMaxDim / 64;

  for (uint32_t kk = (uint32_t)wave; kk < kGenQ; kk += kWaves) {
    const uint32_t n = kt * kGenQ + kk;
    if (n >= a.N) break;  // wave-uniform
    for (uint32_t k = (uint32_t)lane; k < Kd; k += 64) ks[wave][k] = ld_elem(K + (size_t)n * a.ldk + k);
    for (uint32_t d = (uint32_t)lane; d < Dv; d += 64) vs[wave][d] = ld_elem(V + (size_t)n * a.ldv + d);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // Queries that see key n: m >= n - diag (causal), all otherwise.
    int64_t first = CAUSAL ? (int64_t)n - diag : 0;
    first = first < 0 ? 0 : first;
    const uint32_t mbeg = first > (int64_t)a.M ? a.M : (uint32_t)first;
    float gk[DPL], gv[DPL];
#pragma unroll
    for (int j = 0; j < DPL; ++j) gk[j] = gv[j] = 0.0f;
    for (uint32_t m0 = mbeg; m0 < a.M; m0 += 64) {
      const uint32_t m = m0 + (uint32_t)lane;
      float p = 0.0f, ds = 0.0f;
      if (m < a.M) {
        const T *qr = Q + (size_t)m * a.ldq;
        const T *gr = dO + (size_t)m * a.ldo;
        float s = 0.0f, dp = 0.0f;
        for (uint32_t k = 0; k < Kd; ++k) s += ld_elem(qr + k) * ks[wave][k];
        for (uint32_t d = 0; d < Dv; ++d) dp += ld_elem(gr + d) * vs[wave][d];
        p = expf(s * scale - lse[m]);
        ds = p * (dp - dsum[m]);
      }
      __builtin_amdgcn_wave_barrier();
      pp[wave][lane] = p;
      dd[wave][lane] = ds;
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const uint32_t cnt = min(64u, a.M - m0);
      for (uint32_t t = 0; t < cnt; ++t) {
        const float pm = pp[wave][t], dm = dd[wave][t];
        const T *qr = Q + (size_t)(m0 + t) * a.ldq;
        const T *gr = dO + (size_t)(m0 + t) * a.ldo;
#pragma unroll
        for (int j = 0; j < DPL; ++j) {
          const uint32_t c = (uint32_t)lane + 64u * j;
          if (c < Kd) gk[j] += dm * ld_elem(qr + c);
          if (c < Dv) gv[j] += pm * ld_elem(gr + c);
        }
      }
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int j = 0; j < DPL; ++j) {
      const uint32_t c = (uint32_t)lane + 64u * j;
      if (c < Kd) st_elem(dK + (size_t)n * a.ldk + c, gk[j] * scale);
      if (c < Dv) st_elem(dV + (size_t)n * a.ldv + c, gv[j]);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

#define BWPP_ATTN_BWD(NAME, T, CAUSAL)                                                      \
  extern "C" __global__ __launch_bounds__(256) void NAME##_dq(const BwppAttnArgs a) {       \
    attn_bwd_dq<T, CAUSAL>(a);                                                             \
  }                                                                                        \
  extern "C" __global__ __launch_bounds__(256) void NAME##_dkdv(const BwppAttnArgs a) {     \
    attn_bwd_dkdv<T, CAUSAL>(a);                                                           \
  }
BWPP_ATTN_BWD(bwpp_attn_bwd_f32, float, false)
BWPP_ATTN_BWD(bwpp_attn_bwd_f32_causal, float, true)
BWPP_ATTN_BWD(bwpp_attn_bwd_bf16, uint16_t, false)
BWPP_ATTN_BWD(bwpp_attn_bwd_bf16_causal, uint16_t, true)

// Generic path entry points, one per storage type x mask.
#define BWPP_ATTN_GENERIC(NAME, T, CAUSAL)                                                  \
  extern "C" __global__ __launch_bounds__(256) void NAME(const BwppAttnArgs a) {            \
    attn_generic<T, CAUSAL>(a);                                                            \
  }
BWPP_ATTN_GENERIC(bwpp_attn_generic_f32, float, false)
BWPP_ATTN_GENERIC(bwpp_attn_generic_f32_causal, float, true)
BWPP_ATTN_GENERIC(bwpp_attn_generic_bf16, uint16_t, false)
BWPP_ATTN_GENERIC(bwpp_attn_generic_bf16_causal, uint16_t, true)

extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2))) void
bwpp_attn_bf16_d128(const BwppAttnArgs a) {
  attn_bf16_d128<false>(a);
}
// Persistent unmasked form (a.items (slice, query tile) items over one
// block per CU).
extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2))) void
bwpp_attn_bf16_d128_p(const BwppAttnArgs a) {
  attn_bf16_d128_persist<false>(a);
}
extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2))) void
bwpp_attn_bf16_d128_causal_p(const BwppAttnArgs a) {
  attn_bf16_d128_persist<true>(a);
}
extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(512, 512), amdgpu_waves_per_eu(2, 2))) void
bwpp_attn_bf16_d128_causal(const BwppAttnArgs a) {
  attn_bf16_d128<true>(a);
}
