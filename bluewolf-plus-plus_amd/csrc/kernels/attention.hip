// Flash-style attention forward for gfx950, bf16 Q/K/V/O, fp32 softmax and
// accumulation:  O = softmax(scale * Q K^T [causal mask]) V  per (batch, head).
//
// Semantics: runtime/cpu/bwpp_cpu_ref.c:92-144 (row max, sum of exp, inv =
// sum > 0 ? 1/sum : 0, weighted sum of V) generalised with a score scale and
// a bottom-right aligned causal mask (keys n > m + N - M excluded); the MSL
// kernel it replaces is codegen_metal.c:435-556.
//
// Layout of the work: a block of 4 waves owns 256 queries of one
// (batch, head); each wave owns 64 queries as two 32-query groups.  Keys
// stream through LDS in tiles of 64 (K and V, 16 KiB each for d = 128) in a
// 3-stage ring filled by global -> LDS DMA.
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
// exponentiated with v_exp_f32.
#include "common.h"
#include "../kargs.h"

using namespace bwpp;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef short v4s_t __attribute__((ext_vector_type(4)));
typedef short v8s_t __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) v4s_t lds_v4s_t;

namespace {

constexpr int kWaves = 4;
constexpr int kQW = 64;                 // queries per wave
constexpr int kBQ = kWaves * kQW;       // queries per block
constexpr int kBKV = 64;                // keys per tile
constexpr int kStages = 3;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16 bytes per lane global -> LDS (M0 = destination of lane 0, lane l at
// +16 l); inline asm keeps the compiler from adding vmcnt(0) before every
// LDS read (completion is awaited with wait_vmcnt + a barrier).  M0 cannot
// be declared clobbered (it is reserved); these kernels use M0 for nothing
// else, which the generated code confirms (only these s_mov_b32 m0 write it).
__device__ __forceinline__ void g2lds16(const void *gptr, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off" ::"s"(lds_addr), "v"(gptr)
               : "memory");
}

// K tile [64 keys][D] (256-byte rows for D = 128): chunk c of row r at
// c ^ (r & 15), so the 16 rows read by a ds_read_b128 quarter-wave hit 16
// distinct bank groups.  V tile [64 keys][D]: chunk c of row r at
// c ^ (4 * (r & 3)), conflict-free for the transposing reads (4 rows x 2
// chunks per 16-lane group, two groups per half-wave).
__device__ __forceinline__ uint32_t k_off(uint32_t r, uint32_t c) { return r * 256u + 16u * (c ^ (r & 15u)); }
__device__ __forceinline__ uint32_t v_off(uint32_t r, uint32_t c) { return r * 256u + 16u * (c ^ (4u * (r & 3u))); }

template <bool CAUSAL>
__device__ __forceinline__ void attn_bf16_d128(const BwppAttnArgs &a) {
  constexpr int D = 128;
  constexpr int KS = D / 16;  // k-steps of S over d
  constexpr int DB = D / 32;  // 32-wide d blocks of O^T
  constexpr int kTile = kBKV * D * 2;
  constexpr int kStage = 2 * kTile;
  constexpr int kRing = kStages * kStage;
  constexpr int kOut = kBQ * D * 2;
  __shared__ __attribute__((aligned(1024))) unsigned char smem[kRing > kOut ? kRing : kOut];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const uint32_t nbh = gridDim.x / a.q_tiles;
  const uint32_t qt = a.q_tiles - 1 - blockIdx.x / nbh;  // heaviest query tiles first
  const uint32_t bh = blockIdx.x % nbh;
  const uint32_t b = bh / a.heads, h = bh % a.heads;
  const uint16_t *Q = static_cast<const uint16_t *>(a.q) + b * a.q_bs + h * a.q_hs;
  const uint16_t *K = static_cast<const uint16_t *>(a.k) + b * a.k_bs + h * a.k_hs;
  const uint16_t *V = static_cast<const uint16_t *>(a.v) + b * a.v_bs + h * a.v_hs;
  uint16_t *O = static_cast<uint16_t *>(a.o) + b * a.o_bs + h * a.o_hs;
  const int64_t diag = (int64_t)a.N - (int64_t)a.M;  // key n visible to query m iff n <= m + diag

  const uint32_t qb0 = qt * kBQ;                    // block's first query
  const uint32_t q0 = qb0 + (uint32_t)wave * kQW;   // wave's first query
  const uint32_t lq = (uint32_t)(lane & 31), lh = (uint32_t)(lane >> 5);

  // Key tiles this block needs.
  uint32_t kend = a.N;
  if (CAUSAL) {
    const int64_t last_q = (int64_t)min(qb0 + kBQ, a.M) - 1;
    const int64_t lim = last_q + diag + 1;
    kend = lim <= 0 ? 0u : (uint32_t)min<int64_t>(lim, a.N);
  }
  const uint32_t nkt = (kend + kBKV - 1) / kBKV;

  // Q^T operands: lane holds query q0 + 32 g + lq, d = 16 ks + 8 lh .. +7.
  bf16x8_t qf[2][KS];
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const uint32_t qi = q0 + 32u * g + lq;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint4 v = make_uint4(0, 0, 0, 0);
      if (qi < a.M) v = *reinterpret_cast<const uint4 *>(Q + (size_t)qi * a.ldq + 16 * ks + 8 * lh);
      qf[g][ks] = __builtin_bit_cast(bf16x8_t, v);
    }
  }

  // DMA: each wave loads 4 of the 16 1-KiB blocks of the K tile and of the
  // V tile.  Rows past N re-read row N - 1 (finite data; masked to -inf).
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) unsigned char *)smem;
  auto issue = [&](uint32_t t) {
    const uint32_t st = lds0 + (t % kStages) * kStage;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t blk = (uint32_t)(wave * 4 + i);
      const uint32_t q = blk * 64u + (uint32_t)lane;  // 16-byte slot
      const uint32_t r = q >> 4, pc = q & 15u;
      uint32_t key = t * kBKV + r;
      key = key < a.N ? key : a.N - 1;
      g2lds16(K + (size_t)key * a.ldk + 8u * (pc ^ (r & 15u)), st + blk * 1024u);
      g2lds16(V + (size_t)key * a.ldv + 8u * (pc ^ (4u * (r & 3u))), st + kTile + blk * 1024u);
    }
  };

  f32x16_t o[2][DB];
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[g][d][r] = 0.0f;
  float mrow[2] = {-INFINITY, -INFINITY}, lrow[2] = {0.0f, 0.0f};

#pragma unroll
  for (int s = 0; s < kStages - 1; ++s)
    if ((uint32_t)s < nkt) issue((uint32_t)s);

  for (uint32_t t = 0; t < nkt; ++t) {
    if (t + 1 < nkt) wait_vmcnt<8>();  // tile t + 1 may still be in flight
    else wait_vmcnt<0>();
    __syncthreads();
    if (t + kStages - 1 < nkt) issue(t + kStages - 1);

    const uint32_t k0 = t * kBKV;
    // Whole tile masked for this wave's queries: nothing to do.
    if (CAUSAL && (int64_t)k0 > (int64_t)(q0 + kQW - 1) + diag) continue;
    const bool need_mask = (k0 + kBKV > a.N) || (CAUSAL && (int64_t)(k0 + kBKV - 1) > (int64_t)q0 + diag);

    const unsigned char *Ks = smem + (t % kStages) * kStage;
    const unsigned char *Vs = Ks + kTile;

    // S^T blocks: s[kb][g] = K[kb keys] . Q^T[g queries].
    f32x16_t s[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb][g][r] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint32_t row = 32u * kb + lq;
        const uint32_t c = 2u * ks + lh;
        const bf16x8_t kf = __builtin_bit_cast(bf16x8_t, *reinterpret_cast<const uint4 *>(Ks + k_off(row, c)));
#pragma unroll
        for (int g = 0; g < 2; ++g)
          s[kb][g] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[g][ks], s[kb][g], 0, 0, 0);
      }
    }

    // Online softmax per query (lane-local + partner lane ^ 32), in base 2:
    // the running max m is kept in scaled units (scale * log2 e * score),
    // p = exp2(score * c - m) is one FMA and one v_exp_f32.
    const float c = a.scale_log2;
#pragma unroll
    for (int g = 0; g < 2; ++g) {
      float mx = -INFINITY;
      // Key of register r in block kb is k0 + 4 lh + (32 kb + 8 (r >> 2) +
      // (r & 3)); visible iff that offset is below `lim` (key < N and, when
      // causal, key <= query + diag).
      int64_t lim64 = (int64_t)a.N - (int64_t)(k0 + 4u * lh);
      if (CAUSAL) {
        const int64_t c64 = (int64_t)(q0 + 32u * g + lq) + diag + 1 - (int64_t)(k0 + 4u * lh);
        lim64 = c64 < lim64 ? c64 : lim64;
      }
      const int lim = (int)(lim64 < -1 ? -1 : (lim64 > 64 ? 64 : lim64));
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float x = s[kb][g][r];
          if (need_mask) {
            x = (32 * kb + 8 * (r >> 2) + (r & 3)) < lim ? x : -INFINITY;
            s[kb][g][r] = x;
          }
          mx = fmaxf(mx, x);
        }
      }
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float mnew = fmaxf(mrow[g], mx * c);
      const float muse = mnew == -INFINITY ? 0.0f : mnew;
      const float alpha = __builtin_amdgcn_exp2f(mrow[g] - muse);
      mrow[g] = mnew;
      float sum = 0.0f;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kb][g][r], c, -muse));
          s[kb][g][r] = p;
          sum += p;
        }
      sum += __shfl_xor(sum, 32, 64);
      lrow[g] = lrow[g] * alpha + sum;
      // Rescale the output only when some query's maximum moved.
      if (__ballot(alpha != 1.0f)) {
#pragma unroll
        for (int d = 0; d < DB; ++d)
#pragma unroll
          for (int r = 0; r < 16; ++r) o[g][d][r] *= alpha;
      }
    }

    // O^T += V^T P^T over the 4 blocks of 16 keys.
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
      for (int kq = 0; kq < 2; ++kq) {
        bf16x8_t pf[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const f32x16_t &p = s[kb][g];
          const int r0 = 8 * kq;
          uint4 w;
          w.x = pack_bf16x2(p[r0 + 0], p[r0 + 1]);
          w.y = pack_bf16x2(p[r0 + 2], p[r0 + 3]);
          w.z = pack_bf16x2(p[r0 + 4], p[r0 + 5]);
          w.w = pack_bf16x2(p[r0 + 6], p[r0 + 7]);
          pf[g] = __builtin_bit_cast(bf16x8_t, w);
        }
        // Key rows of this lane's operand: 32 kb + 16 kq + 4 h (+8).
        const uint32_t grp = (uint32_t)((lane >> 4) & 3), L = (uint32_t)(lane & 15);
        const uint32_t kbase = 32u * kb + 16u * kq + 4u * (grp >> 1) + (L >> 2);
#pragma unroll
        for (int d = 0; d < DB; ++d) {
          const uint32_t col = 32u * d + 16u * (grp & 1u) + 4u * (L & 3u);
          const uint32_t c = col >> 3, sub = (col & 7u) * 2u;
          const v4s_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Vs + v_off(kbase, c) + sub));
          const v4s_t hi =
              __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s_t *)(Vs + v_off(kbase + 8u, c) + sub));
          const v8s_t vv = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
          const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, vv);
#pragma unroll
          for (int g = 0; g < 2; ++g)
            o[g][d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[g], o[g][d], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();

  // O = O^T / l, staged through LDS ([query][d] bf16 per wave), then stored
  // with 16-byte row chunks.
  uint16_t *os = reinterpret_cast<uint16_t *>(smem) + (size_t)wave * kQW * D;
#pragma unroll
  for (int g = 0; g < 2; ++g) {
    const float inv = lrow[g] > 0.0f ? 1.0f / lrow[g] : 0.0f;
    const uint32_t ql = 32u * g + lq;
#pragma unroll
    for (int d = 0; d < DB; ++d)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        const uint32_t dd = 32u * d + 8u * q4 + 4u * lh;
        uint2 w;
        w.x = pack_bf16x2(o[g][d][4 * q4 + 0] * inv, o[g][d][4 * q4 + 1] * inv);
        w.y = pack_bf16x2(o[g][d][4 * q4 + 2] * inv, o[g][d][4 * q4 + 3] * inv);
        *reinterpret_cast<uint2 *>(os + ql * D + dd) = w;
      }
  }
  __syncthreads();
  constexpr int kRowChunks = D / 8;
#pragma unroll 4
  for (int it = 0; it < kQW * kRowChunks / 64; ++it) {
    const int q = lane + it * 64;
    const uint32_t ql = (uint32_t)(q / kRowChunks), c = (uint32_t)(q % kRowChunks);
    const uint32_t qi = q0 + ql;
    if (qi < a.M)
      *reinterpret_cast<uint4 *>(O + (size_t)qi * a.ldo + 8u * c) =
          *reinterpret_cast<const uint4 *>(os + ql * D + 8u * c);
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
    __builtin_amdgcn_wave_barrier();
  }
}

}  // namespace

// Generic path entry points, one per storage type x mask.
#define BWPP_ATTN_GENERIC(NAME, T, CAUSAL)                                                  \
  extern "C" __global__ __launch_bounds__(256) void NAME(const BwppAttnArgs a) {            \
    attn_generic<T, CAUSAL>(a);                                                            \
  }
BWPP_ATTN_GENERIC(bwpp_attn_generic_f32, float, false)
BWPP_ATTN_GENERIC(bwpp_attn_generic_f32_causal, float, true)
BWPP_ATTN_GENERIC(bwpp_attn_generic_bf16, uint16_t, false)
BWPP_ATTN_GENERIC(bwpp_attn_generic_bf16_causal, uint16_t, true)

extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1))) void
bwpp_attn_bf16_d128(const BwppAttnArgs a) {
  attn_bf16_d128<false>(a);
}
extern "C" __global__ __attribute__((amdgpu_flat_work_group_size(256, 256), amdgpu_waves_per_eu(1, 1))) void
bwpp_attn_bf16_d128_causal(const BwppAttnArgs a) {
  attn_bf16_d128<true>(a);
}
