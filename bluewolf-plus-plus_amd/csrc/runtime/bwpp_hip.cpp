// libbwpp_hip host runtime: code-object loading, the kernel handle cache,
// argument validation, launch geometry and the device arena.
//
// Replaces runtime/metal/dispatch_stub.m.  Where the Metal stub compiles MSL
// at first dispatch and keeps one function-static PSO per op
// (dispatch_stub.m:6-56, 81), this layer loads prebuilt gfx950 code objects
// once per handle with hipModuleLoad and resolves every kernel symbol up
// front, so a missing kernel is an error at bwpp_hip_create() and never a
// silent no-op at dispatch time (dispatch_stub.m:94-98).
#include "bwpp_hip.h"
#include "internal.h"

#include <hip/hip_runtime_api.h>

#include <dlfcn.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cmath>
#include <cstring>
#include <initializer_list>
#include <string>
#include <unordered_map>
#include <vector>

#include "../kargs.h"

namespace {

thread_local std::string g_create_error;

// Code objects built by the package Makefile, all required.
const char *const kModules[] = {"bwpp_rowops.hsaco", "bwpp_gemm.hsaco", "bwpp_attention.hsaco",
                                 "bwpp_attention_f32.hsaco", "bwpp_attention_bwd.hsaco", "bwpp_grad.hsaco"};

// Row-op kernels: bwpp_row_<op>_v<VPT>_w<WPR>_<f|p>, see rowops.hip.
enum RowOpId { ROW_SOFTMAX, ROW_RMSNORM, ROW_LAYERNORM, ROW_MAX, ROW_MAXGRAD, ROW_MASK, ROW_NOPS };
const char *const kRowOpNames[ROW_NOPS] = {"softmax", "rmsnorm", "layernorm", "max", "maxgrad", "mask"};
// (float4 chunks per thread, waves per row); same list as BWPP_ROW_ALL_CFG.
struct RowCfg {
  int vpt;
  int wpr;
};
constexpr int kRowNCfg = 17;
const RowCfg kRowCfgs[kRowNCfg] = {{1, 1}, {2, 1}, {4, 1}, {8, 1}, {16, 1}, {2, 2}, {4, 2}, {8, 2}, {1, 4},
                                   {2, 4}, {4, 4}, {8, 4}, {16, 4}, {2, 8}, {4, 8}, {8, 8}, {16, 8}};
inline uint32_t row_capacity(const RowCfg &c) { return 256u * (uint32_t)c.wpr * (uint32_t)c.vpt; }
inline uint32_t row_block(const RowCfg &c) { return c.wpr >= 4 ? 64u * (uint32_t)c.wpr : 256u; }
inline uint32_t row_rows_per_block(const RowCfg &c) { return row_block(c) / (64u * (uint32_t)c.wpr); }
int find_cfg(int vpt, int wpr) {
  for (int i = 0; i < kRowNCfg; ++i)
    if (kRowCfgs[i].vpt == vpt && kRowCfgs[i].wpr == wpr) return i;
  return -1;
}

}  // namespace

struct BwppHip {
  int device = 0;
  int cus = 0;
  hipStream_t stream = nullptr;
  std::vector<hipModule_t> modules;
  std::unordered_map<hipFunction_t, uint32_t> max_threads;  // per resolved kernel
  std::unordered_map<hipFunction_t, std::string> names;     // symbol of each resolved kernel
  const std::string *last_kernel = nullptr;                 // symbol of the last launch
  const std::string *recent[4] = {};                        // the last four launches, newest first
  std::string err;
  int row_cfg_override = -1;  // BWPP_ROW_CFG: index into kRowCfgs (tuning)
  uint32_t row_grid_cap = 0;  // BWPP_ROW_GRID: max blocks per row launch (0 = per-op default)

  hipFunction_t row_reg[ROW_NOPS][kRowNCfg][2] = {};
  hipFunction_t row_gen[ROW_NOPS] = {};
  hipFunction_t row_maxgrad_idx = nullptr;
  hipFunction_t row_maxgrad_idx_v4 = nullptr;
  hipFunction_t row_maskgrad = nullptr;
  hipFunction_t col_maskgrad = nullptr;
  hipFunction_t col_max = nullptr;
  hipFunction_t col_maxgrad = nullptr;
  hipFunction_t col_mask = nullptr;
  // bwpp_gemm_<bf16|f32>_t<TA><TB>_<e|f>: [dtype][ta][tb][full]
  hipFunction_t gemm[2][2][2][2] = {};
  hipFunction_t gemm_bf16_w8[2][2] = {};  // 8-wave full-tile bf16: [ta][tb]
  hipFunction_t gemm_f32_split[2][2] = {};  // fp32 full tiles, split-K partials: [ta][tb]
  hipFunction_t gemm_f32p[2][2][2][2] = {};  // fp32 full tiles, DMA ring: [4-stage][ta][tb][split]
  hipFunction_t gemm_f32_reduce = nullptr;
  hipFunction_t attn_flash[2] = {};       // bf16, d = 128: [causal]
  hipFunction_t attn_flash_p[2] = {};     // bf16, d = 128, persistent (one block per CU): [causal]
  // BWPP_ATTN_FLASH_PERSIST: bit c set = persistent kernel when causal == c
  // (default unmasked only: causal C4 321.5 against 321.6 us, B2 H16 S4096
  // N 4096 +0.8 %, only B16 H16 S1024 -4.6 %).
  uint32_t attn_flash_persist = 1;
  hipFunction_t attn_generic[2][2] = {};  // [bf16][causal]
  hipFunction_t attn_bwd_dq[2][2] = {};   // [bf16][causal]
  hipFunction_t attn_bwd_dkdv[2][2] = {};
  // fp32 MFMA attention, head dim 64 / 128: [d128][causal]
  hipFunction_t attn_f32_fwd[2][2] = {}, attn_f32_dq[2][2] = {}, attn_f32_dkdv[2][2] = {};
  // bf16 MFMA attention backward, head dim 64 / 128: [d128][causal]
  hipFunction_t attn_bf16_dq[2][2] = {}, attn_bf16_dkdv[2][2] = {};
  hipFunction_t attn_bf16_dkdv_w8[2] = {};  // d = 128, 8 waves per block; [causal]
  uint32_t attn_w8_mask = 3u;  // BWPP_ATTN_BWD_W8: bit c set = 8-wave dK/dV pass allowed when causal == c
  // bf16 d = 128 backward with a stored dS (D_m pass, dK/dV pass storing
  // dS^T, dQ = dS K pass): [causal]
  hipFunction_t attn_bf16_dsum = nullptr, attn_bf16_dkdv_ds[2] = {}, attn_bf16_dkdv_w8_ds[2] = {},
                attn_bf16_dq_ds[2] = {};
  // The same for the fp32 matrix-core passes: [d128]; [d128][causal]
  hipFunction_t attn_f32_dsum[2] = {}, attn_f32_dkdv_ds[2][2] = {}, attn_f32_dq_ds[2][2] = {};
  uint64_t attn_ds_max = 8ull << 30;  // BWPP_ATTN_BWD_DS_MB: largest dS^T workspace in bytes (0: scheme off)
  hipFunction_t attn_conv_to_f32 = nullptr, attn_conv_to_bf16 = nullptr;  // bf16 <-> fp32 operand copies
  hipFunction_t rmsnorm_grad_w[4] = {};  // wave-per-row rmsnorm_grad, 256 / 512 / 1024 / 2048 columns
  hipFunction_t silu_grad = nullptr, softmax_grad = nullptr, rmsnorm_grad = nullptr, col_partials_sum = nullptr,
                reduce_sum_rows = nullptr, reduce_sum_cols = nullptr, elementwise = nullptr,
                mean_square_part = nullptr, mean_square_final = nullptr, copy_multi = nullptr;
  // Library-owned device workspace (column partials), grown on demand and
  // freed by bwpp_hip_destroy.  Calls on one handle are stream-ordered, so
  // reuse across calls is safe.
  void *ws = nullptr;
  size_t ws_bytes = 0;
  // Device address of this device's scratch array (bwpp_scratch.hip), for
  // the allocation-free entry point; NULL with scratch_why set if the
  // lookup failed.
  void *scratch = nullptr;
  std::string scratch_why;
  uint32_t gemm_group_m = 8;  // BWPP_GEMM_GROUP_M
  uint32_t gemm_waves = 8;    // BWPP_GEMM_WAVES: 4 or 8 waves for full bf16 tiles
  // bf16 256 x 384 tiles (8 waves), row-major A: [trans_b]
  hipFunction_t gemm_bf16_x384[2] = {};
  uint32_t gemm_bn = 0;  // BWPP_GEMM_BN: bf16 full-tile width 256 or 384 (0: chosen per shape)
  uint32_t gemm_splitk = 1;   // BWPP_GEMM_SPLITK=0 turns fp32 split-K off
  uint32_t attn_zigzag = 1;  // BWPP_ATTN_ZIGZAG=0: fp32 causal passes always heaviest-first
  uint32_t gemm_f32_pipe = 1;  // BWPP_GEMM_F32_PIPE: fp32 full tiles 0 staged, 1 auto, 2 ring4, 3 ring2
};

namespace {

BwppHipStatus fail(BwppHip *h, BwppHipStatus s, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (h)
    h->err = buf;
  else
    g_create_error = buf;
  return s;
}

}  // namespace

BwppHipStatus bwpp_hip_set_error(BwppHip *h, BwppHipStatus s, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (h)
    h->err = buf;
  else
    g_create_error = buf;
  return s;
}

const void *bwpp_hip_workspace(const BwppHip *h) { return h ? h->ws : nullptr; }

namespace {

BwppHipStatus resolve(BwppHip *h, const std::string &name, hipFunction_t *out) {
  for (hipModule_t m : h->modules) {
    hipFunction_t f = nullptr;
    if (hipModuleGetFunction(&f, m, name.c_str()) == hipSuccess && f) {
      // The block size each kernel was compiled for (its launch bounds):
      // launch() refuses larger blocks instead of running a kernel whose
      // indexing assumes fewer threads.
      int mt = 0;
      if (hipFuncGetAttribute(&mt, HIP_FUNC_ATTRIBUTE_MAX_THREADS_PER_BLOCK, f) != hipSuccess || mt <= 0)
        return fail(h, BWPP_HIP_ERR_HIP, "hipFuncGetAttribute(%s) failed", name.c_str());
      h->max_threads[f] = (uint32_t)mt;
      h->names[f] = name;
      *out = f;
      return BWPP_HIP_OK;
    }
    // A miss in one code object is expected; do not leave it as the
    // thread's last HIP error for the caller (or torch) to trip over.
    (void)hipGetLastError();
  }
  return fail(h, BWPP_HIP_ERR_NO_KERNEL, "kernel %s not found in any loaded code object", name.c_str());
}

BwppHipStatus resolve_all(BwppHip *h) {
  BwppHipStatus s;
  for (int op = 0; op < ROW_NOPS; ++op) {
    for (int c = 0; c < kRowNCfg; ++c) {
      for (int full = 0; full < 2; ++full) {
        std::string n = std::string("bwpp_row_") + kRowOpNames[op] + "_v" + std::to_string(kRowCfgs[c].vpt) +
                        "_w" + std::to_string(kRowCfgs[c].wpr) + (full ? "_f" : "_p");
        if ((s = resolve(h, n, &h->row_reg[op][c][full])) != BWPP_HIP_OK) return s;
      }
    }
    if ((s = resolve(h, std::string("bwpp_row_") + kRowOpNames[op] + "_gen", &h->row_gen[op])) != BWPP_HIP_OK)
      return s;
  }
  struct {
    const char *name;
    hipFunction_t *slot;
  } singles[] = {
      {"bwpp_row_maxgrad_idx", &h->row_maxgrad_idx}, {"bwpp_row_maxgrad_idx_v4", &h->row_maxgrad_idx_v4},
      {"bwpp_row_maskgrad", &h->row_maskgrad},       {"bwpp_col_maskgrad", &h->col_maskgrad},
      {"bwpp_col_max", &h->col_max},                 {"bwpp_col_maxgrad", &h->col_maxgrad},
      {"bwpp_col_mask", &h->col_mask},
      {"bwpp_silu_grad", &h->silu_grad},             {"bwpp_softmax_grad", &h->softmax_grad},
      {"bwpp_rmsnorm_grad", &h->rmsnorm_grad},       {"bwpp_col_partials_sum", &h->col_partials_sum},
      {"bwpp_reduce_sum_rows", &h->reduce_sum_rows}, {"bwpp_reduce_sum_cols", &h->reduce_sum_cols},
      {"bwpp_mean_square_part", &h->mean_square_part}, {"bwpp_mean_square_final", &h->mean_square_final},
      {"bwpp_copy_multi", &h->copy_multi},
      {"bwpp_elementwise", &h->elementwise},         {"bwpp_gemm_f32_splitk_reduce", &h->gemm_f32_reduce},
      {"bwpp_rmsnorm_grad_w1", &h->rmsnorm_grad_w[0]}, {"bwpp_rmsnorm_grad_w2", &h->rmsnorm_grad_w[1]},
      {"bwpp_rmsnorm_grad_w4", &h->rmsnorm_grad_w[2]}, {"bwpp_rmsnorm_grad_w8", &h->rmsnorm_grad_w[3]},
      {"bwpp_attn_conv_bf16_to_f32", &h->attn_conv_to_f32}, {"bwpp_attn_conv_f32_to_bf16", &h->attn_conv_to_bf16},
      {"bwpp_attn_bwd_bf16_mfma_d128_dkdv_w8", &h->attn_bf16_dkdv_w8[0]},
      {"bwpp_attn_bwd_bf16_mfma_d128_causal_dkdv_w8", &h->attn_bf16_dkdv_w8[1]},
      {"bwpp_attn_bwd_bf16_d128_dsum", &h->attn_bf16_dsum},
      {"bwpp_attn_bwd_f32_d64_dsum", &h->attn_f32_dsum[0]},
      {"bwpp_attn_bwd_f32_d128_dsum", &h->attn_f32_dsum[1]},
      {"bwpp_attn_bwd_f32_mfma_d64_dkdv_ds", &h->attn_f32_dkdv_ds[0][0]},
      {"bwpp_attn_bwd_f32_mfma_d64_causal_dkdv_ds", &h->attn_f32_dkdv_ds[0][1]},
      {"bwpp_attn_bwd_f32_mfma_d128_dkdv_ds", &h->attn_f32_dkdv_ds[1][0]},
      {"bwpp_attn_bwd_f32_mfma_d128_causal_dkdv_ds", &h->attn_f32_dkdv_ds[1][1]},
      {"bwpp_attn_bwd_f32_mfma_d64_dq_ds", &h->attn_f32_dq_ds[0][0]},
      {"bwpp_attn_bwd_f32_mfma_d64_causal_dq_ds", &h->attn_f32_dq_ds[0][1]},
      {"bwpp_attn_bwd_f32_mfma_d128_dq_ds", &h->attn_f32_dq_ds[1][0]},
      {"bwpp_attn_bwd_f32_mfma_d128_causal_dq_ds", &h->attn_f32_dq_ds[1][1]},
      {"bwpp_attn_bwd_bf16_mfma_d128_dkdv_ds", &h->attn_bf16_dkdv_ds[0]},
      {"bwpp_attn_bwd_bf16_mfma_d128_causal_dkdv_ds", &h->attn_bf16_dkdv_ds[1]},
      {"bwpp_attn_bwd_bf16_mfma_d128_dkdv_w8_ds", &h->attn_bf16_dkdv_w8_ds[0]},
      {"bwpp_attn_bwd_bf16_mfma_d128_causal_dkdv_w8_ds", &h->attn_bf16_dkdv_w8_ds[1]},
      {"bwpp_attn_bwd_bf16_mfma_d128_dq_ds", &h->attn_bf16_dq_ds[0]},
      {"bwpp_attn_bwd_bf16_mfma_d128_causal_dq_ds", &h->attn_bf16_dq_ds[1]},
  };
  for (auto &e : singles)
    if ((s = resolve(h, e.name, e.slot)) != BWPP_HIP_OK) return s;
  for (int dt = 0; dt < 2; ++dt)
    for (int ta = 0; ta < 2; ++ta)
      for (int tb = 0; tb < 2; ++tb)
        for (int full = 0; full < 2; ++full) {
          const std::string n = std::string("bwpp_gemm_") + (dt ? "bf16" : "f32") + "_t" + std::to_string(ta) +
                                std::to_string(tb) + (full ? "_f" : "_e");
          if ((s = resolve(h, n, &h->gemm[dt][ta][tb][full])) != BWPP_HIP_OK) return s;
        }
  for (int ta = 0; ta < 2; ++ta)
    for (int tb = 0; tb < 2; ++tb) {
      const std::string n = "bwpp_gemm_bf16w8_t" + std::to_string(ta) + std::to_string(tb) + "_f";
      if ((s = resolve(h, n, &h->gemm_bf16_w8[ta][tb])) != BWPP_HIP_OK) return s;
      if (ta == 0) {
        const std::string nx = "bwpp_gemm_bf16x384w8_t0" + std::to_string(tb) + "_f";
        if ((s = resolve(h, nx, &h->gemm_bf16_x384[tb])) != BWPP_HIP_OK) return s;
      }
      const std::string ns = std::string("bwpp_gemm_f32_t") + char('0' + ta) + char('0' + tb) + "_s";
      if ((s = resolve(h, ns, &h->gemm_f32_split[ta][tb])) != BWPP_HIP_OK) return s;
      for (int sp = 0; sp < 2; ++sp) {
        for (int q = 0; q < 2; ++q) {
          const std::string np = std::string(q ? "bwpp_gemm_f32q_t" : "bwpp_gemm_f32p_t") + char('0' + ta) +
                                 char('0' + tb) + (sp ? "_s" : "_f");
          if ((s = resolve(h, np, &h->gemm_f32p[q][ta][tb][sp])) != BWPP_HIP_OK) return s;
        }
      }
    }
  for (int causal = 0; causal < 2; ++causal) {
    const char *cs = causal ? "_causal" : "";
    if ((s = resolve(h, std::string("bwpp_attn_bf16_d128") + cs, &h->attn_flash[causal])) != BWPP_HIP_OK) return s;
    if ((s = resolve(h, std::string("bwpp_attn_bf16_d128") + cs + "_p", &h->attn_flash_p[causal])) != BWPP_HIP_OK)
      return s;
    if ((s = resolve(h, std::string("bwpp_attn_generic_f32") + cs, &h->attn_generic[0][causal])) != BWPP_HIP_OK)
      return s;
    if ((s = resolve(h, std::string("bwpp_attn_generic_bf16") + cs, &h->attn_generic[1][causal])) != BWPP_HIP_OK)
      return s;
    for (int d128 = 0; d128 < 2; ++d128) {
      const std::string dn = std::string(d128 ? "128" : "64") + cs;
      if ((s = resolve(h, "bwpp_attn_f32_mfma_d" + dn, &h->attn_f32_fwd[d128][causal])) != BWPP_HIP_OK) return s;
      if ((s = resolve(h, "bwpp_attn_bwd_f32_mfma_d" + dn + "_dq", &h->attn_f32_dq[d128][causal])) != BWPP_HIP_OK)
        return s;
      if ((s = resolve(h, "bwpp_attn_bwd_f32_mfma_d" + dn + "_dkdv", &h->attn_f32_dkdv[d128][causal])) !=
          BWPP_HIP_OK)
        return s;
      if ((s = resolve(h, "bwpp_attn_bwd_bf16_mfma_d" + dn + "_dq", &h->attn_bf16_dq[d128][causal])) != BWPP_HIP_OK)
        return s;
      if ((s = resolve(h, "bwpp_attn_bwd_bf16_mfma_d" + dn + "_dkdv", &h->attn_bf16_dkdv[d128][causal])) !=
          BWPP_HIP_OK)
        return s;
    }
    for (int bf = 0; bf < 2; ++bf) {
      const std::string base = std::string("bwpp_attn_bwd_") + (bf ? "bf16" : "f32") + cs;
      if ((s = resolve(h, base + "_dq", &h->attn_bwd_dq[bf][causal])) != BWPP_HIP_OK) return s;
      if ((s = resolve(h, base + "_dkdv", &h->attn_bwd_dkdv[bf][causal])) != BWPP_HIP_OK) return s;
    }
  }
  return BWPP_HIP_OK;
}

std::string library_dir() {
  Dl_info info;
  if (dladdr((void *)&bwpp_hip_create, &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t slash = p.rfind('/');
    if (slash != std::string::npos) return p.substr(0, slash);
  }
  return ".";
}

inline bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

BwppHipStatus enter(BwppHip *h) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  h->err.clear();
  hipError_t e = hipSetDevice(h->device);
  if (e != hipSuccess) return fail(h, BWPP_HIP_ERR_HIP, "hipSetDevice(%d): %s", h->device, hipGetErrorString(e));
  return BWPP_HIP_OK;
}

template <class Args>
BwppHipStatus launch(BwppHip *h, hipFunction_t f, uint32_t gx, uint32_t gy, uint32_t gz, uint32_t bx,
                     const Args &args, uint32_t shmem = 0) {
  if (gx == 0 || gy == 0 || gz == 0) return BWPP_HIP_OK;
  const auto mt = h->max_threads.find(f);
  if (mt == h->max_threads.end() || bx > mt->second)
    return fail(h, BWPP_HIP_ERR_HIP, "launch of %u threads per block exceeds the kernel's limit (%u)", bx,
                mt == h->max_threads.end() ? 0u : mt->second);
  void *params[] = {const_cast<Args *>(&args)};
  hipError_t e = hipModuleLaunchKernel(f, gx, gy, gz, bx, 1, 1, shmem, h->stream, params, nullptr);
  if (e != hipSuccess) return fail(h, BWPP_HIP_ERR_HIP, "hipModuleLaunchKernel: %s", hipGetErrorString(e));
  const auto nm = h->names.find(f);
  h->last_kernel = nm == h->names.end() ? nullptr : &nm->second;
  for (int i = 3; i > 0; --i) h->recent[i] = h->recent[i - 1];
  h->recent[0] = h->last_kernel;
  return BWPP_HIP_OK;
}

inline uint32_t eff_ld(uint32_t ld, uint32_t cols) { return ld ? ld : cols; }

// Picks the register-resident configuration for one operator on rows of
// `cols` floats, or -1 for the multi-pass fallback.  Rows up to 1024 get one
// wave each (no cross-wave reduction, no barrier), and so do the norms' and
// softmax's rows up to 1536; up to 2048 the norms and reduce_max take two
// waves, and up to 3072 the norms take two waves of 8 chunks.  Longer rows
// get a block of 4 waves or, where that measured faster, 8 (every operator
// above 16384 columns; softmax and RMSNorm from 4096, LayerNorm above
// 4096, the reduce_max gradient from 4096 to 8192; never reduce_max), with
// the float4 chunks per thread doubled until the row fits (<= 16, i.e.
// 32768 columns).  These are the fastest layouts measured on MI355X at 768
// - 16384 columns (one wave per row: RMSNorm over 4096 x 1024 9.2 -> 6.5
// us, LayerNorm over 4096 x 768 15.2 -> 7.0 us; eight waves instead of
// four, same bytes: RMSNorm 44.0 -> 43.5 / 46.7 -> 45.5 / 50.7 -> 45.8 us
// at 4096 / 8192 / 16384 columns, LayerNorm 47.5 -> 46.3 / 51.3 -> 46.3 at
// 8192 / 16384, the gradient 43.7 -> 43.0 / 45.0 -> 44.6 at 4096 / 8192
// but 47.5 -> 49.2 at 16384, reduce_max 21.0 -> 24.1 at 4096).
int pick_row_cfg(const BwppHip *h, RowOpId op, uint32_t cols, bool vec_ok) {
  if (!vec_ok) return -1;
  if (h->row_cfg_override >= 0 && h->row_cfg_override < kRowNCfg &&
      row_capacity(kRowCfgs[h->row_cfg_override]) >= cols)
    return h->row_cfg_override;
  if (cols <= 256) return find_cfg(1, 1);
  if (cols <= 512) return find_cfg(2, 1);
  if (cols <= 1024) return find_cfg(4, 1);
  const bool norm = op == ROW_RMSNORM || op == ROW_LAYERNORM;
  if (cols <= 1536 && (norm || op == ROW_SOFTMAX)) return find_cfg(8, 1);
  if (cols <= 2048 && op != ROW_SOFTMAX) return find_cfg(4, 2);
  if (cols <= 3072 && norm) return find_cfg(8, 2);
  if (cols > 32768) return -1;
  bool eight = cols > 16384;
  if (op == ROW_SOFTMAX || op == ROW_RMSNORM) eight = eight || cols >= 4096;
  if (op == ROW_LAYERNORM) eight = eight || cols > 4096;
  if (op == ROW_MAXGRAD) eight = eight || (cols >= 4096 && cols <= 8192);
  const int wpr = eight ? 8 : 4;
  int vpt = 1;
  while (row_capacity(RowCfg{vpt, wpr}) < cols) vpt *= 2;
  return find_cfg(vpt, wpr);
}

// Launches one row-wise (axis = last) operator.  The norms run a persistent
// grid of 2 blocks per CU (measured best of 1 / 2 / 4 / one per row) so each
// block reuses its gamma/beta registers over several rows; the others launch
// one block per row group.
BwppHipStatus row_dispatch(BwppHip *h, RowOpId op, const BwppRowArgs &a, bool vec_ok) {
  const int c = pick_row_cfg(h, op, a.cols, vec_ok);
  if (c < 0) return launch(h, h->row_gen[op], a.rows, 1, 1, 256, a);
  const RowCfg &cfg = kRowCfgs[c];
  const int full = (a.cols == row_capacity(cfg)) ? 1 : 0;
  const uint32_t rpb = row_rows_per_block(cfg);
  uint32_t grid = (a.rows + rpb - 1) / rpb;
  uint32_t cap = h->row_grid_cap;
  if (cap == 0 && (op == ROW_RMSNORM || op == ROW_LAYERNORM) && h->cus > 0) cap = 2u * (uint32_t)h->cus;
  if (cap && grid > cap) grid = cap;
  return launch(h, h->row_reg[op][c][full], grid, 1, 1, row_block(cfg), a);
}

inline uint32_t stream_grid(uint32_t rows) { return rows < (1u << 20) ? rows : (1u << 20); }

BwppHipStatus check_rows(BwppHip *h, uint32_t rows, uint32_t cols, uint32_t ld) {
  if (ld < cols) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "ld (%u) < cols (%u)", ld, cols);
  (void)rows;
  return BWPP_HIP_OK;
}

}  // namespace

extern "C" {

const char *bwpp_hip_status_string(BwppHipStatus s) {
  switch (s) {
    case BWPP_HIP_OK: return "ok";
    case BWPP_HIP_ERR: return "error";
    case BWPP_HIP_ERR_INVALID_ARG: return "invalid argument";
    case BWPP_HIP_ERR_HIP: return "HIP runtime error";
    case BWPP_HIP_ERR_NO_KERNEL: return "kernel or code object missing";
    case BWPP_HIP_ERR_ALIAS: return "output aliases an input";
    case BWPP_HIP_ERR_OUT_OF_MEMORY: return "out of device memory";
    case BWPP_HIP_ERR_UNSUPPORTED: return "unsupported";
    case BWPP_HIP_ERR_NO_DEVICE: return "no HIP device";
  }
  return "unknown status";
}

BwppHipStatus bwpp_hip_create(BwppHip **out, int device, const char *code_object_dir) {
  g_create_error.clear();
  if (!out) return fail(nullptr, BWPP_HIP_ERR_INVALID_ARG, "out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0)
    return fail(nullptr, BWPP_HIP_ERR_NO_DEVICE, "no HIP device (%s)", e == hipSuccess ? "count 0" : hipGetErrorString(e));
  if (device < 0 || device >= n)
    return fail(nullptr, BWPP_HIP_ERR_NO_DEVICE, "device %d out of range (%d devices)", device, n);
  if ((e = hipSetDevice(device)) != hipSuccess)
    return fail(nullptr, BWPP_HIP_ERR_HIP, "hipSetDevice(%d): %s", device, hipGetErrorString(e));

  BwppHip *h = new BwppHip();
  h->device = device;
  {
    const char *why = "";
    if (bwpp_hip_scratch_setup(device, &h->scratch, &why) != BWPP_HIP_OK) h->scratch_why = why;
  }
  (void)hipDeviceGetAttribute(&h->cus, hipDeviceAttributeMultiprocessorCount, device);
  if (const char *cfg = getenv("BWPP_ROW_CFG")) h->row_cfg_override = atoi(cfg);
  if (const char *gc = getenv("BWPP_ROW_GRID")) h->row_grid_cap = (uint32_t)strtoul(gc, nullptr, 10);
  if (const char *gw = getenv("BWPP_GEMM_WAVES")) h->gemm_waves = (uint32_t)strtoul(gw, nullptr, 10) == 4 ? 4 : 8;
  if (const char *bn = getenv("BWPP_GEMM_BN")) {
    const uint32_t v = (uint32_t)strtoul(bn, nullptr, 10);
    h->gemm_bn = v == 256 || v == 384 ? v : 0u;
  }
  if (const char *sk = getenv("BWPP_GEMM_SPLITK")) h->gemm_splitk = atoi(sk) != 0 ? 1u : 0u;
  if (const char *zz = getenv("BWPP_ATTN_ZIGZAG")) h->attn_zigzag = atoi(zz) != 0 ? 1u : 0u;
  if (const char *fp = getenv("BWPP_GEMM_F32_PIPE")) h->gemm_f32_pipe = (uint32_t)std::min(std::max(atoi(fp), 0), 3);
  if (const char *w8 = getenv("BWPP_ATTN_BWD_W8")) h->attn_w8_mask = (uint32_t)strtoul(w8, nullptr, 10) & 3u;
  if (const char *dm = getenv("BWPP_ATTN_BWD_DS_MB")) h->attn_ds_max = (uint64_t)strtoull(dm, nullptr, 10) << 20;
  if (const char *fp = getenv("BWPP_ATTN_FLASH_PERSIST")) h->attn_flash_persist = (uint32_t)strtoul(fp, nullptr, 10) & 3u;
  if (const char *gm = getenv("BWPP_GEMM_GROUP_M")) {
    const uint32_t v = (uint32_t)strtoul(gm, nullptr, 10);
    if (v > 0) h->gemm_group_m = v;
  }

  const std::string dir = code_object_dir ? std::string(code_object_dir) : library_dir();
  for (const char *mod : kModules) {
    const std::string path = dir + "/" + mod;
    hipModule_t m = nullptr;
    e = hipModuleLoad(&m, path.c_str());
    if (e != hipSuccess) {
      (void)hipGetLastError();
      bwpp_hip_destroy(h);
      return fail(nullptr, BWPP_HIP_ERR_NO_KERNEL, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    }
    h->modules.push_back(m);
  }
  BwppHipStatus s = resolve_all(h);
  if (s != BWPP_HIP_OK) {
    g_create_error = h->err;
    bwpp_hip_destroy(h);
    return s;
  }
  *out = h;
  return BWPP_HIP_OK;
}

void bwpp_hip_destroy(BwppHip *h) {
  if (!h) return;
  if (h->ws) {
    (void)hipSetDevice(h->device);
    (void)hipStreamSynchronize(h->stream);
    (void)hipFree(h->ws);
  }
  for (hipModule_t m : h->modules) (void)hipModuleUnload(m);
  delete h;
}

BwppHipStatus bwpp_hip_set_stream(BwppHip *h, void *hip_stream) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  const hipStream_t ns = (hipStream_t)hip_stream;
  if (ns == h->stream) return BWPP_HIP_OK;
  if (h->ws) {
    // The workspace (split-K partial planes, attention D rows, column
    // partials) is ordered on the handle's stream.  Work still queued on the
    // old stream may read or write it, so the new stream waits for that
    // work before anything launched on it can touch the workspace.
    BwppHipStatus s = enter(h);
    if (s != BWPP_HIP_OK) return s;
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    if (e == hipSuccess) e = hipEventRecord(ev, h->stream);
    if (e == hipSuccess) e = hipStreamWaitEvent(ns, ev, 0);
    if (ev) (void)hipEventDestroy(ev);
    if (e != hipSuccess) return fail(h, BWPP_HIP_ERR_HIP, "set_stream: ordering after the old stream: %s",
                                     hipGetErrorString(e));
  }
  h->stream = ns;
  return BWPP_HIP_OK;
}

void *bwpp_hip_get_stream(const BwppHip *h) { return h ? (void *)h->stream : nullptr; }

BwppHipStatus bwpp_hip_sync(BwppHip *h) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  hipError_t e = hipStreamSynchronize(h->stream);
  if (e != hipSuccess) return fail(h, BWPP_HIP_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
  return BWPP_HIP_OK;
}

const char *bwpp_hip_last_error(const BwppHip *h) { return h ? h->err.c_str() : g_create_error.c_str(); }

int bwpp_hip_device_cus(const BwppHip *h) { return h ? h->cus : 0; }

const char *bwpp_hip_last_kernel(const BwppHip *h) {
  return h && h->last_kernel ? h->last_kernel->c_str() : "";
}

const char *bwpp_hip_recent_kernel(const BwppHip *h, int back) {
  return h && back >= 0 && back < 4 && h->recent[back] ? h->recent[back]->c_str() : "";
}

// ---------------------------------------------------------------- memory

BwppHipStatus bwpp_hip_arena_init(BwppHip *h, BwppHipArena *arena, size_t capacity) {
  if (!arena) return BWPP_HIP_ERR_INVALID_ARG;
  arena->buffer = nullptr;
  arena->capacity = 0;
  arena->offset = 0;
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, capacity ? capacity : 1);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(h, BWPP_HIP_ERR_OUT_OF_MEMORY, "hipMalloc(%zu): %s", capacity, hipGetErrorString(e));
  }
  arena->buffer = (unsigned char *)p;
  arena->capacity = capacity;
  arena->offset = 0;
  arena->device = h->device;
  return BWPP_HIP_OK;
}

void bwpp_hip_arena_reset(BwppHipArena *arena) {
  if (arena) arena->offset = 0;
}

void *bwpp_hip_arena_alloc(BwppHipArena *arena, size_t size, size_t align) {
  if (!arena || !arena->buffer) return nullptr;
  if (align == 0) align = 1;
  if (align & (align - 1)) return nullptr;  // power of two only
  const size_t mask = align - 1;
  const uintptr_t base = (uintptr_t)arena->buffer;
  const size_t start = ((base + arena->offset + mask) & ~(uintptr_t)mask) - base;
  if (start > arena->capacity || size > arena->capacity - start) return nullptr;
  arena->offset = start + size;
  return arena->buffer + start;
}

void bwpp_hip_arena_destroy(BwppHipArena *arena) {
  if (!arena) return;
  if (arena->buffer) {
    (void)hipSetDevice(arena->device);
    (void)hipFree(arena->buffer);
  }
  arena->buffer = nullptr;
  arena->capacity = 0;
  arena->offset = 0;
}

static BwppHipStatus copy(BwppHip *h, void *dst, const void *src, size_t bytes, hipMemcpyKind kind) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (bytes == 0) return BWPP_HIP_OK;
  if (!dst || !src) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "NULL copy pointer");
  hipError_t e = hipMemcpyAsync(dst, src, bytes, kind, h->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(h->stream);
  if (e != hipSuccess) return fail(h, BWPP_HIP_ERR_HIP, "hipMemcpyAsync: %s", hipGetErrorString(e));
  return BWPP_HIP_OK;
}

BwppHipStatus bwpp_hip_copy_to_device(BwppHip *h, void *dst, const void *src, size_t bytes) {
  return copy(h, dst, src, bytes, hipMemcpyHostToDevice);
}

BwppHipStatus bwpp_hip_copy_to_host(BwppHip *h, void *dst, const void *src, size_t bytes) {
  return copy(h, dst, src, bytes, hipMemcpyDeviceToHost);
}

// ------------------------------------------------------------- row ops

BwppHipStatus bwpp_hip_dispatch_softmax(BwppHip *h, const float *x, float *y, BwppSoftmaxParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || !y) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "softmax: NULL x or y");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  BwppRowArgs a = {};
  a.x = x;
  a.y = y;
  a.rows = p.rows;
  a.cols = p.cols;
  a.ld = ld;
  const bool vec = aligned16(x) && aligned16(y) && (ld % 4 == 0);
  return row_dispatch(h, ROW_SOFTMAX, a, vec);
}

static BwppHipStatus norm_dispatch(BwppHip *h, RowOpId op, const float *x, const float *gamma, const float *beta,
                                   float *y, BwppRmsnormParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || !y) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "%s: NULL x or y", kRowOpNames[op]);
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  BwppRowArgs a = {};
  a.x = x;
  a.y = y;
  a.gamma = gamma;
  a.beta = beta;
  a.rows = p.rows;
  a.cols = p.cols;
  a.ld = ld;
  a.eps = p.eps;
  const bool vec = aligned16(x) && aligned16(y) && (ld % 4 == 0) && (!gamma || aligned16(gamma)) &&
                   (!beta || aligned16(beta));
  return row_dispatch(h, op, a, vec);
}

BwppHipStatus bwpp_hip_dispatch_rmsnorm(BwppHip *h, const float *x, const float *gamma, const float *beta,
                                        float *y, BwppRmsnormParams p) {
  return norm_dispatch(h, ROW_RMSNORM, x, gamma, beta, y, p);
}

BwppHipStatus bwpp_hip_dispatch_layernorm(BwppHip *h, const float *x, const float *gamma, const float *beta,
                                          float *y, BwppRmsnormParams p) {
  return norm_dispatch(h, ROW_LAYERNORM, x, gamma, beta, y, p);
}

BwppHipStatus bwpp_hip_dispatch_reduce_max(BwppHip *h, const float *x, float *maxv, int32_t *argmax,
                                           BwppReduceParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || (!maxv && !argmax)) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "reduce_max: NULL x or both outputs NULL");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  BwppRowArgs a = {};
  a.x = x;
  a.maxv = maxv;
  a.argmax = argmax;
  a.rows = p.rows;
  a.cols = p.cols;
  a.ld = ld;
  if (p.axis == 0) {
    if (p.cols == 0) return BWPP_HIP_OK;
    return launch(h, h->col_max, (p.cols + 255) / 256, 1, 1, 256, a);
  }
  if (p.rows == 0) return BWPP_HIP_OK;
  if (p.cols == 0) return launch(h, h->row_gen[ROW_MAX], p.rows, 1, 1, 256, a);
  return row_dispatch(h, ROW_MAX, a, aligned16(x) && (ld % 4 == 0));
}

BwppHipStatus bwpp_hip_dispatch_reduce_max_mask(BwppHip *h, const float *x, float *mask, BwppReduceParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || !mask) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "reduce_max_mask: NULL x or mask");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  BwppRowArgs a = {};
  a.x = x;
  a.y = mask;
  a.rows = p.rows;
  a.cols = p.cols;
  a.ld = ld;
  if (p.axis == 0) return launch(h, h->col_mask, (p.cols + 255) / 256, 1, 1, 256, a);
  return row_dispatch(h, ROW_MASK, a, aligned16(x) && aligned16(mask) && (ld % 4 == 0));
}

BwppHipStatus bwpp_hip_dispatch_reduce_max_grad(BwppHip *h, const float *mask, const float *dy, float *dx,
                                                BwppReduceParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!mask || !dy || !dx) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "reduce_max_grad: NULL mask, dy or dx");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  BwppRowArgs a = {};
  a.x = mask;
  a.dy = dy;
  a.y = dx;
  a.rows = p.rows;
  a.cols = p.cols;
  a.ld = ld;
  return launch(h, p.axis == 0 ? h->col_maskgrad : h->row_maskgrad, stream_grid(p.rows), 1, 1, 256, a);
}

BwppHipStatus bwpp_hip_dispatch_reduce_max_grad_argmax(BwppHip *h, const float *x, const int32_t *argmax,
                                                       const float *dy, float *dx, BwppReduceParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if ((!x && !argmax) || !dy || !dx)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "reduce_max_grad_argmax: need x or argmax, and dy, dx");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  BwppRowArgs a = {};
  a.x = x;
  a.idx_in = argmax;
  a.dy = dy;
  a.y = dx;
  a.rows = p.rows;
  a.cols = p.cols;
  a.ld = ld;
  if (p.axis == 0) return launch(h, h->col_maxgrad, (p.cols + 255) / 256, 1, 1, 256, a);
  if (argmax) {
    const bool vec = aligned16(dx) && (ld % 4 == 0);
    return launch(h, vec ? h->row_maxgrad_idx_v4 : h->row_maxgrad_idx, stream_grid(p.rows), 1, 1, 256, a);
  }
  return row_dispatch(h, ROW_MAXGRAD, a, aligned16(x) && aligned16(dx) && (ld % 4 == 0));
}

}  // extern "C"

// ------------------------------------------------------------- matmul

namespace {

// Byte range [lo, hi) of a row-major matrix view.
struct Extent {
  uintptr_t lo = 0, hi = 0;
};
Extent extent(const void *p, uint64_t rows, uint64_t cols, uint64_t ld, uint64_t es) {
  Extent e;
  if (!p || rows == 0 || cols == 0) return e;
  e.lo = (uintptr_t)p;
  e.hi = e.lo + ((rows - 1) * ld + cols) * es;
  return e;
}
bool overlaps(const Extent &a, const Extent &b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; }

// Whether two row-strided blocks of es-byte elements share an element:
// exact when their row strides are equal (column blocks of one wider
// matrix interleave without touching), by byte range otherwise.
bool blocks_overlap(const void *pa, uint64_t ra, uint64_t ca, uint64_t lda, const void *pb, uint64_t rb, uint64_t cb,
                    uint64_t ldb, uint64_t es) {
  if (!overlaps(extent(pa, ra, ca, lda, es), extent(pb, rb, cb, ldb, es))) return false;
  if (lda != ldb || lda == 0) return true;
  intptr_t db = (intptr_t)pb - (intptr_t)pa;
  if (db % (intptr_t)es) return true;
  int64_t d = db / (intptr_t)es;  // b's first element, in elements from a's
  if (d < 0) {                    // make a the earlier block
    d = -d;
    std::swap(ra, rb);
    std::swap(ca, cb);
  }
  const uint64_t ld = lda, q = (uint64_t)d / ld, r = (uint64_t)d % ld;
  // b's row i covers columns [r, r + cb) of a's row q + i, spilling into
  // columns [0, r + cb - ld) of row q + i + 1 when r + cb > ld.
  auto rows_meet = [&](uint64_t first, uint64_t count) { return count > 0 && first < ra; };
  if (r < ca && rows_meet(q, rb)) return true;
  if (r + cb > ld && rows_meet(q + 1, rb)) return true;
  return false;
}

BwppHipStatus ensure_ws(BwppHip *h, size_t bytes);

}  // namespace

namespace {

BwppHipStatus matmul_impl(BwppHip *h, const void *a, const void *b, void *c, const void *bias, BwppMatmulParams p,
                          const float *aux, float *c2, BwppHipFusionParams fz) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!a || !b || !c) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: NULL a, b or c");
  if (p.dtype > BWPP_HIP_BF16) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: unknown dtype %u", p.dtype);
  if (p.epilogue > BWPP_HIP_EPILOGUE_ADD_SILU)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: unknown epilogue %u", p.epilogue);
  const bool ta = p.trans_a != 0, tb = p.trans_b != 0;
  const uint32_t a_cols = ta ? p.M : p.K, b_cols = tb ? p.K : p.N;
  const uint32_t lda = p.lda ? p.lda : a_cols, ldb = p.ldb ? p.ldb : b_cols, ldc = p.ldc ? p.ldc : p.N;
  if (lda < a_cols || ldb < b_cols || ldc < p.N)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: leading dimension smaller than the row (lda %u ldb %u ldc %u)",
                lda, ldb, ldc);
  if (p.M == 0 || p.N == 0) return BWPP_HIP_OK;
  const bool bf16 = p.dtype == BWPP_HIP_BF16;
  const uint64_t es = bf16 ? 2 : 4;
  const Extent ec = extent(c, p.M, p.N, ldc, es);
  const Extent ea = extent(a, ta ? p.K : p.M, a_cols, lda, es);
  const Extent eb = extent(b, tb ? p.N : p.K, b_cols, ldb, es);
  const bool use_bias = (p.epilogue & BWPP_HIP_EPILOGUE_ADD) && bias;
  const Extent ebias = use_bias ? extent(bias, 1, p.N, p.N, es) : Extent{};
  if (overlaps(ec, ea) || overlaps(ec, eb) || overlaps(ec, ebias))
    return fail(h, BWPP_HIP_ERR_ALIAS, "matmul: C overlaps A, B or bias");
  // Fused tail: fp32 only; aux (residual / SiLU input) and c2 (dual output).
  const uint32_t fuse = fz.kind;
  const bool use_aux = fuse == BWPP_HIP_FUSE_RESIDUAL || fuse == BWPP_HIP_FUSE_SILU_GRAD;
  const uint32_t ldaux = fz.ld_aux ? fz.ld_aux : p.N, ldc2 = fz.ld_c2 ? fz.ld_c2 : p.N;
  if (fuse != BWPP_HIP_FUSE_NONE) {
    if (fuse > BWPP_HIP_FUSE_SILU_GRAD) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: unknown fusion %u", fuse);
    if (bf16) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "matmul: fused tails run on fp32 only");
    if (use_aux && (!aux || ldaux < p.N)) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: fusion needs aux (ld >= N)");
    if (fuse == BWPP_HIP_FUSE_DUAL_SILU && (!c2 || ldc2 < p.N))
      return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: dual output needs c2 (ld >= N)");
    if (fuse == BWPP_HIP_FUSE_DUAL_SILU && (p.epilogue & BWPP_HIP_EPILOGUE_SILU))
      return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: the dual output takes SiLU of a result without SiLU");
    if (fuse == BWPP_HIP_FUSE_SILU_GRAD && p.epilogue != BWPP_HIP_EPILOGUE_NONE)
      return fail(h, BWPP_HIP_ERR_INVALID_ARG, "matmul: the SiLU gradient tail takes no epilogue");
    const Extent eaux = use_aux ? extent(aux, p.M, p.N, ldaux, 4) : Extent{};
    const Extent ec2 = fuse == BWPP_HIP_FUSE_DUAL_SILU ? extent(c2, p.M, p.N, ldc2, 4) : Extent{};
    // aux may be C itself (each element is read and written by one thread)
    const bool aux_is_c = use_aux && (const void *)aux == c && ldaux == ldc;
    if ((use_aux && !aux_is_c && overlaps(ec, eaux)) || overlaps(ec2, ea) || overlaps(ec2, eb) ||
        overlaps(ec2, ebias) || overlaps(ec2, ec) || overlaps(ec2, eaux))
      return fail(h, BWPP_HIP_ERR_ALIAS, "matmul: c2 or aux overlaps another operand");
  }

  // Full-tile kernels: bf16 256 x 256 with K in steps of 32 (pipelined),
  // fp32 128 x 128 with K in steps of 32; anything else takes the guarded
  // edge kernels.
  const uint32_t BM = bf16 ? 256 : 128, BN = bf16 ? 256 : 128, BK = 32;
  const uint32_t vecw = bf16 ? 8 : 4;  // elements per 16 bytes
  const bool vec = aligned16(a) && aligned16(b) && aligned16(c) && lda % vecw == 0 && ldb % vecw == 0 &&
                   ldc % vecw == 0 && (!use_aux || (aligned16(aux) && ldaux % 4 == 0)) &&
                   (fuse != BWPP_HIP_FUSE_DUAL_SILU || (aligned16(c2) && ldc2 % 4 == 0));
  // The full-tile kernels also fetch the bias row with 16-byte copies.
  const bool full = vec && (!use_bias || aligned16(bias)) && p.M % BM == 0 && p.N % BN == 0 && p.K % BK == 0;
  BwppGemmArgs g = {};
  g.a = a;
  g.b = b;
  g.bias = use_bias ? bias : nullptr;
  g.c = c;
  g.M = p.M;
  g.N = p.N;
  g.K = p.K;
  g.lda = lda;
  g.ldb = ldb;
  g.ldc = ldc;
  g.epilogue = p.epilogue;
  g.tiles_m = (p.M + BM - 1) / BM;
  g.tiles_n = (p.N + BN - 1) / BN;
  g.group_m = h->gemm_group_m;
  g.vec_ok = vec ? 1u : 0u;
  g.fuse = fuse;
  g.aux = use_aux ? aux : nullptr;
  g.ldaux = ldaux;
  g.c2 = fuse == BWPP_HIP_FUSE_DUAL_SILU ? c2 : nullptr;
  g.ldc2 = ldc2;
  const uint64_t tiles = (uint64_t)g.tiles_m * g.tiles_n;
  if (tiles > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "matmul: too many tiles");
  // bf16 256 x 384 tiles: N a multiple of 8 (a tile column that overhangs
  // N re-reads B's last columns and stores only n < N); the DMA addresses
  // are 32-bit offsets from each tile's origin.  On C3 they run even with
  // the 256 x 256 kernel (a higher clock, less matrix-pipe busy time), so
  // they are taken where that one cannot run -- N not a multiple of 256,
  // which would otherwise go to the register-staged edge kernel -- or when
  // BWPP_GEMM_BN=384 asks.
  const bool wide_ok = bf16 && !ta && vec && (!use_bias || aligned16(bias)) && p.M % BM == 0 && p.K % BK == 0 &&
                       p.N % 8 == 0 && h->gemm_waves == 8 && 384ull * 2ull * std::max(lda, ldb) < (1ull << 31);
  if (wide_ok && (h->gemm_bn == 384 || (h->gemm_bn == 0 && p.N % BN != 0))) {
    g.tiles_n = (p.N + 383) / 384;
    const uint64_t wt = (uint64_t)g.tiles_m * g.tiles_n;
    return launch(h, h->gemm_bf16_x384[tb], (uint32_t)wt, 1, 1, 512, g);
  }
  if (bf16 && full && h->gemm_waves == 8)
    return launch(h, h->gemm_bf16_w8[ta][tb], (uint32_t)tiles, 1, 1, 512, g);
  // fp32 full tiles: one of three kernels, optionally with K split into S
  // ranges (multiples of BK) whose raw partial tiles a reduce pass adds in
  // order, applying the epilogue and the fused tail:
  //   ring2 (bwpp_gemm_f32p): LDS-DMA ring, 2 stages, two blocks per CU;
  //   ring4 (bwpp_gemm_f32q): LDS-DMA ring, 4 stages, one block per CU;
  //   staged (bwpp_gemm_f32): register-staged double buffer, two blocks per
  //     CU (BWPP_GEMM_F32_PIPE=0 only; the rings beat it on every measured
  //     full-tile shape).
  // A launch of b blocks runs in waves of blocks, each taking time
  // proportional to its K range.  The choice minimises
  //   ring4:  ceil(b / cus) (k t4 + o4)
  //   ring2:  floor(b / (2 cus)) k t2 + o4, plus for a last partial wave
  //           k t1 when it holds at most one block per CU (such a block
  //           has its CU to itself), else k t2      (staged: t2 = 0.13)
  // plus (2 S - 1) M N 4 / bw + t_r when split (S - 1 more planes written
  // and S read by the reduce), with t4 = 0.064 us, t2 = 0.119 us and t1 =
  // 0.065 us per k of a 128 x 128 block, o4 = 3 us per block (the prologue
  // and epilogue, which one block per CU does not overlap), bw = 6 TB/s,
  // t_r = 2 us; fitted on MI355X to the twelve GEMMs of the C5 block step
  // (from 1024 x 1024 x 4096 to 4096 x 4096 x 1024, with and without split)
  // and checked on 2048^3 and 8192^3.
  if (!bf16 && full) {
    const int mode = (int)h->gemm_f32_pipe;  // 0 staged, 1 auto, 2 ring4, 3 ring2
    const uint64_t cus = h->cus > 0 ? (uint64_t)h->cus : 256ull;
    auto cost = [&](int kind, uint64_t S, uint32_t kchunk) {  // kind: 0 staged, 1 ring2, 2 ring4
      const uint64_t b = tiles * S;
      double t;
      if (kind == 2) {
        t = (double)((b + cus - 1) / cus) * (kchunk * 0.064 + 3.0);
      } else {
        const double tk = kind ? 0.119 : 0.13;
        const uint64_t full = b / (2 * cus), rem = b % (2 * cus);
        t = (double)full * kchunk * tk + 3.0;
        if (rem > 0) t += kchunk * (rem <= cus ? 0.065 : tk);
      }
      if (S > 1) t += (double)(2 * S - 1) * p.M * p.N * 4.0 / 6e6 + 2.0;
      return t;
    };
    int bestKind = mode == 0 ? 0 : mode == 3 ? 1 : 2;
    uint64_t bestS = 1;
    uint32_t bestChunk = p.K;
    double best = 1e300;
    for (int kind = 0; kind < 3; ++kind) {
      if (mode == 0 ? kind != 0 : mode == 1 ? kind == 0 : kind != bestKind) continue;
      for (uint64_t S = 1; S <= 16 && p.K / S >= BK; ++S) {
        if (S > 1 && !h->gemm_splitk) break;
        const uint32_t kchunk = (uint32_t)(((p.K + S - 1) / S + BK - 1) / BK * BK);
        const uint64_t Se = (p.K + kchunk - 1) / kchunk;
        if (Se != S) continue;
        const double c = cost(kind, Se, kchunk);
        if (c < best) {
          best = c;
          bestKind = kind;
          bestS = Se;
          bestChunk = kchunk;
        }
      }
    }
    const int ring4 = bestKind == 2;
    if (bestS > 1) {
      if ((s = ensure_ws(h, (size_t)bestS * p.M * p.N * sizeof(float))) != BWPP_HIP_OK) return s;
      g.ksplit = (uint32_t)bestS;
      g.kchunk = bestChunk;
      g.part = static_cast<float *>(h->ws);
      if ((s = launch(h, bestKind ? h->gemm_f32p[ring4][ta][tb][1] : h->gemm_f32_split[ta][tb],
                      (uint32_t)(tiles * bestS), 1, 1, 256, g)) != BWPP_HIP_OK)
        return s;
      const uint64_t vecs = (uint64_t)p.M * (p.N / 4);
      const uint64_t grid = std::min<uint64_t>((vecs + 255) / 256, 8ull * cus);
      return launch(h, h->gemm_f32_reduce, (uint32_t)grid, 1, 1, 256, g);
    }
    if (bestKind) return launch(h, h->gemm_f32p[ring4][ta][tb][0], (uint32_t)tiles, 1, 1, 256, g);
  }
  return launch(h, h->gemm[bf16 ? 1 : 0][ta][tb][full ? 1 : 0], (uint32_t)tiles, 1, 1, 256, g);
}

}  // namespace

extern "C" BwppHipStatus bwpp_hip_dispatch_matmul(BwppHip *h, const void *a, const void *b, void *c,
                                                  const void *bias, BwppMatmulParams p) {
  return matmul_impl(h, a, b, c, bias, p, nullptr, nullptr, BwppHipFusionParams{});
}

extern "C" BwppHipStatus bwpp_hip_dispatch_matmul_fused(BwppHip *h, const void *a, const void *b, void *c,
                                                        const void *bias, const float *aux, float *c2,
                                                        BwppMatmulParams p, BwppHipFusionParams f) {
  return matmul_impl(h, a, b, c, bias, p, aux, c2, f);
}

namespace {

BwppHipStatus ensure_ws(BwppHip *h, size_t bytes);

// Validation, default strides and the kernel argument block shared by the
// attention entry points.  `out` is O for the forward (checked against
// Q, K, V for overlap); the backward checks its outputs itself.
BwppHipStatus attn_prepare(BwppHip *h, const void *q, const void *k, const void *v, const void *o,
                           const BwppAttentionParams &p, BwppAttnArgs &g, uint64_t &slices, bool &skip,
                           bool forward = true) {
  skip = false;
  if (!q || !k || !v || !o) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "attention: NULL q, k, v or o");
  if (p.dtype > BWPP_HIP_BF16) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "attention: unknown dtype %u", p.dtype);
  const uint32_t B = p.batch ? p.batch : 1, H = p.heads ? p.heads : 1;
  const uint32_t ldq = p.ldq ? p.ldq : p.K, ldk = p.ldk ? p.ldk : p.K;
  const uint32_t ldv = p.ldv ? p.ldv : p.D, ldo = p.ldo ? p.ldo : p.D;
  if (ldq < p.K || ldk < p.K || ldv < p.D || ldo < p.D)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "attention: leading dimension smaller than the row");
  if (forward && (p.M == 0 || p.D == 0)) {
    skip = true;
    return BWPP_HIP_OK;
  }
  if (p.K == 0 || p.K > 512 || p.D > 512)
    return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention: head dims K=%u D=%u outside 1..512", p.K, p.D);
  const uint64_t es = p.dtype == BWPP_HIP_BF16 ? 2 : 4;
  // Default slice strides: [B, H, rows, ld] contiguous.
  auto def = [](uint64_t st, uint64_t dflt) { return st ? st : dflt; };
  const uint64_t q_hs = def(p.q_head_stride, (uint64_t)p.M * ldq), q_bs = def(p.q_batch_stride, q_hs * H);
  const uint64_t k_hs = def(p.k_head_stride, (uint64_t)p.N * ldk), k_bs = def(p.k_batch_stride, k_hs * H);
  const uint64_t v_hs = def(p.v_head_stride, (uint64_t)p.N * ldv), v_bs = def(p.v_batch_stride, v_hs * H);
  const uint64_t o_hs = def(p.o_head_stride, (uint64_t)p.M * ldo), o_bs = def(p.o_batch_stride, o_hs * H);
  // Byte hull of each tensor over all slices; O must not meet Q, K or V.
  auto hull = [&](const void *ptr, uint64_t bs, uint64_t hs, uint64_t rows, uint64_t cols, uint64_t ld) {
    Extent e;
    if (rows == 0 || cols == 0) return e;
    e.lo = (uintptr_t)ptr;
    e.hi = e.lo + ((uint64_t)(B - 1) * bs + (uint64_t)(H - 1) * hs + (rows - 1) * ld + cols) * es;
    return e;
  };
  const Extent eo = hull(o, o_bs, o_hs, p.M, p.D, ldo);
  if (overlaps(eo, hull(q, q_bs, q_hs, p.M, p.K, ldq)) || overlaps(eo, hull(k, k_bs, k_hs, p.N, p.K, ldk)) ||
      overlaps(eo, hull(v, v_bs, v_hs, p.N, p.D, ldv)))
    return fail(h, BWPP_HIP_ERR_ALIAS, "attention: O overlaps Q, K or V");
  g = BwppAttnArgs{};
  g.q = q;
  g.k = k;
  g.v = v;
  g.o = const_cast<void *>(o);
  g.M = p.M;
  g.N = p.N;
  g.ldq = ldq;
  g.ldk = ldk;
  g.ldv = ldv;
  g.ldo = ldo;
  g.heads = H;
  g.q_bs = q_bs;
  g.q_hs = q_hs;
  g.k_bs = k_bs;
  g.k_hs = k_hs;
  g.v_bs = v_bs;
  g.v_hs = v_hs;
  g.o_bs = o_bs;
  g.o_hs = o_hs;
  g.causal = p.causal ? 1u : 0u;
  g.kdim = p.K;
  g.vdim = p.D;
  slices = (uint64_t)B * H;
  return BWPP_HIP_OK;
}

// Variant of the fp32 MFMA attention kernels for these arguments (0: head
// dim 64, 1: 128), or -1 for the generic path: they need K = D in {64, 128},
// a finite scale and 16-byte rows (pointers, leading dims and slice strides
// in multiples of 4 floats).
// fp32 MFMA causal passes: zigzag tile order when the grid is resident in
// one go at two blocks per CU (more than one block per CU, at most two),
// so the dispatcher's pairing of block b with b + grid / 2 on a CU joins a
// heavy tile with a light one (forward, C5: 512 blocks on 256 CUs, 63 -> 58
// us; B2 H16 S2048 d64: 234 -> 190 us; backward, with both passes at two
// waves per SIMD: C5 187 -> 165 us, B2 H16 S2048 d64 686 -> 529 us).
uint32_t attn_zigzag(const BwppHip *h, bool causal, uint64_t grid) {
  return causal && h->attn_zigzag && h->cus > 0 && grid > (uint64_t)h->cus && grid <= 2ull * (uint64_t)h->cus ? 1u
                                                                                                                : 0u;
}

int attn_f32_variant(const BwppAttentionParams &p, const BwppAttnArgs &g, float scale,
                     std::initializer_list<const void *> ptrs) {
  if (p.dtype != BWPP_HIP_F32 || p.K != p.D || (p.K != 64 && p.K != 128) || !std::isfinite(scale)) return -1;
  for (const void *x : ptrs)
    if (!aligned16(x)) return -1;
  for (uint64_t v : {(uint64_t)g.ldq, (uint64_t)g.ldk, (uint64_t)g.ldv, (uint64_t)g.ldo, g.q_bs, g.q_hs, g.k_bs,
                     g.k_hs, g.v_bs, g.v_hs, g.o_bs, g.o_hs})
    if (v % 4 != 0) return -1;
  return p.K == 128 ? 1 : 0;
}

// Variant of the bf16 MFMA attention backward for these arguments (0: head
// dim 64, 1: 128), or -1: K = D in {64, 128}, a finite scale and 16-byte
// rows (pointers, leading dims and slice strides in multiples of 8 bf16).
int attn_bf16_bwd_variant(const BwppAttentionParams &p, const BwppAttnArgs &g, float scale,
                          std::initializer_list<const void *> ptrs) {
  if (p.dtype != BWPP_HIP_BF16 || p.K != p.D || (p.K != 64 && p.K != 128) || !std::isfinite(scale)) return -1;
  for (const void *x : ptrs)
    if (!aligned16(x)) return -1;
  for (uint64_t v : {(uint64_t)g.ldq, (uint64_t)g.ldk, (uint64_t)g.ldv, (uint64_t)g.ldo, g.q_bs, g.q_hs, g.k_bs,
                     g.k_hs, g.v_bs, g.v_hs, g.o_bs, g.o_hs})
    if (v % 8 != 0) return -1;
  return p.K == 128 ? 1 : 0;
}

constexpr uint32_t kAttnWaves = 4;  // waves (32 rows each) per block of the MFMA attention kernels

BwppHipStatus attn_forward(BwppHip *h, const void *q, const void *k, const void *v, void *o, float *lse,
                           const BwppAttentionParams &p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  BwppAttnArgs g;
  uint64_t slices = 0;
  bool skip = false;
  if ((s = attn_prepare(h, q, k, v, o, p, g, slices, skip)) != BWPP_HIP_OK || skip) return s;
  const float scale = p.scale != 0.0f ? p.scale : 1.0f;
  const int causal = p.causal ? 1 : 0;
  const bool bf16 = p.dtype == BWPP_HIP_BF16;
  // The flash kernel takes the row maximum of the raw scores and scales it
  // afterwards, which needs a positive scale (finite: NaN / inf go generic).
  const bool flash = bf16 && p.K == 128 && p.D == 128 && p.N > 0 && scale > 0.0f && scale < INFINITY &&
                     aligned16(q) && aligned16(k) && aligned16(v) && aligned16(o) && g.ldq % 8 == 0 &&
                     g.ldk % 8 == 0 && g.ldv % 8 == 0 && g.ldo % 8 == 0 && g.q_bs % 8 == 0 && g.q_hs % 8 == 0 &&
                     g.k_bs % 8 == 0 && g.k_hs % 8 == 0 && g.v_bs % 8 == 0 && g.v_hs % 8 == 0 &&
                     g.o_bs % 8 == 0 && g.o_hs % 8 == 0 &&
                     // K / V byte offsets inside a slice are 32-bit in the kernel
                     (uint64_t)(p.N - 1) * g.ldk + p.K < (1ull << 31) &&
                     (uint64_t)(p.N - 1) * g.ldv + p.D < (1ull << 31);
  if (flash) {
    g.scale_log2 = scale * 1.4426950408889634f;
    g.lse = lse;
    g.q_tiles = (p.M + 255) / 256;
    // Causal blocks take two query tiles each (the longest with the shortest).
    const uint64_t grid = slices * (causal ? (g.q_tiles + 1) / 2 : g.q_tiles);
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention: grid too large");
    if (((h->attn_flash_persist >> causal) & 1u) && h->cus > 0 && grid > (uint64_t)h->cus) {
      // One block per CU working through the items (causal: tile pairs).
      g.items = (uint32_t)grid;
      return launch(h, h->attn_flash_p[causal], (uint32_t)h->cus, 1, 1, 512, g);
    }
    return launch(h, h->attn_flash[causal], (uint32_t)grid, 1, 1, 512, g);
  }
  const int f32v = attn_f32_variant(p, g, scale, {q, k, v, o});
  if (f32v >= 0) {
    g.scale = scale;
    g.scale_log2 = scale * 1.4426950408889634f;
    g.lse = lse;
    g.q_tiles = (p.M + 32 * kAttnWaves - 1) / (32 * kAttnWaves);
    const uint64_t grid = slices * g.q_tiles;
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention: grid too large");
    g.zigzag = attn_zigzag(h, causal != 0, grid);
    return launch(h, h->attn_f32_fwd[f32v][causal], (uint32_t)grid, 1, 1, 64 * kAttnWaves, g);
  }
  g.scale_log2 = scale;
  g.lse = lse;
  g.q_tiles = (p.M + 15) / 16;
  const uint64_t grid = slices * g.q_tiles;
  if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention: grid too large");
  return launch(h, h->attn_generic[bf16 ? 1 : 0][causal], (uint32_t)grid, 1, 1, 256, g);
}

}  // namespace

extern "C" BwppHipStatus bwpp_hip_dispatch_attention(BwppHip *h, const void *q, const void *k, const void *v,
                                                     void *o, BwppAttentionParams p) {
  return attn_forward(h, q, k, v, o, nullptr, p);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_attention_lse(BwppHip *h, const void *q, const void *k, const void *v,
                                                         void *o, float *lse, BwppAttentionParams p) {
  if (!lse && h) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "attention_lse: NULL lse");
  return attn_forward(h, q, k, v, o, lse, p);
}

namespace {
BwppHipStatus attn_grad_impl(BwppHip *h, const void *q, const void *k, const void *v, const void *o,
                             const void *dout, const float *lse, void *dq, void *dk, void *dv,
                             const BwppAttentionParams &p, bool check_alias, float *dsum_buf = nullptr,
                             size_t dsum_cap = 0);
}  // namespace

extern "C" BwppHipStatus bwpp_hip_dispatch_attention_grad(BwppHip *h, const void *q, const void *k, const void *v,
                                                          const void *o, const void *dout, const float *lse,
                                                          void *dq, void *dk, void *dv, BwppAttentionParams p) {
  return attn_grad_impl(h, q, k, v, o, dout, lse, dq, dk, dv, p, true);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_attention_grad_noalloc(BwppHip *h, const void *q, const void *k,
                                                                  const void *v, const void *o, const void *dout,
                                                                  const float *lse, void *dq, void *dk, void *dv,
                                                                  BwppAttentionParams p) {
  if (!h) return BWPP_HIP_ERR_INVALID_ARG;
  if (!h->scratch)
    return fail(h, BWPP_HIP_ERR_HIP, "attention_grad_noalloc: device scratch unavailable (%s)", h->scratch_why.c_str());
  return attn_grad_impl(h, q, k, v, o, dout, lse, dq, dk, dv, p, true, static_cast<float *>(h->scratch),
                        BWPP_HIP_NOALLOC_SCRATCH_BYTES);
}

BwppHipStatus bwpp_hip_attention_grad_planned(BwppHip *h, const void *q, const void *k, const void *v,
                                              const void *o, const void *dout, const float *lse, void *dq,
                                              void *dk, void *dv, const BwppAttentionParams &p) {
  return attn_grad_impl(h, q, k, v, o, dout, lse, dq, dk, dv, p, false);
}

namespace {
// dsum_buf (the allocation-free entry point): caller-provided device memory
// of dsum_cap bytes for the per-query row sums instead of the handle's
// workspace; paths that need more workspace than that are refused.
BwppHipStatus attn_grad_impl(BwppHip *h, const void *q, const void *k, const void *v, const void *o,
                             const void *dout, const float *lse, void *dq, void *dk, void *dv,
                             const BwppAttentionParams &p, bool check_alias, float *dsum_buf, size_t dsum_cap) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!dout || !lse || !dq || !dk || !dv)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "attention_grad: NULL dout, lse, dq, dk or dv");
  BwppAttnArgs g;
  uint64_t slices = 0;
  bool skip = false;
  if ((s = attn_prepare(h, q, k, v, o, p, g, slices, skip, false)) != BWPP_HIP_OK) return s;
  if (p.M == 0 && p.N == 0) return BWPP_HIP_OK;
  const uint32_t B = p.batch ? p.batch : 1, H = p.heads ? p.heads : 1;
  const uint64_t es = p.dtype == BWPP_HIP_BF16 ? 2 : 4;
  auto hull = [&](const void *ptr, uint64_t bs, uint64_t hs, uint64_t rows, uint64_t cols, uint64_t ld) {
    Extent e;
    if (rows == 0 || cols == 0) return e;
    e.lo = (uintptr_t)ptr;
    e.hi = e.lo + ((uint64_t)(B - 1) * bs + (uint64_t)(H - 1) * hs + (rows - 1) * ld + cols) * es;
    return e;
  };
  const Extent eq = hull(q, g.q_bs, g.q_hs, p.M, p.K, g.ldq), ek = hull(k, g.k_bs, g.k_hs, p.N, p.K, g.ldk);
  const Extent ev = hull(v, g.v_bs, g.v_hs, p.N, p.D, g.ldv), eo = hull(o, g.o_bs, g.o_hs, p.M, p.D, g.ldo);
  const Extent edo = hull(dout, g.o_bs, g.o_hs, p.M, p.D, g.ldo);
  const Extent edq = hull(dq, g.q_bs, g.q_hs, p.M, p.K, g.ldq), edk = hull(dk, g.k_bs, g.k_hs, p.N, p.K, g.ldk);
  const Extent edv = hull(dv, g.v_bs, g.v_hs, p.N, p.D, g.ldv);
  const Extent else_{(uintptr_t)lse, (uintptr_t)lse + slices * p.M * 4};
  if (check_alias) {
    for (const Extent &out : {edq, edk, edv})
      for (const Extent &in : {eq, ek, ev, eo, edo, else_})
        if (overlaps(out, in)) return fail(h, BWPP_HIP_ERR_ALIAS, "attention_grad: an output overlaps an input");
    if (overlaps(edq, edk) || overlaps(edq, edv) || overlaps(edk, edv))
      return fail(h, BWPP_HIP_ERR_ALIAS, "attention_grad: dq, dk and dv overlap");
  }
  const size_t dsum_bytes = (size_t)slices * p.M * sizeof(float) + 4;
  const int bf = p.dtype == BWPP_HIP_BF16 ? 1 : 0, causal = p.causal ? 1 : 0;
  const float scale = p.scale != 0.0f ? p.scale : 1.0f;
  const int bf16v = attn_bf16_bwd_variant(p, g, scale, {q, k, v, o, dout, dq, dk, dv});
  const int f32v = attn_f32_variant(p, g, scale, {q, k, v, o, dout, dq, dk, dv});
  // Stored-dS scheme (bf16 with d = 128, or the fp32 passes; not the
  // allocation-free entry): the dK / dV pass also stores dS^T (bf16 in
  // 2 KiB / fp32 in 4 KiB blocks of 32 keys x 32 queries, keys padded to 32,
  // queries to whole 128-query blocks: ld_dst) and the dQ pass only
  // multiplies it by K, so S and dP are computed once instead of in both
  // passes.  It needs es * B*H * ceil32(N) * ld_dst bytes of workspace, up
  // to attn_ds_max.
  const uint64_t ld_dst = ((uint64_t)p.M + 127ull) / 128ull * 128ull;
  const uint64_t ds_off = ((uint64_t)dsum_bytes + 255ull) & ~255ull;
  const uint64_t ds_bytes = slices * (((uint64_t)p.N + 31ull) / 32ull * 32ull) * ld_dst * (f32v >= 0 ? 4ull : 2ull);
  bool use_ds = !dsum_buf && (bf16v == 1 || f32v >= 0) && p.M > 0 && p.N > 0 && ds_bytes <= h->attn_ds_max &&
                ld_dst <= 0xffffffffull;
  if (dsum_buf) {
    if (dsum_bytes > dsum_cap)
      return fail(h, BWPP_HIP_ERR_UNSUPPORTED,
                  "attention_grad_noalloc: batch*heads*M = %llu query rows need %zu bytes of scratch, above the "
                  "%zu-byte maximum", (unsigned long long)(slices * p.M), dsum_bytes, dsum_cap);
  } else {
    // A stored-dS workspace the device cannot give: recompute S and dP
    // instead (the same results), with only the row sums in the workspace.
    if (use_ds && (s = ensure_ws(h, (size_t)(ds_off + ds_bytes))) != BWPP_HIP_OK) {
      if (s != BWPP_HIP_ERR_OUT_OF_MEMORY) return s;
      use_ds = false;
      h->err.clear();
    }
    if (!use_ds && (s = ensure_ws(h, dsum_bytes)) != BWPP_HIP_OK) return s;
  }
  g.scale_log2 = scale;
  g.lse = const_cast<float *>(lse);
  g.dout = dout;
  g.dq = dq;
  g.dk = dk;
  g.dv = dv;
  g.dsum = dsum_buf ? dsum_buf : static_cast<float *>(h->ws);
  // Matrix-core passes of the recompute scheme (fp32 or bf16 kernels): dQ
  // (also writes D_m = rowsum(dO * O)), then dK / dV.  wq / wk: waves (32
  // rows each) per block of the dQ / dK-dV kernel, as each was compiled.
  auto run_mfma = [&](BwppAttnArgs f, hipFunction_t fdq, hipFunction_t fdkdv, uint32_t wq = kAttnWaves,
                      uint32_t wk = kAttnWaves) -> BwppHipStatus {
    f.scale = scale;
    f.scale_log2 = scale * 1.4426950408889634f;
    f.q_tiles = (p.M + 32 * wq - 1) / (32 * wq);
    uint64_t grid = slices * f.q_tiles;
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    BwppHipStatus st;
    f.zigzag = attn_zigzag(h, causal != 0, grid);  // read by the fp32 passes
    if (p.M > 0 && (st = launch(h, fdq, (uint32_t)grid, 1, 1, 64 * wq, f)) != BWPP_HIP_OK) return st;
    f.q_tiles = (p.N + 32 * wk - 1) / (32 * wk);  // key tiles
    grid = slices * f.q_tiles;
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    f.zigzag = attn_zigzag(h, causal != 0, grid);
    if (p.N > 0) return launch(h, fdkdv, (uint32_t)grid, 1, 1, 64 * wk, f);
    return BWPP_HIP_OK;
  };
  if (use_ds && f32v >= 0) {
    BwppAttnArgs f = g;
    f.scale = scale;
    f.scale_log2 = scale * 1.4426950408889634f;
    f.dst = static_cast<unsigned char *>(h->ws) + ds_off;
    f.ld_dst = (uint32_t)ld_dst;
    f.q_tiles = (p.M + 32 * kAttnWaves - 1) / (32 * kAttnWaves);
    const uint64_t grid = slices * f.q_tiles;
    f.q_tiles = (p.N + 32 * kAttnWaves - 1) / (32 * kAttnWaves);  // key tiles
    const uint64_t kgrid = slices * f.q_tiles;
    if (grid > 0x7fffffffull || kgrid > 0x7fffffffull)
      return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    f.q_tiles = (p.M + 32 * kAttnWaves - 1) / (32 * kAttnWaves);
    if ((s = launch(h, h->attn_f32_dsum[f32v], (uint32_t)grid, 1, 1, 64 * kAttnWaves, f)) != BWPP_HIP_OK) return s;
    BwppAttnArgs fk = f;
    fk.q_tiles = (p.N + 32 * kAttnWaves - 1) / (32 * kAttnWaves);
    fk.zigzag = attn_zigzag(h, causal != 0, kgrid);
    if ((s = launch(h, h->attn_f32_dkdv_ds[f32v][causal], (uint32_t)kgrid, 1, 1, 64 * kAttnWaves, fk)) != BWPP_HIP_OK)
      return s;
    f.zigzag = attn_zigzag(h, causal != 0, grid);
    return launch(h, h->attn_f32_dq_ds[f32v][causal], (uint32_t)grid, 1, 1, 64 * kAttnWaves, f);
  }
  if (f32v >= 0)
    return run_mfma(g, h->attn_f32_dq[f32v][causal], h->attn_f32_dkdv[f32v][causal]);
  if (use_ds) {
    BwppAttnArgs f = g;
    f.scale = scale;
    f.scale_log2 = scale * 1.4426950408889634f;
    f.dst = static_cast<unsigned char *>(h->ws) + ds_off;
    f.ld_dst = (uint32_t)ld_dst;
    f.q_tiles = (p.M + 127) / 128;  // 4-wave blocks of the D_m and dQ passes
    uint64_t grid = slices * f.q_tiles;
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    if ((s = launch(h, h->attn_bf16_dsum, (uint32_t)grid, 1, 1, 256, f)) != BWPP_HIP_OK) return s;
    const bool w8 = ((h->attn_w8_mask >> causal) & 1u) && slices * ((p.N + 255ull) / 256ull) >= (uint64_t)h->cus;
    const uint32_t wk = w8 ? 8u : kAttnWaves;
    BwppAttnArgs fk = f;
    fk.q_tiles = (p.N + 32 * wk - 1) / (32 * wk);  // key tiles
    const uint64_t kgrid = slices * fk.q_tiles;
    if (kgrid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    if ((s = launch(h, w8 ? h->attn_bf16_dkdv_w8_ds[causal] : h->attn_bf16_dkdv_ds[causal], (uint32_t)kgrid, 1,
                        1, 64 * wk, fk)) != BWPP_HIP_OK)
      return s;
    return launch(h, h->attn_bf16_dq_ds[causal], (uint32_t)grid, 1, 1, 256, f);
  }
  if (bf16v >= 0) {
    // d = 128: the dK/dV pass with 8 waves (256 keys) per block (one block
    // per CU) when that grid still gives every CU a block; below that the
    // 4-wave pass's twice as many blocks win (B2 H8 S1000: 90 against
    // 102 us unmasked, 112 against 130 causal).
    const uint64_t w8_blocks = slices * ((p.N + 255ull) / 256ull);
    if (bf16v == 1 && ((h->attn_w8_mask >> causal) & 1u) && w8_blocks >= (uint64_t)h->cus)
      return run_mfma(g, h->attn_bf16_dq[1][causal], h->attn_bf16_dkdv_w8[causal], kAttnWaves, 8);
    return run_mfma(g, h->attn_bf16_dq[bf16v][causal], h->attn_bf16_dkdv[bf16v][causal]);
  }
  if (bf && p.K == p.D && (p.K == 64 || p.K == 128) && std::isfinite(scale)) {
    // bf16 with head dim 64 / 128 whose rows are not 16-byte aligned: fp32
    // copies of Q, K, V, O, dO in the workspace go through the fp32
    // matrix-core passes, and dQ, dK, dV are rounded back into the caller's
    // bf16 layout.
    const uint64_t D = p.D, nq = slices * p.M * D, nk = slices * p.N * D;
    if (dsum_buf)
      return fail(h, BWPP_HIP_ERR_UNSUPPORTED,
                  "attention_grad_noalloc: bf16 rows that are not 16-byte aligned need fp32 copies in the "
                  "handle's workspace; use bwpp_hip_dispatch_attention_grad");
    if ((s = ensure_ws(h, (4 * nq + 4 * nk + slices * p.M) * sizeof(float))) != BWPP_HIP_OK) return s;
    float *w = static_cast<float *>(h->ws);
    float *q32 = w, *o32 = q32 + nq, *do32 = o32 + nq, *dq32 = do32 + nq;
    float *k32 = dq32 + nq, *v32 = k32 + nk, *dk32 = v32 + nk, *dv32 = dk32 + nk, *ds32 = dv32 + nk;
    auto conv = [&](const void *src, void *dst, uint32_t rows, uint32_t ld, uint64_t bs, uint64_t hs,
                    bool to_bf16) -> BwppHipStatus {
      if (rows == 0) return BWPP_HIP_OK;
      BwppConvArgs c = {};
      c.src = src;
      c.dst = dst;
      c.bs = bs;
      c.hs = hs;
      c.rows = rows;
      c.cols = (uint32_t)D;
      c.ld = ld;
      c.heads = H;
      c.slices = (uint32_t)slices;
      c.vec = (aligned16(to_bf16 ? dst : src) && ld % 8 == 0 && bs % 8 == 0 && hs % 8 == 0) ? 1u : 0u;
      const uint64_t total = slices * rows * (D / 8);
      const uint64_t grid = std::min<uint64_t>((total + 255) / 256, h->cus > 0 ? 8ull * (uint64_t)h->cus : 2048ull);
      return launch(h, to_bf16 ? h->attn_conv_to_bf16 : h->attn_conv_to_f32, (uint32_t)grid, 1, 1, 256, c);
    };
    if ((s = conv(q, q32, p.M, g.ldq, g.q_bs, g.q_hs, false)) != BWPP_HIP_OK ||
        (s = conv(k, k32, p.N, g.ldk, g.k_bs, g.k_hs, false)) != BWPP_HIP_OK ||
        (s = conv(v, v32, p.N, g.ldv, g.v_bs, g.v_hs, false)) != BWPP_HIP_OK ||
        (s = conv(o, o32, p.M, g.ldo, g.o_bs, g.o_hs, false)) != BWPP_HIP_OK ||
        (s = conv(dout, do32, p.M, g.ldo, g.o_bs, g.o_hs, false)) != BWPP_HIP_OK)
      return s;
    BwppAttnArgs f = g;
    f.q = q32;
    f.k = k32;
    f.v = v32;
    f.o = o32;
    f.dout = do32;
    f.dq = dq32;
    f.dk = dk32;
    f.dv = dv32;
    f.dsum = ds32;
    f.ldq = f.ldk = f.ldv = f.ldo = (uint32_t)D;
    f.q_hs = f.o_hs = p.M * D;
    f.q_bs = f.o_bs = (uint64_t)H * p.M * D;
    f.k_hs = f.v_hs = p.N * D;
    f.k_bs = f.v_bs = (uint64_t)H * p.N * D;
    const int dv128 = D == 128 ? 1 : 0;
    if ((s = run_mfma(f, h->attn_f32_dq[dv128][causal], h->attn_f32_dkdv[dv128][causal])) != BWPP_HIP_OK) return s;
    if ((s = conv(dq32, dq, p.M, g.ldq, g.q_bs, g.q_hs, true)) != BWPP_HIP_OK ||
        (s = conv(dk32, dk, p.N, g.ldk, g.k_bs, g.k_hs, true)) != BWPP_HIP_OK)
      return s;
    return conv(dv32, dv, p.N, g.ldv, g.v_bs, g.v_hs, true);
  }
  if (p.M > 0) {
    g.q_tiles = (p.M + 15) / 16;
    const uint64_t grid = slices * g.q_tiles;
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    if ((s = launch(h, h->attn_bwd_dq[bf][causal], (uint32_t)grid, 1, 1, 256, g)) != BWPP_HIP_OK) return s;
  }
  if (p.N > 0) {
    g.q_tiles = (p.N + 15) / 16;  // key tiles
    const uint64_t grid = slices * g.q_tiles;
    if (grid > 0x7fffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "attention_grad: grid too large");
    if ((s = launch(h, h->attn_bwd_dkdv[bf][causal], (uint32_t)grid, 1, 1, 256, g)) != BWPP_HIP_OK) return s;
  }
  return BWPP_HIP_OK;
}
}  // namespace

// ------------------------------------------------------------- grad ops

namespace {

// Ensures the handle's workspace holds `bytes`; waits for queued work on the
// handle's stream before replacing a smaller buffer.
BwppHipStatus ensure_ws(BwppHip *h, size_t bytes) {
  if (h->ws_bytes >= bytes) return BWPP_HIP_OK;
  if (h->ws) {
    hipError_t e = hipStreamSynchronize(h->stream);
    if (e != hipSuccess) return fail(h, BWPP_HIP_ERR_HIP, "hipStreamSynchronize: %s", hipGetErrorString(e));
    (void)hipFree(h->ws);
    h->ws = nullptr;
    h->ws_bytes = 0;
  }
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, bytes);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(h, BWPP_HIP_ERR_OUT_OF_MEMORY, "workspace hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  }
  h->ws = p;
  h->ws_bytes = bytes;
  return BWPP_HIP_OK;
}

uint32_t row_grid(const BwppHip *h, uint32_t rows) {
  const uint32_t cap = h->cus > 0 ? 8u * (uint32_t)h->cus : 2048u;
  return rows < cap ? rows : cap;
}

// bwpp_elementwise over rows x cols: a / out with row stride ld, b (when
// full) with ldb.  The 128-bit path needs 16-byte rows and pointers.
BwppHipStatus elementwise_launch(BwppHip *h, const float *a, const float *b, uint32_t ldb, float *out, uint32_t ld,
                                 uint32_t rows, uint32_t cols, uint32_t op, uint32_t bmode) {
  auto a16 = [](const void *q) { return ((uintptr_t)q & 15u) == 0; };
  BwppGradArgs g = {};
  g.a = a;
  g.b = b;
  g.out = out;
  g.rows = rows;
  g.cols = cols;
  g.ld = ld;
  g.ldb = ldb;
  g.op = op;
  g.bmode = bmode;
  g.vec = cols % 4 == 0 && ld % 4 == 0 && a16(out) && (!a || a16(a)) &&
                  (bmode == BWPP_HIP_BCAST_COL || bmode == BWPP_HIP_BCAST_SCALAR || a16(b)) &&
                  (bmode != BWPP_HIP_BCAST_FULL || ldb % 4 == 0)
              ? 1u
              : 0u;
  return launch(h, h->elementwise, row_grid(h, rows), 1, 1, 256, g);
}

}  // namespace

extern "C" BwppHipStatus bwpp_hip_dispatch_silu_grad(BwppHip *h, const float *x, const float *dy, float *dx,
                                                     uint64_t n) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || !dy || !dx) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "silu_grad: NULL pointer");
  if (n == 0) return BWPP_HIP_OK;
  BwppGradArgs g = {};
  g.a = x;
  g.b = dy;
  g.out = dx;
  g.n = n;
  g.vec = (aligned16(x) && aligned16(dy) && aligned16(dx)) ? 1u : 0u;
  const uint64_t items = g.vec ? (n + 3) / 4 : n;
  const uint64_t blocks = (items + 255) / 256;
  return launch(h, h->silu_grad, (uint32_t)(blocks < 65536 ? blocks : 65536), 1, 1, 256, g);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_softmax_grad(BwppHip *h, const float *y, const float *dy, float *dx,
                                                        BwppSoftmaxParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!y || !dy || !dx) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "softmax_grad: NULL pointer");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  BwppGradArgs g = {};
  g.a = y;
  g.b = dy;
  g.out = dx;
  g.rows = p.rows;
  g.cols = p.cols;
  g.ld = ld;
  return launch(h, h->softmax_grad, row_grid(h, p.rows), 1, 1, 256, g);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_rmsnorm_grad(BwppHip *h, const float *x, const float *gamma,
                                                        const float *dy, float *dx, float *dgamma, float *dbeta,
                                                        BwppRmsnormParams p) {
  return bwpp_hip_dispatch_rmsnorm_grad_acc(h, x, gamma, dy, nullptr, dx, dgamma, dbeta, p);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_rmsnorm_grad_acc(BwppHip *h, const float *x, const float *gamma,
                                                            const float *dy, const float *acc, float *dx,
                                                            float *dgamma, float *dbeta, BwppRmsnormParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || !dy || !dx) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "rmsnorm_grad: NULL x, dy or dx");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.cols == 0) return BWPP_HIP_OK;
  if (acc && acc != dx && overlaps(extent(acc, p.rows, p.cols, ld, 4), extent(dx, p.rows, p.cols, ld, 4)))
    return fail(h, BWPP_HIP_ERR_ALIAS, "rmsnorm_grad: acc overlaps dx without being dx");
  const bool parts = dgamma || dbeta;
  if (parts && p.cols > 8192)
    return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "rmsnorm_grad: dgamma/dbeta need cols <= 8192 (got %u)", p.cols);
  BwppGradArgs g = {};
  g.a = x;
  g.b = dy;
  g.gamma = gamma;
  g.out = dx;
  g.acc = acc;
  g.rows = p.rows;
  g.cols = p.cols;
  g.ld = ld;
  g.eps = p.eps;
  // With column partials, at most kMaxParts blocks (each loops over its
  // rows), which bounds the partial arrays to kMaxParts rows.
  constexpr uint32_t kMaxParts = 512;
  // 16-byte rows of at most 2048 columns: one wave per row (no block
  // barriers in the row loop), 4 rows per block per trip.
  int wv = -1;
  if (p.cols <= 2048 && p.cols % 4 == 0 && ld % 4 == 0 && aligned16(x) && aligned16(dy) && aligned16(dx) &&
      (!gamma || aligned16(gamma)) && (!acc || aligned16(acc)))
    wv = p.cols <= 256 ? 0 : p.cols <= 512 ? 1 : p.cols <= 1024 ? 2 : 3;
  uint32_t grid;
  if (wv >= 0) {
    const uint32_t cap = parts ? kMaxParts : (h->cus > 0 ? 8u * (uint32_t)h->cus : 2048u);
    grid = p.rows == 0 ? 1u : std::min<uint32_t>((p.rows + 3) / 4, cap);
  } else {
    grid = p.rows == 0 ? 1u : row_grid(h, p.rows);
    if (parts && grid > kMaxParts) grid = kMaxParts;
  }
  if (parts) {
    if ((s = ensure_ws(h, (size_t)2 * grid * p.cols * sizeof(float))) != BWPP_HIP_OK) return s;
    g.part_g = static_cast<float *>(h->ws);
    g.part_b = g.part_g + (size_t)grid * p.cols;
  }
  if (p.rows > 0 || parts) {
    s = wv >= 0 ? launch(h, h->rmsnorm_grad_w[wv], grid, 1, 1, 256, g, parts ? 8u * p.cols * 4u : 0u)
                : launch(h, h->rmsnorm_grad, grid, 1, 1, 256, g, parts ? 2u * p.cols * 4u : 0u);
    if (s != BWPP_HIP_OK) return s;
  }
  if (!parts) return BWPP_HIP_OK;
  BwppGradArgs r = {};
  r.part_g = g.part_g;
  r.part_b = g.part_b;
  r.out = dgamma;
  r.out2 = dbeta;
  r.cols = p.cols;
  r.nparts = grid;
  return launch(h, h->col_partials_sum, (p.cols + 15) / 16, 1, 1, 256, r);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_reduce_sum(BwppHip *h, const float *x, float *out, BwppReduceParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || !out) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "reduce_sum: NULL pointer");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  BwppGradArgs g = {};
  g.a = x;
  g.out = out;
  g.rows = p.rows;
  g.cols = p.cols;
  g.ld = ld;
  if (p.axis != 0) {
    if (p.rows == 0) return BWPP_HIP_OK;
    return launch(h, h->reduce_sum_rows, row_grid(h, p.rows), 1, 1, 256, g);
  }
  if (p.cols == 0) return BWPP_HIP_OK;
  const uint32_t bands = p.rows == 0 ? 1u : (p.rows < 64u ? p.rows : 64u);
  if ((s = ensure_ws(h, (size_t)bands * p.cols * sizeof(float))) != BWPP_HIP_OK) return s;
  g.part_g = static_cast<float *>(h->ws);
  if ((s = launch(h, h->reduce_sum_cols, (p.cols + 255) / 256, bands, 1, 256, g)) != BWPP_HIP_OK) return s;
  BwppGradArgs r = {};
  r.part_g = g.part_g;
  r.part_b = g.part_g;
  r.out = out;
  r.cols = p.cols;
  r.nparts = bands;
  return launch(h, h->col_partials_sum, (p.cols + 15) / 16, 1, 1, 256, r);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_mean_square(BwppHip *h, const float *x, const float *loss_scale,
                                                       const float *grad_scale, float *loss, float *dx,
                                                       BwppMeanSquareParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!x || (!loss && !dx)) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "mean_square: NULL x or no output");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (dx && dx != x && overlaps(extent(dx, p.rows, p.cols, ld, 4), extent(x, p.rows, p.cols, ld, 4)))
    return fail(h, BWPP_HIP_ERR_ALIAS, "mean_square: dx overlaps x without being x");
  BwppGradArgs g = {};
  g.a = x;
  g.out = dx;
  g.out2 = loss;
  g.s_loss = loss_scale;
  g.s_grad = grad_scale;
  g.rows = p.rows;
  g.cols = p.cols;
  g.ld = ld;
  g.vec = (p.cols % 4 == 0 && ld % 4 == 0 && aligned16(x) && (!dx || aligned16(dx))) ? 1u : 0u;
  const uint32_t cap = h->cus > 0 ? 4u * (uint32_t)h->cus : 1024u;
  const uint32_t grid = std::max<uint32_t>(1u, std::min<uint32_t>(p.rows, cap));
  if ((s = ensure_ws(h, (size_t)grid * sizeof(float))) != BWPP_HIP_OK) return s;
  g.part_g = static_cast<float *>(h->ws);
  g.nparts = grid;
  if ((s = launch(h, h->mean_square_part, grid, 1, 1, 256, g)) != BWPP_HIP_OK) return s;
  if (!loss) return BWPP_HIP_OK;
  return launch(h, h->mean_square_final, 1, 1, 1, 256, g);
}

extern "C" BwppHipStatus bwpp_hip_dispatch_elementwise(BwppHip *h, const float *a, const float *b, float *out,
                                                       BwppElementwiseParams p) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (p.op > BWPP_HIP_OP_SILU || p.bmode > BWPP_HIP_BCAST_SCALAR)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "elementwise: bad op %u or broadcast %u", p.op, p.bmode);
  const bool unary = p.op == BWPP_HIP_OP_COPY || p.op == BWPP_HIP_OP_SILU;
  if (!b || !out || (!unary && !a))
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "elementwise: NULL pointer");
  const uint32_t ld = eff_ld(p.ld, p.cols);
  if ((s = check_rows(h, p.rows, p.cols, ld)) != BWPP_HIP_OK) return s;
  if (p.rows == 0 || p.cols == 0) return BWPP_HIP_OK;
  return elementwise_launch(h, unary ? nullptr : a, b, ld, out, ld, p.rows, p.cols, p.op, p.bmode);
}

BwppHipStatus bwpp_hip_copy_strided(BwppHip *h, const float *src, uint32_t ld_src, float *dst, uint32_t ld_dst,
                                    uint32_t rows, uint32_t cols) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (!src || !dst) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "copy: NULL pointer");
  if (ld_src < cols || ld_dst < cols)
    return fail(h, BWPP_HIP_ERR_INVALID_ARG, "copy: row strides (%u, %u) below cols (%u)", ld_src, ld_dst, cols);
  if (rows == 0 || cols == 0) return BWPP_HIP_OK;
  return elementwise_launch(h, nullptr, src, ld_src, dst, ld_dst, rows, cols, BWPP_HIP_OP_COPY, BWPP_HIP_BCAST_FULL);
}

BwppHipStatus bwpp_hip_copy_strided_multi(BwppHip *h, uint32_t n, const float *const *src, const uint32_t *ld_src,
                                          float *const *dst, const uint32_t *ld_dst, const uint32_t *rows,
                                          const uint32_t *cols) {
  BwppHipStatus s = enter(h);
  if (s != BWPP_HIP_OK) return s;
  if (n == 0 || n > BWPP_COPY_MULTI_MAX) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "copy: %u segments (1..4)", n);
  BwppCopyArgs a = {};
  a.n = n;
  a.vec = 1;
  uint64_t total = 0;
  for (uint32_t i = 0; i < n; ++i) {
    if (!src[i] || !dst[i]) return fail(h, BWPP_HIP_ERR_INVALID_ARG, "copy: NULL pointer");
    if (ld_src[i] < cols[i] || ld_dst[i] < cols[i])
      return fail(h, BWPP_HIP_ERR_INVALID_ARG, "copy: row strides (%u, %u) below cols (%u)", ld_src[i], ld_dst[i],
                  cols[i]);
    for (uint32_t j = 0; j < n; ++j)
      if (blocks_overlap(dst[i], rows[i], cols[i], ld_dst[i], src[j], rows[j], cols[j], ld_src[j], 4) ||
          (j != i && blocks_overlap(dst[i], rows[i], cols[i], ld_dst[i], dst[j], rows[j], cols[j], ld_dst[j], 4)))
        return fail(h, BWPP_HIP_ERR_ALIAS, "copy: segment %u's destination overlaps another segment", i);
    a.src[i] = src[i];
    a.dst[i] = dst[i];
    a.ld_src[i] = ld_src[i];
    a.ld_dst[i] = ld_dst[i];
    a.cols[i] = cols[i];
    a.row0[i] = (uint32_t)total;
    total += cols[i] ? rows[i] : 0u;
    if (cols[i] % 4 || ld_src[i] % 4 || ld_dst[i] % 4 || !aligned16(src[i]) || !aligned16(dst[i])) a.vec = 0;
  }
  if (total > 0xffffffffull) return fail(h, BWPP_HIP_ERR_UNSUPPORTED, "copy: too many rows");
  a.row0[n] = (uint32_t)total;
  if (total == 0) return BWPP_HIP_OK;
  return launch(h, h->copy_multi, row_grid(h, (uint32_t)total), 1, 1, 256, a);
}
