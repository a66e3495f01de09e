// Host launchers behind the C ABI declared in include/hf_convrot.h. One translation unit: the kernel sources are
// included so a single hipcc invocation builds the shared library.
#include <mutex>

#include "../../include/hf_convrot.h"
#include "int8_gemm.hip"
#include "lowrank.hip"
#include "mid_gemm.hip"
#include "rotate_quant.hip"
#include "skinny.hip"
#include "splitk.hip"
#include "skinny_fused.hip"

namespace {

constexpr int kMaxLds = 160 * 1024;
// Rows up to which the rotation runs one workgroup per row (every tile of a row in flight at once).
constexpr int64_t kRowKernelMaxRows = 1024;

inline bool aligned(const void* p, uintptr_t a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

inline int launch_status() { return hipGetLastError() == hipSuccess ? HF_OK : HF_ERR_LAUNCH; }

int log4_of(int32_t group) {
  switch (group) {
    case 4: return 1;
    case 16: return 2;
    case 64: return 3;
    case 256: return 4;
    case 1024: return 5;
    case 4096: return 6;
    case 16384: return 7;
    default: return -1;
  }
}

// Kernels that use more than 64 KiB of dynamic LDS must say so, once per device (the attribute belongs to the
// kernel's code object on the current device); devices past the 64th set it on every call.
void allow_large_lds() {
  static std::once_flag once[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  std::once_flag spare;
  std::call_once(dev < 64 ? once[dev] : spare, [] {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutI32>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutI32, hf::kActSwiGLU>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutBf16>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutBf16Lr>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutBf16, hf::kActGeluTanh>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutBf16Lr, hf::kActGeluTanh>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutBf16, hf::kActSwiGLU>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<hf::kOutBf16Lr, hf::kActSwiGLU>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
#define HF_LATE_ATTR(OUT, ACT)                                                                                       \
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::int8_gemm_kernel<OUT, ACT, true>),                 \
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::kGemmLds);
    HF_LATE_ATTR(hf::kOutBf16, hf::kActNone) HF_LATE_ATTR(hf::kOutBf16Lr, hf::kActNone)
    HF_LATE_ATTR(hf::kOutBf16, hf::kActGeluTanh) HF_LATE_ATTR(hf::kOutBf16Lr, hf::kActGeluTanh)
    HF_LATE_ATTR(hf::kOutBf16, hf::kActSwiGLU) HF_LATE_ATTR(hf::kOutBf16Lr, hf::kActSwiGLU)
#undef HF_LATE_ATTR
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::skinny_fused_kernel<64, false>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::sf_lds(64));
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::skinny_fused_kernel<64, true>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::sf_lds(64));
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_kernel<1>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_kernel<2>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_kernel<3>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_kernel<4>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_kernel<5>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_row_kernel<1>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_row_kernel<2>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_row_kernel<3>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_row_kernel<4>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_row_kernel<5>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_lowrank_row_kernel<1>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_lowrank_row_kernel<2>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_lowrank_row_kernel<3>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_lowrank_row_kernel<4>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_lowrank_row_kernel<5>),
                        hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
#define HF_LR_ATTR(RB, NW)                                                                                \
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::lowrank_down_kernel<RB, NW>),             \
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::lr_lds(NW));
    HF_LR_ATTR(1, 4) HF_LR_ATTR(1, 5) HF_LR_ATTR(1, 6) HF_LR_ATTR(1, 7) HF_LR_ATTR(1, 8)
    HF_LR_ATTR(2, 4) HF_LR_ATTR(2, 5) HF_LR_ATTR(2, 6) HF_LR_ATTR(2, 7) HF_LR_ATTR(2, 8)
#undef HF_LR_ATTR
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::lowrank_down_wide_kernel<4>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::lw_lds(4));
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::lowrank_down_wide_kernel<5>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::lw_lds(5));
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::lowrank_up_kernel),
                        hipFuncAttributeMaxDynamicSharedMemorySize, hf::kUpLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_wide_kernel<false>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::rotate_quant_wide_kernel<true>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::mid_gemm_kernel<hf::kActNone>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::kMidLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::mid_gemm_kernel<hf::kActGeluTanh>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::kMidLds);
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::lowrank_down_band_kernel),
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::kLbLds);
#define HF_BAND_ATTR(NB)                                                                                            \
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::band_gemm_kernel<NB, hf::kActNone>),              \
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::band_lds(NB));                       \
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::band_gemm_kernel<NB, hf::kActGeluTanh>),          \
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::band_lds(NB));
    HF_BAND_ATTR(3) HF_BAND_ATTR(4) HF_BAND_ATTR(5)
#undef HF_BAND_ATTR
#define HF_SKINNY_ATTR(GLU, MR)                                                                       \
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(&hf::skinny_gemm_kernel<GLU, MR>),             \
                              hipFuncAttributeMaxDynamicSharedMemorySize, hf::skinny_lds(MR));
    HF_SKINNY_ATTR(false, 64) HF_SKINNY_ATTR(true, 64) HF_SKINNY_ATTR(false, 128) HF_SKINNY_ATTR(true, 128)
    HF_SKINNY_ATTR(false, 256) HF_SKINNY_ATTR(true, 256)
#undef HF_SKINNY_ATTR
    (void)hipGetLastError();
  });
}

// Groups of 4096 and more: rotate_quant_wide_kernel, one workgroup per row with the row's fp64 sums in LDS
// (K * 8 bytes, so K <= 20472). The caller has checked the group, the alignment and M > 0.
int launch_rotate_wide(bool f32_recip, int lg, const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx,
                       int64_t M, int64_t K, hipStream_t s) {
  const size_t lds = hf::rotate_quant_wide_lds_bytes((int)std::min<int64_t>(K, 1 << 20));
  if (lds > (size_t)kMaxLds || M >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  allow_large_lds();
  const dim3 grid((unsigned)M), block(hf::kRqWideThreads);
  if (f32_recip)
    hipLaunchKernelGGL(hf::rotate_quant_wide_kernel<true>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, lg);
  else
    hipLaunchKernelGGL(hf::rotate_quant_wide_kernel<false>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, lg);
  return launch_status();
}

// rotate_quant_reg_kernel<lg, tpw, f32> (lg and tpw already range-checked by the caller).
int launch_rotate_reg(int lg, int tpw, bool f32, dim3 grid, dim3 block, size_t lds, hipStream_t s,
                      const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, int64_t M, int K, int wpr,
                      const hf::LrFinish& fin) {
#define HF_RQ_CASE(L, T)                                                                                          \
  if (lg == L && tpw == T) {                                                                                      \
    if (f32)                                                                                                      \
      hipLaunchKernelGGL((hf::rotate_quant_reg_kernel<L, T, true>), grid, block, lds, s, x, ldx, q, ldq, sx, M, K, \
                         wpr, fin);                                                                               \
    else                                                                                                          \
      hipLaunchKernelGGL((hf::rotate_quant_reg_kernel<L, T, false>), grid, block, lds, s, x, ldx, q, ldq, sx, M,   \
                         K, wpr, fin);                                                                            \
    return launch_status();                                                                                       \
  }
#define HF_RQ_CASES(L) HF_RQ_CASE(L, 1) HF_RQ_CASE(L, 2) HF_RQ_CASE(L, 3) HF_RQ_CASE(L, 4) HF_RQ_CASE(L, 5)
  HF_RQ_CASES(1)
  HF_RQ_CASES(2)
  HF_RQ_CASES(3)
  HF_RQ_CASES(4)
  HF_RQ_CASES(5)
#undef HF_RQ_CASES
#undef HF_RQ_CASE
  return HF_ERR_ARGUMENT;
}

// Rows of at most 4 * kRqRegMaxTpw tiles held in registers (rotate_quant_reg_kernel): wpr waves of tpw tiles per
// row, 4 / wpr rows per workgroup. The caller has checked the group, the alignment and M > 0.
int rotate_rows_in_registers(bool f32, int lg, const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx,
                             int64_t M, int64_t K, hipStream_t s, const hf::LrFinish& fin) {
  const int64_t ntiles = (K + hf::kRqTile - 1) / hf::kRqTile;
  const int wpr = (int)((ntiles + hf::kRqRegMaxTpw - 1) / hf::kRqRegMaxTpw);
  const int tpw = (int)((ntiles + wpr - 1) / wpr);
  const int rows_per_wg = std::max(1, 4 / wpr);
  const int nw = wpr * rows_per_wg;
  const int64_t blocks = (M + rows_per_wg - 1) / rows_per_wg;
  if (blocks >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  allow_large_lds();
  return launch_rotate_reg(lg, tpw, f32, dim3((unsigned)blocks), dim3(64 * nw), hf::rotate_quant_reg_lds_bytes(nw),
                           s, x, ldx, q, ldq, sx, M, (int)K, wpr, fin);
}

int check_gemm_operands(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, int64_t M, int64_t N,
                        int64_t K) {
  if (!q || !w || M < 0 || N < 0 || K <= 0 || ldq < K || ldw < K) return HF_ERR_ARGUMENT;
  if ((K % 16) || !aligned(q, 16) || !aligned(w, 16) || (ldq % 16) || (ldw % 16)) return HF_ERR_ALIGNMENT;
  if (256 * ldq >= (int64_t(1) << 31) || 256 * ldw >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  return HF_OK;
}

// CUs of the current device (queried once per device).
int device_cus() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  int n = dev < 64 ? cus[dev] : 0;
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    if (dev < 64) cus[dev] = n;
  }
  return n;
}

// Workgroups for the persistent GEMM: one per CU, at most one per work item.
int gemm_grid(int64_t items) { return (int)std::min<int64_t>(items, device_cus()); }

int launch_gemm(hf::GemmArgs& a, bool i32, hipStream_t stream, int act = hf::kActNone) {
  allow_large_lds();
  a.tiles_m = (a.M + hf::GBM - 1) / hf::GBM;
  a.tiles_n = (a.N + hf::GBN - 1) / hf::GBN;
  if (a.splits <= 0) {
    a.splits = 1;
    a.k_chunk = (int)(((int64_t)a.K + hf::GBK - 1) / hf::GBK * hf::GBK);
  }
  const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n * a.splits;
  if (tiles == 0) return HF_OK;
  if (tiles >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  const dim3 grid((unsigned)gemm_grid(tiles)), block(hf::kThreads);
  if (i32) {
    if (act == hf::kActSwiGLU)  // split-K partials in pair order
      hipLaunchKernelGGL((hf::int8_gemm_kernel<hf::kOutI32, hf::kActSwiGLU>), grid, block, hf::kGemmLds, stream, a);
    else
      hipLaunchKernelGGL(hf::int8_gemm_kernel<hf::kOutI32>, grid, block, hf::kGemmLds, stream, a);
  } else {
    // Stage loads after each K step's MFMAs up to K = kLateLoadsMaxK (int8_gemm_kernel's LATE, measured by K).
    const bool late = a.splits == 1 && a.K <= hf::kLateLoadsMaxK;
    const bool lr = a.r > 0 && a.r <= 64;
#define HF_GEMM_BF16(OUT, ACT)                                                                                      \
    if (late)                                                                                                       \
      hipLaunchKernelGGL((hf::int8_gemm_kernel<OUT, ACT, true>), grid, block, hf::kGemmLds, stream, a);             \
    else                                                                                                            \
      hipLaunchKernelGGL((hf::int8_gemm_kernel<OUT, ACT, false>), grid, block, hf::kGemmLds, stream, a);
    if (act == hf::kActGeluTanh) {
      if (lr) { HF_GEMM_BF16(hf::kOutBf16Lr, hf::kActGeluTanh) } else { HF_GEMM_BF16(hf::kOutBf16, hf::kActGeluTanh) }
    } else if (act == hf::kActSwiGLU) {
      if (lr) { HF_GEMM_BF16(hf::kOutBf16Lr, hf::kActSwiGLU) } else { HF_GEMM_BF16(hf::kOutBf16, hf::kActSwiGLU) }
    } else {
      if (lr) { HF_GEMM_BF16(hf::kOutBf16Lr, hf::kActNone) } else { HF_GEMM_BF16(hf::kOutBf16, hf::kActNone) }
    }
#undef HF_GEMM_BF16
  }
  return launch_status();
}

// Split plan of the low-rank down projection: few row blocks leave most CUs idle, so K is split into chunks of at
// least 4 stages (256 elements) until the grid covers the CUs; the fp32 partials are tiny (M x r per split).
struct LrPlan {
  int splits = 1;
  int k_chunk = 0;
};

LrPlan lowrank_plan(int64_t M, int64_t K) {
  LrPlan p;
  p.k_chunk = (int)K;
  const int64_t blocks = (M + hf::kLrRows - 1) / hf::kLrRows;
  const int64_t stages = (K + hf::kLrStageK - 1) / hf::kLrStageK;
  const int64_t want = std::min<int64_t>(std::min<int64_t>(device_cus() / std::max<int64_t>(blocks, 1), stages / 4),
                                         hf::kMaxSplits);
  if (want >= 2) {
    const int64_t chunk_stages = (stages + want - 1) / want;
    p.k_chunk = (int)(chunk_stages * hf::kLrStageK);
    p.splits = (int)((K + p.k_chunk - 1) / p.k_chunk);
  }
  return p;
}

// Few rows: one workgroup per row (lowrank_down_row_kernel), no split and no workspace.
bool lowrank_by_rows(int64_t M, int64_t K) {
  return M <= hf::kLrRowMaxRows && K <= (int64_t)hf::kLrRowMaxWaves * 1024;
}

// Whether the row kernel is also the faster choice. Its cost grows with M * K while the split MFMA kernel's stays
// nearly flat over few rows: measured (M up to 384, rank 64) the rows win while M * K <= ~1.7 M (up to 384 rows at
// K=3072, ~330 at K=5120, ~240 at K=7168, ~110 at K=14336) and lose beyond, by up to 2.2x (M=384, K=14336: 37.3
// against 16.7 us).
constexpr double kLrRowMaxWork = 1.7e6;
bool lowrank_rows_faster(int64_t M, int64_t K) { return lowrank_by_rows(M, K) && (double)M * K <= kLrRowMaxWork; }

int64_t lowrank_ws_bytes(int64_t M, int64_t K, int32_t r) {
  if (lowrank_rows_faster(M, K)) return 0;
  const LrPlan p = lowrank_plan(M, K);
  return p.splits > 1 ? (int64_t)p.splits * M * r * 4 : 0;
}

// The first choice of lowrank_down_impl (before its wide-rank routes, which need many rows and one pass over K): the
// row kernel, or the MFMA kernel with this K plan. A split needs its workspace (the fp32 partial sums of the first
// 64 ranks); without it the rows are still the faster choice where they apply, else the MFMA kernel takes K in one
// pass.
struct LrRoute {
  bool by_rows;
  LrPlan plan;
};
LrRoute lowrank_route(int64_t M, int64_t K, int32_t r, const void* ws, int64_t ws_bytes) {
  LrRoute rt{lowrank_rows_faster(M, K), lowrank_plan(M, K)};
  const bool ws_ok = ws && aligned(ws, 16) &&
                     ws_bytes >= (int64_t)rt.plan.splits * M * std::min<int32_t>(r, hf::kLrRanks) * 4;
  if (rt.plan.splits > 1 && !ws_ok) {
    if (lowrank_by_rows(M, K)) rt.by_rows = true;
    rt.plan = LrPlan{};
    rt.plan.k_chunk = (int)K;
  }
  return rt;
}

// Whether lowrank_down_impl with these sizes and workspace runs the split MFMA kernel for at most 64 ranks (the
// case in which it can leave its partial sums for the layer's rotation kernel to add).
bool lowrank_split_planned(int64_t M, int64_t K, int32_t r, const void* ws, int64_t ws_bytes) {
  if (M <= 0 || K <= 0 || r <= 0 || r > hf::kLrRanks) return false;
  const LrRoute rt = lowrank_route(M, K, r, ws, ws_bytes);
  return !rt.by_rows && rt.plan.splits > 1;
}

// defer: when the split MFMA kernel runs for at most 64 ranks, its partial sums are left in the workspace and
// described in *defer for the layer's rotation kernel to add (no lowrank_reduce_kernel launch); otherwise
// defer->part stays null.
int lowrank_down_impl(const uint16_t* x, int64_t ldx, const uint16_t* down, int64_t ld_down, uint16_t* u,
                      int64_t ldu, int64_t M, int64_t K, int32_t r, void* ws, int64_t ws_bytes,
                      hf_stream_t stream, hf::LrFinish* defer = nullptr) {
  if (M < 0 || K <= 0 || r < 0 || ldx < K || ld_down < K || ldu < r) return HF_ERR_ARGUMENT;
  if (M == 0 || r == 0) return HF_OK;
  if (!x || !down || !u) return HF_ERR_ARGUMENT;
  if (K % 16 || !aligned(x, 16) || !aligned(down, 16) || (ldx % 8) || (ld_down % 8) || !aligned(u, 8))
    return HF_ERR_ALIGNMENT;
  if (M >= (int64_t(1) << 31) || K >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const LrRoute route = lowrank_route(M, K, r, ws, ws_bytes);
  if (route.by_rows) {
    const int64_t waves = (K + 1023) / 1024, groups = (r + hf::kLrRowRanks - 1) / hf::kLrRowRanks;
    const int64_t blocks = hf::lowrank_row_blocks(M, r);
    if (blocks >= (int64_t(1) << 31)) return HF_ERR_SIZE;
    hipLaunchKernelGGL(hf::lowrank_down_row_kernel, dim3((unsigned)blocks), dim3((unsigned)(64 * waves)), 0, s, x,
                       ldx, down, ld_down, u, ldu, (int)M, (int)K, r, (int)groups);
    return launch_status();
  }
  if (2 * hf::kLrMaxRows * ldx >= (int64_t(1) << 31) || 2 * hf::kLrRanks * ld_down >= (int64_t(1) << 31))
    return HF_ERR_SIZE;
  allow_large_lds();
  const LrPlan plan = route.plan;
  if (plan.splits == 1 && r > 128 && K >= 4096 && 8 * ((M + hf::kLbRows - 1) / hf::kLbRows) >= 7 * device_cus() &&
      8 * ((M + hf::kLbRows - 1) / hf::kLbRows) <= 8 * device_cus()) {
    // Ranks past 128 with 160-row blocks filling 7/8 to all of the CUs: lowrank_down_band_kernel, 256 ranks per pass
    // over x, bitwise the sums of the routes below. Measured at M=37710 against them (same box): K=14336, r=256 387
    // -> 333 us, r=512 731 -> 657 us; K=5376, r=192 149 -> 120 us, r=256 155 -> 147 us, r=512 259 -> 256 us. With a
    // short K (M=40000, K=2064, r=200: 59 -> 80 us) the four-stage x ring does not fill, hence K >= 4096.
    if (2 * hf::kLwRanks * ld_down >= (int64_t(1) << 31)) return HF_ERR_SIZE;
    const unsigned blocks = (unsigned)((M + hf::kLbRows - 1) / hf::kLbRows);
    for (int32_t j0 = 0; j0 < r; j0 += hf::kLwRanks) {
      const int rr = std::min<int32_t>(hf::kLwRanks, r - j0);
      hipLaunchKernelGGL(hf::lowrank_down_band_kernel, dim3(blocks), dim3(512), hf::kLbLds, s, x, ldx,
                         down + (int64_t)j0 * ld_down, ld_down, u + j0, ldu, (int)M, (int)K, rr);
      const int st = launch_status();
      if (st != HF_OK) return st;
    }
    return HF_OK;
  }
  if (plan.splits == 1 && r >= 192 && aligned(u, 16) && (ldu % 8) == 0 &&
      2 * ((M + hf::GBM - 1) / hf::GBM) * ((r + hf::GBN - 1) / hf::GBN) >= device_cus()) {
    // Wide ranks with many rows: the persistent 256 x 256 tiles' bf16 product (x rows against down rows, K in
    // bytes), one pass over x per 256 ranks with the matrix cores at the tile kernel's rate. The summation order
    // (64-element stages, 16-element MFMA steps, K ascending) is lowrank_down_wide_kernel's.
    if (2 * K >= (int64_t(1) << 31) || 2 * hf::GBM * ldx >= (int64_t(1) << 32) ||
        2 * hf::GBN * ld_down >= (int64_t(1) << 32))
      return HF_ERR_SIZE;
    hf::GemmArgs a{};
    a.q = reinterpret_cast<const int8_t*>(x); a.ldq = 2 * ldx;
    a.w = reinterpret_cast<const int8_t*>(down); a.ldw = 2 * ld_down;
    a.out = u; a.ldo = ldu;
    a.M = (int)M; a.N = r; a.K = (int)(2 * K); a.out_vec16 = 1;
    a.tiles_m = (int)((M + hf::GBM - 1) / hf::GBM);
    a.tiles_n = (int)((r + hf::GBN - 1) / hf::GBN);
    a.splits = 1;
    a.k_chunk = (int)((a.K + hf::GBK - 1) / hf::GBK * hf::GBK);
    const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
    hipLaunchKernelGGL(hf::int8_gemm_kernel<hf::kOutMmBf16>, dim3((unsigned)gemm_grid(tiles)), dim3(hf::kThreads),
                       hf::kGemmLds, s, a);
    return launch_status();
  }
  if (plan.splits == 1 && r > hf::kLrRanks) {
    // Ranks past 64 with many rows: 256 ranks per pass over x (lowrank_down_wide_kernel), 4 or 5 row blocks of 32
    // per workgroup (5 when 128-row workgroups would need more than one round of CUs).
    if (2 * hf::kLwRanks * ld_down >= (int64_t(1) << 31)) return HF_ERR_SIZE;
    const int nr = (M + 127) / 128 > device_cus() ? 5 : 4;
    const unsigned blocks = (unsigned)((M + 32 * nr - 1) / (32 * nr));
    for (int32_t j0 = 0; j0 < r; j0 += hf::kLwRanks) {
      const int rr = std::min<int32_t>(hf::kLwRanks, r - j0);
      const uint16_t* d = down + (int64_t)j0 * ld_down;
      if (nr == 5)
        hipLaunchKernelGGL(hf::lowrank_down_wide_kernel<5>, dim3(blocks), dim3(128 * 5), hf::lw_lds(5), s, x, ldx, d,
                           ld_down, u + j0, ldu, (int)M, (int)K, rr);
      else
        hipLaunchKernelGGL(hf::lowrank_down_wide_kernel<4>, dim3(blocks), dim3(128 * 4), hf::lw_lds(4), s, x, ldx, d,
                           ld_down, u + j0, ldu, (int)M, (int)K, rr);
      const int st = launch_status();
      if (st != HF_OK) return st;
    }
    return HF_OK;
  }
  float* part = plan.splits > 1 ? static_cast<float*>(ws) : nullptr;
  // Waves per workgroup (32 rows each): the fewest that cover the rows in one round of one workgroup per CU, from 4
  // (128 rows) to 8; split launches keep 4.
  int nw = 4;
  if (plan.splits == 1) {
    const int64_t per_cu = (M + device_cus() - 1) / device_cus();
    nw = (int)std::min<int64_t>(std::max<int64_t>((per_cu + 31) / 32, 4), hf::kLrMaxWaves);
  }
  const unsigned blocks = (unsigned)((M + 32 * nw - 1) / (32 * nw));
  for (int32_t j0 = 0; j0 < r; j0 += hf::kLrRanks) {
    const int rr = std::min<int32_t>(hf::kLrRanks, r - j0);
    const uint16_t* d = down + (int64_t)j0 * ld_down;
    uint16_t* uo = u + j0;
    const dim3 grid(blocks, (unsigned)plan.splits), block(64 * nw);
#define HF_LR_CASE(NW)                                                                                              \
  if (nw == NW) {                                                                                                   \
    if (rr <= 32)                                                                                                   \
      hipLaunchKernelGGL((hf::lowrank_down_kernel<1, NW>), grid, block, hf::lr_lds(NW), s, x, ldx, d, ld_down, uo,  \
                         ldu, (int)M, (int)K, rr, plan.k_chunk, part);                                              \
    else                                                                                                            \
      hipLaunchKernelGGL((hf::lowrank_down_kernel<2, NW>), grid, block, hf::lr_lds(NW), s, x, ldx, d, ld_down, uo,  \
                         ldu, (int)M, (int)K, rr, plan.k_chunk, part);                                              \
  }
    HF_LR_CASE(4) HF_LR_CASE(5) HF_LR_CASE(6) HF_LR_CASE(7) HF_LR_CASE(8)
#undef HF_LR_CASE
    int st = launch_status();
    if (st != HF_OK) return st;
    if (part && defer && r <= hf::kLrRanks) {
      *defer = hf::LrFinish{part, uo, ldu, M, plan.splits, rr};
    } else if (part) {
      const int64_t n = M * rr;
      hipLaunchKernelGGL(hf::lowrank_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part,
                         plan.splits, uo, ldu, (int)M, rr);
      st = launch_status();
      if (st != HF_OK) return st;
    }
  }
  return HF_OK;
}

// Split plan of the INT8 GEMM: when the 256 x 256 tiles are fewer than the CUs, K is split so more CUs share the
// weight stream. A small cost model picks the split: the MFMA time of one round of work items against the memory
// time of the weight, the activations and the int32 partials (written and read back).
struct GemmPlan {
  int splits = 1;
  int k_chunk = 0;
  bool skinny = false;  // at most 256 rows: 128-row weight slices (skinny_gemm_kernel) instead of 256 x 256 tiles
  int mr = 0;           // the skinny kernel's activation rows (64, 128 or 256)
  double seconds = 0;   // the cost model's estimate of the GEMM's time
};

constexpr double kPlanBw = 5.0e12;  // sustained HBM bytes per second of the cost model
// One 128-byte K stage of one 256 x 256 tile at the sustained (power-bound) matrix-core rate.
constexpr double kTileStageSeconds = 2.0 * 256 * 256 * 128 / (8192.0 * 2.0e9 * 0.55);

// The split-K finishing pass: a launch and a few microseconds of latency, then the int32 partial planes read and the
// bf16 output written (measured: M=512, N=K=4096 in 4 splits, 29.4 us with the GEMM against 29.5 us estimated).
double split_finish_seconds(int64_t splits, int64_t M, int64_t N) {
  return 4e-6 + (4.0 * splits + 2.0) * (double)M * (double)N / kPlanBw;
}

GemmPlan gemm_plan(int64_t M, int64_t N, int64_t K) {
  GemmPlan best;
  const int64_t ntiles = (N + hf::kSkinnyN - 1) / hf::kSkinnyN;
  // 128-row weight slices up to 128 rows, and up to 256 rows while the slices leave room to split K at least in two
  // (one workgroup per CU, one wave per SIMD: with K whole, M=256, N=30720 took 97.7 us against 89.1 us for 256 x 256
  // tiles split in two; M=256, N=5120 / 15360 took 36.7 / 60.2 us against 40.5 / 65.8 us).
  if (M <= 128 || (M <= hf::kSkinnyMaxM && 2 * ntiles <= device_cus())) {
    // Enough 128-row x K-chunk work items for one per CU, each chunk at least 4 stages (512 bytes of K). Two per CU
    // (twice the partial planes to write and add) measured 2.5-4 % slower per layer at M=16..64, N=5120..30720. With
    // more than 64 rows a workgroup fills a CU's LDS, so the items stay within one round (rounded down).
    const int64_t stages = (K + hf::kSkinnyStageK - 1) / hf::kSkinnyStageK;
    best.mr = M <= hf::kSkinnyM ? hf::kSkinnyM : (M <= 128 ? 128 : hf::kSkinnyMaxM);
    int64_t want = best.mr == hf::kSkinnyM ? (device_cus() + ntiles - 1) / ntiles : device_cus() / ntiles;
    want = std::max<int64_t>(1, std::min<int64_t>(want, std::min<int64_t>(stages / 4, hf::kMaxSplits)));
    const int64_t chunk = (stages + want - 1) / want;
    best.skinny = true;
    best.k_chunk = (int)(chunk * hf::kSkinnyStageK);
    best.splits = (int)((stages + chunk - 1) / chunk);
    best.seconds = ((double)N * K + 8.0 * best.splits * M * N) / kPlanBw;
    return best;
  }
  const int64_t stages = (K + hf::GBK - 1) / hf::GBK;
  best.k_chunk = (int)(stages * hf::GBK);
  const int64_t tiles = ((M + hf::GBM - 1) / hf::GBM) * ((N + hf::GBN - 1) / hf::GBN);
  const int64_t cus = device_cus();
  const double fixed_bytes = (double)N * K + (double)M * K + 2.0 * M * N;
  best.seconds = std::max((double)((tiles + cus - 1) / cus) * stages * kTileStageSeconds, fixed_bytes / kPlanBw);
  if (tiles >= cus || stages < 4) return best;
  const double t_whole = best.seconds;
  for (int64_t s = 2; s <= std::min<int64_t>(stages / 2, hf::kMaxSplits); ++s) {
    const int64_t chunk = (stages + s - 1) / s;
    const int64_t splits = (stages + chunk - 1) / chunk;
    const double rounds = (double)((tiles * splits + cus - 1) / cus);
    const double t_mfma = rounds * chunk * kTileStageSeconds;
    const double t_mem = (fixed_bytes + (splits > 1 ? 8.0 * splits * M * N : 0.0)) / kPlanBw;
    const double t = std::max(t_mfma, t_mem);
    if (t < best.seconds * 0.97) {
      best.seconds = t;
      best.splits = (int)splits;
      best.k_chunk = (int)(chunk * hf::GBK);
    }
  }
  // The split plan's partial planes are written during the GEMM and read back by the finishing pass after it: when
  // that pass makes the split slower than one round of whole tiles, the tiles stay whole (M=2048, N=K=5120: 160
  // whole tiles against 3 splits that took 92 us with their finishing pass).
  if (best.splits > 1 && t_whole <= best.seconds + split_finish_seconds(best.splits, M, N)) {
    best.splits = 1;
    best.k_chunk = (int)(stages * hf::GBK);
    best.seconds = t_whole;
  }
  return best;
}

// The persistent GEMM's whole time as planned: the GEMM launch, plus the finishing pass of a split plan.
double persistent_seconds(const GemmPlan& p, int64_t M, int64_t N) {
  return p.seconds + (p.splits > 1 || p.skinny ? split_finish_seconds(p.splits, M, N) : 0.0);
}

// Whether a GEMM runs as 256 x 128 tiles (mid_gemm_kernel): its 256 x 256 tiles are fewer than the CUs, it is too
// tall for the 128-row weight slices (skinny_gemm_kernel), and the 256 x 128 tiles fill at least half the CUs, so no
// K split (with its int32 partial planes and finishing pass) is needed, unless K is deep enough for the split to
// win clearly (below). Between a quarter and half of the CUs the
// tiles' single round is weighed against the split path with times measured on MI355X (M=512-1024, N=2048-5120,
// K=2048-5120, graph replays): the tiles take ~0.9 us per 128-byte K stage plus ~3 us, the split GEMM and its
// finishing pass ~21 us plus ~0.62 us per 10^9 int8 operations (e.g. M=1024, N=K=3072: 25.5 against 31.8 us; at
// M=512, N=4096, K=5120 the split path's 33.4 against 37.7 us). The kernel's epilogue covers rank <= 64 and the
// tanh-GELU; gated (SwiGLU) outputs keep the split path.
bool use_mid_gemm(int64_t M, int64_t N, int64_t K, int32_t r, bool glu) {
  if (glu || r > 64) return false;
  const int64_t cus = device_cus();
  const int64_t tiles_m = (M + hf::GBM - 1) / hf::GBM;
  if (tiles_m * ((N + hf::GBN - 1) / hf::GBN) >= cus) return false;
  const int64_t ntiles = (N + hf::kSkinnyN - 1) / hf::kSkinnyN;
  if (M <= 128 || (M <= hf::kSkinnyMaxM && 2 * ntiles <= cus)) return false;
  const int64_t tiles = tiles_m * ((N + hf::kMidBN - 1) / hf::kMidBN);
  const double stages = (double)((K + hf::kMidBK - 1) / hf::kMidBK);
  const double t_round = 0.9 * stages + 3.0;  // us per round of tiles
  if (tiles > cus) {
    // A second, partly filled round: only when it beats the persistent GEMM's plan (whole tiles, or split with its
    // finishing pass). M=640-1024, N=15360, K=5120: 83-90 us in two rounds against 72-80 us persistent; M=1792,
    // N=5120: 77 us in two rounds.
    const double t_tiles = 1e-6 * t_round * (double)((tiles + cus - 1) / cus);
    return t_tiles < persistent_seconds(gemm_plan(M, N, K), M, N);
  }
  if (2 * tiles >= cus) {
    // One round of tiles, at least half the CUs: they win unless K is deep enough that the persistent GEMM's split
    // plan is clearly (10 %) faster. M=1024, N=5120, K=14336: 108.0 us as these tiles, 94.8 us split; at K=8192
    // the estimates are within 2 % and the tiles are faster (61.3 against 63.2 us).
    return persistent_seconds(gemm_plan(M, N, K), M, N) >= 0.9e-6 * t_round;
  }
  if (4 * tiles < cus) return false;
  const double t_split = 21.0 + 0.62e-9 * 2.0 * (double)M * (double)N * (double)K;
  return t_round < t_split;
}

// Column blocks per 128-row band tile (band_gemm_kernel), or 0: the bands run when one round of them fills at least
// 7/8 of the CUs while the 256 x 128 tiles would fill at most 3/4 (M=1024: N=5120 as 256 tiles of 128 x 160
// against 160 of 256 x 128; N=4096, 128 x 128; N=3072, 128 x 96). The widest such tile wins: it reads the fewest
// operand bytes per output. Rank <= 64, no SwiGLU.
int band_blocks_n(int64_t M, int64_t N, int32_t r, bool glu) {
  if (glu || r > 64) return 0;
  const int64_t cus = device_cus();
  const int64_t mid_tiles = ((M + hf::kMidBM - 1) / hf::kMidBM) * ((N + hf::kMidBN - 1) / hf::kMidBN);
  if (4 * mid_tiles > 3 * cus && mid_tiles <= cus) return 0;
  for (int nb = 5; nb >= 3; --nb) {
    const int64_t tiles = ((M + hf::kBandBM - 1) / hf::kBandBM) * ((N + 32 * nb - 1) / (32 * nb));
    if (tiles <= cus && 8 * tiles >= 7 * cus) return nb;
  }
  return 0;
}

// Whether a GEMM of at most 64 rows runs in one pass (skinny_fused_kernel): its 32-row weight slices fill between a
// quarter of the CUs and one round of them. Each workgroup's weight stream is latency-bound (the codes take two thirds
// of each stage), so against the split-K path (128-row slices over K chunks, partial planes and a finishing pass) it
// wins only while the slices fit one round: M=64, N=5120 16.0 -> 14.8 us, M=16 13.9 -> 12.3 us; at N=30720 (3.75
// rounds) 60 against 44 us, and with 128 rows (21.5 against 17.9 us) the split path stays.
bool use_skinny_fused(int64_t M, int64_t N) {
  const int64_t slices = (N + hf::kSfN - 1) / hf::kSfN;
  return M <= 64 && 4 * slices >= device_cus() && slices <= device_cus();
}

// Rows of a many-tile GEMM that run as whole 256 x 256 tiles; the rest (the trailing tile rows) run as a separate
// few-row GEMM, split over K. The persistent grid takes ceil(tiles / CUs) rounds; when the last round is less than
// half full, its tiles keep a few CUs busy for a whole tile time while the others idle. Peeling off the trailing
// tile rows so the main part fills one round fewer, and splitting the peeled rows' K over every CU, turns that round
// into a fraction of one, plus the partial planes, the finishing pass and a drain between the launches. A lightly
// loaded last round runs at a higher clock than a full one (the full chip is power-bound): at K=5120 one tenth of a
// round measured 0.61 of a full round's time (M=3584 against M=3072, N=5120), so the light round is priced at 0.6
// of a round against the peeled rows' GEMM with its finishing pass (persistent_seconds). Measured with this price:
// M=3584, N=K=5120 127.1 -> 114.8 us, M=7168 193.4 -> 180.3 us; deep K as before (M=37710, N=5376, K=14336:
// 2656 -> 2607 us against no peel); the model's q/k/v and M=41344, N=13824 unchanged. Returns M when nothing is
// peeled; the peeled rows' workspace is that of their own route (gemm_route).
int64_t main_gemm_rows(int64_t M, int64_t N, int64_t K) {
  const int64_t tiles_m = (M + hf::GBM - 1) / hf::GBM, tiles_n = (N + hf::GBN - 1) / hf::GBN;
  const int64_t tiles = tiles_m * tiles_n, cus = device_cus();
  if (tiles < cus) return M;
  const int64_t rounds = (tiles + cus - 1) / cus;
  if (2 * (tiles - (rounds - 1) * cus) > cus) return M;
  const int64_t rows_main = (rounds - 1) * cus / tiles_n;  // tile rows that fit in one round fewer
  if (rows_main <= 0 || rows_main >= tiles_m) return M;
  const int64_t m_tail = M - rows_main * hf::GBM;
  const GemmPlan tail = gemm_plan(m_tail, N, K);
  if (tail.splits <= 1) return M;
  const double t_round = (double)((K + hf::GBK - 1) / hf::GBK) * kTileStageSeconds;
  return persistent_seconds(tail, m_tail, N) < 0.6 * t_round ? rows_main * hf::GBM : M;
}

// Ints per split-K partial plane: ceil(M / 32) x ceil(N / 32) blocks of 32 x 32 (partial_block_offset).
int64_t partial_plane_ints(int64_t M, int64_t N) { return ((M + 31) / 32) * ((N + 31) / 32) * 1024; }

// The kernel path of a GEMM of these sizes, and the workspace that path uses. int8_linear_impl launches by it and the
// size queries report its bytes, so a query gives exactly what the call with the same sizes, rank and activation
// uses (0 for the 256 x 128 tiles, the one-pass few-row kernel and whole tiles).
struct GemmRoute {
  enum Kind { kWhole, kPeel, kBand, kMid, kSkinnyFused, kSplit } kind = kWhole;
  int64_t m_main = 0;    // kPeel: rows run as whole tiles; the rest run by their own route
  GemmPlan plan;         // kSplit: the K split
  int64_t ws_bytes = 0;  // workspace the route uses (kPeel: the peeled rows' route's)
};

GemmRoute gemm_route(int64_t M, int64_t N, int64_t K, int32_t r, bool glu) {
  GemmRoute route;
  const int64_t m_main = main_gemm_rows(M, N, K);
  if (m_main < M) {
    route.kind = GemmRoute::kPeel;
    route.m_main = m_main;
    route.ws_bytes = gemm_route(M - m_main, N, K, r, glu).ws_bytes;
    return route;
  }
  if (band_blocks_n(M, N, r, glu)) {
    route.kind = GemmRoute::kBand;
    return route;
  }
  if (use_mid_gemm(M, N, K, r, glu)) {
    route.kind = GemmRoute::kMid;
    return route;
  }
  if (use_skinny_fused(M, N)) {
    route.kind = GemmRoute::kSkinnyFused;
    return route;
  }
  route.plan = gemm_plan(M, N, K);
  if (route.plan.splits > 1 || route.plan.skinny) {
    route.kind = GemmRoute::kSplit;
    route.ws_bytes = (int64_t)route.plan.splits * partial_plane_ints(M, N) * 4;
  }
  return route;
}

bool is_glu(int act_code) { return act_code == HF_ACT_SWIGLU || act_code == HF_ACT_SWIGLU_GATE_FIRST; }

// Whether the low-rank up projection runs on the persistent 256 x 256 tiles (int8_gemm_kernel's bf16 product): its
// output fills at least one round of them. Its K (the rank) is small, so the output (2 bytes per element) and the
// operand rows re-read per tile are the traffic; 256 x 256 tiles read 4 operand bytes per output element against
// 8 for the 128 x 128 tiles of lowrank_up_kernel, and their stores leave the CU as whole lines behind the next
// tile's loads. From rank 128: at M=37710 the up projection to N=7168 took 180-220 us on the tiles against 207-270
// us at rank 256, but 120-140 against 112-120 us at rank 64, where a tile's two stages (one of them zeros) are too
// short for the persistent pipeline to pay.
bool use_up_tiles(int64_t M, int64_t N, int32_t r) {
  return r >= 128 && ((M + hf::GBM - 1) / hf::GBM) * ((N + hf::GBN - 1) / hf::GBN) >= device_cus();
}

int64_t gemm_ws_bytes(int64_t M, int64_t N, int64_t K, int32_t r, int act_code) {
  if (M <= 0 || N <= 0 || K <= 0 || r < 0) return 0;
  return gemm_route(M, N, K, r, is_glu(act_code)).ws_bytes;
}

int int8_linear_impl(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx, const float* sw,
                     const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r,
                     const uint16_t* bias, uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                     int64_t ws_bytes, hf_stream_t stream, int act_code = HF_ACT_NONE) {
  if (act_code < HF_ACT_NONE || act_code > HF_ACT_SWIGLU_GATE_FIRST) return HF_ERR_ARGUMENT;
  const bool glu = is_glu(act_code);
  const int act = glu ? hf::kActSwiGLU : (act_code == HF_ACT_GELU_TANH ? hf::kActGeluTanh : hf::kActNone);
  // SwiGLU: the N weight rows are F hidden and F gate rows (F = N / 2 output columns), F a multiple of 16.
  if (glu && (N < 0 || N % 32)) return HF_ERR_ARGUMENT;
  const int64_t n_out = glu ? N / 2 : N;
  if (M == 0 || N == 0) return (M < 0 || N < 0) ? HF_ERR_ARGUMENT : HF_OK;
  int st = check_gemm_operands(q, ldq, w, ldw, M, N, K);
  if (st != HF_OK) return st;
  if (!sx || !sw || !y || ldy < n_out || r < 0) return HF_ERR_ARGUMENT;
  if (!aligned(y, 8)) return HF_ERR_ALIGNMENT;
  if (r > 0) {
    if (!u || !up || ldu < r || ld_up < r) return HF_ERR_ARGUMENT;
    if ((r % 8) || !aligned(u, 16) || !aligned(up, 16) || (ldu % 8) || (ld_up % 8)) return HF_ERR_ALIGNMENT;
    if (512 * ldu >= (int64_t(1) << 31) || 512 * ld_up >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  }
  // Pair order reads the weight (and up) through one buffer descriptor each: 32-bit byte offsets.
  if (glu && (N * ldw >= (int64_t(1) << 32) || (r > 0 && N * ld_up * 2 >= (int64_t(1) << 32)))) return HF_ERR_SIZE;
  const int glu_half = (int)(N / 2), glu_gate_first = act_code == HF_ACT_SWIGLU_GATE_FIRST;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const GemmRoute route = gemm_route(M, N, K, r, glu);
  // A route that needs a workspace falls back to whole tiles when the caller's is missing or too small.
  const bool ws_ok = route.ws_bytes == 0 || (ws && aligned(ws, 16) && ws_bytes >= route.ws_bytes);
  if (route.kind == GemmRoute::kPeel && ws_ok) {
    // The trailing rows by their own route (a split-K GEMM, or one of the few-row kernels; bitwise the same
    // outputs: the partial sums are exact and every path applies the same epilogue), then the rest as whole tiles;
    // the same stream orders the two.
    const int64_t m_main = route.m_main;
    st = int8_linear_impl(q + m_main * ldq, ldq, w, ldw, sx + m_main, sw, r > 0 ? u + m_main * ldu : u, ldu, up,
                          ld_up, r, bias, y + m_main * ldy, ldy, M - m_main, N, K, ws, ws_bytes, stream, act_code);
    if (st != HF_OK) return st;
    return int8_linear_impl(q, ldq, w, ldw, sx, sw, u, ldu, up, ld_up, r, bias, y, ldy, m_main, N, K, nullptr, 0,
                            stream, act_code);
  }
  if (route.kind == GemmRoute::kBand) {
    allow_large_lds();
    const int nb = band_blocks_n(M, N, r, glu);
    hf::MidArgs a{};
    a.q = q; a.ldq = ldq; a.w = w; a.ldw = ldw; a.sx = sx; a.sw = sw;
    a.u = r > 0 ? u : nullptr; a.ldu = ldu; a.up = r > 0 ? up : nullptr; a.ldup = ld_up; a.r = r;
    a.bias = bias; a.y = y; a.ldy = ldy; a.M = (int)M; a.N = (int)N; a.K = (int)K;
    a.tiles_m = (int)((M + hf::kBandBM - 1) / hf::kBandBM);
    a.tiles_n = (int)((N + 32 * nb - 1) / (32 * nb));
    a.out_vec16 = aligned(y, 16) && (ldy % 8) == 0;
    const dim3 grid((unsigned)((int64_t)a.tiles_m * a.tiles_n)), block(hf::kBandThreads);
#define HF_BAND_LAUNCH(NB)                                                                                          \
    if (act == hf::kActGeluTanh)                                                                                    \
      hipLaunchKernelGGL((hf::band_gemm_kernel<NB, hf::kActGeluTanh>), grid, block, hf::band_lds(NB), s, a);        \
    else                                                                                                            \
      hipLaunchKernelGGL((hf::band_gemm_kernel<NB, hf::kActNone>), grid, block, hf::band_lds(NB), s, a);
    if (nb == 5) { HF_BAND_LAUNCH(5) } else if (nb == 4) { HF_BAND_LAUNCH(4) } else { HF_BAND_LAUNCH(3) }
#undef HF_BAND_LAUNCH
    return launch_status();
  }
  if (route.kind == GemmRoute::kMid) {
    allow_large_lds();
    hf::MidArgs a{};
    a.q = q; a.ldq = ldq; a.w = w; a.ldw = ldw; a.sx = sx; a.sw = sw;
    a.u = r > 0 ? u : nullptr; a.ldu = ldu; a.up = r > 0 ? up : nullptr; a.ldup = ld_up; a.r = r;
    a.bias = bias; a.y = y; a.ldy = ldy; a.M = (int)M; a.N = (int)N; a.K = (int)K;
    a.tiles_m = (int)((M + hf::kMidBM - 1) / hf::kMidBM);
    a.tiles_n = (int)((N + hf::kMidBN - 1) / hf::kMidBN);
    a.out_vec16 = aligned(y, 16) && (ldy % 8) == 0;
    const dim3 grid((unsigned)((int64_t)a.tiles_m * a.tiles_n)), block(hf::kMidThreads);
    if (act == hf::kActGeluTanh)
      hipLaunchKernelGGL(hf::mid_gemm_kernel<hf::kActGeluTanh>, grid, block, hf::kMidLds, s, a);
    else
      hipLaunchKernelGGL(hf::mid_gemm_kernel<hf::kActNone>, grid, block, hf::kMidLds, s, a);
    return launch_status();
  }
  if (route.kind == GemmRoute::kSkinnyFused) {
    // At most 64 rows: one pass, 32 weight rows per workgroup with the whole K, the epilogue in the same kernel.
    allow_large_lds();
    const int vec = aligned(y, 8) && (ldy % 4) == 0;
    const int gh = glu ? glu_half : 0, gf = glu ? glu_gate_first : 0;
    // Weight rows per workgroup: the fewest (a multiple of 4, at most 32) that spread the slices over every CU; pair
    // order keeps whole 32-column blocks. Against 32-row slices on N / 32 CUs (same box, graph replays): M=64,
    // N=K=5120 20.4 -> 18.4 us, N=4096 18.7 -> 16.3 us, N=K=3072 14.3 -> 12.9 us, M=16 16.9 -> 15.9 us.
    const int64_t cus = device_cus();
    const int rows = glu ? hf::kSfN : (int)std::min<int64_t>(hf::kSfN, ((N + cus - 1) / cus + 3) / 4 * 4);
    const dim3 grid((unsigned)((N + rows - 1) / rows)), block(64 * hf::kSfWaves);
#define HF_SF_LAUNCH(MR, GLU)                                                                                       \
  hipLaunchKernelGGL((hf::skinny_fused_kernel<MR, GLU>), grid, block, hf::sf_lds(MR), s, q, ldq, w, ldw, sx, sw,     \
                     r > 0 ? u : nullptr, ldu, r > 0 ? up : nullptr, ld_up, r, bias, y, ldy, (int)M, (int)N, (int)K, \
                     vec, act, gh, gf, rows)
    if (glu) HF_SF_LAUNCH(64, true); else HF_SF_LAUNCH(64, false);
#undef HF_SF_LAUNCH
    return launch_status();
  }
  const GemmPlan& plan = route.plan;
  const int64_t plane = partial_plane_ints(M, N);
  if (route.kind == GemmRoute::kSplit && ws_ok) {
    // Split K: int32 partial planes (block by block; in pair order with SwiGLU), then one pass that adds them and
    // applies the epilogue.
    if (plan.skinny) {
      allow_large_lds();
      const dim3 grid((unsigned)((N + hf::kSkinnyN - 1) / hf::kSkinnyN), (unsigned)plan.splits);
      int32_t* part = static_cast<int32_t*>(ws);
      const int gh = glu ? glu_half : 0, gf = glu ? glu_gate_first : 0;
#define HF_SKINNY_LAUNCH(GLU, MR)                                                                                   \
  hipLaunchKernelGGL((hf::skinny_gemm_kernel<GLU, MR>), grid, dim3(64 * hf::skinny_waves(MR)), hf::skinny_lds(MR), \
                     s, q, ldq, w, ldw,                                                                            \
                     part, plane, (int)M, (int)N, (int)K, plan.k_chunk, gh, gf)
      if (plan.mr == 64) {
        if (glu) HF_SKINNY_LAUNCH(true, 64); else HF_SKINNY_LAUNCH(false, 64);
      } else if (plan.mr == 128) {
        if (glu) HF_SKINNY_LAUNCH(true, 128); else HF_SKINNY_LAUNCH(false, 128);
      } else {
        if (glu) HF_SKINNY_LAUNCH(true, 256); else HF_SKINNY_LAUNCH(false, 256);
      }
#undef HF_SKINNY_LAUNCH
      st = launch_status();
    } else {
      hf::GemmArgs a{};
      a.q = q; a.ldq = ldq; a.w = w; a.ldw = ldw; a.out = ws; a.ldo = 0;
      a.M = (int)M; a.N = (int)N; a.K = (int)K; a.out_vec16 = 1;
      a.splits = plan.splits; a.k_chunk = plan.k_chunk; a.split_stride = plane;
      a.glu_half = glu_half; a.glu_gate_first = glu_gate_first;
      st = launch_gemm(a, true, s, act);
    }
    if (st != HF_OK) return st;
    const int64_t tiles_n = (N + hf::kSkTileN - 1) / hf::kSkTileN;
    const int64_t blocks = ((M + hf::kSkTileM - 1) / hf::kSkTileM) * tiles_n;
    if (blocks >= (int64_t(1) << 31)) return HF_ERR_SIZE;
    const int vec = aligned(y, 8) && (ldy % 4) == 0;
    hipLaunchKernelGGL(hf::splitk_epilogue_kernel, dim3((unsigned)blocks), dim3(64), 0, s,
                       static_cast<const int32_t*>(ws), plane, plan.splits, sx, sw, r > 0 ? u : nullptr, ldu,
                       r > 0 ? up : nullptr, ld_up, r, bias, y, ldy, (int)M, (int)N, (int)tiles_n, vec, act, glu_half,
                       glu_gate_first);
    return launch_status();
  }
  hf::GemmArgs a{};
  a.q = q; a.ldq = ldq; a.w = w; a.ldw = ldw; a.sx = sx; a.sw = sw;
  a.u = r > 0 ? u : nullptr; a.ldu = ldu; a.up = r > 0 ? up : nullptr; a.ldup = ld_up; a.r = r;
  a.bias = bias; a.out = y; a.ldo = ldy; a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.out_vec16 = aligned(y, 16) && (ldy % 8) == 0;
  a.glu_half = glu_half; a.glu_gate_first = glu_gate_first;
  return launch_gemm(a, false, s, act);
}


// hf_rotate_quant's work. fin: the layer's low-rank partial sums, added by the rotation kernels for their rows
// (the row and register kernels) or by lowrank_reduce_kernel after the rotation; part null: none. dry: only the
// argument checks (the status the call would return before launching anything).
int rotate_quant_bf16(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, int64_t M, int64_t K,
                      int32_t group, hipStream_t s, const hf::LrFinish& fin, bool dry) {
  if (M < 0 || K <= 0 || ldx < K || ldq < K) return HF_ERR_ARGUMENT;
  if (M == 0) return HF_OK;
  if (!x || !q || !sx) return HF_ERR_ARGUMENT;
  const int lg = log4_of(group);
  if (lg < 0 || K % group) return HF_ERR_GROUP;
  if (K % 16 || !aligned(x, 16) || !aligned(q, 16) || (ldx % 8) || (ldq % 16)) return HF_ERR_ALIGNMENT;
  int waves = 4;
  while (waves > 0 && hf::rotate_quant_lds_bytes(waves, (int)std::min<int64_t>(K, 1 << 30)) > (size_t)kMaxLds)
    waves >>= 1;
  if (lg < 6 && (waves == 0 || K > 77312)) return HF_ERR_SIZE;
  if (lg >= 6 && (hf::rotate_quant_wide_lds_bytes((int)std::min<int64_t>(K, 1 << 20)) > (size_t)kMaxLds ||
                  M >= (int64_t(1) << 31)))
    return HF_ERR_SIZE;
  if (dry) return HF_OK;
  // The low-rank sums for the routes whose kernels do not add them.
  auto reduce_after = [&](int st) {
    if (st != HF_OK || !fin.part) return st;
    const int64_t n = fin.M * fin.r;
    hipLaunchKernelGGL(hf::lowrank_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, fin.part,
                       fin.splits, fin.u, fin.ldu, (int)fin.M, fin.r);
    return launch_status();
  };
  if (lg >= 6) return reduce_after(launch_rotate_wide(false, lg, x, ldx, q, ldq, sx, M, K, s));
  allow_large_lds();
  const int64_t ntiles = (K + hf::kRqTile - 1) / hf::kRqTile;
  // Few rows: one workgroup per row, one wave per tile, while the rows fit two rounds of workgroups (the row
  // buffer and transpose areas take up to 157 KiB per workgroup: at M=1024, K=13824 the register kernel below took
  // 15.8 us against 20.3; at K=5120, two workgroups per CU, the row kernel stays ahead up to 1024 rows).
  const int64_t row_wgs_per_cu = std::max<int64_t>(1, kMaxLds / (int64_t)hf::rotate_quant_row_lds_bytes((int)K));
  if (M <= kRowKernelMaxRows && M <= 2 * row_wgs_per_cu * device_cus() && ntiles <= 14) {
    const size_t lds = hf::rotate_quant_row_lds_bytes((int)K);
    const dim3 grid((unsigned)M), block((unsigned)(64 * ntiles));
    switch (lg) {
      case 1: hipLaunchKernelGGL(hf::rotate_quant_row_kernel<1>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, fin); break;
      case 2: hipLaunchKernelGGL(hf::rotate_quant_row_kernel<2>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, fin); break;
      case 3: hipLaunchKernelGGL(hf::rotate_quant_row_kernel<3>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, fin); break;
      case 4: hipLaunchKernelGGL(hf::rotate_quant_row_kernel<4>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, fin); break;
      default: hipLaunchKernelGGL(hf::rotate_quant_row_kernel<5>, grid, block, lds, s, x, ldx, q, ldq, sx, (int)K, fin); break;
    }
    return launch_status();
  }
  if (ntiles <= 4 * hf::kRqRegMaxTpw) return rotate_rows_in_registers(false, lg, x, ldx, q, ldq, sx, M, K, s, fin);
  const size_t lds = hf::rotate_quant_lds_bytes(waves, (int)K);
  const int64_t blocks64 = (M + waves - 1) / waves;
  const unsigned blocks = (unsigned)std::min<int64_t>(blocks64, int64_t(1) << 30);
  switch (lg) {
    case 1: hipLaunchKernelGGL(hf::rotate_quant_kernel<1>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    case 2: hipLaunchKernelGGL(hf::rotate_quant_kernel<2>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    case 3: hipLaunchKernelGGL(hf::rotate_quant_kernel<3>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    case 4: hipLaunchKernelGGL(hf::rotate_quant_kernel<4>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    default: hipLaunchKernelGGL(hf::rotate_quant_kernel<5>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
  }
  return reduce_after(launch_status());
}

}  // namespace

extern "C" {

const char* hf_version(void) { return "hf_convrot 0.1.0 gfx950"; }

const char* hf_strerror(int status) {
  switch (status) {
    case HF_OK: return "ok";
    case HF_ERR_ARGUMENT: return "invalid argument (null pointer, negative size or stride smaller than the row)";
    case HF_ERR_GROUP: return "unsupported Hadamard group (a power of 4 from 4 to 16384, dividing K)";
    case HF_ERR_ALIGNMENT: return "pointer or stride breaks the 16-byte alignment rules";
    case HF_ERR_LAUNCH: return "HIP kernel launch failed";
    case HF_ERR_SIZE: return "size exceeds the kernels' index range";
    case HF_ERR_SCRATCH:
      return "the call needs more workspace than hf_convrot_linear_noalloc's 64 MiB scratch (use hf_convrot_linear_ws)";
    default: return "unknown status";
  }
}

int hf_rotate_quant(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, int64_t M, int64_t K,
                    int32_t group, hf_stream_t stream) {
  return rotate_quant_bf16(x, ldx, q, ldq, sx, M, K, group, static_cast<hipStream_t>(stream), hf::LrFinish{}, false);
}

int hf_rotate_quant_ex(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, int64_t M, int64_t K,
                       int32_t group, int32_t arithmetic, hf_stream_t stream) {
  if (arithmetic == HF_ROTATE_BF16_DIV) return hf_rotate_quant(x, ldx, q, ldq, sx, M, K, group, stream);
  if (arithmetic != HF_ROTATE_F32_RECIP) return HF_ERR_ARGUMENT;
  if (M < 0 || K <= 0 || ldx < K || ldq < K) return HF_ERR_ARGUMENT;
  if (M == 0) return HF_OK;
  if (!x || !q || !sx) return HF_ERR_ARGUMENT;
  const int lg = log4_of(group);
  if (lg < 0 || K % group) return HF_ERR_GROUP;
  if (K % 16 || !aligned(x, 16) || !aligned(q, 16) || (ldx % 8) || (ldq % 16)) return HF_ERR_ALIGNMENT;
  if (K >= (int64_t(1) << 30)) return HF_ERR_SIZE;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (lg >= 6) return launch_rotate_wide(true, lg, x, ldx, q, ldq, sx, M, K, s);
  // Up to 20 tiles the row stays in registers and x is read once; wider rows take the two-pass kernel below.
  if ((K + hf::kRqTile - 1) / hf::kRqTile <= 4 * hf::kRqRegMaxTpw)
    return rotate_rows_in_registers(true, lg, x, ldx, q, ldq, sx, M, K, s, hf::LrFinish{});
  constexpr int waves = 4;
  const size_t lds = hf::rotate_quant_f32_recip_lds_bytes(waves);
  const unsigned blocks = (unsigned)std::min<int64_t>((M + waves - 1) / waves, int64_t(1) << 30);
  switch (lg) {
    case 1: hipLaunchKernelGGL(hf::rotate_quant_f32_recip_kernel<1>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    case 2: hipLaunchKernelGGL(hf::rotate_quant_f32_recip_kernel<2>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    case 3: hipLaunchKernelGGL(hf::rotate_quant_f32_recip_kernel<3>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    case 4: hipLaunchKernelGGL(hf::rotate_quant_f32_recip_kernel<4>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
    default: hipLaunchKernelGGL(hf::rotate_quant_f32_recip_kernel<5>, dim3(blocks), dim3(64 * waves), lds, s, x, ldx, q, ldq, sx, M, (int)K); break;
  }
  return launch_status();
}

int hf_lowrank_down(const uint16_t* x, int64_t ldx, const uint16_t* down, int64_t ld_down, uint16_t* u,
                    int64_t ldu, int64_t M, int64_t K, int32_t r, hf_stream_t stream) {
  return lowrank_down_impl(x, ldx, down, ld_down, u, ldu, M, K, r, nullptr, 0, stream);
}

int hf_lowrank_up(const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias,
                  uint16_t* y, int64_t ldy, int64_t M, int64_t N, hf_stream_t stream) {
  if (M < 0 || N < 0 || r < 0 || ldu < r || ld_up < r || ldy < N) return HF_ERR_ARGUMENT;
  if (M == 0 || N == 0) return HF_OK;
  if (!y || (r > 0 && (!u || !up))) return HF_ERR_ARGUMENT;
  if ((r % 8) || (r > 0 && (!aligned(u, 16) || !aligned(up, 16))) || (ldu % 8) || (ld_up % 8) || !aligned(y, 2))
    return HF_ERR_ALIGNMENT;
  if (M >= (int64_t(1) << 31) || N >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  if (2 * hf::kUpTile * std::max(ldu, ld_up) >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  allow_large_lds();
  const int vec16 = aligned(y, 16) && (ldy % 8) == 0;
  if (vec16 && use_up_tiles(M, N, r)) {
    // At least a round of 256 x 256 output tiles: the persistent tile kernel's bf16 product (kOutMmBf16), the
    // operands' rows as bytes (2r bytes of rank per row).
    hf::GemmArgs a{};
    a.q = reinterpret_cast<const int8_t*>(u); a.ldq = 2 * ldu;
    a.w = reinterpret_cast<const int8_t*>(up); a.ldw = 2 * ld_up;
    a.bias = bias; a.out = y; a.ldo = ldy;
    a.M = (int)M; a.N = (int)N; a.K = 2 * r; a.out_vec16 = 1;
    a.tiles_m = (int)((M + hf::GBM - 1) / hf::GBM);
    a.tiles_n = (int)((N + hf::GBN - 1) / hf::GBN);
    a.splits = 1;
    a.k_chunk = (int)((a.K + hf::GBK - 1) / hf::GBK * hf::GBK);
    const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
    if (tiles >= (int64_t(1) << 31)) return HF_ERR_SIZE;
    hipLaunchKernelGGL(hf::int8_gemm_kernel<hf::kOutMmBf16>, dim3((unsigned)gemm_grid(tiles)), dim3(hf::kThreads),
                       hf::kGemmLds, static_cast<hipStream_t>(stream), a);
    return launch_status();
  }
  const int64_t tiles_n = (N + hf::kUpTile - 1) / hf::kUpTile, tiles = ((M + hf::kUpTile - 1) / hf::kUpTile) * tiles_n;
  if (tiles >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  hipLaunchKernelGGL(hf::lowrank_up_kernel, dim3((unsigned)tiles), dim3(hf::kUpThreads), hf::kUpLds,
                     static_cast<hipStream_t>(stream), u, ldu, up, ld_up, bias, y, ldy, (int)M, (int)N, (int)r,
                     (int)tiles_n, vec16);
  return launch_status();
}

int hf_int8_linear(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx, const float* sw,
                   const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias,
                   uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hf_stream_t stream) {
  return int8_linear_impl(q, ldq, w, ldw, sx, sw, u, ldu, up, ld_up, r, bias, y, ldy, M, N, K, nullptr, 0, stream);
}

int64_t hf_int8_linear_ws_bytes(int64_t M, int64_t N, int64_t K, int32_t r, int32_t activation) {
  return gemm_ws_bytes(M, N, K, r, activation);
}

int hf_int8_linear_ws(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx, const float* sw,
                      const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r,
                      const uint16_t* bias, uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                      int64_t ws_bytes, hf_stream_t stream) {
  return int8_linear_impl(q, ldq, w, ldw, sx, sw, u, ldu, up, ld_up, r, bias, y, ldy, M, N, K, ws, ws_bytes, stream);
}

int hf_int8_linear_act_ws(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx,
                          const float* sw, const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up,
                          int32_t r, const uint16_t* bias, int32_t activation, uint16_t* y, int64_t ldy, int64_t M,
                          int64_t N, int64_t K, void* ws, int64_t ws_bytes, hf_stream_t stream) {
  return int8_linear_impl(q, ldq, w, ldw, sx, sw, u, ldu, up, ld_up, r, bias, y, ldy, M, N, K, ws, ws_bytes, stream,
                          activation);
}

int64_t hf_lowrank_down_ws_bytes(int64_t M, int64_t K, int32_t r) {
  if (M <= 0 || K <= 0 || r <= 0) return 0;
  return lowrank_ws_bytes(M, K, std::min<int32_t>(r, hf::kLrRanks));
}

int hf_lowrank_down_ws(const uint16_t* x, int64_t ldx, const uint16_t* down, int64_t ld_down, uint16_t* u,
                       int64_t ldu, int64_t M, int64_t K, int32_t r, void* ws, int64_t ws_bytes, hf_stream_t stream) {
  return lowrank_down_impl(x, ldx, down, ld_down, u, ldu, M, K, r, ws, ws_bytes, stream);
}

int hf_int8_gemm_i32(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, int32_t* acc, int64_t ldacc,
                     int64_t M, int64_t N, int64_t K, hf_stream_t stream) {
  if (M == 0 || N == 0) return (M < 0 || N < 0) ? HF_ERR_ARGUMENT : HF_OK;
  int st = check_gemm_operands(q, ldq, w, ldw, M, N, K);
  if (st != HF_OK) return st;
  if (!acc || ldacc < N) return HF_ERR_ARGUMENT;
  if (!aligned(acc, 16)) return HF_ERR_ALIGNMENT;
  hf::GemmArgs a{};
  a.q = q; a.ldq = ldq; a.w = w; a.ldw = ldw; a.out = acc; a.ldo = ldacc;
  a.M = (int)M; a.N = (int)N; a.K = (int)K;
  a.out_vec16 = (ldacc % 4) == 0;
  return launch_gemm(a, true, static_cast<hipStream_t>(stream));
}

int hf_convrot_linear(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* sw,
                      const uint16_t* down, int64_t ld_down, const uint16_t* up, int64_t ld_up, int32_t r,
                      const uint16_t* bias, int32_t group, int8_t* q_ws, float* sx_ws, uint16_t* u_ws, uint16_t* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, hf_stream_t stream) {
  int st = hf_rotate_quant(x, ldx, q_ws, K, sx_ws, M, K, group, stream);
  if (st != HF_OK) return st;
  if (r > 0) {
    st = hf_lowrank_down(x, ldx, down, ld_down, u_ws, r, M, K, r, stream);
    if (st != HF_OK) return st;
  }
  return hf_int8_linear(q_ws, K, w, ldw, sx_ws, sw, u_ws, r, up, ld_up, r, bias, y, ldy, M, N, K, stream);
}

}  // extern "C"

namespace {

// The rotation (bf16_div arithmetic) and the low-rank down projection of a few rows in one launch
// (rotate_lowrank_row_kernel): the argument rules of hf_rotate_quant and hf_lowrank_down together. Used when both
// would run their row kernels and the rows are few: the low-rank workgroups take the rotation's dynamic LDS (about
// 11 KiB per 1024-element tile), so with more rows they fit fewer per CU than alone. Layer A/B (HIP graph, N=5120,
// rank 64): one launch ahead by 1-5 us up to 128 rows at every K and up to 192 rows at 7 or fewer tiles; behind by
// 1-8 us at 256-384 rows with K=5120 or K=14336.
bool rotate_lowrank_by_rows(int64_t M, int64_t K) {
  const int64_t ntiles = (K + hf::kRqTile - 1) / hf::kRqTile;
  return lowrank_by_rows(M, K) && M <= kRowKernelMaxRows && ntiles <= 14 && (M <= 128 || (M <= 192 && ntiles <= 7));
}

int rotate_lowrank_rows(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, const uint16_t* down,
                        int64_t ld_down, uint16_t* u, int64_t ldu, int64_t M, int64_t K, int32_t r, int32_t group,
                        hf_stream_t stream) {
  if (M < 0 || K <= 0 || r < 0 || ldx < K || ldq < K || ld_down < K || ldu < r) return HF_ERR_ARGUMENT;
  if (M == 0) return HF_OK;
  if (!x || !q || !sx || !down || !u) return HF_ERR_ARGUMENT;
  const int lg = log4_of(group);
  if (lg < 0 || lg > 5 || K % group) return HF_ERR_GROUP;
  if (K % 16 || !aligned(x, 16) || !aligned(q, 16) || (ldx % 8) || (ldq % 16) || !aligned(down, 16) ||
      (ld_down % 8) || !aligned(u, 8))
    return HF_ERR_ALIGNMENT;
  const int64_t groups = (r + hf::kLrRowRanks - 1) / hf::kLrRowRanks;
  const int64_t blocks = hf::lowrank_row_blocks(M, r) + M;
  if (blocks >= (int64_t(1) << 31)) return HF_ERR_SIZE;
  allow_large_lds();
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t lds = hf::rotate_quant_row_lds_bytes((int)K);
  const dim3 grid((unsigned)blocks), block((unsigned)(64 * ((K + hf::kRqTile - 1) / hf::kRqTile)));
#define HF_RLR(G)                                                                                                   \
  hipLaunchKernelGGL(hf::rotate_lowrank_row_kernel<G>, grid, block, lds, s, x, ldx, q, ldq, sx, down, ld_down, u, \
                     ldu, (int)M, (int)K, r, (int)groups)
  switch (lg) {
    case 1: HF_RLR(1); break;
    case 2: HF_RLR(2); break;
    case 3: HF_RLR(3); break;
    case 4: HF_RLR(4); break;
    default: HF_RLR(5); break;
  }
#undef HF_RLR
  return launch_status();
}

}  // namespace

extern "C" {

int64_t hf_convrot_linear_ws_bytes(int64_t M, int64_t N, int64_t K, int32_t r, int32_t activation) {
  if (M <= 0 || N <= 0 || K <= 0 || r < 0) return 0;
  const int64_t lr = r > 0 ? lowrank_ws_bytes(M, K, std::min<int32_t>(r, hf::kLrRanks)) : 0;
  return std::max<int64_t>(lr, gemm_ws_bytes(M, N, K, r, activation));
}

int hf_convrot_linear_ws(const uint16_t* x, int64_t ldx, int8_t* q, float* sx, int32_t quantized, int32_t arithmetic,
                         const int8_t* w, int64_t ldw, const float* sw, const uint16_t* down, int64_t ld_down,
                         const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias, int32_t activation,
                         int32_t group, uint16_t* u, uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                         void* ws, int64_t ws_bytes, hf_stream_t stream) {
  if (M < 0 || N < 0 || K <= 0 || r < 0) return HF_ERR_ARGUMENT;
  if (M == 0 || N == 0) return HF_OK;
  int st = HF_OK;
  if (!quantized && r > 0 && arithmetic == HF_ROTATE_BF16_DIV && group <= 1024 && rotate_lowrank_by_rows(M, K)) {
    st = rotate_lowrank_rows(x, ldx, q, K, sx, down, ld_down, u, r, M, K, r, group, stream);
    if (st != HF_OK) return st;
  } else if (!quantized && r > 0 && arithmetic == HF_ROTATE_BF16_DIV && lowrank_split_planned(M, K, r, ws, ws_bytes)) {
    // The low-rank projection splits K: it runs first and the rotation kernel adds its partial sums for the rows it
    // rotates (one launch fewer; the same sums in the same order: M=1024, K=N=3072, rank 32, bias 37.9 -> 35.1 us, M=1024, N=K=5120
    // 59.9 -> 57.4 us). Without a split the projection stays the last reader of x (its loads keep x out of the
    // Infinity Cache, over the codes the GEMM reads next): run first, it cost 0.6-0.8 % at M=32768 and M=256. The
    // rotation's arguments are checked before anything runs. The low-rank partials and the GEMM's partial planes
    // share the workspace: they are used one after the other.
    hipStream_t s = static_cast<hipStream_t>(stream);
    st = rotate_quant_bf16(x, ldx, q, K, sx, M, K, group, s, hf::LrFinish{}, true);
    if (st != HF_OK) return st;
    hf::LrFinish fin{};
    st = lowrank_down_impl(x, ldx, down, ld_down, u, r, M, K, r, ws, ws_bytes, stream, &fin);
    if (st != HF_OK) return st;
    st = rotate_quant_bf16(x, ldx, q, K, sx, M, K, group, s, fin, false);
    if (st != HF_OK) return st;
  } else {
    if (!quantized) {
      st = hf_rotate_quant_ex(x, ldx, q, K, sx, M, K, group, arithmetic, stream);
      if (st != HF_OK) return st;
    }
    if (r > 0) {
      // The low-rank partials and the GEMM's partial planes share the workspace: they are used one after the other.
      st = lowrank_down_impl(x, ldx, down, ld_down, u, r, M, K, r, ws, ws_bytes, stream);
      if (st != HF_OK) return st;
    }
  }
  return int8_linear_impl(q, K, w, ldw, sx, sw, u, r, up, ld_up, r, bias, y, ldy, M, N, K, ws, ws_bytes, stream,
                          activation);
}

}  // extern "C"

// ------------------------------------------------------------------------------------- allocation-free entry point

// The workspace of hf_convrot_linear_noalloc: the split-K partial planes and low-rank partial sums of one call, in
// device memory that the code object itself holds (each device that loads the library keeps its own copy until the
// process ends). Every call on a device reuses that device's copy; nothing in it needs clearing, since each split
// writes every element of its partial plane (or partial sums) before the finishing pass reads it.
constexpr int64_t kScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;

// The device address of `scratch` on the current device, looked up once per device (the host-side name is a
// stand-in, not a device address). Null when the lookup fails.
void* scratch_address() {
  static std::mutex lock;
  static void* addr[kMaxScratchDevices] = {nullptr};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return nullptr;
  std::lock_guard<std::mutex> guard(lock);
  if (!addr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    addr[dev] = p;
  }
  return addr[dev];
}

}  // namespace

extern "C" {

int64_t hf_convrot_linear_noalloc_max_bytes(void) { return kScratchBytes; }

int hf_convrot_linear_noalloc(const uint16_t* x, int64_t ldx, int8_t* q, float* sx, int32_t quantized,
                              int32_t arithmetic, const int8_t* w, int64_t ldw, const float* sw, const uint16_t* down,
                              int64_t ld_down, const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias,
                              int32_t activation, int32_t group, uint16_t* u, uint16_t* y, int64_t ldy, int64_t M,
                              int64_t N, int64_t K, hf_stream_t stream) {
  if (M < 0 || N < 0 || K <= 0 || r < 0) return HF_ERR_ARGUMENT;
  if (M == 0 || N == 0) return HF_OK;
  const int64_t need = hf_convrot_linear_ws_bytes(M, N, K, r, activation);
  if (need > kScratchBytes) return HF_ERR_SCRATCH;
  void* ws = need > 0 ? scratch_address() : nullptr;
  if (need > 0 && !ws) return HF_ERR_LAUNCH;
  return hf_convrot_linear_ws(x, ldx, q, sx, quantized, arithmetic, w, ldw, sw, down, ld_down, up, ld_up, r, bias,
                              activation, group, u, y, ldy, M, N, K, ws, need > 0 ? kScratchBytes : 0, stream);
}

}  // extern "C"
