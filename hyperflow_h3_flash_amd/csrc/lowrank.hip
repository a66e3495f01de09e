// Low-rank down projection u = bf16(x @ down^T), the first half of LowRankLinear.forward
// (src/hyperflow_h3_flash/transformer.py:57-58: `self.up(self.down(x))`, whose bf16 nn.Linear rounds `down(x)` to
// bf16 before `up`). Its output feeds the low-rank term of the fused INT8 GEMM epilogue.
//
// x is [M, K] bf16 and down is [r, K] bf16 (nn.Linear weight layout), both K-major; r <= 64 per launch (the host
// splits larger ranks). The kernel is a single streaming read of x: a workgroup owns 128 rows and walks K in stages
// of 64 elements. Each stage (the 128 x 64 slab of x, 16 KiB, and the 64 x 64 slab of down, 8 KiB) goes global -> LDS
// with buffer_load ... lds as whole 128-byte row segments into a 6-stage ring, so five stages (120 KiB) are in flight
// per CU while one is consumed. Each of the 4 waves multiplies its 32 rows against all ranks with
// v_mfma_f32_32x32x16_bf16 (first operand down, second x: lanes end with four consecutive rank columns of one row).
// The MFMA work is a few percent of the stage's memory time; `down` (r x K) streams from L2 once per 128 rows.
#include "common.h"

namespace hf {

constexpr int kLrRows = 128;                          // x rows per workgroup
constexpr int kLrRanks = 64;                          // ranks per launch
constexpr int kLrStageK = 64;                         // K elements per stage (128-byte row segments)
constexpr int kLrXBytes = kLrRows * kLrStageK * 2;    // 16 KiB
constexpr int kLrDBytes = kLrRanks * kLrStageK * 2;   // 8 KiB
constexpr int kLrStageBytes = kLrXBytes + kLrDBytes;  // 24 KiB
constexpr int kLrStages = 6;
constexpr int kLrLds = kLrStages * kLrStageBytes;     // 144 KiB
constexpr int kLrThreads = 256;

// LDS rows are 128 bytes (eight 16-byte chunks), swizzled with swizzle128 so fragment reads are conflict-free.
__device__ __forceinline__ int lr_swizzle(int row, int c) { return swizzle128(row, c); }

// One wave's share of a stage: `count` loads of 1 KiB (8 rows x 128 bytes) starting at LDS block `first_blk`.
// Rows at or past `rows_valid`, and chunks at or past K, read as zero (offset `oob` is past the descriptor).
template <int COUNT>
__device__ __forceinline__ void lr_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t oob, uint32_t ld_bytes, int rows_valid,
                                        int k0, int K, unsigned char HF_LDS* dst, int first_blk, int lane) {
#pragma unroll
  for (int i = 0; i < COUNT; ++i) {
    const int blk = first_blk + i;
    const int row = blk * 8 + (lane >> 3);
    const int c = lr_swizzle(row, lane & 7);
    const int k = k0 + c * 8;
    const uint32_t voff = (row < rows_valid && k < K) ? (uint32_t)row * ld_bytes + (uint32_t)k * 2u : oob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void HF_LDS*)(dst + blk * 1024), 16, voff, 0, 0, 0);
  }
}

template <int RB>
__global__ __launch_bounds__(kLrThreads, 1) void lowrank_down_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                     const uint16_t* __restrict__ down, int64_t ldd,
                                                                     uint16_t* __restrict__ u, int64_t ldu, int M,
                                                                     int K, int r) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char lr_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)lr_smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = blockIdx.x * kLrRows;
  const int rows_m = min(kLrRows, M - m0);

  const uint32_t ldx_bytes = (uint32_t)ldx * 2u, ldd_bytes = (uint32_t)ldd * 2u;
  const uint32_t bytes_x = (uint32_t)rows_m * ldx_bytes, bytes_d = (uint32_t)r * ldd_bytes;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (int64_t)m0 * ldx, bytes_x);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(down, bytes_d);

  // Stage t -> slot t % kLrStages; every stage issues 6 loads per wave (4 of x, 2 of down), stages past the end
  // load zeros, so "stage t has landed" is always vmcnt(24) with the four later stages in flight.
  auto issue = [&](int t) {
    unsigned char HF_LDS* st = smem + (t % kLrStages) * kLrStageBytes;
    lr_load<4>(rx, bytes_x, ldx_bytes, rows_m, t * kLrStageK, K, st, wave * 4, lane);
    lr_load<2>(rd, bytes_d, ldd_bytes, r, t * kLrStageK, K, st + kLrXBytes, wave * 2, lane);
  };

  v16f acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = (v16f){0};

  const int nst = (K + kLrStageK - 1) / kLrStageK;
#pragma unroll
  for (int t = 0; t < kLrStages - 1; ++t) issue(t);
  const int xrow = wave * 32 + sub;
  for (int t = 0; t < nst; ++t) {
    // This wave's loads of stage t have landed and its reads of slot (t - 1) % 6 have returned; the barrier (no
    // memory fence, which would also wait for the four stages behind) makes that true for every wave.
    asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(t + kLrStages - 1);
    const unsigned char HF_LDS* st = smem + (t % kLrStages) * kLrStageBytes;
#pragma unroll
    for (int s = 0; s < kLrStageK / 16; ++s) {
      const int c = 2 * s + half;
      const v8bf xf = *reinterpret_cast<const v8bf HF_LDS*>(st + xrow * 128 + lr_swizzle(xrow, c) * 16);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int drow = rb * 32 + sub;
        const v8bf df =
            *reinterpret_cast<const v8bf HF_LDS*>(st + kLrXBytes + drow * 128 + lr_swizzle(drow, c) * 16);
        acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(df, xf, acc[rb], 0, 0, 0);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // zero-fill loads past the end may still be landing

  const int row = m0 + xrow;
  if (row >= M) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int j = rb * 32 + 8 * g + 4 * half;
      uint16_t* dst = u + (int64_t)row * ldu + j;
      if (j + 3 < r && (ldu & 3) == 0) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(pack_bf16x2(acc[rb][4 * g], acc[rb][4 * g + 1]),
                                                    pack_bf16x2(acc[rb][4 * g + 2], acc[rb][4 * g + 3]));
      } else {
        for (int e = 0; e < 4; ++e)
          if (j + e < r) dst[e] = (uint16_t)f32_to_bf16_rne(acc[rb][4 * g + e]);
      }
    }
  }
}

template __global__ void lowrank_down_kernel<1>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                int64_t, int, int, int);
template __global__ void lowrank_down_kernel<2>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                int64_t, int, int, int);

}  // namespace hf
