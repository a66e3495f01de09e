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
#pragma once

#include "common.h"

namespace hf {

// A workgroup of NW waves (4..8) owns 32 NW x rows. The host picks NW so one round of workgroups covers the rows
// when it can (at most one workgroup per CU fits): 4 waves up to 256 CUs x 128 rows, more for a few more rows (the
// 5.2 s clip's 37710 tokens take 236 workgroups of 160 rows instead of 295 of 128, whose last 39 would run alone).
constexpr int kLrRows = 128;                          // x rows per workgroup with 4 waves (the split-K launches)
constexpr int kLrMaxWaves = 8;
constexpr int kLrMaxRows = 32 * kLrMaxWaves;
constexpr int kLrRanks = 64;                          // ranks per launch
constexpr int kLrStageK = 64;                         // K elements per stage (128-byte row segments)
constexpr int kLrDBytes = kLrRanks * kLrStageK * 2;   // 8 KiB of down per stage
constexpr int kLrThreads = 256;                       // with 4 waves

__host__ __device__ constexpr int lr_stage_bytes(int nw) { return nw * 32 * kLrStageK * 2 + kLrDBytes; }
// Ring depth: as many stages as fit 160 KiB, at most 6 (6 stages of 24 KiB with 4 waves).
__host__ __device__ constexpr int lr_stages(int nw) {
  return (160 * 1024) / lr_stage_bytes(nw) < 6 ? (160 * 1024) / lr_stage_bytes(nw) : 6;
}
__host__ __device__ constexpr int lr_lds(int nw) { return lr_stages(nw) * lr_stage_bytes(nw); }
constexpr int kLrLds = lr_lds(4);                     // 144 KiB

// LDS rows are 128 bytes (eight 16-byte chunks), swizzled with swizzle128 so fragment reads are conflict-free.
__device__ __forceinline__ int lr_swizzle(int row, int c) { return swizzle128(row, c); }

// One wave's share of a stage: `count` loads of 1 KiB (8 rows x 128 bytes) starting at LDS block `first_blk`.
// Rows at or past `rows_valid`, and chunks at or past K, read as zero (offset `oob` is past the descriptor).
// CPOL is the loads' cache policy: kCpolStream for x, which this pass reads last in a layer (after the rotation),
// so its 2 bytes per element are not kept in the Infinity Cache over the codes the GEMM reads next.
constexpr int kCpolStream = 2;  // the nt (non-temporal) bit
template <int COUNT, int CPOL = 0>
__device__ __forceinline__ void lr_load(__amdgpu_buffer_rsrc_t rsrc, uint32_t oob, uint32_t ld_bytes, int rows_valid,
                                        int k0, int K, unsigned char HF_LDS* dst, int first_blk, int lane) {
#pragma unroll
  for (int i = 0; i < COUNT; ++i) {
    const int blk = first_blk + i;
    const int row = blk * 8 + (lane >> 3);
    const int c = lr_swizzle(row, lane & 7);
    const int k = k0 + c * 8;
    const uint32_t voff = ((row < rows_valid) & (k < K)) ? (uint32_t)row * ld_bytes + (uint32_t)k * 2u : oob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void HF_LDS*)(dst + blk * 1024), 16, voff, 0, 0, CPOL);
  }
}

// Split K (few rows): blockIdx.y = s covers K elements [s * k_chunk, (s + 1) * k_chunk) and writes its fp32 partial
// sums to plane s of `part` ([splits][M][r]); lowrank_reduce_kernel, or in a layer the rotation kernel (LrFinish),
// adds the planes and rounds to bf16. Unsplit launches (gridDim.y == 1, part == nullptr) write u directly.
template <int RB, int NW = 4>
__global__ __launch_bounds__(64 * NW, 1) void lowrank_down_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                  const uint16_t* __restrict__ down, int64_t ldd,
                                                                  uint16_t* __restrict__ u, int64_t ldu, int M,
                                                                  int K, int r, int k_chunk,
                                                                  float* __restrict__ part) {
  constexpr int kRows = 32 * NW;
  constexpr int kXBytes = kRows * kLrStageK * 2;
  constexpr int kStageBytes = lr_stage_bytes(NW);
  constexpr int kStages = lr_stages(NW);
  static_assert(kStages >= 4 && kStages <= 6, "ring depth");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lr_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)lr_smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = blockIdx.x * kRows;
  const int rows_m = min(kRows, M - m0);

  const int k_lo = blockIdx.y * k_chunk;
  const int k_len = min(K - k_lo, k_chunk);
  const uint32_t ldx_bytes = (uint32_t)ldx * 2u, ldd_bytes = (uint32_t)ldd * 2u;
  const uint32_t bytes_x = (uint32_t)rows_m * ldx_bytes, bytes_d = (uint32_t)r * ldd_bytes;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (int64_t)m0 * ldx + k_lo, bytes_x - 2u * (uint32_t)k_lo);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(down + k_lo, bytes_d - 2u * (uint32_t)k_lo);

  // Stage t -> slot t % kStages; every stage issues 6 loads per wave (4 of its 32 x rows, 2 of the 8 blocks of
  // down: waves past the fourth load the first waves' blocks again, the same bytes to the same place, so every wave
  // issues the same count), stages past the end load zeros, so "stage t has landed" is always a constant vmcnt with
  // the kStages - 2 later stages in flight.
  auto issue = [&](int t) {
    unsigned char HF_LDS* st = smem + (t % kStages) * kStageBytes;
    lr_load<4, kCpolStream>(rx, bytes_x, ldx_bytes, rows_m, t * kLrStageK, k_len, st, wave * 4, lane);
    lr_load<2>(rd, bytes_d, ldd_bytes, r, t * kLrStageK, k_len, st + kXBytes, (wave % 4) * 2, lane);
  };

  v16f acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = (v16f){0};

  const int nst = (k_len + kLrStageK - 1) / kLrStageK;
#pragma unroll
  for (int t = 0; t < kStages - 1; ++t) issue(t);
  const int xrow = wave * 32 + sub;
  for (int t = 0; t < nst; ++t) {
    // This wave's loads of stage t have landed and its reads of slot (t - 1) % kStages have returned; the barrier (no
    // memory fence, which would also wait for the stages behind) makes that true for every wave.
    if constexpr (kStages == 6) {
      asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else if constexpr (kStages == 5) {
      asm volatile("s_waitcnt vmcnt(18) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
    issue(t + kStages - 1);
    const unsigned char HF_LDS* st = smem + (t % kStages) * kStageBytes;
    // All of the stage's fragments are read before its MFMAs (with one wave per SIMD nothing else hides a read the
    // compiler would otherwise place right before its MFMA): 0-1.6 % faster, the same sums in the same order.
    v8bf xf[kLrStageK / 16], df[kLrStageK / 16][RB];
#pragma unroll
    for (int s = 0; s < kLrStageK / 16; ++s) {
      const int c = 2 * s + half;
      xf[s] = *reinterpret_cast<const v8bf HF_LDS*>(st + xrow * 128 + lr_swizzle(xrow, c) * 16);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int drow = rb * 32 + sub;
        df[s][rb] = *reinterpret_cast<const v8bf HF_LDS*>(st + kXBytes + drow * 128 + lr_swizzle(drow, c) * 16);
      }
    }
#pragma unroll
    for (int s = 0; s < kLrStageK / 16; ++s)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
        acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(df[s][rb], xf[s], acc[rb], 0, 0, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, (kLrStageK / 16) * (1 + RB), 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, (kLrStageK / 16) * RB, 0);        // MFMA
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // zero-fill loads past the end may still be landing

  const int row = m0 + xrow;
  if (row >= M) return;
  if (part) {
    float* dst = part + ((int64_t)blockIdx.y * M + row) * r;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = rb * 32 + 8 * g + 4 * half + e;
          if (j < r) dst[j] = acc[rb][4 * g + e];
        }
    return;
  }
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

#define HF_LR_DOWN(RB, NW)                                                                                          \
  template __global__ void lowrank_down_kernel<RB, NW>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*, \
                                                       int64_t, int, int, int, int, float*);
HF_LR_DOWN(1, 4) HF_LR_DOWN(1, 5) HF_LR_DOWN(1, 6) HF_LR_DOWN(1, 7) HF_LR_DOWN(1, 8)
HF_LR_DOWN(2, 4) HF_LR_DOWN(2, 5) HF_LR_DOWN(2, 6) HF_LR_DOWN(2, 7) HF_LR_DOWN(2, 8)
#undef HF_LR_DOWN

// Ranks past 64 (the standalone low-rank linear's ranks are typically several hundred): lowrank_down_kernel would
// stream x once per 64 ranks. This kernel takes 256 ranks per pass over x: a workgroup of NR row blocks of 32 rows
// has two waves per row block, each multiplying its 32 rows against 128 of the ranks (four 32 x 32 MFMA blocks, the
// fragment layout and summation order of lowrank_down_kernel, so every u element is the same sum). A stage is the
// 32 NR x 64 slab of x and the 256 x 64 slab of down (48 or 52 KiB), in a 3-stage ring. Every wave issues the same
// six loads per stage (two of the x blocks of 8 rows, four of the 32 down blocks; with NR = 5 the last two waves
// load the first down blocks again: the same bytes to the same place).
constexpr int kLwRanks = 256;  // ranks per pass
constexpr int kLwStages = 3;
__host__ __device__ constexpr int lw_stage_bytes(int nr) { return nr * 32 * kLrStageK * 2 + kLwRanks * kLrStageK * 2; }
__host__ __device__ constexpr int lw_lds(int nr) { return kLwStages * lw_stage_bytes(nr); }

template <int NR>
__global__ __launch_bounds__(128 * NR, 1) void lowrank_down_wide_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                       const uint16_t* __restrict__ down,
                                                                       int64_t ldd, uint16_t* __restrict__ u,
                                                                       int64_t ldu, int M, int K, int r) {
  constexpr int kRows = 32 * NR;
  constexpr int kXBytes = kRows * kLrStageK * 2;
  constexpr int kStageBytes = lw_stage_bytes(NR);
  constexpr int kRB = 4;  // 32-rank blocks per wave
  static_assert(lw_lds(NR) <= 160 * 1024, "ring exceeds the LDS");
  static_assert((kRows / 8) % (2 * NR) == 0 && (kRows / 8) / (2 * NR) == 2, "two x blocks per wave");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lw_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)lw_smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 31, half = lane >> 5;
  const int rblock = wave % NR, rhalf = wave / NR;  // this wave's 32 rows and 128 ranks
  const int m0 = blockIdx.x * kRows;
  const int rows_m = min(kRows, M - m0);
  const uint32_t ldx_bytes = (uint32_t)ldx * 2u, ldd_bytes = (uint32_t)ldd * 2u;
  const uint32_t bytes_x = (uint32_t)rows_m * ldx_bytes, bytes_d = (uint32_t)r * ldd_bytes;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (int64_t)m0 * ldx, bytes_x);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(down, bytes_d);

  // Stages past the end load zeros, so "stage t has landed" is always vmcnt(6): one later stage (6 loads) in flight.
  auto issue = [&](int t) {
    unsigned char HF_LDS* st = smem + (t % kLwStages) * kStageBytes;
    lr_load<2, kCpolStream>(rx, bytes_x, ldx_bytes, rows_m, t * kLrStageK, K, st, wave * 2, lane);
    lr_load<4>(rd, bytes_d, ldd_bytes, r, t * kLrStageK, K, st + kXBytes, (wave * 4) % 32, lane);
  };

  v16f acc[kRB];
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) acc[rb] = (v16f){0};
  const bool live = rhalf * 128 < r;  // a wave whose ranks are all past r only loads
  const int nst = (K + kLrStageK - 1) / kLrStageK;
#pragma unroll
  for (int t = 0; t < kLwStages - 1; ++t) issue(t);
  const int xrow = rblock * 32 + sub;
  for (int t = 0; t < nst; ++t) {
    // This wave's loads of stage t have landed and its reads of slot (t - 1) % 3 have returned; the barrier makes
    // that true for every wave, so slot (t - 1) % 3 can take stage t + 2.
    asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(t + kLwStages - 1);
    if (!live) continue;
    const unsigned char HF_LDS* st = smem + (t % kLwStages) * kStageBytes;
#pragma unroll
    for (int s = 0; s < kLrStageK / 16; ++s) {
      const int c = 2 * s + half;
      const v8bf xf = *reinterpret_cast<const v8bf HF_LDS*>(st + xrow * 128 + lr_swizzle(xrow, c) * 16);
#pragma unroll
      for (int rb = 0; rb < kRB; ++rb) {
        const int drow = rhalf * 128 + rb * 32 + sub;
        const v8bf df =
            *reinterpret_cast<const v8bf HF_LDS*>(st + kXBytes + drow * 128 + lr_swizzle(drow, c) * 16);
        acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(df, xf, acc[rb], 0, 0, 0);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // zero-fill loads past the end may still be landing

  const int row = m0 + xrow;
  if (row >= M || !live) return;
#pragma unroll
  for (int rb = 0; rb < kRB; ++rb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int j = rhalf * 128 + rb * 32 + 8 * g + 4 * half;
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

template __global__ void lowrank_down_wide_kernel<4>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                     int64_t, int, int, int);
template __global__ void lowrank_down_wide_kernel<5>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                     int64_t, int, int, int);

// lowrank_down_wide_kernel's tile (160 rows of x against 256 ranks per pass) on 8 waves instead of 10. Wave w
// multiplies all five 32-row blocks against ranks 32 w .. 32 w + 31 (five MFMA blocks, one down fragment and five x
// fragments per K step), so every SIMD holds two waves; with ten, two SIMDs held three and set the pace. x streams
// from HBM through a 4-slot LDS ring, loaded three stages ahead; the 256-rank down slab, read from L2, takes two
// 32 KiB LDS slots and is staged through registers: each stage is loaded three stages ahead into one of three
// register buffers and written into its LDS slot one stage ahead, which gives it two stages of lead where an LDS-DMA
// ring in the same space gave one (M=37710: K=14336, r=384 597 -> 516 us, K=8192, r=320 353 -> 309 us, K=5376, r=512
// 267 -> 251 us, r=192 122 -> 110 us; within 1 % at K=14336, r=256). Every wave issues the same memory operations
// in the same order (per stage 4 down loads into registers, then 3 x loads; x's 20 blocks of a stage go 3 to a wave
// and the last four read zeros into a sink past the rings), so the waits the compiler places before the register
// writes to LDS are exact for every wave and never include the x loads of that stage. The fragments of the next K
// step are read while the current one's MFMAs run. Each u element is the same sum in the same order as
// lowrank_down_wide_kernel's (and the 64-rank passes'): K ascending in 16-element MFMA steps, down as the first
// operand.
constexpr int kLbRows = 160;
constexpr int kLbXBytes = kLbRows * kLrStageK * 2;   // 20 KiB a stage of x
constexpr int kLbDBytes = kLwRanks * kLrStageK * 2;  // 32 KiB a stage of down
constexpr int kLbXSlots = 4, kLbDSlots = 2;
constexpr int kLbRings = kLbXSlots * kLbXBytes + kLbDSlots * kLbDBytes;  // 144 KiB
constexpr int kLbLds = kLbRings + 1024;                                  // + the sink of the x loads past a stage
constexpr int kLbXLoads = 3;                 // x blocks (8 rows) per wave and stage: 24 >= 20
constexpr int kLbDLoads = kLwRanks / 8 / 8;  // down blocks per wave and stage: 4

__global__ __launch_bounds__(512, 1) void lowrank_down_band_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                   const uint16_t* __restrict__ down, int64_t ldd,
                                                                   uint16_t* __restrict__ u, int64_t ldu, int M, int K,
                                                                   int r) {
  static_assert(kLbLds <= 160 * 1024, "rings exceed the LDS");
  static_assert(8 * kLbXLoads >= kLbRows / 8, "x blocks");
  extern __shared__ __attribute__((aligned(1024))) unsigned char lb_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)lb_smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = blockIdx.x * kLbRows;
  const int rows_m = min(kLbRows, M - m0);
  const uint32_t ldx_bytes = (uint32_t)ldx * 2u, ldd_bytes = (uint32_t)ldd * 2u;
  const uint32_t bytes_x = (uint32_t)rows_m * ldx_bytes, bytes_d = (uint32_t)r * ldd_bytes;
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(x + (int64_t)m0 * ldx, bytes_x);
  const __amdgpu_buffer_rsrc_t rd = make_rsrc(down, bytes_d);
  auto xslot = [&](int t) { return smem + (t % kLbXSlots) * kLbXBytes; };
  auto dslot = [&](int t) { return smem + kLbXSlots * kLbXBytes + (t % kLbDSlots) * kLbDBytes; };
  // This wave's x loads of stage t (LDS-DMA): blocks 3 w .. 3 w + 2 in lr_load's LDS layout; rows past the block and
  // stages past the end read zeros, and blocks past the stage's 20 go to the sink.
  auto issue_x = [&](int t) {
    const int k0 = t * kLrStageK;
#pragma unroll
    for (int i = 0; i < kLbXLoads; ++i) {
      const int blk = wave * kLbXLoads + i;
      const int row = blk * 8 + (lane >> 3);
      const int c = lr_swizzle(row, lane & 7);
      const int k = k0 + c * 8;
      const bool in = blk < kLbRows / 8;
      const uint32_t voff = (in & (row < rows_m) & (k < K)) ? (uint32_t)row * ldx_bytes + (uint32_t)k * 2u : bytes_x;
      unsigned char HF_LDS* dst = in ? xslot(t) + blk * 1024 : smem + kLbRings;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (void HF_LDS*)dst, 16, voff, 0, 0, kCpolStream);
    }
  };
  // This wave's down blocks 4 w .. 4 w + 3 of stage t into registers, and from registers into the stage's LDS slot,
  // in lr_load's layout (lane l of a block: row 8 blk + l / 8, chunk lr_swizzle(row, l % 8)).
  auto load_d = [&](v4u (&b)[kLbDLoads], int t) {
#pragma unroll
    for (int i = 0; i < kLbDLoads; ++i) {
      const int blk = wave * kLbDLoads + i;
      const int row = blk * 8 + (lane >> 3);
      const int c = lr_swizzle(row, lane & 7);
      const int k = t * kLrStageK + c * 8;
      const uint32_t voff = ((row < r) & (k < K)) ? (uint32_t)row * ldd_bytes + (uint32_t)k * 2u : bytes_d;
      b[i] = __builtin_amdgcn_raw_buffer_load_b128(rd, voff, 0, 0);
    }
  };
  auto write_d = [&](const v4u (&b)[kLbDLoads], int t) {
    unsigned char HF_LDS* dst = dslot(t);
#pragma unroll
    for (int i = 0; i < kLbDLoads; ++i)
      *reinterpret_cast<v4u HF_LDS*>(dst + (wave * kLbDLoads + i) * 1024 + lane * 16) = b[i];
  };

  v16f acc[5];
#pragma unroll
  for (int rb = 0; rb < 5; ++rb) acc[rb] = (v16f){0};
  const bool live = wave * 32 < r;  // a wave whose ranks are all past r only loads
  const int nst = (K + kLrStageK - 1) / kLrStageK;
  // Three register buffers of down stages. A stage's down loads go before its x loads (held there by the scheduling
  // barriers), so waiting for them before their LDS writes never waits for the x loads of the same stage.
  v4u db0[kLbDLoads], db1[kLbDLoads], db2[kLbDLoads];
  load_d(db0, 0);
  __builtin_amdgcn_sched_barrier(0);
  issue_x(0);
  load_d(db1, 1);
  __builtin_amdgcn_sched_barrier(0);
  issue_x(1);
  load_d(db2, 2);
  __builtin_amdgcn_sched_barrier(0);
  issue_x(2);
  write_d(db0, 0);
  const int drow = wave * 32 + sub;
  struct Frags {
    v8bf d;
    v8bf x[5];
  };
  auto read = [&](Frags& f, const unsigned char HF_LDS* xs, const unsigned char HF_LDS* ds, int s) {
    const int c = 2 * s + half;
    f.d = *reinterpret_cast<const v8bf HF_LDS*>(ds + drow * 128 + lr_swizzle(drow, c) * 16);
#pragma unroll
    for (int rb = 0; rb < 5; ++rb) {
      const int xrow = rb * 32 + sub;
      f.x[rb] = *reinterpret_cast<const v8bf HF_LDS*>(xs + xrow * 128 + lr_swizzle(xrow, c) * 16);
    }
  };
  auto mma = [&](const Frags& f) {
#pragma unroll
    for (int rb = 0; rb < 5; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.d, f.x[rb], acc[rb], 0, 0, 0);
  };
  Frags f0, f1;
  // Stage t, with down stage t + 1 in register buffer wbuf and buffer lbuf free (its stage, t, is in LDS).
  auto body = [&](int t, v4u (&wbuf)[kLbDLoads], v4u (&lbuf)[kLbDLoads]) {
    // x stage t has landed once at most the next two stages' 2 x (4 + 3) operations are in flight, and this wave's
    // LDS writes of down stage t are done; the barrier makes both true for every wave and frees the slots of stage
    // t - 1, which take down stage t + 1 (from registers) and x stage t + 3.
    static_assert(2 * (kLbDLoads + kLbXLoads) == 14, "the wait count below");
    asm volatile("s_waitcnt vmcnt(14) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    write_d(wbuf, t + 1);
    load_d(lbuf, t + 3);
    __builtin_amdgcn_sched_barrier(0);
    issue_x(t + 3);
    if (!live) return;
    const unsigned char HF_LDS* xs = xslot(t);
    const unsigned char HF_LDS* ds = dslot(t);
    read(f0, xs, ds, 0);
    read(f1, xs, ds, 1);
    mma(f0);
    read(f0, xs, ds, 2);
    mma(f1);
    read(f1, xs, ds, 3);
    mma(f0);
    mma(f1);
    // Keep that order: left to itself the compiler moves each fragment read down to its MFMA, which then waits for
    // it (lgkmcnt(0) before most MFMAs; 8-11 % slower). K steps 0 and 1 are read up front, K steps 2 and 3 among
    // the MFMAs of the two steps before them.
    __builtin_amdgcn_sched_group_barrier(0x100, 12, 0);  // DS read
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
      for (int i = 1; i < 5; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 10, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // Stage t writes buffer (t + 1) % 3 and loads buffer t % 3. Whole rounds of three stages in the loop (so every path
  // through it runs all three and the compiler's waits stay exact), then the last one or two.
  int t = 0;
  for (; t + 3 <= nst; t += 3) {
    body(t, db1, db0);
    body(t + 1, db2, db1);
    body(t + 2, db0, db2);
  }
  if (t < nst) body(t, db1, db0);
  if (t + 1 < nst) body(t + 1, db2, db1);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // zero-fill loads past the end may still be landing
  if (!live) return;
#pragma unroll
  for (int rb = 0; rb < 5; ++rb) {
    const int row = m0 + rb * 32 + sub;
    if (row >= M) continue;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int j = wave * 32 + 8 * g + 4 * half;
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

constexpr int kMaxSplits = 32;  // K chunks of a split launch, at most

// bf16(sum_s part[s][i]) for element i = m r + j of the [splits][M][r] partial sums: the planes added in a fixed
// order from plane 0, one rounding (round to nearest even). All loads first (splits <= kMaxSplits), then the adds.
__device__ __forceinline__ void lr_reduce_load(const float* __restrict__ part, int splits, int64_t M, int r, int64_t i,
                                               float (&p)[kMaxSplits]) {
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s) p[s] = s < splits ? part[(int64_t)s * M * r + i] : 0.0f;
}
__device__ __forceinline__ uint16_t lr_reduce_sum(const float (&p)[kMaxSplits], int splits) {
  float v = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxSplits; ++s)
    if (s < splits) v += p[s];
  return (uint16_t)f32_to_bf16_rne(v);
}
__device__ __forceinline__ uint16_t lr_reduce_value(const float* __restrict__ part, int splits, int64_t M, int r,
                                                    int64_t i) {
  float p[kMaxSplits];
  lr_reduce_load(part, splits, M, r, i, p);
  return lr_reduce_sum(p, splits);
}

// u[m, j] = bf16(sum_s part[s][m][j]) (lr_reduce_value).
__global__ __launch_bounds__(256) void lowrank_reduce_kernel(const float* __restrict__ part, int splits,
                                                             uint16_t* __restrict__ u, int64_t ldu, int M, int r) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (int64_t)M * r) return;
  const int m = (int)(i / r), j = (int)(i % r);
  u[(int64_t)m * ldu + j] = lr_reduce_value(part, splits, M, r, i);
}

// The same sums added by the rotation kernels of a layer for the rows they rotate, in place of a launch of
// lowrank_reduce_kernel between the two passes over x (the low-rank projection then runs first). `part` null: none.
struct LrFinish {
  const float* part;  // [splits][M][r] fp32 partial sums
  uint16_t* u;        // [M, ldu] bf16
  int64_t ldu;
  int64_t M;
  int splits, r;      // r <= 64: one lane per rank
};

// Row `row`'s r sums, lane j < r taking rank j.
__device__ __forceinline__ void lr_finish_row(const LrFinish& f, int64_t row, int lane) {
  if (lane < f.r) f.u[row * f.ldu + lane] = lr_reduce_value(f.part, f.splits, f.M, f.r, row * f.r + lane);
}

// Few rows: a workgroup per row and group of 8 ranks, which needs no second pass. The MFMA kernel above keeps 32 rows
// per wave, so with few rows it has few row blocks and splits K, and adding the fp32 partials costs another launch.
// Here wave t of the workgroup takes the 1024-element tile [1024 t, 1024 t + 1024) of x, lane p the 16 consecutive
// elements from 1024 t + 16 p (K % 16 == 0: all in or all out), loads its 16 elements of the 8 down rows at once (one
// round trip to memory) and accumulates x[k] down[j, k] in fp32 (fma, k ascending). The 64 lanes' sums are added in a
// fixed butterfly (lane_fold, then the lane groups of 8, 16 and 32), the waves' sums in wave order through LDS, and
// each result is rounded to bf16 once (round to nearest even). The order is fixed, so a row's outputs do not depend
// on the launch it is in (lowrank_down_row_kernel or the rotation's combined row launch). A workgroup reads its row
// of x (2K bytes) and 8 rows of down (16K bytes), mostly from L2: cheap for a few hundred rows. Measured at M=1024,
// K=5120, rank 64, the MFMA kernel and its reduction pass are faster (12 us against 19.5 us); whole layers at K=5120,
// N=5120, rank 32 measured 10 % faster at M=300, 5 % at 384 and equal at 512 by rows, hence the row limit.
// (Two rows per workgroup, sharing the down loads, needed more than the 128 registers a 1024-thread workgroup
// allows; 16 ranks per workgroup with their loads four ranks ahead took 8.9 us at M=64 against 5.2 us, the
// rotation included.)
constexpr int kLrRowMaxRows = 384;  // rows up to which the low-rank down projection runs by rows
constexpr int kLrRowMaxWaves = 16;  // K <= 16384
constexpr int kLrRowRanks = 8;      // ranks per workgroup

// One step of the lane butterfly over 2H values: the lanes with bit H set keep the upper H, the others the lower H,
// and each adds its partner's copy of the kept half.
template <int H>
__device__ __forceinline__ void lane_fold(float (&a)[kLrRowRanks], int lane) {
  const bool upper = lane & H;
#pragma unroll
  for (int i = 0; i < H; ++i) {
    const float keep = upper ? a[H + i] : a[i];
    const float send = upper ? a[i] : a[H + i];
    a[i] = keep + __shfl_xor(send, H, 64);
  }
}

// u[j] = bf16(sum_k x[k] down[j, k]) of one row (urow) for j in [j0, j0 + 8) and j < r; `sums` is LDS for 8 floats
// per wave. Every wave of the workgroup calls it.
__device__ __forceinline__ void lowrank_row_ranks(const uint16_t* __restrict__ xrow,
                                                  const uint16_t* __restrict__ down, int64_t ld_down,
                                                  uint16_t* __restrict__ urow, int K, int r, int j0, float* sums) {
  const int lane = threadIdx.x & 63, t = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), nw = blockDim.x >> 6;
  // Lanes past K (in the last wave) load in-range elements and contribute zero; ranks past r load row r - 1 and are
  // not stored. No load is predicated, so all of them issue at once.
  const bool live = t * 1024 + lane * 16 < K;
  const int k0 = live ? t * 1024 + lane * 16 : K - 16;
  const uint4 xa = *reinterpret_cast<const uint4*>(xrow + k0);
  const uint4 xb = *reinterpret_cast<const uint4*>(xrow + k0 + 8);
  uint4 d[kLrRowRanks][2];
#pragma unroll
  for (int i = 0; i < kLrRowRanks; ++i) {
    const uint16_t* dr = down + (int64_t)min(j0 + i, r - 1) * ld_down + k0;
    d[i][0] = *reinterpret_cast<const uint4*>(dr);
    d[i][1] = *reinterpret_cast<const uint4*>(dr + 8);
  }
  const uint32_t xw[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  float acc[kLrRowRanks];
#pragma unroll
  for (int i = 0; i < kLrRowRanks; ++i) {
    const uint32_t w[8] = {d[i][0].x, d[i][0].y, d[i][0].z, d[i][0].w, d[i][1].x, d[i][1].y, d[i][1].z, d[i][1].w};
    float v = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      v = fmaf(bf16_lo(xw[e]), bf16_lo(w[e]), v);
      v = fmaf(bf16_hi(xw[e]), bf16_hi(w[e]), v);
    }
    acc[i] = live ? v : 0.0f;
  }
  lane_fold<4>(acc, lane);
  lane_fold<2>(acc, lane);
  lane_fold<1>(acc, lane);
  // Lane l holds rank j0 + l % 8 over the 8 lanes l ^ (0..7); add the other lane groups of the wave.
  float total = acc[0] + __shfl_xor(acc[0], 8, 64);
  total = total + __shfl_xor(total, 16, 64);
  total = total + __shfl_xor(total, 32, 64);
  if (lane < kLrRowRanks) sums[t * kLrRowRanks + lane] = total;
  __syncthreads();
  if (t == 0 && lane < kLrRowRanks && j0 + lane < r) {
    float v = sums[lane];
    for (int w = 1; w < nw; ++w) v += sums[w * kLrRowRanks + lane];
    urow[j0 + lane] = (uint16_t)f32_to_bf16_rne(v);
  }
}

// Workgroups for M rows and r ranks: one per row and group of 8 ranks.
__host__ __device__ constexpr int64_t lowrank_row_blocks(int64_t M, int r) {
  return M * ((r + kLrRowRanks - 1) / kLrRowRanks);
}

// Workgroup b: row b / groups, ranks 8 (b % groups) ... (groups = ceil(r / 8)).
__device__ __forceinline__ void lowrank_row_block(int64_t b, int groups, const uint16_t* __restrict__ x, int64_t ldx,
                                                  const uint16_t* __restrict__ down, int64_t ld_down,
                                                  uint16_t* __restrict__ u, int64_t ldu, int M, int K, int r,
                                                  float* sums) {
  const int64_t row = b / groups;
  lowrank_row_ranks(x + row * ldx, down, ld_down, u + row * ldu, K, r, (int)(b % groups) * kLrRowRanks, sums);
}

__global__ __launch_bounds__(1024) void lowrank_down_row_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                const uint16_t* __restrict__ down, int64_t ld_down,
                                                                uint16_t* __restrict__ u, int64_t ldu, int M, int K,
                                                                int r, int groups) {
  __shared__ float sums[kLrRowMaxWaves * kLrRowRanks];
  lowrank_row_block(blockIdx.x, groups, x, ldx, down, ld_down, u, ldu, M, K, r, sums);
}

// Low-rank up projection y = bf16(u @ up^T + bias), the second half of LowRankLinear.forward
// (src/hyperflow_h3_flash/transformer.py:57-58: `self.up(...)`, a bias-free bf16 nn.Linear; the bias is this build's
// extension). u is [M, r] bf16 (the output of lowrank_down_kernel), up is [N, r] bf16 (nn.Linear weight layout).
//
// One workgroup per 128 x 128 output tile, 4 waves of 64 x 64 (2 x 2 blocks of v_mfma_f32_32x32x16_bf16, first
// operand up, second u: lanes end with four consecutive n of one row m). The rank is consumed in chunks of 64: the
// chunk's u rows and up rows (128 bytes each, swizzled with swizzle128) go global -> LDS with buffer_load ... lds,
// 8 lanes per row. The output is the dominant traffic (2 bytes per element); it leaves through LDS so every store
// instruction writes 8 whole 128-byte lines.
constexpr int kUpTile = 128;
constexpr int kUpThreads = 256;
constexpr int kUpLds = 2 * kUpTile * 128 + kUpTile * 4;  // u and up chunks (16 KiB each) + the tile's bias (fp32)

__global__ __launch_bounds__(kUpThreads) void lowrank_up_kernel(const uint16_t* __restrict__ u, int64_t ldu,
                                                                 const uint16_t* __restrict__ up, int64_t ldup,
                                                                 const uint16_t* __restrict__ bias,
                                                                 uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                                 int r, int tiles_n, int out_vec16) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char up_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)up_smem_raw;
  unsigned char HF_LDS* u_lds = smem;
  unsigned char HF_LDS* up_lds = smem + kUpTile * 128;
  float HF_LDS* bias_lds = (float HF_LDS*)(smem + 2 * kUpTile * 128);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = (blockIdx.x / tiles_n) * kUpTile, n0 = (blockIdx.x % tiles_n) * kUpTile;
  const int rows_m = min(kUpTile, M - m0), rows_n = min(kUpTile, N - n0);

  if (threadIdx.x < kUpTile) {
    const int n = n0 + threadIdx.x;
    bias_lds[threadIdx.x] = (bias && n < N) ? __uint_as_float((uint32_t)bias[n] << 16) : 0.0f;
  }
  __syncthreads();  // the bias is read in the epilogue (a rank of zero runs no chunk barrier)
  const uint32_t ldu_bytes = (uint32_t)ldu * 2u, ldup_bytes = (uint32_t)ldup * 2u;
  const uint32_t bytes_u = (uint32_t)rows_m * ldu_bytes, bytes_up = (uint32_t)rows_n * ldup_bytes;
  const __amdgpu_buffer_rsrc_t ru = make_rsrc(u + (int64_t)m0 * ldu, bytes_u);
  const __amdgpu_buffer_rsrc_t rup = make_rsrc(up + (int64_t)n0 * ldup, bytes_up);

  v16f acc[2][2];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) acc[ib][jb] = (v16f){0};

  for (int c0 = 0; c0 < r; c0 += 64) {
    // 16 blocks of 8 rows per operand, 4 per wave; chunks past r and rows past the tile read as zero.
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const bool isup = i >= 4;
      const int blk = 4 * wave + (i & 3), row = 8 * blk + (lane >> 3);
      const int c = (lane & 7) ^ (((lane >> 3) ^ blk) & 7);
      const int rows_valid = isup ? rows_n : rows_m;
      const uint32_t ldb = isup ? ldup_bytes : ldu_bytes, oob = isup ? bytes_up : bytes_u;
      const uint32_t voff = ((row < rows_valid) & (c0 + 8 * c < r)) ? row * ldb + (uint32_t)(c0 + 8 * c) * 2u : oob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isup ? rup : ru, (void HF_LDS*)((isup ? up_lds : u_lds) + blk * 1024),
                                               16, voff, 0, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
    for (int kk = 0; kk < 64; kk += 16) {
      const int chunk = kk / 8 + half;
      v8bf pf[2], uf[2];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const int nl = wn * 64 + ib * 32 + sub;
        pf[ib] = *(const v8bf HF_LDS*)(up_lds + nl * 128 + (swizzle128(nl, chunk) << 4));
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const int ml = wm * 64 + jb * 32 + sub;
        uf[jb] = *(const v8bf HF_LDS*)(u_lds + ml * 128 + (swizzle128(ml, chunk) << 4));
      }
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int jb = 0; jb < 2; ++jb)
          acc[ib][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf[ib], uf[jb], acc[ib][jb], 0, 0, 0);
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // the next chunk (or the staging) rewrites LDS
  }

  // Bias, bf16, and the output through LDS: lane (sub, h) holds columns 16h..16h+15 of row sub of each block after
  // one exchange between the lane halves; the wave stages its 64 x 64 tile (64 rows of 128 bytes) and stores 8 whole
  // rows per instruction.
  unsigned char HF_LDS* stage_out = smem + wave * 8192;
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int row = jb * 32 + sub;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      uint32_t w4[4][2];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = acc[ib][jb][4 * gq + e] + bias_lds[wn * 64 + ib * 32 + 8 * gq + 4 * half + e];
        w4[gq][0] = pack_bf16x2(v[0], v[1]);
        w4[gq][1] = pack_bf16x2(v[2], v[3]);
      }
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const auto s02 = __builtin_amdgcn_permlane32_swap(w4[0][w], w4[2][w], false, false);
        const auto s13 = __builtin_amdgcn_permlane32_swap(w4[1][w], w4[3][w], false, false);
        w4[0][w] = s02[0];
        w4[2][w] = s02[1];
        w4[1][w] = s13[0];
        w4[3][w] = s13[1];
      }
      const int c0 = 4 * ib + 2 * half;
      *(v4i HF_LDS*)(stage_out + row * 128 + (swizzle128(row, c0) << 4)) =
          (v4i){(int)w4[0][0], (int)w4[0][1], (int)w4[2][0], (int)w4[2][1]};
      *(v4i HF_LDS*)(stage_out + row * 128 + (swizzle128(row, c0 + 1) << 4)) =
          (v4i){(int)w4[1][0], (int)w4[1][1], (int)w4[3][0], (int)w4[3][1]};
    }
  }
  wave_lds_sync();
  const bool full = rows_m == kUpTile && rows_n == kUpTile && out_vec16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 8 * i + (lane >> 3), ch = lane & 7;
    const v4i val = *(const v4i HF_LDS*)(stage_out + row * 128 + (swizzle128(row, ch) << 4));
    const int m = m0 + wm * 64 + row, n = n0 + wn * 64 + 8 * ch;
    uint16_t* dst = y + (int64_t)m * ldy + n;
    if (full) {
      *reinterpret_cast<v4i*>(dst) = val;
    } else if (m < M) {
      if (out_vec16 && n + 8 <= N) {
        *reinterpret_cast<v4i*>(dst) = val;
      } else {
        for (int e = 0; e < 8; ++e)
          if (n + e < N) dst[e] = (uint16_t)((uint32_t)val[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

}  // namespace hf
