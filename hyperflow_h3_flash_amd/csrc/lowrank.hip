// Low-rank down projection u = bf16(x @ down^T), the first half of LowRankLinear.forward
// (src/hyperflow_h3_flash/transformer.py:57-58: `self.up(self.down(x))`, whose bf16 nn.Linear rounds `down(x)` to
// bf16 before `up`). Its output feeds the low-rank term of the fused INT8 GEMM epilogue.
//
// x is [M, K] bf16 and down is [r, K] bf16 (nn.Linear weight layout), both K-major. A workgroup owns 128 rows of x;
// each of its 4 waves owns 32 rows and all r outputs and walks the whole of K with v_mfma_f32_32x32x16_bf16 (first
// operand down, second x, so lanes end with four consecutive rank columns of one row). The waves of a workgroup read
// the same `down` rows at the same time, so `down` streams from L2 once per 128 rows. r <= 128 per launch
// (RB = ceil(r / 32) blocks); the host splits larger ranks. The memory-bound part is the single read of x.
#include "common.h"

namespace hf {

constexpr int kLrRowsPerWave = 32;
constexpr int kLrWaves = 4;
constexpr int kLrRows = kLrRowsPerWave * kLrWaves;

template <int RB>
__global__ __launch_bounds__(256) void lowrank_down_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const uint16_t* __restrict__ down, int64_t ldd,
                                                           uint16_t* __restrict__ u, int64_t ldu, int M, int K,
                                                           int r) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = blockIdx.x * kLrRows + wave * kLrRowsPerWave;
  if (m0 >= M) return;
  const int m = min(m0 + sub, M - 1);
  const uint16_t* xrow = x + (int64_t)m * ldx + 8 * half;
  // Rank rows at or past r are clamped to row r-1: they only feed output columns j >= r, which are never stored.
  const uint16_t* drow[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) drow[rb] = down + (int64_t)min(rb * 32 + sub, r - 1) * ldd + 8 * half;
  v16f acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = (v16f){0};

  // K is a multiple of 16: one 16-wide K step per MFMA. Loads run one group of U steps ahead of the MFMAs
  // (software pipelining with two register buffers, unrolled so both stay in registers).
  constexpr int U = RB <= 2 ? 8 : 4;
  struct Group {
    v8bf x[U];
    v8bf d[U][RB];
  };
  auto load_group = [&](Group& g, int st0) {
#pragma unroll
    for (int i = 0; i < U; ++i) {
      g.x[i] = *reinterpret_cast<const v8bf*>(xrow + (st0 + i) * 16);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) g.d[i][rb] = *reinterpret_cast<const v8bf*>(drow[rb] + (st0 + i) * 16);
    }
  };
  auto mma_group = [&](const Group& g) {
#pragma unroll
    for (int i = 0; i < U; ++i)
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(g.d[i][rb], g.x[i], acc[rb], 0, 0, 0);
  };
  const int steps = K / 16;
  const int groups = steps / U;
  Group ga, gb;
  if (groups > 0) load_group(ga, 0);
  int gi = 0;
  for (; gi + 2 <= groups; gi += 2) {
    load_group(gb, (gi + 1) * U);
    mma_group(ga);
    if (gi + 2 < groups) load_group(ga, (gi + 2) * U);
    mma_group(gb);
  }
  if (gi < groups) mma_group(ga);
  for (int st = groups * U; st < steps; ++st) {
    const v8bf x1 = *reinterpret_cast<const v8bf*>(xrow + st * 16);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const v8bf d1 = *reinterpret_cast<const v8bf*>(drow[rb] + st * 16);
      acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(d1, x1, acc[rb], 0, 0, 0);
    }
  }

  const int row = m0 + sub;
  if (row >= M) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int j = rb * 32 + 8 * g + 4 * half;
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) h[e] = f32_to_bf16_rne(acc[rb][4 * g + e]);
      uint16_t* dst = u + (int64_t)row * ldu + j;
      if (j + 3 < r && (ldu & 3) == 0) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
      } else {
        for (int e = 0; e < 4; ++e)
          if (j + e < r) dst[e] = (uint16_t)h[e];
      }
    }
  }
}

template __global__ void lowrank_down_kernel<1>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                int64_t, int, int, int);
template __global__ void lowrank_down_kernel<2>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                int64_t, int, int, int);
template __global__ void lowrank_down_kernel<3>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                int64_t, int, int, int);
template __global__ void lowrank_down_kernel<4>(const uint16_t*, int64_t, const uint16_t*, int64_t, uint16_t*,
                                                int64_t, int, int, int);

}  // namespace hf
