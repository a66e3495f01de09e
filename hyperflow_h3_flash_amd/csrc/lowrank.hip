// Low-rank down projection u = bf16(x @ down^T), the first half of LowRankLinear.forward
// (src/hyperflow_h3_flash/transformer.py:57-58: `self.up(self.down(x))`, whose bf16 nn.Linear rounds `down(x)` to
// bf16 before `up`). Its output feeds the low-rank term of the fused INT8 GEMM epilogue.
//
// x is [M, K] bf16 and down is [r, K] bf16 (nn.Linear weight layout), both K-major. One workgroup owns 32 rows of
// x and all r outputs; its 4 waves split K four ways with v_mfma_f32_32x32x16_bf16 (first operand down, second x,
// so lanes end with four consecutive rank columns of one row) and add their fp32 partial tiles in a fixed order
// through LDS. r <= 128 per launch (RB = ceil(r / 32) blocks); the host splits larger ranks.
#include "common.h"

namespace hf {

template <int RB>
__global__ __launch_bounds__(256) void lowrank_down_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const uint16_t* __restrict__ down, int64_t ldd,
                                                           uint16_t* __restrict__ u, int64_t ldu, int M, int K,
                                                           int r) {
  __shared__ float part[3][RB][16][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = blockIdx.x * 32;
  const int m = min(m0 + sub, M - 1);
  const uint16_t* xrow = x + (int64_t)m * ldx;
  const uint16_t* drow[RB];
  bool dvalid[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int j = rb * 32 + sub;
    dvalid[rb] = j < r;
    drow[rb] = down + (int64_t)min(j, r - 1) * ldd;
  }
  v16f acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = (v16f){0};

  // K is a multiple of 16; wave w takes the 16-element steps w, w + 4, w + 8, ...
  const int steps = K / 16;
  for (int st = wave; st < steps; st += 4) {
    const int k = st * 16 + 8 * half;
    const v8bf xf = *reinterpret_cast<const v8bf*>(xrow + k);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const v8bf df = dvalid[rb] ? *reinterpret_cast<const v8bf*>(drow[rb] + k) : (v8bf){0};
      acc[rb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(df, xf, acc[rb], 0, 0, 0);
    }
  }
  if (wave > 0) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int v = 0; v < 16; ++v) part[wave - 1][rb][v][lane] = acc[rb][v];
  }
  __syncthreads();
  if (wave != 0) return;
  const int row = m0 + sub;
  if (row >= M) return;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int j = rb * 32 + 8 * g + 4 * half;
      uint32_t h[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int v = 4 * g + e;
        float s = acc[rb][v];
        s = s + part[0][rb][v][lane];
        s = s + part[1][rb][v][lane];
        s = s + part[2][rb][v][lane];
        h[e] = f32_to_bf16_rne(s);
      }
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
