// Split-K finish for skinny GEMMs: sums the int32 partial accumulators of the K chunks and applies the convrot
// epilogue of int8_gemm_kernel,
//   y[m, n] = bf16((f32(sum_s acc_s[m, n]) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n]).
// Integer partial sums add exactly in any order, so with no low-rank branch and no bias the output is bitwise the
// reference's (src/hyperflow_h3_flash/int8.py:179), as from the unsplit GEMM. `act` applies the same output activation
// as the GEMM's epilogue (kActNone or kActGeluTanh).
//
// With few rows (M <= a few hundred) the unsplit GEMM has fewer 256 x 256 tiles than the chip has CUs; splitting K
// gives every CU a share of the weight stream, at the cost of writing and re-reading M x N int32 per split.
//
// One wave per 32 (m) x 32 (n) tile (small tiles: few rows give few tiles): lane (sub, h) owns row m0 + sub and the
// four groups of four consecutive columns 8g + 4h + (0..3), the layout of v_mfma_f32_32x32x16_bf16 with up as the
// first operand, so the low-rank term accumulates onto the dequantized values in place.
#include "common.h"

namespace hf {

constexpr int kSkTileM = 32;
constexpr int kSkTileN = 32;
constexpr int kSkMaxSplits = 32;

__global__ __launch_bounds__(64) void splitk_epilogue_kernel(const int32_t* __restrict__ acc, int64_t ld_acc,
                                                             int64_t plane, int splits, const float* __restrict__ sx,
                                                             const float* __restrict__ sw,
                                                             const uint16_t* __restrict__ u, int64_t ldu,
                                                             const uint16_t* __restrict__ up, int64_t ldup, int r,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                             int tiles_n, int vec, int act) {
  const int lane = threadIdx.x;
  const int sub = lane & 31, half = lane >> 5;
  const int m0 = (blockIdx.x / tiles_n) * kSkTileM, n0 = (blockIdx.x % tiles_n) * kSkTileN;
  const int m = m0 + sub;
  const float sxm = sx[min(m, M - 1)];
  v16f c;
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int n = n0 + 8 * gq + 4 * half;
    int32_t s4[4] = {0, 0, 0, 0};
    if (m < M) {
      if (vec && n + 4 <= N) {
        // Every plane's four values are loaded before any is added (splits <= kSkMaxSplits); the sum is exact.
        v4i pl[kSkMaxSplits];
#pragma unroll
        for (int s = 0; s < kSkMaxSplits; ++s)
          pl[s] = s < splits ? *reinterpret_cast<const v4i*>(acc + s * plane + (int64_t)m * ld_acc + n) : (v4i){0};
#pragma unroll
        for (int s = 0; s < kSkMaxSplits; ++s)
#pragma unroll
          for (int e = 0; e < 4; ++e) s4[e] += pl[s][e];
      } else {
        for (int s = 0; s < splits; ++s)
          for (int e = 0; e < 4; ++e)
            if (n + e < N) s4[e] += acc[s * plane + (int64_t)m * ld_acc + n + e];
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float wsn = (n + e < N) ? sw[n + e] : 0.0f;
      c[4 * gq + e] = ((float)s4[e] * sxm) * wsn;
    }
  }
  // Low-rank term, 16 ranks per MFMA: first operand up[n, :], second u[m, :] (rows past the matrix read zero).
  const int nrow = n0 + sub;
  for (int kk = 0; kk < r; kk += 16) {
    const int k = kk + 8 * half;
    const v8bf pf = (k < r && nrow < N) ? *reinterpret_cast<const v8bf*>(up + (int64_t)nrow * ldup + k) : (v8bf){0};
    const v8bf uf = (k < r && m < M) ? *reinterpret_cast<const v8bf*>(u + (int64_t)m * ldu + k) : (v8bf){0};
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c, 0, 0, 0);
  }
  if (m >= M) return;
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int n = n0 + 8 * gq + 4 * half;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = c[4 * gq + e];
      if (bias && n + e < N) v[e] = v[e] + __uint_as_float((uint32_t)bias[n + e] << 16);
    }
    uint32_t p01 = pack_bf16x2(v[0], v[1]), p23 = pack_bf16x2(v[2], v[3]);
    if (act == kActGeluTanh) {
      p01 = activate_bf16x2<kActGeluTanh>(p01);
      p23 = activate_bf16x2<kActGeluTanh>(p23);
    }
    uint16_t* dst = y + (int64_t)m * ldy + n;
    if (vec && n + 4 <= N) {
      *reinterpret_cast<uint2*>(dst) = make_uint2(p01, p23);
    } else {
      const uint16_t h[4] = {(uint16_t)p01, (uint16_t)(p01 >> 16), (uint16_t)p23, (uint16_t)(p23 >> 16)};
      for (int e = 0; e < 4; ++e)
        if (n + e < N) dst[e] = h[e];
    }
  }
}

}  // namespace hf
