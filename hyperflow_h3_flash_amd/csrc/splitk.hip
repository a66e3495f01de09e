// Split-K finish for skinny GEMMs: sums the int32 partial accumulators of the K chunks and applies the convrot
// epilogue of int8_gemm_kernel,
//   y[m, n] = bf16((f32(sum_s acc_s[m, n]) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n]).
// Integer partial sums add exactly in any order, so with no low-rank branch and no bias the output is bitwise the
// reference's (src/hyperflow_h3_flash/int8.py:179), as from the unsplit GEMM. `act` applies the same output activation
// as the GEMM's epilogue (kActNone, kActGeluTanh, or kActSwiGLU).
//
// The planes are stored block by block (partial_block_offset): wave (bm, bn) reads block (bm, bn) of each. kActSwiGLU: the GEMMs that wrote the partials read the weight rows in pair order (column n is weight row
// glu_row(n)), so the epilogue reads wscale, bias and up row glu_row(n) for column n; in each 32-column block register
// v < 8 holds a hidden column and v + 8 its gate column, and the block writes 16 of the N / 2 outputs.
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
// Partial planes gathered per batch of loads. Measured against 8 and 4 (same box, bitwise equal outputs): 8 planes
// held 252 VGPRs, 4 held 188, 2 hold 156, and 2 was fastest at every shape (M=256, N=15360, r=64: 46.2 -> 43.7 us;
// M=64, N=30720: 42.9 -> 41.5 us): more waves per SIMD hide the plane reads better than longer batches per wave.
constexpr int kSkPlanes = 2;

// The epilogue of one 32 (m) x 32 (n) output block whose int32 accumulators a wave holds in the layout of
// v_mfma_i32_32x32x32_i8 with the weight as the first operand. `block_load` issues every load the block needs
// (factors, bias bits, the low-rank operands of the first 64 ranks) so they are in flight while the accumulators are
// gathered; `block_finish` applies (f32(acc) * sx) * sw + u @ up^T + bias, the activation, and stores. Indices are
// clamped into the matrices instead of branched on; values of columns past N or ranks past r are zeroed or not stored.
struct BlockOperands {
  float sxm;
  float wsv[16];
  uint32_t braw[16];
  v8bf pf[4], uf[4];
};

__device__ __forceinline__ void block_load(BlockOperands& o, int m0, int n0, const float* __restrict__ sx,
                                           const float* __restrict__ sw, const uint16_t* __restrict__ u, int64_t ldu,
                                           const uint16_t* __restrict__ up, int64_t ldup, int r,
                                           const uint16_t* __restrict__ bias, int M, int N, bool glu, int glu_half,
                                           int glu_gate_first, int lane) {
  // Accumulator column of logical column n; four consecutive columns from a multiple of 4 stay consecutive.
  auto col = [&](int n) { return glu ? glu_row(n, glu_half, glu_gate_first) : n; };
  const int sub = lane & 31, half = lane >> 5;
  const int m = m0 + sub;
  o.sxm = sx[min(m, M - 1)];
  // Bias bits are loaded unconditionally (from wscale's N x 4 bytes when there is no bias: a load in a branch of its
  // own would be waited for at the branch's end) and converted where they are added.
  const uint16_t* bsrc = bias ? bias : reinterpret_cast<const uint16_t*>(sw);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int na = col(min(n0 + 8 * (i / 4) + 4 * half + i % 4, N - 1));
    o.wsv[i] = sw[na];
    o.braw[i] = bsrc[na];
  }
  // Low-rank operands of the first 64 ranks, 16 ranks per MFMA: first operand up[n, :], second u[m, :].
  const int nrow = col(min(n0 + sub, N - 1)), mrow = min(m, M - 1);
  if (r > 0) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      const int k = 16 * st + 8 * half;
      const int kc = min(k, r - 8);
      o.pf[st] = *reinterpret_cast<const v8bf*>(up + (int64_t)nrow * ldup + kc);
      o.uf[st] = *reinterpret_cast<const v8bf*>(u + (int64_t)mrow * ldu + kc);
    }
  }
}

__device__ __forceinline__ void block_finish(const BlockOperands& o, const int32_t (&sums)[16], int m0, int n0,
                                             const uint16_t* __restrict__ u, int64_t ldu,
                                             const uint16_t* __restrict__ up, int64_t ldup, int r,
                                             const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
                                             int M, int N, int vec, int act, int glu_half, int glu_gate_first,
                                             int lane) {
  const bool glu = act == kActSwiGLU;
  auto col = [&](int n) { return glu ? glu_row(n, glu_half, glu_gate_first) : n; };
  const int sub = lane & 31, half = lane >> 5;
  const int m = m0 + sub;
  const bool n_in = n0 + sub < N;
  const int nrow = col(min(n0 + sub, N - 1));
  v16f c;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int n = n0 + 8 * (i / 4) + 4 * half + i % 4;
    c[i] = ((float)sums[i] * o.sxm) * (n < N ? o.wsv[i] : 0.0f);
  }
  if (r > 0) {
#pragma unroll
    for (int st = 0; st < 4; ++st) {
      if (16 * st >= r) break;
      const bool k_in = 16 * st + 8 * half < r;
      c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(k_in && n_in ? o.pf[st] : (v8bf){0},
                                                k_in && m < M ? o.uf[st] : (v8bf){0}, c, 0, 0, 0);
    }
  }
  for (int kk = 64; kk < r; kk += 16) {  // ranks past 64, loaded as they are used
    const int k = kk + 8 * half;
    const v8bf p = (k < r && n_in) ? *reinterpret_cast<const v8bf*>(up + (int64_t)nrow * ldup + k) : (v8bf){0};
    const v8bf q = (k < r && m < M) ? *reinterpret_cast<const v8bf*>(u + (int64_t)m * ldu + k) : (v8bf){0};
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(p, q, c, 0, 0, 0);
  }
  if (m >= M) return;
  if (bias) {
#pragma unroll
    for (int i = 0; i < 16; ++i)
      if (n0 + 8 * (i / 4) + 4 * half + i % 4 < N) c[i] = c[i] + __uint_as_float(o.braw[i] << 16);
  }
  if (glu) {
    // Outputs n0 / 2 + 8 gq + 4 h + e from the pair (v, v + 8), v = 4 gq + e.
    const int n_out = N / 2;
#pragma unroll
    for (int gq = 0; gq < 2; ++gq) {
      const int oc = n0 / 2 + 8 * gq + 4 * half;
      float v[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = swiglu(round_bf16(c[4 * gq + e]), round_bf16(c[4 * gq + 8 + e]));
      const uint32_t p01 = pack_bf16x2(v[0], v[1]), p23 = pack_bf16x2(v[2], v[3]);
      uint16_t* dst = y + (int64_t)m * ldy + oc;
      if (vec && oc + 4 <= n_out) {
        *reinterpret_cast<uint2*>(dst) = make_uint2(p01, p23);
      } else {
        const uint16_t h[4] = {(uint16_t)p01, (uint16_t)(p01 >> 16), (uint16_t)p23, (uint16_t)(p23 >> 16)};
        for (int e = 0; e < 4; ++e)
          if (oc + e < n_out) dst[e] = h[e];
      }
    }
    return;
  }
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const int n = n0 + 8 * gq + 4 * half;
    float v[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = c[4 * gq + e];
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

__global__ __launch_bounds__(64) void splitk_epilogue_kernel(const int32_t* __restrict__ acc,
                                                             int64_t plane, int splits, const float* __restrict__ sx,
                                                             const float* __restrict__ sw,
                                                             const uint16_t* __restrict__ u, int64_t ldu,
                                                             const uint16_t* __restrict__ up, int64_t ldup, int r,
                                                             const uint16_t* __restrict__ bias,
                                                             uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                             int tiles_n, int vec, int act, int glu_half,
                                                             int glu_gate_first) {
  const int lane = threadIdx.x;
  const int m0 = (blockIdx.x / tiles_n) * kSkTileM, n0 = (blockIdx.x % tiles_n) * kSkTileN;
  // Every load is issued before the first wait (one round trip to memory, not one per operand).
  BlockOperands o;
  block_load(o, m0, n0, sx, sw, u, ldu, up, ldup, r, bias, M, N, act == kActSwiGLU, glu_half, glu_gate_first, lane);
  // The planes' sums at this lane's 16 positions in block (bm, bn) of each plane (partial_block_offset's layout:
  // each of the wave's loads covers 1 KiB of contiguous memory). Loads are issued kSkPlanes planes at a time before
  // any is added; the sums are exact in any order.
  int32_t sums[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) sums[i] = 0;
  const int32_t* blk = acc + partial_block_offset(m0 / 32, n0 / 32, tiles_n) + 4 * lane;
  for (int s0 = 0; s0 < splits; s0 += kSkPlanes) {
    v4i pl[kSkPlanes][4];
#pragma unroll
    for (int s = 0; s < kSkPlanes; ++s)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
        pl[s][gq] = reinterpret_cast<const v4i*>(blk + (int64_t)min(s0 + s, splits - 1) * plane)[64 * gq];
#pragma unroll
    for (int s = 0; s < kSkPlanes; ++s)
#pragma unroll
      for (int gq = 0; gq < 4; ++gq)
#pragma unroll
        for (int e = 0; e < 4; ++e) sums[4 * gq + e] += (s0 + s < splits) ? pl[s][gq][e] : 0;
  }
  block_finish(o, sums, m0, n0, u, ldu, up, ldup, r, bias, y, ldy, M, N, vec, act, glu_half, glu_gate_first, lane);
}

}  // namespace hf
