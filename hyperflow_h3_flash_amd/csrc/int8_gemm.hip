// INT8 x INT8 -> INT32 GEMM on gfx950 MFMA with the convrot epilogue fused.
//
// Replaces the reference's `int8_mm_kernel` (src/hyperflow_h3_flash/int8.py:283-313) and its `rescale_kernel`
// epilogue (int8.py:315-324):
//   acc[m, n] = sum_k q[m, k] * w[n, k]                      exact int32
//   y[m, n]   = bf16((f32(acc) * sx[m]) * sw[n])              two separately rounded fp32 products (int8.py:179)
// extended with the low-rank branch and a bias (the composition with LowRankLinear, transformer.py:57-58):
//   y[m, n]   = bf16((f32(acc) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n])
// With no low-rank branch and no bias the output is bitwise the reference's.
//
// Tiling: 256 (m) x 256 (n) output tile per workgroup, K in steps of 128 bytes, 4 waves in a 2 x 2 grid, each wave
// a 128 x 128 sub-tile of 4 x 4 v_mfma_i32_32x32x32_i8 blocks. The MFMA's first operand is the weight (its rows
// are the output columns n) and the second the activation, so each lane ends with four consecutive n of one row m:
// the epilogue stores 8 contiguous bytes per lane and reads one activation scale per block.
//
// Operands go global -> LDS with buffer_load ... lds (16 bytes per lane, no VGPR round trip), double-buffered.
// A 128-byte LDS row holds one tile row's 128 K-bytes as eight 16-byte chunks, chunk c stored at c ^ (row & 7), so
// the 32 rows one ds_read_b128 touches spread over all banks. Out-of-range rows and K beyond the end read as zero
// through the buffer descriptor's range check.
#include "common.h"

namespace hf {

constexpr int GBM = 256, GBN = 256, GBK = 128;
constexpr int kStageBytes = (GBM + GBN) * GBK;  // 64 KiB: activation tile then weight tile
constexpr int kGemmLds = 2 * kStageBytes;       // double buffered

struct GemmArgs {
  const int8_t* q;
  int64_t ldq;
  const int8_t* w;
  int64_t ldw;
  const float* sx;
  const float* sw;
  const uint16_t* u;   // [M, r] bf16 or null
  int64_t ldu;
  const uint16_t* up;  // [N, r] bf16 or null
  int64_t ldup;
  int r;
  const uint16_t* bias;  // [N] bf16 or null
  void* out;             // bf16 [M, ldo] or int32 [M, ldo]
  int64_t ldo;
  int M, N, K;
  int tiles_m, tiles_n;
};

// Workgroup id -> (tile_m, tile_n). Workgroups are dealt to the 8 XCDs round robin; renumber them so each XCD gets
// a contiguous run of tiles, then walk that run in groups of 8 tile rows so tiles sharing weight columns (and
// activation rows) run close together on one XCD's L2.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int per = total / 8, rem = total % 8;
  const int xcd = bid % 8, local = bid / 8;
  const int logical = (xcd < rem) ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  constexpr int kGroupM = 8;
  const int group = kGroupM * tiles_n;
  const int first_m = (logical / group) * kGroupM;
  const int size_m = min(tiles_m - first_m, kGroupM);
  tm = first_m + (logical % group) % size_m;
  tn = (logical % group) / size_m;
}

__device__ __forceinline__ void load_tile_rows(__amdgpu_buffer_rsrc_t rsrc, uint32_t oob, int64_t ld, int rows_valid,
                                               int k0, int K, unsigned char HF_LDS* dst, int wave, int lane) {
  // 256 rows x 128 bytes = 32 loads of 1 KiB (8 rows) per tile; 8 per wave.
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int blk = wave * 8 + i;
    const int r = blk * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (r & 7);
    const int kb = k0 + c * 16;
    const uint32_t voff = (r < rows_valid && kb < K) ? (uint32_t)(r * ld + kb) : oob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void HF_LDS*)(dst + blk * 1024), 16, voff, 0, 0, 0);
  }
}

template <bool I32OUT>
__global__ __launch_bounds__(256, 1) void int8_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)smem_raw;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  int tm, tn;
  tile_of(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int rows_m = min(GBM, a.M - m0), rows_n = min(GBN, a.N - n0);

  const uint32_t bytes_q = (uint32_t)(rows_m * a.ldq), bytes_w = (uint32_t)(rows_n * a.ldw);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + (int64_t)m0 * a.ldq, bytes_q);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + (int64_t)n0 * a.ldw, bytes_w);

  v16i acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v16i){0};

  const int nk = (a.K + GBK - 1) / GBK;
  load_tile_rows(rq, bytes_q, a.ldq, rows_m, 0, a.K, smem, wave, lane);
  load_tile_rows(rw, bytes_w, a.ldw, rows_n, 0, a.K, smem + GBM * GBK, wave, lane);

  const int sub = lane & 31, half = lane >> 5;
  for (int kt = 0; kt < nk; ++kt) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (kt + 1 < nk) {
      unsigned char HF_LDS* nxt = smem + ((kt + 1) & 1) * kStageBytes;
      load_tile_rows(rq, bytes_q, a.ldq, rows_m, (kt + 1) * GBK, a.K, nxt, wave, lane);
      load_tile_rows(rw, bytes_w, a.ldw, rows_n, (kt + 1) * GBK, a.K, nxt + GBM * GBK, wave, lane);
    }
    const unsigned char HF_LDS* As = smem + (kt & 1) * kStageBytes;
    const unsigned char HF_LDS* Bs = As + GBM * GBK;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int chunk = ((2 * ks + half) ^ (sub & 7)) * 16;
      v4i wf[4], af[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
        wf[ib] = *(const v4i HF_LDS*)(Bs + (wn * 128 + ib * 32 + sub) * GBK + chunk);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
        af[jb] = *(const v4i HF_LDS*)(As + (wm * 128 + jb * 32 + sub) * GBK + chunk);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
          acc[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf[ib], af[jb], acc[ib][jb], 0, 0, 0);
    }
  }

  // Output layout of a 32x32 block: lane holds column j = lane % 32 (the row m here) and, in register v, row
  // i = 8*(v/4) + 4*(lane/32) + v%4 (the column n here): four consecutive n per group of four registers.
  if constexpr (I32OUT) {
    int32_t* out = static_cast<int32_t*>(a.out);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int m = m0 + wm * 128 + jb * 32 + sub;
      if (m >= a.M) continue;
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * 128 + ib * 32 + 8 * g + 4 * half;
          int32_t* dst = out + (int64_t)m * a.ldo + n;
          const v16i& c = acc[ib][jb];
          if (n + 3 < a.N && ((a.ldo & 3) == 0)) {
            *reinterpret_cast<int4*>(dst) = make_int4(c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]);
          } else {
            for (int e = 0; e < 4; ++e)
              if (n + e < a.N) dst[e] = c[4 * g + e];
          }
        }
    }
  } else {
    // One 32-wide block of output columns at a time keeps a single 64-register fp32 tile live next to the
    // accumulators: dequantize, add the low-rank product on bf16 MFMA, add the bias, round, store.
    float sxv[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int m = m0 + wm * 128 + jb * 32 + sub;
      sxv[jb] = m < a.M ? a.sx[m] : 0.0f;
    }
    uint16_t* out = static_cast<uint16_t*>(a.out);
    const bool vec = (a.ldo & 3) == 0;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      const int nb = n0 + wn * 128 + ib * 32;
      float ws[16], bv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int n = nb + 8 * (v >> 2) + 4 * half + (v & 3);
        ws[v] = n < a.N ? a.sw[n] : 0.0f;
        bv[v] = (a.bias && n < a.N) ? __uint_as_float((uint32_t)a.bias[n] << 16) : 0.0f;
      }
      v16f c[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float t = (float)acc[ib][jb][v] * sxv[jb];
          c[jb][v] = t * ws[v];
        }
      if (a.r > 0) {
        // Low-rank term on bf16 MFMA into the same fp32 tile: first operand up[n, :], second u[m, :].
        const int nrow = min(nb + sub, a.N - 1);
        for (int kk = 0; kk < a.r; kk += 16) {
          const int k = kk + 8 * half;
          const v8bf pf = (k < a.r) ? *reinterpret_cast<const v8bf*>(a.up + (int64_t)nrow * a.ldup + k) : (v8bf){0};
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) {
            const int mrow = min(m0 + wm * 128 + jb * 32 + sub, a.M - 1);
            const v8bf uf = (k < a.r) ? *reinterpret_cast<const v8bf*>(a.u + (int64_t)mrow * a.ldu + k) : (v8bf){0};
            c[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c[jb], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int m = m0 + wm * 128 + jb * 32 + sub;
        if (m >= a.M) continue;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = nb + 8 * g + 4 * half;
          uint32_t h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float v = c[jb][4 * g + e];
            if (a.bias) v = v + bv[4 * g + e];
            h[e] = f32_to_bf16_rne(v);
          }
          uint16_t* dst = out + (int64_t)m * a.ldo + n;
          if (vec && n + 3 < a.N) {
            *reinterpret_cast<uint2*>(dst) = make_uint2(h[0] | (h[1] << 16), h[2] | (h[3] << 16));
          } else {
            for (int e = 0; e < 4; ++e)
              if (n + e < a.N) dst[e] = (uint16_t)h[e];
          }
        }
      }
    }
  }
}

template __global__ void int8_gemm_kernel<false>(GemmArgs);
template __global__ void int8_gemm_kernel<true>(GemmArgs);

}  // namespace hf
