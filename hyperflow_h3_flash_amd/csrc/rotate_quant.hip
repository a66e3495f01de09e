// Online block-Hadamard rotation + per-token absmax INT8 quantization (one pass over x).
//
// Replaces the reference's `rotate_quant` (src/hyperflow_h3_flash/int8.py:194-221, host 326-344) with the
// arithmetic of its torch path (int8.py:176-178):
//   xr = bf16(x @ blockdiag(R))   R = regular Hadamard of order G = 4^n, entries +-2^-n
//   sx = max(absmax_row(xr), 1e-12) / 127          (fp32, correctly rounded division)
//   xq = clamp(rint(xr / sx), -127, 127)           (fp32, correctly rounded quotient, ties to even)
//
// The rotation is the unnormalised radix-4 butterfly H4 v = S - 2 reverse(v) (S = sum of the four), applied along
// each base-4 digit of the in-group index, in fp64. Every product with +-1 and every partial sum is exact in fp64
// whenever a group's nonzero inputs span at most 33 binades, so the single rounding to bf16 below is the rounding
// of the exact sum. The 2^-n normalisation is a power of two and is folded into the scale.
//
// Layout: one wave processes one row. A row is walked in tiles of 1024 elements; lane p holds the 16 consecutive
// elements 16p..16p+15 (a "pencil", two 16-byte loads). Digits 0 and 1 (bits 0-3 of the index) are transformed in
// registers. For G >= 64 the fp64 pencils go through LDS once so that each lane holds 16 values along digits 2
// and 3, transformed in registers again. The bf16-rounded values wait in a per-wave row buffer in LDS until the
// row's absmax is known, then each lane quantizes 16 consecutive values and writes 16 bytes.
#pragma once

#include "common.h"
#include "lowrank.hip"

namespace hf {

constexpr int kRqTile = 1024;                            // elements per wave step (64 lanes x 16)
constexpr int kRqStride = 18;                            // doubles per pencil in the transpose scratch (16 + pad)
constexpr int kRqScratchBytes = 64 * kRqStride * 8;      // 9216 bytes per wave
constexpr int kRqRegMaxTpw = 5;  // tiles per wave of the register-resident kernel (four waves per SIMD at five)

__device__ __forceinline__ void h4(double& a, double& b, double& c, double& d) {
  double s = (a + b) + (c + d);
  double na = fma(-2.0, d, s), nb = fma(-2.0, c, s), nc = fma(-2.0, b, s), nd = fma(-2.0, a, s);
  a = na;
  b = nb;
  c = nc;
  d = nd;
}

// Radix-4 stage along the 16-entry array with digit stride S (1 or 4).
template <int S>
__device__ __forceinline__ void h4_stage(double (&v)[16]) {
#pragma unroll
  for (int base = 0; base < 16; ++base) {
    if ((base / S) % 4 == 0) h4(v[base], v[base + S], v[base + 2 * S], v[base + 3 * S]);
  }
}

// RN(a / d) for a bf16-precision a (at most 8 significant bits) and inv = RN(1 / d), in three operations: the
// remainder of q0 = RN(a * inv) is exact in one fma and one more fma corrects q0 (Markstein). Checked exhaustively
// against the correctly rounded division for every fp32 significand of d (tests/proofs/markstein_quotient.c).
__device__ __forceinline__ float quotient(float a, float d, float inv) {
  const float q0 = a * inv;
  const float r = fmaf(-q0, d, a);
  return fmaf(r, inv, q0);
}

size_t rotate_quant_lds_bytes(int waves, int K) { return (size_t)waves * (kRqScratchBytes + 2 * (size_t)K); }

// Element offset, within its 1024-element tile, of value 2i + h (h = 0, 1) of the 16 a lane holds after
// rotate_tile_packed (the layout its last butterfly stage leaves):
//   LOG4G <= 2: 16 lane + 2i + h                                   (natural order)
//   LOG4G == 3: lane = 4 gi + cq: 64 gi + 16 (i / 2) + 4 cq + 2 (i % 2) + h
//   LOG4G == 4: lane = 16 gi + b: 256 gi + 16 (2i + h) + b
//   LOG4G == 5: lane = 16 A + b, value v = 2i + h = 4k + g: 256 g + 16 (4A + k) + b   (the tile is one group)
template <int LOG4G>
__device__ __forceinline__ int held_offset(int lane, int i, int h) {
  if constexpr (LOG4G <= 2) return 16 * lane + 2 * i + h;
  if constexpr (LOG4G == 3) return 64 * (lane >> 2) + 16 * (i >> 1) + 4 * (lane & 3) + 2 * (i & 1) + h;
  if constexpr (LOG4G == 4) return 256 * (lane >> 4) + 16 * (2 * i + h) + (lane & 15);
  const int v = 2 * i + h;
  return 256 * (v & 3) + 16 * (4 * (lane >> 4) + (v >> 2)) + (lane & 15);
}

// Rows of the second transpose (LOG4G == 5): 17 doubles apart, so the four 16-lane groups of a read land on
// distinct banks.
constexpr int kRqStride2 = 17;
static_assert(64 * kRqStride2 <= 64 * kRqStride, "the second transpose fits the wave's scratch");

// Rotates one 1024-element tile (this lane's 16 consecutive inputs 16 lane .. 16 lane + 15 in cur0, cur1): v[2i + h]
// receives the exact unnormalised sum of value 2i + h of the layout of held_offset. `scratch` is the wave's fp64
// transpose area.
template <int LOG4G>
__device__ __forceinline__ void rotate_tile_f64(uint4 cur0, uint4 cur1, int lane, double* scratch, double (&v)[16]) {
  const uint32_t w[8] = {cur0.x, cur0.y, cur0.z, cur0.w, cur1.x, cur1.y, cur1.z, cur1.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    v[2 * i] = (double)bf16_lo(w[i]);
    v[2 * i + 1] = (double)bf16_hi(w[i]);
  }
  if constexpr (LOG4G >= 1) h4_stage<1>(v);
  if constexpr (LOG4G >= 2) h4_stage<4>(v);
  if constexpr (LOG4G >= 3) {
    // Transpose the fp64 pencils through LDS so each lane holds 16 values along digits 2 (and 3).
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      double2 pr;
      pr.x = v[2 * i];
      pr.y = v[2 * i + 1];
      *reinterpret_cast<double2*>(scratch + lane * kRqStride + 2 * i) = pr;
    }
    wave_lds_sync();
    if constexpr (LOG4G >= 4) {
      // lane = 16*gi + b; v[a] = pencil (16*gi + a), column b
      const int gi = lane >> 4, b = lane & 15;
#pragma unroll
      for (int a = 0; a < 16; ++a) v[a] = scratch[(16 * gi + a) * kRqStride + b];
      h4_stage<1>(v);
      h4_stage<4>(v);
      if constexpr (LOG4G == 5) {
        // Digit 4 is gi (lane bits 4-5): a second pass through LDS gives lane (A, b) the values of a = 4A + k for
        // every gi, v[4k + gi], and one more radix-4 stage runs along gi.
        wave_lds_sync();  // every lane has read the first transpose
#pragma unroll
        for (int a = 0; a < 16; ++a) scratch[(16 * gi + a) * kRqStride2 + b] = v[a];
        wave_lds_sync();
        const int A = lane >> 4;
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int g = 0; g < 4; ++g) v[4 * k + g] = scratch[(16 * g + 4 * A + k) * kRqStride2 + b];
        h4_stage<1>(v);
      }
    } else {
      // lane = 4*gi + cq; v[4a + cc] = pencil (4*gi + a), column 4*cq + cc
      const int gi = lane >> 2, cq = lane & 3;
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) v[4 * a + cc] = scratch[(4 * gi + a) * kRqStride + 4 * cq + cc];
      h4_stage<4>(v);
    }
    wave_lds_sync();  // scratch is rewritten by the next tile
  }
}

// rotate_tile_f64, then every value rounded once to bf16, returned as 8 packed pairs (low half first) in the layout
// of held_offset, with this lane's absmax of the rounded, still unnormalised sums.
template <int LOG4G>
__device__ __forceinline__ float rotate_tile_packed(uint4 cur0, uint4 cur1, int lane, double* scratch,
                                                    uint32_t (&packed)[8]) {
  float amax = 0.0f;
  double v[16];
  rotate_tile_f64<LOG4G>(cur0, cur1, lane, scratch, v);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float lo = round_f64_to_bf16_value(v[2 * i]);
    const float hi = round_f64_to_bf16_value(v[2 * i + 1]);
    amax = fmaxf(amax, fmaxf(fabsf(lo), fabsf(hi)));
    packed[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
  }
  return amax;
}

// rotate_tile_f64, then every value rounded once to bf16 (F32: to fp32), returned as fp32 values (the layout of
// held_offset), with this lane's absmax of the rounded, still unnormalised sums.
template <int LOG4G, bool F32 = false>
__device__ __forceinline__ float rotate_tile_rounded(uint4 cur0, uint4 cur1, int lane, double* scratch,
                                                     float (&f)[16]) {
  float amax = 0.0f;
  double v[16];
  rotate_tile_f64<LOG4G>(cur0, cur1, lane, scratch, v);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    f[i] = F32 ? (float)v[i] : round_f64_to_bf16_value(v[i]);
    amax = fmaxf(amax, fabsf(f[i]));
  }
  return amax;
}

// Rotates tile t of a row and parks the rounded bf16 bits in `rowbuf` (the row's buffer) at their natural positions
// (elements at or past K are not written). Returns this lane's absmax.
template <int LOG4G>
__device__ __forceinline__ float rotate_tile(uint4 cur0, uint4 cur1, int t, int K, int lane, double* scratch,
                                             uint16_t* rowbuf) {
  uint32_t packed[8];
  const float amax = rotate_tile_packed<LOG4G>(cur0, cur1, lane, scratch, packed);
  const int base = t * kRqTile;
  if constexpr (LOG4G <= 2) {
    if (base + lane * 16 < K) {
      uint4* dst = reinterpret_cast<uint4*>(rowbuf + base + lane * 16);
      dst[0] = make_uint4(packed[0], packed[1], packed[2], packed[3]);
      dst[1] = make_uint4(packed[4], packed[5], packed[6], packed[7]);
    }
  } else {
    // A lane's 16 values lie in one Hadamard group, which is wholly inside or wholly past K.
    if (base + held_offset<LOG4G>(lane, 0, 0) < K) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if constexpr (LOG4G == 3) {
          *reinterpret_cast<uint32_t*>(rowbuf + base + held_offset<LOG4G>(lane, i, 0)) = packed[i];
        } else {
          rowbuf[base + held_offset<LOG4G>(lane, i, 0)] = (uint16_t)packed[i];
          rowbuf[base + held_offset<LOG4G>(lane, i, 1)] = (uint16_t)(packed[i] >> 16);
        }
      }
    }
  }
  return amax;
}

// The row's scale and its quotient helpers from the absmax of the unnormalised rounded sums: amax of xr = amax *
// 2^-n (exact); then the reference's clamp and division (int8.py:177).
struct RowScale {
  float sx, d, inv;
};

__device__ __forceinline__ RowScale row_scale_n(float amax, int log4g) {
  RowScale r;
  r.sx = fmaxf(ldexpf(amax, -log4g), 1e-12f) / 127.0f;
  r.d = ldexpf(r.sx, log4g);  // (t * 2^n) / (sx * 2^n) == xr / sx exactly
  r.inv = 1.0f / r.d;         // correctly rounded; the per-element quotients use it
  return r;
}

template <int LOG4G>
__device__ __forceinline__ RowScale row_scale(float amax) {
  return row_scale_n(amax, LOG4G);
}

// Quantizes 8 packed bf16 pairs (int8.py:178): value v = 2i + h of the pairs becomes byte v % 4 of out[v / 4].
// The quotient of a value by the row's scale is at most 127 in magnitude (the absmax maps to 127 and nothing is
// larger), so the reference's clamp never acts on finite input. Rounding to an integer is an add of 1.5 * 2^23: the
// sum's exponent leaves units in the last place, so the add rounds the quotient to an integer, ties to even (torch's
// round), and the integer's two's-complement low byte is the sum's low byte; v_perm_b32 gathers four such bytes.
// (Non-finite input gives unspecified codes, as the reference's int8 cast of NaN does.)
constexpr float kRoundMagic = 12582912.0f;  // 1.5 * 2^23

// The 16 codes of 8 packed bf16 pairs, each in the low byte of its word (value v = 2i + h of the pairs in word v).
__device__ __forceinline__ void quantize_bytes(const uint32_t (&w)[8], const RowScale& rs, uint32_t (&b)[16]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    b[2 * i] = __float_as_uint(quotient(bf16_lo(w[i]), rs.d, rs.inv) + kRoundMagic);
    b[2 * i + 1] = __float_as_uint(quotient(bf16_hi(w[i]), rs.d, rs.inv) + kRoundMagic);
  }
}

// The same for 16 values held as fp32 (each exactly a bf16 value).
__device__ __forceinline__ void quantize_values(const float (&f)[16], const RowScale& rs, uint32_t (&b)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) b[i] = __float_as_uint(quotient(f[i], rs.d, rs.inv) + kRoundMagic);
}

// The low bytes of 16 words packed into 4 (word v's byte becomes byte v % 4 of out[v / 4]).
__device__ __forceinline__ void pack_low_bytes(const uint32_t (&b)[16], uint32_t (&out)[4]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    // perm(a, b, sel): selector byte k picks byte k of b (0-3) or of a (4-7); 0x0c gives zero.
    const uint32_t lo = __builtin_amdgcn_perm(b[4 * i + 1], b[4 * i], 0x0c0c0400u);      // bytes: v0, v1, 0, 0
    const uint32_t hi = __builtin_amdgcn_perm(b[4 * i + 3], b[4 * i + 2], 0x04000c0cu);  // bytes: 0, 0, v2, v3
    out[i] = lo | hi;
  }
}

__device__ __forceinline__ void quantize_packed(const uint32_t (&w)[8], const RowScale& rs, uint32_t (&out)[4]) {
  uint32_t b[16];
  quantize_bytes(w, rs, b);
  pack_low_bytes(b, out);
}

// Quantizes this lane's 16 elements of tile t from the row buffer (int8.py:178) and writes them (16 bytes).
__device__ __forceinline__ void quantize_tile(const uint16_t* rowbuf, int t, int K, int lane, const RowScale& rs,
                                              int8_t* qrow) {
  const int e0 = t * kRqTile + lane * 16;
  if (e0 >= K) return;
  const uint4* src = reinterpret_cast<const uint4*>(rowbuf + e0);
  const uint4 a = src[0], b = src[1];
  const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t out[4];
  quantize_packed(w, rs, out);
  *reinterpret_cast<uint4*>(qrow + e0) = make_uint4(out[0], out[1], out[2], out[3]);
}

__device__ __forceinline__ void load_pencil(const uint16_t* xrow, int e, int K, uint4& a, uint4& b) {
  a = make_uint4(0, 0, 0, 0);
  b = a;
  if (e < K) {
    a = *reinterpret_cast<const uint4*>(xrow + e);
    b = *reinterpret_cast<const uint4*>(xrow + e + 8);
  }
}

// Many rows: one wave per row, walking the row's tiles with the next tile's loads in flight.
template <int LOG4G>
__global__ __launch_bounds__(256) void rotate_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           int8_t* __restrict__ q, int64_t ldq,
                                                           float* __restrict__ s, int64_t M, int K) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar addressing
  const int waves = blockDim.x >> 6;
  unsigned char* mine = smem + (size_t)wave * (kRqScratchBytes + 2 * (size_t)K);
  double* scratch = reinterpret_cast<double*>(mine);
  uint16_t* rowbuf = reinterpret_cast<uint16_t*>(mine + kRqScratchBytes);
  const int ntiles = (K + kRqTile - 1) / kRqTile;

  for (int64_t row = (int64_t)blockIdx.x * waves + wave; row < M; row += (int64_t)gridDim.x * waves) {
    const uint16_t* xrow = x + row * ldx;
    float amax = 0.0f;
    uint4 nxt0, nxt1;
    load_pencil(xrow, lane * 16, K, nxt0, nxt1);
    for (int t = 0; t < ntiles; ++t) {
      const uint4 cur0 = nxt0, cur1 = nxt1;
      if (t + 1 < ntiles) load_pencil(xrow, (t + 1) * kRqTile + lane * 16, K, nxt0, nxt1);
      amax = fmaxf(amax, rotate_tile<LOG4G>(cur0, cur1, t, K, lane, scratch, rowbuf));
    }
    const RowScale rs = row_scale<LOG4G>(wave_max(amax));
    if (lane == 0) s[row] = rs.sx;
    wave_lds_sync();
    int8_t* qrow = q + row * ldq;
    for (int t = 0; t < ntiles; ++t) quantize_tile(rowbuf, t, K, lane, rs, qrow);
    wave_lds_sync();  // the row buffer is rewritten by the next row
  }
}

// Few rows: one workgroup per row, one wave per 1024-element tile (the whole row's loads in flight at once); the
// row's absmax goes through LDS. Same arithmetic as rotate_quant_kernel.
size_t rotate_quant_row_lds_bytes(int K) {
  const int ntiles = (K + kRqTile - 1) / kRqTile;
  return (size_t)ntiles * kRqScratchBytes + 2 * (size_t)ntiles * kRqTile + 64 * sizeof(float);
}

template <int LOG4G>
__device__ __forceinline__ void rotate_quant_row(const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ q,
                                                 int64_t ldq, float* __restrict__ s, int K, int64_t row,
                                                 unsigned char* smem) {
  const int lane = threadIdx.x & 63;
  const int t = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // this wave's tile (uniform)
  const int ntiles = blockDim.x >> 6;
  double* scratch = reinterpret_cast<double*>(smem + (size_t)t * kRqScratchBytes);
  uint16_t* rowbuf = reinterpret_cast<uint16_t*>(smem + (size_t)ntiles * kRqScratchBytes);
  float* maxes = reinterpret_cast<float*>(smem + (size_t)ntiles * kRqScratchBytes + 2 * (size_t)ntiles * kRqTile);
  uint4 a, b;
  load_pencil(x + row * ldx, t * kRqTile + lane * 16, K, a, b);
  const float amax = wave_max(rotate_tile<LOG4G>(a, b, t, K, lane, scratch, rowbuf));
  if (lane == 0) maxes[t] = amax;
  __syncthreads();
  float m = 0.0f;
  for (int i = 0; i < ntiles; ++i) m = fmaxf(m, maxes[i]);
  const RowScale rs = row_scale<LOG4G>(m);
  if (threadIdx.x == 0) s[row] = rs.sx;
  quantize_tile(rowbuf, t, K, lane, rs, q + row * ldq);  // this wave's own tile: its writes are visible to it
}

// `fin`: the layer's low-rank partial sums of this row, added by the row's first wave (LrFinish; part null: none);
// their loads are issued before the rotation so they land while it runs.
template <int LOG4G>
__global__ __launch_bounds__(1024) void rotate_quant_row_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                int8_t* __restrict__ q, int64_t ldq,
                                                                float* __restrict__ s, int K, LrFinish fin) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const bool lr = fin.part && threadIdx.x < fin.r;
  float p[kMaxSplits];
  if (lr) lr_reduce_load(fin.part, fin.splits, fin.M, fin.r, (int64_t)blockIdx.x * fin.r + threadIdx.x, p);
  rotate_quant_row<LOG4G>(x, ldx, q, ldq, s, K, blockIdx.x, smem);
  if (lr) fin.u[(int64_t)blockIdx.x * fin.ldu + threadIdx.x] = lr_reduce_sum(p, fin.splits);
}

// The row rotation and the row-wise low-rank down projection (lowrank_row_block) of the same few rows in one launch:
// both read x and neither depends on the other, so workgroups [0, lowrank_row_blocks) project (row, group of 8
// ranks) and the next M workgroups rotate a row, side by side on the CUs, in place of two (or, with the split
// low-rank kernel, three) launches in a row. Each row's results are those of the separate kernels, bit for bit.
template <int LOG4G>
__global__ __launch_bounds__(1024) void rotate_lowrank_row_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                  int8_t* __restrict__ q, int64_t ldq,
                                                                  float* __restrict__ s,
                                                                  const uint16_t* __restrict__ down, int64_t ld_down,
                                                                  uint16_t* __restrict__ u, int64_t ldu, int M, int K,
                                                                  int r, int groups) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int64_t b = blockIdx.x, lr_blocks = lowrank_row_blocks(M, r);
  if (b < lr_blocks)
    lowrank_row_block(b, groups, x, ldx, down, ld_down, u, ldu, M, K, r, reinterpret_cast<float*>(smem));
  else
    rotate_quant_row<LOG4G>(x, ldx, q, ldq, s, K, b - lr_blocks, smem);
}

// Many rows, rows up to 20 tiles: the rounded row stays in registers (as fp32) instead of an LDS row buffer, so a
// workgroup needs only the fp64 transpose areas and occupancy is set by registers (3 waves per SIMD at 5 tiles per
// wave). A row is split over `wpr` waves of TPW <= 5 consecutive tiles each; a workgroup holds 4 / wpr rows (one when
// wpr = 3). The waves of a row combine their absmax through LDS, then each quantizes its own tiles; the bytes of a
// tile go back to natural order through the (now free) transpose area so every lane stores 16 consecutive bytes.
// Same arithmetic as rotate_quant_kernel.
// Writes a tile's 16 codes per lane (each in the low byte of its word, in the layout of held_offset) to the row in
// natural order: directly for LOG4G <= 2, else through the wave's staging bytes (each code written straight from
// its word, then 16 consecutive bytes read back per lane).
template <int LOG4G>
__device__ __forceinline__ void store_codes(const uint32_t (&b)[16], int base, int K, int lane, unsigned char* stage,
                                            int8_t* qrow) {
  if constexpr (LOG4G <= 2) {
    uint32_t out[4];
    pack_low_bytes(b, out);
    if (base + lane * 16 < K)
      *reinterpret_cast<uint4*>(qrow + base + lane * 16) = make_uint4(out[0], out[1], out[2], out[3]);
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (LOG4G == 3) {
        *reinterpret_cast<uint16_t*>(stage + held_offset<LOG4G>(lane, j, 0)) =
            (uint16_t)__builtin_amdgcn_perm(b[2 * j + 1], b[2 * j], 0x0c0c0400u);
      } else {
        stage[held_offset<LOG4G>(lane, j, 0)] = (unsigned char)b[2 * j];
        stage[held_offset<LOG4G>(lane, j, 1)] = (unsigned char)b[2 * j + 1];
      }
    }
    wave_lds_sync();
    if (base + lane * 16 < K)
      *reinterpret_cast<uint4*>(qrow + base + lane * 16) = *reinterpret_cast<const uint4*>(stage + lane * 16);
    wave_lds_sync();  // the next tile rewrites the staging bytes
  }
}

// Quantizes one held tile (16 fp32 values in the layout of held_offset) and writes its codes (store_codes).
template <int LOG4G>
__device__ __forceinline__ void quantize_store_tile(const float (&f)[16], const RowScale& rs, int base, int K,
                                                    int lane, unsigned char* stage, int8_t* qrow) {
  uint32_t b[16];
  quantize_values(f, rs, b);
  store_codes<LOG4G>(b, base, K, lane, stage, qrow);
}

size_t rotate_quant_reg_lds_bytes(int waves) { return (size_t)waves * kRqScratchBytes + 16; }

// Five tiles per wave held as fp32 (80 VGPRs; 118 in all with the wave index and the row descriptor in scalar
// registers) leave four waves per SIMD (three with the 1024 group's second transpose).
//
// F32: the arithmetic of the reference's GPU kernels (rotate_quant_f32_recip_kernel's: each sum rounded once to
// fp32, codes by the reciprocal multiply) in this one-pass layout; the rounded row is held in the same registers.
template <int LOG4G, int TPW, bool F32>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(TPW == kRqRegMaxTpw ? (LOG4G == 5 ? 3 : 4) : 1)))
void rotate_quant_reg_kernel(const uint16_t* __restrict__ x, int64_t ldx, int8_t* __restrict__ q, int64_t ldq,
                             float* __restrict__ s, int64_t M, int K, int wpr, LrFinish fin) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar addressing
  const int nwaves = blockDim.x >> 6;
  double* scratch = reinterpret_cast<double*>(smem + (size_t)wave * kRqScratchBytes);
  float* maxes = reinterpret_cast<float*>(smem + (size_t)nwaves * kRqScratchBytes);
  const int64_t row = (int64_t)blockIdx.x * (nwaves / wpr) + wave / wpr;
  const int part = wave % wpr;
  const bool live = row < M;
  const int kvalid = live ? K : 0;  // a row past the matrix reads zeros and stores nothing
  const uint16_t* xrow = x + (live ? row : 0) * ldx;
  const int t0 = part * TPW;

  // held[i] first receives tile i's raw pencil in its first 8 words (all of this wave's loads in flight at once),
  // then the tile's 16 rounded values. The loads go through a buffer descriptor that covers the row's valid bytes
  // (none for a row past the matrix): a pencil at or past K reads as zeros without a branch, so every load is issued
  // unconditionally in order and tile i waits only for its own two loads, not for the whole row's.
  const __amdgpu_buffer_rsrc_t rx = make_rsrc(xrow, 2u * (uint32_t)kvalid);
  float held[TPW][16];
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int off = 2 * ((t0 + i) * kRqTile + lane * 16);
    const v4u a = __builtin_amdgcn_raw_buffer_load_b128(rx, off, 0, 0);
    const v4u b = __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16, 0, 0);
    const uint32_t raw[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int j = 0; j < 8; ++j) held[i][j] = __uint_as_float(raw[j]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    // A tile wholly past K (the last wave of a row whose tiles do not split evenly) costs no rotation work.
    if ((t0 + i) * kRqTile >= kvalid) continue;
    const uint4 a = make_uint4(__float_as_uint(held[i][0]), __float_as_uint(held[i][1]), __float_as_uint(held[i][2]),
                               __float_as_uint(held[i][3]));
    const uint4 b = make_uint4(__float_as_uint(held[i][4]), __float_as_uint(held[i][5]), __float_as_uint(held[i][6]),
                               __float_as_uint(held[i][7]));
    amax = fmaxf(amax, rotate_tile_rounded<LOG4G, F32>(a, b, lane, scratch, held[i]));
  }
  amax = wave_max(amax);
  float m = amax;
  if (wpr > 1) {
    // The waves of a row combine their maxima. With one wave per row there is nothing to combine and no barrier:
    // the workgroup's waves (rows) run independently.
    if (lane == 0) maxes[wave] = amax;
    __syncthreads();
    m = 0.0f;
    for (int w = 0; w < wpr; ++w) m = fmaxf(m, maxes[(wave / wpr) * wpr + w]);
  }
  if (!live) return;
  int8_t* qrow = q + row * ldq;
  unsigned char* stage = reinterpret_cast<unsigned char*>(scratch);  // the transpose area is free from here on
  if constexpr (F32) {
    // rotate_quant_f32_recip_kernel's scale and codes (|xr * inv| <= 127: the clamp never acts on finite input).
    const float sx = fmaxf(ldexpf(m, -LOG4G), 1e-12f) / 127.0f;
    const float inv_n = ldexpf(1.0f / sx, -LOG4G);
    if (part == 0 && lane == 0) s[row] = sx;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int base = (t0 + i) * kRqTile;
      if (base < K) {
        uint32_t codes[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) codes[j] = __float_as_uint(held[i][j] * inv_n + kRoundMagic);
        store_codes<LOG4G>(codes, base, K, lane, stage, qrow);
      }
    }
  } else {
    const RowScale rs = row_scale<LOG4G>(m);
    if (part == 0 && lane == 0) s[row] = rs.sx;
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int base = (t0 + i) * kRqTile;
      if (base < K) quantize_store_tile<LOG4G>(held[i], rs, base, K, lane, stage, qrow);
    }
  }
  // The layer's low-rank partial sums of this row (LrFinish; part null: none), added by the row's first wave.
  if (fin.part && part == 0) lr_finish_row(fin, row, lane);
}

// The arithmetic of the reference's GPU kernels (rotate_quant_kernel / rotate_quant_factored_kernel,
// src/hyperflow_h3_flash/int8.py:194-262): the rotated value is the exact sum rounded once to fp32 (not bf16),
//   sx = max(absmax_row(xr), 1e-12) / 127,  inv = 1 / sx  (fp32),  xq = clamp(rint(fp32(xr * inv)), -127, 127).
// Two passes over the row like the reference's kernels (the absmax, then the rotation again for the codes): one wave
// per row, tiles of 1024, the fp64 butterfly of rotate_tile_f64. The 2^-n normalisation is a power of two folded
// into the scale: fp32(t 2^-n) = fp32(t) 2^-n and xr * inv = fp32(t) * (inv 2^-n) exactly.
template <int LOG4G>
__global__ __launch_bounds__(256) void rotate_quant_f32_recip_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                     int8_t* __restrict__ q, int64_t ldq,
                                                                     float* __restrict__ s, int64_t M, int K) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: scalar addressing
  const int waves = blockDim.x >> 6;
  double* scratch = reinterpret_cast<double*>(smem + (size_t)wave * kRqScratchBytes);
  unsigned char* stage = reinterpret_cast<unsigned char*>(scratch);
  const int ntiles = (K + kRqTile - 1) / kRqTile;
  for (int64_t row = (int64_t)blockIdx.x * waves + wave; row < M; row += (int64_t)gridDim.x * waves) {
    const uint16_t* xrow = x + row * ldx;
    float amax = 0.0f;
    for (int t = 0; t < ntiles; ++t) {
      uint4 a, b;
      load_pencil(xrow, t * kRqTile + lane * 16, K, a, b);
      double v[16];
      rotate_tile_f64<LOG4G>(a, b, lane, scratch, v);
#pragma unroll
      for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf((float)v[i]));
    }
    const float sx = fmaxf(ldexpf(wave_max(amax), -LOG4G), 1e-12f) / 127.0f;
    const float inv_n = ldexpf(1.0f / sx, -LOG4G);
    if (lane == 0) s[row] = sx;
    int8_t* qrow = q + row * ldq;
    for (int t = 0; t < ntiles; ++t) {
      uint4 a, b;
      load_pencil(xrow, t * kRqTile + lane * 16, K, a, b);
      double v[16];
      rotate_tile_f64<LOG4G>(a, b, lane, scratch, v);
      // |xr * inv| <= 127 (the absmax maps to 127): the clamp never acts on finite input; the rounding add of
      // quantize_bytes gives rint and the code in the low byte.
      uint32_t codes[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) codes[i] = __float_as_uint((float)v[i] * inv_n + kRoundMagic);
      store_codes<LOG4G>(codes, t * kRqTile, K, lane, stage, qrow);
    }
  }
}

size_t rotate_quant_f32_recip_lds_bytes(int waves) { return (size_t)waves * kRqScratchBytes; }

// Hadamard groups of 4^5 = 1024 elements and more (a group spans one or more whole 1024-element tiles): one
// workgroup per row keeps the row's unnormalised fp64 sums in LDS, 8 bytes per element. Each thread loads 16
// consecutive elements and transforms digits 0-1 in registers; every higher digit of the in-group index is then a
// radix-4 pass over the LDS row (stride 4^d; consecutive threads take consecutive quadruples), a barrier between
// passes. The butterflies are those of the tile kernels (exact while a group's nonzero inputs span at most
// 53 - 8 - 2 log4(G) binades). The rounding and quantization are rotate_quant_kernel's (each sum rounded once to bf16,
// true division) or, with F32_RECIP, rotate_quant_f32_recip_kernel's (rounded once to fp32, reciprocal multiply).
constexpr int kRqWideThreads = 256;
size_t rotate_quant_wide_lds_bytes(int K) { return 8 * (size_t)K + 4 * sizeof(float); }

template <bool F32_RECIP>
__global__ __launch_bounds__(kRqWideThreads) void rotate_quant_wide_kernel(const uint16_t* __restrict__ x,
                                                                          int64_t ldx, int8_t* __restrict__ q,
                                                                          int64_t ldq, float* __restrict__ s, int K,
                                                                          int log4g) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  double* rowbuf = reinterpret_cast<double*>(smem);
  float* maxes = reinterpret_cast<float*>(smem + 8 * (size_t)K);
  const int t = threadIdx.x, lane = t & 63, wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int64_t row = blockIdx.x;
  const uint16_t* xrow = x + row * ldx;

  for (int p = t; p < K / 16; p += kRqWideThreads) {
    const uint4 a = *reinterpret_cast<const uint4*>(xrow + 16 * p);
    const uint4 b = *reinterpret_cast<const uint4*>(xrow + 16 * p + 8);
    const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    double v[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[2 * i] = (double)bf16_lo(w[i]);
      v[2 * i + 1] = (double)bf16_hi(w[i]);
    }
    h4_stage<1>(v);
    h4_stage<4>(v);
    double2* dst = reinterpret_cast<double2*>(rowbuf + 16 * p);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = make_double2(v[2 * i], v[2 * i + 1]);
  }
  __syncthreads();
  for (int d = 2; d < log4g; ++d) {
    const int sh = 2 * d, S = 1 << sh;
    for (int qd = t; qd < K / 4; qd += kRqWideThreads) {
      const int i = ((qd >> sh) << (sh + 2)) | (qd & (S - 1));
      double a = rowbuf[i], b = rowbuf[i + S], c = rowbuf[i + 2 * S], e = rowbuf[i + 3 * S];
      h4(a, b, c, e);
      rowbuf[i] = a;
      rowbuf[i + S] = b;
      rowbuf[i + 2 * S] = c;
      rowbuf[i + 3 * S] = e;
    }
    __syncthreads();
  }

  auto rounded = [](double v) { return F32_RECIP ? (float)v : round_f64_to_bf16_value(v); };
  float amax = 0.0f;
  for (int e = t; e < K; e += kRqWideThreads) amax = fmaxf(amax, fabsf(rounded(rowbuf[e])));
  amax = wave_max(amax);
  if (lane == 0) maxes[wave] = amax;
  __syncthreads();
  const float m = fmaxf(fmaxf(maxes[0], maxes[1]), fmaxf(maxes[2], maxes[3]));
  const RowScale rs = row_scale_n(m, log4g);
  const float inv_n = ldexpf(1.0f / rs.sx, -log4g);  // the reciprocal arithmetic's factor (F32_RECIP)
  if (t == 0) s[row] = rs.sx;

  // Four consecutive codes per thread, one 4-byte store.
  int8_t* qrow = q + row * ldq;
  for (int c = t; c < K / 4; c += kRqWideThreads) {
    const double2 lo = *reinterpret_cast<const double2*>(rowbuf + 4 * c);
    const double2 hi = *reinterpret_cast<const double2*>(rowbuf + 4 * c + 2);
    const double v[4] = {lo.x, lo.y, hi.x, hi.y};
    uint32_t code[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float f = rounded(v[i]);
      code[i] = __float_as_uint((F32_RECIP ? f * inv_n : quotient(f, rs.d, rs.inv)) + kRoundMagic);
    }
    const uint32_t word = __builtin_amdgcn_perm(code[1], code[0], 0x0c0c0400u) |
                          __builtin_amdgcn_perm(code[3], code[2], 0x04000c0cu);
    *reinterpret_cast<uint32_t*>(qrow + 4 * c) = word;
  }
}

template __global__ void rotate_quant_f32_recip_kernel<1>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t,
                                                          int);
template __global__ void rotate_quant_f32_recip_kernel<2>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t,
                                                          int);
template __global__ void rotate_quant_f32_recip_kernel<3>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t,
                                                          int);
template __global__ void rotate_quant_f32_recip_kernel<4>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t,
                                                          int);
template __global__ void rotate_quant_f32_recip_kernel<5>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t,
                                                          int);

template __global__ void rotate_quant_wide_kernel<false>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int, int);
template __global__ void rotate_quant_wide_kernel<true>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int, int);

#define HF_RQ_REG(L, T)                                                                                            \
  template __global__ void rotate_quant_reg_kernel<L, T, false>(const uint16_t*, int64_t, int8_t*, int64_t, float*,\
                                                                int64_t, int, int, LrFinish);                     \
  template __global__ void rotate_quant_reg_kernel<L, T, true>(const uint16_t*, int64_t, int8_t*, int64_t, float*, \
                                                               int64_t, int, int, LrFinish);
#define HF_RQ_REG_ALL(L) HF_RQ_REG(L, 1) HF_RQ_REG(L, 2) HF_RQ_REG(L, 3) HF_RQ_REG(L, 4) HF_RQ_REG(L, 5)
HF_RQ_REG_ALL(1)
HF_RQ_REG_ALL(2)
HF_RQ_REG_ALL(3)
HF_RQ_REG_ALL(4)
HF_RQ_REG_ALL(5)
#undef HF_RQ_REG_ALL
#undef HF_RQ_REG

template __global__ void rotate_quant_kernel<1>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t, int);
template __global__ void rotate_quant_kernel<2>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t, int);
template __global__ void rotate_quant_kernel<3>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t, int);
template __global__ void rotate_quant_kernel<4>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t, int);
template __global__ void rotate_quant_kernel<5>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int64_t, int);
template __global__ void rotate_quant_row_kernel<1>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int,
                                                    LrFinish);
template __global__ void rotate_quant_row_kernel<2>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int,
                                                    LrFinish);
template __global__ void rotate_quant_row_kernel<3>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int,
                                                    LrFinish);
template __global__ void rotate_quant_row_kernel<4>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int,
                                                    LrFinish);
template __global__ void rotate_quant_row_kernel<5>(const uint16_t*, int64_t, int8_t*, int64_t, float*, int,
                                                    LrFinish);
#define HF_RQ_LR_ROW(G)                                                                                             \
  template __global__ void rotate_lowrank_row_kernel<G>(const uint16_t*, int64_t, int8_t*, int64_t, float*,         \
                                                        const uint16_t*, int64_t, uint16_t*, int64_t, int, int, int, \
                                                        int);
HF_RQ_LR_ROW(1)
HF_RQ_LR_ROW(2)
HF_RQ_LR_ROW(3)
HF_RQ_LR_ROW(4)
HF_RQ_LR_ROW(5)
#undef HF_RQ_LR_ROW

}  // namespace hf
