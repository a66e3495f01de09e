// INT8 x INT8 -> INT32 GEMM with the convrot epilogue for a few hundred to a few thousand rows: 256 (m) x 128 (n)
// output tiles, one per workgroup (not persistent: these shapes fill the CUs about once).
//
// Same arithmetic as int8_gemm_kernel (the reference's int8_mm_kernel + rescale, src/hyperflow_h3_flash/int8.py:
// 283-324, extended with the low-rank term of transformer.py:57-58 and a bias):
//   y[m, n] = bf16((f32(acc[m, n]) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n])   (acc exact int32)
// optionally followed by the tanh-GELU of the FFN up-projection (rounded to bf16 again). With no low-rank branch and
// no bias the output is bitwise the reference's.
//
// Why this tile: with 256 x 256 tiles a shape such as M = 256, N = 30720 or M = 1024, N = 5120 gives fewer tiles
// than CUs, and splitting K writes and re-reads int32 partial planes. Halving the tile's n side doubles the tiles
// and keeps the operand stream at (256 + 128) x 128 bytes per 4.2 M multiply-adds per stage: 48 KiB per 1024 MFMA
// cycles, inside what one CU's L2 -> LDS path delivers (about 64 bytes per clock). Smaller tiles would be bound by
// that path rather than by the matrix cores.
//
// 8 waves in a 4 (m) x 2 (n) grid, each a 64 x 64 sub-tile of 2 x 2 v_mfma_i32_32x32x32_i8 blocks (the weight is the
// MFMA's first operand, so each lane ends with four consecutive n of one row m, as in int8_gemm_kernel). K runs in
// stages of 128 bytes through a 3-slot LDS ring (48 KiB a slot: 256 q rows and 128 w rows of 128 bytes, loaded with
// buffer_load ... lds as whole 128-byte lines), so each stage's loads are issued two stages ahead. The slot freed at
// the second-to-last boundary receives the tile's low-rank operands (u rows m, up rows n, rank <= 64); after the
// K loop the other two slots stage the bf16 output for whole-line stores.
#pragma once

#include "common.h"

namespace hf {

constexpr int kMidBM = 256;
constexpr int kMidBN = 128;
constexpr int kMidBK = 128;
constexpr int kMidAStage = kMidBM * kMidBK;          // 32 KiB
constexpr int kMidSlot = kMidAStage + kMidBN * kMidBK;  // 48 KiB
constexpr int kMidSlots = 3;
constexpr int kMidParamBytes = (kMidBM + 2 * kMidBN) * 4;  // sx of the tile's rows, wscale and bias of its columns
constexpr int kMidLds = kMidSlots * kMidSlot + kMidParamBytes;
constexpr int kMidThreads = 512;
constexpr int kMidLoads = 6;  // 1 KiB loads per wave and stage: 4 blocks of q rows, 2 of w rows

struct MidArgs {
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
  int r;               // 0 or a multiple of 8 up to 64
  const uint16_t* bias;
  uint16_t* y;
  int64_t ldy;
  int M, N, K;
  int tiles_m, tiles_n;
  int out_vec16;       // 16-byte aligned output rows
};

// Chunk c of LDS row r (128-byte rows) sits at c ^ mid_swz(r): conflict-free for the 16 rows a ds_read_b128 cycle
// serves, and the same for every 32-row MFMA block.
__device__ __forceinline__ int mid_swz(int r) { return (r & 7) ^ ((r >> 3) & 3); }

// Workgroup -> tile. Workgroups are dealt to the 8 XCDs round robin; XCD x takes a contiguous range of the tiles
// ordered column-major (tile rows fastest), so the tiles sharing a weight panel run on one XCD and read it once from
// its L2.
__device__ __forceinline__ void mid_tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n, per = total / 8, rem = total % 8, xcd = bid % 8, local = bid / 8;
  const int logical = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  tm = logical % tiles_m;
  tn = logical / tiles_m;
}

template <int ACT>
__global__ __launch_bounds__(kMidThreads, 1) void mid_gemm_kernel(MidArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char mid_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)mid_smem_raw;
  float HF_LDS* params = (float HF_LDS*)(smem + kMidSlots * kMidSlot);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 3, wn = wave >> 2;  // 4 (m) x 2 (n) waves of 64 x 64
  const int sub = lane & 31, half = lane >> 5;
  int tm = 0, tn = 0;
  mid_tile_of(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  tm = __builtin_amdgcn_readfirstlane(tm);
  tn = __builtin_amdgcn_readfirstlane(tn);
  const int m0 = tm * kMidBM, n0 = tn * kMidBN;
  const int rows_m = min(kMidBM, a.M - m0), rows_n = min(kMidBN, a.N - n0);
  const uint32_t bytes_q = (uint32_t)(rows_m * a.ldq), bytes_w = (uint32_t)(rows_n * a.ldw);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + (int64_t)m0 * a.ldq, bytes_q);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + (int64_t)n0 * a.ldw, bytes_w);
  const bool lowrank = a.r > 0;

  // The epilogue's per-row and per-column factors (clamped indices; the zero factors of rows and columns past the
  // matrix are written below), issued before the stage loads so they land first.
  const int pt = threadIdx.x;
  float p_val;
  if (pt < kMidBM) {
    p_val = a.sx[min(m0 + pt, a.M - 1)];
  } else if (pt < kMidBM + kMidBN) {
    p_val = a.sw[min(n0 + pt - kMidBM, a.N - 1)];
  } else {
    const uint16_t* bsrc = a.bias ? a.bias : reinterpret_cast<const uint16_t*>(a.sw);
    p_val = __uint_as_float((uint32_t)bsrc[min(n0 + pt - kMidBM - kMidBN, a.N - 1)] << 16);
  }

  auto slot = [&](int s) { return smem + (s % kMidSlots) * kMidSlot; };
  // The low-rank operands' sources: u rows m0.. and up rows n0.. (rank r <= 64: one 128-byte row each; ranks past r
  // read zero).
  const uint32_t bytes_u = lowrank ? (uint32_t)(rows_m * a.ldu * 2) : 0u;
  const uint32_t bytes_up = lowrank ? (uint32_t)(rows_n * a.ldup * 2) : 0u;
  const __amdgpu_buffer_rsrc_t ru = make_rsrc(lowrank ? a.u + (int64_t)m0 * a.ldu : a.u, bytes_u);
  const __amdgpu_buffer_rsrc_t rup = make_rsrc(lowrank ? a.up + (int64_t)n0 * a.ldup : a.up, bytes_up);
  // Six loads per wave into slot `dst`: stage kt of q and w (K bytes kt * 128 ..), or, with `lr`, the low-rank
  // operands (u rows in the q half, up rows in the w half). Branch-free: the sources are scalar selects, so every
  // call issues the same instructions.
  auto issue = [&](int kt, bool lr, unsigned char HF_LDS* dst) {
    const __amdgpu_buffer_rsrc_t ra = lr ? ru : rq, rb = lr ? rup : rw;
    const uint32_t oob_a = lr ? bytes_u : bytes_q, oob_b = lr ? bytes_up : bytes_w;
    const int64_t ld_a = lr ? a.ldu * 2 : a.ldq, ld_b = lr ? a.ldup * 2 : a.ldw;
    const int col0 = lr ? 0 : kt * kMidBK, limit = lr ? 2 * a.r : a.K;
#pragma unroll
    for (int i = 0; i < kMidLoads; ++i) {
      const bool isb = i >= 4;
      const int blk = isb ? 2 * wave + i - 4 : 4 * wave + i;
      const int row = 8 * blk + (lane >> 3);
      const uint32_t chunk = (uint32_t)(((lane & 7) ^ mid_swz(row)) << 4);
      const int rows = isb ? rows_n : rows_m;
      const uint32_t col = (uint32_t)col0 + chunk;
      const uint32_t voff = ((row < rows) & (col < (uint32_t)limit)) ? (uint32_t)(row * (isb ? ld_b : ld_a)) + col
                                                                       : (isb ? oob_b : oob_a);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isb ? rb : ra, (void HF_LDS*)(dst + (isb ? kMidAStage : 0) + blk * 1024),
                                               16, voff, 0, 0, 0);
    }
  };

  const int nk = (a.K + kMidBK - 1) / kMidBK;
  issue(0, false, slot(0));
  issue(1, false, slot(1));
  // Two stages or fewer: the third slot is free from the start and takes the low-rank operands.
  issue(2, lowrank && nk <= 2, slot(2));
  // Park the factors (the vmcnt wait below covers them: they were issued first).
  asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  if (pt < kMidBM) {
    params[pt] = (m0 + pt < a.M) ? p_val : 0.0f;
  } else if (pt < kMidBM + kMidBN) {
    params[pt] = (n0 + pt - kMidBM < a.N) ? p_val : 0.0f;
  } else {
    params[pt] = (n0 + pt - kMidBM - kMidBN < a.N) ? p_val : 0.0f;
  }
  __syncthreads();

  int ca[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ca[ks] = sub * kMidBK + (((2 * ks + half) ^ mid_swz(sub)) << 4);
  v4i fa0[2], fb0[2], fa1[2], fb1[2];
  auto read = [&](v4i (&fa)[2], v4i (&fb)[2], const unsigned char HF_LDS* st, int ks) {
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) fa[jb] = *(const v4i HF_LDS*)(st + (wm * 64 + jb * 32) * kMidBK + ca[ks]);
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
      fb[ib] = *(const v4i HF_LDS*)(st + kMidAStage + (wn * 64 + ib * 32) * kMidBK + ca[ks]);
  };
  v16i acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (v16i){0};
  // One K step: the next step's four fragment reads go out first, each pair ahead of an MFMA, then (at a boundary)
  // the ring refill's six loads, two after each remaining MFMA.
  auto kstep = [&](const v4i (&fa)[2], const v4i (&fb)[2], auto&& reads, auto&& loads) {
    reads();
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
        acc[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fb[ib], fa[jb], acc[ib][jb], 0, 0, 0);
    loads();
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x020, 3, 0);  // VMEM (ring refill)
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto nothing = [] {};

  read(fa0, fb0, slot(0), 0);
  for (int s = 0; s < nk; ++s) {
    const unsigned char HF_LDS* st = slot(s);
    kstep(fa0, fb0, [&] { read(fa1, fb1, st, 1); }, nothing);
    kstep(fa1, fb1, [&] { read(fa0, fb0, st, 2); }, nothing);
    kstep(fa0, fb0, [&] { read(fa1, fb1, st, 3); }, nothing);
    // Boundary: stage s + 1 has landed once only stage s + 2's six loads (issued a boundary ago) are in flight; the
    // barrier makes that true for every wave and frees slot s (stage s's fragments are all in registers). Slot s
    // then receives stage s + 3 (zero-fill loads past K), or the low-rank operands when s + 3 is the stage count
    // (they land during the last two stages). After the last stage the first fragments read here are unused.
    asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const bool lr_now = lowrank && s + 3 == nk;
    unsigned char HF_LDS* refill = slot(s);
    kstep(fa1, fb1, [&] { read(fa0, fb0, slot(s + 1), 0); }, [&] { issue(s + 3, lr_now, refill); });
  }
  // Every load (the low-rank operands included) has landed and every wave is done with the ring.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();

  // --------------------------------------------------------------------------------------------------- epilogue
  // Output layout of a 32x32 block: lane holds row m = lane % 32 and, in register v, column
  // n = 8 (v / 4) + 4 (lane / 32) + v % 4.
  const int lr_slot = (nk >= 3) ? nk % kMidSlots : 2;  // the slot that received the low-rank operands
  const unsigned char HF_LDS* u_lds = slot(lr_slot);
  const unsigned char HF_LDS* up_lds = slot(lr_slot) + kMidAStage;
  v16f c[2][2];
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const float sxv = params[wm * 64 + jb * 32 + sub];
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int nl = wn * 64 + ib * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        c[ib][jb][v] = ((float)acc[ib][jb][v] * sxv) * params[kMidBM + nl];
      }
  }
  if (lowrank) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int chunk = 2 * kk + half;
      v8bf pf[2], uf[2];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
        const int nl = wn * 64 + ib * 32 + sub;
        pf[ib] = *(const v8bf HF_LDS*)(up_lds + nl * kMidBK + ((chunk ^ mid_swz(nl)) << 4));
      }
#pragma unroll
      for (int jb = 0; jb < 2; ++jb) {
        const int ml = wm * 64 + jb * 32 + sub;
        uf[jb] = *(const v8bf HF_LDS*)(u_lds + ml * kMidBK + ((chunk ^ mid_swz(ml)) << 4));
      }
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int jb = 0; jb < 2; ++jb) c[ib][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf[ib], uf[jb], c[ib][jb],
                                                                                          0, 0, 0);
    }
  }
  if (a.bias) {
#pragma unroll
    for (int ib = 0; ib < 2; ++ib)
#pragma unroll
      for (int jb = 0; jb < 2; ++jb)
#pragma unroll
        for (int v = 0; v < 16; ++v)
          c[ib][jb][v] = c[ib][jb][v] + params[kMidBM + kMidBN + wn * 64 + ib * 32 + 8 * (v >> 2) + 4 * half + (v & 3)];
  }
  // bf16 and the activation; after one exchange between the lane halves (v_permlane32_swap) lane (sub, h) holds
  // columns 16 h .. 16 h + 15 of row sub of the block: chunk 2 h in w4[0], w4[2] and chunk 2 h + 1 in w4[1], w4[3].
  uint32_t pk[2][2][8];
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 2; ++jb) {
      uint32_t w4[4][2];
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        w4[gq][0] = activate_bf16x2<ACT>(pack_bf16x2(c[ib][jb][4 * gq], c[ib][jb][4 * gq + 1]));
        w4[gq][1] = activate_bf16x2<ACT>(pack_bf16x2(c[ib][jb][4 * gq + 2], c[ib][jb][4 * gq + 3]));
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
      pk[ib][jb][0] = w4[0][0];
      pk[ib][jb][1] = w4[0][1];
      pk[ib][jb][2] = w4[2][0];
      pk[ib][jb][3] = w4[2][1];
      pk[ib][jb][4] = w4[1][0];
      pk[ib][jb][5] = w4[1][1];
      pk[ib][jb][6] = w4[3][0];
      pk[ib][jb][7] = w4[3][1];
    }
  // Stage the wave's 64 x 64 outputs (64 rows of 128 bytes, swizzled) in the slots after the low-rank one (every
  // wave is past the ring and the low-rank reads of other waves touch only lr_slot), then store 8 whole lines per
  // instruction.
  unsigned char HF_LDS* stage =
      slot(lr_slot + 1 + (wave >> 2)) + (wave & 3) * 8192;  // 4 waves x 8 KiB in each of the two other slots
#pragma unroll
  for (int jb = 0; jb < 2; ++jb) {
    const int row = jb * 32 + sub;
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int c0 = 4 * ib + 2 * half;
      *(v4i HF_LDS*)(stage + row * 128 + ((c0 ^ mid_swz(row)) << 4)) =
          (v4i){(int)pk[ib][jb][0], (int)pk[ib][jb][1], (int)pk[ib][jb][2], (int)pk[ib][jb][3]};
      *(v4i HF_LDS*)(stage + row * 128 + (((c0 + 1) ^ mid_swz(row)) << 4)) =
          (v4i){(int)pk[ib][jb][4], (int)pk[ib][jb][5], (int)pk[ib][jb][6], (int)pk[ib][jb][7]};
    }
  }
  wave_lds_sync();
  const bool full = rows_m == kMidBM && rows_n == kMidBN && a.out_vec16;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int row = 8 * i + (lane >> 3), ch = lane & 7;
    const v4i val = *(const v4i HF_LDS*)(stage + row * 128 + ((ch ^ mid_swz(row)) << 4));
    const int m = m0 + wm * 64 + row;
    const int n = n0 + wn * 64 + 8 * ch;
    uint16_t* dst = a.y + (int64_t)m * a.ldy + n;
    if (full) {
      *reinterpret_cast<v4i*>(dst) = val;
    } else if (m < a.M) {
      if (a.out_vec16 && n + 8 <= a.N) {
        *reinterpret_cast<v4i*>(dst) = val;
      } else {
        for (int e = 0; e < 8; ++e)
          if (n + e < a.N) dst[e] = (uint16_t)((uint32_t)val[e >> 1] >> (16 * (e & 1)));
      }
    }
  }
}

template __global__ void mid_gemm_kernel<kActNone>(MidArgs);
template __global__ void mid_gemm_kernel<kActGeluTanh>(MidArgs);

// ------------------------------------------------------------------------------------------------- 128-row bands
// band_gemm_kernel<NB>: 128 (m) x 32 NB (n) output tiles, one per workgroup, for shapes whose 256 x 128 tiles leave
// a third or more of the CUs idle while 128-row tiles fill them in one round (M=1024: N=5120 gives 160 tiles of
// 256 x 128 but 256 of 128 x 160; N=3072, 96 against 256 of 128 x 96). Same arithmetic and epilogue as
// mid_gemm_kernel.
//
// 8 waves: wave w takes row block wm = w % 4 (32 rows) and, of every 128-byte K stage, the two 32-byte K steps
// 2 kh and 2 kh + 1, kh = w / 4, against all NB column blocks (NB accumulators of 16 registers). The two waves of a
// SIMD (w and w + 4) thus share a row block and split each stage's K steps, so every SIMD keeps two waves to
// interleave while the LDS serves one A and NB B fragments per NB MFMAs. After the K loop each wave adds its partner's
// int32 sums for half of the column blocks (exact, through LDS) and finishes those blocks. K runs through a 4-slot
// ring of (128 + 32 NB) rows x 128 bytes (36 KiB at NB = 5), each stage's loads issued three stages ahead; the slot
// of the first stage past K receives the tile's low-rank operands.
constexpr int kBandBM = 128;
constexpr int kBandSlots = 4;
constexpr int kBandThreads = 512;
__host__ __device__ constexpr int band_slot(int nb) { return (kBandBM + 32 * nb) * 128; }
__host__ __device__ constexpr int band_blocks(int nb) { return 16 + 4 * nb; }               // 1 KiB loads a stage
__host__ __device__ constexpr int band_loads(int nb) { return (band_blocks(nb) + 7) / 8; }  // per wave and stage
__host__ __device__ constexpr int band_lds(int nb) {
  return kBandSlots * band_slot(nb) + (kBandBM + 64 * nb) * 4;
}

template <int NB, int ACT>
__global__ __launch_bounds__(kBandThreads, 1) void band_gemm_kernel(MidArgs a) {
  constexpr int BN = 32 * NB, kSlot = band_slot(NB), kAStage = kBandBM * 128, kLoads = band_loads(NB);
  constexpr int kBlocks = band_blocks(NB);
  constexpr int kH = (NB + 1) / 2;          // column blocks the kh = 0 wave finishes; the kh = 1 wave the rest
  constexpr int kXPerSlot = kSlot / 4096;   // 4 KiB exchange blocks per slot
  static_assert(8 * kH <= 3 * kXPerSlot, "the K-half exchange fits the three slots besides the low-rank one");
  static_assert(3 * kLoads <= 63, "wait counts");
  extern __shared__ __attribute__((aligned(1024))) unsigned char band_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)band_smem_raw;
  float HF_LDS* params = (float HF_LDS*)(smem + kBandSlots * kSlot);  // sx (128), wscale (BN), bias (BN)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave & 3, kh = wave >> 2;
  const int sub = lane & 31, half = lane >> 5;
  int tm = 0, tn = 0;
  mid_tile_of(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  tm = __builtin_amdgcn_readfirstlane(tm);
  tn = __builtin_amdgcn_readfirstlane(tn);
  const int m0 = tm * kBandBM, n0 = tn * BN;
  const int rows_m = min(kBandBM, a.M - m0), rows_n = min(BN, a.N - n0);
  const uint32_t bytes_q = (uint32_t)(rows_m * a.ldq), bytes_w = (uint32_t)(rows_n * a.ldw);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + (int64_t)m0 * a.ldq, bytes_q);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + (int64_t)n0 * a.ldw, bytes_w);
  const bool lowrank = a.r > 0;

  // The epilogue's factors (clamped indices; rows and columns past the matrix get zero below), issued first.
  const int pt = threadIdx.x;
  float p_val = 0.0f;
  if (pt < kBandBM) {
    p_val = a.sx[min(m0 + pt, a.M - 1)];
  } else if (pt < kBandBM + BN) {
    p_val = a.sw[min(n0 + pt - kBandBM, a.N - 1)];
  } else if (pt < kBandBM + 2 * BN) {
    const uint16_t* bsrc = a.bias ? a.bias : reinterpret_cast<const uint16_t*>(a.sw);
    p_val = __uint_as_float((uint32_t)bsrc[min(n0 + pt - kBandBM - BN, a.N - 1)] << 16);
  }

  auto slot = [&](int s) { return smem + (s % kBandSlots) * kSlot; };
  const uint32_t bytes_u = lowrank ? (uint32_t)(rows_m * a.ldu * 2) : 0u;
  const uint32_t bytes_up = lowrank ? (uint32_t)(rows_n * a.ldup * 2) : 0u;
  const __amdgpu_buffer_rsrc_t ru = make_rsrc(lowrank ? a.u + (int64_t)m0 * a.ldu : a.u, bytes_u);
  const __amdgpu_buffer_rsrc_t rup = make_rsrc(lowrank ? a.up + (int64_t)n0 * a.ldup : a.up, bytes_up);
  // kLoads loads per wave into slot `dst`: 1 KiB block b = wave + 8 j of the stage (blocks 0-15 the 128 q rows,
  // the rest the w rows; indices past the last block repeat it, the same bytes to the same place), stage kt of
  // q and w, or with `lr` the low-rank operands (u rows in the q part, up rows in the w part). Every call issues the
  // same instructions.
  auto issue = [&](int kt, bool lr, unsigned char HF_LDS* dst) {
    const __amdgpu_buffer_rsrc_t ra = lr ? ru : rq, rb = lr ? rup : rw;
    const uint32_t oob_a = lr ? bytes_u : bytes_q, oob_b = lr ? bytes_up : bytes_w;
    const int64_t ld_a = lr ? a.ldu * 2 : a.ldq, ld_b = lr ? a.ldup * 2 : a.ldw;
    const int col0 = lr ? 0 : kt * 128, limit = lr ? 2 * a.r : a.K;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int b = min(wave + 8 * j, kBlocks - 1);
      const bool isb = b >= 16;
      const int blk = isb ? b - 16 : b;
      const int row = 8 * blk + (lane >> 3);
      const uint32_t chunk = (uint32_t)(((lane & 7) ^ mid_swz(row)) << 4);
      const int rows = isb ? rows_n : rows_m;
      const uint32_t col = (uint32_t)col0 + chunk;
      const uint32_t voff = ((row < rows) & (col < (uint32_t)limit)) ? (uint32_t)(row * (isb ? ld_b : ld_a)) + col
                                                                       : (isb ? oob_b : oob_a);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isb ? rb : ra, (void HF_LDS*)(dst + (isb ? kAStage : 0) + blk * 1024),
                                               16, voff, 0, 0, 0);
    }
  };

  const int nk = (a.K + 127) / 128;
  // Stages 0-3 (zero-fill past K); the first slot past the last stage takes the low-rank operands.
#pragma unroll
  for (int t = 0; t < kBandSlots; ++t) issue(t, lowrank && t == nk, slot(t));
  // Stage 0 and the factors (issued before it) have landed once stages 1-3 remain.
  static_assert(kLoads == 4 || kLoads == 5, "wait counts below");
  if constexpr (kLoads == 4) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(15)" ::: "memory");
  if (pt < kBandBM) {
    params[pt] = (m0 + pt < a.M) ? p_val : 0.0f;
  } else if (pt < kBandBM + BN) {
    params[pt] = (n0 + pt - kBandBM < a.N) ? p_val : 0.0f;
  } else if (pt < kBandBM + 2 * BN) {
    params[pt] = (n0 + pt - kBandBM - BN < a.N) ? p_val : 0.0f;
  }
  __syncthreads();

  // Fragment offsets of this wave's two K steps (2 kh and 2 kh + 1): lane half h reads chunk 2 ks + h of row sub.
  const int ca0 = sub * 128 + (((4 * kh + half) ^ mid_swz(sub)) << 4);
  const int ca1 = sub * 128 + (((4 * kh + 2 + half) ^ mid_swz(sub)) << 4);
  struct BandFrags {
    v4i a;
    v4i b[NB];
  };
  BandFrags f0, f1;
  auto read = [&](BandFrags& f, const unsigned char HF_LDS* st, int ca) {
    f.a = *(const v4i HF_LDS*)(st + wm * 32 * 128 + ca);
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) f.b[ib] = *(const v4i HF_LDS*)(st + kAStage + ib * 32 * 128 + ca);
  };
  v16i acc[NB];
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) acc[ib] = (v16i){0};
  // One K step: the next fragments' reads first, interleaved with the MFMAs, then (at a boundary) the ring refill
  // after the last MFMA.
  auto kstep = [&](const BandFrags& f, auto&& reads, auto&& loads) {
    reads();
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) acc[ib] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[ib], f.a, acc[ib], 0, 0, 0);
    loads();
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
#pragma unroll
    for (int i = 1; i < NB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x020, kLoads, 0);  // VMEM (ring refill)
    __builtin_amdgcn_sched_barrier(0);
  };
  auto nothing = [] {};

  read(f0, slot(0), ca0);
  for (int s = 0; s < nk; ++s) {
    kstep(f0, [&] { read(f1, slot(s), ca1); }, nothing);
    // Boundary: stage s + 1 has landed once stages s + 2 and s + 3 remain in flight; the barrier makes it so for
    // every wave and frees slot s, which receives stage s + 4 (or, when that is the stage count, the low-rank
    // operands). After the last stage the fragments read here are unused.
    if constexpr (kLoads == 4) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(10) lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    const bool lr_now = lowrank && s + kBandSlots == nk;
    unsigned char HF_LDS* refill = slot(s);
    kstep(f1, [&] { read(f0, slot(s + 1), ca0); }, [&] { issue(s + kBandSlots, lr_now, refill); });
  }
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
  __syncthreads();

  // --------------------------------------------------------------------------------------------------- epilogue
  // The K halves: wave (wm, kh) hands its partner (wm, 1 - kh) the sums of the partner's column blocks through 4 KiB
  // exchange blocks in the three slots besides the low-rank one, and adds the partner's sums of its own blocks.
  const int lr_slot = nk % kBandSlots;
  auto xblk = [&](int j) {
    return smem + ((lr_slot + 1 + j / kXPerSlot) % kBandSlots) * kSlot + (j % kXPerSlot) * 4096;
  };
  auto mine = [&](int ib) { return (ib < kH) == (kh == 0); };
  const int partner = wave ^ 4;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    if (!mine(ib)) {
      unsigned char HF_LDS* dst = xblk(wave * kH + (kh == 0 ? ib - kH : ib));
#pragma unroll
      for (int g = 0; g < 4; ++g)
        *(v4i HF_LDS*)(dst + (g * 64 + lane) * 16) =
            (v4i){acc[ib][4 * g], acc[ib][4 * g + 1], acc[ib][4 * g + 2], acc[ib][4 * g + 3]};
    }
  }
  __syncthreads();
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    if (mine(ib)) {
      const unsigned char HF_LDS* src = xblk(partner * kH + (kh == 0 ? ib : ib - kH));
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const v4i o = *(const v4i HF_LDS*)(src + (g * 64 + lane) * 16);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[ib][4 * g + e] += o[e];
      }
    }
  }

  // Output layout of a 32x32 block: lane holds row m = lane % 32 and, in register v, column
  // n = 8 (v / 4) + 4 (lane / 32) + v % 4.
  const unsigned char HF_LDS* u_lds = slot(lr_slot);
  const unsigned char HF_LDS* up_lds = slot(lr_slot) + kAStage;
  const float sxv = params[wm * 32 + sub];
  const bool full = rows_m == kBandBM && rows_n == BN && a.out_vec16;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    if (!mine(ib)) continue;
    v16f c;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int nl = ib * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
      c[v] = ((float)acc[ib][v] * sxv) * params[kBandBM + nl];
    }
    if (lowrank) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const int chunk = 2 * kk + half;
        const int nl = ib * 32 + sub, ml = wm * 32 + sub;
        const v8bf pf = *(const v8bf HF_LDS*)(up_lds + nl * 128 + ((chunk ^ mid_swz(nl)) << 4));
        const v8bf uf = *(const v8bf HF_LDS*)(u_lds + ml * 128 + ((chunk ^ mid_swz(ml)) << 4));
        c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c, 0, 0, 0);
      }
    }
    if (a.bias) {
#pragma unroll
      for (int v = 0; v < 16; ++v) c[v] = c[v] + params[kBandBM + BN + ib * 32 + 8 * (v >> 2) + 4 * half + (v & 3)];
    }
    // bf16 and the activation; after one exchange between the lane halves lane (sub, h) holds columns
    // 16 h .. 16 h + 15 of row sub of the block: chunk 2 h in w4[0], w4[2] and chunk 2 h + 1 in w4[1], w4[3].
    uint32_t w4[4][2];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      w4[gq][0] = activate_bf16x2<ACT>(pack_bf16x2(c[4 * gq], c[4 * gq + 1]));
      w4[gq][1] = activate_bf16x2<ACT>(pack_bf16x2(c[4 * gq + 2], c[4 * gq + 3]));
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
    // Stage the block (32 rows of 64 bytes) in the exchange block this wave read (no other wave touches it again),
    // then store 16 rows x 64 bytes per instruction.
    unsigned char HF_LDS* stage = xblk(partner * kH + (kh == 0 ? ib : ib - kH));
    *(v4i HF_LDS*)(stage + sub * 64 + (swizzle64(sub, 2 * half) << 4)) =
        (v4i){(int)w4[0][0], (int)w4[0][1], (int)w4[2][0], (int)w4[2][1]};
    *(v4i HF_LDS*)(stage + sub * 64 + (swizzle64(sub, 2 * half + 1) << 4)) =
        (v4i){(int)w4[1][0], (int)w4[1][1], (int)w4[3][0], (int)w4[3][1]};
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int row = 16 * i + (lane >> 2), ch = lane & 3;
      const v4i val = *(const v4i HF_LDS*)(stage + row * 64 + (swizzle64(row, ch) << 4));
      const int m = m0 + wm * 32 + row;
      const int n = n0 + ib * 32 + 8 * ch;
      uint16_t* dst = a.y + (int64_t)m * a.ldy + n;
      if (full) {
        *reinterpret_cast<v4i*>(dst) = val;
      } else if (m < a.M) {
        if (a.out_vec16 && n + 8 <= a.N) {
          *reinterpret_cast<v4i*>(dst) = val;
        } else {
          for (int e = 0; e < 8; ++e)
            if (n + e < a.N) dst[e] = (uint16_t)((uint32_t)val[e >> 1] >> (16 * (e & 1)));
        }
      }
    }
  }
}

#define HF_BAND_INSTANTIATE(NB)                                                                                       \
  template __global__ void band_gemm_kernel<NB, kActNone>(MidArgs);                                                 \
  template __global__ void band_gemm_kernel<NB, kActGeluTanh>(MidArgs);
HF_BAND_INSTANTIATE(3) HF_BAND_INSTANTIATE(4) HF_BAND_INSTANTIATE(5)
#undef HF_BAND_INSTANTIATE

}  // namespace hf
