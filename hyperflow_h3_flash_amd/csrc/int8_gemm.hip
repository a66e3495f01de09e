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
// Tiling: 256 (m) x 256 (n) output tile per workgroup (one per CU), K in stages of 64 bytes, 8 waves (two per SIMD,
// so one wave's barrier wait and load issue run under the other's MFMAs) in a 2 (m) x 4 (n) grid, each wave a
// 128 x 64 sub-tile of 4 x 2 v_mfma_i32_32x32x32_i8 blocks (128 accumulator registers). The
// MFMA's first operand is the weight (its rows are the output columns n) and the second the activation, so each
// lane ends with four consecutive n of one row m and reads one activation scale per block.
//
// Operands go global -> LDS with buffer_load ... lds (16 bytes per lane, no VGPR round trip) into a 4-stage ring
// (128 KiB); the waits are partial (vmcnt counts the loads still allowed in flight) and the barrier carries no
// memory fence, so three stages stay in flight while one is consumed. MFMA operands are double-buffered in
// registers: the LDS reads of one 32-byte K step overlap the MFMAs of the previous one. Out-of-range rows and K
// beyond the end read as zero through the buffer descriptor's range check. A rank <= 64 low-rank branch rides the
// last two refills into the ring, so the epilogue reads its operands from LDS. The epilogue goes through LDS so the
// output is written as whole 64-byte row segments, 16 bytes per lane.
#include "common.h"

namespace hf {

constexpr int GBM = 256;                          // activation rows (m) per workgroup tile
constexpr int GBN = 256;                          // weight rows (n) per workgroup tile
constexpr int GBK = 64;                           // K bytes per pipeline stage
constexpr int kStages = 4;                        // LDS ring depth
constexpr int kAStage = GBM * GBK;                // 16 KiB
constexpr int kBStage = GBN * GBK;                // 16 KiB
constexpr int kStageBytes = kAStage + kBStage;    // 32 KiB
constexpr int kRingBytes = kStages * kStageBytes; // 128 KiB; the epilogue reuses it as a 256 x 256 bf16 tile
constexpr int kParamBytes = 3 * 256 * 4;          // the tile's sx, wscale and bias (fp32), staged at kernel start
constexpr int kGemmLds = kRingBytes + kParamBytes;
constexpr int kWaves = 8;                         // 2 per SIMD: one wave's barrier and load issue hide under the other's MFMAs
constexpr int kThreads = 64 * kWaves;

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
  int out_vec16;         // bf16 rows may be written 16 bytes at a time (16-byte aligned base and ldo % 8 == 0)
};

// Workgroup id -> (tile_m, tile_n). The dispatcher deals workgroup ids round robin to the 8 XCDs (XCD = id % 8,
// in id order within an XCD), and each XCD has its own L2. The map gives XCD x the x-th contiguous share of a
// grouped order in which 8 tile rows are walked column by column, so the 32 tiles an XCD runs at once form an 8 x 4
// block: 12 operand panels for 32 tiles instead of ~36 for the row-major order. Measured on the 32768 x 15360 x 5120
// GEMM: L2->fabric fetch 3.7 GiB instead of 11.3 GiB per launch, same duration.
constexpr int kGroupRows = 8;

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n, per = total / 8, rem = total % 8, xcd = bid % 8, local = bid / 8;
  const int logical = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int group = kGroupRows * tiles_n, first = (logical / group) * kGroupRows;
  const int rows = min(tiles_m - first, kGroupRows), within = logical % group;
  tm = first + within % rows;
  tn = within / rows;
}

// LDS rows are 64 bytes (four 16-byte chunks of K); chunk c of row r lives at c ^ ((r >> 1) & 3), which spreads the
// 32 rows of one fragment read over all banks (measured conflict-free on gfx950 for ds_read_b128).
__device__ __forceinline__ int swizzle(int r, int c) { return c ^ ((r >> 1) & 3); }

// Per-lane byte offsets of one wave's stage loads, computed once per tile. Load i of a wave fills LDS block
// blk = first_blk + i (16 rows x 64 bytes): lane l fills row 16*blk + l/4, physical chunk l%4, from the logical chunk
// the swizzle stores there. Rows past the tile's valid rows get the descriptor size as base offset, so adding any
// K offset keeps them out of range (they read as zero).
template <int COUNT>
struct StageOffsets {
  uint32_t off[COUNT];
  __device__ __forceinline__ void init(uint32_t oob, int64_t ld, int rows_valid, int first_blk, int lane) {
#pragma unroll
    for (int i = 0; i < COUNT; ++i) {
      const int r = (first_blk + i) * 16 + (lane >> 2);
      const int c = swizzle(r, lane & 3);
      off[i] = r < rows_valid ? (uint32_t)(r * ld + c * 16) : oob;
    }
  }
};

// Issue one wave's loads of a stage at K offset k0 into `dst` (LDS, wave-uniform). Chunks at or past K (only in a
// partial last stage) read as zero; so does every load of a stage past the end (k0 >= K).
template <int COUNT>
__device__ __forceinline__ void load_stage(__amdgpu_buffer_rsrc_t rsrc, const StageOffsets<COUNT>& so, uint32_t oob,
                                           int k0, int K, unsigned char HF_LDS* dst, int first_blk, int lane) {
  const bool partial = k0 + GBK > K;
#pragma unroll
  for (int i = 0; i < COUNT; ++i) {
    uint32_t voff = so.off[i] + (uint32_t)k0;
    if (partial) {
      const int kb = k0 + swizzle((first_blk + i) * 16 + (lane >> 2), lane & 3) * 16;
      if (kb >= K) voff = oob;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void HF_LDS*)(dst + (first_blk + i) * 1024), 16, voff, 0, 0, 0);
  }
}

// The low-rank operands of a tile (u rows m or up rows n, rank r <= 64, as 128-byte rows of 8 chunks of 8 bf16,
// chunk c of row i stored at c ^ (i & 7)) are loaded into a free ring slot: 256 rows x 128 bytes = 32 loads of
// 1 KiB, 4 per wave. Rows past the tile's valid rows and chunks past r read as zero.
__device__ __forceinline__ void load_lowrank_rows(__amdgpu_buffer_rsrc_t rsrc, uint32_t oob, int64_t ld_bytes,
                                                  int rows_valid, int r, unsigned char HF_LDS* dst, int wave,
                                                  int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = wave * 4 + i;
    const int row = blk * 8 + (lane >> 3);
    const int c = (lane & 7) ^ (row & 7);
    const uint32_t voff = (row < rows_valid && c * 8 < r) ? (uint32_t)(row * ld_bytes + c * 16) : oob;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void HF_LDS*)(dst + blk * 1024), 16, voff, 0, 0, 0);
  }
}

struct Frags {
  v4i a[4];  // activation rows: 4 blocks of 32 (the wave's 128 m)
  v4i b[2];  // weight rows: 2 blocks of 32 (the wave's 64 n)
};

__device__ __forceinline__ void read_frags(Frags& f, const unsigned char HF_LDS* stage, int wm, int wn, int ks,
                                           int sub, int half) {
  const int chunk = swizzle(sub, 2 * ks + half) * 16;  // (row >> 1) & 3 == (sub >> 1) & 3: blocks start at 32k
  const unsigned char HF_LDS* As = stage;
  const unsigned char HF_LDS* Bs = stage + kAStage;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) f.a[jb] = *(const v4i HF_LDS*)(As + (wm * 128 + jb * 32 + sub) * GBK + chunk);
#pragma unroll
  for (int ib = 0; ib < 2; ++ib) f.b[ib] = *(const v4i HF_LDS*)(Bs + (wn * 64 + ib * 32 + sub) * GBK + chunk);
}

__device__ __forceinline__ void mma(v16i (&acc)[2][4], const Frags& f) {
#pragma unroll
  for (int ib = 0; ib < 2; ++ib)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
      acc[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[ib], f.a[jb], acc[ib][jb], 0, 0, 0);
}

#define HF_BARRIER() asm volatile("s_barrier" ::: "memory")

template <bool I32OUT>
__global__ __launch_bounds__(kThreads, 1) void int8_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps LDS addresses scalar
  const int wm = wave & 1, wn = wave >> 1;  // 2 (m) x 4 (n) waves of 128 x 64
  const int sub = lane & 31, half = lane >> 5;
  int tm, tn;
  tile_of(blockIdx.x, a.tiles_m, a.tiles_n, tm, tn);
  const int m0 = tm * GBM, n0 = tn * GBN;
  const int rows_m = min(GBM, a.M - m0), rows_n = min(GBN, a.N - n0);

  const uint32_t bytes_q = (uint32_t)(rows_m * a.ldq), bytes_w = (uint32_t)(rows_n * a.ldw);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.q + (int64_t)m0 * a.ldq, bytes_q);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w + (int64_t)n0 * a.ldw, bytes_w);

  StageOffsets<2> offq, offw;
  offq.init(bytes_q, a.ldq, rows_m, wave * 2, lane);
  offw.init(bytes_w, a.ldw, rows_n, wave * 2, lane);
  // Stage kt into slot kt % 4; a stage past the end (kt >= nk) loads zeros, which keeps the loop branch-free.
  auto issue_stage = [&](int kt) {
    unsigned char HF_LDS* st = smem + (kt % kStages) * kStageBytes;
    load_stage<2>(rq, offq, bytes_q, kt * GBK, a.K, st, wave * 2, lane);
    load_stage<2>(rw, offw, bytes_w, kt * GBK, a.K, st + kAStage, wave * 2, lane);
  };

  // The epilogue's per-row and per-column factors, loaded into registers now and parked in LDS beside the ring when
  // the epilogue starts, so no epilogue instruction waits on global memory. Threads 0..255 take row m0 + t and
  // column n0 + t (sx, wscale); threads 256..511 take the bias of column n0 + t - 256.
  float HF_LDS* params = (float HF_LDS*)(smem + kRingBytes);
  float p_val = 0.0f;
  uint32_t p_bias = 0;
  const int pt = threadIdx.x & 255;
  if (!I32OUT) {
    // Branch-free (clamped indices, a stand-in array when there is no bias) so no wait lands here; rows and columns
    // past the edge are masked when the values are parked.
    if (threadIdx.x < 256) {
      p_val = a.sx[min(m0 + pt, a.M - 1)];
      p_bias = __float_as_uint(a.sw[min(n0 + pt, a.N - 1)]);
    } else {
      const uint16_t* bsrc = a.bias ? a.bias : reinterpret_cast<const uint16_t*>(a.sw);
      p_bias = bsrc[min(n0 + pt, a.N - 1)];
    }
  }

  v16i acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = (v16i){0};

  const int nk = (a.K + GBK - 1) / GBK;
  // Prologue: stages 0..3 in flight (4 loads per wave per stage), wait for stage 0.
  issue_stage(0);
  issue_stage(1);
  issue_stage(2);
  issue_stage(3);
  asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
  HF_BARRIER();
  Frags f0, f1;
  read_frags(f0, smem, wm, wn, 0, sub, half);

  // With a rank <= 64 low-rank branch, the u tile [256 m][r] and the up tile [256 n][r] take the places of the
  // stage loads the last iterations would not need; they land in the ring slots nk % 4 and (nk + 1) % 4.
  const bool lr_lds = !I32OUT && a.r > 0 && a.r <= 64 && nk >= kStages;
  __amdgpu_buffer_rsrc_t ru = rq, rup = rw;
  uint32_t bytes_u = 0, bytes_up = 0;
  if (lr_lds) {
    bytes_u = (uint32_t)(rows_m * a.ldu * 2);
    bytes_up = (uint32_t)(rows_n * a.ldup * 2);
    ru = make_rsrc(a.u + (int64_t)m0 * a.ldu, bytes_u);
    rup = make_rsrc(a.up + (int64_t)n0 * a.ldup, bytes_up);
  }

  // Stage kt lives in slot kt % 4. Per stage: read the second K half while multiplying the first; wait for this
  // wave's loads of stage kt+1 (two more stages stay in flight) and for the reads of slot kt % 4; barrier; read
  // stage kt+1's first half, refill slot kt % 4 and multiply the second half, with the LDS reads and loads spread
  // between the MFMAs. The wait relies on every iteration issuing the same 4 loads per wave.
  auto stage_body = [&](int kt, int refill) {
    const unsigned char HF_LDS* st = smem + (kt % kStages) * kStageBytes;
    read_frags(f1, st, wm, wn, 1, sub, half);
    mma(acc, f0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
    __builtin_amdgcn_sched_barrier(0);  // every MFMA of the first half issues before the wait and barrier
    asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    HF_BARRIER();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(f0, smem + ((kt + 1) % kStages) * kStageBytes, wm, wn, 0, sub, half);
    unsigned char HF_LDS* slot = smem + (kt % kStages) * kStageBytes;
    if (refill == 0) {
      load_stage<2>(rq, offq, bytes_q, (kt + 4) * GBK, a.K, slot, wave * 2, lane);
      load_stage<2>(rw, offw, bytes_w, (kt + 4) * GBK, a.K, slot + kAStage, wave * 2, lane);
    } else if (refill == 1) {
      load_lowrank_rows(ru, bytes_u, a.ldu * 2, rows_m, a.r, slot, wave, lane);
    } else if (refill == 2) {
      load_lowrank_rows(rup, bytes_up, a.ldup * 2, rows_n, a.r, slot, wave, lane);
    }
    mma(acc, f1);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);  // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);  // MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);  // VMEM (stage load)
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 1);
    __builtin_amdgcn_sched_group_barrier(0x008, 2, 1);
    __builtin_amdgcn_sched_barrier(0);
  };
  const int steady = nk - kStages;  // iterations whose refill is a real stage
  int kt = 0;
  for (; kt < steady; ++kt) stage_body(kt, 0);
  for (; kt < nk; ++kt) {
    // Stages past the end load zeros, so every iteration issues exactly 4 loads per wave and vmcnt(8) always
    // means "stage kt + 1 has landed" (with fewer loads behind it the wait would let it through early).
    int refill = 0;
    if (lr_lds && kt == steady) refill = 1;
    if (lr_lds && kt == steady + 1) refill = 2;
    stage_body(kt, refill);
  }
  // Zero-fill loads past the end may still be landing in the ring; the epilogue reuses it.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Output layout of a 32x32 block: lane holds column j = lane % 32 (the row m here) and, in register v, row
  // i = 8*(v/4) + 4*(lane/32) + v%4 (the column n here): four consecutive n per group of four registers.
  if constexpr (I32OUT) {
    int32_t* out = static_cast<int32_t*>(a.out);
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      const int m = m0 + wm * 128 + jb * 32 + sub;
      if (m >= a.M) continue;
#pragma unroll
      for (int ib = 0; ib < 2; ++ib)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = n0 + wn * 64 + ib * 32 + 8 * g + 4 * half;
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
    // Dequantize one 32-wide block of output columns at a time (add the low-rank product on bf16 MFMA and the
    // bias), round to bf16 and park it in LDS (this wave's 128 x 32 block: rows of 64 bytes, 16-byte chunk c of row
    // i at c ^ ((i >> 1) & 3)), then write 64-byte row segments, 16 bytes per lane, 16 rows per instruction. The
    // staging uses the two ring slots the low-rank tiles do not: waves 0-3 slot (nk + 2) % 4, waves 4-7 slot
    // (nk + 3) % 4, 8 KiB each.
    if (threadIdx.x < 256) {
      params[pt] = (m0 + pt < a.M) ? p_val : 0.0f;
      params[256 + pt] = (n0 + pt < a.N) ? __uint_as_float(p_bias) : 0.0f;
    } else {
      params[512 + pt] = (n0 + pt < a.N && a.bias) ? __uint_as_float(p_bias << 16) : 0.0f;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    HF_BARRIER();
    float sxv[4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) sxv[jb] = params[wm * 128 + jb * 32 + sub];
    const unsigned char HF_LDS* u_lds = smem + (nk % kStages) * kStageBytes;
    const unsigned char HF_LDS* up_lds = smem + ((nk + 1) % kStages) * kStageBytes;
    unsigned char HF_LDS* tile =
        smem + ((nk + 2 + (wave >> 2)) % kStages) * kStageBytes + (wave & 3) * (128 * 64);
    const bool has_bias = a.bias != nullptr;
    uint16_t* out = static_cast<uint16_t*>(a.out);
#pragma unroll
    for (int ib = 0; ib < 2; ++ib) {
      const int nb = n0 + wn * 64 + ib * 32;
      float ws[16], bv[16];
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int nl = wn * 64 + ib * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
        ws[v] = params[256 + nl];
        bv[v] = params[512 + nl];
      }
      v16f c[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float t = (float)acc[ib][jb][v] * sxv[jb];
          c[jb][v] = t * ws[v];
        }
      if (lr_lds) {
        // Low-rank term from the LDS tiles: first operand up[n, :], second u[m, :], 16 ranks per MFMA.
        const int nl = wn * 64 + ib * 32 + sub;
        for (int kk = 0; kk < a.r; kk += 16) {
          const int chunk = kk / 8 + half;
          const v8bf pf = *(const v8bf HF_LDS*)(up_lds + nl * 128 + ((chunk ^ (nl & 7)) * 16));
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) {
            const int ml = wm * 128 + jb * 32 + sub;
            const v8bf uf = *(const v8bf HF_LDS*)(u_lds + ml * 128 + ((chunk ^ (ml & 7)) * 16));
            c[jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c[jb], 0, 0, 0);
          }
        }
      } else if (a.r > 0) {
        // Ranks above 64 (or a K too short to carry them in the ring): the same product from global memory.
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
        const int rr = jb * 32 + sub;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = c[jb][4 * g + e];
            if (has_bias) v[e] = v[e] + bv[4 * g + e];
          }
          const int chunk = g ^ ((rr >> 1) & 3);
          typedef unsigned int v2u __attribute__((ext_vector_type(2)));
          *(v2u HF_LDS*)(tile + rr * 64 + chunk * 16 + 8 * half) = (v2u){pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      }
      wave_lds_sync();
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int rr = i * 16 + (lane >> 2);
        const int p = lane & 3;
        const int cc = p ^ ((rr >> 1) & 3);
        const v4i v = *(const v4i HF_LDS*)(tile + rr * 64 + p * 16);
        const int m = m0 + wm * 128 + rr;
        const int n = nb + cc * 8;
        if (m < a.M) {
          uint16_t* dst = out + (int64_t)m * a.ldo + n;
          if (a.out_vec16 && n + 7 < a.N) {
            *reinterpret_cast<v4i*>(dst) = v;
          } else {
            const uint32_t wds[4] = {(uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]};
            for (int e = 0; e < 8; ++e)
              if (n + e < a.N) dst[e] = (uint16_t)(wds[e >> 1] >> (16 * (e & 1)));
          }
        }
      }
      wave_lds_sync();  // the block is overwritten by the next one
    }
  }
}

template __global__ void int8_gemm_kernel<false>(GemmArgs);
template __global__ void int8_gemm_kernel<true>(GemmArgs);

}  // namespace hf
