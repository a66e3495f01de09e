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
#include <type_traits>

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

// LDS rows are 64 bytes (four 16-byte chunks of K), swizzled with swizzle64.
__device__ __forceinline__ int swizzle(int r, int c) { return swizzle64(r, c); }

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

// Issue one wave's loads of a stage at K offset k0 into `dst` (LDS, wave-uniform). A lane's 16-byte chunk sits at
// the same K byte of the stage for every load (the swizzle of its row, 16*blk + lane/4, only sees row bits 1-3, i.e.
// lane bits 3-5). Chunks at or past K read as zero (the offset moves past the descriptor), branch-free; so does every
// load of a stage past the end (k0 >= K).
template <int COUNT>
__device__ __forceinline__ void load_stage(__amdgpu_buffer_rsrc_t rsrc, const StageOffsets<COUNT>& so, uint32_t oob,
                                           int k0, int K, unsigned char HF_LDS* dst, int first_blk, int lane) {
  const int kb = k0 + (swizzle(lane >> 2, lane & 3) << 4);
  const uint32_t kadd = kb < K ? (uint32_t)k0 : oob;
#pragma unroll
  for (int i = 0; i < COUNT; ++i) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (void HF_LDS*)(dst + (first_blk + i) * 1024), 16, so.off[i] + kadd,
                                             0, 0, 0);
  }
}

// The low-rank operands of a tile (u rows m or up rows n, rank r <= 64, as 128-byte rows of 8 chunks of 8 bf16,
// swizzled with swizzle128) are loaded into a free ring slot: 256 rows x 128 bytes = 32 loads of
// 1 KiB, 4 per wave. Rows past the tile's valid rows and chunks past r read as zero.
__device__ __forceinline__ void load_lowrank_rows(__amdgpu_buffer_rsrc_t rsrc, uint32_t oob, int64_t ld_bytes,
                                                  int rows_valid, int r, unsigned char HF_LDS* dst, int wave,
                                                  int lane) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int blk = wave * 4 + i;
    const int row = blk * 8 + (lane >> 3);
    const int c = swizzle128(row, lane & 7);
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
  const int chunk = swizzle(sub, 2 * ks + half) * 16;  // blocks start at multiples of 32 rows: f(row) == f(sub)
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

// s_waitcnt vmcnt(n) for the wave-uniform counts the persistent loop uses (an unlisted count waits for everything,
// which is always safe). The loop's accounting relies on vector memory operations completing in issue order (loads,
// LDS-DMA loads and stores share one in-order counter on gfx9).
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
    case 8: asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory"); break;
    case 10: asm volatile("s_waitcnt vmcnt(10) lgkmcnt(0)" ::: "memory"); break;
    case 12: asm volatile("s_waitcnt vmcnt(12) lgkmcnt(0)" ::: "memory"); break;
    case 26: asm volatile("s_waitcnt vmcnt(26) lgkmcnt(0)" ::: "memory"); break;
    case 28: asm volatile("s_waitcnt vmcnt(28) lgkmcnt(0)" ::: "memory"); break;
    case 40: asm volatile("s_waitcnt vmcnt(40) lgkmcnt(0)" ::: "memory"); break;
    case 44: asm volatile("s_waitcnt vmcnt(44) lgkmcnt(0)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); break;
  }
}

// One output tile's operand source: the q rows m0.. and w rows n0.. as buffer descriptors (rows past the matrix and
// every row of a tile past the last one read as zero) and the per-lane stage offsets.
struct TileSrc {
  int m0, n0, rows_m, rows_n;
  uint32_t bytes_q, bytes_w;
  __amdgpu_buffer_rsrc_t rq, rw;
  StageOffsets<2> offq, offw;
};

__device__ __forceinline__ void tile_src(const GemmArgs& a, int id, int wave, int lane, TileSrc& t) {
  int tm = 0, tn = 0;
  const bool live = id < a.tiles_m * a.tiles_n;
  if (live) tile_of(id, a.tiles_m, a.tiles_n, tm, tn);
  t.m0 = tm * GBM;
  t.n0 = tn * GBN;
  t.rows_m = live ? min(GBM, a.M - t.m0) : 0;
  t.rows_n = live ? min(GBN, a.N - t.n0) : 0;
  t.bytes_q = (uint32_t)(t.rows_m * a.ldq);
  t.bytes_w = (uint32_t)(t.rows_n * a.ldw);
  t.rq = make_rsrc(a.q + (int64_t)t.m0 * a.ldq, t.bytes_q);
  t.rw = make_rsrc(a.w + (int64_t)t.n0 * a.ldw, t.bytes_w);
  t.offq.init(t.bytes_q, a.ldq, t.rows_m, wave * 2, lane);
  t.offw.init(t.bytes_w, a.ldw, t.rows_n, wave * 2, lane);
}

// Stage kt of tile t into ring slot `slot`: 4 loads per wave (2 of q, 2 of w).
__device__ __forceinline__ void load_tile_stage(const TileSrc& t, const GemmArgs& a, int kt,
                                                unsigned char HF_LDS* slot, int wave, int lane) {
  load_stage<2>(t.rq, t.offq, t.bytes_q, kt * GBK, a.K, slot, wave * 2, lane);
  load_stage<2>(t.rw, t.offw, t.bytes_w, kt * GBK, a.K, slot + kAStage, wave * 2, lane);
}

// Output modes: int32 accumulators; bf16 with the dequantization (and, for r > 64, the low-rank term from global
// memory) and bias; bf16 with a rank <= 64 low-rank term whose operands ride the ring.
constexpr int kOutI32 = 0, kOutBf16 = 1, kOutBf16Lr = 2;

// Persistent kernel: one workgroup per CU walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... The ring of 4 stages
// runs continuously across tiles: the last 4 iterations of a tile refill their slots with the next tile's first
// stages (after the tile's u and up tiles in low-rank mode), so a tile starts with its operands in flight and the
// epilogue's output stores drain while the next tile computes. Every ring step issues exactly 4 loads per wave
// (past the last tile they read zeros), which keeps every wait a fixed vmcnt.
template <int OUT>
__global__ __launch_bounds__(kThreads, 1) void int8_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps LDS addresses scalar
  const int wm = wave & 1, wn = wave >> 1;  // 2 (m) x 4 (n) waves of 128 x 64
  const int sub = lane & 31, half = lane >> 5;
  constexpr bool kLr = OUT == kOutBf16Lr;
  constexpr int kParamLoads = OUT == kOutI32 ? 0 : 2;  // per thread and tile
  constexpr int kFastStores = OUT == kOutI32 ? 32 : 16;  // per wave and tile, full tiles only
  float HF_LDS* params = (float HF_LDS*)(smem + kRingBytes);
  const int pt = threadIdx.x & 255;
  auto slot_at = [&](int step) { return smem + (step & (kStages - 1)) * kStageBytes; };

  // K steps per tile, at least 7 so the three first steps, the steady loop and the four refill steps never overlap
  // (stages past K read zeros and add nothing).
  const int nk = max((a.K + GBK - 1) / GBK, kStages + 3);
  const int total = a.tiles_m * a.tiles_n;
  int id = blockIdx.x;
  TileSrc cur;
  tile_src(a, id, wave, lane, cur);
#pragma unroll
  for (int j = 0; j < kStages; ++j) load_tile_stage(cur, a, j, slot_at(j), wave, lane);

  int g = 0;             // ring step of the current tile's stage 0
  bool stores_behind = false;  // the previous tile's epilogue left kFastStores stores behind its stage 3
  Frags f0, f1;
  v16i acc[2][4];

  // One tile; SPILL counts the stores the previous epilogue issued after this tile's stage 3 (they precede the
  // parameter loads), so every wait count below is a constant.
  auto tile = [&](auto spill_tag) -> bool {
    constexpr int spill = decltype(spill_tag)::value;
    const int next_id = id + gridDim.x;
    TileSrc nxt;
    tile_src(a, next_id, wave, lane, nxt);

    // Stage 0 landed (stages 1..3 and the previous tile's stores may still be in flight).
    wait_vm(12 + spill);
    HF_BARRIER();
    read_frags(f0, slot_at(g), wm, wn, 0, sub, half);

    // The epilogue's per-row and per-column factors, loaded now and parked in LDS when the epilogue starts:
    // threads 0..255 take sx of row m0 + t and wscale of column n0 + t, threads 256..511 the bias of column
    // n0 + t - 256 (and a second, unused load so every wave issues the same count). Clamped, branch-free.
    float p_val = 0.0f;
    uint32_t p_bias = 0;
    if (OUT != kOutI32) {
      const int mr = min(cur.m0 + pt, a.M - 1), nc = min(cur.n0 + pt, a.N - 1);
      const uint16_t* bsrc = a.bias ? a.bias : reinterpret_cast<const uint16_t*>(a.sw);
      p_val = a.sx[mr];
      p_bias = threadIdx.x < 256 ? __float_as_uint(a.sw[nc]) : (uint32_t)bsrc[nc];
    }
    constexpr int early = 8 + spill + kParamLoads;  // wait count while those operations sit behind the stage

#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (v16i){0};

    // Step kt: read the second K half of slot kt while multiplying the first; wait until stage kt + 1 landed (for
    // this wave) and the slot's reads returned; barrier; read stage kt + 1's first half, refill slot kt and multiply
    // the second half, with LDS reads and loads spread between the MFMAs.
    auto step = [&](int kt, int vm, bool read_next, auto&& refill) {
      read_frags(f1, slot_at(g + kt), wm, wn, 1, sub, half);
      mma(acc, f0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 5, 0);
      __builtin_amdgcn_sched_barrier(0);  // every MFMA of the first half issues before the wait and barrier
      wait_vm(vm);
      HF_BARRIER();
      __builtin_amdgcn_sched_barrier(0);
      if (read_next) read_frags(f0, slot_at(g + kt + 1), wm, wn, 0, sub, half);
      refill(slot_at(g + kt));
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
    auto own_stage = [&](int kt) {
      return [&, kt](unsigned char HF_LDS* s) { load_tile_stage(cur, a, kt, s, wave, lane); };
    };
    auto next_stage = [&](int kt) {
      return [&, kt](unsigned char HF_LDS* s) { load_tile_stage(nxt, a, kt, s, wave, lane); };
    };

    // Steps 0..nk-5 refill with this tile's stages 4..nk-1; the first three still have the stores and parameter
    // loads behind the stage they wait for.
    step(0, early, true, own_stage(kStages));
    step(1, early, true, own_stage(kStages + 1));
    step(2, early, true, own_stage(kStages + 2));
    int kt = 3;
    for (; kt < nk - kStages; ++kt) step(kt, 8, true, own_stage(kt + kStages));
    // The last four steps refill with the tile's low-rank operands and the next tile's first stages.
    const __amdgpu_buffer_rsrc_t ru =
        make_rsrc(a.u + (int64_t)cur.m0 * a.ldu, kLr ? (uint32_t)(cur.rows_m * a.ldu * 2) : 0u);
    const __amdgpu_buffer_rsrc_t rup =
        make_rsrc(a.up + (int64_t)cur.n0 * a.ldup, kLr ? (uint32_t)(cur.rows_n * a.ldup * 2) : 0u);
    if constexpr (kLr) {
      step(kt, 8, true, [&](unsigned char HF_LDS* s) {
        load_lowrank_rows(ru, (uint32_t)(cur.rows_m * a.ldu * 2), a.ldu * 2, cur.rows_m, a.r, s, wave, lane);
      });
      step(kt + 1, 8, true, [&](unsigned char HF_LDS* s) {
        load_lowrank_rows(rup, (uint32_t)(cur.rows_n * a.ldup * 2), a.ldup * 2, cur.rows_n, a.r, s, wave, lane);
      });
      step(kt + 2, 8, true, next_stage(0));
      step(kt + 3, 8, false, next_stage(1));
    } else {
      step(kt, 8, true, next_stage(0));
      step(kt + 1, 8, true, next_stage(1));
      step(kt + 2, 8, true, next_stage(2));
      step(kt + 3, 8, false, next_stage(3));
    }

    // ------------------------------------------------------------------------------------------------ epilogue
    // Output layout of a 32x32 block: lane holds column j = lane % 32 (the row m here) and, in register v, row
    // i = 8*(v/4) + 4*(lane/32) + v%4 (the column n here): four consecutive n per group of four registers.
    const int m0 = cur.m0, n0 = cur.n0;
    bool full;
    if constexpr (OUT == kOutI32) {
      full = cur.rows_m == GBM && cur.rows_n == GBN && a.out_vec16;
      int32_t* out = static_cast<int32_t*>(a.out);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int m = m0 + wm * 128 + jb * 32 + sub;
#pragma unroll
        for (int ib = 0; ib < 2; ++ib)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int n = n0 + wn * 64 + ib * 32 + 8 * gq + 4 * half;
            int32_t* dst = out + (int64_t)m * a.ldo + n;
            const v16i& c = acc[ib][jb];
            if (full) {
              *reinterpret_cast<v4i*>(dst) = (v4i){c[4 * gq], c[4 * gq + 1], c[4 * gq + 2], c[4 * gq + 3]};
            } else if (m < a.M) {
              for (int e = 0; e < 4; ++e)
                if (n + e < a.N) dst[e] = c[4 * gq + e];
            }
          }
      }
    } else {
      full = cur.rows_m == GBM && cur.rows_n == GBN && a.out_vec16 && (kLr || a.r == 0);
      if (threadIdx.x < 256) {
        params[pt] = (m0 + pt < a.M) ? p_val : 0.0f;
        params[256 + pt] = (n0 + pt < a.N) ? __uint_as_float(p_bias) : 0.0f;
      } else {
        params[512 + pt] = (n0 + pt < a.N && a.bias) ? __uint_as_float(p_bias << 16) : 0.0f;
      }
      // Low-rank mode: the up tile (step g + nk + 1) has landed once only the next tile's stages 0 and 1 are
      // behind it. The barrier also publishes the parameters.
      if constexpr (kLr) {
        wait_vm(8);
      } else {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      }
      HF_BARRIER();
      float sxv[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) sxv[jb] = params[wm * 128 + jb * 32 + sub];
      const unsigned char HF_LDS* u_lds = slot_at(g + nk);
      const unsigned char HF_LDS* up_lds = slot_at(g + nk + 1);
      v16f c[2][4];
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int nl = wn * 64 + ib * 32 + 8 * (v >> 2) + 4 * half + (v & 3);
            c[ib][jb][v] = ((float)acc[ib][jb][v] * sxv[jb]) * params[256 + nl];
          }
        if constexpr (kLr) {
          // Low-rank term from the LDS tiles (rows of 128 bytes, swizzle128): first operand
          // up[n, :], second u[m, :], 16 ranks per MFMA, accumulated onto the dequantized values.
          const int nl = wn * 64 + ib * 32 + sub;
          for (int kk = 0; kk < a.r; kk += 16) {
            const int chunk = kk / 8 + half;
            const v8bf pf = *(const v8bf HF_LDS*)(up_lds + nl * 128 + swizzle128(nl, chunk) * 16);
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
              const int ml = wm * 128 + jb * 32 + sub;
              const v8bf uf = *(const v8bf HF_LDS*)(u_lds + ml * 128 + swizzle128(ml, chunk) * 16);
              c[ib][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c[ib][jb], 0, 0, 0);
            }
          }
        } else if (a.r > 0) {
          // Ranks above 64: the same product from global memory.
          const int nrow = min(n0 + wn * 64 + ib * 32 + sub, a.N - 1);
          for (int kk = 0; kk < a.r; kk += 16) {
            const int k = kk + 8 * half;
            const v8bf pf =
                (k < a.r) ? *reinterpret_cast<const v8bf*>(a.up + (int64_t)nrow * a.ldup + k) : (v8bf){0};
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
              const int mrow = min(m0 + wm * 128 + jb * 32 + sub, a.M - 1);
              const v8bf uf =
                  (k < a.r) ? *reinterpret_cast<const v8bf*>(a.u + (int64_t)mrow * a.ldu + k) : (v8bf){0};
              c[ib][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c[ib][jb], 0, 0, 0);
            }
          }
        }
      }
      if constexpr (kLr) {
        // Every wave is done with the u and up slots: refill them with the next tile's stages 2 and 3.
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        HF_BARRIER();
        load_tile_stage(nxt, a, 2, slot_at(g + nk), wave, lane);
        load_tile_stage(nxt, a, 3, slot_at(g + nk + 1), wave, lane);
      }
      // Bias, bf16, and the stores: after one exchange between the lane halves (v_permlane32_swap: lanes 32..63 of
      // the first operand <-> lanes 0..31 of the second), lane (sub, h) holds columns 16h..16h+15 of row sub of
      // the block, 32 contiguous bytes written as two 16-byte stores; the two halves cover the row's 64 bytes.
      uint16_t* out = static_cast<uint16_t*>(a.out);
      const bool has_bias = a.bias != nullptr;
#pragma unroll
      for (int ib = 0; ib < 2; ++ib) {
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          uint32_t pk[4][2];
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              v[e] = c[ib][jb][4 * gq + e];
              if (has_bias) v[e] = v[e] + params[512 + wn * 64 + ib * 32 + 8 * gq + 4 * half + e];
            }
            pk[gq][0] = pack_bf16x2(v[0], v[1]);
            pk[gq][1] = pack_bf16x2(v[2], v[3]);
          }
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            const auto s02 = __builtin_amdgcn_permlane32_swap(pk[0][w], pk[2][w], false, false);
            const auto s13 = __builtin_amdgcn_permlane32_swap(pk[1][w], pk[3][w], false, false);
            pk[0][w] = s02[0];
            pk[2][w] = s02[1];
            pk[1][w] = s13[0];
            pk[3][w] = s13[1];
          }
          const int m = m0 + wm * 128 + jb * 32 + sub;
          const int n = n0 + wn * 64 + ib * 32 + 16 * half;
          uint16_t* dst = out + (int64_t)m * a.ldo + n;
          const v4i lo = (v4i){(int)pk[0][0], (int)pk[0][1], (int)pk[2][0], (int)pk[2][1]};
          const v4i hi = (v4i){(int)pk[1][0], (int)pk[1][1], (int)pk[3][0], (int)pk[3][1]};
          if (full) {
            *reinterpret_cast<v4i*>(dst) = lo;
            *reinterpret_cast<v4i*>(dst + 8) = hi;
          } else if (m < a.M) {
            const uint32_t wds[8] = {pk[0][0], pk[0][1], pk[2][0], pk[2][1], pk[1][0], pk[1][1], pk[3][0], pk[3][1]};
            for (int e = 0; e < 16; ++e)
              if (n + e < a.N) dst[e] = (uint16_t)(wds[e >> 1] >> (16 * (e & 1)));
          }
        }
      }
    }
    // A partial tile's guarded stores (and the r > 64 global reads) are not a fixed count: drain everything.
    if (!full) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    g += nk + (kLr ? 2 : 0);
    id = next_id;
    cur = nxt;
    return full;
  };
  while (id < total) {
    stores_behind = stores_behind ? tile(std::integral_constant<int, kFastStores>{})
                                  : tile(std::integral_constant<int, 0>{});
  }
  // Zero-fill loads for the tile after the last may still be landing in LDS.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template __global__ void int8_gemm_kernel<kOutI32>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr>(GemmArgs);

}  // namespace hf
