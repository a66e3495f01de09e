// INT8 x INT8 -> INT32 GEMM on gfx950 MFMA with the convrot epilogue fused.
//
// Replaces the reference's `int8_mm_kernel` (src/hyperflow_h3_flash/int8.py:283-313) and its `rescale_kernel`
// epilogue (int8.py:315-324):
//   acc[m, n] = sum_k q[m, k] * w[n, k]                      exact int32
//   y[m, n]   = bf16((f32(acc) * sx[m]) * sw[n])              two separately rounded fp32 products (int8.py:179)
// extended with the low-rank branch and a bias (the composition with LowRankLinear, transformer.py:57-58):
//   y[m, n]   = bf16((f32(acc) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n])
// With no low-rank branch and no bias the output is bitwise the reference's. Optionally the bf16 output then goes
// through an activation and is rounded again (ACT: the FFN up-projection's tanh-GELU, transformer.py:75-99).
//
// Tiling: 256 (m) x 256 (n) output tile per workgroup (one workgroup per CU, persistent), 8 waves (two per SIMD) in
// a 2 (m) x 4 (n) grid, each a 128 x 64 sub-tile of 4 x 2 v_mfma_i32_32x32x32_i8 blocks (128 accumulator
// registers). The MFMA's first operand is the weight (its rows are the output columns n) and the second the
// activation, so each lane ends with four consecutive n of one row m.
//
// Operands: K is consumed in stages of 128 bytes. A stage (256 rows of q and 256 rows of w, 128 bytes each: 64 KiB)
// goes global -> LDS with buffer_load ... lds, 16 bytes per lane, 8 lanes per row, so every load instruction moves
// 8 whole 128-byte lines (half-line requests measured 11 % slower: the texture-address FIFOs fill). Two stage slots
// alternate (double buffering): the loads of stage s + 2 are issued after the MFMAs of a K step, while stage s + 1
// is multiplied. Waits are exact vmcnt counts; the barrier carries no memory fence. MFMA operands are
// double-buffered in registers (the LDS reads of one 32-byte K step overlap the MFMAs of the previous one).
// Out-of-range rows and K beyond the end read as zero through the buffer descriptor's range check.
//
// The slot of a tile's last stage is the epilogue's: once every wave has read its last fragments it receives the
// tile's low-rank operands (u rows m and up rows n, rank <= 64, one 128-byte row each) while the last K step is
// multiplied, then stages the bf16 output so each store instruction writes 8 whole 128-byte lines. Meanwhile the
// other slot already receives the next tile's first stage, and the next tile's second stage is issued into the
// epilogue slot once the stores are out: loads never stop at a tile boundary.
#include <type_traits>

#include "common.h"

namespace hf {

constexpr int GBM = 256;                          // activation rows (m) per workgroup tile
constexpr int GBN = 256;                          // weight rows (n) per workgroup tile
constexpr int GBK = 128;                          // K bytes per pipeline stage
constexpr int kAStage = GBM * GBK;                // 32 KiB
constexpr int kBStage = GBN * GBK;                // 32 KiB
constexpr int kSlotBytes = kAStage + kBStage;     // 64 KiB
constexpr int kRingBytes = 2 * kSlotBytes;        // 128 KiB
constexpr int kParamBytes = 3 * 256 * 4;          // the tile's sx, wscale and bias (fp32)
constexpr int kGemmLds = kRingBytes + kParamBytes;
// Waves per workgroup: 2 (m) x 4 (n) waves of 128 x 64, two per SIMD. The index arithmetic below is written for
// any even count, but only 8 is built: 4 waves of 128 x 128 (one per SIMD, accumulators in AGPRs) measured slower,
// and the pair-order (SwiGLU) epilogue is laid out for 8.
constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int WN = 2 * GBN / kWaves;              // n columns per wave
constexpr int NB = WN / 32;                       // 32-column MFMA blocks per wave
constexpr int kBlkPerWave = 32 / kWaves;          // 1 KiB load blocks per operand per wave and stage
constexpr int kStageLoads = 2 * kBlkPerWave;      // load instructions per wave per stage

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
  // Split K (int32 output only): work item w covers tile w % tiles and K bytes [s * k_chunk, (s + 1) * k_chunk) with
  // s = w / tiles, and writes its partial accumulators to plane s, split_stride elements after plane s - 1, block by
  // block (partial_block_offset, nbn = ceil(N / 32); the planes hold ceil(M / 32) x nbn whole blocks).
  int splits;            // 1: no split
  int k_chunk;           // multiple of GBK
  int64_t split_stride;
  // Gated-linear-unit pair order (the ACT == kActSwiGLU kernels): column n multiplies weight row
  // glu_row(n, glu_half, glu_gate_first), the per-column wscale, bias and up rows follow it, and the output has
  // N / 2 columns.
  int glu_half, glu_gate_first;
};

// Workgroup id -> (tile_m, tile_n). The dispatcher deals workgroup ids round robin to the 8 XCDs (XCD = id % 8,
// in id order within an XCD), and each XCD has its own L2. The map gives XCD x the x-th contiguous share of a
// grouped order in which 8 tile rows are walked column by column, so the 32 tiles an XCD runs at once form an 8 x 4
// block: 12 operand panels for 32 tiles instead of ~36 for the row-major order.
constexpr int kGroupRows = 8;

__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n, per = total / 8, rem = total % 8, xcd = bid % 8, local = bid / 8;
  const int logical = xcd < rem ? xcd * (per + 1) + local : rem * (per + 1) + (xcd - rem) * per + local;
  const int group = kGroupRows * tiles_n, first = (logical / group) * kGroupRows;
  const int rows = min(tiles_m - first, kGroupRows), within = logical % group;
  tm = first + within % rows;
  tn = within / rows;
}

// LDS rows are 128 bytes (eight 16-byte chunks); chunk c of row r is stored at c ^ f(r) with
// f(r) = (r & 7) ^ ((r >> 3) & 3). The 16 lanes a ds_read_b128 serves per cycle read rows R..R+15 (R a multiple of
// 16) at one logical chunk and land on 16 distinct 16-byte slots of a 256-byte bank window. f only sees row bits
// 0-4, so it is the same for every 32-row MFMA block.
__device__ __forceinline__ int row_swz(int r) { return (r & 7) ^ ((r >> 3) & 3); }

// One tile's operand source: buffer descriptors for its q rows and w rows (rows past the matrix, and every row of a
// tile past the last one, read as zero). Wave-uniform: it lives in scalar registers.
struct TileSrc {
  int m0, n0, rows_m, rows_n;
  int k_lo, k_hi;  // the work item's K range
  int split;
  uint32_t bytes_q, bytes_w;
  __amdgpu_buffer_rsrc_t rq, rw;
};

template <bool GLU>
__device__ __forceinline__ void tile_src(const GemmArgs& a, int id, TileSrc& t) {
  int tm = 0, tn = 0;
  const int tiles = a.tiles_m * a.tiles_n;
  const bool live = id < tiles * a.splits;
  t.split = live ? id / tiles : 0;
  if (live) tile_of(id - t.split * tiles, a.tiles_m, a.tiles_n, tm, tn);
  // The divisions above run on the vector unit; their results are uniform. Keeping them (and so the descriptors)
  // in scalar registers avoids a per-load loop over lanes.
  tm = __builtin_amdgcn_readfirstlane(tm);
  tn = __builtin_amdgcn_readfirstlane(tn);
  t.split = __builtin_amdgcn_readfirstlane(t.split);
  t.k_lo = t.split * a.k_chunk;
  t.k_hi = min(a.K, t.k_lo + a.k_chunk);
  t.m0 = tm * GBM;
  t.n0 = tn * GBN;
  t.rows_m = live ? min(GBM, a.M - t.m0) : 0;
  t.rows_n = live ? min(GBN, a.N - t.n0) : 0;
  t.bytes_q = (uint32_t)(t.rows_m * a.ldq);
  t.rq = make_rsrc(a.q + (int64_t)t.m0 * a.ldq, t.bytes_q);
  if (GLU) {
    // Pair order scatters the tile's columns over both halves of the weight: one descriptor for all of it.
    t.bytes_w = (uint32_t)((int64_t)a.N * a.ldw);
    t.rw = make_rsrc(a.w, t.bytes_w);
  } else {
    t.bytes_w = (uint32_t)(t.rows_n * a.ldw);
    t.rw = make_rsrc(a.w + (int64_t)t.n0 * a.ldw, t.bytes_w);
  }
}

// The weight row of tile column `col` (0..255) relative to the tile's descriptor: the column itself, or in pair
// order its global row. Eight consecutive columns starting at a multiple of 8 map to eight consecutive rows.
template <bool GLU>
__device__ __forceinline__ int weight_row(const GemmArgs& a, const TileSrc& t, int col) {
  return GLU ? glu_row(t.n0 + col, a.glu_half, a.glu_gate_first) : col;
}

// The per-lane part of a stage load's address, the same for every tile. Load i of a wave fills the 1 KiB block
// blk = kBlkPerWave * wave + i of its operand (8 rows): lane l fills row r = 8 * blk + l / 8, physical chunk l % 8,
// from logical chunk (l % 8) ^ f(r) = (l % 8) ^ (l / 8) ^ (i % 4) (f sees r % 8 = l / 8 and (r / 8) % 4 = i % 4).
struct LaneLoad {
  uint32_t row_q, row_w;  // (l / 8) * ld of q and of w
  uint32_t chunk;         // ((l % 8) ^ (l / 8)) * 16
  int lrow;               // l / 8
};

// Load j of this wave's share of stage kt, into slot `slot`: j < kBlkPerWave fills q block kBlkPerWave * wave + j,
// the others w block kBlkPerWave * wave + j - kBlkPerWave. Rows past the tile's valid rows and chunks at or past K read as zero (the offset moves
// past the descriptor), branch-free; so does every load of a stage past the end.
template <bool GLU>
__device__ __forceinline__ void load_one(const GemmArgs& a, const TileSrc& t, const LaneLoad& ll, int kt, int j,
                                         unsigned char HF_LDS* slot, int wave) {
  const int i = j % kBlkPerWave;
  const bool isw = j >= kBlkPerWave;
  const int64_t ld = isw ? a.ldw : a.ldq;
  const int rows_valid = isw ? t.rows_n : t.rows_m;
  const uint32_t oob = isw ? t.bytes_w : t.bytes_q;
  const int row0 = 8 * (kBlkPerWave * wave + i);
  const int row = row0 + ll.lrow;
  const uint32_t cb = ll.chunk ^ (uint32_t)(16 * (i & 3));
  const uint32_t k0 = (uint32_t)(t.k_lo + kt * GBK);
  const int src_row0 = isw ? weight_row<GLU>(a, t, row0) : row0;
  const uint32_t off = (isw ? ll.row_w : ll.row_q) + (uint32_t)(src_row0 * ld) + cb + k0;
  const uint32_t voff = ((row < rows_valid) & (k0 + cb < (uint32_t)t.k_hi)) ? off : oob;  // '&': no branch
  __builtin_amdgcn_raw_ptr_buffer_load_lds(isw ? t.rw : t.rq,
                                           (void HF_LDS*)(slot + (isw ? kAStage : 0) + (row0 / 8) * 1024), 16,
                                           voff, 0, 0, 0);
}

// The low-rank operands of a tile (u rows m into the slot's q half, up rows n into its w half, rank r <= 64: one
// 128-byte row each; chunks past r and rows past the tile's valid rows read as zero), in as many loads per wave as
// a stage.
template <bool GLU>
__device__ __forceinline__ void load_lowrank(const GemmArgs& a, const TileSrc& t, unsigned char HF_LDS* slot,
                                             int wave, int lane) {
#pragma unroll
  for (int j = 0; j < kStageLoads; ++j) {
    const bool isup = j >= kBlkPerWave;
    const int64_t ld_bytes = (isup ? a.ldup : a.ldu) * 2;
    const int rows_valid = isup ? t.rows_n : t.rows_m;
    const bool whole = isup && GLU;  // pair order: up rows follow the weight rows, anywhere in up
    const uint32_t bytes = (uint32_t)((whole ? a.N : rows_valid) * ld_bytes);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(
        isup ? (const void*)(a.up + (whole ? 0 : (int64_t)t.n0 * a.ldup)) : (const void*)(a.u + (int64_t)t.m0 * a.ldu),
        bytes);
    const int blk = kBlkPerWave * wave + j % kBlkPerWave, r = 8 * blk + (lane >> 3);
    const int src_r = (isup ? weight_row<GLU>(a, t, 8 * blk) : 8 * blk) + (lane >> 3);
    const int c = (lane & 7) ^ row_swz(r);
    const uint32_t voff = ((r < rows_valid) & (c * 8 < a.r)) ? (uint32_t)(src_r * ld_bytes + c * 16) : bytes;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (void HF_LDS*)(slot + (isup ? kAStage : 0) + blk * 1024), 16,
                                             voff, 0, 0, 0);
  }
}

struct Frags {
  v4i a[4];   // activation rows: 4 blocks of 32 (the wave's 128 m)
  v4i b[NB];  // weight rows: NB blocks of 32 (the wave's WN n)
};

// Operand fragments of K step ks (32 bytes: chunks 2ks and 2ks + 1; lane half h reads chunk 2ks + h of row sub of
// each 32-row block). `ca` is this lane's byte offset of that chunk within its row block (sub * 128 + swizzled
// chunk); the block and slot offsets are wave-uniform.
__device__ __forceinline__ void read_frags(Frags& f, const unsigned char HF_LDS* slot, int wm, int wn, int ca) {
  const unsigned char HF_LDS* As = slot + wm * 128 * GBK + ca;
  const unsigned char HF_LDS* Bs = slot + kAStage + wn * WN * GBK + ca;
#pragma unroll
  for (int jb = 0; jb < 4; ++jb) f.a[jb] = *(const v4i HF_LDS*)(As + jb * 32 * GBK);
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) f.b[ib] = *(const v4i HF_LDS*)(Bs + ib * 32 * GBK);
}

// BF16 = false: the INT8 product (v_mfma_i32_32x32x32_i8, int32 sums). BF16 = true: the operands are bf16 and the
// sums fp32 (v_mfma_f32_32x32x16_bf16, kept in the same registers): its fragment of a 32-byte K step is the same 16
// bytes per lane (lane half h: elements 8h .. 8h + 7 of the step's 16) and its 32 x 32 result has the same layout.
template <bool BF16 = false>
__device__ __forceinline__ void mma(v16i (&acc)[NB][4], const Frags& f) {
#pragma unroll
  for (int ib = 0; ib < NB; ++ib)
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
      if constexpr (BF16) {
        acc[ib][jb] = __builtin_bit_cast(
            v16i, __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(v8bf, f.b[ib]),
                                                          __builtin_bit_cast(v8bf, f.a[jb]),
                                                          __builtin_bit_cast(v16f, acc[ib][jb]), 0, 0, 0));
      } else {
        acc[ib][jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.b[ib], f.a[jb], acc[ib][jb], 0, 0, 0);
      }
    }
}

#define HF_BARRIER() asm volatile("s_barrier" ::: "memory")

// s_waitcnt vmcnt(n) for the wave-uniform counts the loop uses (an unlisted count waits for everything, which is
// always safe). The accounting relies on vector memory operations completing in issue order (loads, LDS-DMA loads
// and stores share one in-order counter on gfx9).
__device__ __forceinline__ void wait_vm(int n) {
  switch (n) {
    case 8: asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory"); break;
    case 16: asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)" ::: "memory"); break;
    case 24: asm volatile("s_waitcnt vmcnt(24) lgkmcnt(0)" ::: "memory"); break;
    case 40: asm volatile("s_waitcnt vmcnt(40) lgkmcnt(0)" ::: "memory"); break;
    case 48: asm volatile("s_waitcnt vmcnt(48) lgkmcnt(0)" ::: "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory"); break;
  }
}

// Output modes: int32 accumulators; bf16 with the dequantization (and, for r > 64, the low-rank term from global
// memory) and bias; bf16 with a rank <= 64 low-rank term whose operands ride the ring; and kOutMmBf16, a bf16
// product: q and w hold bf16 rows (ldq, ldw and K in bytes), the sums are fp32 and the output is bf16(sum + bias)
// (the low-rank up projection, whose small K and large output suit the persistent tiles and their whole-line stores).
constexpr int kOutI32 = 0, kOutBf16 = 1, kOutBf16Lr = 2, kOutMmBf16 = 3;
// Deepest K for which the bf16-output GEMMs issue their stage loads after a K step's MFMAs (LATE).
constexpr int kLateLoadsMaxK = 8192;


// Persistent kernel: one workgroup per CU walks tiles blockIdx.x, blockIdx.x + gridDim.x, ... Every wave issues the
// same number of memory operations in the same order, so every wait is a constant vmcnt. LATE places each stage's
// loads after the MFMAs of the K step that issues them instead of two per MFMA among them (the host's choice by K).
template <int OUT, int ACT = kActNone, bool LATE = false>
__global__ __launch_bounds__(kThreads, 1) void int8_gemm_kernel(GemmArgs a) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // uniform: keeps LDS addresses scalar
  const int wm = wave & 1, wn = wave >> 1;  // 2 (m) x (kWaves / 2) (n) waves of 128 x WN
  const int sub = lane & 31, half = lane >> 5;
  constexpr bool kLr = OUT == kOutBf16Lr;
  constexpr bool kGlu = ACT == kActSwiGLU;  // pair order (the glu fields of GemmArgs)
  // Stores per wave of a full tile, when the wait for the next stage 0 behind them fits the 6-bit wait counter
  // (else they are drained).
  constexpr int kTileStores =
      GBM * GBN * (OUT == kOutI32 ? 4 : 2) / (ACT == kActSwiGLU && OUT != kOutI32 ? 2 : 1) / (kWaves * 1024);
  constexpr int kFastStores = kTileStores + kStageLoads <= 63 ? kTileStores : 0;
  float HF_LDS* params = (float HF_LDS*)(smem + kRingBytes);
  const int pt = threadIdx.x & 255;
  auto slot_at = [&](int s) { return smem + (s & 1) * kSlotBytes; };

  // This lane's fragment offsets for the four K steps of a stage.
  int ca[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) ca[ks] = sub * GBK + (((2 * ks + half) ^ row_swz(sub)) << 4);

  // K stages per work item, at least 2 (stages past its K range read zeros and add nothing).
  const int nk = max((a.k_chunk + GBK - 1) / GBK, 2);
  const int total = a.tiles_m * a.tiles_n * a.splits;
  int id = blockIdx.x;
  LaneLoad ll;
  ll.lrow = lane >> 3;
  ll.row_q = (uint32_t)((lane >> 3) * a.ldq);
  ll.row_w = (uint32_t)((lane >> 3) * a.ldw);
  ll.chunk = (uint32_t)(((lane & 7) ^ (lane >> 3)) << 4);
  TileSrc cur;
  tile_src<kGlu>(a, id, cur);
#pragma unroll
  for (int j = 0; j < kStageLoads; ++j) load_one<kGlu>(a, cur, ll, 0, j, slot_at(0), wave);
#pragma unroll
  for (int j = 0; j < kStageLoads; ++j) load_one<kGlu>(a, cur, ll, 1, j, slot_at(1), wave);

  int g = 0;  // slot parity of the current tile's stage 0
  Frags f0, f1;
  v16i acc[NB][4];

  // MFMAs of one K step on `use` with the LDS reads of the next fragments (`read`) spread between them, two per
  // MFMA, and, when `loads` issues a stage's loads, those two per MFMA after them or (LATE) after the step's last
  // MFMA. Every wave issues its share of a stage right after the barrier; issued late, a load whose issue waits for
  // the texture unit holds up no MFMA of the step. Measured (GEMM with the rank-64 epilogue, same box, bitwise
  // equal): late 0.7-1.1 % faster at K = 5120-7168 (M=32768, N=15360: 2135 -> 2112 us; M=37710, K=5376, N=7168:
  // 1257 -> 1240 us), but 2.7-4.4 % slower at K = 13824-14336 (M=37710, K=14336, N=5376: 2486 -> 2583 us).
  auto kstep = [&](const Frags& use, auto&& read, auto&& loads) {
    read();
    mma<OUT == kOutMmBf16>(acc, use);
    loads();
#pragma unroll
    for (int i = 0; i < (4 + NB) / 2; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS read
    }
    if constexpr (LATE) {
      __builtin_amdgcn_sched_group_barrier(0x008, 4 * NB, 0);
      __builtin_amdgcn_sched_group_barrier(0x020, kStageLoads, 0);  // VMEM (stage loads)
    } else {
#pragma unroll
      for (int i = 0; i < kStageLoads / 2; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);  // VMEM (stage loads)
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 4 * NB, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto nothing = [] {};

  // One tile. SPILL is the number of the previous epilogue's stores that sit between this tile's stage 0 and stage
  // 1 loads (0 when they were drained), so every wait count below is a constant.
  auto tile = [&](auto spill_tag) -> bool {
    constexpr int spill = decltype(spill_tag)::value;
    // An opaque copy of the wave id for this tile's load addressing: keeps the compiler from hoisting the
    // per-load scalar offsets out of the tile loop (they would stay live, and spill, across it).
    int wv = wave;
    asm volatile("" : "+s"(wv));

    // Stage 0 has landed for this wave once only the stores and stage 1's loads remain; the barrier makes it so for
    // every wave.
    wait_vm(spill + kStageLoads);
    HF_BARRIER();
    read_frags(f0, slot_at(g), wm, wn, ca[0]);

    // The epilogue's per-row and per-column factors, loaded now and parked in LDS after the first boundary: thread
    // t < 256 takes sx of row m0 + t and wscale of column n0 + t, thread 256 + t (with 4 waves: thread t too) the
    // bias of column n0 + t. Every wave issues the same loads. Clamped, branch-free.
    float p_val = 0.0f, p_ws = 0.0f;
    uint32_t p_bias = 0;
    if (OUT != kOutI32) {
      const int mr = min(cur.m0 + pt, a.M - 1);
      const int ncol = min(cur.n0 + pt, a.N - 1);
      const int nc = kGlu ? glu_row(ncol, a.glu_half, a.glu_gate_first) : ncol;
      if constexpr (OUT == kOutMmBf16) {
        // A bf16 product has no scales; the bias is optional.
        if ((kThreads == 256 || threadIdx.x >= 256) && a.bias) p_bias = (uint32_t)a.bias[nc];
      } else {
        const uint16_t* bsrc = a.bias ? a.bias : reinterpret_cast<const uint16_t*>(a.sw);
        if (kThreads == 256 || threadIdx.x < 256) {
          p_val = a.sx[mr];
          p_ws = a.sw[nc];
        }
        if (kThreads == 256 || threadIdx.x >= 256) p_bias = (uint32_t)bsrc[nc];
      }
    }

#pragma unroll
    for (int i = 0; i < NB; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (v16i){0};

    // Stage s: K steps 0..2, then (unless s is the last stage) wait for stage s + 1, barrier (every wave is done
    // with slot s), and K step 3 with the reads of stage s + 1's first fragments and the refill of slot s.
    auto first_steps = [&](int s) {
      const unsigned char HF_LDS* sl = slot_at(g + s);
      kstep(f0, [&] { read_frags(f1, sl, wm, wn, ca[1]); }, nothing);
      kstep(f1, [&] { read_frags(f0, sl, wm, wn, ca[2]); }, nothing);
      kstep(f0, [&] { read_frags(f1, sl, wm, wn, ca[3]); }, nothing);
    };
    auto boundary = [&](int s, auto&& loads) {
      wait_vm(0);
      HF_BARRIER();
      if (OUT != kOutI32 && s == 0) {
        // The parameter loads have landed (vmcnt(0)); park them in LDS for the epilogue. Nothing reads this area
        // until then, and the barriers in between publish it.
        if (kThreads == 256 || threadIdx.x < 256) {
          params[pt] = (cur.m0 + pt < a.M) ? p_val : 0.0f;
          params[256 + pt] = (cur.n0 + pt < a.N) ? p_ws : 0.0f;
        }
        if (kThreads == 256 || threadIdx.x >= 256) {
          params[512 + pt] = (cur.n0 + pt < a.N) ? __uint_as_float(p_bias << 16) : 0.0f;
        }
      }
      kstep(f1, [&] { read_frags(f0, slot_at(g + s + 1), wm, wn, ca[0]); }, loads);
    };
    int s = 0;
    for (; s < nk - 2; ++s) {
      first_steps(s);
      boundary(s, [&] {
#pragma unroll
        for (int j = 0; j < kStageLoads; ++j) load_one<kGlu>(a, cur, ll, s + 2, j, slot_at(g + s), wv);
      });
    }
    // Stage nk - 2 refills its slot with the next tile's stage 0; stage nk - 1 has no successor.
    const int next_id = id + gridDim.x;
    TileSrc nxt;
    tile_src<kGlu>(a, next_id, nxt);
    first_steps(s);
    boundary(s, [&] {
#pragma unroll
      for (int j = 0; j < kStageLoads; ++j) load_one<kGlu>(a, nxt, ll, 0, j, slot_at(g + s), wv);
    });
    first_steps(s + 1);
    // The last K step multiplies fragments already in registers, so once every wave's reads have returned the last
    // stage's slot is free: it becomes the epilogue slot E. In low-rank mode E receives the tile's low-rank operands
    // (issued between the last K step's MFMAs), which land while the accumulators are dequantized; then E stages
    // the output.
    unsigned char HF_LDS* eslot = slot_at(g + nk - 1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    HF_BARRIER();
    if constexpr (kLr) {
      kstep(f1, nothing, [&] { load_lowrank<kGlu>(a, cur, eslot, wv, lane); });
    } else {
      kstep(f1, nothing, nothing);
    }

    // ------------------------------------------------------------------------------------------------ epilogue

    // Per-lane epilogue indices from an opaque copy of the lane id: keeps the compiler from hoisting their address
    // arithmetic out of the tile loop, where it would stay live (and spill) across the main loop.
    int el = lane;
    asm volatile("" : "+v"(el));
    const int esub = el & 31, ehalf = el >> 5;
    // Output layout of a 32x32 block: lane holds column j = lane % 32 (the row m here) and, in register v, row
    // i = 8*(v/4) + 4*(lane/32) + v%4 (the column n here): four consecutive n per group of four registers.
    const int m0 = cur.m0, n0 = cur.n0;
    bool full;
    if constexpr (OUT == kOutI32) {
      full = cur.rows_m == GBM && cur.rows_n == GBN && a.out_vec16;
      if (a.splits > 1) {
        // Split-K partial plane, block by block: every block that starts inside the matrix is written whole (four
        // 1 KiB contiguous stores per wave); the stores are a fixed count only for a full tile.
        int32_t* plane = static_cast<int32_t*>(a.out) + cur.split * a.split_stride;
        const int nbn = (a.N + 31) / 32;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          const int bm = (m0 + wm * 128) / 32 + jb;
#pragma unroll
          for (int ib = 0; ib < NB; ++ib) {
            const int bn = (n0 + wn * WN) / 32 + ib;
            if (32 * bm < a.M && 32 * bn < a.N) {
              v4i* dst = reinterpret_cast<v4i*>(plane + partial_block_offset(bm, bn, nbn) + 4 * el);
              const v16i& c = acc[ib][jb];
#pragma unroll
              for (int gq = 0; gq < 4; ++gq)
                dst[64 * gq] = (v4i){c[4 * gq], c[4 * gq + 1], c[4 * gq + 2], c[4 * gq + 3]};
            }
          }
        }
      } else {
      int32_t* out = static_cast<int32_t*>(a.out);
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) {
        const int m = m0 + wm * 128 + jb * 32 + esub;
#pragma unroll
        for (int ib = 0; ib < NB; ++ib)
#pragma unroll
          for (int gq = 0; gq < 4; ++gq) {
            const int n = n0 + wn * WN + ib * 32 + 8 * gq + 4 * ehalf;
            int32_t* dst = out + (int64_t)m * a.ldo + n;
            const v16i& c = acc[ib][jb];
            if (full) {
              store_stream(reinterpret_cast<v4i*>(dst), (v4i){c[4 * gq], c[4 * gq + 1], c[4 * gq + 2], c[4 * gq + 3]});
            } else if (m < a.M) {
              if (a.out_vec16 && n + 4 <= a.N) {
                store_stream(reinterpret_cast<v4i*>(dst), (v4i){c[4 * gq], c[4 * gq + 1], c[4 * gq + 2], c[4 * gq + 3]});
              } else {
                for (int e = 0; e < 4; ++e)
                  if (n + e < a.N) dst[e] = c[4 * gq + e];
              }
            }
          }
      }
      }
    } else {
      full = cur.rows_m == GBM && cur.rows_n == GBN && a.out_vec16 && (kLr || a.r == 0);
      float sxv[4];
#pragma unroll
      for (int jb = 0; jb < 4; ++jb) sxv[jb] = params[wm * 128 + jb * 32 + esub];
      const unsigned char HF_LDS* u_lds = eslot;             // u rows m (128-byte rows)
      const unsigned char HF_LDS* up_lds = eslot + kAStage;  // up rows n
      // Packed bf16 results, two 16-byte chunks per block: pk[ib][jb][0..3] is chunk 4ib + 2h, pk[ib][jb][4..7]
      // chunk 4ib + 2h + 1 of row esub of block (ib, jb), h = ehalf.
      uint32_t pk[NB][4][8];
      uint32_t gk[NB][4][4];  // pair order: the 16 outputs of a block, 8 per lane half
      const bool has_bias = a.bias != nullptr;
      // Two column blocks at a time (the fp32 values of two blocks are 128 registers): dequantize, add the low-rank
      // term, the bias, convert.
#pragma unroll
      for (int pb = 0; pb < NB; pb += 2) {
        v16f c[2][4];
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int ib = pb + i2;
#pragma unroll
          for (int jb = 0; jb < 4; ++jb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int nl = wn * WN + ib * 32 + 8 * (v >> 2) + 4 * ehalf + (v & 3);
              if constexpr (OUT == kOutMmBf16)
                c[i2][jb][v] = __int_as_float(acc[ib][jb][v]);  // the fp32 sum
              else
                c[i2][jb][v] = ((float)acc[ib][jb][v] * sxv[jb]) * params[256 + nl];
            }
        }
        if constexpr (kLr) {
          // Low-rank term: first operand up[n, :], second u[m, :], 16 ranks per MFMA, accumulated onto the
          // dequantized values. The operands have landed once nothing is in flight; the barrier makes that true
          // for every wave's loads. Rank steps outermost and unrolled: the 6 fragment reads of a step serve its 8
          // independent MFMAs (the u fragments are shared by both column blocks), and the next step's reads are
          // issued while they run. Always four steps, straight-line: ranks past r read as zero (load_lowrank), so
          // they add exact zeros.
          if (pb == 0) {
            wait_vm(0);
            HF_BARRIER();
          }
          auto lr_step = [&](int kk) {
            const int chunk = 2 * kk + ehalf;
            v8bf pf[2], uf[4];
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
              const int nl = wn * WN + (pb + i2) * 32 + esub;
              pf[i2] = *(const v8bf HF_LDS*)(up_lds + nl * GBK + ((chunk ^ row_swz(nl)) << 4));
            }
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
              const int ml = wm * 128 + jb * 32 + esub;
              uf[jb] = *(const v8bf HF_LDS*)(u_lds + ml * GBK + ((chunk ^ row_swz(ml)) << 4));
            }
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2)
#pragma unroll
              for (int jb = 0; jb < 4; ++jb)
                c[i2][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf[i2], uf[jb], c[i2][jb], 0, 0, 0);
          };
#pragma unroll
          for (int kk = 0; kk < 4; ++kk) lr_step(kk);
        }
#pragma unroll
        for (int i2 = 0; i2 < 2; ++i2) {
          const int ib = pb + i2;
          if (!kLr && a.r > 0) {
            // Ranks above 64: the same product from global memory.
            const int ncol = min(n0 + wn * WN + ib * 32 + esub, a.N - 1);
            const int nrow = kGlu ? glu_row(ncol, a.glu_half, a.glu_gate_first) : ncol;
            for (int kk = 0; kk < a.r; kk += 16) {
              const int k = kk + 8 * ehalf;
              const v8bf pf =
                  (k < a.r) ? *reinterpret_cast<const v8bf*>(a.up + (int64_t)nrow * a.ldup + k) : (v8bf){0};
#pragma unroll
              for (int jb = 0; jb < 4; ++jb) {
                const int mrow = min(m0 + wm * 128 + jb * 32 + esub, a.M - 1);
                const v8bf uf =
                    (k < a.r) ? *reinterpret_cast<const v8bf*>(a.u + (int64_t)mrow * a.ldu + k) : (v8bf){0};
                c[i2][jb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pf, uf, c[i2][jb], 0, 0, 0);
              }
            }
          }
          // Bias and bf16. After one exchange between the lane halves (v_permlane32_swap: lanes 32..63 of the
          // first operand <-> lanes 0..31 of the second), lane (sub, h) holds columns 16h..16h+15 of row sub of
          // the block: chunk 4ib + 2h in w4[0], w4[2] and chunk 4ib + 2h + 1 in w4[1], w4[3].
          if (has_bias) {
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
#pragma unroll
              for (int v = 0; v < 16; ++v)
                c[i2][jb][v] = c[i2][jb][v] + params[512 + wn * WN + ib * 32 + 8 * (v >> 2) + 4 * ehalf + (v & 3)];
          }
          if constexpr (ACT == kActSwiGLU) {
            // Pair order: register v < 8 is the hidden column and v + 8 the gate column of output
            // 8 (v / 4) + 4 h + v % 4 of the block's 16. After one exchange between the lane halves, lane (sub, h)
            // holds outputs 8h .. 8h + 7 of row sub: gk[ib][jb][0..3].
#pragma unroll
            for (int jb = 0; jb < 4; ++jb) {
              uint32_t w[4];
#pragma unroll
              for (int i = 0; i < 4; ++i)
                w[i] = pack_bf16x2(swiglu(round_bf16(c[i2][jb][2 * i]), round_bf16(c[i2][jb][2 * i + 8])),
                                   swiglu(round_bf16(c[i2][jb][2 * i + 1]), round_bf16(c[i2][jb][2 * i + 9])));
              const auto s02 = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
              const auto s13 = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
              gk[ib][jb][0] = s02[0];
              gk[ib][jb][1] = s13[0];
              gk[ib][jb][2] = s02[1];
              gk[ib][jb][3] = s13[1];
            }
            continue;
          }
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) {
            uint32_t w4[4][2];
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
              w4[gq][0] = activate_bf16x2<ACT>(pack_bf16x2(c[i2][jb][4 * gq], c[i2][jb][4 * gq + 1]));
              w4[gq][1] = activate_bf16x2<ACT>(pack_bf16x2(c[i2][jb][4 * gq + 2], c[i2][jb][4 * gq + 3]));
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
        }
      }
      // Every wave is done with the low-rank operands: the epilogue slot stages the output, 8 KiB per wave (64 rows
      // of 128 bytes, swizzled like the operands), one round per pair of column blocks and half of the rows. Each
      // lane then reads back 16 bytes of each of 8 rows, and each store instruction writes 8 whole 128-byte lines.
      if constexpr (kLr) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        HF_BARRIER();
      }
      unsigned char HF_LDS* stage_out = eslot + wave * 8192;
      uint16_t* out = static_cast<uint16_t*>(a.out);
      if constexpr (ACT == kActSwiGLU) {
        // Pair order: the wave's outputs are 128 rows x 16 NB columns (64-byte rows, swizzle64) in one round; each
        // store instruction writes 16 rows x 64 bytes, and the four waves of a row band fill whole lines together.
        static_assert(NB == 2, "pair order is laid out for 8 waves");
        const int n_out = a.N / 2, no0 = n0 / 2 + wn * (WN / 2);
#pragma unroll
        for (int ib = 0; ib < NB; ++ib)
#pragma unroll
          for (int jb = 0; jb < 4; ++jb) {
            const int row = jb * 32 + esub;
            *(v4i HF_LDS*)(stage_out + row * 64 + (swizzle64(row, 2 * ib + ehalf) << 4)) =
                (v4i){(int)gk[ib][jb][0], (int)gk[ib][jb][1], (int)gk[ib][jb][2], (int)gk[ib][jb][3]};
          }
        wave_lds_sync();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int row = 16 * i + (el >> 2), ch = el & 3;
          const v4i val = *(const v4i HF_LDS*)(stage_out + row * 64 + (swizzle64(row, ch) << 4));
          const int m = m0 + wm * 128 + row;
          const int n = no0 + 8 * ch;
          uint16_t* dst = out + (int64_t)m * a.ldo + n;
          if (full) {
            store_stream(reinterpret_cast<v4i*>(dst), val);
          } else if (m < a.M) {
            if (a.out_vec16 && n + 8 <= n_out) {
              store_stream(reinterpret_cast<v4i*>(dst), val);
            } else {
              for (int e = 0; e < 8; ++e)
                if (n + e < n_out) dst[e] = (uint16_t)((uint32_t)val[e >> 1] >> (16 * (e & 1)));
            }
          }
        }
      } else {
#pragma unroll
      for (int pb = 0; pb < NB; pb += 2) {
#pragma unroll
        for (int rd = 0; rd < 2; ++rd) {
#pragma unroll
          for (int jj = 0; jj < 2; ++jj) {
            const int jb = 2 * rd + jj;
            const int row = jj * 32 + esub;
#pragma unroll
            for (int i2 = 0; i2 < 2; ++i2) {
              const int ib = pb + i2;
              const int c0 = 4 * i2 + 2 * ehalf;
              *(v4i HF_LDS*)(stage_out + row * GBK + ((c0 ^ row_swz(row)) << 4)) =
                  (v4i){(int)pk[ib][jb][0], (int)pk[ib][jb][1], (int)pk[ib][jb][2], (int)pk[ib][jb][3]};
              *(v4i HF_LDS*)(stage_out + row * GBK + (((c0 + 1) ^ row_swz(row)) << 4)) =
                  (v4i){(int)pk[ib][jb][4], (int)pk[ib][jb][5], (int)pk[ib][jb][6], (int)pk[ib][jb][7]};
            }
          }
          wave_lds_sync();
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int row = 8 * i + (el >> 3), ch = el & 7;
            const v4i val = *(const v4i HF_LDS*)(stage_out + row * GBK + ((ch ^ row_swz(row)) << 4));
            const int m = m0 + wm * 128 + 64 * rd + row;
            const int n = n0 + wn * WN + 32 * pb + 8 * ch;
            uint16_t* dst = out + (int64_t)m * a.ldo + n;
            if (full) {
              store_stream(reinterpret_cast<v4i*>(dst), val);
            } else if (m < a.M) {
              if (a.out_vec16 && n + 8 <= a.N) {
                store_stream(reinterpret_cast<v4i*>(dst), val);
              } else {
                for (int e = 0; e < 8; ++e)
                  if (n + e < a.N) dst[e] = (uint16_t)((uint32_t)val[e >> 1] >> (16 * (e & 1)));
              }
            }
          }
          wave_lds_sync();  // the next round rewrites this wave's staging area
        }
      }
      }
    }
    // A partial tile's guarded stores (and the r > 64 global reads) are not a fixed count, and too many stores do
    // not fit the wait counter next to the next tile's loads: drain everything.
    if (!full || kFastStores == 0) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      full = false;
    }
    // Every wave is done with the epilogue slot: it receives the next tile's stage 1.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    HF_BARRIER();
#pragma unroll
    for (int j = 0; j < kStageLoads; ++j) load_one<kGlu>(a, nxt, ll, 1, j, eslot, wv);
    g += nk - 2;
    id = next_id;
    cur = nxt;
    return full;
  };
  bool stores_behind = false;  // the previous tile's epilogue left kFastStores stores behind the next stage 0
  while (id < total) {
    stores_behind = stores_behind ? tile(std::integral_constant<int, kFastStores>{})
                                  : tile(std::integral_constant<int, 0>{});
  }
  // Zero-fill loads for the tile after the last may still be landing in LDS.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template __global__ void int8_gemm_kernel<kOutI32>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutI32, kActSwiGLU>(GemmArgs);  // split-K partials in pair order
template __global__ void int8_gemm_kernel<kOutBf16>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16, kActGeluTanh>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr, kActGeluTanh>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16, kActSwiGLU>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr, kActSwiGLU>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutMmBf16>(GemmArgs);  // bf16 product (the low-rank up projection)
// Late stage loads (whole-K bf16-output GEMMs with K <= kLateLoadsMaxK).
template __global__ void int8_gemm_kernel<kOutBf16, kActNone, true>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr, kActNone, true>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16, kActGeluTanh, true>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr, kActGeluTanh, true>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16, kActSwiGLU, true>(GemmArgs);
template __global__ void int8_gemm_kernel<kOutBf16Lr, kActSwiGLU, true>(GemmArgs);

}  // namespace hf
