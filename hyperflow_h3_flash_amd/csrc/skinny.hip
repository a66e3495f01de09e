// INT8 x INT8 -> INT32 partial products for at most 256 rows (timestep / text-conditioning modulation, short audio
// streams): the accumulator of int8_mm_kernel (src/hyperflow_h3_flash/int8.py:302-306) for a K chunk, written as an
// int32 plane (block by block, partial_block_offset) that splitk_epilogue_kernel adds up and finishes.
//
// With few rows the weight stream is most of the traffic (N x K bytes against MR x K of activations), so the work is
// cut into many small weight slices: a work item is 128 weight rows x one K chunk (blockIdx.x = n tile, blockIdx.y =
// chunk), about as many items as CUs. A stage is 128 bytes of K for the 128 weight rows and the MR activation rows
// (MR = 64, 128 or 256: 24, 32 or 48 KiB), global -> LDS with buffer_load ... lds as whole 128-byte lines (8 lanes per
// row), in a 3-stage ring (72, 96 or 144 KiB; with MR = 64 two work items share a CU and one's start overlaps the
// other's tail): two stages in flight while one is multiplied. Wave w multiplies weight rows 32(w % 4)..+31 against
// the activation rows (all MR of them with 4 waves; half of them each with the 8 waves of MR = 256):
// v_mfma_i32_32x32x32_i8 with the weight as the first operand, up to 4 blocks per K step. Against
// 256 x 256 tiles split over K (the persistent GEMM's few-row mode), 128-row slices give a few-row GEMM four times as
// many work items before K is split, so fewer partial planes are written and added.
#include "common.h"

namespace hf {

constexpr int kSkinnyM = 64;                          // activation rows of the smallest form
constexpr int kSkinnyMaxM = 256;                      // activation rows of the largest form
constexpr int kSkinnyN = 128;                         // weight rows per work item
constexpr int kSkinnyStageK = 128;                    // K bytes per stage
constexpr int kSkinnyWBytes = kSkinnyN * kSkinnyStageK;   // 16 KiB
constexpr int kSkinnyStages = 3;
// LDS per stage and per workgroup for MR activation rows.
__host__ __device__ constexpr int skinny_stage_bytes(int mr) { return kSkinnyWBytes + mr * kSkinnyStageK; }
__host__ __device__ constexpr int skinny_lds(int mr) { return kSkinnyStages * skinny_stage_bytes(mr); }
// Waves per workgroup: 4 (one per 32 weight rows), 8 with 256 activation rows (the two halves of the rows on
// different waves, so each SIMD runs two waves while one workgroup fills the CU's LDS).
__host__ __device__ constexpr int skinny_waves(int mr) { return mr == 256 ? 8 : 4; }
constexpr int kSkinnyLds = skinny_lds(kSkinnyM);      // 72 KiB

__device__ __forceinline__ int skinny_swz(int r) { return (r & 7) ^ ((r >> 3) & 3); }

// GLU: the weight rows are read in pair order (tile column n is weight row glu_row(n, glu_half, glu_gate_first)),
// the order the split-K epilogue's SwiGLU pairs columns in.
template <bool GLU, int MR = kSkinnyM>
__global__ __launch_bounds__(64 * skinny_waves(MR), MR == kSkinnyM ? 2 : 1) void skinny_gemm_kernel(const int8_t* __restrict__ q, int64_t ldq,
                                                             const int8_t* __restrict__ w, int64_t ldw,
                                                             int32_t* __restrict__ acc, int64_t plane, int M, int N,
                                                             int K, int k_chunk, int glu_half, int glu_gate_first) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char sk_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)sk_smem_raw;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 31, half = lane >> 5;
  const int n0 = blockIdx.x * kSkinnyN;
  const int k_lo = blockIdx.y * k_chunk;
  const int k_len = min(K - k_lo, k_chunk);
  const int rows_n = min(kSkinnyN, N - n0);
  // Pair order scatters the tile's rows over both halves of the weight: one descriptor for all of it.
  const uint32_t bytes_w = (uint32_t)((GLU ? N : rows_n) * ldw), bytes_q = (uint32_t)(M * ldq);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + (GLU ? 0 : (int64_t)n0 * ldw) + k_lo, bytes_w - (uint32_t)k_lo);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(q + k_lo, bytes_q - (uint32_t)k_lo);

  // Stage t -> slot t % 3. Every stage issues kLoads loads per wave (4 weight blocks and MR / 32 activation blocks
  // of 1 KiB), stages past the chunk read zeros, so "stage t has landed" is always vmcnt(kLoads) with the next stage
  // in flight.
  constexpr int kWaves = skinny_waves(MR);
  constexpr int kQBlocks = MR / 32 / (kWaves / 4);     // 32-row activation blocks per wave
  constexpr int kWLoads = 16 / kWaves;                 // 1 KiB loads per wave and stage: weight
  constexpr int kQLoads = MR / 8 / kWaves;             // and activations
  constexpr int kLoads = kWLoads + kQLoads;
  constexpr int kStageBytes = skinny_stage_bytes(MR);
  const int wn = wave % 4, wm = wave / 4;              // weight rows 32 wn.., activation blocks kQBlocks wm..
  auto issue = [&](int t) {
    unsigned char HF_LDS* st = smem + (t % kSkinnyStages) * kStageBytes;
    const int k0 = t * kSkinnyStageK;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const bool isq = i >= kWLoads;
      const int blk = isq ? kQLoads * wave + (i - kWLoads) : kWLoads * wave + i;
      const int row = 8 * blk + (lane >> 3);
      const int c = (lane & 7) ^ skinny_swz(row);
      const int64_t ld = isq ? ldq : ldw;
      const int rows_valid = isq ? M : rows_n;
      const uint32_t oob = isq ? bytes_q : bytes_w;
      // the source row: eight consecutive tile rows from a multiple of 8 are eight consecutive weight rows
      const int src = (GLU && !isq) ? glu_row(n0 + 8 * blk, glu_half, glu_gate_first) + (lane >> 3) : row;
      const uint32_t voff = ((row < rows_valid) & (k0 + c * 16 < k_len)) ? (uint32_t)(src * ld + k0 + c * 16) : oob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isq ? rq : rw,
                                               (void HF_LDS*)(st + (isq ? kSkinnyWBytes : 0) + blk * 1024), 16, voff,
                                               0, 0, 0);
    }
  };

  v16i acc_r[kQBlocks];
#pragma unroll
  for (int jb = 0; jb < kQBlocks; ++jb) acc_r[jb] = (v16i){0};
  const int nst = (k_len + kSkinnyStageK - 1) / kSkinnyStageK;
#pragma unroll
  for (int t = 0; t < kSkinnyStages - 1; ++t) issue(t);
  const int wrow = wn * 32 + sub;
  static_assert(kLoads == 6 || kLoads == 8, "wait counts");
  for (int t = 0; t < nst; ++t) {
    if constexpr (kLoads == 6)
      asm volatile("s_waitcnt vmcnt(6) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(t + kSkinnyStages - 1);
    const unsigned char HF_LDS* st = smem + (t % kSkinnyStages) * kStageBytes;
    // A K step's fragments: the weight's and the activation blocks'.
    struct Frags {
      v4i w;
      v4i q[kQBlocks];
    };
    auto read = [&](Frags& f, int ks) {
      const int chunk = 2 * ks + half;
      f.w = *(const v4i HF_LDS*)(st + wrow * 128 + ((chunk ^ skinny_swz(wrow)) << 4));
#pragma unroll
      for (int jb = 0; jb < kQBlocks; ++jb) {
        const int qrow = (wm * kQBlocks + jb) * 32 + sub;
        f.q[jb] = *(const v4i HF_LDS*)(st + kSkinnyWBytes + qrow * 128 + ((chunk ^ skinny_swz(qrow)) << 4));
      }
    };
    auto mma = [&](const Frags& f) {
#pragma unroll
      for (int jb = 0; jb < kQBlocks; ++jb)
        acc_r[jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(f.w, f.q[jb], acc_r[jb], 0, 0, 0);
    };
    if constexpr (MR == kSkinnyM) {
#pragma unroll
      for (int ks = 0; ks < kSkinnyStageK / 32; ++ks) {
        Frags f;
        read(f, ks);
        mma(f);
      }
    } else {
      // Steps 0 and 1 read up front, steps 2 and 3 among the MFMAs of the two steps before them; the scheduling
      // groups keep that order (left to itself the compiler moves each read down to its MFMA, which then waits for
      // it): 2-3 % faster per layer with 128 and 256 rows, 2 % slower with 64, which keeps the plain loop.
      Frags f0, f1;
      read(f0, 0);
      read(f1, 1);
      mma(f0);
      read(f0, 2);
      mma(f1);
      read(f1, 3);
      mma(f0);
      mma(f1);
      constexpr int kReads = 1 + kQBlocks;
      __builtin_amdgcn_sched_group_barrier(0x100, 2 * kReads, 0);  // DS read
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
#pragma unroll
        for (int i = 1; i < kQBlocks; ++i) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        }
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 2 * kQBlocks, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // zero-fill loads past the chunk may still be landing

  // Lane (sub, h) holds row m = 32jb + sub, columns n0 + 32w + 8g + 4h + (0..3) in registers 4g..4g+3: block
  // (jb, n0 / 32 + w) of this chunk's plane, written whole (partial_block_offset's layout).
  int32_t* out = acc + blockIdx.y * plane;
  const int nbn = (N + 31) / 32, bn = n0 / 32 + wn;
  if (32 * bn >= N) return;
#pragma unroll
  for (int jb = 0; jb < kQBlocks; ++jb) {
    const int bm = wm * kQBlocks + jb;
    if (32 * bm >= M) continue;
    v4i* dst = reinterpret_cast<v4i*>(out + partial_block_offset(bm, bn, nbn) + 4 * lane);
    const v16i& c = acc_r[jb];
#pragma unroll
    for (int g = 0; g < 4; ++g) dst[64 * g] = (v4i){c[4 * g], c[4 * g + 1], c[4 * g + 2], c[4 * g + 3]};
  }
}

#define HF_SKINNY(GLU, MR)                                                                                          \
  template __global__ void skinny_gemm_kernel<GLU, MR>(const int8_t*, int64_t, const int8_t*, int64_t, int32_t*,     \
                                                       int64_t, int, int, int, int, int, int);
HF_SKINNY(false, 64) HF_SKINNY(true, 64) HF_SKINNY(false, 128) HF_SKINNY(true, 128) HF_SKINNY(false, 256)
HF_SKINNY(true, 256)
#undef HF_SKINNY

}  // namespace hf
