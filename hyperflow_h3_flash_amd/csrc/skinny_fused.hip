// The convrot linear for at most 64 rows in one pass: INT8 x INT8 with the whole K per workgroup and the epilogue
// applied in the same kernel (int8_mm_kernel and its rescale, src/hyperflow_h3_flash/int8.py:283-324, with the
// low-rank/bias extension and the output activation):
//   y[m, n] = bf16((f32(acc) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n]),   acc = q @ w^T exact int32.
//
// With few rows the weight stream is the traffic (N x K bytes against MR x K of codes that stay in L2), so each
// workgroup takes a slice of at most 32 weight rows (`rows`, chosen by the host so the slices cover every CU: 20 at
// N = 5120 on 256 CUs; rows past the slice read as zero and their columns are not stored) and all MR code rows,
// streams the slice's whole K through an LDS ring (D stages of 32 + MR rows x 128 bytes, LDS-DMA whole lines,
// D - 1 stages in flight), and splits each 128-byte stage's four 32-byte K steps over its four waves. At the end the waves' int32
// partial sums are added through LDS (exact in any order) and each 32 x 32 output block goes through the split-K
// finishing pass's epilogue (block_load / block_finish), so the outputs are bitwise those of the split path and of
// the tile GEMM. Against splitting K over workgroups, there are no int32 partial planes to write and read back and no
// second launch.
#include "common.h"

namespace hf {

constexpr int kSfN = 32;        // weight rows per workgroup, at most (the rows of a stage's weight part)
constexpr int kSfWaves = 4;
constexpr int kSfSub = 1;                 // 128-byte K pieces per stage (2 measured no faster)
constexpr int kSfStageK = 128 * kSfSub;   // K bytes per stage
// A stage holds kSfSub pieces, each (32 + mr) rows x 128 bytes laid out like one 128-byte stage.
__host__ __device__ constexpr int sf_piece_bytes(int mr) { return (kSfN + mr) * 128; }
__host__ __device__ constexpr int sf_stage_bytes(int mr) { return kSfSub * sf_piece_bytes(mr); }
// Ring depth: 8 stages (96 KiB with 64 code rows). Measured at M=64 (graph replays over weight copies, runtime slice
// heights): 4, 6, 8 and 12 stages took 19.1, 18.5, 18.4 and 19.3 us at N=K=5120, 17.2, 16.4, 16.3 and 17.2 us at
// N=4096, 36.0, 33.1, 32.6 and 33.6 us at M=48, K=14336, N=5376: past 8 the extra requests in flight only queue.
__host__ __device__ constexpr int sf_depth(int mr) { return 8; }
__host__ __device__ constexpr int sf_lds(int mr) { return sf_depth(mr) * sf_stage_bytes(mr); }

template <int MR, bool GLU>
__global__ __launch_bounds__(64 * kSfWaves, 1) void skinny_fused_kernel(
    const int8_t* __restrict__ q, int64_t ldq, const int8_t* __restrict__ w, int64_t ldw, const float* __restrict__ sx,
    const float* __restrict__ sw, const uint16_t* __restrict__ u, int64_t ldu, const uint16_t* __restrict__ up,
    int64_t ldup, int r, const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K,
    int vec, int act, int glu_half, int glu_gate_first, int rows) {
  extern __shared__ __attribute__((aligned(1024))) unsigned char sf_smem_raw[];
  unsigned char HF_LDS* smem = (unsigned char HF_LDS*)sf_smem_raw;
  constexpr int kD = sf_depth(MR);
  constexpr int kStage = sf_stage_bytes(MR);
  constexpr int kJB = MR / 32;                 // 32-row code blocks
  constexpr int kPieceLoads = 4 + MR / 8;                 // 1 KiB blocks per piece: 4 weight, MR / 8 code
  constexpr int kLoads = kSfSub * kPieceLoads / kSfWaves;  // per wave and stage
  static_assert((kSfSub * kPieceLoads) % kSfWaves == 0, "loads split evenly over the waves");
  static_assert(kD >= 3 && (kD - 2) * kLoads <= 63, "wait count");
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int sub = lane & 31, half = lane >> 5;
  const int n0 = blockIdx.x * rows;
  const int rows_n = min(rows, N - n0);
  const int n_end = min(N, n0 + rows);  // this workgroup's columns end here (pair order: rows == 32)
  // Pair order scatters the slice's rows over both halves of the weight: one descriptor for all of it.
  const uint32_t bytes_w = (uint32_t)((GLU ? N : rows_n) * ldw), bytes_q = (uint32_t)(M * ldq);
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(w + (GLU ? 0 : (int64_t)n0 * ldw), bytes_w);
  const __amdgpu_buffer_rsrc_t rq = make_rsrc(q, bytes_q);

  // This wave's epilogue blocks (code block jb = wave + 4 i) load their factors and low-rank operands now; the
  // loads land while the K loop runs.
  constexpr int kMine = (kJB + kSfWaves - 1) / kSfWaves;
  BlockOperands ops[kMine];
#pragma unroll
  for (int i = 0; i < kMine; ++i)
    if (wave + kSfWaves * i < kJB)
      block_load(ops[i], 32 * (wave + kSfWaves * i), n0, sx, sw, u, ldu, up, ldup, r, bias, M, GLU ? N : n_end, GLU,
                 glu_half, glu_gate_first, lane);

  // Stage t -> slot t % kD. Load j of this wave fills 1 KiB block b = kLoads * wave + j of the stage: blocks 0-3 are
  // the 32 weight rows, the rest the code rows. Stages past K read zeros, so every stage issues the same loads.
  const int nst = (K + kSfStageK - 1) / kSfStageK;
  auto issue = [&](int t) {
    unsigned char HF_LDS* st = smem + (t % kD) * kStage;
    const int k0 = t * kSfStageK;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int bb = kLoads * wave + j;
      const int piece = bb / kPieceLoads, b = bb % kPieceLoads;
      const bool isq = b >= 4;
      const int blk = isq ? b - 4 : b;
      const int row = 8 * blk + (lane >> 3);
      const int c = (lane & 7) ^ skinny_swz(row);
      const int64_t ld = isq ? ldq : ldw;
      const int rows_valid = isq ? M : rows_n;
      const uint32_t oob = isq ? bytes_q : bytes_w;
      const int src = (GLU && !isq) ? glu_row(n0 + 8 * blk, glu_half, glu_gate_first) + (lane >> 3) : row;
      const int kp = k0 + 128 * piece;
      const uint32_t voff = ((row < rows_valid) & (kp + c * 16 < K)) ? (uint32_t)(src * ld + kp + c * 16) : oob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(isq ? rq : rw,
                                               (void HF_LDS*)(st + piece * sf_piece_bytes(MR) + b * 1024), 16, voff,
                                               0, 0, 0);
    }
  };

  v16i acc[kJB];
#pragma unroll
  for (int jb = 0; jb < kJB; ++jb) acc[jb] = (v16i){0};
#pragma unroll
  for (int t = 0; t < kD - 1; ++t) issue(t);
  // Wave w multiplies K step w of every stage: logical chunks 2w and 2w + 1 (lane half h reads chunk 2w + h).
  const int chunk = 2 * wave + half;
  // Stage t has landed for this wave once only the next kD - 2 stages' loads are outstanding.
  constexpr int kWaitVm = (kD - 2) * kLoads;
  for (int t = 0; t < nst; ++t) {
    // Every wave's share of stage t has landed; every wave is done with stage t - 1's slot, which stage t + kD - 1
    // refills.
    static_assert(kWaitVm == 18, "the wait count below");
    asm volatile("s_waitcnt vmcnt(18) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    issue(t + kD - 1);
    const unsigned char HF_LDS* stg = smem + (t % kD) * kStage;
#pragma unroll
    for (int piece = 0; piece < kSfSub; ++piece) {
      const unsigned char HF_LDS* st = stg + piece * sf_piece_bytes(MR);
      const v4i wf = *(const v4i HF_LDS*)(st + sub * 128 + ((chunk ^ skinny_swz(sub)) << 4));
#pragma unroll
      for (int jb = 0; jb < kJB; ++jb) {
        const int qrow = jb * 32 + sub;
        const v4i qf = *(const v4i HF_LDS*)(st + 4096 + qrow * 128 + ((chunk ^ skinny_swz(qrow)) << 4));
        acc[jb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(wf, qf, acc[jb], 0, 0, 0);
      }
    }
  }
  // The zero-fill loads past K may still be landing; then the ring is free for the reduction.
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // Each wave's partial sums, block by block: value v of lane l of block jb at int (((wave * kJB + jb) * 16 + v) * 64
  // + l), so a wave's writes and reads of one value are 64 consecutive ints.
  int HF_LDS* red = (int HF_LDS*)smem;
#pragma unroll
  for (int jb = 0; jb < kJB; ++jb)
#pragma unroll
    for (int v = 0; v < 16; ++v) red[((wave * kJB + jb) * 16 + v) * 64 + lane] = acc[jb][v];
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int i = 0; i < kMine; ++i) {
    const int jb = wave + kSfWaves * i;
    if (jb >= kJB) break;
    int32_t sums[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      int s = 0;
#pragma unroll
      for (int wv = 0; wv < kSfWaves; ++wv) s += red[((wv * kJB + jb) * 16 + v) * 64 + lane];
      sums[v] = s;
    }
    block_finish(ops[i], sums, 32 * jb, n0, u, ldu, up, ldup, r, bias, y, ldy, M, GLU ? N : n_end, vec, act,
                 glu_half, glu_gate_first, lane);
  }
}

#define HF_SF_INSTANTIATE(MR, GLU)                                                                                    \
  template __global__ void skinny_fused_kernel<MR, GLU>(const int8_t*, int64_t, const int8_t*, int64_t,              \
                                                        const float*, const float*, const uint16_t*, int64_t,       \
                                                        const uint16_t*, int64_t, int, const uint16_t*, uint16_t*,  \
                                                        int64_t, int, int, int, int, int, int, int, int);
HF_SF_INSTANTIATE(64, false) HF_SF_INSTANTIATE(64, true)
#undef HF_SF_INSTANTIATE

}  // namespace hf
