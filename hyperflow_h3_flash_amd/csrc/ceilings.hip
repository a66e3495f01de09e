// Calibration kernels for the benchmark (libhf_ceilings.so): what the matrix cores of this device sustain with no
// memory traffic, and what HBM sustains for a streaming pass, so a kernel's rate can be read against a measured
// ceiling as well as the published peak. Not part of the convrot linear's library or its C ABI.
//
// mfma_i8_ceiling_kernel: 512-thread workgroups (8 waves, two per SIMD, the INT8 GEMM's layout), each wave issuing
// `rounds` x 8 independent v_mfma_i32_32x32x32_i8 (8 accumulators of 16 registers, the GEMM's 128). The operands
// come from a 512 x 16-byte table the caller fills (zeros, uniform codes, ...): the toggling of the operand bits sets
// the clock the chip can hold, so the table's values matter. Each lane writes the xor of its accumulators so the
// MFMAs cannot be dropped. Multiply-adds per launch: grid x 8 waves x rounds x 8 x 32768.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8;
constexpr int kAcc = 8;
constexpr int kTableEntries = 512;  // 16-byte operand entries in the caller's table (8 KiB)

__global__ __launch_bounds__(64 * kWaves) void mfma_i8_ceiling_kernel(const v4i* __restrict__ table, int rounds,
                                                                        int32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  v4i w[2], a[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) w[i] = table[i * 64 + lane];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = table[128 + i * 64 + lane];
  v16i acc[kAcc];
#pragma unroll
  for (int i = 0; i < kAcc; ++i) acc[i] = (v16i){0};
  for (int it = 0; it < rounds; ++it) {
#pragma unroll
    for (int i = 0; i < kAcc; ++i) acc[i] = __builtin_amdgcn_mfma_i32_32x32x32_i8(w[i & 1], a[i >> 1], acc[i], 0, 0, 0);
  }
  int32_t fold = 0;
#pragma unroll
  for (int i = 0; i < kAcc; ++i)
#pragma unroll
    for (int j = 0; j < 16; ++j) fold ^= acc[i][j];
  out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = fold;
}

// stream_kernel<R, W, U>: the bandwidth HBM sustains for a streaming pass, to read the memory-bound kernels
// against. Work is counted in units of one 16-byte vector per lane: unit i of wave-group g = i / 64 reads R vectors
// src[(g R + r) 64 + i % 64] (each load instruction of a wave covers 1 KiB of consecutive bytes) and writes W
// vectors dst[(g W + w) 64 + i % 64] (the xor of the unit's loads), so a launch moves units x 16 x (R + W) bytes.
// R = 2, W = 1 is the rotation pass's ratio (2 bytes of bf16 read per byte of int8 written); R = 2, W = 0 the
// low-rank projection's (x read, almost nothing written: each lane's xor goes to `out` once). Each thread takes U
// units per round (all U x R loads issued before the first use), rounds striding over the whole grid. Loads and
// stores carry the non-temporal hint: the streams are touched once.
template <int R, int W, int U>
__global__ __launch_bounds__(256) void stream_kernel(const v4i* __restrict__ src, v4i* __restrict__ dst,
                                                     int64_t units, int32_t* __restrict__ out) {
  const int64_t threads = (int64_t)gridDim.x * blockDim.x;
  const int64_t first = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int lane = threadIdx.x & 63;
  v4i fold = (v4i){0};
  for (int64_t base = first; base < units; base += threads * U) {
    v4i v[U][R];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * threads;
      const int64_t g = i >> 6;
#pragma unroll
      for (int r = 0; r < R; ++r)
        v[u][r] = i < units ? __builtin_nontemporal_load(src + ((g * R + r) << 6) + lane) : (v4i){0};
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = base + (int64_t)u * threads;
      const int64_t g = i >> 6;
      v4i x = v[u][0];
#pragma unroll
      for (int r = 1; r < R; ++r) x ^= v[u][r];
      if constexpr (W > 0) {
        if (i < units) {
#pragma unroll
          for (int w = 0; w < W; ++w) __builtin_nontemporal_store(x, dst + ((g * W + w) << 6) + lane);
        }
      } else {
        fold ^= x;
      }
    }
  }
  if constexpr (W == 0) out[first] = fold[0] ^ fold[1] ^ fold[2] ^ fold[3];
}

}  // namespace

extern "C" {

// Launches `grid` workgroups of the INT8 MFMA ceiling kernel on `stream`. table: 8 KiB of int8 operands (512
// entries of 16 bytes; entries 0-127 feed the first MFMA operand, 128-383 the second); out: grid x 512 int32.
// Returns 0, -1 for a bad argument, -4 when the launch fails.
int hf_ceiling_mfma_i8(const void* table, int32_t rounds, int32_t grid, int32_t* out, hipStream_t stream) {
  static_assert(128 + 4 * 64 <= kTableEntries, "operand entries past the table");
  if (!table || !out || rounds < 1 || grid < 1) return -1;
  hipLaunchKernelGGL(mfma_i8_ceiling_kernel, dim3(grid), dim3(64 * kWaves), 0, stream,
                     reinterpret_cast<const v4i*>(table), rounds, out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

// Multiply-adds one launch performs.
int64_t hf_ceiling_mfma_i8_macs(int32_t rounds, int32_t grid) {
  return (int64_t)grid * kWaves * rounds * kAcc * 32 * 32 * 32;
}

// Launches one streaming pass on `stream`: `units` (a multiple of 64) units of `reads` 16-byte loads from src and
// `writes` 16-byte stores to dst (reads, writes) in {(2, 0), (2, 1), (1, 1)}; `unroll` units per thread and round
// (4 or 8); `grid` workgroups of 256 threads; out: grid x 256 int32 (used when writes == 0). src must hold
// units x reads x 16 bytes and dst units x writes x 16. Returns 0, -1 for a bad argument, -4 when the launch fails.
int hf_ceiling_stream(const void* src, void* dst, int64_t units, int32_t reads, int32_t writes, int32_t unroll,
                      int32_t grid, int32_t* out, hipStream_t stream) {
  if (!src || units <= 0 || units % 64 || grid < 1 || (unroll != 4 && unroll != 8)) return -1;
  if (writes > 0 && !dst) return -1;
  if (writes == 0 && !out) return -1;
  const v4i* s = reinterpret_cast<const v4i*>(src);
  v4i* d = reinterpret_cast<v4i*>(dst);
#define HF_STREAM(R, W, U) \
  hipLaunchKernelGGL((stream_kernel<R, W, U>), dim3(grid), dim3(256), 0, stream, s, d, units, out)
  if (reads == 2 && writes == 0) {
    if (unroll == 4) HF_STREAM(2, 0, 4); else HF_STREAM(2, 0, 8);
  } else if (reads == 2 && writes == 1) {
    if (unroll == 4) HF_STREAM(2, 1, 4); else HF_STREAM(2, 1, 8);
  } else if (reads == 1 && writes == 1) {
    if (unroll == 4) HF_STREAM(1, 1, 4); else HF_STREAM(1, 1, 8);
  } else {
    return -1;
  }
#undef HF_STREAM
  return hipGetLastError() == hipSuccess ? 0 : -4;
}

}  // extern "C"
