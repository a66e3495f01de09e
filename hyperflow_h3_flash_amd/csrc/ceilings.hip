// Calibration kernels for the benchmark (libhf_ceilings.so): what the matrix cores of this device sustain with no
// memory traffic, so a GEMM's rate can be read against a measured ceiling as well as the published peak. Not part
// of the convrot linear's library or its C ABI.
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

}  // extern "C"
