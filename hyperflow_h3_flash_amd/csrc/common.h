// Shared device helpers for the convrot kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hf {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned int v4u __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

#define HF_LDS __attribute__((address_space(3)))

// bf16 bit pattern -> fp32 (exact).
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }

// fp32 -> bf16 bits, round to nearest even, NaN kept quiet (torch's `.to(torch.bfloat16)`).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : r;
}

// Two fp32 -> packed bf16 pair (lo, hi) with gfx950's v_cvt_pk_bf16_f32: round to nearest even, NaN kept quiet.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2){lo, hi}, b2));
}

// Output activations a GEMM epilogue can apply to the bf16-rounded linear output (the input of the reference's
// activation module is the bf16 linear output, so the value is rounded once before the activation and once after).
constexpr int kActNone = 0;
constexpr int kActGeluTanh = 1;
constexpr int kActSwiGLU = 2;  // the output is hidden * silu(gate) of column pairs (see glu_row)

// tanh-approximate GELU in fp32, torch's `gelu(approximate="tanh")` formula: 0.5 x (1 + tanh(u)) with
// u = sqrt(2/pi) (x + 0.044715 x^3). tanh(u) = 1 - 2 / (exp(2u) + 1) from the hardware exp2 and reciprocal
// (absolute error of tanh ~1e-7, the rounding error of fp32 near 1); exp2 saturates to 0 or inf, giving -1 or 1.
__device__ __forceinline__ float gelu_tanh(float x) {
  constexpr float kTwoBetaLog2e = 2.0f * 0.7978845608028654f * 1.4426950408889634f;  // 2 sqrt(2/pi) log2(e)
  const float p = fmaf(0.044715f * x, x, 1.0f);                                       // 1 + 0.044715 x^2
  const float e = __builtin_amdgcn_exp2f((x * p) * kTwoBetaLog2e);                    // exp(2u)
  const float t = fmaf(-2.0f, __builtin_amdgcn_rcpf(e + 1.0f), 1.0f);                 // tanh(u)
  return (0.5f * x) * (1.0f + t);
}

// Gated-linear-unit weights (2F rows: F "hidden" rows and F "gate" rows, the feed-forward's SwiGLU projection) are
// multiplied in pair order: GEMM column n uses weight row glu_row(n). Within each 32 columns come 16 hidden rows and
// then the 16 gate rows of the same outputs, so in the 32x32 MFMA layout one lane holds both columns of an output
// (registers v and v + 8, v < 8). gate_first: the weight's first F rows are the gates.
__device__ __forceinline__ int glu_row(int n, int half_n, int gate_first) {
  return ((n >> 5) << 4) + (n & 15) + ((((n >> 4) & 1) ^ gate_first) ? half_n : 0);
}

// fp32 -> the nearest bf16 value (round to nearest even), as a float.
__device__ __forceinline__ float round_bf16(float x) { return bf16_lo(pack_bf16x2(x, x)); }

// SiLU in fp32, torch's formula x / (1 + exp(-x)). exp(-x) comes from the hardware exp2 (inf below x = -88.7, as
// fp32 exp overflows there, giving -0). The quotient is the hardware reciprocal's product refined by one residual
// step, q - (q d - x) / d (Markstein's correction; this sign arrangement keeps silu(-0) = -0), which rounds as the
// IEEE division does in all but rare cases: the bare product is off by one fp32 ulp often enough to move bf16
// roundings. The reciprocal of d > 2^100 is taken of d 2^-100 and the quotient scaled back (exact powers of two),
// so values of 1 / d below the normal range are not flushed to zero.
__device__ __forceinline__ float silu(float x) {
  const float e = __builtin_amdgcn_exp2f(x * -1.4426950408889634f);
  const float d = 1.0f + e;
  const bool big = e > 0x1p100f;
  const float ds = big ? d * 0x1p-100f : d;
  const float r = __builtin_amdgcn_rcpf(ds);
  float q = x * r;
  const float refined = fmaf(-fmaf(q, ds, -x), r, q);
  q = __builtin_fabsf(q) < __builtin_inff() ? refined : q;  // x = inf: the residual is NaN, the product is the value
  q = big ? q * 0x1p-100f : q;
  return e == __builtin_inff() ? x * 0.0f : q;
}

// The reference's SwiGLU on bf16 tensors: bf16(h * bf16(silu(g))) of the bf16 linear outputs h and g.
__device__ __forceinline__ float swiglu(float h_bf16, float g_bf16) {
  return round_bf16(h_bf16 * round_bf16(silu(g_bf16)));
}

// The activation of a packed bf16 pair, rounded back to a packed bf16 pair.
template <int ACT>
__device__ __forceinline__ uint32_t activate_bf16x2(uint32_t pair) {
  if constexpr (ACT == kActGeluTanh) return pack_bf16x2(gelu_tanh(bf16_lo(pair)), gelu_tanh(bf16_hi(pair)));
  return pair;
}

// Rounds an fp64 value to 8 significant bits (bf16 precision) with round-to-nearest-even, once, and returns it as
// fp32 (exact: 8 significant bits; inf beyond the fp32 range). Adding c = +-2^(e + 45) (the value's sign and binade
// e, from its high word) leaves the sum in binade e + 45, whose unit in the last place is 2^(e - 7), so the fp64 add
// rounds the value to 8 significant bits, ties to even; subtracting c again is exact. A zero input gives +0 (c is a
// tiny normal number). Two fp64 adds and two integer operations in place of the bit-level rounding (sticky bit,
// carry, mask: five), checked identical to it on 2e7 random and tie-valued inputs.
__device__ __forceinline__ float round_f64_to_bf16_value(double t) {
  const uint32_t hi = (uint32_t)((unsigned long long)__double_as_longlong(t) >> 32);
  const double c = __longlong_as_double((long long)((unsigned long long)((hi & 0xfff00000u) + (45u << 20)) << 32));
  return (float)((t + c) - c);
}

// Wave-level exchange through LDS: make this wave's LDS writes visible to its own later reads, without a
// workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// LDS row swizzles (16-byte chunk c of row r is stored at chunk c ^ f(r)). gfx950's LDS serves a ds_read_b128 16
// lanes per cycle from 64 banks (256 bytes), so the rows read in one cycle must land on distinct 16-byte slots of a
// 256-byte window; both swizzles also keep any 8 consecutive rows distinct within a 128-byte window. Measured: the
// simpler c ^ ((r >> 1) & 3) for 64-byte rows stalled every fragment read on a 2-way bank conflict.
__device__ __forceinline__ int swizzle64(int r, int c) {  // 64-byte rows: 4 chunks
  return c ^ ((((r >> 1) ^ (r >> 3)) & 1) | ((r >> 1) & 2));
}
__device__ __forceinline__ int swizzle128(int r, int c) {  // 128-byte rows: 8 chunks
  return c ^ ((r ^ (r >> 3)) & 7);
}

// Split-K partial planes are stored block by block: the int32 accumulators of the 32 x 32 block (bm, bn) of a plane
// with nbn = ceil(N / 32) block columns occupy the 1024 ints at (bm * nbn + bn) * 1024, in the layout of
// v_mfma_i32_32x32x32_i8 with the weight as the first operand (lane l: row 32 bm + l % 32; value v: column
// 32 bn + 8 (v / 4) + 4 (l / 32) + v % 4): values 4g .. 4g + 3 of lane l at 256 g + 4 l, so each of a wave's four
// 16-byte stores or loads per block covers 1 KiB of contiguous memory. Blocks past M or N are never read.
__device__ __forceinline__ int64_t partial_block_offset(int bm, int bn, int nbn) {
  return ((int64_t)bm * nbn + bn) * 1024;
}

// A 16-byte store of a result nothing in the same kernel reads again (a GEMM's output tile), with the non-temporal
// hint. Written with the normal policy, a GEMM's output (1 GB at M=32768, N=15360) is allocated in the 256 MiB
// Infinity Cache and displaces the operands (codes and weight, ~250 MB) whose panels every XCD's L2 fetches again
// each round; those fetches then come from HBM. Measured at M=32768, K=5120, N=15360 with the rotation and low-rank
// pass before it: the same number of L2 fetches, their mean latency at the L2's fabric interface ~600 -> ~490
// cycles, MFMA busy 66 -> 69.5 % at the same clock, the layer 2413 -> 2324 us (same box).
__device__ __forceinline__ void store_stream(v4i* dst, v4i v) { __builtin_nontemporal_store(v, dst); }

// Buffer resource for raw (stride 0) buffer loads: offsets at or beyond `bytes` read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

}  // namespace hf
