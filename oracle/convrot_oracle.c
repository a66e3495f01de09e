/*
 * ORACLE — test infrastructure only. Nothing in the product imports, links or runs this file: the tests, the
 * smoke check and bench.py's cpu_baseline leg use it for the reference results the device output is compared with.
 *
 * A plain-C restatement of the reference's CPU arithmetic for the INT8 convrot linear,
 * `Int8RotLinear._forward_torch` (src/hyperflow_h3_flash/int8.py:173-179):
 *
 *   xr  = bf16( x.view(M, K/G, G) @ R )          int8.py:176   (R = regular Hadamard, int8.py:100-109)
 *   sx  = max(absmax_row(xr), 1e-12) / 127.0     int8.py:177   (fp32 true division)
 *   xq  = clamp(round_half_even(xr / sx), ±127)  int8.py:178   (fp32 true division)
 *   acc = xq @ qweight^T                          int8.py:179   (integer-valued; exact int64 here)
 *   y   = bf16((f32(acc) * sx) * wscale)          int8.py:179
 *
 * plus the low-rank branch of LowRankLinear (src/hyperflow_h3_flash/transformer.py:57-58,
 * `up(down(x))` with a bf16 intermediate) and a bias, for the fused extension.
 *
 * The rotation sum is computed EXACTLY (exact products, exact sum) and rounded once to bf16 with
 * round-to-nearest-even. The reference's torch CPU GEMM accumulates in fp32 in an ISA-dependent order; its result
 * equals this one whenever that fp32 accumulation is exact or does not move the sum across a bf16 rounding
 * boundary. The exact sum is the order-independent statement of `bf16(x @ R)`.
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so no multiply-add is fused behind our back).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- bf16 helpers */

static inline float bf16_to_f32(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static inline uint32_t f32_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}

/* fp32 -> bf16, round to nearest even; NaN stays NaN (torch's `.to(torch.bfloat16)`). */
uint16_t oracle_f32_to_bf16(float f) {
  uint32_t u = f32_bits(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* fp64 -> bf16 rounded ONCE to nearest even (no intermediate fp32 rounding). Handles bf16 subnormals
 * (quantum 2^-133), overflow to inf, and NaN. */
uint16_t oracle_f64_to_bf16(double d) {
  if (isnan(d)) return 0x7fc0;
  uint16_t sign = signbit(d) ? 0x8000 : 0;
  double a = fabs(d);
  if (isinf(a)) return sign | 0x7f80;
  if (a == 0.0) return sign;
  int e;
  frexp(a, &e);                   /* a = f * 2^e, f in [0.5, 1) */
  int q = e - 8;                  /* exponent of the last kept bit for 8 significant bits */
  if (q < -133) q = -133;         /* bf16 subnormal quantum */
  double scaled = ldexp(a, -q);   /* exact */
  double r = nearbyint(scaled);   /* round half to even in the default rounding mode */
  double v = ldexp(r, q);         /* exact: at most 9 significant bits, and 2^k when 9 */
  if (v >= 0x1p128) return sign | 0x7f80;
  float f = (float)v;             /* exact: v has <= 8 significant bits and is in range */
  return sign | (uint16_t)(f32_bits(f) >> 16);
}

/* ---------------------------------------------------------------- regular Hadamard, int8.py:100-109 */

/* Sign of H[i][j] for H = kron(H4/2, ..., H4/2) with H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]:
 * the H4 entry at (a, b) is -1 exactly when a + b == 3, and the Kronecker product multiplies the entries of the
 * base-4 digits of i and j. Magnitude is 2^-n for G = 4^n. */
static inline int hadamard_negative(int i, int j, int n) {
  int neg = 0;
  for (int t = 0; t < n; ++t) {
    neg ^= (((i >> (2 * t)) & 3) + ((j >> (2 * t)) & 3)) == 3;
  }
  return neg;
}

/* Dense G x G regular Hadamard in float64 (for the tests' closed-form checks). Returns -1 if G is not 4^n. */
int oracle_regular_hadamard(int G, double* out) {
  int n = 0;
  while ((1 << (2 * n)) < G) ++n;
  if ((1 << (2 * n)) != G) return -1;
  double mag = ldexp(1.0, -n);
  for (int i = 0; i < G; ++i)
    for (int j = 0; j < G; ++j) out[(int64_t)i * G + j] = hadamard_negative(i, j, n) ? -mag : mag;
  return 0;
}

/* ---------------------------------------------------------------- exact sums */

/* A 320-bit two's-complement fixed-point accumulator whose least significant bit is 2^-160. Every finite bf16
 * value times 2^-n (n <= 12) is an integer multiple of 2^-145 below 2^129, so sums of up to 2^20 such terms are
 * exact. */
#define ACC_LIMBS 5
#define ACC_LSB_EXP (-160)

typedef struct {
  uint64_t w[ACC_LIMBS];
} superacc;

static void acc_add_term(superacc* a, uint32_t mant, int exp2, int negative) {
  /* adds (-1)^negative * mant * 2^exp2, mant < 2^9 */
  int pos = exp2 - ACC_LSB_EXP;
  int limb = pos >> 6, sh = pos & 63;
  uint64_t lo = (uint64_t)mant << sh;
  uint64_t hi = sh ? ((uint64_t)mant >> (64 - sh)) : 0;
  uint64_t t[ACC_LIMBS] = {0};
  t[limb] = lo;
  if (limb + 1 < ACC_LIMBS) t[limb + 1] = hi;
  if (negative) { /* two's complement negate t */
    int carry = 1;
    for (int k = 0; k < ACC_LIMBS; ++k) {
      uint64_t v = ~t[k] + (uint64_t)carry;
      carry = carry && (v == 0);
      t[k] = v;
    }
  }
  unsigned __int128 c = 0;
  for (int k = 0; k < ACC_LIMBS; ++k) {
    c += (unsigned __int128)a->w[k] + t[k];
    a->w[k] = (uint64_t)c;
    c >>= 64;
  }
}

/* Round the exact accumulator value to a float with `bits` significant bits (8: bf16, 24: fp32), nearest even,
 * with the subnormal quantum 2^qmin_exp; returns the rounded value (exact in a double) or +-inf past 2^128. */
static double acc_round(const superacc* a, int bits, int qmin_exp) {
  uint64_t m[ACC_LIMBS];
  memcpy(m, a->w, sizeof m);
  int negative = (int64_t)m[ACC_LIMBS - 1] < 0;
  if (negative) {
    int carry = 1;
    for (int k = 0; k < ACC_LIMBS; ++k) {
      uint64_t v = ~m[k] + (uint64_t)carry;
      carry = carry && (v == 0);
      m[k] = v;
    }
  }
  int top = -1;
  for (int k = ACC_LIMBS - 1; k >= 0 && top < 0; --k)
    if (m[k]) top = k * 64 + 63 - __builtin_clzll(m[k]);
  if (top < 0) return 0.0; /* an exact zero sum is +0 */
  int q = top - (bits - 1);
  int qmin = qmin_exp - ACC_LSB_EXP;
  if (q < qmin) q = qmin;
#define BIT(i) ((i) < 0 ? 0u : (unsigned)((m[(i) >> 6] >> ((i) & 63)) & 1u))
  uint64_t kept = 0;
  for (int b = top; b >= q; --b) kept = (kept << 1) | BIT(b);
  unsigned round = BIT(q - 1);
  unsigned sticky = 0;
  for (int b = q - 2; b >= 0 && !sticky; --b) sticky = BIT(b);
#undef BIT
  if (round && (sticky || (kept & 1))) kept += 1;
  double v = ldexp((double)kept, q + ACC_LSB_EXP);
  if (v >= 0x1p128) v = INFINITY;
  return negative ? -v : v;
}

/* Round the exact accumulator value to bf16, nearest even. */
static uint16_t acc_to_bf16(const superacc* a) {
  uint64_t m[ACC_LIMBS];
  memcpy(m, a->w, sizeof m);
  int negative = (int64_t)m[ACC_LIMBS - 1] < 0;
  if (negative) {
    int carry = 1;
    for (int k = 0; k < ACC_LIMBS; ++k) {
      uint64_t v = ~m[k] + (uint64_t)carry;
      carry = carry && (v == 0);
      m[k] = v;
    }
  }
  int top = -1;
  for (int k = ACC_LIMBS - 1; k >= 0 && top < 0; --k)
    if (m[k]) top = k * 64 + 63 - __builtin_clzll(m[k]);
  uint16_t sign = negative ? 0x8000 : 0;
  if (top < 0) return 0; /* an exact zero sum is +0, as x + (-x) is in IEEE arithmetic */
  int q = top - 7;                         /* bit index of the last kept bit */
  int qmin = -133 - ACC_LSB_EXP;           /* bf16 subnormal quantum 2^-133 */
  if (q < qmin) q = qmin;
#define BIT(i) ((i) < 0 ? 0u : (unsigned)((m[(i) >> 6] >> ((i) & 63)) & 1u))
  uint64_t kept = 0;
  for (int b = top; b >= q; --b) kept = (kept << 1) | BIT(b);
  unsigned round = BIT(q - 1);
  unsigned sticky = 0;
  for (int b = q - 2; b >= 0 && !sticky; --b) sticky = BIT(b);
#undef BIT
  if (round && (sticky || (kept & 1))) kept += 1;
  double v = ldexp((double)kept, q + ACC_LSB_EXP);
  if (v >= 0x1p128) return sign | 0x7f80;
  float f = (float)v;
  return sign | (uint16_t)(f32_bits(f) >> 16);
}

/* bf16 bits -> (mantissa, exponent) with value = mant * 2^exp, mant < 2^8. Returns 0 for zero, -1 for inf/nan. */
static inline int bf16_decompose(uint16_t b, uint32_t* mant, int* exp2, int* negative) {
  uint32_t e = (b >> 7) & 0xff, f = b & 0x7f;
  *negative = b >> 15;
  if (e == 0xff) return -1;
  if (e == 0) {
    if (f == 0) return 0;
    *mant = f;
    *exp2 = -133;
    return 1;
  }
  *mant = f | 0x80;
  *exp2 = (int)e - 127 - 7;
  return 1;
}

/* ---------------------------------------------------------------- the rotation, int8.py:176 */

/* xr[m, g*G + j] = bf16( sum_i x[m, g*G + i] * H[i][j] ), summed exactly. force_exact=1 always uses the 320-bit
 * accumulator; otherwise a group whose nonzero inputs span at most 32 binades is summed in float64, which is exact
 * there (every term is a multiple of 2^(emin-n) below 2^(emax+1), partial sums of <= 4096 terms need at most
 * span + 21 <= 53 bits). */
int oracle_rotate(const uint16_t* x, int64_t M, int64_t K, int G, uint16_t* xr, int force_exact) {
  int n = 0;
  while ((1 << (2 * n)) < G) ++n;
  if ((1 << (2 * n)) != G || K % G) return -1;
  char* neg = (char*)malloc((size_t)G * G);
  for (int i = 0; i < G; ++i)
    for (int j = 0; j < G; ++j) neg[(size_t)i * G + j] = (char)hadamard_negative(i, j, n);
  double* xd = (double*)malloc(sizeof(double) * G);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t g0 = 0; g0 < K; g0 += G) {
      const uint16_t* xg = x + m * K + g0;
      int emin = 1 << 20, emax = -(1 << 20), nonfinite = 0;
      for (int i = 0; i < G; ++i) {
        uint32_t mt;
        int ex, ng;
        int kind = bf16_decompose(xg[i], &mt, &ex, &ng);
        if (kind < 0) nonfinite = 1;
        if (kind > 0) {
          if (ex < emin) emin = ex;
          if (ex > emax) emax = ex;
        }
        xd[i] = (double)bf16_to_f32(xg[i]);
      }
      int fast = !force_exact && (nonfinite || emax - emin <= 32);
      for (int j = 0; j < G; ++j) {
        if (fast) {
          double s = 0.0;
          for (int i = 0; i < G; ++i) s += neg[(size_t)i * G + j] ? -xd[i] : xd[i];
          xr[m * K + g0 + j] = oracle_f64_to_bf16(ldexp(s, -n));
        } else {
          superacc a;
          memset(&a, 0, sizeof a);
          for (int i = 0; i < G; ++i) {
            uint32_t mt;
            int ex, ng;
            if (bf16_decompose(xg[i], &mt, &ex, &ng) <= 0) continue;
            acc_add_term(&a, mt, ex - n, ng ^ neg[(size_t)i * G + j]);
          }
          xr[m * K + g0 + j] = acc_to_bf16(&a);
        }
      }
    }
  }
  free(xd);
  free(neg);
  return 0;
}

/* The reference's GPU kernels' rotation (rotate_quant_kernel and rotate_quant_factored_kernel, int8.py:194-262):
 * the same exact sum, rounded once to fp32 instead of bf16 (their fp32 dot products; the factored kernel's 3-term
 * bf16 split makes its second product exact). */
int oracle_rotate_f32(const uint16_t* x, int64_t M, int64_t K, int G, float* xr, int force_exact) {
  int n = 0;
  while ((1 << (2 * n)) < G) ++n;
  if ((1 << (2 * n)) != G || K % G) return -1;
  char* neg = (char*)malloc((size_t)G * G);
  for (int i = 0; i < G; ++i)
    for (int j = 0; j < G; ++j) neg[(size_t)i * G + j] = (char)hadamard_negative(i, j, n);
  double* xd = (double*)malloc(sizeof(double) * G);
  for (int64_t m = 0; m < M; ++m) {
    for (int64_t g0 = 0; g0 < K; g0 += G) {
      const uint16_t* xg = x + m * K + g0;
      int emin = 1 << 20, emax = -(1 << 20), nonfinite = 0;
      for (int i = 0; i < G; ++i) {
        uint32_t mt;
        int ex, ng;
        int kind = bf16_decompose(xg[i], &mt, &ex, &ng);
        if (kind < 0) nonfinite = 1;
        if (kind > 0) {
          if (ex < emin) emin = ex;
          if (ex > emax) emax = ex;
        }
        xd[i] = (double)bf16_to_f32(xg[i]);
      }
      int fast = !force_exact && (nonfinite || emax - emin <= 32);
      for (int j = 0; j < G; ++j) {
        if (fast) {
          double s = 0.0;
          for (int i = 0; i < G; ++i) s += neg[(size_t)i * G + j] ? -xd[i] : xd[i];
          xr[m * K + g0 + j] = (float)ldexp(s, -n); /* the exact sum, rounded once */
        } else {
          superacc a;
          memset(&a, 0, sizeof a);
          for (int i = 0; i < G; ++i) {
            uint32_t mt;
            int ex, ng;
            if (bf16_decompose(xg[i], &mt, &ex, &ng) <= 0) continue;
            acc_add_term(&a, mt, ex - n, ng ^ neg[(size_t)i * G + j]);
          }
          xr[m * K + g0 + j] = (float)acc_round(&a, 24, -149);
        }
      }
    }
  }
  free(xd);
  free(neg);
  return 0;
}

/* The GPU kernels' quantization (int8.py:208-220): scale = max(amax, 1e-12) / 127 and inv = 1 / scale in fp32,
 * q = clamp(rint(fp32(v * inv)), -127, 127) (a reciprocal multiply, not a division). */
void oracle_quantize_recip(const float* xr, int64_t M, int64_t K, float* sx, int8_t* xq) {
  for (int64_t m = 0; m < M; ++m) {
    const float* row = xr + m * K;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float v = fabsf(row[k]);
      if (v > amax || isnan(v)) amax = v;
    }
    float s = (amax > 1e-12f ? amax : 1e-12f) / 127.0f; /* tl.maximum(amax, 1e-12) / 127.0 */
    float inv = 1.0f / s;
    sx[m] = s;
    for (int64_t k = 0; k < K; ++k) {
      float t = row[k] * inv;
      float r = rintf(t);
      if (r < -127.0f) r = -127.0f;
      if (r > 127.0f) r = 127.0f;
      xq[m * K + k] = (int8_t)r;
    }
  }
}

/* ---------------------------------------------------------------- per-token quantization, int8.py:177-178 */

void oracle_quantize(const uint16_t* xr, int64_t M, int64_t K, float* sx, int8_t* xq) {
  for (int64_t m = 0; m < M; ++m) {
    const uint16_t* row = xr + m * K;
    float amax = 0.0f;
    for (int64_t k = 0; k < K; ++k) {
      float v = fabsf(bf16_to_f32(row[k]));
      if (v > amax || isnan(v)) amax = v;
    }
    float s = (amax < 1e-12f ? 1e-12f : amax) / 127.0f; /* clamp_min(1e-12) then a true fp32 division */
    sx[m] = s;
    for (int64_t k = 0; k < K; ++k) {
      float t = bf16_to_f32(row[k]) / s;          /* true division, like torch's CPU div */
      float r = rintf(t);                         /* round half to even (torch.round) */
      if (r < -127.0f) r = -127.0f;
      if (r > 127.0f) r = 127.0f;
      xq[m * K + k] = (int8_t)r;
    }
  }
}

/* ---------------------------------------------------------------- int8 GEMM and epilogue, int8.py:179 */

/* acc[m, n] = sum_k xq[m, k] * w[n, k], exactly (int64), stored as int32. Returns -1 if a sum leaves int32. */
int oracle_int8_gemm(const int8_t* xq, const int8_t* w, int64_t M, int64_t N, int64_t K, int32_t* acc) {
  int status = 0;
  for (int64_t m = 0; m < M; ++m) {
    const int8_t* a = xq + m * K;
    for (int64_t n = 0; n < N; ++n) {
      const int8_t* b = w + n * K;
      int64_t s = 0;
      for (int64_t k = 0; k < K; ++k) s += (int64_t)a[k] * (int64_t)b[k];
      if (s > INT32_MAX || s < INT32_MIN) status = -1;
      acc[m * N + n] = (int32_t)s;
    }
  }
  return status;
}

/* y = bf16((f32(acc) * sx) * wscale): two separately rounded fp32 products, then round to bf16. */
void oracle_epilogue(const int32_t* acc, const float* sx, const float* ws, int64_t M, int64_t N, uint16_t* y) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float v = (float)acc[m * N + n];
      v = v * sx[m];
      v = v * ws[n];
      y[m * N + n] = oracle_f32_to_bf16(v);
    }
}

/* ---------------------------------------------------------------- low-rank branch, transformer.py:57-58 */

/* u[m, j] = bf16(sum_k x[m, k] * down[j, k]) — nn.Linear(K, r) in bf16, summed in float64 and rounded once. */
void oracle_lowrank_down(const uint16_t* x, const uint16_t* down, int64_t M, int64_t K, int64_t r, uint16_t* u) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t j = 0; j < r; ++j) {
      double s = 0.0;
      for (int64_t k = 0; k < K; ++k) s += (double)bf16_to_f32(x[m * K + k]) * (double)bf16_to_f32(down[j * K + k]);
      u[m * r + j] = oracle_f64_to_bf16(s);
    }
}

/* Fused extension: y = bf16( (f32(acc)*sx)*ws + sum_j u[m,j]*up[n,j] + bias[n] ) with one final rounding to bf16.
 * The sum is an fp32 sum (the extension's definition; the composition Int8RotLinear(x) + LowRankLinear(x) + bias of
 * transformer.py:57-58 rounds to bf16 after every term instead). With a low-rank term (r > 0) the order of the fp32
 * additions is unspecified, so the oracle takes the exact sum (float64) and device results are held to one bf16 ulp
 * of it; with the bias alone the sum is the single fp32 addition fl32(v + bias), then one rounding to bf16.
 * up is [N, r] (LowRankLinear.up.weight); bias may be NULL, u/up NULL when r == 0. */
void oracle_fused_epilogue(const int32_t* acc, const float* sx, const float* ws, const uint16_t* u,
                           const uint16_t* up, int64_t r, const uint16_t* bias, int64_t M, int64_t N, uint16_t* y) {
  for (int64_t m = 0; m < M; ++m)
    for (int64_t n = 0; n < N; ++n) {
      float v = (float)acc[m * N + n];
      v = v * sx[m];
      v = v * ws[n];
      if (r == 0) {
        if (bias) v = v + bf16_to_f32(bias[n]);
        y[m * N + n] = oracle_f32_to_bf16(v);
        continue;
      }
      double s = (double)v;
      for (int64_t j = 0; j < r; ++j) s += (double)bf16_to_f32(u[m * r + j]) * (double)bf16_to_f32(up[n * r + j]);
      if (bias) s += (double)bf16_to_f32(bias[n]);
      y[m * N + n] = oracle_f64_to_bf16(s);
    }
}

/* ---------------------------------------------------------------- whole layer */

/* The reference layer end to end (bias-free, no low-rank): x bf16 [M,K], w int8 [N,K], ws fp32 [N] -> y bf16
 * [M,N], with the intermediates written when their pointers are non-NULL. */
int oracle_convrot_linear(const uint16_t* x, const int8_t* w, const float* ws, int64_t M, int64_t N, int64_t K,
                          int G, uint16_t* y, uint16_t* xr_out, float* sx_out, int8_t* xq_out, int32_t* acc_out) {
  uint16_t* xr = xr_out ? xr_out : (uint16_t*)malloc(sizeof(uint16_t) * M * K);
  float* sx = sx_out ? sx_out : (float*)malloc(sizeof(float) * M);
  int8_t* xq = xq_out ? xq_out : (int8_t*)malloc((size_t)(M * K));
  int32_t* acc = acc_out ? acc_out : (int32_t*)malloc(sizeof(int32_t) * M * N);
  int status = oracle_rotate(x, M, K, G, xr, 0);
  if (status == 0) {
    oracle_quantize(xr, M, K, sx, xq);
    status = oracle_int8_gemm(xq, w, M, N, K, acc);
    oracle_epilogue(acc, sx, ws, M, N, y);
  }
  if (!xr_out) free(xr);
  if (!sx_out) free(sx);
  if (!xq_out) free(xq);
  if (!acc_out) free(acc);
  return status;
}
