/*
 * hf_convrot — C ABI of the MI355X (gfx950) INT8 "convrot" linear: a W8A8 linear whose input is rotated by a
 * block-diagonal regular Hadamard matrix and quantized per token.
 *
 * Every entry point takes plain device pointers, element strides (leading dimensions, in elements) and sizes,
 * launches on `stream` (a hipStream_t; NULL is the legacy default stream) of the current HIP device, never
 * synchronizes, never allocates, and returns HF_OK or a negative HF_ERR_* code. Callers own every buffer.
 *
 * bf16 tensors are passed as `uint16_t*` bit patterns. All matrices are row-major with the reduction dimension K
 * contiguous ("NT" GEMM: activations [M, K], weights [N, K]).
 *
 * Reference interfaces replaced (Video-Rebirth/hyperflow-h3-flash, src/hyperflow_h3_flash/):
 *   hf_rotate_quant   <- `_kernels().rotate_quant(x2, group)`              int8.py:326-344 (kernel int8.py:194-221)
 *   hf_int8_linear    <- `_kernels().int8_matmul(a, b, sa, sb)`            int8.py:376-390 (kernel int8.py:283-313)
 *                        extended with the low-rank + bias epilogue of      transformer.py:57-58
 *   hf_lowrank_down   <- `LowRankLinear.down(x)` (bf16 nn.Linear)          transformer.py:57-58
 *   hf_lowrank_up     <- `LowRankLinear.up(u)` (bf16 nn.Linear)            transformer.py:57-58
 *   hf_int8_linear_act_ws <- the FFN up-projection + its activation       transformer.py:75-99
 *   hf_int8_gemm_i32  <- the int32 accumulator of `int8_mm_kernel`         int8.py:302-306 (torch._int_mm, :362)
 *   hf_convrot_linear <- `Int8RotLinear.forward` device branch             int8.py:161-171
 *   hf_convrot_linear_ws <- the same with the shared quantized input,      int8.py:150-171
 *                        the activation, the arithmetic and a workspace
 */
#ifndef HF_CONVROT_H
#define HF_CONVROT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HF_OK 0
#define HF_ERR_ARGUMENT (-1)  /* null pointer, negative size, stride smaller than the row */
#define HF_ERR_GROUP (-2)     /* group is not a power of 4 from 4 to 16384, or does not divide K */
#define HF_ERR_ALIGNMENT (-3) /* a pointer or stride breaks the 16-byte vector-access rules below */
#define HF_ERR_LAUNCH (-4)    /* the HIP launch failed (hipGetLastError) */
#define HF_ERR_SIZE (-5)      /* a size exceeds what the kernels index (see each function) */
#define HF_ERR_SCRATCH (-6)   /* hf_convrot_linear_noalloc: the call needs more than its scratch holds */

typedef void* hf_stream_t; /* hipStream_t */

/* Library version string, e.g. "hf_convrot 0.1.0 gfx950". */
const char* hf_version(void);

/* Human-readable text for a status code. */
const char* hf_strerror(int status);

/*
 * Rotate and quantize activations (one pass over x):
 *   xr = bf16(x[m, g*G:(g+1)*G] @ H_G)   exact sum, rounded once to nearest even   (int8.py:176)
 *   sx[m] = max(max_k |xr[m, k]|, 1e-12) / 127                                    (int8.py:177)
 *   q[m, k] = clamp(rint(xr[m, k] / sx[m]), -127, 127)                             (int8.py:178)
 * x: bf16 [M, ldx]; q: int8 [M, ldq]; sx: fp32 [M].
 * Requires: group a power of 4 from 4 to 16384 dividing K; K % 16 == 0; x and q 16-byte aligned; ldx % 8 == 0;
 * ldq % 16 == 0; K <= 77312, and K <= 20472 for groups of 4096 and more (a row's fp64 sums are held in LDS).
 */
int hf_rotate_quant(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, int64_t M, int64_t K,
                    int32_t group, hf_stream_t stream);

/*
 * hf_rotate_quant with a choice of arithmetic:
 *   HF_ROTATE_BF16_DIV   the reference's torch path above (int8.py:176-178); exactly hf_rotate_quant
 *   HF_ROTATE_F32_RECIP  the reference's GPU kernels (rotate_quant_kernel and rotate_quant_factored_kernel,
 *                        int8.py:194-262, the arithmetic its pipeline runs on CUDA devices):
 *                          xr = fp32(x[m, g*G:(g+1)*G] @ H_G)   exact sum, rounded once to nearest even
 *                          sx[m] = max(max_k |xr[m, k]|, 1e-12) / 127,  inv = 1 / sx[m]   (fp32)
 *                          q[m, k] = clamp(rint(fp32(xr[m, k] * inv)), -127, 127)
 *                        Two passes over each row (the absmax, then the codes), as the reference's kernels do.
 * Same operand rules as hf_rotate_quant (any K below 2^30 for HF_ROTATE_F32_RECIP with groups up to 256); any
 * other arithmetic value is HF_ERR_ARGUMENT. Replaces `rotate_quant(x2, group)` (int8.py:326-344) under the
 * reference's CUDA arithmetic.
 */
#define HF_ROTATE_BF16_DIV 0
#define HF_ROTATE_F32_RECIP 1
int hf_rotate_quant_ex(const uint16_t* x, int64_t ldx, int8_t* q, int64_t ldq, float* sx, int64_t M, int64_t K,
                       int32_t group, int32_t arithmetic, hf_stream_t stream);

/*
 * Low-rank down projection u = bf16(x @ down^T) (LowRankLinear's bf16 intermediate, transformer.py:57-58).
 * x: bf16 [M, ldx]; down: bf16 [r, ld_down] (nn.Linear(K, r).weight); u: bf16 [M, ldu].
 * Requires: K % 16 == 0; x, down 16-byte aligned; ldx % 8 == 0; ld_down % 8 == 0; u 8-byte aligned.
 */
int hf_lowrank_down(const uint16_t* x, int64_t ldx, const uint16_t* down, int64_t ld_down, uint16_t* u,
                    int64_t ldu, int64_t M, int64_t K, int32_t r, hf_stream_t stream);

/*
 * hf_lowrank_down with a caller-provided workspace: with a few hundred to a few thousand rows the kernel splits K
 * across workgroups (fp32 partial sums in `ws`, added in a fixed order and rounded once to bf16); up to 384 rows a
 * workgroup per row and 8 ranks needs no workspace. `hf_lowrank_down_ws_bytes` gives the bytes it uses for these
 * sizes (0: no split); a NULL or smaller workspace runs the unsplit kernel.
 * Replaces the same reference interface as hf_lowrank_down (transformer.py:57-58).
 */
int64_t hf_lowrank_down_ws_bytes(int64_t M, int64_t K, int32_t r);
int hf_lowrank_down_ws(const uint16_t* x, int64_t ldx, const uint16_t* down, int64_t ld_down, uint16_t* u,
                       int64_t ldu, int64_t M, int64_t K, int32_t r, void* ws, int64_t ws_bytes, hf_stream_t stream);

/*
 * Low-rank up projection y = bf16(u @ up^T [+ bias]) (LowRankLinear.up, a bias-free bf16 nn.Linear,
 * transformer.py:57-58; the bias is an extension, NULL for none). Together with hf_lowrank_down this is the whole
 * LowRankLinear forward. fp32 accumulation over the rank, one rounding to bf16 (round to nearest even).
 * u: bf16 [M, ldu]; up: bf16 [N, ld_up] (nn.Linear(r, N).weight); bias: bf16 [N] or NULL; y: bf16 [M, ldy].
 * Requires: r % 8 == 0 (zero-pad the rank: an exact no-op); u and up 16-byte aligned; ldu % 8 == 0;
 * ld_up % 8 == 0; y 2-byte aligned (16-byte aligned with ldy % 8 == 0 for whole-line stores).
 */
int hf_lowrank_up(const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias,
                  uint16_t* y, int64_t ldy, int64_t M, int64_t N, hf_stream_t stream);

/*
 * Fused INT8 linear:
 *   acc = q @ w^T (exact int32)
 *   y = bf16((f32(acc) * sx[m]) * sw[n] + sum_j u[m, j] * up[n, j] + bias[n])
 * With r == 0 and bias == NULL this is bitwise the reference's `bf16((acc * sx) * wscale)` (int8.py:179).
 * q: int8 [M, ldq]; w: int8 [N, ldw] (qweight); sx: fp32 [M]; sw: fp32 [N] (wscale);
 * u: bf16 [M, ldu] or NULL; up: bf16 [N, ld_up] (LowRankLinear.up.weight) or NULL; r: rank (0 = none);
 * bias: bf16 [N] or NULL; y: bf16 [M, ldy].
 * Requires: K % 16 == 0; q, w 16-byte aligned; ldq, ldw multiples of 16; 256 * ldq and 256 * ldw < 2^31; y 8-byte aligned;
 * when r > 0: r % 8 == 0, u and up 16-byte aligned, ldu and ld_up multiples of 8, 512 * ldu and 512 * ld_up < 2^31.
 */
int hf_int8_linear(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx, const float* sw,
                   const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias,
                   uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, hf_stream_t stream);

/*
 * hf_int8_linear with a caller-provided workspace (16-byte aligned): at most 64 rows whose 32-row weight slices fill
 * between a quarter and one round of the CUs run in one pass with no workspace; otherwise, when the output has fewer
 * 256 x 256 tiles than the device has CUs (few rows), K is split across workgroups; their int32 partial accumulators (`ws`) are added
 * exactly and the same epilogue is applied, so the result equals hf_int8_linear's bit for bit. With many tiles
 * whose last round on the CUs would be less than half full and deep K, the trailing tile rows run that way and the
 * rest as whole tiles. `hf_int8_linear_ws_bytes` gives the bytes the call with these sizes, rank and activation
 * uses (0 when its kernels need none: whole tiles, the 256 x 128 tiles, the one-pass few-row kernel); a NULL or
 * smaller workspace runs the unsplit kernel. Replaces the same reference interface as hf_int8_linear (int8.py:376-390).
 */
int64_t hf_int8_linear_ws_bytes(int64_t M, int64_t N, int64_t K, int32_t r, int32_t activation);
int hf_int8_linear_ws(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx, const float* sw,
                      const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up, int32_t r,
                      const uint16_t* bias, uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K, void* ws,
                      int64_t ws_bytes, hf_stream_t stream);

/*
 * hf_int8_linear_ws followed by an output activation: the bf16 output y above goes through `activation` and is
 * rounded to bf16 again, inside the GEMM's epilogue (no extra pass over y):
 *   HF_ACT_NONE       y unchanged (this is hf_int8_linear_ws)
 *   HF_ACT_GELU_TANH  y = bf16(gelu_tanh(y)), gelu_tanh(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))) in fp32
 *   HF_ACT_SWIGLU     gated linear unit: the N weight rows are F = N / 2 "hidden" rows followed by F "gate" rows, and
 *                     the output has F columns, out[m, j] = bf16(y[m, j] * bf16(silu(y[m, F + j]))) with
 *                     silu(g) = g / (1 + exp(-g)) in fp32 (y[m, j], y[m, F + j] the bf16 linear outputs above); ldy
 *                     >= F. N must be a multiple of 32 (else HF_ERR_ARGUMENT), and N * ldw (with r > 0 also
 *                     N * ld_up * 2) must stay below 2^32 bytes (else HF_ERR_SIZE).
 *   HF_ACT_SWIGLU_GATE_FIRST  the same with the gate rows first: out[m, j] = bf16(y[m, F + j] * bf16(silu(y[m, j]))).
 * Replaces the feed-forward's up-projection followed by its activation module (transformer.py:75-99, the FFN `net`
 * run by ChunkedFeedForward: the model's SwiGLU `net[0]`, a linear 2F wide whose output is split in two halves,
 * hidden * silu(gate); torch's `gelu(approximate="tanh")` for a GELU feed-forward). The weight keeps its natural
 * row order: the kernel reads the rows of each hidden/gate pair side by side. Any other activation value is
 * HF_ERR_ARGUMENT.
 */
#define HF_ACT_NONE 0
#define HF_ACT_GELU_TANH 1
#define HF_ACT_SWIGLU 2
#define HF_ACT_SWIGLU_GATE_FIRST 3
int hf_int8_linear_act_ws(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, const float* sx,
                          const float* sw, const uint16_t* u, int64_t ldu, const uint16_t* up, int64_t ld_up,
                          int32_t r, const uint16_t* bias, int32_t activation, uint16_t* y, int64_t ldy, int64_t M,
                          int64_t N, int64_t K, void* ws, int64_t ws_bytes, hf_stream_t stream);
/*
 * The int32 accumulator alone: acc = q @ w^T (for parity checks). acc: int32 [M, ldacc], 16-byte aligned.
 * Same operand rules as hf_int8_linear.
 */
int hf_int8_gemm_i32(const int8_t* q, int64_t ldq, const int8_t* w, int64_t ldw, int32_t* acc, int64_t ldacc,
                     int64_t M, int64_t N, int64_t K, hf_stream_t stream);

/*
 * The whole layer on caller-provided workspaces: hf_rotate_quant into (q_ws [M, K], sx_ws [M]), then, when r > 0,
 * hf_lowrank_down into u_ws [M, r], then hf_int8_linear into y. Same rules as the three calls.
 */
int hf_convrot_linear(const uint16_t* x, int64_t ldx, const int8_t* w, int64_t ldw, const float* sw,
                      const uint16_t* down, int64_t ld_down, const uint16_t* up, int64_t ld_up, int32_t r,
                      const uint16_t* bias, int32_t group, int8_t* q_ws, float* sx_ws, uint16_t* u_ws, uint16_t* y,
                      int64_t ldy, int64_t M, int64_t N, int64_t K, hf_stream_t stream);

/*
 * The whole layer in one call, with the activation, the rotation arithmetic, the split-K workspace and the shared
 * quantized input of `Int8RotLinear.forward` (int8.py:150-171):
 *   quantized == 0: hf_rotate_quant_ex(x -> q [M, K] (ldq = K), sx [M], group, arithmetic);
 *   quantized != 0: q and sx already hold x's codes and scales (the input shared by q/k/v projections,
 *                   int8.py:150-159), and x is read only by the low-rank term;
 * then, when r > 0, hf_lowrank_down_ws(x -> u [M, r] (ldu = r)), then hf_int8_linear_act_ws(q, ..., activation ->
 * y). `ws` serves both split-K passes (one after the other): hf_convrot_linear_ws_bytes gives its size for these
 * sizes, rank and activation (a NULL or smaller workspace runs the unsplit kernels). Same rules as the calls it makes,
 * and the same results bit for bit; when the low-rank projection splits K (quantized == 0, HF_ROTATE_BF16_DIV, r <= 64)
 * it runs before the rotation, whose kernel then adds its partial sums (one launch fewer).
 */
int64_t hf_convrot_linear_ws_bytes(int64_t M, int64_t N, int64_t K, int32_t r, int32_t activation);
int hf_convrot_linear_ws(const uint16_t* x, int64_t ldx, int8_t* q, float* sx, int32_t quantized, int32_t arithmetic,
                         const int8_t* w, int64_t ldw, const float* sw, const uint16_t* down, int64_t ld_down,
                         const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias, int32_t activation,
                         int32_t group, uint16_t* u, uint16_t* y, int64_t ldy, int64_t M, int64_t N, int64_t K,
                         void* ws, int64_t ws_bytes, hf_stream_t stream);

/*
 * hf_convrot_linear_ws without the workspace argument, for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the reference. It allocates
 * nothing: the split-K partial planes and low-rank partial sums live in a 64 MiB scratch array inside the library's
 * code object (hf_convrot_linear_noalloc_max_bytes), one per device, held until the process ends. A call that would
 * need more than that (hf_convrot_linear_ws_bytes(M, N, K, r, activation) > 64 MiB) returns HF_ERR_SCRATCH and launches
 * nothing.
 * Calls on one device share its scratch: calls that overlap on one device (other streams, other host threads) race
 * and must be ordered by the caller. Otherwise exactly hf_convrot_linear_ws with a workspace of the needed size.
 */
int64_t hf_convrot_linear_noalloc_max_bytes(void);
int hf_convrot_linear_noalloc(const uint16_t* x, int64_t ldx, int8_t* q, float* sx, int32_t quantized,
                              int32_t arithmetic, const int8_t* w, int64_t ldw, const float* sw, const uint16_t* down,
                              int64_t ld_down, const uint16_t* up, int64_t ld_up, int32_t r, const uint16_t* bias,
                              int32_t activation, int32_t group, uint16_t* u, uint16_t* y, int64_t ldy, int64_t M,
                              int64_t N, int64_t K, hf_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* HF_CONVROT_H */
