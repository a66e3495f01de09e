"""ORACLE — test infrastructure only.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this module, and only as
the reference results the device output is compared with (or, in the baseline, as the timed CPU path). The product
(``hyperflow_h3_flash_amd``) never imports it.

A CPU restatement of the reference's INT8 convrot linear (``Int8RotLinear._forward_torch``,
src/hyperflow_h3_flash/int8.py:173-179) backed by ``convrot_oracle.c`` (built by ``oracle/Makefile``), plus the
numpy closed forms the tests pin it with:

* ``regular_hadamard`` — int8.py:100-109 (``kron(H4/2, ...)``, float64);
* ``hadamard_factors`` — int8.py:112-119;
* ``quantize_weight`` — the checkpoint quantizer of tests/test_int8.py:31-36 (float64);
* ``rotate`` / ``quantize`` / ``int8_gemm`` / ``epilogue`` — int8.py:176-179 step by step;
* ``rotate_f32`` / ``quantize_recip`` — the arithmetic of the reference's GPU rotate+quantize kernels
  (int8.py:194-262): the exact rotation rounded to fp32 (not bf16) and a reciprocal multiply (not a division).
  Pinned by exact arithmetic; parity against those CUDA kernels' own outputs is unpinned (no fixture holds them);
* ``lowrank_down`` / ``fused_epilogue`` — LowRankLinear (src/hyperflow_h3_flash/transformer.py:57-58) and a bias;
* ``composition`` — the reference's own composition ``Int8RotLinear(x) + LowRankLinear(x) + bias`` in bf16 tensor
  arithmetic, which is what the fused extension is graded against;
* ``gelu_tanh`` — the feed-forward's activation module on a bf16 tensor (torch's ``gelu(approximate="tanh")``,
  applied to the up-projection output, transformer.py:75-99), in float64 and rounded once;
* ``silu`` / ``swiglu`` — the model's gated feed-forward input module (``ff.net[0]``, run by ChunkedFeedForward,
  transformer.py:75-99; the module itself is diffusers' ``SwiGLU``, a dependency absent from the reference tree):
  the bf16 projection output split in halves, ``hidden * silu(gate)`` in bf16 tensor arithmetic.

Every array crossing into C is a contiguous numpy array; bf16 tensors are carried as ``uint16`` bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from functools import lru_cache

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")


def build() -> str:
    """Compile ``convrot_oracle.c`` with gcc (oracle/Makefile). Returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


@lru_cache(maxsize=None)
def _lib() -> ctypes.CDLL:
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    p, i64, i32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.oracle_regular_hadamard.argtypes = [i32, p]
    lib.oracle_rotate.argtypes = [p, i64, i64, i32, p, i32]
    lib.oracle_quantize.argtypes = [p, i64, i64, p, p]
    lib.oracle_rotate_f32.argtypes = [p, i64, i64, i32, p, i32]
    lib.oracle_quantize_recip.argtypes = [p, i64, i64, p, p]
    lib.oracle_int8_gemm.argtypes = [p, p, i64, i64, i64, p]
    lib.oracle_epilogue.argtypes = [p, p, p, i64, i64, p]
    lib.oracle_lowrank_down.argtypes = [p, p, i64, i64, i64, p]
    lib.oracle_fused_epilogue.argtypes = [p, p, p, p, p, i64, p, i64, i64, p]
    lib.oracle_convrot_linear.argtypes = [p, p, p, i64, i64, i64, i32, p, p, p, p, p]
    lib.oracle_f64_to_bf16.argtypes = [ctypes.c_double]
    lib.oracle_f64_to_bf16.restype = ctypes.c_uint16
    lib.oracle_f32_to_bf16.argtypes = [ctypes.c_float]
    lib.oracle_f32_to_bf16.restype = ctypes.c_uint16
    return lib


def _ptr(a: np.ndarray | None):
    if a is None:
        return None
    assert a.flags.c_contiguous, "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# ----------------------------------------------------------------------------------------------------- bf16 helpers


def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """uint16 bf16 bit patterns -> float32 values (exact)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def f64_to_bf16(x: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bits rounded once (no fp32 double rounding), via the C routine."""
    lib = _lib()
    flat = np.ascontiguousarray(x, dtype=np.float64).ravel()
    out = np.fromiter((lib.oracle_f64_to_bf16(float(v)) for v in flat), dtype=np.uint16, count=flat.size)
    return out.reshape(np.shape(x))


# ------------------------------------------------------------------------------------------- Hadamard closed forms


def regular_hadamard(group: int) -> np.ndarray:
    """``kron(H4/2, ..., H4/2)`` of size ``group`` in float64 (int8.py:100-109). ValueError unless a power of 4."""
    h4 = np.array([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=np.float64) / 2
    h, n = np.ones((1, 1)), 1
    while n < group:
        h, n = np.kron(h, h4), n * 4
    if n != group:
        raise ValueError(f"Hadamard group {group} is not a power of 4")
    return h


def regular_hadamard_c(group: int) -> np.ndarray:
    """The C oracle's sign-rule construction of the same matrix (digit sums of 3 give -1)."""
    out = np.empty((group, group), dtype=np.float64)
    if _lib().oracle_regular_hadamard(group, _ptr(out)) != 0:
        raise ValueError(f"Hadamard group {group} is not a power of 4")
    return out


def hadamard_factors(group: int) -> tuple[int, int] | None:
    """``(GA, GB)`` with ``kron(H_GA, H_GB) == H_group``, both >= 16; None otherwise (int8.py:112-119)."""
    n = group.bit_length() - 1
    if group < 256 or group != 1 << n or n % 2:
        return None
    ga = 4 ** (n // 4)
    return ga, group // ga


def quantize_weight(weight: np.ndarray, group: int) -> tuple[np.ndarray, np.ndarray]:
    """The checkpoint format of tests/test_int8.py:31-36: ``qweight = round(W R / wscale)``, in float64."""
    w = np.asarray(weight, dtype=np.float64)
    k = w.shape[1]
    h = regular_hadamard(group)
    rotated = (w.reshape(w.shape[0], k // group, group) @ h).reshape(w.shape)
    wscale = np.abs(rotated).max(axis=1) / 127.0
    q = np.clip(np.round(rotated / wscale[:, None]), -127, 127).astype(np.int8)
    return q, wscale.astype(np.float32)


# ------------------------------------------------------------------------------------------------- the restatement


def rotate(x_bits: np.ndarray, group: int, *, force_exact: bool = False) -> np.ndarray:
    """``bf16(x.view(M, K/G, G) @ R)`` with the sum computed exactly and rounded once (int8.py:176)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    m, k = x.shape
    out = np.empty_like(x)
    if _lib().oracle_rotate(_ptr(x), m, k, group, _ptr(out), int(force_exact)) != 0:
        raise ValueError(f"bad rotation shape K={k} group={group}")
    return out


def quantize(xr_bits: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-token scale and int8 codes (int8.py:177-178). Returns (sx float32 [M], xq int8 [M, K])."""
    xr = np.ascontiguousarray(xr_bits, dtype=np.uint16)
    m, k = xr.shape
    sx = np.empty(m, dtype=np.float32)
    xq = np.empty((m, k), dtype=np.int8)
    _lib().oracle_quantize(_ptr(xr), m, k, _ptr(sx), _ptr(xq))
    return sx, xq


def rotate_f32(x_bits: np.ndarray, group: int, *, force_exact: bool = False) -> np.ndarray:
    """The reference's GPU rotation (int8.py:194-262): the exact ``x.view(M, K/G, G) @ R`` rounded once to fp32."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    m, k = x.shape
    out = np.empty((m, k), dtype=np.float32)
    if _lib().oracle_rotate_f32(_ptr(x), m, k, group, _ptr(out), int(force_exact)) != 0:
        raise ValueError(f"bad rotation shape K={k} group={group}")
    return out


def quantize_recip(xr: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The reference's GPU quantization (int8.py:208-220): ``s = max(amax, 1e-12) / 127``, ``inv = 1 / s`` and
    ``q = clamp(rint(v * inv), -127, 127)`` in fp32 on the fp32 rotated values. Returns (sx [M], xq int8 [M, K])."""
    v = np.ascontiguousarray(xr, dtype=np.float32)
    m, k = v.shape
    sx = np.empty(m, dtype=np.float32)
    xq = np.empty((m, k), dtype=np.int8)
    _lib().oracle_quantize_recip(_ptr(v), m, k, _ptr(sx), _ptr(xq))
    return sx, xq


def int8_gemm(xq: np.ndarray, qweight: np.ndarray) -> np.ndarray:
    """Exact ``xq @ qweight^T`` as int32 [M, N] (int8.py:179). Raises if a sum leaves int32."""
    a = np.ascontiguousarray(xq, dtype=np.int8)
    b = np.ascontiguousarray(qweight, dtype=np.int8)
    m, k = a.shape
    n = b.shape[0]
    acc = np.empty((m, n), dtype=np.int32)
    if _lib().oracle_int8_gemm(_ptr(a), _ptr(b), m, n, k, _ptr(acc)) != 0:
        raise OverflowError("int8 GEMM sum outside int32")
    return acc


def epilogue(acc: np.ndarray, sx: np.ndarray, wscale: np.ndarray) -> np.ndarray:
    """``bf16((f32(acc) * sx) * wscale)`` (int8.py:179). Returns bf16 bits [M, N]."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, n = acc.shape
    y = np.empty((m, n), dtype=np.uint16)
    _lib().oracle_epilogue(_ptr(acc), _ptr(np.ascontiguousarray(sx, np.float32)),
                           _ptr(np.ascontiguousarray(wscale, np.float32)), m, n, _ptr(y))
    return y


def convrot_linear(x_bits: np.ndarray, qweight: np.ndarray, wscale: np.ndarray, group: int) -> dict:
    """The whole bias-free reference layer. Returns ``{"xr", "sx", "xq", "acc", "y"}``."""
    xr = rotate(x_bits, group)
    sx, xq = quantize(xr)
    acc = int8_gemm(xq, qweight)
    return {"xr": xr, "sx": sx, "xq": xq, "acc": acc, "y": epilogue(acc, sx, wscale)}


def lowrank_down(x_bits: np.ndarray, down_bits: np.ndarray) -> np.ndarray:
    """``bf16(x @ down^T)``, the bf16 intermediate of LowRankLinear (transformer.py:57-58). down is [r, K]."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    d = np.ascontiguousarray(down_bits, dtype=np.uint16)
    m, k = x.shape
    r = d.shape[0]
    u = np.empty((m, r), dtype=np.uint16)
    _lib().oracle_lowrank_down(_ptr(x), _ptr(d), m, k, r, _ptr(u))
    return u


def lowrank_up(u_bits: np.ndarray, up_bits: np.ndarray, bias_bits: np.ndarray | None = None) -> np.ndarray:
    """``bf16(u @ up^T [+ bias])``: LowRankLinear's second bf16 nn.Linear (transformer.py:57-58), the exact sum
    (float64: products of bf16 values are exact and r <= 2^20 terms stay far inside 53 bits for these magnitudes)
    rounded once. The bias is this build's extension."""
    u = bf16_to_f32(np.asarray(u_bits, dtype=np.uint16)).astype(np.float64)
    up = bf16_to_f32(np.asarray(up_bits, dtype=np.uint16)).astype(np.float64)
    y = u @ up.T
    if bias_bits is not None:
        y = y + bf16_to_f32(np.asarray(bias_bits, dtype=np.uint16)).astype(np.float64)[None, :]
    return f64_to_bf16(y)


def fused_epilogue(acc, sx, wscale, u_bits=None, up_bits=None, bias_bits=None) -> np.ndarray:
    """The fused extension's definition: ``bf16((f32(acc)*sx)*ws + u @ up^T + bias)`` rounded once."""
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    m, n = acc.shape
    r = 0 if u_bits is None else u_bits.shape[1]
    y = np.empty((m, n), dtype=np.uint16)
    _lib().oracle_fused_epilogue(
        _ptr(acc), _ptr(np.ascontiguousarray(sx, np.float32)), _ptr(np.ascontiguousarray(wscale, np.float32)),
        _ptr(None if u_bits is None else np.ascontiguousarray(u_bits, np.uint16)),
        _ptr(None if up_bits is None else np.ascontiguousarray(up_bits, np.uint16)), r,
        _ptr(None if bias_bits is None else np.ascontiguousarray(bias_bits, np.uint16)), m, n, _ptr(y))
    return y


def composition(y_int8_bits, x_bits, down_bits=None, up_bits=None, bias_bits=None) -> np.ndarray:
    """``Int8RotLinear(x) + LowRankLinear(x) + bias`` in bf16 tensor arithmetic, as three reference modules compose:
    the low-rank branch is ``bf16(bf16(x @ down^T) @ up^T)`` (transformer.py:57-58) and each ``+`` rounds to bf16."""
    y = bf16_to_f32(y_int8_bits)
    if down_bits is not None:
        u = bf16_to_f32(lowrank_down(x_bits, down_bits)).astype(np.float64)
        lr = bf16_to_f32(f64_to_bf16(u @ bf16_to_f32(up_bits).astype(np.float64).T))
        y = bf16_to_f32(f32_to_bf16(y + lr))
    if bias_bits is not None:
        y = bf16_to_f32(f32_to_bf16(y + bf16_to_f32(bias_bits)[None, :]))
    return f32_to_bf16(y)


def gelu_tanh(y_bits: np.ndarray) -> np.ndarray:
    """``bf16(0.5 y (1 + tanh(sqrt(2/pi) (y + 0.044715 y^3))))`` of a bf16 tensor: the activation the reference's
    feed-forward applies to its bf16 up-projection output (transformer.py:75-99, torch's ``gelu(approximate="tanh")``).
    Evaluated like torch's CPU kernel: the bf16 values widened to fp32, then ``x*x*x``, ``kBeta*(x + kKappa*x^3)``,
    ``0.5*x*(1 + tanh(inner))`` in fp32 with tanh correctly rounded to fp32, then rounded to bf16 (only the last bit
    of torch's fp32 tanh can differ)."""
    x = bf16_to_f32(np.asarray(y_bits, dtype=np.uint16)).astype(np.float32)
    k_beta = np.float32(np.sqrt(2.0) * (2.0 / np.sqrt(np.pi)) * 0.5)
    k_kappa = np.float32(0.044715)
    with np.errstate(over="ignore"):  # |x| near the bf16 maximum: x^3 is inf and tanh saturates, as in fp32
        inner = k_beta * (x + k_kappa * (x * x * x))
    t = np.tanh(inner.astype(np.float64)).astype(np.float32)  # tanh correctly rounded to fp32
    g = np.float32(0.5) * x * (np.float32(1.0) + t)
    return f32_to_bf16(g.astype(np.float32))


def silu(x_bits: np.ndarray) -> np.ndarray:
    """``bf16(x / (1 + exp(-x)))`` of a bf16 tensor, torch's ``silu`` formula evaluated in fp32 (exp correctly
    rounded to fp32, then the fp32 add and divide), rounded once to bf16."""
    x = bf16_to_f32(np.asarray(x_bits, dtype=np.uint16)).astype(np.float32)
    # x below about -88.7: exp(-x) is inf in fp32 and the quotient is -0 (NaN for x = -inf, as in torch)
    with np.errstate(over="ignore", invalid="ignore"):
        e = np.exp(-x.astype(np.float64)).astype(np.float32)
        s = x / (np.float32(1.0) + e)
    return f32_to_bf16(s.astype(np.float32))


def swiglu(y_bits: np.ndarray, gate_first: bool = False) -> np.ndarray:
    """The gated feed-forward's activation on the bf16 projection output ``y`` [..., 2F]: ``hidden, gate =
    y.chunk(2, -1)`` (``gate, hidden`` when ``gate_first``), then ``hidden * silu(gate)`` in bf16 tensor arithmetic
    (the product of two bf16 values is exact in fp32, so one rounding to bf16). Returns [..., F] bf16 bits."""
    y = np.asarray(y_bits, dtype=np.uint16)
    f = y.shape[-1] // 2
    if y.shape[-1] != 2 * f:
        raise ValueError(f"the projection output width {y.shape[-1]} is odd")
    first, second = y[..., :f], y[..., f:]
    hidden, gate = (second, first) if gate_first else (first, second)
    return f32_to_bf16(bf16_to_f32(hidden) * bf16_to_f32(silu(gate)))


# ------------------------------------------------------------------------------------------------ seeded inputs


def make_inputs(m: int, k: int, n: int, group: int, *, rank: int = 0, bias: bool = False,
                outlier_frac: float = 0.01, outlier_scale: float = 20.0, seed: int = 0,
                weight_dist: str = "uniform", x_rows=None) -> dict:
    """Deterministic synthetic inputs of the benchmark's distributions (numpy PCG64, one seed, fixed draw order:
    x, outlier channels, qweight, wscale, down, up, bias).

    x ~ N(0, 1) with ceil(p*K) outlier channels scaled in float32 before the single bf16 cast. ``weight_dist``
    "uniform" draws qweight ~ U{-127..127} and wscale ~ U(1e-3, 1e-2); "quantized" draws W ~ 0.02 N(0,1) and
    quantizes it with `quantize_weight` (the reference tests' recipe, tests/test_int8.py:93-99).

    ``x_rows`` (sorted row indices) keeps only those rows of x: the whole stream is still drawn, in blocks of rows
    (the same values as one draw), so the other tensors are unchanged; for checks on a few rows of a large shape.
    """
    rng = np.random.default_rng(seed)
    if x_rows is None:
        x = rng.standard_normal((m, k)).astype(np.float32)
    else:
        x_rows = np.asarray(x_rows, dtype=np.int64)
        x = np.empty((x_rows.size, k), dtype=np.float32)
        for r0 in range(0, m, 1024):
            block = rng.standard_normal((min(1024, m - r0), k))
            sel = (x_rows >= r0) & (x_rows < r0 + block.shape[0])
            x[sel] = block[x_rows[sel] - r0]
    n_out = int(np.ceil(outlier_frac * k)) if outlier_frac > 0 else 0
    if n_out:
        cols = rng.choice(k, size=n_out, replace=False)
        x[:, cols] *= np.float32(outlier_scale)
    out = {"x": f32_to_bf16(x)}
    if weight_dist == "uniform":
        out["qweight"] = rng.integers(-127, 128, size=(n, k), dtype=np.int64).astype(np.int8)
        out["wscale"] = rng.uniform(1e-3, 1e-2, size=n).astype(np.float32)
    else:
        w = rng.standard_normal((n, k)) * 0.02
        out["qweight"], out["wscale"] = quantize_weight(w, group)
    if rank:
        out["down"] = f32_to_bf16((rng.standard_normal((rank, k)) * 0.02).astype(np.float32))
        out["up"] = f32_to_bf16((rng.standard_normal((n, rank)) * 0.02).astype(np.float32))
    if bias:
        out["bias"] = f32_to_bf16((rng.standard_normal(n) * 0.01).astype(np.float32))
    return out
