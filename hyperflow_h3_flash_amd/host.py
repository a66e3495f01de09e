"""The convrot linear's arithmetic on host (CPU) tensors, for layers whose input lives in host memory.

The reference runs its torch statements (`Int8RotLinear._forward_torch`, src/hyperflow_h3_flash/int8.py:173-179)
for CPU tensors; a drop-in has to compute on the host too. This module evaluates the same definition as the gfx950
kernels. Without a low-rank term (with or without the bias) a layer gives the same bits on either side of the PCIe
link; with one, the host sums the term exactly while the device's matrix cores sum it in fp32, so the two agree
within one bf16 ulp (bitwise on almost every element):

1. the rotated activation is the exact block sum ``x[m, gG:(g+1)G] @ H_G`` rounded once to bf16 (ties to even);
2. ``sx = max(absmax_row, 1e-12) / 127`` and ``xq = clamp(round_half_even(xr / sx), -127, 127)`` in fp32, true
   divisions;
3. ``acc = xq @ qweight^T`` as an exact integer;
4. ``y = bf16((f32(acc) * sx) * wscale)``, two rounded fp32 products and one rounding to bf16;

and the fused extension ``y = bf16((f32(acc) * sx) * wscale + bf16(x @ down^T) @ up^T + bias)``: the bias alone
added in fp32, a low-rank product (and the bias beside it) summed in float64; one rounding; then the optional output
activation of torch's own modules. The low-rank intermediate ``bf16(x @ down^T)`` is the exact sum rounded once
(the device's fp32 sum is within one bf16 ulp of it).

Exactness: the rotation's products ``x * (+-2^-n)`` are exact and float64 holds their sums exactly while a group's
nonzero inputs span fewer than about 37 binades (the device's fp64 butterfly: 33); the integer product is exact in
float64 up to |acc| < 2^53, far above what int8 codes over K <= 2^20 reach. Every power-of-4 group is accepted here
(the device kernels stop at 256). Device tensors never come here: the module sends them to the HIP kernels.
"""

from __future__ import annotations

import torch
from torch import Tensor

#: The unnormalized order-4 block of the regular Hadamard matrix (int8.py:102): H_G = kron(H4 / 2, ..., H4 / 2).
_H4 = ((1, 1, 1, -1), (1, 1, -1, 1), (1, -1, 1, 1), (-1, 1, 1, 1))


def _digits(group: int) -> int:
    n, g = 0, 1
    while g < group:
        g, n = g * 4, n + 1
    if g != group:
        raise ValueError(f"Hadamard group {group} is not a power of 4")
    return n


def rotate_exact(x2: Tensor, group: int) -> Tensor:
    """float64 ``x2.view(M, K/G, G) @ H_G`` (exact while a group's inputs span < ~37 binades), shape [M, K].

    The transform runs as one radix-4 step per base-4 digit of the in-group index: a [..., 4, 4^d] view multiplied
    by the ±1 matrix H4 along its digit axis, then the 2^-n normalisation (a power of two, exact)."""
    n = _digits(group)
    m, k = x2.shape
    if k % group:
        raise ValueError(f"in_features {k} is not a multiple of the Hadamard group {group}")
    h4 = torch.tensor(_H4, dtype=torch.float64)
    t = x2.to(torch.float64).reshape(-1, 4, 1)  # [blocks, digit, rest]
    rest = 1
    for _ in range(n):
        t = t.reshape(-1, 4, rest)
        t = torch.einsum("ij,bjr->bir", h4, t)
        rest *= 4
    return (t.reshape(m, k) * 2.0 ** (-n)).contiguous()


def round_to_bf16(t: Tensor) -> Tensor:
    """float64 -> the nearest bf16 value (8 significant bits, ties to even) with one rounding, as float32.

    A direct ``.to(torch.bfloat16)`` of a float64 tensor would round twice (to fp32, then to bf16)."""
    mant, expo = torch.frexp(t)  # t = mant * 2^expo, 0.5 <= |mant| < 1
    return torch.ldexp(torch.round(mant * 256.0) / 256.0, expo).to(torch.float32)


def quantize_rows(xr: Tensor) -> tuple[Tensor, Tensor]:
    """Per-token scale and codes of the rotated rows ``xr`` (fp32 [M, K]): (int8 [M, K], fp32 [M])."""
    amax = xr.abs().amax(dim=1) if xr.shape[1] else torch.zeros(xr.shape[0])
    scale = torch.clamp(amax, min=1e-12) / 127.0
    codes = torch.round(xr / scale[:, None]).clamp_(-127, 127)
    return codes.to(torch.int8), scale


def rotate_quant(x2: Tensor, group: int) -> tuple[Tensor, Tensor]:
    """The host counterpart of the device ``rotate_quant``: bf16 [M, K] -> (int8 codes [M, K], fp32 scales [M])."""
    return quantize_rows(round_to_bf16(rotate_exact(x2, group)))


def int8_gemm_exact(a: Tensor, b: Tensor) -> Tensor:
    """``a @ b^T`` of int8 codes as exact integers, held in float64 ([M, N])."""
    return a.to(torch.float64) @ b.to(torch.float64).t()


def lowrank_down(x2: Tensor, down: Tensor) -> Tensor:
    """``bf16(x @ down^T)`` with the float64 sum rounded once (LowRankLinear.down, transformer.py:57)."""
    u = x2.to(torch.bfloat16).to(torch.float64) @ down.to(torch.bfloat16).to(torch.float64).t()
    return round_to_bf16(u).to(torch.bfloat16)


def dequantize(acc: Tensor, sx: Tensor, wscale: Tensor, *, u: Tensor | None = None, up: Tensor | None = None,
               bias: Tensor | None = None) -> Tensor:
    """``bf16((f32(acc) * sx) * wscale [+ u @ up^T] [+ bias])``: the two fp32 products, then (extension) with the
    bias alone one fp32 addition, as the device kernels make it; with a low-rank term the term and the bias added in
    float64 to the fp32 value (the exact sum; the device sums in fp32 in an unspecified order). One rounding to
    bf16."""
    y = (acc.to(torch.float32) * sx[:, None]) * wscale.to(torch.float32)[None, :]
    if u is None:
        if bias is not None:
            y = y + bias.to(torch.bfloat16).to(torch.float32)[None, :]
        return y.to(torch.bfloat16)
    s = y.to(torch.float64)
    if u is not None:
        s = s + u.to(torch.float64) @ up.to(torch.bfloat16).to(torch.float64).t()
    if bias is not None:
        s = s + bias.to(torch.bfloat16).to(torch.float64)[None, :]
    return round_to_bf16(s).to(torch.bfloat16)


def activate(y: Tensor, activation: str | None) -> Tensor:
    """The output activation modules of the feed-forward on the bf16 linear output (transformer.py:75-99): torch's
    ``gelu(approximate="tanh")``, or SwiGLU's ``hidden * silu(gate)`` of ``y.chunk(2, -1)`` (gate first: swapped)."""
    if activation is None:
        return y
    if activation == "gelu_tanh":
        return torch.nn.functional.gelu(y, approximate="tanh")
    first, second = y.chunk(2, dim=-1)
    hidden, gate = (second, first) if activation == "swiglu_gate_first" else (first, second)
    return hidden * torch.nn.functional.silu(gate)


__all__ = ["activate", "dequantize", "int8_gemm_exact", "lowrank_down", "quantize_rows", "rotate_exact",
           "rotate_quant", "round_to_bf16"]
