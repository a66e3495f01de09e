"""ORACLE — test infrastructure only (the CPU baseline leg of bench.py and the tests use it; the product does not).

A PyTorch-CPU restatement of the reference's host path ``Int8RotLinear._forward_torch``
(src/hyperflow_h3_flash/int8.py:173-179), with the low-rank branch of LowRankLinear (transformer.py:57-58) and a
bias for the fused extension. It runs torch's own CPU kernels (oneDNN bf16 GEMM for the rotation, fp32 GEMM for the
integer-valued product), so its rotation rounding follows the host ISA's fp32 accumulation order; this is the
workload the reference runs on a CPU, timed as the baseline.
"""

from __future__ import annotations

import torch


def regular_hadamard(group: int) -> torch.Tensor:
    """int8.py:100-109."""
    h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=torch.float64) / 2
    h, n = torch.ones(1, 1, dtype=torch.float64), 1
    while n < group:
        h, n = torch.kron(h, h4), n * 4
    if n != group:
        raise ValueError(f"Hadamard group {group} is not a power of 4")
    return h.float()


def forward_torch(x2: torch.Tensor, qweight: torch.Tensor, wscale: torch.Tensor, group: int,
                  down: torch.Tensor | None = None, up: torch.Tensor | None = None,
                  bias: torch.Tensor | None = None) -> torch.Tensor:
    """x2 bf16 [M, K] -> bf16 [M, N], the statements of int8.py:176-179 (plus the low-rank composition)."""
    rot = regular_hadamard(group).to(torch.bfloat16)
    k = x2.shape[1]
    xr = (x2.reshape(-1, k // group, group) @ rot).reshape(x2.shape).float()
    sx = xr.abs().amax(1, keepdim=True).clamp_min(1e-12) / 127.0
    xq = (xr / sx).round().clamp(-127, 127)
    y = ((xq @ qweight.float().t()) * sx * wscale[None, :]).to(torch.bfloat16)
    if down is not None:
        y = y + torch.nn.functional.linear(torch.nn.functional.linear(x2, down), up)
    if bias is not None:
        y = y + bias
    return y
