"""The layer's launches under HIP graph capture: the kernels allocate nothing and record no memset, so a captured
forward replays to the eager result every time, with eager work and synchronizations between the replays."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.mark.parametrize("m,k,n,rank,bias", [(64, 5120, 5120, 32, False), (40, 1024, 3000, 0, True),
                                             (1024, 3072, 3072, 32, True)])
def test_captured_forward_replays_to_the_eager_result(m, k, n, rank, bias):
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import Int8RotLinear

    torch.manual_seed(m + n)
    layer = Int8RotLinear(k, n, 256, rank=rank, bias=bias).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.randint(-127, 128, (n, k), dtype=torch.int8))
        layer.wscale.copy_(torch.rand(n) * 9e-3 + 1e-3)
        if rank:
            layer.down.weight.copy_(torch.randn(rank, k) * 0.02)
            layer.up.weight.copy_(torch.randn(n, rank) * 0.02)
        if bias:
            layer.bias.copy_(torch.randn(n) * 0.01)
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        eager = layer(x).clone()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = layer(x)
        for i in range(4):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {i}"
            layer(torch.randn_like(x))  # eager work between replays
            torch.cuda.synchronize()
