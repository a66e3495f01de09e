"""The library on several streams at once: every entry point launches on the caller's stream and keeps no state
between calls, so layers run concurrently on two side streams (each with its own workspace from the caching
allocator) give bitwise the outputs they give one after another on the default stream. The shapes take different
paths: persistent whole tiles with a peeled split-K tail, the few-row split GEMM with its finishing pass and split
low-rank projection, and the mid-size tiles."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")

LAYERS = [(3584, 5120, 5120, 32, True), (64, 5120, 30720, 32, False), (1000, 2304, 4096, 0, False)]


def _layer(k, n, rank, bias, seed):
    from hyperflow_h3_flash_amd import Int8RotLinear

    gen = torch.Generator().manual_seed(seed)
    layer = Int8RotLinear(k, n, 256, rank=rank, bias=bias)
    with torch.no_grad():
        layer.qweight.copy_(torch.randint(-127, 128, (n, k), dtype=torch.int8, generator=gen))
        layer.wscale.copy_(torch.rand(n, generator=gen) * 9e-3 + 1e-3)
        if rank:
            layer.down.weight.copy_(torch.randn(rank, k, generator=gen) * 0.02)
            layer.up.weight.copy_(torch.randn(n, rank, generator=gen) * 0.02)
        if bias:
            layer.bias.copy_(torch.randn(n, generator=gen) * 0.01)
    return layer.to(DEV)


def test_concurrent_streams_match_serial_results():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    layers, xs = [], []
    for i, (m, k, n, rank, bias) in enumerate(LAYERS):
        print(f"stream test layer {i}: M={m} K={k} N={n} rank={rank} bias={bias}", flush=True)
        layers.append(_layer(k, n, rank, bias, seed=100 + i))
        gen = torch.Generator().manual_seed(200 + i)
        xs.append((torch.randn(m, k, generator=gen) * 2.0).to(torch.bfloat16).to(DEV))
    with torch.no_grad():
        serial = [layer(x).clone() for layer, x in zip(layers, xs)]
        torch.cuda.synchronize()
        side = [torch.cuda.Stream(DEV), torch.cuda.Stream(DEV)]
        for s in side:
            s.wait_stream(torch.cuda.current_stream(DEV))
        # each stream runs every layer, in a different order, three times over
        outs = {0: [], 1: []}
        for rep in range(3):
            for j, s in enumerate(side):
                with torch.cuda.stream(s):
                    order = range(len(layers)) if j == 0 else reversed(range(len(layers)))
                    for i in order:
                        outs[j].append((i, layers[i](xs[i])))
        torch.cuda.synchronize()
    for j in (0, 1):
        for i, y in outs[j]:
            assert torch.equal(y, serial[i]), f"stream {j}, layer {i}"
