"""`Int8RotLinear.forward` as one library call (hf_convrot_linear_ws) against the composed calls (rotate_quant,
lowrank_down, int8_matmul): the same kernels and arithmetic, so the outputs must be bitwise equal, including the
shared quantized input of q/k/v projections (int8.py:150-159), both rotation arithmetics and the activations.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def composed(fn):
    """Run `fn` with the kernels namespace's functions wrapped, which routes forward through the composed calls."""
    from hyperflow_h3_flash_amd.int8 import _kernels

    kernels = _kernels()
    saved = kernels.rotate_quant
    kernels.rotate_quant = lambda *a, **k: saved(*a, **k)
    try:
        return fn()
    finally:
        kernels.rotate_quant = saved


def make_layer(k, n, group, rank, bias, activation=None, seed=0):
    from hyperflow_h3_flash_amd import Int8RotLinear

    gen = torch.Generator(device=DEV).manual_seed(seed)
    layer = Int8RotLinear(k, n, group, rank=rank, bias=bias, activation=activation).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen))
        layer.wscale.copy_(torch.rand(n, device=DEV, generator=gen) * 9e-3 + 1e-3)
        if rank:
            layer.down.weight.copy_(torch.randn(rank, k, device=DEV, generator=gen) * 0.02)
            layer.up.weight.copy_(torch.randn(n, rank, device=DEV, generator=gen) * 0.02)
        if bias:
            layer.bias.copy_(torch.randn(n, device=DEV, generator=gen) * 0.01)
    return layer


@pytest.mark.parametrize("m,k,n,rank,bias,activation", [
    (1024, 3072, 3072, 32, True, None),     # the reference's CPU-runnable case (split K)
    (40, 1024, 320, 64, False, None),       # the skinny kernel
    (600, 2048, 768, 64, True, "gelu_tanh"),
    (300, 1024, 544, 96, False, "swiglu"),  # rank above 64: two low-rank launches
    (257, 512, 300, 0, False, None),
    (100, 5376, 640, 32, True, "gelu_tanh"),  # rotation and low-rank rows in one launch, a partial last tile
    (256, 5376, 640, 32, False, None),        # 256 rows in that launch
    (3, 14336, 256, 136, False, None),        # its widest row (14 tiles), ranks in nine passes of 16
    (5, 16384, 256, 32, False, None),         # 16 tiles: the rotation's wide-row kernel, the low-rank row kernel
])
@pytest.mark.parametrize("arithmetic", ["bf16_div", "f32_recip"])
def test_one_call_forward_is_the_composed_forward(m, k, n, rank, bias, activation, arithmetic):
    from hyperflow_h3_flash_amd import set_arithmetic_options

    layer = make_layer(k, n, 256, rank, bias, activation, seed=m + n)
    x = torch.randn(2, m, k, device=DEV).to(torch.bfloat16)
    try:
        set_arithmetic_options(rotate_quant=arithmetic)
        with torch.no_grad():
            fast = layer(x)
            slow = composed(lambda: layer(x))
    finally:
        set_arithmetic_options(rotate_quant="bf16_div")
    assert fast.shape == slow.shape
    np.testing.assert_array_equal(bits_of(fast), bits_of(slow))


@pytest.mark.parametrize("m,k,n,group,rank", [
    (700, 2048, 384, 256, 1),      # the row rotation kernel adds the sums; rank 1
    (2000, 3072, 640, 256, 64),    # the register rotation kernel adds them
    (3000, 1024, 256, 256, 48),    # the register kernel, one tile per row
    (4096, 5120, 512, 256, 32),
    (1100, 24576, 256, 256, 64),   # rows past 20 tiles: the reduce runs after the rotation kernel
    (1500, 8192, 256, 4096, 64),   # group 4096: the wide rotation kernel, the reduce after it
])
def test_one_call_split_low_rank_sums_in_the_rotation(m, k, n, group, rank):
    """Layers whose low-rank projection splits K: the one library call runs the projection first and the rotation
    adds its partial sums (or, for rotation kernels that do not, a reduce launch after them); the result equals the
    composed calls (rotation, projection with its own reduce, GEMM) bit for bit."""
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    assert lib.hf_lowrank_down_ws_bytes(m, k, rank) > 0  # the projection splits K at this size
    layer = make_layer(k, n, group, rank, False, seed=m + k)
    x = torch.randn(m, k, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        fast = layer(x)
        slow = composed(lambda: layer(x))
    np.testing.assert_array_equal(bits_of(fast), bits_of(slow))


def test_one_call_forward_shares_the_quantized_input():
    """q/k/v on one input: the first (keep_input) quantizes, the next two reuse its codes; the outputs equal those of
    layers that each quantize for themselves, and nothing outlives the projections."""
    from hyperflow_h3_flash_amd import Int8RotLinear

    layers = [make_layer(1024, 512, 256, 32, False, seed=s) for s in range(3)]
    layers[0].keep_input = layers[1].keep_input = True
    x = torch.randn(700, 1024, device=DEV).to(torch.bfloat16)
    with torch.no_grad():
        shared = [layer(x) for layer in layers]
        assert not Int8RotLinear._last_input
        for layer in layers:
            layer.keep_input = False
        alone = [layer(x) for layer in layers]
    for a, b in zip(shared, alone):
        np.testing.assert_array_equal(bits_of(a), bits_of(b))
