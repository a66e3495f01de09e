"""The benchmark workloads at full size on the device, checked against the oracle on sampled rows.

Rows of the convrot linear are independent (per-token rotation and scale, per-row output), so a seeded sample of
rows, plus the first and the last rows (the ragged last tile), pins the device's results against the oracle at the
real shapes, while size-independent properties are checked on every row. Bars, per layer:

* no low-rank branch and no bias: codes, scales and bf16 outputs bitwise the oracle's (the reference's torch path);
* with a low-rank branch and/or a bias (the fused extension): every element within one bf16 ulp of the oracle's
  fused definition ``bf16((f32(acc)*sx)*ws + u @ up^T + bias)``, and max |y - y_ref| / max |y_ref| <= 1e-2 against
  the reference's module composition ``Int8RotLinear(x) + LowRankLinear(x) + bias``;
* the low-rank intermediate ``u`` within the fp32-summation bound of the oracle's exactly rounded ``bf16(x @ down^T)``;
* tanh-GELU fused in the epilogue: the oracle's GELU of the same layer's unfused device output, within 1e-3 of its
  maximum everywhere and bitwise on >= 99.9 % of the elements whose input is >= -3 (the bar of
  test_gpu_activation.py). The next layer of a chain is graded on the device's own activation output (so each layer
  sees identical bf16 inputs on both sides).

Workloads: one convrot layer at M=1024, K=N=3072, rank 32, bias; the fused QKV projection at M=32768, K=5120,
N=15360, rank 64; the FFN pair (5120 -> 13824 with tanh-GELU, then 13824 -> 5120, rank 64 each) at M=32768; a full
DiT block's linears at M=40320 + 1024 = 41344 (QKV 15360, out 5120, FFN up 13824, down 5120); the small-M sweep
M in {64, 256, 1024} x N in {5120, 30720}, K=5120, rank 32. Inputs: x ~ N(0, 1) with outlier channels (1 % x20 for
the single layer, 0.5 % x30 elsewhere), int8 weights uniform in [-127, 127], scales U(1e-3, 1e-2), low-rank
factors N(0, 0.02), bias N(0, 0.01); all seeded.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from golden_utils import check_against_composition, device_lowrank_slack, within_fp32_sum_bound

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
G = 256


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def activations(m: int, k: int, seed: int, frac: float = 0.005, scale: float = 30.0) -> torch.Tensor:
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k, device=DEV, generator=gen)
    cols = torch.randperm(k, device=DEV, generator=gen)[: int(np.ceil(frac * k))]
    x[:, cols] *= scale
    return x.to(torch.bfloat16)


def make_layer(k: int, n: int, seed: int, rank: int = 0, bias: bool = False, activation: str | None = None):
    from hyperflow_h3_flash_amd import Int8RotLinear

    gen = torch.Generator(device=DEV).manual_seed(seed)
    layer = Int8RotLinear(k, n, G, rank=rank, bias=bias, activation=activation).to(DEV)
    with torch.no_grad():
        layer.qweight.copy_(torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen))
        layer.wscale.copy_(torch.rand(n, device=DEV, generator=gen) * 9e-3 + 1e-3)
        if rank:
            layer.down.weight.copy_((torch.randn(rank, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16))
            layer.up.weight.copy_((torch.randn(n, rank, device=DEV, generator=gen) * 0.02).to(torch.bfloat16))
        if bias:
            layer.bias.copy_((torch.randn(n, device=DEV, generator=gen) * 0.01).to(torch.bfloat16))
    return layer


def sample_rows(m: int, seed: int, count: int = 12) -> np.ndarray:
    rng = np.random.default_rng(seed)
    picked = rng.choice(m, size=min(count, m), replace=False)
    return np.unique(np.concatenate([picked, [0], np.arange(max(0, m - 3), m)]))


def check_layer(lib, layer, x: torch.Tensor, y: torch.Tensor, rows: np.ndarray) -> None:
    """`y` = layer(x) (no activation) against the oracle on `rows`; codes and scales on every row's properties."""
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    q, s = rotate_quant(x, G)
    torch.cuda.synchronize()
    # every row: its absmax element quantizes to +-127 (rows here are never all zero); no code leaves [-127, 127]
    assert int(q.abs().amax(dim=1).min()) == 127 and int(q.min()) >= -127
    assert bool(torch.isfinite(y.float()).all())
    xb = bits_of(x[rows])
    w = layer.qweight.cpu().numpy()
    ws = layer.wscale.cpu().numpy()
    out = lib.convrot_linear(xb, w, ws, G)
    np.testing.assert_array_equal(s[rows].cpu().numpy(), out["sx"])
    np.testing.assert_array_equal(q[rows].cpu().numpy(), out["xq"])
    got_bits = bits_of(y[rows])
    if not layer.rank and layer.bias is None:
        np.testing.assert_array_equal(got_bits, out["y"])
        return
    down = bits_of(layer.down.weight) if layer.rank else None
    up = bits_of(layer.up.weight) if layer.rank else None
    bias = bits_of(layer.bias) if layer.bias is not None else None
    if layer.rank:
        from hyperflow_h3_flash_amd.int8 import lowrank_down

        u_dev = lowrank_down(x[torch.from_numpy(rows).to(DEV)], layer.down.weight)
        u_ref = lib.lowrank_down(xb, down)
        assert within_fp32_sum_bound(lib.bf16_to_f32(bits_of(u_dev)), lib.bf16_to_f32(u_ref),
                                     lib.bf16_to_f32(xb), lib.bf16_to_f32(down))
        fused = lib.fused_epilogue(out["acc"], out["sx"], ws, u_ref, up, bias)
    else:
        fused = lib.fused_epilogue(out["acc"], out["sx"], ws, None, None, bias)
    got = lib.bf16_to_f32(got_bits)
    want = lib.bf16_to_f32(fused)
    assert (np.abs(got - want) <= np.abs(want) * 2.0**-7 + 1e-6).all()
    # against the reference's composition Int8RotLinear(x) + LowRankLinear(x) + bias, elementwise
    lowrank = lib.lowrank_up(u_ref, up) if layer.rank else None
    extra = device_lowrank_slack(xb, down, u_ref, up, out["y"], bias) if layer.rank else None
    check_against_composition(got_bits, out["y"], lowrank, bias, lib.composition(out["y"], xb, down, up, bias),
                              extra=extra)


def check_gelu(lib, fused_act: torch.Tensor, pre: torch.Tensor, rows: np.ndarray) -> None:
    """The fused tanh-GELU output against the oracle's GELU of the unfused device output."""
    pre_bits = bits_of(pre[rows])
    got = lib.bf16_to_f32(bits_of(fused_act[rows]))
    ref = lib.bf16_to_f32(lib.gelu_tanh(pre_bits))
    assert np.abs(got - ref).max() <= 1e-3 * np.abs(ref).max()
    region = lib.bf16_to_f32(pre_bits) >= -3.0
    assert (got[region] == ref[region]).mean() >= 0.999


def run(layer, x):
    with torch.no_grad():
        y = layer(x)
    torch.cuda.synchronize()
    return y


def test_single_layer_m1024_k3072_n3072_rank32_bias(oracle_lib):
    x = activations(1024, 3072, seed=101, frac=0.01, scale=20.0)
    layer = make_layer(3072, 3072, seed=102, rank=32, bias=True)
    y = run(layer, x)
    check_layer(oracle_lib, layer, x, y, sample_rows(1024, 103, count=24))


@pytest.mark.parametrize("rank", [0, 64])
def test_fused_qkv_m32768_k5120_n15360(oracle_lib, rank):
    x = activations(32768, 5120, seed=201)
    layer = make_layer(5120, 15360, seed=202 + rank, rank=rank)
    y = run(layer, x)
    check_layer(oracle_lib, layer, x, y, sample_rows(32768, 203 + rank))


def test_ffn_pair_m32768_gelu_then_down(oracle_lib):
    """The up-projection with its tanh-GELU fused, then the down-projection on the device's own GELU output."""
    m = 32768
    x = activations(m, 5120, seed=301)
    up = make_layer(5120, 13824, seed=302, rank=64, activation="gelu_tanh")
    rows = sample_rows(m, 303)
    h = run(up, x)
    up.activation = None
    pre = run(up, x)
    up.activation = "gelu_tanh"
    check_layer(oracle_lib, up, x, pre, rows)
    check_gelu(oracle_lib, h, pre, rows)
    del pre
    down = make_layer(13824, 5120, seed=304, rank=64)
    y = run(down, h)
    check_layer(oracle_lib, down, h, y, rows)


def test_dit_block_linears_m41344(oracle_lib):
    """QKV (fused, 15360), attention out (5120), FFN up (13824, tanh-GELU) and down (5120) of one block at the
    5.2 s clip's token count (40320 video + 1024 audio), rank 64 on every layer."""
    m = 40320 + 1024
    rows = sample_rows(m, 401)
    x = activations(m, 5120, seed=402)
    qkv = make_layer(5120, 15360, seed=403, rank=64)
    check_layer(oracle_lib, qkv, x, run(qkv, x), rows)
    out = make_layer(5120, 5120, seed=404, rank=64)
    check_layer(oracle_lib, out, x, run(out, x), rows)
    up = make_layer(5120, 13824, seed=405, rank=64, activation="gelu_tanh")
    h = run(up, x)
    up.activation = None
    pre = run(up, x)
    check_layer(oracle_lib, up, x, pre, rows)
    check_gelu(oracle_lib, h, pre, rows)
    del pre
    down = make_layer(13824, 5120, seed=406, rank=64)
    check_layer(oracle_lib, down, h, run(down, h), rows)


@pytest.mark.parametrize("m", [64, 256, 1024])
@pytest.mark.parametrize("n", [5120, 30720])
def test_small_m_sweep_k5120_rank32(oracle_lib, m, n):
    """The small-M workloads (few-row kernels: skinny and split-K GEMMs, row-wise rotation and low-rank)."""
    x = activations(m, 5120, seed=500 + m)
    layer = make_layer(5120, n, seed=501 + n, rank=32)
    y = run(layer, x)
    check_layer(oracle_lib, layer, x, y, sample_rows(m, 502 + m + n, count=12 if n > 5120 else 24))
    # the r = 0 layer on the same rows: outputs bitwise the oracle's
    plain = make_layer(5120, n, seed=503 + n)
    check_layer(oracle_lib, plain, x, run(plain, x), sample_rows(m, 504 + m, count=8))
