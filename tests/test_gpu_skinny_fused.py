"""The single-pass few-row GEMM (at most 64 rows, 32 weight rows per workgroup with the whole K, the epilogue in the
same kernel) against the oracle.

The shapes below take that path: M <= 64 and between 64 and 256 slices of 32 weight rows. Bars, as for the other
GEMM paths: without a low-rank branch the outputs are bitwise the oracle's (the reference's `bf16((acc * sx) * ws)`,
plus the bias as the fused definition adds it); with one, every element within one bf16 ulp of the oracle's fused
definition computed on the device's own low-rank intermediate u; tanh-GELU and SwiGLU outputs against the oracle's
activation of the same layer's output without the activation (test_gpu_activation.py's bars). The shapes cover a K
that ends inside a 128-byte stage, a ragged N, one row, ranks above 64 and both gated half orders.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from test_gpu_activation import act_linear, check_gelu, check_swiglu

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def to_dev_bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(DEV)


def bits_of(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def layer_operands(oracle_lib, m, k, n, rank, bias, seed):
    from hyperflow_h3_flash_amd.int8 import lowrank_down, rotate_quant

    g = 256 if k % 256 == 0 else 16
    inp = oracle_lib.make_inputs(m, k, n, g, rank=rank, bias=bias, outlier_frac=0.01, outlier_scale=20.0, seed=seed)
    x = to_dev_bf16(inp["x"])
    q, sx = rotate_quant(x, g)
    kw = {}
    if rank:
        kw = dict(u=lowrank_down(x, to_dev_bf16(inp["down"])), up=to_dev_bf16(inp["up"]))
    if bias:
        kw["bias"] = to_dev_bf16(inp["bias"])
    w = torch.from_numpy(inp["qweight"]).to(DEV)
    ws = torch.from_numpy(inp["wscale"]).to(DEV)
    return inp, g, q, sx, w, ws, kw


@pytest.mark.parametrize("m,k,n,rank,bias", [(1, 5120, 2048, 0, False), (64, 5120, 5120, 0, False),
                                             (64, 5120, 5120, 0, True), (17, 2064, 3008, 32, True),
                                             (64, 1040, 8192, 96, False), (40, 3072, 4096, 64, True),
                                             (64, 4096, 2080, 8, False)])
def test_single_pass_gemm_matches_oracle(oracle_lib, m, k, n, rank, bias):
    from hyperflow_h3_flash_amd.int8 import int8_matmul

    inp, g, q, sx, w, ws, kw = layer_operands(oracle_lib, m, k, n, rank, bias, seed=m + k + n + rank)
    print(f"single-pass GEMM M={m} K={k} N={n} rank={rank} bias={bias}", flush=True)
    y = int8_matmul(q, w, sx, ws, **kw)
    torch.cuda.synchronize()
    ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), ref["sx"].view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), ref["xq"])
    if not rank:
        want = ref["y"] if not bias else oracle_lib.fused_epilogue(ref["acc"], ref["sx"], inp["wscale"], None, None,
                                                                   inp["bias"])
        np.testing.assert_array_equal(bits_of(y), want)
        return
    fused = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(ref["acc"], ref["sx"], inp["wscale"], bits_of(kw["u"]),
                                                             inp["up"], inp["bias"] if bias else None))
    got = oracle_lib.bf16_to_f32(bits_of(y))
    assert (np.abs(got - fused) <= np.abs(fused) * 2.0**-7 + 1e-6).all()
    assert (got == fused).mean() > 0.98


@pytest.mark.parametrize("m,k,n,rank,bias", [(64, 3072, 4096, 64, True), (9, 1024, 2048, 0, False)])
def test_single_pass_gelu(oracle_lib, m, k, n, rank, bias):
    from hyperflow_h3_flash_amd.int8 import int8_matmul

    _, _, q, sx, w, ws, kw = layer_operands(oracle_lib, m, k, n, rank, bias, seed=7 * m + n)
    plain = int8_matmul(q, w, sx, ws, **kw)
    fused = act_linear(q, w, sx, ws, kw, "gelu_tanh", True)
    torch.cuda.synchronize()
    check_gelu(bits_of(fused), bits_of(plain), oracle_lib)


@pytest.mark.parametrize("gate_first", [False, True])
@pytest.mark.parametrize("m,k,n,rank,bias", [(64, 1024, 4096, 32, True), (3, 5120, 2048, 0, False)])
def test_single_pass_swiglu(oracle_lib, m, k, n, rank, bias, gate_first):
    from hyperflow_h3_flash_amd.int8 import int8_matmul

    _, _, q, sx, w, ws, kw = layer_operands(oracle_lib, m, k, n, rank, bias, seed=11 * m + n + gate_first)
    plain = int8_matmul(q, w, sx, ws, **kw)
    fused = act_linear(q, w, sx, ws, kw, "swiglu_gate_first" if gate_first else "swiglu", True)
    torch.cuda.synchronize()
    assert fused.shape == (m, n // 2)
    check_swiglu(bits_of(fused), bits_of(plain), oracle_lib, gate_first)
