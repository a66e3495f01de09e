"""Seeded random layers against the oracle: group, K, M, N, low-rank rank, bias and output activation drawn together,
so the dispatch (single-pass, split, mid-size and persistent GEMMs; row, register and LDS-row rotations; row-wise,
split and MFMA low-rank projections) meets combinations no hand-picked test lists.

The draw is fixed (numpy PCG64, seed 2026) and each case prints its parameters before it runs. Bars, as in the other
GEMM tests: codes and scales bitwise the oracle's; without a low-rank branch, bias or activation the output bitwise the
oracle's; with a low-rank branch or bias every output within one bf16 ulp of the oracle's fused definition on the
device's own low-rank intermediate; tanh-GELU and SwiGLU outputs against the oracle's activation of the same layer
without it (test_gpu_activation.py's bars).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from test_gpu_activation import check_gelu, check_swiglu
from test_gpu_skinny_fused import bits_of, to_dev_bf16

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _device():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    _native.library()


def _cases(n_cases: int = 40):
    rng = np.random.default_rng(2026)
    cases = []
    while len(cases) < n_cases:
        g = int(rng.choice([16, 64, 256]))
        k = g * int(rng.integers(1, 6144 // g + 1))
        if k % 16:
            continue
        m = int(np.exp(rng.uniform(0.0, np.log(6000.0))))
        n = 32 * int(np.exp(rng.uniform(0.0, np.log(9000.0 / 32))))
        if m * n * k > 3e9:
            continue
        rank = int(rng.choice([0, 0, 8, 32, 64, 96]))
        bias = bool(rng.integers(0, 2))
        act = str(rng.choice(["none", "none", "gelu_tanh", "swiglu"]))
        cases.append((m, k, n, g, rank, bias, act))
    return cases


def _operands(oracle_lib, m, k, n, g, rank, bias, seed):
    from hyperflow_h3_flash_amd.int8 import lowrank_down, rotate_quant

    inp = oracle_lib.make_inputs(m, k, n, g, rank=rank, bias=bias, outlier_frac=0.01, outlier_scale=20.0, seed=seed)
    x = to_dev_bf16(inp["x"])
    q, sx = rotate_quant(x, g)
    kw = {}
    if rank:
        kw = dict(u=lowrank_down(x, to_dev_bf16(inp["down"])), up=to_dev_bf16(inp["up"]))
    if bias:
        kw["bias"] = to_dev_bf16(inp["bias"])
    w = torch.from_numpy(inp["qweight"]).to(x.device)
    ws = torch.from_numpy(inp["wscale"]).to(x.device)
    return inp, q, sx, w, ws, kw


@pytest.mark.parametrize("case", _cases(), ids=lambda c: "m{}_k{}_n{}_g{}_r{}_b{}_{}".format(*c))
def test_random_layer_matches_oracle(oracle_lib, case):
    from hyperflow_h3_flash_amd.int8 import int8_matmul

    m, k, n, g, rank, bias, act = case
    print(f"random layer M={m} K={k} N={n} G={g} rank={rank} bias={bias} act={act}", flush=True)
    inp, q, sx, w, ws, kw = _operands(oracle_lib, m, k, n, g, rank, bias, seed=m * 31 + n * 7 + k)
    plain = int8_matmul(q, w, sx, ws, **kw)
    fused = int8_matmul(q, w, sx, ws, activation=act, **kw) if act != "none" else None
    torch.cuda.synchronize()
    ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
    np.testing.assert_array_equal(sx.cpu().numpy().view(np.uint32), ref["sx"].view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), ref["xq"])
    if not rank and not bias:
        np.testing.assert_array_equal(bits_of(plain), ref["y"])
    else:
        want = oracle_lib.bf16_to_f32(oracle_lib.fused_epilogue(
            ref["acc"], ref["sx"], inp["wscale"], bits_of(kw["u"]) if rank else None, inp["up"] if rank else None,
            inp["bias"] if bias else None))
        got = oracle_lib.bf16_to_f32(bits_of(plain))
        assert (np.abs(got - want) <= np.abs(want) * 2.0**-7 + 1e-6).all()
        assert (got == want).mean() > 0.98
    if act == "gelu_tanh":
        check_gelu(bits_of(fused), bits_of(plain), oracle_lib)
    elif act == "swiglu":
        assert fused.shape == (m, n // 2)
        check_swiglu(bits_of(fused), bits_of(plain), oracle_lib)
