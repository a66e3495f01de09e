"""Few-row shapes: the split-K GEMM (int32 partial planes + the epilogue pass) and the split-K low-rank down
projection against the unsplit kernels and the oracle.

Bars: the split GEMM bitwise equal to the unsplit one (integer partial sums add exactly; the epilogue is the same
arithmetic in the same order), and bitwise equal to the oracle without a low-rank branch or bias; the split
low-rank down projection within the error bound of an fp32 sum in any order plus one bf16 rounding of the oracle's
exactly rounded sum, and bitwise on almost every element.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch
from golden_utils import within_fp32_sum_bound

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


def p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def run_linear(lib, q, w, sx, ws, u, up, bias, split):
    m, k = q.shape
    n = w.shape[0]
    r = 0 if u is None else u.shape[1]
    y = torch.full((m, n), -1, device=DEV, dtype=torch.int16).view(torch.bfloat16)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (p(q), k, p(w), k, p(sx), p(ws), p(u), r if r else 0, p(up), r if r else 0, r, p(bias), p(y), n, m, n, k)
    if split:
        nbytes = lib.hf_int8_linear_ws_bytes(m, n, k, r, 0)
        assert nbytes > 0, "this shape should take the split path"
        work = torch.empty(nbytes, device=DEV, dtype=torch.uint8)
        status = lib.hf_int8_linear_ws(*args, p(work), nbytes, stream)
    else:
        status = lib.hf_int8_linear(*args, stream)
    assert status == 0
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("m,n,k,r,bias", [(1, 30720, 5120, 0, False), (64, 16384, 2048, 0, False),
                                          (64, 15000, 5120, 32, True), (200, 3072, 3072, 64, False),
                                          (37, 1000, 2048, 136, True), (256, 5120, 5120, 32, False),
                                          (100, 3000, 3072, 32, True), (128, 30720, 1024, 0, False),
                                          (256, 8192, 2048, 0, False),
                                          # K a multiple of 16 but not of the 128-byte stage: partial last stages
                                          (64, 12288, 1040, 0, False), (200, 2048, 2064, 0, False),
                                          (256, 3072, 1040, 32, True), (17, 10000, 2064, 8, False)])
def test_split_gemm_is_bitwise_the_unsplit_gemm(oracle_lib, m, n, k, r, bias):
    from hyperflow_h3_flash_amd import _native
    from hyperflow_h3_flash_amd.int8 import rotate_quant

    lib = _native.library()
    g = 256 if k % 256 == 0 else 16
    inp = oracle_lib.make_inputs(m, k, n, g, rank=r, bias=bias, seed=m + n + r)
    x = to_dev_bf16(inp["x"])
    q, sx = rotate_quant(x, g)
    w = torch.from_numpy(inp["qweight"]).to(DEV)
    ws = torch.from_numpy(inp["wscale"]).to(DEV)
    u = up = b = None
    if r:
        from hyperflow_h3_flash_amd.int8 import lowrank_down

        u = lowrank_down(x, to_dev_bf16(inp["down"]))
        up = to_dev_bf16(inp["up"])
    if bias:
        b = to_dev_bf16(inp["bias"])
    split = run_linear(lib, q, w, sx, ws, u, up, b, True)
    whole = run_linear(lib, q, w, sx, ws, u, up, b, False)
    assert torch.equal(split.view(torch.int16), whole.view(torch.int16))
    if not r and not bias:
        ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
        np.testing.assert_array_equal(bits_of(split), ref["y"])
    elif not r:
        ref = oracle_lib.convrot_linear(inp["x"], inp["qweight"], inp["wscale"], g)
        fused = oracle_lib.fused_epilogue(ref["acc"], ref["sx"], inp["wscale"], None, None, inp["bias"])
        np.testing.assert_array_equal(bits_of(split), fused)


@pytest.mark.parametrize("m,k,r", [(400, 5120, 136), (1100, 5120, 136), (2000, 13824, 32), (1500, 5120, 64)])
def test_split_lowrank_down_matches_oracle(oracle_lib, m, k, r):
    from hyperflow_h3_flash_amd import _native
    from hyperflow_h3_flash_amd.int8 import lowrank_down

    assert _native.library().hf_lowrank_down_ws_bytes(m, k, r) > 0, "this shape should take the split path"
    inp = oracle_lib.make_inputs(m, k, 8, 256, rank=r, seed=k + r)
    u = lowrank_down(to_dev_bf16(inp["x"]), to_dev_bf16(inp["down"]))
    got = oracle_lib.bf16_to_f32(bits_of(u))
    ref = oracle_lib.bf16_to_f32(oracle_lib.lowrank_down(inp["x"], inp["down"]))
    assert within_fp32_sum_bound(got, ref, oracle_lib.bf16_to_f32(inp["x"]), oracle_lib.bf16_to_f32(inp["down"]))
    assert (got == ref).mean() > 0.99


@pytest.mark.parametrize("m,k,r", [(1, 5120, 32), (7, 1024, 8), (64, 5120, 64), (100, 13824, 32), (256, 5376, 32),
                                   (33, 16384, 136), (200, 3072, 40), (250, 7168, 64), (9, 2048, 12), (5, 1024, 1),
                                   (384, 5120, 32)])
def test_lowrank_down_by_rows_matches_oracle(oracle_lib, m, k, r):
    """Up to 384 rows, without a workspace, the down projection runs a workgroup per row and 8 ranks (no split):
    within the fp32-sum bound of the oracle's exactly rounded sum, bitwise on almost every element; a partial last
    1024-element tile (K=5376), the widest row (K=16384), rank counts of 1 to 17 groups of 8 and ranks that are not
    a multiple of 8 (12, 1). With a workspace the same rows take the row kernel while M * K <= 1.7e6 (the size query
    then asks for none) and the split MFMA kernel beyond (250 x 7168, 384 x 5120)."""
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    assert (lib.hf_lowrank_down_ws_bytes(m, k, r) == 0) == (m * k <= 1.7e6)
    inp = oracle_lib.make_inputs(m, k, 8, 256, rank=r, seed=k + r + m)
    x, down = to_dev_bf16(inp["x"]), to_dev_bf16(inp["down"])
    u = torch.empty(m, r, device=DEV, dtype=torch.bfloat16)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.hf_lowrank_down(ctypes.c_void_p(x.data_ptr()), k, ctypes.c_void_p(down.data_ptr()), k,
                               ctypes.c_void_p(u.data_ptr()), r, m, k, r, stream) == 0
    torch.cuda.synchronize()
    got = oracle_lib.bf16_to_f32(bits_of(u))
    ref = oracle_lib.bf16_to_f32(oracle_lib.lowrank_down(inp["x"], inp["down"]))
    assert within_fp32_sum_bound(got, ref, oracle_lib.bf16_to_f32(inp["x"]), oracle_lib.bf16_to_f32(inp["down"]))
    assert (got == ref).mean() > 0.99


def test_lowrank_down_by_rows_strides_and_launch_independence(oracle_lib):
    """Row strides wider than K and r; a row's outputs are the same whichever rows share its launch (the rows run
    independently), so a one-row launch reproduces every row of a 200-row launch bit for bit."""
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    m, k, r = 200, 3072, 24
    inp = oracle_lib.make_inputs(m, k, 8, 256, rank=r, seed=3)
    xw = np.zeros((m, k + 40), dtype=np.uint16)
    xw[:, :k] = inp["x"]
    dw = np.zeros((r, k + 8), dtype=np.uint16)
    dw[:, :k] = inp["down"]
    x, d = to_dev_bf16(xw), to_dev_bf16(dw)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    u = torch.full((m, r + 8), -1, device=DEV, dtype=torch.int16).view(torch.bfloat16)
    assert lib.hf_lowrank_down(p(x), k + 40, p(d), k + 8, p(u), r + 8, m, k, r, stream) == 0
    rows = [0, 77, 199]
    one = torch.empty((1, r), device=DEV, dtype=torch.bfloat16)
    for row in rows:
        assert lib.hf_lowrank_down(p(x[row:]), k + 40, p(d), k + 8, p(one), r, 1, k, r, stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(one[0].view(torch.int16), u[row, :r].view(torch.int16))
    torch.cuda.synchronize()
    assert (u[:, r:].view(torch.int16) == -1).all()
    got = oracle_lib.bf16_to_f32(bits_of(u[:, :r]))
    ref = oracle_lib.bf16_to_f32(oracle_lib.lowrank_down(inp["x"], inp["down"]))
    assert within_fp32_sum_bound(got, ref, oracle_lib.bf16_to_f32(inp["x"]), oracle_lib.bf16_to_f32(inp["down"]))
    assert (got == ref).mean() > 0.99


def test_large_shapes_do_not_split():
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    assert lib.hf_int8_linear_ws_bytes(32768, 15360, 5120, 64, 0) == 0
    assert lib.hf_lowrank_down_ws_bytes(32768, 5120, 64) == 0


@pytest.mark.parametrize("m,n,k,r,bias,act", [
    (37710, 5376, 14336, 0, False, 0),   # the model's FFN down projection at M=37710: 334 trailing rows split over K
    (37710, 5376, 14336, 64, True, 0),   # with the low-rank term and bias
    (37408, 5376, 14336, 0, False, 1),   # 32 trailing rows (the one-pass few-row kernel, no workspace), tanh-GELU
    (37710, 7168, 14336, 32, True, 2),   # SwiGLU: the split partials in pair order
])
def test_trailing_tile_rows_split_is_bitwise_the_whole_gemm(oracle_lib, m, n, k, r, bias, act):
    """Many-tile GEMMs whose last round of the persistent grid would be less than half full run their trailing tile
    rows as a few-row GEMM: split over K (hf_int8_linear_ws_bytes > 0 for them; the result equals the whole unsplit
    GEMM that runs without the workspace, bitwise), or, for at most 64 trailing rows, the one-pass kernel, which
    needs no workspace (so both calls peel). Both parts against the oracle on sampled rows."""
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    nbytes = lib.hf_int8_linear_ws_bytes(m, n, k, r, act)
    one_pass_tail = m % 256 <= 64
    assert (nbytes == 0) if one_pass_tail else (nbytes > 0), nbytes
    gen = torch.Generator(device=DEV).manual_seed(m + n + k)
    q = torch.randint(-127, 128, (m, k), device=DEV, dtype=torch.int8, generator=gen)
    sx = torch.rand(m, device=DEV, generator=gen) * 1e-2 + 1e-3
    w = torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen)
    sw = torch.rand(n, device=DEV, generator=gen) * 9e-3 + 1e-3
    u = (torch.randn(m, r, device=DEV, generator=gen) * 0.5).to(torch.bfloat16) if r else None
    up = (torch.randn(n, r, device=DEV, generator=gen) * 0.02).to(torch.bfloat16) if r else None
    b = (torch.randn(n, device=DEV, generator=gen) * 0.01).to(torch.bfloat16) if bias else None
    n_out = n // 2 if act >= 2 else n
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run(split):
        y = torch.full((m, n_out), -1, device=DEV, dtype=torch.int16).view(torch.bfloat16)
        work = torch.empty(nbytes, device=DEV, dtype=torch.uint8) if split and nbytes else None
        status = lib.hf_int8_linear_act_ws(p(q), k, p(w), k, p(sx), p(sw), p(u), r, p(up), r, r, p(b), act, p(y),
                                           n_out, m, n, k, p(work), nbytes if split else 0, stream)
        assert status == 0
        torch.cuda.synchronize()
        return y

    split, whole = run(True), run(False)
    assert torch.equal(split.view(torch.int16), whole.view(torch.int16))
    if not r and not bias:
        tail = m - m % 256
        rows = np.sort(np.concatenate([np.random.default_rng(m).choice(tail, size=6, replace=False),
                                       np.random.default_rng(n).choice(np.arange(tail - 512, m), size=6,
                                                                       replace=False)]))
        want = oracle_lib.epilogue(oracle_lib.int8_gemm(q[rows].cpu().numpy(), w.cpu().numpy()),
                                   sx[rows].cpu().numpy(), sw.cpu().numpy())
        if act == 1:
            from test_gpu_activation import check_gelu

            check_gelu(bits_of(split[rows]), want, oracle_lib)
        else:
            np.testing.assert_array_equal(bits_of(split[rows]), want)
