"""hf_convrot_linear_noalloc, the entry point that allocates nothing (its workspace is a scratch array in the
library's code object), against hf_convrot_linear_ws with a workspace of the size it asks for: bitwise equal outputs
(the same kernels and the same split plan), on two calls in a row, the second with a smaller input, so the second
call runs on scratch that still holds the first call's partial sums. Also: a call needing more than the scratch holds
is refused before anything is launched."""

from __future__ import annotations

import ctypes

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


def p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def case(m, k, n, r, bias, seed):
    gen = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(m, k, device=DEV, generator=gen)
    x[:, :: max(1, k // 25)] *= 30.0
    return {
        "x": x.to(torch.bfloat16),
        "w": torch.randint(-127, 128, (n, k), device=DEV, dtype=torch.int8, generator=gen),
        "ws": torch.rand(n, device=DEV, generator=gen) * 9e-3 + 1e-3,
        "down": (torch.randn(r, k, device=DEV, generator=gen) * 0.02).to(torch.bfloat16) if r else None,
        "up": (torch.randn(n, r, device=DEV, generator=gen) * 0.02).to(torch.bfloat16) if r else None,
        "bias": (torch.randn(n, device=DEV, generator=gen) * 0.01).to(torch.bfloat16) if bias else None,
        "m": m, "k": k, "n": n, "r": r,
    }


def run(lib, c, noalloc: bool, act: int = 0):
    m, k, n, r = c["m"], c["k"], c["n"], c["r"]
    q = torch.empty(m, k, device=DEV, dtype=torch.int8)
    sx = torch.empty(m, device=DEV, dtype=torch.float32)
    u = torch.empty(m, max(r, 1), device=DEV, dtype=torch.bfloat16)
    width = n // 2 if act >= 2 else n
    y = torch.full((m, width), -1, device=DEV, dtype=torch.int16).view(torch.bfloat16)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    head = (p(c["x"]), k, p(q), p(sx), 0, 0, p(c["w"]), k, p(c["ws"]), p(c["down"]), k, p(c["up"]), r, r,
            p(c["bias"]), act, 256, p(u), p(y), width, m, n, k)
    if noalloc:
        status = lib.hf_convrot_linear_noalloc(*head, stream)
    else:
        nbytes = lib.hf_convrot_linear_ws_bytes(m, n, k, r, act)
        work = torch.empty(max(nbytes, 1), device=DEV, dtype=torch.uint8)
        status = lib.hf_convrot_linear_ws(*head, p(work) if nbytes else None, nbytes, stream)
    assert status == 0, status
    torch.cuda.synchronize()
    return y.view(torch.int16).cpu().numpy()


# (m, k, n, rank, bias, activation), every call using the scratch: the split low-rank down projection ahead of the
# 128-row band tiles, then the skinny kernel's K split; the skinny K split at 128 and at 64 rows (too many weight slices
# for the one-pass kernel); SwiGLU in pair order, then tanh-GELU, both split over K. Each pair runs the larger input
# first.
PAIRS = [
    ((1024, 5120, 5120, 32, True, 0), (300, 3072, 3072, 64, False, 0)),
    ((128, 5120, 30720, 32, False, 0), (64, 5120, 30720, 32, True, 0)),
    ((200, 5376, 14336, 64, True, 2), (17, 2048, 16384, 16, False, 1)),
]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_the_workspace_entry_point_twice(first, second):
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    limit = lib.hf_convrot_linear_noalloc_max_bytes()
    for i, (m, k, n, r, bias, act) in enumerate((first, second)):
        print(f"noalloc call {i}: M={m} K={k} N={n} r={r} bias={bias} act={act}", flush=True)
        need = lib.hf_convrot_linear_ws_bytes(m, n, k, r, act)
        assert 0 < need <= limit, "the case should use the scratch"
        c = case(m, k, n, r, bias, seed=m + n + i)
        got = run(lib, c, True, act)
        want = run(lib, c, False, act)
        np.testing.assert_array_equal(got, want)
        assert (got != -1).all()


def test_noalloc_refuses_calls_beyond_its_scratch():
    from hyperflow_h3_flash_amd import _native

    lib = _native.library()
    m, k, n, r = 2048, 14336, 5120, 32  # split over K: 126 MB of int32 partial planes
    assert lib.hf_convrot_linear_ws_bytes(m, n, k, r, 0) > lib.hf_convrot_linear_noalloc_max_bytes()
    c = case(8, k, n, r, False, seed=1)  # the buffers are never touched: the size check comes first
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    status = lib.hf_convrot_linear_noalloc(p(c["x"]), k, None, None, 0, 0, p(c["w"]), k, p(c["ws"]), p(c["down"]), k,
                                           p(c["up"]), r, r, None, 0, 256, None, None, n, m, n, k, stream)
    assert status == -6
    assert "scratch" in _native.status_text(status)
