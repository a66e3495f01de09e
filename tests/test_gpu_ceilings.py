"""The benchmark's matrix-core ceiling kernel (libhf_ceilings.so) runs its MFMAs: zero operands leave every
accumulator zero, and random codes give the same nonzero fold on every launch (integer sums are exact)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_mfma_ceiling_kernel_runs_its_products():
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    lib = _native.ceilings_library()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev).cuda_stream
    grid, rounds = 8, 16
    print(f"ceiling kernel grid={grid} rounds={rounds}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(3)
    outs = []
    for table in (torch.zeros(8192, dtype=torch.int8, device=dev),
                  torch.randint(-127, 128, (8192,), dtype=torch.int8, device=dev, generator=gen)):
        for _ in range(2):
            out = torch.full((grid * 512,), -1, dtype=torch.int32, device=dev)
            assert lib.hf_ceiling_mfma_i8(table.data_ptr(), rounds, grid, out.data_ptr(), stream) == 0
            outs.append(out.cpu())
    assert (outs[0] == 0).all() and (outs[1] == 0).all()
    assert torch.equal(outs[2], outs[3]) and (outs[2] != 0).any()
    # every workgroup computes the same products
    per_group = outs[2].view(grid, 512)
    assert (per_group == per_group[0]).all()


@pytest.mark.parametrize("reads,writes,unroll,grid", [(2, 1, 4, 3), (2, 1, 8, 5), (1, 1, 4, 2), (2, 0, 8, 4)])
def test_stream_ceiling_kernel_moves_every_byte(reads, writes, unroll, grid):
    """The streaming ceiling kernel reads every source vector and writes the xor of each unit's loads to every
    destination vector (a grid smaller than the units, so the rounds stride); the read-only form folds each
    thread's loads into `out`."""
    if not torch.cuda.is_available():
        pytest.fail("no ROCm device visible")
    from hyperflow_h3_flash_amd import _native

    lib = _native.ceilings_library()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev).cuda_stream
    units = 64 * 97
    print(f"stream ceiling reads={reads} writes={writes} unroll={unroll} grid={grid} units={units}", flush=True)
    gen = torch.Generator(device=dev).manual_seed(reads + writes + unroll)
    src = torch.randint(-2**31, 2**31 - 1, (units * reads * 4,), dtype=torch.int32, device=dev, generator=gen)
    dst = torch.full((max(units * writes * 4, 4),), -1, dtype=torch.int32, device=dev)
    out = torch.full((grid * 256,), -1, dtype=torch.int32, device=dev)
    assert lib.hf_ceiling_stream(src.data_ptr(), dst.data_ptr() if writes else None, units, reads, writes, unroll,
                                 grid, out.data_ptr(), stream) == 0
    torch.cuda.synchronize()
    # unit i of wave-group g reads vectors (g * reads + r) * 64 + i % 64
    v = src.view(units // 64, reads, 64, 4)
    x = v[:, 0]
    for r in range(1, reads):
        x = x ^ v[:, r]
    if writes:
        assert torch.equal(dst.view(units // 64, 64, 4), x)
    else:
        threads = grid * 256  # thread t folds units t, t + threads, ...
        per_unit = x.reshape(units, 4).cpu().numpy()
        lanes = np.bitwise_xor.reduce(per_unit, axis=1)
        padded = np.zeros(-(-units // threads) * threads, dtype=np.int32)
        padded[:units] = lanes
        want = np.bitwise_xor.reduce(padded.reshape(-1, threads), axis=0)
        np.testing.assert_array_equal(out.cpu().numpy(), want)
