"""The benchmark's matrix-core ceiling kernel (libhf_ceilings.so) runs its MFMAs: zero operands leave every
accumulator zero, and random codes give the same nonzero fold on every launch (integer sums are exact)."""

from __future__ import annotations

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
