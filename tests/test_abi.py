"""The C ABI: the built library loads and exports every function include/hf_convrot.h declares, and argument checks
reject bad calls before any HIP call. CPU only: no kernel is launched here."""

from __future__ import annotations

import ctypes
import os
import re

import pytest

from hyperflow_h3_flash_amd import _native

HEADER = os.path.join(_native.REPO_DIR, "include", "hf_convrot.h")


def declared_functions() -> list[str]:
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(hf_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_native.LIB_PATH):
        pytest.fail(f"{_native.LIB_PATH} not built: run __graft_entry__.build()")
    return _native.library()


def test_header_and_binding_agree():
    names = declared_functions()
    assert sorted(names) == sorted(_native.SIGNATURES), names


def test_library_exports_every_declared_function(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name


def test_version_and_status_text(lib):
    assert lib.hf_version().decode().startswith("hf_convrot ")
    assert "gfx950" in lib.hf_version().decode()
    for code in (0, -1, -2, -3, -4, -5):
        assert lib.hf_strerror(code)
    assert lib.hf_strerror(-99) == b"unknown status"


def test_argument_checks_reject_before_launching(lib):
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: every call below fails validation first
    odd = ctypes.c_void_p((1 << 20) + 4)
    null = None
    # null pointers
    assert lib.hf_rotate_quant(null, 256, fake, 256, fake, 4, 256, 256, null) == -1
    # zero rows is a no-op success
    assert lib.hf_rotate_quant(null, 256, null, 256, null, 0, 256, 256, null) == 0
    # unsupported group / group not dividing K
    assert lib.hf_rotate_quant(fake, 256, fake, 256, fake, 4, 256, 32, null) == -2
    assert lib.hf_rotate_quant(fake, 320, fake, 320, fake, 4, 320, 256, null) == -2
    # misaligned pointer, K not a multiple of 16
    assert lib.hf_rotate_quant(odd, 256, fake, 256, fake, 4, 256, 256, null) == -3
    assert lib.hf_rotate_quant(fake, 8, fake, 8, fake, 4, 8, 4, null) == -3
    # the arithmetic selector: unknown codes are rejected; both known codes check operands the same way
    assert lib.hf_rotate_quant_ex(fake, 256, fake, 256, fake, 4, 256, 256, 2, null) == -1
    for arith in (0, 1):
        assert lib.hf_rotate_quant_ex(null, 256, null, 256, null, 0, 256, 256, arith, null) == 0
        assert lib.hf_rotate_quant_ex(fake, 256, fake, 256, fake, 4, 256, 32, arith, null) == -2
        assert lib.hf_rotate_quant_ex(odd, 256, fake, 256, fake, 4, 256, 256, arith, null) == -3
    # GEMM: stride smaller than K, misaligned stride, low-rank rank not a multiple of 8
    assert lib.hf_int8_linear(fake, 64, fake, 128, fake, fake, null, 0, null, 0, 0, null, fake, 64, 4, 64, 128,
                              null) == -1
    assert lib.hf_int8_linear(fake, 136, fake, 136, fake, fake, null, 0, null, 0, 0, null, fake, 64, 4, 64, 130,
                              null) == -3
    assert lib.hf_int8_linear(fake, 128, fake, 128, fake, fake, fake, 12, fake, 12, 12, null, fake, 64, 4, 64, 128,
                              null) == -3
    assert lib.hf_int8_gemm_i32(fake, 128, fake, 128, odd, 64, 4, 64, 128, null) == -3
    assert lib.hf_lowrank_down(fake, 128, fake, 128, fake, 4, 4, 128, 8, null) == -1  # ldu < r
    assert lib.hf_lowrank_down(fake, 128, fake, 128, fake, 8, 4, 120, 8, null) == -3  # K % 16
    assert lib.hf_lowrank_up(fake, 8, fake, 8, 16, null, fake, 64, 4, 64, null) == -1  # ldu < r
    assert lib.hf_lowrank_up(fake, 16, fake, 16, 12, null, fake, 64, 4, 64, null) == -3  # r % 8
    assert lib.hf_lowrank_up(odd, 16, fake, 16, 16, null, fake, 64, 4, 64, null) == -3  # u alignment
    assert lib.hf_lowrank_up(null, 16, null, 16, 16, null, null, 64, 0, 64, null) == 0  # no rows: no-op
    # an activation code the epilogue does not know, even with nothing to compute
    assert lib.hf_int8_linear_act_ws(fake, 128, fake, 128, fake, fake, null, 0, null, 0, 0, null, 7, fake, 64, 4, 64,
                                     128, null, 0, null) == -1
    assert lib.hf_int8_linear_act_ws(null, 128, null, 128, null, null, null, 0, null, 0, 0, null, 4, null, 64, 0, 64,
                                     128, null, 0, null) == -1
    for act in (1, 2, 3):  # known activation, no rows: no-op
        assert lib.hf_int8_linear_act_ws(null, 128, null, 128, null, null, null, 0, null, 0, 0, null, act, null, 64, 0,
                                         64, 128, null, 0, null) == 0
    # SwiGLU: the width must split into two halves of a multiple of 16; the output is N / 2 wide, so ldy >= N / 2
    assert lib.hf_int8_linear_act_ws(fake, 128, fake, 128, fake, fake, null, 0, null, 0, 0, null, 2, fake, 64, 4, 48,
                                     128, null, 0, null) == -1
    assert lib.hf_int8_linear_act_ws(fake, 128, fake, 128, fake, fake, null, 0, null, 0, 0, null, 3, fake, 16, 4, 64,
                                     128, null, 0, null) == -1
    # pair order reads the whole weight through one 32-bit descriptor
    assert lib.hf_int8_linear_act_ws(fake, 1 << 16, fake, 1 << 16, fake, fake, null, 0, null, 0, 0, null, 2, fake,
                                     1 << 15, 4, 1 << 16, 128, null, 0, null) == -5
    # sizes beyond the kernels' index range
    assert lib.hf_int8_gemm_i32(fake, 1 << 24, fake, 128, fake, 64, 4, 64, 128, null) == -5


def test_split_planner_follows_the_measured_cost_models(lib):
    """The workspace size query reports whether a GEMM splits K (or peels its trailing tile rows into a split GEMM):
    0 means whole tiles. The choices below are the ones the measured cost models make on MI355X's 256 CUs (the
    count the library assumes when no device answers, as here): whole tiles where one round of them beats the split
    with its finishing pass (M=2048, N=K=5120: 65 against 85 us), a split where the tiles would leave three quarters
    of the CUs idle (M=512, N=4096, K=5120), a peel of the rows that would leave the last round a tenth full
    (M=3584, N=K=5120: 115 against 127 us), and whole tiles for the headline shape, whose 7680 tiles fill 30 rounds."""
    assert lib.hf_int8_linear_ws_bytes(2048, 5120, 5120, 0, 0) == 0
    assert lib.hf_int8_linear_ws_bytes(512, 4096, 5120, 0, 0) > 0
    assert lib.hf_int8_linear_ws_bytes(3584, 5120, 5120, 0, 0) > 0
    assert lib.hf_int8_linear_ws_bytes(32768, 15360, 5120, 64, 0) == 0
    assert lib.hf_int8_linear_ws_bytes(37710, 5376, 14336, 64, 0) > 0  # the model's down projection: peeled


def test_workspace_queries_report_what_the_route_uses(lib):
    """The size queries follow the kernel route the call takes: no workspace for the one-pass few-row kernel
    (M <= 64 with 32-row weight slices on a quarter to one round of CUs), for the 128-row band tiles (the M=1024, K=N=3072
    layer) or for the 256 x 128 tiles, the split plan's partial planes otherwise; both tile kernels cover rank <= 64
    without SwiGLU, so the same sizes with rank 96 or SwiGLU take the split path and report its planes."""
    assert lib.hf_int8_linear_ws_bytes(64, 5120, 5120, 32, 0) == 0  # one pass
    assert lib.hf_int8_linear_ws_bytes(17, 2048, 4096, 16, 1) == 0  # one pass, tanh-GELU
    assert lib.hf_int8_linear_ws_bytes(1024, 3072, 3072, 32, 0) == 0  # 128 x 96 band tiles
    assert lib.hf_int8_linear_ws_bytes(1024, 5120, 5120, 64, 1) == 0  # 128 x 160 band tiles, tanh-GELU
    assert lib.hf_int8_linear_ws_bytes(1024, 3072, 3072, 96, 0) > 0
    assert lib.hf_int8_linear_ws_bytes(1024, 3072, 3072, 32, 2) > 0  # SwiGLU
    assert lib.hf_int8_linear_ws_bytes(256, 30720, 5120, 32, 0) == 0  # 256 x 128 tiles
    assert lib.hf_int8_linear_ws_bytes(64, 30720, 5120, 32, 0) > 0  # 960 slices: more than one round, split
    # the whole layer adds the low-rank projection's split partials (or needs nothing more)
    assert lib.hf_convrot_linear_ws_bytes(64, 5120, 5120, 32, 0) == 0
    assert 0 < lib.hf_convrot_linear_ws_bytes(2241, 3072, 14336, 32, 0) <= lib.hf_convrot_linear_noalloc_max_bytes()
    assert lib.hf_convrot_linear_ws_bytes(2048, 5120, 14336, 32, 0) > lib.hf_convrot_linear_noalloc_max_bytes()


def test_ceilings_library_loads_and_rejects_bad_arguments():
    """The benchmark's calibration library (matrix-core ceiling) is built beside the C ABI's and checks its
    arguments before launching anything."""
    if not os.path.exists(_native.CEILINGS_LIB_PATH):
        pytest.fail(f"{_native.CEILINGS_LIB_PATH} not built: run __graft_entry__.build()")
    lib = _native.ceilings_library()
    assert lib.hf_ceiling_mfma_i8_macs(12000, 256) == 256 * 8 * 12000 * 8 * 32**3
    buf = ctypes.create_string_buffer(16)
    assert lib.hf_ceiling_mfma_i8(None, 1, 1, buf, None) == -1
    assert lib.hf_ceiling_mfma_i8(buf, 0, 1, buf, None) == -1
    assert lib.hf_ceiling_mfma_i8(buf, 1, 0, buf, None) == -1
    # the streaming ceiling: units a multiple of 64, a supported (reads, writes) pair and unroll, buffers present
    assert lib.hf_ceiling_stream(buf, buf, 100, 2, 1, 4, 1, buf, None) == -1
    assert lib.hf_ceiling_stream(buf, buf, 64, 3, 1, 4, 1, buf, None) == -1
    assert lib.hf_ceiling_stream(buf, buf, 64, 2, 1, 6, 1, buf, None) == -1
    assert lib.hf_ceiling_stream(buf, None, 64, 2, 1, 4, 1, buf, None) == -1
    assert lib.hf_ceiling_stream(buf, None, 64, 2, 0, 4, 1, None, None) == -1
    assert lib.hf_ceiling_stream(None, buf, 64, 1, 1, 4, 1, buf, None) == -1


def test_one_call_layer_checks_the_rotation_before_the_low_rank_projection(lib):
    """A layer whose low-rank projection splits K runs that projection before the rotation (the rotation kernel then
    adds the partial sums of its rows); the rotation's arguments are still checked before anything is launched."""
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: the calls below fail validation first
    odd = ctypes.c_void_p((1 << 20) + 4)
    m, n, k, r = 1024, 5120, 5120, 32
    ws_bytes = lib.hf_convrot_linear_ws_bytes(m, n, k, r, 0)
    assert ws_bytes > 0  # the projection splits K at this size

    def call(x, group):
        return lib.hf_convrot_linear_ws(x, k, fake, fake, 0, 0, fake, k, fake, fake, k, fake, r, r, None, 0, group,
                                        fake, fake, n, m, n, k, fake, ws_bytes, None)

    assert call(fake, 32) == -2  # 32 is not a power of 4
    assert call(fake, 4096) == -2  # does not divide K
    assert call(odd, 256) == -3  # x not 16-byte aligned
