"""ctypes binding of ``libhf_convrot.so`` (the C ABI of include/hf_convrot.h) and the build recipe that makes it.

The library is built in-tree by ``build_library()`` (hipcc, gfx950) and loaded from next to this file. There is no
fallback: when the library is missing or does not load, ``library()`` raises.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from functools import lru_cache

PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PACKAGE_DIR)
LIB_PATH = os.path.join(PACKAGE_DIR, "libhf_convrot.so")
SOURCE = os.path.join(PACKAGE_DIR, "csrc", "convrot_abi.hip")
#: The benchmark's calibration kernels (matrix-core ceiling), a library of their own outside the C ABI.
CEILINGS_LIB_PATH = os.path.join(PACKAGE_DIR, "libhf_ceilings.so")
CEILINGS_SOURCE = os.path.join(PACKAGE_DIR, "csrc", "ceilings.hip")
ARCH = "gfx950"

#: hipcc flags: CDNA4 only; fp-contract off keeps every multiply and add separately rounded as written; packed
#: fp32 instructions are disabled.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]

HF_OK = 0
STATUS_NAMES = {
    -1: "HF_ERR_ARGUMENT",
    -2: "HF_ERR_GROUP",
    -3: "HF_ERR_ALIGNMENT",
    -4: "HF_ERR_LAUNCH",
    -5: "HF_ERR_SIZE",
    -6: "HF_ERR_SCRATCH",
}

#: Every function include/hf_convrot.h declares, with its ctypes signature.
_P, _I64, _I32 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32
SIGNATURES = {
    "hf_version": ([], ctypes.c_char_p),
    "hf_strerror": ([ctypes.c_int], ctypes.c_char_p),
    "hf_rotate_quant": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I32, _P], ctypes.c_int),
    "hf_rotate_quant_ex": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I32, _I32, _P], ctypes.c_int),
    "hf_lowrank_down": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I32, _P], ctypes.c_int),
    "hf_lowrank_down_ws_bytes": ([_I64, _I64, _I32], ctypes.c_int64),
    "hf_lowrank_down_ws": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I32, _P, _I64, _P], ctypes.c_int),
    "hf_int8_linear_ws_bytes": ([_I64, _I64, _I64, _I32, _I32], ctypes.c_int64),
    "hf_int8_linear_ws": ([_P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _I32, _P, _P, _I64, _I64, _I64, _I64, _P,
                           _I64, _P], ctypes.c_int),
    "hf_int8_linear_act_ws": ([_P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _I32, _P, _I32, _P, _I64, _I64, _I64,
                               _I64, _P, _I64, _P], ctypes.c_int),
    "hf_lowrank_up": ([_P, _I64, _P, _I64, _I32, _P, _P, _I64, _I64, _I64, _P], ctypes.c_int),
    "hf_int8_linear": ([_P, _I64, _P, _I64, _P, _P, _P, _I64, _P, _I64, _I32, _P, _P, _I64, _I64, _I64, _I64, _P],
                       ctypes.c_int),
    "hf_int8_gemm_i32": ([_P, _I64, _P, _I64, _P, _I64, _I64, _I64, _I64, _P], ctypes.c_int),
    "hf_convrot_linear_ws_bytes": ([_I64, _I64, _I64, _I32, _I32], ctypes.c_int64),
    "hf_convrot_linear_ws": ([_P, _I64, _P, _P, _I32, _I32, _P, _I64, _P, _P, _I64, _P, _I64, _I32, _P, _I32, _I32,
                              _P, _P, _I64, _I64, _I64, _I64, _P, _I64, _P], ctypes.c_int),
    "hf_convrot_linear": ([_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I32, _P, _I32, _P, _P, _P, _P, _I64, _I64,
                           _I64, _I64, _P], ctypes.c_int),
    "hf_convrot_linear_noalloc_max_bytes": ([], ctypes.c_int64),
    "hf_convrot_linear_noalloc": ([_P, _I64, _P, _P, _I32, _I32, _P, _I64, _P, _P, _I64, _P, _I64, _I32, _P, _I32,
                                   _I32, _P, _P, _I64, _I64, _I64, _I64, _P], ctypes.c_int),
}


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = os.path.join(rocm, "bin", "hipcc")
    return path if os.path.exists(path) else "hipcc"


def _compile(source: str, target: str, verbose: bool) -> None:
    tmp = target + ".tmp"
    proc = subprocess.run([hipcc(), *HIPCC_FLAGS, "-o", tmp, source], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}) on {source}:\n{proc.stderr[-4000:]}")
    if verbose and proc.stderr:
        print(proc.stderr[-2000:])
    os.replace(tmp, target)


def build_library(verbose: bool = False) -> str:
    """Compile csrc/ into libhf_convrot.so, and the benchmark's libhf_ceilings.so, for gfx950 (always recompiles).
    Returns the convrot library's path."""
    _compile(SOURCE, LIB_PATH, verbose)
    _compile(CEILINGS_SOURCE, CEILINGS_LIB_PATH, verbose)
    library.cache_clear()
    ceilings_library.cache_clear()
    return LIB_PATH


@lru_cache(maxsize=None)
def library() -> ctypes.CDLL:
    """The loaded library with argument types set. Raises RuntimeError when it is missing or does not load."""
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950)"
        )
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:
        raise RuntimeError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


@lru_cache(maxsize=None)
def ceilings_library() -> ctypes.CDLL:
    """The benchmark's calibration library (csrc/ceilings.hip). Raises RuntimeError when it is missing."""
    if not os.path.exists(CEILINGS_LIB_PATH):
        raise RuntimeError(f"{CEILINGS_LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; "
                           "g.build()'`")
    lib = ctypes.CDLL(CEILINGS_LIB_PATH)
    lib.hf_ceiling_mfma_i8.argtypes = [_P, _I32, _I32, _P, _P]
    lib.hf_ceiling_mfma_i8.restype = ctypes.c_int
    lib.hf_ceiling_mfma_i8_macs.argtypes = [_I32, _I32]
    lib.hf_ceiling_mfma_i8_macs.restype = ctypes.c_int64
    lib.hf_ceiling_stream.argtypes = [_P, _P, _I64, _I32, _I32, _I32, _I32, _P, _P]
    lib.hf_ceiling_stream.restype = ctypes.c_int
    return lib


def status_text(status: int) -> str:
    return f"{STATUS_NAMES.get(status, status)}: {library().hf_strerror(status).decode()}"
