"""MI355X-native INT8 "convrot" linear for HyperFlow H3 Flash: a drop-in for ``hyperflow_h3_flash.int8``.

Importing the package does not touch the GPU or load the HIP library; the first device forward does.
"""

from .int8 import (
    ACTIVATIONS,
    ARITHMETIC_OPTIONS,
    INT8_GEMMS,
    KERNEL_OPTIONS,
    ROTATE_ARITHMETICS,
    ROTATE_QUANTS,
    Int8RotLinear,
    hadamard_factors,
    regular_hadamard,
    resolve_int8_gemm,
    set_arithmetic_options,
    set_kernel_options,
)
from .lowrank import RANK_MULTIPLE, LowRankLinear, fuse_qkv, set_lowrank_rank_multiple

__version__ = "0.1.0"

__all__ = [
    "ACTIVATIONS",
    "ARITHMETIC_OPTIONS",
    "INT8_GEMMS",
    "KERNEL_OPTIONS",
    "ROTATE_ARITHMETICS",
    "ROTATE_QUANTS",
    "Int8RotLinear",
    "LowRankLinear",
    "RANK_MULTIPLE",
    "fuse_qkv",
    "hadamard_factors",
    "regular_hadamard",
    "resolve_int8_gemm",
    "set_arithmetic_options",
    "set_kernel_options",
    "set_lowrank_rank_multiple",
]
