"""INT8 W8A8 linears with a Hadamard-rotated input dimension, on MI355X (gfx950) HIP kernels.

A drop-in for the reference's ``hyperflow_h3_flash.int8`` (src/hyperflow_h3_flash/int8.py): the same
``Int8RotLinear(in_features, out_features, group)`` constructor, ``forward``, ``keep_input`` sharing and state dict
(``qweight`` int8 [N, K], ``wscale`` fp32 [N], frozen parameters, no buffers), the same ``regular_hadamard`` /
``hadamard_factors`` helpers and the same ``KERNEL_OPTIONS`` / ``set_kernel_options`` / ``resolve_int8_gemm`` API.

``y = (q(x R) @ qweight^T) * s_x * wscale`` with ``R = blockdiag(regular Hadamard of order group)``. For a device
tensor the layer is two launches of the hand-written kernels in ``csrc/`` (through the C ABI of include/hf_convrot.h):
the rotation + per-token quantization, then the INT8 MFMA GEMM with the rescale fused in its epilogue. The arithmetic
is that of the reference's torch path (int8.py:173-179): the rotated activation is rounded to bf16 before the absmax,
and the scale and code divisions are true fp32 divisions; the int32 accumulators are exact.

Host tensors run the same definition on the CPU (``host.py``), as the reference runs its torch statements for CPU
inputs (int8.py:161-167); a device tensor always runs the HIP kernels, at every row count, and raises when the HIP
library is missing (there is no other device backend).

Extension (opt-in, adds no tensors when unused): ``rank > 0`` adds the low-rank branch of the reference's
``LowRankLinear`` (``up(down(x))``, src/hyperflow_h3_flash/transformer.py:48-58) and ``bias=True`` a bf16 bias, both
fused into the GEMM epilogue: ``y = bf16((acc*sx)*wscale + bf16(x @ down^T) @ up^T + bias)``.

There is one backend. Every ``int8_gemm`` choice the reference accepts resolves to it, and both ``rotate_quant``
choices run the same exactly-rounded rotation (the reference's "factored" kernel differs from its dense one by
rare one-code roundings, int8.py:23-25; this build always produces the torch-path rounding).
"""

from __future__ import annotations

import ctypes
import functools
from types import SimpleNamespace
from typing import Any, ClassVar

import torch
from torch import Tensor, nn

from . import _native, host

#: Run-time kernel choices accepted for API compatibility with the reference (int8.py:37-39).
INT8_GEMMS = ("auto", "triton", "cublas", "sgl", "bf16")
ROTATE_QUANTS = ("dense", "factored")

#: The single backend every choice runs on.
BACKEND = "hip-gfx950"

#: Run-time kernel choices for every `Int8RotLinear` (int8.py:45-46).
KERNEL_OPTIONS: dict[str, Any] = {"int8_gemm": "auto", "rotate_quant": "dense"}

#: The arithmetic of the activation rotation + quantization (this build's option; the C ABI's HF_ROTATE_* codes):
#: "bf16_div" is the reference's torch path (int8.py:176-178: the rotated value rounded to bf16, a true division),
#: "f32_recip" the reference's GPU kernels (int8.py:194-262: the rotated value in fp32, a reciprocal multiply), the
#: arithmetic its pipeline runs on CUDA devices.
ROTATE_ARITHMETICS = {"bf16_div": 0, "f32_recip": 1}
ARITHMETIC_OPTIONS: dict[str, Any] = {"rotate_quant": "bf16_div"}


def set_kernel_options(*, int8_gemm: str | None = None, rotate_quant: str | None = None) -> None:
    """Validate and store kernel choices (int8.py:49-57): ValueError for names outside the reference's sets."""
    if int8_gemm is not None:
        if int8_gemm not in INT8_GEMMS:
            raise ValueError(f"int8_gemm must be one of {INT8_GEMMS}, got {int8_gemm!r}")
        KERNEL_OPTIONS["int8_gemm"] = int8_gemm
    if rotate_quant is not None:
        if rotate_quant not in ROTATE_QUANTS:
            raise ValueError(f"rotate_quant must be one of {ROTATE_QUANTS}, got {rotate_quant!r}")
        KERNEL_OPTIONS["rotate_quant"] = rotate_quant


def set_arithmetic_options(*, rotate_quant: str | None = None) -> None:
    """Select the rotation + quantization arithmetic for every later call (ValueError for other names)."""
    if rotate_quant is not None:
        if rotate_quant not in ROTATE_ARITHMETICS:
            raise ValueError(f"rotate_quant arithmetic must be one of {tuple(ROTATE_ARITHMETICS)}, got {rotate_quant!r}")
        ARITHMETIC_OPTIONS["rotate_quant"] = rotate_quant


def resolve_int8_gemm(device: torch.device | None = None) -> str:
    """The GEMM ``KERNEL_OPTIONS["int8_gemm"]`` runs as (int8.py:85-97): always the gfx950 HIP kernel here."""
    return BACKEND


@functools.cache
def regular_hadamard(group: int) -> Tensor:
    """The regular Hadamard matrix of order ``group`` as fp32 (int8.py:100-109): the Kronecker power of the
    normalised order-4 block, so every entry is +-2^-n, the matrix is its own transpose and inverse, and each row adds
    up to one. Computed in float64; ValueError unless ``group`` is 4^n."""
    h4 = torch.tensor([[1, 1, 1, -1], [1, 1, -1, 1], [1, -1, 1, 1], [-1, 1, 1, 1]], dtype=torch.float64) / 2
    h, n = torch.ones(1, 1, dtype=torch.float64), 1
    while n < group:
        h, n = torch.kron(h, h4), n * 4
    if n != group:
        raise ValueError(f"Hadamard group {group} is not a power of 4")
    return h.float()


def hadamard_factors(group: int) -> tuple[int, int] | None:
    """A split of ``group`` into two regular Hadamard orders, each 16 or more, whose Kronecker product is
    ``regular_hadamard(group)`` (int8.py:112-119): the smaller factor takes a quarter of the base-4 digits, rounded
    down. None below 256 or for an odd power of two."""
    n = group.bit_length() - 1
    if group < 256 or group != 1 << n or n % 2:
        return None
    ga = 4 ** (n // 4)
    return ga, group // ga


#: Groups the device rotation implements (powers of 4 up to 16384 that divide K; from 4096 on, K <= 20472).
DEVICE_GROUPS = (4, 16, 64, 256, 1024, 4096, 16384)


def _check_group(group: int) -> None:
    # ValueError for a non-power of 4, as the reference raises at first use; decided from the number alone (building
    # the matrix first would take 2 GiB at 16384 and 32 GiB at 65536).
    if group < 1 or group & (group - 1) or (group.bit_length() - 1) % 2:
        raise ValueError(f"Hadamard group {group} is not a power of 4")
    if group not in DEVICE_GROUPS:
        raise ValueError(f"Hadamard group {group} is not supported by the gfx950 kernels (supported: {DEVICE_GROUPS})")


class Int8RotLinear(nn.Module):
    """W8A8 linear on a block-Hadamard-rotated input, no bias by default (int8.py:127-179): the input is rotated,
    quantized to int8 with one scale per token, multiplied by the int8 ``qweight`` with an exact integer sum, and
    rescaled by the token scale and the per-output-channel ``wscale``.

    Projections that share one input (q, k and v of an attention block) rotate and quantize it once: a layer whose
    ``keep_input`` is set leaves ``(codes, scales)`` behind keyed by the input tensor's identity and version, the
    next layer takes them when it is handed that very tensor unchanged, and every layer call drops what it did not
    leave itself, so the codes never outlive the block (the cache of int8.py:150-159).

    ``rank``, ``bias`` and ``activation`` are this build's fused extension; with their defaults the module and its
    state dict are exactly the reference's. ``activation="gelu_tanh"`` applies torch's ``gelu(approximate="tanh")``
    to the bf16 output inside the GEMM (a feed-forward up-projection and its activation module in one kernel,
    transformer.py:75-99); ``activation="swiglu"`` is the gated feed-forward's input module: the ``out_features``
    outputs are split in halves and the layer returns ``hidden * silu(gate)``, ``out_features // 2`` wide
    (``"swiglu_gate_first"``: the gate half first). Activations add no state.
    """

    _last_input: ClassVar[dict[str, Any]] = {}

    def __init__(self, in_features: int, out_features: int, group: int, *, rank: int = 0, bias: bool = False,
                 activation: str | None = None) -> None:
        super().__init__()
        if _activation_code(activation) in _GLU_CODES and out_features % 32:
            raise ValueError(f"a gated activation needs out_features divisible by 32, got {out_features}")
        self.activation = activation
        if in_features % group:
            raise ValueError(f"in_features {in_features} is not a multiple of the Hadamard group {group}")
        if rank < 0:
            raise ValueError(f"rank must be >= 0, got {rank}")
        self.in_features, self.out_features, self.group = in_features, out_features, group
        self.rank = rank
        self.keep_input = False
        # Parameters, not buffers: offload hooks move parameters back to the host (int8.py:143-145).
        self.qweight = nn.Parameter(torch.zeros(out_features, in_features, dtype=torch.int8), requires_grad=False)
        self.wscale = nn.Parameter(torch.ones(out_features, dtype=torch.float32), requires_grad=False)
        if rank:
            # LowRankLinear's layout (transformer.py:52-54): down.weight [rank, in], up.weight [out, rank].
            self.down = nn.Linear(in_features, rank, bias=False, dtype=torch.bfloat16)
            self.up = nn.Linear(rank, out_features, bias=False, dtype=torch.bfloat16)
            for p in (self.down.weight, self.up.weight):
                p.requires_grad_(False)
        if bias:
            self.bias = nn.Parameter(torch.zeros(out_features, dtype=torch.bfloat16), requires_grad=False)
        else:
            self.bias = None

    def extra_repr(self) -> str:
        text = f"in_features={self.in_features}, out_features={self.out_features}, group={self.group}"
        if self.rank:
            text += f", rank={self.rank}"
        if self.bias is not None:
            text += ", bias=True"
        if self.activation is not None:
            text += f", activation={self.activation}"
        return text

    def _quantize(self, x: Tensor, x2: Tensor, kernels: SimpleNamespace) -> tuple[Tensor, Tensor]:
        cache = Int8RotLinear._last_input
        # Inference tensors (`torch.inference_mode`) have no version counter.
        version = None if x.is_inference() else x._version
        arithmetic = ARITHMETIC_OPTIONS["rotate_quant"]
        hit = (cache.get("x") is x and cache.get("version") == version and cache.get("group") == self.group
               and cache.get("arithmetic") == arithmetic)
        quantized = cache["value"] if hit else kernels.rotate_quant(x2, self.group)
        cache.clear()
        if self.keep_input:
            cache.update(x=x, version=version, group=self.group, arithmetic=arithmetic, value=quantized)
        return quantized

    def _forward_one_call(self, x: Tensor, x2: Tensor) -> Tensor:
        """The device layer as one library call (hf_convrot_linear_ws): the same kernels and arithmetic as the
        rotate_quant / lowrank_down / int8_matmul composition, with the host work of a call done once (the shared
        quantized input of int8.py:150-159 is handled here the same way)."""
        _check_group(self.group)
        M, K = x2.shape
        N = self.out_features
        dev = x2.device
        act = _activation_code(self.activation)
        _same_device(dev, self.qweight, self.wscale, self.bias)
        cache = Int8RotLinear._last_input
        version = None if x.is_inference() else x._version
        arithmetic = ARITHMETIC_OPTIONS["rotate_quant"]
        hit = (cache.get("x") is x and cache.get("version") == version and cache.get("group") == self.group
               and cache.get("arithmetic") == arithmetic)
        if hit:
            xq, sx = cache["value"]
        else:
            xq = torch.empty(M, K, device=dev, dtype=torch.int8)
            sx = torch.empty(M, device=dev, dtype=torch.float32)
        cache.clear()
        if self.keep_input:
            cache.update(x=x, version=version, group=self.group, arithmetic=arithmetic, value=(xq, sx))
        r = self.rank
        down = up = u = None
        if r:
            down, up = self.down.weight, self.up.weight
            _same_device(dev, down, up)
            if down.dtype != torch.bfloat16 or not down.is_contiguous():
                down = down.to(torch.bfloat16).contiguous()
            if up.dtype != torch.bfloat16 or not up.is_contiguous():
                up = up.to(torch.bfloat16).contiguous()
            u = torch.empty(M, r, device=dev, dtype=torch.bfloat16)
        bias = self.bias
        if bias is not None and (bias.dtype != torch.bfloat16 or not bias.is_contiguous()):
            bias = bias.to(torch.bfloat16).contiguous()
        w, ws_ = self.qweight, self.wscale
        if not w.is_contiguous():
            w = w.contiguous()
        if ws_.dtype != torch.float32 or not ws_.is_contiguous():
            ws_ = ws_.to(torch.float32).contiguous()
        y = torch.empty(M, N // 2 if act in _GLU_CODES else N, device=dev, dtype=torch.bfloat16)
        lib = _native.library()
        key = (M, N, K, r, act)
        nbytes = _ONE_CALL_WS.get(key)
        if nbytes is None:
            nbytes = _ONE_CALL_WS[key] = lib.hf_convrot_linear_ws_bytes(M, N, K, r, act)
        with torch.cuda.device(dev):
            work = torch.empty(nbytes, device=dev, dtype=torch.uint8) if nbytes > 0 else None
            status = lib.hf_convrot_linear_ws(
                _ptr(x2), x2.stride(0), _ptr(xq), _ptr(sx), int(hit), ROTATE_ARITHMETICS[arithmetic],
                _ptr(w), w.stride(0), _ptr(ws_), _ptr(down), down.stride(0) if r else 0, _ptr(up),
                up.stride(0) if r else 0, r, _ptr(bias), act, self.group, _ptr(u), _ptr(y), y.stride(0), M, N, K,
                _ptr(work), nbytes if work is not None else 0, _stream(dev))
        _check(status, "hf_convrot_linear_ws")
        return y

    def _forward_torch(self, x2: Tensor, rot: Tensor | None = None) -> Tensor:
        """The layer on host tensors (int8.py:173-179): ``host.py``'s evaluation of the device kernels' definition:
        the device's bits without a low-rank term (with or without the bias), within one bf16 ulp of them with one
        (the host sums the term exactly, the device in fp32). ``rot`` is accepted for the reference's signature; the
        rotation is always the regular Hadamard of ``self.group``."""
        xq, sx = host.rotate_quant(x2, self.group)
        acc = host.int8_gemm_exact(xq, self.qweight)
        u = host.lowrank_down(x2, self.down.weight) if self.rank else None
        y = host.dequantize(acc, sx, self.wscale, u=u, up=self.up.weight if self.rank else None, bias=self.bias)
        return host.activate(y, self.activation)

    def forward(self, x: Tensor) -> Tensor:
        shape = x.shape
        x2 = x.reshape(-1, self.in_features).to(torch.bfloat16).contiguous()
        if not x2.is_cuda:
            # Host tensors: the same arithmetic on the CPU (the reference's torch branch, int8.py:164-167).
            Int8RotLinear._last_input.clear()
            y = self._forward_torch(x2)
            return y.reshape(*shape[:-1], y.shape[-1]).to(x.dtype)
        kernels = _kernels()
        if kernels is None:
            Int8RotLinear._last_input.clear()
            raise RuntimeError(
                f"Int8RotLinear on {x2.device} needs the gfx950 HIP library ({_native.LIB_PATH}); build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (there is no other device backend)"
            )
        if (kernels.rotate_quant is rotate_quant and kernels.lowrank_down is lowrank_down
                and kernels.int8_matmul is int8_matmul and self.rank % 8 == 0):
            y = self._forward_one_call(x, x2)
            return y.reshape(*shape[:-1], y.shape[-1]).to(x.dtype)
        xq, sx = self._quantize(x, x2, kernels)
        if self.rank:
            u = kernels.lowrank_down(x2, self.down.weight)
            y = kernels.int8_matmul(xq, self.qweight, sx, self.wscale, u=u, up=self.up.weight, bias=self.bias,
                                    activation=self.activation)
        else:
            y = kernels.int8_matmul(xq, self.qweight, sx, self.wscale, bias=self.bias, activation=self.activation)
        return y.reshape(*shape[:-1], y.shape[-1]).to(x.dtype)


# ------------------------------------------------------------------------------------------------ device kernels


def _ptr(t: Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _workspace(device: torch.device, nbytes: int) -> tuple[Tensor | None, int]:
    """A device workspace of ``nbytes`` (None for 0) from torch's caching allocator; the kernels never allocate."""
    if nbytes <= 0:
        return None, 0
    return torch.empty(nbytes, device=device, dtype=torch.uint8), nbytes


def _check(status: int, what: str) -> None:
    if status == _native.HF_OK:
        return
    text = _native.status_text(status)
    if status in (-1, -2, -3, -5):
        raise ValueError(f"{what}: {text}")
    raise RuntimeError(f"{what}: {text}")


def _same_device(device: torch.device, *tensors: Tensor | None) -> None:
    for t in tensors:
        if t is not None and t.device != device:
            raise ValueError(f"tensor on {t.device}, expected {device}")


def rotate_quant(x: Tensor, group: int, arithmetic: str | None = None) -> tuple[Tensor, Tensor]:
    """(int8 codes [M, K], fp32 per-token scales [M]) of ``x`` (bf16 [M, K], rows contiguous), int8.py:326-344.

    ``arithmetic`` (default ``ARITHMETIC_OPTIONS["rotate_quant"]``): "bf16_div" (the reference's torch path) or
    "f32_recip" (the reference's GPU kernels)."""
    _check_group(group)
    if x.dtype != torch.bfloat16 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("rotate_quant expects a bf16 [M, K] tensor with contiguous rows")
    arithmetic = ARITHMETIC_OPTIONS["rotate_quant"] if arithmetic is None else arithmetic
    if arithmetic not in ROTATE_ARITHMETICS:
        raise ValueError(f"rotate_quant arithmetic must be one of {tuple(ROTATE_ARITHMETICS)}, got {arithmetic!r}")
    M, K = x.shape
    q = torch.empty(M, K, device=x.device, dtype=torch.int8)
    s = torch.empty(M, device=x.device, dtype=torch.float32)
    with torch.cuda.device(x.device):
        status = _native.library().hf_rotate_quant_ex(_ptr(x), x.stride(0), _ptr(q), q.stride(0), _ptr(s), M, K,
                                                      group, ROTATE_ARITHMETICS[arithmetic], _stream(x.device))
    _check(status, "hf_rotate_quant_ex")
    return q, s


def lowrank_down(x: Tensor, down: Tensor) -> Tensor:
    """``bf16(x @ down^T)`` for x bf16 [M, K] and down bf16 [r, K] (LowRankLinear.down, transformer.py:57)."""
    M, K = x.shape
    r = down.shape[0]
    _same_device(x.device, down)
    down = down.to(torch.bfloat16).contiguous()
    u = torch.empty(M, r, device=x.device, dtype=torch.bfloat16)
    lib = _native.library()
    with torch.cuda.device(x.device):
        ws, nbytes = _workspace(x.device, lib.hf_lowrank_down_ws_bytes(M, K, r))
        status = lib.hf_lowrank_down_ws(_ptr(x), x.stride(0), _ptr(down), down.stride(0), _ptr(u), u.stride(0), M, K,
                                        r, _ptr(ws), nbytes, _stream(x.device))
    _check(status, "hf_lowrank_down_ws")
    return u


def lowrank_up(u: Tensor, up: Tensor, bias: Tensor | None = None) -> Tensor:
    """``bf16(u @ up^T [+ bias])`` for u bf16 [M, r] and up bf16 [N, r] (LowRankLinear.up, transformer.py:57-58)."""
    M, r = u.shape
    N = up.shape[0]
    if up.shape[1] != r:
        raise ValueError(f"rank mismatch: {tuple(u.shape)} vs {tuple(up.shape)}")
    _same_device(u.device, up, bias)
    u, up = _pad_rank(u.to(torch.bfloat16), up.to(torch.bfloat16))
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    y = torch.empty(M, N, device=u.device, dtype=torch.bfloat16)
    with torch.cuda.device(u.device):
        status = _native.library().hf_lowrank_up(_ptr(u), u.stride(0), _ptr(up), up.stride(0), u.shape[1],
                                                 _ptr(bias), _ptr(y), y.stride(0), M, N, _stream(u.device))
    _check(status, "hf_lowrank_up")
    return y


def _pad_rank(u: Tensor, up: Tensor) -> tuple[Tensor, Tensor]:
    # The kernel reads the rank in 8-wide chunks; zero columns add exact zeros (transformer.py:60-73).
    r = u.shape[1]
    pad = -r % 8
    if pad:
        u = torch.nn.functional.pad(u, (0, pad))
        up = torch.nn.functional.pad(up, (0, pad))
    return u.contiguous(), up.contiguous()


#: Workspace bytes of the one-call layer per (M, N, K, rank), asked of the library once.
_ONE_CALL_WS: dict[tuple[int, int, int, int], int] = {}

#: Output activations the GEMM epilogue applies (the C ABI's HF_ACT_* codes). The gated ones halve the output width.
ACTIVATIONS = {None: 0, "gelu_tanh": 1, "swiglu": 2, "swiglu_gate_first": 3}
_GLU_CODES = (2, 3)


def _activation_code(activation: str | None) -> int:
    if activation not in ACTIVATIONS:
        raise ValueError(f"unsupported activation {activation!r}; expected one of {sorted(map(str, ACTIVATIONS))}")
    return ACTIVATIONS[activation]


def int8_matmul(a: Tensor, b: Tensor, sa: Tensor, sb: Tensor, *, u: Tensor | None = None, up: Tensor | None = None,
                bias: Tensor | None = None, activation: str | None = None) -> Tensor:
    """``bf16((f32(a @ b^T) * sa) * sb [+ u @ up^T] [+ bias])`` for a int8 [M, K], b int8 [N, K] (int8.py:376-390).

    ``activation="gelu_tanh"`` then applies torch's ``gelu(approximate="tanh")`` to that bf16 output in the same
    kernel (rounded to bf16 again), the feed-forward up-projection's activation (transformer.py:75-99);
    ``activation="swiglu"`` returns ``bf16(h * bf16(silu(g)))`` of the output's halves ``h, g = out.chunk(2, -1)``
    ([M, N / 2]; ``"swiglu_gate_first"``: ``g, h``), the gated feed-forward's input module."""
    act = _activation_code(activation)
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError(f"K mismatch: {a.shape} vs {b.shape}")
    if act in _GLU_CODES and N % 32:
        raise ValueError(f"a gated activation needs N divisible by 32, got {N}")
    _same_device(a.device, b, sa, sb, u, up, bias)
    a, b = a.contiguous(), b.contiguous()
    sa = sa.to(torch.float32).contiguous()
    sb = sb.to(torch.float32).contiguous()
    r = 0
    if u is not None:
        u, up = _pad_rank(u.to(torch.bfloat16), up.to(torch.bfloat16))
        r = u.shape[1]
    if bias is not None:
        bias = bias.to(torch.bfloat16).contiguous()
    c = torch.empty(M, N // 2 if act in _GLU_CODES else N, device=a.device, dtype=torch.bfloat16)
    lib = _native.library()
    with torch.cuda.device(a.device):
        ws, nbytes = _workspace(a.device, lib.hf_int8_linear_ws_bytes(M, N, K, r, act))
        status = lib.hf_int8_linear_act_ws(
            _ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(sa), _ptr(sb),
            _ptr(u), u.stride(0) if u is not None else 0, _ptr(up), up.stride(0) if up is not None else 0, r,
            _ptr(bias), act, _ptr(c), c.stride(0), M, N, K, _ptr(ws), nbytes, _stream(a.device))
    _check(status, "hf_int8_linear_act_ws")
    return c


def int8_gemm_i32(a: Tensor, b: Tensor) -> Tensor:
    """The exact int32 accumulator ``a @ b^T`` (the sum inside int8.py:302-306), for parity checks."""
    M, K = a.shape
    N = b.shape[0]
    _same_device(a.device, b)
    a, b = a.contiguous(), b.contiguous()
    acc = torch.empty(M, N, device=a.device, dtype=torch.int32)
    with torch.cuda.device(a.device):
        status = _native.library().hf_int8_gemm_i32(_ptr(a), a.stride(0), _ptr(b), b.stride(0), _ptr(acc),
                                                    acc.stride(0), M, N, K, _stream(a.device))
    _check(status, "hf_int8_gemm_i32")
    return acc


@functools.cache
def _kernels() -> SimpleNamespace | None:
    """The device kernels as a namespace shaped like the reference's ``_kernels()`` (int8.py:182-398); None when the
    HIP library is missing or does not load, as the reference returns None without Triton (int8.py:184-187). The
    layers then raise for device tensors (no device fallback) and still compute host tensors."""
    try:
        _native.library()
    except RuntimeError:
        return None
    return SimpleNamespace(
        rotate_quant=rotate_quant,
        int8_matmul=int8_matmul,
        lowrank_down=lowrank_down,
        lowrank_up=lowrank_up,
        int8_gemm_i32=int8_gemm_i32,
        backend=BACKEND,
    )


__all__ = [
    "ACTIVATIONS",
    "ARITHMETIC_OPTIONS",
    "INT8_GEMMS",
    "KERNEL_OPTIONS",
    "ROTATE_ARITHMETICS",
    "ROTATE_QUANTS",
    "Int8RotLinear",
    "hadamard_factors",
    "regular_hadamard",
    "resolve_int8_gemm",
    "set_arithmetic_options",
    "set_kernel_options",
]
