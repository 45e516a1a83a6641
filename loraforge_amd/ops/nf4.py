"""Exact NF4 tensor operations on gfx950 (mirror of ``loraforge.ops.nf4``).

Reference: ``src/loraforge/ops/nf4.py`` -- ``dequantize_nf4`` (:44-106) and
``prepare_scales`` (:109-148). The kernels are the HIP ones in
``csrc/nf4_dequant.hip``; ``prepare_scales`` reconstructs double-quantised
block scales natively instead of calling bitsandbytes.

``NF4State`` carries the attribute names of a bitsandbytes ``QuantState``
(``absmax, shape, code, dtype, blocksize, quant_type, offset, state2,
nested``) so either object can be passed; ``quantize_nf4`` is an offline
input-preparation utility equivalent to ``quantize_4bit(blocksize=64,
quant_type="nf4")`` and is not on the serving path.
"""

from __future__ import annotations

from dataclasses import dataclass

from .. import _lib
from ..annotations import ExperimentalAPI
from . import _checks

# ops/nf4.py:120-141.
NF4_CODE = (
    -1.0,
    -0.6961928009986877,
    -0.5250730514526367,
    -0.39491748809814453,
    -0.28444138169288635,
    -0.18477343022823334,
    -0.09105003625154495,
    0.0,
    0.07958029955625534,
    0.16093020117282867,
    0.24611230194568634,
    0.33791524171829224,
    0.44070982933044434,
    0.5626170039176941,
    0.7229568362236023,
    1.0,
)


@dataclass
class NestedState:
    """Second-level (double-quant) state: fp32 scales per ``blocksize`` absmax codes."""

    absmax: object
    code: object
    blocksize: int = 256


@dataclass
class NF4State:
    absmax: object  # fp32 [N*K/64], or uint8 codes when nested
    shape: tuple
    code: object  # fp32 [16]
    dtype: object = None
    blocksize: int = 64
    quant_type: str = "nf4"
    offset: object = None  # fp32 scalar tensor when nested
    state2: NestedState | None = None

    @property
    def nested(self) -> bool:
        return self.state2 is not None


def _code_tensor(device):
    import torch

    return torch.tensor(NF4_CODE, dtype=torch.float32, device=device)


def dynamic_map(device="cpu"):
    """Signed 8-bit dynamic code table used for double quantisation.

    Restates bitsandbytes' ``create_dynamic_map(signed=True)``: for decade
    ``i`` in 0..6, the midpoints of ``linspace(0.1, 1, 2**i + 1)`` scaled by
    ``10**(i-6)``, with both signs, plus 0 and 1, sorted (256 entries).
    """
    import torch

    data = []
    for i in range(7):
        bounds = torch.linspace(0.1, 1.0, 2**i + 1, dtype=torch.float32)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        data += ((10.0 ** (i - 6)) * means).tolist()
        data += (-(10.0 ** (i - 6)) * means).tolist()
    data += [0.0, 1.0]
    data.sort()
    return torch.tensor(data, dtype=torch.float32, device=device)


def quantize_nf4(weight, *, blocksize: int = 64, compress_statistics: bool = False):
    """Quantise a bf16 ``[N, K]`` weight to packed NF4; returns ``(qweight, NF4State)``.

    Offline utility (the reference uses bitsandbytes ``quantize_4bit``,
    ``benchmarks/prepare_qwen35_nf4.py:40-42``). Runs on the weight's device
    with PyTorch tensor ops. ``qweight`` is ``[N*K/2, 1]`` uint8, high nibble
    first.
    """
    import torch

    if blocksize != 64:
        raise ValueError("only blocksize 64 is supported")
    if weight.ndim != 2 or any(v % 64 for v in weight.shape):
        raise ValueError("weight must be 2D with dimensions that are multiples of 64")
    n, k = weight.shape
    device = weight.device
    w = weight.detach().float().reshape(-1, blocksize)
    absmax = w.abs().amax(dim=1)
    safe = torch.where(absmax > 0, absmax, torch.ones_like(absmax))
    normalised = w * (1.0 / safe)[:, None]
    code = _code_tensor(device)
    mids = (code[:-1].double() + code[1:].double()).div(2).float()
    nib = torch.bucketize(normalised, mids, right=True).to(torch.uint8)
    nib = torch.where(absmax[:, None] > 0, nib, torch.full_like(nib, 7)).reshape(-1)
    packed = ((nib[0::2] << 4) | nib[1::2]).to(torch.uint8).reshape(-1, 1)
    if not compress_statistics:
        return packed, NF4State(absmax.contiguous(), torch.Size((n, k)), code, weight.dtype, blocksize)
    offset = absmax.mean()
    centred = absmax - offset
    nb2 = (centred.numel() + 255) // 256
    padded = torch.zeros(nb2 * 256, dtype=torch.float32, device=device)
    padded[: centred.numel()] = centred
    absmax2 = padded.reshape(nb2, 256).abs().amax(dim=1)
    safe2 = torch.where(absmax2 > 0, absmax2, torch.ones_like(absmax2))
    norm2 = centred / safe2.repeat_interleave(256)[: centred.numel()]
    code2 = dynamic_map(device)
    idx = torch.bucketize(norm2, code2).clamp(1, 255)
    lower, upper = code2[idx - 1], code2[idx]
    q = torch.where((norm2 - lower).abs() <= (upper - norm2).abs(), idx - 1, idx).to(torch.uint8)
    state = NF4State(
        q.contiguous(),
        torch.Size((n, k)),
        code,
        weight.dtype,
        blocksize,
        offset=offset.reshape(()),
        state2=NestedState(absmax2.contiguous(), code2, 256),
    )
    return packed, state


def _check_code(code):
    import torch

    expected = _code_tensor(code.device)
    if code.dtype != torch.float32 or not torch.equal(expected, code.reshape(-1)):
        raise ValueError("requires the canonical NF4 codebook")


@ExperimentalAPI(reason="gfx950 native NF4 scale reconstruction; run once per weight version, before capture.")
def prepare_scales(state):
    """Own a lossless FP32 scale vector for immutable NF4 weights (``ops/nf4.py:109-148``).

    Nested (double-quantised) states are reconstructed on the GPU as
    ``fl32(fl32(code2[absmax[j]] * absmax2[j // blocksize2]) + offset)``.
    """
    import torch

    if state.quant_type != "nf4" or state.blocksize != 64 or state.dtype != torch.bfloat16:
        raise ValueError("requires NF4 block64 BF16 source weights")
    _check_code(state.code)
    if not state.nested:
        return state.absmax.contiguous()
    absmax = state.absmax.contiguous()
    state2 = state.state2
    device = absmax.device
    if device.type != "cuda":
        raise ValueError("nested scale reconstruction requires the same CUDA/ROCm GPU")
    _checks.require_arch(device)
    absmax2 = state2.absmax.contiguous().float()
    code2 = state2.code.contiguous().float()
    offset = state.offset.reshape(1).float().contiguous()
    if absmax.dtype != torch.uint8 or code2.numel() != 256:
        raise ValueError("nested state requires uint8 absmax codes and a 256-entry code2")
    if absmax2.numel() != -(-absmax.numel() // state2.blocksize):
        raise ValueError("nested absmax2 length disagrees with blocksize")
    out = torch.empty(absmax.numel(), dtype=torch.float32, device=device)
    lib = _lib.library()
    with torch.cuda.device(device):
        _lib.check(
            lib.lf_nf4_prepare_scales_dq(
                absmax.data_ptr(),
                absmax2.data_ptr(),
                code2.data_ptr(),
                offset.data_ptr(),
                int(state2.blocksize),
                out.data_ptr(),
                absmax.numel(),
                _lib.stream_of(device),
            )
        )
    return out


@ExperimentalAPI(reason="Validated on gfx950 with canonical NF4/block64 and BF16 output.")
def dequantize_nf4(qweight, scales, code, shape: tuple[int, int], *, out=None):
    """Reconstruct exact BF16 weights from contiguous packed NF4 bytes (``ops/nf4.py:44-106``).

    ``qweight`` holds N*K/2 uint8 bytes (high nibble first), ``scales`` N*K/64
    FP32 block scales and ``code`` the 16-entry FP32 codebook, all contiguous
    on one gfx950 device. ``out`` (optional) is a non-aliasing contiguous BF16
    ``[N, K]`` tensor. Runs on the current stream; there is no BF16 cache.
    """
    import torch

    if (
        not isinstance(shape, tuple)
        or len(shape) != 2
        or any(type(v) is not int or v <= 0 or v % 64 for v in shape)
    ):
        raise ValueError("shape must contain two positive multiples of64")
    size = shape[0] * shape[1]
    if any(not isinstance(t, torch.Tensor) for t in (qweight, scales, code)):
        raise TypeError("packed weights, scales and code must be tensors")
    device = qweight.device
    if device.type != "cuda" or any(t.device != device for t in (scales, code)):
        raise ValueError("all tensors must share one CUDA/ROCm device")
    _checks.require_arch(device)
    if (
        qweight.dtype != torch.uint8
        or qweight.numel() != size // 2
        or scales.dtype != torch.float32
        or scales.numel() != size // 64
        or code.dtype != torch.float32
        or code.numel() != 16
        or any(not t.is_contiguous() or t.requires_grad for t in (qweight, scales, code))
    ):
        raise ValueError("requires contiguous uint8 bytes, FP32 block64 scales and a 16-entry codebook")
    if out is not None:
        if (
            not isinstance(out, torch.Tensor)
            or out.device != device
            or out.dtype != torch.bfloat16
            or tuple(out.shape) != shape
            or not out.is_contiguous()
            or out.requires_grad
        ):
            raise ValueError("out must be contiguous BF16 [N,K] on the input device")
        if any(out.untyped_storage().data_ptr() == t.untyped_storage().data_ptr() for t in (qweight, scales, code)):
            raise ValueError("out must not alias an input storage")
    lib = _lib.library()
    with torch.cuda.device(device):
        if out is None:
            out = torch.empty(shape, device=device, dtype=torch.bfloat16)
        _lib.check(
            lib.lf_nf4_dequant(
                qweight.data_ptr(), scales.data_ptr(), code.data_ptr(), out.data_ptr(), size, _lib.stream_of(device)
            )
        )
    return out


def dequantize_nf4_nested(qweight, state, *, out=None):
    """Dequantise with double-quantised scales reconstructed inside the kernel."""
    import torch

    if not state.nested:
        return dequantize_nf4(qweight, state.absmax, state.code, tuple(state.shape), out=out)
    n, k = (int(v) for v in state.shape)
    device = qweight.device
    _checks.require_arch(device)
    _check_code(state.code)
    if qweight.dtype != torch.uint8 or qweight.numel() != n * k // 2 or not qweight.is_contiguous():
        raise ValueError("requires contiguous uint8 bytes")
    absmax = state.absmax.contiguous()
    absmax2 = state.state2.absmax.contiguous().float()
    code2 = state.state2.code.contiguous().float()
    offset = state.offset.reshape(1).float().contiguous()
    if absmax.dtype != torch.uint8 or absmax.numel() != n * k // 64 or code2.numel() != 256:
        raise ValueError("nested state requires uint8 absmax codes and a 256-entry code2")
    lib = _lib.library()
    with torch.cuda.device(device):
        if out is None:
            out = torch.empty((n, k), device=device, dtype=torch.bfloat16)
        _lib.check(
            lib.lf_nf4_dequant_dq(
                qweight.data_ptr(),
                absmax.data_ptr(),
                absmax2.data_ptr(),
                code2.data_ptr(),
                offset.data_ptr(),
                int(state.state2.blocksize),
                state.code.data_ptr(),
                out.data_ptr(),
                n * k,
                _lib.stream_of(device),
            )
        )
    return out
