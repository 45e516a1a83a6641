"""Structural argument checks shared by the operators.

They mirror the reference's host-side contract checks
(``src/loraforge/ops/lora_rows.py:20-48``, ``ops/nf4.py:58-104``): exception
types and message fragments are kept so callers and tests match on the same
text ("same CUDA", "aligned", "inference", "length", "threads",
"share storage", "alias"). No check reads device memory.
"""

from __future__ import annotations

import functools

ARCH = "gfx950"


def tensor(t, name, ndim, dtype, device=None):
    import torch

    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.ndim != ndim or t.dtype != dtype:
        raise ValueError(f"{name} must be {ndim}D with dtype {dtype}")
    if any(size >= 2**31 for size in t.shape):
        raise ValueError(f"{name} dimensions must fit signed int32 indexing")
    if t.device.type != "cuda" or (device is not None and t.device != device):
        raise ValueError(f"{name} must be on the same CUDA/ROCm GPU")
    if t.requires_grad:
        raise ValueError("row operators are inference-only")


def vector(t, name, dtype, device, size=None):
    tensor(t, name, 1, dtype, device)
    if not t.is_contiguous() or (size is not None and t.numel() != size):
        raise ValueError(f"{name} must be contiguous with the required length")


def distinct_output(output, inputs):
    """Reject outputs sharing storage with any input, including disjoint views."""
    ptr = output.untyped_storage().data_ptr()
    if output.numel() and any(t is not None and t.numel() and t.untyped_storage().data_ptr() == ptr for t in inputs):
        raise ValueError("output must not share storage with an input")


@functools.lru_cache(maxsize=None)
def _arch(index: int) -> str:
    import torch

    return torch.cuda.get_device_properties(index).gcnArchName.split(":")[0]


def require_arch(device) -> None:
    """The kernels are built for gfx950 only (the reference pins gfx90a, ops/nf4.py:68-75)."""
    import torch

    if not torch.version.hip or _arch(device.index if device.index is not None else torch.cuda.current_device()) != ARCH:
        raise RuntimeError(f"loraforge_amd kernels require ROCm {ARCH}")
