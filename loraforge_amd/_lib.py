"""ctypes binding of ``libloraforge_amd.so`` (the C ABI in ``include/loraforge_amd.h``).

The library is loaded after ``torch`` so that it binds to the HIP runtime
PyTorch already loaded (both carry the soname ``libamdhip64.so.7``); pointers
and streams handed over here are therefore valid in both. There is no CPU or
PyTorch fallback: a missing library raises ``RuntimeError`` naming the build
step.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "_lib" / "libloraforge_amd.so"

LF_OK = 0
LF_EINVAL = 1
LF_EHIP = 2
LF_EXACT_WEIGHTS = 1
LF_SWIGLU_OUTPUT = 2
LF_PLAN_DECODE_CHUNKS = 4
LF_PLAN_PREFILL = 8
LF_TEST_WITHHOLD_PARTIALS = 0x100
NOALLOC_SCRATCH_BYTES = 8 * 1024 * 1024
ABI_VERSION = 4

_lock = threading.Lock()
_handle: ctypes.CDLL | None = None

c_void_p = ctypes.c_void_p
c_int64 = ctypes.c_int64
c_int32 = ctypes.c_int32
c_float_p = ctypes.c_void_p


class NF4Weight(ctypes.Structure):
    _fields_ = [
        ("qweight", c_void_p),
        ("scales", c_void_p),
        ("absmax_q", c_void_p),
        ("absmax2", c_void_p),
        ("code2", c_void_p),
        ("offset", c_void_p),
        ("dq_block", c_int64),
        ("code", c_void_p),
        ("n", c_int64),
        ("k", c_int64),
    ]


class Lora(ctypes.Structure):
    _fields_ = [
        ("a_store", c_void_p),
        ("a_offsets", c_void_p),
        ("b_store", c_void_p),
        ("b_offsets", c_void_p),
        ("b_strides", c_void_p),
        ("ranks", c_void_p),
        ("scales", c_void_p),
        ("token_slots", c_void_p),
        ("slice_offsets", c_void_p),
        ("num_slices", c_int32),
        ("max_rank", c_int32),
        ("num_slots", c_int32),
    ]


_PROTOTYPES = {
    "lf_last_error": (ctypes.c_char_p, []),
    "lf_abi_version": (ctypes.c_int, []),
    "lf_device_arch": (ctypes.c_int, [ctypes.c_int, ctypes.c_char_p, ctypes.c_int]),
    "lf_nf4_dequant": (ctypes.c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "lf_nf4_dequant_dq": (
        ctypes.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p],
    ),
    "lf_nf4_prepare_scales_dq": (
        ctypes.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p],
    ),
    "lf_row_shrink": (
        ctypes.c_int,
        [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int32, c_int64, c_int32]
        + [c_void_p, c_int64, c_int32, c_void_p],
    ),
    "lf_row_shrink_workspace_size": (
        c_int64,
        [c_int64, c_int64, c_int64, c_int32, c_int32],
    ),
    "lf_row_expand": (
        ctypes.c_int,
        [c_void_p] * 12 + [c_int64, c_int64, c_int64, c_int64, c_int32, c_int64, c_int32, c_int32, c_void_p],
    ),
    "lf_row_expand_tiled": (
        ctypes.c_int,
        [c_void_p] * 12 + [c_int64, c_int64, c_int64, c_int64, c_int32, c_int64, c_int32, c_int32, c_int32, c_void_p],
    ),
    "lf_nf4_lora_workspace_size": (c_int64, [c_int64, c_int64, c_int64, c_int32, c_int32]),
    "lf_nf4_lora_linear": (
        ctypes.c_int,
        [
            c_void_p,
            c_int64,
            c_int64,
            ctypes.POINTER(NF4Weight),
            c_void_p,
            ctypes.POINTER(Lora),
            c_void_p,
            c_int64,
            c_void_p,
            c_int64,
            c_int32,
            c_void_p,
        ],
    ),
    "lf_nf4_lora_linear_noalloc": (
        ctypes.c_int,
        [
            c_void_p,
            c_int64,
            c_int64,
            ctypes.POINTER(NF4Weight),
            c_void_p,
            ctypes.POINTER(Lora),
            c_void_p,
            c_int64,
            c_int32,
            c_void_p,
        ],
    ),
    "lf_lora_apply": (
        ctypes.c_int,
        [c_void_p, c_int64, c_int64, c_int64, c_int64, ctypes.POINTER(Lora), c_void_p, c_int64, c_void_p, c_int64,
         c_int32, c_void_p],
    ),
    "lf_nf4_lora_status": (ctypes.c_int, [c_void_p, c_void_p, ctypes.POINTER(c_int32)]),
    "lf_swiglu": (ctypes.c_int, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
}

EXPORTS = tuple(_PROTOTYPES)


def library() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if it was not built."""
    global _handle
    if _handle is not None:
        return _handle
    with _lock:
        if _handle is None:
            import torch  # noqa: F401  (binds the HIP runtime torch ships)

            if not LIBRARY.exists():
                raise RuntimeError(
                    f"loraforge_amd native library missing at {LIBRARY}; "
                    "build it with `python -c 'import __graft_entry__ as g; g.build()'` "
                    "or `python -m loraforge_amd._build`"
                )
            lib = ctypes.CDLL(str(LIBRARY))
            for name, (restype, argtypes) in _PROTOTYPES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if lib.lf_abi_version() != ABI_VERSION:
                raise RuntimeError("loraforge_amd native library ABI mismatch; rebuild it")
            _handle = lib
    return _handle


def check(status: int) -> None:
    """Map a C status to the reference's exception types."""
    if status == LF_OK:
        return
    message = (library().lf_last_error() or b"").decode(errors="replace")
    if status == LF_EINVAL:
        raise ValueError(message)
    raise RuntimeError(message)


def ptr(tensor) -> int | None:
    """Device address of a tensor's first element (None for None)."""
    return None if tensor is None else tensor.data_ptr()


def stream_of(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream
