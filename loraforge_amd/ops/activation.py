"""SwiGLU between an MLP's gate/up and down projections, on gfx950.

The reference applies ``bf16(bf16(silu(gate)) * up)`` to the LoRA-updated bf16
gate and up values (``benchmarks/qwen35_decode_silu.py:60-61``; the prefill
variant ``benchmarks/qwen35_prefill_fused.py:14-93``). Here the gate/up
projection is one fused NF4 + LoRA call with two slices writing
``gate_up = [gate | up]`` (``[T, 2N]``); this op reads that output and writes
the down projection's input ``[T, N]`` (``csrc/swiglu.hip``).
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from .. import _lib
from ..annotations import ExperimentalAPI
from ._checks import distinct_output, require_arch, tensor

if TYPE_CHECKING:
    from torch import Tensor


@ExperimentalAPI(reason="SwiGLU step of the c3 MLP chain; gfx950 HIP kernel.")
def silu_mul(gate_up: Tensor, *, out: Tensor | None = None) -> Tensor:
    """``out[t, c] = bf16(bf16(silu(gate_up[t, c])) * gate_up[t, N + c])`` for ``gate_up`` ``[T, 2N]``.

    silu is evaluated in fp32 as ``g / (1 + exp(-g))``. ``out`` (``[T, N]``,
    bf16, unit column stride) is allocated when omitted and must not share
    storage with ``gate_up``.
    """
    import torch

    tensor(gate_up, "gate_up", 2, torch.bfloat16)
    if gate_up.shape[1] % 2 or gate_up.shape[1] == 0 or gate_up.stride(1) != 1:
        raise ValueError("gate_up must be [tokens, 2 * n] with unit column stride")
    n = gate_up.shape[1] // 2
    if out is None:
        out = torch.empty(gate_up.shape[0], n, dtype=torch.bfloat16, device=gate_up.device)
    tensor(out, "out", 2, torch.bfloat16, gate_up.device)
    if out.shape != (gate_up.shape[0], n) or out.stride(1) != 1:
        raise ValueError("out must be [tokens, n] with unit column stride")
    distinct_output(out, (gate_up,))
    if gate_up.shape[0] == 0:
        return out
    require_arch(gate_up.device)
    lib = _lib.library()
    with torch.cuda.device(gate_up.device):
        _lib.check(
            lib.lf_swiglu(
                gate_up.data_ptr(),
                gate_up.shape[0],
                n,
                gate_up.stride(0),
                out.data_ptr(),
                out.stride(0),
                _lib.stream_of(gate_up.device),
            )
        )
    return out
