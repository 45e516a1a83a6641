"""The standalone LoRA row operators (shrink to z, expand onto y) on gfx950.

Drop-in for ``loraforge.ops.row_shrink`` / ``row_expand``
(``src/loraforge/ops/lora_rows.py:51-239``): the signatures, tensor layouts,
structural checks and the exception types and message fragments that
callers match on are the contract kept here. The work runs in the MFMA
kernels of ``csrc/row_ops.hip`` through the C ABI. Metadata on the device is
used as given: the checks below look at shapes, strides, dtypes, devices
and alignment only, so a call never reads device memory back or waits for
the stream.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from .. import _lib
from ..annotations import ExperimentalAPI
from ._checks import distinct_output, require_arch, tensor, vector

if TYPE_CHECKING:
    from torch import Tensor


def _shrink_workspace(x, adapters: int, slices: int, max_rank: int) -> tuple:
    """(pointer, bytes) of the cached workspace a shrink of ``x`` needs (none: (None, 0))."""
    from .fused import _workspace

    need = _lib.library().lf_row_shrink_workspace_size(x.shape[0], x.shape[1], adapters, slices, max_rank)
    if need < 0:
        raise ValueError("invalid shrink problem size")
    if need == 0:
        return None, 0
    ws = _workspace(x.device, _lib.stream_of(x.device), int(need), kind="rows")
    return ws.data_ptr(), ws.numel()


@ExperimentalAPI(reason="BF16 retained-rank inference operator; gfx950 HIP kernel, caller-owned device metadata.")
def row_shrink(
    x: Tensor,
    a: Tensor,
    output: Tensor,
    slots: Tensor,
    ranks: Tensor,
    *,
    num_slices: int = 1,
    max_rank: int = 64,
) -> None:
    """z rows of the routed tokens: ``output[t, s*r + k] = bf16(x[t] . a[g, s*r + k])``.

    ``g = slots[t]`` and ``r = ranks[g]``; tokens routed to -1 or to a rank-0
    slot, and every column at or past ``num_slices * r``, keep their values.
    Shapes: x [tokens, width] (width and row stride multiples of 8, 16-byte
    aligned), a [slots, num_slices * capacity, width] contiguous, output
    [tokens, num_slices * capacity] contiguous; every live rank is at most
    ``max_rank``. Runs on the caller's current stream; no host sync.
    """
    import torch

    tensor(x, "x", 2, torch.bfloat16)
    tensor(a, "a", 3, torch.bfloat16, x.device)
    tensor(output, "output", 2, torch.bfloat16, x.device)
    if type(num_slices) is not int or not 1 <= num_slices <= 3:
        raise ValueError("num_slices must be in 1..3")
    if type(max_rank) is not int or not 1 <= max_rank <= 64:
        raise ValueError("max_rank must be in 1..64")
    if (
        a.shape[0] < 1
        or a.shape[1] % num_slices
        or a.shape[1] // num_slices < max_rank
        or a.shape[2] != x.shape[1]
        or output.shape != (x.shape[0], a.shape[1])
    ):
        raise ValueError("A/output shapes must agree with slices and rank capacity")
    if (
        x.shape[1] < 1
        or x.shape[1] % 8
        or x.stride(1) != 1
        or x.stride(0) < x.shape[1]
        or x.stride(0) % 8
        or x.data_ptr() % 16
        or a.data_ptr() % 16
        or not a.is_contiguous()
        or not output.is_contiguous()
    ):
        raise ValueError("expected aligned A/x and contiguous A/output")
    vector(slots, "slots", torch.int32, x.device, x.shape[0])
    vector(ranks, "ranks", torch.int32, x.device, a.shape[0])
    distinct_output(output, (x, a, slots, ranks))
    if x.shape[0] == 0:
        return
    require_arch(x.device)
    lib = _lib.library()
    with torch.cuda.device(x.device):
        _lib.check(
            lib.lf_row_shrink(
                x.data_ptr(),
                a.data_ptr(),
                output.data_ptr(),
                slots.data_ptr(),
                ranks.data_ptr(),
                x.shape[0],
                x.shape[1],
                x.stride(0),
                a.shape[0],
                num_slices,
                a.shape[1] // num_slices,
                max_rank,
                *_shrink_workspace(x, a.shape[0], num_slices, max_rank),
                0,
                _lib.stream_of(x.device),
            )
        )


@ExperimentalAPI(reason="Compact-B RowExpand; gfx950 HIP kernel, fixed-address metadata/lifetime contract.")
def row_expand(
    z: Tensor,
    b: Tensor,
    output: Tensor,
    *,
    b_offsets: Tensor,
    b_strides: Tensor,
    ranks: Tensor,
    scales: Tensor,
    segment_indptr: Tensor,
    segment_slots: Tensor,
    token_indices: Tensor,
    slice_offsets: Tensor,
    segment_count: Tensor,
    blocks: int | None = None,
    threads: int = 256,
) -> None:
    """Adds each segment's LoRA expansion to its tokens' rows of ``output``, in place.

    A segment is at most 16 distinct tokens routed to one slot g (rank r,
    scale ``scales[g]``); for a column n of slice s it adds
    ``bf16(scales[g] * sum_{k<r} z[t, s*r + k] * B_g[n, k])`` to the bf16
    value and rounds again. ``B_g`` is ``[out, b_strides[g]]`` at element
    ``b_offsets[g]`` of the flat store ``b`` (strides are powers of two in
    1..64, zero padded past r); ``slice_offsets`` partitions the output
    columns and ``segment_count`` (one int32 on the device) says how many
    segments are live, so nothing is read back to the host. Slot -1 and
    rank-0 segments change nothing; a token may sit in one live segment only.
    ``blocks`` / ``threads`` size the persistent grid.
    """
    import torch

    tensor(z, "z", 2, torch.bfloat16)
    tensor(b, "b", 1, torch.bfloat16, z.device)
    tensor(output, "output", 2, torch.bfloat16, z.device)
    vector(ranks, "ranks", torch.int32, z.device)
    nslots = ranks.numel()
    for t, name, dtype in (
        (b_offsets, "b_offsets", torch.int64),
        (b_strides, "b_strides", torch.int32),
        (scales, "scales", torch.float32),
    ):
        vector(t, name, dtype, z.device, nslots)
    vector(segment_slots, "segment_slots", torch.int32, z.device)
    vector(segment_indptr, "segment_indptr", torch.int32, z.device, segment_slots.numel() + 1)
    vector(token_indices, "token_indices", torch.int32, z.device)
    vector(slice_offsets, "slice_offsets", torch.int32, z.device)
    vector(segment_count, "segment_count", torch.int32, z.device, 1)
    slices = slice_offsets.numel() - 1
    if (
        nslots < 1
        or not 1 <= slices <= 3
        or z.shape[1] < slices
        or z.shape[1] % slices
        or output.shape[0] != z.shape[0]
        or output.shape[1] < 1
    ):
        raise ValueError("invalid slots, slice count or activation/output shape")
    if (
        not z.is_contiguous()
        or not b.is_contiguous()
        or b.data_ptr() % 16
        or output.stride(1) != 1
        or output.stride(0) < output.shape[1]
    ):
        raise ValueError("expected contiguous z/aligned B and nonoverlapping output rows")
    if blocks is not None and (type(blocks) is not int or not 1 <= blocks <= 65535):
        raise ValueError("blocks must be in 1..65535")
    if type(threads) is not int or threads not in (128, 256):
        raise ValueError("threads must be 128 or 256")
    column_blocks = (output.shape[1] + threads - 1) // threads
    if segment_slots.numel() * column_blocks >= 2**31:
        raise ValueError("segment work count must fit signed int32 indexing")
    distinct_output(
        output,
        (z, b, b_offsets, b_strides, ranks, scales, segment_indptr, segment_slots, token_indices, slice_offsets, segment_count),
    )
    if z.shape[0] == 0:
        return
    require_arch(z.device)
    lib = _lib.library()
    with torch.cuda.device(z.device):
        if blocks is None:
            blocks = 2 * torch.cuda.get_device_properties(z.device).multi_processor_count
        _lib.check(
            lib.lf_row_expand(
                z.data_ptr(),
                b.data_ptr(),
                b_offsets.data_ptr(),
                b_strides.data_ptr(),
                output.data_ptr(),
                segment_indptr.data_ptr(),
                segment_slots.data_ptr(),
                token_indices.data_ptr(),
                ranks.data_ptr(),
                scales.data_ptr(),
                slice_offsets.data_ptr(),
                segment_count.data_ptr(),
                segment_slots.numel(),
                z.shape[0],
                output.shape[1],
                output.stride(0),
                slices,
                z.shape[1] // slices,
                blocks,
                threads,
                _lib.stream_of(z.device),
            )
        )
