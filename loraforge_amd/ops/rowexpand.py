"""The Fleet row operators' API (mirror of ``loraforge.ops.rowexpand``).

Reference: ``src/loraforge/ops/rowexpand.py:34-92`` (``direct_shrink``,
``row_expand``) over ``ops/csrc/rowexpand.cu:87-127``. The arithmetic is the
retained-rank shrink/expand of ``lora_rows`` (same rounding chain), with the
Fleet argument order, up to four slices and the ``row_tile`` knob. The
reference splits a segment's B work into items of 2/4/8/16 token rows and
documents the outputs as bitwise-equal to the untiled kernel; here an item is
a segment times a run of output columns (the MFMA tile covers all 16 tokens of
a segment), and ``row_tile`` bounds that run: 16 lets the library choose it
from the work count, 8 caps it at 128 columns (256 threads), 4 and 2 at 64.
Outputs are bitwise identical for every value. ``direct_shrink`` goes to
``lf_row_shrink`` (as ``lora_rows.row_shrink`` does), ``row_expand`` to
``lf_row_expand_tiled``.
"""

from __future__ import annotations

from typing import TYPE_CHECKING

from .. import _lib
from .lora_rows import _shrink_workspace
from ._checks import distinct_output, require_arch, tensor, vector

if TYPE_CHECKING:
    from torch import Tensor

_AUTOGRAD = "RowExpand serving operators do not support autograd"


def _no_grad(*tensors) -> None:
    if any(t is not None and t.requires_grad for t in tensors):
        raise ValueError(_AUTOGRAD)


def direct_shrink(x: Tensor, weights: Tensor, output: Tensor, routes: Tensor, ranks: Tensor, slices: int, max_rank: int) -> Tensor:
    """Write live retained A rows ``output[t, s*r + k] = bf16(x[t] . weights[g, s*r + k])``.

    ``weights`` is ``[G, slices * R, K]``, ``output`` ``[T, slices * R]``;
    ``routes[t]`` (length >= T) is the token's slot, -1 for none. Inactive
    output columns are left as they are (the reference leaves them
    unspecified). ``slices`` 1..4, ``max_rank`` 1..64.
    """
    import torch

    _no_grad(x, weights, output)
    tensor(x, "x", 2, torch.bfloat16)
    tensor(weights, "weights", 3, torch.bfloat16, x.device)
    tensor(output, "output", 2, torch.bfloat16, x.device)
    if type(slices) is not int or not 1 <= slices <= 4:
        raise ValueError("slices must be in 1..4")
    if type(max_rank) is not int or not 1 <= max_rank <= 64:
        raise ValueError("max_rank must be in 1..64")
    if (
        weights.shape[1] % slices
        or weights.shape[1] // slices < max_rank
        or weights.shape[2] != x.shape[1]
        or output.shape != (x.shape[0], weights.shape[1])
    ):
        raise ValueError("weights/output shapes must agree with slices and rank capacity")
    if (
        x.shape[1] % 8
        or x.stride(1) != 1
        or x.stride(0) % 8
        or x.data_ptr() % 16
        or weights.data_ptr() % 16
        or not weights.is_contiguous()
        or not output.is_contiguous()
    ):
        raise ValueError("unaligned shrink operands")
    tensor(routes, "routes", 1, torch.int32, x.device)
    if not routes.is_contiguous() or routes.numel() < x.shape[0]:
        raise ValueError("routes must be contiguous with at least one entry per token")
    vector(ranks, "ranks", torch.int32, x.device, weights.shape[0])
    distinct_output(output, (x, weights, routes, ranks))
    if x.shape[0] == 0:
        return output
    require_arch(x.device)
    lib = _lib.library()
    with torch.cuda.device(x.device):
        _lib.check(
            lib.lf_row_shrink(
                x.data_ptr(),
                weights.data_ptr(),
                output.data_ptr(),
                routes.data_ptr(),
                ranks.data_ptr(),
                x.shape[0],
                x.shape[1],
                x.stride(0),
                weights.shape[0],
                slices,
                weights.shape[1] // slices,
                max_rank,
                *_shrink_workspace(x, weights.shape[0], slices, max_rank),
                0,
                _lib.stream_of(x.device),
            )
        )
    return output


def row_expand(
    z: Tensor,
    store: Tensor,
    offsets: Tensor,
    buckets: Tensor,
    output: Tensor,
    segments: Tensor,
    slots: Tensor,
    permutation: Tensor,
    ranks: Tensor,
    scales: Tensor,
    slice_offsets: Tensor,
    segment_count: Tensor,
    capacity: int,
    *,
    blocks: int = 880,
    threads: int = 256,
    row_tile: int = 16,
) -> Tensor:
    """Accumulate the bf16-rounded scaled delta into ``output`` on its current stream.

    ``z`` is ``[T, S * capacity]`` (effective-rank packed slices), ``store``
    the flat compact B regions (``offsets`` int64 elements, ``buckets`` int32
    row widths), ``segments`` the int32 segment pointers of ``slots``
    (int32 slot per segment, at most 16 tokens each), ``permutation`` the
    token of each segment row, ``slice_offsets`` S + 1 int32 bounds (S 1..4)
    and ``segment_count`` one int32 of active segments.
    ``y = bf16(bf16(y) + bf16(scale * z B_g^T))`` per token of an active
    segment; slot -1 and rank 0 leave rows unchanged.
    """
    import torch

    _no_grad(z, store, output, scales)
    if type(row_tile) is not int or row_tile not in (2, 4, 8, 16):
        raise ValueError("row_tile must be 2, 4, 8, or 16")
    if type(threads) is not int or threads not in (128, 256):
        raise ValueError("threads must be 128 or 256")
    if type(blocks) is not int or not 1 <= blocks <= 65535:
        raise ValueError("blocks must be in 1..65535")
    tensor(z, "z", 2, torch.bfloat16)
    tensor(store, "store", 1, torch.bfloat16, z.device)
    tensor(output, "output", 2, torch.bfloat16, z.device)
    vector(ranks, "ranks", torch.int32, z.device)
    for t, name, dtype in ((offsets, "offsets", torch.int64), (buckets, "buckets", torch.int32), (scales, "scales", torch.float32)):
        vector(t, name, dtype, z.device, ranks.numel())
    vector(slots, "slots", torch.int32, z.device)
    vector(segments, "segments", torch.int32, z.device)
    if segments.numel() < slots.numel() + 1:
        raise ValueError("segments must hold one pointer more than slots")
    vector(permutation, "permutation", torch.int32, z.device)
    if permutation.numel() < z.shape[0]:
        raise ValueError("permutation must cover every token")
    vector(slice_offsets, "slice_offsets", torch.int32, z.device)
    vector(segment_count, "segment_count", torch.int32, z.device, 1)
    nslices = slice_offsets.numel() - 1
    if type(capacity) is not int or capacity < 1:
        raise ValueError("capacity must be a positive int")
    if not 1 <= nslices <= 4 or z.shape[1] != capacity * nslices or output.shape[0] != z.shape[0] or output.shape[1] < 1:
        raise ValueError("z/output shapes must agree with the slices and capacity")
    if not z.is_contiguous() or not store.is_contiguous() or store.data_ptr() % 16 or output.stride(1) != 1 or output.stride(0) < output.shape[1]:
        raise ValueError("expected contiguous z/aligned B and nonoverlapping output rows")
    distinct_output(output, (z, store, offsets, buckets, ranks, scales, segments, slots, permutation, slice_offsets, segment_count))
    if z.shape[0] == 0:
        return output
    require_arch(z.device)
    lib = _lib.library()
    with torch.cuda.device(z.device):
        _lib.check(
            lib.lf_row_expand_tiled(
                z.data_ptr(),
                store.data_ptr(),
                offsets.data_ptr(),
                buckets.data_ptr(),
                output.data_ptr(),
                segments.data_ptr(),
                slots.data_ptr(),
                permutation.data_ptr(),
                ranks.data_ptr(),
                scales.data_ptr(),
                slice_offsets.data_ptr(),
                segment_count.data_ptr(),
                slots.numel(),
                z.shape[0],
                output.shape[1],
                output.stride(0),
                nslices,
                capacity,
                blocks,
                threads,
                row_tile,
                _lib.stream_of(z.device),
            )
        )
    return output
