"""The Fleet row operators (``direct_shrink`` / ``row_expand`` with ``row_tile``)
against the oracle: the reference's ``ops/rowexpand.py:34-92`` API with up to
four slices (``rowexpand.cu:87-108``). The reference documents tiled expand
outputs as bitwise-equal to the untiled kernel; every ``row_tile`` here must
give the same bits, and the values must meet the row-operator gates.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import rowexpand
from loraforge_amd.ops import row_expand as lora_row_expand
from oracle import rows
from tests import _cases
from tests.test_rows_gpu import bits, close, gpu_case

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("slices", [1, 3, 4])
def test_fleet_shrink_and_tiled_expand(slices, device):
    c = _cases.row_case(slices, columns=37 if slices == 4 else None, seed=274)
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    before = output.clone()
    max_rank = 64
    rowexpand.direct_shrink(x, a, z, routes, meta["ranks"], slices, max_rank)
    torch.cuda.synchronize()
    expected_z = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"], num_slices=slices)
    zb = bits(z)
    for row, slot in enumerate(c["routes"].tolist()):
        rank = int(c["meta"]["ranks"][slot]) if slot >= 0 else 0
        if rank:
            close(zb[row, : slices * rank], expected_z[row, : slices * rank])
    capacity = z.shape[1] // slices
    args = (meta["b_offsets"], meta["b_strides"])
    outs = []
    for tile in (2, 4, 8, 16):
        out = before.clone()
        rowexpand.row_expand(
            z, b, *args, out, meta["segment_indptr"], meta["segment_slots"], meta["token_indices"], meta["ranks"],
            meta["scales"], meta["slice_offsets"], meta["segment_count"], capacity, row_tile=tile,
        )
        outs.append(out)
    torch.cuda.synchronize()
    for out in outs[1:]:
        assert torch.equal(out, outs[0])
    close(bits(outs[0]), rows.row_expand(zb, c["b"], bits(before), **c["meta"]))
    if slices <= 3:
        ref = before.clone()
        lora_row_expand(z, b, ref, **meta)
        torch.cuda.synchronize()
        assert torch.equal(ref, outs[0])


@pytest.mark.parametrize("threads", [128, 256])
def test_fleet_item_widths_give_identical_bits(threads, device):
    """5700 output columns over 12 segments: row_tile 16 runs the widest items
    (64 columns per wave), 8 at most 32 and 4 / 2 at most 16; every variant must
    give the bits of ``lora_rows.row_expand`` and meet the oracle."""
    slices = 3
    c = _cases.row_case(slices, columns=1900, seed=275)
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    before = output.clone()
    rowexpand.direct_shrink(x, a, z, routes, meta["ranks"], slices, 64)
    torch.cuda.synchronize()
    zb = bits(z)
    outs = []
    for tile in (16, 8, 4, 2):
        out = before.clone()
        rowexpand.row_expand(
            z, b, meta["b_offsets"], meta["b_strides"], out, meta["segment_indptr"], meta["segment_slots"],
            meta["token_indices"], meta["ranks"], meta["scales"], meta["slice_offsets"], meta["segment_count"],
            z.shape[1] // slices, row_tile=tile, threads=threads,
        )
        outs.append(out)
    ref = before.clone()
    lora_row_expand(z, b, ref, **meta, threads=threads)
    torch.cuda.synchronize()
    for out in outs:
        assert torch.equal(out, ref)
    close(bits(ref), rows.row_expand(zb, c["b"], bits(before), **c["meta"]))


def test_fleet_contract_errors(device):
    c = _cases.row_case(1, seed=15)
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    with pytest.raises(ValueError, match="row_tile"):
        rowexpand.row_expand(
            z, b, meta["b_offsets"], meta["b_strides"], output, meta["segment_indptr"], meta["segment_slots"],
            meta["token_indices"], meta["ranks"], meta["scales"], meta["slice_offsets"], meta["segment_count"],
            z.shape[1], row_tile=3,
        )
    with pytest.raises(ValueError, match="slices"):
        rowexpand.direct_shrink(x, a, z, routes, meta["ranks"], 5, 64)
    with pytest.raises(ValueError, match="autograd"):
        rowexpand.direct_shrink(x.float().requires_grad_(), a, z, routes, meta["ranks"], 1, 64)
