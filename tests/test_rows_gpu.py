"""Row shrink/expand on gfx950 against the oracle, following the reference's GPU
tests (``tests/test_row_operators_gpu.py``): mixed ranks 0..64 in a
capacity-128 pool, 1-3 slices, 128/256 threads, segmented routing, column
views, graph replay after metadata mutation, the rounding KATs, rejection
cases and empty batches. Gates: relative L2 < 0.005 on live values (the
reference's), max abs/rel 2e-2, exact equality where nothing may change.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from loraforge_amd.ops import row_expand, row_shrink
from oracle import nf4 as onf4, rows
from tests import _cases

pytestmark = pytest.mark.gpu
KAT = json.loads((Path(__file__).parent / "golden" / "kat_rows.json").read_text())


def t16(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits)).view(torch.bfloat16).to(device)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def close(actual_bits, expected_bits):
    a = onf4.bf16_to_f32(actual_bits).astype(np.float64)
    e = onf4.bf16_to_f32(expected_bits).astype(np.float64)
    rel = np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30)
    assert rel < 0.005, rel
    np.testing.assert_allclose(a, e, rtol=2e-2, atol=2e-2)


def gpu_case(c, device):
    meta = {k: torch.from_numpy(v).to(device) for k, v in c["meta"].items()}
    x = t16(c["x_full"], device)[:, : c["x"].shape[1]]
    storage = t16(c["storage"], device)
    lo, hi = c["out_cols"]
    return x, t16(c["a"], device), t16(c["z"], device), t16(c["b"], device), storage, storage[:, lo:hi], torch.from_numpy(c["routes"]).to(device), meta


@pytest.mark.parametrize("slices", [1, 2, 3])
@pytest.mark.parametrize("threads", [128, 256])
def test_mixed_ranks_slices_segments_and_base(slices, threads, device):
    c = _cases.row_case(slices)
    x, a, z, b, storage, output, routes, meta = gpu_case(c, device)
    before, all_before = output.clone(), storage.clone()
    expected_z = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"], num_slices=slices)
    row_shrink(x, a, z, routes, meta["ranks"], num_slices=slices)
    torch.cuda.synchronize()
    zb = bits(z)
    for row, slot in enumerate(c["routes"].tolist()):
        rank = int(c["meta"]["ranks"][slot]) if slot >= 0 else 0
        if rank:
            close(zb[row, : slices * rank], expected_z[row, : slices * rank])
        assert np.array_equal(zb[row, slices * rank :], expected_z[row, slices * rank :])
    expected = rows.row_expand(zb, c["b"], bits(before), **c["meta"])
    row_expand(z, b, output, **meta, threads=threads, blocks=1)
    torch.cuda.synchronize()
    close(bits(output), expected)
    delta = torch.zeros_like(output)
    row_expand(z, b, delta, **meta, threads=threads, blocks=2)
    torch.cuda.synchronize()
    close(bits(delta), rows.row_expand(zb, c["b"], np.zeros_like(bits(delta)), **c["meta"]))
    assert torch.equal(storage[:, :3], all_before[:, :3]) and torch.equal(storage[:, -3:], all_before[:, -3:])
    skipped = (routes == -1) | (routes == 8)
    assert torch.equal(output[skipped], before[skipped])


@pytest.mark.parametrize("width,columns", [(4096, 14336), (14336, 4096)])
def test_model_projection_sizes(width, columns, device):
    c = _cases.row_case(width=width, columns=columns)
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    expected_z = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"])
    row_shrink(x, a, z, routes, meta["ranks"])
    torch.cuda.synchronize()
    zb = bits(z)
    live = np.arange(128)[None, :] < np.where(c["routes"] >= 0, c["meta"]["ranks"][c["routes"]], 0)[:, None]
    close(zb[live], expected_z[live])
    expected = rows.row_expand(zb, c["b"], bits(output), **c["meta"])
    row_expand(z, b, output, **meta)
    torch.cuda.synchronize()
    close(bits(output), expected)


def test_graph_replay_changed_routes_ranks_offsets_and_weights(device):
    c = _cases.row_case(slices=3)
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    base = output.clone()

    def run():
        row_shrink(x, a, z, routes, meta["ranks"], num_slices=3)
        row_expand(z, b, output, **meta)

    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        run()
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        run()
    # Slot 2 reloaded with rank 7, pointing at slot 3's compact region.
    meta["ranks"][2] = 7
    meta["b_strides"][2] = 8
    meta["b_offsets"][2] = meta["b_offsets"][3]
    a[2].mul_(0.5)
    b.mul_(0.75)
    x.mul_(0.75)
    meta["scales"].mul_(0.5)
    meta["token_indices"].copy_(meta["token_indices"].flip(0))
    for seg, slot in enumerate(meta["segment_slots"].tolist()):
        start, end = meta["segment_indptr"][seg : seg + 2].tolist()
        routes[meta["token_indices"][start:end].long()] = slot
    meta["segment_count"].sub_(2)
    host_meta = {k: v.cpu().numpy() for k, v in meta.items()}
    for _ in range(3):
        output.copy_(base)
        z.fill_(3)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        expected_z = rows.row_shrink(bits(x), bits(a), bits(torch.full_like(z, 3)), routes.cpu().numpy(), host_meta["ranks"], num_slices=3)
        close(bits(output), rows.row_expand(expected_z, bits(b), bits(base), **host_meta))
    replay = output.clone()
    output.copy_(base)
    run()
    torch.cuda.synchronize()
    assert torch.equal(output, replay)


def test_scaled_delta_rounding_contract(device):
    k = KAT["scaled_delta_rounding"]

    def i(v, dtype=torch.int32):
        return torch.tensor(v, device=device, dtype=dtype)

    y = torch.tensor(k["y"], device=device, dtype=torch.bfloat16)
    row_expand(
        torch.tensor(k["z"], device=device, dtype=torch.bfloat16),
        torch.tensor(k["b"], device=device, dtype=torch.bfloat16),
        y,
        b_offsets=i(k["b_offsets"], torch.int64),
        b_strides=i(k["b_strides"]),
        ranks=i(k["ranks"]),
        scales=i(k["scales"], torch.float32),
        segment_indptr=i(k["segment_indptr"]),
        segment_slots=i(k["segment_slots"]),
        token_indices=i(k["token_indices"]),
        slice_offsets=i(k["slice_offsets"]),
        segment_count=i(k["segment_count"]),
    )
    assert y.item() == k["expected_y"][0][0]


def test_example_known_answer(device):
    k = KAT["example_row_operators"]

    def i(v, dtype=torch.int32):
        return torch.tensor(v, device=device, dtype=dtype)

    x = torch.tensor(k["x"], device=device, dtype=torch.bfloat16)
    a = torch.tensor(k["a"], device=device, dtype=torch.bfloat16)
    z = torch.tensor(k["z"], device=device, dtype=torch.bfloat16)
    y = torch.tensor(k["y"], device=device, dtype=torch.bfloat16)
    ranks = i(k["ranks"])
    row_shrink(x, a, z, i(k["slots"]), ranks, max_rank=k["max_rank"])
    row_expand(
        z,
        torch.tensor(k["b"], device=device, dtype=torch.bfloat16),
        y,
        b_offsets=i(k["b_offsets"], torch.int64),
        b_strides=i(k["b_strides"]),
        ranks=ranks,
        scales=i(k["scales"], torch.float32),
        segment_indptr=i(k["segment_indptr"]),
        segment_slots=i(k["segment_slots"]),
        token_indices=i(k["token_indices"]),
        slice_offsets=i(k["slice_offsets"]),
        segment_count=i(k["segment_count"]),
    )
    assert y.float().cpu().tolist() == k["expected_y"]


def test_reject_invalid_structures_and_aliases(device):
    c = _cases.row_case()
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    with pytest.raises(ValueError, match="same CUDA"):
        row_shrink(x, a.cpu(), z, routes, meta["ranks"])
    with pytest.raises(ValueError, match="aligned"):
        row_shrink(x[:, 1:513], a[:, :, :512].contiguous(), z, routes, meta["ranks"])
    with pytest.raises(ValueError, match="inference"):
        row_expand(z.requires_grad_(), b, output, **meta)
    z.requires_grad_(False)
    with pytest.raises(ValueError, match="length"):
        row_expand(z, b, output, **(meta | {"b_offsets": meta["b_offsets"][:2]}))
    with pytest.raises(ValueError, match="threads"):
        row_expand(z, b, output, **meta, threads=64)
    with pytest.raises(ValueError, match="share storage"):
        row_expand(z, b, z[:, : output.shape[1]], **meta)


def test_empty_batch_and_zero_active_segments(device):
    c = _cases.row_case()
    x, a, z, b, _, output, routes, meta = gpu_case(c, device)
    before = output.clone()
    meta["segment_count"].zero_()
    row_expand(z, b, output, **meta)
    torch.cuda.synchronize()
    assert torch.equal(output, before)
    row_shrink(x[:0], a, z[:0], routes[:0], meta["ranks"])
    row_expand(z[:0], b, output[:0], **meta)


def _shrink_case(tokens, seed, adapters=32, rank=16, k=4096):
    c = _cases.c2_case(seed=seed, tokens=tokens, k=k, n=64, adapters=adapters, rank=rank)
    c["z"] = np.full(c["z"].shape, _cases.bf16(3.0), np.uint16)
    return c


@pytest.mark.parametrize("tokens", [1, 17, 64, 200, 256, 257, 700])
def test_shrink_token_counts_across_the_k_split(tokens, device):
    """Up to 256 tokens split K over workgroups (tagged partials, elected sum); above, one pass."""
    c = _shrink_case(tokens, seed=900 + tokens)
    x, a, z = t16(c["x"], device), t16(c["a"], device), t16(c["z"], device)
    routes = torch.from_numpy(c["routes"]).to(device)
    ranks = torch.from_numpy(c["meta"]["ranks"]).to(device)
    for _ in range(2):  # the second call reuses the workspace with a new tag
        row_shrink(x, a, z, routes, ranks, max_rank=16)
        torch.cuda.synchronize()
        zb = bits(z)
        expected = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"])
        live = c["routes"] >= 0
        if live.any():
            close(zb[live], expected[live])
        assert np.array_equal(zb[~live], c["z"][~live])


def test_shrink_gives_up_on_withheld_partials_and_recomputes(device):
    """Host-forced give-up: chunks past the first never publish; the summing workgroup's bounded
    wait ends, it recomputes those chunks from x and A, flags the status word, and z is exact."""
    import ctypes

    from loraforge_amd import _lib

    c = _shrink_case(64, seed=933)
    x, a, z = t16(c["x"], device), t16(c["a"], device), t16(c["z"], device)
    routes = torch.from_numpy(c["routes"]).to(device)
    ranks = torch.from_numpy(c["meta"]["ranks"]).to(device)
    lib = _lib.library()
    need = lib.lf_row_shrink_workspace_size(64, 4096, 32, 1, 16)
    assert need > 0  # 64 tokens split K
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    expected = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"])
    live = c["routes"] >= 0

    def call(flags):
        _lib.check(
            lib.lf_row_shrink(
                x.data_ptr(), a.data_ptr(), z.data_ptr(), routes.data_ptr(), ranks.data_ptr(), 64, 4096, 4096, 32, 1, 16, 16,
                ws.data_ptr(), need, flags, _lib.stream_of(device),
            )
        )
        status = ctypes.c_int32(-1)
        _lib.check(lib.lf_nf4_lora_status(ws.data_ptr(), _lib.stream_of(device), ctypes.byref(status)))
        return status.value

    assert call(0) == 0
    close(bits(z)[live], expected[live])
    z.copy_(t16(c["z"], device))
    assert call(_lib.LF_TEST_WITHHOLD_PARTIALS) == 1
    zb = bits(z)
    close(zb[live], expected[live])
    assert np.array_equal(zb[~live], c["z"][~live])
    ws[8:12].zero_()  # clear the status word; a normal call afterwards is clean again
    z.copy_(t16(c["z"], device))
    assert call(0) == 0
    close(bits(z)[live], expected[live])


def test_shrink_shapes_alternate_on_one_workspace(device):
    """Calls of different shapes share the cached workspace: the election counters of one shape
    land where another shape kept partials, so they must be at a place of their own."""
    for tokens, rank, adapters in [(64, 16, 32), (40, 64, 8), (64, 16, 32), (9, 8, 100), (64, 16, 32)]:
        c = _shrink_case(tokens, seed=tokens * rank + adapters, adapters=adapters, rank=rank)
        x, a, z = t16(c["x"], device), t16(c["a"], device), t16(c["z"], device)
        routes = torch.from_numpy(c["routes"]).to(device)
        ranks = torch.from_numpy(c["meta"]["ranks"]).to(device)
        row_shrink(x, a, z, routes, ranks, max_rank=rank)
        torch.cuda.synchronize()
        live = c["routes"] >= 0
        expected = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"])
        close(bits(z)[live], expected[live])
