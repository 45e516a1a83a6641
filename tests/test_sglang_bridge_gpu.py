"""The SGLang bridge on gfx950: batch_info -> one nf4_lora_linear launch per projection.

Routes come from an independent per-segment expansion (tests/test_sglang_bridge.py);
the expected output is the oracle chain over the same adapter layout. A HIP graph
captured once follows new metadata written into the same batch_info buffers.
Gate: max abs/rel 2e-2 and relative L2 < 0.005 on bf16 outputs.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.integrations import apply_lora, apply_nf4_lora, lora_batch_from_batch_info
from loraforge_amd.runtime import AdapterTable, RetainedLayout
from oracle import linear
from oracle import nf4 as onf4
from tests import _cases
from tests.test_fused_gpu import bits, close, t16, to_device
from tests.test_sglang_bridge import random_info

pytestmark = pytest.mark.gpu


def expected(x_bits, w_bits, batch, routes, n):
    y = linear.nf4_linear(x_bits, w_bits)
    as_np = lambda t: t.cpu().numpy()  # noqa: E731
    return linear.lora_apply(
        x_bits, y, a_store=bits(batch.a_store), a_offsets=as_np(batch.a_offsets), b_store=bits(batch.b_store),
        b_offsets=as_np(batch.b_offsets), b_strides=as_np(batch.b_strides), ranks=as_np(batch.ranks),
        scales=as_np(batch.scales), token_slots=routes, slice_offsets=as_np(batch.slice_offsets), n_total=n,
    )


@pytest.fixture(scope="module")
def weight(device):
    case = _cases.fused_case(1, 1024, 512, ranks=(1,), seed=61)
    _, q, state, _, _ = to_device(case, device)
    st = case["state"]
    return onf4.dequantize(st["qweight"], st["scales"], st["shape"]), q, state


def retained_pool(rng, device, slots=6, cap=32, k=512, n=1024):
    ranks = [8, 0, 32, 16, 4, 32][:slots]
    a = torch.zeros(slots, cap, k, dtype=torch.bfloat16, device=device)
    b = torch.zeros(slots, n, cap, dtype=torch.bfloat16, device=device)
    catalog = {}
    for s, r in enumerate(ranks):
        if r:
            a[s, :r] = torch.from_numpy(rng.standard_normal((r, k)).astype(np.float32) * 0.05).bfloat16().to(device)
            b[s, :, :r] = torch.from_numpy(rng.standard_normal((n, r)).astype(np.float32) * 0.05).bfloat16().to(device)
        catalog[f"c{s}"] = {"base_model.model.model.layers.0.self_attn.o_proj.lora_A.weight": r}
    layout = RetainedLayout(a, b, "o_proj", 0, catalog)
    for s in range(slots):
        layout.load(f"c{s}", s, cap)
    return layout


@pytest.mark.parametrize("tokens", [7, 64, 300])
def test_bridge_over_retained_layout(weight, tokens, device):
    w_bits, q, state = weight
    rng = np.random.default_rng(tokens)
    layout = retained_pool(rng, device)
    info, routes = random_info(rng, tokens, 6, padded=2, device=device)
    info.scalings = torch.tensor([2.0, 1.0, 0.5, 1.5, 0.25, 1.0], device=device)
    x_bits = _cases.bf16(rng.standard_normal((tokens, 512)))
    y = apply_nf4_lora(t16(x_bits, device), q, state, info, layout)
    torch.cuda.synchronize()
    batch = lora_batch_from_batch_info(info, layout, tokens=tokens)
    np.testing.assert_array_equal(batch.token_slots.cpu().numpy(), routes)
    close(bits(y), expected(x_bits, w_bits, batch, routes, 1024))


def test_bridge_graph_replay_follows_new_metadata(weight, device):
    w_bits, q, state = weight
    tokens = 24
    rng = np.random.default_rng(5)
    table = AdapterTable(6, in_features=512, out_features=1024, max_rank=32, device=device)
    from loraforge_amd.adapters import AdapterModule

    for s, r in enumerate([8, 16, 4, 32, 8, 16]):
        a = torch.from_numpy(rng.standard_normal((r, 512)).astype(np.float32) * 0.05).bfloat16().to(device)
        b = torch.from_numpy(rng.standard_normal((1024, r)).astype(np.float32) * 0.05).bfloat16().to(device)
        table.publish(s, [AdapterModule("proj", a, b, 2.0 * r)])
    info, routes = random_info(rng, tokens, 6, padded=3, device=device)
    info.scalings = table.scales.clone()
    x_bits = _cases.bf16(rng.standard_normal((tokens, 512)))
    x = t16(x_bits, device)
    slots_buf = torch.empty(tokens, dtype=torch.int32, device=device)
    out = torch.empty(tokens, 1024, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        apply_nf4_lora(x, q, state, info, table, out=out, token_slots=slots_buf)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            apply_nf4_lora(x, q, state, info, table, out=out, token_slots=slots_buf)
    torch.cuda.synchronize()
    batch = table.batch(slots_buf)
    batch.scales = info.scalings
    for rep in range(3):
        # New routing written into the same metadata buffers (same segment count).
        fresh, routes = random_info(np.random.default_rng(100 + rep), tokens, 6, padded=3,
                                    segments=info.num_segments, device=device)
        assert fresh.num_segments == info.num_segments
        info.seg_indptr.copy_(fresh.seg_indptr)
        info.weight_indices.copy_(fresh.weight_indices)
        info.permutation.copy_(fresh.permutation)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(slots_buf.cpu().numpy(), routes)
        close(bits(out), expected(x_bits, w_bits, batch, routes, 1024))


def test_bridge_graph_replay_over_retained_layout(weight, device):
    """A graph captured over a RetainedLayout (after one eager call built its slice bounds)
    replays new routing written into the same batch_info buffers."""
    w_bits, q, state = weight
    tokens = 24
    rng = np.random.default_rng(7)
    layout = retained_pool(rng, device)
    info, routes = random_info(rng, tokens, 6, padded=3, device=device)
    info.scalings = torch.tensor([2.0, 1.0, 0.5, 1.5, 0.25, 1.0], device=device)
    x_bits = _cases.bf16(rng.standard_normal((tokens, 512)))
    x = t16(x_bits, device)
    slots_buf = torch.empty(tokens, dtype=torch.int32, device=device)
    out = torch.empty(tokens, 1024, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        apply_nf4_lora(x, q, state, info, layout, out=out, token_slots=slots_buf)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            apply_nf4_lora(x, q, state, info, layout, out=out, token_slots=slots_buf)
    torch.cuda.synchronize()
    batch = lora_batch_from_batch_info(info, layout, tokens=tokens)
    for rep in range(3):
        fresh, routes = random_info(np.random.default_rng(300 + rep), tokens, 6, padded=3,
                                    segments=info.num_segments, device=device)
        info.seg_indptr.copy_(fresh.seg_indptr)
        info.weight_indices.copy_(fresh.weight_indices)
        info.permutation.copy_(fresh.permutation)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(slots_buf.cpu().numpy(), routes)
        close(bits(out), expected(x_bits, w_bits, batch, routes, 1024))


@pytest.mark.parametrize("tokens", [5, 64, 150])
def test_bridge_lora_only_update(tokens, device):
    """apply_lora: SGLang's batch over a retained layout, y (the caller's base output) updated in place."""
    rng = np.random.default_rng(200 + tokens)
    layout = retained_pool(rng, device)
    info, routes = random_info(rng, tokens, 6, padded=2, device=device)
    info.scalings = torch.tensor([2.0, 1.0, 0.5, 1.5, 0.25, 1.0], device=device)
    x_bits = _cases.bf16(rng.standard_normal((tokens, 512)))
    y_bits = _cases.bf16(rng.standard_normal((tokens, 1024)))
    y = t16(y_bits, device)
    apply_lora(t16(x_bits, device), y, info, layout)
    torch.cuda.synchronize()
    batch = lora_batch_from_batch_info(info, layout, tokens=tokens)
    as_np = lambda t: t.cpu().numpy()  # noqa: E731
    want = linear.lora_apply(
        x_bits, y_bits, a_store=bits(batch.a_store), a_offsets=as_np(batch.a_offsets), b_store=bits(batch.b_store),
        b_offsets=as_np(batch.b_offsets), b_strides=as_np(batch.b_strides), ranks=as_np(batch.ranks),
        scales=as_np(batch.scales), token_slots=routes, slice_offsets=as_np(batch.slice_offsets), n_total=1024,
    )
    close(bits(y), want)
    idle = routes < 0
    assert np.array_equal(bits(y)[idle], y_bits[idle])
