"""GPU runtime path: PEFT files -> GPUAdapterSlots -> AdapterTable -> fused linear.

Checks that the fixed-address table holds exactly the borrowed factors (A
packed per slice, B zero padded to the rank bucket), that ``nf4_lora_linear``
on the table matches the oracle chain, and that a HIP graph captured once
sees an adapter republished into the same slot (addresses never move). Also
the c4 configuration: retained-rank adapters of ranks {4, 8, 16, 32, 64}
routed with Zipf(1.1) over 128 slots, through both the decode (<= 64 tokens)
and prefill kernels.
"""

import json

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from loraforge_amd.ops import nf4_lora_linear
from loraforge_amd.runtime import AdapterTable, GPUAdapterSlots
from oracle import linear
from oracle import nf4 as onf4
from tests import _cases
from tests.test_fused_gpu import bits, close, t16, to_device, workspace_clean

pytestmark = pytest.mark.gpu


def write_adapter(root, name, rank, k, n, seed, alpha):
    rng = np.random.default_rng(seed)
    d = root / name
    d.mkdir()
    (d / "adapter_config.json").write_text(
        json.dumps({"peft_type": "LORA", "r": rank, "lora_alpha": alpha, "target_modules": ["proj"], "bias": "none"})
    )
    a = torch.from_numpy(rng.standard_normal((rank, k)).astype(np.float32) * 0.05).bfloat16()
    b = torch.from_numpy(rng.standard_normal((n, rank)).astype(np.float32) * 0.05).bfloat16()
    save_file({"base_model.model.proj.lora_A.weight": a, "base_model.model.proj.lora_B.weight": b}, str(d / "adapter_model.safetensors"))
    return d, a, b


def weight(n, k, seed, device):
    case = _cases.fused_case(1, n, k, ranks=(1,), seed=seed)
    _, q, state, _, _ = to_device(case, device)
    return case["state"], q, state


def expected_from_table(x_bits, st, table, token_slots):
    w = onf4.dequantize(st["qweight"], st["scales"], st["shape"])
    y = linear.nf4_linear(x_bits, w)
    return linear.lora_apply(
        x_bits,
        y,
        a_store=bits(table.a_store),
        a_offsets=table.a_offsets.cpu().numpy(),
        b_store=bits(table.b_store),
        b_offsets=table.b_offsets.cpu().numpy(),
        b_strides=table.b_strides.cpu().numpy(),
        ranks=table.ranks.cpu().numpy(),
        scales=table.scales.cpu().numpy(),
        token_slots=np.asarray(token_slots, np.int32),
        slice_offsets=table.slice_offsets.cpu().numpy(),
        n_total=table.out_features,
    )


def test_slots_table_and_graph_replay(tmp_path, device):
    k, n, m = 512, 256, 12
    specs = [("r8", 8, 16.0), ("r16", 16, 8.0), ("r4", 4, 4.0), ("r12", 12, 24.0)]
    adapters = {name: write_adapter(tmp_path, name, r, k, n, i, alpha) for i, (name, r, alpha) in enumerate(specs)}
    pool = GPUAdapterSlots(4, device=str(device))
    handles = {name: pool.load(adapters[name][0], i) for i, (name, _, _) in enumerate(specs)}
    table = AdapterTable(3, in_features=k, out_features=n, max_rank=16, device=device)
    addresses = [t.data_ptr() for t in (table.a_store, table.b_store, table.ranks, table.b_strides, table.scales)]
    for slot, name in enumerate(["r8", "r16", "r4"]):
        table.publish_from(pool, handles[name], slot, ["proj"])
    torch.cuda.synchronize()

    # Table content: A rows of the slot, B zero padded to bucket(rank), metadata.
    for slot, (name, rank, alpha) in enumerate(specs[:3]):
        _, a, b = adapters[name]
        a_rows = table.a_store[slot * table.a_rows * k : slot * table.a_rows * k + rank * k].view(rank, k).cpu()
        torch.testing.assert_close(a_rows, a)
        bucket = int(table.b_strides[slot])
        assert bucket == _cases.bucket_of(rank)
        b_view = table.b_store[slot * n * table.b_width : slot * n * table.b_width + n * bucket].view(n, bucket).cpu()
        torch.testing.assert_close(b_view[:, :rank], b)
        assert not b_view[:, rank:].any()
        assert int(table.ranks[slot]) == rank and float(table.scales[slot]) == pytest.approx(alpha / rank)

    st, q, state = weight(n, k, 5, device)
    rng = np.random.default_rng(9)
    x_bits = _cases.bf16(rng.standard_normal((m, k)))
    x = t16(x_bits, device)
    routes = np.array([0, 1, 2, -1, 2, 1, 0, 0, -1, 1, 2, 0], np.int32)
    slots = torch.from_numpy(routes).to(device)
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    nf4_lora_linear(x, q, state, lora=table.batch(slots), out=out)
    torch.cuda.synchronize()
    close(bits(out), expected_from_table(x_bits, st, table, routes))

    # Capture once, then republish slot 1 with another adapter: the replay must see it.
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    batch = table.batch(slots)
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, state, lora=batch, out=out)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, state, lora=batch, out=out)
    torch.cuda.current_stream().wait_stream(stream)
    table.publish_from(pool, handles["r12"], 1, ["proj"])
    table.clear(2)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        close(bits(out), expected_from_table(x_bits, st, table, routes))
    assert addresses == [t.data_ptr() for t in (table.a_store, table.b_store, table.ranks, table.b_strides, table.scales)]

    # Leases block eviction; evicted handles turn stale.
    with pool.borrow(handles["r4"]):
        with pytest.raises(RuntimeError, match="lease"):
            pool.evict(handles["r4"])
    pool.evict(handles["r4"])
    with pytest.raises(ValueError, match="stale"):
        table.publish_from(pool, handles["r4"], 0, ["proj"])


def zipf_routes(rng, m, adapters, s=1.1):
    p = 1.0 / np.arange(1, adapters + 1) ** s
    return rng.choice(adapters, size=m, p=p / p.sum()).astype(np.int32)


@pytest.mark.parametrize("m", [64, 256])
def test_c4_retained_ranks_zipf(m, device):
    """c4: 128 retained-rank adapters (ranks uniform over {4,8,16,32,64}), Zipf(1.1) routing."""
    k = n = 1024
    rng = np.random.default_rng(736)
    ranks = rng.choice([4, 8, 16, 32, 64], size=128).tolist()
    routes = zipf_routes(rng, m, 128)
    if m == 256:
        assert len(np.unique(routes)) > 64  # one prefill tile holds more than 64 distinct slots
    case = _cases.fused_case(m, n, k, ranks=ranks, seed=737, token_slots=routes)
    x, q, state, lora, _ = to_device(case, device)
    assert lora.max_rank == 64
    y = nf4_lora_linear(x, q, state, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)
