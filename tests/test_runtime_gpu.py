"""GPU runtime path: PEFT files -> GPUAdapterSlots -> AdapterTable -> fused linear.

Checks that the fixed-address table holds exactly the borrowed factors (A
packed per slice, B zero padded to the rank bucket), that ``nf4_lora_linear``
on the table matches the oracle chain, and that a HIP graph captured once
sees an adapter republished into the same slot (addresses never move). The
pool's stream contract (reference tests/test_runtime_gpu.py:45-102): a load
on one stream is ordered before a lease on another, leases block reloads and
evictions, images outlive the queued work that reads them. And the c4
configuration (retained ranks {4, 8, 16, 32, 64}, Zipf(1.1) over 128 slots)
at 4096 x 4096 through both adapter layouts the fused kernels take: a compact
AdapterTable and an SGLang-style padded pool behind RetainedLayout.
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
        a_off, b_off, held = table.region_of(slot)
        assert held == rank and int(table.a_offsets[slot]) == a_off and int(table.b_offsets[slot]) == b_off
        a_rows = table.a_store[a_off : a_off + rank * k].view(rank, k).cpu()
        torch.testing.assert_close(a_rows, a)
        bucket = int(table.b_strides[slot])
        assert bucket == _cases.bucket_of(rank)
        b_view = table.b_store[b_off : b_off + n * bucket].view(n, bucket).cpu()
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


@pytest.fixture(scope="module")
def square_weight(device):
    from loraforge_amd.ops.quant_state import NF4State

    st = _cases.torch_quantized_state(4096, 4096, seed=731)
    w_bits = onf4.dequantize(st["qweight"], st["scales"], st["shape"])
    q = torch.from_numpy(st["qweight"]).to(device)
    state = NF4State(torch.from_numpy(st["absmax"]).to(device), torch.Size(st["shape"]), torch.from_numpy(st["code"]).to(device), torch.bfloat16)
    return w_bits, q, state


def _expected_from_batch(x_bits, w_bits, batch, n):
    y = linear.nf4_linear(x_bits, w_bits)
    as_np = lambda t: t.cpu().numpy()  # noqa: E731
    return linear.lora_apply(
        x_bits,
        y,
        a_store=bits(batch.a_store),
        a_offsets=as_np(batch.a_offsets),
        b_store=bits(batch.b_store),
        b_offsets=as_np(batch.b_offsets),
        b_strides=as_np(batch.b_strides),
        ranks=as_np(batch.ranks),
        scales=as_np(batch.scales),
        token_slots=as_np(batch.token_slots),
        slice_offsets=as_np(batch.slice_offsets),
        n_total=n,
    )


@pytest.mark.filterwarnings("error::pytest.PytestUnraisableExceptionWarning")
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rslora", [False, True])
def test_pool_cross_stream_lease_and_lifetime(tmp_path, device, dtype, rslora):
    """A load on one stream is ordered before a lease on another; the image outlives queued readers."""
    rank, k, n = 3, 64, 32
    d = tmp_path / "first"
    d.mkdir()
    (d / "adapter_config.json").write_text(
        json.dumps({"peft_type": "LORA", "r": rank, "lora_alpha": 6, "target_modules": ["proj"], "use_rslora": rslora})
    )
    a = (torch.arange(rank * k).reshape(rank, k) / 100).to(dtype)
    b = (torch.arange(n * rank).reshape(n, rank) / 100).to(dtype)
    save_file({"base_model.model.proj.lora_A.weight": a, "base_model.model.proj.lora_B.weight": b}, str(d / "adapter_model.safetensors"))
    other, _, _ = write_adapter(tmp_path, "other", 1, k, n, 3, 2.0)
    pool = GPUAdapterSlots(1, device=str(device))
    producer, consumer = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(producer):
        handle = pool.load(d, 0)
    with torch.cuda.stream(consumer):
        with pool.borrow(handle) as modules:
            (mod,) = modules
            assert mod.a.device == device and mod.a.dtype == dtype and mod.a.is_contiguous() and mod.b.is_contiguous()
            result = (mod.b.float() @ mod.a.float()) * mod.scaling
            with pytest.raises(RuntimeError, match="active"):
                pool.load(other, 0)
            with pytest.raises(RuntimeError, match="active"):
                pool.evict(handle)
        del modules, mod
    with torch.cuda.stream(producer):
        replacement = pool.load(other, 0)
    with pytest.raises(ValueError, match="stale"):
        with pool.borrow(handle):
            pass
    pool.evict(replacement)
    del pool
    churn = [torch.empty((rank, k), device=device, dtype=dtype) for _ in range(32)]
    consumer.synchronize()
    scale = 6 / (rank**0.5 if rslora else rank)
    torch.testing.assert_close(result.cpu(), (b.float() @ a.float()) * scale)
    del churn


@pytest.mark.filterwarnings("error::pytest.PytestUnraisableExceptionWarning")
def test_pool_budget_and_exception_release(tmp_path, device):
    small, _, _ = write_adapter(tmp_path, "small", 1, 64, 32, 1, 2.0)
    large, _, _ = write_adapter(tmp_path, "large", 3, 64, 32, 2, 2.0)
    small_bytes = (64 + 32) * 2
    pool = GPUAdapterSlots(1, device=str(device), max_tensor_bytes=small_bytes)
    handle = pool.load(small, 0)
    assert pool.tensor_bytes == small_bytes
    with pytest.raises(ValueError, match="limit"):
        pool.load(large, 0)
    with pytest.raises(ValueError, match="different"):
        with GPUAdapterSlots(1, device=str(device)).borrow(handle):
            pass
    with pytest.raises(RuntimeError, match="consumer failure"):
        with pool.borrow(handle):
            raise RuntimeError("consumer failure")
    pool.collect()
    pool.evict(handle)
    assert pool.tensor_bytes == 0
    with pytest.raises(ValueError, match="stale"):
        pool.evict(handle)


def _c4_adapters(rng, k, n):
    from loraforge_amd.adapters import AdapterModule

    ranks = rng.choice([4, 8, 16, 32, 64], size=128).tolist()
    mods = []
    for r in ranks:
        a = torch.from_numpy(rng.standard_normal((r, k)).astype(np.float32) * 0.02).bfloat16()
        b = torch.from_numpy(rng.standard_normal((n, r)).astype(np.float32) * 0.02).bfloat16()
        mods.append(AdapterModule("proj", a, b, 2.0 * r))
    return ranks, mods


@pytest.mark.parametrize("m", [64, 256])
def test_c4_compact_table_full_size(square_weight, m, device):
    """c4 at 4096 x 4096 through a compact AdapterTable: 128 ragged ranks, Zipf(1.1) routes."""
    w_bits, q, state = square_weight
    k = n = 4096
    rng = np.random.default_rng(741)
    ranks, mods = _c4_adapters(rng, k, n)
    probe = AdapterTable(1, in_features=k, out_features=n, device="cpu", a_elements=1, b_elements=1)
    need = [sum(x) for x in zip(*(probe.region_elements(r) for r in ranks))]
    table = AdapterTable(128, in_features=k, out_features=n, device=device, a_elements=need[0], b_elements=need[1])
    # Compact: exactly sum(r) A rows and sum(bucket(r)) = sum(r) B columns, not 128 x 64 of each.
    assert table.a_store.numel() == k * sum(ranks) and table.b_store.numel() == n * sum(ranks)
    for slot, mod in enumerate(mods):
        table.publish(slot, [_on_device(mod, device)])
    routes = _cases.zipf_routes(rng, m, 128)
    x_bits = _cases.bf16(rng.standard_normal((m, k)))
    batch = table.batch(torch.from_numpy(routes).to(device))
    y = nf4_lora_linear(t16(x_bits, device), q, state, lora=batch)
    torch.cuda.synchronize()
    close(bits(y), _expected_from_batch(x_bits, w_bits, batch, n))
    workspace_clean(device)


def _on_device(mod, device):
    from loraforge_amd.adapters import AdapterModule

    return AdapterModule(mod.name, mod.a.to(device), mod.b.to(device), mod.alpha, mod.use_rslora)


@pytest.mark.parametrize("m", [64, 256])
def test_c4_retained_layout_full_size(square_weight, m, device):
    """An SGLang-style padded pool (128 slots, capacity 64) served through RetainedLayout.lora_batch."""
    from loraforge_amd.runtime import RetainedLayout

    w_bits, q, state = square_weight
    k = n = 4096
    rng = np.random.default_rng(742)
    ranks = rng.choice([4, 8, 16, 32, 64], size=128).tolist()
    a = torch.zeros(128, 64, k, dtype=torch.bfloat16, device=device)
    b = torch.zeros(128, n, 64, dtype=torch.bfloat16, device=device)
    catalog = {}
    for slot, r in enumerate(ranks):
        a[slot, :r] = torch.from_numpy(rng.standard_normal((r, k)).astype(np.float32) * 0.02).bfloat16().to(device)
        b[slot, :, :r] = torch.from_numpy(rng.standard_normal((n, r)).astype(np.float32) * 0.02).bfloat16().to(device)
        catalog[f"ckpt{slot}"] = {f"base_model.model.model.layers.0.self_attn.o_proj.lora_A.weight": r}
    layout = RetainedLayout(a, b, "o_proj", 0, catalog)
    for slot in range(128):
        layout.load(f"ckpt{slot}", slot, 64)
    assert layout.store.numel() == sum(n * r for r in ranks)  # ranks are powers of two: buckets equal ranks
    routes = _cases.zipf_routes(rng, m, 128)
    x_bits = _cases.bf16(rng.standard_normal((m, k)))
    scales = torch.full((128,), 2.0, device=device)
    batch = layout.lora_batch(torch.from_numpy(routes).to(device), scales)
    y = nf4_lora_linear(t16(x_bits, device), q, state, lora=batch)
    torch.cuda.synchronize()
    close(bits(y), _expected_from_batch(x_bits, w_bits, batch, n))
    workspace_clean(device)
