"""Host-side runtime: slot pools, PEFT files, retained-rank layout, slot table.

Behaviour restated from the reference's CPU tests (tests/test_runtime_slots.py:40-144,
tests/test_retained_layout.py:24-67) with this build's own fixtures: handles
go stale on replacement/eviction, failed loads keep the occupant and the byte
budget, compact exports keep the scaling, corrupt files fail the manifest
check, retained regions are frozen (addresses never change) and repack A to
the effective-rank prefix of each slice.
"""

import json
import math
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

from loraforge_amd.adapters import load_peft_adapter, save_peft_adapter
from loraforge_amd.runtime import AdapterSlots, AdapterTable, GPUAdapterSlots, RetainedLayout, effective_rank
from loraforge_amd.runtime.retained import bucket_of


def write_adapter(root, name, *, rank=4, in_features=6, out_features=5, alpha=8.0, rslora=False, modules=("proj",)):
    directory = root / name
    directory.mkdir()
    config = {
        "peft_type": "LORA",
        "r": rank,
        "lora_alpha": alpha,
        "target_modules": list(modules),
        "bias": "none",
        "use_rslora": rslora,
    }
    (directory / "adapter_config.json").write_text(json.dumps(config))
    tensors = {}
    for i, module in enumerate(modules):
        a = (torch.arange(rank * in_features, dtype=torch.float32).reshape(rank, in_features) + i) / 7.0
        b = torch.full((out_features, rank), 0.5 + i)
        tensors[f"base_model.model.{module}.lora_A.weight"] = a
        tensors[f"base_model.model.{module}.lora_B.weight"] = b
    save_file(tensors, str(directory / "adapter_model.safetensors"))
    return directory


@pytest.mark.parametrize("rslora", [False, True])
def test_slot_reuse_scaling_and_stale_handles(tmp_path, rslora):
    first = write_adapter(tmp_path, "first", rank=4, rslora=rslora)
    second = write_adapter(tmp_path, "second", rank=2)
    pool = AdapterSlots(1)
    handle = pool.load(first, 0)
    (module,) = pool.resolve(handle)
    assert module.rank == 4
    assert module.scaling == pytest.approx(8.0 / (math.sqrt(4) if rslora else 4))
    assert pool.tensor_bytes == (4 * 6 + 5 * 4) * 4
    module.a.zero_()  # resolve hands out copies
    assert pool.resolve(handle)[0].a.abs().sum() > 0
    replacement = pool.load(second, 0)
    for op in (pool.resolve, pool.evict):
        with pytest.raises(ValueError, match="stale"):
            op(handle)
    assert pool.resolve(replacement)[0].rank == 2
    pool.evict(replacement)
    assert pool.tensor_bytes == 0


def test_failed_load_keeps_occupant_and_budget(tmp_path):
    small = write_adapter(tmp_path, "small", rank=1)
    large = write_adapter(tmp_path, "large", rank=4)
    small_bytes = (1 * 6 + 5 * 1) * 4
    pool = AdapterSlots(2, max_tensor_bytes=small_bytes)
    handle = pool.load(small, 0)
    for path, slot in [(large, 0), (small, 1), (tmp_path / "absent", 0)]:
        with pytest.raises((ValueError, FileNotFoundError)):
            pool.load(path, slot)
        assert pool.resolve(handle)[0].rank == 1
        assert pool.tensor_bytes == small_bytes
    with pytest.raises(ValueError, match="different pool"):
        AdapterSlots(2).resolve(handle)


@pytest.mark.parametrize("capacity", [0, -3, True, 2.5])
def test_pool_capacity_validation(capacity):
    with pytest.raises(ValueError):
        AdapterSlots(capacity)


@pytest.mark.parametrize("limit", [-1, True, 0.5])
def test_pool_limit_validation(limit):
    with pytest.raises(ValueError):
        AdapterSlots(1, max_tensor_bytes=limit)


@pytest.mark.parametrize("slot", [-1, 1, True, 0.5])
def test_pool_slot_validation(tmp_path, slot):
    with pytest.raises(ValueError, match="slot"):
        AdapterSlots(1).load(tmp_path / "absent", slot)


def test_compact_export_keeps_scaling_and_manifest_guards_files(tmp_path):
    original = write_adapter(tmp_path, "original", rank=4, rslora=True)
    snapshot = load_peft_adapter(original)
    (module,) = snapshot.modules
    compact = save_peft_adapter(snapshot, tmp_path / "compact", factors={module.name: (module.a[:2].clone(), module.b[:, :2].clone())})
    pool = AdapterSlots(1)
    handle = pool.load(compact, 0)
    (resident,) = pool.resolve(handle)
    assert resident.rank == 2
    assert resident.scaling == pytest.approx(module.scaling)
    (compact / "adapter_model.safetensors").write_bytes(b"not a tensor file")
    with pytest.raises(ValueError, match="integrity"):
        pool.load(compact, 0)
    assert pool.resolve(handle)[0].rank == 2
    with pytest.raises(FileExistsError):
        save_peft_adapter(snapshot, compact)


def test_loader_rejects_inconsistent_files(tmp_path):
    bad_rank = write_adapter(tmp_path, "bad_rank", rank=3)
    config = json.loads((bad_rank / "adapter_config.json").read_text())
    config["r"] = 5
    (bad_rank / "adapter_config.json").write_text(json.dumps(config))
    with pytest.raises(ValueError, match="rank"):
        load_peft_adapter(bad_rank)
    bias = write_adapter(tmp_path, "bias")
    config = json.loads((bias / "adapter_config.json").read_text())
    config["bias"] = "all"
    (bias / "adapter_config.json").write_text(json.dumps(config))
    with pytest.raises(ValueError, match="bias"):
        load_peft_adapter(bias)


def test_concurrent_loads_into_independent_slots(tmp_path):
    path = write_adapter(tmp_path, "shared")
    pool = AdapterSlots(4)
    with ThreadPoolExecutor(max_workers=4) as ex:
        handles = list(ex.map(lambda s: pool.load(path, s), range(4)))
    assert pool.tensor_bytes == 4 * (4 * 6 + 5 * 4) * 4
    with ThreadPoolExecutor(max_workers=4) as ex:
        list(ex.map(pool.evict, handles))
    assert pool.tensor_bytes == 0


@pytest.mark.parametrize("device", ["cpu", "cuda", "meta"])
def test_gpu_pool_requires_an_indexed_gpu(device):
    with pytest.raises(ValueError, match="explicitly"):
        GPUAdapterSlots(1, device=device)


def catalog_ranks(gate, up=None, layer=0):
    prefix = f"base_model.model.model.layers.{layer}.mlp"
    return {
        f"{prefix}.gate_proj.lora_A.weight": gate,
        f"{prefix}.up_proj.lora_A.weight": gate if up is None else up,
    }


def test_effective_rank_takes_the_fused_maximum():
    assert effective_rank(catalog_ranks(2, 5), "gate_up_proj", 0) == 5
    assert effective_rank(catalog_ranks(2), "gate_up_proj", 1) == 0
    assert effective_rank(catalog_ranks(2), "qkv_proj", 0) == 0
    assert [bucket_of(k) for k in (0, 1, 3, 4, 5, 33, 64)] == [1, 1, 4, 4, 8, 64, 64]


def test_retained_layout_regions_repack_and_fixed_addresses():
    slots, width, cap = 2, 24, 96
    a = torch.arange(slots * 2 * cap * 8).reshape(slots, 2 * cap, 8).to(torch.bfloat16)
    b = (torch.arange(slots * width * cap) % 251).reshape(slots, width, cap).to(torch.bfloat16)
    catalog = {"small": catalog_ranks(5, 3), "mid": catalog_ranks(40), "wide": catalog_ranks(96)}
    layout = RetainedLayout(a, b, "gate_up_proj", 0, catalog)
    a0, b0 = a.clone(), b.clone()
    fields = (layout.a, layout.b, layout.store, layout.rank, layout.low, layout.high, layout.boff, layout.bucket)
    addresses = [t.data_ptr() for t in fields]

    off, bucket, k = layout.regions["small"]
    assert (bucket, k) == (8, 5) and off % 8 == 0
    layout.load("small", 1, cap)
    # A of slot 1 repacked to the rank-5 prefix of each of the two slices.
    torch.testing.assert_close(a[1, :10], torch.cat((a0[1, :5], a0[1, cap : cap + 5])))
    region = layout.store[off : off + width * bucket].view(width, bucket)
    torch.testing.assert_close(region[:, :5], b0[1, :, :5])
    assert not region[:, 5:].any()
    assert layout.low.tolist() == [0, 5] and layout.high.tolist() == [0, 0]
    assert layout.bucket.tolist() == [0, 8] and layout.boff.tolist() == [0, off]

    a[1].copy_(a0[1])
    layout.load("wide", 1, cap)  # rank above 64: unsupported by the compact path
    assert layout.unsupported.tolist() == [0, 96] and layout.supported.tolist() == [0, 0]
    a[1].copy_(a0[1])
    layout.load("mid", 1, cap)
    assert layout.high.tolist() == [0, 40] and layout.supported.tolist() == [0, 40]
    layout.load(None, 1)
    assert not layout.rank.any() and not layout.bucket.any()
    assert addresses == [t.data_ptr() for t in fields]
    torch.testing.assert_close(b, b0)
    before = a.clone()
    with pytest.raises(ValueError, match="catalog"):
        layout.load("absent", 1, cap)
    torch.testing.assert_close(a, before)


def test_retained_layout_rejects_bad_buffers():
    a = torch.zeros(2, 64, 8, dtype=torch.bfloat16)
    b = torch.zeros(2, 16, 32, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        RetainedLayout(a.float(), b, "gate_up_proj", 0, {"x": catalog_ranks(4)})
    with pytest.raises(ValueError, match="capacity"):
        RetainedLayout(a, b, "gate_up_proj", 0, {"x": catalog_ranks(48)})


def test_adapter_table_argument_validation():
    with pytest.raises(ValueError):
        AdapterTable(0, in_features=64, out_features=64, device="cpu")
    with pytest.raises(ValueError):
        AdapterTable(2, in_features=64, out_features=64, max_rank=65, device="cpu")
    with pytest.raises(ValueError):
        AdapterTable(2, in_features=60, out_features=64, device="cpu")
    with pytest.raises(ValueError):
        AdapterTable(2, in_features=64, out_features=64, slice_offsets=[0, 40, 30, 64], device="cpu")


def test_region_allocator_first_fit_merge_and_claim():
    from loraforge_amd.runtime.table import RegionAllocator

    regions = RegionAllocator(104)
    a, b, c = regions.take(10), regions.take(3), regions.take(20)
    assert (a, b, c) == (0, 16, 24)  # 8-element alignment
    assert regions.take(60) is None and regions.free == 56
    regions.give(b, 3)
    assert regions.take(8) == 16  # first fit reuses the hole
    regions.give(16, 8)
    regions.give(a, 10)
    regions.give(c, 20)
    assert regions.free == 104 and regions.take(104) == 0  # neighbours merged back into one range
    regions.give(0, 104)
    regions.claim(40, 8)
    with pytest.raises(ValueError, match="not free"):
        regions.claim(44, 8)
    assert regions.take(48) == 48 and regions.take(40) == 0


def _module(name, rank, k, n, seed, alpha=8.0):
    from loraforge_amd.adapters import AdapterModule

    g = torch.Generator().manual_seed(seed)
    a = (torch.randn(rank, k, generator=g) * 0.1).bfloat16()
    b = (torch.randn(n, rank, generator=g) * 0.1).bfloat16()
    return AdapterModule(name, a, b, alpha)


def _dense_lora(x_bits, y_bits, slots, factors, bounds):
    """y + bf16(scale * B_s (bf16(A_s x))) per routed token, in dense float64 algebra."""
    from oracle import nf4 as onf4

    x = onf4.bf16_to_f32(x_bits).astype(np.float64)
    out = y_bits.copy()
    for t, g in enumerate(slots):
        if g < 0 or g not in factors:
            continue
        a_parts, b_parts, scale = factors[g]
        for s, (lo, hi) in enumerate(zip(bounds, bounds[1:])):
            a = onf4.bf16_to_f32(a_parts[s]).astype(np.float64)
            b = onf4.bf16_to_f32(b_parts[s]).astype(np.float64)
            z = onf4.bf16_to_f32(onf4.f64_to_bf16_bits(a @ x[t])).astype(np.float64)
            delta = onf4.f64_to_bf16_bits(scale * (b @ z))
            base = onf4.bf16_to_f32(out[t, lo:hi]).astype(np.float64)
            out[t, lo:hi] = onf4.f64_to_bf16_bits(base + onf4.bf16_to_f32(delta))
    return out


def _batch_apply(batch, x_bits, y_bits, n):
    from oracle import linear

    as_np = lambda t: t.cpu().numpy()  # noqa: E731
    return linear.lora_apply(
        x_bits,
        y_bits,
        a_store=as_np(batch.a_store.view(torch.int16)).view(np.uint16),
        a_offsets=as_np(batch.a_offsets),
        b_store=as_np(batch.b_store.view(torch.int16)).view(np.uint16),
        b_offsets=as_np(batch.b_offsets),
        b_strides=as_np(batch.b_strides),
        ranks=as_np(batch.ranks),
        scales=as_np(batch.scales),
        token_slots=as_np(batch.token_slots),
        slice_offsets=as_np(batch.slice_offsets),
        n_total=n,
    )


def _bits(t):
    return t.view(torch.int16).numpy().view(np.uint16)


def test_adapter_table_compact_regions_and_full_store():
    k, bounds = 32, [0, 16, 40]
    n = bounds[-1]
    ranks = {0: 4, 1: 3, 2: 16}
    need = [sum(x) for x in zip(*(AdapterTable(1, in_features=k, out_features=n, slice_offsets=bounds, device="cpu").region_elements(r) for r in ranks.values()))]
    table = AdapterTable(4, in_features=k, out_features=n, max_rank=16, slice_offsets=bounds, device="cpu", a_elements=need[0], b_elements=need[1])
    assert table.a_store.numel() == 2 * (4 + 3 + 16) * k  # compact: no rank-16 padding per slot
    factors = {}
    for slot, r in ranks.items():
        mods = [_module(f"s{s}", r, k, hi - lo, seed=10 * slot + s) for s, (lo, hi) in enumerate(zip(bounds, bounds[1:]))]
        table.publish(slot, mods)
        factors[slot] = ([_bits(m.a) for m in mods], [_bits(m.b) for m in mods], mods[0].scaling)
    assert table.ranks.tolist()[:3] == [4, 3, 16] and table.b_strides.tolist()[:3] == [4, 4, 16]
    a_off, b_off, r = table.region_of(1)
    assert r == 3 and a_off % 8 == 0 and b_off % 8 == 0
    assert not table.b_store[b_off : b_off + n * 4].view(n, 4)[:, 3:].any()  # B zero padded to the bucket

    # The store is full: a fourth adapter is refused and nothing changes.
    before = [t.clone() for t in (table.a_offsets, table.b_offsets, table.ranks)]
    with pytest.raises(ValueError, match="full"):
        table.publish(3, [_module("s0", 2, k, 16, 1), _module("s1", 2, k, 24, 2)])
    with pytest.raises(ValueError, match="full"):
        table.publish(1, [_module("s0", 16, k, 16, 1), _module("s1", 16, k, 24, 2)])
    assert all(torch.equal(x, y) for x, y in zip(before, (table.a_offsets, table.b_offsets, table.ranks)))
    assert table.region_of(1) == (a_off, b_off, 3)

    # Clearing a slot frees its regions for another adapter of the same size.
    table.clear(1)
    assert table.region_of(1) is None and table.ranks.tolist()[1] == 0
    mods = [_module("s0", 3, k, 16, 77), _module("s1", 3, k, 24, 78)]
    table.publish(3, mods)
    factors.pop(1)
    factors[3] = ([_bits(m.a) for m in mods], [_bits(m.b) for m in mods], mods[0].scaling)

    rng = np.random.default_rng(4)
    m_tokens = 9
    x_bits = _bits(torch.from_numpy(rng.standard_normal((m_tokens, k)).astype(np.float32)).bfloat16())
    y_bits = _bits(torch.from_numpy(rng.standard_normal((m_tokens, n)).astype(np.float32)).bfloat16())
    slots = np.array([0, 1, 2, 3, -1, 3, 2, 0, 1], np.int32)
    got = _batch_apply(table.batch(torch.from_numpy(slots)), x_bits, y_bits, n)
    want = _dense_lora(x_bits, y_bits, slots.tolist(), factors, bounds)
    np.testing.assert_array_equal(got[slots == 1], y_bits[slots == 1])  # cleared slot: base only
    np.testing.assert_allclose(
        onf4_f32(got), onf4_f32(want), rtol=1e-2, atol=1e-2
    )


def onf4_f32(bits):
    from oracle import nf4 as onf4

    return onf4.bf16_to_f32(bits)


def test_retained_layout_feeds_the_fused_batch():
    """lora_batch over a loaded layout computes the LoRA of the pool's original padded factors."""
    slots, cap, k, width = 3, 8, 16, 24
    g = torch.Generator().manual_seed(3)
    a = (torch.randn(slots, 2 * cap, k, generator=g) * 0.1).bfloat16()
    b = (torch.randn(slots, width, cap, generator=g) * 0.1).bfloat16()
    a0, b0 = a.clone(), b.clone()
    catalog = {"p5": catalog_ranks(5, 3), "p8": catalog_ranks(8), "p0": catalog_ranks(2, layer=1)}
    layout = RetainedLayout(a, b, "gate_up_proj", 0, catalog)
    layout.load("p5", 0, cap)
    layout.load("p8", 2, cap)
    layout.load("p0", 1, cap)  # no module of this projection: rank 0, base only
    scales = torch.tensor([2.0, 1.0, 0.5])
    rng = np.random.default_rng(5)
    m_tokens = 7
    x_bits = _bits(torch.from_numpy(rng.standard_normal((m_tokens, k)).astype(np.float32)).bfloat16())
    y_bits = _bits(torch.from_numpy(rng.standard_normal((m_tokens, width)).astype(np.float32)).bfloat16())
    route = np.array([0, 2, 1, -1, 2, 0, 0], np.int32)
    batch = layout.lora_batch(torch.from_numpy(route), scales)
    assert batch.max_rank == 8 and batch.slice_offsets.tolist() == [0, 12, 24]
    got = _batch_apply(batch, x_bits, y_bits, width)
    factors = {}
    for slot, r in ((0, 5), (2, 8)):
        a_parts = [_bits(a0[slot, s * cap : s * cap + r].contiguous()) for s in range(2)]
        b_parts = [_bits(b0[slot, s * 12 : (s + 1) * 12, :r].contiguous()) for s in range(2)]
        factors[slot] = (a_parts, b_parts, float(scales[slot]))
    want = _dense_lora(x_bits, y_bits, route.tolist(), factors, [0, 12, 24])
    np.testing.assert_array_equal(got[route == 1], y_bits[route == 1])
    np.testing.assert_allclose(onf4_f32(got), onf4_f32(want), rtol=1e-2, atol=1e-2)
    with pytest.raises(ValueError, match="slice_offsets"):
        layout.lora_batch(torch.from_numpy(route), scales, slice_offsets=[0, 24])
    # The device bounds of a partition are built once and reused (no host copy per call);
    # a partition first seen under graph capture is refused.
    again = layout.lora_batch(torch.from_numpy(route), scales)
    assert again.slice_offsets is batch.slice_offsets
    from loraforge_amd.runtime import retained

    capturing = retained._capturing
    try:
        retained._capturing = lambda device: True
        assert layout.lora_batch(torch.from_numpy(route), scales).slice_offsets is batch.slice_offsets
        with pytest.raises(RuntimeError, match="before capturing"):
            layout.lora_batch(torch.from_numpy(route), scales, slice_offsets=[0, 8, 24])
    finally:
        retained._capturing = capturing


def test_retained_layout_refuses_wide_slots_in_the_fused_batch():
    a = torch.zeros(2, 2 * 96, 8, dtype=torch.bfloat16)
    b = torch.zeros(2, 16, 96, dtype=torch.bfloat16)
    layout = RetainedLayout(a, b, "gate_up_proj", 0, {"wide": catalog_ranks(96)})
    layout.load("wide", 0, 96)
    with pytest.raises(ValueError, match="above 64"):
        layout.lora_batch(torch.zeros(1, dtype=torch.int32), torch.ones(2))


def _padded_checkpoint(root, name, rank, retained=None, nonzero_tail=False):
    directory = root / name
    directory.mkdir()
    (directory / "adapter_config.json").write_text(json.dumps({"peft_type": "LORA", "r": rank, "lora_alpha": 16, "target_modules": ["gate_proj", "up_proj"]}))
    tensors, module_ranks = {}, {}
    for i, proj in enumerate(("gate_proj", "up_proj")):
        key = f"base_model.model.model.layers.0.mlp.{proj}"
        keep = rank if retained is None else retained[i]
        a = torch.zeros(rank, 8)
        b = torch.zeros(16, rank)
        a[:keep] = 1.0
        b[:, :keep] = 1.0
        if nonzero_tail:
            b[0, -1] = 1.0
        tensors[key + ".lora_A.weight"], tensors[key + ".lora_B.weight"] = a, b
        module_ranks[key + ".lora_A.weight"] = keep
    save_file(tensors, str(directory / "adapter_model.safetensors"))
    if retained is not None:
        (directory / "compression.json").write_text(json.dumps({"module_ranks": module_ranks}))
    return directory


def test_rank_catalog_reads_headers_and_retained_ranks(tmp_path):
    from loraforge_amd.runtime import read_rank_catalog

    plain = _padded_checkpoint(tmp_path, "plain", 16)
    reduced = _padded_checkpoint(tmp_path, "reduced", 16, retained=(3, 7))
    catalog = read_rank_catalog([plain, reduced])
    assert effective_rank(catalog[str(plain)], "gate_up_proj", 0) == 16
    assert effective_rank(catalog[str(reduced)], "gate_up_proj", 0) == 7
    bad = _padded_checkpoint(tmp_path, "bad", 16, retained=(3, 7), nonzero_tail=True)
    with pytest.raises(ValueError, match="truncates nonzero"):
        read_rank_catalog([bad])
    over = _padded_checkpoint(tmp_path, "over", 4, retained=(3, 4))
    meta = json.loads((over / "compression.json").read_text())
    meta["module_ranks"] = {key: 5 for key in meta["module_ranks"]}
    (over / "compression.json").write_text(json.dumps(meta))
    with pytest.raises(ValueError, match="exceeds checkpoint rank"):
        read_rank_catalog([over])
    with pytest.raises(ValueError, match="nonempty"):
        read_rank_catalog([])


def test_safetensors_reader_rejects_malformed_files(tmp_path):
    from loraforge_amd.adapters import read_safetensors

    good = write_adapter(tmp_path, "good") / "adapter_model.safetensors"
    tensors = read_safetensors(good)
    assert tensors["base_model.model.proj.lora_B.weight"].shape == (5, 4)
    blob = good.read_bytes()
    size = int.from_bytes(blob[:8], "little")
    header = json.loads(blob[8 : 8 + size])
    cases = {
        "length": (10**9).to_bytes(8, "little") + blob[8:],
        "covered": blob + b"\0" * 8,
    }
    wrong_dtype = dict(header)
    key = "base_model.model.proj.lora_A.weight"
    wrong_dtype[key] = dict(header[key], dtype="I64")
    raw = json.dumps(wrong_dtype).encode()
    cases["dtype"] = len(raw).to_bytes(8, "little") + raw + blob[8 + size :]
    for match, data in cases.items():
        path = tmp_path / f"{match}.safetensors"
        path.write_bytes(data)
        with pytest.raises(ValueError, match=match):
            read_safetensors(path)
