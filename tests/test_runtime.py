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
