"""NF4 weights on disk: bitsandbytes' packed QuantState entries in safetensors.

The layout is the one the reference writes with ``state.as_dict(packed=True)``
(``benchmarks/prepare_qwen35_nf4.py:59-60``) and reads back by key prefix
(``benchmarks/check_qwen35_nf4_ops.py:73-85``). bitsandbytes itself is absent,
so the byte-level format (key names, the JSON fields of the packed entry) is
pinned by the restated layout only; what the tests pin independently is the
round trip (stored and reloaded weights dequantise bit-identically through the
oracle) and the rejection of foreign or inconsistent states.
"""

import json

import numpy as np
import pytest
import torch

from loraforge_amd.ops.nf4 import quantize_nf4
from loraforge_amd.ops.quant_state import (
    load_nf4_weight,
    quant_state_entries,
    quant_state_from_entries,
    save_nf4_weights,
)
from oracle import nf4 as onf4


def weight(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)


def oracle_dequant(qweight, state):
    q = qweight.reshape(-1).numpy()
    if state.nested:
        scales = onf4.dq_scales(
            state.absmax.numpy(),
            state.state2.absmax.numpy(),
            state.state2.code.numpy(),
            np.float32(state.offset.item()),
            dq_block=state.state2.blocksize,
        )
    else:
        scales = state.absmax.numpy()
    return onf4.dequantize(q, scales, tuple(state.shape), code=state.code.numpy())


@pytest.mark.parametrize("nested", [False, True])
def test_file_round_trip_dequantises_identically(tmp_path, nested):
    w1, w2 = weight(128, 192, 1), weight(64, 256, 2)
    q1, s1 = quantize_nf4(w1, compress_statistics=nested)
    q2, s2 = quantize_nf4(w2, compress_statistics=nested)
    path = tmp_path / "model.safetensors"
    save_nf4_weights(path, {"layers.0.up.weight": (q1, s1), "layers.0.up.weight_b": (q2, s2)})
    for name, q, s in (("layers.0.up.weight", q1, s1), ("layers.0.up.weight_b", q2, s2)):
        lq, ls = load_nf4_weight(path, name)
        assert torch.equal(lq, q) and ls.shape == s.shape and ls.nested == nested
        assert ls.dtype == torch.bfloat16 and ls.blocksize == 64 and ls.quant_type == "nf4"
        assert torch.equal(ls.absmax, s.absmax) and torch.equal(ls.code, s.code)
        if nested:
            assert torch.equal(ls.state2.absmax, s.state2.absmax) and ls.state2.blocksize == 256
            assert float(ls.offset) == float(s.offset)
        np.testing.assert_array_equal(oracle_dequant(lq, ls), oracle_dequant(q, s))


def test_packed_entry_layout():
    q, s = quantize_nf4(weight(64, 128, 3), compress_statistics=True)
    entries = quant_state_entries(q, s, "w")
    assert set(entries) == {
        "w",
        "w.absmax",
        "w.quant_map",
        "w.nested_absmax",
        "w.nested_quant_map",
        "w.quant_state.bitsandbytes__nf4",
    }
    blob = entries["w.quant_state.bitsandbytes__nf4"]
    assert blob.dtype == torch.uint8 and blob.ndim == 1
    fields = json.loads(bytes(blob.tolist()).decode("utf-8"))
    assert fields == {
        "quant_type": "nf4",
        "blocksize": 64,
        "dtype": "bfloat16",
        "shape": [64, 128],
        "nested_blocksize": 256,
        "nested_dtype": "float32",
        "nested_offset": float(s.offset),
    }
    assert entries["w.absmax"].dtype == torch.uint8 and entries["w.nested_quant_map"].numel() == 256


def _edit(entries, name, **fields):
    blob = entries[f"{name}.quant_state.bitsandbytes__nf4"]
    data = json.loads(bytes(blob.tolist()).decode("utf-8"))
    data.update(fields)
    out = dict(entries)
    out[f"{name}.quant_state.bitsandbytes__nf4"] = torch.tensor(list(json.dumps(data).encode()), dtype=torch.uint8)
    return out


def test_rejects_foreign_and_inconsistent_states():
    q, s = quantize_nf4(weight(64, 128, 4))
    good = quant_state_entries(q, s, "w")
    quant_state_from_entries(good, "w")
    with pytest.raises(ValueError, match="not nf4"):
        quant_state_from_entries(_edit(good, "w", quant_type="fp4"), "w")
    with pytest.raises(ValueError, match="not 64"):
        quant_state_from_entries(_edit(good, "w", blocksize=128), "w")
    with pytest.raises(ValueError, match="bytes for shape"):
        quant_state_from_entries(_edit(good, "w", shape=[128, 128]), "w")
    with pytest.raises(ValueError, match="unexpected"):
        quant_state_from_entries(_edit(good, "w", extra=1), "w")
    missing = {k: v for k, v in good.items() if "quant_state" not in k}
    with pytest.raises(ValueError, match="exactly one"):
        quant_state_from_entries(missing, "w")
    wrong = dict(good)
    wrong["w.absmax"] = good["w.absmax"].to(torch.uint8)
    with pytest.raises(ValueError, match="does not match nested"):
        quant_state_from_entries(wrong, "w")
    with pytest.raises(ValueError, match="no packed weight"):
        quant_state_from_entries(good, "v")
