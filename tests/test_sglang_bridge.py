"""SGLang batch metadata -> per-token slot map -> one fused call per projection.

``batch_info`` is faked with ``SimpleNamespace`` as the reference's own SGLang
tests do (tests/test_sglang_gpu.py:30-41; SGLang is not installed). The slot
map is checked against a direct per-segment expansion written independently
here; the GPU test checks the fused call on it against the oracle (routes
from the same expansion), graph replay with new metadata, and both adapter
layouts (RetainedLayout over padded pools, AdapterTable).
"""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

from loraforge_amd.integrations import lora_batch_from_batch_info, token_slots_from_batch_info


def expand_segments(tokens, seg_indptr, weight_indices, permutation, nseg):
    """Per-token slots by walking the segments one by one (-1 for tokens no live segment covers)."""
    routes = [-1] * tokens
    for s in range(nseg):
        for j in range(seg_indptr[s], seg_indptr[s + 1]):
            t = j if permutation is None else permutation[j]
            routes[t] = weight_indices[s]
    return np.asarray(routes, np.int32)


def random_info(rng, tokens, slots, *, padded=0, permuted=True, uncovered=0, segments=None, device="cpu"):
    covered = tokens - uncovered
    want = int(rng.integers(1, 9)) - 1 if segments is None else segments - 1  # cuts between segments
    cuts = np.sort(rng.choice(np.arange(1, covered), size=min(covered - 1, want), replace=False)) if covered > 1 else np.array([], int)
    indptr = np.concatenate([[0], cuts, [covered]]).astype(np.int32)
    nseg = len(indptr) - 1
    weights = rng.integers(0, slots, nseg).astype(np.int32)
    perm = rng.permutation(tokens).astype(np.int32) if permuted else None
    # Capacity-padded metadata as in captured graphs: entries past num_segments are junk.
    indptr_p = np.concatenate([indptr, np.full(padded, 10**6, np.int32)])
    weights_p = np.concatenate([weights, rng.integers(0, slots, padded).astype(np.int32)])
    t = lambda a: None if a is None else torch.from_numpy(a).to(device)  # noqa: E731
    info = SimpleNamespace(num_segments=nseg, seg_indptr=t(indptr_p), weight_indices=t(weights_p), permutation=t(perm))
    return info, expand_segments(tokens, indptr, weights, perm, nseg)


@pytest.mark.parametrize("seed", range(6))
def test_token_slots_follow_segments_and_permutation(seed):
    rng = np.random.default_rng(seed)
    tokens = int(rng.integers(1, 70))
    info, expect = random_info(rng, tokens, 9, padded=int(rng.integers(0, 4)), permuted=seed % 2 == 0,
                               uncovered=int(rng.integers(0, min(3, tokens))))
    np.testing.assert_array_equal(token_slots_from_batch_info(info, tokens).numpy(), expect)


def test_token_slots_reuse_a_buffer_and_handle_empty_batches():
    rng = np.random.default_rng(3)
    out = torch.full((12,), 77, dtype=torch.int32)
    address = out.data_ptr()
    for _ in range(3):
        info, expect = random_info(rng, 12, 5)
        assert token_slots_from_batch_info(info, 12, out=out).data_ptr() == address
        np.testing.assert_array_equal(out.numpy(), expect)
    info.num_segments = 0
    assert token_slots_from_batch_info(info, 12, out=out).tolist() == [-1] * 12
    assert token_slots_from_batch_info(info, 0).numel() == 0
    with pytest.raises(ValueError, match="int32"):
        token_slots_from_batch_info(info, 12, out=torch.zeros(12, dtype=torch.int64))
    with pytest.raises(ValueError, match="seg_indptr"):
        token_slots_from_batch_info(SimpleNamespace(num_segments=4, seg_indptr=torch.zeros(3, dtype=torch.int32),
                                                    weight_indices=torch.zeros(4, dtype=torch.int32)), 5)


def test_batch_from_a_retained_layout_takes_sglang_scalings():
    from loraforge_amd.runtime import RetainedLayout

    a = torch.zeros(3, 2 * 8, 16, dtype=torch.bfloat16)
    b = torch.zeros(3, 24, 8, dtype=torch.bfloat16)
    key = "base_model.model.model.layers.0.mlp.{}_proj.lora_A.weight"
    layout = RetainedLayout(a, b, "gate_up_proj", 0, {"x": {key.format("gate"): 4, key.format("up"): 4}})
    layout.load("x", 1, 8)
    rng = np.random.default_rng(1)
    info, expect = random_info(rng, 10, 3)
    info.scalings = torch.tensor([0.5, 2.0, 1.0])
    batch = lora_batch_from_batch_info(info, layout, tokens=10)
    np.testing.assert_array_equal(batch.token_slots.numpy(), expect)
    assert batch.scales is info.scalings and batch.ranks.tolist() == [0, 4, 0]
    del info.scalings
    with pytest.raises(ValueError, match="scalings"):
        lora_batch_from_batch_info(info, layout, tokens=10)
