"""The product's offline NF4 quantiser (torch) agrees with the oracle's input generator."""

import numpy as np
import pytest
import torch

from loraforge_amd.ops.nf4 import NF4_CODE, dynamic_map, quantize_nf4
from oracle import nf4 as onf4


def _weight(seed=731, shape=(128, 256)):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * 0.1).bfloat16()


def test_plain_quantiser_matches_oracle():
    w = _weight()
    q, st = quantize_nf4(w)
    ref = onf4.quantize(w.float().numpy())
    assert np.array_equal(q.reshape(-1).numpy(), ref["qweight"])
    assert np.array_equal(st.absmax.numpy(), ref["absmax"])
    assert torch.equal(st.code, torch.tensor(NF4_CODE, dtype=torch.float32))
    assert not st.nested and st.shape == (128, 256)


def test_nested_quantiser_round_trip():
    w = _weight(seed=1)
    q, st = quantize_nf4(w, compress_statistics=True)
    assert st.nested and st.absmax.dtype == torch.uint8
    scales = onf4.dq_scales(st.absmax.numpy(), st.state2.absmax.numpy(), st.state2.code.numpy(), st.offset.item())
    dq = onf4.bf16_to_f32(onf4.dequantize(q.reshape(-1).numpy(), scales, (128, 256)))
    err = np.abs(dq - w.float().numpy()).reshape(-1, 64).max(axis=1)
    absmax = np.abs(w.float().numpy()).reshape(-1, 64).max(axis=1)
    assert np.all(err <= 0.2 * absmax + 1e-6)


def test_dynamic_map_agrees_with_oracle_table():
    # Both restate the same recipe; torch's linspace is the one the oracle emulates.
    assert np.array_equal(dynamic_map().numpy(), onf4.dynamic_map())


@pytest.mark.parametrize("shape", [(64, 63), (3, 64)])
def test_quantiser_rejects_ragged_shapes(shape):
    with pytest.raises(ValueError):
        quantize_nf4(torch.zeros(shape, dtype=torch.bfloat16))
