"""Host-side contract checks that run without a GPU (CPU tensors are rejected).

Mirrors the structural rejection cases of the reference
(``tests/test_row_operators_gpu.py:262-276``, ``tests/test_nf4_gpu.py:40-48``,
``tests/test_gemv_contracts.py``): wrong device, alignment, autograd,
lengths, thread counts and output aliasing raise before any launch.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import LoraBatch, dequantize_nf4, nf4_lora_linear, quantize_nf4, row_expand, row_shrink
from loraforge_amd.ops.nf4 import NF4State


def test_row_ops_reject_cpu_tensors():
    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    a = torch.zeros(1, 4, 8, dtype=torch.bfloat16)
    z = torch.zeros(2, 4, dtype=torch.bfloat16)
    slots = torch.zeros(2, dtype=torch.int32)
    ranks = torch.ones(1, dtype=torch.int32)
    with pytest.raises(ValueError, match="same CUDA"):
        row_shrink(x, a, z, slots, ranks, max_rank=4)
    meta = dict(
        b_offsets=torch.zeros(1, dtype=torch.int64),
        b_strides=torch.ones(1, dtype=torch.int32),
        ranks=ranks,
        scales=torch.ones(1),
        segment_indptr=torch.tensor([0, 1], dtype=torch.int32),
        segment_slots=torch.zeros(1, dtype=torch.int32),
        token_indices=torch.zeros(1, dtype=torch.int32),
        slice_offsets=torch.tensor([0, 4], dtype=torch.int32),
        segment_count=torch.ones(1, dtype=torch.int32),
    )
    with pytest.raises(ValueError, match="same CUDA"):
        row_expand(z, torch.zeros(4, dtype=torch.bfloat16), torch.zeros(2, 4, dtype=torch.bfloat16), **meta)


def test_row_ops_reject_bad_types_and_slices():
    with pytest.raises(TypeError):
        row_shrink([1], None, None, None, None)
    x = torch.zeros(2, 8, dtype=torch.float32)
    with pytest.raises(ValueError, match="dtype"):
        row_shrink(x, x, x, x, x)


def test_dequant_rejects_bad_shapes_and_devices():
    q = torch.zeros(64 * 32, dtype=torch.uint8)
    s = torch.ones(64, dtype=torch.float32)
    c = torch.zeros(16, dtype=torch.float32)
    with pytest.raises(ValueError, match="multiples of64"):
        dequantize_nf4(q, s, c, (64, 63))
    with pytest.raises(ValueError, match="multiples of64"):
        dequantize_nf4(q, s, c, [64, 64])
    with pytest.raises(TypeError):
        dequantize_nf4(q.numpy(), s, c, (64, 64))
    with pytest.raises(ValueError, match="CUDA"):
        dequantize_nf4(q, s, c, (64, 64))


def test_fused_rejects_cpu_and_bad_shapes():
    w = torch.randn(128, 64, dtype=torch.bfloat16) * 0.02
    q, st = quantize_nf4(w)
    x = torch.zeros(2, 64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="same CUDA"):
        nf4_lora_linear(x, q, st)
    with pytest.raises(ValueError, match="unit column stride|\\[..., K\\]"):
        nf4_lora_linear(torch.zeros(2, 32, dtype=torch.bfloat16), q, st)
    bad = NF4State(st.absmax, st.shape, st.code, torch.bfloat16, blocksize=128)
    with pytest.raises(ValueError, match="block64"):
        nf4_lora_linear(x, q, bad)
    with pytest.raises(ValueError, match="inference"):
        nf4_lora_linear(x.clone().float().requires_grad_().bfloat16(), q, st)


def test_lora_batch_from_padded_offsets():
    a = torch.zeros(3, 32, 64, dtype=torch.bfloat16)
    lb = LoraBatch.from_padded(
        a,
        torch.zeros(8, dtype=torch.bfloat16),
        b_offsets=torch.zeros(3, dtype=torch.int64),
        b_strides=torch.ones(3, dtype=torch.int32),
        ranks=torch.zeros(3, dtype=torch.int32),
        scales=torch.zeros(3),
        token_slots=torch.zeros(1, dtype=torch.int32),
        slice_offsets=torch.tensor([0, 16, 32], dtype=torch.int32),
    )
    assert lb.a_offsets.tolist() == [0, 32 * 64, 2 * 32 * 64]
    assert lb.num_slices == 2 and lb.a_store.ndim == 1


def test_silu_mul_rejects_cpu_and_bad_types():
    from loraforge_amd.ops.activation import silu_mul

    with pytest.raises(ValueError, match="same CUDA"):
        silu_mul(torch.zeros(2, 16, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="dtype"):
        silu_mul(torch.zeros(2, 16, dtype=torch.float32))
    with pytest.raises(TypeError):
        silu_mul(np.zeros((2, 16)))
