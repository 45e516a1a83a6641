"""NF4 base linear + per-token multi-LoRA chain in numpy. TEST INFRASTRUCTURE ONLY.

The reference serving path for one quantised projection with LoRA is three
steps (``src/loraforge/integrations/_sglang_nf4_linear.py:116-129`` for the
base, ``integrations/_sglang_fleet.py:271-407`` for the LoRA calls):

1. ``y = bf16(x @ dequant(W)^T)`` with fp32 accumulation (hipBLASLt ``F.linear``),
   then ``y = bf16(y + bias)`` when a bias exists;
2. ``z = bf16(A_g @ x)`` per token (``row_shrink``);
3. ``y = bf16(y + bf16(scale_g * B_g @ z))`` per token and slice (``row_expand``).

Here the adapter of token ``m`` is ``token_slots[m]`` and slot ``g``'s A rows
(``S * r`` rows of width K, packed at ``s * r`` as in ``row_shrink``) start at
element ``a_offsets[g]`` of a flat store. Prefill uses the same chain with the
token -> slot map expanded from contiguous segments
(``benchmarks/qwen35_prefill_fused.py:95-171``, ``segmented_ab_kernel``).

The SwiGLU step (``benchmarks/qwen35_decode_silu.py:50-61``,
``qwen35_prefill_fused.py:74-87`` with ``ROUND_ACT``) is
``h = bf16(bf16(silu(gate)) * up)`` on the LoRA-updated bf16 gate/up values.

Dot products use float64 and round through fp32 to bf16 (reference test
convention). Pinning: tests/test_oracle_rows.py checks these functions
against the already pinned ``oracle.rows`` operators (shrink + expand with
one-token segments must equal the per-token chain), against ``torch`` CPU
``F.linear`` on the dequantised weight, and a brute-force scalar loop.
"""

from __future__ import annotations

import numpy as np

from .nf4 import bf16_to_f32, bf16_bits, f64_to_bf16_bits
from .rows import add_bf16, expand_delta, slot_b


def nf4_linear(x_bits, w_bits, bias_bits=None, *, rows=None) -> np.ndarray:
    """``bf16(x @ W^T)`` (+ bias). ``rows`` restricts the output columns computed."""
    x64 = bf16_to_f32(x_bits).astype(np.float64)
    w = np.asarray(w_bits)
    if rows is not None:
        w = w[rows]
    y = f64_to_bf16_bits(x64 @ bf16_to_f32(w).astype(np.float64).T)
    if bias_bits is not None:
        b = np.asarray(bias_bits)
        y = add_bf16(y, b if rows is None else b[rows])
    return y


def slot_a(a_store, offset: int, rows: int, width: int) -> np.ndarray:
    flat = bf16_to_f32(np.asarray(a_store).reshape(-1)[offset : offset + rows * width])
    return flat.astype(np.float64).reshape(rows, width)


def lora_apply(
    x_bits,
    y_bits,
    *,
    a_store,
    a_offsets,
    b_store,
    b_offsets,
    b_strides,
    ranks,
    scales,
    token_slots,
    slice_offsets,
    n_total=None,
    columns=None,
) -> np.ndarray:
    """Per-token shrink + expand onto the bf16 base ``y`` (returns a new array).

    ``n_total`` is the full output width that B rows are indexed by; ``columns``
    optionally restricts the columns present in ``y`` (sampled checks).
    """
    x64 = bf16_to_f32(x_bits).astype(np.float64)
    out = np.array(y_bits, dtype=np.uint16, copy=True)
    bounds = np.asarray(slice_offsets).tolist()
    n_all = bounds[-1] if n_total is None else n_total
    width = x64.shape[1]
    slices = len(bounds) - 1
    for m, g in enumerate(np.asarray(token_slots).tolist()):
        if g < 0 or int(ranks[g]) == 0:
            continue
        r = int(ranks[g])
        a = slot_a(a_store, int(a_offsets[g]), slices * r, width)
        z = bf16_to_f32(f64_to_bf16_bits(a @ x64[m])).astype(np.float64)
        bg = slot_b(b_store, int(b_offsets[g]), int(b_strides[g]), n_all)
        full = np.empty(n_all, dtype=np.uint16)
        base_full = np.zeros(n_all, dtype=np.uint16)
        if columns is None:
            base_full[:] = out[m]
        else:
            base_full[columns] = out[m]
        for s, (start, end) in enumerate(zip(bounds, bounds[1:])):
            delta = expand_delta(z, bg, r, scales[g], start, end, s)
            full[start:end] = add_bf16(base_full[start:end], delta)
        out[m] = full if columns is None else full[columns]
    return out


def segments_to_slots(segment_lengths, segment_slots) -> np.ndarray:
    """Contiguous prefill segments -> per-token slot map."""
    return np.repeat(np.asarray(segment_slots, dtype=np.int32), np.asarray(segment_lengths))


def silu_mul(gate_bits, up_bits) -> np.ndarray:
    """``bf16(bf16(silu(gate)) * up)`` in fp32 (``qwen35_decode_silu.py:60-61``)."""
    g = bf16_to_f32(gate_bits)
    u = bf16_to_f32(up_bits)
    with np.errstate(over="ignore"):
        act = (g / (np.float32(1) + np.exp(-g, dtype=np.float32))).astype(np.float32)
        act = bf16_to_f32(bf16_bits(act))
        return bf16_bits((act * u).astype(np.float32))
