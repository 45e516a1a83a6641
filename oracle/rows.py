"""Retained-rank row shrink / RowExpand restated in numpy. TEST INFRASTRUCTURE ONLY.

Follows ``src/loraforge/ops/csrc/lora_rows.cu`` and the dense float64 oracles
of ``tests/test_row_operators_gpu.py:99-134``:

* shrink (``lora_rows.cu:35-65``): for token ``t`` with ``g = slots[t] >= 0``
  and ``r = ranks[g] > 0``, ``z[t, s*r + k] = bf16(sum_w x[t, w] * A[g, s*r + k, w])``
  for every slice ``s < S`` and ``k < r``; all other z entries are untouched.
* expand (``lora_rows.cu:67-162``): for each active segment (one slot, at
  most 16 tokens) and each output column ``n`` of slice ``s``:
  ``y[t, n] = bf16(bf16(y[t, n]) + bf16(scale[g] * sum_{k<r} z[t, s*r + k] * B_g[n, k]))``
  where ``B_g`` is ``[N, b_strides[g]]`` at element offset ``b_offsets[g]``
  of the flat store. Slot -1 and rank 0 segments are skipped.

Dot products are taken in float64 and rounded through fp32 to bf16, as the
reference tests do (``.double() ... .bfloat16()``). All arrays hold bf16 bit
patterns as ``uint16``.

Pinning (tests/test_oracle_rows.py): the two-stage rounding KAT of
``tests/test_row_operators_gpu.py:233-259``; the ``examples/row_operators.py``
KAT; a brute-force scalar loop on tiny inputs against these vectorised forms;
and a dense ``numpy.matmul`` formulation of the same contraction.
"""

from __future__ import annotations

import numpy as np

from .nf4 import bf16_to_f32, f64_to_bf16_bits

MAX_SEGMENT_ROWS = 16
MAX_RANK = 64


def row_shrink(x, a, z, slots, ranks, *, num_slices: int = 1) -> np.ndarray:
    """Return a copy of ``z`` with the live packed prefixes of ``A @ x`` written."""
    x64 = bf16_to_f32(x).astype(np.float64)
    a64 = bf16_to_f32(a).astype(np.float64)
    out = np.array(z, dtype=np.uint16, copy=True)
    for t, g in enumerate(np.asarray(slots).tolist()):
        if g < 0:
            continue
        r = int(ranks[g])
        if r == 0:
            continue
        live = num_slices * r
        out[t, :live] = f64_to_bf16_bits(a64[g, :live] @ x64[t])
    return out


def slot_b(b_store, offset: int, stride: int, rows: int) -> np.ndarray:
    """The ``[rows, stride]`` compact B region of one slot as float64."""
    flat = bf16_to_f32(np.asarray(b_store).reshape(-1)[offset : offset + rows * stride])
    return flat.astype(np.float64).reshape(rows, stride)


def expand_delta(zrow64, bg, rank: int, scale: float, start: int, end: int, s: int) -> np.ndarray:
    """bf16 bits of ``scale * B_g[start:end, :r] @ z[s*r:(s+1)*r]``."""
    value = bg[start:end, :rank] @ zrow64[s * rank : (s + 1) * rank]
    return f64_to_bf16_bits(value * float(np.float32(scale)))


def add_bf16(base_bits, delta_bits) -> np.ndarray:
    """``bf16(fp32(base) + fp32(delta))``."""
    return f64_to_bf16_bits(bf16_to_f32(base_bits).astype(np.float64) + bf16_to_f32(delta_bits))


def row_expand(
    z,
    b_store,
    y,
    *,
    b_offsets,
    b_strides,
    ranks,
    scales,
    segment_indptr,
    segment_slots,
    token_indices,
    slice_offsets,
    segment_count,
) -> np.ndarray:
    """Return a copy of ``y`` (bf16 bits ``[T, N]``) with the RowExpand deltas added."""
    out = np.array(y, dtype=np.uint16, copy=True)
    n_out = out.shape[1]
    bounds = np.asarray(slice_offsets).tolist()
    indptr = np.asarray(segment_indptr).tolist()
    zf = bf16_to_f32(z).astype(np.float64)
    count = int(np.asarray(segment_count).reshape(-1)[0])
    for seg in range(count):
        g = int(segment_slots[seg])
        if g < 0 or int(ranks[g]) == 0:
            continue
        r = int(ranks[g])
        rows = np.asarray(token_indices)[indptr[seg] : indptr[seg + 1]].tolist()
        if len(rows) > MAX_SEGMENT_ROWS or r > MAX_RANK:
            raise ValueError("segment exceeds 16 rows or rank exceeds 64")
        bg = slot_b(b_store, int(b_offsets[g]), int(b_strides[g]), n_out)
        for t in rows:
            for s, (start, end) in enumerate(zip(bounds, bounds[1:])):
                delta = expand_delta(zf[t], bg, r, scales[g], start, end, s)
                out[t, start:end] = add_bf16(out[t, start:end], delta)
    return out
