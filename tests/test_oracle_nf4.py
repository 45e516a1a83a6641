"""Pin the NF4 oracle (CPU) against the reference's literals and closed forms.

Each check is chosen so a plausible restatement mistake fails it: a wrong
codebook entry, swapped nibble order, truncation instead of round-to-nearest-
even, a block index off by a factor, or a fused multiply-add in the
double-quant reconstruction.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import nf4 as o

GOLDEN = Path(__file__).parent / "golden"


def test_codebook_matches_reference_literals():
    ref = json.loads((GOLDEN / "nf4_codebook.json").read_text())["code"]
    assert np.array_equal(o.NF4_CODE, np.array(ref, dtype=np.float32))
    from loraforge_amd.ops.nf4 import NF4_CODE

    assert np.array_equal(np.array(NF4_CODE, dtype=np.float32), o.NF4_CODE)
    assert o.NF4_CODE[7] == 0 and o.NF4_CODE[0] == -1 and o.NF4_CODE[15] == 1
    assert np.all(np.diff(o.NF4_CODE) > 0)


def test_bf16_rounding_matches_torch_including_specials():
    rng = np.random.default_rng(3)
    vals = np.concatenate(
        [
            rng.standard_normal(4096).astype(np.float32) * 10.0 ** rng.integers(-40, 38, 4096),
            np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1e-45, 1.00390625, 1.01171875], np.float32),
        ]
    ).astype(np.float32)
    ours = o.bf16_bits(vals)
    theirs = torch.from_numpy(vals).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    finite = np.isfinite(vals)
    assert np.array_equal(ours[finite], theirs[finite])
    assert np.array_equal(ours[np.isinf(vals)], theirs[np.isinf(vals)])
    nan_bits = ours[np.isnan(vals)]
    assert np.all((nan_bits & 0x7F80) == 0x7F80) and np.all(nan_bits & 0x7F)


def test_round_to_nearest_even_ties():
    # code[15] = 1 times a scale that lands exactly on a bf16 midpoint.
    q = np.array([0xFF] * 32, dtype=np.uint8)  # 64 elements of nibble 15
    w = o.dequantize(np.tile(q, 64), np.full(64, 1.00390625, np.float32), (64, 64))
    assert np.all(w == 0x3F80)  # tie between 1.0 and 1.0078125 -> even (1.0)
    w = o.dequantize(np.tile(q, 64), np.full(64, 1.01171875, np.float32), (64, 64))
    assert np.all(w == 0x3F82)  # tie between 1.0078125 and 1.015625 -> even (1.015625)


def test_nibble_order_and_special_codes():
    s = np.float32(0.0234375)  # bf16-representable absmax
    q = np.zeros(64 * 32, dtype=np.uint8)
    q[0] = 0x0F  # element 0 = code[0] (high nibble), element 1 = code[15]
    q[1] = 0x70  # element 2 = code[7] = 0, element 3 = code[0]
    q[2] = 0x77
    w = o.bf16_to_f32(o.dequantize(q, np.full(64, s, np.float32), (64, 64))).reshape(-1)
    assert w[0] == -s and w[1] == s
    assert w[2] == 0 and w[3] == -s
    assert w[4] == 0 and w[5] == 0


def test_zero_block_gives_zeros_and_block_index():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 256, 64 * 128 // 2, dtype=np.uint8)
    scales = rng.uniform(0.01, 0.1, 64 * 128 // 64).astype(np.float32)
    scales[5] = 0
    w = o.bf16_to_f32(o.dequantize(q, scales, (64, 128))).reshape(-1)
    assert np.all(w[5 * 64 : 6 * 64] == 0)
    # Every element uses the scale of its own 64-element block: |w| <= scale.
    assert np.all(np.abs(w).reshape(-1, 64) <= scales[:, None] * (1 + 2**-8))


def test_exhaustive_bytes_against_independent_torch_evaluation():
    rng = np.random.default_rng(1)
    scales = np.concatenate([rng.uniform(1e-4, 10, 60), [1.0, 0.5, 3.0e-5, 7.0]]).astype(np.float32)
    shape = (256, 64)
    q = np.resize(np.arange(256, dtype=np.uint8), shape[0] * shape[1] // 2)
    sc = np.resize(scales, shape[0] * shape[1] // 64).astype(np.float32)
    ours = o.dequantize(q, sc, shape).reshape(-1)
    # Independent: per-byte python unpacking, torch fp32 multiply, torch bf16 cast.
    code = torch.tensor(o.NF4_CODE.tolist(), dtype=torch.float32)
    nibbles = []
    for b in q.tolist():
        nibbles += [b >> 4, b & 15]
    nib = torch.tensor(nibbles)
    scale = torch.from_numpy(sc).repeat_interleave(64)
    expect = (code[nib] * scale).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, expect)


@pytest.mark.parametrize("double_quant", [False, True])
def test_quantize_round_trip(double_quant):
    rng = np.random.default_rng(731)
    w = o.bf16_to_f32(o.bf16_bits((rng.standard_normal((128, 256)) * 0.1).astype(np.float32)))
    state = o.quantize(w, double_quant=double_quant)
    dq = o.bf16_to_f32(o.dequantize(state["qweight"], state["scales"], (128, 256)))
    blocks_w = w.reshape(-1, 64)
    blocks_d = dq.reshape(-1, 64)
    absmax = np.abs(blocks_w).max(axis=1)
    gap = np.max(np.diff(o.NF4_CODE)) / 2
    err = np.abs(blocks_w - blocks_d).max(axis=1)
    if not double_quant:
        assert np.all(err <= gap * absmax * (1 + 2**-7) + 1e-12)
        # The block maximum maps to code +/-1 and is reproduced exactly.
        idx = np.abs(blocks_w).argmax(axis=1)
        assert np.array_equal(blocks_d[np.arange(len(idx)), idx], blocks_w[np.arange(len(idx)), idx])
    else:
        # Double quantisation perturbs the scale by at most the code2 spacing.
        assert np.all(err <= (gap + 0.02) * absmax + 1e-6)
        assert state["absmax_q"].dtype == np.uint8 and state["absmax2"].size == -(-state["absmax_q"].size // 256)


def test_double_quant_closed_form():
    code2 = o.dynamic_map()
    zero = int(np.flatnonzero(code2 == 0)[0])
    one = int(np.flatnonzero(code2 == 1)[0])
    absmax_q = np.array([zero] * 256 + [one] * 256 + [3] * 10, dtype=np.uint8)
    absmax2 = np.array([0.5, 2.0, 0.125], dtype=np.float32)
    offset = np.float32(0.0371)
    s = o.dq_scales(absmax_q, absmax2, code2, offset)
    assert np.all(s[:256] == offset)  # code2 = 0 -> the offset, exactly
    assert np.all(s[256:512] == np.float32(np.float32(2.0) + offset))
    # No fused multiply-add: fl32(fl32(c * a) + offset), checked with scalar fp32 steps.
    for j in range(512, 522):
        prod = np.float32(code2[absmax_q[j]]) * np.float32(absmax2[j // 256])
        assert s[j] == np.float32(np.float32(prod) + offset)


def test_dynamic_map_properties():
    m = o.dynamic_map()
    assert m.size == 256 and np.all(np.diff(m) >= 0)
    assert (m == 0).sum() == 1 and m.max() == 1.0
    assert (m > 0).sum() == 128 and (m < 0).sum() == 127
    pos = m[(m > 0) & (m < 1)]
    for i in range(7):  # 2**i means per decade 10**(i-6)
        lo, hi = 10.0 ** (i - 6) * 0.1, 10.0 ** (i - 6) * 1.0
        assert ((pos > lo * 0.999) & (pos < hi * 1.0001)).sum() == 2**i
