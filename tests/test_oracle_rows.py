"""Pin the row-operator and fused-chain oracles (CPU).

* The reference's two known-answer tests (two-stage bf16 rounding of the
  scaled delta; ``examples/row_operators.py``) run through the oracle.
* A brute-force scalar loop (written element by element, independently of
  the vectorised oracle) checks shrink/expand on the reference's mixed-rank,
  multi-slice, segmented generator.
* The fused per-token chain equals shrink + expand with one-token segments,
  and its base part equals torch's ``F.linear`` on the dequantised weight.
"""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import linear, nf4 as onf4, rows
from tests import _cases

KAT = json.loads((Path(__file__).parent / "golden" / "kat_rows.json").read_text())


def _meta(d):
    keys = ("b_offsets", "b_strides", "ranks", "scales", "segment_indptr", "segment_slots", "token_indices", "slice_offsets", "segment_count")
    dtypes = dict(b_offsets=np.int64, scales=np.float32)
    return {key: np.array(d[key], dtypes.get(key, np.int32)) for key in keys}


def test_kat_scaled_delta_rounding():
    k = KAT["scaled_delta_rounding"]
    y = rows.row_expand(_cases.bf16(k["z"]), _cases.bf16(k["b"]), _cases.bf16(k["y"]), **_meta(k))
    assert onf4.bf16_to_f32(y).item() == k["expected_y"][0][0]
    single = onf4.bf16_to_f32(_cases.bf16([k["scales"][0] + k["y"][0][0]])).item()
    assert single == k["single_rounding_would_give"] != k["expected_y"][0][0]


def test_kat_example_row_operators():
    k = KAT["example_row_operators"]
    z = rows.row_shrink(_cases.bf16(k["x"]), _cases.bf16(k["a"]), _cases.bf16(k["z"]), np.array(k["slots"], np.int32), np.array(k["ranks"], np.int32))
    assert onf4.bf16_to_f32(z).tolist() == [[8, 8], [0, 0], [8, 8]]
    y = rows.row_expand(z, _cases.bf16(k["b"]), _cases.bf16(k["y"]), **_meta(k))
    assert onf4.bf16_to_f32(y).tolist() == k["expected_y"]


def _brute_shrink(x, a, z, routes, ranks, slices):
    out = z.copy()
    xf, af = onf4.bf16_to_f32(x), onf4.bf16_to_f32(a)
    for t in range(x.shape[0]):
        g = int(routes[t])
        if g < 0 or ranks[g] == 0:
            continue
        r = int(ranks[g])
        for s in range(slices):
            for kk in range(r):
                total = 0.0
                for w in range(x.shape[1]):
                    total += float(af[g, s * r + kk, w]) * float(xf[t, w])
                out[t, s * r + kk] = onf4.bf16_bits(np.float32(total))
    return out


def _brute_expand(z, b, y, meta):
    out = y.copy()
    zf, bflat = onf4.bf16_to_f32(z), onf4.bf16_to_f32(b)
    bounds = meta["slice_offsets"].tolist()
    n = out.shape[1]
    for seg in range(int(meta["segment_count"][0])):
        g = int(meta["segment_slots"][seg])
        if g < 0 or meta["ranks"][g] == 0:
            continue
        r, off, br = int(meta["ranks"][g]), int(meta["b_offsets"][g]), int(meta["b_strides"][g])
        for t in meta["token_indices"][meta["segment_indptr"][seg] : meta["segment_indptr"][seg + 1]].tolist():
            for col in range(n):
                s = sum(col >= bound for bound in bounds[1:-1])
                acc = 0.0
                for kk in range(r):
                    acc += float(zf[t, s * r + kk]) * float(bflat[off + col * br + kk])
                delta = onf4.bf16_to_f32(onf4.bf16_bits(np.float32(acc * float(meta["scales"][g]))))
                base = onf4.bf16_to_f32(out[t, col])
                out[t, col] = onf4.bf16_bits(np.float32(float(base) + float(delta)))
    return out


@pytest.mark.parametrize("slices", [1, 3])
def test_rows_oracle_against_brute_force(slices):
    c = _cases.row_case(slices=slices, width=24, seed=5)
    meta = c["meta"]
    z_or = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], meta["ranks"], num_slices=slices)
    z_bf = _brute_shrink(c["x"], c["a"], c["z"], c["routes"], meta["ranks"], slices)
    # float64 sums in different order may flip a bf16 rounding in rare ties only.
    assert np.mean(z_or != z_bf) < 1e-3
    lo, hi = c["out_cols"]
    y = c["storage"][:, lo:hi]
    y_or = rows.row_expand(z_or, c["b"], y, **meta)
    y_bf = _brute_expand(z_or, c["b"], y, meta)
    assert np.mean(y_or != y_bf) < 2e-3
    diff = np.abs(onf4.bf16_to_f32(y_or) - onf4.bf16_to_f32(y_bf))
    assert diff.max() <= 2 ** -6 * max(1.0, np.abs(onf4.bf16_to_f32(y_bf)).max())
    # Skipped routes (slot -1 and rank 0) leave output untouched.
    skipped = (c["routes"] == -1) | (c["routes"] == 8)
    assert np.array_equal(y_or[skipped], y[skipped])


def test_fused_chain_equals_rows_composition():
    case = _cases.fused_case(6, 128, 192, ranks=(3, 0, 8, 16), seed=2, null_frac=0.2, token_slots=[0, 1, 2, 3, -1, 2])
    lora = case["lora"]
    st = case["state"]
    w_bits = onf4.dequantize(st["qweight"], st["scales"], st["shape"])
    base = linear.nf4_linear(case["x"], w_bits)
    fused = _cases.fused_expected(case)
    # Same result through row_shrink + row_expand with one-token segments.
    cap = 16
    a = np.zeros((4, cap, 192), np.uint16)
    for g, r in enumerate(lora["ranks"].tolist()):
        off = int(lora["a_offsets"][g])
        a[g, :r] = lora["a_store"][off : off + r * 192].reshape(r, 192)
    z = rows.row_shrink(case["x"], a, np.zeros((6, cap), np.uint16), lora["token_slots"], lora["ranks"])
    meta = dict(
        b_offsets=lora["b_offsets"],
        b_strides=lora["b_strides"],
        ranks=lora["ranks"],
        scales=lora["scales"],
        segment_indptr=np.arange(7, dtype=np.int32),
        segment_slots=lora["token_slots"],
        token_indices=np.arange(6, dtype=np.int32),
        slice_offsets=lora["slice_offsets"],
        segment_count=np.array([6], np.int32),
    )
    composed = rows.row_expand(z, lora["b_store"], base, **meta)
    assert np.array_equal(fused, composed)


def test_base_linear_matches_torch_linear():
    case = _cases.fused_case(5, 64, 256, seed=4)
    st = case["state"]
    w_bits = onf4.dequantize(st["qweight"], st["scales"], st["shape"])
    ours = onf4.bf16_to_f32(linear.nf4_linear(case["x"], w_bits))
    x = torch.from_numpy(onf4.bf16_to_f32(case["x"])).double()
    w = torch.from_numpy(onf4.bf16_to_f32(w_bits)).double()
    ref = torch.nn.functional.linear(x, w).float().bfloat16().float().numpy()
    assert np.array_equal(ours, ref)


def test_sampled_columns_match_full_evaluation():
    case = _cases.fused_case(3, 128, 64, ranks=(4, 8), seed=9)
    full = _cases.fused_expected(case)
    cols = np.array([0, 5, 64, 127])
    assert np.array_equal(_cases.fused_expected(case, rows=cols), full[:, cols])


def test_silu_mul_against_float64():
    rng = np.random.default_rng(0)
    g = _cases.bf16(rng.standard_normal(4096) * 3)
    u = _cases.bf16(rng.standard_normal(4096))
    ours = onf4.bf16_to_f32(linear.silu_mul(g, u)).astype(np.float64)
    gf, uf = onf4.bf16_to_f32(g).astype(np.float64), onf4.bf16_to_f32(u).astype(np.float64)
    exact = gf / (1 + np.exp(-gf)) * uf
    assert np.all(np.abs(ours - exact) <= 2 ** -7 * np.abs(exact) + 1e-30)
