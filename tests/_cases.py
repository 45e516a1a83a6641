"""Seeded numpy case builders shared by the CPU oracle tests and the GPU parity tests.

All bf16 tensors are uint16 bit patterns. ``row_case`` restates the generator
of the reference's row-operator tests (``tests/test_row_operators_gpu.py:40-96``:
ranks 1/2/3/7/16/17/33/64/0 in a capacity-128 pool, segments of 1..16 rows, an
empty segment, an unused trailing segment, a column view of a wider output).
``fused_case`` builds the NF4 + multi-LoRA configurations of BASELINE.json.
"""

from __future__ import annotations

import numpy as np

from oracle import nf4 as onf4

RANKS = [1, 2, 3, 7, 16, 17, 33, 64, 0]
SIZES = [1, 2, 3, 4, 8, 16, 15, 16, 3, 2]
SCALES = [1, -0.7, 0.5, 1.25, 2, 0, 0.3, -1, 1]


def bf16(values) -> np.ndarray:
    return onf4.bf16_bits(np.asarray(values, dtype=np.float32))


def bucket_of(k: int) -> int:
    return 1 << (max(1, k) - 1).bit_length()


def row_case(slices=1, width=520, columns=None, seed=31):
    rng = np.random.default_rng(seed)
    m, capacity = sum(SIZES), 128
    widths = [19, 13, 11][:slices] if columns is None else [columns] * slices
    n = sum(widths)
    x_full = bf16(rng.standard_normal((m, width + 8)) * 0.1)
    a = bf16(rng.standard_normal((len(RANKS), slices * capacity, width)) * 0.1)
    z = np.full((m, slices * capacity), bf16(3.0), dtype=np.uint16)
    storage = bf16(rng.standard_normal((m, n + 6)) * 0.1)
    perm = rng.permutation(m)
    starts, seg_slots = [0], []
    routes = [-1] * m
    for slot, size in enumerate(SIZES):
        actual = slot if slot < len(RANKS) else -1
        seg_slots.append(actual)
        for t in perm[starts[-1] : starts[-1] + size]:
            routes[int(t)] = actual
        starts.append(starts[-1] + size)
    seg_slots += [0, -1]  # an empty active segment and an unused capacity entry
    starts += [m, m]
    pieces, offsets, buckets, cursor = [], [], [], 0
    for rank in RANKS:
        pad = (-cursor) % 8
        pieces.append(np.zeros(pad, np.uint16))
        cursor += pad
        bucket = bucket_of(rank)
        b = bf16(rng.standard_normal((n, bucket)) * 0.1)
        b[:, rank:] = 0
        offsets.append(cursor)
        buckets.append(bucket)
        pieces.append(b.reshape(-1))
        cursor += b.size
    bounds = [0]
    for w in widths:
        bounds.append(bounds[-1] + w)
    meta = dict(
        b_offsets=np.array(offsets, np.int64),
        b_strides=np.array(buckets, np.int32),
        ranks=np.array(RANKS, np.int32),
        scales=np.array(SCALES, np.float32),
        segment_indptr=np.array(starts, np.int32),
        segment_slots=np.array(seg_slots, np.int32),
        token_indices=perm.astype(np.int32),
        slice_offsets=np.array(bounds, np.int32),
        segment_count=np.array([len(seg_slots) - 1], np.int32),
    )
    return dict(
        x_full=x_full,
        x=x_full[:, :width],
        a=a,
        z=z,
        b=np.concatenate(pieces),
        storage=storage,
        out_cols=(3, 3 + n),
        routes=np.array(routes, np.int32),
        meta=meta,
        slices=slices,
    )


def lora_tables(rng, k, n, ranks, slices=1, bounds=None, alpha_over_r=2.0, std=0.02):
    """Ragged A/B stores for adapters of the given ranks (A packed at s*r)."""
    bounds = bounds or [0, n]
    a_parts, b_parts, a_off, b_off, strides = [], [], [], [], []
    a_cur = b_cur = 0
    for r in ranks:
        a_off.append(a_cur)
        rows = slices * r
        a = bf16(rng.standard_normal((rows, k)) * std) if rows else np.zeros((0, k), np.uint16)
        a_parts.append(a.reshape(-1))
        a_cur += a.size
        pad = (-a_cur) % 8
        a_parts.append(np.zeros(pad, np.uint16))
        a_cur += pad
        bucket = bucket_of(r)
        b = bf16(rng.standard_normal((n, bucket)) * std)
        b[:, r:] = 0
        b_off.append(b_cur)
        strides.append(bucket)
        b_parts.append(b.reshape(-1))
        b_cur += b.size
        pad = (-b_cur) % 8
        b_parts.append(np.zeros(pad, np.uint16))
        b_cur += pad
    return dict(
        a_store=np.concatenate(a_parts) if a_parts else np.zeros(8, np.uint16),
        a_offsets=np.array(a_off, np.int64),
        b_store=np.concatenate(b_parts),
        b_offsets=np.array(b_off, np.int64),
        b_strides=np.array(strides, np.int32),
        ranks=np.array(ranks, np.int32),
        scales=np.full(len(ranks), alpha_over_r, np.float32),
        slice_offsets=np.array(bounds, np.int32),
    )


def torch_quantized_state(n, k, *, double_quant=False, seed=0, w_std=0.02) -> dict:
    """NF4 state dict of a seeded ``N(0, w_std)`` bf16 weight, quantised with PyTorch on the CPU.

    Input generation only (the full-size configs hold up to 100M weights,
    which the numpy quantiser takes tens of seconds for): the packed bytes and
    scales it returns are what the oracle dequantises, so parity does not
    depend on how they were chosen.
    """
    import torch

    from loraforge_amd.ops.nf4 import quantize_nf4

    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n, k, generator=g) * w_std).bfloat16()
    q, st = quantize_nf4(w, compress_statistics=double_quant)
    state = {
        "qweight": q.reshape(-1).numpy().copy(),
        "shape": (n, k),
        "blocksize": 64,
        "code": st.code.numpy().copy(),
    }
    if double_quant:
        absmax_q = st.absmax.numpy().copy()
        absmax2 = st.state2.absmax.numpy().copy()
        code2 = st.state2.code.numpy().copy()
        offset = np.float32(st.offset.item())
        state.update(
            absmax_q=absmax_q,
            absmax2=absmax2,
            code2=code2,
            offset=offset,
            dq_block=256,
            scales=onf4.dq_scales(absmax_q, absmax2, code2, offset, dq_block=256),
        )
    else:
        state.update(absmax=st.absmax.numpy().copy(), scales=st.absmax.numpy().copy())
    return state


def fused_case(
    m,
    n,
    k,
    *,
    ranks=(16,) * 32,
    slices=1,
    bounds=None,
    double_quant=False,
    null_frac=0.1,
    bias=False,
    seed=731,
    token_slots=None,
    w_std=0.02,
    state=None,
):
    rng = np.random.default_rng(seed)
    x = bf16(rng.standard_normal((m, k)))
    if state is None:
        w = onf4.bf16_to_f32(bf16(rng.standard_normal((n, k)) * w_std))
        state = onf4.quantize(w, double_quant=double_quant)
    lora = lora_tables(rng, k, n, list(ranks), slices=slices, bounds=bounds)
    if token_slots is None:
        token_slots = rng.integers(0, len(ranks), m).astype(np.int32)
        token_slots[rng.random(m) < null_frac] = -1
    lora["token_slots"] = np.asarray(token_slots, np.int32)
    return dict(x=x, state=state, lora=lora, bias=bf16(rng.standard_normal(n) * 0.5) if bias else None, m=m, n=n, k=k)


def fused_expected(case, rows=None):
    """Oracle output of ``fused_case`` (optionally only output columns ``rows``)."""
    from oracle import linear

    st = case["state"]
    w_bits = case.get("w_bits")
    if w_bits is None:
        w_bits = onf4.dequantize(st["qweight"], st["scales"], st["shape"])
    y = linear.nf4_linear(case["x"], w_bits, case["bias"], rows=rows)
    lora = case["lora"]
    return linear.lora_apply(
        case["x"],
        y,
        a_store=lora["a_store"],
        a_offsets=lora["a_offsets"],
        b_store=lora["b_store"],
        b_offsets=lora["b_offsets"],
        b_strides=lora["b_strides"],
        ranks=lora["ranks"],
        scales=lora["scales"],
        token_slots=lora["token_slots"],
        slice_offsets=lora["slice_offsets"],
        n_total=case["n"],
        columns=rows,
    )


def segments_of(routes, max_rows=16):
    """Group tokens by slot into segments of at most ``max_rows`` tokens (the
    reference row_expand's segment contract, ``ops/lora_rows.py:112-239``).
    Returns (segment_indptr, segment_slots, token_indices); base-only tokens
    are left out."""
    routes = np.asarray(routes)
    indptr, seg_slots, order = [0], [], []
    for g in sorted(set(routes.tolist()) - {-1}):
        tokens = np.nonzero(routes == g)[0].tolist()
        for i in range(0, len(tokens), max_rows):
            chunk = tokens[i : i + max_rows]
            order += chunk
            seg_slots.append(g)
            indptr.append(indptr[-1] + len(chunk))
    return np.array(indptr, np.int32), np.array(seg_slots, np.int32), np.array(order, np.int32)


def c2_case(seed=733, tokens=64, k=4096, n=4096, adapters=32, rank=16, null_frac=0.1, scale=2.0):
    """BASELINE c2: BF16 multi-LoRA shrink/expand with no quantised base.

    x bf16 [64, 4096] ~N(0,1); A [32, 16, 4096] and compact B [32][4096, 16]
    ~N(0, 0.02); per-token slot uniform in [0, 32) with 10 % set to -1;
    y (the base output) bf16 ~N(0, 1); ``y += 2.0 * B[idx] (A[idx] x)``.
    """
    rng = np.random.default_rng(seed)
    x = bf16(rng.standard_normal((tokens, k)))
    a = bf16(rng.standard_normal((adapters, rank, k)) * 0.02)
    b = bf16(rng.standard_normal((adapters, n, rank)) * 0.02)
    y = bf16(rng.standard_normal((tokens, n)))
    routes = rng.integers(0, adapters, tokens).astype(np.int32)
    routes[rng.random(tokens) < null_frac] = -1
    indptr, seg_slots, order = segments_of(routes)
    meta = dict(
        b_offsets=np.arange(adapters, dtype=np.int64) * (n * rank),
        b_strides=np.full(adapters, rank, np.int32),
        ranks=np.full(adapters, rank, np.int32),
        scales=np.full(adapters, scale, np.float32),
        segment_indptr=indptr,
        segment_slots=seg_slots,
        token_indices=order,
        slice_offsets=np.array([0, n], np.int32),
        segment_count=np.array([len(seg_slots)], np.int32),
    )
    return dict(x=x, a=a, b=b.reshape(-1), y=y, z=np.zeros((tokens, rank), np.uint16), routes=routes, meta=meta)


def zipf_routes(rng, m, adapters, s=1.1):
    p = 1.0 / np.arange(1, adapters + 1) ** s
    return rng.choice(adapters, size=m, p=p / p.sum()).astype(np.int32)
