"""Fused NF4 + multi-LoRA linear on gfx950 against the oracle chain.

Tolerance: bf16 outputs within max abs/rel 2e-2 of
the reference chain on the same seeded inputs; additionally relative L2
< 0.005 (the reference row-operator gate). Covers decode batch sizes 1..64
(both kernel shapes), plain and double-quantised scales, bias, 3 slices,
mixed ranks 0..64, all-base batches, counters left at zero, repeated calls,
graph replay, and the prefill GEMM with segmented adapters.
"""

import dataclasses

import numpy as np
import pytest
import torch

from loraforge_amd.ops import LoraBatch, nf4_lora_linear
from loraforge_amd.ops.fused import decode_status
from loraforge_amd.ops.nf4 import NF4State, NestedState
from oracle import nf4 as onf4
from tests import _cases

pytestmark = pytest.mark.gpu


def t16(bits, device):
    return torch.from_numpy(np.ascontiguousarray(bits)).view(torch.bfloat16).to(device)


def bits(t):
    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def close(actual_bits, expected_bits):
    a = onf4.bf16_to_f32(actual_bits).astype(np.float64)
    e = onf4.bf16_to_f32(expected_bits).astype(np.float64)
    rel = np.linalg.norm(a - e) / max(np.linalg.norm(e), 1e-30)
    assert rel < 0.005, rel
    np.testing.assert_allclose(a, e, rtol=2e-2, atol=2e-2)


def to_device(case, device):
    st = case["state"]
    code = torch.from_numpy(st["code"]).to(device)
    q = torch.from_numpy(st["qweight"]).to(device)
    if "absmax_q" in st:
        state = NF4State(
            torch.from_numpy(st["absmax_q"]).to(device),
            torch.Size(st["shape"]),
            code,
            torch.bfloat16,
            offset=torch.tensor(st["offset"], dtype=torch.float32, device=device),
            state2=NestedState(torch.from_numpy(st["absmax2"]).to(device), torch.from_numpy(st["code2"]).to(device), 256),
        )
    else:
        state = NF4State(torch.from_numpy(st["absmax"]).to(device), torch.Size(st["shape"]), code, torch.bfloat16)
    lo = case["lora"]
    lora = LoraBatch(
        t16(lo["a_store"], device),
        torch.from_numpy(lo["a_offsets"]).to(device),
        t16(lo["b_store"], device),
        torch.from_numpy(lo["b_offsets"]).to(device),
        torch.from_numpy(lo["b_strides"]).to(device),
        torch.from_numpy(lo["ranks"]).to(device),
        torch.from_numpy(lo["scales"]).to(device),
        torch.from_numpy(lo["token_slots"]).to(device),
        torch.from_numpy(lo["slice_offsets"]).to(device),
        max_rank=int(max(1, lo["ranks"].max())),
    )
    bias = t16(case["bias"], device) if case["bias"] is not None else None
    return t16(case["x"], device), q, state, lora, bias


def workspace_clean(device):
    assert decode_status(device=device) == 0


@pytest.mark.parametrize("m", [1, 7, 16, 17, 40, 64])
@pytest.mark.parametrize("dq", [False, True])
def test_decode_exact_weights(m, dq, device):
    """exact=True multiplies the reference's bf16(code * scale) weights."""
    case = _cases.fused_case(m, 512, 1024, ranks=(16,) * 8, double_quant=dq, seed=200 + m)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora, exact=True)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)


def test_decode_half_chunk_k(device):
    """K % 128 == 64: the last chunk holds a single NF4 block."""
    for m in (3, 20):
        for exact in (False, True):
            case = _cases.fused_case(m, 256, 320, ranks=(8, 4), double_quant=bool(m % 2), seed=m)
            x, q, st, lora, _ = to_device(case, device)
            y = nf4_lora_linear(x, q, st, lora=lora, exact=exact)
            torch.cuda.synchronize()
            close(bits(y), _cases.fused_expected(case))


@pytest.mark.parametrize("m", [1, 2, 5, 16, 17, 33, 48, 64])
@pytest.mark.parametrize("dq", [False, True])
def test_decode_batches(m, dq, device):
    case = _cases.fused_case(m, 512, 1024, ranks=(16,) * 8, double_quant=dq, seed=100 + m)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)


@pytest.mark.parametrize("m", [3, 5, 8])
def test_decode_small_batches_on_wide_rows(m, device):
    """3..8 tokens at N >= 8192 run the wide kernel (one token tile, 32-row groups):
    with LoRA (slices, bias, base-only tokens) and without, against the oracle."""
    case = _cases.fused_case(m, 8192, 1024, ranks=(0, 8, 16, 32), slices=2, bounds=[0, 4096, 8192], bias=True,
                             seed=500 + m, null_frac=0.3)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)
    base = nf4_lora_linear(x, q, st, bias=bias)
    torch.cuda.synchronize()
    close(bits(base), _cases.fused_expected(dict(case, lora=dict(case["lora"], token_slots=np.full(m, -1, np.int32)))))


@pytest.mark.parametrize("m", [9, 12, 16, 17, 24, 32])
def test_decode_narrow_tiles_where_wide_declines(m, device):
    """9..32 tokens run the wide kernel where it takes the shape. With LoRA it needs N a
    multiple of 256, so N = 448 keeps these batches on the narrow kernel's 16- and 32-token
    tiles; without LoRA at K = 12288 the narrow kernel keeps 9..16 tokens (the wide one
    takes 17..32)."""
    ranks = (0, 4, 16, 33)
    case = _cases.fused_case(m, 448, 1024, ranks=ranks, slices=2, bounds=[0, 192, 448], bias=True,
                             double_quant=bool(m % 2), seed=300 + m)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)
    case = _cases.fused_case(m, 192, 12288, ranks=(1,), seed=400 + m, token_slots=[-1] * m)
    x, q, st, _, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))


def test_decode_mixed_ranks_slices_bias(device):
    ranks = (0, 1, 3, 8, 16, 17, 33, 64)
    bounds = [0, 320, 448, 512]
    case = _cases.fused_case(24, 512, 768, ranks=ranks, slices=3, bounds=bounds, bias=True, seed=7, null_frac=0.2)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    case1 = _cases.fused_case(7, 512, 768, ranks=ranks, slices=3, bounds=bounds, bias=True, seed=8, null_frac=0.2)
    x, q, st, lora, bias = to_device(case1, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case1))


def test_decode_base_only_and_all_null_routes(device):
    case = _cases.fused_case(9, 256, 512, ranks=(8, 8), seed=3, token_slots=[-1] * 9)
    x, q, st, lora, _ = to_device(case, device)
    base = nf4_lora_linear(x, q, st)
    routed = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    assert torch.equal(base, routed)
    close(bits(base), _cases.fused_expected(case))


@pytest.mark.parametrize("m", [8, 20, 64])
def test_decode_repeated_calls_and_graph_replay(m, device):
    """Repeated calls on one workspace and graph replays give the eager bits: the narrow
    kernel (8 tokens) and the wide one (one token tile at 20, two at 64)."""
    case = _cases.fused_case(m, 1024, 1024, ranks=(16,) * 4, seed=11 + m)
    x, q, st, lora, _ = to_device(case, device)
    expect = _cases.fused_expected(case)
    out = torch.empty(m, 1024, dtype=torch.bfloat16, device=device)
    for _ in range(5):
        nf4_lora_linear(x, q, st, lora=lora, out=out)
    torch.cuda.synchronize()
    close(bits(out), expect)
    eager = out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, st, lora=lora, out=out)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, st, lora=lora, out=out)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    workspace_clean(device)


@pytest.mark.parametrize("m", [1, 64])
def test_north_star_shape(m, device):
    case = _cases.fused_case(m, 4096, 4096, ranks=(16,) * 32, seed=731)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)


@pytest.mark.parametrize("m", [65, 200, 256, 520])
@pytest.mark.parametrize("dq", [False, True])
def test_prefill_segments(m, dq, device):
    rng = np.random.default_rng(m)
    cuts = np.sort(rng.choice(np.arange(1, m), 3, replace=False))
    lengths = np.diff(np.concatenate([[0], cuts, [m]]))
    seg_slots = [0, 2, -1, 1]
    slots = np.repeat(np.array(seg_slots, np.int32), lengths)
    case = _cases.fused_case(m, 384, 512, ranks=(32, 4, 16), double_quant=dq, seed=m, token_slots=slots, bias=True)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora, plan="prefill")
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)


@pytest.mark.parametrize("k", [64, 192, 320])
@pytest.mark.parametrize("dq", [False, True])
def test_prefill_short_and_odd_k(k, dq, device):
    """One, three and five k-steps (the pipeline's requests past the end), ragged N and M."""
    m = 300
    slots = np.repeat(np.array([0, 1, -1], np.int32), [100, 150, 50])
    case = _cases.fused_case(m, 320, k, ranks=(8, 32), double_quant=dq, seed=k + dq, token_slots=slots)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora, plan="prefill")
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))


@pytest.mark.parametrize("dq", [False, True])
def test_prefill_exact_weights(dq, device):
    """exact=True hands the nested state to the launch, which rebuilds the fp32 scales in its workspace."""
    m = 200
    slots = np.repeat(np.array([1, -1, 0], np.int32), [90, 30, 80])
    case = _cases.fused_case(m, 384, 512, ranks=(16, 8), double_quant=dq, seed=77, token_slots=slots, bias=True)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora, exact=True, plan="prefill")
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))


def test_prefill_slices_and_interleaved_routes(device):
    ranks = (8, 64, 0, 17)
    case = _cases.fused_case(300, 512, 256, ranks=ranks, slices=3, bounds=[0, 200, 448, 512], seed=5, null_frac=0.1)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora, plan="prefill")
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))


@pytest.mark.parametrize("offset", [8, 4, 1])
def test_prefill_strided_output(offset, device):
    """Output rows 16-, 8- and 2-byte aligned (column views of a wider tensor): all three store paths."""
    m, n = 300, 384
    slots = np.repeat(np.array([1, -1, 0], np.int32), [120, 30, 150])
    case = _cases.fused_case(m, n, 256, ranks=(16, 8), seed=90 + offset, token_slots=slots, bias=True)
    x, q, st, lora, bias = to_device(case, device)
    big = torch.full((m, n + 24), -7.0, dtype=torch.bfloat16, device=device)
    out = big[:, offset : offset + n]
    nf4_lora_linear(x, q, st, bias=bias, lora=lora, out=out, plan="prefill")
    torch.cuda.synchronize()
    close(bits(out), _cases.fused_expected(case))
    # Nothing outside the view was written.
    assert torch.all(big[:, :offset] == -7.0) and torch.all(big[:, offset + n :] == -7.0)


def test_prefill_repeated_calls_and_graph_replay(device):
    """The in-launch z producers publish per call (call-epoch tags): eager repeats and graph replays agree."""
    m = 600  # three token tiles, the last one ragged
    slots = np.repeat(np.array([2, 0, -1, 1, 0], np.int32), [150, 130, 40, 200, 80])
    case = _cases.fused_case(m, 448, 512, ranks=(16, 32, 8), seed=41, token_slots=slots)
    x, q, st, lora, _ = to_device(case, device)
    expect = _cases.fused_expected(case)
    out = torch.empty(m, 448, dtype=torch.bfloat16, device=device)
    for _ in range(3):
        nf4_lora_linear(x, q, st, lora=lora, out=out, plan="prefill")
    torch.cuda.synchronize()
    close(bits(out), expect)
    eager = out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, st, lora=lora, out=out, plan="prefill")
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, st, lora=lora, out=out, plan="prefill")
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_prefill_c5_shape_sampled(device):
    m, n, k = 2048, 11008, 4096
    rng = np.random.default_rng(735)
    cuts = np.sort(rng.choice(np.arange(1, m), 7, replace=False))
    lengths = np.diff(np.concatenate([[0], cuts, [m]]))
    slots = np.repeat(np.arange(8, dtype=np.int32), lengths)
    case = _cases.fused_case(m, n, k, ranks=(32,) * 8, double_quant=True, seed=735, token_slots=slots)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    tokens = np.unique(np.concatenate([rng.choice(m, 24, replace=False), np.cumsum(lengths)[:-1], [0, m - 1]]))
    cols = np.unique(np.concatenate([rng.choice(n, 48, replace=False), [0, n - 1, 128, 127]]))
    sub = dict(case, x=case["x"][tokens], m=len(tokens))
    sub["lora"] = dict(case["lora"], token_slots=case["lora"]["token_slots"][tokens])
    expect = _cases.fused_expected(sub, rows=cols)
    close(bits(y)[np.ix_(tokens, cols)], expect)


def _torch_chain(x, w, lora, n):
    """The fused linear's rounding chain in PyTorch fp32 on the GPU (no bias):
    bf16(x W^T), z = bf16(x A_g^T), bf16(bf16(y) + bf16(scale_g z B_g^T)) per routed token."""
    y = (x.float() @ w.float().t()).bfloat16().float()
    slots = lora.token_slots.cpu().numpy()
    ranks = lora.ranks.cpu().numpy()
    a_off = lora.a_offsets.cpu().numpy()
    b_off = lora.b_offsets.cpu().numpy()
    strides = lora.b_strides.cpu().numpy()
    scales = lora.scales.cpu().numpy()
    k = x.shape[1]
    for g in np.unique(slots[slots >= 0]):
        r = int(ranks[g])
        if r == 0:
            continue
        rows = torch.from_numpy(np.nonzero(slots == g)[0]).to(x.device)
        a = lora.a_store[int(a_off[g]) : int(a_off[g]) + r * k].view(r, k).float()
        b = lora.b_store[int(b_off[g]) : int(b_off[g]) + n * int(strides[g])].view(n, int(strides[g]))[:, :r].float()
        z = (x[rows].float() @ a.t()).bfloat16().float()
        delta = ((z @ b.t()) * float(scales[g])).bfloat16().float()
        y[rows] = (y[rows] + delta).bfloat16().float()
    return y.bfloat16()


def test_prefill_c5_full_output_against_torch_fp32(device):
    """Every element of the c5 output (2048 x 11008: both dispatch rounds of the 464 tiles, every
    tile edge, the 8 segment boundaries) against the same rounding chain in PyTorch fp32 on the
    GPU over the bit-exact dequantised weight (lf_nf4_dequant_dq, pinned by the oracle), at the
    oracle tests' gate."""
    from loraforge_amd.ops import dequantize_nf4_nested

    m, n, k = 2048, 11008, 4096
    rng = np.random.default_rng(736)
    cuts = np.sort(rng.choice(np.arange(1, m), 7, replace=False))
    lengths = np.diff(np.concatenate([[0], cuts, [m]]))
    slots = np.repeat(np.arange(8, dtype=np.int32), lengths)
    case = _cases.fused_case(m, n, k, ranks=(32,) * 8, double_quant=True, seed=736, token_slots=slots)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    w = dequantize_nf4_nested(q, st)
    want = _torch_chain(x, w, lora, n)
    torch.cuda.synchronize()
    close(bits(y), bits(want))


def test_decode_after_prefill_on_one_workspace(device):
    """Prefill and decode calls share one workspace: one call epoch, z rows clear of the header."""
    ws = torch.zeros(1 << 22, dtype=torch.uint8, device=device)
    pre = _cases.fused_case(96, 1024, 1024, ranks=(64, 16, 8), seed=21)
    dec = _cases.fused_case(64, 1024, 1024, ranks=(64, 16, 8, 32), seed=22)
    xp, qp, sp, lp, _ = to_device(pre, device)
    xd, qd, sd, ld, _ = to_device(dec, device)
    for call in range(1, 3):
        yp = nf4_lora_linear(xp, qp, sp, lora=lp, workspace=ws, plan="prefill")
        yd = nf4_lora_linear(xd, qd, sd, lora=ld, workspace=ws)
        torch.cuda.synchronize()
        close(bits(yp), _cases.fused_expected(pre))
        close(bits(yd), _cases.fused_expected(dec))
        assert decode_status(workspace=ws) == 0
        # Control header: the epoch moved on once per LoRA call (prefill and decode); the arrival
        # counts are back to zero.
        head = ws[:2048].view(torch.int32)
        assert int(head[0]) == 2 * call
        assert not head[32:512].any()


@pytest.mark.parametrize("dq", [False, True])
def test_weights_loaded_from_quant_state_file(tmp_path, dq, device):
    """NF4 weights stored as packed QuantState entries feed the fused call unchanged."""
    from loraforge_amd.ops.quant_state import load_nf4_weight, save_nf4_weights

    case = _cases.fused_case(8, 256, 512, ranks=(16, 8), double_quant=dq, seed=41)
    x, q, st, lora, _ = to_device(case, device)
    path = tmp_path / "w.safetensors"
    save_nf4_weights(path, {"proj.weight": (q, st)})
    lq, lst = load_nf4_weight(path, "proj.weight", device=device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    y_loaded = nf4_lora_linear(x, lq, lst, lora=lora)
    torch.cuda.synchronize()
    assert torch.equal(y, y_loaded)
    close(bits(y_loaded), _cases.fused_expected(case))


def test_empty_batch_and_smallest_shapes(device):
    """Zero tokens launch nothing; K = N = 64 (one NF4 block per row) works on both paths."""
    case = _cases.fused_case(4, 64, 64, ranks=(16, 64), seed=51, null_frac=0.0)
    x, q, st, lora, _ = to_device(case, device)
    empty = nf4_lora_linear(x[:0], q, st)
    assert empty.shape == (0, 64)
    for m in (1, 4):
        sub = dict(case, x=case["x"][:m], m=m)
        sub["lora"] = dict(case["lora"], token_slots=case["lora"]["token_slots"][:m])
        xs, _, _, lora_m, _ = to_device(sub, device)
        y = nf4_lora_linear(xs, q, st, lora=lora_m)
        torch.cuda.synchronize()
        close(bits(y), _cases.fused_expected(sub))
    big = _cases.fused_case(96, 64, 64, ranks=(16, 64), seed=52)
    x, q, st, lora, _ = to_device(big, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(big))


def test_workspace_grown_after_capture_keeps_the_captured_buffer(device):
    """A larger eager call on a stream after a capture replaces the cached workspace; the
    graph keeps writing into the buffer it captured, which must stay allocated."""
    from loraforge_amd.ops import fused

    dec = _cases.fused_case(8, 1024, 1024, ranks=(16,) * 4, seed=61)
    x, q, st, lora, _ = to_device(dec, device)
    expect = _cases.fused_expected(dec)
    big = _cases.fused_case(96, 4096, 4096, ranks=(16, 8), double_quant=True, seed=62)
    xb, qb, sb, lb, _ = to_device(big, device)
    out = torch.empty(8, 1024, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, st, lora=lora, out=out)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, st, lora=lora, out=out)
        captured = fused._WORKSPACES[(device.index, stream.cuda_stream)]
        retired = len(fused._RETIRED)
        # exact=True hands the nested state to the prefill launch, whose workspace then holds
        # the rebuilt scales: more than the buffer the capture used.
        yb = nf4_lora_linear(xb, qb, sb, lora=lb, exact=True)
    torch.cuda.synchronize()
    assert fused._WORKSPACES[(device.index, stream.cuda_stream)].data_ptr() != captured.data_ptr()
    assert len(fused._RETIRED) == retired + 1 and fused._RETIRED[-1].data_ptr() == captured.data_ptr()
    ref_big = yb.clone()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
            yb2 = nf4_lora_linear(xb, qb, sb, lora=lb, exact=True)
        torch.cuda.synchronize()
        close(bits(out), expect)
        assert torch.equal(yb2, ref_big)


def test_prepared_scales_follow_in_place_weight_updates(device):
    """The cached fp32 scales of a double-quant state are keyed on the tensors' versions
    (reference integrations/_sglang_nf4_linear.py:44-57): an in-place reload is seen."""
    first = _cases.fused_case(8, 512, 1024, ranks=(16,) * 4, double_quant=True, seed=71)
    second = _cases.fused_case(8, 512, 1024, ranks=(16,) * 4, double_quant=True, seed=71, w_std=0.05)
    x, q, st, lora, _ = to_device(first, device)
    y1 = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y1), _cases.fused_expected(first))
    s2 = second["state"]
    q.copy_(torch.from_numpy(s2["qweight"]))
    st.absmax.copy_(torch.from_numpy(s2["absmax_q"]))
    st.state2.absmax.copy_(torch.from_numpy(s2["absmax2"]))
    st.offset.copy_(torch.tensor(s2["offset"], dtype=torch.float32))
    y2 = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y2), _cases.fused_expected(second))
    # Only the absmax codes change: the key still moves and the output follows.
    st.absmax.copy_(torch.from_numpy(first["state"]["absmax_q"]))
    y3 = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    mixed = dict(second, state=dict(second["state"], absmax_q=first["state"]["absmax_q"]))
    mixed["state"]["scales"] = _dq_scales(mixed["state"])
    close(bits(y3), _cases.fused_expected(mixed))


def _dq_scales(st):
    return onf4.dq_scales(st["absmax_q"], st["absmax2"], st["code2"], st["offset"], dq_block=256)


@pytest.mark.parametrize("m", [65, 130, 256, 300])
@pytest.mark.parametrize("plan", [None, "decode", "prefill"])
def test_plans_above_64_tokens(m, plan, device):
    """Above 64 tokens both plans (decode over 64-token chunks, one prefill launch) match the oracle."""
    case = _cases.fused_case(m, 1024, 1024, ranks=(16, 8, 32, 64, 4), seed=500 + m, bias=True)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora, plan=plan)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    if plan == "decode":
        # Each chunk is exactly the decode call on its rows.
        for t0 in range(0, m, 64):
            rows = slice(t0, min(m, t0 + 64))
            part = dataclasses.replace(lora, token_slots=lora.token_slots[rows])
            yc = nf4_lora_linear(x[rows], q, st, bias=bias, lora=part)
            assert torch.equal(yc, y[rows])
    workspace_clean(device)


def test_chunked_decode_graph_replay_and_strided_rows(device):
    """The chunked plan's launches replay in a graph; strided x/y rows (views of wider tensors) are honoured."""
    m, n, k = 200, 512, 1024
    case = _cases.fused_case(m, n, k, ranks=(16, 32, 8), seed=61)
    _, q, st, lora, _ = to_device(case, device)
    xw = torch.zeros(m, k + 64, dtype=torch.bfloat16, device=device)
    xw[:, :k] = t16(case["x"], device)
    x = xw[:, :k]
    big = torch.full((m, n + 40), -3.0, dtype=torch.bfloat16, device=device)
    out = big[:, 8 : 8 + n]
    expect = _cases.fused_expected(case)
    nf4_lora_linear(x, q, st, lora=lora, out=out, plan="decode")
    torch.cuda.synchronize()
    close(bits(out), expect)
    eager = out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, st, lora=lora, out=out, plan="decode")  # the stream's workspace exists before capture
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, st, lora=lora, out=out, plan="decode")
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
    assert torch.all(big[:, :8] == -3.0) and torch.all(big[:, 8 + n :] == -3.0)
