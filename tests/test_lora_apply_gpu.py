"""One-launch LoRA update of existing outputs (``lora_apply`` / ``lf_lora_apply``).

Oracle: ``oracle.linear.lora_apply`` -- per token, ``z = bf16(A_g x)`` and
``y = bf16(bf16(y) + bf16(scale * B_g z))`` per slice, the reference chain of
``row_shrink`` + ``row_expand`` (``ops/csrc/lora_rows.cu:35-117``). Gate:
max abs/rel 2e-2 and relative L2 < 0.005; rows of tokens without an adapter
must keep their bits.
"""

import ctypes

import numpy as np
import pytest
import torch

from loraforge_amd import _lib
from loraforge_amd.ops import LoraBatch, lora_apply
from loraforge_amd.ops.fused import _lora_struct, decode_status, workspace_bytes
from oracle import linear
from tests import _cases
from tests.test_fused_gpu import bits, close, t16

pytestmark = pytest.mark.gpu


def make_case(m, n, k, ranks, *, slices=1, bounds=None, seed=0, null_frac=0.1, routes=None):
    rng = np.random.default_rng(seed)
    lora = _cases.lora_tables(rng, k, n, list(ranks), slices=slices, bounds=bounds)
    if routes is None:
        routes = rng.integers(0, len(ranks), m).astype(np.int32)
        routes[rng.random(m) < null_frac] = -1
    lora["token_slots"] = np.asarray(routes, np.int32)
    x = _cases.bf16(rng.standard_normal((m, k)))
    y = _cases.bf16(rng.standard_normal((m, n)))
    return dict(x=x, y=y, lora=lora, m=m, n=n, k=k)


def expected(case):
    lo = case["lora"]
    return linear.lora_apply(case["x"], case["y"], **{key: lo[key] for key in (
        "a_store", "a_offsets", "b_store", "b_offsets", "b_strides", "ranks", "scales", "token_slots", "slice_offsets")})


def on_device(case, device):
    lo = case["lora"]
    batch = LoraBatch(
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
    return t16(case["x"], device), t16(case["y"], device), batch


def check(case, y):
    out = bits(y)
    close(out, expected(case))
    idle = case["lora"]["token_slots"] < 0
    idle |= case["lora"]["ranks"][np.maximum(case["lora"]["token_slots"], 0)] == 0
    assert np.array_equal(out[idle], case["y"][idle])


def test_c2_full_shape(device):
    """BASELINE c2: 64 tokens, 32 rank-16 adapters, K = N = 4096, 10 % base only."""
    case = make_case(64, 4096, 4096, (16,) * 32, seed=733)
    x, y, batch = on_device(case, device)
    lora_apply(x, y, batch)
    torch.cuda.synchronize()
    check(case, y)
    assert decode_status(device=device) == 0


@pytest.mark.parametrize("m", [1, 7, 33, 64, 130])
def test_mixed_ranks_and_slices(m, device):
    """Ranks 0..64 (rank 0 = untouched), three slices, and 64-token chunks above 64 tokens."""
    ranks = (8, 64, 0, 17, 32, 4, 1)
    case = make_case(m, 512, 1024, ranks, slices=3, bounds=[0, 128, 320, 512], seed=40 + m)
    x, y, batch = on_device(case, device)
    lora_apply(x, y, batch)
    torch.cuda.synchronize()
    check(case, y)


def test_strided_rows_and_graph_replay(device):
    """x and y as column views of wider tensors; a captured call replays to the eager result."""
    m, n, k = 48, 256, 512
    case = make_case(m, n, k, (16, 32, 8), seed=5)
    x0, _, batch = on_device(case, device)
    xw = torch.zeros(m, k + 64, dtype=torch.bfloat16, device=device)
    xw[:, :k] = x0
    x = xw[:, :k]
    yw = torch.full((m, n + 16), -5.0, dtype=torch.bfloat16, device=device)
    y = yw[:, 8 : 8 + n]
    base = t16(case["y"], device)
    y.copy_(base)
    lora_apply(x, y, batch)
    torch.cuda.synchronize()
    check(case, y)
    eager = y.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        y.copy_(base)
        lora_apply(x, y, batch)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            lora_apply(x, y, batch)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(base)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
    assert torch.all(yw[:, :8] == -5.0) and torch.all(yw[:, 8 + n :] == -5.0)


def test_withheld_partials_are_recomputed(device):
    """The producers publish nothing: every consumer gives up its bounded wait, recomputes z, flags the status."""
    case = make_case(40, 512, 1024, (16, 8, 32), seed=9, null_frac=0.0)
    x, y, batch = on_device(case, device)
    need = workspace_bytes(40, 512, 1024, num_slices=1, max_rank=batch.max_rank)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    lib = _lib.library()
    ls = _lora_struct(batch, 40, 1024, 512, device)
    _lib.check(lib.lf_lora_apply(x.data_ptr(), 40, x.stride(0), 512, 1024, ls, y.data_ptr(), y.stride(0),
                                 ws.data_ptr(), need, _lib.LF_TEST_WITHHOLD_PARTIALS, _lib.stream_of(device)))
    status = ctypes.c_int32(-1)
    _lib.check(lib.lf_nf4_lora_status(ws.data_ptr(), _lib.stream_of(device), ctypes.byref(status)))
    assert status.value == 1
    check(case, y)


def test_matches_row_operators_chain(device):
    """Same inputs through row_shrink + row_expand (segments of <= 16 rows): both within the gate of each other."""
    from loraforge_amd.ops import row_expand, row_shrink

    c = _cases.c2_case(seed=77, tokens=64, k=1024, n=512)
    meta = {key: torch.from_numpy(v).to(device) for key, v in c["meta"].items()}
    x, a, b, y = (t16(c[key], device) for key in ("x", "a", "b", "y"))
    z = torch.zeros(64, 16, dtype=torch.bfloat16, device=device)
    routes = torch.from_numpy(c["routes"]).to(device)
    row_shrink(x, a, z, routes, meta["ranks"], max_rank=16)
    y_rows = y.clone()
    row_expand(z, b, y_rows, **meta)
    batch = LoraBatch(
        a.reshape(-1), torch.arange(32, dtype=torch.int64, device=device) * (16 * 1024), b,
        meta["b_offsets"], meta["b_strides"], meta["ranks"], meta["scales"], routes, meta["slice_offsets"], max_rank=16,
    )
    y_fused = y.clone()
    lora_apply(x, y_fused, batch)
    torch.cuda.synchronize()
    close(bits(y_fused), bits(y_rows))
    idle = c["routes"] < 0
    assert np.array_equal(bits(y_fused)[idle], c["y"][idle])


def test_contract_errors(device):
    case = make_case(4, 128, 128, (8,), seed=1)
    x, y, batch = on_device(case, device)
    with pytest.raises(ValueError, match="multiples of 64"):
        lora_apply(x[:, :96], y, batch)
    with pytest.raises(ValueError, match="same number of rows"):
        lora_apply(x[:3], y, batch)
    with pytest.raises(ValueError, match="share storage"):
        lora_apply(x, x, batch)
