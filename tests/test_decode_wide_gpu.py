"""The wide-batch decode kernel (32 rows x 32 tokens per workgroup over the whole K) on gfx950.

Base NF4 linear above 32 tokens against the oracle: ragged token tiles, more
than 64 tokens in one launch (the c4 token count), row-group counts that do not
fill whole XCD octets, K of one block up to 12288 (the c3 down projection, where
the weight ring is shorter), default and exact weights, bias, strided x and y,
and graph replays. Gate: max abs/rel 2e-2 and relative L2 < 0.005; the exact
weights are also compared with F.linear on the dequantised weight.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import nf4_lora_linear
from tests import _cases
from tests.test_fused_gpu import bits, close, t16, to_device

pytestmark = pytest.mark.gpu


def _base_expected(case):
    base = dict(case)
    base["lora"] = dict(case["lora"], token_slots=np.full(case["m"], -1, np.int32))
    return _cases.fused_expected(base)


@pytest.mark.parametrize(
    "m,n,k",
    [
        (33, 4096, 4096),
        (64, 4096, 4096),  # north-star base at B = 64
        (65, 1024, 1024),
        (100, 320, 512),  # 10 row groups: the second XCD octet is partly idle
        (256, 4096, 4096),  # c4's token count in one launch
        (48, 64, 64),  # one NF4 block: seven of the eight waves have no blocks
        (40, 128, 320),
        (64, 256, 12288),  # K of the c3 down projection: the shorter weight ring
        (37, 192, 8192),
    ],
)
@pytest.mark.parametrize("exact", [False, True])
def test_wide_base(m, n, k, exact, device):
    case = _cases.fused_case(m, n, k, ranks=(8,), seed=m + n + k + int(exact), bias=(m % 2 == 1))
    x, q, st, _, bias = to_device(case, device)
    print(f"[wide] m={m} n={n} k={k} exact={exact}", flush=True)
    y = nf4_lora_linear(x, q, st, bias=bias, exact=exact, plan="decode" if m > 64 else None)
    torch.cuda.synchronize()
    close(bits(y), _base_expected(case))


def test_wide_exact_matches_linear_on_dequantised_weight(device):
    """exact=True multiplies the reference's dequantised bf16 weights: compare with
    F.linear (fp32 accumulation) on those weights, to a tighter gate."""
    from loraforge_amd.ops import dequantize_nf4

    m, n, k = 64, 1024, 2048
    case = _cases.fused_case(m, n, k, ranks=(8,), seed=77)
    x, q, st, _, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, exact=True)
    w = dequantize_nf4(q, st.absmax, st.code, (n, k))
    ref = torch.nn.functional.linear(x.float(), w.float())
    torch.cuda.synchronize()
    err = (y.float() - ref).abs().max().item()
    assert err <= 2e-2 * max(1.0, ref.abs().max().item()) * 0.25, err


@pytest.mark.parametrize("offset", [0, 24])
def test_wide_strided_rows_and_graph_replay(offset, device):
    m, n, k = 72, 512, 1024
    case = _cases.fused_case(m, n, k, ranks=(8,), seed=91 + offset, bias=True)
    x, q, st, _, bias = to_device(case, device)
    xs = torch.zeros(m, k + 64, dtype=torch.bfloat16, device=device)
    xs[:, 8 : 8 + k] = x
    xv = xs[:, 8 : 8 + k]
    ys = torch.full((m, n + offset + 8), 5.0, dtype=torch.bfloat16, device=device)
    yv = ys[:, offset : offset + n]
    expect = _base_expected(case)
    nf4_lora_linear(xv, q, st, bias=bias, out=yv, plan="decode")
    torch.cuda.synchronize()
    close(bits(yv), expect)
    assert (ys[:, :offset] == 5.0).all() and (ys[:, offset + n :] == 5.0).all()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(xv, q, st, bias=bias, out=yv, plan="decode")  # warms this stream's workspace
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(xv, q, st, bias=bias, out=yv, plan="decode")
    torch.cuda.synchronize()
    for _ in range(3):
        yv.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        close(bits(yv), expect)


def test_wide_matches_across_token_tiles(device):
    """Every 32-token tile computes its rows the same way: the first 64 tokens of a
    256-token call equal a 64-token call bit for bit."""
    m, n, k = 256, 1024, 1024
    case = _cases.fused_case(m, n, k, ranks=(8,), seed=5)
    x, q, st, _, _ = to_device(case, device)
    big = nf4_lora_linear(x, q, st, plan="decode")
    small = nf4_lora_linear(x[:64].contiguous(), q, st)
    torch.cuda.synchronize()
    assert torch.equal(big[:64], small)


@pytest.mark.parametrize("slots", [1, 65, 256, 300])
def test_wide_lora_slot_counts(slots, device):
    """The LoRA wave loads the per-slot arrays whole (lane l: slots l, l + 64,
    ...) when the pool has at most 256 slots and looks each token up by lane
    shuffle; above that it reads each token's slot entries. Both against the
    oracle, with tokens spread over the whole pool."""
    m, n, k = 64, 1024, 2048
    rng = np.random.default_rng(slots)
    ranks = tuple(int(r) for r in rng.choice([4, 8, 16], slots))
    token_slots = rng.integers(0, slots, m).astype(np.int32)
    token_slots[:4] = [slots - 1, 0, -1, slots // 2]
    case = _cases.fused_case(m, n, k, ranks=ranks, seed=slots, token_slots=token_slots)
    x, q, st, lora, _ = to_device(case, device)
    print(f"[wide-lora] slots={slots}", flush=True)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))


def test_wide_lora_slots_past_the_pool_run_base_only(device):
    """With the pool's slot count given (it always is through nf4_lora_linear),
    a token slot at or past it runs the base linear alone in the wide kernel."""
    m, n, k = 48, 512, 1024
    slots = 8
    token_slots = np.arange(m, dtype=np.int32) % (slots + 4)  # 8..11 are past the pool
    case = _cases.fused_case(m, n, k, ranks=(16,) * slots, seed=12, token_slots=token_slots)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    expect_case = dict(case)
    expect_case["lora"] = dict(case["lora"], token_slots=np.where(token_slots >= slots, -1, token_slots).astype(np.int32))
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(expect_case))
