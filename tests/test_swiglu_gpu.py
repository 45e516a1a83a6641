"""SwiGLU step and the c3 MLP chain (gate/up -> SwiGLU -> down) on gfx950.

The activation follows ``benchmarks/qwen35_decode_silu.py:60-61``:
``bf16(bf16(silu(g)) * u)`` with silu in fp32. The oracle evaluates the same
chain in numpy (``oracle/linear.py`` ``silu_mul``); fp32 ``exp`` may differ in
its last bit between the two, so activations are allowed one bf16 ulp and
must be bit-identical almost everywhere. The chain runs at a c3-like MLP
(hidden 1024, intermediate 3072, double-quantised NF4, 16 rank-8 adapters on
gate/up and down, B in {1, 8, 64}) and at the real c3 down-projection shape
(K = 12288); projections are held to the fused tolerance of the other tests.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import nf4_lora_linear
from loraforge_amd.ops.activation import silu_mul
from oracle import linear
from oracle import nf4 as onf4
from tests import _cases
from tests.test_fused_gpu import bits, close, t16, to_device

pytestmark = pytest.mark.gpu


def assert_activation(actual_bits, expected_bits):
    a = actual_bits.astype(np.int32)
    e = expected_bits.astype(np.int32)
    ulps = np.abs(a - e)
    assert ulps.max() <= 1, ulps.max()
    assert (ulps == 0).mean() > 0.99


@pytest.mark.parametrize("rows,n", [(37, 1000), (64, 4096), (1, 8)])
def test_silu_mul_matches_oracle(rows, n, device):
    rng = np.random.default_rng(rows * 7 + n)
    vals = rng.standard_normal((rows, 2 * n)) * 3.0
    vals[0, :6] = [0.0, -0.0, 40.0, -40.0, 88.0, -100.0]
    gu = _cases.bf16(vals)
    out = silu_mul(t16(gu, device))
    torch.cuda.synchronize()
    assert out.shape == (rows, n)
    assert_activation(bits(out), linear.silu_mul(gu[:, :n], gu[:, n:]))


def test_silu_mul_strided_views_and_aliasing(device):
    rng = np.random.default_rng(5)
    n = 64
    base = t16(_cases.bf16(rng.standard_normal((9, 2 * n + 8))), device)
    view = base[:, : 2 * n]
    out_store = torch.zeros(9, n + 8, dtype=torch.bfloat16, device=device)
    out = out_store[:, :n]
    silu_mul(view, out=out)
    torch.cuda.synchronize()
    gu = bits(view)
    assert_activation(bits(out), linear.silu_mul(gu[:, :n], gu[:, n:]))
    assert torch.equal(out_store[:, n:], torch.zeros_like(out_store[:, n:]))
    with pytest.raises(ValueError, match="share storage"):
        silu_mul(base[:, : 2 * n], out=base[:, :n])
    with pytest.raises(ValueError, match="2 \\* n"):
        silu_mul(base[:, :7])


@pytest.fixture(scope="module")
def mlp_cases():
    hidden, inter = 1024, 3072
    gate_up = _cases.fused_case(
        64, 2 * inter, hidden, ranks=(8,) * 16, slices=2, bounds=[0, inter, 2 * inter], double_quant=True, seed=733
    )
    down = _cases.fused_case(64, hidden, inter, ranks=(8,) * 16, double_quant=True, seed=734)
    down["lora"]["token_slots"] = gate_up["lora"]["token_slots"].copy()
    return gate_up, down


def rows_of(case, m):
    sub = dict(case, x=case["x"][:m], m=m)
    sub["lora"] = dict(case["lora"], token_slots=case["lora"]["token_slots"][:m])
    return sub


@pytest.mark.parametrize("m", [1, 8, 64])
def test_c3_mlp_chain(mlp_cases, m, device):
    gate_up_case, down_case = (rows_of(c, m) for c in mlp_cases)
    x, q1, st1, lora1, _ = to_device(gate_up_case, device)
    gu = nf4_lora_linear(x, q1, st1, lora=lora1)
    h = silu_mul(gu)
    torch.cuda.synchronize()
    gu_bits = bits(gu)
    close(gu_bits, _cases.fused_expected(gate_up_case))
    inter = gu.shape[1] // 2
    assert_activation(bits(h), linear.silu_mul(gu_bits[:, :inter], gu_bits[:, inter:]))
    down_case = dict(down_case, x=bits(h))
    _, q2, st2, lora2, _ = to_device(down_case, device)
    y = nf4_lora_linear(h, q2, st2, lora=lora2)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(down_case))


def test_c3_down_projection_shape(device):
    case = _cases.fused_case(64, 4096, 12288, ranks=(8,) * 16, double_quant=True, seed=736, null_frac=0.0)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    cols = np.unique(np.concatenate([np.arange(0, 4096, 61), [4095]]))
    close(bits(y)[:, cols], _cases.fused_expected(case, rows=cols))


def test_c3_chain_graph_replay(mlp_cases, device):
    """gate/up -> SwiGLU -> down captured in one HIP graph: every replay equals the eager chain."""
    gate_up_case, down_case = (rows_of(c, 8) for c in mlp_cases)
    x, q1, st1, lora1, _ = to_device(gate_up_case, device)
    _, q2, st2, lora2, _ = to_device(dict(down_case, x=np.zeros((8, 3072), np.uint16)), device)
    gu = torch.empty(8, 6144, dtype=torch.bfloat16, device=device)
    h = torch.empty(8, 3072, dtype=torch.bfloat16, device=device)
    y = torch.empty(8, 1024, dtype=torch.bfloat16, device=device)

    def chain():
        nf4_lora_linear(x, q1, st1, lora=lora1, out=gu)
        silu_mul(gu, out=h)
        nf4_lora_linear(h, q2, st2, lora=lora2, out=y)

    chain()
    torch.cuda.synchronize()
    eager = y.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        chain()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        chain()
    for _ in range(3):
        y.zero_()
        h.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, eager)
