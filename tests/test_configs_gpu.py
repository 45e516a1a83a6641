"""BASELINE.json's configurations at their own sizes on gfx950, against the oracle.

c1: NF4 4096 -> 4096 (block 64, fp32 absmax), B = 1, one rank-16 adapter, scale 2.0.
North star: the same linear at B = 1..64 with 32 rank-16 adapters (10 % base-only tokens);
  every batch the bench times is compared here (B = 1 and 64 also in test_fused_gpu).
c2: BF16 multi-LoRA row_shrink + row_expand, 64 tokens, 32 x rank 16, K = N = 4096.
c3: the NF4 + double-quant SwiGLU MLP 4096 / 12288 (gate/up [2 x 12288, 4096] as two
  slices, SwiGLU, down [4096, 12288]), 16 rank-8 adapters, B = 1 / 8 / 64.
c4: NF4 4096 -> 4096 with 128 retained-rank adapters (ranks uniform over {4..64},
  ragged stores), Zipf(1.1) routing, T = 256 (prefill path) and 64 (decode path).
Gates: max abs/rel 2e-2 and relative L2 < 0.005 on bf16 outputs (BASELINE tolerance).
Weights are quantised with PyTorch on the CPU (input generation only); the oracle
dequantises exactly those bytes.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import nf4_lora_linear, row_expand, row_shrink
from loraforge_amd.ops.activation import silu_mul
from oracle import linear, nf4 as onf4, rows
from tests import _cases
from tests.test_fused_gpu import bits, close, t16, to_device, workspace_clean

pytestmark = pytest.mark.gpu


def _with_w_bits(state):
    return onf4.dequantize(state["qweight"], state["scales"], state["shape"])


@pytest.fixture(scope="module")
def square_weight():
    state = _cases.torch_quantized_state(4096, 4096, seed=731)
    return state, _with_w_bits(state)


@pytest.mark.parametrize("exact", [False, True])
def test_c1_single_adapter(square_weight, exact, device):
    state, w_bits = square_weight
    case = _cases.fused_case(1, 4096, 4096, ranks=(16,), null_frac=0.0, seed=732, state=state)
    case["w_bits"] = w_bits
    assert case["lora"]["token_slots"].tolist() == [0]
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora, exact=exact)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)


@pytest.mark.parametrize("m", [2, 4, 8, 16, 32])
def test_north_star_batches(square_weight, m, device):
    state, w_bits = square_weight
    case = _cases.fused_case(m, 4096, 4096, ranks=(16,) * 32, seed=731 + m, state=state)
    case["w_bits"] = w_bits
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)


def test_c2_row_operators(device):
    c = _cases.c2_case()
    meta = {k: torch.from_numpy(v).to(device) for k, v in c["meta"].items()}
    x, a, b, y = (t16(c[key], device) for key in ("x", "a", "b", "y"))
    z = t16(c["z"], device)
    routes = torch.from_numpy(c["routes"]).to(device)
    row_shrink(x, a, z, routes, meta["ranks"], max_rank=16)
    torch.cuda.synchronize()
    zb = bits(z)
    expected_z = rows.row_shrink(c["x"], c["a"], c["z"], c["routes"], c["meta"]["ranks"])
    live = c["routes"] >= 0
    close(zb[live], expected_z[live])
    assert np.array_equal(zb[~live], c["z"][~live])
    row_expand(z, b, y, **meta)
    torch.cuda.synchronize()
    expected = rows.row_expand(zb, c["b"], c["y"], **c["meta"])
    close(bits(y), expected)
    assert np.array_equal(bits(y)[~live], c["y"][~live])


@pytest.fixture(scope="module")
def c3_mlp():
    hidden, inter = 4096, 12288
    gu_state = _cases.torch_quantized_state(2 * inter, hidden, double_quant=True, seed=733)
    down_state = _cases.torch_quantized_state(hidden, inter, double_quant=True, seed=734)
    gate_up = _cases.fused_case(
        64, 2 * inter, hidden, ranks=(8,) * 16, slices=2, bounds=[0, inter, 2 * inter], null_frac=0.0, seed=735,
        state=gu_state,
    )
    gate_up["w_bits"] = _with_w_bits(gu_state)
    down = _cases.fused_case(64, hidden, inter, ranks=(8,) * 16, null_frac=0.0, seed=736, state=down_state)
    down["w_bits"] = _with_w_bits(down_state)
    down["lora"]["token_slots"] = gate_up["lora"]["token_slots"].copy()
    return gate_up, down


def _rows_of(case, m):
    sub = dict(case, x=case["x"][:m], m=m)
    sub["lora"] = dict(case["lora"], token_slots=case["lora"]["token_slots"][:m])
    return sub


@pytest.mark.parametrize("m", [1, 8, 64])
def test_c3_swiglu_mlp(c3_mlp, m, device):
    gate_up_case, down_case = (_rows_of(c, m) for c in c3_mlp)
    x, q1, st1, lora1, _ = to_device(gate_up_case, device)
    gu = nf4_lora_linear(x, q1, st1, lora=lora1)
    h = silu_mul(gu)
    torch.cuda.synchronize()
    gu_bits = bits(gu)
    close(gu_bits, _cases.fused_expected(gate_up_case))
    inter = gu.shape[1] // 2
    expect_h = linear.silu_mul(gu_bits[:, :inter], gu_bits[:, inter:])
    np.testing.assert_allclose(onf4.bf16_to_f32(bits(h)), onf4.bf16_to_f32(expect_h), rtol=2e-2, atol=2e-2)
    down_case = dict(down_case, x=bits(h))
    _, q2, st2, lora2, _ = to_device(down_case, device)
    y = nf4_lora_linear(h, q2, st2, lora=lora2)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(down_case))
    workspace_clean(device)


@pytest.mark.parametrize("m,plan", [(64, None), (256, None), (256, "prefill")])
def test_c4_retained_ranks_zipf_full_size(square_weight, m, plan, device):
    """c4 at its full shape; 256 tokens run the chunked decode plan by default, the prefill GEMM when forced."""
    state, w_bits = square_weight
    rng = np.random.default_rng(737)
    ranks = rng.choice([4, 8, 16, 32, 64], size=128).tolist()
    routes = _cases.zipf_routes(rng, m, 128)
    case = _cases.fused_case(m, 4096, 4096, ranks=ranks, seed=738, token_slots=routes, state=state)
    case["w_bits"] = w_bits
    x, q, st, lora, _ = to_device(case, device)
    assert lora.max_rank == 64
    y = nf4_lora_linear(x, q, st, lora=lora, plan=plan)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    workspace_clean(device)
