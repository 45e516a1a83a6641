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

from loraforge_amd.ops import LoraBatch, nf4_lora_linear, quantize_nf4
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
    # Zeros of both signs, around the overflow of e^-g (g near -88.7), past the exponent
    # clamp of the activation (|g| >= 126) and huge gates.
    vals[0, :8] = [0.0, -0.0, 40.0, -40.0, 88.0, -100.0, -88.5, -89.0]
    if n >= 16:
        vals[0, 8:16] = [126.0, 127.0, -126.5, -127.0, 1e30, -1e30, 3e38, -3e38]
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


@pytest.mark.parametrize("m", [1, 2, 7, 16, 20, 33, 64, 100])
@pytest.mark.parametrize("with_lora", [True, False])
def test_fused_swiglu_output_equals_the_separate_chain(m, with_lora, device):
    """swiglu=True (decode: the activation in the kernel's epilogue, 16- and 32-row groups;
    prefill: linear then silu_mul) gives exactly the bits of the linear followed by silu_mul,
    and the oracle's activation of the oracle's gate/up."""
    inter = 1024
    case = _cases.fused_case(
        m, 2 * inter, 512, ranks=(8, 16, 4), slices=2, bounds=[0, inter, 2 * inter], seed=880 + m, bias=True
    )
    x, q, st, lora, bias = to_device(case, device)
    lora = lora if with_lora else None
    if not with_lora:
        case = dict(case, lora=dict(case["lora"], token_slots=np.full(m, -1, np.int32)))
    h = nf4_lora_linear(x, q, st, bias=bias, lora=lora, swiglu=True)
    gu = nf4_lora_linear(x, q, st, bias=bias, lora=lora)
    sep = silu_mul(gu)
    torch.cuda.synchronize()
    assert h.shape == (m, inter)
    assert torch.equal(h, sep)
    expect_gu = _cases.fused_expected(case)
    close(bits(gu), expect_gu)
    assert_activation(bits(h), linear.silu_mul(bits(gu)[:, :inter], bits(gu)[:, inter:]))


@pytest.mark.parametrize("plan", ["prefill", "decode"])
@pytest.mark.parametrize("m", [100, 300])
def test_fused_swiglu_above_64_tokens_on_both_plans(m, plan, device):
    """Above 64 tokens the activation is formed in the prefill GEMM's epilogue (each tile's
    96 gate rows with the matching up rows; 1024 columns end in a partial tile) or in each
    64-token decode chunk: the same bits as the linear on that plan followed by silu_mul."""
    inter = 1024
    case = _cases.fused_case(
        m, 2 * inter, 512, ranks=(8, 16, 4), slices=2, bounds=[0, inter, 2 * inter], seed=980 + m, bias=True
    )
    x, q, st, lora, bias = to_device(case, device)
    h = nf4_lora_linear(x, q, st, bias=bias, lora=lora, swiglu=True, plan=plan)
    gu = nf4_lora_linear(x, q, st, bias=bias, lora=lora, plan=plan)
    sep = silu_mul(gu)
    base = nf4_lora_linear(x, q, st, bias=bias, swiglu=True, plan=plan)
    base_sep = silu_mul(nf4_lora_linear(x, q, st, bias=bias, plan=plan))
    # An output whose rows are not 16-byte aligned: the linear, then the activation.
    backing = torch.zeros(m * inter + 1, dtype=torch.bfloat16, device=device)
    odd = backing[1:].view(m, inter)
    nf4_lora_linear(x, q, st, bias=bias, lora=lora, swiglu=True, plan=plan, out=odd)
    torch.cuda.synchronize()
    assert torch.equal(h, sep)
    assert torch.equal(base, base_sep)
    assert torch.equal(odd, sep)
    if plan == "prefill":
        close(bits(gu), _cases.fused_expected(case))


def test_prefill_swiglu_c5_scale(device):
    """The prefill GEMM with the activation in its epilogue at M = 2048 over c5's weight read as
    a merged gate/up projection (N = 11008: 5504 activation columns, 58 column tiles, the last
    partial), double quant, 8 segments of rank 32 over the gate/up slices: bit-identical to the
    linear followed by silu_mul."""
    m, inter, k, rank, segs = 2048, 5504, 4096, 32, 8
    g = torch.Generator(device="cpu").manual_seed(736)
    w = (torch.randn(2 * inter, k, generator=g) * 0.02).bfloat16().to(device)
    q, st = quantize_nf4(w, compress_statistics=True)
    del w
    x = torch.randn(m, k, generator=g).bfloat16().to(device)
    slots = torch.repeat_interleave(torch.arange(segs, dtype=torch.int32), m // segs).to(device)
    i64 = dict(dtype=torch.int64, device=device)
    n = 2 * inter
    lora = LoraBatch(
        (torch.randn(segs * 2 * rank * k, generator=g) * 0.02).bfloat16().to(device),
        torch.arange(segs, **i64) * (2 * rank * k),
        (torch.randn(segs * n * rank, generator=g) * 0.02).bfloat16().to(device),
        torch.arange(segs, **i64) * (n * rank),
        torch.full((segs,), rank, dtype=torch.int32, device=device),
        torch.full((segs,), rank, dtype=torch.int32, device=device),
        torch.full((segs,), 2.0, device=device),
        slots,
        torch.tensor([0, inter, n], dtype=torch.int32, device=device),
        max_rank=rank,
    )
    h = nf4_lora_linear(x, q, st, lora=lora, swiglu=True, plan="prefill")
    sep = silu_mul(nf4_lora_linear(x, q, st, lora=lora, plan="prefill"))
    torch.cuda.synchronize()
    assert torch.equal(h, sep)


@pytest.mark.parametrize("m", [16, 48])
def test_fused_swiglu_checks_out_like_the_linear(m, device):
    """swiglu=True checks out for every batch size the same way (device and storage of the
    inputs), also where the library runs the linear and the activation as two launches."""
    inter = 256
    case = _cases.fused_case(m, 2 * inter, 512, ranks=(8,), slices=2, bounds=[0, inter, 2 * inter], seed=890 + m)
    x, q, st, lora, _ = to_device(case, device)
    with pytest.raises(ValueError, match="input device"):
        nf4_lora_linear(x, q, st, lora=lora, swiglu=True, out=torch.empty(m, inter, dtype=torch.bfloat16))
    backing = torch.zeros(m * (512 + inter), dtype=torch.bfloat16, device=device)
    xs = backing[: m * 512].view(m, 512)
    xs.copy_(x)
    with pytest.raises(ValueError, match="share storage"):
        nf4_lora_linear(xs, q, st, lora=lora, swiglu=True, out=backing[m * 512 :].view(m, inter))
    torch.cuda.synchronize()


@pytest.mark.parametrize("m", [1, 8, 64])
def test_c3_gate_up_swiglu_fused_full_size(m, device):
    """c3's gate/up [2 x 12288, 4096] (double quant, 16 rank-8 adapters) with the SwiGLU in the epilogue."""
    inter = 12288
    state = _cases.torch_quantized_state(2 * inter, 4096, double_quant=True, seed=733)
    case = _cases.fused_case(
        m, 2 * inter, 4096, ranks=(8,) * 16, slices=2, bounds=[0, inter, 2 * inter], null_frac=0.0, seed=935 + m,
        state=state,
    )
    case["w_bits"] = onf4.dequantize(state["qweight"], state["scales"], state["shape"])
    x, q, st, lora, _ = to_device(case, device)
    h = nf4_lora_linear(x, q, st, lora=lora, swiglu=True)
    gu = nf4_lora_linear(x, q, st, lora=lora)
    sep = silu_mul(gu)
    torch.cuda.synchronize()
    # gate/up against the oracle at the projection tolerance; the fused activation is then
    # bit for bit the activation of those outputs (comparing h itself with the oracle's
    # activation would multiply the projection tolerance by the other operand).
    close(bits(gu), _cases.fused_expected(case))
    assert torch.equal(h, sep)


def test_fused_swiglu_graph_replay(device):
    case = _cases.fused_case(24, 2048, 512, ranks=(8, 8), slices=2, bounds=[0, 1024, 2048], seed=71)
    x, q, st, lora, _ = to_device(case, device)
    out = torch.empty(24, 1024, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, st, lora=lora, out=out, swiglu=True)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, st, lora=lora, out=out, swiglu=True)
    torch.cuda.synchronize()
    eager = out.clone()
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


@pytest.mark.parametrize("m", [9, 24, 32, 33, 48, 64])
def test_swiglu_flag_through_the_c_abi_at_32_row_groups(m, device):
    """LF_SWIGLU_OUTPUT at 9..64 tokens (the wide kernel's 32-row groups: gate tile and up
    tile meet in LDS; one token tile up to 32 tokens, two above), called through the C-ABI."""
    from loraforge_amd import _lib
    from loraforge_amd.ops.fused import _lora_struct, _weight_struct

    inter = 1024
    case = _cases.fused_case(m, 2 * inter, 512, ranks=(8, 16), slices=2, bounds=[0, inter, 2 * inter], seed=950 + m)
    x, q, st, lora, _ = to_device(case, device)
    w, keep = _weight_struct(q, st, None, 2 * inter, 512, x.device, m)
    ls = _lora_struct(lora, m, 512, 2 * inter, x.device)
    ws = torch.zeros(1 << 20, dtype=torch.uint8, device=device)
    h = torch.empty(m, inter, dtype=torch.bfloat16, device=device)
    lib = _lib.library()
    _lib.check(lib.lf_nf4_lora_linear(x.data_ptr(), m, 512, w, None, ls, h.data_ptr(), inter, ws.data_ptr(), ws.numel(),
                                      _lib.LF_SWIGLU_OUTPUT, _lib.stream_of(device)))
    sep = silu_mul(nf4_lora_linear(x, q, st, lora=lora))
    torch.cuda.synchronize()
    assert torch.equal(h, sep)
    del keep
