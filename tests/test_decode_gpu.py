"""Base NF4 decode (1..64 tokens, no adapters) on gfx950 against the oracle.

Every tile shape of the decode kernel (16 rows x 2 / 8 / 16 / 32 staged
tokens, 32 rows x 32 tokens with two token tiles), token counts that leave
ragged tiles, bias, a strided x, widths that are not a multiple of the row
tile, long K (12288, and 131072 where the block scales no longer fit LDS),
repeated calls on one workspace and graph replays.
Gate: max abs/rel 2e-2 and relative L2 < 0.005.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import nf4_lora_linear
from loraforge_amd.ops.fused import decode_status
from tests import _cases
from tests.test_fused_gpu import bits, close, t16, to_device

pytestmark = pytest.mark.gpu


def _base_expected(case):
    base = dict(case)
    base["lora"] = dict(case["lora"], token_slots=np.full(case["m"], -1, np.int32))
    return _cases.fused_expected(base)


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 16, 17, 31, 32, 33, 48, 64])
def test_decode_base_batches(m, device):
    case = _cases.fused_case(m, 1024, 2048, ranks=(8,), seed=300 + m, bias=(m % 2 == 1))
    x, q, st, _, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias)
    torch.cuda.synchronize()
    close(bits(y), _base_expected(case))
    assert decode_status(device=device) == 0


@pytest.mark.parametrize("m,n,k", [(64, 64, 64), (40, 192, 320), (12, 64, 1024), (64, 128, 12288), (7, 320, 576)])
def test_decode_base_odd_shapes(m, n, k, device):
    """Widths below or not a multiple of the row tile, K of one NF4 block per wave or less, and
    a long K (12288, the c3 down projection)."""
    case = _cases.fused_case(m, n, k, ranks=(8,), seed=n + k + m)
    x, q, st, _, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st)
    torch.cuda.synchronize()
    close(bits(y), _base_expected(case))


@pytest.mark.parametrize("m,with_lora", [(2, False), (2, True), (8, True), (12, False), (20, True), (24, False), (64, True)])
def test_decode_very_long_k(m, with_lora, device):
    """K = 131072: a wave's block scales no longer fit in LDS beside its ring, so
    the launch takes the variant that stages the scales with the weights (every
    tile; the 32-row tile already does at K = 12288, covered above). W is drawn
    8x narrower than elsewhere so the outputs stay O(1): the default arithmetic
    (bf16 codes, fp32 block scale on the block sum) differs from the
    dequantised-weight product by one bf16 rounding per weight, a difference
    that grows as sqrt(K) (at W ~ N(0, 0.02) about 0.014 rms here)."""
    case = _cases.fused_case(m, 64, 131072, ranks=(8, 16), seed=990 + m, null_frac=0.0, w_std=0.0025)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, lora=lora if with_lora else None)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case) if with_lora else _base_expected(case))
    assert decode_status(device=device) == 0


@pytest.mark.parametrize("m", [1, 64])
def test_decode_base_north_star_shape(m, device):
    state = _cases.torch_quantized_state(4096, 4096, seed=731)
    case = _cases.fused_case(m, 4096, 4096, ranks=(16,), seed=731, state=state)
    x, q, st, _, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st)
    torch.cuda.synchronize()
    close(bits(y), _base_expected(case))


def test_decode_base_strided_x_and_graph_replay(device):
    case = _cases.fused_case(24, 512, 1024, ranks=(8,), seed=77, bias=True)
    x, q, st, _, bias = to_device(case, device)
    wide = torch.zeros(24, 1024 + 64, dtype=torch.bfloat16, device=device)
    wide[:, 8 : 8 + 1024] = x
    xs = wide[:, 8 : 8 + 1024]
    expect = _base_expected(case)
    out = torch.empty(24, 512, dtype=torch.bfloat16, device=device)
    for _ in range(3):
        nf4_lora_linear(xs, q, st, bias=bias, out=out)
    torch.cuda.synchronize()
    close(bits(out), expect)
    eager = out.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(xs, q, st, bias=bias, out=out)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(xs, q, st, bias=bias, out=out)
    torch.cuda.synchronize()
    for _ in range(4):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_decode_base_without_workspace(device):
    """From C a base-only decode call may pass no workspace."""
    from loraforge_amd import _lib
    from loraforge_amd.ops.fused import _weight_struct

    case = _cases.fused_case(40, 512, 1024, ranks=(8,), seed=88)
    x, q, st, _, _ = to_device(case, device)
    w, keep = _weight_struct(q, st, None, 512, 1024, device, 40)
    y = torch.empty(40, 512, dtype=torch.bfloat16, device=device)
    lib = _lib.library()
    _lib.check(lib.lf_nf4_lora_linear(x.data_ptr(), 40, 1024, w, None, None, y.data_ptr(), 512, None, 0, 0, _lib.stream_of(device)))
    torch.cuda.synchronize()
    close(bits(y), _base_expected(case))
    del keep


@pytest.mark.parametrize("m,n", [(64, 1024), (16, 1024), (40, 512)])
def test_decode_base_consecutive_inputs(m, n, device):
    """Calls on one workspace with new inputs each time: nothing of one call stands in for the
    next call's results."""
    for seed in range(3):
        case = _cases.fused_case(m, n, 1024, ranks=(8,), seed=500 + seed)
        x, q, st, _, _ = to_device(case, device)
        y = nf4_lora_linear(x, q, st)
        torch.cuda.synchronize()
        close(bits(y), _base_expected(case))
        assert decode_status(device=device) == 0
