"""The decode kernels reading a double-quant (nested) NF4 state themselves.

Each base wave stages the uint8 absmax codes and absmax2 entries of its rows
into LDS and converts them with the closed form of ``lf_nf4_dequant_dq``
(reference ``ops/nf4.py:109-148``, the nested branch of ``prepare_scales``), so
a call given the nested state (``scales="nested"``) must give exactly the bits
of the same call given the prepared fp32 scales (whose path the oracle tests pin), in every
narrow tile (1..8 tokens, 9..16 at K = 12288), the wide kernel (the rest up to 64), the chunked plan, with
and without LoRA, with the default and the exact-weights arithmetic. Through
the C-ABI with a workspace of only the control header, the call can only
succeed if the kernel read the state itself (a rebuild of fp32 scales needs
room for them): that pins which path ran. Shapes the kernels do not take
(K % 256 != 0, a second-level block that is not a power of two) fall back to
scales rebuilt into the workspace, with the same bits.
"""

import numpy as np
import pytest
import torch

from loraforge_amd import _lib
from loraforge_amd.ops import LoraBatch, nf4_lora_linear, prepare_scales, quantize_nf4
from loraforge_amd.ops.fused import _lora_struct, _weight_struct
from loraforge_amd.ops.nf4 import NestedState, NF4State
from tests import _cases
from tests.test_fused_gpu import bits, close, to_device

pytestmark = pytest.mark.gpu

HEADER_BYTES = 262144  # the decode workspace's control header (no room for rebuilt scales)
_WEIGHTS = {}


def _weight(n, k, device, seed=0):
    key = (n, k, seed)
    if key not in _WEIGHTS:
        g = torch.Generator(device="cpu").manual_seed(1000 + k + seed)
        w = (torch.randn(n, k, generator=g) * 0.02).bfloat16().to(device)
        _WEIGHTS[key] = quantize_nf4(w, compress_statistics=True)
    return _WEIGHTS[key]


def _lora(m, n, k, device, seed, slices=1):
    case = _cases.fused_case(
        m, n, k, ranks=(16, 8, 32, 4), slices=slices, bounds=None if slices == 1 else [0, n // 2, n], seed=seed
    )
    x, _, _, lora, _ = to_device(dict(case, state=_cases.fused_case(1, 64, 64, ranks=(1,))["state"]), device)
    return x, lora


def _capi(x, q, st, lora, n, ws_bytes, exact=False, swiglu=False):
    device = x.device
    m, k = x.shape
    width = n // 2 if swiglu else n
    out = torch.empty(m, width, dtype=torch.bfloat16, device=device)
    w, keep = _weight_struct(q, st, "nested", n, k, device, m, exact)
    assert not w.scales, "the nested state itself"
    ls = _lora_struct(lora, m, k, n, device) if lora is not None else None
    ws = torch.zeros(ws_bytes, dtype=torch.uint8, device=device)
    flags = (_lib.LF_EXACT_WEIGHTS if exact else 0) | (_lib.LF_SWIGLU_OUTPUT if swiglu else 0)
    lib = _lib.library()
    _lib.check(
        lib.lf_nf4_lora_linear(
            x.data_ptr(), m, x.stride(0), w, None, ls, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), flags,
            _lib.stream_of(device),
        )
    )
    del keep
    return out


@pytest.mark.parametrize("k", [256, 1024, 4096, 12288])
@pytest.mark.parametrize("m", [1, 2, 5, 8, 16, 32, 33, 64])
def test_nested_state_read_in_kernel(m, k, device):
    """Every narrow tile and the wide kernel, with and without LoRA, default and exact
    arithmetic: the nested state read in-kernel (a header-only workspace: no rebuild
    possible) gives the bits of the call with prepared fp32 scales."""
    n = 256
    q, st = _weight(n, k, device)
    x, lora = _lora(m, n, k, device, seed=7 * m + k)
    scales = prepare_scales(st)
    print(f"[dq] m={m} k={k}", flush=True)
    for exact in (False, True):
        for lo in (lora, None):
            got = _capi(x, q, st, lo, n, HEADER_BYTES, exact=exact)
            want = nf4_lora_linear(x, q, st, scales=scales, lora=lo, exact=exact)
            torch.cuda.synchronize()
            assert torch.equal(got, want), (exact, lo is not None)
            via_py = nf4_lora_linear(x, q, st, scales="nested", lora=lo, exact=exact)
            torch.cuda.synchronize()
            assert torch.equal(via_py, want)


@pytest.mark.parametrize("m", [12, 24, 32])
def test_nested_state_narrow_tiles_where_wide_declines(m, device):
    """N = 448 with LoRA is no multiple of 256, so 9..32 tokens stay on the narrow kernel's
    16- and 32-token tiles: the nested state read there in-kernel."""
    n, k = 448, 4096
    q, st = _weight(n, k, device, seed=13)
    x, lora = _lora(m, n, k, device, seed=110 + m)
    scales = prepare_scales(st)
    for exact in (False, True):
        got = _capi(x, q, st, lora, n, HEADER_BYTES, exact=exact)
        want = nf4_lora_linear(x, q, st, scales=scales, lora=lora, exact=exact)
        torch.cuda.synchronize()
        assert torch.equal(got, want), exact


@pytest.mark.parametrize("m", [1, 8, 48])
def test_nested_state_swiglu_and_gated_rows(m, device):
    """The SwiGLU output (a row group's gate rows and the matching up rows N / 2 further on,
    so the two row halves read different absmax2 runs) with the nested state read in-kernel."""
    n, k = 1024, 4096
    q, st = _weight(n, k, device, seed=3)
    x, lora = _lora(m, n, k, device, seed=90 + m, slices=2)
    got = _capi(x, q, st, lora, n, HEADER_BYTES, swiglu=True)
    want = nf4_lora_linear(x, q, st, scales=prepare_scales(st), lora=lora, swiglu=True)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("m", [100, 300])
def test_nested_state_chunked_plan(m, device):
    """Above 64 tokens the decode plan's chunks (wide kernel, narrow tail) read the state."""
    n, k = 512, 1024
    q, st = _weight(n, k, device, seed=5)
    x, lora = _lora(m, n, k, device, seed=40 + m)
    got = nf4_lora_linear(x, q, st, scales="nested", lora=lora, plan="decode")
    want = nf4_lora_linear(x, q, st, scales=prepare_scales(st), lora=lora, plan="decode")
    torch.cuda.synchronize()
    assert torch.equal(got, want)


@pytest.mark.parametrize("m", [1, 16, 40])
def test_nested_state_fallbacks_rebuild_scales(m, device):
    """K % 256 != 0 and a second-level block of 192 (not a power of two): the library rebuilds
    fp32 scales into the workspace (a header-only workspace is refused) with the same bits."""
    n, k = 256, 320
    q, st = _weight(n, k, device, seed=9)
    x, lora = _lora(m, n, k, device, seed=60 + m)
    want = nf4_lora_linear(x, q, st, scales=prepare_scales(st), lora=lora)
    w, keep = _weight_struct(q, st, "nested", n, k, device, m)
    assert not w.scales
    ls = _lora_struct(lora, m, k, n, device)
    lib = _lib.library()
    out = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    small = torch.zeros(HEADER_BYTES, dtype=torch.uint8, device=device)
    rc = lib.lf_nf4_lora_linear(x.data_ptr(), m, k, w, None, ls, out.data_ptr(), n, small.data_ptr(), small.numel(), 0,
                                _lib.stream_of(device))
    assert rc == _lib.LF_EINVAL and b"rebuilt scales" in lib.lf_last_error()
    need = lib.lf_nf4_lora_workspace_size(m, n, k, 1, 64)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    _lib.check(lib.lf_nf4_lora_linear(x.data_ptr(), m, k, w, None, ls, out.data_ptr(), n, ws.data_ptr(), ws.numel(), 0,
                                      _lib.stream_of(device)))
    torch.cuda.synchronize()
    assert torch.equal(out, want)
    del keep
    # A second-level block of 192 entries at K = 4096 (the closed form indexes absmax2 by
    # block // 192): rebuilt, and equal to the prepared scales' call.
    k2 = 4096
    q2, st2 = _weight(n, k2, device, seed=11)
    codes = st2.absmax
    blocks = codes.numel()
    g = torch.Generator(device="cpu").manual_seed(12)
    a2 = (torch.rand(-(-blocks // 192), generator=g) + 0.5).to(device)
    st192 = NF4State(codes, st2.shape, st2.code, st2.dtype, offset=st2.offset,
                     state2=NestedState(a2, st2.state2.code, 192))
    x2, lora2 = _lora(m, n, k2, device, seed=70 + m)
    w2, keep2 = _weight_struct(q2, st192, "nested", n, k2, device, m)
    assert not w2.scales and w2.dq_block == 192
    ls2 = _lora_struct(lora2, m, k2, n, device)
    need2 = lib.lf_nf4_lora_workspace_size(m, n, k2, 1, 64)
    ws2 = torch.zeros(need2, dtype=torch.uint8, device=device)
    got = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    _lib.check(lib.lf_nf4_lora_linear(x2.data_ptr(), m, k2, w2, None, ls2, got.data_ptr(), n, ws2.data_ptr(),
                                      ws2.numel(), 0, _lib.stream_of(device)))
    want = nf4_lora_linear(x2, q2, st192, scales=prepare_scales(st192), lora=lora2)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    del keep2


def test_nested_state_oracle_and_graph_replay(device):
    """The in-kernel path against the oracle (a double-quant case built on the CPU), and
    replayed from a captured graph between eager calls."""
    case = _cases.fused_case(8, 512, 1024, ranks=(16,) * 4, double_quant=True, seed=77)
    x, q, st, lora, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st, scales="nested", lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    out = torch.empty_like(y)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        nf4_lora_linear(x, q, st, scales="nested", lora=lora, out=out)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            nf4_lora_linear(x, q, st, scales="nested", lora=lora, out=out)
    torch.cuda.synchronize()
    for _ in range(3):
        out.zero_()
        nf4_lora_linear(x, q, st, scales="nested", lora=lora)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y)
