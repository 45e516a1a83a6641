"""The allocation-free fused linear (lf_nf4_lora_linear_noalloc) against lf_nf4_lora_linear.

Both entry points run the same kernels; the allocation-free one takes its
workspace from a library-owned device array instead of a caller buffer, so
its outputs must equal the workspace entry point's bit for bit (and the
oracle within the 2e-2 gate). Each case makes two calls in a row, the second
with a smaller input, then a captured call is replayed between eager work.
"""

import numpy as np
import pytest
import torch

from loraforge_amd import _lib
from loraforge_amd.ops.fused import _lora_struct, _weight_struct
from tests import _cases
from tests.test_fused_gpu import bits, close, to_device

pytestmark = pytest.mark.gpu


def _call(entry, x, q, st, lora, out, ws=None, exact=False):
    device = x.device
    m, k = x.shape
    n = out.shape[1]
    w, keep = _weight_struct(q, st, None, n, k, device, m, exact)
    ls = _lora_struct(lora, m, k, n, device) if lora is not None else None
    lib = _lib.library()
    stream = _lib.stream_of(device)
    flags = _lib.LF_EXACT_WEIGHTS if exact else 0
    if entry == "noalloc":
        rc = lib.lf_nf4_lora_linear_noalloc(
            x.data_ptr(), m, x.stride(0), w, None, ls, out.data_ptr(), out.stride(0), flags, stream
        )
    else:
        rc = lib.lf_nf4_lora_linear(
            x.data_ptr(), m, x.stride(0), w, None, ls, out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), flags, stream
        )
    _lib.check(rc)
    del keep


def _subset(case, m):
    sub = dict(case, x=case["x"][:m], m=m)
    sub["lora"] = dict(case["lora"], token_slots=case["lora"]["token_slots"][:m])
    return sub


def test_noalloc_first_calls_on_two_streams(device):
    """The device's first allocation-free call runs on stream A and the next on stream B,
    issued right after the first returned with no host synchronisation between them (B only
    waits for A's work, as calls sharing the scratch must be ordered): the second must find
    the scratch cleared (first in this file, so in a fresh process it is the device's first
    call)."""
    case = _cases.fused_case(24, 1024, 2048, ranks=(16, 8, 32), seed=86)
    x, q, st, lora, _ = to_device(case, device)
    expect = _cases.fused_expected(case)
    ws = torch.zeros(_lib.library().lf_nf4_lora_workspace_size(24, 1024, 2048, 1, lora.max_rank), dtype=torch.uint8, device=device)
    ref = torch.empty(24, 1024, dtype=torch.bfloat16, device=device)
    _call("workspace", x, q, st, lora, ref, ws=ws)
    torch.cuda.synchronize()
    outs = [torch.full((24, 1024), 3.0, dtype=torch.bfloat16, device=device) for _ in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    print("[noalloc] first call on stream A, second on stream B", flush=True)
    with torch.cuda.stream(streams[0]):
        _call("noalloc", x, q, st, lora, outs[0])
    streams[1].wait_stream(streams[0])
    with torch.cuda.stream(streams[1]):
        _call("noalloc", x, q, st, lora, outs[1])
    torch.cuda.synchronize()
    for out in outs:
        assert torch.equal(out, ref)
        close(bits(out), expect)


@pytest.mark.parametrize(
    "shape",
    [
        (64, 5, 4096, 4096, (16,) * 32, False, False),  # north-star decode, then a smaller batch
        (600, 200, 512, 1024, (16, 32, 8), True, True),  # prefill with the nested state rebuilt in the scratch
    ],
)
def test_noalloc_matches_workspace_entry(shape, device):
    m_big, m_small, n, k, ranks, dq, exact = shape
    if m_big > 64:
        slots = np.repeat(np.array([2, 0, -1, 1], np.int32), [150, 200, 50, 200])
        case = _cases.fused_case(m_big, n, k, ranks=ranks, double_quant=dq, seed=81, token_slots=slots)
    else:
        case = _cases.fused_case(m_big, n, k, ranks=ranks, double_quant=dq, seed=81)
    print(f"[noalloc] m={m_big}/{m_small} n={n} k={k} dq={dq} exact={exact}", flush=True)
    for m in (m_big, m_small):
        sub = _subset(case, m)
        x, q, st, lora, _ = to_device(sub, device)
        ws = torch.zeros(max(_lib.library().lf_nf4_lora_workspace_size(m, n, k, 1, lora.max_rank), 1), dtype=torch.uint8, device=device)
        ref = torch.empty(m, n, dtype=torch.bfloat16, device=device)
        got = torch.full((m, n), 3.0, dtype=torch.bfloat16, device=device)
        _call("workspace", x, q, st, lora, ref, ws=ws, exact=exact)
        _call("noalloc", x, q, st, lora, got, exact=exact)
        torch.cuda.synchronize()
        assert torch.equal(got, ref)
        close(bits(got), _cases.fused_expected(sub))


def test_noalloc_graph_replay(device):
    """After the first (eager) call on the device, calls may be captured; replays between
    eager calls of another shape keep matching."""
    case = _cases.fused_case(16, 1024, 1024, ranks=(16,) * 4, seed=83)
    other = _cases.fused_case(40, 512, 1024, ranks=(8, 8), seed=84)
    x, q, st, lora, _ = to_device(case, device)
    xo, qo, so, lo, _ = to_device(other, device)
    out = torch.empty(16, 1024, dtype=torch.bfloat16, device=device)
    out_o = torch.empty(40, 512, dtype=torch.bfloat16, device=device)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        _call("noalloc", x, q, st, lora, out)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            _call("noalloc", x, q, st, lora, out)
    torch.cuda.synchronize()
    expect = _cases.fused_expected(case)
    expect_o = _cases.fused_expected(other)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            graph.replay()
            _call("noalloc", xo, qo, so, lo, out_o)
        torch.cuda.synchronize()
        close(bits(out), expect)
        close(bits(out_o), expect_o)


def test_noalloc_rejects_oversized_problem(device):
    """A problem whose workspace exceeds the scratch array is refused before any launch."""
    m, n, k = 65536, 64, 64
    assert _lib.library().lf_nf4_lora_workspace_size(m, n, k, 1, 16) > _lib.NOALLOC_SCRATCH_BYTES
    case = _cases.fused_case(4, n, k, ranks=(16,), seed=85)
    _, q, st, lora, _ = to_device(case, device)
    x = torch.zeros(m, k, dtype=torch.bfloat16, device=device)
    out = torch.zeros(m, n, dtype=torch.bfloat16, device=device)
    lora = lora.with_tokens(torch.full((m,), -1, dtype=torch.int32, device=device))
    with pytest.raises(ValueError, match="allocation-free entry point holds"):
        _call("noalloc", x, q, st, lora, out)
    torch.cuda.synchronize()
    assert not out.any()
