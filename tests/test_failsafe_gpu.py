"""Bounded waits of the fused linear give up safely.

A test-only flag (LF_TEST_WITHHOLD_PARTIALS) makes the producers publish
nothing: decode shrink producers store no tagged partials, prefill z
producers store no z and set no flag. Every consumer's bounded wait then
runs out (a shortened limit under the flag), the consumer recomputes what it
was waiting for from x and A, the status word reports the give-up, and the
output still matches the oracle. Every kernel runs to its end; nothing is
left waiting. Gate: max abs/rel 2e-2 and relative L2 < 0.005.
"""

import ctypes

import numpy as np
import pytest
import torch

from loraforge_amd import _lib
from loraforge_amd.ops.fused import _lora_struct, _weight_struct, workspace_bytes
from tests import _cases
from tests.test_fused_gpu import bits, close, to_device

pytestmark = pytest.mark.gpu


def call(case, device, flags):
    x, q, st, lora, bias = to_device(case, device)
    m, n, k = case["m"], case["state"]["shape"][0], case["state"]["shape"][1]
    w, keep = _weight_struct(q, st, None, n, k, device, m)
    ls = _lora_struct(lora, m, k, n, device)
    need = workspace_bytes(m, n, k, num_slices=lora.num_slices, max_rank=lora.max_rank)
    ws = torch.zeros(need, dtype=torch.uint8, device=device)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    lib = _lib.library()
    _lib.check(lib.lf_nf4_lora_linear(x.data_ptr(), m, x.stride(0), w, _lib.ptr(bias), ls, y.data_ptr(), y.stride(0),
                                      ws.data_ptr(), need, flags, _lib.stream_of(device)))
    status = ctypes.c_int32(-1)
    _lib.check(lib.lf_nf4_lora_status(ws.data_ptr(), _lib.stream_of(device), ctypes.byref(status)))
    del keep
    return bits(y), status.value


@pytest.mark.parametrize("m,plan", [(1, 0), (7, 0), (40, 0), (64, 0), (300, "prefill"), (300, "decode")])
def test_withheld_producers_are_recomputed(m, plan, device):
    plan = {0: 0, "prefill": _lib.LF_PLAN_PREFILL, "decode": _lib.LF_PLAN_DECODE_CHUNKS}[plan]
    case = _cases.fused_case(m, 1024, 1024, ranks=(16, 8, 32, 4), seed=990 + m, bias=(m % 2 == 1),
                             null_frac=0.0)
    expect = _cases.fused_expected(case)
    y, status = call(case, device, plan)
    assert status == 0
    close(y, expect)
    y, status = call(case, device, plan | _lib.LF_TEST_WITHHOLD_PARTIALS)
    assert status == 1
    close(y, expect)
    y, status = call(case, device, plan)  # a fresh workspace after a give-up
    assert status == 0
    close(y, expect)


def test_withheld_producers_with_slices_and_many_adapters(device):
    """Prefill tile with dozens of adapters (many producers, all recomputed by the consumer) and 2 slices."""
    rng = np.random.default_rng(12)
    m = 256
    routes = _cases.zipf_routes(rng, m, 48)
    case = _cases.fused_case(m, 1024, 512, ranks=[int(r) for r in rng.choice([4, 8, 16, 32], 48)], slices=2,
                             bounds=[0, 512, 1024], seed=13, token_slots=routes)
    y, status = call(case, device, _lib.LF_PLAN_PREFILL | _lib.LF_TEST_WITHHOLD_PARTIALS)
    assert status == 1
    close(y, _cases.fused_expected(case))
