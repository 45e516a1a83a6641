"""Stream-K prefill (base linear, tiles beyond one round of CUs) against the oracle.

When the 256 x 192 tiles of a call without LoRA would leave at least an
eighth of the CUs idle in their last round, the GEMM workgroups split the
tiles' k-steps evenly; a tile split between workgroups is finished by the one
holding its first k-step, which adds the others' fp32 partial tiles from the
workspace (flags tagged with the call). These shapes put more tiles than CUs
on an MI355X (256 CUs): every tile of the short-K case is split. The test-only
flag LF_TEST_WITHHOLD_PARTIALS keeps the partials unpublished, so every
owner's bounded wait runs out and it computes the missing k-steps itself.
Gate: max abs/rel 2e-2 and relative L2 < 0.005.
"""

import ctypes

import numpy as np
import pytest
import torch

from loraforge_amd import _lib
from loraforge_amd.ops import nf4_lora_linear
from loraforge_amd.ops.fused import _weight_struct, workspace_bytes
from tests import _cases
from tests.test_fused_gpu import bits, close, to_device

pytestmark = [
    pytest.mark.gpu,
    pytest.mark.skip(
        reason="stream-K prefill is switched off: its first GPU run took a memory fault whose cause was not "
        "found by reading the code, so the kernel was reverted to one tile per workgroup"
    ),
]


def _base_only(case):
    base = dict(case)
    base["lora"] = dict(case["lora"], token_slots=np.full(case["m"], -1, np.int32))
    return base


def _call(case, device, flags, ws=None):
    x, q, st, _, bias = to_device(case, device)
    m, n, k = case["m"], case["state"]["shape"][0], case["state"]["shape"][1]
    w, keep = _weight_struct(q, st, None, n, k, device, m)
    need = workspace_bytes(m, n, k)
    if ws is None:
        ws = torch.zeros(need, dtype=torch.uint8, device=device)
    y = torch.empty(m, n, dtype=torch.bfloat16, device=device)
    lib = _lib.library()
    _lib.check(lib.lf_nf4_lora_linear(x.data_ptr(), m, x.stride(0), w, _lib.ptr(bias), None, y.data_ptr(), y.stride(0),
                                      ws.data_ptr(), ws.numel(), flags, _lib.stream_of(device)))
    status = ctypes.c_int32(-1)
    _lib.check(lib.lf_nf4_lora_status(ws.data_ptr(), _lib.stream_of(device), ctypes.byref(status)))
    del keep
    return bits(y), status.value


@pytest.mark.parametrize("m,n,k", [(256, 192 * 300, 512), (300, 192 * 150, 320), (256, 192 * 260 - 64, 1024)])
def test_streamk_split_tiles(m, n, k, device):
    """More tiles than CUs with few k-steps each, so every tile is split between workgroups; ragged M
    and N, bias."""
    case = _base_only(_cases.fused_case(m, n, k, ranks=(8,), seed=m + n + k, bias=True))
    y, status = _call(case, device, _lib.LF_PLAN_PREFILL)
    assert status == 0
    close(y, _cases.fused_expected(case))


def test_streamk_withheld_partials_are_recomputed(device):
    case = _base_only(_cases.fused_case(256, 192 * 300, 512, ranks=(8,), seed=77, bias=True))
    expect = _cases.fused_expected(case)
    y, status = _call(case, device, _lib.LF_PLAN_PREFILL | _lib.LF_TEST_WITHHOLD_PARTIALS)
    assert status == 1
    close(y, expect)
    y, status = _call(case, device, _lib.LF_PLAN_PREFILL)
    assert status == 0
    close(y, expect)


def test_streamk_consecutive_calls_on_one_workspace(device):
    """New inputs on one workspace each time: a flag of one call never stands for the next."""
    m, n, k = 256, 192 * 300, 512
    ws = torch.zeros(workspace_bytes(m, n, k), dtype=torch.uint8, device=device)
    for seed in range(3):
        case = _base_only(_cases.fused_case(m, n, k, ranks=(8,), seed=400 + seed))
        y, status = _call(case, device, _lib.LF_PLAN_PREFILL, ws)
        assert status == 0
        close(y, _cases.fused_expected(case))


def test_streamk_c5_shape_base_sampled(device):
    """c5's GEMM (2048 x 11008 x 4096, double quant) without adapters: 464 tiles on 256 CUs."""
    m, n, k = 2048, 11008, 4096
    rng = np.random.default_rng(736)
    case = _base_only(_cases.fused_case(m, n, k, ranks=(32,), double_quant=True, seed=736))
    x, q, st, _, _ = to_device(case, device)
    y = nf4_lora_linear(x, q, st)
    torch.cuda.synchronize()
    tokens = np.unique(np.concatenate([rng.choice(m, 24, replace=False), [0, 255, 256, m - 1]]))
    cols = np.unique(np.concatenate([rng.choice(n, 48, replace=False), [0, 191, 192, n - 1]]))
    sub = dict(case, x=case["x"][tokens], m=len(tokens))
    sub["lora"] = dict(case["lora"], token_slots=case["lora"]["token_slots"][tokens])
    close(bits(y)[np.ix_(tokens, cols)], _cases.fused_expected(sub, rows=cols))
