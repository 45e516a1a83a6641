"""Seeded random sweep of the fused NF4 + multi-LoRA call against the oracle.

Each case draws the batch (decode 1..64 and prefill 65..200 tokens), the
weight shape (multiples of 64), one to three slices with random bounds, one
to eight adapters with ranks from 0 to 64 (strides are the next power of
two), plain or double-quantised scales, bias, and the share of base-only
tokens; the output is held to the same tolerance as the other fused tests.
The seeds are fixed, so a failure names a reproducible case.
"""

import numpy as np
import pytest
import torch

from loraforge_amd.ops import nf4_lora_linear
from loraforge_amd.ops.fused import decode_status
from tests import _cases
from tests.test_fused_gpu import bits, close, to_device

pytestmark = pytest.mark.gpu

RANKS = [0, 1, 2, 3, 4, 7, 8, 15, 16, 17, 31, 32, 33, 48, 63, 64]


def draw(seed):
    rng = np.random.default_rng(seed)
    m = int(rng.integers(1, 65)) if seed % 3 else int(rng.integers(65, 201))
    slices = int(rng.integers(1, 4))
    n = 64 * int(rng.integers(slices, 9))
    k = 64 * int(rng.integers(1, 13))
    cuts = sorted(rng.choice(np.arange(1, n // 64), slices - 1, replace=False).tolist()) if slices > 1 else []
    bounds = [0] + [64 * c for c in cuts] + [n]
    ranks = tuple(int(r) for r in rng.choice(RANKS, int(rng.integers(1, 9))))
    return dict(
        m=m,
        n=n,
        k=k,
        ranks=ranks,
        slices=slices,
        bounds=bounds,
        double_quant=bool(rng.integers(0, 2)),
        bias=bool(rng.integers(0, 2)),
        null_frac=float(rng.choice([0.0, 0.1, 0.5])),
    )


@pytest.mark.parametrize("seed", range(24))
def test_random_case(seed, device):
    spec = draw(seed)
    m, n, k = spec.pop("m"), spec.pop("n"), spec.pop("k")
    print(f"[random] seed={seed} m={m} n={n} k={k} {spec}", flush=True)
    case = _cases.fused_case(m, n, k, seed=1000 + seed, **spec)
    x, q, st, lora, bias = to_device(case, device)
    y = nf4_lora_linear(x, q, st, bias=bias, lora=lora)
    torch.cuda.synchronize()
    close(bits(y), _cases.fused_expected(case))
    assert decode_status(device=device) == 0
