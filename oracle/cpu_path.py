"""PyTorch-CPU restatement of the reference serving path. TEST INFRASTRUCTURE ONLY.

Used solely as ``bench.py``'s ``cpu_baseline`` leg. The reference has no CPU
path (its operators reject CPU tensors, ``tests/test_gemv_contracts.py``), so
this restates its per-call arithmetic on host cores, as planned in the
baseline notes:

1. NF4 dequantisation by the closed form on every call, no bf16 weight cache
   (``src/loraforge/integrations/_sglang_nf4_linear.py:1-7,116-129``):
   ``bf16(code[nibble] * scale[block])``;
2. ``F.linear`` in bf16 (fp32 accumulation inside the CPU GEMM);
3. LoRA grouped by adapter: ``z = bf16(x A_g^T)``, then
   ``y = bf16(y + bf16(scale_g * (z B_g^T)))`` with the expand product in fp32
   (``ops/csrc/lora_rows.cu:113`` rounding points).
"""

from __future__ import annotations


def make_inputs(batch, n, k, adapters, rank, *, seed=731, null_frac=0.1):
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(batch, k, generator=g).bfloat16()
    w = (torch.randn(n, k, generator=g) * 0.02).bfloat16()
    blocks = w.float().reshape(-1, 64)
    absmax = blocks.abs().amax(dim=1)
    from .nf4 import NF4_CODE

    code = torch.tensor(NF4_CODE.tolist(), dtype=torch.float32)
    mids = (code[:-1].double() + code[1:].double()).div(2).float()
    nib = torch.bucketize(blocks / absmax.clamp_min(1e-30)[:, None], mids, right=True).to(torch.uint8).reshape(-1)
    qweight = (nib[0::2] << 4) | nib[1::2]
    a = (torch.randn(adapters, rank, k, generator=g) * 0.02).bfloat16()
    b = (torch.randn(adapters, n, rank, generator=g) * 0.02).bfloat16()
    scales = torch.full((adapters,), 2.0)
    slots = torch.randint(0, adapters, (batch,), generator=g, dtype=torch.int32)
    slots[torch.rand(batch, generator=g) < null_frac] = -1
    return dict(x=x, qweight=qweight, absmax=absmax, code=code, shape=(n, k), a=a, b=b, scales=scales, slots=slots)


def reference_call(x, qweight, absmax, code, shape, a, b, scales, slots):
    """One call of the reference chain on the CPU; returns bf16 ``[B, N]``."""
    import torch
    import torch.nn.functional as F

    n, k = shape
    nib = torch.stack((qweight >> 4, qweight & 15), dim=1).reshape(-1).long()
    w = (code[nib] * absmax.repeat_interleave(64)).to(torch.bfloat16).view(n, k)
    y = F.linear(x, w)
    for g in torch.unique(slots).tolist():
        if g < 0:
            continue
        rows = (slots == g).nonzero().reshape(-1)
        z = x[rows] @ a[g].T
        delta = ((z.float() @ b[g].float().T) * float(scales[g])).bfloat16()
        y[rows] = (y[rows].float() + delta.float()).bfloat16()
    return y
