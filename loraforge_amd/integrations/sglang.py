"""Contract-level bridge from SGLang's LoRA batch metadata to one fused call per projection.

Reference interface: the Fleet backend's use of ``batch_info``
(``src/loraforge/integrations/_sglang_fleet.py:239-407``) -- ``seg_indptr``,
``weight_indices``, ``permutation``, ``scalings`` and the host-side
``num_segments`` -- and the NF4 ``_apply_4bit_weight`` hook
(``integrations/_sglang_nf4_linear.py:86-139``). The reference spends two
or three launches per projection (dequant + GEMM, shrink, expand); here the
same metadata drives a single ``nf4_lora_linear`` launch.

SGLang is not installed in this image, so this module touches only the
attributes named above (any object with them works, as the reference's own
tests do with ``SimpleNamespace``):

* segment ``s`` covers positions ``seg_indptr[s] .. seg_indptr[s + 1]`` of the
  permuted token order (position ``j`` holds token ``permutation[j]``, or
  token ``j`` when ``permutation`` is None) and routes them to adapter slot
  ``weight_indices[s]``;
* ``scalings[slot]`` is the slot's LoRA scaling.

``apply_lora`` does the same for a projection whose base output the caller
already holds (y updated in place by ``lora_apply``).

The per-token slot map is built on the device with a few tensor kernels and
no read-back (``num_segments`` is the host count SGLang keeps; under graph
capture it is a constant of the captured batch), into a caller-owned
buffer when one is given, so a captured graph keeps its address.
"""

from __future__ import annotations

from ..ops.fused import LoraBatch, lora_apply, nf4_lora_linear


def token_slots_from_batch_info(info, tokens: int, *, out=None):
    """int32 [tokens] slot of every token (-1: no adapter) from SGLang's segment metadata."""
    import torch

    seg_indptr = info.seg_indptr
    weight_indices = info.weight_indices
    device = seg_indptr.device
    nseg = int(info.num_segments)
    if type(tokens) is not int or tokens < 0:
        raise ValueError("tokens must be a nonnegative integer")
    if seg_indptr.dtype not in (torch.int32, torch.int64) or seg_indptr.ndim != 1 or seg_indptr.numel() < nseg + 1:
        raise ValueError("seg_indptr must be an integer vector of at least num_segments + 1 entries")
    if weight_indices.ndim != 1 or weight_indices.numel() < nseg or weight_indices.device != device:
        raise ValueError("weight_indices must hold one slot per segment on the metadata device")
    if out is None:
        out = torch.empty(tokens, dtype=torch.int32, device=device)
    elif out.dtype != torch.int32 or out.shape != (tokens,) or out.device != device or not out.is_contiguous():
        raise ValueError("out must be a contiguous int32 vector of one entry per token on the metadata device")
    out.fill_(-1)
    if tokens == 0 or nseg == 0:
        return out
    positions = torch.arange(tokens, dtype=seg_indptr.dtype, device=device)
    bounds = seg_indptr[: nseg + 1]
    seg = torch.searchsorted(bounds[1:].contiguous(), positions, right=True).clamp_(max=nseg - 1)
    inside = (positions >= bounds[0]) & (positions < bounds[nseg])
    slots = torch.where(inside, weight_indices[:nseg].to(torch.int32)[seg], torch.full_like(out, -1))
    permutation = getattr(info, "permutation", None)
    if permutation is None:
        out.copy_(slots)
    else:
        if permutation.ndim != 1 or permutation.numel() < tokens or permutation.device != device:
            raise ValueError("permutation must hold one token index per position on the metadata device")
        out.scatter_(0, permutation[:tokens].to(torch.int64), slots)
    return out


def lora_batch_from_batch_info(info, table, *, tokens: int, token_slots=None, slice_offsets=None) -> LoraBatch:
    """The ``LoraBatch`` of one projection for SGLang's current batch.

    ``table`` is a ``RetainedLayout`` over SGLang's own A/B pools (the layout
    the Fleet backend serves) or an ``AdapterTable``; slot scalings come from
    ``info.scalings``. ``token_slots`` is an optional int32 [tokens] buffer
    reused across calls (needed for graph capture).
    """
    from ..runtime import RetainedLayout

    slots = token_slots_from_batch_info(info, tokens, out=token_slots)
    scalings = getattr(info, "scalings", None)
    if isinstance(table, RetainedLayout):
        if scalings is None:
            raise ValueError("a retained layout takes its slot scalings from info.scalings")
        return table.lora_batch(slots, scalings, slice_offsets=slice_offsets)
    if slice_offsets is not None:
        raise ValueError("an AdapterTable carries its own slice offsets")
    batch = table.batch(slots)
    if scalings is not None:
        batch.scales = scalings
    return batch


def apply_nf4_lora(x, qweight, state, info, table, *, bias=None, out=None, token_slots=None, slice_offsets=None):
    """y = NF4 base linear + every token's LoRA for SGLang's batch, in one launch."""
    lora = lora_batch_from_batch_info(info, table, tokens=x.shape[0], token_slots=token_slots, slice_offsets=slice_offsets)
    return nf4_lora_linear(x, qweight, state, bias=bias, lora=lora, out=out)


def apply_lora(x, y, info, table, *, token_slots=None, slice_offsets=None):
    """``y += LoRA(x)`` in place for SGLang's batch, one launch per 64 tokens.

    For projections whose base output SGLang computes itself (unquantised
    layers): the Fleet backend's A pass then B pass over ``batch_info``
    (``integrations/_sglang_fleet.py:271-407``) as one ``lora_apply`` call on
    the same slot map.
    """
    lora = lora_batch_from_batch_info(info, table, tokens=x.shape[0], token_slots=token_slots, slice_offsets=slice_offsets)
    return lora_apply(x, y, lora)
