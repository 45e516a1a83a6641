"""Fixed-address adapter table for one projection, read by ``nf4_lora_linear``.

The reference documents that ``GPUAdapterSlots`` reallocates on every load,
so it cannot by itself serve captured graphs (``docs/row-operators.md:82-84``);
``RetainedLayout`` (``runtime/retained.py:119-205``) solves it for the SGLang
pools. ``AdapterTable`` is the same idea for the fused kernels: every slot
owns a preallocated A region (``num_slices * max_rank`` rows of width K) and a
compact B region (``[N, bucket(max_rank)]``), and the per-slot metadata
(ranks, B strides, scales, offsets) lives in device vectors whose addresses
never change. ``publish`` copies a borrowed adapter into a slot on the
current stream (A packed at ``s * r``, B zero padded to ``bucket(r)``), so a
captured graph sees new adapters at the same addresses.
"""

from __future__ import annotations

from ..ops.fused import LoraBatch
from .retained import bucket_of


class AdapterTable:
    def __init__(self, capacity: int, *, in_features: int, out_features: int, max_rank: int = 64, slice_offsets=None, device):
        import torch

        if type(capacity) is not int or capacity < 1:
            raise ValueError("capacity must be a positive integer")
        if type(max_rank) is not int or not 1 <= max_rank <= 64:
            raise ValueError("max_rank must be in 1..64")
        if in_features % 8 or in_features <= 0 or out_features <= 0:
            raise ValueError("in_features must be a positive multiple of 8")
        self.device = torch.device(device)
        bounds = list(slice_offsets) if slice_offsets is not None else [0, out_features]
        if bounds[0] != 0 or bounds[-1] != out_features or any(a >= b for a, b in zip(bounds, bounds[1:])):
            raise ValueError("slice_offsets must increase from 0 to out_features")
        if not 1 <= len(bounds) - 1 <= 3:
            raise ValueError("one to three slices are supported")
        self.capacity = capacity
        self.in_features = in_features
        self.out_features = out_features
        self.max_rank = max_rank
        self.num_slices = len(bounds) - 1
        self.bounds = bounds
        self.a_rows = self.num_slices * max_rank
        self.b_width = bucket_of(max_rank)
        kw = dict(device=self.device)
        self.a_store = torch.zeros(capacity * self.a_rows * in_features, dtype=torch.bfloat16, **kw)
        self.b_store = torch.zeros(capacity * out_features * self.b_width, dtype=torch.bfloat16, **kw)
        self.a_offsets = torch.arange(capacity, dtype=torch.int64, **kw) * (self.a_rows * in_features)
        self.b_offsets = torch.arange(capacity, dtype=torch.int64, **kw) * (out_features * self.b_width)
        self.b_strides = torch.ones(capacity, dtype=torch.int32, **kw)
        self.ranks = torch.zeros(capacity, dtype=torch.int32, **kw)
        self.scales = torch.zeros(capacity, dtype=torch.float32, **kw)
        self.slice_offsets = torch.tensor(bounds, dtype=torch.int32, **kw)
        self.names: list = [None] * capacity

    def _slot(self, slot) -> None:
        if type(slot) is not int or not 0 <= slot < self.capacity:
            raise ValueError("slot outside table capacity")

    def publish(self, slot: int, modules) -> None:
        """Copy one adapter (one ``AdapterModule`` per slice) into ``slot``.

        The copies are enqueued on the current stream; use inside
        ``GPUAdapterSlots.borrow`` so they are ordered after the H2D load.
        """
        import torch

        self._slot(slot)
        modules = list(modules)
        if len(modules) != self.num_slices:
            raise ValueError("one module per slice is required")
        r = modules[0].rank
        if any(m.rank != r for m in modules) or not 1 <= r <= self.max_rank:
            raise ValueError("slice ranks must agree and fit max_rank")
        if any(abs(m.scaling - modules[0].scaling) > 1e-12 * max(1.0, abs(m.scaling)) for m in modules):
            raise ValueError("slices of one slot must share a scaling")
        for s, m in enumerate(modules):
            if m.a.shape != (r, self.in_features) or m.b.shape != (self.bounds[s + 1] - self.bounds[s], r):
                raise ValueError("factor shapes disagree with the table")
        bucket = bucket_of(r)
        with torch.cuda.device(self.device):
            a_base = slot * self.a_rows * self.in_features
            a_view = self.a_store[a_base : a_base + self.num_slices * r * self.in_features].view(self.num_slices * r, self.in_features)
            b_base = slot * self.out_features * self.b_width
            b_view = self.b_store[b_base : b_base + self.out_features * bucket].view(self.out_features, bucket)
            b_view.zero_()
            for s, m in enumerate(modules):
                a_view[s * r : (s + 1) * r].copy_(m.a, non_blocking=True)
                b_view[self.bounds[s] : self.bounds[s + 1], :r].copy_(m.b, non_blocking=True)
            self.ranks[slot] = r
            self.b_strides[slot] = bucket
            self.scales[slot] = float(modules[0].scaling)
        self.names[slot] = tuple(m.name for m in modules)

    def publish_from(self, pool, handle, slot: int, names) -> None:
        """Borrow ``handle`` from a ``GPUAdapterSlots`` pool and publish modules ``names``."""
        with pool.borrow(handle) as modules:
            by_name = {m.name: m for m in modules}
            missing = [n for n in names if n not in by_name]
            if missing:
                raise ValueError(f"adapter lacks modules: {missing}")
            self.publish(slot, [by_name[n] for n in names])

    def clear(self, slot: int) -> None:
        """Mark ``slot`` inactive (rank 0); tokens routed to it get the base output."""
        self._slot(slot)
        self.ranks[slot] = 0
        self.names[slot] = None

    def batch(self, token_slots) -> LoraBatch:
        return LoraBatch(
            self.a_store,
            self.a_offsets,
            self.b_store,
            self.b_offsets,
            self.b_strides,
            self.ranks,
            self.scales,
            token_slots,
            self.slice_offsets,
            self.max_rank,
        )
