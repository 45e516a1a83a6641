"""Fixed-address adapter table for one projection, read by ``nf4_lora_linear``.

The reference documents that ``GPUAdapterSlots`` reallocates on every load,
so it cannot by itself serve captured graphs (``docs/row-operators.md:82-84``);
its SGLang pools solve that with ``RetainedLayout`` (``runtime/retained.py:119-205``).
``AdapterTable`` does it for adapters published from ``GPUAdapterSlots``:

* Two device stores whose addresses never change: A (bf16 rows of width K)
  and B (bf16). Each published slot owns a compact region in each: exactly
  ``num_slices * r`` A rows, packed at ``s * r`` per slice, and a
  ``[N, bucket(r)]`` B block zero padded past ``r``. Regions are carved from
  the stores by a first-fit allocator on the host (8-element aligned, freed
  regions merge with their neighbours), so ragged ranks cost what they hold:
  128 adapters of ranks {4 .. 64} at 4096 x 4096 take about 52 MB rather than
  the 134 MB of rank-64 padding.
* Per-slot metadata in device vectors (A and B offsets, B stride, rank,
  scale); the kernels read them at run time, so a graph captured once sees
  every later publish at the same addresses.

``publish`` and ``clear`` enqueue their device writes on the current stream.
The table is meant to be used from one stream (the one the projections run
on): a region freed by one publish may be rewritten by the next, which stream
order places after every earlier reader on that stream.
"""

from __future__ import annotations

from bisect import insort
from contextlib import nullcontext

from ..ops.fused import LoraBatch
from .retained import bucket_of

_ALIGN = 8  # elements: 16-byte aligned regions, as the kernels' 16-byte loads need


class RegionAllocator:
    """First-fit ranges of a fixed-size store (host bookkeeping, in elements)."""

    def __init__(self, size: int):
        self.size = size
        self._free = [(0, size)]  # sorted (start, length), never adjacent

    @staticmethod
    def _round(n: int) -> int:
        return -(-n // _ALIGN) * _ALIGN

    def take(self, n: int) -> int | None:
        n = self._round(max(n, 1))
        for i, (start, length) in enumerate(self._free):
            if length >= n:
                if length == n:
                    del self._free[i]
                else:
                    self._free[i] = (start + n, length - n)
                return start
        return None

    def give(self, start: int, n: int) -> None:
        n = self._round(max(n, 1))
        insort(self._free, (start, n))
        merged = []
        for s, length in self._free:
            if merged and merged[-1][0] + merged[-1][1] == s:
                merged[-1] = (merged[-1][0], merged[-1][1] + length)
            else:
                merged.append((s, length))
        self._free = merged

    def claim(self, start: int, n: int) -> None:
        """Take the given range back (it must lie inside one free range)."""
        n = self._round(max(n, 1))
        for i, (s, length) in enumerate(self._free):
            if s <= start and start + n <= s + length:
                pieces = [(s, start - s), (start + n, s + length - start - n)]
                self._free[i : i + 1] = [(a, b) for a, b in pieces if b > 0]
                return
        raise ValueError("range is not free")

    @property
    def free(self) -> int:
        return sum(length for _, length in self._free)


class AdapterTable:
    """Fixed-address A/B stores and slot metadata for one (possibly fused) projection.

    ``a_elements`` / ``b_elements`` size the stores; by default they hold
    every slot at ``max_rank``, so a publish never runs out of room. Pass the
    sum over the adapters that will be resident (``region_elements``) for a
    compact table.
    """

    def __init__(
        self,
        capacity: int,
        *,
        in_features: int,
        out_features: int,
        max_rank: int = 64,
        slice_offsets=None,
        device,
        a_elements: int | None = None,
        b_elements: int | None = None,
    ):
        import torch

        if type(capacity) is not int or capacity < 1:
            raise ValueError("capacity must be a positive integer")
        if type(max_rank) is not int or not 1 <= max_rank <= 64:
            raise ValueError("max_rank must be in 1..64")
        if in_features % 8 or in_features <= 0 or out_features <= 0:
            raise ValueError("in_features must be a positive multiple of 8")
        bounds = list(slice_offsets) if slice_offsets is not None else [0, out_features]
        if bounds[0] != 0 or bounds[-1] != out_features or any(lo >= hi for lo, hi in zip(bounds, bounds[1:])):
            raise ValueError("slice_offsets must increase from 0 to out_features")
        if not 1 <= len(bounds) - 1 <= 3:
            raise ValueError("one to three slices are supported")
        self.capacity = capacity
        self.in_features = in_features
        self.out_features = out_features
        self.max_rank = max_rank
        self.num_slices = len(bounds) - 1
        self.bounds = bounds
        worst_a, worst_b = self.region_elements(max_rank)
        a_size = capacity * worst_a if a_elements is None else int(a_elements)
        b_size = capacity * worst_b if b_elements is None else int(b_elements)
        if a_size < 1 or b_size < 1:
            raise ValueError("store sizes must be positive")
        self.device = torch.device(device)
        on = dict(device=self.device)
        self.a_store = torch.zeros(a_size, dtype=torch.bfloat16, **on)
        self.b_store = torch.zeros(b_size, dtype=torch.bfloat16, **on)
        self.a_offsets = torch.zeros(capacity, dtype=torch.int64, **on)
        self.b_offsets = torch.zeros(capacity, dtype=torch.int64, **on)
        self.b_strides = torch.ones(capacity, dtype=torch.int32, **on)
        self.ranks = torch.zeros(capacity, dtype=torch.int32, **on)
        self.scales = torch.zeros(capacity, dtype=torch.float32, **on)
        self.slice_offsets = torch.tensor(bounds, dtype=torch.int32, **on)
        self._a_regions = RegionAllocator(a_size)
        self._b_regions = RegionAllocator(b_size)
        self._held: list = [None] * capacity  # slot -> (a_start, a_len, b_start, b_len, rank)
        self.names: list = [None] * capacity

    def region_elements(self, rank: int) -> tuple[int, int]:
        """(A, B) store elements one slot of ``rank`` occupies."""
        return self.num_slices * rank * self.in_features, self.out_features * bucket_of(rank)

    def _check_slot(self, slot) -> None:
        if type(slot) is not int or not 0 <= slot < self.capacity:
            raise ValueError("slot outside table capacity")

    def _release(self, slot: int) -> None:
        held = self._held[slot]
        if held is not None:
            a_start, a_len, b_start, b_len, _ = held
            self._a_regions.give(a_start, a_len)
            self._b_regions.give(b_start, b_len)
            self._held[slot] = None

    def _reserve(self, slot: int, rank: int) -> tuple[int, int]:
        """Regions for ``slot`` at ``rank`` (its old regions count as free); on failure nothing changes."""
        a_len, b_len = self.region_elements(rank)
        previous = self._held[slot]
        self._release(slot)
        a_start = self._a_regions.take(a_len)
        b_start = self._b_regions.take(b_len) if a_start is not None else None
        if b_start is None:
            if a_start is not None:
                self._a_regions.give(a_start, a_len)
            if previous is not None:  # the old occupant keeps its regions, untouched
                self._a_regions.claim(previous[0], previous[1])
                self._b_regions.claim(previous[2], previous[3])
                self._held[slot] = previous
            raise ValueError("adapter table store is full: size a_elements / b_elements for the resident adapters")
        self._held[slot] = (a_start, a_len, b_start, b_len, rank)
        return a_start, b_start

    def publish(self, slot: int, modules) -> None:
        """Copy one adapter (one ``AdapterModule`` per slice) into ``slot``.

        The copies are enqueued on the current stream; call it inside
        ``GPUAdapterSlots.borrow`` so they are ordered after the adapter's load.
        """
        import torch

        self._check_slot(slot)
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
        a_start, b_start = self._reserve(slot, r)
        bucket = bucket_of(r)
        k, n = self.in_features, self.out_features
        with torch.cuda.device(self.device) if self.device.type == "cuda" else nullcontext():
            a_view = self.a_store[a_start : a_start + self.num_slices * r * k].view(self.num_slices, r, k)
            b_view = self.b_store[b_start : b_start + n * bucket].view(n, bucket)
            if bucket > r:
                b_view[:, r:].zero_()
            for s, m in enumerate(modules):
                a_view[s].copy_(m.a, non_blocking=True)
                b_view[self.bounds[s] : self.bounds[s + 1], :r].copy_(m.b, non_blocking=True)
            self._write_meta(slot, a_start, b_start, bucket, r, float(modules[0].scaling))
        self.names[slot] = tuple(m.name for m in modules)

    def _write_meta(self, slot, a_off, b_off, stride, rank, scale) -> None:
        import torch

        offsets = torch.tensor([a_off, b_off], dtype=torch.int64)
        small = torch.tensor([stride, rank], dtype=torch.int32)
        self.a_offsets[slot : slot + 1].copy_(offsets[:1])
        self.b_offsets[slot : slot + 1].copy_(offsets[1:])
        self.b_strides[slot : slot + 1].copy_(small[:1])
        self.ranks[slot : slot + 1].copy_(small[1:])
        self.scales[slot : slot + 1].fill_(scale)

    def publish_from(self, pool, handle, slot: int, names) -> None:
        """Borrow ``handle`` from a ``GPUAdapterSlots`` pool and publish modules ``names``."""
        with pool.borrow(handle) as modules:
            by_name = {m.name: m for m in modules}
            missing = [n for n in names if n not in by_name]
            if missing:
                raise ValueError(f"adapter lacks modules: {missing}")
            self.publish(slot, [by_name[n] for n in names])

    def clear(self, slot: int) -> None:
        """Make ``slot`` inactive (rank 0: its tokens get the base output) and free its regions."""
        self._check_slot(slot)
        self.ranks[slot : slot + 1].fill_(0)
        self._release(slot)
        self.names[slot] = None

    def region_of(self, slot: int):
        """(a_offset, b_offset, rank) of a published slot, from host bookkeeping; None if empty."""
        self._check_slot(slot)
        held = self._held[slot]
        return None if held is None else (held[0], held[2], held[4])

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

