"""Adapter residency pools: slot ownership, handles and packed snapshots.

Reference interface: ``src/loraforge/runtime/slots.py`` (``SlotHandle``
:14-20, ``AdapterSlots`` :23-111); the behaviour its tests pin
(``tests/test_runtime_slots.py:40-144``) is kept: handles go stale when their
slot is reloaded or evicted, a failed load leaves the occupant and the byte
budget as they were, and resolved factors are private copies.

Every resident adapter is held as one packed snapshot: all of its A and B
factors in a single contiguous byte buffer, each factor at a 256-byte aligned
offset, with the modules as views into it. A snapshot is copied, pinned, moved
to a GPU and freed as one allocation (one host->device copy per adapter in
``GPUAdapterSlots``). ``SlotBook`` holds what the CPU and GPU pools share:
slot and handle checks, per-slot generations and the payload byte budget.
"""

from __future__ import annotations

from dataclasses import dataclass
from threading import RLock
from uuid import uuid4

from ..adapters import AdapterModule, load_peft_adapter

ALIGN = 256  # byte alignment of every factor inside a packed snapshot


@dataclass(frozen=True)
class SlotHandle:
    """Names one occupancy of one slot of one pool; stale once the slot is reloaded or evicted."""

    pool: str
    slot: int
    generation: int


@dataclass(frozen=True)
class Packed:
    """One adapter's factors in one byte buffer; ``modules`` view into ``buffer``."""

    buffer: object  # torch.uint8 [size]
    modules: tuple
    payload: int  # factor bytes, alignment padding excluded


def _factors(modules):
    for m in modules:
        yield m.a
        yield m.b


def _offsets(modules) -> tuple[list, int]:
    offsets, end = [], 0
    for t in _factors(modules):
        end = -(-end // ALIGN) * ALIGN
        offsets.append(end)
        end += t.numel() * t.element_size()
    return offsets, max(end, 1)


def _views(buffer, like, offsets) -> tuple:
    """Modules shaped like ``like`` whose factors view ``buffer`` at ``offsets``."""
    out, it = [], iter(offsets)
    for m in like:
        pair = []
        for t in (m.a, m.b):
            start = next(it)
            size = t.numel() * t.element_size()
            pair.append(buffer[start : start + size].view(t.dtype).view(t.shape))
        out.append(AdapterModule(m.name, pair[0], pair[1], m.alpha, m.use_rslora))
    return tuple(out)


def pack(modules, *, pin: bool = False) -> Packed:
    """Copy ``modules`` into a new packed snapshot in host memory (pinned on request)."""
    import torch

    offsets, size = _offsets(modules)
    buffer = torch.zeros(size, dtype=torch.uint8, pin_memory=pin)
    payload = 0
    for start, t in zip(offsets, _factors(modules)):
        raw = t.detach().contiguous().reshape(-1).view(torch.uint8)
        buffer[start : start + raw.numel()].copy_(raw)
        payload += raw.numel()
    return Packed(buffer, _views(buffer, modules, offsets), payload)


def repack(packed: Packed, buffer) -> Packed:
    """The snapshot ``packed`` over another buffer of the same size (a copy or a device image)."""
    offsets, _ = _offsets(packed.modules)
    return Packed(buffer, _views(buffer, packed.modules, offsets), packed.payload)


class SlotBook:
    """Slots, generations and the byte budget of one pool (callers hold ``lock``)."""

    def __init__(self, capacity, max_tensor_bytes):
        if type(capacity) is not int or capacity <= 0:
            raise ValueError("capacity must be a positive integer")
        if max_tensor_bytes is not None and (type(max_tensor_bytes) is not int or max_tensor_bytes < 0):
            raise ValueError("max_tensor_bytes must be a nonnegative integer")
        self.capacity = capacity
        self.limit = max_tensor_bytes
        self.pool_id = uuid4().hex
        self.lock = RLock()
        self.generation = [0] * capacity
        self.occupant: dict = {}  # slot -> entry with a ``payload`` attribute

    def check_slot(self, slot) -> None:
        if type(slot) is not int or not 0 <= slot < self.capacity:
            raise ValueError("slot outside pool capacity")

    def entry(self, handle):
        if not isinstance(handle, SlotHandle) or handle.pool != self.pool_id:
            raise ValueError("handle belongs to a different pool")
        self.check_slot(handle.slot)
        if handle.generation != self.generation[handle.slot] or handle.slot not in self.occupant:
            raise ValueError("stale or evicted slot handle")
        return self.occupant[handle.slot]

    def payload(self) -> int:
        return sum(e.payload for e in self.occupant.values())

    def admit(self, slot: int, payload: int) -> None:
        """Raise unless ``payload`` bytes fit the budget once ``slot``'s occupant is gone."""
        if self.limit is None:
            return
        current = self.occupant.get(slot)
        others = self.payload() - (current.payload if current is not None else 0)
        if others + payload > self.limit:
            raise ValueError("resident tensor byte limit exceeded")

    def install(self, slot: int, entry):
        """Make ``entry`` the occupant of ``slot``; returns (new handle, previous occupant)."""
        previous = self.occupant.get(slot)
        self.occupant[slot] = entry
        self.generation[slot] += 1
        return SlotHandle(self.pool_id, slot, self.generation[slot]), previous

    def remove(self, handle):
        entry = self.entry(handle)
        del self.occupant[handle.slot]
        self.generation[handle.slot] += 1
        return entry


class AdapterSlots:
    """A bounded pool of CPU adapter snapshots in explicitly chosen slots (thread-safe)."""

    def __init__(self, capacity: int, *, max_tensor_bytes: int | None = None):
        self._book = SlotBook(capacity, max_tensor_bytes)

    @property
    def tensor_bytes(self) -> int:
        """Factor payload bytes held by the pool."""
        with self._book.lock:
            return self._book.payload()

    def load(self, source, slot: int) -> SlotHandle:
        """Read the adapter directory ``source`` into ``slot``; a failure changes nothing."""
        book = self._book
        with book.lock:
            book.check_slot(slot)
            snapshot = pack(load_peft_adapter(source).modules)
            book.admit(slot, snapshot.payload)
            handle, _ = book.install(slot, snapshot)
            return handle

    def resolve(self, handle: SlotHandle) -> tuple:
        """Private copies of the modules held under ``handle``."""
        with self._book.lock:
            snapshot = self._book.entry(handle)
            return repack(snapshot, snapshot.buffer.clone()).modules

    def evict(self, handle: SlotHandle) -> None:
        with self._book.lock:
            self._book.remove(handle)
