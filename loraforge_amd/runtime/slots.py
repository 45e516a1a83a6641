"""Synchronous CPU residency with generation-checked slot reuse.

Mirror of ``src/loraforge/runtime/slots.py`` (``SlotHandle`` :14-20,
``AdapterSlots`` :23-111): a bounded pool of explicitly managed slots holding
compact CPU snapshots. A failed load keeps the previous occupant and handle;
replacement or eviction bumps the slot generation so old handles turn stale.
"""

from __future__ import annotations

from dataclasses import dataclass
from threading import RLock
from uuid import uuid4

from ..adapters import AdapterModule, load_peft_adapter


@dataclass(frozen=True)
class SlotHandle:
    """Opaque ownership token; valid only in its originating pool generation."""

    pool: str
    slot: int
    generation: int


def module_bytes(modules) -> int:
    return sum(t.numel() * t.element_size() for m in modules for t in (m.a, m.b))


class AdapterSlots:
    """Own compact CPU snapshots in a bounded number of slots (serialised by a lock)."""

    def __init__(self, capacity: int, *, max_tensor_bytes: int | None = None):
        if type(capacity) is not int or capacity <= 0:
            raise ValueError("capacity must be a positive integer")
        if max_tensor_bytes is not None and (type(max_tensor_bytes) is not int or max_tensor_bytes < 0):
            raise ValueError("max_tensor_bytes must be a nonnegative integer")
        self._capacity = capacity
        self._limit = max_tensor_bytes
        self._id = uuid4().hex
        self._lock = RLock()
        self._generations = [0] * capacity
        self._entries: dict[int, tuple] = {}

    def _slot(self, slot) -> None:
        if type(slot) is not int or not 0 <= slot < self._capacity:
            raise ValueError("slot outside pool capacity")

    def _check(self, handle) -> None:
        if not isinstance(handle, SlotHandle) or handle.pool != self._id:
            raise ValueError("handle belongs to a different pool")
        self._slot(handle.slot)
        if handle.generation != self._generations[handle.slot] or handle.slot not in self._entries:
            raise ValueError("stale or evicted slot handle")

    @staticmethod
    def _clone(modules) -> tuple:
        return tuple(
            AdapterModule(m.name, m.a.detach().clone().contiguous(), m.b.detach().clone().contiguous(), m.alpha, m.use_rslora)
            for m in modules
        )

    @property
    def tensor_bytes(self) -> int:
        with self._lock:
            return sum(module_bytes(mods) for mods in self._entries.values())

    def load(self, source, slot: int) -> SlotHandle:
        with self._lock:
            self._slot(slot)
            modules = self._clone(load_peft_adapter(source).modules)
            resident = self.tensor_bytes - module_bytes(self._entries.get(slot, ()))
            if self._limit is not None and resident + module_bytes(modules) > self._limit:
                raise ValueError("resident tensor byte limit exceeded")
            self._entries[slot] = modules
            self._generations[slot] += 1
            return SlotHandle(self._id, slot, self._generations[slot])

    def resolve(self, handle: SlotHandle) -> tuple:
        with self._lock:
            self._check(handle)
            return self._clone(self._entries[handle.slot])

    def evict(self, handle: SlotHandle) -> None:
        with self._lock:
            self._check(handle)
            del self._entries[handle.slot]
            self._generations[handle.slot] += 1
