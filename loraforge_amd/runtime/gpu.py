"""Compact GPU residency with event-ordered copies and scoped stream leases.

Mirror of ``src/loraforge/runtime/gpu.py`` (``GPUAdapterSlots`` :25-186):
``load`` validates on the CPU, stages pinned copies and enqueues H2D copies on
the current stream of the pool device followed by a ready event; ``borrow``
makes the consumer's current stream wait on that event and records the stream
on every factor, so allocator reuse stays ordered after lease exit. Active
leases block replacement and eviction. Graph capture is rejected.

Each load allocates new storage, so factor addresses change across loads; the
fixed-address table the fused kernels read is ``runtime.table.AdapterTable``,
fed from ``borrow`` leases.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
from threading import RLock
from uuid import uuid4

from ..adapters import AdapterModule, load_peft_adapter
from .slots import AdapterSlots, SlotHandle, module_bytes


@dataclass
class _Resident:
    modules: tuple
    staging: tuple
    ready: object
    readers: int = 0


class GPUAdapterSlots:
    """Explicit GPU slots; use factors only inside ``borrow()`` on its current stream."""

    def __init__(self, capacity: int, *, device: str, max_tensor_bytes: int | None = None):
        import torch

        AdapterSlots(capacity, max_tensor_bytes=max_tensor_bytes)  # shared argument validation
        selected = torch.device(device)
        if selected.type != "cuda" or selected.index is None:
            raise ValueError("device must explicitly select a CUDA/ROCm GPU index")
        with torch.cuda.device(selected):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("GPU slots do not support graph capture")
        self.device = selected
        self._capacity = capacity
        self._limit = max_tensor_bytes
        self._id = uuid4().hex
        self._lock = RLock()
        self._generations = [0] * capacity
        self._entries: dict[int, _Resident] = {}
        self._pending: list[_Resident] = []

    def _slot(self, slot) -> None:
        if type(slot) is not int or not 0 <= slot < self._capacity:
            raise ValueError("slot outside pool capacity")

    def _entry(self, handle) -> _Resident:
        if not isinstance(handle, SlotHandle) or handle.pool != self._id:
            raise ValueError("handle belongs to a different pool")
        self._slot(handle.slot)
        if handle.generation != self._generations[handle.slot] or handle.slot not in self._entries:
            raise ValueError("stale or evicted slot handle")
        return self._entries[handle.slot]

    def _stream(self):
        import torch

        with torch.cuda.device(self.device):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("GPU slots do not support graph capture")
            return torch.cuda.current_stream(self.device)

    def _reap(self) -> None:
        self._pending = [e for e in self._pending if not e.ready.query()]
        for entry in self._entries.values():
            if entry.staging and entry.ready.query():
                entry.staging = ()

    @property
    def tensor_bytes(self) -> int:
        """Committed factor payload bytes, excluding staging and retired allocations."""
        with self._lock:
            return sum(module_bytes(e.modules) for e in self._entries.values())

    def load(self, source, slot: int) -> SlotHandle:
        """Validate on CPU, stage pinned copies, enqueue H2D on the pool stream.

        Failure preserves the previous occupant and generation.
        """
        import torch

        with self._lock:
            self._slot(slot)
            stream = self._stream()
            self._reap()
            old = self._entries.get(slot)
            if old is not None and old.readers:
                raise RuntimeError("slot has active leases")
            adapter = load_peft_adapter(source)
            size = module_bytes(adapter.modules)
            resident = self.tensor_bytes - (module_bytes(old.modules) if old else 0)
            if self._limit is not None and resident + size > self._limit:
                raise ValueError("resident tensor byte limit exceeded")
            staging, modules = [], []
            try:
                with torch.cuda.device(self.device), torch.cuda.stream(stream):
                    for module in adapter.modules:
                        host = AdapterModule(
                            module.name, module.a.pin_memory(), module.b.pin_memory(), module.alpha, module.use_rslora
                        )
                        staging.append(host)
                        modules.append(
                            AdapterModule(
                                host.name,
                                host.a.to(self.device, non_blocking=True),
                                host.b.to(self.device, non_blocking=True),
                                host.alpha,
                                host.use_rslora,
                            )
                        )
                    ready = torch.cuda.Event()
                    ready.record(stream)
            except BaseException:
                stream.synchronize()  # keep partial pinned buffers alive until copies end
                raise
            entry = _Resident(tuple(modules), tuple(staging), ready)
            if old is not None and old.staging:
                self._pending.append(old)
            self._entries[slot] = entry
            self._generations[slot] += 1
            return SlotHandle(self._id, slot, self._generations[slot])

    @contextmanager
    def borrow(self, handle: SlotHandle):
        """Lease read-only factors for work enqueued on the current pool-device stream."""
        with self._lock:
            stream = self._stream()
            self._reap()
            entry = self._entry(handle)
            stream.wait_event(entry.ready)
            for module in entry.modules:
                module.a.record_stream(stream)
                module.b.record_stream(stream)
            entry.readers += 1
        try:
            yield entry.modules
        finally:
            with self._lock:
                entry.readers -= 1

    def evict(self, handle: SlotHandle) -> None:
        """Invalidate residency; allocator stream tracking protects queued consumers."""
        with self._lock:
            self._stream()
            self._reap()
            entry = self._entry(handle)
            if entry.readers:
                raise RuntimeError("slot has active leases")
            if entry.staging:
                self._pending.append(entry)
            del self._entries[handle.slot]
            self._generations[handle.slot] += 1

    def collect(self) -> None:
        """Release completed pinned staging without waiting for GPU completion."""
        with self._lock:
            self._stream()
            self._reap()
