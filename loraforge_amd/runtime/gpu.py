"""GPU adapter residency: one packed device image per adapter, leases on streams.

Reference interface: ``src/loraforge/runtime/gpu.py`` (``GPUAdapterSlots``
:25-186, constructor, ``load``, ``borrow``, ``evict``, ``collect``,
``tensor_bytes``); the behaviour its tests pin
(``tests/test_runtime_gpu.py:45-140``) is kept: a load is ordered before the
consumers of the borrowing stream, active leases block reload and eviction,
handles go stale, graph capture is refused and the caller's current device is
left alone.

How residency works here:

* ``load`` reads and validates the adapter on the CPU, packs all of its
  factors into one pinned host buffer (``slots.pack``), and enqueues ONE
  host->device copy into ONE device buffer on the pool device's current
  stream, followed by a ready event. The resident modules are views of that
  buffer.
* ``borrow`` makes the caller's current stream wait for the ready event and,
  when the lease ends, records a "last use" event on that stream.
* A replaced or evicted image is retired, not freed: it stays referenced
  until its ready event and every last-use event have completed (checked on
  each pool call and by ``collect``), so device memory is never handed back
  to the allocator while a queued consumer may still read it. When the pool
  itself goes away, its finalizer waits for those events.

Factor addresses change from load to load; the fixed-address table that the
fused kernels and captured graphs read is ``runtime.table.AdapterTable``,
filled from ``borrow`` leases.
"""

from __future__ import annotations

import weakref
from contextlib import contextmanager
from dataclasses import dataclass, field

from ..adapters import load_peft_adapter
from .slots import Packed, SlotBook, SlotHandle, pack, repack


@dataclass
class _Image:
    """One resident adapter: device buffer + module views, its pinned staging and events."""

    device: Packed
    staging: Packed | None
    ready: object
    leases: int = 0
    uses: list = field(default_factory=list)

    @property
    def payload(self) -> int:
        return self.device.payload

    @property
    def modules(self) -> tuple:
        return self.device.modules

    def settle(self) -> bool:
        """Drop what has completed; True once nothing queued can still touch the image."""
        if not self.ready.query():
            return False
        self.staging = None
        self.uses = [e for e in self.uses if not e.query()]
        return not self.uses and self.leases == 0


def _wait_all(*groups) -> None:
    for images in groups:
        for image in list(images):
            image.ready.synchronize()
            for event in image.uses:
                event.synchronize()


class GPUAdapterSlots:
    """Explicit GPU slots; use the factors only inside ``borrow()``, on its current stream."""

    def __init__(self, capacity: int, *, device: str, max_tensor_bytes: int | None = None):
        import torch

        self._book = SlotBook(capacity, max_tensor_bytes)
        selected = torch.device(device)
        if selected.type != "cuda" or selected.index is None:
            raise ValueError("device must explicitly select a GPU index, e.g. 'cuda:0'")
        self.device = selected
        self._stream()  # refuses construction under capture
        self._retired: list = []
        finalizer = weakref.finalize(self, _wait_all, self._retired, self._book.occupant.values())
        finalizer.atexit = False  # at interpreter exit the process releases the device anyway

    def _stream(self):
        import torch

        with torch.cuda.device(self.device):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("GPU slots do not support graph capture")
            return torch.cuda.current_stream(self.device)

    def _reap(self) -> None:
        for image in self._book.occupant.values():
            image.settle()
        self._retired[:] = [image for image in self._retired if not image.settle()]

    def _retire(self, image: _Image) -> None:
        if not image.settle():
            self._retired.append(image)

    @property
    def tensor_bytes(self) -> int:
        """Factor payload bytes resident on the device (staging and retired images excluded)."""
        with self._book.lock:
            return self._book.payload()

    def load(self, source, slot: int) -> SlotHandle:
        """Validate on the CPU, then one pinned host->device copy on the current stream.

        On failure the slot keeps its occupant, handle and budget.
        """
        import torch

        book = self._book
        with book.lock:
            book.check_slot(slot)
            stream = self._stream()
            self._reap()
            current = book.occupant.get(slot)
            if current is not None and current.leases:
                raise RuntimeError("slot has active leases")
            host = pack(load_peft_adapter(source).modules, pin=True)
            book.admit(slot, host.payload)
            with torch.cuda.device(self.device), torch.cuda.stream(stream):
                try:
                    buffer = torch.empty_like(host.buffer, device=self.device)
                    buffer.copy_(host.buffer, non_blocking=True)
                    ready = torch.cuda.Event()
                    ready.record(stream)
                except BaseException:
                    stream.synchronize()  # the pinned source must outlive a copy already queued
                    raise
            image = _Image(repack(host, buffer), host, ready)
            handle, previous = book.install(slot, image)
            if previous is not None:
                self._retire(previous)
            return handle

    @contextmanager
    def borrow(self, handle: SlotHandle):
        """Lease the modules of ``handle`` for work enqueued on the current stream."""
        import torch

        book = self._book
        with book.lock:
            stream = self._stream()
            self._reap()
            image = book.entry(handle)
            stream.wait_event(image.ready)
            image.leases += 1
        try:
            yield image.modules
        finally:
            with book.lock:
                with torch.cuda.device(self.device):
                    done = torch.cuda.Event()
                    done.record(stream)
                image.uses.append(done)
                image.leases -= 1

    def evict(self, handle: SlotHandle) -> None:
        """End residency; the image is released once queued consumers are done with it."""
        book = self._book
        with book.lock:
            self._stream()
            self._reap()
            if book.entry(handle).leases:
                raise RuntimeError("slot has active leases")
            self._retire(book.remove(handle))

    def collect(self) -> None:
        """Release staging buffers and retired images whose work has completed (never waits)."""
        with self._book.lock:
            self._stream()
            self._reap()
