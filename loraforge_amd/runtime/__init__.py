"""Adapter residency and fixed-address slot tables (mirror of ``loraforge.runtime``)."""

from .gpu import GPUAdapterSlots
from .retained import RetainedLayout, effective_rank, read_rank_catalog
from .slots import AdapterSlots, SlotHandle
from .table import AdapterTable

__all__ = [
    "AdapterSlots",
    "AdapterTable",
    "GPUAdapterSlots",
    "RetainedLayout",
    "SlotHandle",
    "effective_rank",
    "read_rank_catalog",
]
