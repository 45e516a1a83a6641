"""Retained-rank compact layout of an SGLang LoRA pool, and its rank catalog.

Reference interface: ``src/loraforge/runtime/retained.py`` --
``read_rank_catalog`` (:17-92), ``effective_rank`` (:95-116) and
``RetainedLayout`` (:119-205), with the per-slot metadata names
(``rank / supported / unsupported / low / high / bucket``, ``boff``) that
the SGLang backend reads.

Two things are kept exactly because other code depends on them: the region
rule (per checkpoint, in catalog order: an 8-element aligned offset,
``bucket = next_pow2(k)``, and ``width * bucket`` elements reserved only when
``0 < k <= 64``; reference :146-154) and the fused-module name table of
``effective_rank``. Everything else is this module's own:

* the per-slot int32 fields are rows of one ``[6, slots]`` device matrix, so a
  load writes a slot's metadata with a single host->device copy;
* A is repacked with one gather (``index_select`` of each slice's first k
  rows) instead of per-slice copies;
* ``lora_batch`` hands the layout to ``nf4_lora_linear``: SGLang's padded A
  pool (``[slots, slices * capacity, K]``, repacked to ``s * k`` per slice) is
  exactly the fused kernels' A layout, and the compact B regions with their
  power-of-two strides are exactly their B layout, so the fused NF4 + LoRA
  projection runs on the layout without copying anything.
"""

from __future__ import annotations

import json
import re
from pathlib import Path
from typing import NamedTuple

from ..adapters.peft import CONFIG, WEIGHTS, read_safetensors, safetensors_header

# Modules whose LoRA factors share one fused projection (SGLang's stacking).
_FUSED = {
    "qkv_proj": {"qkv_proj", "q_proj", "k_proj", "v_proj"},
    "gate_up_proj": {"gate_up_proj", "gate_proj", "up_proj"},
    "in_proj_qkvz": {"in_proj_qkvz", "in_proj_qkv", "in_proj_q", "in_proj_k", "in_proj_v", "in_proj_z"},
    "in_proj_ba": {"in_proj_ba", "in_proj_b", "in_proj_a"},
}
_A_SUFFIX = ".lora_A.weight"
_B_SUFFIX = ".lora_B.weight"
COMPRESSION = "compression.json"


def bucket_of(k: int) -> int:
    """Smallest power of two >= k (1 for k <= 1)."""
    return 1 << (max(1, k) - 1).bit_length()


def _checkpoint_ranks(directory: Path) -> dict:
    """{A tensor key: retained rank} of one padded SGLang checkpoint."""
    config = json.loads((directory / CONFIG).read_text())
    rank = config.get("r")
    if type(rank) is not int or rank < 1:
        raise ValueError("invalid checkpoint rank")
    if config.get("rank_pattern") or config.get("alpha_pattern") or config.get("use_rslora"):
        raise ValueError("convert per-module rank/scaling to SGLang padding first")
    header = safetensors_header(directory / WEIGHTS)
    ranks = {}
    for key in (k for k in header if k.endswith(_A_SUFFIX)):
        partner = header.get(key[: -len(_A_SUFFIX)] + _B_SUFFIX)
        a_shape = header[key].get("shape")
        if not (isinstance(a_shape, list) and len(a_shape) == 2 and a_shape[0] == rank) or not (
            isinstance(partner, dict) and partner.get("shape") and partner["shape"][-1] == rank
        ):
            raise ValueError("native SGLang requires padded global-rank tensors")
        ranks[key] = rank
    if not ranks:
        raise ValueError("no linear LoRA A/B pairs found")
    metadata = directory / COMPRESSION
    if not metadata.exists():
        return ranks
    declared = json.loads(metadata.read_text())["module_ranks"]
    if set(declared) != set(ranks):
        raise ValueError("retained rank metadata must cover exactly the A tensors")
    if any(type(k) is not int or not 0 < k <= rank for k in declared.values()):
        raise ValueError("retained rank exceeds checkpoint rank")
    truncated = {key: k for key, k in declared.items() if k < rank}
    if truncated:
        tensors = read_safetensors(directory / WEIGHTS)
        for key, k in truncated.items():
            a, b = tensors[key], tensors[key[: -len(_A_SUFFIX)] + _B_SUFFIX]
            if a[k:].any() or b[:, k:].any():
                raise ValueError("retained-rank metadata truncates nonzero padded factors")
    return {key: declared[key] for key in ranks}


def read_rank_catalog(paths) -> dict:
    """{checkpoint directory: {A key: retained rank}} for local padded PEFT checkpoints.

    Ranks are the checkpoint rank unless a ``compression.json`` declares
    smaller retained ranks (whose padded tail must then be zero).
    """
    catalog = {str(Path(p).resolve()): _checkpoint_ranks(Path(p).resolve()) for p in paths}
    if not catalog:
        raise ValueError("a nonempty frozen adapter catalog is required")
    return catalog


def effective_rank(ranks: dict, name: str, layer: int) -> int:
    """Largest retained rank among the modules that fuse into projection ``name`` of ``layer``."""
    members = _FUSED.get(name, {name})
    layer_tag = re.compile(rf"\.layers\.{layer}\.")
    found = [r for key, r in ranks.items() if layer_tag.search(key) and key.split(".")[-3] in members]
    return max(found, default=0)


class Region(NamedTuple):
    offset: int  # element offset of the checkpoint's [width, bucket] block in ``store``
    bucket: int
    rank: int  # effective rank k


def plan_regions(catalog: dict, name: str, layer: int, width: int) -> tuple[dict, int]:
    """The frozen region of every catalog checkpoint and the store size in elements."""
    regions, end = {}, 0
    for path, ranks in catalog.items():
        k = effective_rank(ranks, name, layer)
        end = -(-end // 8) * 8
        regions[path] = Region(end, bucket_of(k), k)
        if 0 < k <= 64:
            end += width * bucket_of(k)
    return regions, end


def _capturing(device) -> bool:
    """Whether the current stream of a CUDA/ROCm device is being captured into a graph."""
    import torch

    return device.type == "cuda" and torch.cuda.is_current_stream_capturing()


class RetainedLayout:
    """Compact B regions and fixed per-slot metadata for one fused projection of an SGLang pool.

    ``a``: the pool's padded A buffer ``[slots, slices * capacity, K]``;
    ``b``: its padded B buffer ``[slots, width, capacity]`` (both bf16,
    contiguous, one device). Regions are frozen at construction from
    ``catalog``; ``load`` never reallocates, so every address stays fixed
    for graph replay. Loads are host-driven and must not race consumers.
    """

    FIELDS = ("rank", "supported", "unsupported", "low", "high", "bucket")

    def __init__(self, a, b, name, layer, catalog):
        import torch

        if a.ndim != 3 or b.ndim != 3 or a.dtype != torch.bfloat16 or b.dtype != a.dtype or a.device != b.device:
            raise ValueError("retained layout requires matching BF16 3D buffers")
        slots, width, capacity = b.shape
        if a.shape[0] != slots or capacity < 1 or a.shape[1] % capacity or not 1 <= a.shape[1] // capacity <= 4:
            raise ValueError("invalid fused A/B capacity")
        if not (a.is_contiguous() and b.is_contiguous()):
            raise ValueError("native buffers must be contiguous")
        self.a, self.b, self.name, self.layer = a, b, name, layer
        self.capacity, self.slices = capacity, a.shape[1] // capacity
        self.regions, size = plan_regions(catalog, name, layer, width)
        if any(region.rank > capacity for region in self.regions.values()):
            raise ValueError("effective rank exceeds native capacity")
        on = dict(device=b.device)
        self.store = torch.zeros(max(1, size), dtype=b.dtype, **on)
        self._fields = torch.zeros(len(self.FIELDS), slots, dtype=torch.int32, **on)
        for row, field in enumerate(self.FIELDS):
            setattr(self, field, self._fields[row])
        self.boff = torch.zeros(slots, dtype=torch.int64, **on)
        self.a_offsets = torch.arange(slots, dtype=torch.int64, **on) * (a.shape[1] * a.shape[2])
        ks = [region.rank for region in self.regions.values()]
        self.has_high = any(k > 16 for k in ks)
        self.has_unsupported = any(k > 64 for k in ks)
        self.max_rank = max([1] + [min(64, region.bucket) for region in self.regions.values()])
        self.loaded: dict = {}
        self._bounds: dict = {}  # slice_offsets tuple -> int32 device bounds (built once, eagerly)

    def validate_load(self, path, checkpoint_rank) -> None:
        if path is None:
            return
        if path not in self.regions:
            raise ValueError("checkpoint is absent from frozen rank catalog")
        if not self.regions[path].rank <= checkpoint_rank <= self.capacity:
            raise ValueError("checkpoint rank does not fit retained layout")

    def load(self, path, slot: int, checkpoint_rank: int = 0) -> None:
        """Point ``slot`` at checkpoint ``path`` (None: empty) after the native loader filled a/b[slot].

        A of the slot is repacked in place to the effective-rank prefix of
        each slice; B goes into the checkpoint's zero-padded compact region.
        """
        import torch

        self.validate_load(path, checkpoint_rank)
        if type(slot) is not int or not 0 <= slot < self.b.shape[0]:
            raise ValueError("slot out of range")
        offset, bucket, k = (0, 0, 0) if path is None else self.regions[path]
        if 0 < k != checkpoint_rank:
            rows = torch.arange(k, device=self.a.device)
            keep = torch.cat([rows + s * checkpoint_rank for s in range(self.slices)])
            self.a[slot, : self.slices * k] = self.a[slot].index_select(0, keep)
        if 0 < k <= 64:
            width = self.b.shape[1]
            block = self.store[offset : offset + width * bucket].view(width, bucket)
            block.zero_()
            block[:, :k] = self.b[slot, :, :k]
        low_rank = k <= 16
        values = [k, k if k <= 64 else 0, k if k > 64 else 0, k if low_rank else 0, 0 if low_rank else k, bucket]
        self._fields[:, slot].copy_(torch.tensor(values, dtype=torch.int32))
        self.boff[slot] = offset
        self.loaded[slot] = dict(path=path, rank=k, checkpoint_rank=checkpoint_rank)

    def lora_batch(self, token_slots, scales, *, slice_offsets=None):
        """A ``LoraBatch`` that runs ``nf4_lora_linear`` directly on this layout.

        ``scales``: fp32 per-slot scalings on the layout's device (SGLang's
        ``batch_info.scalings``); ``slice_offsets``: the output partition of
        the fused projection (default: ``slices`` equal parts of the width).
        Slots whose rank exceeds 64 are served by another path and are refused.
        The device copy of each distinct ``slice_offsets`` is built on its first
        (eager) call and reused, so later calls copy nothing from the host and
        may be captured; a partition first seen under capture is refused.
        """
        import torch

        from ..ops.fused import LoraBatch

        wide = sorted(slot for slot, info in self.loaded.items() if info["rank"] > 64)
        if wide:
            raise ValueError(f"slots {wide} hold ranks above 64, which the fused kernels do not take")
        width = self.b.shape[1]
        if slice_offsets is None:
            if width % self.slices:
                raise ValueError("pass slice_offsets: the width does not split evenly into slices")
            slice_offsets = [s * (width // self.slices) for s in range(self.slices + 1)]
        key = tuple(int(v) for v in slice_offsets)
        if len(key) != self.slices + 1:
            raise ValueError("slice_offsets must have slices + 1 entries")
        bounds = self._bounds.get(key)
        if bounds is None:
            if _capturing(self.b.device):
                raise RuntimeError("warm each projection's slice_offsets with an eager call before capturing")
            bounds = self._bounds[key] = torch.tensor(key, dtype=torch.int32, device=self.b.device)
        return LoraBatch(
            self.a.view(-1),
            self.a_offsets,
            self.store,
            self.boff,
            self.bucket,
            self.supported,
            scales,
            token_slots,
            bounds,
            self.max_rank,
        )
