"""PEFT adapter directories (``adapter_config.json`` + ``adapter_model.safetensors``).

Reference interface: ``src/loraforge/adapters/peft.py`` -- ``AdapterModule``
(:42-57), ``PeftAdapter`` (:60-67), ``load_peft_adapter`` (:124-198) and the
``loraforge_manifest.json`` integrity record (:98-121); the file names, the
manifest schema and the error fragments the reference's tests match on
(``rank``, ``bias``, ``integrity``, ``stale`` ...) are the contract kept here.

How a directory is read: each file is read into memory exactly once. Its
sha256 is taken over those bytes, a manifest (when present) is compared with
them, and the factors are cut out of the same bytes by the safetensors parser
below (8-byte little-endian header length, a JSON header of dtype / shape /
data_offsets, then the raw little-endian data, fully covered by the tensors).
So the tensors always come from exactly the bytes that were hashed, and no
second pass over the files is needed to notice a concurrent rewrite. Nothing
in the files is executed: JSON and raw tensor bytes only.
"""

from __future__ import annotations

import hashlib
import json
import math
import re
from dataclasses import dataclass
from pathlib import Path

CONFIG = "adapter_config.json"
WEIGHTS = "adapter_model.safetensors"
MANIFEST = "loraforge_manifest.json"
_FACTOR_KEY = re.compile(r"base_model\.model\.(?P<module>.+)\.lora_(?P<side>[AB])\.weight")
_MAX_HEADER = 64 << 20


@dataclass(frozen=True)
class AdapterModule:
    """One LoRA pair: ``delta = scaling * b @ a`` with ``a`` [rank, in] and ``b`` [out, rank]."""

    name: str
    a: object
    b: object
    alpha: float
    use_rslora: bool = False

    @property
    def rank(self) -> int:
        return self.a.shape[0]

    @property
    def scaling(self) -> float:
        return self.alpha / (math.sqrt(self.rank) if self.use_rslora else self.rank)


@dataclass(frozen=True)
class PeftAdapter:
    """A CPU snapshot of one adapter directory (treat it as read-only)."""

    source: Path
    config: dict
    modules: tuple
    source_sha256: dict


def _json_object(raw: bytes, what: str) -> dict:
    """A JSON object whose keys are unique (a repeated key would hide a value)."""

    def no_repeats(pairs):
        keys = [k for k, _ in pairs]
        if len(set(keys)) != len(keys):
            dup = next(k for k in keys if keys.count(k) > 1)
            raise ValueError(f"duplicate JSON key in {what}: {dup}")
        return dict(pairs)

    try:
        value = json.loads(raw.decode("utf-8"), object_pairs_hook=no_repeats)
    except UnicodeDecodeError as exc:
        raise ValueError(f"{what} is not UTF-8 JSON") from exc
    if not isinstance(value, dict):
        raise ValueError(f"{what} must contain a JSON object")
    return value


def _positive_int(value, what: str) -> int:
    if type(value) is not int or value < 1:
        raise ValueError(f"{what} must be a positive integer")
    return value


def _finite(value, what: str) -> float:
    if isinstance(value, bool) or not isinstance(value, (int, float)) or not math.isfinite(value):
        raise ValueError(f"{what} must be a finite number")
    return float(value)


def _validate_config(config: dict) -> None:
    if config.get("peft_type", "LORA") != "LORA":
        raise ValueError("only LoRA adapters are supported")
    _positive_int(config.get("r"), "config rank r")
    _finite(config.get("lora_alpha"), "config lora_alpha")
    if config.get("bias", "none") != "none":
        raise ValueError("only bias='none' adapters are supported")
    if not isinstance(config.get("use_rslora", False), bool):
        raise ValueError("use_rslora must be a boolean")
    for flag in ("use_dora", "fan_in_fan_out", "lora_bias"):
        if config.get(flag, False) is not False:
            raise ValueError(f"unsupported LoRA configuration: {flag}")
    targets = config.get("target_modules")
    if not targets or not (isinstance(targets, str) or all(isinstance(t, str) and t for t in targets)):
        raise ValueError("explicit target_modules (a regex or a list of names) are required")
    for field, check in (("rank_pattern", _positive_int), ("alpha_pattern", _finite)):
        patterns = config.get(field) or {}
        if not isinstance(patterns, dict):
            raise ValueError(f"{field} must be an object")
        for key, value in patterns.items():
            if not isinstance(key, str) or not key:
                raise ValueError(f"{field} keys must be nonempty strings")
            check(value, f"{field}[{key}]")


def _per_module(patterns, module: str, default):
    """PEFT's pattern rule: the first key that matches a dotted suffix of the module name."""
    for key, value in (patterns or {}).items():
        if re.fullmatch(rf"(?:.*\.)?(?:{key})", module):
            return value
    return default


def _targeted(targets, module: str) -> bool:
    if not targets:
        return False
    if isinstance(targets, str):
        return re.fullmatch(targets, module) is not None
    return any(module == t or module.endswith("." + t) for t in targets)


def _verify_manifest(raw: bytes, files: dict) -> None:
    manifest = _json_object(raw, MANIFEST)
    if type(manifest.get("schema_version")) is not int or manifest["schema_version"] != 1:
        raise ValueError("unsupported LoRAForge manifest version or format")
    if manifest.get("format") != "loraforge.peft":
        raise ValueError("unsupported LoRAForge manifest version or format")
    records = (manifest.get("output") or {}).get("files") if isinstance(manifest.get("output"), dict) else None
    if not isinstance(records, dict):
        raise ValueError("manifest output.files must be an object")
    for name in (CONFIG, WEIGHTS):
        record = records.get(name)
        blob = files[name]
        if (
            not isinstance(record, dict)
            or record.get("bytes") != len(blob)
            or record.get("sha256") != hashlib.sha256(blob).hexdigest()
        ):
            raise ValueError(f"manifest integrity check failed for {name}")


def _header_size(prefix: bytes, total: int) -> int:
    if len(prefix) < 8:
        raise ValueError(f"{WEIGHTS} is truncated")
    size = int.from_bytes(prefix[:8], "little")
    if not 2 <= size <= _MAX_HEADER or 8 + size > total:
        raise ValueError("invalid safetensors header length")
    return size


def safetensors_header(path) -> dict:
    """The tensor entries (dtype, shape, data_offsets) of a safetensors file, reading only its header."""
    path = Path(path)
    with path.open("rb") as fh:
        size = _header_size(fh.read(8), path.stat().st_size)
        header = _json_object(fh.read(size), path.name)
    header.pop("__metadata__", None)
    return header


def read_safetensors(path) -> dict:
    """Every tensor of a safetensors file (F32 / F16 / BF16), as CPU tensors."""
    return _safetensors(Path(path).read_bytes())


def _safetensors(blob: bytes) -> dict:
    """Tensors of a safetensors file held in memory (F32 / F16 / BF16 only)."""
    import torch

    dtypes = {"F32": torch.float32, "F16": torch.float16, "BF16": torch.bfloat16}
    size = _header_size(blob[:8], len(blob))
    header = _json_object(blob[8 : 8 + size], WEIGHTS)
    header.pop("__metadata__", None)
    data = memoryview(blob)[8 + size :]
    spans, tensors = [], {}
    for key, info in header.items():
        dtype = dtypes.get(info.get("dtype")) if isinstance(info, dict) else None
        shape, offsets = (info.get("shape"), info.get("data_offsets")) if isinstance(info, dict) else (None, None)
        if (
            dtype is None
            or not isinstance(shape, list)
            or not all(type(d) is int and d >= 0 for d in shape)
            or not isinstance(offsets, list)
            or len(offsets) != 2
            or not all(type(o) is int for o in offsets)
        ):
            raise ValueError(f"unsupported tensor layout or dtype: {key}")
        start, end = offsets
        itemsize = torch.empty((), dtype=dtype).element_size()
        if not 0 <= start <= end <= len(data) or end - start != math.prod(shape) * itemsize:
            raise ValueError(f"tensor data outside the file or of the wrong size: {key}")
        spans.append((start, end))
        raw = bytearray(data[start:end])
        tensors[key] = (torch.frombuffer(raw, dtype=dtype) if raw else torch.empty(0, dtype=dtype)).reshape(shape)
    covered = 0
    for start, end in sorted(spans):
        if start != covered:
            raise ValueError("safetensors data is not exactly covered by its tensors")
        covered = end
    if covered != len(data):
        raise ValueError("safetensors data is not exactly covered by its tensors")
    return tensors


def load_peft_adapter(directory) -> PeftAdapter:
    """Read a local single-file safetensors PEFT adapter into CPU tensors.

    Unsupported configurations and inconsistent tensors are rejected rather
    than dropped; a present manifest must match both files byte for byte.
    """
    import torch

    source = Path(directory).resolve(strict=True)
    if not source.is_dir() or not all((source / n).is_file() for n in (CONFIG, WEIGHTS)):
        raise ValueError("expected adapter_config.json and adapter_model.safetensors in a directory")
    files = {name: (source / name).read_bytes() for name in (CONFIG, WEIGHTS)}
    if (source / MANIFEST).is_file():
        files[MANIFEST] = (source / MANIFEST).read_bytes()
        _verify_manifest(files[MANIFEST], files)
    config = _json_object(files[CONFIG], CONFIG)
    _validate_config(config)
    pairs: dict = {}
    for key, tensor in _safetensors(files[WEIGHTS]).items():
        found = _FACTOR_KEY.fullmatch(key)
        if found is None:
            raise ValueError(f"unsupported tensor key: {key}")
        if tensor.ndim != 2:
            raise ValueError(f"unsupported tensor layout or dtype: {key}")
        pairs.setdefault(found["module"], {})[found["side"]] = tensor
    if not pairs:
        raise ValueError("adapter has no LoRA tensor pairs")
    rslora = bool(config.get("use_rslora", False))
    modules = []
    for module in sorted(pairs):
        pair = pairs[module]
        if set(pair) != {"A", "B"}:
            raise ValueError(f"incomplete A/B pair: {module}")
        a, b = pair["A"], pair["B"]
        rank = _per_module(config.get("rank_pattern"), module, config["r"])
        alpha = _per_module(config.get("alpha_pattern"), module, config["lora_alpha"])
        if a.dtype != b.dtype or a.shape[0] != rank or b.shape[1] != rank or 0 in (*a.shape, *b.shape):
            raise ValueError(f"factor shape/dtype disagrees with configured rank: {module}")
        if not (torch.isfinite(a).all() and torch.isfinite(b).all()):
            raise ValueError(f"nonfinite factors: {module}")
        if not _targeted(config["target_modules"], module) or _targeted(config.get("exclude_modules"), module):
            raise ValueError(f"tensor module disagrees with target/exclude configuration: {module}")
        modules.append(AdapterModule(module, a, b, float(alpha), rslora))
    digests = {name: hashlib.sha256(blob).hexdigest() for name, blob in files.items()}
    return PeftAdapter(source, config, tuple(modules), digests)


def save_peft_adapter(adapter: PeftAdapter, output, *, factors: dict | None = None) -> Path:
    """Write a (possibly rank-reduced) copy of ``adapter`` with an integrity manifest.

    ``factors`` maps module names to replacement ``(a, b)``; each module's
    alpha is rewritten through ``alpha_pattern`` so that its scaling is kept
    (reference behaviour of compact exports, ``tests/test_runtime_slots.py:87-104``).
    """
    from safetensors.torch import save_file

    out = Path(output).absolute()
    if out.exists():
        raise FileExistsError(f"output must be a new directory: {out}")
    out.mkdir(parents=True)
    replaced = factors or {}
    tensors, ranks, alphas = {}, {}, {}
    for module in adapter.modules:
        a, b = replaced.get(module.name, (module.a, module.b))
        rank = a.shape[0]
        ranks[module.name] = rank
        alphas[module.name] = module.scaling * (math.sqrt(rank) if module.use_rslora else rank)
        prefix = f"base_model.model.{module.name}"
        tensors[prefix + ".lora_A.weight"] = a.contiguous()
        tensors[prefix + ".lora_B.weight"] = b.contiguous()
    config = dict(adapter.config, rank_pattern=ranks, alpha_pattern=alphas)
    (out / CONFIG).write_text(json.dumps(config, indent=2, sort_keys=True) + "\n")
    save_file(tensors, str(out / WEIGHTS))
    records = {}
    for name in (CONFIG, WEIGHTS):
        blob = (out / name).read_bytes()
        records[name] = {"sha256": hashlib.sha256(blob).hexdigest(), "bytes": len(blob)}
    manifest = {"schema_version": 1, "format": "loraforge.peft", "output": {"files": records}}
    (out / MANIFEST).write_text(json.dumps(manifest, indent=2) + "\n")
    return out
