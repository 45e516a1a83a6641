"""Local PEFT adapter files: the subset ``GPUAdapterSlots.load`` consumes.

Reference: ``src/loraforge/adapters/peft.py`` -- ``AdapterModule`` (:42-57),
``load_peft_adapter`` (:124-198) and the sha256 manifest check (:98-121).
Single-file safetensors adapters with ``base_model.model.<module>.lora_A/B.weight``
keys; nothing is executed from the files (safetensors + JSON only).
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
_KEY = re.compile(r"^base_model\.model\.(.+)\.lora_([AB])\.weight$")


@dataclass(frozen=True)
class AdapterModule:
    name: str
    a: object  # [rank, in_features]
    b: object  # [out_features, rank]
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
    source: Path
    config: dict
    modules: tuple
    source_sha256: dict


def _sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as fh:
        for chunk in iter(lambda: fh.read(1 << 20), b""):
            digest.update(chunk)
    return digest.hexdigest()


def _json(path: Path) -> dict:
    def unique(pairs):
        out = {}
        for key, value in pairs:
            if key in out:
                raise ValueError(f"duplicate JSON key in {path.name}: {key}")
            out[key] = value
        return out

    data = json.loads(path.read_text(), object_pairs_hook=unique)
    if not isinstance(data, dict):
        raise ValueError(f"{path.name} must contain a JSON object")
    return data


def _matches(targets, name: str) -> bool:
    if targets is None:
        return False
    if isinstance(targets, str):
        return re.fullmatch(targets, name) is not None
    return any(name == t or name.endswith("." + t) for t in targets)


def _pattern_value(pattern: dict, name: str, default):
    for key, value in (pattern or {}).items():
        if name == key or name.endswith("." + key) or re.fullmatch(key, name):
            return value
    return default


def _check_config(config: dict) -> None:
    if config.get("peft_type", "LORA") != "LORA":
        raise ValueError("only LoRA adapters are supported")
    rank = config.get("r")
    if type(rank) is not int or rank < 1:
        raise ValueError("config r must be a positive integer")
    alpha = config.get("lora_alpha")
    if isinstance(alpha, bool) or not isinstance(alpha, (int, float)) or not math.isfinite(alpha):
        raise ValueError("config lora_alpha must be a finite number")
    if not isinstance(config.get("target_modules"), (str, list)):
        raise ValueError("config target_modules must be a string or list")
    if config.get("bias", "none") != "none":
        raise ValueError("only bias='none' adapters are supported")


def _check_manifest(directory: Path) -> None:
    path = directory / MANIFEST
    if not path.exists():
        return
    manifest = _json(path)
    if manifest.get("schema_version") != 1 or manifest.get("format") != "loraforge.peft":
        raise ValueError("unsupported LoRAForge manifest version or format")
    files = (manifest.get("output") or {}).get("files")
    if not isinstance(files, dict):
        raise ValueError("manifest output.files must be an object")
    for name in (CONFIG, WEIGHTS):
        record = files.get(name, {})
        if (
            not isinstance(record, dict)
            or record.get("sha256") != _sha256(directory / name)
            or record.get("bytes") != (directory / name).stat().st_size
        ):
            raise ValueError(f"manifest integrity check failed for {name}")


def load_peft_adapter(directory) -> PeftAdapter:
    """Read a local single-file safetensors PEFT adapter into CPU tensors."""
    import torch
    from safetensors.torch import load_file

    source = Path(directory).resolve(strict=True)
    if not source.is_dir() or not all((source / n).is_file() for n in (CONFIG, WEIGHTS)):
        raise ValueError("expected adapter_config.json and adapter_model.safetensors in a directory")
    _check_manifest(source)
    names = [CONFIG, WEIGHTS] + ([MANIFEST] if (source / MANIFEST).exists() else [])
    hashes = {n: _sha256(source / n) for n in names}
    config = _json(source / CONFIG)
    _check_config(config)
    weights = load_file(source / WEIGHTS, device="cpu")
    pairs: dict = {}
    for key, value in weights.items():
        match = _KEY.fullmatch(key)
        if match is None:
            raise ValueError(f"unsupported tensor key: {key}")
        if value.ndim != 2 or value.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"unsupported tensor layout or dtype: {key}")
        pairs.setdefault(match.group(1), {})[match.group(2)] = value
    if not pairs:
        raise ValueError("adapter has no LoRA tensor pairs")
    modules = []
    for name, pair in sorted(pairs.items()):
        if pair.keys() != {"A", "B"}:
            raise ValueError(f"incomplete A/B pair: {name}")
        a, b = pair["A"], pair["B"]
        rank = _pattern_value(config.get("rank_pattern"), name, config["r"])
        alpha = _pattern_value(config.get("alpha_pattern"), name, config["lora_alpha"])
        if min(*a.shape, *b.shape) < 1 or a.shape[0] != rank or b.shape[1] != rank or a.dtype != b.dtype:
            raise ValueError(f"factor shape/dtype disagrees with configured rank: {name}")
        if not torch.isfinite(a).all().item() or not torch.isfinite(b).all().item():
            raise ValueError(f"nonfinite factors: {name}")
        if not _matches(config["target_modules"], name) or _matches(config.get("exclude_modules"), name):
            raise ValueError(f"tensor module disagrees with target/exclude configuration: {name}")
        modules.append(AdapterModule(name, a.clone(), b.clone(), float(alpha), bool(config.get("use_rslora", False))))
    if any(_sha256(source / n) != digest for n, digest in hashes.items()):
        raise ValueError("source adapter changed while it was being read")
    return PeftAdapter(source, config, tuple(modules), hashes)


def save_peft_adapter(adapter: PeftAdapter, output, *, factors: dict | None = None) -> Path:
    """Write a (possibly rank-reduced) copy with a sha256 manifest.

    ``factors`` maps module names to replacement ``(a, b)``; the per-module
    alpha is rescaled so ``scaling`` is preserved (reference behaviour of
    compact exports, ``tests/test_runtime_slots.py:87-104``).
    """
    from safetensors.torch import save_file

    out = Path(output).absolute()
    if out.exists():
        raise FileExistsError(f"output must be a new directory: {out}")
    out.mkdir(parents=True)
    tensors, ranks, alphas = {}, {}, {}
    for module in adapter.modules:
        a, b = (factors or {}).get(module.name, (module.a, module.b))
        rank = a.shape[0]
        scaling = module.scaling
        alphas[module.name] = scaling * (math.sqrt(rank) if module.use_rslora else rank)
        ranks[module.name] = rank
        tensors[f"base_model.model.{module.name}.lora_A.weight"] = a.contiguous()
        tensors[f"base_model.model.{module.name}.lora_B.weight"] = b.contiguous()
    config = dict(adapter.config)
    config["rank_pattern"] = ranks
    config["alpha_pattern"] = alphas
    (out / CONFIG).write_text(json.dumps(config, indent=2, sort_keys=True) + "\n")
    save_file(tensors, str(out / WEIGHTS))
    manifest = {
        "schema_version": 1,
        "format": "loraforge.peft",
        "output": {
            "files": {
                name: {"sha256": _sha256(out / name), "bytes": (out / name).stat().st_size} for name in (CONFIG, WEIGHTS)
            }
        },
    }
    (out / MANIFEST).write_text(json.dumps(manifest, indent=2) + "\n")
    return out
