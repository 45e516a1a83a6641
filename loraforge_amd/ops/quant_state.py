"""NF4 weights as they are stored on disk: bitsandbytes' packed QuantState entries.

The reference writes quantised checkpoints with ``state.as_dict(packed=True)``
next to each packed weight (``benchmarks/prepare_qwen35_nf4.py:59-60``) and
reads them back with ``QuantState.from_dict`` over the keys that start with the
weight's name (``benchmarks/check_qwen35_nf4_ops.py:73-85``). The format is
bitsandbytes 0.50.2's (pinned at ``integrations/sglang_experimental.py:54-55``);
bitsandbytes is not a dependency here, so this module restates its published
layout:

- ``<name>``: the packed nibbles, uint8 ``[N*K/2, 1]``;
- ``<name>.absmax``: fp32 block scales, or uint8 codes when double-quantised;
- ``<name>.quant_map``: the fp32 ``[16]`` codebook;
- ``<name>.nested_absmax`` / ``<name>.nested_quant_map``: the second-level fp32
  scales and the fp32 ``[256]`` dynamic map (double-quantised only);
- ``<name>.quant_state.bitsandbytes__nf4``: uint8 bytes of a UTF-8 JSON object
  holding the non-tensor fields ``quant_type``, ``blocksize``, ``dtype``
  (``"bfloat16"``), ``shape`` and, when nested, ``nested_blocksize``,
  ``nested_dtype`` and ``nested_offset``.

Only safetensors and JSON are read: nothing in a file is executed.
"""

from __future__ import annotations

import json

from .nf4 import NF4State, NestedState

_PACKED_KEY = "quant_state.bitsandbytes__nf4"
_TENSOR_KEYS = ("absmax", "quant_map", "nested_absmax", "nested_quant_map")
_FIELDS = {"quant_type", "blocksize", "dtype", "shape", "nested_blocksize", "nested_dtype", "nested_offset"}


def _dtype_name(dtype) -> str:
    return str(dtype).replace("torch.", "")


def _torch_dtype(name: str):
    import torch

    value = getattr(torch, name, None)
    if not isinstance(value, torch.dtype):
        raise ValueError(f"unknown dtype {name!r} in the quant state")
    return value


def quant_state_entries(qweight, state: NF4State, name: str) -> dict:
    """Tensors to store for one NF4 weight under ``name`` (``as_dict(packed=True)`` layout)."""
    import torch

    if state.quant_type != "nf4":
        raise ValueError("only nf4 quant states are supported")
    fields = {
        "quant_type": "nf4",
        "blocksize": int(state.blocksize),
        "dtype": _dtype_name(state.dtype if state.dtype is not None else torch.bfloat16),
        "shape": [int(v) for v in state.shape],
    }
    out = {name: qweight, f"{name}.absmax": state.absmax, f"{name}.quant_map": state.code}
    if state.nested:
        out[f"{name}.nested_absmax"] = state.state2.absmax
        out[f"{name}.nested_quant_map"] = state.state2.code
        fields.update(
            nested_blocksize=int(state.state2.blocksize),
            nested_dtype="float32",
            nested_offset=float(state.offset),
        )
    blob = json.dumps(fields).encode("utf-8")
    out[f"{name}.{_PACKED_KEY}"] = torch.tensor(list(blob), dtype=torch.uint8)
    return {k: v.detach().contiguous().cpu() for k, v in out.items()}


def quant_state_from_entries(entries: dict, name: str, *, device=None):
    """``(qweight, NF4State)`` from the stored tensors of weight ``name``.

    ``entries`` maps full keys to tensors (e.g. everything in a safetensors
    file, or just the keys that start with ``name + "."``). Raises
    ``ValueError`` for a missing or foreign quant state, a non-NF4 type, a
    block size other than 64 or shapes that disagree with the packed data.
    """
    import torch

    if name not in entries:
        raise ValueError(f"no packed weight named {name!r}")
    prefix = name + "."
    own = {k[len(prefix) :]: v for k, v in entries.items() if k.startswith(prefix)}
    packed = [k for k in own if k.startswith("quant_state.")]
    if len(packed) != 1 or packed[0] != _PACKED_KEY:
        raise ValueError(f"{name}: expected exactly one {_PACKED_KEY!r} entry, found {sorted(packed)}")
    raw = own.pop(_PACKED_KEY)
    fields = json.loads(bytes(raw.reshape(-1).to(torch.uint8).tolist()).decode("utf-8"))
    unknown = set(fields) - _FIELDS
    extra = set(own) - set(_TENSOR_KEYS)
    if unknown or extra:
        raise ValueError(f"{name}: unexpected quant state items {sorted(unknown | extra)}")
    if fields.get("quant_type") != "nf4":
        raise ValueError(f"{name}: quant_type {fields.get('quant_type')!r} is not nf4")
    if int(fields.get("blocksize", 0)) != 64:
        raise ValueError(f"{name}: blocksize {fields.get('blocksize')} is not 64")
    shape = torch.Size(int(v) for v in fields["shape"])
    if len(shape) != 2 or shape[0] % 64 or shape[1] % 64:
        raise ValueError(f"{name}: shape {tuple(shape)} must be 2D with dimensions that are multiples of 64")
    qweight = entries[name]
    numel = shape[0] * shape[1]
    if qweight.dtype != torch.uint8 or qweight.numel() * 2 != numel:
        raise ValueError(f"{name}: packed weight holds {qweight.numel()} bytes for shape {tuple(shape)}")
    nested = "nested_absmax" in own
    absmax = own.get("absmax")
    if absmax is None or own.get("quant_map") is None:
        raise ValueError(f"{name}: absmax and quant_map are required")
    if absmax.numel() != numel // 64:
        raise ValueError(f"{name}: {absmax.numel()} block scales for {numel // 64} blocks")
    if absmax.dtype != (torch.uint8 if nested else torch.float32):
        raise ValueError(f"{name}: absmax dtype {absmax.dtype} does not match nested={nested}")
    move = (lambda t: t.to(device)) if device is not None else (lambda t: t)
    offset, state2 = None, None
    if nested:
        if "nested_quant_map" not in own or "nested_offset" not in fields or "nested_blocksize" not in fields:
            raise ValueError(f"{name}: incomplete double-quant state")
        blocks2 = int(fields["nested_blocksize"])
        if blocks2 <= 0 or own["nested_absmax"].numel() != -(-absmax.numel() // blocks2):
            raise ValueError(f"{name}: nested scales do not cover the absmax codes")
        offset = move(torch.tensor(float(fields["nested_offset"]), dtype=torch.float32))
        state2 = NestedState(
            move(own["nested_absmax"].float().reshape(-1).contiguous()),
            move(own["nested_quant_map"].float().reshape(-1).contiguous()),
            blocks2,
        )
    state = NF4State(
        move(absmax.reshape(-1).contiguous()),
        shape,
        move(own["quant_map"].float().reshape(-1).contiguous()),
        _torch_dtype(fields.get("dtype", "bfloat16")),
        64,
        "nf4",
        offset=offset,
        state2=state2,
    )
    return move(qweight.reshape(-1, 1).contiguous()), state


def save_nf4_weights(path, weights: dict, *, metadata: dict | None = None) -> None:
    """Writes ``{name: (qweight, NF4State)}`` to one safetensors file."""
    from safetensors.torch import save_file

    tensors = {}
    for name, (qweight, state) in weights.items():
        tensors.update(quant_state_entries(qweight, state, name))
    save_file(tensors, str(path), metadata=metadata)


def load_nf4_weight(path, name: str, *, device=None):
    """``(qweight, NF4State)`` of weight ``name`` from a safetensors file (tensors only)."""
    from safetensors import safe_open

    with safe_open(str(path), framework="pt", device="cpu") as f:
        keys = [k for k in f.keys() if k == name or k.startswith(name + ".")]
        entries = {k: f.get_tensor(k) for k in keys}
    return quant_state_from_entries(entries, name, device=device)
