"""gfx950 operators of the NF4 + multi-LoRA serving path (mirror of ``loraforge.ops``)."""

from .fused import LoraBatch, lora_apply, nf4_lora_linear, segments_to_slots, workspace_bytes
from .lora_rows import row_expand, row_shrink
from .nf4 import NF4State, NestedState, dequantize_nf4, dequantize_nf4_nested, prepare_scales, quantize_nf4
from . import rowexpand
from .quant_state import load_nf4_weight, quant_state_entries, quant_state_from_entries, save_nf4_weights

__all__ = [
    "LoraBatch",
    "NF4State",
    "NestedState",
    "dequantize_nf4",
    "dequantize_nf4_nested",
    "load_nf4_weight",
    "lora_apply",
    "nf4_lora_linear",
    "prepare_scales",
    "quant_state_entries",
    "quant_state_from_entries",
    "quantize_nf4",
    "row_expand",
    "row_shrink",
    "rowexpand",
    "save_nf4_weights",
    "segments_to_slots",
    "workspace_bytes",
]
