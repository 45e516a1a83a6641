"""Serving-framework bridges (contract level: the frameworks themselves are not installed here)."""

from .sglang import apply_lora, apply_nf4_lora, lora_batch_from_batch_info, token_slots_from_batch_info

__all__ = ["apply_lora", "apply_nf4_lora", "lora_batch_from_batch_info", "token_slots_from_batch_info"]
