"""PEFT adapter file contract consumed by the runtime (mirror of ``loraforge.adapters``)."""

from .peft import AdapterModule, PeftAdapter, load_peft_adapter, read_safetensors, safetensors_header, save_peft_adapter

__all__ = ["AdapterModule", "PeftAdapter", "load_peft_adapter", "read_safetensors", "safetensors_header", "save_peft_adapter"]
