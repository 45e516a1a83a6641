"""loraforge_amd: the NF4 + multi-LoRA serving path of LoRAForge, native to MI355X (gfx950).

Public API mirrors the reference package: ``loraforge_amd.ops`` (``dequantize_nf4``,
``prepare_scales``, ``row_shrink``, ``row_expand`` and the fused
``nf4_lora_linear``), ``loraforge_amd.runtime`` (``GPUAdapterSlots``,
``AdapterSlots``, ``SlotHandle``, ``RetainedLayout``, ``AdapterTable``) and
``loraforge_amd.adapters`` (``load_peft_adapter``). Kernels live in one C-ABI
library built from ``loraforge_amd/csrc`` (``include/loraforge_amd.h``).
Submodules import torch lazily.
"""

__version__ = "0.1.0.dev0"
