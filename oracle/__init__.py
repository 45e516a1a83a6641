"""CPU oracle for the NF4 + multi-LoRA serving path. TEST INFRASTRUCTURE ONLY.

This package restates, in numpy, the arithmetic of the reference
(lishenghui/loraforge) for the quantized-serving linear:

* ``oracle.nf4``   -- NF4 block dequantisation, the double-quant scale
  reconstruction and an input quantiser (``src/loraforge/ops/nf4.py``,
  ``src/loraforge/ops/_nf4_kernels.py``).
* ``oracle.rows``  -- retained-rank ``row_shrink`` / ``row_expand``
  (``src/loraforge/ops/csrc/lora_rows.cu``, ``tests/test_row_operators_gpu.py``).
* ``oracle.linear`` -- the NF4 base linear followed by the per-token LoRA
  chain, decode and segmented prefill, and the SwiGLU MLP chain
  (``src/loraforge/integrations/_sglang_nf4_linear.py``,
  ``benchmarks/qwen35_prefill_fused.py``, ``benchmarks/qwen35_decode_silu.py``).
* ``oracle.cpu_path`` -- the PyTorch-CPU restatement of the reference serving
  path that ``bench.py`` times as the CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as a checker or a baseline.
The product (``loraforge_amd``) never imports it and has no CPU fallback.

Parity status of each function is stated in its docstring. One function is
"parity unpinned" with respect to bitsandbytes 0.50.2 (absent from the
reference tree and not installable offline): ``oracle.nf4.dynamic_map``
(the second-level code table of double quantisation). The double-quant
*reconstruction* formula is pinned by closed-form special cases; the exact
table bitsandbytes would produce is not.
"""
