"""The C-ABI library loads and exports every symbol the public header declares (CPU only).

Only argument-validation paths are exercised here: they return before any HIP
call, so no GPU is needed.
"""

import ctypes
import re
from pathlib import Path

import pytest

from loraforge_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "loraforge_amd.h"


def declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(lf_[a-z0-9_]+)\s*\(", text)))


def test_header_and_binding_agree():
    assert declared() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    for name in declared():
        assert hasattr(lib, name), name
    version = int(re.search(r"#define LF_ABI_VERSION (\d+)", HEADER.read_text()).group(1))
    assert lib.lf_abi_version() == version == _lib.ABI_VERSION


def test_validation_errors_without_device_work():
    lib = _lib.library()
    status = lib.lf_nf4_dequant(None, ctypes.c_void_p(16), None, None, 5, None)
    assert status == _lib.LF_EINVAL
    assert b"multiple of 4096" in lib.lf_last_error()
    with pytest.raises(ValueError, match="threads"):
        _lib.check(lib.lf_row_expand(*([ctypes.c_void_p(8)] * 12), 2, 4, 4, 4, 1, 4, 64, 64, None))
    with pytest.raises(ValueError, match="num_slices"):
        _lib.check(lib.lf_row_shrink(*([ctypes.c_void_p(16)] * 5), 4, 64, 64, 2, 5, 64, 16, None, 0, 0, None))
    with pytest.raises(ValueError, match="null pointer"):
        _lib.check(lib.lf_swiglu(None, 1, 8, 16, None, 8, None))
    with pytest.raises(ValueError, match="2 \\* n"):
        _lib.check(lib.lf_swiglu(ctypes.c_void_p(16), 1, 8, 8, ctypes.c_void_p(16), 8, None))
    w = _lib.NF4Weight(n=100, k=64)
    with pytest.raises(ValueError, match="multiples of 64"):
        _lib.check(lib.lf_nf4_lora_linear(ctypes.c_void_p(16), 1, 64, ctypes.byref(w), None, None, ctypes.c_void_p(16), 64, None, 0, 0, None))
    both = _lib.LF_PLAN_DECODE_CHUNKS | _lib.LF_PLAN_PREFILL
    with pytest.raises(ValueError, match="exclude each other"):
        _lib.check(lib.lf_nf4_lora_linear(ctypes.c_void_p(16), 100, 64, ctypes.byref(w), None, None, ctypes.c_void_p(16), 64, None, 0, both, None))
    with pytest.raises(ValueError, match="unknown flags"):
        _lib.check(lib.lf_nf4_lora_linear(ctypes.c_void_p(16), 100, 64, ctypes.byref(w), None, None, ctypes.c_void_p(16), 64, None, 0, 0x40, None))


def test_workspace_size_is_host_arithmetic():
    lib = _lib.library()
    small = lib.lf_nf4_lora_workspace_size(1, 4096, 4096, 1, 16)
    big = lib.lf_nf4_lora_workspace_size(64, 4096, 4096, 1, 16)
    prefill = lib.lf_nf4_lora_workspace_size(2048, 11008, 4096, 1, 32)
    # Decode: the 256 KiB control header (tagged shrink partials inside), the prefill's
    # 16 KiB flag region, then room for fp32 scales rebuilt from a nested state.
    assert small == big == 262144 + 16384 + 4096 * (4096 // 64) * 4
    assert prefill >= 262144 + 2048 * 64 * 2  # prefill z rows sit after that header
    assert lib.lf_nf4_lora_workspace_size(-1, 64, 64, 1, 1) == -1
