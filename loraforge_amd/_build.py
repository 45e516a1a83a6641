"""Build the gfx950 shared library ``loraforge_amd/_lib/libloraforge_amd.so``.

Every ``csrc/*.hip`` file is compiled by ``hipcc --offload-arch=gfx950`` into
one position-independent object and the objects are linked into a single
C-ABI library (declared in ``include/loraforge_amd.h``). The build is in-tree
so the library travels with the source tree; nothing is JIT-compiled at run
time.
"""

from __future__ import annotations

import os
import re
import shutil
import subprocess
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
LIBDIR = PACKAGE / "_lib"
LIBRARY = LIBDIR / "libloraforge_amd.so"
ARCH = "gfx950"

HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-mcode-object-version=5",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-variable",
    f"-I{ROOT / 'include'}",
]


# Sources whose kernels must not use scratch: the decode and prefill kernels
# issue loads the compiler does not track (waited for explicitly), and a
# register spill of such a result would store it before the load returned.
NO_SCRATCH = {"nf4_gemv.hip", "nf4_decode_wide.hip", "nf4_lora_prefill.hip", "row_ops.hip"}


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build loraforge_amd")
    return found


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _scratch_users(remarks: list[str]) -> list[str]:
    """Kernels with a non-zero ScratchSize in -Rpass-analysis=kernel-resource-usage remarks."""
    users, name = [], None
    for line in remarks:
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            name = m.group(1)
            continue
        m = re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)
        if m and int(m.group(1)) > 0:
            users.append(f"{name} ({m.group(1)} bytes/lane)")
    return users


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    check = src.name in NO_SCRATCH
    extra = ["-Rpass-analysis=kernel-resource-usage"] if check else []
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    messages = [line for line in (result.stderr or "").splitlines() if noise not in line]
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(messages))
    if check:
        users = _scratch_users(messages)
        if users:
            obj.unlink(missing_ok=True)
            raise RuntimeError(f"{src.name}: kernels use scratch (register spills): " + "; ".join(users))
        messages = [line for line in messages if "kernel-resource-usage" not in line]
    if verbose and messages:
        print("\n".join(messages), flush=True)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source and link the library; returns its path."""
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    objs = [objdir / (s.stem + ".o") for s in srcs]
    workers = jobs or min(len(srcs), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda pair: _compile(pair[0], pair[1], verbose), zip(srcs, objs)))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError("link failed:\n" + result.stderr)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
