"""Build `libttsp_hip.so` (gfx950) from `csrc/*.hip` with hipcc.

Each translation unit is compiled to an object in parallel, then linked into
one shared library next to this file, so the built `.so` travels with the
source tree. Flags that matter for results:

* `-ffp-contract=off`: no implicit fused multiply-adds; every fma in the
  kernels is written out, which is what lets a CPU restatement reproduce
  them bit for bit.
* `-Xclang -target-feature -Xclang -packed-fp32-ops`: no packed fp32
  instructions are generated.

And one for speed: `-mllvm -amdgpu-kernarg-preload-count=16` has the command
processor place the first kernel-argument dwords in SGPRs at wave launch, so
a kernel's first loads do not wait for a fetch of its argument block (the
code keeps a prologue that fetches them, for firmware without preloading).

Usage: `python -m ttspipe_amd.build` (or `build()` from Python).
"""

from __future__ import annotations

import concurrent.futures
import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
OBJDIR = HERE / "_build"
LIB = HERE / "libttsp_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-mllvm",
    "-amdgpu-kernarg-preload-count=16",
    f"-I{CSRC}",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.stem + ".o")
    cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    return obj


def build(verbose: bool = False) -> Path:
    """Compile every kernel source and link the library. Always rebuilds."""
    OBJDIR.mkdir(exist_ok=True)
    srcs = sources()
    workers = max(1, min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs = list(pool.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
