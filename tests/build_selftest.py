"""Build tests/libttsp_selftest.so (gfx950) from tests/csrc/selftest.hip - TEST
INFRASTRUCTURE: the numerics self-test kernels, kept out of the product
library. Same compiler flags as the product (ttspipe_amd/build.py)."""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "libttsp_selftest.so"


def build(verbose: bool = False) -> Path:
    from ttspipe_amd import build as product

    src = HERE / "csrc" / "selftest.hip"
    cmd = [product.HIPCC, *product.COMMON_FLAGS, "-shared", str(src), "-o", str(LIB)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
