"""Build the oracle's C library (test infrastructure; never loaded by the product).

gcc, SSE fp32 arithmetic (x86-64 default, no excess precision),
`-ffp-contract=off` so every fp32 operation is a single IEEE operation and
only the explicit fmaf() calls fuse. `python -m oracle.build` or `build()`.
"""

from __future__ import annotations

import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
PORT_LIB = HERE / "libnf4cpu_port.so"


def build(verbose: bool = False) -> Path:
    cmd = ["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", "-fno-fast-math",
           "-fopenmp", str(HERE / "nf4_oracle.c"), "-o", str(LIB), "-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{proc.stderr}")
    port = HERE / "nf4cpu_port.cpp"
    if port.exists():
        cmd = ["g++", "-O3", "-std=c++17", "-fPIC", "-shared", "-fopenmp", str(port), "-o", str(PORT_LIB)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"CPU baseline build failed:\n{proc.stderr}")
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
