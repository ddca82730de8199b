"""CPU baseline for bench.py - TEST/BENCH INFRASTRUCTURE.

Times `nf4cpu_port.cpp` (the reference's CPU NF4 GEMV algorithm,
app/engine/nf4cpu.py:86-146, restated) over the benchmark's layer of seven
linears on this host's cores, threads = the CPUs this process may run on (the
reference's rule, app/engine/cpu.py:25-34). As the reference's CPU path does
(nf4cpu.py:850-860), nested scales are expanded once to dense bf16 absmax and
the code table is rounded to bf16. Weights rotate over copies larger than the
host's last-level cache so the rate is a DRAM rate.

Reported in the benchmark's unit: the layer's algorithmic bytes (the same
count the GPU figure uses) per second of CPU time.
"""

from __future__ import annotations

import ctypes
import math
import os
import platform
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def _lib():
    path = HERE / "libnf4cpu_port.so"
    if not path.exists():
        from oracle import build

        build.build()
    lib = ctypes.CDLL(str(path))
    lib.cpu_nf4_gemv.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                 ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    lib.cpu_nf4_gemv.restype = None
    lib.cpu_has_avx512bf16.restype = ctypes.c_int
    return lib


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def gemv(x_bf16: np.ndarray, packed: np.ndarray, absmax_bf16: np.ndarray, code_bf16: np.ndarray, n_out: int,
         threads: int | None = None, force_scalar: bool = False) -> np.ndarray:
    lib = _lib()
    threads = threads or len(os.sched_getaffinity(0))
    y = np.empty(n_out, dtype=np.uint16)
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    lib.cpu_nf4_gemv(x.ctypes.data, x.size, packed.ctypes.data, absmax_bf16.ctypes.data, code_bf16.ctypes.data,
                     n_out, y.ctypes.data, threads, int(force_scalar))
    return y


def run(layer_shapes, seconds: float = 10.0, threads: int | None = None) -> dict:
    from oracle import oracle as o

    lib = _lib()
    threads = threads or len(os.sched_getaffinity(0))
    rng = np.random.default_rng(0)
    weight_bytes = sum(M * K // 2 for _, M, K in layer_shapes)
    ncopy = max(2, math.ceil(1024 * 2**20 / weight_bytes))  # > 1 GB in rotation: past any L3
    code = o.from_f32(o.NF4_CODE, o.DT_BF16)
    copies = []
    for _ in range(ncopy):
        layer = []
        for _, M, K in layer_shapes:
            packed = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
            absmax = o.from_f32((rng.random(M * K // 64, dtype=np.float32) * 0.02 + 0.03), o.DT_BF16)
            layer.append((M, K, packed, absmax))
        copies.append(layer)
    xs = {K: o.from_f32(rng.standard_normal(K).astype(np.float32), o.DT_BF16) for _, _, K in layer_shapes}
    ys = {M: np.empty(M, dtype=np.uint16) for _, M, _ in layer_shapes}

    def step(layer):
        for M, K, packed, absmax in layer:
            lib.cpu_nf4_gemv(xs[K].ctypes.data, K, packed.ctypes.data, absmax.ctypes.data, code.ctypes.data, M,
                             ys[M].ctypes.data, threads, 0)

    for layer in copies[:2]:
        step(layer)  # warm up threads
    steps = 0
    t0 = time.perf_counter()
    while True:
        step(copies[steps % ncopy])
        steps += 1
        el = time.perf_counter() - t0
        if el >= seconds and steps >= ncopy:
            break
    from bench import LAYER, nf4_bytes  # the GPU figure's byte count for the same step

    step_bytes = sum(nf4_bytes(M, K, True) for _, M, K in LAYER)
    avx = bool(lib.cpu_has_avx512bf16())
    return {
        "value": round(step_bytes * steps / el / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "ms_per_step": round(el / steps * 1e3, 3),
        "sample": f"{steps} steps of the same 7-linear layer (bf16 x, dense bf16 absmax as the reference's CPU "
                  f"path stores it), {ncopy} weight copies rotated, {el:.1f} s; "
                  f"{'AVX512-BF16 kernel' if avx else 'scalar fallback (no AVX512-BF16 on this host)'}; "
                  f"{_cpu_model()}, {os.cpu_count()} logical CPUs",
    }
