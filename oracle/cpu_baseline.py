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


def host() -> dict:
    """This host as the baseline ran on it: CPU model, the logical CPUs this
    process may run on (the threads used), the physical cores those CPUs
    belong to (distinct (package, core) pairs in sysfs), and the machine's
    logical CPU count."""
    cpus = sorted(os.sched_getaffinity(0))
    cores = set()
    for c in cpus:
        base = Path(f"/sys/devices/system/cpu/cpu{c}/topology")
        try:
            cores.add((int((base / "physical_package_id").read_text()), int((base / "core_id").read_text())))
        except (OSError, ValueError):
            cores.add((0, c))
    return {"model": _cpu_model(), "logical_cpus_used": len(cpus), "physical_cores_used": len(cores),
            "logical_cpus_on_host": os.cpu_count()}


def _host_text() -> str:
    h = host()
    return (f"{h['model']}; {h['logical_cpus_used']} logical CPUs on {h['physical_cores_used']} physical cores "
            f"available to this process (host has {h['logical_cpus_on_host']} logical CPUs)")


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
                  f"{_host_text()}",
        "host": host(),
    }


def run_decode(frames: int = 3, threads: int | None = None) -> dict:
    """One synthetic Dual-AR frame on the CPU (the GPU decode's structure): 36
    slow blocks at position 2048+, the semantic head, the fast projection, the
    fast prime (4 blocks at fast position 0), then 9 codebooks of 4 fast
    blocks + head each, every block through `cpu_decode_block` (the reference
    CPU path's decode_block structure, nf4cpu.py:479-617) and every linear
    through the port's AVX512-BF16 GEMV. Random NF4 bytes and bf16 scales,
    distinct per layer (2 GB, past any last-level cache)."""
    from ttspipe_amd.dualar import DualARConfig

    cfg = DualARConfig()
    lib = _lib()
    threads = threads or len(os.sched_getaffinity(0))
    u16p, u8p, fp, i64 = ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64
    lib.cpu_decode_block.argtypes = ([u16p, u16p, i64, i64, i64, i64, u16p, u16p, u16p, u16p, ctypes.c_float]
                                     + [u8p, u16p] * 4 + [u16p, u16p, u16p, i64, i64, fp, ctypes.c_int])
    lib.cpu_decode_block.restype = None
    lib.cpu_argmax_bf16.argtypes = [u16p, i64]
    lib.cpu_argmax_bf16.restype = i64
    rng = np.random.default_rng(1)
    from oracle import oracle as o

    code = o.from_f32(o.NF4_CODE, o.DT_BF16)

    def lin(M, K):
        return (rng.integers(0, 256, M * K // 2, dtype=np.uint8),
                (0x3C00 + rng.integers(0, 0x80, M * K // 64, dtype=np.uint16)).astype(np.uint16))

    def vec(n):
        return (0x3F80 + rng.integers(0, 0x40, n, dtype=np.uint16)).astype(np.uint16)

    def cache(nkv, max_len):
        r = rng.integers(0, 0x80, nkv * max_len * 128, dtype=np.uint16)
        return ((r | 0x3F00) ^ (r << 8 & 0x8000)).astype(np.uint16)

    def block(D, nh, nkv, inter, max_len):
        hd = cfg.head_dim
        return {"D": D, "nh": nh, "nkv": nkv, "inter": inter, "max_len": max_len,
                "an": vec(D), "fn": vec(D), "qn": vec(hd), "kn": vec(hd),
                "qkv": lin((nh + 2 * nkv) * hd, D), "wo": lin(D, nh * hd), "w13": lin(2 * inter, D),
                "w2": lin(D, inter), "kc": cache(nkv, max_len), "vc": cache(nkv, max_len)}

    slow = [block(cfg.dim, cfg.n_head, cfg.n_local_heads, cfg.intermediate_size, cfg.max_seq_len)
            for _ in range(cfg.n_layer)]
    fast = [block(cfg.fast_dim, cfg.fast_n_head, cfg.fast_n_local_heads, cfg.fast_intermediate_size,
                  cfg.fast_max_len) for _ in range(cfg.fast_n_layer)]
    head, proj, fhead = lin(cfg.vocab_size, cfg.dim), lin(cfg.fast_dim, cfg.dim), lin(cfg.codebook_size, cfg.fast_dim)
    freqs = np.stack([np.cos(np.arange(64) * 0.01), np.sin(np.arange(64) * 0.01)], -1).astype(np.float32).ravel()
    x = vec(cfg.dim)
    bufs = {D: (np.empty(D, np.uint16), np.empty(D, np.uint16)) for D in (cfg.dim, cfg.fast_dim)}
    logits = np.empty(max(cfg.vocab_size, cfg.codebook_size), np.uint16)
    fx = np.empty(cfg.fast_dim, np.uint16)

    def run_block(b, xin, out, pos):
        p = lambda a: a.ctypes.data  # noqa: E731
        lib.cpu_decode_block(p(xin), p(out), b["D"], b["nh"], b["nkv"], b["inter"], p(b["an"]), p(b["fn"]),
                             p(b["qn"]), p(b["kn"]), cfg.norm_eps, p(b["qkv"][0]), p(b["qkv"][1]), p(b["wo"][0]),
                             p(b["wo"][1]), p(b["w13"][0]), p(b["w13"][1]), p(b["w2"][0]), p(b["w2"][1]), p(code),
                             p(b["kc"]), p(b["vc"]), pos, b["max_len"], p(freqs), threads)

    def gemv_into(w, xin, M, K, out):
        lib.cpu_nf4_gemv(xin.ctypes.data, K, w[0].ctypes.data, w[1].ctypes.data, code.ctypes.data, M,
                         out.ctypes.data, threads, 0)

    def blocks(stack, xin, D, pos):
        cur = xin
        for i, blk in enumerate(stack):  # outputs alternate between two buffers
            out = bufs[D][i % 2]
            run_block(blk, cur, out, pos)
            cur = out
        return cur

    def frame(pos):
        cur = blocks(slow, x, cfg.dim, pos)
        gemv_into(head, cur, cfg.vocab_size, cfg.dim, logits)
        lib.cpu_argmax_bf16(logits.ctypes.data, cfg.vocab_size)
        gemv_into(proj, cur, cfg.fast_dim, cfg.dim, fx)
        for cb in range(cfg.num_codebooks):  # the prime at fast position 0, then one step per codebook
            fcur = blocks(fast, fx, cfg.fast_dim, cb)
            if cb:
                gemv_into(fhead, fcur, cfg.codebook_size, cfg.fast_dim, logits)
                lib.cpu_argmax_bf16(logits.ctypes.data, cfg.codebook_size)

    frame(cfg.prefill_len)  # warm up threads and pages
    t0 = time.perf_counter()
    for i in range(frames):
        frame(cfg.prefill_len + 1 + i)
    el = time.perf_counter() - t0
    return {"ms_per_step": round(el / frames * 1e3, 2), "frames": frames, "cores": threads,
            "sample": f"{frames} synthetic Dual-AR frames after one warm-up (36 slow blocks at positions 2049+, "
                      f"semantic head, fast projection, fast prime + 9 codebooks of 4 fast blocks and head), "
                      f"distinct random NF4 weights per layer (dense bf16 absmax), "
                      f"{'AVX512-BF16 GEMV' if lib.cpu_has_avx512bf16() else 'scalar GEMV'}"}
