"""Benchmark: NF4 GEMV HBM GB/s (% of peak) + decode step ms/token, one MI355X.

Step (the `value`): the seven batch-1 linears of one Qwen3-4B-shaped decoder
layer in NF4 with double-quant absmax (uint8, bs2 256, fp32 scale + offset),
bf16 activations - q 2560->4096, k/v 2560->1024, o 4096->2560, gate/up
2560->9728, down 9728->2560 - executed as the fused decode block executes them
(q/k/v as one wqkv GEMV, gate/up as one SwiGLU GEMV: four launches,
52,149,332 algorithmic bytes: the same weights and scales, x read once per
launch, one gated output instead of gate and up); the same linears as seven separate launches
(52,186,204 bytes) are reported beside it.
Weights rotate over enough distinct copies (> 512 MB) that every step streams
from HBM, not from the 256 MB Infinity Cache; launches are replayed from a
HIP graph so the GPU runs them back to back. value = bytes / time (GB/s).

Also reported: the dominant kernel (gate 9728x2560) timed alone with HIP
events on its stream -> `roofline`; the single fp16 GEMV of the reference's
CPU-runnable case (plain fp32 absmax) -> `gemv_fp16_plain`; the synthetic
Dual-AR decode step -> `decode`; and the CPU baseline (the reference's CPU
NF4 GEMV algorithm restated in C++, on this host's cores) -> `cpu_baseline`,
with the same Dual-AR frame on the CPU through it -> `cpu_baseline.decode`.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 * 2**20
#: A spin of about 100 us queued ahead of each timed region: the host's submission
#: of the first graph replay then overlaps it instead of idling inside the region.
SPIN_CYCLES = 200_000

#: Figures measured off-line for the gate-shape GEMV launch (9728 x 2560, nested,
#: bf16), keyed by the launch they were measured on: its shape and grid and a
#: digest of the kernel source. bench.py prints them only while the key matches
#: the launch it makes (else null, marked stale).
#: traffic_bytes: HBM bytes per launch, rocprofv3 --pmc FETCH_SIZE then WRITE_SIZE
#: per dispatch (bench.py --only kernel --direct; medians over 88 dispatches),
#: each scaled by the same counter on a plain 64 MiB copy (FETCH_SIZE x 1.99925,
#: WRITE_SIZE x 1.0): (6444.06 x 1.99925 + 22.81) KiB.
#: rocprof_*_us: dispatch durations of that kernel in rocprofv3 --kernel-trace
#: --stats -- python3 bench.py --only kernel (2156 graph-replayed dispatches).
#: The tracer reads 3-10 % above the untraced launch-to-launch interval (6.04
#: median against 5.89 us in the same session; 6.2-6.6 us means across boxes).
GEMV_PROFILE = {
    "key": {"M": 9728, "K": 2560, "J": 5, "KS": 1, "RPW": 5, "grid": 244, "source_sha16": "066d1767a696e109"},
    "traffic_bytes": 13_211_723,
    "rocprof_mean_us": 6.245,
    "rocprof_median_us": 6.119,
    "summary": "profiles/nf4_gemv_gate_9728x2560_bf16_nested.md",
}


#: the GEMV's translation unit: its source and the headers it includes
GEMV_SOURCES = ("nf4_gemv.hip", "gemv_common.h", "attn_common.h", "ttsp_common.h")


def gemv_launch_key(M: int, K: int) -> dict:
    """The launch the GEMV makes for [M, K] (one row), as GEMV_PROFILE keys it."""
    import ctypes
    import hashlib

    from ttspipe_amd import _lib

    J, KS, RPW = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    _lib.load().ttsp_gemv_shape(M, K, ctypes.byref(J), ctypes.byref(KS), ctypes.byref(RPW))
    rows_wg = (8 // KS.value) * RPW.value
    h = hashlib.sha256()
    for name in GEMV_SOURCES:
        h.update((ROOT / "ttspipe_amd" / "csrc" / name).read_bytes())
    return {"M": M, "K": K, "J": J.value, "KS": KS.value, "RPW": RPW.value, "grid": -(-M // rows_wg),
            "source_sha16": h.hexdigest()[:16]}


def spin():
    """Queue SPIN_CYCLES of GPU work on the current stream."""
    import torch

    torch.cuda._sleep(SPIN_CYCLES)

# (name, out_features, in_features) of one decoder layer's linears
LAYER = [("q", 4096, 2560), ("k", 1024, 2560), ("v", 1024, 2560), ("o", 2560, 4096),
         ("gate", 9728, 2560), ("up", 9728, 2560), ("down", 2560, 9728)]


def nf4_bytes(M: int, K: int, nested: bool, dsize: int = 2, bs: int = 64, bs2: int = 256) -> int:
    """Algorithmic bytes of one GEMV: packed weight + scales + x + y."""
    nblk = M * K // bs
    if nested:
        scales = nblk + 4 * math.ceil(nblk / bs2) + 256 * 4 + 4  # a8, absmax2, code2, offset
    else:
        scales = 4 * nblk
    return M * K // 2 + scales + dsize * K + dsize * M


class Linear:
    """Device buffers of one NF4 linear, random codes and scales."""

    def __init__(self, M, K, nested, seed, device):
        import torch

        from ttspipe_amd.quant import create_dynamic_map

        g = torch.Generator(device=device).manual_seed(seed)
        self.M, self.K, self.nested = M, K, nested
        nblk = M * K // 64
        self.w = torch.randint(0, 256, (M * K // 2,), dtype=torch.uint8, device=device, generator=g)
        if nested:
            self.a8 = torch.randint(0, 256, (nblk,), dtype=torch.uint8, device=device, generator=g)
            self.amax = torch.rand(-(-nblk // 256), device=device, generator=g) * 0.01 + 0.01
            self.code2 = create_dynamic_map().to(device)
            self.offset = 0.04
        else:
            self.a8, self.code2, self.offset = None, None, 0.0
            self.amax = torch.rand(nblk, device=device, generator=g) * 0.04 + 0.02


# The same layer as the fused decode block executes it: q/k/v as one wqkv
# matrix, and gate/up as one SwiGLU launch streaming both weights.
FUSED_LAYER = [("wqkv", 6144, 2560), ("o", 2560, 4096), ("gate_up", 9728, 2560), ("down", 2560, 9728)]


def fused_layer_bytes() -> int:
    """Algorithmic bytes of FUSED_LAYER: every weight byte and scale once, x and
    the code2 table once per launch (the SwiGLU launch reads two code2 tables),
    y once."""
    total = 0
    for name, M, K in FUSED_LAYER:
        n = 2 if name == "gate_up" else 1
        nblk = M * K // 64
        total += n * (M * K // 2 + nblk + 4 * math.ceil(nblk / 256) + 256 * 4 + 4) + 2 * K + 2 * M
    return total


def launch(lib, lut, lin, x, y, dt, stream):
    from ttspipe_amd import _lib

    rc = lib.ttsp_nf4_gemm(x.data_ptr(), dt, lin.w.data_ptr(), _lib.ptr(lin.a8), lin.amax.data_ptr(),
                           _lib.ptr(lin.code2), lin.offset, lut.data_ptr(), y.data_ptr(), 0, 0, lin.M, lin.K, 1,
                           64, 256, stream)
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemm failed: {rc}")


def launch_swiglu(lib, lut, l1, l3, x, y, stream):
    from ttspipe_amd import _lib

    rc = lib.ttsp_nf4_gemv_fused(x.data_ptr(), _lib.DT_BF16, 0, 1e-6, l1.w.data_ptr(), _lib.ptr(l1.a8),
                                 l1.amax.data_ptr(), _lib.ptr(l1.code2), l1.offset, l3.w.data_ptr(), _lib.ptr(l3.a8),
                                 l3.amax.data_ptr(), _lib.ptr(l3.code2), l3.offset, lut.data_ptr(), y.data_ptr(), 0, 0,
                                 l1.M, l1.K, 64, 256, stream)
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemv_fused failed: {rc}")


def time_graph(graph, replays: int, stream) -> float:
    """Seconds per replay, HIP events on the graph's launch stream."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spin()
    start.record(stream)
    for _ in range(replays):
        graph.replay()
    end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / replays


def capture(fn):
    import torch

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn()
    return graph


def time_exact_steps(body, ncopy: int, steps: int, warmup: int, sustained_replays: int = 100):
    """Run exactly `warmup` untimed steps, then time exactly `steps` steps; a
    step is one pass over one weight copy, and consecutive steps walk the
    copies in order. `body(n)` launches the first n copies' steps. Steps go
    as replays of a graph over all ncopy copies plus one graph over the first
    steps % ncopy of them (copy 0 follows the last copy, so every step still
    reads weights the cache no longer holds). The timed region is bracketed by
    device synchronisation and timed with HIP events on the launch stream.
    Also returns a sustained figure over `sustained_replays` full replays."""
    import torch

    stream = torch.cuda.current_stream()
    graphs = {ncopy: capture(lambda: body(ncopy))}
    for n in {steps % ncopy, warmup % ncopy} - {0}:
        graphs[n] = capture(lambda n=n: body(n))

    def run(n_steps):
        for _ in range(n_steps // ncopy):
            graphs[ncopy].replay()
        if n_steps % ncopy:
            graphs[n_steps % ncopy].replay()

    run(warmup)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    spin()
    start.record(stream)
    run(steps)
    end.record(stream)
    end.synchronize()
    torch.cuda.synchronize()
    sec = start.elapsed_time(end) / 1e3 / steps
    sustained = time_graph(graphs[ncopy], sustained_replays, stream) / ncopy
    return sec, sustained


def bench_layer(steps: int, warmup: int):
    """C2: the seven linears of one layer, nested absmax, bf16 x."""
    import torch

    from ttspipe_amd import _lib
    from ttspipe_amd.quant import NF4_CODE

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    step_bytes = sum(nf4_bytes(M, K, True) for _, M, K in LAYER)
    weight_bytes = sum(M * K // 2 for _, M, K in LAYER)
    ncopy = max(2, math.ceil(2 * MALL_BYTES / weight_bytes))  # > 512 MB of weights in rotation
    copies = [[Linear(M, K, True, seed=1000 * c + i, device=dev) for i, (_, M, K) in enumerate(LAYER)]
              for c in range(ncopy)]
    xs = {K: torch.randn(K, device=dev).to(torch.bfloat16) for K in {K for _, _, K in LAYER}}
    ys = {name: torch.empty(M, dtype=torch.bfloat16, device=dev) for name, M, _ in LAYER}

    def body(n):
        st = torch.cuda.current_stream().cuda_stream
        for layer in copies[:n]:
            for (name, M, K), lin in zip(LAYER, layer):
                launch(lib, lut, lin, xs[K], ys[name], _lib.DT_BF16, st)

    body(ncopy)
    torch.cuda.synchronize()
    sec, sustained = time_exact_steps(body, ncopy, steps, warmup)
    return {"step_bytes": step_bytes, "sec_per_step": sec, "steps": steps, "copies": ncopy, "warmup": warmup,
            "sustained_sec_per_step": sustained}


def bench_fused_layer(steps: int, warmup: int):
    """The decode block's launch structure for one layer's linears (4 launches)."""
    import torch

    from ttspipe_amd import _lib
    from ttspipe_amd.quant import NF4_CODE

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    step_bytes = fused_layer_bytes()
    weight_bytes = sum(M * K // 2 * (2 if n == "gate_up" else 1) for n, M, K in FUSED_LAYER)
    ncopy = max(2, math.ceil(2 * MALL_BYTES / weight_bytes))
    copies = []
    for c in range(ncopy):
        layer = {}
        for i, (name, M, K) in enumerate(FUSED_LAYER):
            layer[name] = Linear(M, K, True, seed=3000 + 10 * c + i, device=dev)
            if name == "gate_up":
                layer["up"] = Linear(M, K, True, seed=7000 + 10 * c + i, device=dev)
        copies.append(layer)
    xs = {K: torch.randn(K, device=dev).to(torch.bfloat16) for K in {K for _, _, K in FUSED_LAYER}}
    ys = {name: torch.empty(M, dtype=torch.bfloat16, device=dev) for name, M, _ in FUSED_LAYER}

    def body(n):
        st = torch.cuda.current_stream().cuda_stream
        for layer in copies[:n]:
            for name, M, K in FUSED_LAYER:
                if name == "gate_up":
                    launch_swiglu(lib, lut, layer[name], layer["up"], xs[K], ys[name], st)
                else:
                    launch(lib, lut, layer[name], xs[K], ys[name], _lib.DT_BF16, st)

    body(ncopy)
    torch.cuda.synchronize()
    sec, sustained = time_exact_steps(body, ncopy, steps, warmup)
    return {"step_bytes": step_bytes, "sec_per_step": sec, "steps": steps, "copies": ncopy, "warmup": warmup,
            "sustained_sec_per_step": sustained}


def bench_kernel(M, K, nested, dtype_name, launches_per_copy=1, min_bytes=2 * MALL_BYTES, direct=False):
    """One GEMV shape alone: average seconds per launch over > 512 MB of distinct weights.

    direct=True launches each copy once without a graph (for counter runs,
    where every dispatch is profiled on its own)."""
    import torch

    from ttspipe_amd import _lib
    from ttspipe_amd.quant import NF4_CODE

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    dt = _lib.DT_BF16 if dtype_name == "bf16" else _lib.DT_F16
    tdt = torch.bfloat16 if dt == _lib.DT_BF16 else torch.float16
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    ncopy = max(2, math.ceil(min_bytes / (M * K // 2)))
    lins = [Linear(M, K, nested, seed=77 + c, device=dev) for c in range(ncopy)]
    x = torch.randn(K, device=dev).to(tdt)
    y = torch.empty(M, dtype=tdt, device=dev)

    def body():
        st = torch.cuda.current_stream().cuda_stream
        for lin in lins:
            launch(lib, lut, lin, x, y, dt, st)

    body()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    if direct:
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        spin()
        start.record(stream)
        body()
        end.record(stream)
        end.synchronize()
        reps, sec = 1, start.elapsed_time(end) / 1e3 / ncopy
    else:
        # back to back: the launch-to-launch interval of graph-replayed launches
        graph = capture(body)
        time_graph(graph, 3, stream)
        reps = max(3, 2000 // ncopy)
        sec = time_graph(graph, reps, stream) / ncopy
    nbytes = nf4_bytes(M, K, nested, 2)
    del lins
    return {"M": M, "K": K, "nested": nested, "dtype": dtype_name, "sec": sec, "bytes": nbytes,
            "gbs": nbytes / sec / 1e9, "launches": reps * ncopy, "copies": ncopy}


MFMA_PEAK_TFLOPS = 2500.0  # dense bf16


def bench_gemm(rows: int = 512, copies: int = 4, reps: int = 20):
    """C4: a `rows`-token prefill through the seven projections of one layer
    (X bf16 [rows, K] x NF4 nested weights -> bf16 [rows, M]), each projection
    timed alone, graph-replayed over `copies` weight copies."""
    import torch

    from ttspipe_amd import _lib
    from ttspipe_amd.quant import NF4_CODE

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    res, total_s, total_flop = [], 0.0, 0
    # the seven projections of the reference's table, then wqkv as the
    # prefill block runs it (q, k and v rows of one weight, one launch)
    for i, (name, M, K) in enumerate(LAYER + [("qkv", 6144, 2560)]):
        lins = [Linear(M, K, True, seed=500 + 10 * i + c, device=dev) for c in range(copies)]
        x = torch.randn(rows, K, device=dev).to(torch.bfloat16)
        y = torch.empty(rows, M, dtype=torch.bfloat16, device=dev)
        # the K split nf4gemv.matmul uses for this shape (fp32 partials in a workspace)
        splits = lib.ttsp_nf4_gemm_splits(M, K, rows)
        work = torch.empty(splits * rows * M, dtype=torch.float32, device=dev)

        def body():
            st = torch.cuda.current_stream().cuda_stream
            for lin in lins:
                rc = lib.ttsp_nf4_gemm_split(x.data_ptr(), _lib.DT_BF16, lin.w.data_ptr(), _lib.ptr(lin.a8),
                                             lin.amax.data_ptr(), _lib.ptr(lin.code2), lin.offset, lut.data_ptr(),
                                             y.data_ptr(), 0, 0, M, K, rows, 64, 256, work.data_ptr(), splits, st)
                if rc:
                    raise RuntimeError(f"ttsp_nf4_gemm_split failed: {rc}")

        body()
        torch.cuda.synchronize()
        graph = capture(body)
        stream = torch.cuda.current_stream()
        time_graph(graph, 2, stream)
        sec = time_graph(graph, reps, stream) / copies
        flop = 2 * rows * M * K
        res.append({"name": name, "M": M, "K": K, "k_splits": splits, "us": round(sec * 1e6, 2),
                    "tflops": round(flop / sec / 1e12, 1)})
        if name != "qkv":
            total_s += sec
            total_flop += flop
        del lins
    out = {"rows": rows, "projections": res, "layer_us": round(total_s * 1e6, 1),
           "tflops": round(total_flop / total_s / 1e12, 1),
           "pct_of_mfma_peak": round(100 * total_flop / total_s / 1e12 / MFMA_PEAK_TFLOPS, 2)}
    # gate and up as the prefill block runs them: one SwiGLU launch
    (_, M, K), = [p for p in LAYER if p[0] == "gate"]
    if lib.ttsp_nf4_gemm_swiglu_fits(M, K, rows, 64, 256, 1):
        pairs = [(Linear(M, K, True, seed=700 + c, device=dev), Linear(M, K, True, seed=750 + c, device=dev))
                 for c in range(copies)]
        x = torch.randn(rows, K, device=dev).to(torch.bfloat16)
        y = torch.empty(rows, M, dtype=torch.bfloat16, device=dev)

        def body_sw():
            st = torch.cuda.current_stream().cuda_stream
            for l1, l3 in pairs:
                rc = lib.ttsp_nf4_gemm_swiglu(x.data_ptr(), _lib.DT_BF16, l1.w.data_ptr(), l1.a8.data_ptr(),
                                              l1.amax.data_ptr(), l1.code2.data_ptr(), l1.offset, l3.w.data_ptr(),
                                              l3.a8.data_ptr(), l3.amax.data_ptr(), l3.code2.data_ptr(), l3.offset,
                                              lut.data_ptr(), y.data_ptr(), M, K, rows, 64, 256, st)
                if rc:
                    raise RuntimeError(f"ttsp_nf4_gemm_swiglu failed: {rc}")

        body_sw()
        torch.cuda.synchronize()
        graph = capture(body_sw)
        stream = torch.cuda.current_stream()
        time_graph(graph, 2, stream)
        sec = time_graph(graph, reps, stream) / copies
        flop = 2 * 2 * rows * M * K
        sep = sum(r["us"] for r in res if r["name"] in ("gate", "up")) * 1e-6
        layer = total_s - sep + sec
        out["swiglu_gate_up"] = {"us": round(sec * 1e6, 2), "tflops": round(flop / sec / 1e12, 1),
                                 "two_launches_us": round(sep * 1e6, 2)}
        out["layer_us_with_one_swiglu_launch"] = round(layer * 1e6, 1)
        out["pct_of_mfma_peak_with_one_swiglu_launch"] = round(
            100 * total_flop / layer / 1e12 / MFMA_PEAK_TFLOPS, 2)
        # the prefill block's four launches: wqkv, wo, the SwiGLU pair, w2
        us = {r["name"]: r["us"] * 1e-6 for r in res}
        block = us["qkv"] + us["o"] + sec + us["down"]
        out["prefill_block_launches_us"] = round(block * 1e6, 1)
        out["pct_of_mfma_peak_prefill_block_launches"] = round(
            100 * total_flop / block / 1e12 / MFMA_PEAK_TFLOPS, 2)
        del pairs
    return out


def bench_small_n(ns=(1, 2, 4, 8, 16, 32), min_bytes: int = 2 * MALL_BYTES, replays: int = 20):
    """The reference's small-N table (nf4gemv.py:20-28: a frame of matmuls at
    N = 1, 8, 16, 32 input rows): the seven projections of one layer at N
    bf16 rows each (N = 1 through the GEMV, N > 1 through the MFMA GEMM),
    graph-replayed over > 512 MB of distinct weight copies. Reports us per
    layer and the effective rate (the layer's algorithmic bytes at N rows per
    second), the reference's "effective" column."""
    import torch

    from ttspipe_amd import _lib
    from ttspipe_amd.quant import NF4_CODE

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
    weight_bytes = sum(M * K // 2 for _, M, K in LAYER)
    ncopy = max(2, math.ceil(min_bytes / weight_bytes))
    copies = [[Linear(M, K, True, seed=9000 + 10 * c + i, device=dev) for i, (_, M, K) in enumerate(LAYER)]
              for c in range(ncopy)]
    out = []
    for n in ns:
        xs = {K: torch.randn(n, K, device=dev).to(torch.bfloat16) for K in {K for _, _, K in LAYER}}
        ys = {name: torch.empty(n, M, dtype=torch.bfloat16, device=dev) for name, M, _ in LAYER}

        def body():
            st = torch.cuda.current_stream().cuda_stream
            for layer in copies:
                for (name, M, K), lin in zip(LAYER, layer):
                    rc = lib.ttsp_nf4_gemm(xs[K].data_ptr(), _lib.DT_BF16, lin.w.data_ptr(), _lib.ptr(lin.a8),
                                           lin.amax.data_ptr(), _lib.ptr(lin.code2), lin.offset, lut.data_ptr(),
                                           ys[name].data_ptr(), 0, 0, M, K, n, 64, 256, st)
                    if rc:
                        raise RuntimeError(f"ttsp_nf4_gemm failed: {rc}")

        def body_pair():  # gate and up as the prefill block runs them: one launch (silu(gate) * up)
            st = torch.cuda.current_stream().cuda_stream
            for layer in copies:
                for (name, M, K), lin in zip(LAYER, layer):
                    if name == "gate":
                        continue
                    if name != "up":
                        rc = lib.ttsp_nf4_gemm(xs[K].data_ptr(), _lib.DT_BF16, lin.w.data_ptr(), _lib.ptr(lin.a8),
                                               lin.amax.data_ptr(), _lib.ptr(lin.code2), lin.offset, lut.data_ptr(),
                                               ys[name].data_ptr(), 0, 0, M, K, n, 64, 256, st)
                        if rc:
                            raise RuntimeError(f"ttsp_nf4_gemm failed: {rc}")
                        continue
                    g = layer[[nm for nm, _, _ in LAYER].index("gate")]
                    pair = (g.w.data_ptr(), _lib.ptr(g.a8), g.amax.data_ptr(), _lib.ptr(g.code2), g.offset,
                            lin.w.data_ptr(), _lib.ptr(lin.a8), lin.amax.data_ptr(), _lib.ptr(lin.code2), lin.offset,
                            lut.data_ptr(), ys[name].data_ptr())
                    if n <= 2:
                        rc = lib.ttsp_nf4_gemv_fused_rows(xs[K].data_ptr(), _lib.DT_BF16, None, 0.0, *pair, 0, 0, M,
                                                          K, n, 64, 256, st)
                    else:
                        rc = lib.ttsp_nf4_gemm_swiglu(xs[K].data_ptr(), _lib.DT_BF16, *pair, M, K, n, 64, 256, st)
                    if rc:
                        raise RuntimeError(f"gate and up in one launch failed: {rc}")

        stream = torch.cuda.current_stream()
        point = {"rows": n}
        for key, fn in (("", body), ("_gate_up_one_launch", body_pair)):
            if key and n > 2 and not lib.ttsp_nf4_gemm_swiglu_fits(9728, 2560, n, 64, 256, 1):
                continue
            fn()
            torch.cuda.synchronize()
            graph = capture(fn)
            time_graph(graph, 2, stream)
            sec = time_graph(graph, replays, stream) / ncopy
            point["layer_us" + key] = round(sec * 1e6, 2)
            if not key:
                nbytes = sum(nf4_bytes(M, K, True, 2) + 2 * (n - 1) * (M + K) for _, M, K in LAYER)
                point["effective_gbs"] = round(nbytes / sec / 1e9, 1)
            del graph
        out.append(point)
    for r in out:
        r["rel_to_n1"] = round(r["layer_us"] / out[0]["layer_us"], 2)
        if "layer_us_gate_up_one_launch" in r:
            r["rel_to_n1_gate_up_one_launch"] = round(
                r["layer_us_gate_up_one_launch"] / out[0]["layer_us_gate_up_one_launch"], 2)
    return {"layer": "q, k, v, o, gate, up, down (7 launches), NF4 nested, bf16; "
            "_gate_up_one_launch: gate and up as one launch, as the prefill block runs them (6 launches)",
            "copies": ncopy, "points": out}


def bench_norm_rope(min_bytes: int = 2 * MALL_BYTES, replays: int = 20):
    """RMSNorm of hidden [S, 2560] and rotary of q [S, 32, 128] and k
    [S, 8, 128] (bf16, theta 1e6 table, random positions in [0, 4096)) at
    decode (S = 1) and prefill (S = 512), each op over distinct input copies
    (> 512 MB for the prefill shapes) so the inputs stream from HBM.
    Algorithmic bytes: norm 2*S*D*2 + 2*D; rotary per tensor 2*S*H*128*2 plus
    its S rows of the table (read once per tensor: q and k are two launches)."""
    import torch

    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    lib = _lib.load()
    dev = torch.device("cuda", 0)
    D, nh, nkv, hd, eps = 2560, 32, 8, 128, 1e-6
    g = torch.Generator(device=dev).manual_seed(31)
    table = precompute_freqs_cis(4096, hd, 1e6).to(dev)
    out = {}
    for S in (1, 512):
        per = 2 * S * D * 2 + 2 * (S * (nh + nkv) * hd * 2)
        ncopy = max(4, min(400, math.ceil(min_bytes / per)))
        xs = [torch.randn(S, D, device=dev, generator=g).to(torch.bfloat16) for _ in range(ncopy)]
        w = (1.0 + 0.1 * torch.randn(D, device=dev, generator=g)).to(torch.bfloat16)
        q = [torch.randn(1, S, nh, hd, device=dev, generator=g).to(torch.bfloat16) for _ in range(ncopy)]
        k = [torch.randn(1, S, nkv, hd, device=dev, generator=g).to(torch.bfloat16) for _ in range(ncopy)]
        pos = torch.randint(0, 4096, (S,), device=dev, generator=g)
        f = table.index_select(0, pos).contiguous()
        yn = torch.empty(S, D, dtype=torch.bfloat16, device=dev)
        yq, yk = torch.empty_like(q[0]), torch.empty_like(k[0])

        def norm_body():
            st = torch.cuda.current_stream().cuda_stream
            for x in xs:
                _lib.check(lib.ttsp_rms_norm(x.data_ptr(), w.data_ptr(), yn.data_ptr(), S, D, eps, _lib.DT_BF16, st),
                           "ttsp_rms_norm")

        def rope_body():
            st = torch.cuda.current_stream().cuda_stream
            for a, b in zip(q, k):
                for t, y, h in ((a, yq, nh), (b, yk, nkv)):
                    _lib.check(lib.ttsp_rope(t.data_ptr(), f.data_ptr(), _lib.DT_BF16, y.data_ptr(), t.numel() // 2,
                                             hd // 2, h, S, _lib.DT_BF16, st), "ttsp_rope")

        res = {}
        for name, body, launches, nbytes in (
                ("rms_norm", norm_body, 1, 2 * S * D * 2 + 2 * D),
                ("rope_qk", rope_body, 2, 2 * S * (nh + nkv) * hd * 2 + 2 * S * (hd // 2) * 2 * 2)):
            body()
            torch.cuda.synchronize()
            graph = capture(body)
            stream = torch.cuda.current_stream()
            time_graph(graph, 2, stream)
            sec = time_graph(graph, replays, stream) / ncopy
            res[name] = {"us": round(sec * 1e6, 3), "launches": launches, "bytes": nbytes,
                         "gbs": round(nbytes / sec / 1e9, 1),
                         "pct_of_hbm_peak": round(100 * nbytes / sec / 1e9 / HBM_PEAK_GBS, 2)}
        res["copies"] = ncopy
        out["decode_1" if S == 1 else f"prefill_{S}"] = res
        del xs, q, k
    return out


def bench_prefill_attention(cases=((512, 0), (512, 1536), (64, 2000)), n_head: int = 32, n_kv: int = 8,
                            reps: int = 20):
    """Prefill attention of `rows` new positions (32 q / 8 kv heads of 128,
    bf16) over a cached prefix, for each (rows, prefix) case, with the fork's
    causal mask, as the HIP path runs it (one launch, or a key split and its
    merge for a short run over a long cache); torch's
    scaled_dot_product_attention with the same boolean mask (the reference's
    path beyond 64 positions) timed beside it, and the causal form the
    prefill block runs (`positions=`: the mask computed from the rows'
    positions, `us_causal`). FLOPs count the allowed (query, key) pairs:
    4 * 128 per pair and head."""
    import torch
    import torch.nn.functional as F

    from ttspipe_amd import _lib, fastpath

    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev).manual_seed(11)
    out = []
    for rows, prefix in cases:
        L = prefix + rows
        splits = _lib.lib().ttsp_prefill_attention_splits(rows, n_kv, L)
        work = torch.empty(max(fastpath.prefill_work_floats(rows, n_head, splits), 4), device=dev)
        max_len = ((L + 255) // 256) * 256
        q = torch.randn(1, rows, n_head, 128, device=dev, generator=g).to(torch.bfloat16).transpose(1, 2)
        kc = torch.randn(1, n_kv, max_len, 128, device=dev, generator=g).to(torch.bfloat16)
        vc = torch.randn(1, n_kv, max_len, 128, device=dev, generator=g).to(torch.bfloat16)
        k, v = kc[:, :, :L], vc[:, :, :L]
        causal = torch.tril(torch.ones(max_len, max_len, dtype=torch.bool, device=dev))
        pos = torch.arange(prefix, L, device=dev)
        mask = causal[None, None, pos][..., :L]
        y = torch.empty(1, rows, n_head * 128, dtype=torch.bfloat16, device=dev)

        def ours():
            if fastpath.prefill_attention(q, k, v, mask, n_head, n_kv, 128, out=y, work=work) is None:
                raise RuntimeError("prefill attention declined")

        def ours_causal():
            if fastpath.prefill_attention(q, k, v, None, n_head, n_kv, 128, out=y, work=work, positions=pos) is None:
                raise RuntimeError("prefill attention declined")

        def sdpa():
            F.scaled_dot_product_attention(q, k, v, attn_mask=mask, enable_gqa=True)

        times = {}
        for name, fn in (("hip", ours), ("causal", ours_causal), ("sdpa", sdpa)):
            fn()
            torch.cuda.synchronize()
            graph = capture(lambda fn=fn: [fn() for _ in range(4)])
            stream = torch.cuda.current_stream()
            time_graph(graph, 2, stream)
            times[name] = time_graph(graph, reps, stream) / 4
        pairs = rows * prefix + rows * (rows + 1) // 2
        flop = 4 * 128 * pairs * n_head
        out.append({"rows": rows, "prefix": prefix, "key_splits": splits, "us": round(times["hip"] * 1e6, 2),
                    "tflops": round(flop / times["hip"] / 1e12, 1),
                    "pct_of_mfma_peak": round(100 * flop / times["hip"] / 1e12 / MFMA_PEAK_TFLOPS, 2),
                    "us_causal": round(times["causal"] * 1e6, 2),
                    "tflops_causal": round(flop / times["causal"] / 1e12, 1),
                    "pct_of_mfma_peak_causal": round(100 * flop / times["causal"] / 1e12 / MFMA_PEAK_TFLOPS, 2),
                    "torch_sdpa_us": round(times["sdpa"] * 1e6, 1)})
    return out


def bench_copy(nbytes: int = 64 * 2**20, launches: int = 8):
    """A plain device copy of known size (reads and writes `nbytes` each), the
    calibration kernel for the HBM byte counters."""
    import torch

    src = torch.randint(0, 255, (launches, nbytes), dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(launches):
        dst[i].copy_(src[i])
    end.record()
    end.synchronize()
    sec = start.elapsed_time(end) / 1e3 / launches
    return {"bytes_read": nbytes, "bytes_written": nbytes, "sec": sec, "gbs_rw": 2 * nbytes / sec / 1e9}


def cpu_baseline(seconds: float = 10.0, decode_frames: int = 3):
    """The reference's CPU NF4 GEMV algorithm (restated in C++) on this host,
    and the synthetic Dual-AR frame through the same kernels (`decode`)."""
    try:
        from oracle import cpu_baseline as cb
    except Exception as exc:  # noqa: BLE001
        return {"value": None, "unit": "GB/s", "cores": None, "kind": "port", "sample": f"unavailable: {exc}"}
    out = cb.run(LAYER, seconds=seconds)
    if decode_frames > 0:
        out["decode"] = cb.run_decode(frames=decode_frames)
    return out


def roofline_entry(kern: dict) -> dict:
    """The dominant kernel against HBM. `achieved`: algorithmic bytes per
    launch over the live launch-to-launch interval of graph-replayed launches
    (HIP events on the launch stream). Beside it the kernel trace's dispatch
    durations of the same command and the counter traffic, both only while
    their launch key matches the launch made here."""
    key = gemv_launch_key(kern["M"], kern["K"])
    current = key == GEMV_PROFILE["key"]
    nbytes = kern["bytes"]
    out = {
        "bound": "hbm",
        "kernel": "nf4_gemv_kernel (gate 9728x2560, nested, bf16)",
        "achieved": round(kern["gbs"], 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(kern["gbs"] / HBM_PEAK_GBS, 4),
        "traffic": GEMV_PROFILE["traffic_bytes"] if current else None,
        "bytes_per_launch": nbytes,
        "avg_launch_us": round(kern["sec"] * 1e6, 3),
        "avg_launch_us_is": "launch-to-launch interval of back-to-back graph-replayed launches (HIP events), "
                            "weights rotated past the Infinity Cache",
        "launch_key": key,
        "rocprof_summary": GEMV_PROFILE["summary"],
    }
    if current:
        med, mean = GEMV_PROFILE["rocprof_median_us"], GEMV_PROFILE["rocprof_mean_us"]
        out["rocprof"] = {"median_us": med, "mean_us": mean,
                          "frac_at_median": round(nbytes / (med * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                          "frac_at_mean": round(nbytes / (mean * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    else:
        out["stale"] = ("the committed rocprof figures were measured on another launch "
                        f"({GEMV_PROFILE['key']}); re-profile")
    return out


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--only", choices=["layer", "kernel", "c1", "copy", "decode", "gemm", "pattn", "prefill",
                                       "prefill512", "smalln", "normrope"],
                    default=None,
                    help="run one GPU measurement only (for profiling runs)")
    ap.add_argument("--decode-steps", type=int, default=256, help="greedy frames the decode benchmark times")
    ap.add_argument("--cpu-decode-frames", type=int, default=3, help="frames the CPU baseline's decode times")
    ap.add_argument("--direct", action="store_true",
                    help="with --only kernel/c1: one launch per weight copy, no graph (counter runs)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this path has no multi-GPU mode (the value is one GPU's "
              "throughput; sharded, each GPU would stream its own share of every weight's rows)",
              file=sys.stderr)
        return 2

    import torch

    torch.cuda.set_device(0)
    out = {}
    if args.only in (None, "layer"):
        out["layer_fused"] = bench_fused_layer(args.steps, args.warmup)
        out["layer"] = bench_layer(args.steps, args.warmup)
    if args.only in (None, "kernel"):
        out["kernel"] = bench_kernel(9728, 2560, True, "bf16", direct=args.direct)
    if args.only in (None, "c1"):
        out["c1"] = bench_kernel(9728, 2560, False, "fp16", direct=args.direct)
    if args.only == "copy":
        out["copy"] = bench_copy()
    if args.only in (None, "gemm"):
        out["gemm"] = bench_gemm()
    if args.only in (None, "pattn"):
        out["pattn"] = bench_prefill_attention()
    if args.only in (None, "smalln"):
        out["smalln"] = bench_small_n()
    if args.only in (None, "normrope"):
        out["normrope"] = bench_norm_rope()
    if args.only in (None, "prefill", "prefill512"):
        from ttspipe_amd import dualar

        out["prefill"] = dualar.prefill_benchmark(512)
        if args.only != "prefill512":  # (the 512-token prompt alone: its kernel trace)
            out["prefill_tail"] = dualar.prefill_tail_benchmark()
    decode = None
    if args.only in (None, "decode") and not args.skip_decode:
        from ttspipe_amd import dualar

        decode = dualar.benchmark(n_steps=args.decode_steps)
        decode["pct_of_hbm_peak"] = round(100 * decode["achieved_gbs"] / HBM_PEAK_GBS, 1)
        out["decode"] = decode
    if args.only is not None:
        print(json.dumps(out))
        return 0
    cpu = None if args.skip_cpu else cpu_baseline(args.cpu_seconds, 0 if args.skip_decode else args.cpu_decode_frames)

    layer, kern, c1, fused = out["layer"], out["kernel"], out["c1"], out["layer_fused"]
    value = fused["step_bytes"] / fused["sec_per_step"] / 1e9
    separate = layer["step_bytes"] / layer["sec_per_step"] / 1e9
    line = {
        "metric": "NF4 GEMV HBM GB/s (% of peak) + decode step ms/token, 4B-dim model, 1 GPU",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": fused["steps"],
        "warmup": fused["warmup"],
        "ms_per_step": round(fused["sec_per_step"] * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "all batch-1 linears of one Qwen3-4B-shaped decoder layer: q 2560->4096, k/v 2560->1024, "
                        "o 4096->2560, gate/up 2560->9728, down 9728->2560; NF4 bs64, double-quant absmax "
                        "(uint8, bs2 256, fp32 scale+offset); x bf16; run as the fused decode block runs them "
                        "(q/k/v as one wqkv GEMV, gate/up as one SwiGLU GEMV: 4 launches)",
            "bytes_per_step": fused["step_bytes"],
            "weight_copies_rotated": fused["copies"],
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 1),
            "sustained_over_100_replays": {
                "steps": 100 * fused["copies"],
                "gbs": round(fused["step_bytes"] / fused["sustained_sec_per_step"] / 1e9, 1),
                "ms_per_step": round(fused["sustained_sec_per_step"] * 1e3, 5)},
            "seven_separate_launches": {"gbs": round(separate, 1), "ms_per_step": round(layer["sec_per_step"] * 1e3, 5),
                                        "bytes_per_step": layer["step_bytes"]},
        },
        "roofline": roofline_entry(kern),
        "gemv_fp16_plain": {
            "shape": "9728x2560 fp16 x, fp32 absmax bs64",
            "gbs": round(c1["gbs"], 1),
            "pct_of_peak": round(100 * c1["gbs"] / HBM_PEAK_GBS, 1),
            "avg_launch_us": round(c1["sec"] * 1e6, 3),
            "bytes_per_launch": c1["bytes"],
        },
        "decode": decode,
        "prefill_gemm": out["gemm"],
        "small_n_gemm": out["smalln"],
        "norm_rope": out["normrope"],
        "prefill_attention": out["pattn"],
        "prefill_512": out["prefill"],
        "prefill_tail": out["prefill_tail"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
