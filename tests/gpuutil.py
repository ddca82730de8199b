"""Helpers for GPU tests: torch <-> numpy bit patterns, oracle-side views."""

from __future__ import annotations

import ctypes

import numpy as np
import torch

from oracle import oracle as o


def bits(t: torch.Tensor) -> np.ndarray:
    """16-bit tensor (any device) -> flat uint16 numpy bit pattern; fp32 -> float32."""
    t = t.detach().contiguous().cpu()
    if t.dtype == torch.float32:
        return t.numpy().reshape(-1)
    return t.view(torch.int16).numpy().view(np.uint16).reshape(-1)


def from_bits(a: np.ndarray, dtype, device="cuda") -> torch.Tensor:
    a = np.ascontiguousarray(a)
    if dtype == torch.float32:
        return torch.from_numpy(a.astype(np.float32)).to(device)
    return torch.from_numpy(a.view(np.int16).copy()).view(dtype).to(device)


def dt_code(dtype) -> int:
    return {torch.float16: o.DT_F16, torch.bfloat16: o.DT_BF16, torch.float32: o.DT_F32}[dtype]


def randn_bits(n: int, dtype, seed: int, scale: float = 1.0) -> np.ndarray:
    x = (np.random.default_rng(seed).standard_normal(n) * scale).astype(np.float32)
    return o.from_f32(x, dt_code(dtype))


def gemv_shape(M: int, K: int):
    from ttspipe_amd import _lib

    J, KS, RPW = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = _lib.load().ttsp_gemv_shape(M, K, ctypes.byref(J), ctypes.byref(KS), ctypes.byref(RPW))
    assert rc == 0
    return J.value, KS.value, RPW.value


def gemv_rows_shape(M: int, K: int, N: int):
    """(J, KS, RPW) of N activation rows through the GEMV, or None when those
    rows take the MFMA kernels."""
    from ttspipe_amd import _lib

    J, KS, RPW = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = _lib.load().ttsp_gemv_rows_shape(M, K, N, ctypes.byref(J), ctypes.byref(KS), ctypes.byref(RPW))
    return (J.value, KS.value, RPW.value) if rc == 0 else None


def first_mismatch(a: np.ndarray, b: np.ndarray) -> str:
    idx = np.flatnonzero(a != b)
    if idx.size == 0:
        return "identical"
    i = int(idx[0])
    return f"{idx.size} of {a.size} differ; first at {i}: {a[i]} vs {b[i]}"
