"""ctypes binding of `libttsp_hip.so`, the C-ABI the Python modules call.

This replaces the reference's NVRTC/driver FFI (app/engine/nvrtc.py:76-198):
the kernels are compiled ahead of time by hipcc for gfx950 (see `build.py`),
and every entry point takes raw device pointers, sizes and a `hipStream_t`
and returns a `hipError_t` (0 = success). Nothing in the library allocates.

Loading is lazy. `gpu_present()` answers whether a GPU is visible without
raising; `lib()` raises if the library is missing, because on a machine with a
GPU the kernels are the product and there is no silent substitute for them.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libttsp_hip.so"

#: Element-type codes of the C-ABI (`include/ttsp_hip.h`).
DT_F16, DT_BF16, DT_F32 = 0, 1, 2

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_ll = ctypes.c_longlong



class Nf4Weight(ctypes.Structure):
    """`ttsp_nf4_weight`: one NF4 weight's device pointers (A8 NULL: plain scales)."""

    _fields_ = [("W", _vp), ("A8", _vp), ("AMAX", _vp), ("CODE2", _vp), ("offset", _f)]


class FastLayer(ctypes.Structure):
    """`ttsp_fast_layer`: one fast-transformer layer for `ttsp_fast_steps`."""

    _fields_ = [("wqkv", Nf4Weight), ("wo", Nf4Weight), ("w1", Nf4Weight), ("w3", Nf4Weight), ("w2", Nf4Weight),
                ("attention_norm", _vp), ("ffn_norm", _vp), ("q_norm", _vp), ("k_norm", _vp), ("k_cache", _vp),
                ("v_cache", _vp)]


#: `ttsp_fast_steps`' barrier words and the index of its failed-wait count.
FAST_SYNC_WORDS, FAST_SYNC_FAILED = 192, 128

#: name -> argtypes (restype is int for all of them)
SIGNATURES: dict[str, list] = {
    "ttsp_nf4_gemm": [_vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp],
    "ttsp_nf4_gemm_splits": [_i, _i, _i],
    "ttsp_nf4_gemm_split": [_vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _vp],
    "ttsp_nf4_gemm_partials": [_vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _i, _i, _vp, _i, _vp],
    "ttsp_nf4_gemm_split_norm": [_vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _i,
                                 _vp, _f, _vp, _vp],
    "ttsp_nf4_gemm_swiglu": [_vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _i, _i,
                             _vp],
    "ttsp_nf4_gemm_swiglu_fits": [_i, _i, _i, _i, _i, _i],
    "ttsp_nf4_gemv_fused": [_vp, _i, _vp, _f, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp,
                            _i, _i, _i, _i, _i, _vp],
    "ttsp_nf4_gemv_fused_rows": [_vp, _i, _vp, _f, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp, _vp, _f, _vp, _vp, _vp,
                                 _i, _i, _i, _i, _i, _i, _vp],
    "ttsp_nf4_dequant": [_vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _ll, _i, _i, _vp],
    "ttsp_gemv_shape": [_i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "ttsp_gemv_rows_shape": [_i, _i, _i, ctypes.POINTER(_i), ctypes.POINTER(_i), ctypes.POINTER(_i)],
    "ttsp_rms_norm": [_vp, _vp, _vp, _i, _i, _f, _i, _vp],
    "ttsp_rope": [_vp, _vp, _i, _vp, _ll, _i, _i, _i, _i, _vp],
    "ttsp_qk_rope_kv": [_vp, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp],
    "ttsp_attn_decode": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp],
    "ttsp_attn_decode_qkv": [_vp, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f,
                             _i, _vp],
    "ttsp_attn_nf4_gemv": [_vp, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _i, _i, _i, _f, _vp, _vp, _vp, _vp, _f,
                           _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "ttsp_attn_chunk": [],
    "ttsp_attn_decode_qkv_noalloc": [_vp, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _vp],
    "ttsp_attn_decode_qkv_noalloc_max_slots": [],
    "ttsp_qk_rope_kv_rows": [_vp, _ll, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    "ttsp_attn_decode_rows": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _i, _i, _vp],
    "ttsp_attn_decode_qkv_rows": [_vp, _i, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i,
                                  _f, _i, _i, _vp],
    "ttsp_qk_rope_kv_rows_partials": [_vp, _i, _vp, _vp, _f, _vp, _i, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i,
                                      _vp],
    "ttsp_prefill_attention": [_vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _vp, _i, _i, _i, _i, _f, _i,
                               _vp],
    "ttsp_prefill_max_groups": [],
    "ttsp_prefill_attention_splits": [_i, _i, _i],
    "ttsp_prefill_attention_split": [_vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _vp, _i, _i, _i, _i, _f,
                                     _i, _vp, _i, _vp],
    "ttsp_prefill_attention_causal": [_vp, _ll, _ll, _vp, _ll, _ll, _vp, _ll, _ll, _vp, _vp, _i, _i, _i, _i, _f, _i,
                                      _vp, _i, _vp],
    "ttsp_sample_topk": [_vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp],
    "ttsp_sample_max_top_k": [],
    "ttsp_sample_max_vocab": [],
    "ttsp_embed_sum": [_vp, _vp, _i, _i, _i, _vp, _i, _vp],
    "ttsp_embed_sum_rows": [_vp, _vp, _ll, _i, _i, _i, _i, _vp, _i, _vp],
    "ttsp_argmax": [_vp, _i, _i, _vp, _vp],
    "ttsp_argmax_embed": [_vp, _i, _i, _vp, _vp, _vp, _i, _i, _vp, _vp],
    "ttsp_frame_advance": [_vp, _i, _vp, _i, _vp, _vp, _vp, _i, _i, _vp, _vp],
    "ttsp_synth_fill": [_vp, _ll, ctypes.c_ulonglong, _i, _f, _f, _vp],
    "ttsp_fast_steps": [ctypes.POINTER(FastLayer), _i, ctypes.POINTER(Nf4Weight), _vp, _vp, _vp, _vp, _i, _vp, _vp,
                        _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _i, _i, _f, _i, _i, _i, _vp],
    "ttsp_fast_steps_grid": [_i, _i, _i, _i, _i, _i, _i, _i],
    "ttsp_fast_steps_work_bytes": [_i, _i, _i, _i],
}


def load() -> ctypes.CDLL:
    """Load the library and bind every signature. Raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m ttspipe_amd.build` "
                "(the HIP kernels have no substitute)"
            )
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        _lib = handle
        return _lib


def lib() -> ctypes.CDLL:
    return load()


def gpu_present() -> bool:
    """Whether a ROCm device is visible (never raises)."""
    try:
        import torch

        return bool(torch.cuda.is_available())
    except Exception:  # noqa: BLE001
        return False


def dtype_code(dtype) -> int | None:
    import torch

    return {torch.float16: DT_F16, torch.bfloat16: DT_BF16, torch.float32: DT_F32}.get(dtype)


def stream() -> int:
    """torch's current stream on the current device, as a raw hipStream_t."""
    import torch

    return torch.cuda.current_stream().cuda_stream


def check(rc: int, what: str) -> None:
    if rc:
        raise RuntimeError(f"{what} failed: hipError_t {rc}")


def ptr(t) -> int:
    return 0 if t is None else t.data_ptr()
