"""The two elementwise chains around every matmul, one HIP kernel each.

Drop-in for the reference's `app/engine/fusedops.py`: `rms_norm(x, weight,
eps)`, `rope(x, freqs_cis)`, `install()`, `stats()`, `note_rope_fallback()`,
`enabled`, `_built()`, and class attributes `_fused_patched` /
`_fused_original_forward` on the patched `RMSNorm`.

* `rms_norm` is the fork's RMSNorm, `_norm(x.float()).type_as(x) * weight`:
  fp32 sum of squares, r = 1/sqrt(mean + eps) (correctly rounded sqrt and
  divide), rounded to the activation type after `x * r` and again after the
  weight multiply (reference: fusedops.py:8-14, 61-94).
* `rope` is `apply_rotary_emb` on interleaved pairs with separately rounded
  products and sum (no fma), bit-identical to the fork's fp32 chain
  (reference: fusedops.py:103-133).

fp16 and bf16 activations are served (the reference: fp16 only); fp32 and
non-contiguous inputs are declined with `None`, as the reference declines them
(fusedops.py:169-236).
"""

from __future__ import annotations

import logging

from ttspipe_amd import _lib

logger = logging.getLogger(__name__)

enabled = True

_stats = {"norm": 0, "norm_fallback": 0, "rope": 0, "rope_fallback": 0}


def stats() -> dict:
    return dict(_stats)


def _built():
    """The loaded library when a GPU is present, else None (the reference's contract)."""
    if not _lib.gpu_present():
        return None
    return _lib.load()


def rms_norm(x, weight, eps: float, out=None):
    """The fork's RMSNorm of x over its last axis on the GPU kernel (two
    roundings: after the normalisation and after the weight), or None when
    the kernel cannot take these tensors."""
    lib = _built()
    if lib is None or not enabled:
        return None
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or weight.dtype != x.dtype:
        return None
    if x.device.type != "cuda" or not x.is_contiguous() or not weight.is_contiguous():
        return None
    width = x.shape[-1]
    if width != weight.numel() or width == 0 or width % 8:
        return None
    if x.data_ptr() % 16 or weight.data_ptr() % 16 or (out is not None and out.data_ptr() % 16):
        return None
    if out is None:
        import torch

        out = torch.empty_like(x)
    rc = lib.ttsp_rms_norm(x.data_ptr(), weight.data_ptr(), out.data_ptr(), x.numel() // width, width,
                           float(eps), dt, _lib.stream())
    _lib.check(rc, "ttsp_rms_norm")
    _stats["norm"] += 1
    return out


def rope(x, freqs_cis, out=None):
    """Rotary embedding of `x` (B, S, H, D) against `freqs_cis` (S, D/2, 2), or None."""
    lib = _built()
    if lib is None or not enabled:
        return None
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or x.device.type != "cuda" or not x.is_contiguous():
        return None
    if not freqs_cis.is_contiguous() or x.dim() != 4 or freqs_cis.device != x.device:
        return None
    ftype = _lib.dtype_code(freqs_cis.dtype)
    if ftype is None:
        return None
    bsz, seq, heads, head_dim = x.shape
    half_dim = head_dim // 2
    if head_dim % 2 or freqs_cis.numel() != seq * half_dim * 2 or x.numel() == 0:
        return None
    if x.data_ptr() % 4 or (out is not None and out.data_ptr() % 4):  # a pair is one 32-bit word
        return None
    if out is None:
        import torch

        out = torch.empty_like(x)
    rc = lib.ttsp_rope(x.data_ptr(), freqs_cis.data_ptr(), ftype, out.data_ptr(), x.numel() // 2,
                       half_dim, heads, seq, dt, _lib.stream())
    _lib.check(rc, "ttsp_rope")
    _stats["rope"] += 1
    return out


def note_rope_fallback() -> None:
    """Called by an attention forward that had to use the unfused rotary."""
    _stats["rope_fallback"] += 1


def _norm_classes():
    from ttspipe_amd.llama import RMSNorm

    classes = [RMSNorm]
    try:
        from fish_speech.models.text2semantic.llama import RMSNorm as ForkRMSNorm

        classes.append(ForkRMSNorm)
    except Exception:  # noqa: BLE001
        pass
    return classes


def install() -> bool:
    """Route `RMSNorm.forward` through the fused kernel. Idempotent."""
    if _built() is None:
        return False
    for cls in _norm_classes():
        if getattr(cls, "_fused_patched", False):
            continue
        original_forward = cls.forward

        def forward(self, x, _original=original_forward):
            out = rms_norm(x, self.weight, self.eps)
            if out is not None:
                return out
            _stats["norm_fallback"] += 1
            return _original(self, x)

        cls.forward = forward
        cls._fused_patched = True
        cls._fused_original_forward = original_forward
    return True
