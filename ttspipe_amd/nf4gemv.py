"""NF4 linear layers on MI355X: one kernel library serves single-token decode and prompt prefill.

Drop-in for the reference's `app/engine/nf4gemv.py` (same public names and
behaviour: `MAX_N`, `NF4_CODE`, `EPI_*`, `available`, `prepare`, `matmul`,
`install`, `stats`, `module._nf4_fast`, class attributes `_nf4_patched` /
`_nf4_original_forward`). The packed codes and their scales stay where
bitsandbytes put them; `libttsp_hip.so` reads them directly:

* a single activation row goes to the GEMV (`csrc/nf4_gemv.hip`), a pure
  stream of the packed weight: 256-byte wave loads, both codes of a byte
  looked up at once in an LDS table, fp32 fma chains and DPP lane sums in a
  fixed order (so results are reproducible bit for bit);
* two or more rows go to the GEMM (`csrc/nf4_gemm.hip`), where each K-step's
  weight tile is dequantised into LDS and multiplied by
  `v_mfma_f32_32x32x16`: one dequantisation serves a whole tile of rows.

Unlike the reference (fp16 only, nf4gemv.py:439) both fp16 and bf16
activations are served; anything else is declined (`None`), exactly where the
reference declines (nf4gemv.py:328-376, 436-456), and the patched forward then
uses the layer's own dequantise-and-matmul path. `MAX_N` is kept for callers
that size buffers by it; a launch here takes any number of rows.
"""

from __future__ import annotations

import logging
import threading

from ttspipe_amd import _lib
from ttspipe_amd.quant import NF4_CODE

logger = logging.getLogger(__name__)

#: Rows the reference's kernel took per launch (nf4gemv.py:71). Kept for
#: callers that bucket prompts by it; `matmul` takes any count in one launch.
MAX_N = 32

#: Epilogues `matmul` can fold into the kernel's store (nf4gemv.py:424).
EPI_NONE, EPI_RESIDUAL, EPI_SILU_GATE = 0, 1, 2

_lock = threading.Lock()
_state = {"ready": None, "lut": {}}
_stats = {"fast": 0, "fallback": 0, "layers": 0}


def stats() -> dict:
    """Counters: `fast` (matmuls the kernels ran), `fallback` (calls the layer's
    own forward took), `layers` (modules prepared for the kernels)."""
    return dict(_stats)


def available() -> bool:
    """Whether the kernels are usable here.

    False without a GPU (nothing raises for that, nf4gemv.py:26-28 of the
    reference's FFI). With a GPU the library must load: a missing build is an
    error, not a slow path.
    """
    if _state["ready"] is not None:
        return _state["ready"]
    with _lock:
        if _state["ready"] is None:
            if not _lib.gpu_present():
                _state["ready"] = False
            else:
                _lib.load()
                _state["ready"] = True
    return _state["ready"]


def _lut(device):
    import torch

    key = str(device)
    t = _state["lut"].get(key)
    if t is None:
        t = torch.tensor(NF4_CODE, dtype=torch.float32, device=device)
        _state["lut"][key] = t
    return t


def prepare(module) -> bool:
    """Check one 4-bit layer once and cache the verdict on it as `_nf4_fast`.

    The cached value is the launch description (a dict) or None when the
    kernels cannot read this layer; later calls return the cached verdict.
    The conditions match the reference's (nf4gemv.py:333-376): NF4 codes on
    the GPU; a power-of-two blocksize of at least 64; in_features divisible by
    128 and by the blocksize; a 16-byte aligned packed weight; scales that are
    either fp32 per block or the uint8 + fp32 double-quantised pair, one row of
    blocks per output feature.
    """
    import torch

    cached = getattr(module, "_nf4_fast", -1)
    if cached != -1:
        return cached is not None

    def reject(why: str) -> bool:
        module._nf4_fast = None
        logger.debug("%s stays on its own forward (%s)", type(module).__name__, why)
        return False

    weight = getattr(module, "weight", None)
    quant_state = getattr(weight, "quant_state", None)
    if quant_state is None:
        return reject("no quant_state: the weight has not been packed")
    if getattr(quant_state, "quant_type", None) != "nf4":
        return reject(f"codes are {getattr(quant_state, 'quant_type', None)!r}, the kernels read only 'nf4'")
    if weight.device.type != "cuda":
        return reject(f"packed weight lives on {weight.device.type}")

    out_features, in_features = tuple(quant_state.shape)
    blocksize = int(quant_state.blocksize)
    if blocksize < 64 or blocksize & (blocksize - 1):
        return reject(f"scale block of {blocksize} codes (needs 64, 128, 256, ...)")
    if in_features % blocksize or in_features % 128:
        return reject(f"{in_features} input features do not split into 128-code steps and {blocksize}-code blocks")
    if weight.data_ptr() % 16:
        return reject("packed weight starts off a 16-byte boundary")

    nblk = in_features // blocksize
    nested = bool(getattr(quant_state, "nested", False))
    if nested:
        state2 = quant_state.state2
        bs2 = int(state2.blocksize)
        if bs2 <= 0 or bs2 & (bs2 - 1):
            return reject(f"double-quant group of {bs2} blocks is not a power of two")
        if quant_state.absmax.dtype != torch.uint8 or state2.absmax.dtype != torch.float32:
            return reject(f"double-quant scales are {quant_state.absmax.dtype}/{state2.absmax.dtype}, "
                          "the kernels read uint8 indices and fp32 group maxima")
        if state2.code.dtype != torch.float32 or state2.code.numel() != 256:
            return reject("double-quant code table is not 256 fp32 values")
        scales = (quant_state.absmax, state2.absmax, state2.code)
        offset = float(quant_state.offset)
    else:
        if quant_state.absmax.dtype != torch.float32:
            return reject(f"per-block scales are {quant_state.absmax.dtype}; the kernels read fp32")
        scales = (None, quant_state.absmax, None)
        offset = 0.0
        bs2 = 0
    if quant_state.absmax.numel() != out_features * nblk:
        return reject(f"{quant_state.absmax.numel()} scales for {out_features} rows of {nblk} blocks")
    for t in scales:
        if t is not None and (t.device != weight.device or not t.is_contiguous()):
            return reject("a scale tensor is strided or on another device than the weight")

    module._nf4_fast = {
        "nested": nested,
        "held": tuple(t for t in scales if t is not None),  # keeps the pointed-to tensors alive
        "w": weight.data_ptr(),
        "a8": _lib.ptr(scales[0]),
        "amax": scales[1].data_ptr(),
        "code2": _lib.ptr(scales[2]),
        "offset": offset,
        "lut": _lut(weight.device),
        "bs": blocksize,
        "bs2": bs2,
        "M": out_features,
        "K": in_features,
    }
    _stats["layers"] += 1
    return True


def matmul(module, x, *, epi: int = EPI_NONE, operand=None, out=None):
    """Return x times the layer's weight transposed (fp16 or bf16 rows, any
    count), or None when the kernels cannot take this call.

    `epi` folds the operation that follows in the fork into the store:
    EPI_RESIDUAL gives `operand + y`, EPI_SILU_GATE `silu(operand) * y`, each
    rounded exactly where the separate torch ops would round. `operand` must
    match the output in shape, dtype and device and be contiguous; `out`, if
    given, is written in place.
    """
    import torch

    fast = getattr(module, "_nf4_fast", None)
    if fast is None:
        return None
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or x.device.type != "cuda":
        return None
    K, M = fast["K"], fast["M"]
    if x.shape[-1] != K:
        return None
    flat = x.reshape(-1, K)
    if not flat.is_contiguous() or flat.data_ptr() % 16:
        flat = flat.contiguous()
        if flat.data_ptr() % 16:
            return None
    rows = flat.shape[0]
    if rows == 0:
        return x.new_empty(*x.shape[:-1], M)
    if epi != EPI_NONE:
        if operand is None or operand.numel() != rows * M or operand.dtype != x.dtype:
            return None
        if operand.device != x.device or not operand.is_contiguous():
            return None
    if out is None:
        out = torch.empty((rows, M), dtype=x.dtype, device=x.device)
    elif out.dtype != x.dtype or out.numel() != rows * M or not out.is_contiguous():
        return None
    lib = _lib.lib()
    splits = lib.ttsp_nf4_gemm_splits(M, K, rows) if rows > 1 else 1
    if splits > 1:
        # K split over workgroups (too few output tiles to fill the GPU): fp32
        # partials in a workspace, summed in split order by a second kernel
        work = torch.empty(splits * rows * M, dtype=torch.float32, device=x.device)
        rc = lib.ttsp_nf4_gemm_split(
            flat.data_ptr(), dt, fast["w"], fast["a8"], fast["amax"], fast["code2"], fast["offset"],
            fast["lut"].data_ptr(), out.data_ptr(), _lib.ptr(operand) if epi else 0, epi, M, K, rows,
            fast["bs"], fast["bs2"], work.data_ptr(), splits, _lib.stream())
    else:
        rc = lib.ttsp_nf4_gemm(
            flat.data_ptr(), dt, fast["w"], fast["a8"], fast["amax"], fast["code2"], fast["offset"],
            fast["lut"].data_ptr(), out.data_ptr(), _lib.ptr(operand) if epi else 0, epi, M, K, rows,
            fast["bs"], fast["bs2"], _lib.stream())
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemm failed: hipError_t {rc}")
    _stats["fast"] += 1
    return out.view(*x.shape[:-1], M)


#: Widest output row whose RMSNorm the split-K reduce folds in (eight 8-value
#: chunks per lane of one wave).
NORM_MAX_M = 4096


def matmul_partials(module, x):
    """`(work, splits)`: the K-split launch of `matmul(module, x)` without its
    reduce, work the fp32 partial sums [splits, rows, M] for a consumer that
    adds them in split order; None where the shape runs unsplit (or the
    kernels do not take the call)."""
    import torch

    fast = getattr(module, "_nf4_fast", None)
    if fast is None:
        return None
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or x.device.type != "cuda":
        return None
    K, M = fast["K"], fast["M"]
    if x.shape[-1] != K or not x.is_contiguous() or x.data_ptr() % 16:
        return None
    rows = x.numel() // K
    if rows < 2:
        return None
    lib = _lib.lib()
    splits = lib.ttsp_nf4_gemm_splits(M, K, rows)
    if splits < 2:
        return None
    work = torch.empty(splits, rows, M, dtype=torch.float32, device=x.device)
    rc = lib.ttsp_nf4_gemm_partials(
        x.data_ptr(), dt, fast["w"], fast["a8"], fast["amax"], fast["code2"], fast["offset"],
        fast["lut"].data_ptr(), M, K, rows, fast["bs"], fast["bs2"], work.data_ptr(), splits, _lib.stream())
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemm_partials failed: hipError_t {rc}")
    _stats["fast"] += 1
    return work, splits


def matmul_norm(module, x, norm_weight, eps: float, *, epi: int = EPI_NONE, operand=None):
    """`(y, rms_norm(y))` for several rows with the norm folded into the
    split-K reduce, or None where that form does not serve the call (one row,
    an unsplit shape, M over NORM_MAX_M); y is `matmul(module, x, epi=epi,
    operand=operand)` and the second output is `fusedops.rms_norm(y,
    norm_weight, eps)`, both bit for bit."""
    import torch

    fast = getattr(module, "_nf4_fast", None)
    if fast is None:
        return None
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or x.device.type != "cuda":
        return None
    K, M = fast["K"], fast["M"]
    if x.shape[-1] != K or not x.is_contiguous() or x.data_ptr() % 16 or M % 8 or M > NORM_MAX_M:
        return None
    rows = x.numel() // K
    if rows < 2:
        return None
    if (norm_weight.dtype != x.dtype or norm_weight.numel() != M or not norm_weight.is_contiguous()
            or norm_weight.data_ptr() % 16 or norm_weight.device != x.device):
        return None
    if epi != EPI_NONE:
        if operand is None or operand.numel() != rows * M or operand.dtype != x.dtype:
            return None
        if operand.device != x.device or not operand.is_contiguous() or operand.data_ptr() % 16:
            return None
    lib = _lib.lib()
    splits = lib.ttsp_nf4_gemm_splits(M, K, rows)
    if splits not in (2, 4, 8):
        return None
    out = torch.empty((rows, M), dtype=x.dtype, device=x.device)
    out_n = torch.empty((rows, M), dtype=x.dtype, device=x.device)
    work = torch.empty(splits * rows * M, dtype=torch.float32, device=x.device)
    rc = lib.ttsp_nf4_gemm_split_norm(
        x.data_ptr(), dt, fast["w"], fast["a8"], fast["amax"], fast["code2"], fast["offset"],
        fast["lut"].data_ptr(), out.data_ptr(), _lib.ptr(operand) if epi else 0, epi, M, K, rows,
        fast["bs"], fast["bs2"], work.data_ptr(), splits, norm_weight.data_ptr(), float(eps), out_n.data_ptr(),
        _lib.stream())
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemm_split_norm failed: hipError_t {rc}")
    _stats["fast"] += 1
    shape = (*x.shape[:-1], M)
    return out.view(shape), out_n.view(shape)


#: Widest input whose RMSNorm the single-row kernel folds in (one 8-value
#: chunk per thread of its 512).
NORM_MAX_K = 4096


def gemv_fits(M: int, K: int) -> bool:
    """Whether the single-row kernel takes an [M, K] weight (rows of at most
    32768 codes). `matmul` serves longer rows through the tiled kernel; the
    fused single-row forms decline them."""
    return _lib.lib().ttsp_gemv_shape(M, K, None, None, None) == 0


#: Most activation rows `matmul_fused` takes in one launch.
FUSED_MAX_ROWS = 2


def matmul_fused(module, x, *, norm_weight=None, eps: float = 1e-6, module3=None, epi: int = EPI_NONE,
                 operand=None, out=None):
    """Up to `FUSED_MAX_ROWS` input rows through `module` in a single launch
    (each weight byte looked up once for all of them), or None if not applicable.

    `norm_weight` folds the fork's RMSNorm of each row in (bit-identical to
    `fusedops.rms_norm` then `matmul`); `module3` (same shape and scales
    layout as `module`) makes it the SwiGLU pair: silu(x W1) * (x W3), rounded
    as the two-launch form `matmul(w3, epi=EPI_SILU_GATE, operand=matmul(w1))`.
    """
    import torch

    fast = getattr(module, "_nf4_fast", None)
    if fast is None:
        return None
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or x.device.type != "cuda":
        return None
    K, M = fast["K"], fast["M"]
    rows = x.numel() // K if x.shape[-1] == K else 0
    if rows < 1 or rows > FUSED_MAX_ROWS or not x.is_contiguous() or x.data_ptr() % 16:
        return None
    if rows > 1 and _lib.lib().ttsp_gemv_rows_shape(M, K, rows, None, None, None):
        return None
    if not gemv_fits(M, K):
        return None
    fast3 = None
    if module3 is not None:
        fast3 = getattr(module3, "_nf4_fast", None)
        if fast3 is None or epi != EPI_NONE:
            return None
        if (fast3["M"], fast3["K"], fast3["nested"], fast3["bs"], fast3["bs2"]) != (M, K, fast["nested"], fast["bs"],
                                                                                  fast["bs2"]):
            return None
    if norm_weight is not None:
        if K > NORM_MAX_K:
            return None
        if (norm_weight.dtype != x.dtype or norm_weight.numel() != K or not norm_weight.is_contiguous()
                or norm_weight.data_ptr() % 16 or norm_weight.device != x.device):
            return None
    if epi != EPI_NONE:
        if operand is None or operand.numel() != rows * M or operand.dtype != x.dtype:
            return None
        if operand.device != x.device or not operand.is_contiguous():
            return None
    if out is None:
        out = torch.empty((rows, M), dtype=x.dtype, device=x.device)
    elif out.dtype != x.dtype or out.numel() != rows * M or not out.is_contiguous():
        return None
    f3 = fast3 or {"w": 0, "a8": 0, "amax": 0, "code2": 0, "offset": 0.0}
    if rows > 1:
        rc = _lib.lib().ttsp_nf4_gemv_fused_rows(
            x.data_ptr(), dt, _lib.ptr(norm_weight), float(eps), fast["w"], fast["a8"], fast["amax"], fast["code2"],
            fast["offset"], f3["w"], f3["a8"], f3["amax"], f3["code2"], f3["offset"], fast["lut"].data_ptr(),
            out.data_ptr(), _lib.ptr(operand) if epi else 0, epi, M, K, rows, fast["bs"], fast["bs2"], _lib.stream())
        if rc:
            raise RuntimeError(f"ttsp_nf4_gemv_fused_rows failed: hipError_t {rc}")
        _stats["fast"] += 2 if fast3 is not None else 1
        return out.view(*x.shape[:-1], M)
    rc = _lib.lib().ttsp_nf4_gemv_fused(
        x.data_ptr(), dt, _lib.ptr(norm_weight), float(eps),
        fast["w"], fast["a8"], fast["amax"], fast["code2"], fast["offset"],
        f3["w"], f3["a8"], f3["amax"], f3["code2"], f3["offset"],
        fast["lut"].data_ptr(), out.data_ptr(), _lib.ptr(operand) if epi else 0, epi, M, K,
        fast["bs"], fast["bs2"], _lib.stream())
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemv_fused failed: hipError_t {rc}")
    _stats["fast"] += 2 if fast3 is not None else 1
    return out.view(*x.shape[:-1], M)


def matmul_swiglu(module1, module3, x, *, out=None):
    """silu(x W1^T) * (x W3^T) for several rows in one launch, rounded as the
    two-launch form `matmul(w3, x, epi=EPI_SILU_GATE, operand=matmul(w1, x))`
    and with its bits; None where one launch does not serve the shape (it
    serves where both GEMMs would run the direct-to-LDS kernel unsplit, e.g.
    385 to 512 rows of 9728 x 2560, and where both would run the few-row
    kernel, 3 to 32 rows, whose pair form reads each row tile of w1 and w3
    in one workgroup)."""
    import torch

    if not (prepare(module1) and prepare(module3)):
        return None
    f1, f3 = module1._nf4_fast, module3._nf4_fast
    dt = _lib.dtype_code(x.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16) or x.device.type != "cuda":
        return None
    K, M = f1["K"], f1["M"]
    if (f3["M"], f3["K"], f3["nested"], f3["bs"], f3["bs2"]) != (M, K, f1["nested"], f1["bs"], f1["bs2"]):
        return None
    if x.shape[-1] != K or not x.is_contiguous() or x.data_ptr() % 16:
        return None
    rows = x.numel() // K
    lib = _lib.lib()
    if not lib.ttsp_nf4_gemm_swiglu_fits(M, K, rows, f1["bs"], f1["bs2"], int(f1["nested"])):
        return None
    if out is None:
        out = torch.empty((rows, M), dtype=x.dtype, device=x.device)
    elif out.dtype != x.dtype or out.numel() != rows * M or not out.is_contiguous():
        return None
    rc = lib.ttsp_nf4_gemm_swiglu(
        x.data_ptr(), dt, f1["w"], f1["a8"], f1["amax"], f1["code2"], f1["offset"],
        f3["w"], f3["a8"], f3["amax"], f3["code2"], f3["offset"], f1["lut"].data_ptr(), out.data_ptr(),
        M, K, rows, f1["bs"], f1["bs2"], _lib.stream())
    if rc:
        raise RuntimeError(f"ttsp_nf4_gemm_swiglu failed: hipError_t {rc}")
    _stats["fast"] += 2
    return out.view(*x.shape[:-1], M)


def _classes():
    """Linear4bit classes to patch: ours, and bitsandbytes' where it is importable."""
    from ttspipe_amd.quant import Linear4bit

    classes = [Linear4bit]
    try:  # a real bitsandbytes model is served the same way (same quant_state fields)
        import bitsandbytes as bnb  # noqa: F401

        classes.append(bnb.nn.Linear4bit)
    except Exception:  # noqa: BLE001
        pass
    return classes


def install(model=None) -> bool:
    """Patch `Linear4bit.forward` (ours, and bitsandbytes' when importable) so
    that fp16/bf16 calls on NF4 layers run on the kernels; layers or calls the
    kernels cannot take keep the original forward. Class-level, so instances
    created later are covered too. Returns False when the kernels are not
    usable here (no GPU); with `model`, every layer is prepared immediately.
    """
    if not available():
        return False
    for cls in _classes():
        if getattr(cls, "_nf4_patched", False):
            continue
        original_forward = cls.forward

        def forward(self, x, _original=original_forward):
            if prepare(self):
                out = matmul(self, x)
                if out is not None:
                    if self.bias is not None:
                        out = out + self.bias.to(out.dtype)
                    return out
            _stats["fallback"] += 1
            return _original(self, x)

        cls.forward = forward
        cls._nf4_patched = True
        cls._nf4_original_forward = original_forward
    if model is not None:
        _prepare_all(model)
    return True


def _prepare_all(model) -> None:
    """Run `prepare` on every 4-bit layer of `model` up front (the checks and
    pointer gathering then never happen inside a decode step or a capture)."""
    classes = tuple(_classes())
    served = declined = 0
    for module in model.modules():
        if isinstance(module, classes):
            if prepare(module):
                served += 1
            else:
                declined += 1
    logger.info("NF4 kernels serve %d 4-bit layers; %d keep their own forward", served, declined)
