"""bitsandbytes-compatible NF4 weights without bitsandbytes.

The reference reads bitsandbytes' `Linear4bit` / `Params4bit` / `QuantState`
in place (app/engine/nf4gemv.py:315-420, duck-typed: `weight.quant_state.
{quant_type, shape, blocksize, nested, absmax, offset, state2.{absmax, code,
blocksize}}`). bitsandbytes is not part of this stack, so this module
provides the same objects and the same byte layout:

* `quantize_4bit` - NF4 with per-block absmax (bitsandbytes'
  `functional.quantize_4bit`, restated): over the row-major flattened weight,
  block b is elements [b*bs, (b+1)*bs); absmax_b = max |w| in fp32; each
  w * (1 / absmax_b) goes to the nearest NF4 code (midpoint thresholds, a
  value exactly on a midpoint takes the lower code); two codes per byte, the
  even flattened index in the high nibble.
* `compress_statistics=True` - "double quant": offset = mean(absmax);
  absmax - offset is quantised blockwise (bs2 = 256) to uint8 indices into the
  256-point signed dynamic map with fp32 absmax2 per block. The scale the
  kernels reconstruct is code2[a8[b]] * absmax2[b // bs2] + offset.
* `Linear4bit` - an `nn.Module` with `weight.quant_state`; its own forward
  is the dequantise-then-matmul path bitsandbytes' forward takes (HIP
  dequantisation kernel + torch matmul). `nf4gemv.install()` patches it.

Quantisation is a load-time data-format step (torch ops on whatever device
the weight lives on); every operation on the decode path is a HIP kernel.
"""

from __future__ import annotations

import math

import torch

#: bitsandbytes' NF4 code points (the reference's table: app/engine/nf4gemv.py:75-92).
NF4_CODE = (
    -1.0,
    -0.6961928009986877,
    -0.5250730514526367,
    -0.39491748809814453,
    -0.28444138169288635,
    -0.18477343022823334,
    -0.09105003625154495,
    0.0,
    0.07958029955625534,
    0.16093020141124725,
    0.24611230194568634,
    0.33791524171829224,
    0.44070982933044434,
    0.5626170039176941,
    0.7229568362236023,
    1.0,
)


def create_dynamic_map(signed: bool = True, max_exponent_bits: int = 7, total_bits: int = 8):
    """The 256-point signed dynamic quantisation map (bitsandbytes
    `functional.create_dynamic_map`, restated): for exponent i < 7, 2^i
    midpoints of linspace(0.1, 1, 2^i + 1) scaled by 10^(i - 6), with both
    signs, plus 0 and 1, sorted ascending."""
    data: list[float] = []
    non_sign_bits = total_bits - 1
    additional = 2 ** (non_sign_bits - max_exponent_bits) - 1
    for i in range(max_exponent_bits):
        items = int(
            2 ** (i + non_sign_bits - max_exponent_bits) + 1
            if signed
            else 2 ** (i + non_sign_bits - max_exponent_bits + 1) + 1
        )
        bounds = torch.linspace(0.1, 1, items)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + i)) * means).tolist()
    if additional > 0:
        bounds = torch.linspace(0.1, 1, additional + 1)
        means = (bounds[:-1] + bounds[1:]) / 2.0
        data += ((10 ** (-(max_exponent_bits - 1) + max_exponent_bits - 1)) * means).tolist()
        if signed:
            data += (-(10 ** (-(max_exponent_bits - 1) + max_exponent_bits - 1)) * means).tolist()
    data.append(0.0)
    data.append(1.0)
    data += [0.0] * (2**total_bits - len(data))
    data.sort()
    return torch.tensor(data, dtype=torch.float32)


class QuantState:
    """What bitsandbytes' `QuantState` carries, under the same attribute names."""

    def __init__(self, absmax, shape, code, blocksize, quant_type="nf4", dtype=None,
                 offset=None, state2=None):
        self.absmax = absmax
        self.shape = tuple(shape)
        self.code = code
        self.blocksize = int(blocksize)
        self.quant_type = quant_type
        self.dtype = dtype
        self.offset = offset
        self.state2 = state2
        self.nested = state2 is not None

    def to(self, device):
        self.absmax = self.absmax.to(device)
        self.code = self.code.to(device)
        if self.offset is not None:
            self.offset = self.offset.to(device)
        if self.state2 is not None:
            self.state2.to(device)
        return self


def _nearest_sorted(values, table):
    """Index of the nearest entry of the ascending `table` (ties: lower)."""
    mids = (table[:-1] + table[1:]) / 2
    return torch.bucketize(values, mids, right=False)


def quantize_blockwise(A, code, blocksize: int = 256):
    """uint8 indices into `code` per element, fp32 absmax per block."""
    flat = A.reshape(-1).float()
    n = flat.numel()
    nb = -(-n // blocksize)
    pad = nb * blocksize - n
    blocks = torch.nn.functional.pad(flat, (0, pad)).view(nb, blocksize)
    absmax = blocks.abs().amax(dim=1)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    q = _nearest_sorted((blocks * inv[:, None]).reshape(-1)[:n], code.to(flat.device))
    state = QuantState(absmax=absmax, shape=A.shape, code=code.to(flat.device), blocksize=blocksize,
                       quant_type="dynamic", dtype=torch.float32)
    return q.to(torch.uint8), state


def dequantize_blockwise_scales(qabsmax, state2, offset):
    """code2[a8] * absmax2[b // bs2] + offset, two fp32 roundings (torch order)."""
    blocks = torch.arange(qabsmax.numel(), device=qabsmax.device)
    return state2.code[qabsmax.long()] * state2.absmax[blocks // state2.blocksize] + offset


def quantize_4bit(A, blocksize: int = 64, compress_statistics: bool = False, quant_type: str = "nf4"):
    """(packed uint8 [n/2, 1], QuantState) in bitsandbytes' NF4 layout."""
    if quant_type != "nf4":
        raise ValueError("only nf4 is supported")
    if blocksize < 64 or blocksize & (blocksize - 1):
        raise ValueError("blocksize must be a power of two >= 64")
    flat = A.reshape(-1).float()
    n = flat.numel()
    if n % 2:
        raise ValueError("NF4 packs two codes per byte: the element count must be even")
    nb = -(-n // blocksize)
    pad = nb * blocksize - n
    blocks = torch.nn.functional.pad(flat, (0, pad)).view(nb, blocksize)
    absmax = blocks.abs().amax(dim=1)
    code = torch.tensor(NF4_CODE, dtype=torch.float32, device=flat.device)
    inv = torch.where(absmax > 0, 1.0 / absmax, torch.zeros_like(absmax))
    normed = (blocks * inv[:, None]).reshape(-1)[:n]
    q = _nearest_sorted(normed, code).to(torch.uint8)
    packed = ((q[0::2] << 4) | q[1::2]).view(-1, 1)
    state2 = None
    offset = None
    if compress_statistics:
        offset = absmax.mean()
        qabsmax, state2 = quantize_blockwise(absmax - offset, create_dynamic_map(), blocksize=256)
        absmax = qabsmax
    state = QuantState(absmax=absmax, shape=A.shape, code=code, blocksize=blocksize, quant_type="nf4",
                       dtype=A.dtype, offset=offset, state2=state2)
    return packed, state


def dequantize_4bit(packed, state, out_dtype=None):
    """Dense weight, round(code * scale) in `out_dtype` (default: state.dtype).

    The HIP dequantisation kernel; GPU tensors only."""
    from ttspipe_amd import _lib

    if packed.device.type != "cuda":
        raise RuntimeError("dequantize_4bit runs on the GPU (HIP kernel); move the weight there")
    dt = out_dtype or state.dtype or torch.float16
    code = _lib.dtype_code(dt)
    if code is None:
        raise ValueError(f"unsupported output dtype {dt}")
    n = math.prod(state.shape)
    out = torch.empty(state.shape, dtype=dt, device=packed.device)
    if state.nested:
        a8, amax, code2, offset = state.absmax, state.state2.absmax, state.state2.code, float(state.offset)
        bs2 = state.state2.blocksize
    else:
        a8, amax, code2, offset, bs2 = None, state.absmax, None, 0.0, 0
    lut = state.code.to(device=packed.device, dtype=torch.float32).contiguous()
    rc = _lib.lib().ttsp_nf4_dequant(
        packed.data_ptr(), _lib.ptr(a8), amax.data_ptr(), _lib.ptr(code2), offset, lut.data_ptr(),
        out.data_ptr(), code, n, state.blocksize, bs2, _lib.stream())
    _lib.check(rc, "ttsp_nf4_dequant")
    return out


class Linear4bit(torch.nn.Module):
    """NF4 linear layer with bitsandbytes' attribute layout.

    `weight` is the packed uint8 tensor with `.quant_state` attached;
    `forward` dequantises (HIP kernel) and multiplies in `compute_dtype`, the
    arithmetic of bitsandbytes' own forward. `nf4gemv.install()` routes calls
    through the fused NF4 matmul instead.
    """

    def __init__(self, in_features, out_features, bias=False, compute_dtype=None,
                 quant_type="nf4", compress_statistics=True, blocksize=64, device=None):
        super().__init__()
        self.in_features = in_features
        self.out_features = out_features
        self.compute_dtype = compute_dtype
        self.quant_type = quant_type
        self.compress_statistics = compress_statistics
        self.blocksize = blocksize
        self.device = torch.device(device) if device is not None else None  # where loaded weights go
        self.weight = None
        self.bias = (torch.nn.Parameter(torch.zeros(out_features, device=device,
                                                    dtype=compute_dtype or torch.float16),
                                        requires_grad=False) if bias else None)

    def load_weight(self, dense):
        """Quantise a dense [out, in] weight into this layer (on its device)."""
        if tuple(dense.shape) != (self.out_features, self.in_features):
            raise ValueError("weight shape mismatch")
        packed, state = quantize_4bit(dense, blocksize=self.blocksize,
                                      compress_statistics=self.compress_statistics,
                                      quant_type=self.quant_type)
        return self.set_quantized(packed, state)

    def set_quantized(self, packed, state):
        w = torch.nn.Parameter(packed, requires_grad=False)
        w.quant_state = state
        self.weight = w
        self.__dict__.pop("_nf4_fast", None)
        return self

    def forward(self, x):
        dt = self.compute_dtype or x.dtype
        w = dequantize_4bit(self.weight.data, self.weight.quant_state, out_dtype=dt)
        out = torch.nn.functional.linear(x.to(dt), w.view(self.out_features, self.in_features),
                                         None if self.bias is None else self.bias.to(dt))
        return out.to(x.dtype)


# --------------------------------------------------------------------------
# bitsandbytes' serialised form of a 4-bit weight (what a prequantised
# checkpoint such as the reference's NF4 `model.pth` holds, loaded by the
# fork through bitsandbytes' Params4bit / QuantState): for a Linear4bit at
# `prefix`,
#   prefix + "weight"                       packed uint8 codes [n/2, 1]
#   prefix + "weight.absmax"                fp32 [nblocks], or uint8 when nested
#   prefix + "weight.quant_map"             the 16 NF4 code points, fp32
#   prefix + "weight.nested_absmax"         fp32 [nblocks / bs2]          (nested)
#   prefix + "weight.nested_quant_map"      the 256-point dynamic map     (nested)
#   prefix + "weight.quant_state.bitsandbytes__nf4"
#       uint8 bytes of a JSON object: quant_type, blocksize, dtype, shape and,
#       nested, nested_blocksize, nested_dtype, nested_offset.

_PACKED_KEY = "quant_state.bitsandbytes__"


def _dtype_name(dt) -> str:
    return str(dt).replace("torch.", "")


def _dtype_from(name: str):
    dt = getattr(torch, name, None)
    if not isinstance(dt, torch.dtype):
        raise ValueError(f"unknown dtype {name!r} in a 4-bit weight's state")
    return dt


def quant_state_to_dict(packed, state) -> dict:
    """The tensors bitsandbytes stores for one 4-bit weight, keyed relative to
    the module prefix ("weight", "weight.absmax", ...)."""
    import json

    meta = {"quant_type": state.quant_type, "blocksize": int(state.blocksize),
            "dtype": _dtype_name(state.dtype or torch.float16), "shape": list(state.shape)}
    out = {"weight": packed, "weight.absmax": state.absmax, "weight.quant_map": state.code}
    if state.nested:
        out["weight.nested_absmax"] = state.state2.absmax
        out["weight.nested_quant_map"] = state.state2.code
        meta.update({"nested_blocksize": int(state.state2.blocksize),
                     "nested_dtype": _dtype_name(state.state2.dtype or torch.float32),
                     "nested_offset": float(state.offset)})
    blob = json.dumps(meta).encode("utf-8")
    out["weight." + _PACKED_KEY + state.quant_type] = torch.tensor(list(blob), dtype=torch.uint8)
    return out


def quant_state_from_dict(tensors: dict, device=None):
    """(packed, QuantState) from the tensors `quant_state_to_dict` names (the
    bitsandbytes layout). Raises ValueError on a malformed entry."""
    import json

    packed_key = [k for k in tensors if k.startswith("weight." + _PACKED_KEY)]
    if len(packed_key) != 1:
        raise ValueError("a 4-bit weight needs exactly one packed quant_state entry")
    qt = packed_key[0][len("weight." + _PACKED_KEY):]
    if qt != "nf4":
        raise ValueError(f"quant_type {qt!r} is not served (nf4 only)")
    meta = json.loads(bytes(tensors[packed_key[0]].to("cpu", torch.uint8).tolist()).decode("utf-8"))
    dev = device if device is not None else tensors["weight"].device
    shape = tuple(int(v) for v in meta["shape"])
    code = tensors["weight.quant_map"].to(dev, torch.float32)
    packed = tensors["weight"].to(dev)
    if packed.dtype != torch.uint8 or packed.numel() * 2 != math.prod(shape):
        raise ValueError("packed codes do not match the weight's shape")
    nested = "weight.nested_absmax" in tensors
    state2 = offset = None
    absmax = tensors["weight.absmax"].to(dev)
    if nested:
        state2 = QuantState(absmax=tensors["weight.nested_absmax"].to(dev, torch.float32),
                            shape=(absmax.numel(),), code=tensors["weight.nested_quant_map"].to(dev, torch.float32),
                            blocksize=int(meta["nested_blocksize"]), quant_type="dynamic",
                            dtype=_dtype_from(meta.get("nested_dtype", "float32")))
        offset = torch.tensor(float(meta["nested_offset"]), device=dev)
    state = QuantState(absmax=absmax, shape=shape, code=code, blocksize=int(meta["blocksize"]), quant_type=qt,
                       dtype=_dtype_from(meta["dtype"]), offset=offset, state2=state2)
    return packed.view(-1, 1), state


def nf4_state_dict(model) -> dict:
    """`model.state_dict()` with every Linear4bit's weight in bitsandbytes'
    serialised form (the layout of a prequantised checkpoint)."""
    sd = {}
    lin = {name: m for name, m in model.named_modules() if isinstance(m, Linear4bit)}
    for k, v in model.state_dict().items():
        owner = k.rsplit(".", 1)[0] if "." in k else ""
        if owner in lin and k.endswith("weight"):
            continue
        sd[k] = v
    for name, m in lin.items():
        prefix = f"{name}." if name else ""
        for k, v in quant_state_to_dict(m.weight.data, m.weight.quant_state).items():
            sd[prefix + k] = v
    return sd


def load_nf4_state_dict(model, state_dict: dict, strict: bool = True):
    """Load a prequantised checkpoint's state dict (bitsandbytes' 4-bit layout)
    into `model`, whose quantised linears are `Linear4bit`s (no bitsandbytes
    needed). A layer's tensors go to the device it was built on (else where its
    current weight lives, else where the state dict's tensors are). Every other
    entry goes through `load_state_dict`. Returns the (missing, unexpected) keys
    of that remainder. Read a checkpoint file with `torch.load(path,
    weights_only=True)` first."""
    lin = {name: m for name, m in model.named_modules() if isinstance(m, Linear4bit)}
    used = set()
    for name, m in lin.items():
        prefix = f"{name}." if name else ""
        sub = {k[len(prefix):]: v for k, v in state_dict.items()
               if k == prefix + "weight" or k.startswith(prefix + "weight.")}
        if "weight" not in sub:
            if strict:
                raise KeyError(f"{prefix}weight missing from the state dict")
            continue
        dev = m.device if getattr(m, "device", None) is not None else (
            m.weight.device if m.weight is not None else None)
        packed, state = quant_state_from_dict(sub, device=dev)
        if tuple(state.shape) != (m.out_features, m.in_features):
            raise ValueError(f"{prefix}weight: shape {state.shape} for a {m.out_features}x{m.in_features} layer")
        m.set_quantized(packed, state)
        used.update(prefix + k for k in sub)
    rest = {k: v for k, v in state_dict.items() if k not in used}
    missing, unexpected = model.load_state_dict(rest, strict=False)
    missing = [k for k in missing if not any(k == (f"{n}." if n else "") + "weight" for n in lin)]
    if strict and (missing or unexpected):
        raise KeyError(f"missing {missing}, unexpected {unexpected}")
    return missing, unexpected
