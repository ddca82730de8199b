"""Seeded NF4 layers for tests: the same bytes go to the oracle (numpy) and the GPU (torch)."""

from __future__ import annotations

import numpy as np


def random_layer(M: int, K: int, nested: bool, seed: int, bs: int = 64, bs2: int = 256) -> dict:
    """Uniform random codes (what NF4 of normal weights looks like: each code
    holds equal mass) and positive scales around 0.04, plain or nested."""
    from ttspipe_amd.quant import create_dynamic_map

    rng = np.random.default_rng(seed)
    packed = rng.integers(0, 256, size=M * K // 2, dtype=np.uint8)
    nblk = M * K // bs
    layer = {"M": M, "K": K, "W": packed, "bs": bs, "nested": nested}
    if nested:
        layer["A8"] = rng.integers(0, 256, size=nblk, dtype=np.uint8)
        layer["AMAX"] = (rng.random(-(-nblk // bs2), dtype=np.float32) * 0.01 + 0.01).astype(np.float32)
        layer["CODE2"] = create_dynamic_map().numpy().astype(np.float32)
        layer["offset"] = np.float32(0.04)
        layer["bs2"] = bs2
    else:
        layer["A8"] = None
        layer["AMAX"] = (rng.random(nblk, dtype=np.float32) * 0.04 + 0.02).astype(np.float32)
        layer["CODE2"] = None
        layer["offset"] = np.float32(0.0)
        layer["bs2"] = 0
    return layer


def oracle_args(layer: dict) -> dict:
    return {k: layer[k] for k in ("W", "A8", "AMAX", "CODE2", "offset")}


def to_linear(layer: dict, dtype, device="cuda"):
    """A `quant.Linear4bit` holding exactly these bytes."""
    import torch

    from ttspipe_amd.quant import NF4_CODE, Linear4bit, QuantState

    M, K = layer["M"], layer["K"]
    lin = Linear4bit(K, M, bias=False, compute_dtype=dtype, compress_statistics=layer["nested"],
                     blocksize=layer["bs"], device=device)
    code = torch.tensor(NF4_CODE, dtype=torch.float32, device=device)
    packed = torch.from_numpy(layer["W"].copy()).to(device).view(-1, 1)
    if layer["nested"]:
        state2 = QuantState(absmax=torch.from_numpy(layer["AMAX"]).to(device), shape=(layer["A8"].size,),
                            code=torch.from_numpy(layer["CODE2"]).to(device), blocksize=layer["bs2"],
                            quant_type="dynamic", dtype=torch.float32)
        state = QuantState(absmax=torch.from_numpy(layer["A8"]).to(device), shape=(M, K), code=code,
                           blocksize=layer["bs"], dtype=dtype,
                           offset=torch.tensor(float(layer["offset"]), device=device), state2=state2)
    else:
        state = QuantState(absmax=torch.from_numpy(layer["AMAX"]).to(device), shape=(M, K), code=code,
                           blocksize=layer["bs"], dtype=dtype)
    return lin.set_quantized(packed, state)


def dequant_numpy(layer: dict, out_dtype: int) -> np.ndarray:
    """Closed form, independent of the C oracle: round(code[q] * s) per element."""
    from oracle import oracle as o

    q = o.unpack_nf4(layer["W"])
    s = o.scales(layer["A8"], layer["AMAX"], layer["CODE2"], layer["offset"], layer["bs2"] or 1)
    v = (o.NF4_CODE[q] * np.repeat(s, layer["bs"])[: q.size]).astype(np.float32)
    return o.from_f32(v, out_dtype)
