"""Prequantised checkpoints in bitsandbytes' serialised 4-bit layout (what the
reference's NF4 model.pth holds and the fork loads through Params4bit /
QuantState) load into this package's Linear4bit without bitsandbytes (CPU)."""

from __future__ import annotations

import json

import pytest
import torch

from ttspipe_amd import quant


def _model(nested: bool):
    torch.manual_seed(0)
    m = torch.nn.Module()
    m.norm = torch.nn.Parameter(torch.randn(256))
    m.a = quant.Linear4bit(256, 128, bias=False, compress_statistics=nested)
    m.a.load_weight(torch.randn(128, 256) * 0.02)
    m.b = quant.Linear4bit(128, 64, bias=True, compute_dtype=torch.float16, compress_statistics=nested)
    m.b.load_weight(torch.randn(64, 128) * 0.02)
    return m


@pytest.mark.parametrize("nested", [True, False])
def test_the_serialised_layout_is_bitsandbytes(nested):
    m = _model(nested)
    sd = quant.nf4_state_dict(m)
    keys = {"a.weight", "a.weight.absmax", "a.weight.quant_map", "a.weight.quant_state.bitsandbytes__nf4"}
    if nested:
        keys |= {"a.weight.nested_absmax", "a.weight.nested_quant_map"}
    assert keys <= set(sd)
    meta = json.loads(bytes(sd["a.weight.quant_state.bitsandbytes__nf4"].tolist()).decode())
    assert meta["quant_type"] == "nf4" and meta["blocksize"] == 64 and meta["shape"] == [128, 256]
    assert sd["a.weight"].dtype == torch.uint8 and sd["a.weight"].shape == (128 * 256 // 2, 1)
    assert sd["a.weight.absmax"].dtype == (torch.uint8 if nested else torch.float32)
    if nested:
        assert meta["nested_blocksize"] == 256 and isinstance(meta["nested_offset"], float)


@pytest.mark.parametrize("nested", [True, False])
def test_round_trip_restores_every_byte(nested):
    src = _model(nested)
    sd = quant.nf4_state_dict(src)
    dst = _model(not nested)  # other contents, same module tree
    quant.load_nf4_state_dict(dst, sd)
    for name in ("a", "b"):
        s, d = getattr(src, name), getattr(dst, name)
        assert torch.equal(s.weight.data, d.weight.data)
        qs, qd = s.weight.quant_state, d.weight.quant_state
        assert qd.nested == nested and qd.shape == qs.shape and qd.blocksize == qs.blocksize
        assert torch.equal(qs.absmax, qd.absmax) and torch.equal(qs.code, qd.code)
        if nested:
            assert torch.equal(qs.state2.absmax, qd.state2.absmax) and torch.equal(qs.state2.code, qd.state2.code)
            assert float(qs.offset) == float(qd.offset) and qd.state2.blocksize == 256
    assert torch.equal(src.norm, dst.norm) and torch.equal(src.b.bias, dst.b.bias)


def test_malformed_entries_are_rejected():
    m = _model(True)
    sd = quant.nf4_state_dict(m)
    bad = dict(sd)
    bad["a.weight"] = bad["a.weight"][:-1]
    with pytest.raises(ValueError):
        quant.load_nf4_state_dict(_model(True), bad)
    bad = {k: v for k, v in sd.items() if not k.startswith("a.weight.quant_state")}
    with pytest.raises(ValueError):
        quant.load_nf4_state_dict(_model(True), bad)
    bad = {k: v for k, v in sd.items() if k != "norm"}
    with pytest.raises(KeyError):
        quant.load_nf4_state_dict(_model(True), bad)
    # a state dict saved by torch and read back with weights_only=True (the safe loader) loads
    import io

    buf = io.BytesIO()
    torch.save(sd, buf)
    buf.seek(0)
    quant.load_nf4_state_dict(_model(True), torch.load(buf, weights_only=True))
