"""The allocation-free decode attention (ttsp_attn_decode_qkv_noalloc) against
the entry point that takes caller scratch (ttsp_attn_decode_qkv), through the
C-ABI (GPU).

Bar: bit for bit - the attention output and the K/V cache rows - on two calls
in a row, the second with a smaller problem (fewer heads, a shorter cache and
fewer chunks), so it reads the library's scratch after a larger call left
other values in it; requests beyond the scratch are refused before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.gpuutil import from_bits, randn_bits

pytestmark = pytest.mark.gpu


def _case(pos, max_len, nh, nkv, dtype, seed):
    from ttspipe_amd.llama import precompute_freqs_cis

    dt = o.DT_BF16 if dtype == torch.bfloat16 else o.DT_F16
    qkv = from_bits(randn_bits((nh + 2 * nkv) * 128, dtype, seed=seed, scale=2.0), dtype)
    qw = from_bits(o.from_f32((np.random.default_rng(seed + 1).random(128) + 0.5).astype(np.float32), dt), dtype)
    kw = from_bits(o.from_f32((np.random.default_rng(seed + 2).random(128) + 0.5).astype(np.float32), dt), dtype)
    freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos:pos + 1].contiguous().cuda()
    kc = from_bits(randn_bits(nkv * max_len * 128, dtype, seed=seed + 3), dtype)
    vc = from_bits(randn_bits(nkv * max_len * 128, dtype, seed=seed + 4), dtype)
    posd = torch.tensor([pos], dtype=torch.long, device="cuda")
    return qkv, qw, kw, freqs, kc, vc, posd


def _both(hip, pos, max_len, nh, nkv, dtype, seed):
    from ttspipe_amd import _lib

    nchunk = -(-max_len // 64)
    qkv, qw, kw, freqs, kc, vc, posd = _case(pos, max_len, nh, nkv, dtype, seed)
    dt = _lib.DT_BF16 if dtype == torch.bfloat16 else _lib.DT_F16
    scale = float(128 ** -0.5)
    # with caller scratch
    f32 = dict(dtype=torch.float32, device="cuda")
    pm, pl, pacc = torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk * 128, **f32)
    kc1, vc1 = kc.clone(), vc.clone()
    y1 = torch.empty(nh * 128, dtype=dtype, device="cuda")
    rc = hip.ttsp_attn_decode_qkv(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), 1e-6, freqs.data_ptr(), _lib.DT_BF16,
                                  posd.data_ptr(), kc1.data_ptr(), vc1.data_ptr(), pm.data_ptr(), pl.data_ptr(),
                                  pacc.data_ptr(), y1.data_ptr(), nh, nkv, max_len, nchunk, scale, dt, _lib.stream())
    assert rc == 0
    # the library's own scratch
    kc2, vc2 = kc.clone(), vc.clone()
    y2 = torch.empty(nh * 128, dtype=dtype, device="cuda")
    rc = hip.ttsp_attn_decode_qkv_noalloc(qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), 1e-6, freqs.data_ptr(),
                                          _lib.DT_BF16, posd.data_ptr(), kc2.data_ptr(), vc2.data_ptr(), y2.data_ptr(),
                                          nh, nkv, max_len, nchunk, scale, dt, _lib.stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(y1, y2), "attention outputs differ"
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), "cache rows differ"
    assert not torch.equal(kc1, kc), "the new K row was not written"
    return nchunk


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_attention_equals_the_scratch_entry_twice(hip, dtype):
    big = _both(hip, pos=2100, max_len=2304, nh=32, nkv=8, dtype=dtype, seed=7)
    small = _both(hip, pos=300, max_len=512, nh=8, nkv=2, dtype=dtype, seed=8)
    assert big == 36 and small == 8


def test_noalloc_attention_refuses_beyond_its_scratch(hip):
    from ttspipe_amd import _lib

    slots = hip.ttsp_attn_decode_qkv_noalloc_max_slots()
    assert slots == 4096
    nh, nkv = 64, 8
    nchunk = slots // nh + 1  # one chunk too many
    max_len = 64 * nchunk
    # buffers of the full size, so the refusal is the only thing under test
    bf = dict(dtype=torch.bfloat16, device="cuda")
    qkv = torch.zeros((nh + 2 * nkv) * 128, **bf)
    kc, vc = torch.zeros(nkv * max_len * 128, **bf), torch.zeros(nkv * max_len * 128, **bf)
    freqs = torch.zeros(128, **bf)
    y = torch.zeros(nh * 128, **bf)
    posd = torch.tensor([0], dtype=torch.long, device="cuda")
    rc = hip.ttsp_attn_decode_qkv_noalloc(qkv.data_ptr(), 0, 0, 1e-6, freqs.data_ptr(), _lib.DT_BF16,
                                          posd.data_ptr(), kc.data_ptr(), vc.data_ptr(), y.data_ptr(),
                                          nh, nkv, max_len, nchunk, 0.1, _lib.DT_BF16, _lib.stream())
    assert rc != 0
    assert not y.any() and not kc.any()
    torch.cuda.synchronize()
