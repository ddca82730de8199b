"""Seeded random shapes through the decode attention kernels, RMSNorm and
rotary (GPU).

The fixed-shape tests take the model's head counts and cache lengths. These
draw what a caller of the same entry points may pass: 1 to 8 kv heads with 1
to 16 query heads each, caches of 1 to 4096 positions, the position anywhere
in the cache and chunk counts from the fewest that reach it to the whole
cache; the attention + wo launch over every head count and cache its LDS
holds and up to 8192 output rows; RMSNorm rows of any multiple of 8 wide up
to 12288; rotary of any even head width. Bar: bit for bit against the
oracle's emulation of each kernel's order (attention and the KV rows it
writes, the norm, the rotary), as the fixed-shape tests.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.gpuutil import bits, dt_code, first_mismatch, from_bits, gemv_shape, randn_bits
from tests.nf4data import oracle_args, random_layer

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _norm_weights(rng, dt):
    qwb = o.from_f32((rng.random(128) + 0.5).astype(np.float32), dt)
    kwb = o.from_f32((rng.random(128) + 0.5).astype(np.float32), dt)
    return qwb, kwb


@pytest.mark.parametrize("case", range(6))
def test_attention_from_qkv_random_shapes(hip, orc, case):
    """Head norms, rotary, the KV write and split-K attention (+ merge) from
    the QKV row, against qk_rope_kv then the attention in the oracle."""
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    rng = np.random.default_rng(4000 + case)
    for i in range(6):
        nkv = int(rng.choice([1, 2, 4, 8]))
        groups = int(rng.choice([1, 2, 3, 4, 8, 16]))
        nh = nkv * groups
        max_len = int(rng.integers(1, 4097))
        pos = int(rng.integers(0, max_len))
        nchunk = int(rng.integers(pos // 64 + 1, -(-max_len // 64) + 1))
        qk_norm = bool(rng.integers(0, 2))
        dtype = DTYPES[int(rng.integers(0, 2))]
        dt = dt_code(dtype)
        where = f"nh={nh} nkv={nkv} max_len={max_len} pos={pos} nchunk={nchunk} qk_norm={qk_norm} {dtype}"
        qkvb = randn_bits((nh + 2 * nkv) * 128, dtype, seed=case * 10 + i, scale=2.0)
        qwb, kwb = _norm_weights(rng, dt)
        freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos : pos + 1].contiguous()
        kcb = randn_bits(nkv * max_len * 128, dtype, seed=case * 10 + i + 100)
        vcb = randn_bits(nkv * max_len * 128, dtype, seed=case * 10 + i + 200)
        KC, VC = from_bits(kcb, dtype), from_bits(vcb, dtype)
        f32 = dict(dtype=torch.float32, device="cuda")
        pm, pl = torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk, **f32)
        pacc = torch.empty(nh * nchunk * 128, **f32)
        y = torch.empty(nh * 128, dtype=dtype, device="cuda")
        qw = from_bits(qwb, dtype) if qk_norm else None
        kw = from_bits(kwb, dtype) if qk_norm else None
        posd = torch.tensor([pos], dtype=torch.long, device="cuda")
        fd, qkv = freqs.cuda(), from_bits(qkvb, dtype)
        rc = hip.ttsp_attn_decode_qkv(qkv.data_ptr(), _lib.ptr(qw), _lib.ptr(kw), 1e-6, fd.data_ptr(), o.DT_BF16,
                                      posd.data_ptr(), KC.data_ptr(), VC.data_ptr(), pm.data_ptr(), pl.data_ptr(),
                                      pacc.data_ptr(), y.data_ptr(), nh, nkv, max_len, nchunk, float(128**-0.5), dt,
                                      _lib.stream())
        assert rc == 0, where
        Qo = np.zeros(nh * 128, np.uint16)
        KCo, VCo = kcb.copy(), vcb.copy()
        orc.qk_rope_kv(qkvb, qwb if qk_norm else None, kwb if qk_norm else None, 1e-6, bits(freqs), o.DT_BF16, pos,
                       Qo, KCo, VCo, nh, nkv, max_len, dt)
        expect = orc.attn_emul(Qo, KCo, VCo, pos, nh, nkv, max_len, nchunk, 128**-0.5, dt)
        assert np.array_equal(bits(y), expect), f"{where}: {first_mismatch(bits(y), expect)}"
        assert np.array_equal(bits(KC), KCo), f"{where}: K rows"
        assert np.array_equal(bits(VC), VCo), f"{where}: V rows"


@pytest.mark.parametrize("case", range(6))
def test_attention_and_wo_random_shapes(hip, orc, case):
    """The one-chunk attention recomputed by every wo workgroup, then wo with
    the residual: against the oracle's qk_rope_kv, attention and GEMV."""
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis
    from ttspipe_amd.quant import NF4_CODE

    rng = np.random.default_rng(5000 + case)
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device="cuda")
    for i in range(6):
        nkv = int(rng.choice([1, 2, 4, 8]))
        nh = nkv * int(rng.choice([g for g in (1, 2, 4, 8) if nkv * g <= 8]))
        max_len = int(rng.integers(1, min(64, 128 // nkv) + 1))
        pos = int(rng.integers(0, max_len))
        K = nh * 128
        M = int(rng.integers(1, 8193))
        nested = bool(rng.integers(0, 2))
        qk_norm = bool(rng.integers(0, 2))
        dtype = DTYPES[int(rng.integers(0, 2))]
        dt = dt_code(dtype)
        J, KS, RPW = gemv_shape(M, K)
        where = f"nh={nh} nkv={nkv} max_len={max_len} pos={pos} M={M} J={J} RPW={RPW} nested={nested} {dtype}"
        layer = random_layer(M, K, nested, seed=case * 10 + i + 300)
        W = torch.from_numpy(layer["W"]).cuda()
        A8 = torch.from_numpy(layer["A8"]).cuda() if nested else None
        AM = torch.from_numpy(layer["AMAX"]).cuda()
        C2 = torch.from_numpy(layer["CODE2"]).cuda() if nested else None
        qkvb = randn_bits((nh + 2 * nkv) * 128, dtype, seed=case * 10 + i + 400, scale=2.0)
        qwb, kwb = _norm_weights(rng, dt)
        freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos : pos + 1].contiguous()
        kcb = randn_bits(nkv * max_len * 128, dtype, seed=case * 10 + i + 500)
        vcb = randn_bits(nkv * max_len * 128, dtype, seed=case * 10 + i + 600)
        rb = randn_bits(M, dtype, seed=case * 10 + i + 700)
        KC, VC = from_bits(kcb, dtype), from_bits(vcb, dtype)
        qkv, R = from_bits(qkvb, dtype), from_bits(rb, dtype)
        qw = from_bits(qwb, dtype) if qk_norm else None
        kw = from_bits(kwb, dtype) if qk_norm else None
        posd = torch.tensor([pos], dtype=torch.long, device="cuda")
        fd = freqs.cuda()
        h = torch.empty(M, dtype=dtype, device="cuda")
        rc = hip.ttsp_attn_nf4_gemv(qkv.data_ptr(), _lib.ptr(qw), _lib.ptr(kw), 1e-6, fd.data_ptr(), o.DT_BF16,
                                    posd.data_ptr(), KC.data_ptr(), VC.data_ptr(), nh, nkv, max_len,
                                    float(128**-0.5), W.data_ptr(), _lib.ptr(A8), AM.data_ptr(), _lib.ptr(C2),
                                    float(layer["offset"]), lut.data_ptr(), h.data_ptr(), R.data_ptr(), 1, M, 64,
                                    layer["bs2"] or 0, dt, _lib.stream())
        assert rc == 0, where
        Qo = np.zeros(nh * 128, np.uint16)
        KCo, VCo = kcb.copy(), vcb.copy()
        orc.qk_rope_kv(qkvb, qwb if qk_norm else None, kwb if qk_norm else None, 1e-6, bits(freqs), o.DT_BF16, pos,
                       Qo, KCo, VCo, nh, nkv, max_len, dt)
        y = orc.attn_emul(Qo, KCo, VCo, pos, nh, nkv, max_len, 1, 128**-0.5, dt)
        expect = orc.gemv_emul(y, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, bs2=layer["bs2"] or 256,
                               R=rb, epi=1)
        assert np.array_equal(bits(h), expect), f"{where}: {first_mismatch(bits(h), expect)}"
        assert np.array_equal(bits(KC), KCo), f"{where}: K rows"
        assert np.array_equal(bits(VC), VCo), f"{where}: V rows"


@pytest.mark.parametrize("case", range(4))
def test_rms_norm_random_shapes(orc, case):
    from ttspipe_amd import fusedops

    rng = np.random.default_rng(6000 + case)
    for i in range(8):
        rows = int(rng.integers(1, 601))
        width = 8 * int(rng.integers(1, 1537))
        dtype = DTYPES[int(rng.integers(0, 2))]
        dt = dt_code(dtype)
        xb = randn_bits(rows * width, dtype, seed=case * 10 + i, scale=float(rng.choice([0.01, 1.0, 30.0])))
        wb = o.from_f32((rng.standard_normal(width) * 0.1 + 1).astype(np.float32), dt)
        y = fusedops.rms_norm(from_bits(xb, dtype).view(1, rows, width), from_bits(wb, dtype), 1e-6)
        assert y is not None
        expect = orc.rms_norm_emul(xb, wb, rows, width, 1e-6, dt)
        assert np.array_equal(bits(y), expect), f"rows={rows} width={width} {dtype}: {first_mismatch(bits(y), expect)}"


@pytest.mark.parametrize("case", range(4))
def test_rope_random_shapes(orc, case):
    from ttspipe_amd import fusedops
    from ttspipe_amd.llama import apply_rotary_emb

    rng = np.random.default_rng(7000 + case)
    fdts = [torch.bfloat16, torch.float32, torch.float16]
    for i in range(8):
        b, s, h = int(rng.integers(1, 4)), int(rng.integers(1, 300)), int(rng.integers(1, 41))
        d = 2 * int(rng.integers(1, 129))
        dtype, fdt = DTYPES[int(rng.integers(0, 2))], fdts[int(rng.integers(0, 3))]
        g = torch.Generator().manual_seed(case * 100 + i)
        x = torch.randn(b, s, h, d, generator=g).to(dtype)
        f = torch.randn(s, d // 2, 2, generator=g).to(fdt)
        y = fusedops.rope(x.cuda(), f.cuda())
        where = f"shape={(b, s, h, d)} {dtype} freqs {fdt}"
        assert y is not None, where
        assert torch.equal(y.cpu(), apply_rotary_emb(x, f)), where
        ours = orc.rope(bits(x), bits(f), dt_code(fdt), d // 2, h, s, dt_code(dtype))
        assert np.array_equal(bits(y), ours), where


@pytest.mark.parametrize("case", range(4))
def test_prefill_attention_random_shapes(case):
    """Causal prefill attention over S new positions after a cached prefix,
    every head grouping the kernel takes, against fp64 within the 5e-3 bar;
    and the same call with a random key split."""
    from tests.conftest import relative_error
    from tests.test_prefill_gpu import _fp64, _run, _setup, _split_call
    from ttspipe_amd import _lib

    rng = np.random.default_rng(8000 + case)
    gmax = _lib.load().ttsp_prefill_max_groups()
    for i in range(4):
        nkv = int(rng.choice([1, 2, 4, 8]))
        nh = nkv * int(rng.choice([g for g in (1, 2, 4, 8, 16) if g <= gmax]))
        S, prefix = int(rng.integers(1, 601)), int(rng.integers(0, 3001))
        dtype = DTYPES[int(rng.integers(0, 2))]
        where = f"S={S} prefix={prefix} nh={nh} nkv={nkv} {dtype}"
        q, k, v, mask = _setup(S, prefix, nh, nkv, dtype, seed=case * 10 + i)
        ref = _fp64(q, k, v, mask)
        y = _run(q, k, v, mask, nh, nkv)
        assert relative_error(y[0].double().cpu().numpy(), ref) < 5e-3, where
        splits = int(rng.integers(2, 9))
        ys = _split_call(q, k, v, mask, nh, nkv, splits)  # [nh, S, D] on the host
        assert relative_error(ys, ref) < 5e-3, f"{where} splits={splits}"
