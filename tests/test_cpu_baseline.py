"""The CPU baseline (oracle/nf4cpu_port.cpp, the reference's CPU NF4 GEMV
algorithm restated, app/engine/nf4cpu.py:86-146, and a decode block on it,
nf4cpu.py:479-617) against fp64 numpy restatements of the same formulas on
small shapes. It is a timing baseline, so the bar is the bf16 roundings the
algorithm makes, not bit-exactness."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as o
from tests.conftest import beyond_rounding_error

BF = o.DT_BF16


def _bf(a):
    return o.to_f32(o.from_f32(np.asarray(a, np.float32), BF), BF).astype(np.float64)


def _dequant(packed, absmax_bits, M, K, code_bits):
    q = np.empty(M * K, np.int64)
    q[0::2] = packed >> 4
    q[1::2] = packed & 15
    code = o.to_f32(code_bits, BF).astype(np.float64)
    s = np.repeat(o.to_f32(absmax_bits, BF).astype(np.float64), 64)
    return (code[q] * s).reshape(M, K)


def _layer(rng, M, K):
    packed = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    absmax = o.from_f32((rng.random(M * K // 64, dtype=np.float32) * 0.05 + 0.02), BF)
    return packed, absmax


@pytest.fixture(scope="module")
def cb():
    from oracle import cpu_baseline

    return cpu_baseline


@pytest.mark.parametrize("M,K", [(13, 64), (64, 256), (40, 1024)])
@pytest.mark.parametrize("force_scalar", [False, True])
def test_cpu_gemv_matches_fp64(cb, M, K, force_scalar):
    rng = np.random.default_rng(M + K)
    packed, absmax = _layer(rng, M, K)
    code = o.from_f32(o.NF4_CODE, BF)
    xb = o.from_f32(rng.standard_normal(K).astype(np.float32), BF)
    y = cb.gemv(xb, packed, absmax, code, M, threads=2, force_scalar=force_scalar)
    ref = _dequant(packed, absmax, M, K, code) @ o.to_f32(xb, BF).astype(np.float64)
    assert beyond_rounding_error(o.to_f32(y, BF), ref, BF) < 1e-3


def test_cpu_decode_block_matches_fp64(cb):
    """One block at small dims through `cpu_decode_block` against a numpy
    fp64 restatement (bf16 roundings where the block rounds)."""
    import ctypes

    rng = np.random.default_rng(3)
    D, nh, nkv, inter, max_len, pos, hd = 256, 4, 2, 512, 16, 9, 128
    lib = cb._lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.cpu_decode_block.argtypes = ([vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, ctypes.c_float] + [vp, vp] * 4
                                     + [vp, vp, vp, i64, i64, vp, ctypes.c_int])
    code = o.from_f32(o.NF4_CODE, BF)
    vec = lambda n: o.from_f32((rng.standard_normal(n) * 0.1 + 1).astype(np.float32), BF)  # noqa: E731
    an, fn, qn, kn = vec(D), vec(D), vec(hd), vec(hd)
    qkv, wo, w13, w2 = (_layer(rng, (nh + 2 * nkv) * hd, D), _layer(rng, D, nh * hd), _layer(rng, 2 * inter, D),
                        _layer(rng, D, inter))
    kc = o.from_f32(rng.standard_normal(nkv * max_len * hd).astype(np.float32), BF)
    vc = o.from_f32(rng.standard_normal(nkv * max_len * hd).astype(np.float32), BF)
    kc0, vc0 = kc.copy(), vc.copy()
    ang = pos * 1e6 ** (-np.arange(0, hd, 2) / hd)
    freqs = np.stack([np.cos(ang), np.sin(ang)], -1).astype(np.float32).ravel()
    x = o.from_f32(rng.standard_normal(D).astype(np.float32), BF)
    out = np.empty(D, np.uint16)
    p = lambda a: a.ctypes.data  # noqa: E731
    lib.cpu_decode_block(p(x), p(out), D, nh, nkv, inter, p(an), p(fn), p(qn), p(kn), 1e-6, p(qkv[0]), p(qkv[1]),
                         p(wo[0]), p(wo[1]), p(w13[0]), p(w13[1]), p(w2[0]), p(w2[1]), p(code), p(kc), p(vc), pos,
                         max_len, p(freqs), 2)

    # fp64 restatement, rounding to bf16 where the block rounds
    f = lambda b: o.to_f32(b, BF).astype(np.float64)  # noqa: E731
    W = lambda lay, M, K: _dequant(lay[0], lay[1], M, K, code)  # noqa: E731
    xf = f(x)

    def norm(v, w):
        return _bf(_bf(v / np.sqrt(np.mean(v * v) + 1e-6)) * f(w))

    t = _bf(W(qkv, (nh + 2 * nkv) * hd, D) @ norm(xf, an))
    heads = t.reshape(nh + 2 * nkv, hd)
    for h in range(nh + nkv):
        r = heads[h]
        r = _bf(r / np.sqrt(np.mean(r * r) + 1e-6) * f(qn if h < nh else kn))
        c, s = freqs.astype(np.float64)[0::2], freqs.astype(np.float64)[1::2]
        a, b = r[0::2].copy(), r[1::2].copy()
        r[0::2], r[1::2] = _bf(a * c - b * s), _bf(b * c + a * s)
        heads[h] = r
    K3 = f(kc0).reshape(nkv, max_len, hd)
    V3 = f(vc0).reshape(nkv, max_len, hd)
    K3[:, pos], V3[:, pos] = _bf(heads[nh:nh + nkv]), _bf(heads[nh + nkv:])
    att = np.empty((nh, hd))
    for h in range(nh):
        kv = h // (nh // nkv)
        sc = _bf(K3[kv, :pos + 1] @ heads[h]) / np.sqrt(hd)
        e = np.exp(sc - sc.max())
        att[h] = _bf(_bf(e / e.sum()) @ V3[kv, :pos + 1])
    hres = _bf(xf + _bf(W(wo, D, nh * hd) @ att.ravel()))
    ab = _bf(W(w13, 2 * inter, D) @ norm(hres, fn))
    g = _bf(_bf(ab[:inter] / (1 + np.exp(-ab[:inter]))) * ab[inter:])
    ref = hres + _bf(W(w2, D, inter) @ g)
    assert beyond_rounding_error(o.to_f32(out, BF), ref, BF) < 2e-2
    # the new K/V row landed at pos, nothing else changed
    kc3, vc3 = kc.reshape(nkv, max_len, hd), vc.reshape(nkv, max_len, hd)
    assert np.array_equal(np.delete(kc3, pos, 1), np.delete(kc0.reshape(nkv, max_len, hd), pos, 1))
    assert np.array_equal(np.delete(vc3, pos, 1), np.delete(vc0.reshape(nkv, max_len, hd), pos, 1))
    assert np.abs(f(kc3[:, pos]) - K3[:, pos]).max() <= 0.02 * np.abs(K3[:, pos]).max()
