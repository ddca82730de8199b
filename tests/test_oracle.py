"""Pins the CPU oracle before anything is compared against it.

Each oracle function is checked against something it does not share code
with: the reference's own literal table (golden fixture), numpy / torch
implementations of the same closed form, fp64 brute force, or an identity the
mathematics fixes. Each check is chosen so a plausible slip - swapped
nibbles, a dropped rounding, a transposed operand, the wrong KV head - fails.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.conftest import beyond_rounding_error, relative_error
from tests.nf4data import dequant_numpy, oracle_args, random_layer

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_nf4_code_matches_the_reference_literal():
    ref = json.loads((GOLDEN / "nf4_code.json").read_text())["NF4_CODE"]
    from ttspipe_amd.quant import NF4_CODE

    assert np.array_equal(np.float32(ref), o.NF4_CODE)
    assert np.array_equal(np.float32(ref), np.float32(NF4_CODE))
    assert list(ref) == sorted(ref) and ref[0] == -1.0 and ref[7] == 0.0 and ref[15] == 1.0


@pytest.mark.parametrize("dt", [o.DT_F16, o.DT_BF16])
def test_conversions_match_numpy_and_torch(orc, dt):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * 300,
        np.float32([0.0, -0.0, 1e-8, 6e-8, 65504.0, 65520.0, 7e4, np.inf, -np.inf, 3e38, 1.0000001, 2.9802322e-08]),
    ])
    ours = np.array([(orc.lib().orc_f32_to_f16 if dt == o.DT_F16 else orc.lib().orc_f32_to_bf16)(float(v)) for v in x], np.uint16)
    tdt = torch.float16 if dt == o.DT_F16 else torch.bfloat16
    theirs = torch.from_numpy(x).to(tdt).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert np.array_equal(o.from_f32(x, dt), theirs)
    back = o.to_f32(theirs, dt)
    assert np.array_equal(back, torch.from_numpy(x).to(tdt).float().numpy(), equal_nan=True)


def _round_f32(x) -> float:
    """Exact rational -> nearest fp32, ties to even (subnormals included)."""
    from fractions import Fraction

    if x == 0:
        return 0.0
    sign, a = (-1 if x < 0 else 1), abs(Fraction(x))
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    q = max(e - 23, -149)  # the ulp's exponent
    m = a / Fraction(2) ** q
    n, rem = divmod(m.numerator, m.denominator)
    if 2 * rem > m.denominator or (2 * rem == m.denominator and n % 2):
        n += 1
    return sign * float(Fraction(n) * Fraction(2) ** q)


def test_fma16_chain_is_two_exactly_rounded_fmas(orc):
    """orc_fma16_chain (the GEMV's v_fma_mix chain: fma(a.hi, b.hi,
    fma(a.lo, b.lo, c)), fp16 operands, fp32 accumulator) against exact
    rational arithmetic with one fp32 rounding per fma, over random operands
    and the edge cases (zeros, signs, subnormal and large fp16, tiny and huge
    c). (A product of two fp16 values is exact in fp32, so an fma and a
    multiply-then-add agree; what the chain fixes is the rounding after each
    add and the order.) The chain rounded once at the end, or the pair taken
    in the other order, disagrees on a visible share of the same inputs."""
    from fractions import Fraction

    rng = np.random.default_rng(16)
    n = 4000
    h = rng.integers(0, 1 << 16, size=(2, n), dtype=np.uint32)
    h[:, :200] = rng.choice(np.array([0x0000, 0x8000, 0x0001, 0x03ff, 0x7bff, 0xfbff, 0x3c00, 0xbc00], np.uint32),
                            size=(2, 200))
    h2 = rng.integers(0, 1 << 16, size=(2, n), dtype=np.uint32)
    finite = lambda u: (u & 0x7c00) != 0x7c00  # noqa: E731
    keep = finite(h[0]) & finite(h[1]) & finite(h2[0]) & finite(h2[1])
    a = (h[0] | (h2[0] << 16))[keep].astype(np.uint32)
    b = (h[1] | (h2[1] << 16))[keep].astype(np.uint32)
    c = (rng.standard_normal(a.size) * np.exp2(rng.integers(-30, 30, a.size))).astype(np.float32)
    c[:50] = 0.0
    got = orc.fma16_chain(a, b, c)
    f16 = lambda u: float(np.uint16(u).view(np.float16))  # noqa: E731
    diff_once = diff_order = 0
    for i in range(a.size):
        alo, ahi, blo, bhi = f16(a[i] & 0xFFFF), f16(a[i] >> 16), f16(b[i] & 0xFFFF), f16(b[i] >> 16)
        t = _round_f32(Fraction(alo) * Fraction(blo) + Fraction(float(c[i])))
        want = _round_f32(Fraction(ahi) * Fraction(bhi) + Fraction(t))
        if math.isinf(want) or abs(want) > 3.4e38:
            continue
        assert got[i] == np.float32(want), (i, hex(a[i]), hex(b[i]), c[i], got[i], want)
        once = _round_f32(Fraction(alo) * Fraction(blo) + Fraction(float(c[i])) + Fraction(ahi) * Fraction(bhi))
        diff_once += np.float32(once) != np.float32(want)
        t2 = _round_f32(Fraction(ahi) * Fraction(bhi) + Fraction(float(c[i])))
        diff_order += np.float32(_round_f32(Fraction(alo) * Fraction(blo) + Fraction(t2))) != np.float32(want)
    assert diff_once > a.size // 50 and diff_order > a.size // 50, (diff_once, diff_order)


def test_packing_layout_is_high_nibble_first():
    """The product quantiser's bytes decode, through the oracle's unpacking,
    to the nearest-code indices computed independently (the reference's
    layout check, tests/test_nf4gemv.py:69-92)."""
    from ttspipe_amd.quant import quantize_4bit

    torch.manual_seed(0)
    w = torch.randn(8, 256)
    packed, state = quantize_4bit(w, blocksize=64, compress_statistics=False)
    absmax = w.reshape(-1, 64).abs().amax(1)
    assert torch.equal(state.absmax, absmax)
    code = torch.tensor(o.NF4_CODE)
    ratio = (w.reshape(-1, 64) * (1.0 / absmax)[:, None]).reshape(-1)
    idx = (ratio[:, None] - code[None, :]).abs().argmin(1)  # nearest code by brute force
    q = o.unpack_nf4(packed.numpy())
    assert np.array_equal(q, idx.numpy())
    assert np.array_equal(o.pack_nf4(q), packed.numpy().reshape(-1))
    # the first byte holds element 0 in its high nibble
    assert int(packed.reshape(-1)[0]) >> 4 == int(idx[0])


def test_nested_scales_closed_form():
    """code2[a8] * absmax2[b // bs2] + offset, as torch evaluates it (tests/test_nf4gemv.py:95-111)."""
    from ttspipe_amd.quant import dequantize_blockwise_scales, quantize_4bit

    torch.manual_seed(1)
    w = torch.randn(64, 512) * 0.02
    _, state = quantize_4bit(w, blocksize=64, compress_statistics=True)
    theirs = dequantize_blockwise_scales(state.absmax, state.state2, state.offset).numpy()
    ours = o.scales(state.absmax.numpy(), state.state2.absmax.numpy(), state.state2.code.numpy(),
                    float(state.offset), state.state2.blocksize)
    assert np.array_equal(ours, theirs)
    # and the reconstruction is close to the true absmax (double quant works)
    true = w.reshape(-1, 64).abs().amax(1).numpy()
    assert np.max(np.abs(ours - true)) < 0.02 * np.max(true)


@pytest.mark.parametrize("nested", [False, True])
@pytest.mark.parametrize("dt", [o.DT_F16, o.DT_BF16, o.DT_F32])
def test_dequant_matches_closed_form(orc, nested, dt):
    layer = random_layer(48, 384, nested, seed=3)
    n = 48 * 384
    ours = orc.nf4_dequant(**oracle_args(layer), out_dtype=dt, n=n, bs=64, bs2=layer["bs2"] or 256)
    assert np.array_equal(ours, dequant_numpy(layer, dt))


def test_dequant_mutant_nibble_order_is_caught(orc):
    """Planted slip: decoding the low nibble first disagrees with the closed form."""
    layer = random_layer(4, 128, False, seed=4)
    swapped = dict(layer)
    swapped["W"] = ((layer["W"] << 4) | (layer["W"] >> 4)).astype(np.uint8)
    bad = orc.nf4_dequant(**oracle_args(swapped), out_dtype=o.DT_F32, n=512, bs=64)
    assert not np.array_equal(bad, dequant_numpy(layer, o.DT_F32))


@pytest.mark.parametrize("dt", [o.DT_F16, o.DT_BF16])
def test_gemm_ref_is_fp64_brute_force(orc, dt):
    layer = random_layer(24, 256, True, seed=5)
    rng = np.random.default_rng(6)
    x = o.from_f32(rng.standard_normal((3, 256)).astype(np.float32), dt)
    y = orc.nf4_gemm_ref(x, dt, **oracle_args(layer), M=24, K=256, N=3, bs=64)
    w = o.to_f32(dequant_numpy(layer, dt), dt).astype(np.float64).reshape(24, 256)
    expect = o.to_f32(x, dt).astype(np.float64) @ w.T
    assert np.allclose(y, expect, rtol=1e-12, atol=1e-12)
    # planted slip: the transposed product is a different number
    assert not np.allclose(y, (o.to_f32(x, dt).astype(np.float64) @ w[:, :].T)[:, ::-1])


def test_gemv_closed_form_constant_codes(orc):
    """All codes 15 (1.0), one scale s, x = 1: y = round(s * K) exactly."""
    M, K = 8, 512
    layer = {"W": np.full(M * K // 2, 0xFF, np.uint8), "A8": None,
             "AMAX": np.full(M * K // 64, 0.5, np.float32), "CODE2": None, "offset": 0.0}
    x = o.from_f32(np.ones(K, np.float32), o.DT_F16)
    y = orc.gemv_emul(x, o.DT_F16, **layer, M=M, K=K, bs=64, KS=1, J=1)
    assert np.all(o.to_f32(y, o.DT_F16) == 256.0)


@pytest.mark.parametrize("shape", [(64, 2560), (40, 9728), (96, 1024), (32, 4096)])
@pytest.mark.parametrize("nested", [False, True])
@pytest.mark.parametrize("dt", [o.DT_F16, o.DT_BF16])
@pytest.mark.parametrize("KS", [1, 2, 4])
def test_gemv_emul_agrees_with_fp64(orc, shape, nested, dt, KS):
    M, K = shape
    KD = K // 8
    if KD < 64 * KS:
        pytest.skip("slice narrower than a wave")
    J = -(-KD // (64 * KS))
    layer = random_layer(M, K, nested, seed=M + K + KS)
    x = o.from_f32(np.random.default_rng(7).standard_normal(K).astype(np.float32), dt)
    y = orc.gemv_emul(x, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, bs2=layer["bs2"] or 256)
    # against bitsandbytes' arithmetic (weights rounded to dt) and against exact NF4 weights
    for exact in (False, True):
        ref = orc.nf4_gemm_ref(x, dt, **oracle_args(layer), M=M, K=K, N=1, bs=64, bs2=layer["bs2"] or 256,
                               exact=exact)
        assert beyond_rounding_error(o.to_f32(y, dt), ref.reshape(-1), dt) < (5e-4 if exact else 2e-3)


@pytest.mark.parametrize("epi", [1, 2])
def test_gemv_epilogues_closed_form(orc, epi):
    M, K, dt = 64, 1024, o.DT_BF16
    layer = random_layer(M, K, True, seed=8)
    rng = np.random.default_rng(9)
    x = o.from_f32(rng.standard_normal(K).astype(np.float32), dt)
    r = o.from_f32(rng.standard_normal(M).astype(np.float32) * 2, dt)
    plain = o.to_f32(orc.gemv_emul(x, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=1, J=2), dt)
    got = o.to_f32(orc.gemv_emul(x, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=1, J=2, R=r, epi=epi), dt)
    rf = o.to_f32(r, dt).astype(np.float64)
    if epi == 1:
        expect = rf + plain
    else:
        expect = (rf / (1 + np.exp(-rf))) * plain
    assert relative_error(got, expect) < 8e-3


@pytest.mark.parametrize("rows,width", [(1, 2560), (32, 128), (8, 128), (1, 9728), (3, 2560), (1, 40)])
@pytest.mark.parametrize("dt", [o.DT_F16, o.DT_BF16])
def test_rms_norm_emul_matches_the_fork_formula(orc, rows, width, dt):
    """Against torch running the fork's formula on the CPU (fusedops.py:8-14):
    the reference's own bar - >= 99.5% identical, worst < 2e-3 (test_fusedops.py:103-107)."""
    from ttspipe_amd.llama import RMSNorm

    g = torch.Generator().manual_seed(rows * 1000 + width)
    tdt = torch.float16 if dt == o.DT_F16 else torch.bfloat16
    x = torch.randn(1, rows, width, generator=g).to(tdt)
    norm = RMSNorm(width, 1e-6, dtype=tdt)
    norm.weight.data.copy_((torch.randn(width, generator=g) * 0.1 + 1).to(tdt))
    theirs = RMSNorm.forward(norm, x).reshape(-1)
    xu = x.view(torch.int16).numpy().view(np.uint16).reshape(-1)
    wu = norm.weight.data.view(torch.int16).numpy().view(np.uint16)
    ours = orc.rms_norm_emul(xu, wu, rows, width, 1e-6, dt)
    ours_f = o.to_f32(ours, dt)
    theirs_f = theirs.float().numpy()
    identical = float(np.mean(ours_f == theirs_f))
    worst = float(np.max(np.abs(ours_f - theirs_f) / np.maximum(np.abs(theirs_f), 1e-4)))
    assert identical > 0.995 and worst < 2e-2 if dt == o.DT_BF16 else worst < 2e-3
    ref = orc.rms_norm_ref(xu, wu, rows, width, 1e-6, dt)
    assert float(np.mean(ours_f == ref.astype(np.float32))) > 0.995


def test_rms_norm_mutant_single_rounding_is_caught(orc):
    """Skipping the round before the weight multiply leaves far fewer elements identical."""
    rows, width, dt = 4, 2560, o.DT_F16
    rng = np.random.default_rng(11)
    x = o.from_f32(rng.standard_normal(rows * width).astype(np.float32), dt)
    w = o.from_f32((rng.standard_normal(width) * 0.1 + 1).astype(np.float32), dt)
    ours = o.to_f32(orc.rms_norm_emul(x, w, rows, width, 1e-6, dt), dt)
    xf = o.to_f32(x, dt).astype(np.float64).reshape(rows, width)
    r = 1 / np.sqrt((xf * xf).mean(1, keepdims=True) + 1e-6)
    single = o.to_f32(o.from_f32((xf * r * o.to_f32(w, dt)).astype(np.float32).reshape(-1), dt), dt)
    assert np.mean(ours == single) < 0.99


@pytest.mark.parametrize("shape", [(1, 1, 32, 128), (1, 1, 8, 128), (1, 4, 32, 128), (2, 3, 8, 64)])
@pytest.mark.parametrize("fdt", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("xdt", [torch.float16, torch.bfloat16])
def test_rope_is_bit_exact_against_torch(orc, shape, fdt, xdt):
    from ttspipe_amd.llama import apply_rotary_emb

    b, s, h, d = shape
    g = torch.Generator().manual_seed(hash(shape) % 9973)
    x = torch.randn(*shape, generator=g).to(xdt)
    f = torch.randn(s, d // 2, 2, generator=g).to(fdt)
    theirs = apply_rotary_emb(x, f)
    dt = o.DT_F16 if xdt == torch.float16 else o.DT_BF16
    ft = {torch.float32: o.DT_F32, torch.float16: o.DT_F16, torch.bfloat16: o.DT_BF16}[fdt]
    fv = f.numpy() if fdt == torch.float32 else f.view(torch.int16).numpy().view(np.uint16)
    ours = orc.rope(x.view(torch.int16).numpy().view(np.uint16).reshape(-1), fv.reshape(-1), ft, d // 2, h, s, dt)
    assert np.array_equal(ours, theirs.view(torch.int16).numpy().view(np.uint16).reshape(-1))


def test_rope_reads_its_own_position(orc):
    from ttspipe_amd.llama import apply_rotary_emb

    s, h, d = 5, 2, 8
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, s, h, d, generator=g).to(torch.float16)
    f = torch.randn(s, d // 2, 2, generator=g).to(torch.bfloat16)
    whole = orc.rope(x.view(torch.int16).numpy().view(np.uint16).reshape(-1),
                     f.view(torch.int16).numpy().view(np.uint16).reshape(-1), o.DT_BF16, d // 2, h, s, o.DT_F16)
    whole = whole.reshape(1, s, h, d)
    for i in range(s):
        alone = apply_rotary_emb(x[:, i : i + 1], f[i : i + 1])
        assert np.array_equal(whole[:, i : i + 1], alone.view(torch.int16).numpy().view(np.uint16))
    # planted slip: reading row 0 for every position changes positions 1..s-1
    f0 = f[0:1].expand(s, -1, -1).contiguous()
    wrong = orc.rope(x.view(torch.int16).numpy().view(np.uint16).reshape(-1),
                     f0.view(torch.int16).numpy().view(np.uint16).reshape(-1), o.DT_BF16, d // 2, h, s, o.DT_F16)
    assert not np.array_equal(wrong.reshape(1, s, h, d)[:, 1:], whole[:, 1:])


def _kv(nkv, max_len, dt, seed):
    rng = np.random.default_rng(seed)
    kc = o.from_f32(rng.standard_normal(nkv * max_len * 128).astype(np.float32), dt)
    vc = o.from_f32(rng.standard_normal(nkv * max_len * 128).astype(np.float32), dt)
    return kc, vc


@pytest.mark.parametrize("L", [1, 10, 63, 64, 65, 401, 2048])
@pytest.mark.parametrize("dt", [o.DT_F16, o.DT_BF16])
def test_attn_emul_agrees_with_fp64(orc, L, dt):
    nh, nkv, max_len = 32, 8, 2304
    kc, vc = _kv(nkv, max_len, dt, seed=L)
    q = o.from_f32(np.random.default_rng(L + 1).standard_normal(nh * 128).astype(np.float32) * 2, dt)
    nchunk = -(-max_len // 64)
    y = orc.attn_emul(q, kc, vc, L - 1, nh, nkv, max_len, nchunk, 128**-0.5, dt)
    ref = orc.attn_ref(q, kc, vc, L, nh, nkv, max_len, 128**-0.5, dt)
    assert relative_error(o.to_f32(y, dt), ref) < 5e-3


def test_attn_heads_map_onto_their_kv_head(orc):
    """Query head i reads KV head i // groups (tests/test_nf4gemv.py:297-319): identical
    keys make attention a plain average, so each head reads back its group's value."""
    nh, nkv, max_len, dt = 8, 2, 3, o.DT_F16
    q = o.from_f32(np.zeros(nh * 128, np.float32), dt)
    kc = o.from_f32(np.zeros(nkv * max_len * 128, np.float32), dt)
    v = np.zeros((nkv, max_len, 128), np.float32)
    for h in range(nkv):
        v[h] = h + 1
    y = orc.attn_emul(q, kc, o.from_f32(v.reshape(-1), dt), max_len - 1, nh, nkv, max_len, 1, 128**-0.5, dt)
    y = o.to_f32(y, dt).reshape(nh, 128)
    for head in range(nh):
        assert np.all(y[head] == head // (nh // nkv) + 1)


def test_attn_ignores_positions_past_pos(orc):
    nh, nkv, max_len, dt = 32, 8, 256, o.DT_BF16
    kc, vc = _kv(nkv, max_len, dt, seed=3)
    q = o.from_f32(np.random.default_rng(4).standard_normal(nh * 128).astype(np.float32), dt)
    a = orc.attn_emul(q, kc, vc, 40, nh, nkv, max_len, 4, 128**-0.5, dt)
    kc2, vc2 = kc.reshape(nkv, max_len, 128).copy(), vc.reshape(nkv, max_len, 128).copy()
    kc2[:, 41:] = o.from_f32(np.float32([1e3]), dt)[0]
    vc2[:, 41:] = o.from_f32(np.float32([-1e3]), dt)[0]
    b = orc.attn_emul(q, kc2.reshape(-1), vc2.reshape(-1), 40, nh, nkv, max_len, 4, 128**-0.5, dt)
    assert np.array_equal(a, b)


def test_qk_rope_kv_matches_unfused_ops(orc):
    """Head norm (one rounding) + rotary + cache write against torch's unfused ops."""
    from ttspipe_amd.llama import HeadNorm, apply_rotary_emb, precompute_freqs_cis

    nh, nkv, max_len, pos = 4, 2, 16, 9
    tdt, dt = torch.bfloat16, o.DT_BF16
    g = torch.Generator().manual_seed(12)
    qkv = torch.randn((nh + 2 * nkv) * 128, generator=g).to(tdt)
    qn, kn = HeadNorm(128, 1e-6, dtype=tdt), HeadNorm(128, 1e-6, dtype=tdt)
    qn.weight.data.copy_((torch.rand(128, generator=g) + 0.5).to(tdt))
    kn.weight.data.copy_((torch.rand(128, generator=g) + 0.5).to(tdt))
    freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos : pos + 1]
    u16 = lambda t: t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)  # noqa: E731
    Q = np.zeros(nh * 128, np.uint16)
    KC = np.zeros(nkv * max_len * 128, np.uint16)
    VC = np.zeros(nkv * max_len * 128, np.uint16)
    orc.qk_rope_kv(u16(qkv), u16(qn.weight.data), u16(kn.weight.data), 1e-6, u16(freqs), o.DT_BF16, pos,
                   Q, KC, VC, nh, nkv, max_len, dt)
    q = qkv[: nh * 128].view(1, 1, nh, 128)
    k = qkv[nh * 128 : (nh + nkv) * 128].view(1, 1, nkv, 128)
    v = qkv[(nh + nkv) * 128 :].view(nkv, 128)
    q_ref = apply_rotary_emb(qn(q), freqs)
    k_ref = apply_rotary_emb(kn(k), freqs)
    assert relative_error(o.to_f32(Q, dt), q_ref.float().numpy().reshape(-1)) < 1e-2
    KC = KC.reshape(nkv, max_len, 128)
    assert relative_error(o.to_f32(KC[:, pos], dt), k_ref.float().numpy().reshape(nkv, 128)) < 1e-2
    assert np.array_equal(VC.reshape(nkv, max_len, 128)[:, pos], u16(v).reshape(nkv, 128))
    assert not KC[:, :pos].any() and not KC[:, pos + 1 :].any()


@pytest.mark.parametrize("dt", [o.DT_BF16, o.DT_F16])
def test_qk_head_norm_rounds_once_bitwise(orc, dt):
    """The head norm is y = round((x * r) * w) with a single rounding to the
    16-bit type, r = 1 / sqrt(ss / 128 + eps) in fp32 (reference
    fusedlayer.py:75-83), followed by the no-fma rotary; restated here in
    numpy float32 and compared bit for bit. x are multiples of 1/16 below 4,
    so every square and every partial sum of squares is exact in fp32 and the
    sum does not depend on its order. A double-rounding mutant,
    round(round(x * r) * w), differs on a visible fraction of elements."""
    from ttspipe_amd.llama import precompute_freqs_cis

    nh, nkv, max_len, pos, eps = 6, 2, 32, 21, 1e-6
    rng = np.random.default_rng(40 + dt)
    xf = (rng.integers(-63, 64, (nh + 2 * nkv, 128)) / 16.0).astype(np.float32)
    wf = o.to_f32(o.from_f32((rng.random((2, 128)) + 0.5).astype(np.float32), dt), dt)
    qkv = o.from_f32(xf.reshape(-1), dt)
    assert np.array_equal(o.to_f32(qkv, dt).reshape(xf.shape), xf)  # exact in the 16-bit type
    freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos]
    fb = freqs.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)
    Q = np.zeros(nh * 128, np.uint16)
    KC = np.zeros(nkv * max_len * 128, np.uint16)
    VC = np.zeros(nkv * max_len * 128, np.uint16)
    orc.qk_rope_kv(qkv, o.from_f32(wf[0], dt), o.from_f32(wf[1], dt), eps, fb, o.DT_BF16, pos, Q, KC, VC,
                   nh, nkv, max_len, dt)
    f = o.to_f32(fb, o.DT_BF16).reshape(64, 2)
    c, s = f[:, 0], f[:, 1]

    def expect(x, w, double):
        ss = np.float32((x.astype(np.float64) ** 2).sum())  # exact, so any order
        r = np.float32(1.0) / np.sqrt(ss / np.float32(128.0) + np.float32(eps))
        xr = x * r
        if double:
            xr = o.to_f32(o.from_f32(xr, dt), dt)
        y = o.to_f32(o.from_f32(xr * w, dt), dt)
        x0, x1 = y[0::2], y[1::2]
        out = np.empty(128, np.float32)
        out[0::2] = x0 * c - x1 * s
        out[1::2] = x1 * c + x0 * s
        return o.from_f32(out, dt)

    got_q = Q.reshape(nh, 128)
    got_k = KC.reshape(nkv, max_len, 128)[:, pos]
    differ = 0
    for h in range(nh + nkv):
        got = got_q[h] if h < nh else got_k[h - nh]
        w = wf[0] if h < nh else wf[1]
        assert np.array_equal(got, expect(xf[h], w, False)), f"head {h}: {first_diff(got, expect(xf[h], w, False))}"
        differ += int((got != expect(xf[h], w, True)).sum())
    assert differ > 0.02 * (nh + nkv) * 128, f"the double-rounding mutant differs on only {differ} elements"
    assert np.array_equal(VC.reshape(nkv, max_len, 128)[:, pos], qkv.reshape(-1, 128)[nh + nkv:])


def first_diff(a, b):
    i = np.flatnonzero(a != b)
    return "identical" if i.size == 0 else f"{i.size} differ, first at {i[0]}: {a[i[0]]:#06x} vs {b[i[0]]:#06x}"


def test_exp_is_within_a_few_ulp(orc):
    x = np.linspace(-86.9, 88.5, 20001, dtype=np.float32)
    got = orc.exp_cw(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - ref) / ulp) <= 3.0
    assert orc.exp_cw(np.float32([-87.5, -200.0])).tolist() == [0.0, 0.0]
    assert math.isinf(float(orc.exp_cw(np.float32([89.0]))[0]))


def _splitmix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = z + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


@pytest.mark.parametrize("kind", [0, 1, 3])
def test_synth_fill_matches_numpy_splitmix(orc, kind):
    n, seed = 10007, 123456789
    got = orc.synth_fill(n, seed, kind, 0.5, 0.25)
    ms = _splitmix(np.array([seed], np.uint64))[0]
    h = _splitmix(ms ^ np.arange(n, dtype=np.uint64))
    if kind == 0:
        expect = (h >> np.uint64(56)).astype(np.uint8)
    else:
        u = (h >> np.uint64(40)).astype(np.float32) * np.float32(2.0**-23) - np.float32(1.0)
        v = (u * np.float32(0.5) + np.float32(0.25)).astype(np.float32)
        expect = o.f32_to_bf16(v) if kind == 1 else v
    assert np.array_equal(got, expect)


def test_embed_sum_and_argmax(orc):
    rng = np.random.default_rng(13)
    vocab, D, ntok = 50, 64, 3
    E = o.from_f32(rng.standard_normal(ntok * vocab * D).astype(np.float32), o.DT_BF16)
    tok = np.array([4, 0, 49], np.int32)
    got = orc.embed_sum(E, tok, vocab, D, o.DT_BF16)
    Ef = o.to_f32(E, o.DT_BF16).reshape(ntok, vocab, D)
    expect = o.from_f32((Ef[0, 4] + Ef[1, 0]) + Ef[2, 49], o.DT_BF16)
    assert np.array_equal(got, expect)
    x = o.from_f32(np.float32([1, 5, 3, 5, -2]), o.DT_F16)
    assert orc.argmax(x, o.DT_F16) == 1


# ------------------------------------------------------------------ sampler


def test_sampler_ref_closed_forms():
    """top_k = 1 and top_p = 0 keep only the largest logit (first index among
    ties); equal uniforms make the draw the largest kept logit."""
    rng = np.random.default_rng(0)
    l = rng.standard_normal(300)
    l[17] = l[200] = l.max() + 1.0
    u = rng.random(300)
    assert o.sample_topk_ref(l, 0.7, 0.9, 1, u)[0] == 17
    assert o.sample_topk_ref(l, 0.7, 0.0, 40, u)[0] == 17
    best, kept, c, _ = o.sample_topk_ref(l, 1.0, 1.0, 64, np.full(300, 0.5))
    assert best == 17 and kept.size == 64 and np.all(np.diff(l[kept]) <= 0)


def test_sampler_ref_draws_from_the_truncated_tempered_softmax():
    """Gumbel-max over the kept set with fresh uniforms: empirical frequencies
    match softmax(l / T) restricted to the kept candidates (a dropped
    temperature or a wrong cut fails this)."""
    rng = np.random.default_rng(1)
    l = np.array([2.0, 1.5, 1.0, 0.5, 0.0, -0.5, -1.0, -3.0])
    T, top_p, top_k, n = 0.8, 0.93, 6, 40000
    counts = np.zeros(l.size)
    for _ in range(n):
        counts[o.sample_topk_ref(l, T, top_p, top_k, rng.random(l.size))[0]] += 1
    _, kept, _, _ = o.sample_topk_ref(l, T, top_p, top_k, np.full(l.size, 0.5))
    q = np.zeros(l.size)
    q[kept] = np.exp(l[kept] / T)
    q /= q.sum()
    assert np.abs(counts / n - q).max() < 0.01
    # the cut: softmax(l) cumulative <= top_p, first always kept
    p = np.exp(l - l.max()) / np.exp(l - l.max()).sum()
    assert set(kept) == {i for i in range(top_k) if i == 0 or np.cumsum(p)[i] <= top_p}
