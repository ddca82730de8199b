"""Fused RMSNorm, rotary, qk-norm/rope/KV write, decode attention and the
whole fused decode block against the oracle (GPU).

Bar: bit for bit against the oracle's emulation (each kernel's fixed order);
RMSNorm also against the fork's formula at the reference's thresholds
(tests/test_fusedops.py:103-107), rotary bit for bit against torch's unfused
chain (tests/test_fusedops.py:151-163), attention within 5e-3 of fp64, the
fused block against the unfused block at the reference's 5e-3
(tests/test_fused_decode.py:96-103).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.conftest import relative_error, ulp16
from tests.gpuutil import bits, dt_code, first_mismatch, from_bits, gemv_shape, randn_bits

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


@pytest.fixture(scope="module")
def fused():
    from ttspipe_amd import fusedops

    assert fusedops._built() is not None
    return fusedops


# ------------------------------------------------------------------ RMSNorm

# rows up to 4096 wide are held in registers, wider ones streamed twice;
# 520 and 4104 leave the last 64-chunk step partly filled
@pytest.mark.parametrize("rows,width", [(1, 2560), (32, 128), (8, 128), (1, 9728), (3, 2560), (1, 40),
                                        (512, 2560), (1, 1024), (5, 520), (2, 4096), (2, 4104)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_rms_norm_bit_exact_and_matches_the_fork(fused, orc, rows, width, dtype):
    from ttspipe_amd.llama import RMSNorm

    dt = dt_code(dtype)
    xb = randn_bits(rows * width, dtype, seed=rows * 1000 + width)
    wb = o.from_f32((np.random.default_rng(width).standard_normal(width) * 0.1 + 1).astype(np.float32), dt)
    x = from_bits(xb, dtype).view(1, rows, width)
    w = from_bits(wb, dtype)
    before = fused.stats()["norm"]
    y = fused.rms_norm(x, w, 1e-6)
    assert y is not None and fused.stats()["norm"] == before + 1
    assert y.shape == x.shape and y.dtype == dtype
    expect = orc.rms_norm_emul(xb, wb, rows, width, 1e-6, dt)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)
    norm = RMSNorm(width, 1e-6, dtype=dtype, device="cuda")
    norm.weight.data.copy_(w)
    theirs = getattr(RMSNorm, "_fused_original_forward", RMSNorm.forward)(norm, x)
    identical = (y == theirs).float().mean().item()
    worst = ((y.float() - theirs.float()).abs() / theirs.float().abs().clamp(min=1e-4)).max().item()
    assert identical > 0.995, f"only {identical:.4f} identical"
    # one 16-bit ulp apart at most (bf16's ulp is 2^-7 relative)
    assert worst < (2e-3 if dtype == torch.float16 else 8e-3)


def test_rms_norm_declines_fp32_and_views(fused):
    w = torch.ones(256, device="cuda")
    assert fused.rms_norm(torch.randn(1, 1, 256, device="cuda"), w, 1e-6) is None
    wide = torch.randn(1, 4, 256, device="cuda", dtype=torch.float16)
    assert fused.rms_norm(wide[..., :128], torch.ones(128, device="cuda", dtype=torch.float16), 1e-6) is None


def test_patched_norm_falls_back_without_changing_the_answer(fused):
    from ttspipe_amd.llama import RMSNorm

    assert fused.install()
    norm = RMSNorm(256, 1e-6, dtype=torch.float32, device="cuda")
    x = torch.randn(1, 2, 256, device="cuda")
    before = fused.stats()["norm_fallback"]
    ours = norm(x)
    assert fused.stats()["norm_fallback"] == before + 1
    assert torch.equal(ours, RMSNorm._fused_original_forward(norm, x))


# ------------------------------------------------------------------ rotary

# head dims that are multiples of 8 take four pairs a thread; 6 and 10 one
@pytest.mark.parametrize("shape", [(1, 1, 32, 128), (1, 1, 8, 128), (1, 4, 32, 128), (2, 3, 8, 64),
                                   (1, 512, 32, 128), (1, 3, 4, 6), (2, 5, 3, 10)])
@pytest.mark.parametrize("fdt", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("dtype", DTYPES)
def test_rope_is_bit_exact(fused, orc, shape, fdt, dtype):
    from ttspipe_amd.llama import apply_rotary_emb

    b, s, h, d = shape
    g = torch.Generator().manual_seed(hash(shape) % 9973)
    x = torch.randn(*shape, generator=g).to(dtype)
    f = torch.randn(s, d // 2, 2, generator=g).to(fdt)
    y = fused.rope(x.cuda(), f.cuda())
    assert y is not None and y.shape == x.shape and y.dtype == dtype
    theirs = apply_rotary_emb(x, f)
    assert torch.equal(y.cpu(), theirs)
    ours = orc.rope(bits(x), bits(f), dt_code(fdt), d // 2, h, s, dt_code(dtype))
    assert np.array_equal(bits(y), ours)


@pytest.mark.parametrize("offset", [0, 2, 8])
def test_rope_on_a_buffer_not_16_byte_aligned(fused, offset):
    """A contiguous tensor starting 4 or 16 bytes into its buffer gives the same bits."""
    from ttspipe_amd.llama import apply_rotary_emb

    shape = (1, 6, 8, 128)
    n = int(np.prod(shape))
    g = torch.Generator().manual_seed(offset + 5)
    buf = torch.randn(n + 8, generator=g).to(torch.bfloat16)
    x = buf.cuda()[offset : offset + n].view(shape)
    f = torch.randn(6, 64, 2, generator=g).to(torch.float32).cuda()
    y = fused.rope(x, f)
    assert y is not None
    assert torch.equal(y.cpu(), apply_rotary_emb(x.cpu(), f.cpu()))


def test_rope_uses_the_frequencies_of_its_own_position(fused):
    from ttspipe_amd.llama import apply_rotary_emb

    seq, heads, d = 5, 2, 8
    x = torch.randn(1, seq, heads, d, device="cuda", dtype=torch.float16)
    f = torch.randn(seq, d // 2, 2, device="cuda", dtype=torch.bfloat16)
    whole = fused.rope(x, f)
    for s in range(seq):
        alone = apply_rotary_emb(x[:, s : s + 1].cpu(), f[s : s + 1].cpu())
        assert torch.equal(whole[:, s : s + 1].cpu(), alone)


def test_rope_declines(fused):
    packed = torch.randn(1, 4, 32, 256, device="cuda", dtype=torch.float16)
    freqs = torch.randn(4, 64, 2, device="cuda", dtype=torch.bfloat16)
    assert fused.rope(packed[..., :128], freqs) is None
    x = torch.randn(1, 4, 32, 128, device="cuda", dtype=torch.float16)
    assert fused.rope(x, torch.randn(2, 64, 2, device="cuda", dtype=torch.bfloat16)) is None


# ------------------------------------------------- qk norm + rope + KV write

@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("pos", [0, 37, 2047])
def test_qk_rope_kv_bit_exact(hip, orc, qk_norm, dtype, pos):
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    nh, nkv, max_len, dt = 32, 8, 2304, dt_code(dtype)
    qkvb = randn_bits((nh + 2 * nkv) * 128, dtype, seed=pos)
    qwb = o.from_f32((np.random.default_rng(1).random(128) + 0.5).astype(np.float32), dt)
    kwb = o.from_f32((np.random.default_rng(2).random(128) + 0.5).astype(np.float32), dt)
    freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos : pos + 1].contiguous()
    kcb = randn_bits(nkv * max_len * 128, dtype, seed=3)
    vcb = randn_bits(nkv * max_len * 128, dtype, seed=4)
    Q = torch.empty(nh * 128, dtype=dtype, device="cuda")
    KC, VC = from_bits(kcb, dtype), from_bits(vcb, dtype)
    qw = from_bits(qwb, dtype) if qk_norm else None
    kw = from_bits(kwb, dtype) if qk_norm else None
    posd = torch.tensor([pos], dtype=torch.long, device="cuda")
    fd = freqs.cuda()
    qkv = from_bits(qkvb, dtype)  # held: the launch is asynchronous
    rc = hip.ttsp_qk_rope_kv(qkv.data_ptr(), _lib.ptr(qw), _lib.ptr(kw), 1e-6, fd.data_ptr(),
                             o.DT_BF16, posd.data_ptr(), Q.data_ptr(), KC.data_ptr(), VC.data_ptr(), nh, nkv,
                             max_len, dt, _lib.stream())
    assert rc == 0
    Qo = np.zeros(nh * 128, np.uint16)
    KCo, VCo = kcb.copy(), vcb.copy()
    orc.qk_rope_kv(qkvb, qwb if qk_norm else None, kwb if qk_norm else None, 1e-6, bits(freqs), o.DT_BF16, pos,
                   Qo, KCo, VCo, nh, nkv, max_len, dt)
    assert np.array_equal(bits(Q), Qo), first_mismatch(bits(Q), Qo)
    assert np.array_equal(bits(KC), KCo), first_mismatch(bits(KC), KCo)
    assert np.array_equal(bits(VC), VCo)


# ------------------------------------------------------------ decode attention

@pytest.mark.parametrize("L", [1, 10, 17, 64, 65, 401, 2048, 2304])
@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_attention_bit_exact(hip, orc, L, dtype):
    from ttspipe_amd import _lib

    nh, nkv, max_len, dt = 32, 8, 2304, dt_code(dtype)
    nchunk = -(-max_len // 64)
    qb = randn_bits(nh * 128, dtype, seed=L, scale=2.0)
    kcb = randn_bits(nkv * max_len * 128, dtype, seed=L + 1)
    vcb = randn_bits(nkv * max_len * 128, dtype, seed=L + 2)
    f32 = dict(dtype=torch.float32, device="cuda")
    pm, pl, pacc = torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk * 128, **f32)
    y = torch.empty(nh * 128, dtype=dtype, device="cuda")
    posd = torch.tensor([L - 1], dtype=torch.long, device="cuda")
    qd, kd, vd = from_bits(qb, dtype), from_bits(kcb, dtype), from_bits(vcb, dtype)  # held across the launch
    rc = hip.ttsp_attn_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), posd.data_ptr(), pm.data_ptr(), pl.data_ptr(),
                              pacc.data_ptr(), y.data_ptr(), nh, nkv, max_len, nchunk, float(128**-0.5), dt,
                              _lib.stream())
    assert rc == 0
    expect = orc.attn_emul(qb, kcb, vcb, L - 1, nh, nkv, max_len, nchunk, 128**-0.5, dt)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)
    ref = orc.attn_ref(qb, kcb, vcb, L, nh, nkv, max_len, 128**-0.5, dt)
    assert relative_error(o.to_f32(bits(y), dt), ref) < 5e-3


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("positions,max_len,nh,nkv,nchunk", [
    ([512, 513], 2304, 32, 8, 36),                  # a 2-token tail after 512 cached positions
    ([0, 1, 2, 3, 4], 8, 8, 2, 1),                  # a first span: the window ends with it
    ([60, 61, 62, 63, 64, 65, 66, 67], 128, 4, 1, 2),  # a span across a chunk edge
    (list(range(2290, 2304)), 2304, 32, 8, 36),     # the cache's last positions
    ([7, 300, 41, 2000, 64, 65], 2304, 16, 4, 36)])  # rows in any order, one a row
def test_decode_attention_rows_equal_one_position_each(hip, orc, dtype, positions, max_len, nh, nkv, nchunk):
    """ttsp_attn_decode_rows == ttsp_attn_decode for each row's position, bit
    for bit, and row 0 against the oracle's emulation."""
    from ttspipe_amd import _lib

    S, dt = len(positions), dt_code(dtype)
    qb = randn_bits(S * nh * 128, dtype, seed=S + nh, scale=2.0)
    kcb = randn_bits(nkv * max_len * 128, dtype, seed=S + 1)
    vcb = randn_bits(nkv * max_len * 128, dtype, seed=S + 2)
    f32 = dict(dtype=torch.float32, device="cuda")
    qd, kd, vd = from_bits(qb, dtype), from_bits(kcb, dtype), from_bits(vcb, dtype)
    posd = torch.tensor(positions, dtype=torch.long, device="cuda")
    pm, pl = torch.empty(S * nh * nchunk, **f32), torch.empty(S * nh * nchunk, **f32)
    pacc = torch.empty(S * nh * nchunk * 128, **f32)
    y = torch.empty(S, nh * 128, dtype=dtype, device="cuda")
    rc = hip.ttsp_attn_decode_rows(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), posd.data_ptr(), pm.data_ptr(),
                                   pl.data_ptr(), pacc.data_ptr(), y.data_ptr(), nh, nkv, max_len, nchunk,
                                   float(128**-0.5), S, dt, _lib.stream())
    assert rc == 0
    for r, p in enumerate(positions):
        one = torch.empty(nh * 128, dtype=dtype, device="cuda")
        pr = torch.tensor([p], dtype=torch.long, device="cuda")
        rc = hip.ttsp_attn_decode(qd[r * nh * 128:].data_ptr(), kd.data_ptr(), vd.data_ptr(), pr.data_ptr(),
                                  pm.data_ptr(), pl.data_ptr(), pacc.data_ptr(), one.data_ptr(), nh, nkv, max_len,
                                  nchunk, float(128**-0.5), dt, _lib.stream())
        assert rc == 0
        assert np.array_equal(bits(y[r]), bits(one)), (r, p)
    expect = orc.attn_emul(qb[:nh * 128], kcb, vcb, positions[0], nh, nkv, max_len, nchunk, 128**-0.5, dt)
    assert np.array_equal(bits(y[0]), expect), first_mismatch(bits(y[0]), expect)


@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("positions,max_len,nh,nkv", [
    ([37], 2304, 32, 8),                             # one row
    ([512, 513], 2304, 32, 8),                       # a 2-token tail after 512 cached positions
    ([60, 61, 62, 63, 64, 65, 66, 67], 128, 4, 1),  # eight rows across a chunk edge
    ([2297, 2298, 2299, 2300, 2301, 2302, 2303], 2304, 16, 4),  # the cache's last positions
    ([7, 300, 41, 2000, 64, 65], 2304, 8, 2),        # rows in any order, one a chunk's first position
    ([0, 1, 2], 16, 8, 8)])                          # one head per kv head, a one-chunk cache
def test_rows_attention_from_qkv_equals_the_rows_kernels(hip, qk_norm, dtype, positions, max_len, nh, nkv):
    """ttsp_attn_decode_qkv_rows (each workgroup computing its row's query and
    the span rows its chunk holds) == ttsp_qk_rope_kv_rows then
    ttsp_attn_decode_rows, bit for bit: the output and every cache row."""
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    S, dt = len(positions), dt_code(dtype)
    nchunk = -(-max_len // 64)
    rs = (nh + 2 * nkv) * 128
    qkvb = randn_bits(S * rs, dtype, seed=S + nh, scale=2.0)
    qwb = o.from_f32((np.random.default_rng(7).random(128) + 0.5).astype(np.float32), dt)
    kwb = o.from_f32((np.random.default_rng(8).random(128) + 0.5).astype(np.float32), dt)
    table = precompute_freqs_cis(max_len, 128, 1e6)
    freqs = table[torch.tensor(positions)].contiguous().cuda()
    kcb = randn_bits(nkv * max_len * 128, dtype, seed=S + 12)
    vcb = randn_bits(nkv * max_len * 128, dtype, seed=S + 13)
    qkv = from_bits(qkvb, dtype)
    qw = from_bits(qwb, dtype) if qk_norm else None
    kw = from_bits(kwb, dtype) if qk_norm else None
    posd = torch.tensor(positions, dtype=torch.long, device="cuda")
    f32 = dict(dtype=torch.float32, device="cuda")
    outs = []
    for fused in (True, False):
        KC, VC = from_bits(kcb, dtype), from_bits(vcb, dtype)
        pm, pl = torch.empty(S * nh * nchunk, **f32), torch.empty(S * nh * nchunk, **f32)
        pacc = torch.empty(S * nh * nchunk * 128, **f32)
        y = torch.empty(S, nh * 128, dtype=dtype, device="cuda")
        if fused:
            rc = hip.ttsp_attn_decode_qkv_rows(qkv.data_ptr(), rs, _lib.ptr(qw), _lib.ptr(kw), 1e-6, freqs.data_ptr(),
                                               o.DT_BF16, posd.data_ptr(), KC.data_ptr(), VC.data_ptr(), pm.data_ptr(),
                                               pl.data_ptr(), pacc.data_ptr(), y.data_ptr(), nh, nkv, max_len, nchunk,
                                               float(128**-0.5), S, dt, _lib.stream())
            assert rc == 0
        else:
            q = torch.empty(S, nh * 128, dtype=dtype, device="cuda")
            rc = hip.ttsp_qk_rope_kv_rows(qkv.data_ptr(), rs, _lib.ptr(qw), _lib.ptr(kw), 1e-6, freqs.data_ptr(),
                                          o.DT_BF16, posd.data_ptr(), q.data_ptr(), KC.data_ptr(), VC.data_ptr(), nh,
                                          nkv, max_len, S, dt, _lib.stream())
            assert rc == 0
            rc = hip.ttsp_attn_decode_rows(q.data_ptr(), KC.data_ptr(), VC.data_ptr(), posd.data_ptr(), pm.data_ptr(),
                                           pl.data_ptr(), pacc.data_ptr(), y.data_ptr(), nh, nkv, max_len, nchunk,
                                           float(128**-0.5), S, dt, _lib.stream())
            assert rc == 0
        outs.append((bits(y), bits(KC), bits(VC)))
    for a, b in zip(*outs):
        assert np.array_equal(a, b), first_mismatch(a, b)


@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("pos,max_len,nh,nkv", [(0, 2304, 32, 8), (37, 2304, 32, 8), (63, 2304, 32, 8),
                                                (64, 2304, 32, 8), (2047, 2304, 32, 8), (2303, 2304, 32, 8),
                                                (0, 16, 8, 2), (9, 16, 8, 2), (15, 16, 8, 2), (100, 128, 4, 1),
                                                (70, 256, 8, 8), (130, 256, 4, 2), (200, 1024, 16, 1),
                                                (5000, 8192, 16, 1)])
def test_attention_from_qkv_bit_exact(hip, orc, qk_norm, dtype, pos, max_len, nh, nkv):
    """One pass (head norms, rotary, KV write, attention, merge) == qk_rope_kv then
    the split-K attention, through the oracle's emulations, and the cache rows."""
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    dt = dt_code(dtype)
    nchunk = -(-max_len // 64)
    qkvb = randn_bits((nh + 2 * nkv) * 128, dtype, seed=pos + 11, scale=2.0)
    qwb = o.from_f32((np.random.default_rng(5).random(128) + 0.5).astype(np.float32), dt)
    kwb = o.from_f32((np.random.default_rng(6).random(128) + 0.5).astype(np.float32), dt)
    freqs = precompute_freqs_cis(max_len, 128, 1e6)[pos : pos + 1].contiguous()
    kcb = randn_bits(nkv * max_len * 128, dtype, seed=pos + 12)
    vcb = randn_bits(nkv * max_len * 128, dtype, seed=pos + 13)
    KC, VC = from_bits(kcb, dtype), from_bits(vcb, dtype)
    f32 = dict(dtype=torch.float32, device="cuda")
    pm, pl, pacc = torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk * 128, **f32)
    y = torch.empty(nh * 128, dtype=dtype, device="cuda")
    qw = from_bits(qwb, dtype) if qk_norm else None
    kw = from_bits(kwb, dtype) if qk_norm else None
    posd = torch.tensor([pos], dtype=torch.long, device="cuda")
    fd, qkv = freqs.cuda(), from_bits(qkvb, dtype)
    rc = hip.ttsp_attn_decode_qkv(qkv.data_ptr(), _lib.ptr(qw), _lib.ptr(kw), 1e-6, fd.data_ptr(), o.DT_BF16,
                                  posd.data_ptr(), KC.data_ptr(), VC.data_ptr(), pm.data_ptr(), pl.data_ptr(),
                                  pacc.data_ptr(), y.data_ptr(), nh, nkv, max_len, nchunk, float(128**-0.5), dt,
                                  _lib.stream())
    assert rc == 0
    Qo = np.zeros(nh * 128, np.uint16)
    KCo, VCo = kcb.copy(), vcb.copy()
    orc.qk_rope_kv(qkvb, qwb if qk_norm else None, kwb if qk_norm else None, 1e-6, bits(freqs), o.DT_BF16, pos,
                   Qo, KCo, VCo, nh, nkv, max_len, dt)
    expect = orc.attn_emul(Qo, KCo, VCo, pos, nh, nkv, max_len, nchunk, 128**-0.5, dt)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)
    assert np.array_equal(bits(KC), KCo), first_mismatch(bits(KC), KCo)
    assert np.array_equal(bits(VC), VCo)


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("pos,max_len,nh,nkv,M", [(0, 16, 8, 2, 1024), (9, 16, 8, 2, 1024), (15, 16, 8, 2, 1024),
                                                  (37, 64, 4, 1, 640), (63, 64, 8, 2, 2048), (5, 8, 2, 2, 256),
                                                  (20, 32, 8, 4, 1024), (0, 1, 1, 1, 64)])
def test_attention_and_wo_in_one_launch(hip, nested, qk_norm, dtype, pos, max_len, nh, nkv, M):
    """ttsp_attn_nf4_gemv (every wo workgroup recomputes the one-chunk attention)
    == ttsp_attn_decode_qkv then the wo GEMV with the residual, bit for bit,
    and the same KV-cache rows."""
    from tests.nf4data import random_layer
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis
    from ttspipe_amd.quant import NF4_CODE

    dt = dt_code(dtype)
    K = nh * 128
    layer = random_layer(M, K, nested, seed=M + K + pos)
    W = torch.from_numpy(layer["W"]).cuda()
    A8 = torch.from_numpy(layer["A8"]).cuda() if nested else None
    AM = torch.from_numpy(layer["AMAX"]).cuda()
    C2 = torch.from_numpy(layer["CODE2"]).cuda() if nested else None
    lut = torch.tensor(NF4_CODE, dtype=torch.float32, device="cuda")
    qkvb = randn_bits((nh + 2 * nkv) * 128, dtype, seed=pos + 21, scale=2.0)
    qwb = o.from_f32((np.random.default_rng(5).random(128) + 0.5).astype(np.float32), dt)
    kwb = o.from_f32((np.random.default_rng(6).random(128) + 0.5).astype(np.float32), dt)
    freqs = precompute_freqs_cis(max(max_len, pos + 1), 128, 1e6)[pos : pos + 1].contiguous().cuda()
    kcb = randn_bits(nkv * max_len * 128, dtype, seed=pos + 22)
    vcb = randn_bits(nkv * max_len * 128, dtype, seed=pos + 23)
    rb = randn_bits(M, dtype, seed=pos + 24)
    qkv, R = from_bits(qkvb, dtype), from_bits(rb, dtype)
    qw = from_bits(qwb, dtype) if qk_norm else None
    kw = from_bits(kwb, dtype) if qk_norm else None
    posd = torch.tensor([pos], dtype=torch.long, device="cuda")
    scale = float(128**-0.5)
    offset = float(layer["offset"])
    bs2 = layer["bs2"] or 0

    # two launches
    KC1, VC1 = from_bits(kcb, dtype), from_bits(vcb, dtype)
    y = torch.empty(nh * 128, dtype=dtype, device="cuda")
    h1 = torch.empty(M, dtype=dtype, device="cuda")
    rc = hip.ttsp_attn_decode_qkv(qkv.data_ptr(), _lib.ptr(qw), _lib.ptr(kw), 1e-6, freqs.data_ptr(), o.DT_BF16,
                                  posd.data_ptr(), KC1.data_ptr(), VC1.data_ptr(), None, None, None, y.data_ptr(),
                                  nh, nkv, max_len, 1, scale, dt, _lib.stream())
    assert rc == 0
    rc = hip.ttsp_nf4_gemm(y.data_ptr(), dt, W.data_ptr(), _lib.ptr(A8), AM.data_ptr(), _lib.ptr(C2), offset,
                           lut.data_ptr(), h1.data_ptr(), R.data_ptr(), 1, M, K, 1, 64, bs2, _lib.stream())
    assert rc == 0
    # one launch
    KC2, VC2 = from_bits(kcb, dtype), from_bits(vcb, dtype)
    h2 = torch.empty(M, dtype=dtype, device="cuda")
    rc = hip.ttsp_attn_nf4_gemv(qkv.data_ptr(), _lib.ptr(qw), _lib.ptr(kw), 1e-6, freqs.data_ptr(), o.DT_BF16,
                                posd.data_ptr(), KC2.data_ptr(), VC2.data_ptr(), nh, nkv, max_len, scale,
                                W.data_ptr(), _lib.ptr(A8), AM.data_ptr(), _lib.ptr(C2), offset, lut.data_ptr(),
                                h2.data_ptr(), R.data_ptr(), 1, M, 64, bs2, dt, _lib.stream())
    assert rc == 0
    assert np.array_equal(bits(h2), bits(h1)), first_mismatch(bits(h2), bits(h1))
    assert np.array_equal(bits(KC2), bits(KC1)), first_mismatch(bits(KC2), bits(KC1))
    assert np.array_equal(bits(VC2), bits(VC1))


def test_attention_and_wo_declines_what_it_cannot_serve(hip):
    """Shapes outside the one-launch form are rejected with an error code (the
    caller then runs the two-launch form), never launched."""
    from ttspipe_amd import _lib

    d = torch.zeros(1 << 16, dtype=torch.float32, device="cuda")
    p = d.data_ptr()
    st = _lib.stream()
    # (nh, nkv, max_len): too many heads, a cache longer than one chunk, too many staged rows
    for nh, nkv, max_len in ((16, 2, 16), (8, 2, 65), (8, 4, 64), (6, 4, 16)):
        rc = hip.ttsp_attn_nf4_gemv(p, None, None, 1e-6, p, o.DT_F32, p, p, p, nh, nkv, max_len, 0.088, p, None, p,
                                    None, 0.0, p, p, p, 1, 64, 64, 0, o.DT_BF16, st)
        assert rc != 0, (nh, nkv, max_len)


def test_decode_attention_matches_torch_gqa():
    """Against torch SDPA with enable_gqa on the CPU, the reference's check
    (tests/test_nf4gemv.py:224-242)."""
    import torch.nn.functional as F

    from ttspipe_amd import _lib

    nh, nkv, L = 32, 8, 401
    torch.manual_seed(0)
    q = torch.randn(1, nh, 1, 128, dtype=torch.float16)
    k = torch.randn(1, nkv, L, 128, dtype=torch.float16)
    v = torch.randn(1, nkv, L, 128, dtype=torch.float16)
    theirs = F.scaled_dot_product_attention(q.float(), k.float(), v.float(), enable_gqa=True)
    f32 = dict(dtype=torch.float32, device="cuda")
    nchunk = -(-L // 64)
    pm, pl, pacc = torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk, **f32), torch.empty(nh * nchunk * 128, **f32)
    y = torch.empty(nh * 128, dtype=torch.float16, device="cuda")
    posd = torch.tensor([L - 1], dtype=torch.long, device="cuda")
    qd, kd, vd = q.cuda(), k.cuda().contiguous(), v.cuda().contiguous()  # held across the launch
    rc = _lib.load().ttsp_attn_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), posd.data_ptr(), pm.data_ptr(), pl.data_ptr(),
                                      pacc.data_ptr(), y.data_ptr(), nh, nkv, L, nchunk, float(128**-0.5), 0,
                                      _lib.stream())
    assert rc == 0
    assert relative_error(y.cpu().float().numpy(), theirs.reshape(-1).numpy()) < 5e-3


# ------------------------------------------------------------ the whole block

def _block(dtype, qk_norm, dim=512, n_head=4, n_local_heads=2, inter=1024, max_len=256, seed=0):
    """A small block on the GPU with seeded NF4 weights (the reference's test
    block: dim 512, 4 q / 2 kv heads of 128, FFN 1024, tests/test_fused_decode.py:46-71)."""
    from ttspipe_amd.llama import BaseModelArgs, KVCache, TransformerBlock
    from tests.nf4data import random_layer, to_linear

    cfg = BaseModelArgs(dim=dim, n_head=n_head, n_local_heads=n_local_heads, head_dim=128,
                        intermediate_size=inter, attention_qk_norm=qk_norm, norm_eps=1e-6)
    block = TransformerBlock(cfg, dtype=dtype, device="cuda")
    layers = {}
    for i, (parent, name, shape) in enumerate([
        (block.attention, "wqkv", ((n_head + 2 * n_local_heads) * 128, dim)),
        (block.attention, "wo", (dim, n_head * 128)),
        (block.feed_forward, "w1", (inter, dim)),
        (block.feed_forward, "w3", (inter, dim)),
        (block.feed_forward, "w2", (dim, inter)),
    ]):
        layers[name] = random_layer(*shape, True, seed=seed * 10 + i)
        setattr(parent, name, to_linear(layers[name], dtype))
    g = torch.Generator().manual_seed(seed)
    norms = [block.attention_norm, block.ffn_norm] + ([block.attention.q_norm, block.attention.k_norm] if qk_norm else [])
    for norm in norms:
        norm.weight.data.copy_((torch.rand(norm.weight.shape, generator=g) + 0.5).to(dtype))
    block.attention.kv_cache = KVCache(1, max_len, n_local_heads, 128, dtype=dtype, device="cuda")
    return block, layers


def _oracle_block(orc, block, layers, xb, pos, window, dt, freqs_row_bits, kcb, vcb):
    """The fused block composed from oracle emulations, kernel by kernel."""
    a = block.attention
    nh, nkv, D = a.n_head, a.n_local_heads, xb.size
    max_len = a.kv_cache.k_cache.shape[2]
    inter = block.feed_forward.w1.out_features
    wb = lambda p: bits(p.data)  # noqa: E731

    def gemv(name, x, R=None, epi=0):
        L = layers[name]
        J, KS, _ = gemv_shape(L["M"], L["K"])
        return orc.gemv_emul(x, dt, L["W"], L["A8"], L["AMAX"], L["CODE2"], L["offset"], M=L["M"], K=L["K"],
                             bs=64, KS=KS, J=J, bs2=L["bs2"], R=R, epi=epi)

    xn = orc.rms_norm_emul(xb, wb(block.attention_norm.weight), 1, D, 1e-6, dt)
    qkv = gemv("wqkv", xn)
    Q = np.zeros(nh * 128, np.uint16)
    qw = wb(a.q_norm.weight) if a.attention_qk_norm else None
    kw = wb(a.k_norm.weight) if a.attention_qk_norm else None
    orc.qk_rope_kv(qkv, qw, kw, 1e-6, freqs_row_bits, o.DT_BF16, pos, Q, kcb, vcb, nh, nkv, max_len, dt)
    nchunk = -(-min(window, max_len) // 64)
    y = orc.attn_emul(Q, kcb, vcb, pos, nh, nkv, max_len, nchunk, 128**-0.5, dt)
    h = gemv("wo", y, R=xb, epi=1)
    hn = orc.rms_norm_emul(h, wb(block.ffn_norm.weight), 1, D, 1e-6, dt)
    g1 = gemv("w1", hn)
    g = gemv("w3", hn, R=g1, epi=2)
    return gemv("w2", g, R=h, epi=1), kcb, vcb


@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("pos,window", [(0, 1), (37, 64), (200, 256)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_decode_block_matches_oracle_and_unfused_block(orc, qk_norm, pos, window, dtype):
    from ttspipe_amd import fusedlayer, fusedops, nf4gemv
    from ttspipe_amd.llama import TransformerBlock, precompute_freqs_cis

    assert nf4gemv.install() and fusedops.install() and fusedlayer.install()
    block, layers = _block(dtype, qk_norm, seed=pos)
    cache = block.attention.kv_cache
    dt = dt_code(dtype)
    kcb = randn_bits(cache.k_cache.numel(), dtype, seed=5)
    vcb = randn_bits(cache.v_cache.numel(), dtype, seed=6)
    cache.k_cache.copy_(from_bits(kcb, dtype).view_as(cache.k_cache))
    cache.v_cache.copy_(from_bits(vcb, dtype).view_as(cache.v_cache))
    freqs = precompute_freqs_cis(256, 128, 10000).cuda()
    xb = randn_bits(512, dtype, seed=pos + 7)
    x = from_bits(xb, dtype).view(1, 1, 512)
    ip = torch.tensor([pos], device="cuda", dtype=torch.long)
    mask = torch.ones(256, 256, dtype=torch.bool, device="cuda").tril()[None, None, ip, :window]
    f = freqs[ip].contiguous()
    k0, v0 = cache.k_cache.clone(), cache.v_cache.clone()
    with torch.inference_mode():
        theirs = TransformerBlock._fused_original_forward(block, x, f, mask, ip)
        k_ref, v_ref = cache.k_cache.clone(), cache.v_cache.clone()
        cache.k_cache.copy_(k0)
        cache.v_cache.copy_(v0)
        before = fusedlayer.stats()["fused"]
        ours = block(x, f, mask, ip)
    assert fusedlayer.stats()["fused"] == before + 1
    # the unfused block (fork arithmetic, torch ops) - the reference's bar, 5e-3 of
    # max |y|, plus one output ulp: two separately rounded 16-bit results may sit
    # one ulp apart, and bf16's ulp at the largest outputs is itself ~5e-3 of them
    got, ref = bits_f(ours, dt).astype(np.float64), bits_f(theirs, dt).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 5e-3 * np.abs(ref).max() + ulp16(ref, dt))
    assert relative_error(bits_f(cache.k_cache[:, :, pos], dt), bits_f(k_ref[:, :, pos], dt)) < 1e-2
    assert torch.equal(cache.v_cache[:, :, pos], v_ref[:, :, pos])
    # the oracle composition - bit for bit
    expect, kco, vco = _oracle_block(orc, block, layers, xb, pos, window, dt, bits(f), kcb.copy(), vcb.copy())
    assert np.array_equal(bits(ours), expect), first_mismatch(bits(ours), expect)
    assert np.array_equal(bits(cache.k_cache), kco)
    assert np.array_equal(bits(cache.v_cache), vco)


def bits_f(t, dt):
    return o.to_f32(bits(t), dt)


def test_decode_block_declines_a_prefill():
    from ttspipe_amd import fusedlayer

    block, _ = _block(torch.bfloat16, True)
    x = torch.randn(1, 3, 512, device="cuda", dtype=torch.bfloat16)
    ip = torch.arange(3, device="cuda")
    mask = torch.ones(1, 1, 3, 3, dtype=torch.bool, device="cuda")
    assert fusedlayer.decode_block(block, x, None, mask, ip) is None
