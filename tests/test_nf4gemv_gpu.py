"""The NF4 GEMV / GEMM / dequantisation kernels against the oracle (GPU).

Bar (written per test): dequantised weights and the one-row GEMV bit for bit
against the oracle's emulation of the kernel's fixed order; the GEMV and the
MFMA GEMM within 2e-3 (relative to max |y|, beyond the output type's own
half-ulp rounding) of the fp64 product on the dequantised weights; epilogues
bit for bit. Shapes are the reference's (tests/test_nf4gemv.py:119-186) plus
the Dual-AR fast transformer's.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.conftest import beyond_rounding_error, relative_error
from tests.gpuutil import bits, dt_code, first_mismatch, from_bits, gemv_rows_shape, gemv_shape, randn_bits
from tests.nf4data import dequant_numpy, oracle_args, random_layer, to_linear

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


@pytest.fixture(scope="module")
def nf4():
    from ttspipe_amd import nf4gemv

    assert nf4gemv.install(), "nf4 kernels unavailable on a GPU machine"
    return nf4gemv


# ------------------------------------------------------------ numerics primitives

def test_fp16_fma_chain_is_ieee(selftest, orc):
    """The GEMV's inner step, fma(a.hi, b.hi, fma(a.lo, b.lo, c)) on fp16 halves
    (v_fma_mix_f32), equals IEEE fmaf bit for bit - over random, tiny, huge and
    exactly cancelling operands."""
    from ttspipe_amd import _lib

    rng = np.random.default_rng(0)
    n = 1 << 16
    va = (rng.standard_normal(2 * n) * 10.0 ** rng.integers(-7, 4, 2 * n)).astype(np.float32)
    vb = (rng.standard_normal(2 * n) * 10.0 ** rng.integers(-3, 4, 2 * n)).astype(np.float32)
    a = o.from_f32(va, o.DT_F16).view(np.uint32).copy()
    b = o.from_f32(vb, o.DT_F16).view(np.uint32).copy()
    c = (rng.standard_normal(n) * 10.0 ** rng.integers(-4, 4, n)).astype(np.float32)
    af = o.to_f32(a.view(np.uint16), o.DT_F16).reshape(-1, 2)
    bf = o.to_f32(b.view(np.uint16), o.DT_F16).reshape(-1, 2)
    c[:1000] = -(af[:1000, 0] * bf[:1000, 0])  # exact cancellation in the first fma
    at = torch.from_numpy(a.view(np.int32)).cuda()
    bt = torch.from_numpy(b.view(np.int32)).cuda()
    ct = torch.from_numpy(c).cuda()
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    assert selftest.ttsp_selftest_fma16(at.data_ptr(), bt.data_ptr(), ct.data_ptr(), n, out.data_ptr(), _lib.stream()) == 0
    got = out.cpu().numpy()
    expect = o.fma16_chain(a, b, c)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), first_mismatch(got, expect)


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_device_math_matches_the_oracle_bit_for_bit(selftest, orc, op):
    from ttspipe_amd import _lib

    rng = np.random.default_rng(op)
    if op == 0:
        x = np.concatenate([np.linspace(-90, 90, 40001), rng.uniform(-87, 0, 20000)]).astype(np.float32)
    elif op in (1, 2):
        x = np.concatenate([10.0 ** rng.uniform(-6, 6, 40000), rng.uniform(1e-6, 4, 20000)]).astype(np.float32)
    else:
        x = rng.uniform(-30, 30, 40000).astype(np.float32)
    xt = torch.from_numpy(x).cuda()
    out = torch.empty_like(xt)
    assert selftest.ttsp_selftest_math(xt.data_ptr(), x.size, op, out.data_ptr(), _lib.stream()) == 0
    got = out.cpu().numpy()
    if op == 0:
        expect = orc.exp_cw(x)
    elif op == 1:
        expect = np.sqrt(x)  # numpy's float32 sqrt is correctly rounded
    elif op == 2:
        expect = (np.float32(1.0) / np.sqrt(x)).astype(np.float32)
    else:
        e = orc.exp_cw(-x)
        expect = (x / (np.float32(1.0) + e)).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), expect.view(np.uint32)), first_mismatch(got, expect)


# ------------------------------------------------------------------ dequant

@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("out_dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("shape", [(9728, 2560), (13, 64 * 3), (1, 64)])
def test_dequant_is_bit_exact(nested, out_dtype, shape):
    from ttspipe_amd.quant import dequantize_4bit

    layer = random_layer(*shape, nested, seed=shape[0])
    lin = to_linear(layer, torch.bfloat16)
    got = dequantize_4bit(lin.weight.data, lin.weight.quant_state, out_dtype=out_dtype)
    expect = dequant_numpy(layer, dt_code(out_dtype))
    assert np.array_equal(bits(got), expect), first_mismatch(bits(got), expect)


# ------------------------------------------------------------------ GEMV

GEMV_SHAPES = [
    (6144, 2560),  # wqkv
    (2560, 4096),  # wo
    (9728, 2560),  # w1 / w3
    (2560, 9728),  # w2
    (1544, 2560),  # rows that do not divide into tiles
    (4096, 2560),  # q
    (1024, 2560),  # k / v
    (1536, 1024),  # fast wqkv
    (3072, 1024),  # fast w1 / w3
    (1024, 3072),  # fast w2
    (4096, 1024),  # fast head
    (1024, 2560),  # fast_project_in
    (64, 128),     # smallest
]


@pytest.mark.parametrize("shape", GEMV_SHAPES)
@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
def test_gemv_bit_exact_and_within_bar(nf4, orc, shape, nested, dtype):
    M, K = shape
    layer = random_layer(M, K, nested, seed=M * 7 + K)
    lin = to_linear(layer, dtype)
    xb = randn_bits(K, dtype, seed=K)
    x = from_bits(xb, dtype).view(1, 1, K)
    before = nf4.stats()["fast"]
    y = lin(x)
    assert nf4.stats()["fast"] == before + 1
    assert y.shape == (1, 1, M) and y.dtype == dtype
    J, KS, _ = gemv_shape(M, K)
    dt = dt_code(dtype)
    expect = orc.gemv_emul(xb, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, bs2=layer["bs2"] or 256)
    got = bits(y)
    assert np.array_equal(got, expect), f"M={M} K={K} KS={KS} J={J}: {first_mismatch(got, expect)}"
    ref = orc.nf4_gemm_ref(xb, dt, **oracle_args(layer), M=M, K=K, N=1, bs=64, bs2=layer["bs2"] or 256)
    assert beyond_rounding_error(o.to_f32(got, dt), ref.reshape(-1), dt) < 2e-3


@pytest.mark.parametrize("shape", GEMV_SHAPES)
@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
def test_two_rows_through_the_gemv(nf4, orc, shape, nested, dtype):
    """Two activation rows take the GEMV (one code lookup per weight byte, one
    fp32 chain per row) with the one-row launch's K split: row n equals the
    oracle's one-row emulation of x[n] bit for bit (so two rows give exactly
    what two one-row calls give), and each is within the bar. Three rows take
    the MFMA kernels."""
    M, K = shape
    rows = 2
    sh = gemv_rows_shape(M, K, rows)
    assert sh is not None, f"{rows} rows of {M}x{K} should take the GEMV"
    assert sh == gemv_shape(M, K), "two rows keep the one-row launch shape"
    assert gemv_rows_shape(M, K, 3) is None
    J, KS, _ = sh
    layer = random_layer(M, K, nested, seed=M * 3 + K + rows)
    lin = to_linear(layer, dtype)
    dt = dt_code(dtype)
    xb = randn_bits(rows * K, dtype, seed=K + rows)
    before = nf4.stats()["fast"]
    y = lin(from_bits(xb, dtype).view(1, rows, K))
    assert nf4.stats()["fast"] == before + 1 and y.shape == (1, rows, M)
    got = bits(y).reshape(rows, M)
    bs2 = layer["bs2"] or 256
    for n in range(rows):
        expect = orc.gemv_emul(xb[n * K:(n + 1) * K], dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, bs2=bs2)
        assert np.array_equal(got[n], expect), f"row {n} of {rows}, {M}x{K}: {first_mismatch(got[n], expect)}"
    ref = orc.nf4_gemm_ref(xb, dt, **oracle_args(layer), M=M, K=K, N=rows, bs=64, bs2=bs2)
    assert beyond_rounding_error(o.to_f32(got, dt).reshape(-1), ref.reshape(-1), dt) < 2e-3


@pytest.mark.parametrize("rows", [2])
@pytest.mark.parametrize("epi", [1, 2])
def test_rows_through_the_gemv_with_epilogues(nf4, orc, rows, epi):
    """The residual and gate epilogues of the two-row form read each row's own
    operand row."""
    M, K, dtype = 2560, 9728, torch.bfloat16
    dt = dt_code(dtype)
    J, KS, _ = gemv_rows_shape(M, K, rows)
    layer = random_layer(M, K, True, seed=rows * 10 + epi)
    lin = to_linear(layer, dtype)
    assert nf4.prepare(lin)
    xb = randn_bits(rows * K, dtype, seed=rows + 40, scale=0.5)
    rb = randn_bits(rows * M, dtype, seed=rows + 50)
    y = nf4.matmul(lin, from_bits(xb, dtype).view(rows, K), epi=epi, operand=from_bits(rb, dtype).view(rows, M))
    got = bits(y).reshape(rows, M)
    for n in range(rows):
        expect = orc.gemv_emul(xb[n * K:(n + 1) * K], dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J,
                               R=rb[n * M:(n + 1) * M], epi=epi)
        assert np.array_equal(got[n], expect), f"row {n}: {first_mismatch(got[n], expect)}"


@pytest.mark.parametrize("shape", [(4961, 384), (16000, 256), (4100, 128), (9000, 512)])
@pytest.mark.parametrize("pair", [False, True])
def test_one_chunk_rows_with_three_or_more_rows_a_wave(nf4, orc, shape, pair):
    """K <= 512 (one 64-dword chunk per lane) with more than 4096 rows (3 to 8
    rows a wave): the code lookups run ahead of the arithmetic, and must not
    reach a weight row before its load is issued. They once did, and every
    wave's third row came out wrong. Plain one-weight form and the SwiGLU
    pair, against the oracle bit for bit."""
    M, K = shape
    dtype = torch.bfloat16
    dt = dt_code(dtype)
    J, KS, RPW = gemv_shape(M, K)
    assert J == 1 and RPW >= 3
    l1 = random_layer(M, K, False, seed=M + K)
    w1 = to_linear(l1, dtype)
    assert nf4.prepare(w1)
    xb = randn_bits(K, dtype, seed=K + 3)
    x = from_bits(xb, dtype).view(1, 1, K)
    g1 = orc.gemv_emul(xb, dt, **oracle_args(l1), M=M, K=K, bs=64, KS=KS, J=J)
    if pair:
        l3 = random_layer(M, K, False, seed=M + K + 1)
        w3 = to_linear(l3, dtype)
        assert nf4.prepare(w3)
        y = nf4.matmul_fused(w1, x, module3=w3)
        expect = orc.gemv_emul(xb, dt, **oracle_args(l3), M=M, K=K, bs=64, KS=KS, J=J, R=g1, epi=2)
    else:
        y = nf4.matmul(w1, x)
        expect = g1
    assert np.array_equal(bits(y), expect), f"M={M} K={K} RPW={RPW}: {first_mismatch(bits(y), expect)}"


@pytest.mark.parametrize("epi", [1, 2])
@pytest.mark.parametrize("dtype", DTYPES)
def test_gemv_epilogues_bit_exact(nf4, orc, epi, dtype):
    M, K = 2560, 9728
    layer = random_layer(M, K, True, seed=11)
    lin = to_linear(layer, dtype)
    xb = randn_bits(K, dtype, seed=12, scale=0.5)
    rb = randn_bits(M, dtype, seed=13)
    assert nf4.prepare(lin)
    y = nf4.matmul(lin, from_bits(xb, dtype).view(1, 1, K), epi=epi, operand=from_bits(rb, dtype).view(1, 1, M))
    J, KS, _ = gemv_shape(M, K)
    expect = orc.gemv_emul(xb, dt_code(dtype), **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, R=rb, epi=epi)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)


@pytest.mark.parametrize("shape", [(1, 1, 2560), (1, 2560), (2560,)])
def test_every_single_vector_shape_is_served(nf4, shape):
    layer = random_layer(512, 2560, True, seed=3)
    lin = to_linear(layer, torch.float16)
    x = torch.randn(*shape, device="cuda", dtype=torch.float16)
    before = nf4.stats()["fast"]
    y = lin(x)
    assert nf4.stats()["fast"] == before + 1
    assert y.shape == (*shape[:-1], 512)


def test_gemv_is_deterministic(nf4):
    layer = random_layer(9728, 2560, True, seed=21)
    lin = to_linear(layer, torch.bfloat16)
    x = torch.randn(1, 1, 2560, device="cuda", dtype=torch.bfloat16)
    first = lin(x).clone()
    for _ in range(5):
        assert torch.equal(lin(x), first)


def test_unsupported_layer_is_declined_not_broken(nf4):
    """A blocksize that is not a power of two goes to the layer's own forward."""
    layer = random_layer(256, 2560, True, seed=4)
    lin = to_linear(layer, torch.float16)
    lin.weight.quant_state.blocksize = 96
    x = torch.randn(1, 1, 2560, device="cuda", dtype=torch.float16)
    assert not nf4.prepare(lin)
    before = nf4.stats()["fallback"]
    with pytest.raises(Exception):
        lin(x)  # the layer's own dequantisation refuses blocksize 96 too
    assert nf4.stats()["fallback"] == before + 1


def test_fp32_activations_are_declined(nf4):
    layer = random_layer(256, 2560, True, seed=5)
    lin = to_linear(layer, torch.float16)
    assert nf4.prepare(lin)
    assert nf4.matmul(lin, torch.randn(1, 2560, device="cuda")) is None


# ------------------------------------------------------------------ GEMM (N > 1)

@pytest.mark.parametrize("rows", [2, 5, 8, 9, 16, 17, 19, 32, 33, 48, 64, 65, 70])
@pytest.mark.parametrize("shape", [(6144, 2560), (2560, 9728), (1544, 2560)])
@pytest.mark.parametrize("dtype", DTYPES)
def test_several_positions_within_bar(nf4, orc, shape, rows, dtype):
    M, K = shape
    layer = random_layer(M, K, True, seed=M + rows)
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=rows, scale=0.5)
    before = nf4.stats()["fast"]
    y = lin(from_bits(xb, dtype).view(1, rows, K))
    assert nf4.stats()["fast"] == before + 1
    dt = dt_code(dtype)
    ref = orc.nf4_gemm_ref(xb, dt, **oracle_args(layer), M=M, K=K, N=rows, bs=64, bs2=256)
    assert beyond_rounding_error(o.to_f32(bits(y), dt), ref.reshape(-1), dt) < 2e-3


@pytest.mark.parametrize("rows", [3, 16, 17, 40])
def test_few_rows_over_a_long_row(nf4, orc, rows):
    """K = 16384: up to 16 rows the few-row kernel splits K over 16 waves; more
    rows than its limit for that K go to the tiled GEMM. Both within the bar."""
    M, K, dtype = 272, 16384, torch.bfloat16
    layer = random_layer(M, K, True, seed=rows + 7)
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=rows + 8, scale=0.5)
    y = lin(from_bits(xb, dtype).view(rows, K))
    ref = orc.nf4_gemm_ref(xb, o.DT_BF16, **oracle_args(layer), M=M, K=K, N=rows, bs=64, bs2=256)
    assert beyond_rounding_error(o.to_f32(bits(y), o.DT_BF16), ref.reshape(-1), o.DT_BF16) < 2e-3


@pytest.mark.parametrize("K", [12416, 16384, 32768])
@pytest.mark.parametrize("nested", [True, False])
def test_one_row_over_a_long_row(nf4, orc, K, nested):
    """One activation row past 12288 codes (the reference serves any K with
    K % 128 == 0, nf4gemv.py:346-347): the GEMV stages the rest of x after
    requesting its weight rows, bit for bit against the oracle - the plain
    form, the residual epilogue and the SwiGLU pair."""
    M, dtype = 200, torch.bfloat16
    dt = dt_code(dtype)
    assert nf4.gemv_fits(M, K)
    J, KS, _ = gemv_shape(M, K)
    l1 = random_layer(M, K, nested, seed=K + nested)
    l3 = random_layer(M, K, nested, seed=K + nested + 2)
    w1, w3 = to_linear(l1, dtype), to_linear(l3, dtype)
    assert nf4.prepare(w1) and nf4.prepare(w3)
    xb = randn_bits(K, dtype, seed=K + 5, scale=0.5)
    rb = randn_bits(M, dtype, seed=K + 6)
    x = from_bits(xb, dtype).view(1, 1, K)
    kw = dict(M=M, K=K, bs=64, KS=KS, J=J, bs2=l1["bs2"] or 256)
    g1 = orc.gemv_emul(xb, dt, **oracle_args(l1), **kw)
    y = nf4.matmul(w1, x)
    assert np.array_equal(bits(y), g1), f"K={K} KS={KS} J={J}: {first_mismatch(bits(y), g1)}"
    ref = orc.nf4_gemm_ref(xb, dt, **oracle_args(l1), M=M, K=K, N=1, bs=64, bs2=l1["bs2"] or 256)
    assert beyond_rounding_error(o.to_f32(bits(y), dt), ref.reshape(-1), dt) < 2e-3
    y = nf4.matmul(w1, x, epi=nf4.EPI_RESIDUAL, operand=from_bits(rb, dtype).view(1, 1, M))
    expect = orc.gemv_emul(xb, dt, **oracle_args(l1), **kw, R=rb, epi=1)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)
    y = nf4.matmul_fused(w1, x, module3=w3)
    expect = orc.gemv_emul(xb, dt, **oracle_args(l3), **kw, R=g1, epi=2)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)


@pytest.mark.parametrize("nested", [True, False])
def test_one_row_longer_than_the_gemv_holds(nf4, orc, nested):
    """K = 65536 (beyond the GEMV's 32768): `matmul` serves the row through the
    tiled kernel within the bar; the fused single-row forms decline (None),
    never raise."""
    M, K, dtype = 96, 65536, torch.bfloat16
    assert not nf4.gemv_fits(M, K)
    layer = random_layer(M, K, nested, seed=31 + nested)
    lin = to_linear(layer, dtype)
    assert nf4.prepare(lin)
    xb = randn_bits(K, dtype, seed=33, scale=0.5)
    x = from_bits(xb, dtype).view(1, 1, K)
    before = nf4.stats()["fast"]
    y = lin(x)
    assert nf4.stats()["fast"] == before + 1 and y.shape == (1, 1, M)
    ref = orc.nf4_gemm_ref(xb, o.DT_BF16, **oracle_args(layer), M=M, K=K, N=1, bs=64, bs2=layer["bs2"] or 256)
    assert beyond_rounding_error(o.to_f32(bits(y), o.DT_BF16), ref.reshape(-1), o.DT_BF16) < 2e-3
    assert nf4.matmul_fused(lin, x) is None
    assert nf4.matmul_fused(lin, x, module3=lin) is None


@pytest.mark.parametrize("rows", [128, 256, 512])
@pytest.mark.parametrize("name,shape", [("q", (4096, 2560)), ("k", (1024, 2560)), ("o", (2560, 4096)),
                                        ("gate", (9728, 2560)), ("down", (2560, 9728)), ("qkv", (6144, 2560)),
                                        ("narrow", (1024, 4096))])
def test_prefill_gemm_bucket_rows(nf4, orc, name, shape, rows):
    """The prefill workload: 128, 256 and 512 bf16 rows (prompt buckets)
    through each projection shape; between them the launch plan takes every
    K split it has (none, 2, 4 and 8 ways: 8 for the narrow shape at 128)."""
    M, K = shape
    dtype = torch.bfloat16
    layer = random_layer(M, K, True, seed=len(name))
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=99)
    y = lin(from_bits(xb, dtype).view(rows, K))
    dt = dt_code(dtype)
    sample = np.arange(0, rows, 37)  # a sample of rows keeps the fp64 reference quick
    ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], dt, **oracle_args(layer), M=M, K=K, N=sample.size, bs=64)
    got = o.to_f32(bits(y), dt).reshape(rows, M)[sample]
    assert beyond_rounding_error(got, ref, dt) < 2e-3


@pytest.mark.parametrize("epi", [1, 2])
@pytest.mark.parametrize("rows,shape", [(24, (2560, 9728)), (512, (2560, 9728)), (512, (9728, 2560))])
def test_gemm_epilogues(nf4, orc, epi, rows, shape):
    """Residual and SwiGLU-gate epilogues of the GEMM (24 rows: unsplit; 512
    rows at 2560 x 9728: the K-split plan, where the reduce kernel applies
    them; 512 rows at 9728 x 2560: the unsplit direct-to-LDS kernel, which
    applies them itself) against the closed forms round(R + round(y)) and
    round(round(silu(R)) * round(y)) evaluated on the oracle's fp64 product,
    within the 2e-3 bar beyond the output's own rounding. An epilogue with its
    operands swapped misses that bar by an order of magnitude."""
    from ttspipe_amd import _lib

    (M, K), dtype = shape, torch.float16
    if rows == 512:
        assert _lib.load().ttsp_nf4_gemm_splits(M, K, rows) == (4 if M == 2560 else 1)
    layer = random_layer(M, K, True, seed=31)
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=32, scale=0.5)
    rb = randn_bits(rows * M, dtype, seed=33)
    assert nf4.prepare(lin)
    y = nf4.matmul(lin, from_bits(xb, dtype).view(rows, K), epi=epi, operand=from_bits(rb, dtype).view(rows, M))
    sample = np.arange(0, rows, 7)
    ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], o.DT_F16, **oracle_args(layer), M=M, K=K,
                           N=sample.size, bs=64, bs2=256).astype(np.float64)
    yr = o.to_f32(o.from_f32(ref.astype(np.float32), o.DT_F16), o.DT_F16).astype(np.float64)
    r = o.to_f32(rb, o.DT_F16).astype(np.float64).reshape(rows, M)[sample]
    silu = o.to_f32(o.from_f32((r / (1 + np.exp(-r))).astype(np.float32), o.DT_F16), o.DT_F16).astype(np.float64)
    expect = r + yr if epi == 1 else silu * yr
    got = o.to_f32(bits(y), o.DT_F16).reshape(rows, M)[sample]
    assert beyond_rounding_error(got, expect, o.DT_F16) < 2e-3
    if epi == 2:
        swapped = (yr / (1 + np.exp(-yr))) * r
        assert beyond_rounding_error(got, swapped, o.DT_F16) > 2e-2


@pytest.mark.parametrize("rows", [512, 300])
def test_split_gemm_with_rows_not_a_multiple_of_four(nf4, orc, rows):
    """1540 output features (M % 4 == 2) at K = 2560: 512 rows take a K split,
    whose fp32 partial sums are then stored without 16-byte vectors."""
    from ttspipe_amd import _lib

    M, K, dtype = 1540, 2560, torch.bfloat16
    splits = _lib.load().ttsp_nf4_gemm_splits(M, K, rows)
    assert splits > 1
    layer = random_layer(M, K, True, seed=1540)
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=41)
    y = lin(from_bits(xb, dtype).view(rows, K))
    sample = np.arange(0, rows, 13)
    ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], o.DT_BF16, **oracle_args(layer), M=M, K=K,
                           N=sample.size, bs=64, bs2=256)
    got = o.to_f32(bits(y), o.DT_BF16).reshape(rows, M)[sample]
    assert beyond_rounding_error(got, ref, o.DT_BF16) < 2e-3


@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape,rows,splits", [((9728, 2560), 512, 1), ((6144, 2560), 512, 2),
                                               ((2560, 4096), 256, 4), ((9730, 2560), 500, 1),
                                               ((9730, 2560), 300, 2)])
def test_direct_lds_gemm_launches(nf4, orc, shape, rows, splits, nested, dtype):
    """Every launch the plan gives the direct-to-LDS kernel (unsplit, 2 and 4
    K-splits) with bf16 and fp16 activations and nested and plain scales,
    including ragged tiles (9730 weight rows: M % 4 == 2, a partial 64-row
    tile; 500 and 300 activation rows: a partial 128-row tile), against the
    oracle's fp64 product within the bar."""
    from ttspipe_amd import _lib

    M, K = shape
    assert _lib.load().ttsp_nf4_gemm_splits(M, K, rows) == splits
    layer = random_layer(M, K, nested, seed=M + rows)
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=rows + 3)
    y = lin(from_bits(xb, dtype).view(rows, K))
    dt = dt_code(dtype)
    sample = np.concatenate([np.arange(0, rows, 41), [rows - 1]])  # the last row sits in the partial tile
    ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], dt, **oracle_args(layer), M=M, K=K, N=sample.size, bs=64)
    got = o.to_f32(bits(y), dt).reshape(rows, M)[sample]
    assert beyond_rounding_error(got, ref, dt) < 2e-3


@pytest.mark.parametrize("shape,rows,bs2", [((9728, 2560), 512, 16), ((2560, 4096), 256, 16),
                                            ((6144, 2560), 512, 32)])
def test_direct_lds_gemm_small_second_level_groups(nf4, orc, shape, rows, bs2):
    """Nested scales with second-level groups of 16 or 32 blocks (1,024 or
    2,048 codes) at launches the plan gives the direct-to-LDS kernel: where a
    workgroup's K range (2,560 codes unsplit) could cross two group
    boundaries the launch falls back to the 64 x 128 kernel; where it spans
    at most one (1,024 codes a split for 16-block groups, 1,280 for 32) the
    kernel switches the group's absmax mid-range. Against the oracle."""
    M, K = shape
    dtype = torch.bfloat16
    layer = random_layer(M, K, True, seed=M + bs2, bs2=bs2)
    lin = to_linear(layer, dtype)
    xb = randn_bits(rows * K, dtype, seed=rows + bs2)
    y = lin(from_bits(xb, dtype).view(rows, K))
    dt = dt_code(dtype)
    sample = np.concatenate([np.arange(0, rows, 37), [rows - 1]])
    ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], dt, **oracle_args(layer), M=M, K=K, N=sample.size, bs=64,
                           bs2=bs2)
    got = o.to_f32(bits(y), dt).reshape(rows, M)[sample]
    assert beyond_rounding_error(got, ref, dt) < 2e-3


# ------------------------------------------------------------ fused forms (one launch)

FUSED_SHAPES = [(6144, 2560), (9728, 2560), (2560, 9728), (1536, 1024), (3072, 1024), (1544, 2560), (64, 128)]


@pytest.mark.parametrize("shape", FUSED_SHAPES)
@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_folded_into_the_matmul_is_bit_exact(nf4, orc, shape, nested, dtype):
    """rmsnorm(x) . W^T in one launch == the standalone norm then the GEMV, bit for bit."""
    M, K = shape
    layer = random_layer(M, K, nested, seed=M + 3 * K)
    lin = to_linear(layer, dtype)
    assert nf4.prepare(lin)
    dt = dt_code(dtype)
    xb = randn_bits(K, dtype, seed=K + 1, scale=3.0)
    gb = o.from_f32((np.random.default_rng(K).random(K) * 0.5 + 0.75).astype(np.float32), dt)
    y = nf4.matmul_fused(lin, from_bits(xb, dtype).view(1, 1, K), norm_weight=from_bits(gb, dtype), eps=1e-6)
    J, KS, _ = gemv_shape(M, K)
    if K > nf4.NORM_MAX_K:  # too wide to fold the norm in: the caller runs it separately
        assert y is None
        return
    xn = orc.rms_norm_emul(xb, gb, 1, K, 1e-6, dt)
    expect = orc.gemv_emul(xn, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, bs2=layer["bs2"] or 256)
    assert np.array_equal(bits(y), expect), f"M={M} K={K}: {first_mismatch(bits(y), expect)}"


@pytest.mark.parametrize("shape", FUSED_SHAPES)
@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("epi", [0, 1, 2])
@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_folded_into_two_rows_is_bit_exact(nf4, orc, shape, nested, epi, dtype):
    """Two rows through `matmul_fused` with the norm folded in (one launch,
    each weight byte looked up once for both rows): each row bit for bit the
    oracle's norm then GEMV (and its epilogue), and the two one-row launches."""
    M, K = shape
    if K > nf4.NORM_MAX_K:
        return
    layer = random_layer(M, K, nested, seed=M + 5 * K + epi)
    lin = to_linear(layer, dtype)
    assert nf4.prepare(lin)
    dt = dt_code(dtype)
    xb = [randn_bits(K, dtype, seed=K + 11 + r, scale=2.0 + r) for r in range(2)]
    rb = [randn_bits(M, dtype, seed=M + 21 + r) for r in range(2)]
    gb = o.from_f32((np.random.default_rng(K + 3).random(K) * 0.5 + 0.75).astype(np.float32), dt)
    g = from_bits(gb, dtype)
    x2 = from_bits(np.concatenate(xb), dtype).view(1, 2, K)
    r2 = from_bits(np.concatenate(rb), dtype).view(1, 2, M) if epi else None
    y = nf4.matmul_fused(lin, x2, norm_weight=g, eps=1e-6, epi=epi, operand=r2)
    assert y is not None and y.shape == (1, 2, M)
    J, KS, _ = gemv_shape(M, K)
    for r in range(2):
        xn = orc.rms_norm_emul(xb[r], gb, 1, K, 1e-6, dt)
        kw = dict(R=rb[r], epi=epi) if epi else {}
        expect = orc.gemv_emul(xn, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, bs2=layer["bs2"] or 256,
                               **kw)
        assert np.array_equal(bits(y[0, r]), expect), f"row {r} M={M} K={K}: {first_mismatch(bits(y[0, r]), expect)}"
        one = nf4.matmul_fused(lin, x2[:, r : r + 1].contiguous(), norm_weight=g, eps=1e-6, epi=epi,
                               operand=None if r2 is None else r2[:, r : r + 1].contiguous())
        assert np.array_equal(bits(one), bits(y[0, r]))


@pytest.mark.parametrize("shape", [(9728, 2560), (3072, 1024), (1000, 2560), (64, 128)])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
def test_swiglu_pair_in_one_launch_is_bit_exact(nf4, orc, shape, norm, dtype):
    """silu(x W1) * (x W3) from one launch == w1, then w3 with the gate epilogue."""
    M, K = shape
    l1, l3 = random_layer(M, K, True, seed=M + 1), random_layer(M, K, True, seed=M + 2)
    w1, w3 = to_linear(l1, dtype), to_linear(l3, dtype)
    assert nf4.prepare(w1) and nf4.prepare(w3)
    dt = dt_code(dtype)
    xb = randn_bits(K, dtype, seed=K + 5)
    gb = o.from_f32((np.random.default_rng(K + 1).random(K) + 0.5).astype(np.float32), dt)
    y = nf4.matmul_fused(w1, from_bits(xb, dtype).view(1, 1, K), norm_weight=from_bits(gb, dtype) if norm else None,
                         eps=1e-6, module3=w3)
    J, KS, _ = gemv_shape(M, K)
    xin = orc.rms_norm_emul(xb, gb, 1, K, 1e-6, dt) if norm else xb
    g1 = orc.gemv_emul(xin, dt, **oracle_args(l1), M=M, K=K, bs=64, KS=KS, J=J)
    expect = orc.gemv_emul(xin, dt, **oracle_args(l3), M=M, K=K, bs=64, KS=KS, J=J, R=g1, epi=2)
    assert np.array_equal(bits(y), expect), f"M={M} K={K}: {first_mismatch(bits(y), expect)}"


@pytest.mark.parametrize("shape", [(9728, 2560), (3072, 1024), (1000, 2560), (64, 128)])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("nested", [True, False])
@pytest.mark.parametrize("dtype", DTYPES)
def test_swiglu_pair_over_two_rows_is_bit_exact(nf4, orc, shape, norm, nested, dtype):
    """The SwiGLU pair over two rows in one launch (norm folded or not): each
    row bit for bit the oracle's w1, then w3 with the gate epilogue, and the
    one-row launch of that row."""
    M, K = shape
    l1, l3 = random_layer(M, K, nested, seed=M + 11), random_layer(M, K, nested, seed=M + 12)
    w1, w3 = to_linear(l1, dtype), to_linear(l3, dtype)
    assert nf4.prepare(w1) and nf4.prepare(w3)
    dt = dt_code(dtype)
    xb = [randn_bits(K, dtype, seed=K + 31 + r) for r in range(2)]
    gb = o.from_f32((np.random.default_rng(K + 7).random(K) + 0.5).astype(np.float32), dt)
    g = from_bits(gb, dtype) if norm else None
    x2 = from_bits(np.concatenate(xb), dtype).view(1, 2, K)
    y = nf4.matmul_fused(w1, x2, norm_weight=g, eps=1e-6, module3=w3)
    assert y is not None and y.shape == (1, 2, M)
    J, KS, _ = gemv_shape(M, K)
    for r in range(2):
        xin = orc.rms_norm_emul(xb[r], gb, 1, K, 1e-6, dt) if norm else xb[r]
        g1 = orc.gemv_emul(xin, dt, **oracle_args(l1), M=M, K=K, bs=64, KS=KS, J=J, bs2=l1["bs2"] or 256)
        expect = orc.gemv_emul(xin, dt, **oracle_args(l3), M=M, K=K, bs=64, KS=KS, J=J, bs2=l3["bs2"] or 256, R=g1,
                               epi=2)
        assert np.array_equal(bits(y[0, r]), expect), f"row {r} M={M} K={K}: {first_mismatch(bits(y[0, r]), expect)}"
        one = nf4.matmul_fused(w1, x2[:, r : r + 1].contiguous(), norm_weight=g, eps=1e-6, module3=w3)
        assert np.array_equal(bits(one), bits(y[0, r]))


@pytest.mark.parametrize("dtype", DTYPES)
def test_norm_folded_with_residual_epilogue(nf4, orc, dtype):
    M, K = 2560, 4096
    layer = random_layer(M, K, True, seed=77)
    lin = to_linear(layer, dtype)
    assert nf4.prepare(lin)
    dt = dt_code(dtype)
    xb, rb = randn_bits(K, dtype, seed=78), randn_bits(M, dtype, seed=79)
    gb = o.from_f32(np.full(K, 1.25, np.float32), dt)
    y = nf4.matmul_fused(lin, from_bits(xb, dtype).view(1, K), norm_weight=from_bits(gb, dtype), eps=1e-5,
                         epi=nf4.EPI_RESIDUAL, operand=from_bits(rb, dtype))
    J, KS, _ = gemv_shape(M, K)
    xn = orc.rms_norm_emul(xb, gb, 1, K, 1e-5, dt)
    expect = orc.gemv_emul(xn, dt, **oracle_args(layer), M=M, K=K, bs=64, KS=KS, J=J, R=rb, epi=1)
    assert np.array_equal(bits(y), expect), first_mismatch(bits(y), expect)


def test_fused_form_declines_what_it_cannot_serve(nf4):
    a = to_linear(random_layer(512, 2560, True, seed=1), torch.bfloat16)
    b = to_linear(random_layer(256, 2560, True, seed=2), torch.bfloat16)
    assert nf4.prepare(a) and nf4.prepare(b)
    x = torch.randn(1, 2560, device="cuda", dtype=torch.bfloat16)
    assert nf4.matmul_fused(a, x, module3=b) is None  # shapes differ
    assert nf4.matmul_fused(a, torch.randn(3, 2560, device="cuda", dtype=torch.bfloat16)) is None  # three rows
    two = torch.randn(2, 2560, device="cuda", dtype=torch.bfloat16)
    assert nf4.matmul_fused(a, two, module3=b) is None  # shapes differ, two rows
    assert nf4.matmul_fused(a, x, norm_weight=torch.ones(2560, device="cuda", dtype=torch.float16)) is None


@pytest.mark.parametrize("nested", [True, False])
def test_prequantised_checkpoint_serves_the_same_bits(nf4, nested):
    """A layer saved in bitsandbytes' serialised layout, read back with the safe
    loader and loaded into a fresh Linear4bit on the GPU, computes bit for bit
    what the original does (GEMV and GEMM paths)."""
    import io

    from ttspipe_amd import quant

    M, K, dtype = 1536, 1024, torch.bfloat16
    layer = random_layer(M, K, nested, seed=5)
    src = to_linear(layer, dtype)
    buf = io.BytesIO()
    torch.save({k: v.cpu() for k, v in quant.quant_state_to_dict(src.weight.data, src.weight.quant_state).items()},
               buf)
    buf.seek(0)
    sd = torch.load(buf, weights_only=True)
    dst = quant.Linear4bit(K, M, bias=False, compute_dtype=dtype, compress_statistics=nested, device="cuda")
    quant.load_nf4_state_dict(dst, sd)
    assert dst.weight.device.type == "cuda"
    for rows in (1, 24):
        x = from_bits(randn_bits(rows * K, dtype, seed=rows), dtype).view(rows, K)
        assert torch.equal(src(x).view(torch.int16), dst(x).view(torch.int16))


# ------------------------------------------------------------ the SwiGLU pair as one GEMM launch


@pytest.mark.parametrize("shape,rows,nested,dtype", [((9728, 2560), 512, True, torch.bfloat16),
                                                     ((9728, 2560), 400, True, torch.bfloat16),
                                                     ((9728, 2560), 512, False, torch.float16),
                                                     ((9730, 2560), 500, True, torch.bfloat16),
                                                     ((9730, 2560), 500, False, torch.float16)])
def test_swiglu_gemm_equals_the_two_launches(nf4, shape, rows, nested, dtype):
    """`matmul_swiglu` (one launch: the gate's waves and w3's waves of the
    same rows meet in LDS) against `matmul(w1)` then `matmul(w3, epi=SILU_GATE)`,
    bit for bit, including ragged tiles (9730 rows: M % 4 == 2 and a partial
    64-row tile; 500 activation rows: a partial 128-row tile), plain and nested
    scales, fp16 and bf16."""
    from ttspipe_amd import _lib

    M, K = shape
    lib = _lib.load()
    assert lib.ttsp_nf4_gemm_swiglu_fits(M, K, rows, 64, 256, int(nested)) == 1
    w1 = to_linear(random_layer(M, K, nested, seed=M + rows), dtype)
    w3 = to_linear(random_layer(M, K, nested, seed=M + rows + 1), dtype)
    x = from_bits(randn_bits(rows * K, dtype, seed=rows + 5, scale=2.0), dtype).view(1, rows, K)
    got = nf4.matmul_swiglu(w1, w3, x)
    assert got is not None and got.shape == (1, rows, M)
    g = nf4.matmul(w1, x)
    ref = nf4.matmul(w3, x, epi=nf4.EPI_SILU_GATE, operand=g)
    torch.cuda.synchronize()
    gb, rb = bits(got), bits(ref)
    assert np.array_equal(gb, rb), first_mismatch(gb, rb)
    assert np.abs(o.to_f32(rb, dt_code(dtype))).max() > 0


@pytest.mark.parametrize("shape,rows,nested,dtype", [((9728, 2560), 3, True, torch.bfloat16),
                                                     ((9728, 2560), 4, True, torch.bfloat16),
                                                     ((9728, 2560), 8, False, torch.float16),
                                                     ((9728, 2560), 9, True, torch.bfloat16),
                                                     ((9728, 2560), 16, True, torch.float16),
                                                     ((9728, 2560), 17, True, torch.bfloat16),
                                                     ((9728, 2560), 32, False, torch.bfloat16),
                                                     ((9730, 2560), 5, True, torch.bfloat16),
                                                     ((3072, 1024), 4, True, torch.bfloat16),
                                                     ((1000, 4096), 12, False, torch.float16),
                                                     ((512, 9728), 24, True, torch.bfloat16)])
def test_swiglu_few_rows_equals_the_two_launches(nf4, shape, rows, nested, dtype):
    """3-32 rows: `matmul_swiglu` runs the few-row kernel's pair form (each
    row tile read from w1 and from w3 by one workgroup) with the bits of
    `matmul(w1)` then `matmul(w3, epi=SILU_GATE)`: one and two X tiles, three
    tiles a workgroup (4-8 rows of 9728 x 2560), ragged M, 8-wave K runs,
    plain and nested scales, fp16 and bf16."""
    from ttspipe_amd import _lib

    M, K = shape
    lib = _lib.load()
    assert lib.ttsp_nf4_gemm_swiglu_fits(M, K, rows, 64, 256, int(nested)) == 1
    w1 = to_linear(random_layer(M, K, nested, seed=M + rows), dtype)
    w3 = to_linear(random_layer(M, K, nested, seed=M + rows + 1), dtype)
    x = from_bits(randn_bits(rows * K, dtype, seed=rows + 5, scale=2.0), dtype).view(1, rows, K)
    got = nf4.matmul_swiglu(w1, w3, x)
    assert got is not None and got.shape == (1, rows, M)
    g = nf4.matmul(w1, x)
    ref = nf4.matmul(w3, x, epi=nf4.EPI_SILU_GATE, operand=g)
    torch.cuda.synchronize()
    gb, rb = bits(got), bits(ref)
    assert np.array_equal(gb, rb), first_mismatch(gb, rb)
    assert np.abs(o.to_f32(rb, dt_code(dtype))).max() > 0


@pytest.mark.parametrize("shape,rows,bs2", [((2560, 9728), 512, 256), ((9728, 2560), 256, 256),
                                            ((9728, 2560), 512, 16), ((1536, 1024), 512, 256)])
def test_swiglu_gemm_declines_what_one_launch_does_not_serve(nf4, shape, rows, bs2):
    """Shapes whose GEMMs the plan splits along K, row counts below the
    direct-to-LDS kernel's, second-level groups a workgroup's K range could
    cross twice, and tile counts below its unsplit rule: None (the caller runs
    the two launches)."""
    M, K = shape
    w1 = to_linear(random_layer(M, K, True, seed=3, bs2=bs2), torch.bfloat16)
    w3 = to_linear(random_layer(M, K, True, seed=4, bs2=bs2), torch.bfloat16)
    x = from_bits(randn_bits(rows * K, torch.bfloat16, seed=9), torch.bfloat16).view(rows, K)
    assert nf4.matmul_swiglu(w1, w3, x) is None


@pytest.mark.parametrize("shape,rows,splits,epi,nested,dtype", [
    ((2560, 4096), 512, 4, 1, True, torch.bfloat16),   # wo of a 512-row span
    ((2560, 9728), 512, 4, 1, True, torch.bfloat16),   # w2 of a 512-row span
    ((2560, 9728), 64, 4, 1, False, torch.float16),
    ((1024, 4096), 128, 8, 0, True, torch.float16),
    ((1536, 1024), 300, 2, 2, True, torch.bfloat16),
    ((512, 1024), 64, 2, 1, True, torch.bfloat16),
    ((4096, 4096), 128, 4, 1, True, torch.bfloat16),  # eight waves a row, the largest M served
    ((520, 2048), 128, 4, 1, True, torch.float16),    # a last step of one 8-value chunk
    ((4088, 2048), 64, 4, 0, False, torch.bfloat16)])
def test_split_gemm_with_the_next_norm_equals_the_two_launches(nf4, shape, rows, splits, epi, nested, dtype):
    """`matmul_norm` (the split-K reduce, its epilogue and the RMSNorm of each
    output row in one launch) against `matmul` then `fusedops.rms_norm`, bit
    for bit: 2, 4 and 8 splits, every epilogue, fp16 and bf16, plain and
    nested scales, a row count that is not a multiple of four, rows of one
    to eight 512-column steps (a wave each) and a ragged last step."""
    from ttspipe_amd import _lib, fusedops

    M, K = shape
    assert _lib.load().ttsp_nf4_gemm_splits(M, K, rows) == splits
    assert fusedops.install()
    lin = to_linear(random_layer(M, K, nested, seed=M + K + rows), dtype)
    assert nf4.prepare(lin)
    x = from_bits(randn_bits(rows * K, dtype, seed=rows + 11, scale=0.5), dtype).view(1, rows, K)
    r = from_bits(randn_bits(rows * M, dtype, seed=rows + 12), dtype).view(1, rows, M) if epi else None
    g = torch.rand(M, generator=torch.Generator().manual_seed(M)).add(0.5).to(dtype).cuda()
    eps = 1e-5
    got = nf4.matmul_norm(lin, x, g, eps, epi=epi, operand=r)
    assert got is not None
    y, yn = got
    ref = nf4.matmul(lin, x, epi=epi, operand=r)
    ref_n = fusedops.rms_norm(ref, g, eps)
    assert ref_n is not None
    torch.cuda.synchronize()
    for a, b in ((y, ref), (yn, ref_n)):
        ab, bb = bits(a), bits(b)
        assert np.array_equal(ab, bb), first_mismatch(ab, bb)
    nb = o.to_f32(bits(ref_n), dt_code(dtype)).reshape(rows, M)
    assert np.all(np.isfinite(nb)) and np.abs(nb).max() > 0


@pytest.mark.parametrize("shape,rows", [((1540, 2560), 512), ((4096, 2560), 512), ((6144, 2560), 256),
                                        ((2560, 9728), 16), ((2560, 9728), 1)])
def test_split_gemm_norm_declines_what_it_does_not_serve(nf4, shape, rows):
    """M % 8 != 0, an unsplit plan, M over 4096, the few-row and one-row
    paths: None (the caller runs the GEMM and the norm separately)."""
    M, K = shape
    lin = to_linear(random_layer(M, K, True, seed=5), torch.bfloat16)
    assert nf4.prepare(lin)
    x = from_bits(randn_bits(rows * K, torch.bfloat16, seed=6), torch.bfloat16).view(rows, K)
    g = torch.ones(M, dtype=torch.bfloat16, device="cuda")
    assert nf4.matmul_norm(lin, x, g, 1e-6) is None


def _row_slice(layer, r0, r1):
    """Rows r0 .. r1 - 1 of a nested layer as a layer of their own (r0 and r1
    on second-level group boundaries)."""
    K, bs, bs2 = layer["K"], layer["bs"], layer["bs2"]
    b0, b1 = r0 * K // bs, r1 * K // bs
    assert b0 % bs2 == 0 and b1 % bs2 == 0
    out = dict(layer)
    out.update(M=r1 - r0, W=layer["W"][r0 * K // 2:r1 * K // 2], A8=layer["A8"][b0:b1],
               AMAX=layer["AMAX"][b0 // bs2:b1 // bs2])
    return out


@pytest.mark.parametrize("rows", [3, 4, 8])
@pytest.mark.parametrize("dtype", DTYPES)
def test_three_tile_workgroups_equal_the_one_tile_launch(nf4, rows, dtype):
    """9728 x 2560 at up to 8 rows runs three row tiles a workgroup; each
    output row is the same fixed function of its weight row as in a
    one-tile-a-workgroup launch (1024-row slices of the same bytes), bit for
    bit, across the slice boundaries."""
    M, K = 9728, 2560
    layer = random_layer(M, K, True, seed=rows)
    full = to_linear(layer, dtype)
    assert nf4.prepare(full)
    x = from_bits(randn_bits(rows * K, dtype, seed=rows + 40), dtype).view(rows, K)
    y = nf4.matmul(full, x)
    assert y is not None
    for r0 in (0, 4096, 8704):
        part = to_linear(_row_slice(layer, r0, r0 + 1024), dtype)
        assert nf4.prepare(part)
        ys = nf4.matmul(part, x)
        torch.cuda.synchronize()
        a, b = bits(y[:, r0:r0 + 1024].contiguous()), bits(ys)
        assert np.array_equal(a, b), (r0, first_mismatch(a, b))
