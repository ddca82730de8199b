"""Seeded random layer shapes through the NF4 matmuls (GPU).

The fixed-shape tests cover the model's own matrices. These sweep what the
launch plans must also get right for any caller of `nf4gemv.matmul`: row
counts that leave the last workgroup partly empty, K from one 128-code step
to 96 of them (every chunk count J and K split KS the GEMV plan picks, and
K-step counts that no GEMM split divides), scale blocks of 64, 128 and 256
codes, plain and nested scales, both activation types.

Bars as the fixed-shape tests: the one-row GEMV bit for bit against the
oracle's emulation of its order (and within 2e-3 of fp64); several rows
within 2e-3 of the fp64 product on bitsandbytes' dequantised weights
(beyond the output type's own half-ulp).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.conftest import beyond_rounding_error
from tests.gpuutil import bits, dt_code, first_mismatch, from_bits, gemv_shape, randn_bits
from tests.nf4data import oracle_args, random_layer, to_linear

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _shapes(n: int, seed: int, max_rows: int):
    """(M, K, bs, nested, dtype, rows) drawn from a seeded generator."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        K = 128 * int(rng.integers(1, 97))
        M = int(rng.integers(1, 6001))
        bs = int(rng.choice([64, 128, 256]))
        if K % bs:
            bs = 128
        out.append((M, K, bs, bool(rng.integers(0, 2)), DTYPES[int(rng.integers(0, 2))],
                    int(rng.integers(2, max_rows + 1))))
    return out


@pytest.fixture(scope="module")
def nf4():
    from ttspipe_amd import nf4gemv

    assert nf4gemv.install(), "nf4 kernels unavailable on a GPU machine"
    return nf4gemv


@pytest.mark.parametrize("case", range(8))
def test_gemv_random_shapes_bit_exact(nf4, orc, case):
    """Ten shapes per case; every one must take the kernel and match the
    oracle's emulation of the plan it got."""
    seen = set()
    for i, (M, K, bs, nested, dtype, _) in enumerate(_shapes(12, 1000 + case, 2)):
        layer = random_layer(M, K, nested, seed=case * 100 + i, bs=bs)
        lin = to_linear(layer, dtype)
        xb = randn_bits(K, dtype, seed=K + i)
        before = nf4.stats()["fast"]
        y = lin(from_bits(xb, dtype).view(1, 1, K))
        assert nf4.stats()["fast"] == before + 1, f"M={M} K={K} bs={bs} was declined"
        J, KS, RPW = gemv_shape(M, K)
        seen.add((J, KS))
        dt = dt_code(dtype)
        bs2 = layer["bs2"] or 256
        expect = orc.gemv_emul(xb, dt, **oracle_args(layer), M=M, K=K, bs=bs, KS=KS, J=J, bs2=bs2)
        got = bits(y)
        where = f"M={M} K={K} bs={bs} nested={nested} {dtype} J={J} KS={KS} RPW={RPW}"
        assert np.array_equal(got, expect), f"{where}: {first_mismatch(got, expect)}"
        ref = orc.nf4_gemm_ref(xb, dt, **oracle_args(layer), M=M, K=K, N=1, bs=bs, bs2=bs2)
        assert beyond_rounding_error(o.to_f32(got, dt), ref.reshape(-1), dt) < 2e-3, where
    assert len(seen) >= 3  # the draw spans several launch plans


@pytest.mark.parametrize("case", range(6))
def test_matmul_random_shapes_within_bar(nf4, orc, case):
    """Eight shapes per case at 2..600 rows: the few-row kernel, the GEMM
    unsplit and with every K split."""
    from ttspipe_amd import _lib

    splits = set()
    for i, (M, K, bs, nested, dtype, rows) in enumerate(_shapes(8, 2000 + case, 600)):
        layer = random_layer(M, K, nested, seed=case * 100 + i + 50, bs=bs)
        lin = to_linear(layer, dtype)
        xb = randn_bits(rows * K, dtype, seed=rows + i)
        y = lin(from_bits(xb, dtype).view(rows, K))
        assert y.shape == (rows, M)
        splits.add(_lib.load().ttsp_nf4_gemm_splits(M, K, rows))
        dt = dt_code(dtype)
        sample = np.unique(np.linspace(0, rows - 1, 6).astype(int))
        ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], dt, **oracle_args(layer), M=M, K=K, N=sample.size,
                               bs=bs, bs2=layer["bs2"] or 256)
        got = o.to_f32(bits(y), dt).reshape(rows, M)[sample]
        where = f"M={M} K={K} rows={rows} bs={bs} nested={nested} {dtype}"
        assert beyond_rounding_error(got, ref, dt) < 2e-3, where
    assert splits  # (recorded for the failure message of a future plan change)


def _dl_shapes(n: int, seed: int, splits: int):
    """(M, K, bs, nested, dtype, rows) the launch plan gives the direct-to-LDS
    kernel with `splits` K splits: 4 where K has 64 or more 64-code steps and
    there are at least 75 64 x 128 tiles; with fewer steps unsplit from 512
    tiles and 2 splits from 300."""
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        rows = int(rng.integers(256, 513))
        nt = -(-rows // 128)
        if splits == 4:
            K = 512 * int(rng.integers(8, 33))  # 64 to 256 steps, a multiple of 8
            M = int(rng.integers(64 * (-(-75 // nt)), 9001))
        elif splits == 1:
            K = 128 * int(rng.integers(1, 32))  # fewer than 64 steps
            M = int(rng.integers(64 * (-(-512 // nt)), 64 * (-(-512 // nt)) + 4001))
        else:
            K = 256 * int(rng.integers(1, 16))  # steps a multiple of 4, fewer than 64
            lo, hi = 64 * (-(-300 // nt)), 64 * (512 // nt) - 1
            if lo > hi:  # 256 rows: 2 row tiles need 150-255 weight tiles
                rows, nt = 512, 4
                lo, hi = 64 * 75, 64 * 128 - 1
            M = int(rng.integers(lo, hi + 1))
        bs = int(rng.choice([64, 128, 256]))
        if K % bs:
            bs = 64
        out.append((M, K, bs, bool(rng.integers(0, 2)), DTYPES[int(rng.integers(0, 2))], rows))
    return out


@pytest.mark.parametrize("splits", [1, 2, 4])
def test_direct_lds_gemm_random_shapes_within_bar(nf4, orc, splits):
    """Six random shapes per launch form of the direct-to-LDS kernel
    (unsplit, 2 and 4 K-splits): ragged weight and activation rows, block
    sizes 64 to 256, plain and nested scales (whose second-level group may
    change inside a workgroup's K range), bf16 and fp16; a sample of rows
    against the oracle's fp64 product within the bar."""
    from ttspipe_amd import _lib
    from tests.test_abi import _dl_split

    for i, (M, K, bs, nested, dtype, rows) in enumerate(_dl_shapes(6, 2700 + splits, splits)):
        where = f"M={M} K={K} rows={rows} bs={bs} nested={nested} {dtype}"
        assert _dl_split(M, K, rows) == splits, where
        assert _lib.load().ttsp_nf4_gemm_splits(M, K, rows) == splits, where
        layer = random_layer(M, K, nested, seed=splits * 100 + i + 7, bs=bs)
        lin = to_linear(layer, dtype)
        xb = randn_bits(rows * K, dtype, seed=rows + i + 11)
        y = lin(from_bits(xb, dtype).view(rows, K))
        dt = dt_code(dtype)
        sample = np.unique(np.concatenate([np.linspace(0, rows - 1, 5).astype(int), [rows - 1]]))
        ref = orc.nf4_gemm_ref(xb.reshape(rows, K)[sample], dt, **oracle_args(layer), M=M, K=K, N=sample.size,
                               bs=bs, bs2=layer["bs2"] or 256)
        got = o.to_f32(bits(y), dt).reshape(rows, M)[sample]
        assert beyond_rounding_error(got, ref, dt) < 2e-3, where


@pytest.mark.parametrize("case", range(6))
def test_few_rows_random_shapes_within_bar(nf4, orc, case):
    """2 to 64 rows (the few-row kernel wherever K allows it) at random layer
    shapes, every row checked."""
    rng = np.random.default_rng(2500 + case)
    for i, (M, K, bs, nested, dtype, _) in enumerate(_shapes(8, 2500 + case, 2)):
        rows = int(rng.integers(2, 65))
        layer = random_layer(M, K, nested, seed=case * 100 + i + 90, bs=bs)
        lin = to_linear(layer, dtype)
        xb = randn_bits(rows * K, dtype, seed=rows + i + 5)
        y = lin(from_bits(xb, dtype).view(rows, K))
        dt = dt_code(dtype)
        ref = orc.nf4_gemm_ref(xb, dt, **oracle_args(layer), M=M, K=K, N=rows, bs=bs, bs2=layer["bs2"] or 256)
        got = o.to_f32(bits(y), dt).reshape(rows, M)
        where = f"M={M} K={K} rows={rows} bs={bs} nested={nested} {dtype}"
        assert beyond_rounding_error(got, ref, dt) < 2e-3, where


FORMS = ("norm", "norm+swiglu", "swiglu", "norm+residual")


@pytest.mark.parametrize("case", range(6))
def test_fused_forms_random_shapes_bit_exact(nf4, orc, case):
    """The one-launch forms of the decode block (the norm folded in, the
    SwiGLU pair, the residual epilogue after a folded norm) at random shapes
    up to the widest K a folded norm takes, against the oracle's composition
    of the unfused steps, bit for bit."""
    rng = np.random.default_rng(3000 + case)
    for i in range(8):
        K = 128 * int(rng.integers(1, nf4.NORM_MAX_K // 128 + 1))
        M = int(rng.integers(1, 6001))
        bs = int(rng.choice([64, 128, 256]))
        if K % bs:
            bs = 128
        nested = bool(rng.integers(0, 2))
        dtype = DTYPES[int(rng.integers(0, 2))]
        form = FORMS[int(rng.integers(0, len(FORMS)))]
        dt = dt_code(dtype)
        l1 = random_layer(M, K, nested, seed=case * 100 + i + 7, bs=bs)
        w1 = to_linear(l1, dtype)
        assert nf4.prepare(w1)
        xb = randn_bits(K, dtype, seed=i + 11 * case, scale=2.0)
        gb = o.from_f32((rng.random(K) * 0.5 + 0.75).astype(np.float32), dt)
        x = from_bits(xb, dtype).view(1, 1, K)
        norm = from_bits(gb, dtype) if "norm" in form else None
        J, KS, _ = gemv_shape(M, K)
        bs2 = l1["bs2"] or 256
        xin = orc.rms_norm_emul(xb, gb, 1, K, 1e-6, dt) if norm is not None else xb
        where = f"{form} M={M} K={K} bs={bs} nested={nested} {dtype} J={J} KS={KS}"
        if "swiglu" in form:
            l3 = random_layer(M, K, nested, seed=case * 100 + i + 8, bs=bs)
            w3 = to_linear(l3, dtype)
            assert nf4.prepare(w3)
            y = nf4.matmul_fused(w1, x, norm_weight=norm, eps=1e-6, module3=w3)
            g1 = orc.gemv_emul(xin, dt, **oracle_args(l1), M=M, K=K, bs=bs, KS=KS, J=J, bs2=bs2)
            expect = orc.gemv_emul(xin, dt, **oracle_args(l3), M=M, K=K, bs=bs, KS=KS, J=J, bs2=bs2, R=g1, epi=2)
        elif form == "norm+residual":
            rb = randn_bits(M, dtype, seed=M + i)
            y = nf4.matmul_fused(w1, x, norm_weight=norm, eps=1e-6, epi=nf4.EPI_RESIDUAL,
                                 operand=from_bits(rb, dtype))
            expect = orc.gemv_emul(xin, dt, **oracle_args(l1), M=M, K=K, bs=bs, KS=KS, J=J, bs2=bs2, R=rb, epi=1)
        else:
            y = nf4.matmul_fused(w1, x, norm_weight=norm, eps=1e-6)
            expect = orc.gemv_emul(xin, dt, **oracle_args(l1), M=M, K=K, bs=bs, KS=KS, J=J, bs2=bs2)
        assert y is not None, f"{where}: declined"
        assert np.array_equal(bits(y), expect), f"{where}: {first_mismatch(bits(y), expect)}"
