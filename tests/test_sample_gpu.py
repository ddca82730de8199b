"""The fused top-k / top-p sampler (ttsp_sample_topk) against the oracle's
float64 restatement of the reference's sampler (fusedsample.py:55-223), with
the same per-index uniform numbers (GPU).

Bar: the same drawn index, except where the decision is within fp32 rounding
of a boundary - a candidate's cumulative probability within 1e-5 of top_p,
or the best two scores within 1e-5 - which the test detects and skips."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o
from tests.gpuutil import bits, dt_code, from_bits

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _draw(row_bits, dtype, temp, topp, topk, u):
    from ttspipe_amd import fusedsample

    row = from_bits(row_bits, dtype)
    t = torch.tensor([temp], dtype=dtype, device="cuda")
    p = torch.tensor([topp], dtype=dtype, device="cuda")
    k = torch.tensor([topk], dtype=torch.int64, device="cuda")
    return int(fusedsample.sample(row, t, p, k, uniform=torch.from_numpy(u).cuda()).item())


def _ambiguous(l, temp, topp, topk, u):
    _, kept, c, scores = o.sample_topk_ref(l, temp, topp, topk, u)
    if np.any(np.abs(c[1:] - topp) < 1e-5 * max(1.0, topp)):
        return True
    s = np.sort(scores)[::-1]
    return s.size > 1 and s[0] - s[1] < 1e-5 * max(1.0, abs(s[0]))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("topk,topp,temp", [(1, 0.9, 0.7), (5, 1.0, 1.0), (30, 0.9, 0.7), (64, 0.95, 1.3),
                                            (100, 0.5, 0.3), (64, 0.0, 1.0), (40, 1.0, 0.05)])
def test_sampler_matches_the_oracle(dtype, topk, topp, temp):
    dt = dt_code(dtype)
    rng = np.random.default_rng(topk * 1000 + int(topp * 100) + int(temp * 10))
    checked = 0
    for trial in range(40):
        V = 4096 if trial % 4 else 1000
        lb = o.from_f32((rng.standard_normal(V) * 2.5).astype(np.float32), dt)
        u = rng.random(V).astype(np.float32)
        tq = float(o.to_f32(o.from_f32(np.float32([temp]), dt), dt)[0])
        pq = float(o.to_f32(o.from_f32(np.float32([topp]), dt), dt)[0])
        l = o.to_f32(lb, dt).astype(np.float64)
        if _ambiguous(l, tq, pq, topk, u):
            continue
        expect = o.sample_topk_ref(l, tq, pq, topk, u)[0]
        assert _draw(lb, dtype, temp, topp, topk, u) == expect, f"trial {trial}"
        checked += 1
    assert checked >= 30


@pytest.mark.parametrize("dtype", DTYPES)
def test_sampler_ties_and_masked_entries(dtype):
    """Many logits equal to the k-th value (the cut takes the lowest indices),
    and -inf entries (never drawn)."""
    dt = dt_code(dtype)
    rng = np.random.default_rng(5)
    V = 4096
    l = np.full(V, -np.inf, np.float32)
    l[::7] = 1.0                 # 586 ties
    l[100:110] = 3.0             # a clear top ten
    lb = o.from_f32(l, dt)
    for topk in (10, 12, 64):
        for _ in range(10):
            u = rng.random(V).astype(np.float32)
            expect = o.sample_topk_ref(o.to_f32(lb, dt).astype(np.float64), 1.0, 1.0, topk, u)[0]
            got = _draw(lb, dtype, 1.0, 1.0, topk, u)
            assert got == expect
            assert np.isfinite(l[got])
            if topk > 10 and got not in range(100, 110):
                assert got % 7 == 0 and got < 7 * (topk - 10)  # the lowest-index ties


def test_sampler_is_deterministic_and_greedy_limits():
    from ttspipe_amd import fusedsample

    rng = np.random.default_rng(9)
    row = torch.from_numpy((rng.standard_normal(4096) * 3).astype(np.float32)).to("cuda", torch.bfloat16)
    u = torch.rand(4096, device="cuda")
    t, p = torch.tensor([0.8], device="cuda"), torch.tensor([0.9], device="cuda")
    k = torch.tensor([30], device="cuda")
    a = [int(fusedsample.sample(row, t, p, k, uniform=u).item()) for _ in range(5)]
    assert len(set(a)) == 1
    am = int(torch.argmax(row.float()).item())
    assert int(fusedsample.sample(row, t, p, torch.tensor([1], device="cuda")).item()) == am
    assert int(fusedsample.sample(row, t, torch.tensor([0.0], device="cuda"), k).item()) == am
    assert fusedsample.MAX_TOP_K == 64 and fusedsample.available()
    # fresh uniforms: every draw lands in the top-k set
    top = set(torch.topk(row.float(), 30).indices.tolist())
    for _ in range(50):
        assert int(fusedsample.sample(row, t, torch.tensor([1.0], device="cuda"), k).item()) in top


@pytest.mark.parametrize("V", [1, 7, 63, 64, 65, 257, 4095, 32768])
def test_sampler_row_lengths(V):
    """Rows shorter than k, rows that do not fill the workgroup's stride and
    the longest row served, against the oracle."""
    dtype = torch.bfloat16
    dt = dt_code(dtype)
    rng = np.random.default_rng(V)
    checked = 0
    for trial in range(6):
        lb = o.from_f32((rng.standard_normal(V) * 2.0).astype(np.float32), dt)
        u = rng.random(V).astype(np.float32)
        l = o.to_f32(lb, dt).astype(np.float64)
        tq = float(o.to_f32(o.from_f32(np.float32([0.8]), dt), dt)[0])
        pq = float(o.to_f32(o.from_f32(np.float32([0.9]), dt), dt)[0])
        if _ambiguous(l, tq, pq, 64, u):
            continue
        assert _draw(lb, dtype, 0.8, 0.9, 64, u) == o.sample_topk_ref(l, tq, pq, 64, u)[0], f"trial {trial}"
        checked += 1
    assert checked >= 4


def test_sampler_declines_rows_longer_than_it_holds():
    from ttspipe_amd import fusedsample

    row = torch.zeros(fusedsample.MAX_VOCAB + 1, device="cuda", dtype=torch.float16)
    t, p = torch.tensor([1.0], device="cuda"), torch.tensor([1.0], device="cuda")
    assert fusedsample.sample(row, t, p, torch.tensor([5], device="cuda")) is None


@pytest.mark.parametrize("case", range(4))
def test_sampler_random_settings(case):
    """Random row lengths (1 to 32768), k (1 to 100), top-p, temperatures and
    logit spreads (down to bf16/fp16 spacing, where ties abound): the drawn
    index equals the oracle's wherever the decision is not within rounding of
    a boundary."""
    rng = np.random.default_rng(9000 + case)
    checked = 0
    for trial in range(40):
        dtype = DTYPES[int(rng.integers(0, 2))]
        dt = dt_code(dtype)
        V = int(rng.integers(1, 32769))
        topk, topp = int(rng.integers(1, 101)), float(rng.choice([0.0, 0.3, 0.8, 0.95, 1.0]))
        temp = float(rng.choice([0.05, 0.5, 1.0, 1.7]))
        spread = float(rng.choice([0.02, 1.0, 4.0]))
        lb = o.from_f32((rng.standard_normal(V) * spread).astype(np.float32), dt)
        u = rng.random(V).astype(np.float32)
        tq = float(o.to_f32(o.from_f32(np.float32([temp]), dt), dt)[0])
        pq = float(o.to_f32(o.from_f32(np.float32([topp]), dt), dt)[0])
        l = o.to_f32(lb, dt).astype(np.float64)
        if _ambiguous(l, tq, pq, topk, u):
            continue
        expect = o.sample_topk_ref(l, tq, pq, topk, u)[0]
        where = f"trial {trial}: V={V} k={topk} p={topp} T={temp} spread={spread} {dtype}"
        assert _draw(lb, dtype, temp, topp, topk, u) == expect, where
        checked += 1
    assert checked >= 25
