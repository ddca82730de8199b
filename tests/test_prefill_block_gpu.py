"""The multi-position (prompt prefill) block and the Dual-AR prompt prefill
with its bucket graphs (GPU), plus the span arithmetic (CPU).

Bar: the fused prefill block against a float64 restatement of the block
with the fork's roundings that no kernel of this repository feeds
(tests/refblock.py; weights from the numpy dequantisation), rel-norm < 3e-3,
a bar each planted mistake of the restatement misses by more than twice
(CPU test); against the block's own unpatched forward (the same GEMMs, the
epilogues keep the unfused roundings; the head norms run in the decode
step's kernel instead of the fork's torch modules), at the reference's block
bar rel-norm < 2e-2 (tests/test_nf4cpu.py:175-191), V rows identical; the many-row head-norm/rotary/KV kernel bit for bit against the
one-position kernel; the model's prompt prefill against the same
positions decoded one at a time through the decode kernels (different GEMM
and attention kernels, so the reference's 2e-2 block bar on the KV rows and
the last position's logits); graph replay against the eager span, bit for
bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch


def _rel(a, b):
    a, b = a.float(), b.float()
    return ((a - b).norm() / b.norm()).item()


def test_prefill_spans_follow_the_buckets():
    from ttspipe_amd.dualar import PREFILL_BUCKETS, prefill_spans

    top = PREFILL_BUCKETS[-1]
    assert prefill_spans(0) == []
    assert PREFILL_BUCKETS[:6] == (1, 2, 4, 8, 16, 32)  # the reference's buckets (graphs.py:137)
    assert prefill_spans(1) == [(0, 1, 1)]
    assert [prefill_spans(n)[0][2] for n in (2, 3, 4, 5, 8, 9)] == [2, 4, 4, 8, 8, 16]
    assert prefill_spans(40) == [(0, 40, 64)]
    assert prefill_spans(top) == [(0, top, top)]
    assert prefill_spans(top + 1) == [(0, top, top), (top, 1, PREFILL_BUCKETS[0])]
    assert prefill_spans(2 * top + 100) == [(0, top, top), (top, top, top), (2 * top, 100, 128)]
    for n in range(1, 1200, 37):
        sp = prefill_spans(n)
        assert sum(s for _, s, _ in sp) == n and all(s <= b for _, s, b in sp)
        assert all(o == sum(s for _, s, _ in sp[:i]) for i, (o, _, _) in enumerate(sp))


@pytest.mark.gpu
@pytest.mark.parametrize("qk_norm", [True, False])
def test_prefill_block_matches_the_unpatched_block(qk_norm):
    from tests.test_fused_gpu import _block
    from ttspipe_amd import fusedlayer, fusedops, nf4gemv
    from ttspipe_amd.llama import TransformerBlock, precompute_freqs_cis

    # the worker's installs (app/engine/worker.py:565-586): the unpatched
    # block's norms and linears then run the same kernels as the prefill
    # block's, whatever ran before this test
    assert nf4gemv.install() and fusedops.install() and fusedlayer.install()
    block, _ = _block(torch.bfloat16, qk_norm, max_len=128, seed=3)
    kc, vc = block.attention.kv_cache.k_cache, block.attention.kv_cache.v_cache
    kc.normal_()
    vc.normal_()
    saved = (kc.clone(), vc.clone())
    pos = torch.arange(24, 64, device="cuda")
    mask = torch.tril(torch.ones(128, 128, dtype=torch.bool, device="cuda"))[None, None, pos]
    freqs = precompute_freqs_cis(128, 128, 1e6).cuda()[pos]
    x = torch.randn(1, 40, 512, device="cuda").to(torch.bfloat16)
    before = fusedlayer.stats()["prefill"]
    ours = block(x, freqs, mask, pos)
    assert fusedlayer.stats()["prefill"] == before + 1
    ours_k, ours_v = kc[:, :, 24:64].clone(), vc[:, :, 24:64].clone()
    kc.copy_(saved[0])
    vc.copy_(saved[1])
    theirs = TransformerBlock._fused_original_forward(block, x, freqs, mask, pos)
    assert _rel(ours, theirs) < 2e-2
    assert _rel(ours_k, kc[:, :, 24:64]) < 2e-2
    assert torch.equal(ours_v, vc[:, :, 24:64])  # V rows are copied as they are


@pytest.mark.gpu
@pytest.mark.parametrize("qk_norm,rows,dtype", [(True, 40, torch.bfloat16), (False, 100, torch.float16)])
def test_prefill_block_folded_reduces_equal_the_separate_launches(monkeypatch, qk_norm, rows, dtype):
    """A block whose wqkv, wo and w2 all take K splits (d = 1024, 8 q / 2 kv
    heads, FFN 2048): wqkv's partial sums added inside the head-norm / rotary
    / KV kernel and the RMSNorms written by wo's and w2's reduces, against
    the block with a reduce and a norm launch of their own: the output, the
    next norm's output and every cache row bit for bit."""
    from tests.gpuutil import bits
    from tests.test_fused_gpu import _block
    from ttspipe_amd import _lib, fusedlayer, fusedops, nf4gemv
    from ttspipe_amd.llama import precompute_freqs_cis

    assert nf4gemv.install() and fusedops.install()
    lib = _lib.load()
    assert min(lib.ttsp_nf4_gemm_splits(1536, 1024, rows), lib.ttsp_nf4_gemm_splits(1024, 1024, rows),
               lib.ttsp_nf4_gemm_splits(1024, 2048, rows)) > 1
    block, _ = _block(dtype, qk_norm, dim=1024, n_head=8, n_local_heads=2, inter=2048, max_len=128, seed=4)
    kc, vc = block.attention.kv_cache.k_cache, block.attention.kv_cache.v_cache
    kc.normal_()
    vc.normal_()
    saved = (kc.clone(), vc.clone())
    start = 128 - rows
    pos = torch.arange(start, 128, device="cuda")
    mask = torch.tril(torch.ones(128, 128, dtype=torch.bool, device="cuda"))[None, None, pos]
    freqs = precompute_freqs_cis(128, 128, 1e6).cuda()[pos].contiguous()
    x = torch.randn(1, rows, 1024, device="cuda").to(dtype)

    def run():
        kc.copy_(saved[0])
        vc.copy_(saved[1])
        r = fusedlayer.prefill_block_chain(block, x, freqs, mask, pos, next_norm=block.attention_norm)
        assert r is not None and r[1] is not None
        torch.cuda.synchronize()
        return [bits(t).copy() for t in (*r, kc, vc)]

    used = []

    def spy(fn, tag):
        def wrapped(*a, **k):
            r = fn(*a, **k)
            used.append((tag, r is not None))
            return r
        return wrapped

    monkeypatch.setattr(nf4gemv, "matmul_partials", spy(nf4gemv.matmul_partials, "partials"))
    monkeypatch.setattr(nf4gemv, "matmul_norm", spy(nf4gemv.matmul_norm, "norm"))
    folded = run()
    assert used == [("partials", True), ("norm", True), ("norm", True)]
    monkeypatch.setattr(nf4gemv, "matmul_norm", lambda *a, **k: None)
    monkeypatch.setattr(nf4gemv, "matmul_partials", lambda *a, **k: None)
    separate = run()
    for name, a_, b_ in zip(["out", "out_n", "k_cache", "v_cache"], folded, separate):
        assert np.array_equal(a_, b_), name
    assert not np.array_equal(separate[2], bits(saved[0]))  # the span was written


# ------------------------------------------------ against an fp64 block

REF_BAR = 3e-3  # rel-norm of the block output against the fp64 block with the fork's roundings
REF_START, REF_ROWS, REF_LEN = 24, 40, 128


def _ref_inputs(dtype, qk_norm, seed=3, nh=4, nkv=2, D=512, inter=1024, start=REF_START, rows=REF_ROWS,
                length=REF_LEN):
    """The fp64 reference's inputs for `_block(dtype, qk_norm, D, nh, nkv,
    inter, max_len=length, seed)`: its dequantised weights (numpy closed
    form) and norm weights (the same seeded generator), seeded x rows at
    positions start.. start + rows - 1 and cache, the positions'
    frequencies."""
    from oracle import oracle as o
    from tests.nf4data import dequant_numpy, random_layer
    from ttspipe_amd.llama import precompute_freqs_cis

    dt = o.DT_BF16 if dtype == torch.bfloat16 else o.DT_F16
    W = {}
    for i, (name, M, K) in enumerate([("wqkv", (nh + 2 * nkv) * 128, D), ("wo", D, nh * 128), ("w1", inter, D),
                                      ("w3", inter, D), ("w2", D, inter)]):
        W[name] = o.to_f32(dequant_numpy(random_layer(M, K, True, seed=seed * 10 + i), dt), dt).astype(
            np.float64).reshape(M, K)
    g = torch.Generator().manual_seed(seed)
    names = ["attention_norm", "ffn_norm"] + (["q_norm", "k_norm"] if qk_norm else [])
    norms = {n: (torch.rand(D if "attention" in n or "ffn" in n else 128, generator=g) + 0.5).to(dtype)
             .double().numpy() for n in names}
    rng = np.random.default_rng(seed + 100)
    q16 = lambda a: o.from_f32(a.astype(np.float32), dt)  # noqa: E731
    xb = q16(rng.standard_normal((rows, D)))
    kcb, vcb = q16(rng.standard_normal((nkv, length, 128))), q16(rng.standard_normal((nkv, length, 128)))
    pos = list(range(start, start + rows))
    freqs = precompute_freqs_cis(length, 128, 1e6)[pos]
    f64 = lambda b: o.to_f32(b, dt).astype(np.float64)  # noqa: E731
    rnd = lambda t: f64(q16(np.asarray(t)))  # noqa: E731
    return dict(W=W, norms=norms, xb=xb, kcb=kcb, vcb=vcb, pos=pos, freqs=freqs, dt=dt, f64=f64, rnd=rnd,
                nh=nh, nkv=nkv, D=D, inter=inter, start=start, rows=rows, length=length, seed=seed)


def _ref(c, qk_norm, mutant=None):
    from tests.refblock import block_fp64

    f64 = c["f64"]
    return block_fp64(c["W"], c["norms"], f64(c["xb"]), c["freqs"].double().numpy(), f64(c["kcb"]), f64(c["vcb"]),
                      c["pos"], c["nh"], c["nkv"], qk_norm, rnd=c["rnd"], mutant=mutant)


@pytest.mark.parametrize("qk_norm", [True, False])
def test_fp64_block_reference_catches_planted_mistakes(qk_norm):
    """Each planted mistake of the reference block (no rotary, no q/k norm,
    query heads mapped to KV heads modulo, a mask one position too wide)
    moves its output more than twice the bar the fused block is held to."""
    from tests.refblock import MUTANTS, rel_norm

    c = _ref_inputs(torch.bfloat16, qk_norm)
    ref = _ref(c, qk_norm)[0]
    for m in MUTANTS:
        if m == "no_qk_norm" and not qk_norm:
            continue
        assert rel_norm(_ref(c, qk_norm, m)[0], ref) > 2 * REF_BAR, m


def _block_against_fp64(dtype, qk_norm, causal=False, **shape):
    """The fused prefill block of `_ref_inputs(dtype, qk_norm, **shape)`'s
    shape on the GPU against the fp64 block: (rel-norm of the output, K-row
    and V-row error in ulps of each head row's largest element). `causal`:
    through `prefill_block_chain(..., causal=True)`, the attention computing
    the causal mask from the positions."""
    from tests.refblock import rel_norm
    from tests.test_fused_gpu import _block
    from ttspipe_amd import fusedlayer, fusedops, nf4gemv

    assert nf4gemv.install() and fusedops.install() and fusedlayer.install()
    c = _ref_inputs(dtype, qk_norm, **shape)
    D, rows, start, length = c["D"], c["rows"], c["start"], c["length"]
    block, _ = _block(dtype, qk_norm, dim=D, n_head=c["nh"], n_local_heads=c["nkv"], inter=c["inter"],
                      max_len=length, seed=c["seed"])
    for n, w in c["norms"].items():
        mod = getattr(block, n, None) or getattr(block.attention, n)
        assert np.array_equal(mod.weight.double().cpu().numpy(), w)
    dev = lambda b, shape: torch.from_numpy(b.view(np.int16).copy()).view(dtype).cuda().view(shape)  # noqa: E731
    kv = block.attention.kv_cache
    kv.k_cache.copy_(dev(c["kcb"], kv.k_cache.shape))
    kv.v_cache.copy_(dev(c["vcb"], kv.v_cache.shape))
    pos = torch.tensor(c["pos"], device="cuda")
    mask = torch.tril(torch.ones(length, length, dtype=torch.bool, device="cuda"))[None, None, pos]
    before = fusedlayer.stats()["prefill"]
    with torch.inference_mode():
        if causal:
            r = fusedlayer.prefill_block_chain(block, dev(c["xb"], (1, rows, D)), c["freqs"].cuda(), mask, pos,
                                               causal=True)
            assert r is not None
            ours = r[0]
        else:
            ours = block(dev(c["xb"], (1, rows, D)), c["freqs"].cuda(), mask, pos)
    assert fusedlayer.stats()["prefill"] == before + 1
    ref, k_ref, v_ref = _ref(c, qk_norm)
    got = ours.double().cpu().numpy().reshape(rows, D)
    rel = rel_norm(got, ref)
    k_got = kv.k_cache[0, :, start : start + rows].double().cpu().numpy().transpose(1, 0, 2)
    v_got = kv.v_cache[0, :, start : start + rows].double().cpu().numpy().transpose(1, 0, 2)
    # in ulps of each head row's largest element (rotation may cancel two
    # rounded inputs into a value far smaller than either)
    mant = 7 if dtype == torch.bfloat16 else 10
    row_ulp = lambda t: 2.0 ** (np.floor(np.log2(np.abs(t).max(-1, keepdims=True))) - mant)  # noqa: E731
    k_ulps = float(np.max(np.abs(k_got - k_ref) / row_ulp(k_ref)))
    v_ulps = float(np.max(np.abs(v_got - v_ref) / row_ulp(v_ref)))
    return rel, k_ulps, v_ulps


@pytest.mark.gpu
@pytest.mark.parametrize("qk_norm", [True, False])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_block_matches_an_fp64_block(qk_norm, dtype):
    """The fused prefill block (40 rows at positions 24..63 over a 128-row
    cache) against the block restated in float64 with the fork's roundings
    (tests/refblock.py; no kernel of this repository feeds it): the output
    within REF_BAR (rel-norm), the new K and V rows within one 16-bit ulp of
    each head row's largest element (the products' own roundings)."""
    rel, k_ulps, v_ulps = _block_against_fp64(dtype, qk_norm)
    print(f"prefill block vs fp64 block: rel {rel:.2e}, K rows {k_ulps:.1f} ulp, V rows {v_ulps:.1f} ulp")
    assert rel < REF_BAR
    assert k_ulps <= 1.0 and v_ulps <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("case", range(6))
def test_random_block_shapes_match_an_fp64_block(case):
    """The same bars at randomly drawn block shapes: width 256-1024, 1-8 kv
    heads with 1-4 query heads each, FFN 256-2048, 2-200 new rows after a
    0-300 position prefix (so the GEMMs take the few-row kernel and every
    split, and the attention one or several key blocks)."""
    rng = np.random.default_rng(900 + case)
    nkv = int(rng.choice([1, 2, 4, 8]))
    shape = dict(nkv=nkv, nh=nkv * int(rng.choice([1, 2, 4])), D=128 * int(rng.integers(2, 9)),
                 inter=128 * int(rng.integers(2, 17)), start=int(rng.integers(0, 301)), rows=int(rng.integers(2, 201)),
                 seed=40 + case)
    shape["length"] = shape["start"] + shape["rows"] + int(rng.integers(0, 64))
    dtype = [torch.bfloat16, torch.float16][int(rng.integers(0, 2))]
    qk_norm = bool(rng.integers(0, 2))
    rel, k_ulps, v_ulps = _block_against_fp64(dtype, qk_norm, **shape)
    where = f"{shape} {dtype} qk_norm={qk_norm}: rel {rel:.2e}, K {k_ulps:.1f} ulp, V {v_ulps:.1f} ulp"
    assert rel < REF_BAR, where
    assert k_ulps <= 1.0 and v_ulps <= 1.0, where


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_causal_512_row_block_matches_an_fp64_block(dtype):
    """A 512-row first span with 32 query / 8 kv heads through the causal
    chain, whose attention then takes two-head workgroups with four key
    splits each: the same bars against the fp64 block."""
    from ttspipe_amd import fastpath

    before = fastpath.stats()["prefill_attn"]
    rel, k_ulps, v_ulps = _block_against_fp64(dtype, True, causal=True, nh=32, nkv=8, D=1024, inter=1024, start=0,
                                              rows=512, length=512, seed=71)
    assert fastpath.stats()["prefill_attn"] == before + 1
    print(f"causal 512-row block vs fp64 block: rel {rel:.2e}, K rows {k_ulps:.1f} ulp, V rows {v_ulps:.1f} ulp")
    assert rel < REF_BAR
    assert k_ulps <= 1.0 and v_ulps <= 1.0


@pytest.mark.gpu
@pytest.mark.parametrize("rows,start,nh,nkv", [(100, 37, 32, 8), (64, 200, 8, 2), (20, 0, 6, 3)])
def test_causal_chain_equals_the_masked_chain(rows, start, nh, nkv):
    """`prefill_block_chain(..., causal=True)` (the mask computed from the
    positions) against the same chain reading the causal mask's bytes: the
    block output, its carried norm and the new K/V rows bit for bit (shapes
    on the two-split attention form)."""
    from tests.test_fused_gpu import _block
    from ttspipe_amd import fusedlayer, fusedops, nf4gemv

    assert nf4gemv.install() and fusedops.install() and fusedlayer.install()
    dtype, D, length = torch.bfloat16, 512, 512
    block, _ = _block(dtype, True, dim=D, n_head=nh, n_local_heads=nkv, inter=1024, max_len=length, seed=rows)
    kv = block.attention.kv_cache
    g = torch.Generator().manual_seed(start)
    kv.k_cache.copy_(torch.randn(kv.k_cache.shape, generator=g).to(dtype))
    kv.v_cache.copy_(torch.randn(kv.v_cache.shape, generator=g).to(dtype))
    x = torch.randn(1, rows, D, generator=g).to(dtype).cuda()
    pos = torch.arange(start, start + rows, device="cuda")
    from ttspipe_amd.llama import precompute_freqs_cis

    freqs = precompute_freqs_cis(length, 128, 10000.0, dtype=dtype).cuda()[pos].contiguous()
    mask = torch.tril(torch.ones(length, length, dtype=torch.bool, device="cuda"))[None, None, pos]
    outs = []
    with torch.inference_mode():
        for causal in (False, True):
            r = fusedlayer.prefill_block_chain(block, x, freqs, mask, pos, next_norm=block.ffn_norm, causal=causal)
            assert r is not None
            k_rows = kv.k_cache[0, :, start : start + rows].clone()
            v_rows = kv.v_cache[0, :, start : start + rows].clone()
            outs.append([t.clone() for t in r] + [k_rows, v_rows])
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("rows,start", [(2, 30), (5, 60), (8, 0)])
def test_short_causal_span_attention_from_qkv_equals_the_rows_kernels(monkeypatch, rows, start):
    """A causal span of up to 8 rows with the head norms, rotary and KV write
    inside the row-by-row attention launch, against the same chain with them
    as their own launch first: the block output and the new K/V rows bit for
    bit."""
    from tests.test_fused_gpu import _block
    from ttspipe_amd import fastpath, fusedlayer, fusedops, nf4gemv
    from ttspipe_amd.llama import precompute_freqs_cis

    assert nf4gemv.install() and fusedops.install() and fusedlayer.install()
    dtype, D, length = torch.bfloat16, 512, 256
    block, _ = _block(dtype, True, dim=D, n_head=8, n_local_heads=2, inter=1024, max_len=length, seed=rows)
    kv = block.attention.kv_cache
    g = torch.Generator().manual_seed(start)
    kc0 = torch.randn(kv.k_cache.shape, generator=g).to(dtype).cuda()
    vc0 = torch.randn(kv.v_cache.shape, generator=g).to(dtype).cuda()
    x = torch.randn(1, rows, D, generator=g).to(dtype).cuda()
    pos = torch.arange(start, start + rows, device="cuda")
    freqs = precompute_freqs_cis(length, 128, 10000.0, dtype=dtype).cuda()[pos].contiguous()
    mask = torch.tril(torch.ones(length, length, dtype=torch.bool, device="cuda"))[None, None, pos]
    outs = []
    orig = fastpath.causal_rows_attention_qkv
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(fastpath, "causal_rows_attention_qkv", lambda *a, **k: None)
        kv.k_cache.copy_(kc0)
        kv.v_cache.copy_(vc0)
        with torch.inference_mode():
            out, _ = fusedlayer.prefill_block_chain(block, x, freqs, mask, pos, causal=True)
        outs.append([out.clone(), kv.k_cache.clone(), kv.v_cache.clone()])
    monkeypatch.setattr(fastpath, "causal_rows_attention_qkv", orig)
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("causal", [True, False])
def test_two_row_chain_with_folded_norms_equals_the_norm_launches(monkeypatch, causal):
    """Two blocks chained over a 2-row span: with the RMSNorms folded into the
    wqkv and w1 / w3 GEMVs (no norm launch) against the same chain running
    them as launches (the carried norm, then w1 and w3 on it): both blocks'
    outputs and the new K/V rows bit for bit."""
    from tests.test_fused_gpu import _block
    from ttspipe_amd import fusedlayer, fusedops, nf4gemv
    from ttspipe_amd.llama import precompute_freqs_cis

    assert nf4gemv.install() and fusedops.install() and fusedlayer.install()
    dtype, D, length, start, rows = torch.bfloat16, 512, 256, 30, 2
    block, _ = _block(dtype, True, dim=D, n_head=8, n_local_heads=2, inter=1024, max_len=length, seed=5)
    kv = block.attention.kv_cache
    g = torch.Generator().manual_seed(6)
    kc0 = torch.randn(kv.k_cache.shape, generator=g).to(dtype).cuda()
    vc0 = torch.randn(kv.v_cache.shape, generator=g).to(dtype).cuda()
    x = torch.randn(1, rows, D, generator=g).to(dtype).cuda()
    pos = torch.arange(start, start + rows, device="cuda")
    freqs = precompute_freqs_cis(length, 128, 10000.0, dtype=dtype).cuda()[pos].contiguous()
    mask = torch.tril(torch.ones(length, length, dtype=torch.bool, device="cuda"))[None, None, pos]
    outs = []
    for fold in (False, True):
        monkeypatch.setattr(nf4gemv, "FUSED_MAX_ROWS", 2 if fold else 1)
        kv.k_cache.copy_(kc0)
        kv.v_cache.copy_(vc0)
        calls = nf4gemv.stats()["fast"]
        with torch.inference_mode():
            o1, n1 = fusedlayer.prefill_block_chain(block, x, freqs, mask, pos, next_norm=block.attention_norm,
                                                    causal=causal)
            assert (n1 is None) == fold
            o2, _ = fusedlayer.prefill_block_chain(block, o1, freqs, mask, pos, xn=n1, causal=causal)
        if fold:
            assert nf4gemv.stats()["fast"] >= calls + 6  # wqkv and the w1 / w3 pair of each block, fused
        outs.append([o1.clone(), o2.clone(), kv.k_cache[0, :, start : start + rows].clone(),
                     kv.v_cache[0, :, start : start + rows].clone()])
    for a, b in zip(*outs):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_rows_kernel_equals_the_one_position_kernel(dtype):
    """ttsp_qk_rope_kv_rows over a run of positions (in any order, one out of
    the cache) gives the one-position kernel's bits, row by row."""
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    lib, st = _lib.load(), _lib.stream()
    nh, nkv, max_len, hd = 8, 2, 64, 128
    pos = torch.tensor([3, 10, 11, 40, 2, 70, 63], dtype=torch.long, device="cuda")  # 70: past the cache
    n, total = pos.numel(), (nh + 2 * nkv) * hd
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(n, total + 64, generator=g).to(dtype).cuda()  # row stride wider than a row
    qw = (torch.rand(hd, generator=g) + 0.5).to(dtype).cuda()
    kw = (torch.rand(hd, generator=g) + 0.5).to(dtype).cuda()
    freqs = precompute_freqs_cis(128, hd, 1e6).cuda()[torch.clamp(pos, max=127)].contiguous()
    dt = _lib.dtype_code(dtype)
    kc1 = torch.randn(1, nkv, max_len, hd, generator=g).to(dtype).cuda()
    vc1 = torch.randn(1, nkv, max_len, hd, generator=g).to(dtype).cuda()
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1 = torch.zeros(n, nh, hd, dtype=dtype, device="cuda")
    q2 = torch.zeros_like(q1)
    rc = lib.ttsp_qk_rope_kv_rows(qkv.data_ptr(), qkv.shape[1], qw.data_ptr(), kw.data_ptr(), 1e-6,
                                  freqs.data_ptr(), _lib.DT_BF16, pos.data_ptr(), q1.data_ptr(), kc1.data_ptr(),
                                  vc1.data_ptr(), nh, nkv, max_len, n, dt, st)
    assert rc == 0
    for r in range(n):
        rc = lib.ttsp_qk_rope_kv(qkv[r].data_ptr(), qw.data_ptr(), kw.data_ptr(), 1e-6, freqs[r].data_ptr(),
                                 _lib.DT_BF16, pos[r:].data_ptr(), q2[r].data_ptr(), kc2.data_ptr(), vc2.data_ptr(),
                                 nh, nkv, max_len, dt, st)
        assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert not torch.equal(q1[3], torch.zeros_like(q1[3])) and torch.equal(q1[5], torch.zeros_like(q1[5]))


@pytest.mark.gpu
@pytest.mark.parametrize("K,rows,splits,dtype,qk_norm", [(1024, 40, 2, torch.float16, True),
                                                         (2048, 64, 4, torch.bfloat16, True),
                                                         (4096, 100, 8, torch.bfloat16, False)])
def test_rows_kernel_from_split_partials_equals_reduce_then_rows(K, rows, splits, dtype, qk_norm):
    """wqkv's K-split partial sums added inside the head-norm / rotary / KV
    kernel (`matmul_partials` + ttsp_qk_rope_kv_rows_partials) against the
    split GEMM's own reduce then ttsp_qk_rope_kv_rows: Q, K and V cache bit
    for bit at 2, 4 and 8 splits, fp16 and bf16, with and without the head
    norms, positions in any order and one past the cache (nothing written)."""
    from tests.nf4data import random_layer, to_linear
    from ttspipe_amd import _lib, nf4gemv
    from ttspipe_amd.llama import precompute_freqs_cis

    nh, nkv, hd, max_len = 8, 2, 128, 256
    M = (nh + 2 * nkv) * hd
    lib, st = _lib.load(), _lib.stream()
    assert lib.ttsp_nf4_gemm_splits(M, K, rows) == splits
    assert nf4gemv.install()
    lin = to_linear(random_layer(M, K, True, seed=K + rows), dtype)
    assert nf4gemv.prepare(lin)
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, K, generator=g).mul(0.5).to(dtype).cuda()
    pos = torch.randperm(max_len, generator=g)[:rows].cuda()
    pos[rows // 2] = max_len + 3  # past the cache: the row writes nothing
    freqs = precompute_freqs_cis(max_len + 8, hd, 1e6).cuda()[pos].contiguous()
    qw = (torch.rand(hd, generator=g) + 0.5).to(dtype).cuda() if qk_norm else None
    kw = (torch.rand(hd, generator=g) + 0.5).to(dtype).cuda() if qk_norm else None
    dt = _lib.dtype_code(dtype)
    kc1 = torch.randn(1, nkv, max_len, hd, generator=g).to(dtype).cuda()
    vc1 = torch.randn(1, nkv, max_len, hd, generator=g).to(dtype).cuda()
    kc2, vc2 = kc1.clone(), vc1.clone()
    q1 = torch.zeros(rows, nh, hd, dtype=dtype, device="cuda")
    q2 = torch.zeros_like(q1)
    qkv = nf4gemv.matmul(lin, x)
    rc = lib.ttsp_qk_rope_kv_rows(qkv.data_ptr(), M, _lib.ptr(qw), _lib.ptr(kw), 1e-6, freqs.data_ptr(), _lib.DT_BF16,
                                  pos.data_ptr(), q1.data_ptr(), kc1.data_ptr(), vc1.data_ptr(), nh, nkv, max_len,
                                  rows, dt, st)
    assert rc == 0
    work, got_splits = nf4gemv.matmul_partials(lin, x)
    assert got_splits == splits
    rc = lib.ttsp_qk_rope_kv_rows_partials(work.data_ptr(), splits, _lib.ptr(qw), _lib.ptr(kw), 1e-6,
                                           freqs.data_ptr(), _lib.DT_BF16, pos.data_ptr(), q2.data_ptr(),
                                           kc2.data_ptr(), vc2.data_ptr(), nh, nkv, max_len, rows, dt, st)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(q1.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(kc1.view(torch.int16), kc2.view(torch.int16))
    assert torch.equal(vc1.view(torch.int16), vc2.view(torch.int16))
    assert torch.equal(q2[rows // 2], torch.zeros_like(q2[rows // 2]))
    assert not torch.equal(q2[0], torch.zeros_like(q2[0]))


@pytest.fixture(scope="module")
def fresh():
    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    return SyntheticDualAR(SMALL)


def _tokens(model, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(0, model.cfg.codebook_size, (model.cfg.n_tokens, n), generator=g, device="cuda",
                         dtype=torch.int32)


def _prefill_state(m):
    from tests.gpuutil import bits

    torch.cuda.synchronize()
    return [bits(t).copy() for b in m.layers for t in (b.attention.kv_cache.k_cache, b.attention.kv_cache.v_cache)
            ] + [bits(m.logits).copy()]


@pytest.mark.gpu
@pytest.mark.parametrize("n,start", [(64, 0), (40, 8)])
def test_chained_norms_equal_the_separate_norm_launches(fresh, monkeypatch, n, start):
    """The prompt's blocks handing each other the next RMSNorm from w2's (and
    wo's) split-K reduce, and wqkv's partial sums going straight to the
    head-norm / rotary / KV kernel, against the same blocks with every norm
    and reduce a launch of its own (`matmul_norm`, `matmul_partials`
    declined): every KV row and the logits bit for bit."""
    import numpy as np

    from ttspipe_amd import nf4gemv

    m = fresh
    toks = _tokens(m, n, 70 + n)
    pos = torch.arange(start, start + n, device="cuda")
    last = torch.tensor([n - 1], device="cuda")
    calls = nf4gemv.stats()["fast"]
    m.prefill_forward(toks, pos, last)
    chained = _prefill_state(m)
    assert nf4gemv.stats()["fast"] > calls
    monkeypatch.setattr(nf4gemv, "matmul_norm", lambda *a, **k: None)
    monkeypatch.setattr(nf4gemv, "matmul_partials", lambda *a, **k: None)
    m.prefill_forward(toks, pos, last)
    separate = _prefill_state(m)
    for i, (a, b) in enumerate(zip(chained, separate)):
        assert np.array_equal(a, b), f"state {i} differs"


@pytest.mark.gpu
@pytest.mark.parametrize("start,n", [(8, 40), (8, 1), (9, 2), (10, 3), (11, 5), (12, 8)])
def test_prompt_prefill_matches_position_by_position_decode(fresh, start, n):
    """Prefill n positions at once (buckets 64, 1, 2, 4, 8, 8: the decode
    block, the two-row GEMV, the few-row kernel), then decode the same
    positions one at a time through the decode kernels: the KV rows and the
    last logits agree."""
    m, cfg = fresh, fresh.cfg
    toks = _tokens(m, n, 1 + n)
    assert m.prefill(toks, start, graphed=False)
    kv = [(b.attention.kv_cache.k_cache[:, :, start:start + n].clone(),
           b.attention.kv_cache.v_cache[:, :, start:start + n].clone()) for b in m.layers]
    logits = m.logits.clone()
    token = int(m.prefill_token.item())
    # the same embeddings, then one position at a time
    rows = torch.clamp(toks.long(), 0, cfg.vocab_size - 1)
    rows = rows + (torch.arange(cfg.n_tokens, device="cuda") * cfg.vocab_size).view(-1, 1)
    emb = m.tensors["embeddings"].view(-1, cfg.dim).index_select(0, rows.reshape(-1))
    emb = emb.view(cfg.n_tokens, n, cfg.dim).float().sum(0).to(m.dtype)
    pos = torch.zeros(1, dtype=torch.long, device="cuda")
    for j in range(n):
        pos.fill_(start + j)
        x = emb[j].view(1, 1, cfg.dim).contiguous()
        for blk in m.layers:
            x = blk(x, m.freqs[start + j].view(1, -1, 2), m.mask, pos)
    m._fused(m.output, x.view(1, 1, -1), m.tensors["norm"], cfg.norm_eps, m.logits)
    for (k0, v0), b in zip(kv, m.layers):
        assert _rel(k0, b.attention.kv_cache.k_cache[:, :, start:start + n]) < 2e-2
        assert _rel(v0, b.attention.kv_cache.v_cache[:, :, start:start + n]) < 2e-2
    assert _rel(logits, m.logits) < 2e-2
    assert token == int(torch.argmax(logits.float()).item())


@pytest.mark.gpu
@pytest.mark.parametrize("start", [5, 0])
@pytest.mark.parametrize("n,bucket", [(100, 128), (1, 1), (2, 2), (3, 4), (6, 8)])
def test_graph_prefill_equals_the_eager_span(fresh, n, bucket, start):
    """One span padded to its bucket: three graph replays, each with eager
    work and synchronisation between them, equal the eager span bit for bit
    (logits, token and the K rows of every layer); at position 0 through the
    graphs whose attention window ends with the span."""
    from ttspipe_amd.dualar import prefill_spans

    m = fresh
    assert prefill_spans(n) == [(0, n, bucket)]
    toks = _tokens(m, n, 2 + n)
    assert m.prefill(toks, start, graphed=False)
    eager = (m.logits.clone(), int(m.prefill_token.item()),
             [b.attention.kv_cache.k_cache[:, :, start:start + n].clone() for b in m.layers])
    m.capture_prefill([bucket], first=start == 0)
    for _ in range(3):
        m.logits.zero_()
        torch.cuda.synchronize()
        assert m.prefill(toks, start, graphed=True)
        torch.cuda.synchronize()
        assert torch.equal(m.logits, eager[0]) and int(m.prefill_token.item()) == eager[1]
        for kc, b in zip(eager[2], m.layers):
            assert torch.equal(kc, b.attention.kv_cache.k_cache[:, :, start:start + n])


@pytest.mark.gpu
def test_prefill_refuses_a_span_padded_past_the_cache(fresh):
    m = fresh
    assert m.cfg.max_seq_len == 320
    before = m.layers[0].attention.kv_cache.k_cache.clone()
    assert not m.prefill(_tokens(m, 300, 3), 0)  # 300 pads to 512 > 320
    assert not m.prefill(_tokens(m, 20, 4), 300)  # 20 pads to 32: 332 > 320
    assert torch.equal(before, m.layers[0].attention.kv_cache.k_cache)


@pytest.fixture(scope="module")
def roomy():
    """The reduced model with a cache long enough for two prompt spans."""
    import dataclasses

    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    return SyntheticDualAR(dataclasses.replace(SMALL, max_seq_len=1280))


def _kv_state(m, upto):
    return [(b.attention.kv_cache.k_cache[:, :, :upto].clone(), b.attention.kv_cache.v_cache[:, :, :upto].clone())
            for b in m.layers]


def _set_kv(m, state):
    for b, (k, v) in zip(m.layers, state):
        b.attention.kv_cache.k_cache[:, :, :k.shape[2]].copy_(k)
        b.attention.kv_cache.v_cache[:, :, :v.shape[2]].copy_(v)


def _assert_same_prefill(m, eager, upto):
    for i, ((k0, v0), (k1, v1)) in enumerate(zip(eager["kv"], _kv_state(m, upto))):
        assert torch.equal(k0, k1) and torch.equal(v0, v1), f"layer {i} KV rows differ from the eager prefill"
    assert torch.equal(m.logits, eager["logits"]) and int(m.prefill_token.item()) == eager["token"]


@pytest.mark.gpu
def test_graphed_prefill_captures_buckets_without_touching_live_kv(roomy):
    """A 600-token prompt with no bucket captured beforehand: the first span
    (at position 0) takes its own window's 512 graph; the second span's
    bucket (128) is captured after the first span's KV rows are written, and
    its warm-up runs at positions 0..127; the result must equal the eager
    prefill, KV rows and logits bit for bit."""
    m = roomy
    m.prefill_graphs.clear()
    m.prefill_first_graphs.clear()
    initial = _kv_state(m, m.cfg.max_seq_len)
    toks = _tokens(m, 600, 5)
    assert m.prefill(toks, 0, graphed=False)
    torch.cuda.synchronize()
    eager = {"kv": _kv_state(m, 600), "logits": m.logits.clone(), "token": int(m.prefill_token.item())}
    _set_kv(m, initial)
    assert m.prefill(toks, 0, graphed=True)
    torch.cuda.synchronize()
    # (the span at position 0 takes the graph whose window ends with it)
    assert sorted(m.prefill_first_graphs) == [512] and sorted(m.prefill_graphs) == [128]
    _assert_same_prefill(m, eager, 600)


@pytest.mark.gpu
def test_graphed_prefill_after_an_eager_one_keeps_its_context(roomy):
    """An eager 64-token prompt at position 0, then 100 more tokens graphed at
    position 64 whose bucket is captured on the spot: the first prompt's KV
    rows survive the capture and the continuation equals the all-eager run."""
    m = roomy
    m.prefill_graphs.clear()
    initial = _kv_state(m, m.cfg.max_seq_len)
    head, tail = _tokens(m, 64, 6), _tokens(m, 100, 7)
    assert m.prefill(head, 0, graphed=False) and m.prefill(tail, 64, graphed=False)
    torch.cuda.synchronize()
    eager = {"kv": _kv_state(m, 164), "logits": m.logits.clone(), "token": int(m.prefill_token.item())}
    _set_kv(m, initial)
    assert m.prefill(head, 0, graphed=False) and m.prefill(tail, 64, graphed=True)
    torch.cuda.synchronize()
    assert 128 in m.prefill_graphs
    _assert_same_prefill(m, eager, 164)


@pytest.mark.gpu
def test_first_span_window_matches_the_whole_cache_window(roomy):
    """A 300-token prompt at position 0 through the window that ends with the
    span (the default there) and through the whole-cache window: the keys past
    the span are masked either way, so the KV rows and the last logits agree
    within the reference's 2e-2 block bar (the attention's key split differs
    with the window, and with it the roundings); layer 0's K/V rows, written
    before any attention, are identical."""
    import numpy as np

    m = roomy
    toks = _tokens(m, 300, 9)
    initial = _kv_state(m, m.cfg.max_seq_len)
    got = {}
    for name, width in (("span", 512), ("cache", None)):
        _set_kv(m, initial)
        inp = torch.empty(m.cfg.n_tokens, 512, dtype=torch.int32, device=m.device)
        inp[:, :300].copy_(toks)
        inp[:, 300:].copy_(toks[:, -1:].expand(-1, 212))
        pos = torch.arange(512, dtype=torch.long, device=m.device)
        last = torch.tensor([299], dtype=torch.long, device=m.device)
        m.prefill_forward(inp, pos, last, width)
        torch.cuda.synchronize()
        got[name] = (m.logits.float().cpu().numpy(), _kv_state(m, 300))
    (la, kva), (lb, kvb) = got["span"], got["cache"]
    assert np.linalg.norm(la - lb) / np.linalg.norm(lb) < 2e-2
    assert torch.equal(kva[0][0], kvb[0][0]) and torch.equal(kva[0][1], kvb[0][1])
    for (ka, va), (kb, vb) in zip(kva, kvb):
        for a, b in ((ka, kb), (va, vb)):
            a, b = a.float(), b.float()
            assert float((a - b).norm() / b.norm()) < 2e-2
    _set_kv(m, initial)
