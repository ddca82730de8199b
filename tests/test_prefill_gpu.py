"""Prefill attention (`fastpath.prefill_attention`, one HIP launch) against
fp64 attention on the CPU and against the reference's formula
(`fastpath.decode_attention`, app/engine/fastpath.py:133-174) on the GPU.

Bar: a floating-point kernel (scores on the matrix cores, probabilities
rounded to the activation type before the second product), so within 5e-3
of fp64 in the reference's measure, max |got - ref| / max |ref| (the bar of
the decode attention, tests/test_nf4gemv.py:224-242), and within twice that
of the reference's own bf16/fp16 result; NaN exactly where the reference's
softmax gives NaN (a row with no allowed key).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.conftest import relative_error

pytestmark = pytest.mark.gpu

TOL = 5e-3
D = 128


def _setup(S, prefix, nh, nkv, dtype, max_len=None, seed=0):
    """q as `llama.Attention` hands it over (a transposed view of the wqkv
    output), k/v as the KV cache sliced to the live length L = prefix + S, and
    the fork's mask: rows input_pos of tril(max_len), cut to L."""
    L = prefix + S
    max_len = max_len or ((L + 255) // 256) * 256
    g = torch.Generator().manual_seed(seed)
    total = (nh + 2 * nkv) * D
    qkv = torch.randn(1, S, total, generator=g).to(dtype).cuda()
    q = qkv[..., : nh * D].view(1, S, nh, D).transpose(1, 2)
    kc = torch.zeros(1, nkv, max_len, D, dtype=dtype, device="cuda")
    vc = torch.zeros_like(kc)
    kc[:, :, :L] = torch.randn(1, nkv, L, D, generator=g).to(dtype).cuda()
    vc[:, :, :L] = torch.randn(1, nkv, L, D, generator=g).to(dtype).cuda()
    causal = torch.tril(torch.ones(max_len, max_len, dtype=torch.bool, device="cuda"))
    pos = torch.arange(prefix, L, device="cuda")
    mask = causal[None, None, pos, :max_len][..., :L]
    return q, kc[:, :, :L], vc[:, :, :L], mask


def _fp64(q, k, v, mask):
    """Exact attention: q (1, nh, S, D), k/v (1, nkv, L, D), mask (1, 1, S, L)."""
    qn = q[0].double().cpu().numpy()
    kn, vn = k[0].double().cpu().numpy(), v[0].double().cpu().numpy()
    m = mask[0, 0].cpu().numpy()
    nh, nkv = qn.shape[0], kn.shape[0]
    out = np.empty_like(qn)
    for hd in range(nh):
        kv = hd // (nh // nkv)
        s = qn[hd] @ kn[kv].T * D**-0.5
        s = np.where(m, s, -np.inf)
        with np.errstate(invalid="ignore"):
            p = np.exp(s - s.max(axis=1, keepdims=True))
            out[hd] = (p / p.sum(axis=1, keepdims=True)) @ vn[kv]
    return out


def _run(q, k, v, mask, nh, nkv):
    from ttspipe_amd import fastpath

    before = fastpath.stats()["prefill_attn"]
    y = fastpath.prefill_attention(q, k, v, mask, nh, nkv, D)
    assert y is not None, "declined"
    assert fastpath.stats()["prefill_attn"] == before + 1
    assert y.shape == q.shape and y.dtype == q.dtype
    assert y.transpose(1, 2).is_contiguous()
    return y


CASES = [  # (S, prefix, nh, nkv)
    (512, 0, 32, 8),      # the 512-token prompt prefill of the 4B-dim layer
    (512, 1536, 32, 8),   # the same after a cached prefix
    (64, 0, 32, 8),       # the reference's largest decode_attention prefill
    (7, 0, 4, 2),         # the test block of the reference (4 q / 2 kv heads)
    (33, 100, 8, 2),      # ragged: S and L off every tile size
    (1, 300, 32, 8),      # one position (a declined decode step)
    (100, 0, 16, 16),     # one query head per kv head
    (65, 5, 8, 1),        # eight query heads per kv head
    (200, 2900, 8, 2),    # the fast transformer's head shape over a long cache
    (64, 2000, 32, 8),    # a short run over a long cached prefix: keys split over workgroups
    (16, 3000, 8, 2),     # the same with the fast transformer's heads (16 splits)
]


@pytest.mark.parametrize("S,prefix,nh,nkv", CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_prefill_attention_matches_fp64_and_the_reference_formula(S, prefix, nh, nkv, dtype):
    from ttspipe_amd.fastpath import decode_attention

    q, k, v, mask = _setup(S, prefix, nh, nkv, dtype, seed=S + prefix + nh)
    y = _run(q, k, v, mask, nh, nkv)
    exact = _fp64(q, k, v, mask)
    got = y[0].float().cpu().numpy()
    assert np.isfinite(got).all()
    assert relative_error(got, exact) < TOL
    # the reference's formula rounds its own output to the activation type: two
    # results each within TOL of fp64 lie within 2 TOL of each other
    theirs = decode_attention(q, k, v, mask, nh, nkv, D)[0].float().cpu().numpy()
    assert relative_error(theirs, exact) < TOL
    assert relative_error(got, theirs) < 2 * TOL


def test_arbitrary_mask_and_rows_with_no_key():
    """Any boolean mask (not only causal), including rows that allow no key:
    NaN there, as the reference's softmax; every other row exact to the bar."""
    S, L, nh, nkv = 70, 90, 8, 2
    q, k, v, _ = _setup(S, L - S, nh, nkv, torch.bfloat16, seed=5)
    g = torch.Generator().manual_seed(9)
    store = torch.rand(S, 96, generator=g) < 0.3  # row stride 96: 16-byte rows, cut to L
    store[3] = False
    store[40, :] = False
    store[40, 89] = True  # only the last key
    mask = store.cuda()[None, None, :, :L]
    y = _run(q, k, v, mask, nh, nkv)[0].float().cpu().numpy()
    exact = _fp64(q, k, v, mask)
    assert np.isnan(y[:, 3]).all()
    keep = [i for i in range(S) if i != 3]
    assert np.isfinite(y[:, keep]).all()
    assert relative_error(y[:, keep], exact[:, keep]) < TOL


def _split_call(q, k, v, mask, nh, nkv, splits):
    from ttspipe_amd import _lib
    from ttspipe_amd.fastpath import prefill_work_floats

    S, L = q.shape[2], k.shape[2]
    out = torch.full((1, S, nh * D), 7.0, dtype=q.dtype, device="cuda")
    work = torch.full((max(prefill_work_floats(S, nh, splits), 4),), float("nan"), device="cuda")
    rc = _lib.load().ttsp_prefill_attention_split(
        q.data_ptr(), q.stride(2), q.stride(1), k.data_ptr(), k.stride(2), k.stride(1), v.data_ptr(), v.stride(2),
        v.stride(1), mask.data_ptr(), mask.stride(2), out.data_ptr(), S, nh, nkv, L, D**-0.5,
        _lib.dtype_code(q.dtype), work.data_ptr(), splits, _lib.stream())
    assert rc == 0
    torch.cuda.synchronize()
    return out.view(1, S, nh, D).transpose(1, 2)[0].float().cpu().numpy()


@pytest.mark.parametrize("S,prefix,nh,nkv", [(64, 2000, 32, 8), (40, 0, 8, 2), (100, 900, 16, 2), (5, 300, 8, 8)])
def test_any_key_split_gives_the_unsplit_result(S, prefix, nh, nkv):
    """Splits 1, 2, 3, 7 and 16 of the keys: every split count (also ones
    the plan never picks, and splits left with no allowed key by the causal
    mask) within the bar of fp64. The probabilities are rounded relative to a
    different running max in each split, so two split counts agree to twice
    the bar."""
    q, k, v, mask = _setup(S, prefix, nh, nkv, torch.bfloat16, seed=11 + S)
    exact = _fp64(q, k, v, mask)
    one = _split_call(q, k, v, mask, nh, nkv, 1)
    assert relative_error(one, exact) < TOL
    for sp in (2, 3, 7, 16):
        got = _split_call(q, k, v, mask, nh, nkv, sp)
        assert np.isfinite(got).all(), sp
        assert relative_error(got, exact) < TOL, sp
        assert relative_error(got, one) < 2 * TOL, sp  # each within TOL of fp64


@pytest.mark.parametrize("S,prefix", [(64, 1500), (512, 0), (200, 700)])
def test_key_split_over_the_whole_cache_splits_the_live_keys(S, prefix):
    """K/V and the mask over the whole cache (4096 positions), as a captured
    prefill passes them, the mask cutting the keys to the live prefix: the
    splits divide the keys the mask allows, and the result keeps the bar."""
    from ttspipe_amd import _lib

    nh, nkv, max_len = 32, 8, 4096
    q, k, v, _ = _setup(S, prefix, nh, nkv, torch.bfloat16, max_len=max_len, seed=S + 1)
    kc, vc = k.new_zeros(1, nkv, max_len, D), v.new_zeros(1, nkv, max_len, D)
    kc[:, :, : prefix + S], vc[:, :, : prefix + S] = k, v
    kc[:, :, prefix + S :] = 1e4  # keys past the live length carry huge values: the mask must cut them
    causal = torch.tril(torch.ones(max_len, max_len, dtype=torch.bool, device="cuda"))
    mask = causal[None, None, torch.arange(prefix, prefix + S, device="cuda")]
    assert _lib.load().ttsp_prefill_attention_splits(S, nkv, max_len) > 1
    y = _run(q, kc, vc, mask, nh, nkv)[0].float().cpu().numpy()
    exact = _fp64(q, k, v, mask[..., : prefix + S])
    assert np.isfinite(y).all()
    assert relative_error(y, exact) < TOL


def test_key_split_rows_with_no_key_are_nan():
    S, L, nh, nkv = 40, 600, 8, 2
    q, k, v, _ = _setup(S, L - S, nh, nkv, torch.float16, seed=4)
    g = torch.Generator().manual_seed(2)
    store = torch.rand(S, 608, generator=g) < 0.05
    store[7] = False
    store[20, :] = False
    store[20, 599] = True  # only the last key (the last split)
    store[21, :] = False
    store[21, 0] = True  # only the first key (the first split)
    mask = store.cuda()[None, None, :, :L]
    exact = _fp64(q, k, v, mask)
    for sp in (4, 16):
        y = _split_call(q, k, v, mask, nh, nkv, sp)
        assert np.isnan(y[:, 7]).all()
        keep = [i for i in range(S) if i != 7]
        assert np.isfinite(y[:, keep]).all()
        assert relative_error(y[:, keep], exact[:, keep]) < TOL


def test_declines_what_it_does_not_take():
    from ttspipe_amd import fastpath

    q, k, v, mask = _setup(40, 8, 8, 2, torch.bfloat16)
    before = fastpath.stats()["prefill_declined"]
    assert fastpath.prefill_attention(q.float(), k.float(), v.float(), mask, 8, 2, D) is None
    assert fastpath.prefill_attention(q, k, v, None, 8, 2, D) is None
    assert fastpath.prefill_attention(q[..., :64], k[..., :64], v[..., :64], mask, 8, 2, 64) is None
    loose = mask.contiguous()[..., :47].contiguous()  # 48 keys cut to 47: row stride 47
    assert fastpath.prefill_attention(q, k[:, :, :47], v[:, :, :47], loose, 8, 2, D) is None
    q16, k16, v16, m16 = _setup(40, 8, 32, 2, torch.bfloat16)  # 16 query heads per kv head
    assert fastpath.prefill_attention(q16, k16, v16, m16, 32, 2, D) is None
    assert fastpath.stats()["prefill_declined"] == before + 5


def test_rejected_arguments_return_an_error():
    from ttspipe_amd import _lib

    hip, st = _lib.load(), _lib.stream()
    buf = torch.zeros(1 << 16, dtype=torch.bfloat16, device="cuda")
    p = buf.data_ptr()
    ok = dict(S=4, nh=8, nkv=2, L=16)
    bad = [dict(ok, nh=7), dict(ok, nh=32, nkv=2), dict(ok, S=0), dict(ok, L=0), dict(ok, L=100)]
    for a in bad:  # L=100 exceeds the mask row stride of 64
        rc = hip.ttsp_prefill_attention(p, 1024, 128, p, 256, 4096, p, 256, 4096, p, 64, p, a["S"], a["nh"],
                                        a["nkv"], a["L"], 0.088, 1, st)
        assert rc != 0, a
    rc = hip.ttsp_prefill_attention(p + 2, 1024, 128, p, 256, 4096, p, 256, 4096, p, 64, p, 4, 8, 2, 16, 0.088,
                                    1, st)
    assert rc != 0  # misaligned Q
    rc = hip.ttsp_prefill_attention(p, 1024, 128, p, 256, 4096, p, 256, 4096, p, 40, p, 4, 8, 2, 16, 0.088, 1,
                                    st)
    assert rc != 0  # mask rows not 16-byte aligned
    torch.cuda.synchronize()


def test_captured_in_a_graph_replays_identically():
    from ttspipe_amd import fastpath

    q, k, v, mask = _setup(96, 40, 8, 2, torch.bfloat16, seed=3)
    out = torch.empty(1, 96, 8 * D, dtype=torch.bfloat16, device="cuda")
    eager = fastpath.prefill_attention(q, k, v, mask, 8, 2, D).clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fastpath.prefill_attention(q, k, v, mask, 8, 2, D, out=out)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(1, 96, 8, D).transpose(1, 2), eager)


def test_key_split_captured_in_a_graph_replays_identically():
    from ttspipe_amd import _lib, fastpath

    S, prefix, nh, nkv = 64, 2000, 32, 8
    assert _lib.load().ttsp_prefill_attention_splits(S, nkv, S + prefix) > 1
    q, k, v, mask = _setup(S, prefix, nh, nkv, torch.bfloat16, seed=6)
    out = torch.empty(1, S, nh * D, dtype=torch.bfloat16, device="cuda")
    work = torch.empty(fastpath.prefill_work_floats(S, nh, 16), device="cuda")
    eager = fastpath.prefill_attention(q, k, v, mask, nh, nkv, D).clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fastpath.prefill_attention(q, k, v, mask, nh, nkv, D, out=out, work=work)
    for _ in range(3):
        out.zero_()
        work.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(1, S, nh, D).transpose(1, 2), eager)


def test_attention_forward_takes_the_kernel_for_a_prefill():
    """`llama.Attention.forward` over 40 new positions after 24 cached ones:
    the HIP prefill attention runs, and the layer output (after wo) agrees
    with the same layer run through the reference's formula."""
    from ttspipe_amd import fastpath
    from ttspipe_amd.llama import Attention, BaseModelArgs, KVCache, precompute_freqs_cis
    from tests.nf4data import random_layer, to_linear

    torch.manual_seed(0)
    args = BaseModelArgs(dim=512, n_head=4, n_local_heads=2, head_dim=128, intermediate_size=1024,
                         attention_qk_norm=True)
    att = Attention(args, dtype=torch.bfloat16, device="cuda")
    att.wqkv = to_linear(random_layer(8 * 128, 512, True, seed=1), torch.bfloat16)
    att.wo = to_linear(random_layer(512, 4 * 128, True, seed=2), torch.bfloat16)
    max_len = 128
    att.kv_cache = KVCache(1, max_len, 2, 128, dtype=torch.bfloat16, device="cuda")
    att.kv_cache.k_cache.normal_()
    att.kv_cache.v_cache.normal_()
    freqs = precompute_freqs_cis(max_len, 128, 1e6).cuda()
    pos = torch.arange(24, 64, device="cuda")
    causal = torch.tril(torch.ones(max_len, max_len, dtype=torch.bool, device="cuda"))
    mask = causal[None, None, pos][..., :64]
    x = torch.randn(1, 40, 512, dtype=torch.bfloat16, device="cuda")
    saved = (att.kv_cache.k_cache.clone(), att.kv_cache.v_cache.clone())
    before = fastpath.stats()["prefill_attn"]
    ours = att(x, freqs[pos], mask, pos)
    assert fastpath.stats()["prefill_attn"] == before + 1
    att.kv_cache.k_cache.copy_(saved[0])
    att.kv_cache.v_cache.copy_(saved[1])
    orig = fastpath.prefill_attention
    fastpath.prefill_attention = lambda *a, **kw: None
    try:
        theirs = att(x, freqs[pos], mask, pos)
    finally:
        fastpath.prefill_attention = orig
    # the layer-level bar of the reference's prefill block test, rel-norm < 2e-2
    # (tests/test_nf4cpu.py:175-191): the attention outputs differ by bf16
    # roundings, which wo then mixes
    rel = ((ours.float() - theirs.float()).norm() / theirs.float().norm()).item()
    assert rel < 2e-2


CAUSAL_CASES = [  # (S, prefix, nh, nkv, window past the span): the masked kernel's own shapes
    (512, 0, 32, 8, 0),       # the 512-token prompt, its window ending with the span (four key splits)
    (480, 0, 32, 8, 0),       # 120 (kv head, query block) pairs: the two-split form, bit for bit
    (512, 0, 32, 8, 1792),    # the same over the whole cache (2304 positions)
    (512, 1536, 32, 8, 0),    # after a cached prefix: two key splits
    (64, 2000, 32, 8, 0),     # a short run over a long prefix: 16 key splits
    (100, 37, 8, 2, 5),       # ragged query and key blocks
    (33, 0, 6, 2, 0),         # three heads per kv head (one key split a workgroup)
    (9, 3, 8, 1, 40),         # eight heads per kv head
    (1, 0, 4, 4, 0),          # one row, one key
]


@pytest.mark.parametrize("S,prefix,nh,nkv,extra", CAUSAL_CASES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_causal_positions_equal_the_causal_mask_bit_for_bit(S, prefix, nh, nkv, extra, dtype):
    """`positions=` (the mask computed from the rows' positions in the kernel)
    against the masked kernel with the fork's causal rows at those positions,
    which it must equal bit for bit (the same keys masked, the same blocks
    taken whole) where both take the same key splits, and against fp64."""
    from ttspipe_amd import _lib, fastpath

    L = prefix + S + extra
    q, k, v, _ = _setup(S, prefix, nh, nkv, dtype, seed=S + prefix + extra)
    g = torch.Generator().manual_seed(L)
    kc, vc = (torch.randn(1, nkv, L, D, generator=g).to(dtype).cuda() for _ in "kv")
    kc[:, :, : prefix + S], vc[:, :, : prefix + S] = k, v
    Lp = (L + 255) // 256 * 256  # the masked kernel takes 16-byte aligned mask rows
    causal = torch.tril(torch.ones(Lp, Lp, dtype=torch.bool, device="cuda"))
    pos = torch.arange(prefix, prefix + S, device="cuda")
    mask = causal[None, None, pos, :Lp][..., :L]
    masked = _run(q, kc, vc, mask, nh, nkv)
    got = fastpath.prefill_attention(q, kc, vc, None, nh, nkv, D, positions=pos)
    assert got is not None
    exact = _fp64(q, kc, vc, mask)
    assert relative_error(got[0].float().cpu().numpy(), exact) < TOL
    splits = _lib.load().ttsp_prefill_attention_splits(S, nkv, L)
    if nh == 4 * nkv and splits == 1 and nkv * -(-S // 32) >= 128:
        # four key splits a workgroup: the same attention, merged in another order
        assert relative_error(got[0].float().cpu().numpy(), masked[0].float().cpu().numpy()) < 2 * TOL
    else:
        assert torch.equal(got.view(torch.int16), masked.view(torch.int16))


def test_causal_positions_in_any_order_and_past_the_window():
    """Rows need not be consecutive: each row's own position sets its keys
    (positions at or past L allow every key), bit for bit the mask that
    states the same."""
    from ttspipe_amd import fastpath

    S, nh, nkv, L = 80, 8, 2, 300
    q, _, _, _ = _setup(S, 0, nh, nkv, torch.bfloat16, seed=11)
    g = torch.Generator().manual_seed(12)
    k = torch.randn(1, nkv, L, D, generator=g).to(torch.bfloat16).cuda()
    v = torch.randn(1, nkv, L, D, generator=g).to(torch.bfloat16).cuda()
    pos = torch.randint(0, L + 40, (S,), generator=g).cuda()
    mask = (torch.arange(L + 20, device="cuda")[None, :] <= pos[:, None])[None, None, :, :L]  # 16-byte rows
    masked = _run(q, k, v, mask, nh, nkv)
    got = fastpath.prefill_attention(q, k, v, None, nh, nkv, D, positions=pos)
    assert torch.equal(got.view(torch.int16), masked.view(torch.int16))


def test_causal_positions_declines_and_argument_checks():
    from ttspipe_amd import _lib, fastpath

    q, k, v, mask = _setup(16, 4, 8, 2, torch.bfloat16)
    pos = torch.arange(4, 20, device="cuda")
    assert fastpath.prefill_attention(q, k, v, None, 8, 2, D, positions=pos.int()) is None
    assert fastpath.prefill_attention(q, k, v, None, 8, 2, D, positions=pos[:15]) is None
    assert fastpath.prefill_attention(q, k, v, None, 8, 2, D, positions=pos.cpu()) is None
    assert fastpath.prefill_attention(q, k, v, None, 8, 2, D) is None
    hip = _lib.load()
    p = q.data_ptr()
    rc = hip.ttsp_prefill_attention_causal(p, 1024, 128, p, 256, 4096, p, 256, 4096, None, p, 16, 8, 2, 20, 0.088, 1,
                                           None, 1, None)
    assert rc != 0


def test_causal_positions_captured_in_a_graph_replay_identically():
    from ttspipe_amd import fastpath

    for S, prefix in ((96, 40), (64, 2000)):
        q, k, v, _ = _setup(S, prefix, 32, 8, torch.bfloat16, seed=5)
        pos = torch.arange(prefix, prefix + S, device="cuda")
        out = torch.empty(1, S, 32 * D, dtype=torch.bfloat16, device="cuda")
        work = torch.empty(fastpath.prefill_work_floats(S, 32, 16), device="cuda")
        eager = fastpath.prefill_attention(q, k, v, None, 32, 8, D, positions=pos).clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fastpath.prefill_attention(q, k, v, None, 32, 8, D, out=out, work=work, positions=pos)
        for _ in range(3):
            out.zero_()
            work.zero_()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out.view(1, S, 32, D).transpose(1, 2), eager)
