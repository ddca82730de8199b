"""The multi-position (prompt prefill) block and the Dual-AR prompt prefill
with its bucket graphs (GPU), plus the span arithmetic (CPU).

Bar: the fused prefill block against the block's own unpatched forward
(the same GEMMs, the epilogues keep the unfused roundings; the head norms
run in the decode step's kernel instead of the fork's torch modules), at the
reference's block bar rel-norm < 2e-2 (tests/test_nf4cpu.py:175-191), V rows
identical; the many-row head-norm/rotary/KV kernel bit for bit against the
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
    assert prefill_spans(1) == [(0, 1, PREFILL_BUCKETS[0])]
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


@pytest.fixture(scope="module")
def fresh():
    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    return SyntheticDualAR(SMALL)


def _tokens(model, n, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randint(0, model.cfg.codebook_size, (model.cfg.n_tokens, n), generator=g, device="cuda",
                         dtype=torch.int32)


@pytest.mark.gpu
def test_prompt_prefill_matches_position_by_position_decode(fresh):
    """Prefill 40 positions at once, then decode the same positions one at a
    time through the decode kernels: the KV rows and the last logits agree."""
    m, cfg = fresh, fresh.cfg
    start, n = 8, 40
    toks = _tokens(m, n, 1)
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
def test_graph_prefill_equals_the_eager_span(fresh):
    m = fresh
    toks = _tokens(m, 100, 2)  # one span, padded to the 128 bucket
    assert m.prefill(toks, 0, graphed=False)
    eager = (m.logits.clone(), int(m.prefill_token.item()),
             [b.attention.kv_cache.k_cache[:, :, :100].clone() for b in m.layers])
    m.capture_prefill([128])
    for _ in range(3):
        m.logits.zero_()
        torch.cuda.synchronize()
        assert m.prefill(toks, 0, graphed=True)
        torch.cuda.synchronize()
        assert torch.equal(m.logits, eager[0]) and int(m.prefill_token.item()) == eager[1]
        for kc, b in zip(eager[2], m.layers):
            assert torch.equal(kc, b.attention.kv_cache.k_cache[:, :, :100])


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
    """A 600-token prompt with no bucket captured beforehand: the second span's
    bucket (128) is captured after the first span's KV rows are written, and
    its warm-up runs at positions 0..127; the result must equal the eager
    prefill, KV rows and logits bit for bit."""
    m = roomy
    m.prefill_graphs.clear()
    initial = _kv_state(m, m.cfg.max_seq_len)
    toks = _tokens(m, 600, 5)
    assert m.prefill(toks, 0, graphed=False)
    torch.cuda.synchronize()
    eager = {"kv": _kv_state(m, 600), "logits": m.logits.clone(), "token": int(m.prefill_token.item())}
    _set_kv(m, initial)
    assert m.prefill(toks, 0, graphed=True)
    torch.cuda.synchronize()
    assert sorted(m.prefill_graphs) == [128, 512]
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
