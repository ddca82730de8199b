"""Greedy Dual-AR decode on the GPU against the oracle's restatement (GPU).

Bar: token ids identical, every frame (the benchmark's acceptance rule), and
the logits and KV rows each frame writes identical bit for bit. The reduced
model runs 256 frames against the oracle live; the benchmark model (36 slow
layers, KV prefilled to 2048) runs 256 frames against a fixture the oracle
wrote on the CPU (tests/golden/make_dualar_c5.py), plus run-to-run
determinism.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpuutil import bits, gemv_shape

pytestmark = pytest.mark.gpu


def _oracle(model):
    from oracle.dualar_oracle import OracleDualAR
    from ttspipe_amd.quant import create_dynamic_map

    return OracleDualAR(model.cfg, (model.specs["linears"], model.specs["vectors"], model.specs["caches"]),
                        lambda M, K: gemv_shape(M, K)[:2], code2=create_dynamic_map().numpy(),
                        freqs_bits=bits(model.freqs), fast_freqs_bits=bits(model.fast_freqs))


@pytest.fixture(scope="module")
def small():
    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    return SyntheticDualAR(SMALL)


def test_synthetic_weights_match_the_oracle_bytes(small, orc):
    """The device fill and the CPU fill give the same bytes (spot check of
    each kind: packed codes, scale indices, fp32 absmax2, bf16 vectors)."""
    lin = small.specs["linears"][0]
    packed, state = small.quant[lin.name]
    assert np.array_equal(packed.view(-1).cpu().numpy(), orc.synth_fill(lin.packed.n, lin.packed.seed, 0))
    assert np.array_equal(state.absmax.cpu().numpy(), orc.synth_fill(lin.a8.n, lin.a8.seed, 0))
    s = lin.absmax2
    assert np.array_equal(state.state2.absmax.cpu().numpy(), orc.synth_fill(s.n, s.seed, 3, s.scale, s.offset))
    v = small.specs["vectors"][0]
    assert np.array_equal(bits(small.tensors[v.name]), orc.synth_fill(v.n, v.seed, 1, v.scale, v.offset))


def test_small_model_256_greedy_frames_match_the_oracle(small):
    from ttspipe_amd.dualar import first_tokens

    cfg = small.cfg
    got = small.decode(256, graphed=True)
    ref = _oracle(small).decode(first_tokens(cfg), cfg.prefill_len, 256)
    assert got.shape == ref.shape == (256, cfg.n_tokens)
    diff = np.flatnonzero((got != ref).any(axis=1))
    assert diff.size == 0, f"first differing frame {diff[0]}: gpu {got[diff[0]]} oracle {ref[diff[0]]}"
    assert len({tuple(r) for r in got}) > 1, "the decode should not be stuck on one frame"


def test_small_model_graph_replay_equals_eager_steps(small):
    eager = small.decode(12, graphed=False)
    graphed = small.decode(12, graphed=True)
    assert np.array_equal(eager, graphed)


def _digest(t) -> str:
    import hashlib

    return hashlib.sha256(np.ascontiguousarray(bits(t)).tobytes()).hexdigest()


def test_benchmark_model_256_frames_match_the_oracle_fixture():
    """The benchmark model (36 slow layers at d=2560, KV prefilled to position
    2048) against the fixture the oracle wrote on the CPU
    (tests/golden/make_dualar_c5.py): for all 256 greedy frames the token
    column, the slow head's logits and the last codebook step's logits, bit
    for bit, and the K/V rows three layers wrote at three frames. The fixture
    records the GEMV launch split of every shape (it fixes the summation
    order the oracle reproduced) and the rotary tables; a library whose plan
    changed fails here first, instead of comparing against stale numbers.
    Then the same 256 frames again: identical (no atomics, fixed orders)."""
    import json
    from pathlib import Path

    from ttspipe_amd.dualar import DualARConfig, SyntheticDualAR, first_tokens

    fx = json.loads((Path(__file__).parent / "golden" / "dualar_c5_tokens.json").read_text())
    cfg = DualARConfig()
    assert fx["config"] == {k: getattr(cfg, k) for k in cfg.__dataclass_fields__}
    assert fx["first_tokens"] == list(first_tokens(cfg)) and fx["position0"] == cfg.prefill_len
    for key, (J, KS) in fx["gemv_shapes"].items():
        M, K = map(int, key.split("x"))
        assert gemv_shape(M, K)[:2] == (J, KS), f"the GEMV plan for {key} changed: regenerate the fixture"
    model = SyntheticDualAR(cfg)
    assert _digest(model.freqs) == fx["freqs_sha256"] and _digest(model.fast_freqs) == fx["fast_freqs_sha256"]
    n = fx["frames"]
    assert n == 256
    model.capture()
    model.reset(n)
    slow, fast = [], []
    for _ in range(n):
        model.graph.replay()
        slow.append(_digest(model.logits))
        fast.append(_digest(model.fast_logits))
    torch.cuda.synchronize()
    got = model.history[:n].cpu().numpy()
    ref = np.asarray(fx["tokens"], np.int32)
    diff = np.flatnonzero((got != ref).any(axis=1))
    assert diff.size == 0, f"{diff.size} frames differ, first {diff[0]}: gpu {got[diff[0]]} oracle {ref[diff[0]]}"
    bad = [f for f in range(n) if slow[f] != fx["slow_logits_sha256"][f]]
    assert not bad, f"slow-head logits differ at {len(bad)} frames, first {bad[0]}"
    bad = [f for f in range(n) if fast[f] != fx["last_fast_logits_sha256"][f]]
    assert not bad, f"last codebook logits differ at {len(bad)} frames, first {bad[0]}"
    p0 = cfg.prefill_len
    for key, ref_digest in fx["kv_rows_sha256"].items():
        which, layer, frame = key.split(".")
        c = getattr(model.layers[int(layer)].attention.kv_cache, f"{which}_cache")
        assert _digest(c[0, :, p0 + int(frame)]) == ref_digest, f"{which} rows of layer {layer} at frame {frame}"
    again = model.decode(n, graphed=True)
    assert np.array_equal(again, got)
    del model
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n,vocab,D", [(4096, 4096, 1024), (4096, 1024, 1024), (700, 4096, 1000), (1, 8, 64),
                                       (40000, 4096, 2560)])
def test_argmax_embed_equals_argmax_then_embed(dtype, n, vocab, D):
    """ttsp_argmax_embed == ttsp_argmax then a one-row ttsp_embed_sum, bit for
    bit: ties (the lowest index), the winner past the table (clamped), -0.0
    entries of the table (0 + -0 rounds to +0, as embed_sum), every row
    element."""
    from ttspipe_amd import _lib

    lib, st = _lib.lib(), _lib.stream()
    dt = _lib.dtype_code(dtype)
    g = torch.Generator(device="cuda").manual_seed(n + vocab)
    for case in range(4):
        x = torch.randn(n, device="cuda", generator=g).to(dtype)
        if case == 1:  # a tie of the maximum at two indices
            top = x.max()
            x[n // 3] = top
            x[n // 2] = top
        if case == 2:  # the winner past the table
            x[n - 1] = 100.0
        E = torch.randn(vocab, D, device="cuda", generator=g).to(dtype)
        E[:, ::7] = -0.0
        tok = torch.full((2,), -5, dtype=torch.int32, device="cuda")
        ref_tok = torch.full((2,), -5, dtype=torch.int32, device="cuda")
        out = torch.empty(D, dtype=dtype, device="cuda")
        ref = torch.empty(D, dtype=dtype, device="cuda")
        _lib.check(lib.ttsp_argmax_embed(x.data_ptr(), n, dt, tok.data_ptr(), tok[1:].data_ptr(), E.data_ptr(), vocab,
                                         D, out.data_ptr(), st), "argmax_embed")
        _lib.check(lib.ttsp_argmax(x.data_ptr(), n, dt, ref_tok.data_ptr(), st), "argmax")
        torch.clamp(ref_tok[:1], 0, vocab - 1, out=ref_tok[1:2])
        _lib.check(lib.ttsp_embed_sum(E.data_ptr(), ref_tok[1:].data_ptr(), 1, vocab, D, ref.data_ptr(), dt, st),
                   "embed_sum")
        assert torch.equal(tok, ref_tok), (case, tok.tolist(), ref_tok.tolist())
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), case
        top = x.float().max()
        assert int(tok[0]) == int((x.float() == top).nonzero()[0])  # the lowest index holding the maximum


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 7, 8, 9, 4096, 4103, 32768, 40000])
@pytest.mark.parametrize("offset", [0, 1, 3])
def test_argmax_is_the_lowest_index_of_the_maximum(dtype, n, offset):
    """ttsp_argmax against torch: the lowest index holding the maximum, with
    ties inside one 8-value chunk and across chunks and threads, NaN entries
    (never chosen), an all -inf row (index 0), lengths off the chunk size and
    logits that do not start 16-byte aligned (offset values in)."""
    from ttspipe_amd import _lib

    lib, st = _lib.lib(), _lib.stream()
    dt = _lib.dtype_code(dtype)
    g = torch.Generator(device="cuda").manual_seed(n * 3 + offset)
    for case in range(5):
        base = torch.randn(n + offset, device="cuda", generator=g).to(dtype)
        x = base[offset:]
        if case == 1 and n > 1:  # ties: two in one chunk, one in another chunk, one in another thread's chunk
            top = x.float().max().to(dtype)
            for i in {n - 1, n // 2, min(n - 1, n // 2 + 1), min(n - 1, 8 * 1024 + 3)}:
                x[i] = top
        if case == 2:  # NaN entries, one of them first
            x[0] = float("nan")
            x[n // 3] = float("nan")
        if case == 3:
            x.fill_(-float("inf"))
        if case == 4 and n > 8:  # the maximum in the tail past the last whole chunk
            x[n - 1] = 100.0
        out = torch.full((1,), -5, dtype=torch.int32, device="cuda")
        _lib.check(lib.ttsp_argmax(x.data_ptr(), n, dt, out.data_ptr(), st), "argmax")
        xf = x.float()
        finite = xf[~xf.isnan()]
        if case == 3 or finite.numel() == 0 or finite.max() == -float("inf"):
            want = 0  # nothing beats -inf
        else:
            want = int((xf == finite.max()).nonzero()[0])
        assert int(out[0]) == want, (case, int(out[0]), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ntok,rows,vocab,D,pad", [(11, 512, 4096, 2560, 0), (5, 37, 512, 512, 3),
                                                   (3, 9, 64, 1000, 0), (1, 4, 16, 8, 1)])
def test_embed_sum_rows_equals_the_one_position_sum(dtype, ntok, rows, vocab, D, pad):
    """ttsp_embed_sum_rows == ttsp_embed_sum of each token column, bit for
    bit (16-byte and one-value paths: D = 1000 is not a multiple of 8), with
    tokens outside the tables (clamped), -0.0 entries, a padded token stride;
    and a sample of rows against the oracle's embed_sum."""
    from oracle import oracle as o
    from ttspipe_amd import _lib

    lib, st = _lib.lib(), _lib.stream()
    dt = _lib.dtype_code(dtype)
    g = torch.Generator(device="cuda").manual_seed(ntok * rows + D)
    E = torch.randn(ntok * vocab, D, device="cuda", generator=g).to(dtype)
    E[:, ::5] = -0.0
    tok = torch.randint(-3, vocab + 3, (ntok, rows + pad), device="cuda", generator=g, dtype=torch.int32)
    out = torch.empty(rows, D, dtype=dtype, device="cuda")
    _lib.check(lib.ttsp_embed_sum_rows(E.data_ptr(), tok.data_ptr(), rows + pad, ntok, rows, vocab, D,
                                       out.data_ptr(), dt, st), "embed_sum_rows")
    ref = torch.empty(rows, D, dtype=dtype, device="cuda")
    col = torch.empty(rows, ntok, dtype=torch.int32, device="cuda")
    col.copy_(tok[:, :rows].t())
    for r in range(rows):
        _lib.check(lib.ttsp_embed_sum(E.data_ptr(), col[r].data_ptr(), ntok, vocab, D, ref[r].data_ptr(), dt, st),
                   "embed_sum")
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    Eb = E.view(torch.int16).cpu().numpy().view(np.uint16)
    for r in sorted({0, rows // 2, rows - 1}):
        want = o.embed_sum(Eb, col[r].cpu().numpy(), vocab, D, dt)
        assert np.array_equal(out[r].view(torch.int16).cpu().numpy().view(np.uint16), want)


def test_frame_advance_equals_the_torch_bookkeeping():
    """ttsp_frame_advance == history.index_copy_(0, step, tokens),
    step.add_(1), pos.add_(1), index_select(freqs, 0, pos): three frames in a
    row, the last one past the history's rows (its row is not written) and
    with pos at the table's end (the row clamps)."""
    from ttspipe_amd import _lib
    from ttspipe_amd.llama import precompute_freqs_cis

    lib, st = _lib.lib(), _lib.stream()
    freqs = precompute_freqs_cis(300, 128, 1e6).cuda()
    ntok, rows = 11, 2
    hist = torch.zeros(rows, ntok, dtype=torch.int32, device="cuda")
    step = torch.zeros(1, dtype=torch.long, device="cuda")
    pos = torch.full((1,), 297, dtype=torch.long, device="cuda")
    frow = torch.empty(1, 64, 2, dtype=freqs.dtype, device="cuda")
    hist_ref = hist.clone()
    for f in range(3):
        tokens = torch.arange(ntok, dtype=torch.int32, device="cuda") * (f + 3)
        _lib.check(lib.ttsp_frame_advance(tokens.data_ptr(), ntok, hist.data_ptr(), rows, step.data_ptr(),
                                          pos.data_ptr(), freqs.data_ptr(), freqs.shape[0], 128, frow.data_ptr(), st),
                   "frame_advance")
        if f < rows:
            hist_ref[f] = tokens
        assert torch.equal(hist, hist_ref)
        assert int(step) == f + 1 and int(pos) == 298 + f
        assert torch.equal(frow[0].view(torch.int16), freqs[min(298 + f, 299)].view(torch.int16))


@pytest.fixture(scope="module")
def roomy():
    """The reduced model with a cache that holds more frames than the
    256-row history the model starts with."""
    import dataclasses

    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    model = SyntheticDualAR(dataclasses.replace(SMALL, max_seq_len=SMALL.prefill_len + 300))
    yield model
    del model
    torch.cuda.empty_cache()


def test_reset_to_a_longer_history_drops_the_captured_frame(roomy):
    """A captured frame writes into the history it was captured with: a reset
    that has to allocate a longer history drops the graph (it is captured
    again on the next graphed decode) instead of leaving it pointing at freed
    memory."""
    roomy.reset(4)
    roomy.capture()
    assert roomy.graph is not None
    roomy.reset(roomy.history.shape[0] + 8)
    assert roomy.graph is None
    roomy.decode(4)
    assert roomy.graph is not None


def test_graphed_decode_longer_than_the_history_equals_eager(roomy):
    """decode(n) with n above the history's rows, after a frame was captured
    for the shorter history: the history grows, the frame is captured again,
    and every frame equals the eager decode's."""
    from ttspipe_amd.dualar import max_frames

    roomy.decode(4)  # a captured frame for the current history
    n = roomy.history.shape[0] + 8
    assert n <= max_frames(roomy.cfg)
    graphed = roomy.decode(n, graphed=True)
    eager = roomy.decode(n, graphed=False)
    assert graphed.shape == (n, roomy.cfg.n_tokens)
    diff = np.flatnonzero((graphed != eager).any(axis=1))
    assert diff.size == 0, f"first differing frame {diff[0]}: graphed {graphed[diff[0]]} eager {eager[diff[0]]}"
    with pytest.raises(ValueError):
        roomy.decode(max_frames(roomy.cfg) + 1)


def _random_config(rng, seed):
    """A small Dual-AR model of random shape (widths multiples of 128, any
    GQA grouping the kernels take, 1-3 layers each side, 2-6 codebooks)."""
    from ttspipe_amd.dualar import DualARConfig

    nkv = int(rng.choice([1, 2, 4]))
    fnkv = int(rng.choice([1, 2]))
    ncb = int(rng.integers(2, 7))
    prefill_len = int(rng.integers(1, 200))
    return DualARConfig(
        dim=128 * int(rng.integers(2, 9)), n_layer=int(rng.integers(1, 4)), n_head=nkv * int(rng.choice([1, 2, 4])),
        n_local_heads=nkv, intermediate_size=128 * int(rng.integers(2, 13)),
        vocab_size=int(rng.choice([256, 512, 640])), fast_dim=128 * int(rng.integers(1, 5)),
        fast_n_layer=int(rng.integers(1, 4)), fast_n_head=fnkv * int(rng.choice([1, 2, 4])),
        fast_n_local_heads=fnkv, fast_intermediate_size=128 * int(rng.integers(1, 9)), num_codebooks=ncb,
        codebook_size=int(rng.choice([128, 256, 512])), max_seq_len=prefill_len + 8 + int(rng.integers(1, 100)),
        prefill_len=prefill_len, qk_norm=bool(rng.integers(0, 2)), seed=seed,
        fast_max_len=int(rng.choice([ncb, 16])))


@pytest.mark.parametrize("case", range(8))
def test_random_model_shapes_match_the_oracle(case):
    """Eight greedy frames of a randomly shaped model, graph-replayed and
    eager, against the oracle: the frame's launch plans (GEMV splits, fused
    or two-launch attention + wo, chunk counts of the slow cache) at shapes
    the two fixed models do not have."""
    from ttspipe_amd.dualar import SyntheticDualAR, first_tokens

    cfg = _random_config(np.random.default_rng(700 + case), seed=31 + case)
    model = SyntheticDualAR(cfg)
    got = model.decode(8, graphed=True)
    ref = _oracle(model).decode(first_tokens(cfg), cfg.prefill_len, 8)
    diff = np.flatnonzero((got != ref).any(axis=1))
    assert diff.size == 0, f"{cfg}: first differing frame {diff[0]}: gpu {got[diff[0]]} oracle {ref[diff[0]]}"
    assert np.array_equal(model.decode(8, graphed=False), got)
    del model
    torch.cuda.empty_cache()
