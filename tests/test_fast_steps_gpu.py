"""The codebook loop as one launch (`ttsp_fast_steps`) against the same loop
launch by launch (GPU).

Bar: bit for bit. Every frame's token column, the last codebook step's
logits and the fast KV caches the steps write are identical between the
one-launch form and the per-launch form (whose results the oracle tests
pin), eager and graph-replayed, and no grid-barrier wait gives up. The
benchmark model's 256-frame oracle fixture is checked through the one-launch
form too.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpuutil import bits

pytestmark = pytest.mark.gpu


def _state(model):
    caches = []
    for blk in model.fast_layers:
        c = blk.attention.kv_cache
        caches += [bits(c.k_cache).copy(), bits(c.v_cache).copy()]
    return bits(model.fast_logits).copy(), caches


def _compare(model, frames, graphed):
    model.use_fast_steps = True
    one = model.decode(frames, graphed=graphed)
    one_logits, one_caches = _state(model)
    assert model.fast_steps_failed() == 0
    model.use_fast_steps = False
    model.graph = None  # a captured frame holds the form it was captured with
    loop = model.decode(frames, graphed=graphed)
    loop_logits, loop_caches = _state(model)
    model.use_fast_steps = True
    model.graph = None
    diff = np.flatnonzero((one != loop).any(axis=1))
    assert diff.size == 0, f"first differing frame {diff[0]}: one launch {one[diff[0]]} per launch {loop[diff[0]]}"
    assert np.array_equal(one_logits, loop_logits)
    for i, (a, b) in enumerate(zip(one_caches, loop_caches)):
        assert np.array_equal(a, b), f"fast cache {i // 2} ({'kv'[i % 2]}) differs"
    assert len({tuple(r) for r in one}) > 1, "the decode should not be stuck on one frame"


@pytest.mark.parametrize("graphed", [False, True])
def test_small_model_fast_steps_equal_the_per_launch_loop(graphed):
    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    model = SyntheticDualAR(SMALL)
    assert model._fast_args is not None and model._fast_args["grid"] == 64
    _compare(model, 24, graphed)
    del model
    torch.cuda.empty_cache()


def test_benchmark_model_fast_steps_equal_the_per_launch_loop():
    from ttspipe_amd.dualar import DualARConfig, SyntheticDualAR

    model = SyntheticDualAR(DualARConfig())
    assert model._fast_args is not None and model._fast_args["grid"] == 128
    _compare(model, 12, graphed=True)
    _compare(model, 4, graphed=False)
    del model
    torch.cuda.empty_cache()


@pytest.mark.parametrize("qk_norm,fast_max_len", [(False, 4), (True, 64)])
def test_fast_steps_without_head_norms_and_with_a_full_chunk_cache(qk_norm, fast_max_len):
    """The reduced model's fast side without q/k head norms and a 4-row cache
    (exactly the codebook steps' positions), and with a 64-position cache."""
    import dataclasses

    from ttspipe_amd.dualar import SMALL, SyntheticDualAR

    model = SyntheticDualAR(dataclasses.replace(SMALL, qk_norm=qk_norm, fast_max_len=fast_max_len))
    assert model._fast_args is not None
    _compare(model, 8, graphed=True)
    del model
    torch.cuda.empty_cache()


def test_benchmark_model_256_frames_through_fast_steps_match_the_oracle_fixture(monkeypatch):
    """The fixture test of test_dualar_gpu.py with the codebook loop as one launch."""
    from tests import test_dualar_gpu
    from ttspipe_amd import dualar

    orig = dualar.SyntheticDualAR.__init__

    def init(self, *a, **kw):
        orig(self, *a, **kw)
        self.use_fast_steps = True
        assert self._fast_args is not None

    monkeypatch.setattr(dualar.SyntheticDualAR, "__init__", init)
    test_dualar_gpu.test_benchmark_model_256_frames_match_the_oracle_fixture()
