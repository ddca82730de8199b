"""The C-ABI boundary and the host-side logic, on the CPU (no GPU calls).

* every function `include/ttsp_hip.h` declares is exported by the built
  library and bound by `_lib.SIGNATURES` with the header's arity;
* host-only entry points (`ttsp_gemv_shape`, argument validation that
  returns before any launch) behave as documented;
* the Python drop-ins decline without a GPU instead of raising (the
  reference's contract, app/engine/nvrtc.py:26-28);
* byte accounting used by the benchmark matches the closed forms.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ttsp_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\bint\s+(ttsp_\w+)\s*\(([^)]*)\)\s*;", text):
        args = m.group(2).strip()
        n = 0 if args in ("", "void") else args.count(",") + 1
        decls[m.group(1)] = n
    return decls


def test_header_declares_the_entry_points():
    decls = _declared()
    for name in ("ttsp_nf4_gemm", "ttsp_nf4_dequant", "ttsp_rms_norm", "ttsp_rope", "ttsp_qk_rope_kv",
                 "ttsp_attn_decode", "ttsp_gemv_shape"):
        assert name in decls


def test_library_exports_every_declared_symbol():
    from ttspipe_amd import _lib

    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _declared():
        assert hasattr(lib, name), f"{name} declared in the header but not exported"


def test_bindings_match_the_header():
    from ttspipe_amd import _lib

    decls = _declared()
    assert set(_lib.SIGNATURES) == set(decls)
    for name, n in decls.items():
        assert len(_lib.SIGNATURES[name]) == n, name


def _shape(M, K):
    from ttspipe_amd import _lib

    J, KS, RPW = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rc = _lib.load().ttsp_gemv_shape(M, K, ctypes.byref(J), ctypes.byref(KS), ctypes.byref(RPW))
    return rc, J.value, KS.value, RPW.value


@pytest.mark.parametrize("M,K", [(9728, 2560), (2560, 9728), (6144, 2560), (2560, 4096), (1024, 2560),
                                 (1536, 1024), (3072, 1024), (1024, 3072), (4096, 1024), (64, 128)])
def test_gemv_shape_covers_every_row_and_column(M, K):
    rc, J, KS, RPW = _shape(M, K)
    assert rc == 0
    assert KS in (1, 2, 4, 8) and 1 <= J <= 8 and RPW >= 1
    assert J * KS * 64 >= K // 8 and (J - 1) * KS * 64 < K // 8  # no wholly idle chunk slot


def _dl_split(M, K, N):
    """The direct-to-LDS kernel's split for 256 to 512 rows, or None: 4 where K
    has 64 or more steps and there are at least 75 64 x 128 tiles; with fewer
    steps none from 512 tiles and 2 from 300."""
    steps, t = K // 64, -(-M // 64) * -(-N // 128)
    if not 256 <= N <= 512:
        return None
    if steps >= 64:
        return 4 if t >= 75 and steps % 8 == 0 and steps // 4 <= 64 else None
    if t >= 512:
        return 1
    if t >= 300 and steps % 4 == 0:
        return 2
    return None


@pytest.mark.parametrize("N", [2, 32, 33, 64, 70, 256, 512, 2048])
@pytest.mark.parametrize("M,K", [(4096, 2560), (1024, 2560), (2560, 4096), (9728, 2560), (2560, 9728),
                                 (6144, 2560), (1536, 1024), (3072, 1024), (1024, 3072), (64, 128)])
def test_gemm_split_plan(M, K, N):
    """The K split a prefill GEMM takes (host-only query): none for N <= 32 or
    when the 64 x 128 output tiles already fill the GPU; otherwise each split
    covers an even number of at least 8 K-steps of 64 codes. 33 to 64 rows:
    4 splits where that allows, else 2. 256 to 512 rows where the
    direct-to-LDS kernel takes the launch: its split. More rows otherwise: up
    to 128 tiles the largest such split whose workgroups fit one to a CU;
    between 128 and 256 tiles, 4 splits when each keeps more than 16 K-steps."""
    from ttspipe_amd import _lib

    lib = _lib.load()
    sp = lib.ttsp_nf4_gemm_splits(M, K, N)
    assert sp in (1, 2, 4, 8)
    steps = K // 64
    t = -(-M // 64) * -(-N // 128)
    if sp > 1:
        assert steps % (2 * sp) == 0 and steps // sp >= 8
    dl = _dl_split(M, K, N) if N > 64 else None
    if dl is not None:
        assert sp == dl
        return
    if N <= 32 or t >= 256:
        assert sp == 1
    if 32 < N <= 64:  # 64 x 64 tiles, the K split 4 ways where each keeps 8 K-steps, else 2
        expect = 4 if steps % 8 == 0 and steps // 4 >= 8 else 2 if steps % 4 == 0 and steps // 2 >= 8 else 1
        assert sp == expect
    elif N > 64 and t > 128:
        assert sp == (4 if t < 256 and steps % 8 == 0 and steps > 64 else 1)
    elif N > 64:
        # the split fits one pass, and twice it would not (or is not allowed)
        assert t * sp <= 256
        nxt = 2 * sp
        assert nxt > 8 or steps % (2 * nxt) or steps // nxt < 8 or t * nxt > 256
    assert lib.ttsp_nf4_gemm_splits(M, K, 1) == 1


def test_gemm_split_entry_rejects_a_mismatched_split():
    from ttspipe_amd import _lib

    lib = _lib.load()
    sp = lib.ttsp_nf4_gemm_splits(2560, 9728, 512)
    assert sp == 4
    for bad in (1, 2, 8):  # anything but the plan's split, before any launch
        assert lib.ttsp_nf4_gemm_split(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 0, 2560, 9728, 512, 64, 256, 16,
                                       bad, None) == 1
    # the plan's split without a workspace
    assert lib.ttsp_nf4_gemm_split(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 0, 2560, 9728, 512, 64, 256, None,
                                   sp, None) == 1
    # rows-kernel arguments
    assert lib.ttsp_qk_rope_kv_rows(8, 100, None, None, 1e-6, 8, 1, 8, 8, 8, 8, 4, 2, 64, 3, 1, None) == 1
    assert lib.ttsp_qk_rope_kv_rows(8, 1024, None, None, 1e-6, 8, 1, 8, 8, 8, 8, 4, 2, 64, 0, 1, None) == 1


@pytest.mark.parametrize("S", [1, 7, 32, 64, 100, 512, 2048])
@pytest.mark.parametrize("nkv", [1, 2, 8, 16])
@pytest.mark.parametrize("L_extra", [0, 64, 500, 2000, 8000])
def test_prefill_key_split_plan(S, nkv, L_extra):
    """The key split of a prefill attention (host-only query): none below 16
    key blocks of 32 or from 256 (kv head, 32-query) workgroups; two for
    128-255 workgroups over a cached prefix of 1024 keys or more, else none;
    below 128 workgroups a power of two up to 16, each split holding at least
    3 key blocks, doubling only while the workgroups stay under 256."""
    from ttspipe_amd import _lib

    lib = _lib.load()
    L = S + L_extra
    sp = lib.ttsp_prefill_attention_splits(S, nkv, L)
    wg = nkv * -(-S // 32)
    blocks = -(-L // 32)
    assert sp in (1, 2, 4, 8, 16)
    if wg >= 256 or blocks < 16:
        assert sp == 1
    elif wg >= 128:
        assert sp == (2 if L_extra >= 1024 else 1)
        return
    if sp > 1:
        assert blocks // sp >= 3 and wg * sp // 2 < 256
    if sp < 16 and wg < 128 and blocks >= 16:  # stopped because it filled the GPU or ran out of blocks
        assert wg * sp >= 256 or blocks // (2 * sp) < 3


def test_prefill_split_entry_rejects_bad_splits_before_any_launch():
    from ttspipe_amd import _lib

    lib = _lib.load()
    p = 1 << 20  # aligned stand-in pointers: every call below is refused before a launch
    args = (p, 1024, 128, p, 256, 4096, p, 256, 4096, p, 64, p, 4, 8, 2, 16, 0.088, 1)
    assert lib.ttsp_prefill_attention_split(*args, p, 0, None) == 1
    assert lib.ttsp_prefill_attention_split(*args, p, 17, None) == 1
    assert lib.ttsp_prefill_attention_split(*args, None, 2, None) == 1  # no workspace
    assert lib.ttsp_prefill_attention_split(*args, p + 4, 2, None) == 1  # workspace not 16-byte aligned


def test_invalid_arguments_are_rejected_before_any_launch():
    from ttspipe_amd import _lib

    lib = _lib.load()
    # N == 0, M == 0, blocksize not a power of two, K not a multiple of 128: hipErrorInvalidValue (1)
    assert lib.ttsp_nf4_gemm(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 0, 64, 128, 0, 64, 256, None) == 1
    assert lib.ttsp_nf4_gemm(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 0, 0, 128, 1, 64, 256, None) == 1
    assert lib.ttsp_nf4_gemm(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 0, 64, 128, 1, 96, 256, None) == 1
    assert lib.ttsp_nf4_gemm(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 0, 64, 192, 1, 64, 256, None) == 1
    # an epilogue without its operand
    assert lib.ttsp_nf4_gemm(8, 1, 8, None, 8, None, 0.0, 8, 8, None, 1, 64, 128, 1, 64, 256, None) == 1
    assert lib.ttsp_nf4_dequant(8, None, 8, None, 0.0, 8, 8, 1, -1, 64, 256, None) == 1
    assert lib.ttsp_attn_decode(8, 8, 8, 8, 8, 8, 8, 8, 32, 7, 64, 1, 0.1, 1, None) == 1  # nh % nkv
    assert lib.ttsp_attn_decode_rows(8, 8, 8, 8, 8, 8, 8, 8, 32, 8, 64, 1, 0.1, 0, 1, None) == 1  # no rows
    assert lib.ttsp_attn_decode_rows(8, 8, 8, 8, 8, 8, 8, 8, 32, 8, 64, 1, 0.1, 70000, 1, None) == 1
    assert lib.ttsp_attn_chunk() == 64
    # the frame's glue: empty rows, tables or histories, missing pointers, an unknown dtype
    assert lib.ttsp_argmax_embed(8, 0, 1, 8, None, 8, 16, 8, 8, None) == 1
    assert lib.ttsp_argmax_embed(8, 16, 1, 8, None, 8, 0, 8, 8, None) == 1
    assert lib.ttsp_argmax_embed(8, 16, 1, None, None, 8, 16, 8, 8, None) == 1
    assert lib.ttsp_argmax_embed(8, 16, 7, 8, None, 8, 16, 8, 8, None) == 1
    assert lib.ttsp_frame_advance(8, 11, 8, 0, 8, 8, 8, 300, 128, 8, None) == 1
    assert lib.ttsp_frame_advance(8, 11, 8, 4, 8, None, 8, 300, 128, 8, None) == 1
    assert lib.ttsp_frame_advance(8, 0, 8, 4, 8, 8, 8, 300, 128, 8, None) == 1


def test_drop_ins_decline_without_a_gpu():
    import torch

    from ttspipe_amd import _lib, fusedlayer, fusedops, nf4gemv
    from ttspipe_amd.quant import Linear4bit

    if _lib.gpu_present():
        pytest.skip("a GPU is present")
    lin = Linear4bit(128, 64, compress_statistics=False, compute_dtype=torch.float16).load_weight(torch.randn(64, 128))
    assert nf4gemv.available() is False
    assert nf4gemv.prepare(lin) is False  # weights on the CPU
    assert nf4gemv.matmul(lin, torch.randn(1, 128, dtype=torch.float16)) is None
    assert nf4gemv.install() is False
    assert fusedops.rms_norm(torch.randn(1, 64, dtype=torch.float16), torch.ones(64, dtype=torch.float16), 1e-6) is None
    assert fusedops.install() is False and fusedlayer.install() is False


def test_benchmark_byte_counts():
    import bench

    # the reference's CPU-runnable case (C1: 9728 x 2560, fp32 absmax) and one decoder layer (C2: the
    # seven nested-scale linears), each total worked out by hand from the NF4 layout
    assert bench.nf4_bytes(9728, 2560, False) == 14_032_896
    assert sum(bench.nf4_bytes(M, K, True) for _, M, K in bench.LAYER) == 52_186_204
    # the fused launches: identical weight and scale bytes; q/k/v read x once (two fewer x reads and code2
    # tables), gate/up read x once and write one gated output instead of two outputs
    saved = 2 * (2560 * 2 + 1028) + 2560 * 2 + 9728 * 2
    assert bench.fused_layer_bytes() == 52_186_204 - saved == 52_149_332


def test_roofline_figures_are_keyed_to_the_launch_they_measured():
    """bench.py's off-line GEMV figures (rocprof durations, counter traffic)
    carry the launch they were measured on - shape, grid and a digest of the
    kernel source - and are printed only while it matches the launch the bench
    makes: the committed figures match the current kernel, and any other key
    reads as stale."""
    import bench

    key = bench.gemv_launch_key(9728, 2560)
    assert key == bench.GEMV_PROFILE["key"], "nf4_gemv.hip or its launch changed: re-profile and update GEMV_PROFILE"
    kern = {"M": 9728, "K": 2560, "sec": 6e-6, "bytes": bench.nf4_bytes(9728, 2560, True), "gbs": 2145.4}
    line = bench.roofline_entry(kern)
    assert line["traffic"] == bench.GEMV_PROFILE["traffic_bytes"] and "stale" not in line
    assert line["rocprof"]["median_us"] == bench.GEMV_PROFILE["rocprof_median_us"]
    assert abs(line["frac"] - 2145.4 / 8000) < 1e-4
    saved = dict(bench.GEMV_PROFILE["key"])
    try:
        bench.GEMV_PROFILE["key"]["source_sha16"] = "0" * 16
        line = bench.roofline_entry(kern)
        assert line["traffic"] is None and "rocprof" not in line and "stale" in line
    finally:
        bench.GEMV_PROFILE["key"].clear()
        bench.GEMV_PROFILE["key"].update(saved)


def test_dualar_specs_and_byte_account():
    from ttspipe_amd import dualar

    cfg = dualar.DualARConfig()
    linears, vectors, caches = dualar.weight_specs(cfg)
    names = [s.name for s in linears + vectors + caches]
    assert len(names) == len(set(names))
    seeds = [t.seed for s in linears for t in (s.packed, s.a8, s.absmax2)] + [s.seed for s in vectors + caches]
    assert len(seeds) == len(set(seeds)), "every synthetic tensor needs its own stream"
    slow = sum(s.packed.n for s in linears if s.name.startswith("layers."))
    assert slow == 36 * (6144 * 2560 + 2560 * 4096 + 3 * 9728 * 2560) // 2
    b0, b1 = dualar.step_bytes(cfg, 2048), dualar.step_bytes(cfg, 2049)
    assert 2.3e9 < b0 < 2.6e9
    assert b1 - b0 == cfg.n_layer * cfg.n_local_heads * cfg.head_dim * 2 * 2  # one more K and V row


def test_decode_longer_than_the_cache_is_refused_on_the_host():
    """Frame i writes slow position prefill_len + i: the benchmark model holds
    2304 - 2048 = 256 frames, and one more is a ValueError before any launch
    (the kernels would clamp the position instead of failing)."""
    from ttspipe_amd import dualar

    cfg = dualar.DualARConfig()
    assert dualar.max_frames(cfg) == 256
    dualar.check_frames(cfg, 256)
    dualar.check_frames(cfg, 1)
    for bad in (257, 512, 0, -1):
        with pytest.raises(ValueError):
            dualar.check_frames(cfg, bad)
    small = dualar.SMALL
    assert dualar.max_frames(small) == small.max_seq_len - small.prefill_len == 256


def test_dualar_oracle_decode_is_deterministic_and_in_range(orc):
    """The reduced model through the CPU restatement: same frames twice, ids in range."""
    from oracle.dualar_oracle import OracleDualAR
    from ttspipe_amd import dualar
    from ttspipe_amd.llama import precompute_freqs_cis
    from ttspipe_amd.quant import create_dynamic_map

    cfg = dualar.SMALL
    bits = lambda t: t.contiguous().view(__import__("torch").int16).numpy().view(np.uint16).reshape(-1)  # noqa: E731

    def make():
        return OracleDualAR(cfg, dualar.weight_specs(cfg), lambda M, K: _shape(M, K)[1:3],
                            code2=create_dynamic_map().numpy(),
                            freqs_bits=bits(precompute_freqs_cis(cfg.max_seq_len, 128, cfg.rope_base)),
                            fast_freqs_bits=bits(precompute_freqs_cis(cfg.fast_max_len, 128, cfg.rope_base)))

    a = make().decode(dualar.first_tokens(cfg), cfg.prefill_len, 6)
    b = make().decode(dualar.first_tokens(cfg), cfg.prefill_len, 6)
    assert np.array_equal(a, b)
    assert (a[:, 0] < cfg.vocab_size).all() and (a[:, 1:] < cfg.codebook_size).all() and (a >= 0).all()
    assert (a[:, 1] == np.minimum(a[:, 0], cfg.codebook_size - 1)).all()


def test_fast_steps_argument_blocks_match_the_header(tmp_path):
    """`ttsp_nf4_weight` / `ttsp_fast_layer` as the C compiler lays them out
    from the header, against the ctypes mirrors the Python side passes."""
    import subprocess

    from ttspipe_amd import _lib

    src = tmp_path / "layout.c"
    src.write_text(
        '#include <stddef.h>\n#include <stdio.h>\n#include "ttsp_hip.h"\n'
        "int main(void) {\n"
        '  printf("%zu %zu %zu %zu %zu %zu\\n", sizeof(ttsp_nf4_weight), offsetof(ttsp_nf4_weight, offset),\n'
        "         sizeof(ttsp_fast_layer), offsetof(ttsp_fast_layer, w2), offsetof(ttsp_fast_layer, attention_norm),\n"
        "         offsetof(ttsp_fast_layer, v_cache));\n"
        '  printf("%d %d\\n", TTSP_FAST_SYNC_WORDS, TTSP_FAST_SYNC_FAILED);\n'
        "  return 0;\n}\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c99", f"-I{ROOT / 'include'}", str(src), "-o", str(exe)], check=True)
    lines = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split("\n")
    got = [int(v) for v in lines[0].split()]
    W, L = _lib.Nf4Weight, _lib.FastLayer
    assert got == [ctypes.sizeof(W), W.offset.offset, ctypes.sizeof(L), L.w2.offset, L.attention_norm.offset,
                   L.v_cache.offset]
    assert [int(v) for v in lines[1].split()] == [_lib.FAST_SYNC_WORDS, _lib.FAST_SYNC_FAILED]


def test_fast_steps_serves_the_fast_transformer_shapes():
    """The one-launch codebook loop's shape plan (host-only): the benchmark's
    fast transformer (d 1024, 8/2 heads, FFN 3072, codebook 4096) on 128
    workgroups, the reduced model's on 64; shapes the GEMV would split along K,
    more than 8 query heads, caches past one 64-position chunk, more than 4
    layers and blocks under 64 codes are declined (0)."""
    from ttspipe_amd import _lib
    from ttspipe_amd.dualar import SMALL, DualARConfig

    lib = _lib.load()

    def grid(c, **kw):
        a = dict(dim=c.fast_dim, n_head=c.fast_n_head, n_kv=c.fast_n_local_heads, inter=c.fast_intermediate_size,
                 vocab=c.codebook_size, max_len=c.fast_max_len, n_layers=c.fast_n_layer, blocksize=64)
        a.update(kw)
        return lib.ttsp_fast_steps_grid(*a.values())

    big = DualARConfig()
    assert grid(big) == 128
    assert grid(SMALL) == 64
    for kw in ({"dim": 2560}, {"inter": 9728}, {"n_head": 16, "n_kv": 4}, {"max_len": 65}, {"n_layers": 5},
               {"n_layers": 0}, {"blocksize": 32}, {"blocksize": 96}, {"n_head": 6, "n_kv": 4}, {"vocab": 0}):
        assert grid(big, **kw) == 0, kw
    # the phases' K splits as the GEMV's own plan gives them: all 1
    for M, K in ((1536, 1024), (1024, 1024), (3072, 1024), (1024, 3072), (4096, 1024)):
        assert _shape(M, K)[2] == 1
    qkv = (big.fast_n_head + 2 * big.fast_n_local_heads) * 128
    rb = lambda e: -(-2 * e // 256) * 256  # noqa: E731
    assert lib.ttsp_fast_steps_work_bytes(1024, 8, 2, 3072) == rb(qkv) + 2 * rb(1024) + rb(3072)
    assert lib.ttsp_fast_steps_work_bytes(0, 8, 2, 3072) == 0


def test_fast_steps_rejects_bad_arguments_before_any_launch():
    """Null pointers, positions past the cache and unserved shapes return
    hipErrorInvalidValue (1) on the host."""
    from ttspipe_amd import _lib

    lib = _lib.load()
    layers = (_lib.FastLayer * 4)()
    head = _lib.Nf4Weight()
    p = 4096  # never dereferenced: every case returns before a launch

    def call(dim=1024, max_len=16, step0=1, n_steps=9, x0=p, n_layers=4):
        return lib.ttsp_fast_steps(layers, n_layers, head, p, p, p, p, 1, x0, p, p, p, p, dim, 8, 2, 3072, 4096,
                                   max_len, step0, n_steps, 1e-6, 64, 256, _lib.DT_BF16, None)

    assert call(x0=None) == 1
    assert call(step0=8, n_steps=9) == 1  # positions 8 .. 16 run past a 16-row cache
    assert call(step0=-1) == 1
    assert call(n_steps=0) == 1
    assert call(dim=2560) == 1
    assert call(n_layers=5) == 1
    assert call() == 1  # the weights' pointers are NULL


def test_swiglu_gemm_plan_on_the_host():
    """`ttsp_nf4_gemm_swiglu_fits`: one launch where both GEMMs of the pair
    would run the direct-to-LDS kernel unsplit (up to 512 rows, >= 512 tiles
    of 64 x 128 with fewer than 64 K-steps: 385-512 rows of 9728 x 2560) or
    the few-row kernel (3-32 rows), nowhere else; the entry rejects a
    shape it does not serve before any launch."""
    from ttspipe_amd import _lib

    lib = _lib.load()
    fits = lib.ttsp_nf4_gemm_swiglu_fits
    assert fits(9728, 2560, 512, 64, 256, 1) == 1
    assert fits(9728, 2560, 400, 64, 256, 0) == 1
    assert fits(9730, 2560, 500, 64, 256, 1) == 1
    for args in ((2560, 9728, 512, 64, 256, 1), (9728, 2560, 128, 64, 256, 1), (9728, 2560, 256, 64, 256, 1), (9728, 2560, 513, 64, 256, 1),
                 (1536, 1024, 512, 64, 256, 1), (9728, 2560, 512, 64, 16, 1), (9728, 2560, 512, 32, 256, 1),
                 (9728, 2560, 512, 96, 256, 0), (9728, 2500, 512, 64, 256, 1)):
        assert fits(*args) == 0, args
    # 3-32 rows where both GEMMs run the few-row kernel unsplit: its pair form
    for rows in (3, 4, 8, 16, 17, 32):
        assert fits(9728, 2560, rows, 64, 256, 1) == 1, rows
        assert fits(2560, 9728, rows, 64, 256, 0) == 1, rows
    for args in ((9728, 2560, 2, 64, 256, 1), (9728, 2560, 33, 64, 256, 1), (9728, 2560, 64, 64, 256, 1),
                 (9728, 10368, 4, 64, 256, 1), (9728, 2560, 4, 32, 256, 1)):
        assert fits(*args) == 0, args  # two rows (the GEMV), a K split, runs past 8 waves, 32-code blocks
    p = 4096
    assert lib.ttsp_nf4_gemm_swiglu(p, 1, p, p, p, p, 0.0, p, p, p, p, 0.0, p, p, 2560, 9728, 512, 64, 256,
                                    None) == 1
    assert lib.ttsp_nf4_gemm_swiglu(p, 1, p, p, p, p, 0.0, p, None, p, p, 0.0, p, p, 9728, 2560, 512, 64, 256,
                                    None) == 1  # one weight nested, the other plain
