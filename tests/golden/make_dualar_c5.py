"""Write the 256-frame greedy token fixture of the benchmark-size Dual-AR frame.

Runs the oracle's CPU restatement of the frame (`oracle.dualar_oracle`) on the
benchmark model - 36 slow layers at d=2560 (32 q / 8 kv heads of 128, FFN
9728, vocab 4096), 4 fast layers at d=1024 over 10 codebooks of 4096, KV
cache filled with seeded bf16 up to position 2048 - for 256 greedy frames, and
records:

* the token column of every frame ([256, 11] ints);
* the GEMV launch split (J, KS) of every linear shape, which fixes the
  kernel's summation order and therefore the bits the oracle reproduces (a
  GPU test asserts the library still reports these, so a kernel whose order
  changed fails loudly instead of comparing against stale ids);
* per frame, sha256 digests of the slow head's logits and of the last
  codebook step's logits (bf16 bit patterns): the decode of this random model
  falls into a few recurring token columns, so the logits carry most of what
  distinguishes one frame from the next;
* sha256 digests of the K and V cache rows written at frames 0, 128 and 255
  in slow layers 0, 17 and 35, and of the rotary tables the frame used.

Run from the repository root (about 21 minutes on 8 cores; the fixture records the run's
seconds in `cpu_seconds`: 1,260.6):

    python -m tests.golden.make_dualar_c5 [--frames 256]

The fixture is data: `tests/golden/dualar_c5_tokens.json`.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
OUT = HERE / "dualar_c5_tokens.json"
KV_FRAMES = (0, 128, 255)
KV_LAYERS = (0, 17, 35)


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def freqs_bits(cfg):
    """The two rotary tables as the frame model builds them (bf16 bit patterns)."""
    import torch

    from ttspipe_amd.llama import precompute_freqs_cis

    def b(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)

    return (b(precompute_freqs_cis(cfg.max_seq_len, cfg.head_dim, cfg.rope_base, dtype=torch.bfloat16)),
            b(precompute_freqs_cis(cfg.fast_max_len, cfg.head_dim, cfg.rope_base, dtype=torch.bfloat16)))


def gemv_shapes(cfg):
    """(M, K) -> (J, KS) of every linear of the model, from the library's planner."""
    import ctypes

    from ttspipe_amd import _lib
    from ttspipe_amd.dualar import weight_specs

    lib = _lib.load()
    out = {}
    for s in weight_specs(cfg)[0]:
        key = (s.out_features, s.in_features)
        if key in out:
            continue
        J, KS, RPW = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
        if lib.ttsp_gemv_shape(key[0], key[1], ctypes.byref(J), ctypes.byref(KS), ctypes.byref(RPW)) != 0:
            raise RuntimeError(f"no GEMV plan for {key}")
        out[key] = (J.value, KS.value)
    return out


def make(frames: int, cfg=None) -> dict:
    from oracle.dualar_oracle import OracleDualAR
    from ttspipe_amd.dualar import DualARConfig, first_tokens, weight_specs
    from ttspipe_amd.quant import create_dynamic_map

    cfg = cfg or DualARConfig()
    shapes = gemv_shapes(cfg)
    fb, ffb = freqs_bits(cfg)
    orc = OracleDualAR(cfg, weight_specs(cfg), lambda M, K: shapes[(M, K)],
                       code2=create_dynamic_map().numpy(), freqs_bits=fb, fast_freqs_bits=ffb)
    t0 = time.time()
    hist = np.zeros((frames, cfg.n_tokens), np.int32)
    slow_logits, fast_logits = [], []
    tok = np.asarray(first_tokens(cfg), np.int32)
    for f in range(frames):
        orc.logits_log = []
        tok = orc.step(tok, cfg.prefill_len + f)
        hist[f] = tok
        slow_logits.append(digest(orc.logits_log[0]))
        fast_logits.append(digest(orc.logits_log[-1]))
        print(f"frame {f}: {tok.tolist()} ({time.time() - t0:.0f} s)", flush=True)
    kv = {}
    for layer in KV_LAYERS:
        if layer >= cfg.n_layer:
            continue
        for which in ("k", "v"):
            c = orc.t[f"layers.{layer}.{which}_cache"].reshape(cfg.n_local_heads, cfg.max_seq_len, cfg.head_dim)
            for f in KV_FRAMES:
                if f < frames:
                    kv[f"{which}.{layer}.{f}"] = digest(c[:, cfg.prefill_len + f])
    return {
        "what": "greedy token ids of the synthetic Dual-AR frame model, from the oracle's CPU restatement",
        "config": {k: getattr(cfg, k) for k in cfg.__dataclass_fields__},
        "frames": frames,
        "first_tokens": list(map(int, first_tokens(cfg))),
        "position0": cfg.prefill_len,
        "gemv_shapes": {f"{m}x{k}": list(v) for (m, k), v in sorted(shapes.items())},
        "freqs_sha256": digest(fb),
        "fast_freqs_sha256": digest(ffb),
        "kv_rows_sha256": kv,
        "tokens": hist.tolist(),
        "slow_logits_sha256": slow_logits,
        "last_fast_logits_sha256": fast_logits,
        "cpu_seconds": round(time.time() - t0, 1),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--frames", type=int, default=256)
    ap.add_argument("--out", type=Path, default=OUT)
    args = ap.parse_args()
    data = make(args.frames)
    args.out.write_text(json.dumps(data, indent=1) + "\n")
    print(f"wrote {args.out} ({data['cpu_seconds']} s)")


if __name__ == "__main__":
    main()
