"""The synthetic Dual-AR frame on the reference's CPU algorithm - TEST INFRASTRUCTURE.

The GPU decode's frame order (reference app/engine/graphs.py:76-132: slow
blocks, semantic head, fast projection, fast prime at fast position 0 with
the last fast layer only writing its KV entries, one fast step per remaining
codebook), with every block through `cpu_decode_block` (the reference CPU
path's decode_block, app/engine/nf4cpu.py:479-617, restated in
nf4cpu_port.cpp) and every head through the port's GEMV (nf4cpu.py:86-146).
Weights take the reference CPU path's form (nf4cpu.py:850-860): each layer's
scales expanded once to dense bf16 absmax and the NF4 code table rounded to
bf16. This is the reference's CPU arithmetic, not the GPU kernels', so the
two agree by tolerance: tests compare each head's logits at the reference's
block bar and count top-1 agreement under teacher forcing (the reference's
own cross-path check, docs/LATENCY.md:194-207).

Only tests import this.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from oracle import oracle as o

BF = o.DT_BF16


def resolve_scales_bf16(a8, absmax2, code2, offset, bs2: int = 256) -> np.ndarray:
    """Nested NF4 scales as the reference CPU path stores them: the fp32 scale
    code2[a8[b]] * absmax2[b // bs2] + offset (two roundings, as bitsandbytes'
    dequantize_blockwise then the offset add), rounded to bf16 bits
    (nf4cpu.py:850-860)."""
    a8 = np.asarray(a8, np.uint8)
    s = (np.asarray(code2, np.float32)[a8] * np.repeat(np.asarray(absmax2, np.float32), bs2)[: a8.size]).astype(
        np.float32)
    s = (s + np.float32(offset)).astype(np.float32)
    return o.from_f32(s, BF)


def _lib():
    from oracle import cpu_baseline

    lib = cpu_baseline._lib()
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.cpu_decode_block.argtypes = ([vp, vp, i64, i64, i64, i64, vp, vp, vp, vp, ctypes.c_float] + [vp, vp] * 4
                                     + [vp, vp, vp, i64, i64, vp, ctypes.c_int])
    lib.cpu_decode_block.restype = None
    return lib


def _p(a):
    return 0 if a is None else a.ctypes.data


class CpuReferenceDualAR:
    """The frame model on the reference CPU path.

    weights: {"linears": {name: (packed u8 [M*K/2], scale bf16 bits [M*K/64])},
    "vectors": {name: bf16 bits} (norms and embedding tables), "caches":
    {name: bf16 bits} (slow K/V caches, copied), "freqs" / "fast_freqs": the
    rotary tables as fp32 [rows, 128]} - the GPU model's own tensors."""

    def __init__(self, cfg, weights, threads: int | None = None):
        self.cfg = cfg
        self.lib = _lib()
        self.threads = threads or len(os.sched_getaffinity(0))
        self.code16 = o.from_f32(o.NF4_CODE, BF)
        self.lin = weights["linears"]
        self.vec = weights["vectors"]
        self.freqs = np.ascontiguousarray(weights["freqs"], np.float32)
        self.fast_freqs = np.ascontiguousarray(weights["fast_freqs"], np.float32)
        self.kv = {k: np.array(v, np.uint16) for k, v in weights["caches"].items()}
        fkv = cfg.fast_n_local_heads * cfg.fast_max_len * cfg.head_dim
        for i in range(cfg.fast_n_layer):
            self.kv[f"fast_layers.{i}.k_cache"] = np.zeros(fkv, np.uint16)
            self.kv[f"fast_layers.{i}.v_cache"] = np.zeros(fkv, np.uint16)
        # w1 | w3 as one weight of 2 * inter rows, the reference block's layout
        self.w13 = {}
        for prefix, n in (("layers", cfg.n_layer), ("fast_layers", cfg.fast_n_layer)):
            for i in range(n):
                p = f"{prefix}.{i}"
                w1, w3 = self.lin[f"{p}.w1"], self.lin[f"{p}.w3"]
                self.w13[p] = (np.concatenate([w1[0], w3[0]]), np.concatenate([w1[1], w3[1]]))

    def gemv(self, name, x, M):
        packed, scales = self.lin[name]
        y = np.empty(M, np.uint16)
        self.lib.cpu_nf4_gemv(x.ctypes.data, x.size, packed.ctypes.data, scales.ctypes.data, self.code16.ctypes.data,
                              M, y.ctypes.data, self.threads, 0)
        return y

    def norm(self, x, name):
        """The fork's RMSNorm (nf4cpu.py's rms_norm_bf): fp32 x, r = 1/sqrt(mean + eps), bf16(bf16(x r) w)."""
        xf = o.to_f32(x, BF).astype(np.float32)
        r = np.float32(1.0) / np.sqrt(np.float32(np.dot(xf.astype(np.float64), xf) / xf.size) + np.float32(self.cfg.norm_eps))
        t = o.to_f32(o.from_f32((xf * r).astype(np.float32), BF), BF)
        return o.from_f32((t * o.to_f32(self.vec[name], BF)).astype(np.float32), BF)

    def block(self, p, x, pos, fast: bool):
        cfg = self.cfg
        D = cfg.fast_dim if fast else cfg.dim
        nh, nkv = (cfg.fast_n_head, cfg.fast_n_local_heads) if fast else (cfg.n_head, cfg.n_local_heads)
        inter = cfg.fast_intermediate_size if fast else cfg.intermediate_size
        max_len = cfg.fast_max_len if fast else cfg.max_seq_len
        freqs = (self.fast_freqs if fast else self.freqs)[pos]
        out = np.empty(D, np.uint16)
        qn = self.vec.get(f"{p}.q_norm") if cfg.qk_norm else None
        kn = self.vec.get(f"{p}.k_norm") if cfg.qk_norm else None
        L = self.lin
        self.lib.cpu_decode_block(
            _p(x), _p(out), D, nh, nkv, inter, _p(self.vec[f"{p}.attention_norm"]), _p(self.vec[f"{p}.ffn_norm"]),
            _p(qn), _p(kn), cfg.norm_eps, _p(L[f"{p}.wqkv"][0]), _p(L[f"{p}.wqkv"][1]), _p(L[f"{p}.wo"][0]),
            _p(L[f"{p}.wo"][1]), _p(self.w13[p][0]), _p(self.w13[p][1]), _p(L[f"{p}.w2"][0]), _p(L[f"{p}.w2"][1]),
            _p(self.code16), _p(self.kv[f"{p}.k_cache"]), _p(self.kv[f"{p}.v_cache"]), pos, max_len,
            freqs.ctypes.data, self.threads)
        return out

    def step(self, tokens, pos, forced=None):
        """One frame from the token column at slow position `pos`. `forced` (the
        other path's next column) teacher-forces the fast steps' input tokens.
        Returns (this path's greedy column, [slow logits, fast logits per
        codebook step]) as bf16 bits."""
        cfg = self.cfg
        tok = np.asarray(tokens, np.int32)
        x = o.embed_sum(self.vec["embeddings"], tok, cfg.vocab_size, cfg.dim, BF)
        for i in range(cfg.n_layer):
            x = self.block(f"layers.{i}", x, pos, fast=False)
        hn = self.norm(x, "norm")
        logits = [self.gemv("output", hn, cfg.vocab_size)]
        out = np.zeros(cfg.n_tokens, np.int32)
        out[0] = o.argmax(logits[0], BF)
        out[1] = min(max(int(out[0]), 0), cfg.codebook_size - 1)
        fx = self.gemv("fast_project_in", hn, cfg.fast_dim)
        for j in range(cfg.fast_n_layer):  # the prime: the last layer's output feeds nothing
            fx = self.block(f"fast_layers.{j}", fx, 0, fast=True)
        feed = out if forced is None else np.asarray(forced, np.int32)
        for i in range(1, cfg.num_codebooks):
            t = int(feed[i]) if forced is not None else int(out[i])
            h = o.embed_sum(self.vec["fast_embeddings"], np.asarray([t], np.int32), cfg.codebook_size, cfg.fast_dim,
                            BF)
            for j in range(cfg.fast_n_layer):
                h = self.block(f"fast_layers.{j}", h, i, fast=True)
            logits.append(self.gemv("fast_output", self.norm(h, "fast_norm"), cfg.codebook_size))
            out[i + 1] = o.argmax(logits[-1], BF)
        return out, logits


def weights_from_gpu_model(model) -> dict:
    """The host copy of a `dualar.SyntheticDualAR`'s weights in the reference
    CPU path's form (packed codes as stored, nested scales resolved to bf16)."""
    import torch

    def bits16(t):
        return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1)

    lin = {}
    for name, (packed, state) in model.quant.items():
        s2 = state.state2
        scales = resolve_scales_bf16(state.absmax.cpu().numpy(), s2.absmax.cpu().numpy(), s2.code.cpu().numpy(),
                                     float(state.offset), int(s2.blocksize))
        lin[name] = (packed.view(-1).cpu().numpy().copy(), scales)
    vec = {s.name: bits16(model.tensors[s.name]) for s in model.specs["vectors"]}
    caches = {s.name: bits16(model.tensors[s.name]) for s in model.specs["caches"]}
    f32 = lambda t: t.float().reshape(t.shape[0], -1).cpu().numpy()  # noqa: E731
    return {"linears": lin, "vectors": vec, "caches": caches, "freqs": f32(model.freqs),
            "fast_freqs": f32(model.fast_freqs)}
