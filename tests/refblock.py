"""A transformer block restated in float64 numpy from the model's definition,
independent of every kernel in this repository: the reference for the fused
prefill block.

The block (the fork's `TransformerBlock`, whose operation order the
reference's fused decode block follows, app/engine/fusedlayer.py:212-269):
x -> RMSNorm -> wqkv -> split q/k/v -> per-head q/k RMSNorm (when the model
has it) -> interleaved-pair rotary -> KV-cache write -> causal GQA attention
(query head h reads KV head h // (n_head / n_local_heads), softmax in full
precision, app/engine/fastpath.py:133-174) -> wo -> + x = h -> RMSNorm ->
w2(silu(w1 .) * w3 .) (app/engine/cpu.py:119-121) -> + h.

`rnd` rounds a tensor where the fork produces a 16-bit tensor (every
activation above), so the result is the exact computation with the fork's
roundings; without it, the exact computation. `mutant` plants one mistake
(tests show each is far outside the bar the kernels are held to).
"""

from __future__ import annotations

import numpy as np

MUTANTS = ("no_rope", "no_qk_norm", "gqa_modulo", "mask_off_by_one")


def block_fp64(W, norms, x, freqs, kc, vc, pos, n_head, n_kv, qk_norm, eps=1e-6, rnd=None, mutant=None):
    """W: name -> [M, K] dequantised weights; norms: name -> vector
    (attention_norm, ffn_norm, q_norm, k_norm); x [S, D]; freqs [S, 64, 2]
    (cos, sin) of each position; kc/vc [n_kv, L, 128] the cache before the
    call; pos: the S positions. Returns (out [S, D], K rows [S, n_kv, 128],
    V rows [S, n_kv, 128]) as written to the cache."""
    r = rnd or (lambda t: t)

    def rms(t, w):  # the per-head q/k norm: one rounding, after the weight
        return t / np.sqrt(np.mean(t * t, axis=-1, keepdims=True) + eps) * w

    def rms2(t, w):  # the block norms: rounded, then times the weight, rounded again
        return r(r(t / np.sqrt(np.mean(t * t, axis=-1, keepdims=True) + eps)) * w)

    S = x.shape[0]
    hd = 128
    xn = rms2(x, norms["attention_norm"])
    qkv = r(xn @ W["wqkv"].T)
    q = qkv[:, : n_head * hd].reshape(S, n_head, hd)
    k = qkv[:, n_head * hd : (n_head + n_kv) * hd].reshape(S, n_kv, hd)
    v = qkv[:, (n_head + n_kv) * hd :].reshape(S, n_kv, hd)
    if qk_norm and mutant != "no_qk_norm":
        q = r(rms(q, norms["q_norm"]))
        k = r(rms(k, norms["k_norm"]))

    def rope(t):
        t2 = t.reshape(S, t.shape[1], hd // 2, 2)
        c, s = freqs[:, None, :, 0], freqs[:, None, :, 1]
        out = np.stack([t2[..., 0] * c - t2[..., 1] * s, t2[..., 1] * c + t2[..., 0] * s], -1)
        return out.reshape(t.shape)

    if mutant != "no_rope":
        q, k = r(rope(q)), r(rope(k))
    K, V = kc.copy(), vc.copy()
    for i, p in enumerate(pos):
        K[:, p] = k[i]
        V[:, p] = v[i]
    groups = n_head // n_kv
    last = np.asarray(pos)[:, None] + (1 if mutant == "mask_off_by_one" else 0)
    allow = np.arange(K.shape[1])[None, :] <= last
    y = np.zeros((S, n_head, hd))
    for h in range(n_head):
        kv = h % n_kv if mutant == "gqa_modulo" else h // groups
        sc = np.where(allow, q[:, h] @ K[kv].T / np.sqrt(hd), -np.inf)
        p = np.exp(sc - sc.max(-1, keepdims=True))
        y[:, h] = (p / p.sum(-1, keepdims=True)) @ V[kv]
    y = r(y.reshape(S, n_head * hd))
    h_ = r(x + r(y @ W["wo"].T))
    hn = rms2(h_, norms["ffn_norm"])
    a1, a3 = r(hn @ W["w1"].T), r(hn @ W["w3"].T)
    g = r(r(a1 / (1 + np.exp(-a1))) * a3)
    return r(h_ + r(g @ W["w2"].T)), k, v


def rel_norm(a, b) -> float:
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))
