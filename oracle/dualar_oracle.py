"""CPU restatement of the synthetic Dual-AR frame - TEST INFRASTRUCTURE.

Follows `ttspipe_amd/dualar.py` step for step (the reference frame:
app/engine/graphs.py:76-132 - slow forward, semantic token, fast prime at
fast position 0 with the last fast layer writing only its KV entries, then one
fast step per remaining codebook), composing the C oracle's emulations of each
kernel (`*_emul`: the kernels' fixed operation order, so every intermediate
matches the GPU bit for bit). Weights are regenerated from the same
`weight_specs` with `orc_synth_fill`, the CPU twin of `ttsp_synth_fill`.

Only tests import this; the GEMV emulation needs the launch split (J, KS) the
kernel uses for each shape, which the caller supplies.
"""

from __future__ import annotations

import numpy as np

from oracle import oracle as o

BF = o.DT_BF16


class OracleDualAR:
    def __init__(self, cfg, specs, gemv_shape, *, code2, freqs_bits, fast_freqs_bits):
        """cfg / specs: `dualar.DualARConfig` / `dualar.weight_specs(cfg)`;
        gemv_shape(M, K) -> (J, KS); code2: the 256-entry fp32 second-level
        scale code; freqs: the rotary tables as bf16 bits [max_len, head_dim]
        and [fast_max_len, head_dim]."""
        self.cfg = cfg
        self.gemv_shape = gemv_shape
        linears, vectors, caches = specs
        self.t = {}
        for s in vectors + caches:
            self.t[s.name] = o.synth_fill(s.n, s.seed, s.kind, s.scale, s.offset)
        code2 = np.ascontiguousarray(code2, np.float32)
        self.lin = {}
        for s in linears:
            self.lin[s.name] = dict(
                W=o.synth_fill(s.packed.n, s.packed.seed, 0),
                A8=o.synth_fill(s.a8.n, s.a8.seed, 0),
                AMAX=o.synth_fill(s.absmax2.n, s.absmax2.seed, 3, s.absmax2.scale, s.absmax2.offset),
                CODE2=code2, offset=np.float32(s.offset), M=s.out_features, K=s.in_features)
        self.freqs = freqs_bits.reshape(cfg.max_seq_len, -1)
        self.fast_freqs = fast_freqs_bits.reshape(cfg.fast_max_len, -1)
        kv = cfg.fast_n_local_heads * cfg.fast_max_len * cfg.head_dim
        for i in range(cfg.fast_n_layer):
            self.t[f"fast_layers.{i}.k_cache"] = np.zeros(kv, np.uint16)
            self.t[f"fast_layers.{i}.v_cache"] = np.zeros(kv, np.uint16)

    # ------------------------------------------------------------- pieces

    def gemv(self, name, x, R=None, epi=0):
        L = self.lin[name]
        J, KS = self.gemv_shape(L["M"], L["K"])
        return o.gemv_emul(x, BF, L["W"], L["A8"], L["AMAX"], L["CODE2"], L["offset"], M=L["M"], K=L["K"],
                           bs=64, KS=KS, J=J, bs2=256, R=R, epi=epi)

    def norm(self, x, name):
        return o.rms_norm_emul(x, self.t[name], 1, x.size, self.cfg.norm_eps, BF)

    def _qkv_rope_kv(self, p, x, freq_row, pos, nh, nkv, max_len):
        cfg = self.cfg
        xn = self.norm(x, f"{p}.attention_norm")
        qkv = self.gemv(f"{p}.wqkv", xn)
        Q = np.zeros(nh * cfg.head_dim, np.uint16)
        qw = self.t[f"{p}.q_norm"] if cfg.qk_norm else None
        kw = self.t[f"{p}.k_norm"] if cfg.qk_norm else None
        o.qk_rope_kv(qkv, qw, kw, cfg.norm_eps, freq_row, BF, pos, Q, self.t[f"{p}.k_cache"],
                     self.t[f"{p}.v_cache"], nh, nkv, max_len, BF)
        return Q

    def block(self, p, x, freq_row, pos, nh, nkv, max_len, window):
        """`fusedlayer.decode_block` (reference fusedlayer.py:212-269)."""
        Q = self._qkv_rope_kv(p, x, freq_row, pos, nh, nkv, max_len)
        nchunk = -(-min(window, max_len) // 64)
        y = o.attn_emul(Q, self.t[f"{p}.k_cache"], self.t[f"{p}.v_cache"], pos, nh, nkv, max_len, nchunk,
                        self.cfg.head_dim ** -0.5, BF)
        h = self.gemv(f"{p}.wo", y, R=x, epi=1)
        hn = self.norm(h, f"{p}.ffn_norm")
        g1 = self.gemv(f"{p}.w1", hn)
        g = self.gemv(f"{p}.w3", hn, R=g1, epi=2)
        return self.gemv(f"{p}.w2", g, R=h, epi=1)

    # -------------------------------------------------------------- frame

    def fast_prime(self, fx):
        """Fast position 0 (reference graphs.py:76-89): every fast layer but the
        last in full; the last only for its KV entries (its output feeds
        nothing)."""
        cfg = self.cfg
        fmax = cfg.fast_max_len
        for i in range(cfg.fast_n_layer - 1):
            fx = self.block(f"fast_layers.{i}", fx, self.fast_freqs[0], 0, cfg.fast_n_head, cfg.fast_n_local_heads,
                            fmax, fmax)
        self._qkv_rope_kv(f"fast_layers.{cfg.fast_n_layer - 1}", fx, self.fast_freqs[0], 0, cfg.fast_n_head,
                          cfg.fast_n_local_heads, fmax)

    def fast_step(self, token, i):
        """Codebook step i >= 1 at fast position i: the embedding of the token
        just chosen through every fast layer, the fast norm and head -> logits."""
        cfg = self.cfg
        fmax = cfg.fast_max_len
        h = o.embed_sum(self.t["fast_embeddings"], np.asarray([token], np.int32), cfg.codebook_size, cfg.fast_dim, BF)
        for j in range(cfg.fast_n_layer):
            h = self.block(f"fast_layers.{j}", h, self.fast_freqs[i], i, cfg.fast_n_head, cfg.fast_n_local_heads,
                           fmax, fmax)
        return self.gemv("fast_output", self.norm(h, "fast_norm"))

    def step(self, tokens, pos):
        """One frame: the token column at slow position pos -> the next column.
        When `self.logits_log` is a list, each head's logits (bf16 bits) are
        appended to it: the slow head's, then one per codebook step."""
        cfg = self.cfg
        log = getattr(self, "logits_log", None)
        tok = np.asarray(tokens, np.int32)
        x = o.embed_sum(self.t["embeddings"], tok, cfg.vocab_size, cfg.dim, BF)
        for i in range(cfg.n_layer):
            x = self.block(f"layers.{i}", x, self.freqs[pos], pos, cfg.n_head, cfg.n_local_heads,
                           cfg.max_seq_len, cfg.max_seq_len)
        hn = self.norm(x, "norm")
        logits = self.gemv("output", hn)
        if log is not None:
            log.append(logits)
        out = np.zeros(cfg.n_tokens, np.int32)
        out[0] = o.argmax(logits, BF)
        self.fast_prime(self.gemv("fast_project_in", hn))
        # codebook 0 is the semantic token, clamped into the codebook
        out[1] = min(max(int(out[0]), 0), cfg.codebook_size - 1)
        for i in range(1, cfg.num_codebooks):
            fl = self.fast_step(int(out[i]), i)
            if log is not None:
                log.append(fl)
            out[i + 1] = o.argmax(fl, BF)
        return out

    def decode(self, first, pos0, n_steps):
        hist = np.zeros((n_steps, self.cfg.n_tokens), np.int32)
        tok = np.asarray(first, np.int32)
        for s in range(n_steps):
            tok = self.step(tok, pos0 + s)
            hist[s] = tok
        return hist
