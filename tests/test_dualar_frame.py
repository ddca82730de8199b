"""The oracle's Dual-AR frame against an independent torch restatement (CPU).

The frame (reference app/engine/graphs.py:76-132): the slow transformer over
the summed token embeddings at the next position, the semantic token from its
head; its normed final state, projected to the fast width, primes the fast
transformer at fast position 0 (every fast layer but the last in full, the
last only for its KV entries); then codebook steps 1..9 at fast positions
1..9, each feeding the embedding of the token just chosen (codebook 1's is the
semantic token clamped into the codebook).

`TorchFrame` restates that frame here with plain torch ops in fp32, on the
weights dequantised by torch (round(code * (code2[a8] * absmax2 + offset)) to
bf16), rounding to bf16 where the fork's bf16 modules round. It shares no
code with the oracle's frame or with `dualar.py`: only the weight generator
and the model's shapes. The oracle runs freely; the torch frame is fed the
oracle's tokens (teacher forcing, so a near tie cannot cascade) and every
head's logits are compared: within a relative bar, and the oracle's greedy
token must be torch's wherever torch's top-2 margin exceeds twice the largest
logit difference. Planted mistakes in the oracle's frame must fail that check.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import oracle as o

LOGITS_BAR = 2e-2  # the reference's block bar (tests/test_nf4cpu.py:175-191)


def _bf16_bits_to_f32(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy((bits.astype(np.uint32) << 16).view(np.float32).copy())


def r16(t: torch.Tensor) -> torch.Tensor:
    """Round to bf16, keep computing in fp32."""
    return t.to(torch.bfloat16).float()


class TorchFrame:
    def __init__(self, cfg):
        from ttspipe_amd.dualar import weight_specs
        from ttspipe_amd.llama import precompute_freqs_cis
        from ttspipe_amd.quant import NF4_CODE, create_dynamic_map

        self.cfg = cfg
        linears, vectors, caches = weight_specs(cfg)
        code = torch.tensor(NF4_CODE, dtype=torch.float32)
        code2 = create_dynamic_map().float()
        self.W = {}
        for s in linears:
            packed = torch.from_numpy(o.synth_fill(s.packed.n, s.packed.seed, 0).astype(np.int64))
            q = torch.stack([packed >> 4, packed & 15], 1).reshape(-1)
            a8 = torch.from_numpy(o.synth_fill(s.a8.n, s.a8.seed, 0).astype(np.int64))
            amax2 = torch.from_numpy(o.synth_fill(s.absmax2.n, s.absmax2.seed, 3, s.absmax2.scale, s.absmax2.offset))
            scale = code2[a8] * amax2.repeat_interleave(256)[: a8.numel()]
            scale = scale + torch.tensor(s.offset, dtype=torch.float32)
            self.W[s.name] = r16(code[q] * scale.repeat_interleave(64)).view(s.out_features, s.in_features)
        self.v = {s.name: _bf16_bits_to_f32(o.synth_fill(s.n, s.seed, s.kind, s.scale, s.offset))
                  for s in vectors + caches}
        for i in range(cfg.n_layer):
            for w in ("k", "v"):
                self.v[f"layers.{i}.{w}_cache"] = self.v[f"layers.{i}.{w}_cache"].view(
                    cfg.n_local_heads, cfg.max_seq_len, cfg.head_dim)
        for i in range(cfg.fast_n_layer):
            for w in ("k", "v"):
                self.v[f"fast_layers.{i}.{w}_cache"] = torch.zeros(cfg.fast_n_local_heads, cfg.fast_max_len,
                                                                   cfg.head_dim)
        self.freqs = precompute_freqs_cis(cfg.max_seq_len, cfg.head_dim, cfg.rope_base).float()
        self.fast_freqs = precompute_freqs_cis(cfg.fast_max_len, cfg.head_dim, cfg.rope_base).float()

    # the fork's modules, bf16 in and out
    def lin(self, name, x):
        return r16(self.W[name] @ x)

    def rmsnorm(self, x, name):
        r = torch.rsqrt((x * x).mean() + self.cfg.norm_eps)
        return r16(r16(x * r) * self.v[name])

    def head_norm(self, x, name):
        r = torch.rsqrt((x * x).mean(-1, keepdim=True) + self.cfg.norm_eps)
        return r16(x * r * self.v[name])

    @staticmethod
    def rope(x, f):
        c, s = f[:, 0], f[:, 1]
        x0, x1 = x[:, 0::2], x[:, 1::2]
        return r16(torch.stack([x0 * c - x1 * s, x1 * c + x0 * s], -1).flatten(1))

    def qkv_kv(self, p, x, f, pos, nh, nkv):
        hd = self.cfg.head_dim
        qkv = self.lin(f"{p}.wqkv", self.rmsnorm(x, f"{p}.attention_norm"))
        q = qkv[: nh * hd].view(nh, hd)
        k = qkv[nh * hd:(nh + nkv) * hd].view(nkv, hd)
        v = qkv[(nh + nkv) * hd:].view(nkv, hd)
        if self.cfg.qk_norm:
            q, k = self.head_norm(q, f"{p}.q_norm"), self.head_norm(k, f"{p}.k_norm")
        q, k = self.rope(q, f), self.rope(k, f)
        self.v[f"{p}.k_cache"][:, pos] = k
        self.v[f"{p}.v_cache"][:, pos] = v
        return q

    def block(self, p, x, f, pos, nh, nkv):
        q = self.qkv_kv(p, x, f, pos, nh, nkv)
        kc, vc = self.v[f"{p}.k_cache"][:, : pos + 1], self.v[f"{p}.v_cache"][:, : pos + 1]
        g = nh // nkv
        sc = torch.einsum("hd,hld->hl", q, kc.repeat_interleave(g, 0)) * self.cfg.head_dim ** -0.5
        y = r16(torch.einsum("hl,hld->hd", torch.softmax(sc, -1), vc.repeat_interleave(g, 0))).reshape(-1)
        h = r16(x + self.lin(f"{p}.wo", y))
        hn = self.rmsnorm(h, f"{p}.ffn_norm")
        gate = r16(r16(torch.nn.functional.silu(self.lin(f"{p}.w1", hn))) * self.lin(f"{p}.w3", hn))
        return r16(h + self.lin(f"{p}.w2", gate))

    def frame(self, tokens, pos, forced):
        """Logits of the slow head and of each codebook step, with the fast
        steps fed `forced` (the column the oracle chose)."""
        cfg = self.cfg
        emb = self.v["embeddings"].view(cfg.n_tokens, cfg.vocab_size, cfg.dim)
        x = torch.zeros(cfg.dim)
        for c, t in enumerate(tokens):
            x = x + emb[c, int(t)]
        x = r16(x)
        for i in range(cfg.n_layer):
            x = self.block(f"layers.{i}", x, self.freqs[pos], pos, cfg.n_head, cfg.n_local_heads)
        hn = self.rmsnorm(x, "norm")
        out = [self.lin("output", hn)]
        fx = self.lin("fast_project_in", hn)
        f0 = self.fast_freqs[0]
        for i in range(cfg.fast_n_layer - 1):
            fx = self.block(f"fast_layers.{i}", fx, f0, 0, cfg.fast_n_head, cfg.fast_n_local_heads)
        self.qkv_kv(f"fast_layers.{cfg.fast_n_layer - 1}", fx, f0, 0, cfg.fast_n_head, cfg.fast_n_local_heads)
        femb = self.v["fast_embeddings"].view(cfg.codebook_size, cfg.fast_dim)
        assert forced[1] == min(max(int(forced[0]), 0), cfg.codebook_size - 1)
        for i in range(1, cfg.num_codebooks):
            h = femb[int(forced[i])]
            for j in range(cfg.fast_n_layer):
                h = self.block(f"fast_layers.{j}", h, self.fast_freqs[i], i, cfg.fast_n_head, cfg.fast_n_local_heads)
            out.append(self.lin("fast_output", self.rmsnorm(h, "fast_norm")))
        return out


def _oracle(cfg, cls=None):
    from oracle.dualar_oracle import OracleDualAR
    from ttspipe_amd.dualar import weight_specs
    from ttspipe_amd.llama import precompute_freqs_cis
    from ttspipe_amd.quant import create_dynamic_map

    def b(t):
        return t.contiguous().view(torch.int16).numpy().view(np.uint16).reshape(-1)

    def shape(M, K):
        # a launch split that covers any row: one K slice of ceil(K / 512) dwords per lane
        return (-(-K // 512), 1)

    return (cls or OracleDualAR)(cfg, weight_specs(cfg), shape, code2=create_dynamic_map().numpy(),
                                 freqs_bits=b(precompute_freqs_cis(cfg.max_seq_len, cfg.head_dim, cfg.rope_base)),
                                 fast_freqs_bits=b(precompute_freqs_cis(cfg.fast_max_len, cfg.head_dim, cfg.rope_base)))


def compare(cfg, orc, frames):
    """Free-running oracle vs the teacher-forced torch frame. Returns
    (worst relative logit difference, heads whose greedy token disagrees
    despite a clear margin, heads where the margin decided, heads)."""
    from ttspipe_amd.dualar import first_tokens

    tf = TorchFrame(cfg)
    tok = np.asarray(first_tokens(cfg), np.int32)
    worst, wrong, decided, heads = 0.0, [], 0, 0
    for f in range(frames):
        pos = cfg.prefill_len + f
        orc.logits_log = []
        out = orc.step(tok, pos)
        ref = tf.frame(tok, pos, out)
        assert len(orc.logits_log) == len(ref) == cfg.num_codebooks
        for h, (lo_bits, lt) in enumerate(zip(orc.logits_log, ref)):
            lo = _bf16_bits_to_f32(lo_bits)
            diff = float((lo - lt).abs().max())
            worst = max(worst, diff / float(lt.abs().max()))
            top2 = torch.topk(lt, 2).values
            heads += 1
            if float(top2[0] - top2[1]) > 2 * diff:
                decided += 1
                if int(out[0 if h == 0 else h + 1]) != int(torch.argmax(lt)):
                    wrong.append((f, h))
        tok = out
    return worst, wrong, decided, heads


FRAMES = 12


def test_oracle_frame_matches_the_torch_frame():
    from ttspipe_amd.dualar import SMALL

    worst, wrong, decided, heads = compare(SMALL, _oracle(SMALL), FRAMES)
    assert worst < LOGITS_BAR, f"logits differ by {worst:.3g} of their range"
    assert not wrong, f"greedy tokens differ at (frame, head) {wrong}"
    assert decided >= 0.8 * heads, f"only {decided} of {heads} heads had a clear margin"


def _mutants():
    from oracle.dualar_oracle import OracleDualAR

    class PrimeAtPositionOne(OracleDualAR):
        def fast_prime(self, fx):
            cfg = self.cfg
            fmax = cfg.fast_max_len
            for i in range(cfg.fast_n_layer - 1):
                fx = self.block(f"fast_layers.{i}", fx, self.fast_freqs[1], 1, cfg.fast_n_head,
                                cfg.fast_n_local_heads, fmax, fmax)
            self._qkv_rope_kv(f"fast_layers.{cfg.fast_n_layer - 1}", fx, self.fast_freqs[1], 1, cfg.fast_n_head,
                              cfg.fast_n_local_heads, fmax)

    class PrimeSkipsTheLastLayer(OracleDualAR):
        def fast_prime(self, fx):
            cfg = self.cfg
            fmax = cfg.fast_max_len
            for i in range(cfg.fast_n_layer - 1):
                fx = self.block(f"fast_layers.{i}", fx, self.fast_freqs[0], 0, cfg.fast_n_head,
                                cfg.fast_n_local_heads, fmax, fmax)

    class CodebookStepsOneBehind(OracleDualAR):
        def fast_step(self, token, i):
            return super().fast_step(token, i - 1)

    class SlowWithoutTheFinalNorm(OracleDualAR):
        def norm(self, x, name):
            return x.copy() if name == "norm" else super().norm(x, name)

    return [PrimeAtPositionOne, PrimeSkipsTheLastLayer, CodebookStepsOneBehind, SlowWithoutTheFinalNorm]


@pytest.mark.parametrize("mutant", _mutants(), ids=lambda c: c.__name__)
def test_planted_frame_mistakes_are_caught(mutant):
    from ttspipe_amd.dualar import SMALL

    worst, wrong, _, _ = compare(SMALL, _oracle(SMALL, mutant), FRAMES)
    assert worst >= LOGITS_BAR or wrong, f"{mutant.__name__} passed the check (worst {worst:.3g})"
