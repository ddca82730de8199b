"""Transformer block of the Dual-AR model, in the fork's own (unfused) form.

The reference patches classes of the vendored fish-speech fork
(`fish_speech.models.text2semantic.llama`: RMSNorm, Attention, FeedForward,
TransformerBlock, KVCache, precompute_freqs_cis, apply_rotary_emb), which is
not part of the reference tree; the reference states their arithmetic where it
replaces them (app/engine/fusedops.py:8-14, app/engine/fusedlayer.py:56-92,
app/engine/fastpath.py:207-271). These are those classes restated with the
same attribute names, so `nf4gemv.install`, `fusedops.install` and
`fusedlayer.install` patch them exactly as the reference patches the fork.
Their forwards are torch ops: the path a declined call falls back to.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from ttspipe_amd.quant import Linear4bit


@dataclass
class BaseModelArgs:
    dim: int = 2560
    n_head: int = 32
    n_local_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 9728
    attention_qk_norm: bool = True
    norm_eps: float = 1e-6
    rope_base: float = 1e6
    max_seq_len: int = 4096


def precompute_freqs_cis(seq_len: int, n_elem: int, base: float = 10000, dtype=torch.bfloat16):
    """(cos, sin) of s * base^(-2i/n_elem) as [seq_len, n_elem/2, 2] (the fork's table, bf16)."""
    freqs = 1.0 / (base ** (torch.arange(0, n_elem, 2)[: (n_elem // 2)].float() / n_elem))
    t = torch.arange(seq_len, device=freqs.device)
    freqs = torch.outer(t, freqs)
    cis = torch.polar(torch.ones_like(freqs), freqs)
    return torch.stack([cis.real, cis.imag], dim=-1).to(dtype)


def apply_rotary_emb(x, freqs_cis):
    """Interleaved-pair rotation in fp32, rounded once to x's dtype."""
    xs = x.float().reshape(*x.shape[:-1], -1, 2)
    fc = freqs_cis.float().view(1, xs.size(1), 1, xs.size(3), 2)
    out = torch.stack(
        [
            xs[..., 0] * fc[..., 0] - xs[..., 1] * fc[..., 1],
            xs[..., 1] * fc[..., 0] + xs[..., 0] * fc[..., 1],
        ],
        -1,
    )
    return out.flatten(3).type_as(x)


class RMSNorm(nn.Module):
    """`_norm(x.float()).type_as(x) * weight` (two roundings)."""

    def __init__(self, dim: int, eps: float = 1e-6, dtype=None, device=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype, device=device), requires_grad=False)

    def _norm(self, x):
        return x * torch.rsqrt(torch.mean(x * x, dim=-1, keepdim=True) + self.eps)

    def forward(self, x):
        return self._norm(x.float()).type_as(x) * self.weight


class HeadNorm(nn.Module):
    """Per-head q/k norm with one rounding: round(x * rsqrt(mean(x^2) + eps) * w)."""

    def __init__(self, dim: int, eps: float = 1e-6, dtype=None, device=None):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim, dtype=dtype, device=device), requires_grad=False)

    def forward(self, x):
        xf = x.float()
        r = torch.rsqrt(torch.mean(xf * xf, dim=-1, keepdim=True) + self.eps)
        return (xf * r * self.weight.float()).to(x.dtype)


class KVCache(nn.Module):
    def __init__(self, max_batch_size, max_seq_len, n_heads, head_dim, dtype=torch.bfloat16, device=None):
        super().__init__()
        shape = (max_batch_size, n_heads, max_seq_len, head_dim)
        self.register_buffer("k_cache", torch.zeros(shape, dtype=dtype, device=device))
        self.register_buffer("v_cache", torch.zeros(shape, dtype=dtype, device=device))

    def update(self, input_pos, k_val, v_val):
        self.k_cache[:, :, input_pos] = k_val
        self.v_cache[:, :, input_pos] = v_val
        return self.k_cache, self.v_cache


def _linear(cin, cout, dtype, device, blocksize=64, nested=True):
    return Linear4bit(cin, cout, bias=False, compute_dtype=dtype, compress_statistics=nested,
                      blocksize=blocksize, device=device)


class Attention(nn.Module):
    def __init__(self, config: BaseModelArgs, dtype=torch.bfloat16, device=None):
        super().__init__()
        total = (config.n_head + 2 * config.n_local_heads) * config.head_dim
        self.wqkv = _linear(config.dim, total, dtype, device)
        self.wo = _linear(config.n_head * config.head_dim, config.dim, dtype, device)
        self.kv_cache = None
        self.n_head = config.n_head
        self.n_local_heads = config.n_local_heads
        self.head_dim = config.head_dim
        self.dim = config.dim
        self.attention_qk_norm = config.attention_qk_norm
        if self.attention_qk_norm:
            self.q_norm = HeadNorm(config.head_dim, config.norm_eps, dtype=dtype, device=device)
            self.k_norm = HeadNorm(config.head_dim, config.norm_eps, dtype=dtype, device=device)

    def forward(self, x, freqs_cis, mask, input_pos=None):
        from ttspipe_amd import fusedops
        from ttspipe_amd.fastpath import decode_attention, prefill_attention

        bsz, seqlen, _ = x.shape
        q_size = self.n_head * self.head_dim
        kv_size = self.n_local_heads * self.head_dim
        q, k, v = self.wqkv(x).split([q_size, kv_size, kv_size], dim=-1)
        q = q.view(bsz, seqlen, self.n_head, self.head_dim)
        k = k.view(bsz, seqlen, self.n_local_heads, self.head_dim)
        v = v.view(bsz, seqlen, self.n_local_heads, self.head_dim)
        if self.attention_qk_norm:
            q = self.q_norm(q)
            k = self.k_norm(k)
        fq = fusedops.rope(q, freqs_cis)
        fk = fusedops.rope(k, freqs_cis) if fq is not None else None
        if fk is not None:
            q, k = fq, fk
        else:
            fusedops.note_rope_fallback()
            q = apply_rotary_emb(q, freqs_cis)
            k = apply_rotary_emb(k, freqs_cis)
        q, k, v = (t.transpose(1, 2) for t in (q, k, v))
        if self.kv_cache is not None:
            k, v = self.kv_cache.update(input_pos, k, v)
        if mask is not None and mask.shape[-1] < k.shape[2]:
            k = k[:, :, : mask.shape[-1]]
            v = v[:, :, : mask.shape[-1]]
        y = prefill_attention(q, k, v, mask, self.n_head, self.n_local_heads, self.head_dim)
        if y is None:
            y = decode_attention(q, k, v, mask, self.n_head, self.n_local_heads, self.head_dim)
        y = y.transpose(1, 2).contiguous().view(bsz, seqlen, q_size)
        return self.wo(y)


class FeedForward(nn.Module):
    def __init__(self, config: BaseModelArgs, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.w1 = _linear(config.dim, config.intermediate_size, dtype, device)
        self.w3 = _linear(config.dim, config.intermediate_size, dtype, device)
        self.w2 = _linear(config.intermediate_size, config.dim, dtype, device)

    def forward(self, x):
        return self.w2(F.silu(self.w1(x)) * self.w3(x))


class TransformerBlock(nn.Module):
    def __init__(self, config: BaseModelArgs, dtype=torch.bfloat16, device=None):
        super().__init__()
        self.attention = Attention(config, dtype=dtype, device=device)
        self.feed_forward = FeedForward(config, dtype=dtype, device=device)
        self.ffn_norm = RMSNorm(config.dim, config.norm_eps, dtype=dtype, device=device)
        self.attention_norm = RMSNorm(config.dim, config.norm_eps, dtype=dtype, device=device)

    def forward(self, x, freqs_cis, mask, input_pos=None):
        h = x + self.attention(self.attention_norm(x), freqs_cis, mask, input_pos)
        return h + self.feed_forward(self.ffn_norm(h))
