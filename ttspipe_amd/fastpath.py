"""Grouped-query attention for a decode step or a short prefill, in torch ops.

Restates the reference's `decode_attention` (app/engine/fastpath.py:133-174):
query head i reads KV head i // groups (the grouping `repeat_interleave` and
`enable_gqa` use), fp32 scores scaled by head_dim^-0.5, the boolean mask
applied with -inf, softmax in fp32, probabilities cast to V's dtype before the
second matmul. This is the unfused attention of `llama.Attention` (prefill and
declined decode calls); a decode step takes the HIP kernels in `fusedlayer`.
"""

from __future__ import annotations

GROUPED_MAX_QUERY = 64


def decode_attention(q, k, v, mask, n_head, n_local_heads, head_dim):
    """q (B, n_head, S, D), k/v (B, n_local_heads, L, D), mask bool (B, 1, S, L) -> (B, n_head, S, D)."""
    import torch

    bsz, _, seqlen, _ = q.shape
    groups = n_head // n_local_heads
    qg = q.reshape(bsz, n_local_heads, groups * seqlen, head_dim)
    # fp32 products on the device: a bf16 batched matmul with a transposed
    # right operand is avoided on purpose.
    scores = torch.matmul(qg.float(), k.float().transpose(-2, -1).contiguous()) * (head_dim**-0.5)
    scores = scores.view(bsz, n_local_heads, groups, seqlen, -1)
    if mask is not None:
        scores = torch.where(mask.unsqueeze(2), scores, float("-inf"))
    probs = torch.softmax(scores, dim=-1).to(v.dtype).view(bsz, n_local_heads, groups * seqlen, -1)
    return torch.matmul(probs.float(), v.float()).to(v.dtype).view(bsz, n_head, seqlen, head_dim)
