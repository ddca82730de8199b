"""Grouped-query attention for a decode step or a short prefill, in torch ops.

Restates the reference's `decode_attention` (app/engine/fastpath.py:133-174):
query head i reads KV head i // groups (the grouping `repeat_interleave` and
`enable_gqa` use), fp32 scores scaled by head_dim^-0.5, the boolean mask
applied with -inf, softmax in fp32, probabilities cast to V's dtype before the
second matmul. This is the unfused attention of `llama.Attention` (prefill and
declined decode calls); a decode step takes the HIP kernels in `fusedlayer`.

`prefill_attention` is the same computation in one HIP launch (flash form on
the matrix cores) for any number of new positions: the reference runs
`decode_attention` for up to `GROUPED_MAX_QUERY` queries and torch's
`scaled_dot_product_attention` with the boolean mask beyond
(app/engine/fastpath.py:244-268). It declines (returns None) what it does not
take, and the caller then runs `decode_attention`. `causal_rows_attention`
serves a short span whose mask is known to be causal with the decode step's
attention kernels, row by row.
"""

from __future__ import annotations

GROUPED_MAX_QUERY = 64
HEAD_DIM = 128
CHUNK = 64  # cache positions per chunk of the decode attention (ttsp_attn_chunk)

_stats = {"prefill_attn": 0, "prefill_declined": 0, "causal_rows": 0}


def stats() -> dict:
    return dict(_stats)


def _prefill_eligible(q, k, v, mask, n_head, n_local_heads, head_dim, positions=None) -> bool:
    import torch

    from ttspipe_amd import _lib

    if head_dim != HEAD_DIM or (mask is None and positions is None) or not q.is_cuda or q.dim() != 4:
        return False
    if k.dim() != 4 or v.dim() != 4:
        return False
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        return False
    bsz, nh, seqlen, d = q.shape
    if bsz != 1 or nh != n_head or d != head_dim or n_head % n_local_heads:
        return False
    if n_head // n_local_heads > _lib.lib().ttsp_prefill_max_groups():
        return False
    L = k.shape[2]
    if k.shape != (1, n_local_heads, L, head_dim) or v.shape != k.shape:
        return False
    for t in (q, k, v):
        if t.stride(3) != 1 or t.stride(1) % 8 or t.stride(2) % 8 or t.data_ptr() % 16:
            return False
    if positions is not None:
        return (positions.dtype == torch.long and positions.is_cuda and positions.is_contiguous()
                and positions.numel() == seqlen)
    if mask.dtype != torch.bool or mask.dim() != 4 or tuple(mask.shape) != (1, 1, seqlen, L) or not mask.is_cuda:
        return False
    return mask.stride(3) == 1 and mask.stride(2) % 16 == 0 and mask.stride(2) >= L and mask.data_ptr() % 16 == 0


def prefill_attention(q, k, v, mask, n_head, n_local_heads, head_dim, out=None, work=None, positions=None):
    """`decode_attention` in one launch: q (1, n_head, S, 128), k/v (1,
    n_local_heads, L, 128) with the last dim contiguous (any seq/head strides
    that keep rows 16-byte aligned, e.g. the KV cache sliced to L), mask bool
    (1, 1, S, L) with 16-byte aligned rows. Returns (1, n_head, S, 128) as a
    transposed view of a contiguous (1, S, n_head * 128) tensor (`out=` may
    supply that tensor), so the caller's `transpose(1, 2).contiguous()` is free;
    None when declined. A query whose mask row allows no key gets NaN, as the
    reference's softmax over all -inf scores. A short run over a long cache
    splits its keys over several workgroups (`ttsp_prefill_attention_splits`)
    through an fp32 workspace: `work=` may supply one of at least
    `prefill_work_floats(...)` elements, else it is allocated per call.
    `positions` (int64 (S,), contiguous): the causal mask at those positions
    (row i allows keys 0 .. positions[i], none at or past L) is computed in
    the kernel instead of read, and `mask` is not read (it may be None); the
    result is bit for bit the one `mask` = those causal rows gives, except
    where the kernel takes four in-workgroup key splits (4 query heads per kv
    head, no split over workgroups, at least 128 (kv head, 32-row block)
    pairs), whose merge order rounds differently."""
    import torch

    from ttspipe_amd import _lib

    if not _lib.gpu_present() or not _prefill_eligible(q, k, v, mask, n_head, n_local_heads, head_dim, positions):
        _stats["prefill_declined"] += 1
        return None
    seqlen, L = q.shape[2], k.shape[2]
    if out is None:
        out = torch.empty(1, seqlen, n_head * head_dim, dtype=q.dtype, device=q.device)
    elif out.shape != (1, seqlen, n_head * head_dim) or out.dtype != q.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous (1, S, n_head * head_dim) tensor of q's dtype")
    lib = _lib.lib()
    splits = lib.ttsp_prefill_attention_splits(seqlen, n_local_heads, L)
    need = prefill_work_floats(seqlen, n_head, splits)
    if splits > 1 and work is None:
        work = torch.empty(need, dtype=torch.float32, device=q.device)
    elif splits > 1 and (work.dtype != torch.float32 or work.numel() < need or not work.is_contiguous()
                         or work.data_ptr() % 16):
        raise ValueError(f"work must be a contiguous 16-byte aligned fp32 tensor of at least {need} elements")
    wp = work.data_ptr() if splits > 1 else None
    if positions is not None:
        rc = lib.ttsp_prefill_attention_causal(
            q.data_ptr(), q.stride(2), q.stride(1), k.data_ptr(), k.stride(2), k.stride(1), v.data_ptr(),
            v.stride(2), v.stride(1), positions.data_ptr(), out.data_ptr(), seqlen, n_head, n_local_heads, L,
            float(head_dim**-0.5), _lib.dtype_code(q.dtype), wp, splits, _lib.stream())
        _lib.check(rc, "ttsp_prefill_attention_causal")
    else:
        rc = lib.ttsp_prefill_attention_split(
            q.data_ptr(), q.stride(2), q.stride(1), k.data_ptr(), k.stride(2), k.stride(1), v.data_ptr(),
            v.stride(2), v.stride(1), mask.data_ptr(), mask.stride(2), out.data_ptr(), seqlen, n_head, n_local_heads,
            L, float(head_dim**-0.5), _lib.dtype_code(q.dtype), wp, splits, _lib.stream())
        _lib.check(rc, "ttsp_prefill_attention_split")
    _stats["prefill_attn"] += 1
    return out.view(1, seqlen, n_head, head_dim).transpose(1, 2)


#: Longest causal span `causal_rows_attention` serves (the grouped decode
#: attention row by row); longer spans take `prefill_attention`.
CAUSAL_ROWS_MAX = 8


def causal_rows_attention(q, k_cache, v_cache, input_pos, n_head, n_local_heads, width):
    """Attention of S query rows (q contiguous (1, S, n_head, 128)) at
    positions `input_pos` (int64 (S,)) over the cache (1, n_local_heads,
    max_len, 128) with the causal mask - row i sees positions 0 .. pos[i],
    which must lie below `width`, the mask's key count - as the decode step's
    attention computes each row (bit for bit the one-position result). Returns
    (1, S, n_head * 128); None when declined (shapes, dtypes, S >
    CAUSAL_ROWS_MAX)."""
    import torch

    from ttspipe_amd import _lib

    if not _lib.gpu_present():
        return None
    S = q.shape[1] if q.dim() == 4 else 0
    if (S < 1 or S > CAUSAL_ROWS_MAX or q.shape != (1, S, n_head, HEAD_DIM) or not q.is_contiguous()
            or k_cache.dim() != 4 or k_cache.shape[0] != 1 or k_cache.shape[1] != n_local_heads
            or k_cache.shape[3] != HEAD_DIM or v_cache.shape != k_cache.shape or not k_cache.is_contiguous()
            or not v_cache.is_contiguous() or k_cache.dtype != q.dtype or v_cache.dtype != q.dtype
            or input_pos.dtype != torch.long or input_pos.numel() != S or not input_pos.is_contiguous()
            or n_head % n_local_heads or _lib.dtype_code(q.dtype) not in (_lib.DT_F16, _lib.DT_BF16)):
        return None
    max_len = k_cache.shape[2]
    nchunk = -(-min(width, max_len) // CHUNK)
    pm = torch.empty(2 * S * n_head * nchunk, dtype=torch.float32, device=q.device)
    pacc = torch.empty(S * n_head * nchunk * HEAD_DIM, dtype=torch.float32, device=q.device)
    y = torch.empty(1, S, n_head * HEAD_DIM, dtype=q.dtype, device=q.device)
    rc = _lib.lib().ttsp_attn_decode_rows(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), input_pos.data_ptr(), pm.data_ptr(),
        pm[S * n_head * nchunk:].data_ptr(), pacc.data_ptr(), y.data_ptr(), n_head, n_local_heads, max_len, nchunk,
        float(HEAD_DIM**-0.5), S, _lib.dtype_code(q.dtype), _lib.stream())
    _lib.check(rc, "ttsp_attn_decode_rows")
    _stats["causal_rows"] += 1
    return y


def causal_rows_attention_qkv(qkv, q_weight, k_weight, eps, freqs_cis, input_pos, k_cache, v_cache, n_head,
                              n_local_heads, width):
    """`causal_rows_attention` straight from the wqkv output: qkv (1, S,
    (n_head + 2 n_local_heads) 128) contiguous, the q/k head-norm weights
    (None: no head norms) and eps, the rows' rotary rows freqs_cis (S x 128
    values, contiguous), positions input_pos (int64 (S,)). The head norms,
    rotary and the KV-cache write of the S rows happen inside the attention
    launch (each workgroup computes the span rows its chunk holds), with the
    bits of the head-norm / rotary / KV kernel followed by
    `causal_rows_attention`. Returns (1, S, n_head * 128); None when declined
    (shapes, dtypes, S > CAUSAL_ROWS_MAX)."""
    import torch

    from ttspipe_amd import _lib

    if not _lib.gpu_present():
        return None
    S = qkv.shape[1] if qkv.dim() == 3 else 0
    width_qkv = (n_head + 2 * n_local_heads) * HEAD_DIM
    ftype = _lib.dtype_code(freqs_cis.dtype)
    if (S < 1 or S > CAUSAL_ROWS_MAX or qkv.shape != (1, S, width_qkv) or not qkv.is_contiguous()
            or k_cache.dim() != 4 or k_cache.shape[0] != 1 or k_cache.shape[1] != n_local_heads
            or k_cache.shape[3] != HEAD_DIM or v_cache.shape != k_cache.shape or not k_cache.is_contiguous()
            or not v_cache.is_contiguous() or k_cache.dtype != qkv.dtype or v_cache.dtype != qkv.dtype
            or input_pos.dtype != torch.long or input_pos.numel() != S or not input_pos.is_contiguous()
            or n_head % n_local_heads or _lib.dtype_code(qkv.dtype) not in (_lib.DT_F16, _lib.DT_BF16)
            or ftype is None or not freqs_cis.is_contiguous() or freqs_cis.numel() != S * HEAD_DIM
            or freqs_cis.data_ptr() % 4):
        return None
    for w in (q_weight, k_weight):
        if w is not None and (w.dtype != qkv.dtype or w.numel() != HEAD_DIM or not w.is_contiguous()):
            return None
    max_len = k_cache.shape[2]
    nchunk = -(-min(width, max_len) // CHUNK)
    pm = torch.empty(2 * S * n_head * nchunk, dtype=torch.float32, device=qkv.device)
    pacc = torch.empty(S * n_head * nchunk * HEAD_DIM, dtype=torch.float32, device=qkv.device)
    y = torch.empty(1, S, n_head * HEAD_DIM, dtype=qkv.dtype, device=qkv.device)
    rc = _lib.lib().ttsp_attn_decode_qkv_rows(
        qkv.data_ptr(), width_qkv, _lib.ptr(q_weight), _lib.ptr(k_weight), float(eps), freqs_cis.data_ptr(), ftype,
        input_pos.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), pm.data_ptr(), pm[S * n_head * nchunk:].data_ptr(),
        pacc.data_ptr(), y.data_ptr(), n_head, n_local_heads, max_len, nchunk, float(HEAD_DIM**-0.5), S,
        _lib.dtype_code(qkv.dtype), _lib.stream())
    _lib.check(rc, "ttsp_attn_decode_qkv_rows")
    _stats["causal_rows"] += 1
    return y


def prefill_work_floats(seqlen: int, n_head: int, splits: int) -> int:
    """fp32 elements of the key-split workspace: per split, position and head
    the unnormalised output (128) and the running max and sum (2); 0 unsplit."""
    return 0 if splits <= 1 else splits * seqlen * n_head * (HEAD_DIM + 2)


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
