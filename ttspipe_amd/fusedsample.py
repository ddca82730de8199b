"""Top-k / top-p sampling of one logit row in one HIP launch.

Drop-in for the reference's `app/engine/fusedsample.py` (`MAX_TOP_K`,
`available`, `sample`): the fork's sampler - temperature, top-k, top-p, then a
draw - which the fork runs as a full sort, a softmax, a cumsum, a scatter and
a second softmax. Here one workgroup holds the row in LDS, finds the k-th
largest value by bisection over its 16-bit pattern, gathers the k winners in
index order, ranks them by pairwise counting, and draws
`argmax(v / temperature - log(-log(u)))` over those that survive the top-p
cut, with `u` one uniform number per vocabulary index from `torch.rand`.
That is the Gumbel form of the fork's `argmax(probs / Exp(1))`: exact
sampling from the truncated, tempered distribution (reference:
fusedsample.py:1-19, 225-257). The cumulative mass is summed in fp32 where the
fork's fp16 cumsum rounds, so a draw whose mass lands exactly on the top-p
boundary can differ; the distribution is the same.
"""

from __future__ import annotations

from ttspipe_amd import _lib

#: Largest `top_k` the kernel takes; larger requests use the caller's sampler.
MAX_TOP_K = 64

#: Longest row the kernel takes (the row is held in LDS); `sample` returns None
#: for a longer one and the caller's sampler runs.
MAX_VOCAB = 32768


def available() -> bool:
    """True when the HIP library is loadable on a GPU machine."""
    if not _lib.gpu_present():
        return False
    try:
        _lib.lib()
    except Exception:  # noqa: BLE001 - the caller's sampler still works
        return False
    return True


def sample(logits, temperature, top_p, top_k, uniform=None):
    """The fork's `sample(...)[0]`: an int32 tensor of shape (1,) holding the
    drawn index, or None for a row longer than `MAX_VOCAB`. `temperature`/`top_p` are one-element tensors, `top_k` a
    one-element int64 tensor, all on the logits' device (so a captured graph
    can change them in place); `uniform` (optional) supplies the per-index
    uniform numbers (default: `torch.rand`)."""
    import torch

    row = logits.reshape(-1)
    if row.numel() > MAX_VOCAB:
        return None
    dt = _lib.dtype_code(row.dtype)
    if dt not in (_lib.DT_F16, _lib.DT_BF16):
        row, dt = row.to(torch.float16), _lib.DT_F16
    row = row.contiguous()
    temp = temperature.reshape(-1)[:1].to(row.dtype).contiguous()
    topp = top_p.reshape(-1)[:1].to(row.dtype).contiguous()
    topk = top_k.reshape(-1)[:1].to(torch.int64).contiguous()
    if uniform is None:
        uniform = torch.rand(row.numel(), device=row.device, dtype=torch.float32)
    elif uniform.dtype != torch.float32 or uniform.numel() != row.numel():
        raise ValueError("uniform must hold one float32 per logit")
    out = torch.empty(1, dtype=torch.int32, device=row.device)
    rc = _lib.lib().ttsp_sample_topk(row.data_ptr(), row.numel(), dt, temp.data_ptr(), topp.data_ptr(),
                                     topk.data_ptr(), uniform.contiguous().data_ptr(), out.data_ptr(), _lib.stream())
    _lib.check(rc, "ttsp_sample_topk")
    return out
