"""numpy front end of the C oracle (`nf4_oracle.c`) - TEST INFRASTRUCTURE.

Arrays in, arrays out; 16-bit element types travel as uint16 bit patterns.
Also restates, in numpy, the pieces of the reference's data format the C file
does not (NF4 packing and the two conversions), so tests can pin each side
against the other.

Parity status of each function is stated in the C file and in the tests that
pin it; the whole-model decode emulation is in `dualar_oracle.py`.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
DT_F16, DT_BF16, DT_F32 = 0, 1, 2

#: bitsandbytes' NF4 code points as the reference holds them (app/engine/nf4gemv.py:75-92).
NF4_CODE = np.array(
    [-1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453, -0.28444138169288635,
     -0.18477343022823334, -0.09105003625154495, 0.0, 0.07958029955625534, 0.16093020141124725,
     0.24611230194568634, 0.33791524171829224, 0.44070982933044434, 0.5626170039176941,
     0.7229568362236023, 1.0],
    dtype=np.float32,
)

_lib = None


def lib():
    global _lib
    if _lib is None:
        path = HERE / "liboracle.so"
        if not path.exists():
            from oracle import build

            build.build()
        _lib = ctypes.CDLL(str(path))
        vp, i, f, ll, d = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong, ctypes.c_double
        sig = {
            "orc_f32_to_bf16": ([f], ctypes.c_uint16),
            "orc_f32_to_f16": ([f], ctypes.c_uint16),
            "orc_exp_cw": ([f], f),
            "orc_rsqrt_rn": ([f], f),
            "orc_fma16_chain": ([vp, vp, vp, i, vp], None),
            "orc_nf4_dequant": ([vp, vp, vp, vp, f, vp, vp, i, ll, i, i], None),
            "orc_nf4_gemm_ref": ([vp, i, vp, vp, vp, vp, f, vp, vp, i, i, i, i, i, i], None),
            "orc_gemv_emul": ([vp, i, vp, vp, vp, vp, f, vp, vp, vp, i, i, i, i, i, i, i], None),
            "orc_rms_norm_ref": ([vp, vp, vp, i, i, f, i], None),
            "orc_rms_norm_emul": ([vp, vp, vp, i, i, f, i], None),
            "orc_rope": ([vp, vp, i, vp, ll, i, i, i, i], None),
            "orc_qk_rope_kv": ([vp, vp, vp, f, vp, i, ll, vp, vp, vp, i, i, i, i], None),
            "orc_attn_ref": ([vp, vp, vp, ll, vp, i, i, i, f, i], None),
            "orc_attn_emul": ([vp, vp, vp, ll, vp, i, i, i, i, f, i], None),
            "orc_synth_fill": ([vp, ll, ctypes.c_uint64, i, f, f], None),
            "orc_embed_sum": ([vp, vp, i, i, i, vp, i], None),
            "orc_argmax": ([vp, i, i], i),
        }
        for name, (args, res) in sig.items():
            fn = getattr(_lib, name)
            fn.argtypes = args
            fn.restype = res
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype=None):
    if a is None:
        return None
    a = np.ascontiguousarray(a if dtype is None else a.astype(dtype, copy=False))
    return a


# ------------------------------------------------------------ conversions

def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even to bf16 bit patterns (numpy restatement)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_to_f32(h) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def to_f32(h, dt) -> np.ndarray:
    if dt == DT_F32:
        return np.asarray(h, dtype=np.float32)
    return f16_to_f32(h) if dt == DT_F16 else bf16_to_f32(h)


def from_f32(x, dt) -> np.ndarray:
    if dt == DT_F32:
        return np.asarray(x, dtype=np.float32)
    return f32_to_f16(x) if dt == DT_F16 else f32_to_bf16(x)


# ------------------------------------------------------------ NF4 format

def unpack_nf4(packed) -> np.ndarray:
    """Codes of the flattened weight: byte j = q[2j] << 4 | q[2j+1] (high nibble first)."""
    b = np.asarray(packed, dtype=np.uint8).reshape(-1)
    q = np.empty(b.size * 2, dtype=np.uint8)
    q[0::2] = b >> 4
    q[1::2] = b & 15
    return q


def pack_nf4(q) -> np.ndarray:
    q = np.asarray(q, dtype=np.uint8).reshape(-1)
    return ((q[0::2] << 4) | q[1::2]).astype(np.uint8)


def scales(a8, amax, code2, offset, bs2) -> np.ndarray:
    """Per-block scale: plain absmax, or code2[a8] * absmax2[b // bs2] + offset (two fp32 roundings)."""
    if a8 is None:
        return np.asarray(amax, dtype=np.float32)
    b = np.arange(a8.size)
    prod = (np.asarray(code2, np.float32)[a8.astype(np.int64)] * np.asarray(amax, np.float32)[b // bs2]).astype(np.float32)
    return (prod + np.float32(offset)).astype(np.float32)


def nf4_dequant(W, A8, AMAX, CODE2, offset, out_dtype, n, bs, bs2=256, lut=NF4_CODE):
    lib()
    out = np.empty(n, dtype=np.float32 if out_dtype == DT_F32 else np.uint16)
    W, A8, AMAX, CODE2, lut = _c(W, np.uint8), _c(A8, np.uint8), _c(AMAX, np.float32), _c(CODE2, np.float32), _c(lut, np.float32)
    _lib.orc_nf4_dequant(_p(W), _p(A8), _p(AMAX), _p(CODE2), float(offset), _p(lut), _p(out), out_dtype, n, bs, bs2)
    return out


def nf4_gemm_ref(X, dt, W, A8, AMAX, CODE2, offset, M, K, N, bs, bs2=256, lut=NF4_CODE, exact=False):
    """fp64 [N, M] of x . dequant(W)^T; weights rounded to dt (bitsandbytes'
    dequantise-then-matmul) or, with exact=True, code*scale unrounded."""
    lib()
    Y = np.empty((N, M), dtype=np.float64)
    X, W, A8, AMAX, CODE2, lut = _c(X), _c(W, np.uint8), _c(A8, np.uint8), _c(AMAX, np.float32), _c(CODE2, np.float32), _c(lut, np.float32)
    _lib.orc_nf4_gemm_ref(_p(X), dt, _p(W), _p(A8), _p(AMAX), _p(CODE2), float(offset), _p(lut), _p(Y), M, K, N, bs, bs2,
                          -1 if exact else dt)
    return Y


def gemv_emul(X, dt, W, A8, AMAX, CODE2, offset, M, K, bs, KS, J, bs2=256, R=None, epi=0, lut=NF4_CODE):
    lib()
    Y = np.empty(M, dtype=np.uint16)
    X, W, A8, AMAX, CODE2, R, lut = _c(X), _c(W, np.uint8), _c(A8, np.uint8), _c(AMAX, np.float32), _c(CODE2, np.float32), _c(R), _c(lut, np.float32)
    _lib.orc_gemv_emul(_p(X), dt, _p(W), _p(A8), _p(AMAX), _p(CODE2), float(offset), _p(lut), _p(Y), _p(R), epi, M, K, bs, bs2, KS, J)
    return Y


def rms_norm_ref(X, Wt, rows, D, eps, dt):
    lib()
    Y = np.empty(rows * D, dtype=np.float64)
    X, Wt = _c(X), _c(Wt)
    _lib.orc_rms_norm_ref(_p(X), _p(Wt), _p(Y), rows, D, float(eps), dt)
    return Y


def rms_norm_emul(X, Wt, rows, D, eps, dt):
    lib()
    Y = np.empty(rows * D, dtype=np.uint16)
    X, Wt = _c(X), _c(Wt)
    _lib.orc_rms_norm_emul(_p(X), _p(Wt), _p(Y), rows, D, float(eps), dt)
    return Y


def rope(X, F, ftype, half_dim, heads, seq, dt):
    lib()
    X, F = _c(X), _c(F)
    Y = np.empty(X.size, dtype=np.uint16)
    _lib.orc_rope(_p(X), _p(F), ftype, _p(Y), X.size // 2, half_dim, heads, seq, dt)
    return Y


def qk_rope_kv(QKV, QW, KW, eps, F, ftype, pos, Q, KC, VC, nh, nkv, max_len, dt):
    """In place on Q, KC, VC (uint16 arrays), like the kernel."""
    lib()
    QKV, QW, KW, F = _c(QKV), _c(QW), _c(KW), _c(F)
    for a in (Q, KC, VC):
        assert a.flags.c_contiguous
    _lib.orc_qk_rope_kv(_p(QKV), _p(QW), _p(KW), float(eps), _p(F), ftype, int(pos), _p(Q), _p(KC), _p(VC), nh, nkv, max_len, dt)


def attn_ref(Q, KC, VC, L, nh, nkv, max_len, scale, dt):
    lib()
    Y = np.empty(nh * 128, dtype=np.float64)
    Q, KC, VC = _c(Q), _c(KC), _c(VC)
    _lib.orc_attn_ref(_p(Q), _p(KC), _p(VC), int(L), _p(Y), nh, nkv, max_len, float(scale), dt)
    return Y


def attn_emul(Q, KC, VC, pos, nh, nkv, max_len, nchunk, scale, dt):
    lib()
    Y = np.empty(nh * 128, dtype=np.uint16)
    Q, KC, VC = _c(Q), _c(KC), _c(VC)
    _lib.orc_attn_emul(_p(Q), _p(KC), _p(VC), int(pos), _p(Y), nh, nkv, max_len, nchunk, float(scale), dt)
    return Y


def fma16_chain(a, b, c):
    """fma(a.hi, b.hi, fma(a.lo, b.lo, c)) with IEEE fmaf, a/b packed fp16 pairs (uint32)."""
    lib()
    a, b, c = _c(a, np.uint32), _c(b, np.uint32), _c(c, np.float32)
    out = np.empty(c.size, dtype=np.float32)
    _lib.orc_fma16_chain(_p(a), _p(b), _p(c), c.size, _p(out))
    return out


def synth_fill(n, seed, kind, scale=1.0, offset=0.0):
    lib()
    out = np.empty(n, dtype={0: np.uint8, 1: np.uint16, 2: np.uint16, 3: np.float32}[kind])
    _lib.orc_synth_fill(_p(out), n, seed, kind, float(scale), float(offset))
    return out


def exp_cw(x) -> np.ndarray:
    lib()
    return np.array([_lib.orc_exp_cw(float(v)) for v in np.asarray(x, np.float32).ravel()], dtype=np.float32)


def embed_sum(E, tok, vocab, D, dt):
    lib()
    E, tok = _c(E), _c(tok, np.int32)
    out = np.empty(D, dtype=np.uint16)
    _lib.orc_embed_sum(_p(E), _p(tok), tok.size, vocab, D, _p(out), dt)
    return out


def argmax(X, dt) -> int:
    lib()
    X = _c(X)
    return int(_lib.orc_argmax(_p(X), X.size, dt))


def sample_topk_ref(logits, temperature: float, top_p: float, top_k: int, u):
    """The fork's top-k / top-p draw as the reference's fused sampler computes
    it (app/engine/fusedsample.py:55-223), in float64: the top_k largest
    logits (ties by lowest index) sorted descending; the first and every one
    whose inclusive cumulative probability under softmax(logits) is <= top_p
    kept; returns (index, kept indices, cumulative probabilities, scores) with
    index = argmax over the kept of l / max(temperature, 1e-5) -
    log(-log(max(u, 1e-20))), ties to the lowest index."""
    l = np.asarray(logits, np.float64)
    V = l.size
    k = int(min(max(int(top_k), 1), 64, V))
    order = np.lexsort((np.arange(V), -l))[:k]  # value descending, then index ascending
    m = l.max()
    p = np.exp(l[order] - m) / np.exp(l - m).sum()
    c = np.cumsum(p)
    keep = np.zeros(k, bool)
    keep[0] = True
    keep[1:] = c[1:] <= top_p
    kept = order[keep]
    uu = np.maximum(np.asarray(u, np.float64)[kept], 1e-20)
    scores = l[kept] / max(float(temperature), 1e-5) - np.log(-np.log(uu))
    mx = scores.max()
    cand = kept[scores == mx]
    best = int(cand.min())
    return best, kept, c, scores
