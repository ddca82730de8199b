"""Greedy decode of a synthetic Dual-AR (slow/fast) transformer on the NF4 kernels.

The reference decodes one audio frame per step (app/engine/graphs.py:76-132,
streamgen.py:654-715): the slow transformer (36 layers at d=2560, GQA
32 q / 8 kv heads of 128, FFN 9728) takes the frame's summed token
embeddings at the next position and yields the semantic token from its head;
its final hidden state, projected to the fast width, primes the fast
transformer at fast position 0 (every fast layer but the last in full, the
last for its KV entries only, graphs.py:76-89); then the fast transformer
runs once per remaining codebook, each step feeding the embedding of the
token it just chose. This module builds that model with seeded random NF4
weights (bitsandbytes layout, double-quant scales) and decodes it greedily -
argmax in place of the sampler, as the benchmark specifies - so the whole
frame is a fixed function of the weights and the starting state.

Every transformer block goes through `fusedlayer.decode_block` (the drop-in
for the reference's fused decode block) and every linear through
`nf4gemv.matmul`; the whole frame is captured once as a HIP graph and
replayed per step, with the position, token and history counters kept on
the device so a replay needs nothing from the host.

Weights are generated on the device by `ttsp_synth_fill` (a counter-based
hash of (seed, index)), so a CPU restatement can regenerate the identical
bytes from `weight_specs()` without copying 2.5 GB.
"""

from __future__ import annotations

from dataclasses import dataclass, field

from ttspipe_amd import _lib

#: absmax of the double-quant scales: s_b = code2[a8[b]] * absmax2 + offset
#: with code2 in [-1, 1], so s_b stays in [offset - absmax2, offset + absmax2].
SCALE_OFFSET = 0.02
ABSMAX2_LO, ABSMAX2_HI = 0.004, 0.008


@dataclass(frozen=True)
class DualARConfig:
    """Shapes of the synthetic frame model (defaults: the benchmark's)."""

    dim: int = 2560
    n_layer: int = 36
    n_head: int = 32
    n_local_heads: int = 8
    intermediate_size: int = 9728
    vocab_size: int = 4096
    fast_dim: int = 1024
    fast_n_layer: int = 4
    fast_n_head: int = 8
    fast_n_local_heads: int = 2
    fast_intermediate_size: int = 3072
    num_codebooks: int = 10
    codebook_size: int = 4096
    head_dim: int = 128
    norm_eps: float = 1e-6
    rope_base: float = 1e6
    max_seq_len: int = 2304
    prefill_len: int = 2048
    qk_norm: bool = True
    seed: int = 20260
    fast_max_len: int = 16

    @property
    def n_tokens(self) -> int:
        """Tokens per frame: the semantic token plus one per codebook."""
        return 1 + self.num_codebooks


#: Padded span lengths a prompt is prefilled at; longer prompts go through in
#: spans of the largest. The reference pads to 1, 2, 4, 8, 16 or 32 rows
#: (graphs.py:137; its MMA kernel takes at most 32); the GEMM here takes any
#: row count, so the buckets go on to 512. A 1-position span runs the decode
#: block (the GEMV), 2 positions the two-row GEMV, 4-64 the few-row kernel.
PREFILL_BUCKETS = (1, 2, 4, 8, 16, 32, 64, 128, 256, 512)

def prefill_spans(n: int):
    """(offset, real length, bucket) of each span an n-token prompt is
    prefilled in: spans of the largest bucket, the rest padded to the
    smallest bucket that holds it (reference: graphs.py:316-320)."""
    if n <= 0:
        return []
    top = PREFILL_BUCKETS[-1]
    full = (n - 1) // top
    sizes = [top] * full + [n - top * full]
    out, off = [], 0
    for size in sizes:
        out.append((off, size, next(b for b in PREFILL_BUCKETS if b >= size)))
        off += size
    return out


SMALL = DualARConfig(dim=512, n_layer=3, n_head=4, n_local_heads=2, intermediate_size=1024,
                     vocab_size=512, fast_dim=256, fast_n_layer=2, fast_n_head=2, fast_n_local_heads=1,
                     fast_intermediate_size=512, num_codebooks=4, codebook_size=512, max_seq_len=320,
                     prefill_len=64, seed=7)


@dataclass
class TensorSpec:
    """One synthetic tensor: `ttsp_synth_fill(n, seed, kind, scale, offset)`.

    kind 0: uint8 bytes; 1 / 3: u * scale + offset (u uniform in [-1, 1)) as
    bf16 / fp32."""

    name: str
    n: int
    seed: int
    kind: int
    scale: float = 1.0
    offset: float = 0.0


@dataclass
class LinearSpec:
    """An NF4 linear [out, in] with double-quant scales (blocksize 64 / 256)."""

    name: str
    out_features: int
    in_features: int
    packed: TensorSpec = field(init=False)
    a8: TensorSpec = field(init=False)
    absmax2: TensorSpec = field(init=False)
    seed: int = 0
    offset: float = SCALE_OFFSET

    def __post_init__(self):
        n = self.out_features * self.in_features
        nblk = n // 64
        mid, half = (ABSMAX2_LO + ABSMAX2_HI) / 2, (ABSMAX2_HI - ABSMAX2_LO) / 2
        self.packed = TensorSpec(self.name + ".packed", n // 2, self.seed, 0)
        self.a8 = TensorSpec(self.name + ".a8", nblk, self.seed + 1, 0)
        self.absmax2 = TensorSpec(self.name + ".absmax2", -(-nblk // 256), self.seed + 2, 3, half, mid)


def _block_specs(prefix, dim, n_head, n_local, inter, head_dim, qk_norm, seed):
    total = (n_head + 2 * n_local) * head_dim
    lin = [LinearSpec(f"{prefix}.wqkv", total, dim, seed=seed + 10),
           LinearSpec(f"{prefix}.wo", dim, n_head * head_dim, seed=seed + 20),
           LinearSpec(f"{prefix}.w1", inter, dim, seed=seed + 30),
           LinearSpec(f"{prefix}.w3", inter, dim, seed=seed + 40),
           LinearSpec(f"{prefix}.w2", dim, inter, seed=seed + 50)]
    vec = [TensorSpec(f"{prefix}.attention_norm", dim, seed + 60, 1, 0.1, 1.0),
           TensorSpec(f"{prefix}.ffn_norm", dim, seed + 61, 1, 0.1, 1.0)]
    if qk_norm:
        vec += [TensorSpec(f"{prefix}.q_norm", head_dim, seed + 62, 1, 0.1, 1.0),
                TensorSpec(f"{prefix}.k_norm", head_dim, seed + 63, 1, 0.1, 1.0)]
    return lin, vec


def weight_specs(cfg: DualARConfig):
    """Every synthetic tensor of the model: (linears, vectors, caches)."""
    s = cfg.seed * 100_000
    linears, vectors = [], []
    for i in range(cfg.n_layer):
        lin, vec = _block_specs(f"layers.{i}", cfg.dim, cfg.n_head, cfg.n_local_heads, cfg.intermediate_size,
                                cfg.head_dim, cfg.qk_norm, s + 1000 * i)
        linears += lin
        vectors += vec
    for i in range(cfg.fast_n_layer):
        lin, vec = _block_specs(f"fast_layers.{i}", cfg.fast_dim, cfg.fast_n_head, cfg.fast_n_local_heads,
                                cfg.fast_intermediate_size, cfg.head_dim, cfg.qk_norm, s + 50_000 + 1000 * i)
        linears += lin
        vectors += vec
    linears += [LinearSpec("output", cfg.vocab_size, cfg.dim, seed=s + 90_000),
                LinearSpec("fast_project_in", cfg.fast_dim, cfg.dim, seed=s + 90_100),
                LinearSpec("fast_output", cfg.codebook_size, cfg.fast_dim, seed=s + 90_200)]
    vectors += [TensorSpec("norm", cfg.dim, s + 90_300, 1, 0.1, 1.0),
                TensorSpec("fast_norm", cfg.fast_dim, s + 90_301, 1, 0.1, 1.0),
                # semantic table then one table per codebook, each [4096, dim]
                TensorSpec("embeddings", cfg.n_tokens * cfg.vocab_size * cfg.dim, s + 90_400, 1, 1.0, 0.0),
                TensorSpec("fast_embeddings", cfg.codebook_size * cfg.fast_dim, s + 90_500, 1, 1.0, 0.0)]
    kv = cfg.n_local_heads * cfg.max_seq_len * cfg.head_dim
    caches = []
    for i in range(cfg.n_layer):
        caches += [TensorSpec(f"layers.{i}.k_cache", kv, s + 95_000 + 2 * i, 1, 1.0, 0.0),
                   TensorSpec(f"layers.{i}.v_cache", kv, s + 95_001 + 2 * i, 1, 1.0, 0.0)]
    return linears, vectors, caches


def max_frames(cfg: DualARConfig) -> int:
    """Frames a decode from position `prefill_len` can run before the slow
    cache is full (frame i writes position prefill_len + i)."""
    return cfg.max_seq_len - cfg.prefill_len


def check_frames(cfg: DualARConfig, n_steps: int) -> None:
    """Raise ValueError unless 1 <= `n_steps` and the frames fit the slow cache."""
    if n_steps < 1 or n_steps > max_frames(cfg):
        raise ValueError(f"{n_steps} frames from position {cfg.prefill_len} run past the "
                         f"{cfg.max_seq_len}-position cache (at most {max_frames(cfg)} fit)")


def first_tokens(cfg: DualARConfig):
    """The frame fed at position `prefill_len` (a fixed, in-range token column)."""
    return [(97 * (c + 1)) % (cfg.vocab_size if c == 0 else cfg.codebook_size) for c in range(cfg.n_tokens)]


class SyntheticDualAR:
    """The frame model on the GPU, weights materialised from `weight_specs`."""

    def __init__(self, cfg: DualARConfig = DualARConfig(), device: str = "cuda"):
        import torch

        from ttspipe_amd import fusedlayer, fusedops, nf4gemv
        from ttspipe_amd.llama import BaseModelArgs, KVCache, TransformerBlock, precompute_freqs_cis
        from ttspipe_amd.quant import NF4_CODE, QuantState, create_dynamic_map

        if not (nf4gemv.install() and fusedops.install()):
            raise RuntimeError("the NF4 kernels are not available (no GPU or library not built)")
        fusedlayer.install()
        self.cfg = cfg
        self.device = torch.device(device)
        self.dtype = torch.bfloat16
        self._lib = _lib.load()
        dev, bf = self.device, self.dtype
        linears, vectors, caches = weight_specs(cfg)
        self.specs = {"linears": linears, "vectors": vectors, "caches": caches}
        code = torch.tensor(NF4_CODE, dtype=torch.float32, device=dev)
        code2 = create_dynamic_map().to(dev)

        def fill(spec: TensorSpec):
            dt = {0: torch.uint8, 1: bf, 3: torch.float32}[spec.kind]
            t = torch.empty(spec.n, dtype=dt, device=dev)
            rc = self._lib.ttsp_synth_fill(t.data_ptr(), spec.n, spec.seed, spec.kind, spec.scale, spec.offset,
                                           _lib.stream())
            _lib.check(rc, "ttsp_synth_fill")
            return t

        self.tensors = {}
        for spec in vectors + caches:
            self.tensors[spec.name] = fill(spec)
        self.quant = {}
        for spec in linears:
            packed, a8, amax2 = fill(spec.packed), fill(spec.a8), fill(spec.absmax2)
            state2 = QuantState(absmax=amax2, shape=(a8.numel(),), code=code2, blocksize=256,
                                quant_type="dynamic", dtype=torch.float32)
            state = QuantState(absmax=a8, shape=(spec.out_features, spec.in_features), code=code, blocksize=64,
                               dtype=bf, offset=torch.tensor(spec.offset, dtype=torch.float32, device=dev),
                               state2=state2)
            self.quant[spec.name] = (packed.view(-1, 1), state)

        def make_linear(name):
            from ttspipe_amd.quant import Linear4bit

            packed, state = self.quant[name]
            out_f, in_f = state.shape
            lin = Linear4bit(in_f, out_f, bias=False, compute_dtype=bf, compress_statistics=True, blocksize=64)
            lin.set_quantized(packed, state)
            if not nf4gemv.prepare(lin):
                raise RuntimeError(f"the NF4 kernel declines {name}")
            return lin

        def make_blocks(prefix, n, dim, n_head, n_local, inter, max_len, k_caches):
            args = BaseModelArgs(dim=dim, n_head=n_head, n_local_heads=n_local, head_dim=cfg.head_dim,
                                 intermediate_size=inter, attention_qk_norm=cfg.qk_norm, norm_eps=cfg.norm_eps,
                                 rope_base=cfg.rope_base, max_seq_len=max_len)
            blocks = []
            for i in range(n):
                with torch.device("meta"):
                    blk = TransformerBlock(args, dtype=bf)
                p = f"{prefix}.{i}"
                a, ff = blk.attention, blk.feed_forward
                a.wqkv, a.wo = make_linear(f"{p}.wqkv"), make_linear(f"{p}.wo")
                ff.w1, ff.w3, ff.w2 = make_linear(f"{p}.w1"), make_linear(f"{p}.w3"), make_linear(f"{p}.w2")
                blk.attention_norm.weight = torch.nn.Parameter(self.tensors[f"{p}.attention_norm"], requires_grad=False)
                blk.ffn_norm.weight = torch.nn.Parameter(self.tensors[f"{p}.ffn_norm"], requires_grad=False)
                if cfg.qk_norm:
                    a.q_norm.weight = torch.nn.Parameter(self.tensors[f"{p}.q_norm"], requires_grad=False)
                    a.k_norm.weight = torch.nn.Parameter(self.tensors[f"{p}.k_norm"], requires_grad=False)
                cache = KVCache.__new__(KVCache)
                torch.nn.Module.__init__(cache)
                if k_caches:
                    kc = self.tensors[f"{p}.k_cache"].view(1, n_local, max_len, cfg.head_dim)
                    vc = self.tensors[f"{p}.v_cache"].view(1, n_local, max_len, cfg.head_dim)
                else:
                    kc = torch.zeros(1, n_local, max_len, cfg.head_dim, dtype=bf, device=dev)
                    vc = torch.zeros_like(kc)
                cache.register_buffer("k_cache", kc)
                cache.register_buffer("v_cache", vc)
                a.kv_cache = cache
                blocks.append(blk)
            return blocks

        self.layers = make_blocks("layers", cfg.n_layer, cfg.dim, cfg.n_head, cfg.n_local_heads,
                                  cfg.intermediate_size, cfg.max_seq_len, True)
        self.fast_layers = make_blocks("fast_layers", cfg.fast_n_layer, cfg.fast_dim, cfg.fast_n_head,
                                       cfg.fast_n_local_heads, cfg.fast_intermediate_size, cfg.fast_max_len, False)
        self.output = make_linear("output")
        self.fast_project_in = make_linear("fast_project_in")
        self.fast_output = make_linear("fast_output")

        self.freqs = precompute_freqs_cis(cfg.max_seq_len, cfg.head_dim, cfg.rope_base, dtype=bf).to(dev)
        self.fast_freqs = precompute_freqs_cis(cfg.fast_max_len, cfg.head_dim, cfg.rope_base, dtype=bf).to(dev)
        self.mask = torch.ones(1, 1, 1, cfg.max_seq_len, dtype=torch.bool, device=dev)
        self.fast_mask = torch.ones(1, 1, 1, cfg.fast_max_len, dtype=torch.bool, device=dev)

        # device-side state of the decode loop
        self.pos = torch.zeros(1, dtype=torch.long, device=dev)
        self.tokens = torch.zeros(cfg.n_tokens, dtype=torch.int32, device=dev)
        self.step_index = torch.zeros(1, dtype=torch.long, device=dev)
        self.history = None
        self.fast_pos = [torch.full((1,), i, dtype=torch.long, device=dev) for i in range(cfg.num_codebooks)]
        self.freq_row = torch.empty(1, cfg.head_dim // 2, 2, dtype=bf, device=dev)

        x1 = torch.empty(1, 1, cfg.dim, dtype=bf, device=dev)
        f1 = torch.empty(1, 1, cfg.fast_dim, dtype=bf, device=dev)
        nchunk = -(-cfg.max_seq_len // fusedlayer.CHUNK)
        fchunk = -(-cfg.fast_max_len // fusedlayer.CHUNK)
        self.ws = [fusedlayer.make_workspace(self.layers[0], x1, nchunk, with_out=True) for _ in range(2)]
        self.fws = [fusedlayer.make_workspace(self.fast_layers[0], f1, fchunk, with_out=True) for _ in range(2)]
        self.x = x1
        self.logits = torch.empty(1, cfg.vocab_size, dtype=bf, device=dev)
        self.fast_h = torch.empty(1, 1, cfg.fast_dim, dtype=bf, device=dev)
        self.fast_logits = torch.empty(1, cfg.codebook_size, dtype=bf, device=dev)
        # the codebook loop as one launch (ttsp_fast_steps), where it serves these
        # shapes, on request: the same bits, but measured slower on MI355X than
        # the graph-replayed launches (its grid barriers cost more than a launch)
        self.use_fast_steps = False
        self.fast_sync = torch.zeros(_lib.FAST_SYNC_WORDS, dtype=torch.int32, device=dev)
        self._fast_args = self._fast_steps_args()
        self.graph = None
        # prompt prefill: the fork's causal mask rows, one captured graph per bucket
        self.causal = torch.tril(torch.ones(cfg.max_seq_len, cfg.max_seq_len, dtype=torch.bool, device=dev))
        self.prefill_graphs = {}
        self.prefill_first_graphs = {}
        self.prefill_token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.reset()

    # ------------------------------------------------------------------ state

    def reset(self, n_steps: int | None = None) -> None:
        """Position `prefill_len`, the first frame's tokens, an empty history
        of `n_steps` rows (default: 256, or as many frames as the cache holds
        if fewer). Raises ValueError when `n_steps` frames would run past the
        cache (the kernels would clamp the position, not fail)."""
        import torch

        if n_steps is None:
            n_steps = min(256, max_frames(self.cfg))
        check_frames(self.cfg, n_steps)
        self.pos.fill_(self.cfg.prefill_len)
        # the first frame's rotary row; each frame's last launch writes the next one's
        torch.index_select(self.freqs, 0, self.pos, out=self.freq_row)
        self.tokens.copy_(torch.tensor(first_tokens(self.cfg), dtype=torch.int32))
        self.step_index.zero_()
        if self.history is None or self.history.shape[0] < n_steps:
            self.history = torch.zeros(n_steps, self.cfg.n_tokens, dtype=torch.int32, device=self.device)
            self.graph = None  # a captured frame holds the old history's address: capture again
        else:
            self.history.zero_()

    # ------------------------------------------------------------------- step

    def _check(self, rc, what):
        _lib.check(rc, what)

    def _fast_kv_only(self, blk, x, freqs, pos):
        """The last fast layer at the prime position: norm, wqkv, KV write."""
        from ttspipe_amd import nf4gemv

        a = blk.attention
        ws = self.fws[0]
        qkv = nf4gemv.matmul_fused(a.wqkv, x, norm_weight=blk.attention_norm.weight, eps=blk.attention_norm.eps,
                                   out=ws["qkv"])
        if qkv is None:
            raise RuntimeError("the fused matmul declined the fast prime's wqkv")
        qn = a.q_norm if self.cfg.qk_norm else None
        kn = a.k_norm if self.cfg.qk_norm else None
        rc = self._lib.ttsp_qk_rope_kv(
            qkv.data_ptr(), _lib.ptr(None if qn is None else qn.weight), _lib.ptr(None if kn is None else kn.weight),
            float(self.cfg.norm_eps), freqs.data_ptr(), _lib.DT_BF16,
            pos.data_ptr(), ws["q"].data_ptr(), a.kv_cache.k_cache.data_ptr(), a.kv_cache.v_cache.data_ptr(),
            a.n_head, a.n_local_heads, a.kv_cache.k_cache.shape[2], _lib.DT_BF16, _lib.stream())
        self._check(rc, "ttsp_qk_rope_kv")

    def _run_blocks(self, blocks, workspaces, x, freqs, mask, pos):
        from ttspipe_amd import fusedlayer

        for i, blk in enumerate(blocks):
            y = fusedlayer.decode_block(blk, x, freqs, mask, pos, workspace=workspaces[i % 2])
            if y is None:
                raise RuntimeError("decode_block declined a layer of the synthetic model")
            x = y
        return x

    @staticmethod
    def _fused(linear, x, norm_weight, eps, out):
        """RMSNorm of x folded into the matmul (one launch, the unfused pair's bits)."""
        from ttspipe_amd import nf4gemv

        y = nf4gemv.matmul_fused(linear, x, norm_weight=norm_weight, eps=eps, out=out)
        if y is None:
            raise RuntimeError("the fused matmul declined a head of the synthetic model")
        return y

    def _fast_steps_args(self):
        """`ttsp_fast_steps`' arguments for this model's fast transformer (the
        codebook loop in one launch), or None where that launch does not serve
        its shapes: the loop then runs launch by launch, with the same bits."""
        import torch

        cfg = self.cfg
        n_steps = cfg.num_codebooks - 1
        if n_steps < 1 or cfg.num_codebooks > cfg.fast_max_len:  # fast positions 1 .. n_steps
            return None
        lins = [self.fast_output]
        for blk in self.fast_layers:
            a, ff = blk.attention, blk.feed_forward
            lins += [a.wqkv, a.wo, ff.w1, ff.w3, ff.w2]
        fast = [getattr(lin, "_nf4_fast", None) for lin in lins]
        if any(f is None for f in fast) or len({(f["bs"], f["bs2"], f["nested"]) for f in fast}) != 1:
            return None
        norms = [blk.attention_norm for blk in self.fast_layers] + [blk.ffn_norm for blk in self.fast_layers]
        if cfg.qk_norm:
            norms += [blk.attention.q_norm for blk in self.fast_layers] + [blk.attention.k_norm for blk in self.fast_layers]
        if any(float(m.eps) != float(cfg.norm_eps) for m in norms):
            return None
        bs, bs2 = fast[0]["bs"], fast[0]["bs2"]
        grid = self._lib.ttsp_fast_steps_grid(cfg.fast_dim, cfg.fast_n_head, cfg.fast_n_local_heads,
                                              cfg.fast_intermediate_size, cfg.codebook_size, cfg.fast_max_len,
                                              cfg.fast_n_layer, bs)
        ftype = _lib.dtype_code(self.fast_freqs.dtype)
        if grid <= 0 or ftype is None or not self.fast_freqs.is_contiguous():
            return None

        def weight(lin):
            f = lin._nf4_fast
            return _lib.Nf4Weight(f["w"], f["a8"] or None, f["amax"], f["code2"] or None, f["offset"])

        layers = (_lib.FastLayer * cfg.fast_n_layer)()
        for i, blk in enumerate(self.fast_layers):
            a, ff = blk.attention, blk.feed_forward
            layers[i] = _lib.FastLayer(
                weight(a.wqkv), weight(a.wo), weight(ff.w1), weight(ff.w3), weight(ff.w2),
                blk.attention_norm.weight.data_ptr(), blk.ffn_norm.weight.data_ptr(),
                a.q_norm.weight.data_ptr() if cfg.qk_norm else None,
                a.k_norm.weight.data_ptr() if cfg.qk_norm else None,
                a.kv_cache.k_cache.data_ptr(), a.kv_cache.v_cache.data_ptr())
        nbytes = self._lib.ttsp_fast_steps_work_bytes(cfg.fast_dim, cfg.fast_n_head, cfg.fast_n_local_heads,
                                                     cfg.fast_intermediate_size)
        work = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return {"layers": layers, "head": weight(self.fast_output), "work": work, "grid": grid, "ftype": ftype,
                "lut": fast[0]["lut"], "bs": bs, "bs2": bs2, "n_steps": n_steps}

    def fast_steps_failed(self) -> int:
        """Grid-barrier waits of `ttsp_fast_steps` that gave up since the model
        was built (0 unless the launch's workgroups were not all resident)."""
        return int(self.fast_sync[_lib.FAST_SYNC_FAILED].item())

    def check_fast_steps(self) -> None:
        """Raise if a `ttsp_fast_steps` barrier wait gave up (its frames' tokens are then not valid)."""
        n = self.fast_steps_failed()
        if n:
            raise RuntimeError(f"ttsp_fast_steps: {n} grid-barrier waits gave up; the decoded tokens are not valid")

    def _codebook_steps(self, st) -> None:
        """The codebook loop as one `ttsp_fast_steps` launch: steps 1 .. n-1 at
        fast positions 1 .. n-1 from `fast_h`, tokens[2 ..] and fast_logits."""
        cfg, f = self.cfg, self._fast_args
        rc = self._lib.ttsp_fast_steps(
            f["layers"], cfg.fast_n_layer, f["head"], self.tensors["fast_norm"].data_ptr(),
            self.tensors["fast_embeddings"].data_ptr(), f["lut"].data_ptr(), self.fast_freqs.data_ptr(), f["ftype"],
            self.fast_h.data_ptr(), f["work"].data_ptr(), self.fast_sync.data_ptr(), self.fast_logits.data_ptr(),
            self.tokens.data_ptr(), cfg.fast_dim, cfg.fast_n_head, cfg.fast_n_local_heads, cfg.fast_intermediate_size,
            cfg.codebook_size, cfg.fast_max_len, 1, f["n_steps"], float(cfg.norm_eps), f["bs"], f["bs2"],
            _lib.DT_BF16, st)
        self._check(rc, "ttsp_fast_steps")

    def _codebook_loop(self, st) -> None:
        """The codebook loop launch by launch: per step the fast blocks, the
        fast head, the greedy token and (but for the last) its embedding row."""
        cfg, lib = self.cfg, self._lib
        emb = self.tensors["fast_embeddings"].data_ptr()
        for i in range(1, cfg.num_codebooks):
            x = self._run_blocks(self.fast_layers, self.fws, self.fast_h, self.fast_freqs[i], self.fast_mask,
                                 self.fast_pos[i])
            self._fused(self.fast_output, x.view(1, 1, -1), self.tensors["fast_norm"], cfg.norm_eps, self.fast_logits)
            tok = self.tokens[i + 1:].data_ptr()
            if i + 1 < cfg.num_codebooks:  # the token and the next codebook step's embedding
                rc = lib.ttsp_argmax_embed(self.fast_logits.data_ptr(), cfg.codebook_size, _lib.DT_BF16, tok, None,
                                           emb, cfg.codebook_size, cfg.fast_dim, self.fast_h.data_ptr(), st)
                self._check(rc, "ttsp_argmax_embed")
            else:
                rc = lib.ttsp_argmax(self.fast_logits.data_ptr(), cfg.codebook_size, _lib.DT_BF16, tok, st)
                self._check(rc, "ttsp_argmax")

    def step(self) -> None:
        """One frame: tokens (device) at position pos -> next frame's tokens; pos += 1."""
        cfg, lib, st = self.cfg, self._lib, _lib.stream()
        # slow transformer
        rc = lib.ttsp_embed_sum(self.tensors["embeddings"].data_ptr(), self.tokens.data_ptr(), cfg.n_tokens,
                                cfg.vocab_size, cfg.dim, self.x.data_ptr(), _lib.DT_BF16, st)
        self._check(rc, "ttsp_embed_sum")
        # (freq_row holds the rotary row of pos: reset() or the last frame wrote it)
        h = self._run_blocks(self.layers, self.ws, self.x, self.freq_row, self.mask, self.pos).view(1, 1, -1)
        # the final norm runs inside both consumers (head and fast projection)
        norm, eps = self.tensors["norm"], cfg.norm_eps
        self._fused(self.output, h, norm, eps, self.logits)
        # fast transformer: prime at fast position 0 with the projected hidden state
        fx = self._fused(self.fast_project_in, h, norm, eps, self.fast_h)
        p0 = self.fast_pos[0]
        x = self._run_blocks(self.fast_layers[:-1], self.fws, fx, self.fast_freqs[0], self.fast_mask, p0)
        self._fast_kv_only(self.fast_layers[-1], x, self.fast_freqs[0], p0)
        # codebook 0 is the semantic token, clamped into the codebook; its
        # embedding starts the fast steps (one launch: argmax, clamp, row)
        emb = self.tensors["fast_embeddings"].data_ptr()
        rc = lib.ttsp_argmax_embed(self.logits.data_ptr(), cfg.vocab_size, _lib.DT_BF16, self.tokens.data_ptr(),
                                   self.tokens[1:].data_ptr(), emb, cfg.codebook_size, cfg.fast_dim,
                                   self.fast_h.data_ptr(), st)
        self._check(rc, "ttsp_argmax_embed")
        if self.use_fast_steps and self._fast_args is not None:
            self._codebook_steps(st)
        else:
            self._codebook_loop(st)
        # bookkeeping on the device: history row, step and position, the next rotary row
        rc = lib.ttsp_frame_advance(self.tokens.data_ptr(), cfg.n_tokens, self.history.data_ptr(),
                                    self.history.shape[0], self.step_index.data_ptr(), self.pos.data_ptr(),
                                    self.freqs.data_ptr(), self.freqs.shape[0], self.freqs[0].numel(),
                                    self.freq_row.data_ptr(), st)
        self._check(rc, "ttsp_frame_advance")

    # ---------------------------------------------------------------- prefill

    def prefill_forward(self, inp, pos, last, width: int | None = None) -> None:
        """The slow transformer over a prompt span: `inp` (n_tokens, n) int32
        token rows at positions `pos` (n,) int64 write their KV entries; the
        final norm and output head run on span index `last` (1,) int64, whose
        greedy token lands in `prefill_token` and logits in `logits`
        (reference: DecodeGraphs._prefill_body, graphs.py:219-231, through
        BaseTransformer.forward_generate with the whole cache as the window).
        `width`: the attention window, the first `width` cache positions
        (default the whole cache; a span that starts at position 0 sees
        nothing past its own end, so its window can stop there)."""
        import torch

        from ttspipe_amd import fusedlayer

        cfg = self.cfg
        width = cfg.max_seq_len if width is None else width
        n = inp.shape[1]
        if inp.dtype != torch.int32 or inp.shape[0] != cfg.n_tokens or inp.stride(1) != 1:
            raise ValueError("inp must be int32 (n_tokens, n) with contiguous rows")
        # every position's summed codebook embeddings, as a decode step sums them
        x = torch.empty(1, n, cfg.dim, dtype=self.dtype, device=inp.device)
        rc = self._lib.ttsp_embed_sum_rows(self.tensors["embeddings"].data_ptr(), inp.data_ptr(), inp.stride(0),
                                           cfg.n_tokens, n, cfg.vocab_size, cfg.dim, x.data_ptr(),
                                           _lib.dtype_code(self.dtype), _lib.stream())
        self._check(rc, "ttsp_embed_sum_rows")
        freqs = self.freqs.index_select(0, pos)
        mask = self.causal.index_select(0, pos)[None, None, :, :width]
        # each block hands the next its attention RMSNorm, written by w2's
        # split-K reduce where that serves the span length
        xn = None
        for i, blk in enumerate(self.layers):
            nxt = self.layers[i + 1].attention_norm if i + 1 < len(self.layers) else None
            r = fusedlayer.prefill_block_chain(blk, x, freqs, mask, pos, xn=xn, next_norm=nxt, causal=True)
            if r is None:
                x, xn = blk(x, freqs, mask, pos), None
            else:
                x, xn = r
        h = x.index_select(1, last)
        self._fused(self.output, h, self.tensors["norm"], cfg.norm_eps, self.logits)
        rc = self._lib.ttsp_argmax(self.logits.data_ptr(), cfg.vocab_size, _lib.DT_BF16, self.prefill_token.data_ptr(),
                                   _lib.stream())
        self._check(rc, "ttsp_argmax")

    def capture_prefill(self, buckets=None, first: bool = False) -> None:
        """One graph per padded span length (after an eager warm-up of each);
        `first`: the graphs for a span at position 0, whose attention window
        ends with the span (`prefill_first_graphs`), else the whole-cache ones
        (`prefill_graphs`).

        The warm-up runs the span at positions 0..b-1, which writes those KV
        rows of every slow layer; they are saved first and put back after, so
        a bucket can be captured while a prompt is live in the cache (the
        logits and `prefill_token` the warm-up leaves are overwritten by the
        next span anyway)."""
        import torch

        graphs = self.prefill_first_graphs if first else self.prefill_graphs
        for b in buckets or PREFILL_BUCKETS:
            if b in graphs or b > self.cfg.max_seq_len:
                continue
            width = b if first else None
            inp = torch.zeros(self.cfg.n_tokens, b, dtype=torch.int32, device=self.device)
            pos = torch.arange(b, dtype=torch.long, device=self.device)
            last = torch.zeros(1, dtype=torch.long, device=self.device)
            saved = [(blk.attention.kv_cache.k_cache[:, :, :b].clone(), blk.attention.kv_cache.v_cache[:, :, :b].clone())
                     for blk in self.layers]
            self.prefill_forward(inp, pos, last, width)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.prefill_forward(inp, pos, last, width)
            for blk, (kc, vc) in zip(self.layers, saved):
                blk.attention.kv_cache.k_cache[:, :, :b].copy_(kc)
                blk.attention.kv_cache.v_cache[:, :, :b].copy_(vc)
            del saved
            graphs[b] = (g, inp, pos, last)

    def prefill(self, tokens, start: int, graphed: bool = True) -> bool:
        """KV entries for `tokens` (n_tokens, n) int32 at [start, start + n),
        in spans of the largest bucket and a last span padded to a bucket (the
        padding repeats the last real token; its KV entries land past the
        prompt, where decoding overwrites them before reading them); the last
        real position's token in `prefill_token`. False (nothing done) when
        the padded span runs past the cache (reference: graphs.py:304-335).
        A span at position 0 attends over its own positions only (the window
        of the reference's causal mask there), not the whole cache."""
        import torch

        n = tokens.shape[-1]
        spans = prefill_spans(n)
        if not spans or start + spans[-1][0] + spans[-1][2] > self.cfg.max_seq_len:
            return False
        for off, size, b in spans:
            first = start + off == 0
            if graphed:
                graphs = self.prefill_first_graphs if first else self.prefill_graphs
                if b not in graphs:
                    self.capture_prefill([b], first=first)
                g, inp, pos, last = graphs[b]
            else:
                inp = torch.empty(self.cfg.n_tokens, b, dtype=torch.int32, device=self.device)
                pos = torch.empty(b, dtype=torch.long, device=self.device)
                last = torch.empty(1, dtype=torch.long, device=self.device)
            inp[:, :size].copy_(tokens[:, off:off + size])
            inp[:, size:].copy_(tokens[:, off + size - 1:off + size].expand(-1, b - size))
            torch.arange(start + off, start + off + b, out=pos)
            last.fill_(size - 1)
            if graphed:
                g.replay()
            else:
                self.prefill_forward(inp, pos, last, b if first else None)
        return True

    def capture(self) -> None:
        """Record one step as a HIP graph (after a warm-up step outside capture)."""
        import torch

        self.step()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g

    def decode(self, n_steps: int, graphed: bool = True):
        """Reset, then n_steps frames; returns the [n_steps, n_tokens] token history (host)."""
        import torch

        # reset first: a reset that grows the history drops a captured frame
        # (it writes into the old history), so capture after it; capture()
        # runs one eager frame, so reset again
        self.reset(n_steps)
        if graphed and self.graph is None:
            self.capture()
            self.reset(n_steps)
        for _ in range(n_steps):
            if graphed:
                self.graph.replay()
            else:
                self.step()
        torch.cuda.synchronize()
        self.check_fast_steps()
        return self.history[:n_steps].cpu().numpy()


def linear_bytes(spec: LinearSpec) -> int:
    """Algorithmic bytes of one batch-1 NF4 matmul: packed codes, uint8 scale
    indices, fp32 absmax2, the 256-entry code2 and offset, x and y (bf16)."""
    return (spec.packed.n + spec.a8.n + 4 * spec.absmax2.n + 4 * 257 + 2 * spec.in_features
            + 2 * spec.out_features)


def step_bytes(cfg: DualARConfig, pos: int) -> int:
    """Algorithmic HBM bytes of one frame at slow position `pos`: every linear
    each time it is applied, the KV rows attention reads and writes, the
    embedding rows gathered and the norm weights."""
    linears, _, _ = weight_specs(cfg)
    by = {s.name: linear_bytes(s) for s in linears}
    slow = sum(v for k, v in by.items() if k.startswith("layers."))
    fast_layer = [sum(v for k, v in by.items() if k.startswith(f"fast_layers.{i}.")) for i in range(cfg.fast_n_layer)]
    fast_passes = cfg.num_codebooks - 1
    prime = sum(fast_layer[:-1]) + by[f"fast_layers.{cfg.fast_n_layer - 1}.wqkv"]
    heads = by["output"] + by["fast_project_in"] + fast_passes * by["fast_output"]
    kv_row = cfg.head_dim * 2
    slow_kv = cfg.n_layer * cfg.n_local_heads * kv_row * (2 * (pos + 1) + 2)
    fast_kv = sum(cfg.fast_n_layer * cfg.fast_n_local_heads * kv_row * (2 * (i + 1) + 2) for i in range(1, cfg.num_codebooks))
    emb = 2 * (cfg.n_tokens * cfg.dim + fast_passes * cfg.fast_dim)
    norms = 2 * cfg.dim * (2 * cfg.n_layer + 1) + 2 * cfg.fast_dim * (2 * cfg.fast_n_layer * (fast_passes + 1) + fast_passes)
    return slow + fast_passes * sum(fast_layer) + prime + heads + slow_kv + fast_kv + emb + norms


def benchmark(n_steps: int = 256, warmup: int = 8, cfg: DualARConfig = DualARConfig(),
              fast_steps: bool = False) -> dict:
    """ms per frame over `n_steps` graph-replayed greedy steps (one MI355X);
    fast_steps True runs the codebook loop as one `ttsp_fast_steps` launch."""
    import torch

    model = SyntheticDualAR(cfg)
    model.use_fast_steps = fast_steps
    one_launch = fast_steps and model._fast_args is not None
    model.reset(max(n_steps, warmup))  # the history the graph writes: grown before capture
    model.capture()
    model.reset(max(n_steps, warmup))
    for _ in range(warmup):
        model.graph.replay()
    torch.cuda.synchronize()
    model.reset(n_steps)
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(n_steps):
        model.graph.replay()
    end.record(stream)
    end.synchronize()
    model.check_fast_steps()
    ms = start.elapsed_time(end) / n_steps
    hist = model.history[:n_steps].cpu().numpy()
    nbytes = sum(step_bytes(cfg, cfg.prefill_len + i) for i in range(n_steps)) / n_steps
    del model
    torch.cuda.empty_cache()
    return {"ms_per_step": round(ms, 4), "steps": n_steps, "bytes_per_step": int(nbytes), "fast_steps": one_launch,
            "achieved_gbs": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "tokens_first_step": hist[0].tolist(), "tokens_last_step": hist[-1].tolist(),
            "config": f"slow {cfg.n_layer}x d{cfg.dim} ({cfg.n_head}q/{cfg.n_local_heads}kv x{cfg.head_dim}, "
                      f"FFN {cfg.intermediate_size}), fast {cfg.fast_n_layer}x d{cfg.fast_dim} "
                      f"({cfg.fast_n_head}q/{cfg.fast_n_local_heads}kv, FFN {cfg.fast_intermediate_size}), "
                      f"{cfg.num_codebooks} codebooks of {cfg.codebook_size}, KV from {cfg.prefill_len}"}


def prefill_benchmark(n_tokens: int = 512, reps: int = 20, cfg: DualARConfig = DualARConfig()) -> dict:
    """ms to prefill an `n_tokens` prompt (one captured bucket graph per span)
    through the slow transformer, from position 0, synthetic tokens."""
    import torch

    model = SyntheticDualAR(cfg)
    g = torch.Generator(device=model.device).manual_seed(cfg.seed)
    toks = torch.randint(0, cfg.codebook_size, (cfg.n_tokens, n_tokens), generator=g, device=model.device,
                         dtype=torch.int32)
    model.capture_prefill(sorted({b for _, _, b in prefill_spans(n_tokens)}))
    assert model.prefill(toks, 0)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(reps):
        model.prefill(toks, 0)
    end.record(stream)
    end.synchronize()
    ms = start.elapsed_time(end) / reps
    token = int(model.prefill_token.item())
    del model
    torch.cuda.empty_cache()
    return {"tokens": n_tokens, "ms": round(ms, 3), "tokens_per_s": round(n_tokens / ms * 1e3, 1),
            "first_token": token, "layers": cfg.n_layer}


def prefill_tail_benchmark(sizes=(1, 2, 4, 8, 16, 32), start: int = 512, reps: int = 20,
                           cfg: DualARConfig = DualARConfig()) -> dict:
    """ms to prefill a prompt tail of n tokens after `start` cached positions
    (the case after a prefix-cache hit, reference streamgen.py:184-253), one
    captured bucket graph per size, through the 36-layer slow transformer."""
    import torch

    model = SyntheticDualAR(cfg)
    g = torch.Generator(device=model.device).manual_seed(cfg.seed + 1)
    stream = torch.cuda.current_stream()
    out = []
    for n in sizes:
        toks = torch.randint(0, cfg.codebook_size, (cfg.n_tokens, n), generator=g, device=model.device,
                             dtype=torch.int32)
        bucket = prefill_spans(n)[-1][2]
        model.capture_prefill([bucket])
        assert model.prefill(toks, start)
        torch.cuda.synchronize()
        torch.cuda._sleep(200_000)  # the host's first submission overlaps this, not the timed region
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(reps):
            model.prefill(toks, start)
        t1.record(stream)
        t1.synchronize()
        out.append({"tokens": n, "bucket": bucket, "ms": round(t0.elapsed_time(t1) / reps, 3)})
    del model
    torch.cuda.empty_cache()
    return {"after_cached_positions": start, "layers": cfg.n_layer, "points": out}
