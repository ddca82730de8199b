"""MI355X-native (gfx950) NF4 decode hot path of a Dual-AR TTS transformer.

Drop-in modules with the reference's Python-facing signatures:

* `nf4gemv`    - NF4 GEMV (decode) / MFMA GEMM (prefill) on bitsandbytes-layout weights
* `fusedops`   - fused RMSNorm and rotary embedding
* `fusedlayer` - a decode step through one transformer block
* `quant`      - NF4 quantisation and the `Linear4bit` / `QuantState` objects
* `llama`      - the transformer block classes the patches apply to
* `dualar`     - the synthetic Dual-AR decode (slow + fast transformer, greedy)

The kernels live in `libttsp_hip.so` (`csrc/*.hip`, built by `build.py`) and
are reached through the C-ABI declared in `include/ttsp_hip.h`.
"""

__all__ = ["nf4gemv", "fusedops", "fusedlayer", "quant", "llama", "dualar"]
