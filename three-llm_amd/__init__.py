"""three-llm_amd: MI355X-native per-token decoder path of three-llm.

The compute lives in libtlm.so (hand-written HIP kernels for gfx950 behind the
C ABI declared in include/tlm.h).  This package is the host side: the ctypes
binding (tlm), the runner that mirrors the reference's DecoderTSLRunner
controls (runner), the restated generate loop and host sampling (generate),
the recipe/RoPE tables (recipe), canonical weights (weights) and local
Hugging Face checkpoints (checkpoint) and the byte-level BPE tokenizer
(tokenizer).
"""
from . import checkpoint, generate, recipe, runner, tlm, tokenizer, weights  # noqa: F401

__all__ = ["checkpoint", "generate", "recipe", "runner", "tlm", "tokenizer", "weights"]
