"""three-llm_amd: MI355X-native per-token decoder path of three-llm.

The compute lives in libtlm.so (hand-written HIP kernels for gfx950 behind the
C ABI declared in include/tlm.h).  This package is the host side: the ctypes
binding, the runner that mirrors the reference's DecoderTSLRunner controls, and
the restated generate loop.
"""
from . import recipe  # noqa: F401

__all__ = ["recipe"]
