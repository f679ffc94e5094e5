"""MI355X-native LLM decode hot path: hand-written HIP kernels for gfx950 behind
a C ABI (include/mxdecode.h), driven from Python through ctypes.

    _lib    ctypes binding of libmxdecode.so (no fallback: it raises if missing)
    ops     operator surface named after the reference's Metal operators
    quant   int8 block-32 weight converter
    build   hipcc driver producing the in-tree libmxdecode.so
"""

__all__ = ["_lib", "ops", "quant"]
