"""saient_quartz_amd -- MI355X (gfx950) quantized dequant-GEMV backend for Quartz.

The product is the C-ABI shared library libquartz_hip.so (include/quartz_hip.h).
This module binds it with ctypes so tests and benchmarks call exactly the
symbols a Rust/C host would.  Importing the package does not touch the GPU;
`lib()` raises if the library has not been built -- there is no CPU fallback.
"""
from .api import (  # noqa: F401
    GGML_TYPES,
    QH_OK,
    QuartzHipError,
    block_elems,
    lib,
    lib_path,
    type_size,
)
