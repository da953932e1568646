"""molla_amd -- MI355X (gfx950) decode hot path for molla.

GGUF block-quantized matvec (Q8_0, Q4_0, Q4_K, Q6_K) and the Llama decoder
layer, as hand-written HIP kernels behind the C ABI in include/molla_mi.h
(libmolla_mi.so).  `molla_amd.gpu` and `molla_amd.block` mirror the
reference's device entry points over that ABI.
"""

from ._lib import LIB_PATH, MiError, lib  # noqa: F401

__version__ = "0.1.0"
