"""Python host binding of libuocr_hip (MI355X INT4 MoE expert path).

The product is the C-ABI library `lib/libuocr_hip.so` (declared in
`include/uocr_hip/moe_capi.h`); this package only binds it with ctypes for
tests, the benchmark and Python callers. Importing it never falls back to a
CPU path: `load()` raises if the library has not been built.
"""
from ._lib import HipError, load, lib_path  # noqa: F401
from .layer import MoELayer, MoELayerInt4, QMatrix  # noqa: F401
from . import ops, synth  # noqa: F401
