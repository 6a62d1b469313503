"""lama32_mojo_amd -- MI355X-native INT8 group-quantized (W8A32) linear layers.

The compute path is libq8hip.so (hand-written gfx950 HIP kernels behind a
C ABI, include/q8hip.h).  ``q8hip`` is its ctypes binding; ``q8`` mirrors the
reference's host interface (Weights, Acts, mm_q8_op, pack_q8, ...).
"""

from . import q8hip  # noqa: F401
from .q8hip import LIB_PATH, Buffer, Context, Q8Error  # noqa: F401

__all__ = ["q8hip", "LIB_PATH", "Buffer", "Context", "Q8Error"]
