"""MI355X (gfx950) quantized-GEMV decode path of RunIT, behind its dispatch API.

`runit_mac_amd.dispatch` mirrors RunIT's `crates/kernels` dispatch functions
over the C ABI in include/runit_hip.h (librunit_hip.so + lib/kernels/*.hsaco).
"""
from . import dispatch  # noqa: F401

__all__ = ["dispatch"]
