"""ztensor_amd: MI355X (gfx950) implementation of ztensor's quantized-weight
decode matmul path (Q4_0, Q8_0, IQ4_NL, W4A16 GPTQ/AWQ, ternary).

The compute lives in libzt_hip.so (ztensor_amd/csrc, C ABI in
include/zt_hip.h); this package is the host-side mirror of the reference's
engine / storage surface and the ctypes binding.
"""
from . import _lib, synth  # noqa: F401
from ._lib import ZTError, load  # noqa: F401

__all__ = ["load", "ZTError", "synth"]
