"""The reference's Dequantizer registry, with device dequantizers.

tensor/quant_registry.go:10-73 keeps a name -> Dequantizer map:
Dequantize(src []byte, dst []float32), BlockSize(), BitsPerWeight(), with
RegisterQuantType (panics on an empty name, a nil dequantizer or a second
registration), GetQuantType and ListQuantTypes (sorted).  The built-in
names are "Q4_0", "Q8_0", "Q4_K", "Q5_K", "Q6_K", "Q5_0", "FP8_E4M3",
"FP8_E5M2" (tensor/quant_registry.go:231-240), "AWQ_4"
(tensor/quantized_awq.go:306-308), "W8A8" (tensor/quantized_w8a8.go:320-322)
and "IQ3_S" (tensor/iq3_storage.go:184-186).

Here every built-in name maps to a libzt_hip.so entry point that decodes the
same bytes on the GPU, bit for bit with the reference; ROCmEngine.dequantize
uploads the source bytes and runs it.  Formats registered later with
register_quant_type carry their own device function.
"""
from __future__ import annotations

import ctypes as C
import threading
from dataclasses import dataclass
from typing import Callable

import numpy as np


# (lib, src_host, src_dev, dst, stream) -> hipError_t.  src_host is the host
# copy of the source bytes (sizes and headers are checked there), src_dev its
# device copy (a uint8 torch tensor), dst the fp32 device tensor of n values.
DeviceFn = Callable[[object, np.ndarray, object, object, int], int]


@dataclass(frozen=True)
class DeviceDequantizer:
    """One registered format: BlockSize / BitsPerWeight as the reference's
    Dequantizer reports them, and the device decode."""

    name: str
    block_size: int
    bits_per_weight: int
    run: DeviceFn
    empty_ok: bool = True  # IQ3_S: the reference rejects zero elements (NewIQ3SStorageFromRaw)


def _short(name: str, need: int, got: int) -> ValueError:
    # errShortData, tensor/quant_registry.go:242-245
    return ValueError(f"tensor: {name} data too short: need {need} bytes, got {got}")


def _q4_0(lib, src, sd, dst, s):
    n = dst.numel()
    need = -(-n // 32) * 18
    if src.size < need:
        raise _short("Q4_0", need, src.size)
    return lib.zt_dequant_q4raw_f32(sd.data_ptr(), src.size, dst.data_ptr(), n, s)


def _q8_0(lib, src, sd, dst, s):
    n = dst.numel()
    need = -(-n // 32) * 36
    if src.size < need:
        raise _short("Q8_0", need, src.size)
    return lib.zt_dequant_q8_f32(sd.data_ptr(), dst.data_ptr(), n, s)


def _blocks(fn: str, name: str, vals: int, block_bytes: int) -> DeviceFn:
    """Raw K-quant / Q5_0 blocks: the device dequantizers decode whole
    blocks (rows of one block each), so a partial last block is decoded into
    a padded buffer and the first n values kept, as the reference's
    Dequantize writes only n."""

    def run(lib, src, sd, dst, s):
        import torch

        n = dst.numel()
        nb = -(-n // vals)
        if src.size < nb * block_bytes:
            raise _short(name, nb * block_bytes, src.size)
        if n == nb * vals:
            return getattr(lib, fn)(sd.data_ptr(), dst.data_ptr(), nb, vals, s)
        tmp = torch.empty(nb * vals, dtype=torch.float32, device=dst.device)
        rc = getattr(lib, fn)(sd.data_ptr(), tmp.data_ptr(), nb, vals, s)
        if rc == 0:
            dst.copy_(tmp[:n])
        return rc

    return run


def _w8a8(lib, src, sd, dst, s):
    # the Q8_0 36-byte groups (tensor/quantized_w8a8.go:285-316)
    n = dst.numel()
    need = -(-n // 32) * 36
    if src.size < need:
        raise _short("W8A8", need, src.size)
    if n == 0:
        return 0
    return lib.zt_dequant_q8_f32(sd.data_ptr(), dst.data_ptr(), n, s)


def _iq3s(lib, src, sd, dst, s):
    # NewIQ3SStorageFromRaw (tensor/iq3_storage.go:98-111): a positive count
    # and ceil(n / 256) super-blocks of 110 bytes
    n = dst.numel()
    if n <= 0:
        raise ValueError(f"numElements must be positive, got {n}")
    nb = -(-n // 256)
    if src.size < nb * 110:
        raise ValueError(f"IQ3_S raw data too short: need {nb * 110} bytes for {nb} blocks, got {src.size}")
    return lib.zt_dequant_iq3s_f32(sd.data_ptr(), src.size, dst.data_ptr(), n, s)


def _awq4(lib, src, sd, dst, s):
    n = dst.numel()
    g, ng = C.c_int(0), C.c_int(0)
    if lib.zt_awq4_wire_header(src.ctypes.data, src.size, n, C.byref(g), C.byref(ng)) != 0:
        raise ValueError("tensor: AWQ_4 header does not match the destination, or the data is short")
    if n == 0:
        return 0
    return lib.zt_dequant_awq4_f32(sd.data_ptr(), src.size, dst.data_ptr(), n, g.value, ng.value, s)


def _fp8(e5m2: int, name: str) -> DeviceFn:
    def run(lib, src, sd, dst, s):
        n = dst.numel()
        if src.size < 4 + n:
            raise _short(name, 4 + n, src.size)
        return lib.zt_dequant_fp8_f32(sd.data_ptr(), src.size, dst.data_ptr(), n, e5m2, s)

    return run


_mu = threading.Lock()
_registry: dict[str, DeviceDequantizer] = {}


def register_quant_type(name: str, d: DeviceDequantizer) -> None:
    """RegisterQuantType (tensor/quant_registry.go:28-44)."""
    if not name:
        raise ValueError("tensor: RegisterQuantType called with empty name")
    if d is None:
        raise ValueError("tensor: RegisterQuantType called with nil Dequantizer")
    with _mu:
        if name in _registry:
            raise ValueError("tensor: RegisterQuantType called twice for " + name)
        _registry[name] = d


def get_quant_type(name: str) -> tuple[DeviceDequantizer | None, bool]:
    """GetQuantType (tensor/quant_registry.go:46-53)."""
    with _mu:
        d = _registry.get(name)
    return d, d is not None


def list_quant_types() -> list[str]:
    """ListQuantTypes (tensor/quant_registry.go:55-66), sorted."""
    with _mu:
        return sorted(_registry)


for _name, _bs, _bits, _fn in [
    ("Q4_0", 32, 4, _q4_0),
    ("Q8_0", 32, 8, _q8_0),
    ("Q4_K", 256, 4, _blocks("zt_dequant_q4k_f32", "Q4_K", 256, 144)),
    ("Q5_K", 256, 5, _blocks("zt_dequant_q5k_f32", "Q5_K", 256, 176)),
    ("Q6_K", 256, 6, _blocks("zt_dequant_q6k_f32", "Q6_K", 256, 210)),
    ("Q5_0", 32, 5, _blocks("zt_dequant_q5_0_f32", "Q5_0", 32, 22)),
    ("FP8_E4M3", 1, 8, _fp8(0, "FP8_E4M3")),
    ("FP8_E5M2", 1, 8, _fp8(1, "FP8_E5M2")),
    ("AWQ_4", 128, 4, _awq4),
    ("W8A8", 32, 8, _w8a8),
    ("IQ3_S", 256, 3, _iq3s),
]:
    register_quant_type(_name, DeviceDequantizer(_name, _bs, _bits, _fn, _name != "IQ3_S"))
