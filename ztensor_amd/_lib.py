"""ctypes binding of libzt_hip.so.

This is the Python twin of the reference's purego layer
(internal/cuda/kernels/purego.go:230-260, internal/hip/kernels/purego.go:44-107):
the library is opened once, every symbol is resolved once into a table, and
every call passes only integers and pointers.  A nonzero return is a
hipError_t and becomes ZTError, which is what the reference's checkKernel
turns into a Go error (internal/cuda/kernels/elementwise_purego.go:11-16).

There is no fallback: if the library is missing, load() raises.
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libzt_hip.so"

P = C.c_void_p
I = C.c_int
L = C.c_long

# name -> (restype, argtypes); mirrors include/zt_hip.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "zt_abi_version": (I, []),
    "zt_gemm_q4_f32": (I, [P, P, P, I, I, I, I, P]),
    "zt_gemm_q4_f16": (I, [P, P, P, I, I, I, I, P]),
    "zt_gemm_q4_group_f32": (I, [P, I, P, I, P]),
    "zt_dequant_q4_f32": (I, [P, P, L, I, P]),
    "zt_q4_gpu_data_offset": (L, [L]),
    "zt_q4_gpu_bytes": (L, [L]),
    "zt_q4_raw_to_gpu": (None, [P, L, P]),
    "zt_gemm_iq4nl_f32": (I, [P, P, P, I, I, I, I, P]),
    "zt_gemm_iq4nl_f16": (I, [P, P, P, I, I, I, I, P]),
    "zt_dequant_iq4nl_f32": (I, [P, P, L, I, P]),
    "zt_iq4nl_tiled_bytes": (L, [I, I]),
    "zt_iq4nl_tiled_scale_bytes": (L, [I, I]),
    "zt_iq4nl_tile": (I, [P, I, I, I, P, P, P]),
    "zt_gemm_iq4nlt_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_iq4nlt_f16": (I, [P, P, P, P, I, I, I, P, L, P]),
    "zt_iq4nl_raw_to_gpu": (None, [P, L, P]),
    "zt_gemm_q8_f32": (I, [P, P, P, I, I, I, P]),
    "zt_gemm_q8sep_f32": (I, [P, P, P, I, I, I, L, P]),
    "zt_dequant_q8_f32": (I, [P, P, L, P]),
    "zt_dequant_q8sep_f32": (I, [P, P, L, L, P]),
    "zt_q8_repack": (I, [P, P, L, P]),
    "zt_q8_gpu_data_offset": (L, [L]),
    "zt_q8_gpu_bytes": (L, [L]),
    "zt_q8_raw_to_gpu": (None, [P, L, P]),
    "zt_gemm_q8gguf_f32": (I, [P, P, P, I, I, I, L, P]),
    "zt_dequant_q8gguf_f32": (I, [P, P, L, L, P]),
    "zt_q8gguf_gpu_data_offset": (L, [L]),
    "zt_q8gguf_gpu_bytes": (L, [L]),
    "zt_q8gguf_raw_to_gpu": (None, [P, L, P]),
    "zt_gemm_w4a16_f32": (I, [P, P, P, P, P, I, I, I, I, P]),
    "zt_dequant_w4_f32": (I, [P, P, P, P, L, I, P]),
    "zt_dequant_w4_f16": (I, [P, P, P, P, L, I, P]),
    "zt_dequant_q4_f16": (I, [P, P, L, I, P]),
    "zt_w4a16_pack_szr": (I, [P, P, I, I, I, P, P]),
    "zt_gemv_w4a16sz_f32": (I, [P, P, P, P, I, I, I, P]),
    "zt_gemm_w4a16sz_f32": (I, [P, P, P, P, I, I, I, I, P]),
    "zt_bench_stream_read": (I, [P, L, P, P]),
    "zt_ternary_gemv_i8_group": (I, [P, I, P, P, I, P]),
    "zt_gemv_w4a16sz_group_f32": (I, [P, I, P, I, I, P]),
    "zt_w4a16_tiled_bytes": (L, [I, I]),
    "zt_w4a16_sz_bytes": (L, [I, I, I]),
    "zt_w4a16_tile": (I, [P, P, P, I, I, I, P, P, P]),
    "zt_gemm_w4a16t_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_w4a16t_f32": (I, [P, P, P, P, I, I, I, I, P, L, P]),
    "zt_q4_tiled_bytes": (L, [I, I]),
    "zt_q4_tiled_scale_bytes": (L, [I, I]),
    "zt_q4_tile": (I, [P, I, I, I, P, P, P]),
    "zt_gemm_q4t_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_q4t_f32": (I, [P, P, P, P, I, I, I, P, L, P]),
    "zt_gemm_q4t_f32_noalloc": (I, [P, P, P, P, I, I, I, P]),
    "zt_q8_tiled_bytes": (L, [I, I]),
    "zt_q8_tiled_scale_bytes": (L, [I, I]),
    "zt_q8_tile": (I, [P, I, I, L, P, P, P]),
    "zt_q8gguf_tile": (I, [P, I, I, L, P, P, P]),
    "zt_gemm_q8t_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_q8t_f32": (I, [P, P, P, P, I, I, I, P, L, P]),
    "zt_q4k_tiled_bytes": (L, [I, I]),
    "zt_q4k_tiled_header_bytes": (L, [I, I]),
    "zt_q4k_tile": (I, [P, I, I, P, P, P]),
    "zt_gemm_q4kt_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_q4kt_f32": (I, [P, P, P, P, I, I, I, P, L, P]),
    "zt_q5_0_tiled_bytes": (L, [I, I]),
    "zt_q5_0_tiled_scale_bytes": (L, [I, I]),
    "zt_q5_0_tiled_qh_bytes": (L, [I, I]),
    "zt_q5_0_tile": (I, [P, I, I, L, L, P, P, P, P]),
    "zt_gemm_q5_0t_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_q5_0t_f32": (I, [P, P, P, P, P, I, I, I, P, L, P]),
    "zt_q5k_tiled_bytes": (L, [I, I]),
    "zt_q5k_tiled_header_bytes": (L, [I, I]),
    "zt_q5k_tiled_qh_bytes": (L, [I, I]),
    "zt_q5k_tile": (I, [P, I, I, P, P, P, P]),
    "zt_gemm_q5kt_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_q5kt_f32": (I, [P, P, P, P, P, I, I, I, P, L, P]),
    "zt_q6k_tiled_bytes": (L, [I, I]),
    "zt_q6k_tiled_scale_bytes": (L, [I, I]),
    "zt_q6k_tile": (I, [P, I, I, P, P, P]),
    "zt_gemm_q6kt_workspace_bytes": (L, [I, I, I]),
    "zt_gemm_q6kt_f32": (I, [P, P, P, P, I, I, I, P, L, P]),
    "zt_ternary_gemv_f32": (I, [P, P, P, I, I, P]),
    "zt_ternary_gemv_i8": (I, [P, P, P, P, P, I, I, P]),
    "zt_dequant_ternary_f32": (I, [P, P, I, I, P]),
    "zt_ternary_repack_rows": (None, [P, L, L, P]),
    "zt_gemv_q4k_f32": (I, [P, P, P, I, I, P]),
    "zt_gemv_q5k_f32": (I, [P, P, P, I, I, P]),
    "zt_gemv_q6k_f32": (I, [P, P, P, I, I, P]),
    "zt_q6k_split_bytes": (L, [I, I]),
    "zt_q6k_split": (I, [P, I, I, P, P]),
    "zt_gemv_q6ks_f32": (I, [P, P, P, I, I, P]),
    "zt_gemv_q5_0_f32": (I, [P, P, P, I, I, I, I, P]),
    "zt_dequant_q4k_f32": (I, [P, P, I, I, P]),
    "zt_dequant_q5k_f32": (I, [P, P, I, I, P]),
    "zt_dequant_q6k_f32": (I, [P, P, I, I, P]),
    "zt_dequant_q5_0_f32": (I, [P, P, I, I, P]),
    "zt_q5_0_gpu_qh_offset": (L, [L]),
    "zt_q5_0_gpu_qs_offset": (L, [L]),
    "zt_q5_0_gpu_bytes": (L, [L]),
    "zt_q5_0_raw_to_gpu": (None, [P, L, P]),
    "zt_dequant_q4raw_f32": (I, [P, L, P, L, P]),
    "zt_awq4_wire_header": (I, [P, L, L, P, P]),
    "zt_dequant_awq4_f32": (I, [P, L, P, L, I, I, P]),
    "zt_dequant_fp8_f32": (I, [P, L, P, L, I, P]),
    "zt_dequant_iq3s_f32": (I, [P, L, P, L, P]),
    "zt_gemm_int8_f32": (I, [P, P, P, I, I, I, P]),
    "zt_gemm_int4_f32": (I, [P, P, P, P, P, I, I, I, I, P]),
    "zt_gemm_int4_f32_rmul": (I, [P, P, P, P, P, I, I, I, I, P]),
}

HIP_ERROR_INVALID_VALUE = 1
GROUP_MAX = 8  # ZT_GROUP_MAX
NOALLOC_SCRATCH_BYTES = 8 << 20  # ZT_NOALLOC_SCRATCH_BYTES
HIP_ERROR_OUT_OF_MEMORY = 2


class Q4GemvDesc(C.Structure):
    """zt_q4_gemv_desc: one matrix of a grouped Q4_0 GEMV."""

    _fields_ = [("A", C.c_void_p), ("data_offset", C.c_long), ("y", C.c_void_p), ("rows", C.c_int),
                ("reserved", C.c_int)]


def q4_gemv_descs(entries) -> C.Array:
    """A host array of zt_q4_gemv_desc from (A, data_offset, y, rows) tuples."""
    arr = (Q4GemvDesc * max(1, len(entries)))()
    for i, (a, off, y, rows) in enumerate(entries):
        arr[i].A, arr[i].data_offset, arr[i].y, arr[i].rows, arr[i].reserved = a, off, y, rows, 0
    return arr


class TernaryGemvDesc(C.Structure):
    """zt_ternary_gemv_desc: one matrix of a grouped BitNet GEMV."""

    _fields_ = [("W", C.c_void_p), ("w_scale", C.c_void_p), ("y", C.c_void_p), ("rows", C.c_int),
                ("reserved", C.c_int)]


def ternary_gemv_descs(entries) -> C.Array:
    """A host array of zt_ternary_gemv_desc from (W, w_scale, y, rows) tuples."""
    arr = (TernaryGemvDesc * max(1, len(entries)))()
    for i, (w, ws, y, rows) in enumerate(entries):
        arr[i].W, arr[i].w_scale, arr[i].y, arr[i].rows, arr[i].reserved = w, ws, y, rows, 0
    return arr


class W4A16GemvDesc(C.Structure):
    """zt_w4a16_gemv_desc: one matrix of a grouped batch-1 W4A16 GEMV."""

    _fields_ = [("W", C.c_void_p), ("szr", C.c_void_p), ("y", C.c_void_p), ("rows", C.c_int), ("reserved", C.c_int)]


def w4a16_gemv_descs(entries) -> C.Array:
    """A host array of zt_w4a16_gemv_desc from (W, szr, y, rows) tuples."""
    arr = (W4A16GemvDesc * max(1, len(entries)))()
    for i, (w, szr, y, rows) in enumerate(entries):
        arr[i].W, arr[i].szr, arr[i].y, arr[i].rows, arr[i].reserved = w, szr, y, rows, 0
    return arr


class ZTError(RuntimeError):
    """A libzt_hip entry point returned a nonzero hipError_t."""

    def __init__(self, name: str, code: int):
        super().__init__(f"{name} failed: hipError_t {code}")
        self.name = name
        self.code = code


class _Lib:
    def __init__(self, path: Path):
        if not path.exists():
            raise FileNotFoundError(
                f"{path} is not built; run `python -m ztensor_amd.build` (no CPU fallback exists)"
            )
        self.path = path
        self.cdll = C.CDLL(str(path))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(self.cdll, name)
            fn.restype = res
            fn.argtypes = args
            setattr(self, name, fn)

    def call(self, name: str, *args) -> None:
        """Calls an int-returning entry point and raises ZTError on failure."""
        rc = getattr(self, name)(*args)
        if rc != 0:
            raise ZTError(name, rc)


_once = threading.Lock()
_lib: _Lib | None = None


def load() -> _Lib:
    """Opens the library once (the sync.Once of the reference loader)."""
    global _lib
    with _once:
        if _lib is None:
            _lib = _Lib(LIB_PATH)
    return _lib
