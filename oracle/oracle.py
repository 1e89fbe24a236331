"""ctypes wrapper of liboracle.so, the CPU restatement of the reference path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker and the CPU baseline.  Never
imported by the ztensor_amd package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

P, L, I, F = C.c_void_p, C.c_int64, C.c_int, C.c_float
_SIG = {
    "orc_f16_to_f32": (F, [C.c_uint16]),
    "orc_f16_bits_to_f32_xblas": (F, [C.c_uint16]),
    "orc_q4_dequant": (None, [P, L, P]),
    "orc_q4_gpu_data_offset": (L, [L]),
    "orc_q4_raw_to_gpu": (None, [P, L, P]),
    "orc_q4_dot_block": (F, [P, F, P, I]),
    "orc_q4_dot_row": (F, [P, P, I]),
    "orc_gemm_f32_q4_nt": (None, [L, L, L, P, P, P, I]),
    "orc_q8_dequant": (None, [P, L, P]),
    "orc_gemm_f32_q8_nt": (None, [L, L, L, P, P, P, I]),
    "orc_iq4nl_table_copy": (None, [P]),
    "orc_iq4nl_dequant": (None, [P, L, P]),
    "orc_gptq_dequant": (None, [P, P, P, L, L, I, P]),
    "orc_awq_dequant": (None, [P, P, P, L, L, P]),
    "orc_f16_slice": (None, [P, L, P]),
    "orc_sgemm_simd": (None, [L, L, L, P, P, P]),
    "orc_w4a16_matmul_gptq": (None, [P, P, P, P, P, L, L, L, L, P, P]),
    "orc_iq4nl_matmul": (None, [P, P, P, L, L, L, P, P]),
    "orc_ternary_get": (I, [P, L]),
    "orc_ternary_gemv": (None, [P, P, L, L, P]),
    "orc_ternary_repack_rows": (None, [P, L, L, P]),
    "orc_ternary_gemv_i8": (None, [P, P, F, F, L, L, P, P]),
    "orc_kq_scales_mins": (None, [P, P, P]),
    "orc_q4k_dequant": (None, [P, L, P]),
    "orc_q5k_dequant": (None, [P, L, P]),
    "orc_q6k_dequant": (None, [P, L, P]),
    "orc_gemm_f32_kq_nt": (None, [I, L, L, L, P, P, P, I]),
    "orc_q5_0_dequant": (None, [P, L, P]),
    "orc_q5_0_gpu_qh_offset": (L, [L]),
    "orc_q5_0_gpu_qs_offset": (L, [L]),
    "orc_q5_0_raw_to_gpu": (None, [P, L, P]),
    "orc_gemm_f32_q5_0_nt": (None, [L, L, L, P, P, P, P, P]),
    "orc_gguf_q8_0_dequant": (None, [P, L, P]),
    "orc_gemm_f32_mmap_nt": (I, [I, L, L, L, P, P, P, I, P]),
    "orc_awq4_wire_dequant": (I, [P, L, P, L]),
    "orc_fp8_dequant": (I, [P, L, P, L, I]),
    "orc_iq3s_dequant": (I, [P, L, P, L]),
    "orc_gemm_int4_f32": (I, [P, P, P, P, P, L, L, L, L, I]),
    "orc_gemm_int4_f32_rmul": (I, [P, P, P, P, P, L, L, L, L, I]),
    "orc_gemm_int8_f32": (None, [P, P, P, L, L, L, I]),
}

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
        for n, (r, a) in _SIG.items():
            f = getattr(_lib, n)
            f.restype, f.argtypes = r, a
    return _lib


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def nthreads() -> int:
    return len(os.sched_getaffinity(0))


# ---- thin typed wrappers ------------------------------------------------

def f16_to_f32(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, np.uint16)
    out = np.empty(bits.size, np.float32)
    lib().orc_f16_slice(_p(bits), bits.size, _p(out))
    return out


def q4_dequant(raw: np.ndarray, nelem: int) -> np.ndarray:
    out = np.empty(nelem, np.float32)
    lib().orc_q4_dequant(_p(raw), nelem, _p(out))
    return out


def q4_raw_to_gpu(raw: np.ndarray, nblk: int) -> np.ndarray:
    off = lib().orc_q4_gpu_data_offset(nblk)
    out = np.empty(off + 16 * nblk, np.uint8)
    lib().orc_q4_raw_to_gpu(_p(raw), nblk, _p(out))
    return out


def gemm_f32_q4_nt(a: np.ndarray, raw: np.ndarray, m: int, n: int, k: int, threads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    c = np.empty(m * n, np.float32)
    lib().orc_gemm_f32_q4_nt(m, n, k, _p(a), _p(raw), _p(c), threads)
    return c


def q8_dequant(raw: np.ndarray, nelem: int) -> np.ndarray:
    out = np.empty(nelem, np.float32)
    lib().orc_q8_dequant(_p(raw), nelem, _p(out))
    return out


def gemm_f32_q8_nt(a: np.ndarray, raw: np.ndarray, m: int, n: int, k: int, threads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    c = np.empty(m * n, np.float32)
    lib().orc_gemm_f32_q8_nt(m, n, k, _p(a), _p(raw), _p(c), threads)
    return c


def iq4nl_table() -> np.ndarray:
    t = np.empty(16, np.float32)
    lib().orc_iq4nl_table_copy(_p(t))
    return t


def iq4nl_dequant(raw: np.ndarray, nelem: int) -> np.ndarray:
    out = np.empty(nelem, np.float32)
    lib().orc_iq4nl_dequant(_p(raw), nelem, _p(out))
    return out


def gptq_dequant(data, scales, zeros, nelem: int, group: int, bits: int = 4) -> np.ndarray:
    data = np.ascontiguousarray(data, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    zeros = np.ascontiguousarray(zeros, np.uint16)
    out = np.empty(nelem, np.float32)
    lib().orc_gptq_dequant(_p(data), _p(scales), _p(zeros), nelem, group, bits, _p(out))
    return out


def awq_dequant(words, scales, zeros, nelem: int, group: int) -> np.ndarray:
    words = np.ascontiguousarray(words, np.uint32)
    scales = np.ascontiguousarray(scales, np.uint16)
    zeros = np.ascontiguousarray(zeros, np.uint16)
    out = np.empty(nelem, np.float32)
    lib().orc_awq_dequant(_p(words), _p(scales), _p(zeros), nelem, group, _p(out))
    return out


def awq4_wire_dequant(src, n: int):
    """(status, values): the registry's AWQ_4 Dequantize on wire bytes;
    status 0 ok, 1 short data, 2 numElements mismatch, 3 bad group fields."""
    src = np.ascontiguousarray(src, np.uint8)
    out = np.zeros(max(n, 1), np.float32)
    rc = lib().orc_awq4_wire_dequant(_p(src), src.size, _p(out), n)
    return rc, out[:n]


def fp8_dequant(src, n: int, e5m2: bool):
    """(status, values): the registry's FP8_E4M3 / FP8_E5M2 Dequantize."""
    src = np.ascontiguousarray(src, np.uint8)
    out = np.zeros(max(n, 1), np.float32)
    rc = lib().orc_fp8_dequant(_p(src), src.size, _p(out), n, int(bool(e5m2)))
    return rc, out[:n]


def iq3s_dequant(src, n: int):
    """(status, values): the registry's IQ3_S Dequantize (status 1 where the
    reference returns an error)."""
    src = np.ascontiguousarray(src, np.uint8)
    out = np.zeros(max(n, 1), np.float32)
    rc = lib().orc_iq3s_dequant(_p(src), src.size, _p(out), n)
    return rc, out[:max(n, 0)]


def sgemm_simd(a: np.ndarray, b: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    c = np.zeros(m * n, np.float32)
    lib().orc_sgemm_simd(m, n, k, _p(a), _p(b), _p(c))
    return c


def w4a16_matmul(data, scales, zeros, x16, m: int, k: int, n: int, group: int) -> np.ndarray:
    """C[m,n] = dequant(W)[m,k] @ f32(x16)[k,n] as MatMulW4A16 computes it."""
    data = np.ascontiguousarray(data, np.uint8)
    scales = np.ascontiguousarray(scales, np.uint16)
    zeros = np.ascontiguousarray(zeros, np.uint16)
    x16 = np.ascontiguousarray(x16, np.uint16)
    c = np.empty(m * n, np.float32)
    wt = np.empty(m * k, np.float32)
    xt = np.empty(k * n, np.float32)
    lib().orc_w4a16_matmul_gptq(_p(data), _p(scales), _p(zeros), _p(x16), _p(c), m, k, n, group, _p(wt), _p(xt))
    return c


def iq4nl_matmul(raw, x16, m: int, k: int, n: int) -> np.ndarray:
    x16 = np.ascontiguousarray(x16, np.uint16)
    c = np.empty(m * n, np.float32)
    wt = np.empty(m * k, np.float32)
    xt = np.empty(k * n, np.float32)
    lib().orc_iq4nl_matmul(_p(raw), _p(x16), _p(c), m, k, n, _p(wt), _p(xt))
    return c


def ternary_gemv(raw: np.ndarray, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty(rows, np.float32)
    lib().orc_ternary_gemv(_p(raw), _p(x), rows, cols, _p(y))
    return y


def ternary_repack_rows(raw: np.ndarray, rows: int, cols: int) -> np.ndarray:
    out = np.zeros(rows * ((cols + 3) // 4), np.uint8)
    lib().orc_ternary_repack_rows(_p(raw), rows, cols, _p(out))
    return out


def ternary_gemv_i8(raw, qx, x_scale, w_scale, rows: int, cols: int) -> np.ndarray:
    qx = np.ascontiguousarray(qx, np.int8)
    y = np.empty(rows, np.float32)
    xt = np.empty(cols, np.float32)
    lib().orc_ternary_gemv_i8(_p(raw), _p(qx), float(x_scale), float(w_scale), rows, cols, _p(y), _p(xt))
    return y


def ternary_get(raw: np.ndarray, i: int) -> int:
    return lib().orc_ternary_get(_p(raw), i)


# ---- K-quants and Q5_0 ----------------------------------------------------

KQ_FMT = {"q4_k": 4, "q5_k": 5, "q6_k": 6}


def kq_scales_mins(block: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    block = np.ascontiguousarray(block, np.uint8)
    sc = np.empty(8, np.uint8)
    mn = np.empty(8, np.uint8)
    lib().orc_kq_scales_mins(_p(block), _p(sc), _p(mn))
    return sc, mn


def kq_dequant(fmt: str, raw: np.ndarray, nelem: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty(nelem, np.float32)
    getattr(lib(), f"orc_{fmt.replace('_', '')}_dequant")(_p(raw), nelem, _p(out))
    return out


def gemm_f32_kq_nt(fmt: str, a: np.ndarray, raw: np.ndarray, m: int, n: int, k: int, threads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    raw = np.ascontiguousarray(raw, np.uint8)
    c = np.empty(m * n, np.float32)
    lib().orc_gemm_f32_kq_nt(KQ_FMT[fmt], m, n, k, _p(a), _p(raw), _p(c), threads)
    return c


def q5_0_dequant(raw: np.ndarray, nelem: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty(nelem, np.float32)
    lib().orc_q5_0_dequant(_p(raw), nelem, _p(out))
    return out


def q5_0_raw_to_gpu(raw: np.ndarray, nblk: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty(lib().orc_q5_0_gpu_qs_offset(nblk) + 16 * nblk, np.uint8)
    lib().orc_q5_0_raw_to_gpu(_p(raw), nblk, _p(out))
    return out


def gemm_f32_q5_0_nt(a: np.ndarray, raw: np.ndarray, m: int, n: int, k: int) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    raw = np.ascontiguousarray(raw, np.uint8)
    c = np.empty(m * n, np.float32)
    wt = np.empty(n * k, np.float32)
    tt = np.empty(n * k, np.float32)
    lib().orc_gemm_f32_q5_0_nt(m, n, k, _p(a), _p(raw), _p(c), _p(wt), _p(tt))
    return c


# ---- GGUF mmap --------------------------------------------------------------

def gguf_q8_0_dequant(raw: np.ndarray, nelem: int) -> np.ndarray:
    raw = np.ascontiguousarray(raw, np.uint8)
    out = np.empty(nelem, np.float32)
    lib().orc_gguf_q8_0_dequant(_p(raw), nelem, _p(out))
    return out


def gemm_f32_mmap_nt(qtype: int, a: np.ndarray, raw: np.ndarray, m: int, n: int, k: int, threads: int = 1) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    raw = np.ascontiguousarray(raw, np.uint8)
    c = np.empty(m * n, np.float32)
    wt = np.empty(n * k if qtype in (2, 6, 8) else 1, np.float32)
    rc = lib().orc_gemm_f32_mmap_nt(qtype, m, n, k, _p(a), _p(raw), _p(c), threads, _p(wt))
    if rc != 0:
        raise ValueError(f"GGML type {qtype} has no quantized GEMV here")
    return c


# ---- int4 / int8 GEMMs (gemm_int4.cu, gemm_int8.cu) ---------------------------

def gemm_int4_f32(a: np.ndarray, b: np.ndarray, scales: np.ndarray, zeros: np.ndarray, m: int, k: int, n: int,
                  gs: int, threads: int = 8) -> np.ndarray:
    """C[m, n] of gemm_int4_f32; raises ValueError where the launcher returns
    InvalidValue (odd K, group_size <= 0)."""
    a = np.ascontiguousarray(a, np.uint8)
    b = np.ascontiguousarray(b, np.float32)
    scales = np.ascontiguousarray(scales, np.float32)
    zeros = np.ascontiguousarray(zeros, np.uint8)
    c = np.empty(m * n, np.float32)
    if lib().orc_gemm_int4_f32(_p(a), _p(b), _p(c), _p(scales), _p(zeros), m, k, n, gs, threads) != 0:
        raise ValueError("gemm_int4_f32: invalid value")
    return c


def gemm_int4_f32_rmul(w: np.ndarray, x: np.ndarray, scales: np.ndarray, zeros: np.ndarray, batch: int, inf: int,
                       outf: int, gs: int, threads: int = 8) -> np.ndarray:
    w = np.ascontiguousarray(w, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    scales = np.ascontiguousarray(scales, np.float32)
    zeros = np.ascontiguousarray(zeros, np.uint8)
    c = np.empty(batch * outf, np.float32)
    if lib().orc_gemm_int4_f32_rmul(_p(w), _p(x), _p(c), _p(scales), _p(zeros), batch, inf, outf, gs, threads) != 0:
        raise ValueError("gemm_int4_f32_rmul: invalid value")
    return c


def gemm_int8_f32(a: np.ndarray, b: np.ndarray, m: int, k: int, n: int, threads: int = 8) -> np.ndarray:
    a = np.ascontiguousarray(a, np.int8)
    b = np.ascontiguousarray(b, np.float32)
    c = np.empty(m * n, np.float32)
    lib().orc_gemm_int8_f32(_p(a), _p(b), _p(c), m, k, n, threads)
    return c
