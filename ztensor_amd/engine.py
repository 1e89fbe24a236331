"""ROCmEngine: the quantized-matmul surface of ztensor's compute engine on MI355X.

Two levels, as in the reference:

* KernelRunner level (internal/gpuapi/kernels.go:45-81): gemm_q4_f32,
  gemm_q8_f32, ... take raw device pointers and integers and call the C ABI
  of libzt_hip.so on the engine's stream.  These replace the ROCm stubs
  that return "not implemented" (internal/gpuapi/rocm_kernels.go:109-135).
* Engine level: upload_weights (WeightUploader.UploadWeights,
  compute/engine.go:36-38; compute/gpu_engine.go:778-1050), matmul with the
  storage-type dispatch of GPUEngine.MatMul (compute/gpu_engine.go:1409-1470,
  2115-2200) and CPUEngine.tryQuantizedMatMul (compute/cpu_engine.go:2277-2523),
  matmul_w4a16 (W4A16MatMuler, compute/w4a16.go:137-168) and ternary_gemv
  (TernaryGEMVGPU, compute/ternary_gemv_gpu.go:18-25).

Device memory and the stream come from PyTorch; every byte of arithmetic on
the path runs in libzt_hip.so.  There is no CPU fallback: a kernel error
raises ZTError (the reference falls back to its CPU engine; here the caller
decides).
"""
from __future__ import annotations

from typing import Any

import numpy as np
import torch

from . import _lib
from .storage import (
    AWQStorage,
    Float16Storage,
    GPTQStorage,
    GPUBuffer,
    IQ4NLStorage,
    MmapStorage,
    GGMLType,
    Q4KStorage,
    Q4Storage,
    Q5_0Storage,
    Q5KStorage,
    Q6KStorage,
    Q8Storage,
    Tensor,
    TernaryStorage,
)

_KQ_GEMV = {Q4KStorage: "zt_gemv_q4k_f32", Q5KStorage: "zt_gemv_q5k_f32", Q6KStorage: "zt_gemv_q6k_f32"}
_KQ_TILED = {Q4KStorage: "q4k", Q5KStorage: "q5k", Q6KStorage: "q6k"}
_KQ_DEQUANT = {Q4KStorage: "zt_dequant_q4k_f32", Q5KStorage: "zt_dequant_q5k_f32", Q6KStorage: "zt_dequant_q6k_f32"}


def _p(t: torch.Tensor | None) -> int:
    return 0 if t is None else t.data_ptr()


def _on_engine_stream(fn):
    """Runs an engine method with the engine's stream as torch's current
    stream, so every temporary it makes (clones, transposes, pads, outputs,
    tiled copies, the workspace) is allocated and written in the same stream
    order as the kernels that read it, and the caching allocator never hands
    one of them to other work while a kernel on the engine stream still uses
    it.  Inputs made on another stream must be ready before the call, and
    outputs used on another stream must wait for the engine stream, as with
    any stream-ordered library."""

    def wrapped(self, *args, **kwargs):
        with torch.cuda.stream(self.stream):
            return fn(self, *args, **kwargs)

    wrapped.__name__, wrapped.__doc__, wrapped.__wrapped__ = fn.__name__, fn.__doc__, fn  # type: ignore[attr-defined]
    return wrapped


def _tiled_cached(s: Any, key: tuple):
    """The tiled device copy cached on a storage for `key`
    (format tag, rows, K, source buffer address), or None."""
    cached = getattr(s, "_gpu_tiled", None)
    if cached is not None and cached[0] == key:
        return cached[1:]
    return None


class ROCmEngine:
    def __init__(self, device: int = 0, stream: torch.cuda.Stream | None = None, q6k_split: bool = True,
                 split_reserve_bytes: int = 1 << 30):
        """q6k_split: Q6_K batch 1 on a split copy of the super-blocks (35-55%
        faster; it doubles the resident Q6_K bytes).  The copy is built only
        while at least split_reserve_bytes of device memory stay free after
        it; otherwise, or with q6k_split=False, batch 1 reads the raw
        super-blocks."""
        if not torch.cuda.is_available():
            raise RuntimeError("ROCmEngine needs a ROCm GPU (torch.cuda.is_available() is False)")
        self.device = torch.device("cuda", device)
        self.stream = stream if stream is not None else torch.cuda.current_stream(self.device)
        self.lib = _lib.load()
        self.q6k_split = q6k_split
        self.split_reserve_bytes = split_reserve_bytes

    @property
    def _s(self) -> int:
        return self.stream.cuda_stream

    def _workspace(self, nbytes: int) -> tuple[int, int]:
        """Scratch for the split-K partials of the tiled GEMMs: one buffer per
        engine, grown on demand; calls on the engine's one stream run in
        order, so they can share it."""
        if nbytes <= 0:
            return 0, 0
        buf = getattr(self, "_wsbuf", None)
        if buf is None or buf.numel() < nbytes:
            buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self._wsbuf = buf
        return _p(buf), buf.numel()

    # ------------------------------------------------------ KernelRunner level

    def gemm_q4_f32(self, a_q4: int, b: int, c: int, m: int, k: int, n: int, data_offset: int) -> None:
        self.lib.call("zt_gemm_q4_f32", a_q4, b, c, m, k, n, data_offset, self._s)

    def gemm_q4_f16(self, a_q4: int, b: int, c: int, m: int, k: int, n: int, data_offset: int) -> None:
        self.lib.call("zt_gemm_q4_f16", a_q4, b, c, m, k, n, data_offset, self._s)

    def gemm_iq4nl_f32(self, a: int, b: int, c: int, m: int, k: int, n: int, data_offset: int) -> None:
        self.lib.call("zt_gemm_iq4nl_f32", a, b, c, m, k, n, data_offset, self._s)

    def gemm_iq4nl_f16(self, a: int, b: int, c: int, m: int, k: int, n: int, data_offset: int) -> None:
        self.lib.call("zt_gemm_iq4nl_f16", a, b, c, m, k, n, data_offset, self._s)

    def gemm_q8_f32(self, a_q8: int, b: int, c: int, m: int, k: int, n: int) -> None:
        self.lib.call("zt_gemm_q8_f32", a_q8, b, c, m, k, n, self._s)

    def gemm_q8sep_f32(self, a_q8: int, b: int, c: int, m: int, k: int, n: int, data_offset: int) -> None:
        self.lib.call("zt_gemm_q8sep_f32", a_q8, b, c, m, k, n, data_offset, self._s)

    def gemm_w4a16_f32(self, w: int, scales: int, zeros: int, b: int, c: int, m: int, k: int, n: int,
                       group_size: int) -> None:
        self.lib.call("zt_gemm_w4a16_f32", w, scales, zeros, b, c, m, k, n, group_size, self._s)

    def w4a16_tile(self, w: int, scales: int, zeros: int, m: int, k: int, group_size: int, w_tiled: int,
                   sz: int) -> None:
        self.lib.call("zt_w4a16_tile", w, scales, zeros, m, k, group_size, w_tiled, sz, self._s)

    def gemm_w4a16t_f32(self, w_tiled: int, sz: int, b: int, c: int, m: int, k: int, n: int, group_size: int) -> None:
        ws, wsb = self._workspace(self.lib.zt_gemm_w4a16t_workspace_bytes(m, k, n))
        self.lib.call("zt_gemm_w4a16t_f32", w_tiled, sz, b, c, m, k, n, group_size, ws, wsb, self._s)

    def gemv_q4k_f32(self, w: int, x: int, y: int, m: int, k: int) -> None:
        self.lib.call("zt_gemv_q4k_f32", w, x, y, m, k, self._s)

    def gemv_q5k_f32(self, w: int, x: int, y: int, m: int, k: int) -> None:
        self.lib.call("zt_gemv_q5k_f32", w, x, y, m, k, self._s)

    def gemv_q6k_f32(self, w: int, x: int, y: int, m: int, k: int) -> None:
        self.lib.call("zt_gemv_q6k_f32", w, x, y, m, k, self._s)

    def gemv_q5_0_f32(self, w: int, x: int, y: int, m: int, k: int, qh_offset: int, qs_offset: int) -> None:
        self.lib.call("zt_gemv_q5_0_f32", w, x, y, m, k, qh_offset, qs_offset, self._s)

    def dequant_q4k_f32(self, src: int, dst: int, rows: int, k: int) -> None:
        self.lib.call("zt_dequant_q4k_f32", src, dst, rows, k, self._s)

    def dequant_q5k_f32(self, src: int, dst: int, rows: int, k: int) -> None:
        self.lib.call("zt_dequant_q5k_f32", src, dst, rows, k, self._s)

    def dequant_q6k_f32(self, src: int, dst: int, rows: int, k: int) -> None:
        self.lib.call("zt_dequant_q6k_f32", src, dst, rows, k, self._s)

    def dequant_q5_0_f32(self, src: int, dst: int, rows: int, k: int) -> None:
        self.lib.call("zt_dequant_q5_0_f32", src, dst, rows, k, self._s)

    def ternary_gemv_f32(self, w: int, x: int, y: int, m: int, k: int) -> None:
        self.lib.call("zt_ternary_gemv_f32", w, x, y, m, k, self._s)

    def ternary_gemv_i8(self, w: int, xq: int, x_scale: int, w_scale: int, y: int, m: int, k: int) -> None:
        self.lib.call("zt_ternary_gemv_i8", w, xq, x_scale, w_scale, y, m, k, self._s)

    def ternary_gemv_i8_group(self, mats: list[tuple[int, int, int, int]], xq: int, x_scale: int, k: int) -> None:
        """Ternary GEMVs over one int8 activation vector (a BitNet layer's
        q/k/v, or gate/up), given as (W, w_scale, y, rows) device pointers:
        one zt_ternary_gemv_i8_group launch per ZT_GROUP_MAX matrices, each
        result the one zt_ternary_gemv_i8 gives (bit for bit)."""
        for i0 in range(0, len(mats), _lib.GROUP_MAX):
            part = mats[i0:i0 + _lib.GROUP_MAX]
            self.lib.call("zt_ternary_gemv_i8_group", _lib.ternary_gemv_descs(part), len(part), xq, x_scale, k,
                          self._s)

    # ------------------------------------------------------------ residency

    def _to_dev(self, host: np.ndarray) -> torch.Tensor:
        t = torch.from_numpy(np.ascontiguousarray(host).view(np.uint8).reshape(-1))
        return t.to(self.device, non_blocking=False)

    @_on_engine_stream
    def upload_weights(self, storages: list[Any]) -> int:
        """Copies each quantized storage to the device once, in its GPU layout,
        and records the buffer with set_gpu_ptr (compute/gpu_engine.go:778-818).
        Returns the number of storages uploaded."""
        n = 0
        for s in storages:
            if isinstance(s, (Q4Storage, IQ4NLStorage, Q8Storage)):
                if s.gpu_ptr() is None:
                    buf = s.raw_bytes_gpu()
                    s.set_gpu_ptr(GPUBuffer(self._to_dev(buf), buf.size, self.device.index or 0,
                                            s.gpu_data_offset()))
                    n += 1
            elif isinstance(s, (Q4KStorage, Q5KStorage, Q6KStorage)):
                if s.gpu_ptr() is None:  # raw super-blocks, as compute/gpu_engine.go:817-874
                    s.set_gpu_ptr(GPUBuffer(self._to_dev(s.raw), s.raw.size, self.device.index or 0))
                    n += 1
            elif isinstance(s, MmapStorage):
                if s.gpu_ptr() is None:  # compute/gpu_engine.go:3072-3100 mmapDevicePtr, plus the repacks
                    buf, offs = s.device_layout()
                    s.set_gpu_ptr(GPUBuffer(self._to_dev(buf), buf.size, self.device.index or 0,
                                            offs.get("data_offset", 0)))
                    s._gpu_offsets = offs  # type: ignore[attr-defined]
                    n += 1
            elif isinstance(s, Q5_0Storage):
                if s.gpu_ptr() is None:  # RawBytesGPU, as compute/gpu_engine.go:876-893
                    buf = s.raw_bytes_gpu()
                    s.set_gpu_ptr(GPUBuffer(self._to_dev(buf), buf.size, self.device.index or 0))
                    n += 1
            elif isinstance(s, (GPTQStorage, AWQStorage)):
                if s.gpu_ptr() is None:
                    packed = s.data if isinstance(s, GPTQStorage) else s.packed_bytes()
                    if isinstance(s, GPTQStorage) and s.bits != 4:
                        raise ValueError("only 4-bit GPTQ weights are on the W4A16 path")
                    t = self._to_dev(packed)
                    sc = self._to_dev(s.scales).view(torch.int16)
                    zr = self._to_dev(s.zeros).view(torch.int16)
                    s.set_gpu_ptr(GPUBuffer(t, packed.size, self.device.index or 0))
                    s._gpu_scales, s._gpu_zeros = sc, zr  # type: ignore[attr-defined]
                    # (scale, zero) packed into one dword per group for batch 1; the
                    # packing is elementwise over the [rows, K/group] arrays
                    szr = None
                    if s.group_size % 32 == 0:
                        szr = torch.empty(s.scales.size, dtype=torch.int32, device=self.device)
                        self.lib.call("zt_w4a16_pack_szr", _p(sc), _p(zr), s.scales.size, s.group_size,
                                      s.group_size, _p(szr), self._s)
                    s._gpu_szr = szr  # type: ignore[attr-defined]
                    n += 1
        return n

    # ---------------------------------------------------------------- matmul

    @_on_engine_stream
    def matmul(self, a: Tensor | torch.Tensor, b: Tensor | torch.Tensor) -> torch.Tensor:
        """C = A @ B where one operand is a quantized weight Tensor and the
        other an fp32 (or fp16, for the W4A16 formats) device tensor.

        A-side weight: A is [M, K] (blocks along K), B is [K, N] -> C [M, N].
        B-side weight: B is the virtually transposed weight, logical [K, N],
        physical [N, K] (compute/cpu_engine.go:1378-1390); A is [M, K];
        C [M, N] is computed as (W[N,K] @ A^T)^T, as matMulQ4BWeight does
        (compute/gpu_engine.go:2115-2200)."""
        if isinstance(a, Tensor):
            rows, k = a.shape[-2], a.shape[-1]
            x = b
            if x.shape[0] != k:
                raise ValueError(f"matmul: A is [{rows},{k}] but B has {x.shape[0]} rows")
            return self._weight_times(a.storage, rows, k, x.contiguous())
        if isinstance(b, Tensor):
            k, nout = b.shape[-2], b.shape[-1]
            if a.shape[-1] != k:
                raise ValueError(f"matmul: A has {a.shape[-1]} columns but B is [{k},{nout}]")
            m = a.numel() // k
            xt = a.reshape(m, k).t().contiguous()  # [K, M]
            ct = self._weight_times(b.storage, nout, k, xt)  # [Nout, M]
            return ct.t().contiguous().reshape(*a.shape[:-1], nout)
        raise TypeError("matmul: neither operand is a quantized weight Tensor")

    def _w4a16_tiled(self, s: Any, rows: int, k: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The tiled copy of uploaded W4A16 weights for batches of 4-16
        columns, built on the device on the first batched call and kept
        beside the row-major upload (which batch 1 reads)."""
        key = ("w4a16t", rows, k, _p(s.gpu_ptr().tensor))
        cached = _tiled_cached(s, key)
        if cached is not None:
            return cached
        nbytes = self.lib.zt_w4a16_tiled_bytes(rows, k)
        szbytes = self.lib.zt_w4a16_sz_bytes(rows, k, s.group_size)
        if nbytes < 0 or szbytes < 0:
            raise ValueError(f"W4A16 tiled layout: unsupported shape [{rows}, {k}] (group {s.group_size})")
        wt = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        sz = torch.empty(szbytes // 4, dtype=torch.int32, device=self.device)
        zeros = _p(s._gpu_zeros) if s._gpu_zeros is not None else 0
        self.w4a16_tile(_p(s.gpu_ptr().tensor), _p(s._gpu_scales), zeros, rows, k, s.group_size, _p(wt), _p(sz))
        s._gpu_tiled = (key, wt, sz)  # type: ignore[attr-defined]
        return wt, sz

    def _iq4nl_tiled(self, s: Any, buf: GPUBuffer, rows: int, k: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The tiled copy of uploaded IQ4_NL weights for batches of 4-16
        fp16 columns, built on the device on first use."""
        key = ("iq4nlt", rows, k, _p(buf.tensor))
        cached = _tiled_cached(s, key)
        if cached is not None:
            return cached
        nbytes, sbytes = self.lib.zt_iq4nl_tiled_bytes(rows, k), self.lib.zt_iq4nl_tiled_scale_bytes(rows, k)
        if nbytes < 0 or sbytes < 0:
            raise ValueError(f"IQ4_NL tiled layout: unsupported shape [{rows}, {k}]")
        wt = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        st = torch.empty(sbytes, dtype=torch.uint8, device=self.device)
        self.lib.call("zt_iq4nl_tile", _p(buf.tensor), rows, k, buf.data_offset, _p(wt), _p(st), self._s)
        s._gpu_tiled = (key, wt, st)  # type: ignore[attr-defined]
        return wt, st

    def _block_tiled(self, s: Any, buf: GPUBuffer, rows: int, k: int, fmt: str) -> tuple[torch.Tensor, torch.Tensor]:
        """The tiled copy of uploaded Q4_0 ("q4") or Q8_0 ("q8") weights for
        batches of 4-16 fp32 columns, built on the device from the separated
        upload on the first batched call and kept beside it (batch 1 reads
        the separated layout)."""
        key = (fmt + "t", rows, k, _p(buf.tensor))
        cached = _tiled_cached(s, key)
        if cached is not None:
            return cached
        size_fmt = "q8" if fmt == "q8gguf" else fmt  # GGUF Q8_0 tiles into the Q8_0 layout
        nbytes = getattr(self.lib, f"zt_{size_fmt}_tiled_bytes")(rows, k)
        sbytes = getattr(self.lib, f"zt_{size_fmt}_tiled_scale_bytes")(rows, k)
        if nbytes < 0 or sbytes < 0:
            raise ValueError(f"{fmt} tiled layout: unsupported shape [{rows}, {k}]")
        wt = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        st = torch.empty(sbytes, dtype=torch.uint8, device=self.device)
        self.lib.call(f"zt_{fmt}_tile", _p(buf.tensor), rows, k, buf.data_offset, _p(wt), _p(st), self._s)
        s._gpu_tiled = (key, wt, st)  # type: ignore[attr-defined]
        return wt, st

    @staticmethod
    def _tiled_ok(s: Any, rows: int, k: int, x: torch.Tensor) -> bool:
        """Whether this weight and activation dtype have a tiled MFMA path."""
        if k % 128 != 0 or isinstance(s, MmapStorage):
            return False
        if isinstance(s, Q4Storage):
            return x.dtype in (torch.float32, torch.float16)
        if isinstance(s, Q8Storage):
            return x.dtype == torch.float32
        if isinstance(s, (Q4KStorage, Q5KStorage, Q6KStorage)):
            return x.dtype == torch.float32 and k % 256 == 0
        if isinstance(s, Q5_0Storage):
            return x.dtype == torch.float32
        if isinstance(s, IQ4NLStorage):
            return x.dtype == torch.float16
        if isinstance(s, (GPTQStorage, AWQStorage)):
            return (x.dtype == torch.float16 and s.group_size % 128 == 0 and
                    rows * (k // s.group_size) < 1 << 29)
        return False

    def _kq_tiled(self, s: Any, buf: GPUBuffer, rows: int, k: int, f: str) -> tuple:
        """The tiled copy of uploaded K-quant super-blocks for batches of
        4-16 fp32 columns, built on the device on the first batched call.
        f = "q4k" / "q5k": data in the Q4_0 tile format, the super-block
        headers and, for Q5_K, the fifth bits; f = "q6k": the 6-bit values in
        the Q8_0 tile format and the per-16 scales d * sc."""
        key = (f + "t", rows, k, _p(buf.tensor))
        cached = _tiled_cached(s, key)
        if cached is not None:
            return cached
        second = "tiled_scale_bytes" if f == "q6k" else "tiled_header_bytes"
        sizes = [getattr(self.lib, f"zt_{f}_tiled_bytes")(rows, k), getattr(self.lib, f"zt_{f}_{second}")(rows, k)]
        if f == "q5k":
            sizes.append(self.lib.zt_q5k_tiled_qh_bytes(rows, k))
        if min(sizes) < 0:
            raise ValueError(f"{f} tiled layout: unsupported shape [{rows}, {k}]")
        bufs = tuple(torch.empty(n, dtype=torch.uint8, device=self.device) for n in sizes)
        self.lib.call(f"zt_{f}_tile", _p(buf.tensor), rows, k, *(_p(b) for b in bufs), self._s)
        s._gpu_tiled = (key,) + bufs  # type: ignore[attr-defined]
        return bufs

    def _kq_tiled_gemm(self, s: Any, buf: GPUBuffer, rows: int, k: int, x: torch.Tensor, n: int, c: torch.Tensor,
                       f: str) -> None:
        bufs = self._kq_tiled(s, buf, rows, k, f)
        ws, wsb = self._workspace(getattr(self.lib, f"zt_gemm_{f}t_workspace_bytes")(rows, k, n))
        self.lib.call(f"zt_gemm_{f}t_f32", *(_p(b) for b in bufs), _p(x), _p(c), rows, k, n, ws, wsb, self._s)

    def _q6k_gemv(self, s: Any, raw_ptr: int, rows: int, k: int, x: torch.Tensor, c: torch.Tensor) -> None:
        """Q6_K batch 1 on the split layout (zt_q6k_split: the same 210 bytes
        a super-block in four aligned arrays), built on the device from the
        uploaded raw super-blocks on the first batch-1 call and kept beside
        them: 35-55% faster than the raw-layout GEMV at the Llama-3-8B
        shapes.  Falls back to the raw-layout GEMV where the split kernel's
        32-bit offsets or x's alignment do not allow it, when the engine was
        made with q6k_split=False, and when building the copy would leave less
        than split_reserve_bytes of device memory free."""
        key = ("q6ks", rows, k, raw_ptr)
        cached = getattr(s, "_gpu_split", None)
        if cached is not None and cached[0] != key:
            s._gpu_split = cached = None  # type: ignore[attr-defined]  # a stale copy goes before a new one
        nbytes = self.lib.zt_q6k_split_bytes(rows, k)
        if (rows * (k // 256) * 210 >= 1 << 31 or _p(x) % 16 != 0 or not self.q6k_split
                or (cached is None and torch.cuda.mem_get_info(self.device)[0] < nbytes + self.split_reserve_bytes)):
            self.lib.call("zt_gemv_q6k_f32", raw_ptr, _p(x), _p(c), rows, k, self._s)
            return
        if cached is None:
            sp = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self.lib.call("zt_q6k_split", raw_ptr, rows, k, _p(sp), self._s)
            cached = (key, sp)
            s._gpu_split = cached  # type: ignore[attr-defined]
        self.lib.call("zt_gemv_q6ks_f32", _p(cached[1]), _p(x), _p(c), rows, k, self._s)

    def _q5_0_tiled(self, s: Any, buf: GPUBuffer, rows: int, k: int, qh: int, qs: int) -> tuple:
        """The tiled copy of uploaded Q5_0 weights (nibbles and scales in the
        Q4_0 tiled layout, plus the fifth bits) for batches of 4-16 fp32
        columns, built on the device on the first batched call."""
        key = ("q5_0t", rows, k, _p(buf.tensor))
        cached = _tiled_cached(s, key)
        if cached is not None:
            return cached
        sizes = [self.lib.zt_q5_0_tiled_bytes(rows, k), self.lib.zt_q5_0_tiled_scale_bytes(rows, k),
                 self.lib.zt_q5_0_tiled_qh_bytes(rows, k)]
        if min(sizes) < 0:
            raise ValueError(f"Q5_0 tiled layout: unsupported shape [{rows}, {k}]")
        wt, st, ht = (torch.empty(n, dtype=torch.uint8, device=self.device) for n in sizes)
        self.lib.call("zt_q5_0_tile", _p(buf.tensor), rows, k, qh, qs, _p(wt), _p(st), _p(ht), self._s)
        s._gpu_tiled = (key, wt, st, ht)  # type: ignore[attr-defined]
        return wt, st, ht

    def _q5_0_tiled_gemm(self, s: Any, buf: GPUBuffer, rows: int, k: int, x: torch.Tensor, n: int, c: torch.Tensor,
                         qh: int, qs: int) -> None:
        wt, st, ht = self._q5_0_tiled(s, buf, rows, k, qh, qs)
        ws, wsb = self._workspace(self.lib.zt_gemm_q5_0t_workspace_bytes(rows, k, n))
        self.lib.call("zt_gemm_q5_0t_f32", _p(wt), _p(st), _p(ht), _p(x), _p(c), rows, k, n, ws, wsb, self._s)

    def _weight_times(self, s: Any, rows: int, k: int, x: torch.Tensor) -> torch.Tensor:
        """dequant(W)[rows, k] @ x[k, n] -> fp32 [rows, n]."""
        n = 1 if x.dim() == 1 else x.shape[1]
        if x.device != self.device:
            raise ValueError("activations must be on the engine's device")
        wide = ((isinstance(s, Q4Storage) and x.dtype in (torch.float32, torch.float16) and _block_wide("q4", rows, k, n))
                or (isinstance(s, Q8Storage) and x.dtype == torch.float32 and _block_wide("q8", rows, k, n)))
        if n > 1 and n not in _TILED_BATCHES and not wide and self._tiled_ok(s, rows, k, x):
            # other batch sizes on the tiled MFMA kernels: columns in chunks of
            # 16, the last one zero-padded to a multiple of 4
            xs = x.reshape(k, n)
            outs = []
            for j0 in range(0, n, 16):
                m = min(16, n - j0)
                mp = -(-m // 4) * 4
                xp = torch.zeros((k, mp), dtype=x.dtype, device=self.device)
                xp[:, :m] = xs[:, j0:j0 + m]
                outs.append(self._weight_times(s, rows, k, xp)[:, :m])
            return torch.cat(outs, dim=1)
        self.upload_weights([s])
        c = torch.empty((rows, n), dtype=torch.float32, device=self.device)
        buf = s.gpu_ptr() if hasattr(s, "gpu_ptr") else None  # ternary: resident per shape, below
        if isinstance(s, MmapStorage):
            return self._mmap_times(s, buf, rows, k, x, n, c)
        if isinstance(s, Q4Storage):
            if wide:
                # the bf16 MFMA tile GEMM behind the entry point (fp16 activations widen exactly)
                x = x.float() if x.dtype == torch.float16 else x
                x = x if _p(x) % 8 == 0 else x.clone()
                self.gemm_q4_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            elif x.dtype in (torch.float32, torch.float16) and _block_rowblock("q4", rows, k, n):
                # one launch on the separated upload (the row-block GEMM): no tiled copy, no workspace
                x = x.float() if x.dtype == torch.float16 else x
                x = x if _p(x) % 16 == 0 else x.clone()
                self.gemm_q4_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            elif x.dtype in (torch.float32, torch.float16) and n in _TILED_BATCHES and k % 128 == 0:
                # fp16 activations widen exactly to fp32 for the tiled kernel
                x = x.float() if x.dtype == torch.float16 or _p(x) % 16 else x
                wt, st = self._block_tiled(s, buf, rows, k, "q4")
                ws, wsb = self._workspace(self.lib.zt_gemm_q4t_workspace_bytes(rows, k, n))
                self.lib.call("zt_gemm_q4t_f32", _p(wt), _p(st), _p(x), _p(c), rows, k, n, ws, wsb, self._s)
            elif x.dtype == torch.float32:
                self.gemm_q4_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            elif x.dtype == torch.float16:
                self.gemm_q4_f16(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            else:
                raise TypeError(f"Q4_0 matmul: unsupported activation dtype {x.dtype}")
        elif isinstance(s, IQ4NLStorage):
            if x.dtype == torch.float32:
                self.gemm_iq4nl_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            elif (x.dtype == torch.float16 and k <= 8192 and _p(x) % 16 == 0
                  and (n in (4, 8) or (n in (12, 16) and rows <= 4096))):
                # one launch on the separated upload (the row-block GEMM): no tiled copy, no workspace;
                # faster than the tiled layout at K <= 8192 (3584 x 3584: 5.0 / 6.0 against 7.3 / 7.5 us at
                # batch 4 / 8), slower past it (K = 18944, batch 8: 23.8 against 15.7 us); batches of 12
                # and 16 up to 4096 rows (4096 x 4096: 7.5 / 8.4 against 9.0 / 8.9 us)
                self.gemm_iq4nl_f16(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            elif x.dtype == torch.float16 and n in _TILED_BATCHES and k % 128 == 0:
                wt, st = self._iq4nl_tiled(s, buf, rows, k)
                ws, wsb = self._workspace(self.lib.zt_gemm_iq4nlt_workspace_bytes(rows, k, n))
                self.lib.call("zt_gemm_iq4nlt_f16", _p(wt), _p(st), _p(x), _p(c), rows, k, n, ws, wsb, self._s)
            elif x.dtype == torch.float16:
                self.gemm_iq4nl_f16(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
            else:
                raise TypeError(f"IQ4_NL matmul: unsupported activation dtype {x.dtype}")
        elif isinstance(s, Q8Storage):
            if x.dtype != torch.float32:
                raise TypeError("Q8_0 matmul takes fp32 activations")
            if wide:
                # the bf16 MFMA tile GEMM behind the entry point
                x = x if _p(x) % 8 == 0 else x.clone()
                self.gemm_q8sep_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
                return c
            if _block_rowblock("q8", rows, k, n) and _p(x) % 16 == 0:
                # one launch on the separated upload (the row-block GEMM)
                self.gemm_q8sep_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
                return c
            if n in _TILED_BATCHES and k % 128 == 0 and _p(x) % 16 == 0:
                wt, st = self._block_tiled(s, buf, rows, k, "q8")
                ws, wsb = self._workspace(self.lib.zt_gemm_q8t_workspace_bytes(rows, k, n))
                self.lib.call("zt_gemm_q8t_f32", _p(wt), _p(st), _p(x), _p(c), rows, k, n, ws, wsb, self._s)
                return c
            self.gemm_q8sep_f32(_p(buf.tensor), _p(x), _p(c), rows, k, n, buf.data_offset)
        elif isinstance(s, (GPTQStorage, AWQStorage)):
            if x.dtype != torch.float16:
                raise TypeError("W4A16 matmul takes fp16 activations")
            tiled_ok = k % 128 == 0 and s.group_size % 128 == 0 and rows * (k // s.group_size) < 1 << 29
            if (n in (4, 8, 12, 16) and s._gpu_szr is not None and rows * k // 2 < 1 << 31 and _p(x) % 16 == 0
                    and _w4a16_rowblock(rows, k, n)):
                # one launch on the row-major upload and the packed (scale, zero) dwords: no tiled copy,
                # no workspace, no second kernel
                self.lib.call("zt_gemm_w4a16sz_f32", _p(buf.tensor), _p(s._gpu_szr), _p(x), _p(c), rows, k, n,
                              s.group_size, self._s)
            elif n in _TILED_BATCHES and tiled_ok:
                wt, sz = self._w4a16_tiled(s, rows, k)
                self.gemm_w4a16t_f32(_p(wt), _p(sz), _p(x), _p(c), rows, k, n, s.group_size)
            elif (n == 1 and s._gpu_szr is not None and k <= 32768 and rows * k // 2 < 1 << 31
                  and _p(x) % 16 == 0):
                # packed (scale, zero) dwords, one load a row and step instead of two: faster at every
                # Llama-3 shape (3.73 against 3.88 us at 4096 x 4096, 26.3 against 27.8 us at K = 28672)
                self.lib.call("zt_gemv_w4a16sz_f32", _p(buf.tensor), _p(s._gpu_szr), _p(x), _p(c), rows, k,
                              s.group_size, self._s)
            else:
                self.gemm_w4a16_f32(_p(buf.tensor), _p(s._gpu_scales), _p(s._gpu_zeros), _p(x), _p(c), rows, k, n,
                                    s.group_size)
        elif isinstance(s, TernaryStorage):
            if x.dtype != torch.float32:
                raise TypeError("ternary matmul takes fp32 activations")
            w = self._ternary_resident(s, rows, k)
            xs = x.reshape(k, n)
            cols = [xs[:, j].contiguous() for j in range(n)] if n > 1 else [xs.reshape(k)]
            outs = [c] if n == 1 else [torch.empty(rows, dtype=torch.float32, device=self.device) for _ in range(n)]
            for xj, yj in zip(cols, outs):  # TernaryGEMV per column (compute/ternary_gemv.go:12)
                self.ternary_gemv_f32(_p(w), _p(xj), _p(yj), rows, k)
            if n > 1:
                c.copy_(torch.stack(outs, dim=1))
        elif isinstance(s, (Q4KStorage, Q5KStorage, Q6KStorage, Q5_0Storage)):
            if x.dtype != torch.float32:
                raise TypeError(f"{type(s).__name__} matmul takes fp32 activations")
            q50 = isinstance(s, Q5_0Storage)
            if q50 and n in _TILED_BATCHES and k % 128 == 0 and _p(x) % 16 == 0:
                self._q5_0_tiled_gemm(s, buf, rows, k, x, n, c, s.gpu_qh_offset(), s.gpu_qs_offset())
                return c
            if not q50 and n in _TILED_BATCHES and k % 256 == 0:
                # batched K-quants on the tiled MFMA kernel
                xs = x if _p(x) % 16 == 0 else x.clone()
                self._kq_tiled_gemm(s, buf, rows, k, xs, n, c, _KQ_TILED[type(s)])
                return c
            if n == 1 and k % (32 if q50 else 256) == 0:
                # fused dequant-GEMV (compute/gpu_engine.go:2224-2238, 2505-2510)
                if q50:
                    self.gemv_q5_0_f32(_p(buf.tensor), _p(x), _p(c), rows, k, s.gpu_qh_offset(), s.gpu_qs_offset())
                elif isinstance(s, Q6KStorage):
                    self._q6k_gemv(s, _p(buf.tensor), rows, k, x, c)
                else:
                    self.lib.call(_KQ_GEMV[type(s)], _p(buf.tensor), _p(x), _p(c), rows, k, self._s)
            else:
                # batched: dequantize on the device, then a dense fp32 GEMM, the
                # reference's dequantSgemm (compute/gpu_engine.go:2240-2255);
                # rocBLAS via torch stands in for its cuBLAS Sgemm
                if q50:
                    # the upload holds RawBytesGPU, which the raw-block dequantizer
                    # does not read: one fused GEMV per activation column
                    xt = x.reshape(k, n).t().contiguous()
                    ct = torch.empty((n, rows), dtype=torch.float32, device=self.device)
                    for j in range(n):
                        self.gemv_q5_0_f32(_p(buf.tensor), _p(xt[j]), _p(ct[j]), rows, k, s.gpu_qh_offset(),
                                           s.gpu_qs_offset())
                    c.copy_(ct.t())
                    return c
                if k % 256 != 0:
                    raise ValueError(f"{type(s).__name__} matmul needs K % 256 == 0")
                w = torch.empty((rows, k), dtype=torch.float32, device=self.device)
                self.lib.call(_KQ_DEQUANT[type(s)], _p(buf.tensor), _p(w), rows, k, self._s)
                torch.matmul(w, x.reshape(k, n), out=c)
        else:
            raise TypeError(f"matmul: {type(s).__name__} is not a quantized weight storage")
        return c

    def _mmap_times(self, s: MmapStorage, buf: GPUBuffer, rows: int, k: int, x: torch.Tensor, n: int,
                    c: torch.Tensor) -> torch.Tensor:
        """GPUEngine.matMulMmap / matMulMmapB (compute/gpu_engine.go:2813-3070):
        the GGML type picks the kernel.  Q4_0, Q4_K, Q5_K, Q6_K, Q5_0 and Q8_0
        batches of 4-16 run on the tiled MFMA kernels, as for the storage types.  Q8_0 runs on its own repacked layout
        (the reference passes the 34-byte blocks to the 36-byte kernel,
        compute/gpu_engine.go:2865-2870); Q5_0, which the reference leaves to
        its CPU engine, runs on the Q5_0 GEMV; types without a quantized
        kernel (F32, F16, BF16, Q4_1, Q5_1) raise."""
        if x.dtype != torch.float32:
            raise TypeError("MmapStorage matmul takes fp32 activations")
        q, p, offs = s.qtype, _p(buf.tensor), s._gpu_offsets
        tiled = n in _TILED_BATCHES and _p(x) % 16 == 0
        if q == GGMLType.Q4_0 and tiled and _block_rowblock("q4", rows, k, n):
            self.gemm_q4_f32(p, _p(x), _p(c), rows, k, n, offs["data_offset"])
        elif q == GGMLType.Q8_0 and tiled and _block_rowblock("q8", rows, k, n):
            self.lib.call("zt_gemm_q8gguf_f32", p, _p(x), _p(c), rows, k, n, offs["data_offset"], self._s)
        elif q == GGMLType.Q4_0 and tiled and k % 128 == 0:
            # batches on the tiled MFMA kernel, as for Q4Storage (the device layout is RawBytesGPU)
            wt, st = self._block_tiled(s, buf, rows, k, "q4")
            ws, wsb = self._workspace(self.lib.zt_gemm_q4t_workspace_bytes(rows, k, n))
            self.lib.call("zt_gemm_q4t_f32", _p(wt), _p(st), _p(x), _p(c), rows, k, n, ws, wsb, self._s)
        elif q in (GGMLType.Q4_K, GGMLType.Q5_K, GGMLType.Q6_K) and tiled and k % 256 == 0:
            self._kq_tiled_gemm(s, buf, rows, k, x, n, c, {GGMLType.Q4_K: "q4k", GGMLType.Q5_K: "q5k"}.get(q, "q6k"))
        elif q == GGMLType.Q8_0 and tiled and k % 128 == 0:
            wt, st = self._block_tiled(s, buf, rows, k, "q8gguf")
            ws, wsb = self._workspace(self.lib.zt_gemm_q8t_workspace_bytes(rows, k, n))
            self.lib.call("zt_gemm_q8t_f32", _p(wt), _p(st), _p(x), _p(c), rows, k, n, ws, wsb, self._s)
        elif q == GGMLType.Q5_0 and tiled and k % 128 == 0:
            self._q5_0_tiled_gemm(s, buf, rows, k, x, n, c, offs["qh_offset"], offs["qs_offset"])
        elif q == GGMLType.Q4_0:
            self.gemm_q4_f32(p, _p(x), _p(c), rows, k, n, offs["data_offset"])
        elif q == GGMLType.Q8_0:
            self.lib.call("zt_gemm_q8gguf_f32", p, _p(x), _p(c), rows, k, n, offs["data_offset"], self._s)
        elif q == GGMLType.Q5_0:
            xt = x.reshape(k, n).t().contiguous()
            ct = torch.empty((n, rows), dtype=torch.float32, device=self.device)
            for j in range(n):
                self.gemv_q5_0_f32(p, _p(xt[j]), _p(ct[j]), rows, k, offs["qh_offset"], offs["qs_offset"])
            c.copy_(ct.t())
        elif q in (GGMLType.Q4_K, GGMLType.Q5_K, GGMLType.Q6_K):
            kind = {GGMLType.Q4_K: Q4KStorage, GGMLType.Q5_K: Q5KStorage, GGMLType.Q6_K: Q6KStorage}[q]
            if k % 256 != 0:
                raise ValueError(f"{q.name} matmul needs K % 256 == 0")
            if n == 1 and q == GGMLType.Q6_K:
                self._q6k_gemv(s, p, rows, k, x, c)
            elif n == 1:
                self.lib.call(_KQ_GEMV[kind], p, _p(x), _p(c), rows, k, self._s)
            else:
                w = torch.empty((rows, k), dtype=torch.float32, device=self.device)
                self.lib.call(_KQ_DEQUANT[kind], p, _p(w), rows, k, self._s)
                torch.matmul(w, x.reshape(k, n), out=c)
        else:
            raise TypeError(f"GGML type {q.name} has no quantized GEMV on this path")
        return c

    @_on_engine_stream
    def matmul_w4a16(self, a: Tensor, b: Tensor) -> torch.Tensor:
        """W4A16MatMuler.MatMulW4A16 (compute/w4a16.go:137-143): one operand
        holds 4-bit weights (Q4_0, GPTQ bits=4 or AWQ), the other a
        Float16Storage; the result is fp32 (compute/w4a16.go:64-119)."""
        w, act, side = _detect_w4a16(a, b)
        if w is None:
            raise ValueError("MatMulW4A16: inputs are not W4A16 - need 4-bit weights and FP16 activations")
        x = torch.from_numpy(act.storage.data.view(np.float16)).to(self.device)
        if side == "A":
            return self.matmul(w, x.reshape(act.shape))
        return self.matmul(x.reshape(act.shape), w)

    @_on_engine_stream
    def gemv_group(self, weights: list[Tensor], x: torch.Tensor) -> list[torch.Tensor]:
        """y_i = W_i @ x for weight Tensors that read the same activation
        vector x[K] (a decode layer's q/k/v, or gate/up).  Q4_0 weights with
        fp32 x run in one zt_gemm_q4_group_f32 launch (up to ZT_GROUP_MAX
        matrices a launch), each in its own upload: the effect of
        MergeQ4Storage (tensor/quantized.go:224-242) without re-laying out
        the storages.  W4A16 weights (GPTQ/AWQ) of one group size with fp16 x
        run in one zt_gemv_w4a16sz_group_f32 launch on their packed (scale,
        zero) dwords, each result the single-matrix GEMV's to the bit.  Other
        formats run one GEMV per matrix."""
        if x.dtype not in (torch.float32, torch.float16) or x.dim() != 1 or x.device != self.device:
            raise ValueError("gemv_group takes one fp32 (fp16 for W4A16) activation vector on the engine's device")
        k = x.shape[0]
        for w in weights:
            if not isinstance(w, Tensor) or w.shape[-1] != k:
                raise ValueError(f"gemv_group: every weight must be a quantized [rows, {k}] Tensor")
        if x.dtype == torch.float16 and all(isinstance(w.storage, (GPTQStorage, AWQStorage)) for w in weights):
            self.upload_weights([w.storage for w in weights])
            groups = {w.storage.group_size for w in weights}
            gs = groups.pop() if len(groups) == 1 else 0
            if (gs and gs % 32 == 0 and k % gs == 0 and k <= 32768 and _p(x) % 16 == 0
                    and all(getattr(w.storage, "_gpu_szr", None) is not None for w in weights)):
                outs = [torch.empty(w.shape[-2], dtype=torch.float32, device=self.device) for w in weights]
                for i0 in range(0, len(weights), _lib.GROUP_MAX):
                    part = list(zip(weights[i0:i0 + _lib.GROUP_MAX], outs[i0:i0 + _lib.GROUP_MAX]))
                    descs = _lib.w4a16_gemv_descs([(_p(w.storage.gpu_ptr().tensor), _p(w.storage._gpu_szr), _p(y),
                                                    w.shape[-2]) for w, y in part])
                    self.lib.call("zt_gemv_w4a16sz_group_f32", descs, len(part), _p(x), k, gs, self._s)
                return outs
            return [self._weight_times(w.storage, w.shape[-2], k, x).reshape(-1) for w in weights]
        if (x.dtype != torch.float32 or not all(isinstance(w.storage, Q4Storage) for w in weights) or _p(x) % 16 != 0
                or k % 32 != 0):
            return [self._weight_times(w.storage, w.shape[-2], k, x).reshape(-1) for w in weights]
        self.upload_weights([w.storage for w in weights])
        outs = [torch.empty(w.shape[-2], dtype=torch.float32, device=self.device) for w in weights]
        for i0 in range(0, len(weights), _lib.GROUP_MAX):
            part = list(zip(weights[i0:i0 + _lib.GROUP_MAX], outs[i0:i0 + _lib.GROUP_MAX]))
            descs = _lib.q4_gemv_descs([(_p(w.storage.gpu_ptr().tensor), w.storage.gpu_ptr().data_offset, _p(y),
                                         w.shape[-2]) for w, y in part])
            self.lib.call("zt_gemm_q4_group_f32", descs, len(part), _p(x), k, self._s)
        return outs

    @_on_engine_stream
    def dequant_w4_to_fp16(self, w: Tensor) -> torch.Tensor:
        """DequantW4ToFP16 (compute/w4a16.go:170-175) on the device: the
        4-bit weights (Q4_0, GPTQ bits=4, AWQ) dequantized in fp32 exactly as
        their Dequantize does, then rounded to fp16 (nearest, ties to even),
        as an fp16 device tensor of the weight's shape - the operand of an
        fp16 GEMM."""
        s = w.storage
        n = int(np.prod(w.shape))
        self.upload_weights([s])
        out = torch.empty(n, dtype=torch.float16, device=self.device)
        buf = s.gpu_ptr()
        if isinstance(s, Q4Storage):
            self.lib.call("zt_dequant_q4_f16", _p(buf.tensor), _p(out), n, buf.data_offset, self._s)
        elif isinstance(s, (GPTQStorage, AWQStorage)):
            if isinstance(s, GPTQStorage) and s.bits != 4:
                raise ValueError("DequantW4ToFP16 takes 4-bit weights")
            self.lib.call("zt_dequant_w4_f16", _p(buf.tensor), _p(s._gpu_scales), _p(s._gpu_zeros), _p(out), n,
                          s.group_size, self._s)
        else:
            raise TypeError(f"DequantW4ToFP16: {type(s).__name__} is not a 4-bit weight storage")
        return out.reshape(w.shape)

    @_on_engine_stream
    def dequantize(self, name: str, src: np.ndarray, n: int) -> torch.Tensor:
        """GetQuantType(name).Dequantize(src, dst) with dst on the device
        (tensor/quant_registry.go:10-73): src holds the registered format's
        bytes on the host; they are copied to the device once and decoded
        there into n fp32 values, bit for bit with the reference."""
        from . import registry

        d, ok = registry.get_quant_type(name)
        if not ok:
            raise ValueError(f"tensor: quantization type {name!r} is not registered")
        src = np.ascontiguousarray(src, np.uint8).reshape(-1)
        dst = torch.empty(n, dtype=torch.float32, device=self.device)
        if n == 0:
            if not d.empty_ok:  # IQ3_S: NewIQ3SStorageFromRaw (tensor/iq3_storage.go:99-101)
                raise ValueError(f"numElements must be positive, got {n}")
            return dst
        sd = self._to_dev(np.concatenate([src, np.zeros(-src.size % 16, np.uint8)]) if src.size % 16 else src)
        rc = d.run(self.lib, src, sd, dst, self._s)
        if rc != 0:
            raise _lib.ZTError(f"dequantize {name}", rc)
        return dst

    # ---------------------------------------------------------------- ternary

    @_on_engine_stream
    def ternary_gemv(self, weights: TernaryStorage, x: np.ndarray, rows: int, cols: int) -> np.ndarray:
        """TernaryGEMVGPU (compute/ternary_gemv_gpu.go:18-91): host x in, host
        y out.  The reference repacks and uploads the weights on every call
        (:34-67); here the row-aligned upload is made once per storage and
        shape and kept resident (_ternary_resident)."""
        w = self._ternary_resident(weights, rows, cols)
        xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(self.device)
        y = torch.empty(rows, dtype=torch.float32, device=self.device)
        self.ternary_gemv_f32(_p(w), _p(xd), _p(y), rows, cols)
        return y.cpu().numpy()

    def _ternary_resident(self, s: TernaryStorage, rows: int, cols: int) -> torch.Tensor:
        """The row-aligned device copy of ternary weights (the layout of
        compute/ternary_gemv_gpu.go:52-67), uploaded on first use."""
        cached = getattr(s, "_gpu_rows", None)
        if cached is not None and cached[0] == (rows, cols):
            return cached[1]
        if s.len != rows * cols:
            raise ValueError(f"ternary weights hold {s.len} values, not [{rows}, {cols}]")
        w = self._to_dev(s.row_aligned(rows, cols))
        s._gpu_rows = ((rows, cols), w)  # type: ignore[attr-defined]
        return w


def _block_rowblock(fmt: str, rows: int, k: int, n: int) -> bool:
    """Whether a batch of fp32 columns on Q4_0 ("q4") or Q8_0 ("q8") weights
    runs faster as one launch of the row-block GEMM on the batch-1 upload
    (zt_gemm_q4_f32 / zt_gemm_q8sep_f32 with N > 1) than on the tiled layout
    with its split-K reduction.  Measured (us, row-block against tiled) at
    batch 4 / 8: Q4_0 4096 x 4096 5.2 / 7.1 against 6.6 / 7.4, 1024 x 4096
    4.4 / 5.6 against 5.6 / 5.6, 14336 x 4096 10.8 / 17.8 against 11.7 /
    13.0, 4096 x 14336 14.1 / 29.8 against 11.5 / 12.7; Q8_0 4096 x 4096
    7.2 / 8.6 against 7.7 / 7.9, 1024 x 4096 4.4 / 5.9 against 5.7 / 5.8.
    The row-block kernel stages each wave step's activations as fp16 hi + lo
    parts (16 KB a wave at batch 8), which caps its occupancy on large
    matrices."""
    if n not in (4, 8) or k > 32768:
        return False
    if fmt == "q4" and n == 4:
        return rows * k <= 4096 * 4096 or k <= 4096
    return rows * k <= 4096 * 4096 and (fmt == "q4" or n == 4)


def _w4a16_rowblock(rows: int, k: int, n: int) -> bool:
    """Whether a batch of 4-16 W4A16 columns runs faster on the single-launch
    row-block GEMM over the row-major upload (zt_gemm_w4a16sz_f32) than on the
    tiled layout with its split-K reduction.  Measured (us, row-block against
    tiled): batch 4 at 8192 x 8192 10.1 / 11.2, 4096 x 14336 (rows x K)
    10.0 / 10.7, 14336 x 4096 10.8 / 11.0, 8192 x 28672 37.1 / 29.7; batch
    8 at 14336 x 4096 11.8 / 11.4, 4096 x 4096 4.9 / 6.8, 1024 x 8192
    4.1 / 6.0, 8192 x 8192 13.2 / 11.1, 4096 x 14336 12.3 / 10.9, 28672 x
    8192 37.7 / 29.0; batch 16 at 1024 x 8192 5.98 / 6.22, 4096 x 4096
    6.4 / 7.1, 8192 x 8192 20.4 / 11.8, 14336 x 4096 20.6 / 12.6.
    A row-block workgroup re-reads
    more activation bytes than weight bytes once the rows are many and K is
    long, more so at 12 and 16 columns."""
    if k > 32768:
        return False
    if n == 4:
        return k <= 16384
    if n in (12, 16):
        return k <= 8192 and rows <= 4096
    return k <= 4096 or rows <= 2048


def _block_wide(fmt: str, rows: int, k: int, n: int) -> bool:
    """Whether zt_gemm_q4_f32 / zt_gemm_q8sep_f32 run a batch of n fp32
    columns (even n, 8-byte aligned) on the bf16 MFMA tile GEMM: from 128
    columns, and for Q8_0 also from 32 at 8192 rows and more and from 64
    past K = 8192 (the rules of zt_q4.hip and zt_q8.hip).  Such batches go
    to the entry point as they are, with no tiled copy and no 16-column
    chunks: 512 columns of 14336 x 4096 (rows x K) take 309 us (Q4_0) and
    256 us (Q8_0) on it."""
    if n % 2:
        return False
    if fmt == "q4":
        return n >= 128
    return n >= 128 or (n >= 32 and rows >= 8192) or (n >= 64 and k > 8192)


_TILED_BATCHES = (4, 8, 12, 16)  # batch sizes on the tiled layouts (W4A16, IQ4_NL, Q4_0, Q8_0, Q4_K, Q5_K, Q5_0)


def _detect_w4a16(a: Tensor, b: Tensor):
    """detectW4A16 (compute/w4a16.go:27-62)."""

    def w4(s):
        return isinstance(s, (Q4Storage, AWQStorage)) or (isinstance(s, GPTQStorage) and s.bits == 4)

    if isinstance(a, Tensor) and isinstance(b, Tensor):
        if w4(a.storage) and isinstance(b.storage, Float16Storage):
            return a, b, "A"
        if w4(b.storage) and isinstance(a.storage, Float16Storage):
            return b, a, "B"
    return None, None, ""
