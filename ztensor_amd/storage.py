"""Host-side quantized storage types, mirroring the reference's tensor package.

Each class holds the reference's serialised bytes on the host (numpy) and
knows its device upload layout.  Names and semantics follow the Go types so a
caller of tensor.Q4Storage & co. finds the same surface:

  Q4Storage      tensor/quantized.go:22-274   (RawBytes, RawBytesGPU, NumBlocks, SetGPUPtr/GPUPtr,
                                               MergeQ4Storage -> merge_q4_storage)
  Q8Storage      tensor/quantized.go:288-478  (36-byte blocks, fp32 scale)
  IQ4NLStorage   tensor/iq4_storage.go:48-142 (MergeIQ4NLStorage -> merge_iq4nl_storage)
  GPTQStorage    tensor/quantized_gptq.go:30-280 (bits = 4 for W4A16)
  AWQStorage     tensor/quantized_awq.go:30-321
  TernaryStorage tensor/ternary_storage.go:7-95
  Float16Storage tensor/fp16_storage.go:14-122
  Q4KStorage     tensor/quantized_kquant.go:236-339 (MergeQ4KStorage -> merge_q4k_storage)
  Q5KStorage     tensor/quantized_kquant.go:552-636
  Q6KStorage     tensor/quantized_kquant.go:385-505 (MergeQ6KStorage -> merge_q6k_storage)
  Q5_0Storage    tensor/quantized_q5_0.go:47-184 (RawBytesGPU, Q5_0GPUQhOffset/QsOffset)
  MmapStorage    tensor/mmap_storage.go:16-189 (GGUF tensors by GGML type; device_layout adds the
                 repacks the engine uploads)

Dequantization on the host is not offered here on purpose: the product path
dequantizes on the GPU (zt_dequant_*), and the CPU restatement used to check
it lives in the test-only oracle.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field
from enum import IntEnum
from typing import Any

import numpy as np

from . import _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data_as(C.c_void_p).value or 0


@dataclass
class GPUBuffer:
    """A device copy set by the engine's upload (SetGPUPtr); the caller (the
    engine) owns the memory, as in tensor/quantized.go:200-212."""

    tensor: Any  # torch.Tensor (uint8, on the device)
    nbytes: int
    device_id: int
    data_offset: int = 0


class _GPUPtrMixin:
    _gpu: GPUBuffer | None

    def set_gpu_ptr(self, buf: GPUBuffer | None) -> None:
        self._gpu = buf
        self._gpu_tiled = None  # a tiled copy built from the previous upload is stale
        self._gpu_split = None  # so is a split copy (Q6_K batch 1)

    def gpu_ptr(self) -> GPUBuffer | None:
        return self._gpu


@dataclass
class Q4Storage(_GPUPtrMixin):
    raw: np.ndarray  # 18-byte blocks
    len: int
    _gpu: GPUBuffer | None = field(default=None, repr=False)

    @staticmethod
    def from_raw(raw: np.ndarray, num_elements: int) -> "Q4Storage":
        """NewQ4StorageFromRaw (tensor/quantized.go:247-264)."""
        if num_elements <= 0:
            raise ValueError(f"numElements must be positive, got {num_elements}")
        nblk = (num_elements + 31) // 32
        raw = np.asarray(raw, np.uint8).reshape(-1)
        if raw.size < nblk * 18:
            raise ValueError(f"Q4_0 raw data too short: need {nblk * 18} bytes for {nblk} blocks, got {raw.size}")
        return Q4Storage(raw[: nblk * 18].copy(), num_elements)

    def num_blocks(self) -> int:
        return (self.len + 31) // 32

    def byte_size(self) -> int:
        return self.num_blocks() * 18

    def raw_bytes(self) -> np.ndarray:
        return self.raw

    def raw_bytes_gpu(self) -> np.ndarray:
        """RawBytesGPU (tensor/quantized.go:168-187), built by the library."""
        lib = _lib.load()
        nblk = self.num_blocks()
        out = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
        lib.zt_q4_raw_to_gpu(_ptr(self.raw), nblk, _ptr(out))
        return out

    def gpu_data_offset(self) -> int:
        """Q4GPUDataOffset (tensor/quantized.go:195-198)."""
        return _lib.load().zt_q4_gpu_data_offset(self.num_blocks())


def merge_q4_storage(*storages: "Q4Storage") -> "Q4Storage":
    """MergeQ4Storage (tensor/quantized.go:224-242): the blocks of every
    storage, in order, as one storage whose length is the sum of the lengths.
    Merging the row-major Q, K and V (or Gate and Up) weights this way gives
    one [sum(rows), K] matrix, so a decode step runs one GEMV instead of
    three (or two)."""
    if not storages:
        raise ValueError("merge_q4_storage: no storages")
    return Q4Storage(np.concatenate([st.raw for st in storages]), sum(st.len for st in storages))


@dataclass
class IQ4NLStorage(_GPUPtrMixin):
    raw: np.ndarray
    len: int
    _gpu: GPUBuffer | None = field(default=None, repr=False)

    @staticmethod
    def from_raw(raw: np.ndarray, num_elements: int) -> "IQ4NLStorage":
        """NewIQ4NLStorageFromRaw (tensor/iq4_storage.go:60-72)."""
        if num_elements <= 0:
            raise ValueError(f"numElements must be positive, got {num_elements}")
        nblk = (num_elements + 31) // 32
        raw = np.asarray(raw, np.uint8).reshape(-1)
        if raw.size < nblk * 18:
            raise ValueError(f"IQ4_NL raw data too short: need {nblk * 18} bytes for {nblk} blocks, got {raw.size}")
        return IQ4NLStorage(raw[: nblk * 18].copy(), num_elements)

    def num_blocks(self) -> int:
        return (self.len + 31) // 32

    def raw_bytes(self) -> np.ndarray:
        return self.raw

    def raw_bytes_gpu(self) -> np.ndarray:
        lib = _lib.load()
        nblk = self.num_blocks()
        out = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
        lib.zt_iq4nl_raw_to_gpu(_ptr(self.raw), nblk, _ptr(out))
        return out

    def gpu_data_offset(self) -> int:
        return _lib.load().zt_q4_gpu_data_offset(self.num_blocks())


def merge_iq4nl_storage(*storages: "IQ4NLStorage") -> "IQ4NLStorage":
    """MergeIQ4NLStorage (tensor/iq4_storage.go:124-140): raw blocks
    concatenated in order, lengths summed."""
    if not storages:
        raise ValueError("merge_iq4nl_storage: no storages")
    return IQ4NLStorage(np.concatenate([st.raw for st in storages]), sum(st.len for st in storages))


@dataclass
class Q8Storage(_GPUPtrMixin):
    raw: np.ndarray  # 36-byte blocks
    len: int
    _gpu: GPUBuffer | None = field(default=None, repr=False)

    @staticmethod
    def from_blocks(scales: np.ndarray, quants: np.ndarray, num_elements: int) -> "Q8Storage":
        """NewQ8StorageFromBlocks (tensor/quantized.go:457-475)."""
        if num_elements <= 0:
            raise ValueError(f"numElements must be positive, got {num_elements}")
        nblk = (num_elements + 31) // 32
        scales = np.asarray(scales, np.float32).reshape(-1)
        quants = np.asarray(quants, np.int8).reshape(-1)
        if scales.size != nblk:
            raise ValueError(f"expected {nblk} scales for {num_elements} elements, got {scales.size}")
        if quants.size != nblk * 32:
            raise ValueError(f"expected {nblk * 32} quants for {nblk} blocks, got {quants.size}")
        raw = np.empty((nblk, 36), np.uint8)
        raw[:, :4] = scales.astype("<f4").reshape(nblk, 1).view(np.uint8)
        raw[:, 4:] = quants.reshape(nblk, 32).view(np.uint8)
        return Q8Storage(raw.reshape(-1), num_elements)

    def num_blocks(self) -> int:
        return (self.len + 31) // 32

    def byte_size(self) -> int:
        return self.num_blocks() * 36

    def raw_bytes(self) -> np.ndarray:
        """RawBytes (tensor/quantized.go:427-438)."""
        return self.raw

    def raw_bytes_gpu(self) -> np.ndarray:
        lib = _lib.load()
        nblk = self.num_blocks()
        out = np.empty(lib.zt_q8_gpu_bytes(nblk), np.uint8)
        lib.zt_q8_raw_to_gpu(_ptr(self.raw), nblk, _ptr(out))
        return out

    def gpu_data_offset(self) -> int:
        return _lib.load().zt_q8_gpu_data_offset(self.num_blocks())


@dataclass
class GPTQStorage(_GPUPtrMixin):
    data: np.ndarray  # packed groups, concatenated
    scales: np.ndarray  # uint16 fp16 bits, one per group
    zeros: np.ndarray  # uint16 fp16 bits, one per group
    len: int
    group_size: int
    bits: int = 4
    _gpu: GPUBuffer | None = field(default=None, repr=False)

    @staticmethod
    def from_raw(data, scales, zeros, num_elements: int, group_size: int, bits: int) -> "GPTQStorage":
        """NewGPTQStorageFromRaw (tensor/quantized_gptq.go:217-277)."""
        if num_elements <= 0:
            raise ValueError(f"numElements must be positive, got {num_elements}")
        if bits not in (4, 8):
            raise ValueError(f"bits must be 4 or 8, got {bits}")
        ng = (num_elements + group_size - 1) // group_size
        scales = np.asarray(scales, np.uint16).reshape(-1)
        zeros = np.asarray(zeros, np.uint16).reshape(-1)
        if scales.size != ng:
            raise ValueError(f"expected {ng} scales for {ng} groups, got {scales.size}")
        if zeros.size != ng:
            raise ValueError(f"expected {ng} zeros for {ng} groups, got {zeros.size}")
        total = 0
        for gi in range(ng):
            cnt = min(group_size, num_elements - gi * group_size)
            total += (cnt + 1) // 2 if bits == 4 else cnt
        data = np.asarray(data, np.uint8).reshape(-1)
        if data.size < total:
            raise ValueError(f"GPTQ data too short: need {total} bytes, got {data.size}")
        return GPTQStorage(data[:total].copy(), scales.copy(), zeros.copy(), num_elements, group_size, bits)

    def num_groups(self) -> int:
        return self.scales.size

    def byte_size(self) -> int:
        return self.data.size + 4 * self.num_groups()


@dataclass
class AWQStorage(_GPUPtrMixin):
    words: np.ndarray  # uint32, 8 nibbles each, groups concatenated
    scales: np.ndarray
    zeros: np.ndarray
    len: int
    group_size: int
    _gpu: GPUBuffer | None = field(default=None, repr=False)

    def packed_bytes(self) -> np.ndarray:
        """The words' little-endian bytes: identical to GPTQ 4-bit packing when
        the group size is a multiple of 8 (tensor/quantized_awq.go:97-105)."""
        return self.words.astype("<u4").view(np.uint8)


@dataclass
class TernaryStorage:
    data: np.ndarray  # flat 2-bit packing
    len: int

    def raw_bytes(self) -> np.ndarray:
        return self.data

    def row_aligned(self, rows: int, cols: int) -> np.ndarray:
        """The per-row byte-aligned layout of compute/ternary_gemv_gpu.go:55-67."""
        lib = _lib.load()
        out = np.empty(rows * ((cols + 3) // 4), np.uint8)
        lib.zt_ternary_repack_rows(_ptr(self.data), rows, cols, _ptr(out))
        return out


@dataclass
class Float16Storage(_GPUPtrMixin):
    data: np.ndarray  # uint16 fp16 bits
    len: int
    _gpu: GPUBuffer | None = field(default=None, repr=False)

    @staticmethod
    def from_raw(raw: np.ndarray, num_elems: int) -> "Float16Storage":
        """NewFloat16StorageFromRaw (tensor/fp16_storage.go:42-46)."""
        return Float16Storage(np.asarray(raw).view(np.uint16).reshape(-1)[:num_elems].copy(), num_elems)


class _KQuantBase(_GPUPtrMixin):
    """Shared body of the K-quant storages: contiguous super-blocks of 256
    values, uploaded to the device unchanged (compute/gpu_engine.go:817-874)."""

    BLOCK_VALUES = 256
    BLOCK_BYTES = 0
    NAME = ""

    def __init__(self, raw: np.ndarray, length: int):
        self.raw = raw
        self.len = length
        self._gpu = None

    @classmethod
    def from_raw(cls, raw: np.ndarray, num_elements: int):
        """NewQ4KStorageFromRaw / NewQ5KStorageFromRaw / NewQ6KStorageFromRaw
        (tensor/quantized_kquant.go:248-261, 564-577, 397-410): the first
        ceil(n/256) super-blocks are copied; shorter data is an error."""
        if num_elements <= 0:
            raise ValueError(f"numElements must be positive, got {num_elements}")
        nb = (num_elements + cls.BLOCK_VALUES - 1) // cls.BLOCK_VALUES
        need = nb * cls.BLOCK_BYTES
        raw = np.asarray(raw, np.uint8).reshape(-1)
        if raw.size < need:
            raise ValueError(f"{cls.NAME} raw data too short: need {need} bytes for {nb} blocks, got {raw.size}")
        return cls(raw[:need].copy(), num_elements)

    def num_blocks(self) -> int:
        return (self.len + self.BLOCK_VALUES - 1) // self.BLOCK_VALUES

    def byte_size(self) -> int:
        return self.num_blocks() * self.BLOCK_BYTES

    def raw_bytes(self) -> np.ndarray:
        return self.raw

    def block_raw(self, i: int) -> np.ndarray:
        """BlockRaw (tensor/quantized_kquant.go:450-454, 618-622)."""
        return self.raw[i * self.BLOCK_BYTES:(i + 1) * self.BLOCK_BYTES]


class Q4KStorage(_KQuantBase):
    """Q4_K: 144-byte super-blocks [fp16 d][fp16 dmin][12 B scales/mins][128 B nibbles]."""

    BLOCK_BYTES = 144
    NAME = "Q4_K"


class Q5KStorage(_KQuantBase):
    """Q5_K: 176-byte super-blocks (Q4_K plus 32 bytes of fifth bits)."""

    BLOCK_BYTES = 176
    NAME = "Q5_K"


class Q6KStorage(_KQuantBase):
    """Q6_K: 210-byte super-blocks [128 ql][64 qh][16 int8 scales][fp16 d]."""

    BLOCK_BYTES = 210
    NAME = "Q6_K"


def merge_q4k_storage(*storages: Q4KStorage) -> Q4KStorage:
    """MergeQ4KStorage (tensor/quantized_kquant.go:316-336)."""
    if not storages:
        raise ValueError("merge_q4k_storage: no storages")
    return Q4KStorage(np.concatenate([st.raw for st in storages]), sum(st.len for st in storages))


def merge_q6k_storage(*storages: Q6KStorage) -> Q6KStorage:
    """MergeQ6KStorage (tensor/quantized_kquant.go:470-490)."""
    if not storages:
        raise ValueError("merge_q6k_storage: no storages")
    return Q6KStorage(np.concatenate([st.raw for st in storages]), sum(st.len for st in storages))


class Q5_0Storage(_GPUPtrMixin):
    """Q5_0: 22-byte blocks of 32 values [fp16 d][uint32 qh][16 B nibbles]."""

    def __init__(self, raw: np.ndarray, length: int):
        self.raw = raw
        self.len = length
        self._gpu = None

    @staticmethod
    def from_raw(raw: np.ndarray, num_elements: int) -> "Q5_0Storage":
        """NewQ5_0StorageFromRaw (tensor/quantized_q5_0.go:60-73)."""
        if num_elements <= 0:
            raise ValueError(f"numElements must be positive, got {num_elements}")
        nb = (num_elements + 31) // 32
        raw = np.asarray(raw, np.uint8).reshape(-1)
        if raw.size < nb * 22:
            raise ValueError(f"Q5_0 raw data too short: need {nb * 22} bytes for {nb} blocks, got {raw.size}")
        return Q5_0Storage(raw[: nb * 22].copy(), num_elements)

    def num_blocks(self) -> int:
        return (self.len + 31) // 32

    def raw_bytes(self) -> np.ndarray:
        return self.raw

    def raw_bytes_gpu(self) -> np.ndarray:
        """RawBytesGPU (tensor/quantized_q5_0.go:118-147), built by the library."""
        lib = _lib.load()
        nb = self.num_blocks()
        out = np.empty(lib.zt_q5_0_gpu_bytes(nb), np.uint8)
        lib.zt_q5_0_raw_to_gpu(_ptr(self.raw), nb, _ptr(out))
        return out

    def gpu_qh_offset(self) -> int:
        """Q5_0GPUQhOffset (tensor/quantized_q5_0.go:151-156)."""
        return _lib.load().zt_q5_0_gpu_qh_offset(self.num_blocks())

    def gpu_qs_offset(self) -> int:
        """Q5_0GPUQsOffset (tensor/quantized_q5_0.go:158-165)."""
        return _lib.load().zt_q5_0_gpu_qs_offset(self.num_blocks())


class GGMLType(IntEnum):
    """tensor/mmap_storage.go:16-30."""

    F32 = 0
    F16 = 1
    Q4_0 = 2
    Q4_1 = 3
    Q5_0 = 6
    Q5_1 = 7
    Q8_0 = 8
    Q4_K = 12
    Q5_K = 13
    Q6_K = 14
    BF16 = 30


# (values per block, bytes per block), tensor/mmap_storage.go:85-119 mmapByteSize
_GGML_BLOCK = {
    GGMLType.F32: (1, 4), GGMLType.F16: (1, 2), GGMLType.BF16: (1, 2),
    GGMLType.Q4_0: (32, 18), GGMLType.Q8_0: (32, 34), GGMLType.Q4_1: (32, 20),
    GGMLType.Q5_0: (32, 22), GGMLType.Q5_1: (32, 24),
    GGMLType.Q4_K: (256, 144), GGMLType.Q5_K: (256, 176), GGMLType.Q6_K: (256, 210),
}


def mmap_byte_size(qtype: int, num_elements: int) -> int:
    """mmapByteSize (tensor/mmap_storage.go:85-119)."""
    try:
        vals, nbytes = _GGML_BLOCK[GGMLType(qtype)]
    except (ValueError, KeyError):
        raise ValueError(f"unsupported GGML type {qtype}") from None
    return (num_elements + vals - 1) // vals * nbytes


class MmapStorage(_GPUPtrMixin):
    """A GGUF tensor's raw bytes (a view of the mmap'd file) with its GGML type."""

    def __init__(self, data: np.ndarray, length: int, qtype: int):
        """NewMmapStorage (tensor/mmap_storage.go:59-83): length > 0, data
        non-empty and at least mmapByteSize long; the storage keeps exactly
        that many bytes."""
        if length <= 0:
            raise ValueError(f"mmap storage: length must be positive, got {length}")
        data = np.asarray(data, np.uint8).reshape(-1)
        if data.size == 0:
            raise ValueError("mmap storage: data must not be empty")
        need = mmap_byte_size(qtype, length)
        if data.size < need:
            raise ValueError(f"mmap storage: data too short for {length} elements of type {int(qtype)}: "
                             f"need {need} bytes, got {data.size}")
        self.data = data[:need]
        self.len = length
        self.qtype = GGMLType(qtype)
        self._gpu = None

    def byte_size(self) -> int:
        return self.data.size

    def raw_bytes(self) -> np.ndarray:
        return self.data

    def num_blocks(self) -> int:
        vals, _ = _GGML_BLOCK[self.qtype]
        return (self.len + vals - 1) // vals

    def raw_bytes_gpu(self) -> np.ndarray:
        """RawBytesGPU (tensor/mmap_storage.go:170-189): Q4_0 in the separated
        layout, every other type unchanged."""
        if self.qtype != GGMLType.Q4_0:
            return self.data
        lib = _lib.load()
        nb = self.data.size // 18
        out = np.empty(lib.zt_q4_gpu_bytes(nb), np.uint8)
        lib.zt_q4_raw_to_gpu(_ptr(self.data), nb, _ptr(out))
        return out

    def device_layout(self) -> tuple[np.ndarray, dict]:
        """The bytes this library's kernels read and their offsets: Q4_0 as
        RawBytesGPU; Q8_0 repacked to [fp16 scales][pad][int8 payloads]
        (zt_q8gguf_raw_to_gpu); Q5_0 as Q5_0Storage.RawBytesGPU; the K-quants
        unchanged."""
        lib = _lib.load()
        nb = self.num_blocks()
        if self.qtype == GGMLType.Q4_0:
            return self.raw_bytes_gpu(), {"data_offset": lib.zt_q4_gpu_data_offset(nb)}
        if self.qtype == GGMLType.Q8_0:
            out = np.empty(lib.zt_q8gguf_gpu_bytes(nb), np.uint8)
            lib.zt_q8gguf_raw_to_gpu(_ptr(self.data), nb, _ptr(out))
            return out, {"data_offset": lib.zt_q8gguf_gpu_data_offset(nb)}
        if self.qtype == GGMLType.Q5_0:
            out = np.empty(lib.zt_q5_0_gpu_bytes(nb), np.uint8)
            lib.zt_q5_0_raw_to_gpu(_ptr(self.data), nb, _ptr(out))
            return out, {"qh_offset": lib.zt_q5_0_gpu_qh_offset(nb), "qs_offset": lib.zt_q5_0_gpu_qs_offset(nb)}
        if self.qtype in (GGMLType.Q4_K, GGMLType.Q5_K, GGMLType.Q6_K):
            return self.data, {}
        raise TypeError(f"GGML type {self.qtype.name} has no quantized GEMV on this path")


@dataclass
class Tensor:
    """A shaped view over a storage (the subset of tensor.TensorNumeric the
    matmul dispatch reads: shape and storage type)."""

    shape: tuple[int, ...]
    storage: Any
