"""CPU checks of the drop-in boundary: libzt_hip.so loads, exports every
entry point include/zt_hip.h declares with the ctypes table matching the
header, and its host-side layout converters produce the reference's device
layouts (checked against the oracle).  No GPU compute is called."""
import re
from pathlib import Path

import numpy as np
import pytest

from ztensor_amd import _lib, synth
from ztensor_amd.storage import IQ4NLStorage, Q4Storage, Q8Storage, TernaryStorage

ROOT = Path(__file__).resolve().parents[1]


def header_functions():
    text = (ROOT / "include" / "zt_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"^\s*(?:int|long|void)\s+(zt_\w+)\s*\(", text, flags=re.M))


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    declared = header_functions()
    assert len(declared) >= 20
    assert declared == set(_lib.SIGNATURES), declared ^ set(_lib.SIGNATURES)
    for name in declared:
        assert hasattr(lib.cdll, name)
    assert lib.zt_abi_version() == 102


def test_header_arity_matches_binding():
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / "zt_hip.h").read_text(), flags=re.S)
    for name, (_, args) in _lib.SIGNATURES.items():
        m = re.search(name + r"\s*\(([^)]*)\)", text)
        params = [p for p in m.group(1).split(",") if p.strip() and p.strip() != "void"]
        assert len(params) == len(args), name


def test_q4_and_iq4_gpu_layout_match_oracle(orc):
    for rows, K in [(1, 32), (3, 96), (16, 4096)]:
        w = synth.q4_0(rows, K, 1)
        s = Q4Storage.from_raw(w.raw, rows * K)
        nblk = rows * K // 32
        assert np.array_equal(s.raw_bytes_gpu(), orc.q4_raw_to_gpu(w.raw, nblk))
        assert s.gpu_data_offset() == orc.lib().orc_q4_gpu_data_offset(nblk)
        iq = IQ4NLStorage.from_raw(w.raw, rows * K)
        assert np.array_equal(iq.raw_bytes_gpu(), s.raw_bytes_gpu())


def test_q8_separated_layout():
    w = synth.q8_0(5, 64, 2)
    s = Q8Storage(w.raw, 5 * 64)
    g = s.raw_bytes_gpu()
    nblk = 10
    off = s.gpu_data_offset()
    assert off == 48 and g.size == off + 32 * nblk
    blocks = w.raw.reshape(nblk, 36)
    assert np.array_equal(g[: 4 * nblk].reshape(nblk, 4), blocks[:, :4])
    assert np.array_equal(g[off:].reshape(nblk, 32), blocks[:, 4:])


def test_ternary_repack_matches_oracle(orc):
    rng = np.random.default_rng(0)
    for rows, cols in [(3, 5), (4, 8), (33, 33), (2, 2560)]:
        w = rng.integers(-1, 2, rows * cols).astype(np.int8)
        raw = synth.pack_ternary(w)
        assert np.array_equal(TernaryStorage(raw, w.size).row_aligned(rows, cols),
                              orc.ternary_repack_rows(raw, rows, cols))


def test_storage_constructors_validate_like_reference():
    with pytest.raises(ValueError):
        Q4Storage.from_raw(np.zeros(10, np.uint8), 32)  # short raw
    with pytest.raises(ValueError):
        Q4Storage.from_raw(np.zeros(18, np.uint8), 0)
    with pytest.raises(ValueError):
        IQ4NLStorage.from_raw(np.zeros(10, np.uint8), 32)  # tensor/iq4_storage_test.go:137-142
    with pytest.raises(ValueError):
        IQ4NLStorage.from_raw(np.zeros(0, np.uint8), -1)
    with pytest.raises(ValueError):
        Q8Storage.from_blocks(np.zeros(1, np.float32), np.zeros(31, np.int8), 32)


def test_merge_storages_concatenate_blocks_like_reference(orc):
    """MergeQ4Storage / MergeIQ4NLStorage (tensor/quantized.go:224-242,
    tensor/iq4_storage.go:124-140): blocks in order, lengths summed; the
    merged Q/K/V storage dequantizes to the three matrices stacked row-wise
    and uploads to the RawBytesGPU layout of the concatenated blocks."""
    from ztensor_amd import synth
    from ztensor_amd.storage import IQ4NLStorage, Q4Storage, merge_iq4nl_storage, merge_q4_storage

    parts = [synth.q4_0(rows, 256, 40 + i) for i, rows in enumerate((64, 16, 16))]
    st = [Q4Storage.from_raw(p.raw, p.rows * p.K) for p in parts]
    m = merge_q4_storage(*st)
    assert m.len == 96 * 256 and m.num_blocks() == sum(s.num_blocks() for s in st)
    want = np.concatenate([orc.q4_dequant(p.raw, p.rows * p.K) for p in parts])
    assert np.array_equal(orc.q4_dequant(m.raw_bytes(), m.len).view(np.uint32), want.view(np.uint32))
    assert np.array_equal(m.raw_bytes_gpu(), orc.q4_raw_to_gpu(np.concatenate([p.raw for p in parts]), m.num_blocks()))
    iparts = [synth.iq4nl(rows, 128, 50 + i) for i, rows in enumerate((8, 4))]
    mi = merge_iq4nl_storage(*[IQ4NLStorage.from_raw(p.raw, p.rows * p.K) for p in iparts])
    want = np.concatenate([orc.iq4nl_dequant(p.raw, p.rows * p.K) for p in iparts])
    assert np.array_equal(orc.iq4nl_dequant(mi.raw_bytes(), mi.len).view(np.uint32), want.view(np.uint32))
    with pytest.raises(ValueError):
        merge_q4_storage()


def test_q5_0_gpu_layout_matches_oracle(orc):
    from ztensor_amd.storage import Q5_0Storage

    for rows, K in [(1, 32), (3, 96), (16, 4096)]:
        w = synth.kquant("q5_0", rows, K, 5)
        s = Q5_0Storage.from_raw(w.raw, rows * K)
        nblk = rows * K // 32
        assert np.array_equal(s.raw_bytes_gpu(), orc.q5_0_raw_to_gpu(w.raw, nblk))
        assert s.gpu_qh_offset() == orc.lib().orc_q5_0_gpu_qh_offset(nblk)
        assert s.gpu_qs_offset() == orc.lib().orc_q5_0_gpu_qs_offset(nblk)


def test_kquant_storage_constructors_validate_like_the_reference():
    from ztensor_amd.storage import Q4KStorage, Q5KStorage, Q6KStorage, merge_q4k_storage

    # NewQ4KStorageFromRaw_InvalidSize (tensor/quantized_kquant_test.go:208-213)
    with pytest.raises(ValueError):
        Q4KStorage.from_raw(np.zeros(10, np.uint8), 256)
    with pytest.raises(ValueError):
        Q6KStorage.from_raw(np.zeros(210, np.uint8), 0)
    s = Q5KStorage.from_raw(np.zeros(3 * 176 + 5, np.uint8), 700)
    assert s.num_blocks() == 3 and s.raw_bytes().size == 3 * 176
    a = Q4KStorage.from_raw(synth.kquant("q4_k", 2, 256, 1).raw, 512)
    b = Q4KStorage.from_raw(synth.kquant("q4_k", 1, 256, 2).raw, 256)
    m = merge_q4k_storage(a, b)  # TestMergeQ4KStorage (tensor/quantized_kquant_test.go:496-543)
    assert m.len == 768 and np.array_equal(m.raw, np.concatenate([a.raw, b.raw]))


def test_gguf_q8_0_device_layout():
    from ztensor_amd.storage import GGMLType, MmapStorage

    rows, K = 5, 64
    raw = synth.gguf_q8_0(rows, K, 7)
    s = MmapStorage(raw, rows * K, GGMLType.Q8_0)
    buf, offs = s.device_layout()
    nblk = rows * K // 32
    off = offs["data_offset"]
    assert off == 32 and buf.size == off + 32 * nblk  # (10*2 + 15) & ~15
    blocks = raw.reshape(nblk, 34)
    assert np.array_equal(buf[: 2 * nblk].reshape(nblk, 2), blocks[:, :2])
    assert not buf[2 * nblk:off].any()
    assert np.array_equal(buf[off:].reshape(nblk, 32), blocks[:, 2:])


def test_mmap_storage_validates_like_the_reference():
    from ztensor_amd.storage import GGMLType, MmapStorage, Q4Storage, mmap_byte_size

    # mmapByteSize (tensor/mmap_storage.go:85-119)
    assert mmap_byte_size(GGMLType.Q8_0, 64) == 68 and mmap_byte_size(GGMLType.Q4_K, 300) == 288
    assert mmap_byte_size(GGMLType.Q5_1, 33) == 48 and mmap_byte_size(GGMLType.BF16, 3) == 6
    with pytest.raises(ValueError):
        mmap_byte_size(99, 32)
    with pytest.raises(ValueError):
        MmapStorage(np.zeros(10, np.uint8), 32, GGMLType.Q8_0)  # too short
    with pytest.raises(ValueError):
        MmapStorage(np.zeros(0, np.uint8), 32, GGMLType.Q4_0)
    w = synth.q4_0(3, 64, 8)
    m = MmapStorage(np.concatenate([w.raw, np.zeros(9, np.uint8)]), 192, GGMLType.Q4_0)
    assert m.raw_bytes().size == 6 * 18
    # RawBytesGPU (tensor/mmap_storage.go:170-189) is Q4Storage's for Q4_0
    assert np.array_equal(m.raw_bytes_gpu(), Q4Storage.from_raw(w.raw, 192).raw_bytes_gpu())
    with pytest.raises(TypeError):
        MmapStorage(np.zeros(40, np.uint8), 32, GGMLType.Q4_1).device_layout()


def test_w4a16_tiled_layout_sizes():
    """The tiled W4A16 layout's byte counts (host helpers, no GPU): rows
    padded to a multiple of 16, K a multiple of 128, one dword per
    (group, row); shapes the layout does not take return -1."""
    from ztensor_amd import _lib

    lib = _lib.load()
    assert lib.zt_w4a16_tiled_bytes(8192, 8192) == 8192 * 4096
    assert lib.zt_w4a16_tiled_bytes(17, 256) == 32 * 128
    assert lib.zt_w4a16_tiled_bytes(1, 128) == 16 * 64
    assert lib.zt_w4a16_tiled_bytes(4, 96) == -1
    assert lib.zt_w4a16_sz_bytes(8192, 8192, 128) == 8192 * 64 * 4
    assert lib.zt_w4a16_sz_bytes(17, 256, 64) == 17 * 4 * 4
    assert lib.zt_w4a16_sz_bytes(4, 96, 64) == -1


def test_iq4nl_tiled_layout_sizes():
    """The tiled IQ4_NL layout's byte counts (host helpers, no GPU)."""
    from ztensor_amd import _lib

    lib = _lib.load()
    assert lib.zt_iq4nl_tiled_bytes(3584, 3584) == 3584 * 1792
    assert lib.zt_iq4nl_tiled_bytes(17, 256) == 32 * 128
    assert lib.zt_iq4nl_tiled_scale_bytes(17, 256) == 32 * 8 * 2
    assert lib.zt_iq4nl_tiled_bytes(4, 96) == -1 and lib.zt_iq4nl_tiled_scale_bytes(4, 96) == -1


def test_q4_q8_tiled_layout_and_workspace_sizes():
    """The tiled Q4_0 / Q8_0 layouts' byte counts and the split-K workspace
    sizes (host helpers, no GPU).  The workspace is one KB per 16-row tile
    per K split and 0 when K is not split; the split counts follow the
    launch heuristic (128 rows a workgroup, up to 4 units of 128 K, at least
    256 workgroups for Q4_0 and 512 for Q8_0)."""
    from ztensor_amd import _lib

    lib = _lib.load()
    assert lib.zt_q4_tiled_bytes(4096, 4096) == 4096 * 2048
    assert lib.zt_q4_tiled_bytes(17, 256) == 32 * 128
    assert lib.zt_q4_tiled_scale_bytes(17, 256) == 32 * 8 * 2
    assert lib.zt_q8_tiled_bytes(17, 256) == 32 * 256
    assert lib.zt_q8_tiled_scale_bytes(17, 256) == 32 * 8 * 4
    for f in ("q4", "q8"):
        assert getattr(lib, f"zt_{f}_tiled_bytes")(4, 96) == -1
        assert getattr(lib, f"zt_{f}_tiled_scale_bytes")(4, 96) == -1
    q4, q8 = lib.zt_gemm_q4t_workspace_bytes, lib.zt_gemm_q8t_workspace_bytes
    # 14336 x 4096: 112 row blocks, 4 units -> 8 splits; 896 tiles
    assert q4(14336, 4096, 8) == 8 * 896 * 1024 and q8(14336, 4096, 8) == 8 * 896 * 1024
    # 4096 x 4096: Q4_0 keeps 4 units (256 workgroups), Q8_0 drops to 2 (512)
    assert q4(4096, 4096, 8) == 8 * 256 * 1024 and q8(4096, 4096, 16) == 16 * 256 * 1024
    # 4096 x 14336: 28 splits
    assert q4(4096, 14336, 4) == 28 * 256 * 1024
    # K of one unit: no split, no workspace; unsupported shapes and batches: -1
    assert q4(100, 128, 8) == 0 and q8(100, 128, 8) == 0
    assert q4(0, 4096, 8) == 0
    assert q4(16, 96, 8) == -1 and q8(16, 128, 6) == -1 and q4(16, 128, 1) == -1


def test_kquant_and_q5_0_tiled_layout_sizes():
    """Byte counts of the tiled Q4_K / Q5_K / Q5_0 layouts (host helpers, no
    GPU): the Q4_0 tile data, 16 header bytes per row and super-block, one
    fifth-bit dword per lane and tile-unit (256 bytes per 16 rows x 128 K)."""
    from ztensor_amd import _lib

    lib = _lib.load()
    for f in ("q4k", "q5k"):
        assert getattr(lib, f"zt_{f}_tiled_bytes")(4096, 4096) == 4096 * 2048
        assert getattr(lib, f"zt_{f}_tiled_header_bytes")(17, 512) == 32 * 2 * 16
        assert getattr(lib, f"zt_{f}_tiled_bytes")(16, 128) == -1  # whole super-blocks only
        assert getattr(lib, f"zt_gemm_{f}t_workspace_bytes")(16, 256, 8) == 0
    assert lib.zt_q5k_tiled_qh_bytes(17, 512) == 2 * 4 * 256
    assert lib.zt_q6k_tiled_bytes(17, 512) == 32 * 512
    assert lib.zt_q6k_tiled_scale_bytes(17, 512) == 32 * 32 * 4
    assert lib.zt_q6k_tiled_bytes(16, 128) == -1
    assert lib.zt_gemm_q6kt_workspace_bytes(16, 256, 8) == 0
    assert lib.zt_q5_0_tiled_bytes(17, 256) == 32 * 128
    assert lib.zt_q5_0_tiled_scale_bytes(17, 256) == 32 * 8 * 2
    assert lib.zt_q5_0_tiled_qh_bytes(17, 256) == 2 * 2 * 256
    assert lib.zt_q5_0_tiled_qh_bytes(17, 96) == -1
    assert lib.zt_gemm_q5_0t_workspace_bytes(14336, 4096, 8) == 8 * 896 * 1024


def test_q4_group_rejects_bad_arguments_without_launching():
    """zt_gemm_q4_group_f32 validates every descriptor before any launch:
    each case returns InvalidValue (1) with no GPU present."""
    lib = _lib.load()
    good = (0x10000, 16, 0x20000, 8)
    x = 0x30000
    cases = [
        ([good], 0, x, 64),                      # n < 1
        ([good] * 9, 9, x, 64),                  # n > ZT_GROUP_MAX
        ([good], 1, x, 48),                      # K % 32 != 0
        ([good], 1, x + 4, 64),                  # misaligned activations
        ([good], 1, 0, 64),                      # null activations
        ([(0, 16, 0x20000, 8)], 1, x, 64),       # null weights
        ([(0x10000, 16, 0, 8)], 1, x, 64),       # null output
        ([(0x10000, 8, 0x20000, 8)], 1, x, 64),  # data not 16-byte aligned
        ([(0x10000, 16, 0x20000, -1)], 1, x, 64),  # negative rows
    ]
    for entries, n, xp, K in cases:
        descs = _lib.q4_gemv_descs(entries)
        assert lib.zt_gemm_q4_group_f32(descs, n, xp, K, None) == _lib.HIP_ERROR_INVALID_VALUE, (entries, n, K)
    assert lib.zt_gemm_q4_group_f32(None, 1, x, 64, None) == _lib.HIP_ERROR_INVALID_VALUE
    d = _lib.q4_gemv_descs([good])
    d[0].reserved = 1
    assert lib.zt_gemm_q4_group_f32(d, 1, x, 64, None) == _lib.HIP_ERROR_INVALID_VALUE


def test_q4t_noalloc_rejects_oversized_and_bad_calls_without_launching():
    """zt_gemm_q4t_f32_noalloc checks the scratch size and the shape before
    touching the GPU: a call whose partials exceed ZT_NOALLOC_SCRATCH_BYTES
    runs in row slices, so only one whose single 128-row slice needs more
    (K past 2^19: 2048 splits x 8 tiles x 1 KB = 16 MiB) returns
    hipErrorOutOfMemory; a bad shape returns InvalidValue."""
    lib = _lib.load()
    assert lib.zt_gemm_q4t_workspace_bytes(28672, 8192, 8) > _lib.NOALLOC_SCRATCH_BYTES  # sliced, not refused
    p = 0x10000
    assert lib.zt_gemm_q4t_workspace_bytes(128, 1 << 20, 8) == 16 << 20
    assert lib.zt_gemm_q4t_f32_noalloc(p, p, p, p, 128, 1 << 20, 8, None) == _lib.HIP_ERROR_OUT_OF_MEMORY
    assert lib.zt_gemm_q4t_f32_noalloc(p, p, p, p, 64, 96, 8, None) == _lib.HIP_ERROR_INVALID_VALUE  # K % 128
    assert lib.zt_gemm_q4t_f32_noalloc(p, p, p, p, 64, 128, 5, None) == _lib.HIP_ERROR_INVALID_VALUE  # N


def test_int4_int8_gemms_reject_like_the_reference_without_launching():
    """zt_gemm_int4_f32 / _rmul return InvalidValue for an odd K (odd
    out_features) or group_size <= 0, as gemm_int4.cu:64-69, 122-127 do, and
    for negative sizes or NULL buffers; empty outputs return 0.  No GPU."""
    lib = _lib.load()
    p, bad = 0x10000, _lib.HIP_ERROR_INVALID_VALUE
    assert lib.zt_gemm_int4_f32(p, p, p, p, p, 4, 33, 4, 32, None) == bad  # odd K
    assert lib.zt_gemm_int4_f32(p, p, p, p, p, 4, 32, 4, 0, None) == bad  # group_size
    assert lib.zt_gemm_int4_f32(p, p, p, p, p, -1, 32, 4, 32, None) == bad
    assert lib.zt_gemm_int4_f32(p, None, p, p, p, 4, 32, 4, 32, None) == bad
    assert lib.zt_gemm_int4_f32(p, p, p, p, p, 0, 32, 4, 32, None) == 0
    assert lib.zt_gemm_int4_f32_rmul(p, p, p, p, p, 4, 32, 33, 32, None) == bad  # odd out
    assert lib.zt_gemm_int4_f32_rmul(p, p, p, p, p, 4, 32, 32, -2, None) == bad
    assert lib.zt_gemm_int4_f32_rmul(p, p, p, p, None, 4, 32, 32, 32, None) == bad
    assert lib.zt_gemm_int4_f32_rmul(p, p, p, p, p, 4, 32, 0, 32, None) == 0
    assert lib.zt_gemm_int8_f32(p, p, p, 4, -1, 4, None) == bad
    assert lib.zt_gemm_int8_f32(None, p, p, 4, 16, 4, None) == bad
    assert lib.zt_gemm_int8_f32(p, p, p, 4, 16, 0, None) == 0


def test_ccall_style_calls_through_all_uintptr_signature(tmp_path):
    """tests/ccall_abi.c, compiled here with gcc, dlopens libzt_hip.so and
    calls entry points through a 20-argument all-uintptr_t function pointer,
    as the reference's Ccall does; only validation paths, no kernel."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / "ccall_abi"
    subprocess.run([cc, "-O1", "-std=c11", "-Wall", "-o", str(exe), str(ROOT / "tests" / "ccall_abi.c"), "-ldl"],
                   check=True)
    r = subprocess.run([str(exe), str(_lib.LIB_PATH)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
