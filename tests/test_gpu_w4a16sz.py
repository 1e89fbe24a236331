"""GPU parity of the batch-1 W4A16 GEMV on packed (scale, zero) dwords
(zt_w4a16_pack_szr, zt_gemv_w4a16sz_f32).

This is the batch-1 form of W4A16MatMuler.MatMulW4A16 (compute/w4a16.go:
137-143) that the engine runs.  Bars:
  * the packing: byte-identical with scale | zero << 16 per (row, group),
    row-major, zero 8.0 (0x4800) when zeros is NULL;
  * the GEMV: max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle's
    restatement of the reference CPU engine (dequantize, then SgemmSimd),
    and within 1e-5 of zt_gemm_w4a16_f32 with N = 1 on the same operands.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5  # every product exact in fp32: only the summation order differs


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return _lib.load()


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def pack_dev(lib, w, zeros=True):
    s = dev(w.scales)
    z = dev(w.zeros) if zeros else None
    szr = torch.empty(w.scales.size, dtype=torch.int32, device="cuda")
    lib.call("zt_w4a16_pack_szr", s.data_ptr(), z.data_ptr() if zeros else 0, w.rows, w.K, w.group, szr.data_ptr(),
             stream())
    return szr


def gemv(lib, w, szr, x16):
    p, xd = dev(w.packed), dev(x16)
    y = torch.empty(w.rows, dtype=torch.float32, device="cuda")
    lib.call("zt_gemv_w4a16sz_f32", p.data_ptr(), szr.data_ptr(), xd.data_ptr(), y.data_ptr(), w.rows, w.K, w.group,
             stream())
    return y.cpu().numpy()


def rowmajor(lib, w, x16, zeros=True):
    p, s, xd = dev(w.packed), dev(w.scales), dev(x16)
    z = dev(w.zeros) if zeros else None
    y = torch.empty(w.rows, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_w4a16_f32", p.data_ptr(), s.data_ptr(), z.data_ptr() if zeros else 0, xd.data_ptr(),
             y.data_ptr(), w.rows, w.K, 1, w.group, stream())
    return y.cpu().numpy()


@pytest.mark.parametrize("zeros", [True, False])
def test_pack_szr_bytes(lib, zeros):
    w = synth.w4a16(37, 512, 81, group=64)
    got = pack_dev(lib, w, zeros).cpu().numpy().view(np.uint32)
    z = w.zeros.astype(np.uint32) if zeros else np.full(w.scales.shape, 0x4800, np.uint32)
    assert np.array_equal(got, (w.scales.astype(np.uint32) | (z << 16)).reshape(-1))


@pytest.mark.parametrize("rows,K,g", [(1, 32, 32), (3, 96, 32), (17, 256, 64), (100, 1024, 128), (1000, 4096, 128),
                                      (33, 4128, 32), (64, 8192, 256), (9, 12288, 128), (40, 32768, 128),
                                      (5, 16384 + 96, 32)])
def test_w4sz_ragged(lib, orc, rows, K, g):
    """Rows that are not a multiple of the rows per wave, every step count
    (K up to 4096: one step; 8192: two; above: four), the largest K (32768),
    partial last steps (4128, 16480) and group sizes 32 .. 256."""
    print(f"w4a16sz rows={rows} K={K} g={g}", flush=True)
    w = synth.w4a16(rows, K, 82, group=g)
    x16 = synth.x_f16(K, 82)
    y = gemv(lib, w, pack_dev(lib, w), x16)
    assert rel_err(y, orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, g)) <= TOL
    assert rel_err(y, rowmajor(lib, w, x16)) <= 1e-5


@pytest.mark.parametrize("rows,K", [(4096, 4096), (8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)])
def test_w4sz_config_shapes(lib, orc, rows, K):
    """The W4A16 configurations' batch-1 shapes (Llama-3-8B 4096 x 4096 and
    the Llama-3-70B layer) at full size."""
    print(f"w4a16sz rows={rows} K={K}", flush=True)
    w = synth.w4a16(rows, K, synth.seed_for(4, rows % 97 + K % 89))
    x16 = synth.x_f16(K, 83)
    y = gemv(lib, w, pack_dev(lib, w), x16)
    assert rel_err(y, orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128)) <= TOL
    assert rel_err(y, rowmajor(lib, w, x16)) <= 1e-5


def test_w4sz_default_zero_and_non_integer_zeros(lib, orc):
    rows, K = 256, 2048
    w = synth.w4a16(rows, K, 84)
    x16 = synth.x_f16(K, 84)
    y = gemv(lib, w, pack_dev(lib, w, zeros=False), x16)
    assert rel_err(y, rowmajor(lib, w, x16, zeros=False)) <= 1e-5
    z8 = np.full(w.zeros.shape, synth.f16_bits(np.float32(8.0)), np.uint16)
    assert rel_err(y, orc.w4a16_matmul(w.packed, w.scales, z8, x16, rows, K, 1, 128)) <= TOL
    rng = np.random.default_rng(84)
    zeros = synth.f16_bits((rng.random(w.zeros.shape, dtype=np.float32) * 15).astype(np.float32))
    w2 = synth.W4Weights(rows, K, w.group, w.packed, w.scales, zeros)
    y2 = gemv(lib, w2, pack_dev(lib, w2), x16)
    assert rel_err(y2, orc.w4a16_matmul(w2.packed, w2.scales, w2.zeros, x16, rows, K, 1, 128)) <= TOL


def test_w4sz_small_activations(lib, orc):
    """Activations of order 1e-4 (many fp16 subnormals): the nibble operands
    are exact and the products are formed in fp32."""
    rows, K = 512, 4096
    w = synth.w4a16(rows, K, 85)
    rng = np.random.default_rng(85)
    x16 = synth.f16_bits(rng.standard_normal(K).astype(np.float32) * np.float32(1e-4))
    y = gemv(lib, w, pack_dev(lib, w), x16)
    assert rel_err(y, orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128)) <= TOL


def test_w4sz_k_zero_writes_zeros(lib):
    y = torch.full((7,), float("nan"), dtype=torch.float32, device="cuda")
    t = torch.zeros(64, dtype=torch.uint8, device="cuda")
    lib.call("zt_gemv_w4a16sz_f32", t.data_ptr(), t.data_ptr(), t.data_ptr(), y.data_ptr(), 7, 0, 32, stream())
    assert torch.equal(y.cpu(), torch.zeros(7))
    c = torch.full((7 * 3,), float("nan"), dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_w4a16_f32", t.data_ptr(), t.data_ptr(), 0, t.data_ptr(), c.data_ptr(), 7, 0, 3, 32, stream())
    assert torch.equal(c.cpu(), torch.zeros(21))


def test_w4sz_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    for rows, K, g in [(2, 96, 48), (2, 128, 96), (2, 32768 + 128, 128), (2, 128, 0)]:
        assert lib.zt_gemv_w4a16sz_f32(p, p, p, p, rows, K, g, stream()) == 1, (rows, K, g)
    assert lib.zt_gemv_w4a16sz_f32(p + 8, p, p, p, 2, 128, 128, stream()) == 1  # W alignment
    assert lib.zt_gemv_w4a16sz_f32(p, p, p + 2, p, 2, 128, 128, stream()) == 1  # x alignment
    assert lib.zt_gemv_w4a16sz_f32(p, p + 2, p, p, 2, 128, 128, stream()) == 1  # szr alignment
    assert lib.zt_w4a16_pack_szr(p, p, 2, 128, 48, p, stream()) == 1
    assert lib.zt_w4a16_pack_szr(p + 1, p, 2, 128, 32, p, stream()) == 1


def test_engine_batch1_w4a16_uses_packed_scales(lib, orc):
    """ROCmEngine.matmul_w4a16 with one activation column packs the
    (scale, zero) dwords at upload and, for 4096 < K <= 16384, runs on them;
    the result matches the oracle."""
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Float16Storage, GPTQStorage, Tensor

    rows, K = 1024, 8192
    w = synth.w4a16(rows, K, 86)
    st = GPTQStorage.from_raw(w.packed.reshape(-1), w.scales.reshape(-1), w.zeros.reshape(-1), rows * K, 128, 4)
    eng = ROCmEngine()
    x16 = synth.x_f16(K, 86)
    act = Tensor((K, 1), Float16Storage.from_raw(x16, K))
    y = eng.matmul_w4a16(Tensor((rows, K), st), act).cpu().numpy()
    assert st._gpu_szr is not None
    assert rel_err(y.reshape(-1), orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128)) <= TOL
