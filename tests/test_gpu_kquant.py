"""GPU parity of the K-quant (Q4_K, Q5_K, Q6_K) and Q5_0 entry points against
the CPU oracle, through the C ABI and the engine.

Bars: dequantizers bit-exact (uint32 view equality); GEMVs
max|y - y_ref| / max|y_ref| <= 1e-5 with fp32 accumulation, y_ref = the
reference CPU engine's GemmF32Q4KNT / Q5KNT / Q6KNT and its Q5_0 B-side
matmul as restated by the oracle.  Shapes: the Llama-3-8B decode layers,
plus ragged cases (one super-block, partial wave steps, odd super-block
counts that leave Q6_K blocks 2-byte aligned, a 2-byte offset base).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402
from ztensor_amd.storage import Q4KStorage, Q5_0Storage, Q6KStorage, Tensor  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5  # every product exact in fp32: only the summation order differs
KQ = ["q4_k", "q5_k", "q6_k"]
LLAMA8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]
RAGGED = [(1, 256), (17, 768), (65, 2560), (5, 6912), (130, 1792)]
# the reference's own GEMV test shapes (internal/cuda/kernels/gemv_q4k_test.go:363-368,
# gemv_q5k_test.go:374-379, gemv_q6k_test.go:329-334; Q5_0: gemv_q5_0_test.go:260-265)
REF_KQ = [(32, 256), (64, 512), (256, 256), (128, 1024), (1024, 256), (512, 2048)]
REF_Q5_0 = [(32, 32), (64, 128), (128, 128), (128, 1024), (1024, 32), (512, 2048)]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return _lib.load()


def dev(a: np.ndarray, pad: int = 0) -> "torch.Tensor":
    b = np.ascontiguousarray(a).view(np.uint8).reshape(-1)
    t = torch.zeros(b.size + pad, dtype=torch.uint8)
    t[pad:] = torch.from_numpy(b.copy())
    return t.cuda()


def devf(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def say(msg: str) -> None:
    print(msg, flush=True)


def kq_gemv(lib, fmt, w_dev_ptr, x, rows, K):
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = devf(x)
    lib.call(f"zt_gemv_{fmt.replace('_', '')}_f32", w_dev_ptr, xd.data_ptr(), y.data_ptr(), rows, K, stream())
    torch.cuda.synchronize()
    return y.cpu().numpy()


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("rows,K", [(1, 256), (3, 768), (64, 4096), (7, 6912)])
def test_kquant_dequant_bit_exact(lib, orc, fmt, rows, K):
    say(f"dequant {fmt} {rows}x{K}")
    w = synth.kquant(fmt, rows, K, synth.seed_for(6, rows % 16))
    d = dev(w.raw)
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call(f"zt_dequant_{fmt.replace('_', '')}_f32", d.data_ptr(), out.data_ptr(), rows, K, stream())
    torch.cuda.synchronize()
    want = orc.kq_dequant(fmt, w.raw, rows * K)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", KQ)
@pytest.mark.parametrize("rows,K", LLAMA8B + RAGGED + REF_KQ)
def test_kquant_gemv_matches_oracle(lib, orc, fmt, rows, K):
    say(f"gemv {fmt} {rows}x{K}")
    w = synth.kquant(fmt, rows, K, synth.seed_for(6, K % 16))
    x = synth.x_f32(K, synth.seed_for(6, K % 16))
    d = dev(w.raw)
    y = kq_gemv(lib, fmt, d.data_ptr(), x, rows, K)
    ref = orc.gemm_f32_kq_nt(fmt, x, w.raw, 1, rows, K, threads=orc.nthreads())
    err = rel_err(y, ref)
    say(f"  rel err {err:.2e}")
    assert err <= TOL


def test_q6k_gemv_on_a_2_byte_aligned_base(lib, orc):
    # Q6_K super-blocks are 210 bytes: a weight slice can start at any even
    # address, which the kernel's aligned-dword reads must handle.
    rows, K = 33, 2560
    w = synth.kquant("q6_k", rows, K, 77)
    x = synth.x_f32(K, 77)
    d = dev(w.raw, pad=2)
    y = kq_gemv(lib, "q6_k", d.data_ptr() + 2, x, rows, K)
    assert rel_err(y, orc.gemm_f32_kq_nt("q6_k", x, w.raw, 1, rows, K)) <= TOL
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_q6k_f32", d.data_ptr() + 2, out.data_ptr(), rows, K, stream())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.kq_dequant("q6_k", w.raw, rows * K).view(np.uint32))


def q6k_split_dev(lib, raw, rows, K, off=0):
    """The split copy of raw Q6_K super-blocks (uploaded at byte offset off)."""
    d = dev(raw, pad=off)
    out = torch.empty(lib.zt_q6k_split_bytes(rows, K), dtype=torch.uint8, device="cuda")
    assert lib.call("zt_q6k_split", d.data_ptr() + off, rows, K, out.data_ptr(), stream()) is None
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("rows,K,off", [(1, 256, 0), (17, 768, 2), (33, 2560, 0)])
def test_q6k_split_layout_bytes(lib, rows, K, off):
    """ql, qh, scales and d of every super-block regrouped into four arrays,
    checked against a numpy regrouping of the raw 210-byte blocks."""
    say(f"q6k split layout {rows}x{K} off {off}")
    w = synth.kquant("q6_k", rows, K, 91)
    raw = np.frombuffer(w.raw, np.uint8).reshape(-1, 210)
    want = np.concatenate([raw[:, :128].reshape(-1), raw[:, 128:192].reshape(-1), raw[:, 192:208].reshape(-1),
                           raw[:, 208:210].reshape(-1)])
    assert lib.zt_q6k_split_bytes(rows, K) == raw.size
    got = q6k_split_dev(lib, w.raw, rows, K, off).cpu().numpy()
    assert np.array_equal(got, want)


@pytest.mark.parametrize("rows,K", LLAMA8B + RAGGED + REF_KQ + [(9, 16640), (300, 28672)])
def test_q6k_split_gemv_matches_oracle(lib, orc, rows, K):
    """zt_gemv_q6ks_f32 on the split layout against GemmF32Q6KNT, at the
    Llama-3-8B shapes, ragged ones and K past one step of 16 waves."""
    say(f"q6ks gemv {rows}x{K}")
    w = synth.kquant("q6_k", rows, K, synth.seed_for(6, K % 16))
    x = synth.x_f32(K, synth.seed_for(6, K % 16))
    ws = q6k_split_dev(lib, w.raw, rows, K)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = devf(x)
    lib.call("zt_gemv_q6ks_f32", ws.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, stream())
    torch.cuda.synchronize()
    err = rel_err(y.cpu().numpy(), orc.gemm_f32_kq_nt("q6_k", x, w.raw, 1, rows, K, threads=orc.nthreads()))
    say(f"  rel err {err:.2e}")
    assert err <= TOL


def test_q6k_split_invalid_arguments(lib):
    t = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    assert lib.zt_q6k_split_bytes(4, 100) == -1
    assert lib.zt_q6k_split(p, 4, 100, p, stream()) == 1     # K % 256
    assert lib.zt_q6k_split(p + 1, 1, 256, p, stream()) == 1  # raw alignment
    assert lib.zt_q6k_split(p, 1, 256, p + 8, stream()) == 1  # split alignment
    assert lib.zt_gemv_q6ks_f32(p, p, p, 4, 100, stream()) == 1
    assert lib.zt_gemv_q6ks_f32(p + 8, p, p, 1, 256, stream()) == 1  # W alignment
    assert lib.zt_gemv_q6ks_f32(p, p + 4, p, 1, 256, stream()) == 1  # x alignment
    assert lib.zt_gemv_q6ks_f32(p, p, p, 1 << 20, 4096, stream()) == 1  # 210 T >= 2^31


@pytest.mark.parametrize("fmt,K,off", [("q4_k", 768, 0), ("q5_k", 4352, 0), ("q6_k", 768, 0), ("q6_k", 768, 2),
                                        ("q6_k", 4352, 2), ("q6_k", 4096, 2)])
def test_kquant_fixed_step_kernel_odd_superblocks_and_offset_base(lib, orc, fmt, K, off):
    """2048-row matrices (the Q4_K / Q5_K fixed-step kernel; the Q6_K loop
    kernel): an odd number of super-blocks per row (3; 17 with a partial
    last wave), and for Q6_K a base 2 bytes past a 4-byte boundary, so
    blocks alternate between both misalignments."""
    rows = 2048
    say(f"{fmt} steps rows={rows} K={K} off={off}")
    w = synth.kquant(fmt, rows, K, 78)
    x = synth.x_f32(K, 78)
    d = dev(w.raw, pad=off)
    y = kq_gemv(lib, fmt, d.data_ptr() + off, x, rows, K)
    assert rel_err(y, orc.gemm_f32_kq_nt(fmt, x, w.raw, 1, rows, K, threads=orc.nthreads())) <= TOL


@pytest.mark.parametrize("fmt", KQ)
def test_kquant_zero_superblocks_give_zero(lib, fmt):
    nbytes = {"q4_k": 144, "q5_k": 176, "q6_k": 210}[fmt]
    d = dev(np.zeros(8 * 2 * nbytes, np.uint8))
    y = kq_gemv(lib, fmt, d.data_ptr(), synth.x_f32(512, 3), 8, 512)
    assert np.all(y == 0)


@pytest.mark.parametrize("fmt", KQ)
def test_kquant_invalid_arguments_rejected(lib, fmt):
    name = f"zt_gemv_{fmt.replace('_', '')}_f32"
    fn = getattr(lib, name)
    w = dev(np.zeros(4096, np.uint8))
    x = devf(np.zeros(512, np.float32))
    y = torch.empty(8, dtype=torch.float32, device="cuda")
    assert fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), 8, 300, stream()) == _lib.HIP_ERROR_INVALID_VALUE  # K % 256
    assert fn(0, x.data_ptr(), y.data_ptr(), 8, 256, stream()) == _lib.HIP_ERROR_INVALID_VALUE
    assert fn(w.data_ptr(), x.data_ptr() + 4, y.data_ptr(), 8, 256, stream()) == _lib.HIP_ERROR_INVALID_VALUE
    assert fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), 0, 256, stream()) == 0
    assert fn(w.data_ptr(), x.data_ptr(), y.data_ptr(), -1, 256, stream()) == _lib.HIP_ERROR_INVALID_VALUE
    deq = getattr(lib, f"zt_dequant_{fmt.replace('_', '')}_f32")
    assert deq(w.data_ptr(), y.data_ptr(), 1, 100, stream()) == _lib.HIP_ERROR_INVALID_VALUE


# ------------------------------------------------------------------ Q5_0


def q5_0_dev(lib, w):
    nblk = w.rows * w.K // 32
    host = np.empty(lib.zt_q5_0_gpu_bytes(nblk), np.uint8)
    lib.zt_q5_0_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    return dev(host), lib.zt_q5_0_gpu_qh_offset(nblk), lib.zt_q5_0_gpu_qs_offset(nblk)


@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (64, 4096)])
def test_q5_0_dequant_bit_exact(lib, orc, rows, K):
    w = synth.kquant("q5_0", rows, K, synth.seed_for(7, rows % 16))
    d = dev(w.raw)
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_q5_0_f32", d.data_ptr(), out.data_ptr(), rows, K, stream())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.q5_0_dequant(w.raw, rows * K).view(np.uint32))


@pytest.mark.parametrize("rows,K", LLAMA8B + [(1, 32), (3, 96), (17, 4128), (65, 2080)] + REF_Q5_0)
def test_q5_0_gemv_matches_oracle(lib, orc, rows, K):
    say(f"gemv q5_0 {rows}x{K}")
    w = synth.kquant("q5_0", rows, K, synth.seed_for(7, K % 16))
    x = synth.x_f32(K, synth.seed_for(7, K % 16))
    d, qh, qs = q5_0_dev(lib, w)
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = devf(x)
    lib.call("zt_gemv_q5_0_f32", d.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, qh, qs, stream())
    torch.cuda.synchronize()
    ref = orc.gemm_f32_q5_0_nt(x, w.raw, 1, rows, K)
    err = rel_err(y.cpu().numpy(), ref)
    say(f"  rel err {err:.2e}")
    assert err <= TOL


def test_q5_0_invalid_arguments_rejected(lib):
    w = dev(np.zeros(4096, np.uint8))
    x = devf(np.zeros(64, np.float32))
    y = torch.empty(4, dtype=torch.float32, device="cuda")
    f = lib.zt_gemv_q5_0_f32
    assert f(w.data_ptr(), x.data_ptr(), y.data_ptr(), 4, 40, 16, 32, stream()) == _lib.HIP_ERROR_INVALID_VALUE
    assert f(w.data_ptr(), x.data_ptr(), y.data_ptr(), 4, 64, 16, 40, stream()) == _lib.HIP_ERROR_INVALID_VALUE
    assert f(w.data_ptr(), x.data_ptr(), y.data_ptr(), 0, 64, 16, 32, stream()) == 0


# ------------------------------------------------------------------ engine


@pytest.mark.parametrize("n", [1, 3])
def test_engine_q4k_both_operand_sides(orc, n):
    from ztensor_amd.engine import ROCmEngine

    eng = ROCmEngine()
    rows, K = 96, 1024
    w = synth.kquant("q4_k", rows, K, 88)
    x = synth.x_f32(K * n, 88).reshape(K, n)
    W = orc.kq_dequant("q4_k", w.raw, rows * K).reshape(rows, K).astype(np.float64)
    # A side: W [rows, K] @ x [K, n]
    a = Tensor((rows, K), Q4KStorage.from_raw(w.raw, rows * K))
    got = eng.matmul(a, devf(x)).cpu().numpy()
    assert rel_err(got, W @ x.astype(np.float64)) <= TOL
    # B side: act [n, K] @ W^T (virtually transposed weight, logical [K, rows])
    b = Tensor((K, rows), Q4KStorage.from_raw(w.raw, rows * K))
    got = eng.matmul(devf(x.T.copy()), b).cpu().numpy()
    assert rel_err(got, x.T.astype(np.float64) @ W.T) <= TOL


def test_engine_q6k_and_q5_0(orc):
    from ztensor_amd.engine import ROCmEngine

    eng = ROCmEngine()
    rows, K = 40, 768
    w6 = synth.kquant("q6_k", rows, K, 89)
    x = synth.x_f32(K, 89)
    got = eng.matmul(Tensor((rows, K), Q6KStorage.from_raw(w6.raw, rows * K)), devf(x)).cpu().numpy()
    assert rel_err(got.reshape(-1), orc.gemm_f32_kq_nt("q6_k", x, w6.raw, 1, rows, K)) <= TOL
    w5 = synth.kquant("q5_0", rows, K, 90)
    x2 = synth.x_f32(2 * K, 90).reshape(K, 2)
    got = eng.matmul(Tensor((rows, K), Q5_0Storage.from_raw(w5.raw, rows * K)), devf(x2)).cpu().numpy()
    W5 = orc.q5_0_dequant(w5.raw, rows * K).reshape(rows, K).astype(np.float64)
    assert rel_err(got, W5 @ x2.astype(np.float64)) <= TOL


def test_engine_q6k_batch1_split_copy(orc):
    """Q6_K batch 1 through the engine runs on the split copy: built once on
    the first call, reused on the next, dropped when the storage is uploaded
    again (then rebuilt from the new buffer)."""
    from ztensor_amd.engine import ROCmEngine

    eng = ROCmEngine()
    rows, K = 96, 2048
    w = synth.kquant("q6_k", rows, K, 93)
    st = Q6KStorage.from_raw(w.raw, rows * K)
    x = synth.x_f32(K, 93)
    ref = orc.gemm_f32_kq_nt("q6_k", x, w.raw, 1, rows, K)
    t = Tensor((rows, K), st)
    assert rel_err(eng.matmul(t, devf(x)).cpu().numpy().reshape(-1), ref) <= TOL
    first = st._gpu_split[1]
    assert first.numel() == rows * (K // 256) * 210
    assert rel_err(eng.matmul(t, devf(x)).cpu().numpy().reshape(-1), ref) <= TOL
    assert st._gpu_split[1] is first
    st.set_gpu_ptr(None)
    assert st._gpu_split is None
    eng.upload_weights([st])
    assert rel_err(eng.matmul(t, devf(x)).cpu().numpy().reshape(-1), ref) <= TOL
    assert st._gpu_split is not None and st._gpu_split[1] is not first


@pytest.mark.parametrize("opts", [dict(q6k_split=False), dict(split_reserve_bytes=1 << 62)])
def test_engine_q6k_split_opt_out(orc, opts):
    """With q6k_split=False, or when the copy would leave less than the
    reserve free, Q6_K batch 1 reads the raw super-blocks: no split copy is
    built and the result is the raw-layout GEMV's, bit for bit."""
    from ztensor_amd import _lib
    from ztensor_amd.engine import ROCmEngine

    eng = ROCmEngine(**opts)
    rows, K = 96, 2048
    w = synth.kquant("q6_k", rows, K, 94)
    st = Q6KStorage.from_raw(w.raw, rows * K)
    x = synth.x_f32(K, 94)
    got = eng.matmul(Tensor((rows, K), st), devf(x)).cpu().numpy().reshape(-1)
    assert getattr(st, "_gpu_split", None) is None
    assert rel_err(got, orc.gemm_f32_kq_nt("q6_k", x, w.raw, 1, rows, K)) <= TOL
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = devf(x)
    _lib.load().call("zt_gemv_q6k_f32", st.gpu_ptr().tensor.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K,
                     torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(got.view(np.uint32), y.cpu().numpy().view(np.uint32))


# ------------------------------------------------------------------ GGUF mmap


def q8gguf_dev(lib, raw, nblk):
    host = np.empty(lib.zt_q8gguf_gpu_bytes(nblk), np.uint8)
    lib.zt_q8gguf_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
    return dev(host), lib.zt_q8gguf_gpu_data_offset(nblk)


@pytest.mark.parametrize("rows,K", [(1, 32), (5, 96), (64, 4096)])
def test_gguf_q8_0_dequant_bit_exact(lib, orc, rows, K):
    raw = synth.gguf_q8_0(rows, K, 91)
    nblk = rows * K // 32
    d, off = q8gguf_dev(lib, raw, nblk)
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_q8gguf_f32", d.data_ptr(), out.data_ptr(), rows * K, off, stream())
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), orc.gguf_q8_0_dequant(raw, rows * K).view(np.uint32))


@pytest.mark.parametrize("N", [1, 3])
@pytest.mark.parametrize("rows,K", LLAMA8B + [(3, 32), (65, 2080)])
def test_gguf_q8_0_gemm_matches_oracle(lib, orc, rows, K, N):
    say(f"gguf q8_0 {rows}x{K} N={N}")
    raw = synth.gguf_q8_0(rows, K, 92)
    d, off = q8gguf_dev(lib, raw, rows * K // 32)
    x = synth.x_f32(K * N, 92)
    xd = devf(x)
    y = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q8gguf_f32", d.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, N, off, stream())
    torch.cuda.synchronize()
    # reference CPU engine on the same weights: GemmF32MmapNT with A = x^T [N, K]
    ref = orc.gemm_f32_mmap_nt(8, x.reshape(K, N).T.copy(), raw, N, rows, K).reshape(N, rows).T
    err = rel_err(y.cpu().numpy().reshape(rows, N), ref)
    say(f"  rel err {err:.2e}")
    assert err <= TOL


@pytest.mark.parametrize("qtype", [2, 6, 8, 12, 13, 14])
def test_engine_mmap_dispatch_by_ggml_type(orc, qtype):
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import GGMLType, MmapStorage

    eng = ROCmEngine()
    rows, K = 48, 1024
    raw = {2: lambda: synth.q4_0(rows, K, 93).raw, 6: lambda: synth.kquant("q5_0", rows, K, 93).raw,
           8: lambda: synth.gguf_q8_0(rows, K, 93), 12: lambda: synth.kquant("q4_k", rows, K, 93).raw,
           13: lambda: synth.kquant("q5_k", rows, K, 93).raw, 14: lambda: synth.kquant("q6_k", rows, K, 93).raw}[qtype]()
    for n in (1, 2, 8):  # 8: every type here on the tiled MFMA kernels
        x = synth.x_f32(K * n, 93 + n)
        ref = orc.gemm_f32_mmap_nt(qtype, x.reshape(K, n).T.copy(), raw, n, rows, K)  # [n, rows]
        # B side (virtually transposed weight): act [n, K] @ W^T
        b = Tensor((K, rows), MmapStorage(raw, rows * K, GGMLType(qtype)))
        got = eng.matmul(devf(x.reshape(K, n).T.copy()), b).cpu().numpy()
        assert rel_err(got.reshape(n, rows), ref.reshape(n, rows)) <= TOL
        # A side: W [rows, K] @ x [K, n]
        a = Tensor((rows, K), MmapStorage(raw, rows * K, GGMLType(qtype)))
        got = eng.matmul(a, devf(x.reshape(K, n))).cpu().numpy()
        assert rel_err(got.reshape(rows, n), ref.reshape(n, rows).T) <= TOL
