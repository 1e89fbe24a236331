"""GPU parity of Q4_0 and Q8_0 with many fp32 activation columns (prefill
widths) on the reference's own batched entry points: zt_gemm_q4_f32,
zt_gemm_q8_f32 (raw 36-byte blocks), zt_gemm_q8sep_f32 and
zt_gemm_q8gguf_f32 with even N from 128 (Q8_0 also from 32 at 8192 rows
and more, from 64 past K = 8192; narrower batches take the row-block
GEMM, also checked here) run the bf16 MFMA tile GEMM
(bf16_gemm_kernel): each fp32 activation as three exact bf16 parts, each
block value as an exact bf16 (Q4_0 as 128 + u with the offset 136 taken off
through an all-ones product, Q8_0 as q), and each 32-element block's sums
times the block's scale.

The reference's contract is GemmQ4F32 / GemmQ8F32 with n > 1
(internal/gpuapi/kernels.go:45-48, 79-81; the CPU GemmF32Q4NT /
GemmF32Q8NT, internal/xblas/gemm_quant.go:81-264), which the oracle
restates.  Bars: max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle;
per output |y - exact| / sum|w x| <= 1e-6 against the fp64 product of the
dequantized weights; the same bits on a second call; rows of C past M never
written.  Shapes: partial 32-, 64- and 128-row tiles and column tiles,
N = 32 .. 512 and N = 2 mod 4, K from 32 to 14336, B 8-byte but not 16-byte
aligned.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return _lib.load()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def run(lib, name, buf, off, x, rows, K, N, xoff=0):
    """C = W x through `name`; x [K, N] float32 placed `xoff` floats into its
    buffer; C carries 8 guard floats past the end."""
    xb = torch.zeros(K * N + xoff, dtype=torch.float32, device="cuda")
    xb[xoff:] = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.full((rows * N + 8,), float("nan"), dtype=torch.float32, device="cuda")
    args = (buf.data_ptr(), xb.data_ptr() + 4 * xoff, c.data_ptr(), rows, K, N) + ((off,) if off is not None else ())
    lib.call(name, *args, stream())
    out = c.cpu().numpy()
    assert np.all(np.isnan(out[rows * N:]))
    return out[:rows * N].reshape(rows, N)


def q4_dev(lib, w):
    nblk = w.rows * w.K // 32
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    return torch.from_numpy(host).cuda(), lib.zt_q4_gpu_data_offset(nblk)


def q8_devs(lib, w):
    nblk = w.rows * w.K // 32
    sep = np.empty(lib.zt_q8_gpu_bytes(nblk), np.uint8)
    lib.zt_q8_raw_to_gpu(w.raw.ctypes.data, nblk, sep.ctypes.data)
    return dev(w.raw), dev(sep), lib.zt_q8_gpu_data_offset(nblk)


def per_element(y, W, x) -> float:
    exact = W @ x.astype(np.float64)
    mag = np.abs(W) @ np.abs(x.astype(np.float64))
    return float(np.max(np.abs(np.asarray(y, np.float64) - exact) / np.maximum(mag, 1e-300)))


SHAPES = [  # rows, K, N
    (1, 32, 32), (100, 4096, 32), (333, 4128, 34), (4099, 1024, 64), (65, 14336, 128), (1000, 2048, 130),
    (4096, 4096, 256), (1024, 4096, 512), (257, 512, 1030),
    # Q8_0's tile GEMM from 32 columns at 8192 rows, from 64 past K = 8192
    (8195, 1024, 32), (300, 9216, 64),
]


@pytest.mark.parametrize("rows,K,N", SHAPES)
def test_q4_0_wide(lib, orc, rows, K, N):
    print(f"q4_0 wide rows={rows} K={K} N={N}", flush=True)
    w = synth.q4_0(rows, K, 900 + rows + N)
    x = synth.x_f32(K * N, 901 + N).reshape(K, N)
    a, off = q4_dev(lib, w)
    y = run(lib, "zt_gemm_q4_f32", a, off, x, rows, K, N)
    ref = orc.gemm_f32_q4_nt(np.ascontiguousarray(x.T), w.raw, N, rows, K, threads=orc.nthreads())
    assert rel_err(y, np.asarray(ref).reshape(N, rows).T) <= TOL


@pytest.mark.parametrize("rows,K,N", SHAPES)
def test_q8_0_wide(lib, orc, rows, K, N):
    print(f"q8_0 wide rows={rows} K={K} N={N}", flush=True)
    w = synth.q8_0(rows, K, 910 + rows + N)
    x = synth.x_f32(K * N, 911 + N).reshape(K, N)
    raw, sep, off = q8_devs(lib, w)
    ref = np.asarray(orc.gemm_f32_q8_nt(np.ascontiguousarray(x.T), w.raw, N, rows, K, threads=orc.nthreads()))
    ref = ref.reshape(N, rows).T
    assert rel_err(run(lib, "zt_gemm_q8_f32", raw, None, x, rows, K, N), ref) <= TOL
    assert rel_err(run(lib, "zt_gemm_q8sep_f32", sep, off, x, rows, K, N), ref) <= TOL


@pytest.mark.parametrize("rows,K,N", [(333, 4128, 34), (1000, 2048, 130), (64, 4096, 256)])
def test_q8_0_gguf_wide(lib, orc, rows, K, N):
    """GGUF Q8_0 (fp16 scales) after its upload repack."""
    raw = synth.gguf_q8_0(rows, K, 920 + rows)
    nblk = rows * K // 32
    host = np.empty(lib.zt_q8gguf_gpu_bytes(nblk), np.uint8)
    lib.zt_q8gguf_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
    d = torch.from_numpy(host).cuda()
    x = synth.x_f32(K * N, 921).reshape(K, N)
    y = run(lib, "zt_gemm_q8gguf_f32", d, lib.zt_q8gguf_gpu_data_offset(nblk), x, rows, K, N)
    ref = orc.gemm_f32_mmap_nt(8, np.ascontiguousarray(x.T), raw, N, rows, K).reshape(N, rows).T
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("N", [64, 256])
def test_wide_per_element_error_and_alignment(lib, orc, N):
    """Each output against the exact product, relative to its own sum of
    |w x|; B placed 2 floats (8 bytes) off a 16-byte boundary."""
    rows, K = 512, 2048
    w4 = synth.q4_0(rows, K, 930)
    w8 = synth.q8_0(rows, K, 931)
    x = synth.x_f32(K * N, 932).reshape(K, N)
    a, off = q4_dev(lib, w4)
    y4 = run(lib, "zt_gemm_q4_f32", a, off, x, rows, K, N, xoff=2)
    W4 = orc.q4_dequant(w4.raw, rows * K).astype(np.float64).reshape(rows, K)
    raw, sep, off8 = q8_devs(lib, w8)
    y8 = run(lib, "zt_gemm_q8_f32", raw, None, x, rows, K, N, xoff=2)
    W8 = orc.q8_dequant(w8.raw, rows * K).astype(np.float64).reshape(rows, K)
    e4, e8 = per_element(y4, W4, x), per_element(y8, W8, x)
    print(f"wide N={N}: per-element |y - exact| / sum|w x|: Q4_0 {e4:.3e}, Q8_0 {e8:.3e}", flush=True)
    assert e4 <= 1e-6 and e8 <= 1e-6


def test_wide_repeat_bit_identical(lib):
    rows, K, N = 4096, 4096, 128
    w = synth.q4_0(rows, K, 940)
    x = synth.x_f32(K * N, 941).reshape(K, N)
    a, off = q4_dev(lib, w)
    y0 = run(lib, "zt_gemm_q4_f32", a, off, x, rows, K, N)
    y1 = run(lib, "zt_gemm_q4_f32", a, off, x, rows, K, N)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q4", "q4_f16", "q8"])
def test_engine_wide_batch_direct(lib, orc, fmt):
    """ROCmEngine sends a 256-column batch to the entry point's tile GEMM:
    no tiled copy, no 16-column chunks, the reference CPU product."""
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Q4Storage, Q8Storage, Tensor

    rows, K, n = 600, 2048, 256
    eng = ROCmEngine()
    x = synth.x_f32(K * n, 950).reshape(K, n)
    if fmt == "q8":
        w = synth.q8_0(rows, K, 951)
        q = w.raw.reshape(-1, 36)
        s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), rows * K)
        ref = orc.gemm_f32_q8_nt(np.ascontiguousarray(x.T), w.raw, n, rows, K, threads=orc.nthreads())
        xd = torch.from_numpy(x).cuda()
    else:
        w = synth.q4_0(rows, K, 952)
        s = Q4Storage.from_raw(w.raw, rows * K)
        if fmt == "q4_f16":  # the reference widens fp16 activations to fp32 (tensor/fp16_storage.go:53-63)
            x = x.astype(np.float16).astype(np.float32)
        ref = orc.gemm_f32_q4_nt(np.ascontiguousarray(x.T), w.raw, n, rows, K, threads=orc.nthreads())
        xd = torch.from_numpy(x.astype(np.float16) if fmt == "q4_f16" else x).cuda()
    y = eng.matmul(Tensor((rows, K), s), xd).cpu().numpy()
    assert rel_err(y, np.asarray(ref).reshape(n, rows).T) <= TOL
    assert getattr(s, "_gpu_tiled", None) is None
