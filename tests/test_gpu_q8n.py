"""GPU parity of Q8_0 with several fp32 activation columns on the three
entry points that take Q8_0 blocks (zt_gemm_q8_f32 on the raw 36-byte
blocks, zt_gemm_q8sep_f32 on the separated layout, zt_gemm_q8gguf_f32 on
the GGUF 34-byte blocks' upload layout): with N % 4 == 0 and 16-byte
aligned B they run rbf_kernel, the row-block MFMA GEMM (groups of 8 columns
for K <= 4096, else of 4), one launch per group; other N keep the
per-column kernel.

This is the reference's batched GemmQ8F32 contract (internal/gpuapi/
kernels.go:79-81; gemm_q8.cu:121-152 for N > 1; the CPU GemmF32Q8NT,
internal/xblas/gemm_quant.go:160-264) and GemmF32MmapNT for GGUF Q8_0.
Bars: max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle; within 1e-6
of the exact (fp64) product, also with activations spread over 2^+-20
inside one wave step; the same bits on a second call; the three layouts of
the same weights give the same bits (one kernel, the same products); rows
of C past M are never written.
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


class Q8Dev:
    """One Q8_0 matrix in the raw and separated layouts."""

    def __init__(self, lib, w):
        self.rows, self.K = w.rows, w.K
        nblk = w.rows * w.K // 32
        sep = np.empty(lib.zt_q8_gpu_bytes(nblk), np.uint8)
        lib.zt_q8_raw_to_gpu(w.raw.ctypes.data, nblk, sep.ctypes.data)
        self.raw, self.sep, self.off = dev(w.raw), dev(sep), lib.zt_q8_gpu_data_offset(nblk)


def gemm(lib, name, buf, off, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.full((rows * N + 8,), float("nan"), dtype=torch.float32, device="cuda")
    args = (buf.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N) + ((off,) if off is not None else ())
    lib.call(name, *args, stream())
    out = c.cpu().numpy()
    assert np.all(np.isnan(out[rows * N:]))
    return out[:rows * N].reshape(rows, N)


def both(lib, m, x, N):
    a = gemm(lib, "zt_gemm_q8_f32", m.raw, None, x, m.rows, m.K, N)
    b = gemm(lib, "zt_gemm_q8sep_f32", m.sep, m.off, x, m.rows, m.K, N)
    return a, b


def oracle(orc, w, x, N):
    return orc.gemm_f32_q8_nt(np.ascontiguousarray(x.T), w.raw, N, w.rows, w.K, threads=orc.nthreads()) \
        .reshape(N, w.rows).T


def exact64(orc, w, x):
    W = orc.q8_dequant(w.raw, w.rows * w.K).astype(np.float64).reshape(w.rows, w.K)
    return W @ np.asarray(x, np.float64)


@pytest.mark.parametrize("N", [4, 8])
@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (17, 544), (100, 4096), (65, 4128), (33, 8192), (9, 16384),
                                    (2049, 1024), (5, 20480), (7, 32768)])
def test_q8n_ragged_both_layouts(lib, orc, rows, K, N):
    """Partial row sets and workgroups, K not a multiple of a step (512),
    one, two and four steps a wave: the oracle's result on both layouts,
    the same bits on both and on a second call."""
    print(f"q8n rows={rows} K={K} N={N}", flush=True)
    w = synth.q8_0(rows, K, 111)
    x = synth.x_f32(K * N, 111 + N).reshape(K, N)
    m = Q8Dev(lib, w)
    a, b = both(lib, m, x, N)
    assert rel_err(a, oracle(orc, w, x, N)) <= TOL
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    assert np.array_equal(b.view(np.uint32), both(lib, m, x, N)[1].view(np.uint32))


@pytest.mark.parametrize("N", [4, 8])
@pytest.mark.parametrize("rows,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_q8n_llama3_8b_shapes(lib, orc, rows, K, N):
    print(f"q8n rows={rows} K={K} N={N}", flush=True)
    w = synth.q8_0(rows, K, synth.seed_for(2, 8 + rows % 5))
    x = synth.x_f32(K * N, 112 + N).reshape(K, N)
    m = Q8Dev(lib, w)
    a, b = both(lib, m, x, N)
    assert rel_err(b, oracle(orc, w, x, N)) <= TOL
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("N", [12, 16, 3, 6])
def test_q8n_column_groups(lib, orc, N):
    """8 + 4 and 8 + 8 columns on the MFMA path; 3 and 6 columns on the
    per-column kernel."""
    rows, K = 300, 2048
    print(f"q8n groups N={N}", flush=True)
    w = synth.q8_0(rows, K, 113)
    x = synth.x_f32(K * N, 113 + N).reshape(K, N)
    m = Q8Dev(lib, w)
    a, b = both(lib, m, x, N)
    ref = oracle(orc, w, x, N)
    assert rel_err(a, ref) <= TOL and rel_err(b, ref) <= TOL


@pytest.mark.parametrize("N", [4, 8])
def test_q8n_close_to_fp64_and_spread(lib, orc, N):
    """Against the exact product: ordinary activations at K = 16384 and
    4096, and activations of magnitudes 2^-20 .. 2^20 mixed inside every
    wave step: within 1e-6 per column (the reference's own fp32 products,
    q scale rounded before the multiply, differ from it by about 1e-7)."""
    for rows, K, spread in [(256, 16384, False), (512, 4096, False), (256, 4096, True)]:
        w = synth.q8_0(rows, K, 114)
        if spread:
            rng = np.random.default_rng(114)
            mag = np.exp2(rng.uniform(-20, 20, (K, N))).astype(np.float32)
            x = (mag * np.sign(rng.standard_normal((K, N)))).astype(np.float32)
        else:
            x = synth.x_f32(K * N, 114).reshape(K, N)
        m = Q8Dev(lib, w)
        c = both(lib, m, x, N)[1]
        ex = exact64(orc, w, x)
        for n in range(N):
            assert rel_err(c[:, n], ex[:, n]) <= 1e-6, (rows, K, spread, n)


@pytest.mark.parametrize("N", [4, 8])
@pytest.mark.parametrize("rows,K", [(4096, 4096), (65, 2080), (300, 14336)])
def test_q8n_gguf(lib, orc, rows, K, N):
    """GGUF Q8_0 (fp16 scales) batches against the reference CPU engine's
    GemmF32MmapNT on the same 34-byte blocks."""
    print(f"q8n gguf rows={rows} K={K} N={N}", flush=True)
    raw = synth.gguf_q8_0(rows, K, 115)
    nblk = rows * K // 32
    host = np.empty(lib.zt_q8gguf_gpu_bytes(nblk), np.uint8)
    lib.zt_q8gguf_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
    d = dev(host)
    x = synth.x_f32(K * N, 115).reshape(K, N)
    c = gemm(lib, "zt_gemm_q8gguf_f32", d, lib.zt_q8gguf_gpu_data_offset(nblk), x, rows, K, N)
    ref = orc.gemm_f32_mmap_nt(8, np.ascontiguousarray(x.T), raw, N, rows, K).reshape(N, rows).T
    assert rel_err(c, ref) <= TOL
