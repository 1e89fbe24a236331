"""GPU parity of the int4 and int8 A B GEMMs at batches 4-64 (N % 4 == 0,
K % 32 == 0, int4 group_size % 32 == 0), the shapes zt_gemm_int4_f32 and
zt_gemm_int8_f32 run on the row-block MFMA GEMM (up to 64 columns while
M N <= 2^19 for int4, 2^18 for int8), against the oracle's
restatement of the reference's kernels (internal/cuda/kernels/gemm_int4.cu:
29-69, gemm_int8.cu:16-40), through the C ABI.

The kernel splits each fp32 activation into fp16 hi and lo parts on a
per-step power-of-two scale, multiplies them by the exact fp16 encodings of
the unsigned nibble u = v + 8 (int4) or byte u = q + 128 (int8), and takes
the offset (8 + z, or 128) times the activation sum off once per 32-element
block.  Bars: max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle, and
per output |y - exact| / sum|w x| <= 1e-6 against the exact product (the
weights are exact in fp16 and hi + lo carries each activation to about
2^-22 of its step's largest value).  Shapes: one,
two and four K steps a wave (K up to 32768), 4- and 8-column launches,
rows not a multiple of a workgroup's, group sizes that are and are not
powers of two, zero points up to 255, and the rows past M and K past the
buffers' ends reading zeros.
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


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def say(msg: str) -> None:
    print(msg, flush=True)


def run_int4(lib, w, b, M, K, N, gs):
    c = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda")
    a, bd, s, z = dev(w.packed), dev(b), dev(w.scales), dev(w.zeros)
    lib.call("zt_gemm_int4_f32", a.data_ptr(), bd.data_ptr(), c.data_ptr(), s.data_ptr(), z.data_ptr(), M, K, N, gs,
             stream())
    return c.cpu().numpy()


def run_int8(lib, a, b, M, K, N):
    c = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda")
    ad, bd = dev(a), dev(b)
    lib.call("zt_gemm_int8_f32", ad.data_ptr(), bd.data_ptr(), c.data_ptr(), M, K, N, stream())
    return c.cpu().numpy()


INT4_CASES = [  # M, K, N, group_size
    (4096, 4096, 4, 128), (4096, 4096, 8, 128), (4096, 4096, 12, 32), (4096, 4096, 16, 128),
    (14336, 4096, 8, 128), (4096, 14336, 4, 128), (4096, 14336, 16, 64),
    # ragged rows; group sizes 96 (three blocks) and the whole row
    (333, 1024, 4, 96), (1001, 2016, 8, 96), (37, 4096, 12, 4096), (5, 64, 16, 32), (1, 32, 4, 32),
    # two and four steps a wave, K past 16384 and at 32768
    (515, 10240, 4, 128), (515, 10240, 8, 128), (259, 20480, 4, 64), (130, 32768, 4, 128), (130, 32768, 16, 256),
    # 20-64 columns while M N <= 2^19
    (4096, 4096, 64, 128), (1000, 2048, 36, 64), (8191, 1024, 60, 32),
    # 8 row sets at one step (4-column groups), 2 row sets at four steps on 10 waves
    (14336, 4096, 4, 32), (4096, 20480, 4, 128), (4096, 20480, 8, 64),
]


@pytest.mark.parametrize("M,K,N,gs", INT4_CASES)
def test_int4_rb(lib, orc, M, K, N, gs):
    say(f"int4 rb M={M} K={K} N={N} gs={gs}")
    w = synth.int4(M, K, gs, 700 + M + K + N, zero_max=15)
    b = synth.x_f32(K * N, 701 + N).reshape(K, N)
    y = run_int4(lib, w, b, M, K, N, gs)
    assert rel_err(y, orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, N, gs)) <= TOL


INT8_CASES = [  # M, K, N
    (4096, 4096, 4), (4096, 4096, 8), (4096, 4096, 12), (4096, 4096, 16), (14336, 4096, 8), (4096, 14336, 4),
    (4096, 14336, 16), (333, 1024, 4), (1001, 2016, 8), (5, 64, 16), (1, 32, 4), (515, 10240, 8), (259, 20480, 4),
    (130, 32768, 4), (130, 32768, 8),
    # 20-64 columns while M N <= 2^18
    (4096, 4096, 64), (1000, 2048, 36), (2047, 1024, 60),
    # 4 row sets at one step, 2 at two and four steps
    (14336, 4096, 4), (4096, 12288, 4), (4096, 20480, 4),
]


@pytest.mark.parametrize("M,K,N", INT8_CASES)
def test_int8_rb(lib, orc, M, K, N):
    say(f"int8 rb M={M} K={K} N={N}")
    a = synth.int8(M, K, 710 + M + K)
    b = synth.x_f32(K * N, 711 + N).reshape(K, N)
    y = run_int8(lib, a, b, M, K, N)
    assert rel_err(y, orc.gemm_int8_f32(a, b, M, K, N)) <= TOL


@pytest.mark.parametrize("zmax", [0, 15, 255])
@pytest.mark.parametrize("N", [4, 8])
def test_int4_rb_per_element_error(lib, orc, zmax, N):
    """Each output against the exact product, relative to its own sum of
    |w x|, beside the same measure of the reference's fp32 loop (the
    oracle).  The offset (8 + z) sum(x) comes off once per 32-element block,
    so zero points up to 255 test the cancellation it carries."""
    M, K, gs = 512, 4096, 128
    w = synth.int4(M, K, gs, 720 + zmax, zero_max=zmax)
    b = synth.x_f32(K * N, 721).reshape(K, N)
    y = run_int4(lib, w, b, M, K, N, gs).reshape(M, N).astype(np.float64)
    W = synth.int4_dense(w, gs).astype(np.float64).reshape(M, K)
    exact = W @ b.astype(np.float64)
    mag = np.abs(W) @ np.abs(b.astype(np.float64))
    ref = np.asarray(orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, N, gs), np.float64).reshape(M, N)
    ours = float(np.max(np.abs(y - exact) / mag))
    theirs = float(np.max(np.abs(ref - exact) / mag))
    say(f"int4 rb N={N} zmax={zmax}: per-element |y - exact| / sum|w x|: {ours:.3e} (reference loop {theirs:.3e})")
    assert ours <= 1e-6 and ours <= 4 * theirs


def test_int8_rb_per_element_error(lib, orc):
    M, K, N = 512, 4096, 8
    a = synth.int8(M, K, 730)
    b = synth.x_f32(K * N, 731).reshape(K, N)
    y = run_int8(lib, a, b, M, K, N).reshape(M, N).astype(np.float64)
    A = a.astype(np.float64).reshape(M, K)
    exact = A @ b.astype(np.float64)
    mag = np.abs(A) @ np.abs(b.astype(np.float64))
    ours = float(np.max(np.abs(y - exact) / mag))
    say(f"int8 rb per-element |y - exact| / sum|w x|: {ours:.3e}")
    assert ours <= 1e-6


def test_int4_rb_scale_spread_and_zero_activations(lib, orc):
    """Activations spanning 2^-60 .. 2^60 across K steps and all-zero steps:
    the per-step power-of-two normalisation keeps each step's hi/lo split
    exact to about 2^-22 of that step's largest value."""
    M, K, N, gs = 257, 8192, 8, 64
    w = synth.int4(M, K, gs, 740, zero_max=15)
    b = synth.x_f32(K * N, 741).reshape(K, N).astype(np.float64)
    step = np.arange(K) // 512
    b *= np.exp2(np.where(step % 4 == 3, -200.0, (step % 8 - 4) * 15.0))[:, None]
    b[step % 4 == 3] = 0.0
    b = b.astype(np.float32)
    y = run_int4(lib, w, b, M, K, N, gs).reshape(M, N).astype(np.float64)
    W = synth.int4_dense(w, gs).astype(np.float64).reshape(M, K)
    exact = W @ b.astype(np.float64)
    mag = np.abs(W) @ np.abs(b.astype(np.float64))
    assert float(np.max(np.abs(y - exact) / mag)) <= 1e-6


def test_int4_rb_repeat_bit_identical(lib):
    M, K, N, gs = 4096, 4096, 8, 128
    w = synth.int4(M, K, gs, 750, zero_max=15)
    b = synth.x_f32(K * N, 751).reshape(K, N)
    y0 = run_int4(lib, w, b, M, K, N, gs)
    y1 = run_int4(lib, w, b, M, K, N, gs)
    assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
