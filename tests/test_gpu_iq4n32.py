"""GPU parity of IQ4_NL with fp32 activations (zt_gemm_iq4nl_f32): batch 1
on the fixed-step GEMV for K <= 4096 (one or two steps a wave; 8197 rows
take two) and the loop GEMV beyond; with N % 4 == 0 and 16-byte aligned B,
the fp32-activation row-block MFMA GEMM (rbf_kernel, groups of 8 columns up
to K = 8192, else 4), one launch per group; other N one GEMV per column.

The reference's IQ4_NL matmul is its fp32 CPU engine: IQ4NLStorage's
Dequantize (tensor/iq4_storage.go:36-46) and then an fp32 GEMM
(tensor/tensor.go:216-219, compute/cpu_engine.go:1215-1245).  Bars:
max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle's dequantized
weights times x; within 1e-6 of the exact (fp64) product per column, also
with activations spread over 2^+-20 inside one wave step (activations and
codebook both enter the MFMAs as fp16 hi + lo parts, each within about
2^-22 of its fp32 value); the same bits on a second call; rows of C past M
never written.
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


def upload(lib, w):
    nblk = w.rows * w.K // 32
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_iq4nl_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    return torch.from_numpy(host).cuda(), lib.zt_q4_gpu_data_offset(nblk)


def gemm(lib, a, off, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.full((rows * N + 8,), float("nan"), dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_iq4nl_f32", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, off, stream())
    out = c.cpu().numpy()
    assert np.all(np.isnan(out[rows * N:]))
    return out[:rows * N].reshape(rows, N)


def dense(orc, w):
    """The reference's dequantized fp32 weights, as float64."""
    return orc.iq4nl_dequant(w.raw, w.rows * w.K).astype(np.float64).reshape(w.rows, w.K)


def reference(orc, w, x):
    """Dequantize, then an fp32 GEMM (the reference CPU engine's path)."""
    W = orc.iq4nl_dequant(w.raw, w.rows * w.K).reshape(w.rows, w.K)
    return (W @ np.asarray(x, np.float32)).astype(np.float32)


@pytest.mark.parametrize("N", [1, 4, 8])
@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (17, 544), (100, 3584), (65, 4128), (33, 8192), (9, 16384),
                                    (2049, 1024), (5, 20480), (3301, 17024)])
def test_iq4n32_ragged(lib, orc, rows, K, N):
    """Partial row sets and workgroups, K not a multiple of a step (512),
    one, two and four steps a wave (3301 x 17024: four row sets at four
    steps, 9 waves, a partial last workgroup): the reference's result and
    the same bits on a second call."""
    print(f"iq4n32 rows={rows} K={K} N={N}", flush=True)
    w = synth.iq4nl(rows, K, 131)
    x = synth.x_f32(K * N, 131 + N).reshape(K, N)
    a, off = upload(lib, w)
    c = gemm(lib, a, off, x, rows, K, N)
    assert rel_err(c, reference(orc, w, x)) <= TOL
    assert np.array_equal(c.view(np.uint32), gemm(lib, a, off, x, rows, K, N).view(np.uint32))


@pytest.mark.parametrize("N", [1, 4, 8])
@pytest.mark.parametrize("rows,K", [(3584, 3584), (18944, 3584), (3584, 18944), (8197, 4096)])
def test_iq4n32_qwen2_shapes(lib, orc, rows, K, N):
    print(f"iq4n32 rows={rows} K={K} N={N}", flush=True)
    w = synth.iq4nl(rows, K, synth.seed_for(5, rows % 7))
    x = synth.x_f32(K * N, 132 + N).reshape(K, N)
    a, off = upload(lib, w)
    assert rel_err(gemm(lib, a, off, x, rows, K, N), reference(orc, w, x)) <= TOL


@pytest.mark.parametrize("N", [12, 16, 3])
def test_iq4n32_column_groups(lib, orc, N):
    """8 + 4 and 8 + 8 columns on the MFMA path, 3 columns one GEMV each."""
    rows, K = 300, 2048
    w = synth.iq4nl(rows, K, 133)
    x = synth.x_f32(K * N, 133 + N).reshape(K, N)
    a, off = upload(lib, w)
    assert rel_err(gemm(lib, a, off, x, rows, K, N), reference(orc, w, x)) <= TOL


@pytest.mark.parametrize("N", [4, 8])
def test_iq4n32_close_to_fp64_and_spread(lib, orc, N):
    """Against the exact product of the dequantized weights: ordinary
    activations at K = 16384 and 3584, and magnitudes 2^-20 .. 2^20 mixed
    inside every wave step: within 1e-6 per column."""
    for rows, K, spread in [(256, 16384, False), (512, 3584, False), (256, 4096, True)]:
        w = synth.iq4nl(rows, K, 134)
        if spread:
            rng = np.random.default_rng(134)
            mag = np.exp2(rng.uniform(-20, 20, (K, N))).astype(np.float32)
            x = (mag * np.sign(rng.standard_normal((K, N)))).astype(np.float32)
        else:
            x = synth.x_f32(K * N, 134).reshape(K, N)
        a, off = upload(lib, w)
        c = gemm(lib, a, off, x, rows, K, N)
        ex = dense(orc, w) @ np.asarray(x, np.float64)
        for n in range(N):
            assert rel_err(c[:, n], ex[:, n]) <= 1e-6, (rows, K, spread, n)


def test_iq4n32_codebook_worst_case(lib, orc):
    """Every weight on T = -0.5250730 (the entry fp16 alone rounds worst,
    by 3.25e-4 relative) and positive activations: only the codebook's hi + lo split
    keeps the result within the bar."""
    rows, K, N = 256, 4096, 8
    nblk = rows * K // 32
    rng = np.random.default_rng(135)
    nib = np.full((nblk, 32), 2, np.uint8)
    scales = synth.f16_bits(np.abs(rng.standard_normal(nblk).astype(np.float32)) * np.float32(0.01) + np.float32(0.001))
    raw = synth.pack_iq4nl(nib, scales)
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_iq4nl_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
    a, off = torch.from_numpy(host).cuda(), lib.zt_q4_gpu_data_offset(nblk)
    x = rng.uniform(0.5, 1.5, (K, N)).astype(np.float32)
    W = orc.iq4nl_dequant(raw, rows * K).reshape(rows, K)
    ref = (W @ x).astype(np.float32)
    assert rel_err(gemm(lib, a, off, x, rows, K, N), ref) <= TOL
