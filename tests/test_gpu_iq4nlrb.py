"""GPU parity of the single-launch batched IQ4_NL GEMM on the separated
upload layout (zt_gemm_iq4nl_f16 with fp16 activations and N = 4, 8, 12 or
16, the row-block kernel; past 4096 rows, N = 12 and 16 run the 16x16x32 MFMA
kernel without a K split).

The reference has no IQ4_NL matmul: CPUEngine.MatMul falls back to
Data() and an fp32 GEMM (tensor/tensor.go:216-219, compute/cpu_engine.go:
1215-1245), which the oracle restates.  Bars:
  * max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle: the codebook
    enters the MFMAs as T_hi + T_lo in fp16 (within 2^-22 of every fp32
    entry) and every product is exact in fp32;
  * the worst-rounded codebook entry everywhere, with positive activations,
    stays within the bar (dropping T_lo would miss by 3.25e-4);
  * bit-identical from call to call (no atomics).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
QWEN = [(3584, 3584), (18944, 3584), (3584, 18944)]


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


def run(lib, raw, x16, rows, K, N):
    nblk = rows * K // 32
    sep = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_iq4nl_raw_to_gpu(raw.ctypes.data, nblk, sep.ctypes.data)
    a, xd = dev(sep), dev(x16)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_iq4nl_f16", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
             lib.zt_q4_gpu_data_offset(nblk), stream())
    return c.cpu().numpy()


@pytest.mark.parametrize("N", [4, 8, 12, 16])
@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (5, 544), (17, 4128), (100, 8192), (64, 12288), (9, 32768),
                                    (2049, 1024), (2100, 1024), (3000, 2080), (4096, 8192), (4097, 1024)])
def test_iq4nl_rb_ragged(lib, orc, rows, K, N):
    """Partial row sets and workgroups, K not a multiple of a step (16
    blocks), one to four steps a wave; at N = 12 and 16 two row sets (2049
    to 3000 rows), four (4096, two steps a wave at K = 8192), and the
    16x16x32 path past 4096 rows."""
    print(f"iq4nl rb rows={rows} K={K} N={N}", flush=True)
    w = synth.iq4nl(rows, K, 81)
    x16 = synth.x_f16(K * N, 81 + N)
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(run(lib, w.raw, x16, rows, K, N), ref) <= TOL


@pytest.mark.parametrize("N", [4, 8])
@pytest.mark.parametrize("rows,K", QWEN)
def test_iq4nl_rb_qwen_shapes(lib, orc, rows, K, N):
    print(f"iq4nl rb rows={rows} K={K} N={N}", flush=True)
    seed = synth.seed_for(5, QWEN.index((rows, K)))
    w = synth.iq4nl(rows, K, seed)
    x16 = synth.x_f16(K * N, seed + N)
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(run(lib, w.raw, x16, rows, K, N), ref) <= TOL


def test_iq4nl_rb_codebook_worst_case(lib, orc):
    """Every weight on T = -0.5250730 (fp16 rounds it by 3.25e-4) and every
    activation positive: only the hi + lo split keeps the result within
    the bar."""
    rows, K, N = 256, 4096, 8
    nblk = rows * K // 32
    rng = np.random.default_rng(82)
    nib = np.full((nblk, 32), 2, np.uint8)
    scales = synth.f16_bits(np.abs(rng.standard_normal(nblk).astype(np.float32)) * np.float32(0.01) + np.float32(0.001))
    raw = synth.pack_iq4nl(nib, scales)
    x16 = synth.f16_bits(rng.uniform(0.5, 1.5, K * N).astype(np.float32))
    ref = orc.iq4nl_matmul(raw, x16, rows, K, N)
    assert rel_err(run(lib, raw, x16, rows, K, N), ref) <= TOL


def test_iq4nl_rb_repeated_calls_bit_identical(lib):
    for rows, K, N in [(3584, 3584, 8), (1024, 8192, 4), (300, 18944, 8), (1000, 4096, 16), (4096, 4096, 16)]:
        w = synth.iq4nl(rows, K, 83)
        x16 = synth.x_f16(K * N, 83)
        a = run(lib, w.raw, x16, rows, K, N)
        b = run(lib, w.raw, x16, rows, K, N)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, K, N)
