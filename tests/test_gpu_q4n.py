"""GPU parity of Q4_0 with several fp32 activation columns on the raw-layout
entry point (zt_gemm_q4_f32 with N > 1):
  * N % 4 == 0 with 16-byte aligned B and K <= 32768: q4_rb_kernel, the
    row-block MFMA GEMM (groups of 8 columns for K <= 4096, else of 4), one
    launch per group, weights read once per group;
  * other even N with 8-byte aligned B and K <= 16384: gemv_q4n_steps_kernel
    in groups of 2 columns (VALU, the batch-1 products);
  * anything else: the per-column GEMV.

This is the reference's batched GemmQ4F32 contract (internal/gpuapi/
kernels.go:45-48; gemm_q4.cu:117-159 for N > 1; the CPU GemmF32Q4NT,
internal/xblas/gemm_quant.go:81-157).  Bars:
  * max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle;
  * MFMA path: within 1e-6 of the exact (fp64) product, also with
    activations spread over 2^+-20 inside one wave step (the fp16 hi + lo
    split after a power-of-two normalisation per step carries each
    activation to about 2^-22 of the step's max |x|), and the same bits on
    a second call (no atomics);
  * 2-column groups: every column bit for bit the batch-1 GEMV of that
    column (the same products, chains and reduction tree);
  * rows of C past M are never written.
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
    lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    return torch.from_numpy(host).cuda(), lib.zt_q4_gpu_data_offset(nblk)


def gemm(lib, a, off, x, rows, K, N, xoff=0):
    """C = A x on the device; x is [K, N] float32, placed `xoff` floats into
    its buffer (to test B alignment); C has 8 guard floats past the end."""
    xb = torch.zeros(K * N + xoff, dtype=torch.float32, device="cuda")
    xb[xoff:] = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.full((rows * N + 8,), float("nan"), dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4_f32", a.data_ptr(), xb.data_ptr() + 4 * xoff, c.data_ptr(), rows, K, N, off, stream())
    out = c.cpu().numpy()
    assert np.all(np.isnan(out[rows * N:]))
    return out[:rows * N].reshape(rows, N)


def batch1(lib, a, off, x, rows, K):
    """Each column through the batch-1 GEMV."""
    cols = []
    for n in range(x.shape[1]):
        xd = torch.from_numpy(np.ascontiguousarray(x[:, n], np.float32)).cuda()
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        lib.call("zt_gemm_q4_f32", a.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, 1, off, stream())
        cols.append(y.cpu().numpy())
    return np.stack(cols, axis=1)


def oracle(orc, w, x, N):
    return orc.gemm_f32_q4_nt(np.ascontiguousarray(x.T), w.raw, N, w.rows, w.K, threads=orc.nthreads()) \
        .reshape(N, w.rows).T


def exact64(orc, w, x):
    W = orc.q4_dequant(w.raw, w.rows * w.K).astype(np.float64).reshape(w.rows, w.K)
    return W @ np.asarray(x, np.float64)


@pytest.mark.parametrize("N", [2, 4, 8])
@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (17, 544), (100, 4096), (65, 4128), (33, 8192), (9, 16384),
                                    (2049, 1024), (5, 20480), (7, 32768), (3301, 17024)])
def test_q4n_ragged(lib, orc, rows, K, N):
    """Partial row sets and workgroups, K not a multiple of a step (512),
    one, two and four steps a wave (3301 x 17024: four row sets at four
    steps, 9 waves, a partial last workgroup): the oracle's result; 2 columns: each
    column the batch-1 kernel's bits; 4 and 8: the same bits on a second
    call."""
    print(f"q4n rows={rows} K={K} N={N}", flush=True)
    w = synth.q4_0(rows, K, 101)
    x = synth.x_f32(K * N, 101 + N).reshape(K, N)
    a, off = upload(lib, w)
    c = gemm(lib, a, off, x, rows, K, N)
    assert rel_err(c, oracle(orc, w, x, N)) <= TOL
    if N == 2 and K <= 16384:
        assert np.array_equal(c.view(np.uint32), batch1(lib, a, off, x, rows, K).view(np.uint32))
    else:
        assert np.array_equal(c.view(np.uint32), gemm(lib, a, off, x, rows, K, N).view(np.uint32))


@pytest.mark.parametrize("N", [4, 8])
@pytest.mark.parametrize("rows,K", [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_q4n_llama3_8b_shapes(lib, orc, rows, K, N):
    print(f"q4n rows={rows} K={K} N={N}", flush=True)
    w = synth.q4_0(rows, K, synth.seed_for(2, rows % 5))
    x = synth.x_f32(K * N, 102 + N).reshape(K, N)
    a, off = upload(lib, w)
    c = gemm(lib, a, off, x, rows, K, N)
    assert rel_err(c, oracle(orc, w, x, N)) <= TOL
    assert np.array_equal(c.view(np.uint32), gemm(lib, a, off, x, rows, K, N).view(np.uint32))


@pytest.mark.parametrize("N,xoff", [(6, 0), (12, 0), (16, 0), (24, 0), (4, 2), (8, 2), (3, 0), (5, 1)])
def test_q4n_column_groups_and_alignment(lib, orc, N, xoff):
    """Column groups on the MFMA path (8 + 4, 8 + 8, 8 + 8 + 8), B rows only
    8-byte aligned or N = 6 (2-column groups, bit-equal to batch 1), and odd
    N (the per-column kernel)."""
    rows, K = 300, 2048
    print(f"q4n groups N={N} xoff={xoff}", flush=True)
    w = synth.q4_0(rows, K, 103)
    x = synth.x_f32(K * N, 103 + N).reshape(K, N)
    a, off = upload(lib, w)
    c = gemm(lib, a, off, x, rows, K, N, xoff)
    assert rel_err(c, oracle(orc, w, x, N)) <= TOL
    if N % 2 == 0 and (N % 4 != 0 or xoff % 4 != 0):
        assert np.array_equal(c.view(np.uint32), batch1(lib, a, off, x, rows, K).view(np.uint32))


@pytest.mark.parametrize("N", [4, 8])
def test_q4n_close_to_fp64(lib, orc, N):
    """The MFMA path against the exact product at K = 16384 (N = 8 as two
    4-column groups) and K = 4096: within 1e-6 (normal-range weight
    operands; subnormal ones would be biased low by several 1e-6 here)."""
    for rows, K in [(256, 16384), (512, 4096)]:
        w = synth.q4_0(rows, K, 105)
        x = synth.x_f32(K * N, 105).reshape(K, N)
        a, off = upload(lib, w)
        assert rel_err(gemm(lib, a, off, x, rows, K, N), exact64(orc, w, x)) <= 1e-6, (rows, K)


@pytest.mark.parametrize("N", [4, 8])
def test_q4n_activations_spanning_2e20(lib, orc, N):
    """Activations of magnitudes 2^-20 .. 2^20 mixed inside every wave step
    (and columns 2^5 and 2^10 apart): each column's normwise error against
    the fp64 product stays within 1e-6, and within 1e-5 of the oracle."""
    rows, K = 256, 4096
    rng = np.random.default_rng(106)
    w = synth.q4_0(rows, K, 106)
    mag = np.exp2(rng.uniform(-20, 20, (K, N))).astype(np.float32)
    x = (mag * np.sign(rng.standard_normal((K, N)))).astype(np.float32) * np.exp2(5.0 * (np.arange(N) % 3))
    x = x.astype(np.float32)
    a, off = upload(lib, w)
    c = gemm(lib, a, off, x, rows, K, N)
    ex = exact64(orc, w, x)
    ref = oracle(orc, w, x, N)
    for n in range(N):
        assert rel_err(c[:, n], ex[:, n]) <= 1e-6, n
        assert rel_err(c[:, n], ref[:, n]) <= TOL, n


def test_q4n_scaled_and_zero_columns(lib, orc):
    """Columns 10^6 apart in scale and an all-zero column (exact zeros)."""
    rows, K, N = 256, 4096, 4
    w = synth.q4_0(rows, K, 104)
    x = synth.x_f32(K * N, 104).reshape(K, N) * np.array([1e3, 1e-3, 0.0, 1.0], np.float32)
    a, off = upload(lib, w)
    c = gemm(lib, a, off, x, rows, K, N)
    ref = oracle(orc, w, x, N)
    for n in (0, 1, 3):
        assert rel_err(c[:, n], ref[:, n]) <= TOL
    assert np.all(c[:, 2] == 0.0)


def test_rowblock_gemms_in_hip_graph_replays(lib, orc):
    """The one-launch batched GEMMs (fp32 row-block on Q4_0, fp16 row-block on
    W4A16 packed scales and on IQ4_NL) captured in a HIP graph: every replay,
    with eager work and synchronisations between replays, gives the eager
    result bit for bit (they need no memset, workspace or second kernel)."""
    rows, K, N = 1024, 4096, 8
    w = synth.q4_0(rows, K, 107)
    a, off = upload(lib, w)
    x = torch.from_numpy(synth.x_f32(K * N, 107)).cuda()
    w4 = synth.w4a16(rows, K, 108)
    p4, s4, z4 = (torch.from_numpy(np.ascontiguousarray(v).view(np.uint8).reshape(-1).copy()).cuda()
                  for v in (w4.packed, w4.scales, w4.zeros))
    szr = torch.empty(w4.scales.size, dtype=torch.int32, device="cuda")
    lib.call("zt_w4a16_pack_szr", s4.data_ptr(), z4.data_ptr(), rows, K, 128, szr.data_ptr(), stream())
    wi = synth.iq4nl(rows, K, 109)
    nblk = rows * K // 32
    sep = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_iq4nl_raw_to_gpu(wi.raw.ctypes.data, nblk, sep.ctypes.data)
    ai = torch.from_numpy(sep).cuda()
    x16 = torch.from_numpy(synth.x_f16(K * N, 109).view(np.uint8).copy()).cuda()
    outs = [torch.empty(rows * N, dtype=torch.float32, device="cuda") for _ in range(3)]

    def launch(s):
        lib.call("zt_gemm_q4_f32", a.data_ptr(), x.data_ptr(), outs[0].data_ptr(), rows, K, N, off, s)
        lib.call("zt_gemm_w4a16sz_f32", p4.data_ptr(), szr.data_ptr(), x16.data_ptr(), outs[1].data_ptr(), rows, K,
                 N, 128, s)
        lib.call("zt_gemm_iq4nl_f16", ai.data_ptr(), x16.data_ptr(), outs[2].data_ptr(), rows, K, N,
                 lib.zt_q4_gpu_data_offset(nblk), s)

    launch(stream())
    torch.cuda.synchronize()
    eager = [o.cpu().numpy().copy() for o in outs]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch(torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        for o in outs:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for o, e in zip(outs, eager):
            assert np.array_equal(o.cpu().numpy().view(np.uint32), e.view(np.uint32)), rep
        launch(stream())  # eager work between replays
        torch.cuda.synchronize()
