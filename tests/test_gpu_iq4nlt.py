"""GPU parity of the tiled IQ4_NL layout (zt_iq4nl_tile, zt_gemm_iq4nlt_f16).

The tiled layout is this build's upload-time repack for batched fp16
activations on IQ4_NL weights (the reference's engine falls back to its CPU
engine for them, compute/cpu_engine.go:1215-1245).  Bars:
  * the repack: byte-identical with the layout restated here in numpy;
  * the GEMM: max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle's
    restatement of the reference CPU engine (DequantizeIQ4NL, then the
    fp32 GEMM); the codebook enters the MFMAs as two fp16 parts, exact to
    2^-22 per entry (measured about 2e-6).
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


def separated(lib, raw: np.ndarray, nblk: int):
    out = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_iq4nl_raw_to_gpu(raw.ctypes.data, nblk, out.ctypes.data)
    return out, lib.zt_q4_gpu_data_offset(nblk)


def tile_ref(raw: np.ndarray, rows: int, K: int):
    """Data: piece 16 g + i of tile (rt, u) = dword g of blocks 4u .. 4u+3 of
    row 16 rt + i; scales: [rt][u][16 rows][4 blocks] fp16."""
    nt, nu, kb = (rows + 15) // 16, K // 128, K // 32
    blk = raw.reshape(rows * kb, 18)
    d = np.zeros((nt * 16, kb, 16), np.uint8)
    d[:rows] = blk[:, 2:].reshape(rows, kb, 16)
    sc = np.zeros((nt * 16, kb), np.uint16)
    sc[:rows] = blk[:, :2].copy().view("<u2").reshape(rows, kb)
    # d: [rt, i, u, s, g, 4] -> [rt, u, g, i, s, 4]
    dt = d.reshape(nt, 16, nu, 4, 4, 4).transpose(0, 2, 4, 1, 3, 5).reshape(-1)
    st = sc.reshape(nt, 16, nu, 4).transpose(0, 2, 1, 3).reshape(-1)
    return dt, st


def tile_dev(lib, raw, rows, K):
    nblk = rows * K // 32
    sep, off = separated(lib, raw, nblk)
    a = dev(sep)
    wt = torch.empty(lib.zt_iq4nl_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
    st = torch.empty(lib.zt_iq4nl_tiled_scale_bytes(rows, K), dtype=torch.uint8, device="cuda")
    lib.call("zt_iq4nl_tile", a.data_ptr(), rows, K, off, wt.data_ptr(), st.data_ptr(), stream())
    torch.cuda.synchronize()
    return wt, st


def workspace(lib, rows, K, N):
    nb = lib.zt_gemm_iq4nlt_workspace_bytes(rows, K, N)
    assert nb >= 0
    return torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda"), nb


def run_t(lib, wt, st, x16, rows, K, N):
    xd = dev(x16)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    ws, nb = workspace(lib, rows, K, N)
    lib.call("zt_gemm_iq4nlt_f16", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
             ws.data_ptr(), nb, stream())
    return c.cpu().numpy()


@pytest.mark.parametrize("rows,K", [(16, 128), (17, 256), (100, 1024), (1, 384)])
def test_tile_layout_bytes(lib, rows, K):
    w = synth.iq4nl(rows, K, 71)
    wt, st = tile_dev(lib, w.raw, rows, K)
    dref, sref = tile_ref(w.raw, rows, K)
    assert np.array_equal(wt.cpu().numpy(), dref)
    assert np.array_equal(st.cpu().numpy().view("<u2"), sref)


@pytest.mark.parametrize("rows,K,N", [(16, 128, 4), (17, 256, 8), (33, 2176, 12), (65, 384, 16), (100, 4096, 8),
                                      (40, 12288, 4), (1, 128, 16), (300, 1024, 16)])
def test_iq4nlt_ragged(lib, orc, rows, K, N):
    print(f"iq4nlt rows={rows} K={K} N={N}", flush=True)
    w = synth.iq4nl(rows, K, 72)
    x16 = synth.x_f16(K * N, 72)
    wt, st = tile_dev(lib, w.raw, rows, K)
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(run_t(lib, wt, st, x16, rows, K, N), ref) <= TOL


@pytest.mark.parametrize("N", [4, 8, 16])
@pytest.mark.parametrize("rows,K", QWEN)
def test_iq4nlt_qwen_shapes(lib, orc, rows, K, N):
    """The Qwen2-7B shapes at full size against the oracle, and against the
    separated-layout MFMA kernel on the same operands."""
    print(f"iq4nlt rows={rows} K={K} N={N}", flush=True)
    seed = synth.seed_for(5, QWEN.index((rows, K)))
    w = synth.iq4nl(rows, K, seed)
    x16 = synth.x_f16(K * N, seed + N)
    wt, st = tile_dev(lib, w.raw, rows, K)
    y = run_t(lib, wt, st, x16, rows, K, N)
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(y, ref) <= TOL
    nblk = rows * K // 32
    sep, off = separated(lib, w.raw, nblk)
    a, xd = dev(sep), dev(x16)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_iq4nl_f16", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, off, stream())
    assert rel_err(y, c.cpu().numpy()) <= TOL


def test_iq4nlt_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    for rows, K, N in [(2, 128, 3), (2, 128, 1), (2, 96, 4), (2, 160, 8)]:
        assert lib.zt_gemm_iq4nlt_f16(p, p, p, p, rows, K, N, p, 1 << 16, stream()) == 1, (rows, K, N)
    assert lib.zt_gemm_iq4nlt_f16(p + 4, p, p, p, 2, 128, 4, p, 1 << 16, stream()) == 1
    need = lib.zt_gemm_iq4nlt_workspace_bytes(3584, 3584, 8)
    assert need > 0
    assert lib.zt_gemm_iq4nlt_f16(p, p, p, p, 3584, 3584, 8, 0, 0, stream()) == 1  # workspace missing
    assert lib.zt_gemm_iq4nlt_f16(p, p, p, p, 3584, 3584, 8, p, need - 1, stream()) == 1  # too short
    assert lib.zt_iq4nl_tile(p, 2, 96, 16, p, p, stream()) == 1  # K % 128
    assert lib.zt_iq4nl_tile(p, 2, 128, 8, p, p, stream()) == 1  # data not 16-byte aligned


@pytest.mark.parametrize("rows", [512, 8192])
@pytest.mark.parametrize("N", [8, 16])
@pytest.mark.parametrize("side", ["A", "B"])
def test_engine_batched_iq4nl_dispatch(lib, orc, side, N, rows):
    """16 columns of the 8192-row matrix build the tiled copy; 8 columns
    at K <= 8192, and 16 up to 4096 rows, run the row-block GEMM on the
    separated upload and build none."""
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import IQ4NLStorage, Tensor

    K = 1024
    w = synth.iq4nl(rows, K, 73)
    s = IQ4NLStorage.from_raw(w.raw, rows * K)
    eng = ROCmEngine()
    x16 = synth.x_f16(K * N, 73)
    ref = np.asarray(orc.iq4nl_matmul(w.raw, x16, rows, K, N)).reshape(rows, N)
    xk = torch.from_numpy(x16.view(np.float16).reshape(K, N)).cuda()
    if side == "A":
        y = eng.matmul(Tensor((rows, K), s), xk).cpu().numpy()
        want = ref
    else:
        y = eng.matmul(xk.t().contiguous(), Tensor((K, rows), s)).cpu().numpy()
        want = ref.T
    assert rel_err(y.reshape(-1), want.reshape(-1)) <= TOL
    assert (getattr(s, "_gpu_tiled", None) is not None) == (N == 16 and rows > 4096)


def test_iq4nlt_repeated_calls_bit_identical(lib):
    """Split-K calls repeat bit for bit (partials summed in split order)."""
    for rows, K, N in [(3584, 3584, 8), (1024, 8192, 16)]:
        assert lib.zt_gemm_iq4nlt_workspace_bytes(rows, K, N) > 0
        w = synth.iq4nl(rows, K, 75)
        x16 = synth.x_f16(K * N, 75)
        wt, st = tile_dev(lib, w.raw, rows, K)
        a = run_t(lib, wt, st, x16, rows, K, N)
        b = run_t(lib, wt, st, x16, rows, K, N)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, K, N)


def test_iq4nlt_split_combine_graph_replays_and_two_streams(lib, orc):
    """Split-K calls (partials to a workspace, then the ordered sum)
    captured in a HIP graph and replayed with eager calls in between, then
    run on two streams at once: every result matches the oracle."""
    rows, K, N = 3584, 3584, 8
    cases = []
    for seed in (73, 74):
        w = synth.iq4nl(rows, K, seed)
        x16 = synth.x_f16(K * N, seed)
        wt, st = tile_dev(lib, w.raw, rows, K)
        cases.append((wt, st, dev(x16), torch.empty(rows * N, dtype=torch.float32, device="cuda"),
                      orc.iq4nl_matmul(w.raw, x16, rows, K, N), workspace(lib, rows, K, N)))

    def call(case, s):
        wt, st, xd, c, _, (ws, nb) = case
        lib.call("zt_gemm_iq4nlt_f16", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
                 ws.data_ptr(), nb, s)

    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        call(cases[0], cs.cuda_stream)
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call(cases[0], torch.cuda.current_stream().cuda_stream)
    for rep in range(4):
        cases[0][3].fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert rel_err(cases[0][3].cpu().numpy(), cases[0][4]) <= TOL, rep
        call(cases[1], stream())
        torch.cuda.synchronize()
        assert rel_err(cases[1][3].cpu().numpy(), cases[1][4]) <= TOL, rep
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for rep in range(3):
        for case, s in zip(cases, streams):
            for _ in range(3):
                call(case, s.cuda_stream)
        torch.cuda.synchronize()
        for i, case in enumerate(cases):
            assert rel_err(case[3].cpu().numpy(), case[4]) <= TOL, (rep, i)
