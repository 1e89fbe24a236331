"""GPU parity of the tiled W4A16 layout (zt_w4a16_tile, zt_gemm_w4a16t_f32).

The tiled layout is this build's upload-time repack for the small-batch path
of W4A16MatMuler.MatMulW4A16 (compute/w4a16.go:137-143); the reference
uploads W4A16 weights as stored.  Bars:
  * the repack: byte-identical with the layout restated here in numpy (each
    16-row x 128-K tile one 1 KB block in lane order, rows past M zero; the
    (scale, zero) dwords laid out [group][row]);
  * the GEMM: max|y - y_ref| / max|y_ref| <= 1e-5 against the oracle's
    restatement of the reference CPU engine (dequantize, then SgemmSimd):
    every product is exact in fp32, so only the summation order differs;
    within 1e-5 of zt_gemm_w4a16_f32 on the same operands; bit-identical
    from call to call (split K ranges are summed through the workspace in a
    fixed order).
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
LLAMA70B = [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)]


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


def tile_ref(packed: np.ndarray, rows: int, K: int) -> np.ndarray:
    """The tiled byte layout: tile (rt, u) = 64 pieces of 16 bytes, piece
    16 g + i = row 16 rt + i, packed bytes [64 u + 16 g, +16)."""
    nt, nu = (rows + 15) // 16, K // 128
    p = np.zeros((nt * 16, K // 2), np.uint8)
    p[:rows] = packed.reshape(rows, K // 2)
    # [rt, i, u, g, 16] -> [rt, u, g, i, 16]
    return p.reshape(nt, 16, nu, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


def sz_ref(scales: np.ndarray, zeros, rows: int, ng: int) -> np.ndarray:
    s = scales.reshape(rows, ng).astype(np.uint32)
    z = np.full((rows, ng), 0x4800, np.uint32) if zeros is None else zeros.reshape(rows, ng).astype(np.uint32)
    return (s | (z << 16)).T.reshape(-1)


def tile_dev(lib, w, zeros=True):
    rows, K, g = w.rows, w.K, w.group
    p, s = dev(w.packed), dev(w.scales)
    z = dev(w.zeros) if zeros else None
    wt = torch.empty(lib.zt_w4a16_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
    sz = torch.empty(lib.zt_w4a16_sz_bytes(rows, K, g) // 4, dtype=torch.int32, device="cuda")
    lib.call("zt_w4a16_tile", p.data_ptr(), s.data_ptr(), z.data_ptr() if zeros else 0, rows, K, g, wt.data_ptr(),
             sz.data_ptr(), stream())
    return wt, sz


def workspace(lib, rows, K, N):
    nb = lib.zt_gemm_w4a16t_workspace_bytes(rows, K, N)
    assert nb >= 0
    return torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda"), nb


def run_w4t(lib, wt, sz, x16, rows, K, N, g):
    xd = dev(x16)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    ws, nb = workspace(lib, rows, K, N)
    lib.call("zt_gemm_w4a16t_f32", wt.data_ptr(), sz.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, g,
             ws.data_ptr(), nb, stream())
    return c.cpu().numpy()


@pytest.mark.parametrize("rows,K,g,zeros", [(16, 128, 128, True), (17, 256, 64, True), (100, 1024, 128, False),
                                            (1, 384, 32, True)])
def test_tile_layout_bytes(lib, rows, K, g, zeros):
    w = synth.w4a16(rows, K, 61, group=g)
    wt, sz = tile_dev(lib, w, zeros)
    assert np.array_equal(wt.cpu().numpy(), tile_ref(w.packed, rows, K))
    assert np.array_equal(sz.cpu().numpy().view(np.uint32), sz_ref(w.scales, w.zeros if zeros else None, rows,
                                                                   K // g))


@pytest.mark.parametrize("rows,K,g,N", [(16, 128, 128, 4), (17, 256, 128, 8), (33, 2176, 128, 12), (65, 384, 128, 16),
                                        (100, 4096, 256, 8), (40, 12288, 128, 4), (1, 128, 128, 16),
                                        (300, 1024, 128, 16)])
def test_w4t_ragged(lib, orc, rows, K, g, N):
    """Partial row tiles and workgroups (17, 33, 65, 100, 300 rows; one row),
    a partial last K range (2176 = 17 units), group 256, N = 12, and few-row
    matrices whose K is split across many workgroups."""
    print(f"w4a16t rows={rows} K={K} g={g} N={N}", flush=True)
    w = synth.w4a16(rows, K, 62, group=g)
    x16 = synth.x_f16(K * N, 62)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, g)
    wt, sz = tile_dev(lib, w)
    assert rel_err(run_w4t(lib, wt, sz, x16, rows, K, N, g), ref) <= TOL


def test_w4t_non_integer_zero_and_default_zero(lib, orc):
    """Any fp16 zero point (y subtracts z * sum(x) exactly); zeros == NULL is
    the symmetric zero-point 8."""
    rows, K, N = 64, 1024, 8
    w = synth.w4a16(rows, K, 63)
    rng = np.random.default_rng(63)
    zeros = synth.f16_bits((rng.random(w.zeros.shape, dtype=np.float32) * 15).astype(np.float32))
    w2 = synth.W4Weights(rows, K, w.group, w.packed, w.scales, zeros)
    x16 = synth.x_f16(K * N, 63)
    wt, sz = tile_dev(lib, w2)
    ref = orc.w4a16_matmul(w2.packed, w2.scales, w2.zeros, x16, rows, K, N, 128)
    assert rel_err(run_w4t(lib, wt, sz, x16, rows, K, N, 128), ref) <= TOL
    wt, sz = tile_dev(lib, w, zeros=False)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128)
    assert rel_err(run_w4t(lib, wt, sz, x16, rows, K, N, 128), ref) <= TOL


def test_w4t_small_activations(lib, orc):
    """Activations of order 1e-4, many below the fp16 normal range: the
    A operands are exact subnormals and X is staged unscaled, so the
    products stay exact in fp32."""
    rows, K, N = 256, 2048, 16
    w = synth.w4a16(rows, K, 64)
    rng = np.random.default_rng(64)
    x = (rng.standard_normal(K * N).astype(np.float32) * np.float32(1e-4))
    x16 = synth.f16_bits(x)
    wt, sz = tile_dev(lib, w)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128)
    assert rel_err(run_w4t(lib, wt, sz, x16, rows, K, N, 128), ref) <= TOL


@pytest.mark.parametrize("N", [4, 8, 16])
@pytest.mark.parametrize("rows,K", LLAMA70B)
def test_w4t_70b_shapes(lib, orc, rows, K, N):
    """The Llama-3-70B layer at full size against the oracle, and against
    the row-major kernel on the same operands."""
    print(f"w4a16t rows={rows} K={K} N={N}", flush=True)
    seed = synth.seed_for(4, LLAMA70B.index((rows, K)))
    w = synth.w4a16(rows, K, seed)
    x16 = synth.x_f16(K * N, seed + N)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128)
    wt, sz = tile_dev(lib, w)
    y = run_w4t(lib, wt, sz, x16, rows, K, N, 128)
    assert rel_err(y, ref) <= TOL
    p, s, z = dev(w.packed), dev(w.scales), dev(w.zeros)
    xd = dev(x16)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_w4a16_f32", p.data_ptr(), s.data_ptr(), z.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
             128, stream())
    assert rel_err(y, c.cpu().numpy()) <= 1e-5


def test_w4t_repeated_calls_bit_identical(lib):
    """Split-K calls repeat bit for bit: the partial tiles go through the
    workspace and are summed in split order (no atomics, no zero fill)."""
    for rows, K, N in [(4096, 4096, 8), (1024, 8192, 16), (300, 12288, 4)]:
        assert lib.zt_gemm_w4a16t_workspace_bytes(rows, K, N) > 0  # the K range is split
        w = synth.w4a16(rows, K, 65)
        x16 = synth.x_f16(K * N, 65)
        wt, sz = tile_dev(lib, w)
        a = run_w4t(lib, wt, sz, x16, rows, K, N, 128)
        b = run_w4t(lib, wt, sz, x16, rows, K, N, 128)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), (rows, K, N)


def test_w4t_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    bad = [
        (2, 128, 3, 128),   # N not in {4, 8, 12, 16}
        (2, 128, 1, 128),
        (2, 96, 4, 32),     # K % 128
        (2, 256, 4, 64),    # group % 128
        (2, 256, 4, 96),    # K % group
    ]
    for rows, K, N, g in bad:
        assert lib.zt_gemm_w4a16t_f32(p, p, p, p, rows, K, N, g, p, 1 << 16, stream()) == 1, (rows, K, N, g)
    assert lib.zt_gemm_w4a16t_f32(p + 4, p, p, p, 2, 128, 4, 128, p, 1 << 16, stream()) == 1  # W_tiled alignment
    need = lib.zt_gemm_w4a16t_workspace_bytes(1024, 8192, 8)
    assert need > 0
    assert lib.zt_gemm_w4a16t_f32(p, p, p, p, 1024, 8192, 8, 128, 0, 0, stream()) == 1  # workspace missing
    assert lib.zt_gemm_w4a16t_f32(p, p, p, p, 1024, 8192, 8, 128, p, need - 1, stream()) == 1  # too short
    assert lib.zt_gemm_w4a16t_f32(p, p, p, p, 1024, 8192, 8, 128, p + 8, need, stream()) == 1  # misaligned
    assert lib.zt_w4a16_tile(p, p, 0, 2, 96, 32, p, p, stream()) == 1  # K % 128
    assert lib.zt_w4a16_tile(p + 8, p, 0, 2, 128, 32, p, p, stream()) == 1  # W_packed alignment


@pytest.mark.parametrize("rows", [512, 8192])
@pytest.mark.parametrize("N", [8, 16])
@pytest.mark.parametrize("side", ["A", "B"])
def test_engine_batched_w4a16_dispatch(lib, orc, side, N, rows):
    """ROCmEngine.matmul_w4a16 with 8 or 16 activation columns (A side) or
    rows (B side) matches the oracle.  16 columns of the 8192-row matrix
    build the tiled copy once; 8 columns, and 16 of the 512-row matrix, run
    the row-block GEMM on the row-major upload and build none."""
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Float16Storage, GPTQStorage, Tensor

    K = 1024
    w = synth.w4a16(rows, K, 66)
    st = GPTQStorage.from_raw(w.packed.reshape(-1), w.scales.reshape(-1), w.zeros.reshape(-1), rows * K, 128, 4)
    eng = ROCmEngine()
    ref = np.asarray(orc.w4a16_matmul(w.packed, w.scales, w.zeros, synth.x_f16(K * N, 66), rows, K, N, 128))
    ref = ref.reshape(rows, N)
    x16 = synth.x_f16(K * N, 66)  # [K, N]
    if side == "A":
        act = Tensor((K, N), Float16Storage.from_raw(x16, K * N))
        y = eng.matmul_w4a16(Tensor((rows, K), st), act).cpu().numpy()
        want = ref
    else:
        xt = np.ascontiguousarray(x16.reshape(K, N).T)  # [N, K]
        act = Tensor((N, K), Float16Storage.from_raw(xt, K * N))
        y = eng.matmul_w4a16(act, Tensor((K, rows), st)).cpu().numpy()
        want = ref.T
    assert rel_err(y.reshape(-1), want.reshape(-1)) <= TOL
    assert (getattr(st, "_gpu_tiled", None) is not None) == (N == 16 and rows > 4096)


def _w4t_call(lib, wt, sz, xd, c, rows, K, N, s, ws):
    lib.call("zt_gemm_w4a16t_f32", wt.data_ptr(), sz.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, 128,
             ws[0].data_ptr(), ws[1], s)


def test_w4t_split_combine_graph_replays(lib, orc):
    """A split-K call (partials to the workspace, then the ordered sum)
    captured in a HIP graph: every replay, with eager calls of the same
    kernel on other operands and another workspace in between, matches the
    oracle and the eager result bit for bit."""
    rows, K, N = 4096, 4096, 8
    w = synth.w4a16(rows, K, 67)
    x16 = synth.x_f16(K * N, 67)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128)
    wt, sz = tile_dev(lib, w)
    xd = dev(x16)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    w2 = synth.w4a16(rows, K, 68)
    x2 = synth.x_f16(K * N, 68)
    ref2 = orc.w4a16_matmul(w2.packed, w2.scales, w2.zeros, x2, rows, K, N, 128)
    wt2, sz2 = tile_dev(lib, w2)
    xd2 = dev(x2)
    c2 = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    ws, ws2 = workspace(lib, rows, K, N), workspace(lib, rows, K, N)
    cs = torch.cuda.Stream()
    cs.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(cs):
        _w4t_call(lib, wt, sz, xd, c, rows, K, N, cs.cuda_stream, ws)
    torch.cuda.current_stream().wait_stream(cs)
    torch.cuda.synchronize()
    eager = c.cpu().numpy().copy()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _w4t_call(lib, wt, sz, xd, c, rows, K, N, torch.cuda.current_stream().cuda_stream, ws)
    for rep in range(4):
        c.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        got = c.cpu().numpy()
        assert rel_err(got, ref) <= TOL, rep
        assert np.array_equal(got.view(np.uint32), eager.view(np.uint32)), rep
        _w4t_call(lib, wt2, sz2, xd2, c2, rows, K, N, stream(), ws2)
        torch.cuda.synchronize()
        assert rel_err(c2.cpu().numpy(), ref2) <= TOL, rep


def test_w4t_split_combine_two_streams(lib, orc):
    """Split-K calls on two streams at once, repeated, both against the
    oracle."""
    rows, K, N = 8192, 8192, 16
    cases = []
    for seed in (69, 70):
        w = synth.w4a16(rows, K, seed)
        x16 = synth.x_f16(K * N, seed)
        wt, sz = tile_dev(lib, w)
        cases.append((wt, sz, dev(x16), torch.empty(rows * N, dtype=torch.float32, device="cuda"),
                      orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128), workspace(lib, rows, K, N)))
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    for rep in range(3):
        for (wt, sz, xd, c, _, ws), s in zip(cases, streams):
            for _ in range(3):
                _w4t_call(lib, wt, sz, xd, c, rows, K, N, s.cuda_stream, ws)
        torch.cuda.synchronize()
        for i, (_, _, _, c, ref, _) in enumerate(cases):
            assert rel_err(c.cpu().numpy(), ref) <= TOL, (rep, i)

