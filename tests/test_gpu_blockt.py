"""GPU parity of the batched Q4_0 / Q8_0 MFMA GEMMs on tiled layouts
(zt_q4_tile / zt_gemm_q4t_f32, zt_q8_tile / zt_gemm_q8t_f32).

The products are the reference's batched Q4_0 / Q8_0 matmuls with fp32
activations (xblas.GemmF32Q4NT / GemmF32Q8NT, internal/xblas/gemm_quant.go:
81-264, run here by the oracle's C restatement).  Bars:
  * the repacks: byte-identical with the layouts restated here in numpy;
  * the GEMMs: max|y - y_ref| / max|y_ref| <= 1e-5 with fp32 accumulation
    (measured about 1e-7: the activations are carried as two fp16 parts
    after a power-of-two normalisation), also for activations far outside
    the fp16 range, tiny activations and columns of very different scale,
    and for the IQ4_NL tiled kernel reached through the engine;
  * split-K results repeat bit for bit from call to call.
"""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5  # every product exact in fp32: only the summation order differs
LLAMA = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


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


def weights(fmt: str, rows: int, K: int, seed: int):
    return synth.q4_0(rows, K, seed) if fmt == "q4" else synth.q8_0(rows, K, seed)


def separated(lib, fmt: str, raw: np.ndarray, nblk: int):
    if fmt == "q4":
        out = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
        lib.zt_q4_raw_to_gpu(raw.ctypes.data, nblk, out.ctypes.data)
        return out, lib.zt_q4_gpu_data_offset(nblk)
    out = np.empty(lib.zt_q8_gpu_bytes(nblk), np.uint8)
    lib.zt_q8_raw_to_gpu(raw.ctypes.data, nblk, out.ctypes.data)
    return out, lib.zt_q8_gpu_data_offset(nblk)


def tile_ref(fmt: str, raw: np.ndarray, rows: int, K: int):
    """Q4_0: piece 16 g + i of tile (rt, u) = dword g of blocks 4u .. 4u+3 of
    row 16 rt + i, fp16 scales [rt][u][16 rows][4 blocks].  Q8_0: half h,
    piece 16 g + i = bytes 8g .. 8g+7 of blocks 4u+2h and 4u+2h+1 of row
    16 rt + i, fp32 scales [rt][u][16 rows][4 blocks]."""
    nt, nu, kb = (rows + 15) // 16, K // 128, K // 32
    if fmt == "q4":
        blk = raw.reshape(rows * kb, 18)
        d = np.zeros((nt * 16, kb, 16), np.uint8)
        d[:rows] = blk[:, 2:].reshape(rows, kb, 16)
        sc = np.zeros((nt * 16, kb), np.uint16)
        sc[:rows] = blk[:, :2].copy().view("<u2").reshape(rows, kb)
        dt = d.reshape(nt, 16, nu, 4, 4, 4).transpose(0, 2, 4, 1, 3, 5).reshape(-1)
    else:
        blk = raw.reshape(rows * kb, 36)
        d = np.zeros((nt * 16, kb, 32), np.uint8)
        d[:rows] = blk[:, 4:].reshape(rows, kb, 32)
        sc = np.zeros((nt * 16, kb), np.float32)
        sc[:rows] = blk[:, :4].copy().view("<f4").reshape(rows, kb)
        # d: [rt, i, u, h, b2, g, 8] -> [rt, u, h, g, i, b2, 8]
        dt = d.reshape(nt, 16, nu, 2, 2, 4, 8).transpose(0, 2, 3, 5, 1, 4, 6).reshape(-1)
    st = sc.reshape(nt, 16, nu, 4).transpose(0, 2, 1, 3).reshape(-1)
    return dt, st


def tile_dev(lib, fmt, raw, rows, K):
    nblk = rows * K // 32
    sep, off = separated(lib, fmt, raw, nblk)
    a = dev(sep)
    wt = torch.empty(getattr(lib, f"zt_{fmt}_tiled_bytes")(rows, K), dtype=torch.uint8, device="cuda")
    st = torch.empty(getattr(lib, f"zt_{fmt}_tiled_scale_bytes")(rows, K), dtype=torch.uint8, device="cuda")
    lib.call(f"zt_{fmt}_tile", a.data_ptr(), rows, K, off, wt.data_ptr(), st.data_ptr(), stream())
    torch.cuda.synchronize()
    return wt, st


def workspace(lib, fmt, rows, K, N):
    nb = getattr(lib, f"zt_gemm_{fmt}t_workspace_bytes")(rows, K, N)
    assert nb >= 0
    return torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda"), nb


def run_t(lib, fmt, wt, st, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    ws, nb = workspace(lib, fmt, rows, K, N)
    lib.call(f"zt_gemm_{fmt}t_f32", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
             ws.data_ptr(), nb, stream())
    return c.cpu().numpy().reshape(rows, N)


def oracle(orc, fmt, raw, x, rows, K, N):
    """The reference CPU GEMM on x [K, N]: C^T = X^T W^T (GemmF32Q{4,8}NT)."""
    xt = np.ascontiguousarray(np.asarray(x, np.float32).reshape(K, N).T)
    f = orc.gemm_f32_q4_nt if fmt == "q4" else orc.gemm_f32_q8_nt
    return f(xt, raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T


@pytest.mark.parametrize("fmt", ["q4", "q8"])
@pytest.mark.parametrize("rows,K", [(16, 128), (17, 256), (100, 1024), (1, 384)])
def test_tile_layout_bytes(lib, fmt, rows, K):
    w = weights(fmt, rows, K, 81)
    wt, st = tile_dev(lib, fmt, w.raw, rows, K)
    dref, sref = tile_ref(fmt, w.raw, rows, K)
    assert np.array_equal(wt.cpu().numpy(), dref)
    got = st.cpu().numpy().view("<u2" if fmt == "q4" else "<f4")
    assert np.array_equal(got.view(np.uint8), sref.view(np.uint8))


@pytest.mark.parametrize("fmt", ["q4", "q8"])
@pytest.mark.parametrize("rows,K,N", [(16, 128, 4), (17, 256, 8), (33, 2176, 12), (65, 384, 16), (100, 4096, 8),
                                      (40, 12288, 4), (1, 128, 16), (300, 1024, 16), (129, 640, 12)])
def test_blockt_ragged(lib, orc, fmt, rows, K, N):
    print(f"{fmt}t rows={rows} K={K} N={N}", flush=True)
    w = weights(fmt, rows, K, 82)
    x = synth.x_f32(K * N, 82).reshape(K, N)
    wt, st = tile_dev(lib, fmt, w.raw, rows, K)
    assert rel_err(run_t(lib, fmt, wt, st, x, rows, K, N), oracle(orc, fmt, w.raw, x, rows, K, N)) <= TOL


@pytest.mark.parametrize("N", [4, 8, 16])
@pytest.mark.parametrize("rows,K", LLAMA)
@pytest.mark.parametrize("fmt", ["q4", "q8"])
def test_blockt_llama3_shapes(lib, orc, fmt, rows, K, N):
    """The Llama-3-8B shapes at full size against the oracle, and against
    the VALU batched kernel on the separated layout."""
    print(f"{fmt}t rows={rows} K={K} N={N}", flush=True)
    seed = synth.seed_for(2, LLAMA.index((rows, K)))
    w = weights(fmt, rows, K, seed)
    x = synth.x_f32(K * N, seed + N).reshape(K, N)
    wt, st = tile_dev(lib, fmt, w.raw, rows, K)
    y = run_t(lib, fmt, wt, st, x, rows, K, N)
    err = rel_err(y, oracle(orc, fmt, w.raw, x, rows, K, N))
    assert err <= 1e-5, err  # fp32-level: two fp16 parts carry each activation
    nblk = rows * K // 32
    sep, off = separated(lib, fmt, w.raw, nblk)
    a, xd = dev(sep), torch.from_numpy(np.ascontiguousarray(x).reshape(-1)).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    name = "zt_gemm_q4_f32" if fmt == "q4" else "zt_gemm_q8sep_f32"
    lib.call(name, a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, off, stream())
    assert rel_err(y, c.cpu().numpy().reshape(rows, N)) <= 1e-5
    # the split-K reduction runs in a fixed order: a second call is bit-identical
    assert np.array_equal(run_t(lib, fmt, wt, st, x, rows, K, N), y)


@pytest.mark.parametrize("fmt", ["q4", "q8"])
@pytest.mark.parametrize("case", ["huge", "tiny", "mixed_columns", "span_2e20", "zero", "one_hot"])
def test_blockt_activation_ranges(lib, orc, fmt, case):
    """Activations outside fp16's range (|x| up to 1e7), far below its normal
    range (1e-7), columns 1e4 apart in scale, magnitudes spread over 2^-20 ..
    2^20 inside every workgroup's K range (the power-of-two scaling follows
    the largest; each hi + lo pair holds an activation to 2^-22 relative down
    to 2^-17 of that largest, and to 2^-25 / c absolute below), all zero, and
    a single nonzero activation (the result is one weight column times x)."""
    rows, K, N = 96, 1024, 8
    w = weights(fmt, rows, K, 83)
    x = synth.x_f32(K * N, 83).reshape(K, N)
    if case == "huge":
        x = x * np.float32(1e7)
    elif case == "tiny":
        x = x * np.float32(1e-7)
    elif case == "mixed_columns":
        x = x * np.float32(1e4) ** (np.arange(N) % 2).astype(np.float32)
    elif case == "span_2e20":
        e = np.random.default_rng(84).uniform(-20.0, 20.0, x.shape)
        x = (x * np.exp2(e)).astype(np.float32)
    elif case == "zero":
        x = np.zeros_like(x)
    else:
        x = np.zeros_like(x)
        x[517, 3] = np.float32(3.25)
    x = np.ascontiguousarray(x, np.float32)
    wt, st = tile_dev(lib, fmt, w.raw, rows, K)
    y = run_t(lib, fmt, wt, st, x, rows, K, N)
    ref = oracle(orc, fmt, w.raw, x, rows, K, N)
    assert np.all(np.isfinite(y))
    if case == "zero":
        assert np.array_equal(y, np.zeros_like(y))
    elif case == "one_hot" and fmt == "q4":
        assert np.array_equal(y, ref)  # scale * ((q - 8) x): one rounding both ways
    elif case == "one_hot":
        # the reference rounds q * scale, then x * that (gemm_quant.go:199-201): one ulp apart at most
        assert rel_err(y, ref) <= 2.0 ** -22
    elif case in ("mixed_columns", "span_2e20"):
        for n in range(N):  # each column on its own scale
            assert rel_err(y[:, n], ref[:, n]) <= TOL, n
    else:
        assert rel_err(y, ref) <= 1e-5


def test_blockt_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    for fmt in ("q4", "q8"):
        g = getattr(lib, f"zt_gemm_{fmt}t_f32")
        for rows, K, N in [(2, 128, 3), (2, 128, 1), (2, 96, 4), (2, 160, 8), (-1, 128, 4)]:
            assert g(p, p, p, p, rows, K, N, p, 1 << 16, stream()) == 1, (fmt, rows, K, N)
        assert g(p + 4, p, p, p, 2, 128, 4, p, 1 << 16, stream()) == 1
        assert g(p, p, p + 4, p, 2, 128, 4, p, 1 << 16, stream()) == 1  # B not 16-byte aligned
        assert g(p, p, p, p, 0, 128, 4, 0, 0, stream()) == 0  # empty: nothing to do
        assert getattr(lib, f"zt_{fmt}_tiled_bytes")(2, 96) == -1
        wsb = getattr(lib, f"zt_gemm_{fmt}t_workspace_bytes")
        assert wsb(2, 96, 4) == -1 and wsb(2, 128, 3) == -1
        assert wsb(16, 128, 4) == 0  # one K range: no split, no workspace
        need = wsb(4096, 4096, 8)
        assert need > 0
        # K split but the workspace is missing, short or misaligned
        assert g(p, p, p, p, 4096, 4096, 8, 0, 0, stream()) == 1
        assert g(p, p, p, p, 4096, 4096, 8, p, need - 16, stream()) == 1
        assert g(p, p, p, p, 4096, 4096, 8, p + 4, need, stream()) == 1
    assert lib.zt_q4_tile(p, 2, 96, 16, p, p, stream()) == 1  # K % 128
    assert lib.zt_q8_tile(p, 2, 96, 16, p, p, stream()) == 1
    assert lib.zt_q8_tile(p, 2, 128, 8, p, p, stream()) == 1  # data not 16-byte aligned


@pytest.mark.parametrize("fmt", ["q4", "q8"])
@pytest.mark.parametrize("side", ["A", "B"])
def test_engine_batched_uses_tiled_layout(lib, orc, fmt, side):
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Q4Storage, Q8Storage, Tensor

    rows, K, N = 8192, 4096, 8  # past the row-block GEMM's shapes (engine._block_rowblock)
    w = weights(fmt, rows, K, 84)
    if fmt == "q4":
        s = Q4Storage.from_raw(w.raw, rows * K)
    else:
        q = w.raw.reshape(-1, 36)
        s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), rows * K)
    eng = ROCmEngine()
    x = synth.x_f32(K * N, 84).reshape(K, N)
    ref = oracle(orc, fmt, w.raw, x, rows, K, N)
    xk = torch.from_numpy(x).cuda()
    if side == "A":
        y = eng.matmul(Tensor((rows, K), s), xk).cpu().numpy()
        want = ref
    else:
        y = eng.matmul(xk.t().contiguous(), Tensor((K, rows), s)).cpu().numpy()
        want = ref.T
    assert rel_err(y.reshape(-1), want.reshape(-1)) <= TOL
    assert getattr(s, "_gpu_tiled", None) is not None


@pytest.mark.parametrize("fmt", ["q4", "q8"])
@pytest.mark.parametrize("rows,K,N", [(512, 1024, 4), (1024, 4096, 8), (4096, 4096, 4), (4100, 4096, 4)])
def test_engine_batched_rowblock_dispatch(lib, orc, fmt, rows, K, N):
    """Batches the row-block GEMM wins run on the batch-1 upload (no tiled
    copy is built); the others keep the tiled layout; both give the
    oracle's result."""
    from ztensor_amd.engine import ROCmEngine, _block_rowblock, _w4a16_rowblock
    from ztensor_amd.storage import Q4Storage, Q8Storage, Tensor

    w = weights(fmt, rows, K, 88)
    if fmt == "q4":
        s = Q4Storage.from_raw(w.raw, rows * K)
    else:
        q = w.raw.reshape(-1, 36)
        s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), rows * K)
    x = synth.x_f32(K * N, 88).reshape(K, N)
    y = ROCmEngine().matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda()).cpu().numpy()
    assert rel_err(y.reshape(-1), oracle(orc, fmt, w.raw, x, rows, K, N).reshape(-1)) <= TOL
    assert (getattr(s, "_gpu_tiled", None) is None) == _block_rowblock(fmt, rows, K, N)


@pytest.mark.parametrize("fmt", ["q4", "q8"])
def test_blockt_split_graph_replays_and_two_streams(lib, orc, fmt):
    """Split-K calls (partials to a workspace, then the reduction kernel)
    captured in a HIP graph and replayed with eager calls in between, then
    run on two streams at once, each with its own workspace: every result
    matches the oracle."""
    rows, K, N = 4096, 4096, 8
    cases = []
    for seed in (85, 86):
        w = weights(fmt, rows, K, seed)
        x = synth.x_f32(K * N, seed).reshape(K, N)
        wt, st = tile_dev(lib, fmt, w.raw, rows, K)
        ws, nb = workspace(lib, fmt, rows, K, N)  # one per case: the two streams overlap
        assert nb > 0
        cases.append((wt, st, torch.from_numpy(np.ascontiguousarray(x).reshape(-1)).cuda(),
                      torch.empty(rows * N, dtype=torch.float32, device="cuda"),
                      oracle(orc, fmt, w.raw, x, rows, K, N).reshape(-1), ws, nb))

    def call(case, s):
        wt, st, xd, c, _, ws, nb = case
        lib.call(f"zt_gemm_{fmt}t_f32", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
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


@pytest.mark.parametrize("n", [2, 3, 5, 20])
@pytest.mark.parametrize("fmt", ["q4", "q4_f16", "q8", "iq4nl", "w4a16"])
def test_engine_other_batch_sizes_on_tiled_kernels(lib, orc, fmt, n):
    """Batches outside {4, 8, 12, 16}: ROCmEngine runs them on the tiled
    kernels in column chunks of 16, zero-padded to a multiple of 4, and the
    result matches the reference CPU product (Q4_0 also with fp16
    activations, widened exactly to fp32); chunks that the row-block GEMM
    takes run on the batch-1 upload instead."""
    from ztensor_amd.engine import ROCmEngine, _block_rowblock, _w4a16_rowblock
    from ztensor_amd.storage import GPTQStorage, IQ4NLStorage, Q4Storage, Q8Storage, Tensor

    rows, K = 200, 1024
    eng = ROCmEngine()
    if fmt in ("q4", "q4_f16", "q8"):
        w = weights(fmt[:2], rows, K, 87)
        if fmt != "q8":
            s = Q4Storage.from_raw(w.raw, rows * K)
        else:
            q = w.raw.reshape(-1, 36)
            s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), rows * K)
        x = synth.x_f32(K * n, 87).reshape(K, n)
        if fmt == "q4_f16":  # fp16 activations: the reference widens them to fp32 (tensor/fp16_storage.go:53-63)
            x = x.astype(np.float16).astype(np.float32)
        ref = oracle(orc, fmt[:2], w.raw, x, rows, K, n)
        xd = torch.from_numpy(x.astype(np.float16) if fmt == "q4_f16" else x).cuda()
    elif fmt == "iq4nl":
        w = synth.iq4nl(rows, K, 87)
        s = IQ4NLStorage.from_raw(w.raw, rows * K)
        x16 = synth.x_f16(K * n, 87)
        ref = np.asarray(orc.iq4nl_matmul(w.raw, x16, rows, K, n)).reshape(rows, n)
        xd = torch.from_numpy(x16.view(np.float16).reshape(K, n)).cuda()
    else:
        w = synth.w4a16(rows, K, 87)
        s = GPTQStorage.from_raw(w.packed.reshape(-1), w.scales.reshape(-1), w.zeros.reshape(-1), rows * K, 128, 4)
        x16 = synth.x_f16(K * n, 87)
        ref = np.asarray(orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, n, 128)).reshape(rows, n)
        xd = torch.from_numpy(x16.view(np.float16).reshape(K, n)).cuda()
    y = eng.matmul(Tensor((rows, K), s), xd).cpu().numpy()
    assert y.shape == (rows, n)
    assert rel_err(y, ref) <= TOL
    chunk = -(-n // 4) * 4 if n < 16 else 16
    if ((fmt == "iq4nl" and K <= 8192 and (chunk <= 8 or rows <= 4096)) or
            (fmt == "w4a16" and _w4a16_rowblock(rows, K, chunk)) or
            (fmt in ("q4", "q4_f16", "q8") and _block_rowblock(fmt[:2], rows, K, chunk))):
        # chunks the row-block GEMM takes run on the batch-1 upload
        assert getattr(s, "_gpu_tiled", None) is None
    else:
        assert getattr(s, "_gpu_tiled", None) is not None


# ---- batched Q4_K on the same kernel (zt_q4k_tile, zt_gemm_q4kt_f32)

def q4k_tile_ref(raw: np.ndarray, rows: int, K: int):
    """Data: every 32-value sub-block rewritten as a 16-byte Q4_0 block (byte
    j = value j | value j+16 << 4), then the Q4_0 tile order; headers: the
    first 16 bytes of every super-block as [tile][super-block][16 rows]."""
    nt, nu, nsb = (rows + 15) // 16, K // 128, K // 256
    sbk = raw.reshape(rows, nsb, 144)
    nib = sbk[:, :, 16:].reshape(rows, nsb, 4, 32)
    q = np.stack([(nib >> 4 * h) & 15 for h in (0, 1)], axis=3).reshape(rows, nsb * 8, 32)  # sub-block 2g+h
    blocks = (q[:, :, :16] | (q[:, :, 16:] << 4)).astype(np.uint8)
    d = np.zeros((nt * 16, K // 32, 16), np.uint8)
    d[:rows] = blocks
    dt = d.reshape(nt, 16, nu, 4, 4, 4).transpose(0, 2, 4, 1, 3, 5).reshape(-1)
    hd = np.zeros((nt * 16, nsb, 16), np.uint8)
    hd[:rows] = sbk[:, :, :16]
    ht = hd.reshape(nt, 16, nsb, 16).transpose(0, 2, 1, 3).reshape(-1)
    return dt, ht


def q4k_tile_dev(lib, raw, rows, K):
    a = dev(raw)
    wt = torch.empty(lib.zt_q4k_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
    ht = torch.empty(lib.zt_q4k_tiled_header_bytes(rows, K), dtype=torch.uint8, device="cuda")
    lib.call("zt_q4k_tile", a.data_ptr(), rows, K, wt.data_ptr(), ht.data_ptr(), stream())
    torch.cuda.synchronize()
    return wt, ht


def run_q4kt(lib, wt, ht, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    nb = lib.zt_gemm_q4kt_workspace_bytes(rows, K, N)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")
    lib.call("zt_gemm_q4kt_f32", wt.data_ptr(), ht.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, ws.data_ptr(),
             nb, stream())
    return c.cpu().numpy().reshape(rows, N)


def q4k_oracle(orc, raw, x, rows, K, N):
    xt = np.ascontiguousarray(np.asarray(x, np.float32).reshape(K, N).T)
    return orc.gemm_f32_kq_nt("q4_k", xt, raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T


@pytest.mark.parametrize("rows,K", [(16, 256), (17, 512), (100, 1024), (1, 768)])
def test_q4k_tile_layout_bytes(lib, rows, K):
    w = synth.kquant("q4_k", rows, K, 91)
    wt, ht = q4k_tile_dev(lib, w.raw, rows, K)
    dref, href = q4k_tile_ref(w.raw, rows, K)
    assert np.array_equal(wt.cpu().numpy(), dref)
    assert np.array_equal(ht.cpu().numpy(), href)


@pytest.mark.parametrize("rows,K,N", [(16, 256, 4), (17, 512, 8), (33, 2304, 12), (65, 768, 16), (100, 4096, 8),
                                      (40, 12288, 4), (1, 256, 16), (300, 1024, 16)])
def test_q4kt_ragged(lib, orc, rows, K, N):
    print(f"q4kt rows={rows} K={K} N={N}", flush=True)
    w = synth.kquant("q4_k", rows, K, 92)
    x = synth.x_f32(K * N, 92).reshape(K, N)
    wt, ht = q4k_tile_dev(lib, w.raw, rows, K)
    assert rel_err(run_q4kt(lib, wt, ht, x, rows, K, N), q4k_oracle(orc, w.raw, x, rows, K, N)) <= TOL


@pytest.mark.parametrize("N", [4, 8, 16])
@pytest.mark.parametrize("rows,K", LLAMA)
def test_q4kt_llama3_shapes(lib, orc, rows, K, N):
    """The Llama-3-8B shapes at full size against the oracle (the reference
    CPU engine's GemmF32Q4KNT), and deterministic across calls."""
    print(f"q4kt rows={rows} K={K} N={N}", flush=True)
    seed = synth.seed_for(6, LLAMA.index((rows, K)))
    w = synth.kquant("q4_k", rows, K, seed)
    x = synth.x_f32(K * N, seed + N).reshape(K, N)
    wt, ht = q4k_tile_dev(lib, w.raw, rows, K)
    y = run_q4kt(lib, wt, ht, x, rows, K, N)
    err = rel_err(y, q4k_oracle(orc, w.raw, x, rows, K, N))
    assert err <= 1e-5, err
    assert np.array_equal(run_q4kt(lib, wt, ht, x, rows, K, N), y)


def test_q4kt_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    g = lib.zt_gemm_q4kt_f32
    for rows, K, N in [(2, 256, 3), (2, 128, 4), (2, 384, 8), (-1, 256, 4)]:
        assert g(p, p, p, p, rows, K, N, p, 1 << 16, stream()) == 1, (rows, K, N)
    assert lib.zt_q4k_tile(p, 2, 128, p, p, stream()) == 1  # K % 256
    assert lib.zt_q4k_tile(p + 4, 2, 256, p, p, stream()) == 1
    assert lib.zt_q4k_tiled_bytes(2, 128) == -1 and lib.zt_gemm_q4kt_workspace_bytes(2, 128, 4) == -1


@pytest.mark.parametrize("n", [3, 8])
def test_engine_batched_q4k_uses_tiled_layout(lib, orc, n):
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Q4KStorage, Tensor

    rows, K = 300, 1024
    w = synth.kquant("q4_k", rows, K, 93)
    s = Q4KStorage(w.raw, rows * K)
    x = synth.x_f32(K * n, 93).reshape(K, n)
    y = ROCmEngine().matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda()).cpu().numpy()
    assert rel_err(y, q4k_oracle(orc, w.raw, x, rows, K, n)) <= TOL
    assert getattr(s, "_gpu_tiled", None) is not None


# ---- batched Q5_0 on the same kernel (zt_q5_0_tile, zt_gemm_q5_0t_f32)

Q5_BITS = [0, 2, 16, 18, 1, 3, 17, 19]  # fifth-bit order in a lane's byte, offset by 4g


def q5_tile_dev(lib, raw, rows, K):
    nblk = rows * K // 32
    host = np.empty(lib.zt_q5_0_gpu_bytes(nblk), np.uint8)
    lib.zt_q5_0_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
    a = dev(host)
    bufs = [torch.empty(f(rows, K), dtype=torch.uint8, device="cuda")
            for f in (lib.zt_q5_0_tiled_bytes, lib.zt_q5_0_tiled_scale_bytes, lib.zt_q5_0_tiled_qh_bytes)]
    lib.call("zt_q5_0_tile", a.data_ptr(), rows, K, lib.zt_q5_0_gpu_qh_offset(nblk), lib.zt_q5_0_gpu_qs_offset(nblk),
             *(b.data_ptr() for b in bufs), stream())
    torch.cuda.synchronize()
    return bufs


def q5_tile_ref(raw, rows, K):
    """Nibbles and scales: the Q4_0 tiled layout of the same 16 + 2 bytes;
    fifth bits: byte s of lane 16g+i's dword = bits 4g + Q5_BITS of block
    4u+s's qh word."""
    nt, nu, kb = (rows + 15) // 16, K // 128, K // 32
    blk = raw.reshape(rows * kb, 22)
    q4like = np.concatenate([blk[:, :2], blk[:, 6:]], axis=1).reshape(-1)
    dt, st = tile_ref("q4", q4like, rows, K)
    qh = np.zeros((nt * 16, kb), np.uint32)
    qh[:rows] = blk[:, 2:6].copy().view("<u4").reshape(rows, kb)
    q = qh.reshape(nt, 16, nu, 4)  # [rt, i, u, s]
    out = np.zeros((nt, nu, 4, 16), np.uint32)  # [rt, u, g, i]
    for g in range(4):
        byte = np.zeros((nt, 16, nu, 4), np.uint32)
        for k, e in enumerate(Q5_BITS):
            byte |= ((q >> np.uint32(4 * g + e)) & np.uint32(1)) << np.uint32(k)
        word = byte[..., 0] | (byte[..., 1] << np.uint32(8)) | (byte[..., 2] << np.uint32(16)) | (byte[..., 3] << np.uint32(24))
        out[:, :, g, :] = word.transpose(0, 2, 1)
    return dt, st, out.reshape(-1)


def run_q5t(lib, bufs, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    nb = lib.zt_gemm_q5_0t_workspace_bytes(rows, K, N)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")
    lib.call("zt_gemm_q5_0t_f32", *(b.data_ptr() for b in bufs), xd.data_ptr(), c.data_ptr(), rows, K, N,
             ws.data_ptr(), nb, stream())
    return c.cpu().numpy().reshape(rows, N)


def q5_oracle(orc, raw, x, rows, K, N):
    xt = np.ascontiguousarray(np.asarray(x, np.float32).reshape(K, N).T)
    return orc.gemm_f32_q5_0_nt(xt, raw, N, rows, K).reshape(N, rows).T


@pytest.mark.parametrize("rows,K", [(16, 128), (17, 256), (100, 1024), (1, 384)])
def test_q5_tile_layout_bytes(lib, rows, K):
    w = synth.kquant("q5_0", rows, K, 94)
    bufs = q5_tile_dev(lib, w.raw, rows, K)
    dref, sref, href = q5_tile_ref(w.raw, rows, K)
    assert np.array_equal(bufs[0].cpu().numpy(), dref)
    assert np.array_equal(bufs[1].cpu().numpy().view("<u2"), sref)
    assert np.array_equal(bufs[2].cpu().numpy().view("<u4"), href)


@pytest.mark.parametrize("rows,K,N", [(16, 128, 4), (17, 256, 8), (33, 2176, 12), (65, 384, 16), (100, 4096, 8),
                                      (1, 128, 16), (300, 1024, 16)])
def test_q5t_ragged(lib, orc, rows, K, N):
    print(f"q5t rows={rows} K={K} N={N}", flush=True)
    w = synth.kquant("q5_0", rows, K, 95)
    x = synth.x_f32(K * N, 95).reshape(K, N)
    bufs = q5_tile_dev(lib, w.raw, rows, K)
    assert rel_err(run_q5t(lib, bufs, x, rows, K, N), q5_oracle(orc, w.raw, x, rows, K, N)) <= TOL


@pytest.mark.parametrize("N", [4, 8, 16])
@pytest.mark.parametrize("rows,K", [(4096, 4096), (14336, 4096), (4096, 14336)])
def test_q5t_llama3_shapes(lib, orc, rows, K, N):
    print(f"q5t rows={rows} K={K} N={N}", flush=True)
    w = synth.kquant("q5_0", rows, K, 96)
    x = synth.x_f32(K * N, 96 + N).reshape(K, N)
    bufs = q5_tile_dev(lib, w.raw, rows, K)
    y = run_q5t(lib, bufs, x, rows, K, N)
    err = rel_err(y, q5_oracle(orc, w.raw, x, rows, K, N))
    assert err <= 1e-5, err


@pytest.mark.parametrize("n", [5, 8])
def test_engine_batched_q5_0_uses_tiled_layout(lib, orc, n):
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Q5_0Storage, Tensor

    rows, K = 300, 1024
    w = synth.kquant("q5_0", rows, K, 97)
    s = Q5_0Storage(w.raw, rows * K)
    x = synth.x_f32(K * n, 97).reshape(K, n)
    y = ROCmEngine().matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda()).cpu().numpy()
    assert rel_err(y, q5_oracle(orc, w.raw, x, rows, K, n)) <= TOL
    assert getattr(s, "_gpu_tiled", None) is not None


# ---- batched Q5_K (zt_q5k_tile, zt_gemm_q5kt_f32)

def q5k_tile_dev(lib, raw, rows, K):
    a = dev(raw)
    bufs = [torch.empty(f(rows, K), dtype=torch.uint8, device="cuda")
            for f in (lib.zt_q5k_tiled_bytes, lib.zt_q5k_tiled_header_bytes, lib.zt_q5k_tiled_qh_bytes)]
    lib.call("zt_q5k_tile", a.data_ptr(), rows, K, *(b.data_ptr() for b in bufs), stream())
    torch.cuda.synchronize()
    return bufs


def run_q5kt(lib, bufs, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    nb = lib.zt_gemm_q5kt_workspace_bytes(rows, K, N)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")
    lib.call("zt_gemm_q5kt_f32", *(b.data_ptr() for b in bufs), xd.data_ptr(), c.data_ptr(), rows, K, N,
             ws.data_ptr(), nb, stream())
    return c.cpu().numpy().reshape(rows, N)


@pytest.mark.parametrize("rows,K", [(16, 256), (17, 512), (1, 768)])
def test_q5k_tile_layout_bytes(lib, rows, K):
    """Data and headers as the Q4_K layout of the same nibbles (bytes 16..143
    of each 176-byte super-block, its first 16 bytes); fifth bits: bit j of
    byte 144 + l is value l of sub-block j, ordered per lane as for Q5_0."""
    w = synth.kquant("q5_k", rows, K, 98)
    nsb = K // 256
    sbk = w.raw.reshape(rows, nsb, 176)
    as_q4k = np.concatenate([sbk[:, :, :144]], axis=2).reshape(-1)
    dref, href = q4k_tile_ref(as_q4k, rows, K)
    bufs = q5k_tile_dev(lib, w.raw, rows, K)
    assert np.array_equal(bufs[0].cpu().numpy(), dref)
    assert np.array_equal(bufs[1].cpu().numpy(), href)
    # fifth bits as a per-block qh word (bit e = value e), then the Q5_0 lane order
    nt, nu = (rows + 15) // 16, K // 128
    qhb = sbk[:, :, 144:].astype(np.uint32)  # [rows, nsb, 32]
    words = np.zeros((nt * 16, nsb * 8), np.uint32)
    for j in range(8):
        for e in range(32):
            words[:rows, np.arange(nsb) * 8 + j] |= ((qhb[:, :, e] >> np.uint32(j)) & np.uint32(1)) << np.uint32(e)
    q = words.reshape(nt, 16, nu, 4)
    out = np.zeros((nt, nu, 4, 16), np.uint32)
    for g in range(4):
        byte = np.zeros((nt, 16, nu, 4), np.uint32)
        for k, e in enumerate(Q5_BITS):
            byte |= ((q >> np.uint32(4 * g + e)) & np.uint32(1)) << np.uint32(k)
        out[:, :, g, :] = (byte[..., 0] | (byte[..., 1] << np.uint32(8)) | (byte[..., 2] << np.uint32(16))
                           | (byte[..., 3] << np.uint32(24))).transpose(0, 2, 1)
    assert np.array_equal(bufs[2].cpu().numpy().view("<u4"), out.reshape(-1))


@pytest.mark.parametrize("rows,K,N", [(16, 256, 4), (33, 2304, 12), (100, 4096, 8), (300, 1024, 16),
                                      (4096, 4096, 8), (14336, 4096, 16), (4096, 14336, 8)])
def test_q5kt_matches_oracle(lib, orc, rows, K, N):
    print(f"q5kt rows={rows} K={K} N={N}", flush=True)
    w = synth.kquant("q5_k", rows, K, 99)
    x = synth.x_f32(K * N, 99).reshape(K, N)
    bufs = q5k_tile_dev(lib, w.raw, rows, K)
    xt = np.ascontiguousarray(x.T)
    ref = orc.gemm_f32_kq_nt("q5_k", xt, w.raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T
    err = rel_err(run_q5kt(lib, bufs, x, rows, K, N), ref)
    assert err <= 1e-5, err


def test_engine_batched_q5k_uses_tiled_layout(lib, orc):
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Q5KStorage, Tensor

    rows, K, n = 300, 1024, 8
    w = synth.kquant("q5_k", rows, K, 100)
    s = Q5KStorage(w.raw, rows * K)
    x = synth.x_f32(K * n, 100).reshape(K, n)
    y = ROCmEngine().matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda()).cpu().numpy()
    ref = orc.gemm_f32_kq_nt("q5_k", np.ascontiguousarray(x.T), w.raw, n, rows, K).reshape(n, rows).T
    assert rel_err(y, ref) <= TOL
    assert getattr(s, "_gpu_tiled", None) is not None


# ---- batched Q6_K (zt_q6k_tile, zt_gemm_q6kt_f32)

def q6k_values(raw, rows, K):
    """The 6-bit values 0..63 of Q6_K super-blocks as [rows, K] and the int8
    scales and fp16 d, per DequantizeQ6K (tensor/quantized_kquant.go:355-382):
    value 128h + 32j + l takes ql[64h + 32(j&1) + l] (low nibble for j < 2,
    high for j >= 2) and bits 2j..2j+1 of qh[32h + l]."""
    sbk = raw.reshape(rows, K // 256, 210).astype(np.int32)
    q = np.zeros((rows, K // 256, 256), np.int32)
    for h in range(2):
        for j in range(4):
            l = np.arange(32)
            lo = (sbk[:, :, 64 * h + 32 * (j & 1) + l] >> (4 * (j >> 1))) & 15
            hi = (sbk[:, :, 128 + 32 * h + l] >> (2 * j)) & 3
            q[:, :, 128 * h + 32 * j + l] = lo | (hi << 4)
    sc = sbk[:, :, 192:208].astype(np.uint8).view(np.int8).astype(np.float32)
    d = raw.reshape(rows, K // 256, 210)[:, :, 208:210].copy().view("<f2").astype(np.float32)
    return q.reshape(rows, K), (d * sc).reshape(rows, K // 16)


def q6k_tile_dev(lib, raw, rows, K):
    a = dev(raw)
    bufs = [torch.empty(f(rows, K), dtype=torch.uint8, device="cuda")
            for f in (lib.zt_q6k_tiled_bytes, lib.zt_q6k_tiled_scale_bytes)]
    lib.call("zt_q6k_tile", a.data_ptr(), rows, K, *(b.data_ptr() for b in bufs), stream())
    torch.cuda.synchronize()
    return bufs


def run_q6kt(lib, bufs, x, rows, K, N):
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32).reshape(-1)).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    nb = lib.zt_gemm_q6kt_workspace_bytes(rows, K, N)
    ws = torch.empty(max(nb, 16), dtype=torch.uint8, device="cuda")
    lib.call("zt_gemm_q6kt_f32", *(b.data_ptr() for b in bufs), xd.data_ptr(), c.data_ptr(), rows, K, N,
             ws.data_ptr(), nb, stream())
    return c.cpu().numpy().reshape(rows, N)


@pytest.mark.parametrize("rows,K", [(16, 256), (17, 512), (1, 768)])
def test_q6k_tile_layout_bytes(lib, rows, K):
    """Values as bytes (lane 16 g + i, half hh: for blocks 4u + 2hh and
    4u + 2hh + 1 of row 16 rt + i, values 4g .. 4g+3 and then 16 + 4g ..
    16 + 4g+3 of the block) and d * sc per 16-value group as [tile-unit]
    [16 rows][8 groups], zero past the last row."""
    w = synth.kquant("q6_k", rows, K, 101)
    q, s = q6k_values(w.raw, rows, K)
    nt, nu = (rows + 15) // 16, K // 128
    qp = np.zeros((nt * 16, K), np.uint8)
    qp[:rows] = q
    sp = np.zeros((nt * 16, K // 16), np.float32)
    sp[:rows] = s
    # [rt, i, u, hh, bb, h2, g, k4] -> [rt, u, hh, g, i, bb, h2, k4]
    dref = qp.reshape(nt, 16, nu, 2, 2, 2, 4, 4).transpose(0, 2, 3, 6, 1, 4, 5, 7).reshape(-1)
    sref = sp.reshape(nt, 16, nu, 8).transpose(0, 2, 1, 3).reshape(-1)
    bufs = q6k_tile_dev(lib, w.raw, rows, K)
    assert np.array_equal(bufs[0].cpu().numpy(), dref)
    assert np.array_equal(bufs[1].cpu().numpy().view(np.float32), sref)


@pytest.mark.parametrize("rows,K,N", [(16, 256, 4), (33, 2304, 12), (100, 4096, 8), (300, 1024, 16),
                                      (4096, 4096, 8), (14336, 4096, 16), (4096, 14336, 8)])
def test_q6kt_matches_oracle(lib, orc, rows, K, N):
    print(f"q6kt rows={rows} K={K} N={N}", flush=True)
    w = synth.kquant("q6_k", rows, K, 102)
    x = synth.x_f32(K * N, 102).reshape(K, N)
    bufs = q6k_tile_dev(lib, w.raw, rows, K)
    xt = np.ascontiguousarray(x.T)
    ref = orc.gemm_f32_kq_nt("q6_k", xt, w.raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T
    err = rel_err(run_q6kt(lib, bufs, x, rows, K, N), ref)
    assert err <= 1e-5, err


def test_q6kt_invalid_arguments(lib):
    assert lib.zt_q6k_tiled_bytes(16, 128) == -1
    assert lib.zt_q6k_tile(0, 16, 384, 0, 0, None) != 0
    assert lib.zt_gemm_q6kt_f32(0, 0, 0, 0, 16, 256, 5, 0, 0, None) != 0  # N not in {4, 8, 12, 16}


def test_engine_batched_q6k_uses_tiled_layout(lib, orc):
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import Q6KStorage, Tensor

    rows, K, n = 300, 1024, 8
    w = synth.kquant("q6_k", rows, K, 103)
    s = Q6KStorage(w.raw, rows * K)
    x = synth.x_f32(K * n, 103).reshape(K, n)
    y = ROCmEngine().matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda()).cpu().numpy()
    ref = orc.gemm_f32_kq_nt("q6_k", np.ascontiguousarray(x.T), w.raw, n, rows, K).reshape(n, rows).T
    assert rel_err(y, ref) <= TOL
    assert getattr(s, "_gpu_tiled", None) is not None


# ---- repeatability of the workspace reduction


@pytest.mark.parametrize("fmt", ["q4", "q8", "q4_k", "q5_k", "q6_k", "q5_0"])
def test_tiled_gemms_repeat_bit_for_bit(lib, fmt):
    """Every workspace-reduced tiled GEMM gives the same bits on two calls in
    a row (the K splits are summed in split order by one thread per output),
    at a shape whose K range is split across workgroups."""
    rows, K, N = 1024, 8192, 8
    x = synth.x_f32(K * N, 96)
    if fmt in ("q4", "q8"):
        assert getattr(lib, f"zt_gemm_{fmt}t_workspace_bytes")(rows, K, N) > 0
        w = weights(fmt, rows, K, 96)
        wt, st = tile_dev(lib, fmt, w.raw, rows, K)
        run = lambda: run_t(lib, fmt, wt, st, x, rows, K, N)
    elif fmt == "q4_k":
        assert lib.zt_gemm_q4kt_workspace_bytes(rows, K, N) > 0
        w = synth.kquant("q4_k", rows, K, 96)
        wt, ht = q4k_tile_dev(lib, w.raw, rows, K)
        run = lambda: run_q4kt(lib, wt, ht, x, rows, K, N)
    elif fmt == "q5_k":
        assert lib.zt_gemm_q5kt_workspace_bytes(rows, K, N) > 0
        bufs = q5k_tile_dev(lib, synth.kquant("q5_k", rows, K, 96).raw, rows, K)
        run = lambda: run_q5kt(lib, bufs, x, rows, K, N)
    elif fmt == "q6_k":
        assert lib.zt_gemm_q6kt_workspace_bytes(rows, K, N) > 0
        bufs = q6k_tile_dev(lib, synth.kquant("q6_k", rows, K, 96).raw, rows, K)
        run = lambda: run_q6kt(lib, bufs, x, rows, K, N)
    else:
        assert lib.zt_gemm_q5_0t_workspace_bytes(rows, K, N) > 0
        bufs = q5_tile_dev(lib, synth.kquant("q5_0", rows, K, 96).raw, rows, K)
        run = lambda: run_q5t(lib, bufs, x, rows, K, N)
    a, b = run(), run()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q4", "q8", "q5_0", "q4_k", "q5_k", "q6_k"])
def test_tiled_close_to_fp64_with_spread_activations(lib, orc, fmt):
    """Activations whose magnitudes spread over 2^-20 .. 2^20 inside every
    workgroup's K range: each column within 2e-6 of the exact (fp64) product
    of the dequantized weights (measured 2-7e-7).  The weights enter the
    MFMAs as normal-range fp16 (2^14 + 2^10 q and the like); as fp16
    subnormals (q 2^-24) the 4- and 5-bit formats came out up to 1.5e-5 off
    here."""
    rows, K, N = 96, 1024, 8
    x = synth.x_f32(K * N, 85).reshape(K, N)
    x = np.ascontiguousarray((x * np.exp2(np.random.default_rng(85).uniform(-20.0, 20.0, x.shape))).astype(np.float32))
    if fmt in ("q4", "q8"):
        w = weights(fmt, rows, K, 85)
        wt, st = tile_dev(lib, fmt, w.raw, rows, K)
        y = run_t(lib, fmt, wt, st, x, rows, K, N)
        deq = orc.q4_dequant(w.raw, rows * K) if fmt == "q4" else orc.q8_dequant(w.raw, rows * K)
    elif fmt == "q5_0":
        w = synth.kquant("q5_0", rows, K, 85)
        y = run_q5t(lib, q5_tile_dev(lib, w.raw, rows, K), x, rows, K, N)
        deq = orc.q5_0_dequant(w.raw, rows * K)
    else:
        w = synth.kquant(fmt, rows, K, 85)
        if fmt == "q4_k":
            wt, ht = q4k_tile_dev(lib, w.raw, rows, K)
            y = run_q4kt(lib, wt, ht, x, rows, K, N)
        elif fmt == "q5_k":
            y = run_q5kt(lib, q5k_tile_dev(lib, w.raw, rows, K), x, rows, K, N)
        else:
            y = run_q6kt(lib, q6k_tile_dev(lib, w.raw, rows, K), x, rows, K, N)
        deq = orc.kq_dequant(fmt, w.raw, rows * K)
    exact = deq.astype(np.float64).reshape(rows, K) @ x.astype(np.float64)
    for n in range(N):
        assert rel_err(y[:, n], exact[:, n]) <= 2e-6, n
