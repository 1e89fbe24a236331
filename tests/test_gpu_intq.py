"""GPU parity of the int4 / int8 GEMMs (zt_gemm_int4_f32, zt_gemm_int4_f32_rmul,
zt_gemm_int8_f32) against the oracle's restatement of the reference's
kernels (internal/cuda/kernels/gemm_int4.cu:29-144, gemm_int8.cu:16-73),
through the C ABI.

Bars: max|y - y_ref| / max|y_ref| <= 1e-5 with y_ref the oracle: every
weight is dequantized as the reference does (one fp32 multiply) and every
product is an fp32 product, so only the summation order differs.  Shapes:
the streaming batch-1..4 kernels (K % 16 == 0, group_size % 16 == 0; K
past one 4096-element activation chunk, rows not a multiple of a
workgroup's; for X W out % 16 == 0, partial column blocks), the bf16 MFMA
GEMM (A B with K % 32 == 0, group_size % 32 == 0, even N; partial 128 x 128
tiles, int4 zero points up to 255) and the fp32 MFMA GEMM (every other
shape: odd group sizes, K not a multiple of 16 or 32, odd N, partial 64-row
and 64-column tiles, X W past batch 4), the reference
benchmark's square GEMMs at 1024 in full and at 4096 on sampled rows, and
its inputs (bytes 0x53, scale 0.1, activations 0.01) at 4096 cubed on every
output against the fp32 FMA chain of its k loop and the exact sum, within
the summation bound K * 2^-24 that equal positive terms call for.
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


def run_rmul(lib, w, x, batch, inf, outf, gs):
    c = torch.full((batch * outf,), float("nan"), dtype=torch.float32, device="cuda")
    wd, xd, s, z = dev(w.packed), dev(x), dev(w.scales), dev(w.zeros)
    lib.call("zt_gemm_int4_f32_rmul", wd.data_ptr(), xd.data_ptr(), c.data_ptr(), s.data_ptr(), z.data_ptr(), batch,
             inf, outf, gs, stream())
    return c.cpu().numpy()


def run_int8(lib, a, b, M, K, N):
    c = torch.full((M * N,), float("nan"), dtype=torch.float32, device="cuda")
    ad, bd = dev(a), dev(b)
    lib.call("zt_gemm_int8_f32", ad.data_ptr(), bd.data_ptr(), c.data_ptr(), M, K, N, stream())
    return c.cpu().numpy()


INT4_CASES = [  # M, K, N, group_size
    (4096, 4096, 1, 32), (4096, 4096, 1, 128), (14336, 4096, 1, 128), (4096, 4096, 4, 32), (333, 1024, 3, 64),
    (1, 16, 1, 16), (4096, 4096, 2, 32), (100, 4112, 4, 16), (33, 8208, 2, 48),
    # batches 2-4 on 8192 rows: 4 rows a wave of the LDS-staged kernel, a partial last 4096-K chunk
    (8192, 4112, 2, 16), (8192, 4112, 3, 16), (8192, 4112, 4, 16),
    # batch 1 on the fixed-step kernel: two steps a wave past K = 16384, K = 32768, the loop kernel beyond
    (65, 20480, 1, 32), (17, 32768, 1, 128), (7, 33024, 1, 64), (2049, 16, 1, 16),
    # MFMA GEMM: group sizes not a multiple of 16, odd shapes, wider batches
    (1000, 1000, 2, 20), (77, 130, 5, 7), (65, 34, 9, 2), (512, 4096, 16, 128), (100, 2048, 64, 32), (3, 2, 1, 1),
    # bf16 MFMA GEMM (K % 32, group % 32, N even): partial 128 x 128 tiles
    (130, 96, 6, 32), (300, 4128, 130, 96), (64, 64, 8, 64),
]


@pytest.mark.parametrize("M,K,N,gs", INT4_CASES)
def test_int4_nt(lib, orc, M, K, N, gs):
    say(f"int4 M={M} K={K} N={N} gs={gs}")
    w = synth.int4(M, K, gs, 300 + M + K, zero_max=15)
    b = synth.x_f32(K * N, 301 + N).reshape(K, N)
    y = run_int4(lib, w, b, M, K, N, gs)
    assert rel_err(y, orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, N, gs)) <= TOL


RMUL_CASES = [  # batch, in, out, group_size
    (1, 4096, 4096, 32), (4, 4096, 4096, 128), (3, 1000, 1002, 7), (2, 64, 30, 16), (1, 1, 2, 1),
    (5, 512, 256, 32), (64, 1024, 1000, 32), (17, 33, 66, 5),
    (3, 100, 272, 16), (2, 1000, 4112, 48), (4, 130, 32, 32), (1, 63, 16, 16),
    # the 16-byte-load kernel (out % 32 == 0, group_size % 32 == 0): partial column blocks, K not a
    # multiple of the 8 waves' rows, batches 1-4
    (2, 1000, 4160, 64), (3, 2048, 96, 32), (1, 8191, 1024, 256), (4, 64, 4096, 32), (1, 14336, 4096, 32),
    (2, 4096, 14336, 128),
    # past batch 4, groups of up to 4 rows of X on the same kernels: the 16-byte-load kernel up to
    # batch 64 (ragged last groups), the 8-byte one up to batch 16 (in > 8192 or out % 32 != 0),
    # the fp32 MFMA GEMM beyond
    (8, 4096, 4096, 128), (13, 1000, 4160, 64), (32, 512, 2048, 32), (64, 256, 512, 32), (16, 9000, 1040, 16),
    (6, 300, 4112, 16), (65, 256, 512, 32), (17, 9000, 1024, 32),
]


@pytest.mark.parametrize("batch,inf,outf,gs", RMUL_CASES)
def test_int4_rmul(lib, orc, batch, inf, outf, gs):
    say(f"int4 rmul batch={batch} in={inf} out={outf} gs={gs}")
    w = synth.int4(inf, outf, gs, 400 + inf + outf, zero_max=15)
    x = synth.x_f32(batch * inf, 401 + batch).reshape(batch, inf)
    y = run_rmul(lib, w, x, batch, inf, outf, gs)
    assert rel_err(y, orc.gemm_int4_f32_rmul(w.packed, x, w.scales, w.zeros, batch, inf, outf, gs)) <= TOL


def test_int4_batch1_large_zero_points(lib, orc):
    """uint8 zero points up to 255 at batch 1 (the fixed-step kernel takes (8 + zero) sum x off a chunk's
    sum), against the oracle and the fp64 product."""
    M, K, gs = 1000, 4096, 32
    w = synth.int4(M, K, gs, 406, zero_max=255)
    b = synth.x_f32(K, 407).reshape(K, 1)
    y = np.asarray(run_int4(lib, w, b, M, K, 1, gs), np.float64).reshape(-1)
    assert rel_err(y, np.asarray(orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, 1, gs)).reshape(-1)) <= TOL
    exact = synth.int4_dense(w, gs) @ np.asarray(b, np.float64).reshape(-1)
    assert rel_err(y, exact) <= 1e-6


@pytest.mark.parametrize("batch", [1, 3])
def test_int4_rmul_large_zero_points(lib, orc, batch):
    """uint8 zero points up to 255 (the 16-byte-load kernel takes sum t (8 + zero) off at the end) and
    activations of mixed sign, against the oracle and the fp64 product."""
    inf, outf, gs = 2048, 1024, 64
    w = synth.int4(inf, outf, gs, 404 + batch, zero_max=255)
    x = synth.x_f32(batch * inf, 405 + batch).reshape(batch, inf)
    y = np.asarray(run_rmul(lib, w, x, batch, inf, outf, gs), np.float64).reshape(batch, outf)
    ref = np.asarray(orc.gemm_int4_f32_rmul(w.packed, x, w.scales, w.zeros, batch, inf, outf, gs)).reshape(batch, outf)
    assert rel_err(y, ref) <= TOL
    exact = np.asarray(x, np.float64) @ synth.int4_dense(w, gs)
    for b in range(batch):
        assert rel_err(y[b], exact[b]) <= 1e-6, b


def test_int4_rmul_repeat_bit_identical(lib):
    """The X W kernels sum in a fixed order: two calls give the same bits."""
    for batch, inf, outf, gs in [(1, 4096, 4096, 32), (4, 2048, 1024, 128), (3, 1000, 1002, 7)]:
        w = synth.int4(inf, outf, gs, 402 + batch, zero_max=15)
        x = synth.x_f32(batch * inf, 403 + batch).reshape(batch, inf)
        a = run_rmul(lib, w, x, batch, inf, outf, gs)
        b = run_rmul(lib, w, x, batch, inf, outf, gs)
        assert np.array_equal(np.asarray(a).view(np.uint32), np.asarray(b).view(np.uint32)), (batch, inf, outf)


INT8_CASES = [  # M, K, N
    (4096, 4096, 1), (4096, 14336, 1), (4096, 4096, 4), (1, 16, 1), (333, 1024, 3),
    (7, 33, 1), (1000, 1000, 3), (256, 512, 64), (100, 4096, 17), (65, 1, 65), (64, 4112, 2), (31, 8208, 4),
    (200, 4128, 130), (129, 32, 6),
    (31, 20496, 1), (9, 33040, 1), (2049, 16, 1), (3, 32768, 1),
    # batches 2-4 on 8192 rows: 4 rows a wave of the LDS-staged kernel, a partial last 4096-K chunk
    (8192, 4112, 2), (8192, 4112, 3), (8192, 4112, 4),
]


@pytest.mark.parametrize("M,K,N", INT8_CASES)
def test_int8(lib, orc, M, K, N):
    say(f"int8 M={M} K={K} N={N}")
    a = synth.int8(M, K, 500 + M + K)
    b = synth.x_f32(K * N, 501 + N).reshape(K, N)
    y = run_int8(lib, a, b, M, K, N)
    assert rel_err(y, orc.gemm_int8_f32(a, b, M, K, N)) <= TOL


@pytest.mark.parametrize("zmax", [255, 0])
def test_int4_nt_zero_points_full_range(lib, orc, zmax):
    """uint8 zero points up to 255 (v - z down to -263) and all zero, on the
    bf16 MFMA GEMM, whose int4 operand is 128 + (v ^ 8) with the offset
    136 + z applied through an all-ones product."""
    M, K, N, gs = 256, 1024, 32, 64
    say(f"int4 zeros<={zmax}")
    w = synth.int4(M, K, gs, 320 + zmax, zero_max=zmax)
    b = synth.x_f32(K * N, 321).reshape(K, N)
    y = run_int4(lib, w, b, M, K, N, gs)
    assert rel_err(y, orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, N, gs)) <= TOL


@pytest.mark.parametrize("zmax", [0, 15, 255])
def test_int4_bf16_per_element_error(lib, orc, zmax):
    """Each output of the bf16 MFMA GEMM against the exact product,
    relative to that output's own sum of |w x| (not to max |y|, which hides
    small outputs), beside the same measure of the reference's fp32 loop
    (the oracle).  The int4 operand is 136 + v and the offset (136 + z) sum(x)
    comes off once per 32-K step, so each step's fp32 sums are about
    (272 + z) / |v - z| times larger than the step's result."""
    M, K, N, gs = 512, 4096, 32, 128
    w = synth.int4(M, K, gs, 330 + zmax, zero_max=zmax)
    b = synth.x_f32(K * N, 331).reshape(K, N)
    y = run_int4(lib, w, b, M, K, N, gs).reshape(M, N).astype(np.float64)
    W = synth.int4_dense(w, gs).astype(np.float64).reshape(M, K)
    exact = W @ b.astype(np.float64)
    mag = np.abs(W) @ np.abs(b.astype(np.float64))
    ref = np.asarray(orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, N, gs), np.float64).reshape(M, N)
    ours = float(np.max(np.abs(y - exact) / mag))
    theirs = float(np.max(np.abs(ref - exact) / mag))
    say(f"int4 bf16 zmax={zmax}: per-element |y - exact| / sum|w x|: {ours:.3e} (reference loop {theirs:.3e})")
    # measured 3.8e-7 / 1.6e-7 / 3.9e-8 against the loop's 2.2e-7 / 2.9e-7 / 2.0e-7 (z <= 0 / 15 / 255)
    assert ours <= 1e-6 and ours <= 4 * theirs


@pytest.mark.parametrize("fmt", ["int4", "int8", "rmul"])
def test_reference_benchmark_square_1024(lib, orc, fmt):
    """The reference benchmark's 1024-cubed GEMM on random operands, every
    output against the oracle."""
    n = 1024
    say(f"{fmt} square {n}")
    x = synth.x_f32(n * n, 600).reshape(n, n)
    if fmt == "int4":
        w = synth.int4(n, n, 32, 601)
        assert rel_err(run_int4(lib, w, x, n, n, n, 32), orc.gemm_int4_f32(w.packed, x, w.scales, w.zeros, n, n, n,
                                                                           32, threads=16)) <= TOL
    elif fmt == "rmul":
        w = synth.int4(n, n, 32, 602)
        assert rel_err(run_rmul(lib, w, x, n, n, n, 32), orc.gemm_int4_f32_rmul(w.packed, x, w.scales, w.zeros, n, n,
                                                                                n, 32, threads=16)) <= TOL
    else:
        a = synth.int8(n, n, 603)
        assert rel_err(run_int8(lib, a, x, n, n, n), orc.gemm_int8_f32(a, x, n, n, n, threads=16)) <= TOL


@pytest.mark.parametrize("fmt", ["int4", "int8"])
def test_reference_benchmark_square_4096_sampled_rows(lib, orc, fmt):
    """4096 cubed on random operands; the oracle runs the first and last 8
    rows of A (all K, all N) against the same rows of the GPU result."""
    n = 4096
    say(f"{fmt} square {n}")
    x = synth.x_f32(n * n, 610).reshape(n, n)
    rows = np.r_[0:8, n - 8:n]
    if fmt == "int4":
        w = synth.int4(n, n, 32, 611)
        y = run_int4(lib, w, x, n, n, n, 32).reshape(n, n)
        ref = orc.gemm_int4_f32(w.packed[rows], x, w.scales[rows], w.zeros[rows], len(rows), n, n, 32, threads=16)
    else:
        a = synth.int8(n, n, 612)
        y = run_int8(lib, a, x, n, n, n).reshape(n, n)
        ref = orc.gemm_int8_f32(a[rows], x, len(rows), n, n, threads=16)
    assert rel_err(y[rows].reshape(-1), ref) <= TOL
    assert np.isfinite(y).all()


def test_reference_benchmark_inputs_4096_every_output(lib):
    """gemm_bench_test.go's inputs at 4096 cubed (int4: bytes 0x53, scale 0.1,
    zero 0, group 32; int8: bytes 42; activations 0.01).  Every term of a sum
    is equal and positive, so the rounding errors of any fp32 summation order
    add up instead of cancelling: the reference kernel's sequential FMA chain
    (replayed exactly in long double) ends 2.0e-5 above the exact sum, and a
    different order may land on the other side.  The bar for these inputs is
    therefore the summation bound K * 2^-24 (2.4e-4), against both the chain
    and the exact value; the random-operand tests above keep 1e-5."""
    n = 4096
    bound = n * 2.0 ** -24
    say("benchmark inputs 4096")
    x = np.full((n, n), 0.01, np.float32)
    w = synth.Int4Weights(np.zeros((1, 1), np.int8), np.full((n, n // 2), 0x53, np.uint8),
                          np.full((n, n // 32), 0.1, np.float32), np.zeros((n, n // 32), np.uint8))
    y = run_int4(lib, w, x, n, n, n, 32)
    dq = [np.float32(np.float32(3) * np.float32(0.1)), np.float32(np.float32(5) * np.float32(0.1))]
    acc = np.float32(0.0)
    for k in range(n):
        acc = np.float32(np.longdouble(acc) + np.longdouble(dq[k & 1]) * np.longdouble(np.float32(0.01)))
    exact = n // 2 * (np.float64(dq[0]) + np.float64(dq[1])) * np.float64(np.float32(0.01))
    assert rel_err(y, np.full(n * n, acc)) <= bound
    assert rel_err(y, np.full(n * n, exact)) <= bound
    assert np.all(y == y[0])  # every output is the same sum
    y8 = run_int8(lib, np.full((n, n), 42, np.int8), x, n, n, n)
    acc8 = np.float32(0.0)
    for _ in range(n):
        acc8 = np.float32(np.longdouble(acc8) + np.longdouble(42) * np.longdouble(np.float32(0.01)))
    exact8 = n * 42 * np.float64(np.float32(0.01))
    assert rel_err(y8, np.full(n * n, acc8)) <= bound
    assert rel_err(y8, np.full(n * n, exact8)) <= bound
    assert np.all(y8 == y8[0])


def test_zero_k_writes_zeros_and_empty_calls(lib):
    c = torch.full((12,), float("nan"), dtype=torch.float32, device="cuda")
    t = torch.zeros(64, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    assert lib.zt_gemm_int8_f32(p, p, c.data_ptr(), 3, 0, 4, stream()) == 0
    torch.cuda.synchronize()
    assert not c.cpu().numpy().any()
    c.fill_(float("nan"))
    assert lib.zt_gemm_int4_f32(p, p, c.data_ptr(), p, p, 4, 0, 3, 32, stream()) == 0
    torch.cuda.synchronize()
    assert not c.cpu().numpy().any()
    c.fill_(float("nan"))
    assert lib.zt_gemm_int4_f32_rmul(p, p, c.data_ptr(), p, p, 2, 0, 6, 32, stream()) == 0
    torch.cuda.synchronize()
    assert not c.cpu().numpy().any()
    # empty outputs: nothing to do, nothing written
    assert lib.zt_gemm_int8_f32(p, p, p, 0, 16, 4, stream()) == 0
    assert lib.zt_gemm_int4_f32(p, p, p, p, p, 4, 32, 0, 32, stream()) == 0
    assert lib.zt_gemm_int4_f32_rmul(p, p, p, p, p, 0, 32, 64, 32, stream()) == 0


def test_repeated_calls_bit_identical(lib):
    M, K, N, gs = 1000, 1000, 40, 20
    w = synth.int4(M, K, gs, 700)
    b = synth.x_f32(K * N, 701).reshape(K, N)
    y1 = run_int4(lib, w, b, M, K, N, gs)
    y2 = run_int4(lib, w, b, M, K, N, gs)
    assert np.array_equal(y1.view(np.uint32), y2.view(np.uint32))
