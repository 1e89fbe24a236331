"""The oracle's int4 / int8 GEMMs (orc_gemm_int4_f32, orc_gemm_int4_f32_rmul,
orc_gemm_int8_f32), restating internal/cuda/kernels/gemm_int4.cu:20-144 and
gemm_int8.cu:16-73, pinned on the CPU.

Pins (the reference's tests hold no known answers for these kernels, only
the benchmark inputs of internal/cuda/kernels/gemm_bench_test.go:46-157):
  * sign extension: every nibble value 0..15 through a one-hot product maps
    to v - 16 for v >= 8, which a kernel that forgot it (or read the high
    nibble first) fails;
  * the benchmark inputs bit for bit: bytes 0x53 (values 3, 5), scale 0.1,
    zero 0, activations 0.01, and int8 bytes 42, against the fp32 FMA chain
    of the reference kernel's k loop replayed exactly in long double;
  * float64 brute force on independent numpy unpacking (pack_int4 /
    int4_dense), with group sizes that do and do not divide K (or out), for
    the NT and the right-multiply forms, zero points up to 255;
  * small integers: int8 weights and activations of small integers are
    exact in fp32, so the result equals the integer product exactly;
  * the launchers' errors: odd K / odd out_features, group_size <= 0.
"""
import numpy as np
import pytest

from ztensor_amd import synth


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def test_int4_sign_extension_every_nibble(orc):
    # one row, K = 16: elements 0..15 hold nibble values 0..15 as stored
    nib = np.arange(16, dtype=np.uint8)
    packed = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8).reshape(1, 8)
    b = np.eye(16, dtype=np.float32)  # B [K, N] = identity: C[0, j] = w_j
    c = orc.gemm_int4_f32(packed, b, np.ones((1, 1), np.float32), np.zeros((1, 1), np.uint8), 1, 16, 16, 16)
    want = np.where(nib >= 8, nib.astype(np.int32) - 16, nib.astype(np.int32)).astype(np.float32)
    assert np.array_equal(c, want)
    # the same through the right-multiply form: W [16, 16/2] with w[k, j] = value of nibble j
    w = np.repeat(packed, 16, axis=0)
    x = np.eye(16, dtype=np.float32)  # X [batch, in] = identity
    cr = orc.gemm_int4_f32_rmul(w, x, np.ones((16, 1), np.float32), np.zeros((16, 1), np.uint8), 16, 16, 16, 16)
    assert np.array_equal(cr.reshape(16, 16), np.tile(want, (16, 1)))


def fma_chain(terms) -> np.float32:
    """acc = fmaf(a, b, acc) over (a, b) pairs in order: a*b and acc + a*b
    are exact in the 64-bit long double mantissa for these operands (at most
    48 + 10 bits), so each step rounds once, to fp32, as an FMA does."""
    acc = np.float32(0.0)
    for a, b in terms:
        acc = np.float32(np.longdouble(acc) + np.longdouble(a) * np.longdouble(b))
    return acc


@pytest.mark.parametrize("K", [32, 1024])
def test_benchmark_inputs_exact_fma_chain(orc, K):
    """gemm_bench_test.go's inputs; every output is the fp32 FMA chain of
    the reference kernel's k loop, bit for bit."""
    assert np.finfo(np.longdouble).nmant >= 63
    M, N, gs = 8, 4, 32
    a = np.full((M, K // 2), 0x53, np.uint8)
    b = np.full((K, N), 0.01, np.float32)
    s = np.full((M, K // gs), 0.1, np.float32)
    z = np.zeros((M, K // gs), np.uint8)
    c = orc.gemm_int4_f32(a, b, s, z, M, K, N, gs)
    dq = [np.float32(np.float32(3) * np.float32(0.1)), np.float32(np.float32(5) * np.float32(0.1))]
    want = fma_chain((dq[k & 1], np.float32(0.01)) for k in range(K))
    assert np.array_equal(c, np.full(M * N, want, np.float32))
    i8 = np.full((M, K), 42, np.int8)
    c8 = orc.gemm_int8_f32(i8, b, M, K, N)
    want8 = fma_chain((np.float32(42), np.float32(0.01)) for _ in range(K))
    assert np.array_equal(c8, np.full(M * N, want8, np.float32))


@pytest.mark.parametrize("M,K,N,gs", [(5, 64, 3, 32), (7, 96, 2, 40), (3, 30, 4, 7), (1, 256, 1, 256), (4, 2, 5, 1)])
def test_int4_nt_float64_brute_force(orc, M, K, N, gs):
    w = synth.int4(M, K, gs, 17 + K, zero_max=255)
    b = synth.x_f32(K * N, 18 + K).reshape(K, N)
    c = orc.gemm_int4_f32(w.packed, b, w.scales, w.zeros, M, K, N, gs)
    ref = synth.int4_dense(w, gs) @ b.astype(np.float64)
    assert rel_err(c, ref.reshape(-1)) <= 1e-6


@pytest.mark.parametrize("batch,inf,outf,gs", [(3, 64, 32, 16), (2, 50, 30, 7), (1, 128, 256, 128), (4, 9, 2, 1)])
def test_int4_rmul_float64_brute_force(orc, batch, inf, outf, gs):
    w = synth.int4(inf, outf, gs, 21 + outf, zero_max=255)  # groups along out
    x = synth.x_f32(batch * inf, 22 + inf).reshape(batch, inf)
    c = orc.gemm_int4_f32_rmul(w.packed, x, w.scales, w.zeros, batch, inf, outf, gs)
    ref = x.astype(np.float64) @ synth.int4_dense(w, gs)
    assert rel_err(c, ref.reshape(-1)) <= 1e-6


def test_int8_small_integers_exact_and_brute_force(orc):
    M, K, N = 9, 77, 5
    g = np.random.default_rng(3)
    a = g.integers(-128, 128, size=(M, K), dtype=np.int8)
    b = g.integers(-20, 21, size=(K, N)).astype(np.float32)
    c = orc.gemm_int8_f32(a, b, M, K, N)
    assert np.array_equal(c, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32).reshape(-1))
    bf = synth.x_f32(K * N, 5).reshape(K, N)
    cf = orc.gemm_int8_f32(a, bf, M, K, N)
    assert rel_err(cf, (a.astype(np.float64) @ bf.astype(np.float64)).reshape(-1)) <= 1e-6


def test_launcher_errors(orc):
    z1, s1 = np.zeros((1, 1), np.uint8), np.ones((1, 1), np.float32)
    with pytest.raises(ValueError):
        orc.gemm_int4_f32(np.zeros((1, 1), np.uint8), np.zeros(3, np.float32), s1, z1, 1, 3, 1, 32)
    with pytest.raises(ValueError):
        orc.gemm_int4_f32(np.zeros((1, 1), np.uint8), np.zeros(2, np.float32), s1, z1, 1, 2, 1, 0)
    with pytest.raises(ValueError):
        orc.gemm_int4_f32_rmul(np.zeros((1, 2), np.uint8), np.zeros(1, np.float32), s1, z1, 1, 1, 3, 32)
    with pytest.raises(ValueError):
        orc.gemm_int4_f32_rmul(np.zeros((1, 1), np.uint8), np.zeros(1, np.float32), s1, z1, 1, 1, 2, -1)
