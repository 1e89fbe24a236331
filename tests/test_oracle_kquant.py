"""Pins the oracle's K-quant (Q4_K, Q5_K, Q6_K) and Q5_0 functions.

The dequantizers are checked against weights written by the packers in
ztensor_amd/synth.py, which follow the reference's *test-side* block builders
(tensor/quantized_kquant_test.go:11-128, 217-292, 366-468) - code written in
the opposite direction from the dequantizers - from known integer codes, so
a wrong bit position, nibble half, sub-block index or qh bit fails.  The
expected values are the formats' element definitions evaluated in numpy fp32
with the reference's rounding order.  The reference's own round-trip tests
(quantize with the test builder, dequantize, compare within its stated
tolerance) are ported too, and the GEMVs are checked against fp64 brute
force and for thread-count invariance.
"""
import numpy as np
import pytest

from ztensor_amd import synth

F = np.float32


def _codes(fmt, nsb, seed):
    g = np.random.default_rng(seed)
    hi = {"q4_k": 16, "q5_k": 32}[fmt]
    q = g.integers(0, hi, size=(nsb, 256), dtype=np.uint8)
    sc = g.integers(0, 64, size=(nsb, 8), dtype=np.uint8)
    mn = g.integers(0, 64, size=(nsb, 8), dtype=np.uint8)
    d = synth.f16_bits(np.abs(g.standard_normal(nsb)).astype(F) * F(0.01))
    dmin = synth.f16_bits(np.abs(g.standard_normal(nsb)).astype(F) * F(0.005))
    return q, sc, mn, d, dmin


def _expect_q45k(q, sc, mn, d, dmin):
    """value v of a super-block: (d*sc[s])*q[v] - dmin*mn[s], s = sub-block
    2*(v//64) + (v%64 >= 32) (tensor/quantized_kquant.go:54-79, 509-549)."""
    nsb = q.shape[0]
    v = np.arange(256)
    s = 2 * (v // 64) + ((v % 64) >= 32)
    dd = d.view(np.float16).astype(F)[:, None]
    dm = dmin.view(np.float16).astype(F)[:, None]
    scl = (dd * sc[:, s].astype(F)).astype(F)
    mnl = (dm * mn[:, s].astype(F)).astype(F)
    return ((scl * q.astype(F)).astype(F) - mnl).astype(F).reshape(nsb * 256)


def test_kq_scales_mins_unpack_inverts_the_test_builders_packing(orc):
    g = np.random.default_rng(3)
    for _ in range(200):
        sc = g.integers(0, 64, 8, dtype=np.uint8)
        mn = g.integers(0, 64, 8, dtype=np.uint8)
        blk = np.zeros(16, np.uint8)
        blk[4:16] = synth.pack_kq_scales_mins(sc[None], mn[None])[0]
        got_sc, got_mn = orc.kq_scales_mins(blk)
        assert np.array_equal(got_sc, sc) and np.array_equal(got_mn, mn)


@pytest.mark.parametrize("fmt", ["q4_k", "q5_k"])
def test_q4k_q5k_dequant_from_known_codes_is_bit_exact(orc, fmt):
    q, sc, mn, d, dmin = _codes(fmt, 24, 11 if fmt == "q4_k" else 12)
    pack = synth.pack_q4_k if fmt == "q4_k" else synth.pack_q5_k
    raw = pack(q, sc, mn, d, dmin)
    assert raw.size == 24 * (144 if fmt == "q4_k" else 176)
    got = orc.kq_dequant(fmt, raw, 24 * 256)
    want = _expect_q45k(q, sc, mn, d, dmin)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q5k_fifth_bit_moves_exactly_one_value_by_16_steps(orc):
    # A qh bit at the wrong position would move a different element.
    q, sc, mn, d, dmin = _codes("q5_k", 1, 5)
    q &= 0xF
    base = orc.kq_dequant("q5_k", synth.pack_q5_k(q, sc, mn, d, dmin), 256)
    for v in (0, 31, 32, 63, 64, 100, 191, 255):
        q2 = q.copy()
        q2[0, v] |= 16
        got = orc.kq_dequant("q5_k", synth.pack_q5_k(q2, sc, mn, d, dmin), 256)
        diff = np.nonzero(got != base)[0]
        s = 2 * (v // 64) + ((v % 64) >= 32)
        if sc[0, s] == 0:
            assert diff.size == 0
        else:
            assert diff.tolist() == [v]


def test_q6k_dequant_from_known_codes_is_bit_exact(orc):
    g = np.random.default_rng(13)
    nsb = 24
    q = g.integers(0, 64, size=(nsb, 256), dtype=np.uint8)
    sc = g.integers(-128, 128, size=(nsb, 16), dtype=np.int16).astype(np.int8)
    d = synth.f16_bits(np.abs(g.standard_normal(nsb)).astype(F) * F(0.001))
    raw = synth.pack_q6_k(q, sc, d)
    assert raw.size == nsb * 210
    got = orc.kq_dequant("q6_k", raw, nsb * 256)
    # value v uses scale v // 16 (tensor/quantized_kquant.go:355-382): (d * sc) * (q - 32)
    v = np.arange(256)
    dd = d.view(np.float16).astype(F)[:, None]
    want = ((dd * sc[:, v // 16].astype(F)).astype(F) * (q.astype(F) - F(32))).astype(F).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_q5_0_dequant_from_known_codes_is_bit_exact(orc):
    g = np.random.default_rng(14)
    nblk = 96
    q = g.integers(0, 32, size=(nblk, 32), dtype=np.uint8)
    d = synth.f16_bits(g.standard_normal(nblk).astype(F) * F(0.02))
    raw = synth.pack_q5_0(q, d)
    got = orc.q5_0_dequant(raw, nblk * 32)
    want = (d.view(np.float16).astype(F)[:, None] * (q.astype(F) - F(16))).astype(F).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ---- the reference's own round-trip tests, ported --------------------------

def _build_q4k_block(values):
    """tensor/quantized_kquant_test.go:11-128 buildQ4KBlock in numpy
    (fp16 rounding by numpy RNE; only the tolerance check depends on it)."""
    v = values.astype(F).reshape(8, 32)
    mnv = np.minimum(v.min(1), 0).astype(F)
    sub_sc = ((v.max(1) - mnv) / F(15)).astype(F)
    sub_mn = (-mnv).astype(F)
    d = F(sub_sc.max() / F(63))
    dmin = F(sub_mn.max() / F(63))
    scq = np.zeros(8, np.uint8) if d == 0 else np.minimum(np.round(sub_sc / d), 63).astype(np.uint8)
    mnq = np.zeros(8, np.uint8) if dmin == 0 else np.minimum(np.round(sub_mn / dmin), 63).astype(np.uint8)
    d16, dmin16 = synth.f16_bits(d), synth.f16_bits(dmin)
    df, dminf = d16.view(np.float16).astype(F), dmin16.view(np.float16).astype(F)
    q = np.zeros(256, np.uint8)
    for s in range(8):
        scf = F(df * F(scq[s]))
        mnf = F(dminf * F(mnq[s]))
        inv = F(1) / scf if scf > 0 else F(0)
        q[32 * s:32 * s + 32] = np.clip(np.round(((v[s] + mnf) * inv).astype(np.float64)), 0, 15)
    # values are in natural order 0..255 = group 2g (first 32) / 2g+1 (next 32)
    return synth.pack_q4_k(q[None], scq[None], mnq[None], np.array([d16]), np.array([dmin16]))


def test_q4k_roundtrip_sine_within_reference_tolerance(orc):
    # TestDequantizeQ4K_RoundTrip: sin(0.1 i) * 2, max error <= 0.6.
    values = (np.sin(np.arange(256) * 0.1) * 2.0).astype(F)
    got = orc.kq_dequant("q4_k", _build_q4k_block(values), 256)
    assert np.abs(got - values).max() <= 0.6


def test_q4k_roundtrip_ramp_within_reference_tolerance(orc):
    # TestNewQ4KStorageFromRaw: i * 0.01, max error <= 0.3.
    values = (np.arange(256) * 0.01).astype(F)
    got = orc.kq_dequant("q4_k", _build_q4k_block(values), 256)
    assert np.abs(got - values).max() <= 0.3


@pytest.mark.parametrize("fmt,nbytes", [("q4_k", 144), ("q5_k", 176), ("q6_k", 210)])
def test_kquant_zero_block_dequantizes_to_zero(orc, fmt, nbytes):
    # TestDequantizeQ4K_Zeros / Q6K_Zeros: an all-zero block (d = dmin = 0).
    got = orc.kq_dequant(fmt, np.zeros(2 * nbytes, np.uint8), 512)
    assert np.all(got == 0)


@pytest.mark.parametrize("fmt", ["q4_k", "q5_k", "q6_k"])
def test_kquant_partial_last_superblock(orc, fmt):
    w = synth.kquant(fmt, 1, 768, 21)
    full = orc.kq_dequant(fmt, w.raw, 768)
    part = orc.kq_dequant(fmt, w.raw, 700)
    assert np.array_equal(part, full[:700])


def test_q5_0_partial_last_block(orc):
    w = synth.kquant("q5_0", 1, 96, 22)
    full = orc.q5_0_dequant(w.raw, 96)
    assert np.array_equal(orc.q5_0_dequant(w.raw, 70), full[:70])


# ---- GEMVs -------------------------------------------------------------------

@pytest.mark.parametrize("fmt", ["q4_k", "q5_k", "q6_k"])
def test_kquant_gemv_matches_fp64_bruteforce(orc, fmt):
    rows, K = 48, 1024
    w = synth.kquant(fmt, rows, K, 31)
    x = synth.x_f32(2 * K, 31)
    y = orc.gemm_f32_kq_nt(fmt, x, w.raw, 2, rows, K)
    W = orc.kq_dequant(fmt, w.raw, rows * K).reshape(rows, K).astype(np.float64)
    ref = x.reshape(2, K).astype(np.float64) @ W.T
    assert np.abs(y.reshape(2, rows) - ref).max() <= 1e-5 * np.abs(ref).max()


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_kquant_gemv_thread_split_is_bit_identical(orc, fmt):
    rows, K = 256, 1024
    w = synth.kquant(fmt, rows, K, 32)
    x = synth.x_f32(K, 32)
    a = orc.gemm_f32_kq_nt(fmt, x, w.raw, 1, rows, K, threads=1)
    b = orc.gemm_f32_kq_nt(fmt, x, w.raw, 1, rows, K, threads=8)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_kquant_gemv_sums_in_element_order(orc):
    # One row: the GEMV equals the sequential fp32 sum of x[p] * w[p], p = 0..K-1.
    w = synth.kquant("q4_k", 1, 512, 33)
    x = synth.x_f32(512, 33)
    deq = orc.kq_dequant("q4_k", w.raw, 512)
    s = F(0)
    for p in range(512):
        s = F(s + F(x[p] * deq[p]))
    got = orc.gemm_f32_kq_nt("q4_k", x, w.raw, 1, 1, 512)
    assert got[0] == s


def test_q5_0_gpu_layout_matches_reference_test_converter(orc):
    # internal/cuda/kernels/gemv_q5_0_test.go:13-33 q5_0ToGPULayout, restated.
    nblk = 37
    w = synth.kquant("q5_0", 1, 32 * nblk, 23)
    raw = w.raw.reshape(nblk, 22)
    sb = (nblk * 2 + 15) & ~15
    qb = (nblk * 4 + 15) & ~15
    want = np.zeros(sb + qb + 16 * nblk, np.uint8)
    for i in range(nblk):
        want[2 * i:2 * i + 2] = raw[i, 0:2]
        want[sb + 4 * i:sb + 4 * i + 4] = raw[i, 2:6]
        want[sb + qb + 16 * i:sb + qb + 16 * i + 16] = raw[i, 6:22]
    got = orc.q5_0_raw_to_gpu(w.raw, nblk)
    assert np.array_equal(got, want)
    lib = orc.lib()
    assert lib.orc_q5_0_gpu_qh_offset(nblk) == sb
    assert lib.orc_q5_0_gpu_qs_offset(nblk) == sb + qb


def test_q5_0_matmul_matches_fp64_bruteforce(orc):
    rows, K = 40, 512
    w = synth.kquant("q5_0", rows, K, 24)
    x = synth.x_f32(K, 24)
    y = orc.gemm_f32_q5_0_nt(x, w.raw, 1, rows, K)
    W = orc.q5_0_dequant(w.raw, rows * K).reshape(rows, K).astype(np.float64)
    ref = W @ x.astype(np.float64)
    assert np.abs(y - ref).max() <= 1e-5 * np.abs(ref).max()


# ---- GGUF mmap ---------------------------------------------------------------

def test_gguf_q8_0_dequant_from_known_codes_is_bit_exact(orc):
    g = np.random.default_rng(41)
    q = g.integers(-128, 128, size=(50, 32), dtype=np.int16).astype(np.int8)
    d = synth.f16_bits(g.standard_normal(50).astype(F) * F(0.02))
    raw = synth.pack_gguf_q8_0(q, d)
    assert raw.size == 50 * 34
    got = orc.gguf_q8_0_dequant(raw, 50 * 32)
    want = (q.astype(F) * d.view(np.float16).astype(F)[:, None]).astype(F).reshape(-1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # partial last block
    assert np.array_equal(orc.gguf_q8_0_dequant(raw, 50 * 32 - 7), got[:-7])


@pytest.mark.parametrize("qtype,fmt", [(12, "q4_k"), (13, "q5_k"), (14, "q6_k")])
def test_mmap_gemv_kquants_equal_the_storage_gemvs(orc, qtype, fmt):
    # GemmF32MmapNT streams super-blocks exactly as GemmF32Q{4,5,6}KNT do.
    rows, K = 20, 768
    w = synth.kquant(fmt, rows, K, 42)
    x = synth.x_f32(K, 42)
    a = orc.gemm_f32_mmap_nt(qtype, x, w.raw, 1, rows, K)
    b = orc.gemm_f32_kq_nt(fmt, x, w.raw, 1, rows, K)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


@pytest.mark.parametrize("qtype", [2, 6, 8])
def test_mmap_gemv_dequantizing_types_match_fp64(orc, qtype):
    rows, K = 24, 512
    if qtype == 2:
        raw = synth.q4_0(rows, K, 43).raw
        W = orc.q4_dequant(raw, rows * K)
    elif qtype == 6:
        raw = synth.kquant("q5_0", rows, K, 43).raw
        W = orc.q5_0_dequant(raw, rows * K)
    else:
        raw = synth.gguf_q8_0(rows, K, 43)
        W = orc.gguf_q8_0_dequant(raw, rows * K)
    x = synth.x_f32(2 * K, 43)
    y = orc.gemm_f32_mmap_nt(qtype, x, raw, 2, rows, K)
    ref = x.reshape(2, K).astype(np.float64) @ W.reshape(rows, K).astype(np.float64).T
    assert np.abs(y.reshape(2, rows) - ref).max() <= 1e-5 * np.abs(ref).max()


def test_mmap_gemv_rejects_types_without_a_kernel(orc):
    with pytest.raises(ValueError):
        orc.gemm_f32_mmap_nt(3, np.zeros(32, np.float32), np.zeros(20, np.uint8), 1, 1, 32)
