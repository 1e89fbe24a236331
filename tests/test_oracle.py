"""Pins the CPU oracle (oracle/zt_oracle.c) before it is trusted as the checker.

Each oracle function is checked against at least one thing that does not
restate it: the reference's own known-answer tests (tests/golden/*.json,
transcribed from the reference test files cited there), IEEE/numpy for fp16,
closed forms and special cases, brute-force fp64 products, exact integer
arithmetic, round trips through independent quantizers, and cross-checks
between two oracle functions that must agree.  A plausible slip - a swapped
nibble order, a dropped -8 / zero-point, a sign error, a transposed operand,
an off-by-one in the tail - fails at least one test here.
"""
import json
from pathlib import Path

import numpy as np
import pytest

from ztensor_amd import synth

GOLD = Path(__file__).resolve().parent / "golden"


def f16(v):
    return synth.f16_bits(np.float32(v))


# ------------------------------------------------------------------ fp16


def test_f16_widening_matches_ieee_for_all_bit_patterns(orc):
    bits = np.arange(65536, dtype=np.uint16)
    got = orc.f16_to_f32(bits)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_xblas_f16_decoder_is_ieee_for_finite_and_zero_for_inf_nan(orc):
    # internal/xblas/q4dot.go:53-78: Inf/NaN -> 0, everything else IEEE.
    lib = orc.lib()
    for b in list(range(0, 65536, 97)) + [0x0001, 0x03FF, 0x8001, 0x7C00, 0xFC00, 0x7E00, 0x7BFF]:
        v = np.uint16(b).view(np.float16).astype(np.float32)
        got = np.float32(lib.orc_f16_bits_to_f32_xblas(b))
        if not np.isfinite(v):
            assert got == 0.0
        else:
            assert got.view(np.uint32) == v.view(np.uint32), hex(b)


# ------------------------------------------------------------------ Q4_0


def quantize_q4(src: np.ndarray) -> np.ndarray:
    """QuantizeQ4 (tensor/quantized.go:37-91) restated in numpy -> 18-byte blocks."""
    n = src.size
    nblk = (n + 31) // 32
    x = np.zeros(nblk * 32, np.float32)
    x[:n] = src
    x = x.reshape(nblk, 32)
    absmax = np.abs(x).max(axis=1)
    scale = np.where(absmax > 0, absmax / np.float32(7.0), 0).astype(np.float32)
    d = synth.f16_bits(scale)
    inv = np.where(scale > 0, np.float32(1.0) / np.where(scale > 0, scale, 1), 0).astype(np.float32)
    q = np.clip(np.round((x * inv[:, None]).astype(np.float64)), -8, 7).astype(np.int64) + 8
    return synth.pack_q4_0(q.astype(np.uint8), d)


def test_q4_dequant_roundtrip_through_independent_quantizer(orc):
    # A swapped nibble order (interleaved instead of split) or a missing -8
    # shows up as errors of the order of the block absmax.
    rng = np.random.default_rng(1)
    src = rng.standard_normal(64 * 32).astype(np.float32)
    raw = quantize_q4(src)
    got = orc.q4_dequant(raw, src.size)
    scale = synth.f16_bits(np.abs(src.reshape(-1, 32)).max(1) / np.float32(7)).view(np.float16).astype(np.float32)
    err = np.abs(got - src).reshape(-1, 32).max(1)
    assert np.all(err <= scale * 0.5 + 1e-3 * scale + 1e-6)


def test_q4_dequant_closed_form_and_registry_pattern(orc):
    # tensor/quant_registry_test.go:169-202 input (i-32)/32 over 64 elements.
    src = (np.arange(64, dtype=np.float32) - 32) / np.float32(32)
    raw = quantize_q4(src)
    got = orc.q4_dequant(raw, 64)
    blk = raw.reshape(2, 18)
    for b in range(2):
        d = blk[b, :2].view("<u2")[0:1].view(np.float16).astype(np.float32)[0]
        for j in range(16):
            lo, hi = blk[b, 2 + j] & 15, blk[b, 2 + j] >> 4
            assert got[32 * b + j] == np.float32(np.float32(int(lo) - 8) * d)
            assert got[32 * b + j + 16] == np.float32(np.float32(int(hi) - 8) * d)


def test_q4_partial_last_block(orc):
    raw = quantize_q4(np.linspace(-1, 1, 40).astype(np.float32))
    full = orc.q4_dequant(raw, 64)
    part = orc.q4_dequant(raw, 40)
    assert np.array_equal(part, full[:40])


def test_q4_raw_to_gpu_layout(orc):
    # tensor/quantized.go:168-198: [scales][pad to 16][data]; offsets pinned by hand.
    for nblk, off in [(1, 16), (7, 16), (8, 16), (9, 32), (128, 256)]:
        assert orc.lib().orc_q4_gpu_data_offset(nblk) == off
    w = synth.q4_0(3, 96, 5)
    nblk = 9
    gpu = orc.q4_raw_to_gpu(w.raw, nblk)
    blocks = w.raw.reshape(nblk, 18)
    assert np.array_equal(gpu[: 2 * nblk].reshape(nblk, 2), blocks[:, :2])
    assert np.array_equal(gpu[32:].reshape(nblk, 16), blocks[:, 2:])
    assert not gpu[2 * nblk:32].any()


def test_q4dot_block_reference_known_answers(orc):
    # internal/xblas/q4dot_test.go:11-140 (tolerances from the test itself).
    for case in json.loads((GOLD / "q4dot_cases.json").read_text()):
        nib = np.array(case["nibbles"], np.uint8)
        packed = (nib[:16] | (nib[16:] << 4)).astype(np.uint8)
        x = np.array(case["x"], np.float32)
        got = np.float32(orc.lib().orc_q4_dot_block(packed.ctypes.data, case["scale"], x.ctypes.data, 32))
        want = np.float32(case["want"])
        tol = 1e-5 if abs(want) <= 1 else abs(want) * 1e-6
        assert abs(float(got) - float(want)) <= tol, case["name"]


def test_q4_gemv_matches_fp64_brute_force_and_threads_do_not_change_bits(orc):
    rows, K = 96, 256
    w = synth.q4_0(rows, K, 11)
    x = synth.x_f32(K, 11)
    wd = orc.q4_dequant(w.raw, rows * K).reshape(rows, K).astype(np.float64)
    ref = wd @ x.astype(np.float64)
    y1 = orc.gemm_f32_q4_nt(x, w.raw, 1, rows, K, threads=1)
    y8 = orc.gemm_f32_q4_nt(x, w.raw, 1, rows, K, threads=8)
    assert np.array_equal(y1, y8)
    assert np.max(np.abs(y1 - ref)) <= 1e-5 * np.max(np.abs(ref))
    # M>1 rows of A are independent GEMVs.
    a = np.stack([x, -x, 2 * x])
    y3 = orc.gemm_f32_q4_nt(a, w.raw, 3, rows, K).reshape(3, rows)
    assert np.array_equal(y3[0], y1) and np.array_equal(y3[1], -y1)


# ------------------------------------------------------------------ Q8_0


def quantize_q8(src: np.ndarray) -> np.ndarray:
    """QuantizeQ8 (tensor/quantized.go:301-341) restated -> 36-byte blocks."""
    x = src.reshape(-1, 32).astype(np.float32)
    absmax = np.abs(x).max(axis=1)
    scale = np.where(absmax > 0, absmax / np.float32(127), 0).astype(np.float32)
    inv = np.where(scale > 0, np.float32(1) / np.where(scale > 0, scale, 1), 0).astype(np.float32)
    q = np.clip(np.round((x * inv[:, None]).astype(np.float64)), -128, 127).astype(np.int8)
    return synth.pack_q8_0(q, scale)


def test_q8_dequant_roundtrip_and_closed_form(orc):
    # tensor/quant_registry_test.go:204-229 input (i-32)/16.
    src = (np.arange(64, dtype=np.float32) - 32) / np.float32(16)
    raw = quantize_q8(src)
    got = orc.q8_dequant(raw, 64)
    b = raw.reshape(2, 36)
    for i in range(2):
        s = b[i, :4].view("<f4")[0]
        q = b[i, 4:].view(np.int8)
        assert np.array_equal(got[32 * i:32 * i + 32], (q.astype(np.float32) * s).astype(np.float32))
    assert np.max(np.abs(got - src)) <= 2.0 / 127 * 0.5 + 1e-6
    # negative values keep their sign (int8, not uint8)
    assert got[0] < 0 and got[-1] > 0


def test_q8_gemv_matches_fp64(orc):
    rows, K = 64, 320
    w = synth.q8_0(rows, K, 3)
    x = synth.x_f32(K, 3)
    wd = orc.q8_dequant(w.raw, rows * K).reshape(rows, K).astype(np.float64)
    ref = wd @ x.astype(np.float64)
    y = orc.gemm_f32_q8_nt(x, w.raw, 1, rows, K, threads=4)
    assert np.array_equal(y, orc.gemm_f32_q8_nt(x, w.raw, 1, rows, K, threads=1))
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.max(np.abs(ref))


# ---------------------------------------------------------------- IQ4_NL


def _iq4_block(scale, nib):
    return synth.pack_iq4nl(np.array(nib, np.uint8).reshape(1, 32), f16(scale).reshape(1))


def test_iq4nl_reference_known_answers(orc):
    gold = json.loads((GOLD / "iq4nl_cases.json").read_text())
    T = orc.iq4nl_table()
    # tensor/iq4_storage_test.go:157-175
    assert T[gold["table_zero_index"]] == 0.0 and np.all(np.diff(T) > 0) and T.size == 16
    # :21-42 single block
    sb = gold["single_block"]
    got = orc.iq4nl_dequant(_iq4_block(sb["scale"], sb["nibbles"]), 32)
    want = np.float32(sb["scale"]) * T[np.array(sb["nibbles"])]
    assert np.max(np.abs(got - want)) <= 1e-6
    # :44-84 two blocks
    raw = np.concatenate([_iq4_block(b["scale"], b["nibbles"]) for b in gold["two_blocks"]])
    got = orc.iq4nl_dequant(raw, 64)
    want = np.concatenate([np.float32(b["scale"]) * T[np.array(b["nibbles"])] for b in gold["two_blocks"]])
    assert np.max(np.abs(got - want)) <= 1e-6
    # :86-120 partial block
    p = gold["partial"]
    raw = np.concatenate([_iq4_block(b["scale"], b["nibbles"]) for b in p["blocks"]])
    got = orc.iq4nl_dequant(raw, p["num_elements"])
    want = T[np.arange(48) % 16]
    assert got.size == 48 and np.max(np.abs(got - want)) <= 1e-6


def test_iq4nl_nibble_order_is_interleaved(orc):
    # element 0 <- low nibble of byte 0, element 1 <- high nibble of byte 0
    nib = np.zeros(32, np.uint8)
    nib[1] = 15
    got = orc.iq4nl_dequant(_iq4_block(1.0, nib), 32)
    T = orc.iq4nl_table()
    assert got[1] == T[15] and got[0] == T[0] and got[16] == T[0]


def test_iq4nl_matmul_matches_fp64(orc):
    rows, K, N = 24, 128, 3
    w = synth.iq4nl(rows, K, 4)
    x16 = synth.x_f16(K * N, 4)
    wd = orc.iq4nl_dequant(w.raw, rows * K).reshape(rows, K).astype(np.float64)
    xf = x16.view(np.float16).astype(np.float64).reshape(K, N)
    ref = wd @ xf
    got = orc.iq4nl_matmul(w.raw, x16, rows, K, N).reshape(rows, N)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


# ------------------------------------------------------------ GPTQ / AWQ


def quantize_awq(src: np.ndarray, group: int):
    """QuantizeAWQ (tensor/quantized_awq.go:44-114) restated."""
    n = src.size
    ng = (n + group - 1) // group
    words, scales, zeros = [], [], []
    for gi in range(ng):
        g = src[gi * group:(gi + 1) * group].astype(np.float32)
        mn, mx = g.min(), g.max()
        scale = np.float32((mx - mn) / np.float32(15)) if mx - mn > 0 else np.float32(0)
        zero = np.float32(-mn / scale) if scale > 0 else np.float32(0)
        sb, zb = f16(scale), f16(zero)
        sf = sb.view(np.float16).astype(np.float32)
        zf = zb.view(np.float16).astype(np.float32)
        inv = np.float32(1) / sf if sf > 0 else np.float32(0)
        q = np.clip((g * inv + zf + np.float32(0.5)).astype(np.int64), 0, 15)  # Go int() truncates
        w = np.zeros((g.size + 7) // 8, np.uint32)
        for j, v in enumerate(q):
            w[j // 8] |= np.uint32(int(v) & 15) << np.uint32(4 * (j % 8))
        words.append(w)
        scales.append(sb)
        zeros.append(zb)
    return np.concatenate(words), np.array(scales, np.uint16), np.array(zeros, np.uint16)


def test_awq_reference_known_vectors(orc):
    # tensor/quantized_awq_test.go:88-118 and :120-133
    src = np.arange(8, dtype=np.float32)
    w, s, z = quantize_awq(src, 8)
    got = orc.awq_dequant(w, s, z, 8, 8)
    assert np.all(np.abs(got - src) <= 1.1)
    assert abs(got[0]) <= 0.1 and abs(got[7] - 7.0) <= 0.1
    w, s, z = quantize_awq(np.full(8, 3.14, np.float32), 8)
    assert np.all(orc.awq_dequant(w, s, z, 8, 8) == 0.0)


def test_gptq_and_awq_share_byte_layout(orc):
    # AWQ's LE uint32 words are GPTQ's 4-bit bytes: the two oracle dequantizers,
    # written from two different reference functions, must agree bit for bit.
    wts = synth.w4a16(4, 256, 9, group=128)
    words = wts.packed.reshape(-1).view("<u4")
    a = orc.gptq_dequant(wts.packed, wts.scales, wts.zeros, 4 * 256, 128)
    b = orc.awq_dequant(words, wts.scales, wts.zeros, 4 * 256, 128)
    assert np.array_equal(a, b)


def test_gptq_dequant_closed_form_with_integer_zero(orc):
    # zero = 8: (q - 8) is exact, so w == (q-8)*s with a single rounding.
    wts = synth.w4a16(2, 128, 2, group=64)
    got = orc.gptq_dequant(wts.packed, wts.scales, wts.zeros, 256, 64).reshape(2, 128)
    p = wts.packed.reshape(2, 64)
    q = np.empty((2, 128), np.int64)
    q[:, 0::2], q[:, 1::2] = p & 15, p >> 4
    s = np.repeat(wts.scales.view(np.float16).astype(np.float32), 64, axis=1)
    assert np.array_equal(got, ((q - 8).astype(np.float32) * s).astype(np.float32))


def test_gptq_non_integer_zero_and_bits8(orc):
    data = np.array([0x21, 0xF0], np.uint8)  # q = 1, 2, 0, 15
    s, z = f16(0.5).reshape(1), f16(2.25).reshape(1)
    got = orc.gptq_dequant(data, s, z, 4, 4, bits=4)
    assert np.array_equal(got, np.array([-0.625, -0.125, -1.125, 6.375], np.float32))
    got8 = orc.gptq_dequant(np.array([3, 250], np.uint8), s, z, 2, 2, bits=8)
    assert np.array_equal(got8, np.array([0.375, 123.875], np.float32))


def test_w4a16_matmul_matches_fp64_and_equals_dequant_plus_gemm(orc):
    m, k, n, g = 8, 256, 4, 128
    wts = synth.w4a16(m, k, 7, group=g)
    x16 = synth.x_f16(k * n, 7)
    c = orc.w4a16_matmul(wts.packed, wts.scales, wts.zeros, x16, m, k, n, g).reshape(m, n)
    wd = orc.gptq_dequant(wts.packed, wts.scales, wts.zeros, m * k, g).reshape(m, k)
    xf = x16.view(np.float16).astype(np.float32).reshape(k, n)
    # compute/w4a16_test.go:255-348: dispatch == dequant + fp32 GEMM exactly
    assert np.array_equal(c.reshape(-1), orc.sgemm_simd(wd, xf, m, n, k))
    ref = wd.astype(np.float64) @ xf.astype(np.float64)
    assert np.max(np.abs(c - ref)) <= 1e-5 * np.max(np.abs(ref))


# -------------------------------------------------------------- SgemmSimd


def test_sgemm_exact_on_small_integers_and_tail_lengths(orc):
    rng = np.random.default_rng(3)
    for m, n, k in [(1, 1, 1), (3, 5, 7), (2, 37, 300), (4, 16, 513)]:
        a = rng.integers(-4, 5, (m, k)).astype(np.float32)
        b = rng.integers(-4, 5, (k, n)).astype(np.float32)
        got = orc.sgemm_simd(a, b, m, n, k).reshape(m, n)
        assert np.array_equal(got, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


def test_sgemm_not_transposed(orc):
    a = np.array([[1, 2, 3]], np.float32)
    b = np.array([[1, 0], [0, 1], [1, 1]], np.float32)
    assert np.array_equal(orc.sgemm_simd(a, b, 1, 2, 3), np.array([4, 5], np.float32))


# --------------------------------------------------------------- Ternary


def test_ternary_reference_known_answers(orc):
    gold = json.loads((GOLD / "ternary_cases.json").read_text())
    for case in gold["gemv"]:
        raw = synth.pack_ternary(np.array(case["w"], np.int8))
        y = orc.ternary_gemv(raw, np.array(case["x"], np.float32), case["rows"], case["cols"])
        assert np.array_equal(y, np.array(case["want"], np.float32)), case["name"]
        # Get() decodes every element back
        assert [orc.ternary_get(raw, i) for i in range(len(case["w"]))] == case["w"]
    for n, want in gold["byte_counts"]:
        assert synth.pack_ternary(np.zeros(n, np.int8)).size == want


def test_ternary_matches_dense_and_repack(orc):
    # compute/ternary_gemv_test.go:47-74 (dense match <= 1e-6), on both the
    # byte-aligned LUT path and the unaligned per-element path.
    rng = np.random.default_rng(42)
    for rows, cols in [(128, 256), (7, 33), (5, 6)]:
        w = rng.integers(-1, 2, rows * cols).astype(np.int8)
        x = (rng.random(cols, dtype=np.float32) * 2 - 1).astype(np.float32)
        raw = synth.pack_ternary(w)
        y = orc.ternary_gemv(raw, x, rows, cols)
        dense = np.zeros(rows, np.float32)
        wf = w.reshape(rows, cols).astype(np.float32)
        for j in range(cols):
            dense = (dense + wf[:, j] * x[j]).astype(np.float32)
        assert np.max(np.abs(y - dense)) <= 1e-6
        rep = orc.ternary_repack_rows(raw, rows, cols)
        bpr = (cols + 3) // 4
        for i in range(rows):
            for j in range(cols):
                code = (rep[i * bpr + j // 4] >> (2 * (j % 4))) & 3
                assert int(code) - 1 == w[i * cols + j]


def test_ternary_i8_is_exact_integer_dot_times_scale(orc):
    rows, K = 40, 2560
    t = synth.ternary(rows, K, 8)
    q, xs = synth.x_i8(K, 8)
    y = orc.ternary_gemv_i8(t.raw, q, xs, t.w_scale, rows, K)
    codes = np.array([orc.ternary_get(t.raw, i) for i in range(rows * K)], np.int64).reshape(rows, K)
    exact = codes @ q.astype(np.int64)
    want = (exact.astype(np.float32) * np.float32(t.w_scale * xs)).astype(np.float32)
    assert np.array_equal(y, want)
