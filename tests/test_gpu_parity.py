"""GPU parity: every HIP entry point against the CPU oracle, through the C ABI.

Bars (written into each assertion):
  * dequantizers: bit-exact (uint32 view equality) with the reference's
    dequantizers as restated by the oracle;
  * GEMV / GEMM: max|y - y_ref| / max|y_ref| <= 1e-5 with fp32 accumulation,
    y_ref = the reference CPU engine's result (oracle): every product is
    exact in fp32 on these kernels, so only the summation order differs
    (measured about 2e-7).  The IQ4_NL fp16-activation kernels carry the
    codebook as two fp16 parts, exact to 2^-22 an entry (measured about
    2e-6), and meet the same bar;
  * ternary int8: bit-exact (integer accumulation).
Shapes: the benchmark configurations at full size plus ragged/edge cases.
"""
import functools
import json
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-5
GOLD = Path(__file__).resolve().parent / "golden"

LLAMA8B = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]  # (rows = out features, K)
BITNET = [(2560, 2560), (6912, 2560), (2560, 6912)]
QWEN = [(3584, 3584), (18944, 3584), (3584, 18944)]
LLAMA70B = [(8192, 8192), (1024, 8192), (28672, 8192), (8192, 28672)]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return _lib.load()


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def devf(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def bits_equal(a, b) -> bool:
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32), np.asarray(b, np.float32).view(np.uint32))


def say(msg: str) -> None:
    print(msg, flush=True)


@functools.lru_cache(maxsize=4)
def w4_cached(rows, K, seed):
    return synth.w4a16(rows, K, seed)


# ------------------------------------------------------------------ Q4_0


def q4_dev(w):
    gpu = synth_gpu_q4(w.raw, w.rows * w.K // 32)
    return dev(gpu), _lib.load().zt_q4_gpu_data_offset(w.rows * w.K // 32)


def synth_gpu_q4(raw, nblk):
    lib = _lib.load()
    out = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_q4_raw_to_gpu(raw.ctypes.data, nblk, out.ctypes.data)
    return out


@pytest.mark.parametrize("rows,K", [(1, 32), (3, 96), (17, 4096)] + LLAMA8B[:2])
def test_q4_dequant_bit_exact(lib, orc, rows, K):
    w = synth.q4_0(rows, K, synth.seed_for(2, rows % 7))
    a, off = q4_dev(w)
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_q4_f32", a.data_ptr(), out.data_ptr(), rows * K, off, stream())
    assert bits_equal(out.cpu().numpy(), orc.q4_dequant(w.raw, rows * K))


@pytest.mark.parametrize("rows,K", LLAMA8B + [(1, 32), (3, 64), (65, 96), (130, 2080), (7, 16384), (64, 28672),
                                    (9, 16416)])
def test_q4_gemv_matches_oracle(lib, orc, rows, K):
    say(f"q4 gemv rows={rows} K={K}")
    seed = synth.seed_for(2, LLAMA8B.index((rows, K)) if (rows, K) in LLAMA8B else 9)
    w = synth.q4_0(rows, K, seed)
    x = synth.x_f32(K, seed)
    a, off = q4_dev(w)
    xd, y = devf(x), torch.empty(rows, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4_f32", a.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, 1, off, stream())
    ref = orc.gemm_f32_q4_nt(x, w.raw, 1, rows, K, threads=orc.nthreads())
    assert rel_err(y.cpu().numpy(), ref) <= TOL


# (2, 32, 4) and (64, 128, 64): the reference's gemm_q4_f32 tests
# (internal/cuda/kernels/gemm_q4_test.go:152, 235)
@pytest.mark.parametrize("rows,K,N", [(100, 512, 2), (100, 512, 3), (100, 512, 8), (2, 32, 4), (64, 128, 64)])
def test_q4_batched_matches_oracle(lib, orc, rows, K, N):
    w = synth.q4_0(rows, K, 21)
    x = synth.x_f32(K * N, 21).reshape(K, N)  # B is [K, N]
    a, off = q4_dev(w)
    xd, c = devf(x), torch.empty(rows * N, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4_f32", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, off, stream())
    ref = orc.gemm_f32_q4_nt(np.ascontiguousarray(x.T), w.raw, N, rows, K).reshape(N, rows).T
    assert rel_err(c.cpu().numpy().reshape(rows, N), ref) <= TOL


@pytest.mark.parametrize("rows,K", [(256, 4096), (1, 32), (17, 544), (100, 4128), (33, 8192), (9, 16384),
                                    (5, 20480), (4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)])
def test_q4_fp16_activations(lib, orc, rows, K):
    """zt_gemm_q4_f16 at batch 1 against the oracle, and bit-identical to
    zt_gemm_q4_f32 on the same activations widened to fp32: both run the
    same kernel (fixed steps up to K = 16384, the loop beyond) with the same
    products in the same order."""
    w = synth.q4_0(rows, K, 5)
    x16 = synth.x_f16(K, 5)
    x32 = np.asarray(orc.f16_to_f32(x16), np.float32)
    a, off = q4_dev(w)
    xd, y = dev(x16), torch.empty(rows, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4_f16", a.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, 1, off, stream())
    ref = orc.gemm_f32_q4_nt(x32, w.raw, 1, rows, K)
    got = y.cpu().numpy()
    assert rel_err(got, ref) <= TOL
    y32 = torch.empty(rows, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4_f32", a.data_ptr(), devf(x32).data_ptr(), y32.data_ptr(), rows, K, 1, off, stream())
    assert np.array_equal(got.view(np.uint32), y32.cpu().numpy().view(np.uint32))


def test_q4_reference_known_answers(lib):
    # internal/xblas/q4dot_test.go:11-140, each case as a 1x32 GEMV.
    for case in json.loads((GOLD / "q4dot_cases.json").read_text()):
        nib = np.array(case["nibbles"], np.uint8).reshape(1, 32)
        raw = synth.pack_q4_0(nib, synth.f16_bits(np.float32(case["scale"])).reshape(1))
        a = dev(synth_gpu_q4(raw, 1))
        x = devf(np.array(case["x"], np.float32))
        y = torch.empty(1, dtype=torch.float32, device="cuda")
        lib.call("zt_gemm_q4_f32", a.data_ptr(), x.data_ptr(), y.data_ptr(), 1, 32, 1, 16, stream())
        got, want = float(y.cpu()[0]), case["want"]
        # the cases' scales (0.5, 100, 0.001, 0.25) pass through fp16; 0.001 is not exact.
        s16 = float(synth.f16_bits(np.float32(case["scale"])).view(np.float16))
        want16 = want * (s16 / case["scale"]) if case["scale"] else 0.0
        # the reference test allows 1e-6 relative for its sequential loop; the
        # kernel's sum(q x) - 8 sum(x) form is held to 1e-5 relative here.
        assert abs(got - want16) <= max(1e-5, 1e-5 * abs(want16)), case["name"]


def test_q4_invalid_arguments_rejected(lib):
    a = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    x = torch.zeros(64, dtype=torch.float32, device="cuda")
    y = torch.zeros(4, dtype=torch.float32, device="cuda")
    # K % 32 != 0 -> hipErrorInvalidValue (internal/cuda/kernels/gemm_q4.cu:169-171)
    assert lib.zt_gemm_q4_f32(a.data_ptr(), x.data_ptr(), y.data_ptr(), 2, 40, 1, 16, stream()) == 1
    # misaligned data region
    assert lib.zt_gemm_q4_f32(a.data_ptr(), x.data_ptr(), y.data_ptr(), 2, 32, 1, 8, stream()) == 1
    assert lib.zt_gemm_q4_f32(0, x.data_ptr(), y.data_ptr(), 2, 32, 1, 16, stream()) == 1
    # empty output: nothing to do
    assert lib.zt_gemm_q4_f32(a.data_ptr(), x.data_ptr(), y.data_ptr(), 0, 32, 1, 16, stream()) == 0
    torch.cuda.synchronize()


def test_q4_zero_scale_gives_zero(lib):
    nib = np.full((4, 32), 15, np.uint8)
    raw = synth.pack_q4_0(nib, np.zeros(4, np.uint16))
    a = dev(synth_gpu_q4(raw, 4))
    x = devf(np.ones(64, np.float32))
    y = torch.full((2,), 7.0, device="cuda")
    lib.call("zt_gemm_q4_f32", a.data_ptr(), x.data_ptr(), y.data_ptr(), 2, 64, 1, 16, stream())
    assert np.array_equal(y.cpu().numpy(), np.zeros(2, np.float32))


# ------------------------------------------------------------------ Q8_0


def q8sep(lib, raw, nblk):
    out = np.empty(lib.zt_q8_gpu_bytes(nblk), np.uint8)
    lib.zt_q8_raw_to_gpu(raw.ctypes.data, nblk, out.ctypes.data)
    return out


@pytest.mark.parametrize("rows,K", [(5, 64), (64, 4096)])
def test_q8_dequant_bit_exact_both_layouts(lib, orc, rows, K):
    w = synth.q8_0(rows, K, 31)
    n = rows * K
    ref = orc.q8_dequant(w.raw, n)
    out = torch.empty(n, dtype=torch.float32, device="cuda")
    raw_d = dev(w.raw)
    lib.call("zt_dequant_q8_f32", raw_d.data_ptr(), out.data_ptr(), n, stream())
    assert bits_equal(out.cpu().numpy(), ref)
    nblk = n // 32
    sep = dev(q8sep(lib, w.raw, nblk))
    out.zero_()
    lib.call("zt_dequant_q8sep_f32", sep.data_ptr(), out.data_ptr(), n, lib.zt_q8_gpu_data_offset(nblk), stream())
    assert bits_equal(out.cpu().numpy(), ref)
    # device-side repack gives the same bytes as the host one
    rep = torch.empty_like(sep)
    lib.call("zt_q8_repack", raw_d.data_ptr(), rep.data_ptr(), nblk, stream())
    off = lib.zt_q8_gpu_data_offset(nblk)
    r, s = rep.cpu().numpy(), sep.cpu().numpy()
    assert np.array_equal(r[: 4 * nblk], s[: 4 * nblk]) and np.array_equal(r[off:], s[off:])


@pytest.mark.parametrize("rows,K", LLAMA8B + [(3, 32), (65, 2080), (17, 8160), (2, 6144), (2048, 16384),
                                              (2047, 8224)])
def test_q8_gemv_matches_oracle_both_layouts(lib, orc, rows, K):
    say(f"q8 gemv rows={rows} K={K}")
    seed = synth.seed_for(2, 8 + (LLAMA8B.index((rows, K)) if (rows, K) in LLAMA8B else 5))
    w = synth.q8_0(rows, K, seed)
    x = synth.x_f32(K, seed)
    ref = orc.gemm_f32_q8_nt(x, w.raw, 1, rows, K, threads=orc.nthreads())
    xd, y = devf(x), torch.empty(rows, dtype=torch.float32, device="cuda")
    raw = dev(w.raw)
    lib.call("zt_gemm_q8_f32", raw.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, 1, stream())
    assert rel_err(y.cpu().numpy(), ref) <= TOL
    del raw
    nblk = rows * K // 32
    sep = dev(q8sep(lib, w.raw, nblk))
    y.zero_()
    lib.call("zt_gemm_q8sep_f32", sep.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, 1,
             lib.zt_q8_gpu_data_offset(nblk), stream())
    assert rel_err(y.cpu().numpy(), ref) <= TOL


def test_q8_batched(lib, orc):
    rows, K, N = 33, 256, 4
    w = synth.q8_0(rows, K, 2)
    x = synth.x_f32(K * N, 2).reshape(K, N)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    # keep every device buffer referenced until the kernel has run: a freed
    # temporary can be handed to the next allocation on the same stream.
    a, xd = dev(w.raw), devf(x)
    lib.call("zt_gemm_q8_f32", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, stream())
    ref = orc.gemm_f32_q8_nt(np.ascontiguousarray(x.T), w.raw, N, rows, K).reshape(N, rows).T
    assert rel_err(c.cpu().numpy().reshape(rows, N), ref) <= TOL


# ---------------------------------------------------------------- IQ4_NL


@pytest.mark.parametrize("rows,K", [(2, 64), (3584, 3584)])
def test_iq4nl_dequant_bit_exact(lib, orc, rows, K):
    w = synth.iq4nl(rows, K, 41)
    nblk = rows * K // 32
    a = dev(synth_gpu_q4(w.raw, nblk))
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_iq4nl_f32", a.data_ptr(), out.data_ptr(), rows * K, lib.zt_q4_gpu_data_offset(nblk),
             stream())
    assert bits_equal(out.cpu().numpy(), orc.iq4nl_dequant(w.raw, rows * K))


def test_iq4nl_partial_block_dequant(lib, orc):
    # tensor/iq4_storage_test.go:86-120: 48 elements over two blocks
    gold = json.loads((GOLD / "iq4nl_cases.json").read_text())["partial"]
    nib = np.array([b["nibbles"] for b in gold["blocks"]], np.uint8)
    raw = synth.pack_iq4nl(nib, synth.f16_bits(np.array([b["scale"] for b in gold["blocks"]], np.float32)))
    a = dev(synth_gpu_q4(raw, 2))
    out = torch.full((64,), -99.0, device="cuda")
    lib.call("zt_dequant_iq4nl_f32", a.data_ptr(), out.data_ptr(), 48, 16, stream())
    o = out.cpu().numpy()
    assert bits_equal(o[:48], orc.iq4nl_dequant(raw, 48)) and np.all(o[48:] == -99.0)


@pytest.mark.parametrize("N", [1, 8])
@pytest.mark.parametrize("rows,K", QWEN + [(5, 96)])
def test_iq4nl_gemm_matches_oracle(lib, orc, rows, K, N):
    say(f"iq4nl rows={rows} K={K} N={N}")
    seed = synth.seed_for(5, QWEN.index((rows, K)) if (rows, K) in QWEN else 7)
    w = synth.iq4nl(rows, K, seed)
    x16 = synth.x_f16(K * N, seed)
    nblk = rows * K // 32
    a = dev(synth_gpu_q4(w.raw, nblk))
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    xd = dev(x16)
    lib.call("zt_gemm_iq4nl_f16", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
             lib.zt_q4_gpu_data_offset(nblk), stream())
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(c.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("rows,K", [(8193, 4096), (9001, 3616), (8200, 128), (7, 2048), (1, 32), (4099, 3584),
                                    (3, 4128)])
def test_iq4nl_f16_gemv_ragged(lib, orc, rows, K):
    """Batch-1 fp16 IQ4_NL on the fixed-step kernel (K <= 4096: two steps
    from 8192 rows, one below; a partial last step at K = 3616) and on the
    loop kernel above 4096 (4128), with row counts that are not a multiple
    of the rows per wave."""
    say(f"iq4nl f16 gemv rows={rows} K={K}")
    w = synth.iq4nl(rows, K, 23)
    x16 = synth.x_f16(K, 23)
    nblk = rows * K // 32
    a = dev(synth_gpu_q4(w.raw, nblk))
    c = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = dev(x16)
    lib.call("zt_gemm_iq4nl_f16", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, 1,
             lib.zt_q4_gpu_data_offset(nblk), stream())
    assert rel_err(c.cpu().numpy(), orc.iq4nl_matmul(w.raw, x16, rows, K, 1)) <= TOL


@pytest.mark.parametrize("rows,K,N", [(33, 2176, 4), (1, 128, 16), (100, 3584, 12), (64, 384, 8)])
def test_iq4nl_mfma_ragged(lib, orc, rows, K, N):
    """Batched IQ4_NL on the MFMA path: partial row tiles, a partial last K
    chunk (2176 = 2048 + 128), a single row, N = 4, 8, 12, 16."""
    say(f"iq4nl mfma rows={rows} K={K} N={N}")
    w = synth.iq4nl(rows, K, 21)
    x16 = synth.x_f16(K * N, 21)
    nblk = rows * K // 32
    a = dev(synth_gpu_q4(w.raw, nblk))
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    xd = dev(x16)
    lib.call("zt_gemm_iq4nl_f16", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N,
             lib.zt_q4_gpu_data_offset(nblk), stream())
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(c.cpu().numpy(), ref) <= TOL


def test_iq4nl_codebook_worst_case(lib, orc):
    """The fp16-activation GEMV carries the fp32 codebook as T_hi + 2^-11
    T_lo' in fp16.  Every weight sits on T = -0.5250730, the entry that
    fp16 alone rounds worst (relative error 3.25e-4), and every activation
    is positive, so no per-weight errors can cancel: a kernel that dropped
    the lo part would miss by 3.25e-4, the split stays within 1e-5."""
    rows, K = 256, 4096
    nblk = rows * K // 32
    rng = np.random.default_rng(5)
    nib = np.full((nblk, 32), 2, np.uint8)
    scales = synth.f16_bits(np.abs(rng.standard_normal(nblk).astype(np.float32)) * np.float32(0.01) + np.float32(0.001))
    raw = synth.pack_iq4nl(nib, scales)
    x16 = synth.f16_bits(rng.uniform(0.5, 1.5, K).astype(np.float32))
    a = dev(synth_gpu_q4(raw, nblk))
    c = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = dev(x16)
    lib.call("zt_gemm_iq4nl_f16", a.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, 1,
             lib.zt_q4_gpu_data_offset(nblk), stream())
    ref = orc.iq4nl_matmul(raw, x16, rows, K, 1)
    err = rel_err(c.cpu().numpy(), ref)
    assert err <= TOL


def test_iq4nl_fp32_activations(lib, orc):
    rows, K = 64, 1024
    w = synth.iq4nl(rows, K, 3)
    x = synth.x_f32(K, 3)
    nblk = rows * K // 32
    a = dev(synth_gpu_q4(w.raw, nblk))
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = devf(x)
    lib.call("zt_gemm_iq4nl_f32", a.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, 1,
             lib.zt_q4_gpu_data_offset(nblk), stream())
    ref = orc.iq4nl_dequant(w.raw, rows * K).reshape(rows, K).astype(np.float64) @ x.astype(np.float64)
    assert rel_err(y.cpu().numpy(), ref) <= TOL


# ----------------------------------------------------------------- W4A16


def w4_dev(w):
    return dev(w.packed), dev(w.scales), dev(w.zeros)


@pytest.mark.parametrize("rows,K,g", [(4, 256, 128), (4096, 4096, 128), (3, 96, 32)])
def test_w4_dequant_bit_exact(lib, orc, rows, K, g):
    w = synth.w4a16(rows, K, 51, group=g)
    p, s, z = w4_dev(w)
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_w4_f32", p.data_ptr(), s.data_ptr(), z.data_ptr(), out.data_ptr(), rows * K, g, stream())
    assert bits_equal(out.cpu().numpy(), orc.gptq_dequant(w.packed, w.scales, w.zeros, rows * K, g))


def test_w4_dequant_non_integer_zero(lib, orc):
    rows, K, g = 8, 256, 64
    w = synth.w4a16(rows, K, 52, group=g)
    zeros = synth.f16_bits(np.random.default_rng(0).uniform(0, 15, w.zeros.shape).astype(np.float32))
    p, s, z = dev(w.packed), dev(w.scales), dev(zeros)
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_w4_f32", p.data_ptr(), s.data_ptr(), z.data_ptr(), out.data_ptr(), rows * K, g, stream())
    assert bits_equal(out.cpu().numpy(), orc.gptq_dequant(w.packed, w.scales, zeros, rows * K, g))


def run_w4a16(lib, w, x16, rows, K, N, zeros=True):
    p, s, z = w4_dev(w)
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    xd = dev(x16)
    lib.call("zt_gemm_w4a16_f32", p.data_ptr(), s.data_ptr(), z.data_ptr() if zeros else 0, xd.data_ptr(),
             c.data_ptr(), rows, K, N, w.group, stream())
    return c.cpu().numpy()


def test_w4a16_gemv_config1(lib, orc):
    rows, K = 4096, 4096
    seed = synth.seed_for(1)
    w = synth.w4a16(rows, K, seed)
    x16 = synth.x_f16(K, seed)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128)
    assert rel_err(run_w4a16(lib, w, x16, rows, K, 1), ref) <= TOL
    # zeros == NULL means the symmetric zero-point 8, equal to explicit zeros of 8
    assert rel_err(run_w4a16(lib, w, x16, rows, K, 1, zeros=False), ref) <= TOL


@pytest.mark.parametrize("N", [1, 4, 8, 16])
@pytest.mark.parametrize("rows,K", LLAMA70B)
def test_w4a16_gemm_70b_shapes(lib, orc, rows, K, N):
    say(f"w4a16 rows={rows} K={K} N={N}")
    seed = synth.seed_for(4, LLAMA70B.index((rows, K)))
    w = w4_cached(rows, K, seed)
    x16 = synth.x_f16(K * N, seed + N)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128)
    assert rel_err(run_w4a16(lib, w, x16, rows, K, N), ref) <= TOL


@pytest.mark.parametrize("rows,K,g,N", [(1, 32, 32, 1), (3, 96, 32, 2), (65, 384, 128, 3), (17, 256, 64, 5)])
def test_w4a16_ragged(lib, orc, rows, K, g, N):
    w = synth.w4a16(rows, K, 7, group=g)
    x16 = synth.x_f16(K * N, 7)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, g)
    assert rel_err(run_w4a16(lib, w, x16, rows, K, N), ref) <= TOL


@pytest.mark.parametrize("rows,K,g,N", [(65, 384, 128, 4), (33, 2176, 128, 8), (17, 4096, 256, 12), (1, 128, 128, 16),
                                        (100, 2048, 128, 16), (100, 4096, 128, 8), (40, 12288, 256, 4)])
def test_w4a16_mfma_ragged(lib, orc, rows, K, g, N):
    """Batched shapes on the MFMA path: partial row tiles, a partial last K
    chunk (2176 = 2048 + 128), group 256, N = 12, one-row matrices, and
    few-row matrices whose K is split across workgroups (100 x 4096: four
    splits of 8 units; 40 x 12288: eight splits of 12 units)."""
    say(f"w4a16 mfma rows={rows} K={K} g={g} N={N}")
    w = synth.w4a16(rows, K, 9, group=g)
    x16 = synth.x_f16(K * N, 9)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, g)
    assert rel_err(run_w4a16(lib, w, x16, rows, K, N), ref) <= TOL


def test_w4a16_mfma_non_integer_zero(lib, orc):
    """Zero points that are not integers (GPTQ allows any fp16): the MFMA
    path subtracts z * sum(x) exactly instead of folding z into the weights."""
    rows, K, N = 64, 1024, 8
    w = synth.w4a16(rows, K, 10)
    rng = np.random.default_rng(10)
    zeros = synth.f16_bits((rng.random(w.zeros.shape, dtype=np.float32) * 15).astype(np.float32))
    w = synth.W4Weights(rows, K, w.group, w.packed, w.scales, zeros)
    x16 = synth.x_f16(K * N, 10)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, N, 128)
    assert rel_err(run_w4a16(lib, w, x16, rows, K, N), ref) <= TOL


def test_w4a16_invalid_group(lib):
    t = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    assert lib.zt_gemm_w4a16_f32(t.data_ptr(), t.data_ptr(), 0, t.data_ptr(), t.data_ptr(), 2, 128, 1, 48,
                                 stream()) == 1
    assert lib.zt_gemm_w4a16_f32(t.data_ptr(), t.data_ptr(), 0, t.data_ptr(), t.data_ptr(), 2, 96, 1, 64,
                                 stream()) == 1


# --------------------------------------------------------------- Ternary


@pytest.mark.parametrize("rows,K", BITNET + [(3, 4), (5, 33), (7, 64), (9, 260), (65, 2560), (33, 4160),
                                              (6, 65536), (4, 65600), (2049, 128),
                                              (1501, 256), (16397, 128), (3, 4096)])
def test_ternary_i8_bit_exact(lib, orc, rows, K):
    say(f"ternary i8 rows={rows} K={K}")
    seed = synth.seed_for(3, BITNET.index((rows, K)) if (rows, K) in BITNET else 6)
    t = synth.ternary(rows, K, seed)
    q, xs = synth.x_i8(K, seed)
    ref = orc.ternary_gemv_i8(t.raw, q, xs, t.w_scale, rows, K)
    W = dev(orc.ternary_repack_rows(t.raw, rows, K))
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    sc = devf(np.array([xs, t.w_scale], np.float32))
    qd = dev(q)
    lib.call("zt_ternary_gemv_i8", W.data_ptr(), qd.data_ptr(), sc.data_ptr(), sc.data_ptr() + 4,
             y.data_ptr(), rows, K, stream())
    assert bits_equal(y.cpu().numpy(), ref)


def test_ternary_f32_reference_known_answers(lib, orc):
    for case in json.loads((GOLD / "ternary_cases.json").read_text())["gemv"]:
        rows, cols = case["rows"], case["cols"]
        raw = synth.pack_ternary(np.array(case["w"], np.int8))
        W = dev(orc.ternary_repack_rows(raw, rows, cols))
        y = torch.empty(rows, dtype=torch.float32, device="cuda")
        xd = devf(np.array(case["x"], np.float32))
        lib.call("zt_ternary_gemv_f32", W.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, cols, stream())
        assert np.array_equal(y.cpu().numpy(), np.array(case["want"], np.float32)), case["name"]


@pytest.mark.parametrize("rows,K", BITNET + [(7, 33), (128, 256), (65, 2560), (6, 65536), (4, 65600), (1501, 256),
                                              (16397, 128), (3, 4096), (2049, 64),
                                              # the quad mapping (K <= 16384, K % 64 == 0): partial row groups,
                                              # lanes past the row's last dword, 1 to 16 waves, 1, 2 or 4 rows
                                              # a wave; past K = 16384 one lane a chunk
                                              (6405, 2560), (8191, 64), (2053, 6912), (4099, 8192), (1, 64),
                                              (131, 1088), (9, 16384), (5, 16448), (300, 4160)])
def test_ternary_f32_matches_oracle(lib, orc, rows, K):
    t = synth.ternary(rows, K, 77)
    x = synth.x_f32(K, 77)
    ref = orc.ternary_gemv(t.raw, x, rows, K)
    W = dev(orc.ternary_repack_rows(t.raw, rows, K))
    y = torch.empty(rows, dtype=torch.float32, device="cuda")
    xd = devf(x)
    lib.call("zt_ternary_gemv_f32", W.data_ptr(), xd.data_ptr(), y.data_ptr(), rows, K, stream())
    assert rel_err(y.cpu().numpy(), ref) <= TOL


def test_ternary_dequant(lib, orc):
    rows, K = 5, 33
    t = synth.ternary(rows, K, 4)
    W = dev(orc.ternary_repack_rows(t.raw, rows, K))
    out = torch.empty(rows * K, dtype=torch.float32, device="cuda")
    lib.call("zt_dequant_ternary_f32", W.data_ptr(), out.data_ptr(), rows, K, stream())
    want = np.array([orc.ternary_get(t.raw, i) for i in range(rows * K)], np.float32)
    assert np.array_equal(out.cpu().numpy(), want)
