"""DequantW4ToFP16 on the device (zt_dequant_q4_f16, zt_dequant_w4_f16,
ROCmEngine.dequant_w4_to_fp16): the reference dequantizes to fp32 and
rounds with github.com/zerfoo/float16's FromFloat32, which no reference test
pins (its only test, compute/w4a16_test.go:230-253, allows 0.01 of error).
These tests fix what the mathematics fixes instead: the fp32 value is the
bit-exact dequantization (the oracle's), and its fp16 rounding is IEEE
round-to-nearest-even, checked against numpy's float32 -> float16
conversion over random weights, on hand-built ties that round down and up
to the even neighbour, on values that overflow to +-inf, and on values that
round into the fp16 subnormal range."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402
from ztensor_amd.engine import ROCmEngine  # noqa: E402
from ztensor_amd.storage import GPTQStorage, Q4Storage, Tensor  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return ROCmEngine(0)


def f16_bits_of(x32: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):  # out-of-range values become +-inf, as intended
        return np.asarray(x32, np.float32).astype(np.float16).view(np.uint16)


def test_q4_0_random_matches_oracle_rounded(eng, orc):
    rows, K = 512, 4096
    w = synth.q4_0(rows, K, 81)
    got = eng.dequant_w4_to_fp16(Tensor((rows, K), Q4Storage.from_raw(w.raw, rows * K)))
    assert got.shape == (rows, K) and got.dtype == torch.float16
    want = f16_bits_of(orc.q4_dequant(w.raw, rows * K))
    assert np.array_equal(got.cpu().numpy().view(np.uint16).reshape(-1), want)


def test_gptq_non_integer_zeros_match_oracle_rounded(eng, orc):
    rows, K, g = 256, 1024, 128
    w = synth.w4a16(rows, K, 82)
    rng = np.random.default_rng(82)
    zeros = synth.f16_bits((rng.random(w.zeros.shape, dtype=np.float32) * 15).astype(np.float32))
    st = GPTQStorage.from_raw(w.packed.reshape(-1), w.scales.reshape(-1), zeros.reshape(-1), rows * K, g, 4)
    got = eng.dequant_w4_to_fp16(Tensor((rows, K), st)).cpu().numpy().view(np.uint16).reshape(-1)
    ref32 = orc.gptq_dequant(w.packed.reshape(-1), w.scales.reshape(-1), zeros.reshape(-1), rows * K, g, 4)
    assert np.array_equal(got, f16_bits_of(ref32))


def q4_block(d_bits: int, codes) -> np.ndarray:
    """One Q4_0 block: fp16 scale, then bytes j = codes[j] | codes[j+16] << 4."""
    c = np.asarray(codes, np.uint8)
    return np.concatenate([np.array([d_bits], "<u2").view(np.uint8), (c[:16] | (c[16:] << 4)).astype(np.uint8)])


def test_ties_round_to_even_and_overflow(eng):
    lib = _lib.load()
    s = torch.cuda.current_stream().cuda_stream
    blocks = [
        # d = 1 + 2^-10: (q - 8) = 3 gives 3 + 3 * 2^-10, 1.5 ulp above 3 -> up to 3 + 2^-8 (mantissa 0x202)
        (0x3C01, [11] * 32, 0x4202),
        # d = 1 + 3 * 2^-10: 3 + 9 * 2^-10, 4.5 ulp above 3 -> down to 3 + 2^-7 (mantissa 0x204)
        (0x3C03, [11] * 32, 0x4204),
        # the same ties negative: (q - 8) = -3
        (0x3C01, [5] * 32, 0xC202),
        (0x3C03, [5] * 32, 0xC204),
        # d = 65504 (fp16 max), q - 8 = -8: -524032 overflows to -inf; +7: 458528 to +inf
        (0x7BFF, [0] * 16 + [15] * 16, None),
    ]
    raw = np.concatenate([q4_block(d, c) for d, c, _ in blocks])
    nblk = len(blocks)
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_q4_raw_to_gpu(raw.ctypes.data, nblk, host.ctypes.data)
    a = torch.from_numpy(host).cuda()
    out = torch.empty(nblk * 32, dtype=torch.float16, device="cuda")
    lib.call("zt_dequant_q4_f16", a.data_ptr(), out.data_ptr(), nblk * 32, lib.zt_q4_gpu_data_offset(nblk), s)
    got = out.cpu().numpy().view(np.uint16).reshape(nblk, 32)
    for i, (_, _, want) in enumerate(blocks[:4]):
        assert np.all(got[i] == want), (i, hex(got[i][0]), hex(want))
    assert np.all(got[4][:16] == 0xFC00) and np.all(got[4][16:] == 0x7C00)
    # numpy's IEEE conversion agrees on every one of them
    d32 = np.array([np.float16(np.uint16(d).view(np.float16)) for d, _, _ in blocks], np.float32)
    for i, (d, c, _) in enumerate(blocks):
        v = (np.asarray(c, np.float32) - 8) * d32[i]
        assert np.array_equal(got[i], f16_bits_of(v))


def test_rounding_into_subnormals(eng, orc):
    """Scale 2^-18 (an fp16 subnormal) with non-integer zeros in [0, 15):
    every |q - z| * 2^-18 is below 2^-14, so each value rounds to an fp16
    subnormal (or zero)."""
    lib = _lib.load()
    s = torch.cuda.current_stream().cuda_stream
    n, g = 4096, 128
    rng = np.random.default_rng(83)
    q = rng.integers(0, 16, size=n, dtype=np.uint8)
    packed = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    scales = np.full(n // g, 0x0040, np.uint16)  # 2^-18
    zeros = synth.f16_bits((rng.random(n // g, dtype=np.float32) * 15).astype(np.float32))
    dev = lambda x: torch.from_numpy(np.ascontiguousarray(x).view(np.uint8)).cuda()  # noqa: E731
    pd, sd, zd = dev(packed), dev(scales), dev(zeros)
    out = torch.empty(n, dtype=torch.float16, device="cuda")
    lib.call("zt_dequant_w4_f16", pd.data_ptr(), sd.data_ptr(), zd.data_ptr(), out.data_ptr(), n, g, s)
    got = out.cpu().numpy().view(np.uint16)
    ref32 = orc.gptq_dequant(packed, scales, zeros, n, g, 4)
    assert np.array_equal(got, f16_bits_of(ref32))
    assert np.all((got & 0x7C00) == 0)  # every value is an fp16 subnormal or zero
    assert np.sum((got & 0x3FF) != 0) > n // 2


def test_invalid_arguments(eng):
    lib = _lib.load()
    assert lib.zt_dequant_w4_f16(0, 0, 0, 0, 64, 48, None) == 1  # group % 32
    assert lib.zt_dequant_w4_f16(0x1008, 0x2000, 0, 0x3000, 64, 32, None) == 1  # W_packed alignment
    assert lib.zt_dequant_q4_f16(0x1001, 0x3000, 32, 16, None) == 1  # odd base
