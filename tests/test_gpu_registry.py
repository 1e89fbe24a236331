"""Device dequantizers of the Dequantizer registry (ROCmEngine.dequantize ->
libzt_hip.so) against the oracle's restatement of each registered format,
bit for bit (NaN positions for FP8_E5M2's NaN codes), including partial last
blocks and AWQ groups that do not divide the element count or 8."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import registry, synth  # noqa: E402
from ztensor_amd.engine import ROCmEngine  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return ROCmEngine(0)


def bits_equal(a, b) -> bool:
    a, b = np.asarray(a, np.float32), np.asarray(b, np.float32)
    nan = np.isnan(b)
    return np.array_equal(np.isnan(a), nan) and np.array_equal(a[~nan].view(np.uint32), b[~nan].view(np.uint32))


@pytest.mark.parametrize("n", [32, 4096, 1000, 7])
def test_q4_0_q8_0(eng, orc, n):
    rows, K = 1, -(-n // 32) * 32
    w4 = synth.q4_0(rows, K, 50)
    assert bits_equal(eng.dequantize("Q4_0", w4.raw, n).cpu().numpy(), orc.q4_dequant(w4.raw, n))
    w8 = synth.q8_0(rows, K, 51)
    assert bits_equal(eng.dequantize("Q8_0", w8.raw, n).cpu().numpy(), orc.q8_dequant(w8.raw, n))


@pytest.mark.parametrize("fmt,name", [("q4_k", "Q4_K"), ("q5_k", "Q5_K"), ("q6_k", "Q6_K"), ("q5_0", "Q5_0")])
@pytest.mark.parametrize("n", [512, 300])
def test_kquants_and_q5_0(eng, orc, fmt, name, n):
    vals = 32 if fmt == "q5_0" else 256
    w = synth.kquant(fmt, 1, -(-n // vals) * vals, 52)
    ref = orc.q5_0_dequant(w.raw, n) if fmt == "q5_0" else orc.kq_dequant(fmt, w.raw, n)
    assert bits_equal(eng.dequantize(name, w.raw, n).cpu().numpy(), ref)


@pytest.mark.parametrize("n,group", [(4096 * 3, 128), (1000, 128), (300, 36), (37, 5), (1, 128)])
def test_awq4_wire(eng, orc, n, group):
    wire, _, _, _ = synth.awq4_wire(n, group, 53)
    rc, ref = orc.awq4_wire_dequant(wire, n)
    assert rc == 0
    assert bits_equal(eng.dequantize("AWQ_4", wire, n).cpu().numpy(), ref)
    with pytest.raises(ValueError):
        eng.dequantize("AWQ_4", wire[:-1], n)
    with pytest.raises(ValueError):
        eng.dequantize("AWQ_4", wire, n + 1)


@pytest.mark.parametrize("name,e5m2", [("FP8_E4M3", False), ("FP8_E5M2", True)])
def test_fp8_all_codes(eng, orc, name, e5m2):
    codes = np.tile(np.arange(256, dtype=np.uint8), 5)
    wire = synth.fp8_wire(codes, 0.0123)
    rc, ref = orc.fp8_dequant(wire, codes.size, e5m2)
    assert rc == 0
    assert bits_equal(eng.dequantize(name, wire, codes.size).cpu().numpy(), ref)
    with pytest.raises(ValueError):
        eng.dequantize(name, wire[:-1], codes.size)


@pytest.mark.parametrize("n", [256, 4096, 300, 1])
def test_iq3s(eng, orc, n):
    raw = synth.iq3s(-(-n // 256), 54 + n)
    rc, ref = orc.iq3s_dequant(raw, n)
    assert rc == 0
    assert bits_equal(eng.dequantize("IQ3_S", raw, n).cpu().numpy(), ref)
    with pytest.raises(ValueError):
        eng.dequantize("IQ3_S", raw[:-1], n)
    with pytest.raises(ValueError):
        eng.dequantize("IQ3_S", raw, 0)  # NewIQ3SStorageFromRaw rejects zero elements


@pytest.mark.parametrize("n", [32, 1000, 7])
def test_w8a8(eng, orc, n):
    # W8A8's 36-byte groups are Q8_0's (tensor/quantized_w8a8.go:285-316)
    w = synth.q8_0(1, -(-n // 32) * 32, 55)
    assert bits_equal(eng.dequantize("W8A8", w.raw, n).cpu().numpy(), orc.q8_dequant(w.raw, n))
    with pytest.raises(ValueError):
        eng.dequantize("W8A8", w.raw[:-1], n)
    assert eng.dequantize("W8A8", w.raw, 0).numel() == 0


def test_unknown_name_and_empty(eng):
    with pytest.raises(ValueError):
        eng.dequantize("NOPE", np.zeros(4, np.uint8), 1)
    assert eng.dequantize("Q4_0", np.zeros(0, np.uint8), 0).numel() == 0
    assert registry.get_quant_type("AWQ_4")[1]
