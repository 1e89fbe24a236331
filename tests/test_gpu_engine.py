"""ROCmEngine (the host mirror of the reference's engine surface) on the GPU.

These follow the reference's own engine tests: the quantized MatMul dispatch
on either operand side (compute/cpu_engine_quant_test.go), the W4A16
dispatch equalling dequantize + GEMM (compute/w4a16_test.go:255-348, there
RMSE <= 1e-6 on one CPU engine; here max|y - y_ref| / max|y_ref| <= 1e-5
against the CPU restatement, fp32 accumulation in both), weight residency
(compute/engine.go:36-38) and TernaryGEMV's known answers
(compute/ternary_gemv_test.go:25-45).  Everything runs through libzt_hip.so.
"""
import json
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import synth  # noqa: E402
from ztensor_amd.engine import ROCmEngine  # noqa: E402
from ztensor_amd.storage import (  # noqa: E402
    AWQStorage,
    Float16Storage,
    GPTQStorage,
    IQ4NLStorage,
    Q4Storage,
    Q8Storage,
    Tensor,
    TernaryStorage,
)

pytestmark = pytest.mark.gpu

TOL = 1e-5  # fp32-exact products: only the summation order differs
GOLD = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def eng():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return ROCmEngine(0)


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("rows,K,N", [(4096, 4096, 1), (1024, 4096, 4), (96, 320, 3)])
def test_q4_matmul_weight_on_a_side(eng, orc, rows, K, N):
    w = synth.q4_0(rows, K, 11)
    s = Q4Storage.from_raw(w.raw, rows * K)
    x = synth.x_f32(K * N, 11).reshape(K, N)
    c = eng.matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda())
    ref = orc.gemm_f32_q4_nt(np.ascontiguousarray(x.T), w.raw, N, rows, K).reshape(N, rows).T
    assert c.shape == (rows, N)
    assert rel_err(c.cpu().numpy(), ref) <= TOL


@pytest.mark.parametrize("M,rows,K", [(1, 4096, 4096), (5, 1024, 4096)])
def test_q4_matmul_weight_on_b_side(eng, orc, M, rows, K):
    """B is the virtually transposed weight: logical [K, rows], physical
    [rows, K] (compute/cpu_engine.go:1378-1390)."""
    w = synth.q4_0(rows, K, 12)
    s = Q4Storage.from_raw(w.raw, rows * K)
    a = synth.x_f32(M * K, 12).reshape(M, K)
    c = eng.matmul(torch.from_numpy(a).cuda(), Tensor((K, rows), s))
    ref = orc.gemm_f32_q4_nt(a, w.raw, M, rows, K).reshape(M, rows)
    assert c.shape == (M, rows)
    assert rel_err(c.cpu().numpy(), ref) <= TOL


def test_upload_weights_is_once_per_storage(eng):
    w = synth.q4_0(64, 256, 13)
    s = Q4Storage.from_raw(w.raw, 64 * 256)
    assert eng.upload_weights([s, s]) == 1
    assert eng.upload_weights([s]) == 0
    buf = s.gpu_ptr()
    assert buf is not None and buf.data_offset == s.gpu_data_offset() and buf.nbytes == s.raw_bytes_gpu().size


def test_q8_matmul(eng, orc):
    rows, K = 1024, 4096
    w = synth.q8_0(rows, K, 14)
    q = w.raw.reshape(-1, 36)
    s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), rows * K)
    assert np.array_equal(s.raw_bytes(), w.raw)
    x = synth.x_f32(K, 14)
    c = eng.matmul(Tensor((rows, K), s), torch.from_numpy(x).cuda())
    ref = orc.gemm_f32_q8_nt(x, w.raw, 1, rows, K)
    assert rel_err(c.cpu().numpy().reshape(-1), ref.reshape(-1)) <= TOL


def test_iq4nl_matmul_fp16_activations(eng, orc):
    rows, K, N = 3584, 3584, 2
    w = synth.iq4nl(rows, K, 15)
    s = IQ4NLStorage.from_raw(w.raw, rows * K)
    x16 = synth.x_f16(K * N, 15)
    c = eng.matmul(Tensor((rows, K), s), torch.from_numpy(x16.view(np.float16).reshape(K, N)).cuda())
    ref = orc.iq4nl_matmul(w.raw, x16, rows, K, N)
    assert rel_err(c.cpu().numpy(), np.asarray(ref).reshape(rows, N)) <= TOL


def _gptq(w):
    return GPTQStorage.from_raw(w.packed.reshape(-1), w.scales.reshape(-1), w.zeros.reshape(-1), w.rows * w.K,
                                w.group, 4)


@pytest.mark.parametrize("side", ["A", "B"])
def test_w4a16_dispatch_equals_dequant_plus_gemm(eng, orc, side):
    rows, K = 4096, 4096
    w = synth.w4a16(rows, K, synth.seed_for(1))
    x16 = synth.x_f16(K, synth.seed_for(1))
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128)
    wt = Tensor((rows, K) if side == "A" else (K, rows), _gptq(w))
    act = Tensor((K, 1) if side == "A" else (1, K), Float16Storage.from_raw(x16, K))
    c = eng.matmul_w4a16(wt, act) if side == "A" else eng.matmul_w4a16(act, wt)
    assert c.dtype == torch.float32
    assert rel_err(c.cpu().numpy().reshape(-1), np.asarray(ref).reshape(-1)) <= TOL


def test_w4a16_awq_words_same_result_as_gptq_bytes(eng, orc):
    rows, K = 256, 1024
    w = synth.w4a16(rows, K, 16)
    words = w.packed.reshape(-1).view("<u4").copy()
    awq = AWQStorage(words, w.scales.reshape(-1).copy(), w.zeros.reshape(-1).copy(), rows * K, 128)
    x16 = synth.x_f16(K, 16)
    act = Tensor((K, 1), Float16Storage.from_raw(x16, K))
    ca = eng.matmul_w4a16(Tensor((rows, K), awq), act).cpu().numpy()
    cg = eng.matmul_w4a16(Tensor((rows, K), _gptq(w)), act).cpu().numpy()
    assert np.array_equal(ca, cg)
    ref = orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128)
    assert rel_err(ca.reshape(-1), np.asarray(ref).reshape(-1)) <= TOL


def test_w4a16_rejects_non_w4a16_inputs(eng):
    w = synth.q8_0(32, 64, 17)
    q = w.raw.reshape(-1, 36)
    s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), 32 * 64)
    act = Tensor((64, 1), Float16Storage.from_raw(synth.x_f16(64, 17), 64))
    with pytest.raises(ValueError):
        eng.matmul_w4a16(Tensor((32, 64), s), act)


def test_q8_rejects_fp16_activations(eng):
    w = synth.q8_0(32, 64, 18)
    q = w.raw.reshape(-1, 36)
    s = Q8Storage.from_blocks(q[:, :4].copy().view("<f4").reshape(-1), q[:, 4:].copy().view(np.int8), 32 * 64)
    with pytest.raises(TypeError):
        eng.matmul(Tensor((32, 64), s), torch.zeros(64, 1, dtype=torch.float16, device="cuda"))


def test_ternary_gemv_reference_known_answers(eng):
    for case in json.loads((GOLD / "ternary_cases.json").read_text())["gemv"]:
        rows, cols = case["rows"], case["cols"]
        st = TernaryStorage(synth.pack_ternary(np.array(case["w"], np.int8)), rows * cols)
        y = eng.ternary_gemv(st, np.array(case["x"], np.float32), rows, cols)
        assert np.array_equal(y, np.array(case["want"], np.float32)), case["name"]


def test_ternary_gemv_matches_oracle(eng, orc):
    rows, cols = 2560, 6912
    t = synth.ternary(rows, cols, 19)
    x = synth.x_f32(cols, 19)
    y = eng.ternary_gemv(TernaryStorage(t.raw, rows * cols), x, rows, cols)
    assert rel_err(y, orc.ternary_gemv(t.raw, x, rows, cols)) <= TOL


def test_ternary_weights_stay_resident(eng, orc):
    """The row-aligned ternary upload is made once per storage and shape
    (the reference repacks and uploads on every TernaryGEMVGPU call) and is
    reused by both ternary_gemv and matmul, including several activation
    columns."""
    rows, cols = 256, 1000
    t = synth.ternary(rows, cols, 23)
    st = TernaryStorage(t.raw, rows * cols)
    x = synth.x_f32(cols, 23)
    y1 = eng.ternary_gemv(st, x, rows, cols)
    first = st._gpu_rows[1]
    y2 = eng.ternary_gemv(st, x, rows, cols)
    assert st._gpu_rows[1] is first and np.array_equal(y1, y2)
    assert rel_err(y1, orc.ternary_gemv(t.raw, x, rows, cols)) <= TOL
    xs = np.stack([synth.x_f32(cols, 30 + j) for j in range(3)], axis=1)  # [cols, 3]
    c = eng.matmul(Tensor((rows, cols), st), torch.from_numpy(np.ascontiguousarray(xs)).cuda()).cpu().numpy()
    assert st._gpu_rows[1] is first
    for j in range(3):
        assert rel_err(c[:, j], orc.ternary_gemv(t.raw, np.ascontiguousarray(xs[:, j]), rows, cols)) <= TOL
    with pytest.raises(ValueError):
        eng.ternary_gemv(st, x, rows + 1, cols)


def test_merged_qkv_storage_equals_separate_gemvs(eng, orc):
    """A merged Q/K/V storage (MergeQ4Storage) gives, in one GEMV, the three
    projections stacked: rows 0..4095 = Q, then K, then V."""
    from ztensor_amd.storage import merge_q4_storage

    K = 4096
    parts = [synth.q4_0(rows, K, 60 + i) for i, rows in enumerate((4096, 1024, 1024))]
    st = [Q4Storage.from_raw(p.raw, p.rows * K) for p in parts]
    x = torch.from_numpy(synth.x_f32(K, 60)).cuda()
    merged = eng.matmul(Tensor((6144, K), merge_q4_storage(*st)), x).cpu().numpy().reshape(-1)
    sep = np.concatenate([eng.matmul(Tensor((p.rows, K), s), x).cpu().numpy().reshape(-1) for p, s in zip(parts, st)])
    assert rel_err(merged, sep) <= 1e-6  # same kernel, row reduction order may differ with the row-tile size
    ref = np.concatenate([orc.gemm_f32_q4_nt(x.cpu().numpy(), p.raw, 1, p.rows, K) for p in parts])
    assert rel_err(merged, ref) <= TOL


def test_gemv_group_equals_separate_gemvs(eng, orc):
    """ROCmEngine.gemv_group: Q/K/V (and 9 matrices, past one launch's
    ZT_GROUP_MAX) in grouped launches equal the per-matrix GEMVs, and a
    non-Q4_0 member falls back to its own GEMV."""
    K = 4096
    parts = [synth.q4_0(rows, K, 70 + i) for i, rows in enumerate((4096, 1024, 1024))]
    ws = [Tensor((p.rows, K), Q4Storage.from_raw(p.raw, p.rows * K)) for p in parts]
    x = torch.from_numpy(synth.x_f32(K, 70)).cuda()
    outs = eng.gemv_group(ws, x)
    for p, y in zip(parts, outs):
        ref = orc.gemm_f32_q4_nt(x.cpu().numpy(), p.raw, 1, p.rows, K)
        assert rel_err(y.cpu().numpy(), ref) <= 1e-5
    many = [synth.q4_0(64 + 8 * i, 256, 80 + i) for i in range(9)]
    mw = [Tensor((p.rows, 256), Q4Storage.from_raw(p.raw, p.rows * 256)) for p in many]
    xs = torch.from_numpy(synth.x_f32(256, 80)).cuda()
    for p, y in zip(many, eng.gemv_group(mw, xs)):
        assert rel_err(y.cpu().numpy(), orc.gemm_f32_q4_nt(xs.cpu().numpy(), p.raw, 1, p.rows, 256)) <= 1e-5
    q8 = synth.q8_0(128, 256, 90)
    qb = q8.raw.reshape(-1, 36)
    q8s = Q8Storage.from_blocks(qb[:, :4].copy().view("<f4").reshape(-1), qb[:, 4:].copy().view(np.int8), 128 * 256)
    mixed = [mw[0], Tensor((128, 256), q8s)]
    y0, y1 = eng.gemv_group(mixed, xs)
    assert rel_err(y1.cpu().numpy(), orc.gemm_f32_q8_nt(xs.cpu().numpy(), q8.raw, 1, 128, 256)) <= 1e-5
    with pytest.raises(ValueError):
        eng.gemv_group(ws, xs)  # K mismatch


def test_engine_on_a_side_stream_runs_torch_work_on_that_stream(orc):
    """An engine built on a side stream makes its temporaries (transposes,
    pads, outputs, tiled copies, the split-K workspace) on that stream: every
    library call sees it as torch's current stream, and the results are right
    while the default stream is busy with other work."""
    side = torch.cuda.Stream()
    eng = ROCmEngine(0, stream=side)
    seen = []
    real_call = eng.lib.call

    def spy(name, *args):
        seen.append(torch.cuda.current_stream().cuda_stream)
        return real_call(name, *args)

    eng.lib = type("L", (), {})()
    for attr in dir(real_call.__self__):
        if attr.startswith("zt_"):
            setattr(eng.lib, attr, getattr(real_call.__self__, attr))
    eng.lib.call = spy
    rows, K = 512, 1024
    w = synth.q4_0(rows, K, 71)
    st = Q4Storage.from_raw(w.raw, rows * K)
    q8 = synth.q8_0(rows, K, 72)
    qb = q8.raw.reshape(-1, 36)
    s8 = Q8Storage.from_blocks(qb[:, :4].copy().view("<f4").reshape(-1), qb[:, 4:].copy().view(np.int8), rows * K)
    x = synth.x_f32(K * 8, 71).reshape(K, 8)
    busy = torch.randn(4096, 4096, device="cuda")
    for _ in range(8):  # keep the default stream busy meanwhile
        busy = busy @ busy * 1e-3
    xb = torch.from_numpy(x).cuda()
    torch.cuda.synchronize()
    c_b = eng.matmul(xb.t().contiguous(), Tensor((K, rows), st))  # B side: transposes on the engine stream
    c_t = eng.matmul(Tensor((rows, K), s8), xb)  # batched tiled Q8_0: tiled copy + workspace
    ys = eng.gemv_group([Tensor((rows, K), st)], xb[:, 0].contiguous())
    side.synchronize()
    assert seen and all(sid == side.cuda_stream for sid in seen)
    ref4 = orc.gemm_f32_q4_nt(np.ascontiguousarray(x.T), w.raw, 8, rows, K)
    ref8 = orc.gemm_f32_q8_nt(np.ascontiguousarray(x.T), q8.raw, 8, rows, K)
    assert rel_err(c_b.cpu().numpy().reshape(-1), ref4.reshape(-1)) <= TOL
    assert rel_err(c_t.cpu().numpy().T.reshape(-1), ref8.reshape(-1)) <= TOL
    assert rel_err(ys[0].cpu().numpy(), ref4.reshape(8, rows)[0]) <= TOL
    torch.cuda.synchronize()
