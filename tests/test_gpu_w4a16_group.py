"""Grouped batch-1 W4A16 GEMV (zt_gemv_w4a16sz_group_f32): matrices on
packed (scale, zero) dwords that read the same fp16 activation vector, one
launch, each in its own upload.

Bars: every matrix bit for bit equal to the single-matrix
zt_gemv_w4a16sz_f32 (the same steps, waves and reduction tree) and within
1e-5 of the oracle's restatement of MatMulW4A16 (dequantize, then
SgemmSimd, compute/w4a16.go:71-119); outputs past a matrix's rows are never
written."""
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


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def run_group(lib, orc, shapes, K, group=128, seed0=120, check_oracle=True):
    x16 = synth.x_f16(K, seed0)
    xd = dev(x16)
    mats, keep, refs, singles = [], [], [], []
    for i, rows in enumerate(shapes):
        w = synth.w4a16(max(rows, 1), K, seed0 + 1 + i, group=group)
        p, s, z = dev(w.packed), dev(w.scales), dev(w.zeros)
        szr = torch.empty(max(w.scales.size, 1), dtype=torch.int32, device="cuda")
        lib.call("zt_w4a16_pack_szr", s.data_ptr(), z.data_ptr(), w.rows, K, group, szr.data_ptr(), stream())
        y = torch.full((max(rows, 1) + 8,), float("nan"), dtype=torch.float32, device="cuda")
        keep += [p, s, z, szr, y]
        mats.append((p.data_ptr(), szr.data_ptr(), y.data_ptr(), rows))
        if rows:
            ys = torch.empty(rows, dtype=torch.float32, device="cuda")
            lib.call("zt_gemv_w4a16sz_f32", p.data_ptr(), szr.data_ptr(), xd.data_ptr(), ys.data_ptr(), rows, K, group,
                     stream())
            singles.append(ys)
            refs.append(orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, group) if check_oracle else None)
        else:
            singles.append(None)
            refs.append(None)
    lib.call("zt_gemv_w4a16sz_group_f32", _lib.w4a16_gemv_descs(mats), len(mats), xd.data_ptr(), K, group, stream())
    torch.cuda.synchronize()
    return [keep[5 * i + 4].cpu().numpy() for i in range(len(shapes))], [
        s.cpu().numpy() if s is not None else None for s in singles], refs


@pytest.mark.parametrize("shapes,K", [([8192, 1024, 1024], 8192), ([28672, 28672], 8192), ([4096, 1024, 1024], 4096),
                                      ([8192], 28672), ([7, 0, 130, 33], 1024), ([3, 5, 9, 11, 13, 17, 19, 23], 256),
                                      ([100, 60], 16384)])
def test_w4a16_group_bit_exact(lib, orc, shapes, K):
    """Llama-3-70B q/k/v (8192 + 2 x 1024 rows at K = 8192) and gate/up,
    Llama-3-8B q/k/v, the down shape alone (K = 28672, 4 steps a wave),
    ragged row counts with an empty matrix, eight matrices, K = 16384."""
    print(f"w4a16 group shapes={shapes} K={K}", flush=True)
    big = sum(shapes) * K > 200_000_000
    grouped, singles, refs = run_group(lib, orc, shapes, K, check_oracle=not big)
    for g, s, r, rows in zip(grouped, singles, refs, shapes):
        if rows == 0:
            assert np.all(np.isnan(g))
            continue
        assert np.array_equal(g[:rows].view(np.uint32), s.view(np.uint32))
        if r is not None:
            assert rel_err(g[:rows], r) <= TOL
        assert np.all(np.isnan(g[rows:]))


def test_w4a16_group_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    one = _lib.w4a16_gemv_descs([(p, p, p, 4)])
    f = lib.zt_gemv_w4a16sz_group_f32
    assert f(one, 0, p, 128, 128, stream()) == 1                                    # n = 0
    assert f(one, _lib.GROUP_MAX + 1, p, 128, 128, stream()) == 1                   # n too large
    assert f(one, 1, p + 8, 128, 128, stream()) == 1                                # misaligned x
    assert f(one, 1, p, 128, 48, stream()) == 1                                     # group % 32
    assert f(one, 1, p, 96, 64, stream()) == 1                                      # K % group
    assert f(_lib.w4a16_gemv_descs([(p + 4, p, p, 4)]), 1, p, 128, 128, stream()) == 1  # W alignment
    assert f(_lib.w4a16_gemv_descs([(p, 0, p, 4)]), 1, p, 128, 128, stream()) == 1      # no scales
    bad = _lib.w4a16_gemv_descs([(p, p, p, 4)])
    bad[0].reserved = 1
    assert f(bad, 1, p, 128, 128, stream()) == 1
    assert f(_lib.w4a16_gemv_descs([(0, 0, 0, 0)]), 1, p, 128, 128, stream()) == 0    # all empty


def test_engine_gemv_group_w4a16(lib, orc):
    """ROCmEngine.gemv_group on GPTQ weights with an fp16 activation vector:
    one grouped launch, each result equal to the engine's own batch-1 matmul
    of that weight, bit for bit, and within 1e-5 of the oracle."""
    from ztensor_amd.engine import ROCmEngine
    from ztensor_amd.storage import GPTQStorage, Tensor

    K = 4096
    x16 = synth.x_f16(K, 125)
    xd = torch.from_numpy(x16.view(np.float16).copy()).cuda()
    eng = ROCmEngine()
    ts, refs = [], []
    for i, rows in enumerate([1024, 256, 256]):
        w = synth.w4a16(rows, K, 126 + i)
        st = GPTQStorage.from_raw(w.packed.reshape(-1), w.scales.reshape(-1), w.zeros.reshape(-1), rows * K, 128, 4)
        ts.append(Tensor((rows, K), st))
        refs.append(orc.w4a16_matmul(w.packed, w.scales, w.zeros, x16, rows, K, 1, 128))
    outs = eng.gemv_group(ts, xd)
    for t, y, r in zip(ts, outs, refs):
        single = eng.matmul(t, xd.reshape(K, 1)).reshape(-1)
        assert np.array_equal(y.cpu().numpy().view(np.uint32), single.cpu().numpy().view(np.uint32))
        assert rel_err(y.cpu().numpy(), r) <= TOL
