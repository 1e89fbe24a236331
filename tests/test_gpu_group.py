"""Grouped Q4_0 GEMV (zt_gemm_q4_group_f32): several matrices that share one
activation vector in one launch, each in its own RawBytesGPU upload.

Bars: every matrix of a group within 1e-5 (normwise, max|y - y_ref| /
max|y_ref|) of the oracle's GemmF32Q4NT (internal/xblas/gemm_quant.go:81-157);
bit-identical to the single-matrix launch when both use the same rows per
wave; rows that a descriptor does not own are never written."""
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


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def upload(lib, rows, K, seed):
    w = synth.q4_0(rows, K, seed)
    nblk = rows * K // 32
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    return w, torch.from_numpy(host).cuda(), lib.zt_q4_gpu_data_offset(nblk)


def run_group(lib, orc, shapes, K, seed0=40):
    s = torch.cuda.current_stream().cuda_stream
    x = synth.x_f32(K, seed0)
    xd = torch.from_numpy(x).cuda()
    mats = [upload(lib, rows, K, seed0 + 1 + i) for i, rows in enumerate(shapes)]
    ys = [torch.full((max(rows, 1) + 8,), 7.0, dtype=torch.float32, device="cuda") for rows in shapes]
    descs = _lib.q4_gemv_descs([(a.data_ptr(), off, y.data_ptr(), rows)
                                for (w, a, off), y, rows in zip(mats, ys, shapes)])
    lib.call("zt_gemm_q4_group_f32", descs, len(shapes), xd.data_ptr(), K, s)
    torch.cuda.synchronize()
    out = []
    for (w, a, off), y, rows in zip(mats, ys, shapes):
        yh = y.cpu().numpy()
        assert np.all(yh[rows:] == 7.0), "a grouped launch wrote past its matrix's rows"
        if rows:
            ref = orc.gemm_f32_q4_nt(x, w.raw, 1, rows, K, threads=orc.nthreads())
            err = rel_err(yh[:rows], ref)
            print(f"group rows={rows} K={K}: rel err {err:.2e}", flush=True)
            assert err <= TOL
        out.append((a, off, yh[:rows]))
    return xd, out


@pytest.mark.parametrize("shapes,K", [
    ([4096, 1024, 1024], 4096),   # Llama-3-8B q, k, v
    ([14336, 14336], 4096),       # gate, up
    ([4096], 14336),              # down (K = 14336: two steps a wave)
    ([17, 0, 3, 130], 96),        # ragged rows, an empty matrix, K not a multiple of 512
    ([5, 9, 33, 64, 65, 1, 2, 8], 2080),  # ZT_GROUP_MAX matrices
])
def test_q4_group_matches_oracle(lib, orc, shapes, K):
    run_group(lib, orc, shapes, K)


def test_q4_group_bit_identical_to_single_launch(lib, orc):
    # every matrix >= 2048 rows: the single launch and the group both run 8 rows per wave
    K = 4096
    xd, out = run_group(lib, orc, [4096, 2048, 14336], K)
    s = torch.cuda.current_stream().cuda_stream
    for a, off, yg in out:
        rows = yg.size
        y1 = torch.empty(rows, dtype=torch.float32, device="cuda")
        lib.call("zt_gemm_q4_f32", a.data_ptr(), xd.data_ptr(), y1.data_ptr(), rows, K, 1, off, s)
        assert np.array_equal(y1.cpu().numpy().view(np.uint32), yg.view(np.uint32))


def test_q4_group_long_rows_fall_back_to_single_launches(lib, orc):
    # K > 16384 is past the fixed-step kernel: one launch per matrix, same results
    run_group(lib, orc, [64, 96], 28672)


def test_q4_group_in_captured_graph_replays(lib, orc):
    K = 4096
    shapes = [1024, 1024]
    mats = [upload(lib, r, K, 60 + i) for i, r in enumerate(shapes)]
    x = synth.x_f32(K, 59)
    xd = torch.from_numpy(x).cuda()
    ys = [torch.empty(r, dtype=torch.float32, device="cuda") for r in shapes]
    descs = _lib.q4_gemv_descs([(a.data_ptr(), off, y.data_ptr(), r) for (w, a, off), y, r in zip(mats, ys, shapes)])
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(g):
            lib.call("zt_gemm_q4_group_f32", descs, 2, xd.data_ptr(), K, torch.cuda.current_stream().cuda_stream)
    refs = [orc.gemm_f32_q4_nt(x, w.raw, 1, r, K, threads=orc.nthreads()) for (w, a, off), r in zip(mats, shapes)]
    for _ in range(3):
        for y in ys:
            y.fill_(0.0)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for y, ref in zip(ys, refs):
            assert rel_err(y.cpu().numpy(), ref) <= TOL
