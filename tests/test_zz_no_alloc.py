"""The allocation-free batched Q4_0 entry point (zt_gemm_q4t_f32_noalloc)
against the entry point it varies (zt_gemm_q4t_f32 with a caller
workspace), through the C ABI.

Bars: bit-identical outputs (the same kernels, the same split order), on two
calls in a row with the second on a smaller matrix (which reuses the
scratch array the first call left filled); within 1e-5 of the oracle's
GemmF32Q4NT; no device memory allocated by the calls after the first (the
static scratch array itself comes with the library's module on the first
call)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")

from ztensor_amd import _lib, synth  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return _lib.load()


def rel_err(y, ref) -> float:
    ref = np.asarray(ref, np.float64)
    return float(np.max(np.abs(np.asarray(y, np.float64) - ref)) / max(np.max(np.abs(ref)), 1e-30))


def tiled(lib, rows, K, seed):
    w = synth.q4_0(rows, K, seed)
    nblk = rows * K // 32
    host = np.empty(lib.zt_q4_gpu_bytes(nblk), np.uint8)
    lib.zt_q4_raw_to_gpu(w.raw.ctypes.data, nblk, host.ctypes.data)
    sep = torch.from_numpy(host).cuda()
    wt = torch.empty(lib.zt_q4_tiled_bytes(rows, K), dtype=torch.uint8, device="cuda")
    st = torch.empty(lib.zt_q4_tiled_scale_bytes(rows, K), dtype=torch.uint8, device="cuda")
    lib.call("zt_q4_tile", sep.data_ptr(), rows, K, lib.zt_q4_gpu_data_offset(nblk), wt.data_ptr(), st.data_ptr(),
             torch.cuda.current_stream().cuda_stream)
    return w, wt, st


def test_noalloc_equals_workspace_entry_point_on_two_calls(lib, orc):
    s = torch.cuda.current_stream().cuda_stream
    free_after = []
    for rows, K, N, seed in [(4096, 4096, 8, 101), (1024, 2048, 4, 102)]:
        need = lib.zt_gemm_q4t_workspace_bytes(rows, K, N)
        print(f"noalloc rows={rows} K={K} N={N} scratch={need}", flush=True)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES  # the K range is split: the scratch is used
        w, wt, st = tiled(lib, rows, K, seed)
        x = synth.x_f32(K * N, seed)
        xd = torch.from_numpy(x).cuda()
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
        c_ws = torch.empty(rows * N, dtype=torch.float32, device="cuda")
        c_na = torch.full((rows * N,), float("nan"), dtype=torch.float32, device="cuda")
        lib.call("zt_gemm_q4t_f32", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c_ws.data_ptr(), rows, K, N,
                 ws.data_ptr(), need, s)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        lib.call("zt_gemm_q4t_f32_noalloc", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c_na.data_ptr(), rows, K, N, s)
        torch.cuda.synchronize()
        free_after.append((free0, torch.cuda.mem_get_info()[0]))
        a, b = c_ws.cpu().numpy(), c_na.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
        xt = np.ascontiguousarray(x.reshape(K, N).T)
        ref = orc.gemm_f32_q4_nt(xt, w.raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T
        assert rel_err(b.reshape(rows, N), ref) <= 1e-5
    # the second call allocated nothing on the device
    assert free_after[1][0] == free_after[1][1], free_after


def test_noalloc_unsplit_call_and_oversized_request(lib, orc):
    s = torch.cuda.current_stream().cuda_stream
    rows, K, N = 64, 256, 16  # K not split: no scratch needed
    assert lib.zt_gemm_q4t_workspace_bytes(rows, K, N) == 0
    w, wt, st = tiled(lib, rows, K, 103)
    x = synth.x_f32(K * N, 103)
    xd = torch.from_numpy(x).cuda()
    c = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4t_f32_noalloc", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c.data_ptr(), rows, K, N, s)
    torch.cuda.synchronize()
    xt = np.ascontiguousarray(x.reshape(K, N).T)
    ref = orc.gemm_f32_q4_nt(xt, w.raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T
    assert rel_err(c.cpu().numpy().reshape(rows, N), ref) <= 1e-5
    p = wt.data_ptr()
    assert lib.zt_gemm_q4t_f32_noalloc(p, p, p, p, 128, 1 << 20, 8, s) == _lib.HIP_ERROR_OUT_OF_MEMORY


@pytest.mark.parametrize("rows,K,N", [(28672, 8192, 8), (8200, 28672, 4)])
def test_noalloc_past_the_scratch_runs_in_row_slices(lib, orc, rows, K, N):
    """Partials larger than the scratch (29 MB and 16 MB here): the call runs
    in slices of whole 128-row workgroup rows with the full call's K split,
    bit-identical to the workspace entry point, then a small call reuses the
    scratch as before.  8200 rows end in a partial slice and a partial tile."""
    s = torch.cuda.current_stream().cuda_stream
    need = lib.zt_gemm_q4t_workspace_bytes(rows, K, N)
    print(f"noalloc sliced rows={rows} K={K} N={N} partials={need}", flush=True)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    w, wt, st = tiled(lib, rows, K, 104)
    x = synth.x_f32(K * N, 104)
    xd = torch.from_numpy(x).cuda()
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    c_ws = torch.empty(rows * N, dtype=torch.float32, device="cuda")
    c_na = torch.full((rows * N,), float("nan"), dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4t_f32", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c_ws.data_ptr(), rows, K, N,
             ws.data_ptr(), need, s)
    lib.call("zt_gemm_q4t_f32_noalloc", wt.data_ptr(), st.data_ptr(), xd.data_ptr(), c_na.data_ptr(), rows, K, N, s)
    torch.cuda.synchronize()
    a, b = c_ws.cpu().numpy(), c_na.cpu().numpy()
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    xt = np.ascontiguousarray(x.reshape(K, N).T)
    ref = orc.gemm_f32_q4_nt(xt, w.raw, N, rows, K, threads=orc.nthreads()).reshape(N, rows).T
    assert rel_err(b.reshape(rows, N), ref) <= 1e-5
    # a smaller call after it, on the scratch the sliced call left filled
    rows2, K2 = 1024, 2048
    w2, wt2, st2 = tiled(lib, rows2, K2, 105)
    x2 = torch.from_numpy(synth.x_f32(K2 * 4, 105)).cuda()
    need2 = lib.zt_gemm_q4t_workspace_bytes(rows2, K2, 4)
    ws2 = torch.empty(max(need2, 16), dtype=torch.uint8, device="cuda")
    c1 = torch.empty(rows2 * 4, dtype=torch.float32, device="cuda")
    c2 = torch.empty(rows2 * 4, dtype=torch.float32, device="cuda")
    lib.call("zt_gemm_q4t_f32", wt2.data_ptr(), st2.data_ptr(), x2.data_ptr(), c1.data_ptr(), rows2, K2, 4,
             ws2.data_ptr(), need2, s)
    lib.call("zt_gemm_q4t_f32_noalloc", wt2.data_ptr(), st2.data_ptr(), x2.data_ptr(), c2.data_ptr(), rows2, K2, 4, s)
    torch.cuda.synchronize()
    assert np.array_equal(c1.cpu().numpy().view(np.uint32), c2.cpu().numpy().view(np.uint32))
