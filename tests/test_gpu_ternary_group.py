"""Grouped BitNet GEMV (zt_ternary_gemv_i8_group): ternary matrices that read
the same int8 activation vector in one launch, each in its own row-aligned
upload.

Bars: every matrix bit for bit equal to the oracle's restatement of
TernaryGEMV (compute/ternary_gemv.go:12-77) on float(q) times the scale
product, and to the single-matrix zt_ternary_gemv_i8 (exact integer sums);
outputs of other matrices are never written."""
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


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()


def run_group(lib, orc, shapes, K, seed0=90):
    """shapes: row counts; returns (grouped outputs, single outputs, references)."""
    q, xs = synth.x_i8(K, seed0)
    qd = dev(q)
    xsd = torch.tensor([xs], dtype=torch.float32, device="cuda")
    mats, refs, keep = [], [], []
    for i, rows in enumerate(shapes):
        t = synth.ternary(rows, K, seed0 + 1 + i)
        W = dev(orc.ternary_repack_rows(t.raw, rows, K))
        ws = torch.tensor([t.w_scale], dtype=torch.float32, device="cuda")
        y = torch.full((max(rows, 1) + 8,), float("nan"), dtype=torch.float32, device="cuda")
        keep += [W, ws, y]
        mats.append((W.data_ptr(), ws.data_ptr(), y.data_ptr(), rows))
        refs.append(orc.ternary_gemv_i8(t.raw, q, xs, t.w_scale, rows, K) if rows else np.zeros(0, np.float32))
    lib.call("zt_ternary_gemv_i8_group", _lib.ternary_gemv_descs(mats), len(mats), qd.data_ptr(), xsd.data_ptr(), K,
             stream())
    torch.cuda.synchronize()
    grouped = [keep[3 * i + 2].cpu().numpy() for i in range(len(shapes))]
    singles = []
    for (w, ws, _, rows), i in zip(mats, range(len(mats))):
        y = torch.empty(max(rows, 1), dtype=torch.float32, device="cuda")
        if rows:
            lib.call("zt_ternary_gemv_i8", w, qd.data_ptr(), xsd.data_ptr(), ws, y.data_ptr(), rows, K, stream())
        singles.append(y.cpu().numpy()[:rows])
    return grouped, singles, refs


@pytest.mark.parametrize("shapes,K", [([2560, 2560, 2560], 2560), ([6912, 6912], 2560), ([2560], 6912),
                                      ([640, 2560, 640], 2560), ([7, 1, 130], 128), ([33, 0, 5], 4096),
                                      ([3, 5, 9, 11], 256), ([100, 60], 96)])
def test_ternary_group_bit_exact(lib, orc, shapes, K):
    """BitNet-2B shapes (q/k/v with the reference config's 2560 rows and
    with 640-row k/v, gate/up, down), ragged row counts, an empty matrix,
    four matrices and K % 64 != 0 (one launch per matrix)."""
    print(f"ternary group shapes={shapes} K={K}", flush=True)
    grouped, singles, refs = run_group(lib, orc, shapes, K)
    for g, s, r, rows in zip(grouped, singles, refs, shapes):
        assert np.array_equal(g[:rows].view(np.uint32), np.asarray(r, np.float32).view(np.uint32))
        assert np.array_equal(g[:rows].view(np.uint32), s.view(np.uint32))
        assert np.all(np.isnan(g[rows:]))  # rows past the matrix are not written


def test_ternary_group_invalid_arguments(lib):
    t = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = t.data_ptr()
    one = _lib.ternary_gemv_descs([(p, p, p, 4)])
    f = lib.zt_ternary_gemv_i8_group
    assert f(one, 0, p, p, 64, stream()) == 1                                  # n = 0
    assert f(one, _lib.GROUP_MAX + 1, p, p, 64, stream()) == 1                 # n too large
    assert f(one, 1, p + 8, p, 64, stream()) == 1                              # misaligned x
    assert f(one, 1, p, 0, 64, stream()) == 1                                  # no x scale
    assert f(_lib.ternary_gemv_descs([(0, p, p, 4)]), 1, p, p, 64, stream()) == 1  # no weights
    bad = _lib.ternary_gemv_descs([(p, p, p, 4)])
    bad[0].reserved = 1
    assert f(bad, 1, p, p, 64, stream()) == 1
    assert f(_lib.ternary_gemv_descs([(0, 0, 0, 0)]), 1, p, p, 64, stream()) == 0  # all empty
