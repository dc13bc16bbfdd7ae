"""The matrix-core MULTISEQ path (kq_gemv_multix_mfma_dev): a tolerance
path, checked against the exact multi-stream GEMV (which equals the
single-stream and oracle arithmetic).  Bound, per output:
    |y_mfma - y_exact| <= 2e-6 * sum_l |w_l| |x_l|
(the row's dequantized weights times |x|: an upper bound on the sizes of the
terms whose binary32 rounding order differs, and on the 2^-21 relative
rounding of x to its two fp16 planes), i.e. a few binary32 ulps of the
terms; the test also prints the max relative error against the oracle
and the share of outputs within the GEMV bound of 1e-5."""
import numpy as np
import pytest

import stratum_amd as K
from oracle import oracle as O
from stratum_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
TOL = 2e-6


@pytest.fixture(scope="module", autouse=True)
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()
    yield
    torch.cuda.synchronize()


def stream():
    return torch.cuda.current_stream().cuda_stream


def run(fn, qtype, dw, xs, B, N, Kd):
    dx = torch.from_numpy(np.ascontiguousarray(xs.reshape(-1))).cuda()
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    fn(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd, stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy().reshape(B, N)


def magnitude(port, qtype, w, xs, rows, Kd):
    """sum_l |w_l| |x_l| per (stream, sampled row), from the oracle's dequant."""
    rb = K.lib().kq_row_bytes(qtype, Kd)
    deq = np.stack([port.dequant(qtype, w[r * rb:(r + 1) * rb], 1, Kd) for r in rows]).astype(np.float64)
    return np.abs(xs.astype(np.float64)) @ np.abs(deq).T          # [B, rows]


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("B,N,Kd", [(16, 200, 2048), (17, 130, 1024), (33, 64, 3072),
                                    (64, 96, 2048), (16, 300, 512)])
def test_mfma_against_exact(port, qtype, B, N, Kd):
    w = synth.tensor(qtype, N, Kd, 950 + qtype + B)
    xs = np.stack([synth.gaussian(synth.rng(960 + s), Kd) for s in range(B)])
    dw = torch.from_numpy(w).cuda()
    got = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    exact = run(K.gemv_multix_dev, qtype, dw, xs, B, N, Kd)
    mag = magnitude(port, qtype, w, xs, range(N), Kd)
    err = np.abs(got.astype(np.float64) - exact.astype(np.float64))
    worst = (err / mag).max()
    rel = O.rel_err(got, exact)
    print(f"{K.TYPE_NAMES[qtype]} B={B} N={N} K={Kd}: max err/mag {worst:.2e}, "
          f"max rel err {rel.max():.2e}, within 1e-5: {np.mean(rel <= 1e-5) * 100:.2f}%")
    assert np.all(np.isfinite(got))
    assert worst <= TOL


@pytest.mark.parametrize("B", [16, 64])
@pytest.mark.parametrize("qtype,N,Kd", [(12, 17408, 5120), (14, 5120, 17408)])
def test_mfma_27b_sampled(port, qtype, N, Kd, B):
    """27B gate / down with 16 and 64 streams: every output against the exact
    path, sampled rows against the oracle."""
    w = synth.tensor(qtype, N, Kd, 970 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(980 + s), Kd) for s in range(B)])
    dw = torch.from_numpy(w).cuda()
    got = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    exact = run(K.gemv_multix_dev, qtype, dw, xs, B, N, Kd)
    rows = np.random.default_rng(5).choice(N, 128, replace=False)
    mag = magnitude(port, qtype, w, xs, rows, Kd)
    err = np.abs(got[:, rows].astype(np.float64) - exact[:, rows].astype(np.float64))
    assert (err / mag).max() <= TOL
    rb = K.lib().kq_row_bytes(qtype, Kd)
    sub = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    want = port.gemv(qtype, sub, xs[3], len(rows), Kd)
    rel = O.rel_err(got[3, rows], want)
    print(f"27B {K.TYPE_NAMES[qtype]}: max rel err vs oracle {rel.max():.2e}, "
          f"within 1e-5: {np.mean(O.rel_err(got, exact) <= 1e-5) * 100:.2f}%")
    assert np.all(np.isfinite(got))


@pytest.mark.parametrize("qtype,N,Kd", [(12, 131100, 256), (14, 65600, 512)])
def test_mfma_whole_row_blocks(port, qtype, N, Kd):
    """Enough row blocks (256 rows for Q4_K, 128 for Q6_K) for at least two
    per workgroup: whole row blocks per workgroup, no partial sums; the last
    block is ragged."""
    B = 16
    w = synth.tensor(qtype, N, Kd, 1000 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(1010 + s), Kd) for s in range(B)])
    dw = torch.from_numpy(w).cuda()
    got = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    exact = run(K.gemv_multix_dev, qtype, dw, xs, B, N, Kd)
    rows = np.concatenate([np.random.default_rng(6).choice(N, 250, replace=False),
                           np.arange(N - 6, N)])
    mag = magnitude(port, qtype, w, xs, rows, Kd)
    err = np.abs(got[:, rows].astype(np.float64) - exact[:, rows].astype(np.float64))
    print(f"{K.TYPE_NAMES[qtype]} N={N}: max err/mag {(err / mag).max():.2e}")
    assert np.all(np.isfinite(got))
    assert (err / mag).max() <= TOL


@pytest.mark.parametrize("qtype", [12, 14])
def test_mfma_more_than_64_streams(port, qtype):
    """B = 100 runs as chunks of 64 and 36 streams on one workspace."""
    B, N, Kd = 100, 96, 1024
    w = synth.tensor(qtype, N, Kd, 1020 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(1030 + s), Kd) for s in range(B)])
    dw = torch.from_numpy(w).cuda()
    got = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    exact = run(K.gemv_multix_dev, qtype, dw, xs, B, N, Kd)
    mag = magnitude(port, qtype, w, xs, range(N), Kd)
    err = np.abs(got.astype(np.float64) - exact.astype(np.float64))
    assert (err / mag).max() <= TOL


@pytest.mark.parametrize("qtype", [12, 14])
def test_mfma_wide_dynamic_range(port, qtype):
    """x scaled per stream to the binary exponent of its largest |x|: streams
    with outliers 1e4 above the rest, a tiny stream (1e-30), an all-zero
    stream, subnormal values and a huge stream (1e30) keep the bound."""
    B, N, Kd = 16, 80, 2048
    w = synth.tensor(qtype, N, Kd, 1040 + qtype)
    r = synth.rng(1041)
    xs = np.stack([synth.gaussian(synth.rng(1050 + s), Kd) for s in range(B)])
    for s in range(0, 6):                       # outliers
        idx = r.choice(Kd, 5, replace=False)
        xs[s, idx] *= np.float32(1e4)
    xs[6] *= np.float32(1e-30)
    xs[7] = 0.0
    xs[8, ::3] = np.float32(1e-40)              # subnormal
    xs[9] *= np.float32(1e30)
    xs = xs.astype(np.float32)
    dw = torch.from_numpy(w).cuda()
    got = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    exact = run(K.gemv_multix_dev, qtype, dw, xs, B, N, Kd)
    mag = magnitude(port, qtype, w, xs, range(N), Kd)
    err = np.abs(got.astype(np.float64) - exact.astype(np.float64))
    assert np.all(got[7] == 0.0)
    live = mag > 0
    print(f"{K.TYPE_NAMES[qtype]}: max err/mag {(err[live] / mag[live]).max():.2e}")
    assert np.all(np.isfinite(got))
    assert (err[live] / mag[live]).max() <= TOL


def test_mfma_repeatable_and_other_types_refused():
    """Two launches give the same bits (the partial sums are added in a
    fixed order); types without a matrix-core path return -1."""
    qtype, B, N, Kd = 12, 20, 150, 4096
    w = synth.tensor(qtype, N, Kd, 990)
    xs = np.stack([synth.gaussian(synth.rng(991 + s), Kd) for s in range(B)])
    dw = torch.from_numpy(w).cuda()
    a = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    b = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    with pytest.raises(RuntimeError, match="no MFMA path"):
        run(K.gemv_multix_mfma_dev, 10, dw, xs, B, N, Kd)
    # an xs that is not 16-byte aligned is refused before any launch (the
    # split kernel reads x as float4)
    dx = torch.from_numpy(np.ascontiguousarray(xs.reshape(-1))).cuda()
    dy = torch.zeros(B * N, dtype=torch.float32, device="cuda")
    for fn in (K.lib().kq_gemv_multix_mfma_dev, K.lib().kq_gemv_multix_mfma_noalloc_dev):
        rc = fn(qtype, dw.data_ptr(), dx.data_ptr() + 4, dy.data_ptr(), B - 1, N, Kd, None)
        assert rc == -1 and b"16-byte aligned" in K.lib().kq_last_error()


def test_mfma_reserved_workspace_allocates_nothing():
    """kq_reserve_mfma_workspace grows the workspace once; calls whose
    workspace fits (kq_gemv_multix_mfma_workspace_bytes) then leave the
    library's scratch unchanged, with the same results as before."""
    L = K.lib()
    qtype, N, Kd = 12, 1000, 4096
    need = {B: L.kq_gemv_multix_mfma_workspace_bytes(qtype, B, N, Kd) for B in (16, 40, 64)}
    assert all(v > 0 for v in need.values()), need
    assert L.kq_gemv_multix_mfma_workspace_bytes(10, 16, N, Kd) == -1
    assert L.kq_reserve_mfma_workspace(max(need.values())) == 0
    held = L.kq_scratch_bytes()
    assert held >= max(need.values())
    w = synth.tensor(qtype, N, Kd, 995)
    dw = torch.from_numpy(w).cuda()
    for B in (64, 16, 40):
        xs = np.stack([synth.gaussian(synth.rng(996 + s), Kd) for s in range(B)])
        a = run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd)
        assert L.kq_scratch_bytes() == held, B
        assert np.array_equal(a.view(np.uint32),
                              run(K.gemv_multix_mfma_dev, qtype, dw, xs, B, N, Kd).view(np.uint32))
    assert L.kq_reserve_mfma_workspace(-1) == -1
