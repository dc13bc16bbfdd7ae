"""The entry point that allocates nothing (kq_gemv_multix_mfma_noalloc_dev),
through the C ABI: the same results as kq_gemv_multix_mfma_dev bit for bit,
on two calls in a row (the second smaller, so it reuses the static scratch
the first one filled), for both matrix-core types; sizes beyond the static
array are refused with a message before any launch."""
import numpy as np
import pytest

import stratum_amd as K
from conftest import same_values
from stratum_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()
    yield
    torch.cuda.synchronize()


def run(fn, qtype, w, xs, N, Kd):
    B = xs.shape[0]
    dw = torch.from_numpy(w).cuda()
    dx = torch.from_numpy(np.ascontiguousarray(xs).reshape(-1)).cuda()
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    sh = torch.cuda.current_stream().cuda_stream
    rc = fn(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd, sh)
    assert rc == 0, K.lib().kq_last_error().decode()
    torch.cuda.synchronize()
    return dy.cpu().numpy().reshape(B, N)


@pytest.mark.parametrize("qtype", [12, 14])
def test_noalloc_matches_allocating_entry(qtype):
    L = K.lib()
    # first call: larger (several K-parts, 3 stream groups); second: smaller
    for B, N, Kd, seed in ((40, 3000, 4096, 1), (17, 700, 1024, 2)):
        w = synth.tensor(qtype, N, Kd, 7000 + seed)
        xs = np.stack([synth.gaussian(synth.rng(7100 + 97 * seed + s), Kd) for s in range(B)])
        got = run(L.kq_gemv_multix_mfma_noalloc_dev, qtype, w, xs, N, Kd)
        want = run(L.kq_gemv_multix_mfma_dev, qtype, w, xs, N, Kd)
        print(f"noalloc type={qtype} B={B} N={N} K={Kd}: "
              f"{int(np.sum(got.view(np.uint32) == want.view(np.uint32)))}/{got.size} identical",
              flush=True)
        assert np.isfinite(got).all()
        assert same_values(got, want), (qtype, B, N, Kd)


def test_noalloc_refuses_sizes_beyond_the_array():
    L = K.lib()
    # B = 64 streams of K = 131072 need 32 MiB of x planes alone, plus the
    # x sums; the buffers are real (and large enough), so nothing could be
    # read out of bounds even if the refusal were missing
    B, N, Kd = 64, 16, 131072
    w = torch.zeros(N * L.kq_row_bytes(14, Kd), dtype=torch.uint8, device="cuda")
    x = torch.zeros(B * Kd, dtype=torch.float32, device="cuda")
    y = torch.zeros(B * N, dtype=torch.float32, device="cuda")
    rc = L.kq_gemv_multix_mfma_noalloc_dev(14, w.data_ptr(), x.data_ptr(), y.data_ptr(), B, N,
                                           Kd, None)
    torch.cuda.synchronize()
    assert rc == -1
    assert torch.count_nonzero(y).item() == 0
    msg = L.kq_last_error().decode()
    assert "scratch" in msg and str(K.NOALLOC_SCRATCH_BYTES) in msg, msg
