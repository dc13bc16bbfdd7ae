"""GPU parity of the remaining dispatch types (stratum_linear.h:533-541):
Q5_K, Q3_K and Q8_0 through the block kernels, F16 and F32 through the
dense kernel, against the CPU oracle (and, through the golden fixtures, the
reference's own compiled scalar routines).

Bars (per test):
  * dequantization: bit-exact;
  * Q5_K / Q3_K / Q8_0 GEMV: per element |y - y_ref| / max(|y_ref|, 1e-6)
    <= 1e-5 with argmax identical (quant_test.c:34-43), bit-identical count
    printed; decomposition-independent and repeatable bit for bit;
  * F16 / F32 GEMV: within one binary32 ulp of the oracle's element-order
    binary64 sum (both round a binary64 sum of exact products; only the
    binary64 grouping differs).
"""
import numpy as np
import pytest

import stratum_amd as K
from conftest import GOLDEN_FILES, load_golden, same_values
from oracle import oracle as O
from stratum_amd import synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
NEW = [13, 11, 8]
DENSE = [1, 0]


@pytest.fixture(scope="module", autouse=True)
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()
    yield
    torch.cuda.synchronize()


def stream():
    return torch.cuda.current_stream().cuda_stream


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_gemv(qtype, w, x, N, Kd, add=None):
    dw, dx = dev(w), dev(x)
    dy = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
    da = dev(add) if add is not None else None
    K.gemv_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), N, Kd,
               add_ptr=da.data_ptr() if da is not None else None, stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy()


def gpu_dequant(qtype, w, nblocks):
    dw = dev(w)
    dy = torch.empty(nblocks * 256, dtype=torch.float32, device="cuda")
    K.dequant_dev(qtype, dw.data_ptr(), dy.data_ptr(), nblocks, stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy()


def check_close(got, want, what):
    fin = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want)), what
    assert np.array_equal(got[np.isinf(want)], want[np.isinf(want)]), what
    rel = O.rel_err(got[fin], want[fin])
    exact = int(np.sum(got[fin].view(np.uint32) == want[fin].view(np.uint32)))
    print(f"{what}: max rel err {rel.max() if rel.size else 0:.3e}, "
          f"bit-identical {exact}/{int(fin.sum())}", flush=True)
    assert rel.size == 0 or rel.max() <= 1e-5, what
    if fin.all() and want.size > 1:
        assert np.argmax(got) == np.argmax(want), what


def check_ulp(got, want, what):
    """|got - want| <= one binary32 ulp of want, per element."""
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ulp = np.spacing(np.abs(want)).astype(np.float64)
    exact = int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
    print(f"{what}: max |d|/ulp {np.max(d / ulp):.2f}, bit-identical {exact}/{want.size}", flush=True)
    assert np.all(d <= ulp), what


# ---------------------------------------------------------------- dequant
@pytest.mark.parametrize("qtype", NEW)
def test_dequant_golden_bit_exact(qtype):
    for case, d in load_golden(GOLDEN_FILES[qtype]).items():
        N, Kd = (int(v) for v in d["shape"])
        print(f"dequant golden type={qtype} case={case}", flush=True)
        assert same_values(gpu_dequant(qtype, d["w"], N * Kd // 256), d["deq"]), (qtype, case)


@pytest.mark.parametrize("qtype", NEW + DENSE)
def test_dequant_random_bit_exact(port, qtype):
    N, Kd = 48, 2048
    w = synth.tensor(qtype, N, Kd, 31)
    assert same_values(gpu_dequant(qtype, w, N * Kd // 256), port.dequant(qtype, w, N, Kd))


# ------------------------------------------------------------------- GEMV
@pytest.mark.parametrize("qtype", NEW)
def test_gemv_golden(qtype):
    for case, d in load_golden(GOLDEN_FILES[qtype]).items():
        N, Kd = (int(v) for v in d["shape"])
        print(f"gemv golden type={qtype} case={case} N={N} K={Kd}", flush=True)
        check_close(gpu_gemv(qtype, d["w"], d["x"], N, Kd), d["y"], f"golden {qtype}/{case}")


@pytest.mark.parametrize("qtype", NEW)
@pytest.mark.parametrize("N,Kd", [(1, 256), (7, 768), (300, 1024), (129, 3072), (64, 6144)])
def test_gemv_shapes(port, qtype, N, Kd):
    w = synth.tensor(qtype, N, Kd, 100 + N)
    x = synth.gaussian(synth.rng(200 + Kd), Kd)
    print(f"gemv type={qtype} N={N} K={Kd}", flush=True)
    check_close(gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd, threads=8),
                f"{K.TYPE_NAMES[qtype]} {N}x{Kd}")


@pytest.mark.parametrize("qtype", NEW)
def test_gemv_add_epilogue(port, qtype):
    N, Kd = 200, 2048
    w = synth.tensor(qtype, N, Kd, 5)
    x = synth.gaussian(synth.rng(6), Kd)
    add = synth.gaussian(synth.rng(7), N)
    got = gpu_gemv(qtype, w, x, N, Kd, add=add)
    check_close(got, port.gemv(qtype, w, x, N, Kd, add=add), f"add {qtype}")
    assert same_values(got, add + gpu_gemv(qtype, w, x, N, Kd))


@pytest.mark.parametrize("qtype,N,Kd", [(13, 17408, 5120), (8, 5120, 5120), (11, 6144, 5120),
                                        (13, 5120, 17408)])
def test_gemv_large_sampled(port, qtype, N, Kd, kq_env):
    """27B-class shapes: sampled rows against the oracle, a bit-identical
    rerun and the same bits under 37 workgroups of 256 lanes."""
    w = synth.tensor(qtype, N, Kd, 33)
    x = synth.gaussian(synth.rng(34), Kd)
    print(f"large type={qtype} N={N} K={Kd}", flush=True)
    y = gpu_gemv(qtype, w, x, N, Kd)
    rows = np.unique(np.concatenate([np.random.default_rng(1).integers(0, N, 380), [0, N - 1]]))
    check_close(y[rows], port.gemv_rows(qtype, w, x, rows, Kd), f"large {qtype} {N}x{Kd}")
    assert same_values(gpu_gemv(qtype, w, x, N, Kd), y)
    kq_env(KQ_GRID=37, KQ_WG_THREADS=256)
    assert same_values(gpu_gemv(qtype, w, x, N, Kd), y)


WINDOW = {"low-out": [2.0 ** -42], "high-out": [2.0 ** 52], "subnormal": [1e-40],
          "zeros-inf-nan": [0.0, -0.0, np.inf, np.nan], "tiny-all": None}


@pytest.mark.parametrize("case", sorted(WINDOW))
@pytest.mark.parametrize("qtype", NEW)
def test_gemv_x_outside_scaled_window(port, qtype, case):
    """Q5_K multiplies by byte select on x staged x 2^64; values outside the
    window send it to the exact convert path.  Q3_K and Q8_0 read x as
    staged; all must give the reference's values."""
    N, Kd = 96, 1024
    w = synth.tensor(qtype, N, Kd, 500 + qtype)
    x = synth.gaussian(synth.rng(501), Kd)
    if WINDOW[case] is None:
        x = (x.astype(np.float64) * 2.0 ** -45).astype(np.float32)
    else:
        sp = np.asarray(WINDOW[case], np.float32)
        x[7:7 + sp.size] = sp
        x[900:900 + sp.size] = sp[::-1]
    got, want = gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd)
    check_close(got, want, f"{K.TYPE_NAMES[qtype]} window {case}")
    if WINDOW[case] is None:
        assert same_values(got, want)


def test_segments_mixed_types_split(port):
    """One segment list mixing the core types with Q5_K, Q3_K, Q8_0 and a
    dense F16 tensor on one x (the host splits it into launches a kernel
    instantiation takes, and x scaled by a Q4_K segment is read by Q3_K
    and Q8_0 ones): every output equals its own single launch."""
    H = 1024
    x = synth.gaussian(synth.rng(650), H)
    specs = [(12, 256), (13, 192), (13, 64), (11, 128), (14, 96), (8, 200), (1, 80), (12, 64)]
    dx = dev(x)
    ws, dws, dys, segs = [], [], [], []
    for i, (t, N) in enumerate(specs):
        ws.append(synth.tensor(t, N, H, 660 + i))
        dws.append(dev(ws[-1]))
        dys.append(torch.full((N,), float("nan"), dtype=torch.float32, device="cuda"))
        segs.append(K.segment(t, H, N, [dws[-1].data_ptr()], dx.data_ptr(), dys[-1].data_ptr()))
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i, (t, N) in enumerate(specs):
        got = dys[i].cpu().numpy()
        assert same_values(got, gpu_gemv(t, ws[i], x, N, H)), (i, t)
        if t not in DENSE:
            check_close(got, port.gemv(t, ws[i], x, N, H), f"mixed seg {i} {K.TYPE_NAMES[t]}")


@pytest.mark.parametrize("qtype", NEW + DENSE)
@pytest.mark.parametrize("N,Kd,B", [(100, 1024, 5), (2100, 512, 9)])
def test_multix_equals_single_stream(qtype, N, Kd, B):
    """Every stream bit-identical to its single-stream launch.  Dense rows:
    the small shape runs one stream per wave, the large one eight streams
    per wave sharing each weight load (the second group partial)."""
    w = synth.tensor(qtype, N, Kd, 700 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(710 + s), Kd) for s in range(B)])
    dw, dx = dev(w), dev(xs.reshape(-1))
    dy = torch.empty(B * N, dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd, stream=stream())
    torch.cuda.synchronize()
    got = dy.cpu().numpy().reshape(B, N)
    for s in range(B):
        assert same_values(got[s], gpu_gemv(qtype, w, xs[s], N, Kd)), s


@pytest.mark.parametrize("qtype", [13, 8])
@pytest.mark.parametrize("B", [1, 3])
def test_moe_gather_other_types(port, qtype, B):
    """MoE experts in Q5_K / Q8_0: one token through the device-selected
    single-stream kernel, several tokens through the multi-x kernel; every
    member equals its slice's single GEMV."""
    n_exp, H, F, k = 16, 512, 256, 4
    gate = synth.tensor(qtype, n_exp * F, H, 720)
    r = np.random.default_rng(721 + B)
    sel = np.stack([r.choice(n_exp, k, replace=False) for _ in range(B)]).astype(np.int32)
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    dg, dx, ds = dev(gate), dev(x), dev(sel.reshape(-1))
    y = torch.full((B * k * F,), float("nan"), dtype=torch.float32, device="cuda")
    sl = F * K.lib().kq_row_bytes(qtype, H)
    op = K.moe_op(qtype, F, H, [dg.data_ptr()], sl, dx.data_ptr(), k, [y.data_ptr()])
    K.moe_gemv_dev(op, ds.data_ptr(), B, k, n_exp, stream())
    torch.cuda.synchronize()
    got = y.cpu().numpy().reshape(B * k, F)
    for m in range(B * k):
        e = sel.reshape(-1)[m]
        xm = x[(m // k) * H:(m // k + 1) * H]
        ws = gate[e * sl:(e + 1) * sl]
        assert same_values(got[m], gpu_gemv(qtype, ws, xm, F, H)), m
    m = B * k - 1
    e = sel.reshape(-1)[m]
    check_close(got[m], port.gemv(qtype, gate[e * sl:(e + 1) * sl],
                                  x[(m // k) * H:(m // k + 1) * H], F, H), f"moe {qtype} B={B}")


# ------------------------------------------------------------------ dense
@pytest.mark.parametrize("qtype", DENSE)
@pytest.mark.parametrize("N,Kd", [(1, 256), (128, 768), (128, 2048), (1000, 4096), (37, 20480)])
def test_dense_gemv(port, qtype, N, Kd):
    """F16 / F32 rows, including K % 512 == 256 (an F16 step half full) and
    K beyond what the kernel stages in LDS (x read from memory)."""
    w = synth.tensor(qtype, N, Kd, 800 + N)
    x = synth.gaussian(synth.rng(801 + Kd), Kd)
    print(f"dense type={qtype} N={N} K={Kd}", flush=True)
    check_ulp(gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd, threads=8),
              f"{K.TYPE_NAMES[qtype]} {N}x{Kd}")


@pytest.mark.parametrize("qtype", DENSE)
def test_dense_add_and_exact_cases(port, qtype):
    N, Kd = 64, 1024
    w = synth.tensor(qtype, N, Kd, 820)
    x = synth.gaussian(synth.rng(821), Kd)
    add = synth.gaussian(synth.rng(822), N)
    got = gpu_gemv(qtype, w, x, N, Kd, add=add)
    assert same_values(got, add + gpu_gemv(qtype, w, x, N, Kd))
    # integer weights and x: every sum exact, so the result is exact
    r = np.random.default_rng(823)
    wi = r.integers(-8, 8, (N, Kd)).astype(np.float32)
    wb = (wi.astype(np.float16).view(np.uint8) if qtype == 1 else wi.view(np.uint8)).reshape(-1).copy()
    xi = r.integers(-50, 50, Kd).astype(np.float32)
    assert np.array_equal(gpu_gemv(qtype, wb, xi, N, Kd),
                          (wi.astype(np.float64) @ xi).astype(np.float32))
