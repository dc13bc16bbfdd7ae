"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Bar (written per test):
  * dequantization: bit-exact (NaN == NaN);
  * GEMV: per-element |y - y_ref| / max(|y_ref|, 1e-6) <= 1e-5, the
    reference's own ASSERT_REL (quant_test.c:34-43), with greedy argmax
    identical; the number of outputs that are not bit-identical is printed.
Full-size tensors (27B shapes) are checked on a row sample against the
oracle plus size-independent properties: determinism across runs and
independence from the launch decomposition.
"""
import ctypes
import os

import numpy as np
import pytest

import stratum_amd as K
from conftest import GOLDEN_FILES, load_golden, same_values
from oracle import oracle as O
from stratum_amd import synth

pytestmark = pytest.mark.gpu

REL_TOL = 1e-5
TYPES = [12, 14, 10, 42]

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def device():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    K.lib()
    yield
    torch.cuda.synchronize()


def stream():
    return torch.cuda.current_stream().cuda_stream


def dev(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def gpu_gemv(qtype, w, x, N, Kd, add=None):
    dw, dx = dev(w), dev(x)
    dy = torch.empty(N, dtype=torch.float32, device="cuda")
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
    assert rel.size == 0 or rel.max() <= REL_TOL, what
    if fin.all() and want.size > 1:
        assert np.argmax(got) == np.argmax(want), what


# ------------------------------------------------------------- dequant
def test_fp16_exhaustive_via_dequant():
    """Every fp16 bit pattern as Q4_K d with scale 1, min 0, quant 1:
    weight 0 of the block is exactly fp16 -> fp32 of d."""
    n = 65536
    b = np.zeros((n, 144), np.uint8)
    b[:, 0:2] = np.arange(n, dtype=np.uint32).astype(np.uint16).view(np.uint8).reshape(n, 2)
    sc = np.ones((n, 8), np.uint8)
    b[:, 4:16] = synth.pack_q4k_scales(sc, np.zeros((n, 8), np.uint8))
    b[:, 16:144] = 0x11
    y = gpu_dequant(12, b.reshape(-1), n).reshape(n, 256)
    want = np.arange(n, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float32)
    assert same_values(y[:, 0], want)


@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_golden_bit_exact(qtype):
    for case, d in load_golden(GOLDEN_FILES[qtype]).items():
        N, Kd = (int(v) for v in d["shape"])
        print(f"dequant golden type={qtype} case={case} N={N} K={Kd}", flush=True)
        got = gpu_dequant(qtype, d["w"], N * Kd // 256)
        assert same_values(got, d["deq"]), (qtype, case)


@pytest.mark.parametrize("qtype", TYPES)
def test_dequant_random_bit_exact(port, qtype):
    N, Kd = 64, 4096
    w = synth.tensor(qtype, N, Kd, 21)
    got = gpu_dequant(qtype, w, N * Kd // 256)
    assert same_values(got, port.dequant(qtype, w, N, Kd))


# ---------------------------------------------------------------- GEMV
@pytest.mark.parametrize("qtype", TYPES)
def test_gemv_golden(qtype):
    for case, d in load_golden(GOLDEN_FILES[qtype]).items():
        N, Kd = (int(v) for v in d["shape"])
        print(f"gemv golden type={qtype} case={case} N={N} K={Kd}", flush=True)
        got = gpu_gemv(qtype, d["w"], d["x"], N, Kd)
        check_close(got, d["y"], f"golden {qtype}/{case}")


def test_gemv_config0_q4k_1024(port):
    """Q4_K 1024 x 1024, batch 1, fixed seed."""
    N = Kd = 1024
    w = synth.tensor(12, N, Kd, 1)
    x = synth.gaussian(synth.rng(2), Kd)
    check_close(gpu_gemv(12, w, x, N, Kd), port.gemv(12, w, x, N, Kd, threads=8), "cfg0")


@pytest.mark.parametrize("qtype", TYPES)
@pytest.mark.parametrize("N,Kd", [(1, 256), (7, 768), (300, 1024), (129, 3072), (64, 6144)])
def test_gemv_shapes(port, qtype, N, Kd):
    w = synth.tensor(qtype, N, Kd, 100 + N)
    x = synth.gaussian(synth.rng(200 + Kd), Kd)
    print(f"gemv type={qtype} N={N} K={Kd}", flush=True)
    check_close(gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd, threads=8),
                f"{qtype} {N}x{Kd}")


@pytest.mark.parametrize("qtype", TYPES)
def test_gemv_add_epilogue(port, qtype):
    N, Kd = 200, 2048
    w = synth.tensor(qtype, N, Kd, 5)
    x = synth.gaussian(synth.rng(6), Kd)
    add = synth.gaussian(synth.rng(7), N)
    got = gpu_gemv(qtype, w, x, N, Kd, add=add)
    check_close(got, port.gemv(qtype, w, x, N, Kd, add=add), f"add {qtype}")
    # the add is one binary32 addition to the row's rounded result
    # (y[r] = add[r] + dot, stratum_linear.h:566-600)
    assert same_values(got, add + gpu_gemv(qtype, w, x, N, Kd))


@pytest.mark.parametrize("qtype,N,Kd", [(12, 17408, 5120), (14, 5120, 17408), (12, 6144, 5120),
                                        (12, 8192, 5120), (14, 8191, 5120), (42, 17408, 5120),
                                        (10, 17408, 5120), (14, 151936, 1024), (12, 5120, 6144),
                                        (12, 1024, 5120)])
def test_gemv_27b_shape_sampled(port, qtype, N, Kd, kq_env):
    """Full-size config shapes: 384 sampled rows against the oracle,
    bit-identical reruns, and the same bits under two other launch shapes
    (37 workgroups of 256 lanes; 512 lanes with two batches in flight per
    wave).  27B-class: gate/up, down, Q, the merged Q/K/V row count 8192 and
    a ragged 8191, type 42 and Q2_K gate, O (5120 x 6144) and K/V (1024 x 5120) alone;
    Qwen3-0.6B: the Q6_K LM head 151936 x 1024 (594 rows per workgroup, and
    several launches under the 37-workgroup decomposition, whose terms would
    not fit one launch's LDS)."""
    w = synth.tensor(qtype, N, Kd, 31)
    x = synth.gaussian(synth.rng(32), Kd)
    print(f"27b shape type={qtype} N={N} K={Kd}", flush=True)
    y = gpu_gemv(qtype, w, x, N, Kd)
    rows = np.unique(np.concatenate([np.random.default_rng(0).integers(0, N, 380),
                                     [0, 1, N - 2, N - 1]]))
    check_close(y[rows], port.gemv_rows(qtype, w, x, rows, Kd), f"27b {qtype} {N}x{Kd}")
    assert same_values(gpu_gemv(qtype, w, x, N, Kd), y)
    kq_env(KQ_GRID=37, KQ_WG_THREADS=256)
    assert same_values(gpu_gemv(qtype, w, x, N, Kd), y)
    kq_env(KQ_GRID=0, KQ_WG_THREADS=512, KQ_DEPTH=2)
    assert same_values(gpu_gemv(qtype, w, x, N, Kd), y)


# -------------------------------------------------- reference-signature ABI
def test_host_abi_dispatch_multix_group(port):
    """kq_linear_init + GgufTensor-style descriptors (offsets into one blob),
    host x/y as in st_linear_dispatch / _add / multix / st_q4k_group."""
    Kd = 1024
    specs = [(12, 512), (14, 256), (10, 128), (42, 64)]
    parts, tensors, off = [], [], 0
    for i, (t, N) in enumerate(specs):
        wb = synth.tensor(t, N, Kd, 40 + i)
        tensors.append((K.make_tensor(t, N, Kd, off, name=f"t{i}".encode()), wb, t, N))
        parts.append(wb)
        off += wb.size
    blob = np.concatenate(parts)
    K.WeightRegion(blob)
    x = synth.gaussian(synth.rng(50), Kd)
    for desc, wb, t, N in tensors:
        check_close(K.linear_dispatch(desc, x, N, Kd), port.gemv(t, wb, x, N, Kd), f"abi {t}")
        add = synth.gaussian(synth.rng(51), N)
        check_close(K.linear_dispatch_add(desc, x, add, N, Kd),
                    port.gemv(t, wb, x, N, Kd, add=add), f"abi add {t}")
        xs = [synth.gaussian(synth.rng(60 + s), Kd) for s in range(5)]
        ys = K.linear_multix(desc, xs, N, Kd)
        for s in range(5):
            assert same_values(ys[s], K.linear_dispatch(desc, xs[s], N, Kd))
    (d0, w0, t0, n0), (d1, w1, t1, n1), (d2, w2, t2, n2) = tensors[:3]
    g = K.q4k_group(x, Kd, (d0, n0), (d1, n1), (d2, n2))
    assert same_values(g[0], K.linear_dispatch(d0, x, n0, Kd))
    assert same_values(g[1], K.linear_dispatch(d1, x, n1, Kd))
    assert same_values(g[2], K.linear_dispatch(d2, x, n2, Kd))
    # a descriptor past the registered bytes is refused (-1), not read
    bad = K.make_tensor(12, 512, Kd, blob.size - 100)
    y = np.empty(512, np.float32)
    assert K.lib().kq_linear_dispatch(ctypes.byref(bad), K._fptr(x), K._fptr(y), 512, Kd) == -1


# ------------------------------------------------------- batched segments
def test_segments_row_limit():
    """A segment of 2^24 rows or more is refused with a message before any
    launch (the kernel's row arithmetic is 24-bit); one row fewer is not
    refused for that reason."""
    import torch
    w = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    x = torch.zeros(256, device="cuda")
    y = torch.zeros(16, device="cuda")
    L = K.lib()
    seg = K.segment(12, 256, 1 << 24, [w.data_ptr()], x.data_ptr(), y.data_ptr())
    assert L.kq_gemv_segments_dev((K.KqSegment * 1)(seg), 1, None) == -1
    assert "2^24" in L.kq_last_error().decode()
    seg = K.segment(12, 256, 16, [w.data_ptr()], x.data_ptr(), y.data_ptr())
    sh = torch.cuda.current_stream().cuda_stream
    assert L.kq_gemv_segments_dev((K.KqSegment * 1)(seg), 1, sh) == 0
    torch.cuda.synchronize()
    assert torch.count_nonzero(y).item() == 0


def test_segments_layer_set_matches_single_launches(port):
    """A layer's matvecs in ONE launch (kq_gemv_segments_dev): each output is
    bit-identical to its own kq_gemv_dev launch, and matches the oracle."""
    H, F, Q, KV = 1024, 3072, 2048, 512
    specs = [("q", 12, Q, H, "h"), ("k", 12, KV, H, "h"), ("v", 14, KV, H, "h"),
             ("gate", 12, F, H, "h"), ("up", 10, F, H, "h"),
             ("o", 12, H, Q, "a"), ("down", 14, H, F, "f"), ("extra", 42, 256, F, "f")]
    xs = {"h": synth.gaussian(synth.rng(1), H), "a": synth.gaussian(synth.rng(2), Q),
          "f": synth.gaussian(synth.rng(3), F)}
    dx = {k: dev(v) for k, v in xs.items()}
    ws, dws, dys, segs = {}, {}, {}, []
    for i, (name, t, N, Kd, xn) in enumerate(specs):
        ws[name] = synth.tensor(t, N, Kd, 70 + i)
        dws[name] = dev(ws[name])
        dys[name] = torch.empty(N, dtype=torch.float32, device="cuda")
        segs.append(K.segment(t, Kd, N, [dws[name].data_ptr()], dx[xn].data_ptr(),
                              dys[name].data_ptr()))
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for name, t, N, Kd, xn in specs:
        got = dys[name].cpu().numpy()
        single = gpu_gemv(t, ws[name], xs[xn], N, Kd)
        assert same_values(got, single), name
        check_close(got, port.gemv(t, ws[name], xs[xn], N, Kd, threads=8), f"seg {name}")


@pytest.mark.parametrize("order", [(12, 12, 14), (14, 12, 14, 14, 12), (14, 14, 12, 12, 14, 12, 12, 14)])
def test_segments_mixed_q4k_q6k(port, order):
    """Q4_K and Q6_K tensors on one x in one segment list (a Q4_K_M layer's
    Q, K, V with a Q6_K V): one launch of the Q4_K+Q6_K kernel; every output
    equals its own single launch bit for bit and the oracle within the GEMV
    bound."""
    H = 2048
    x = synth.gaussian(synth.rng(8450), H)
    rows = [1024, 128, 160, 96, 64, 300, 17, 256]
    dx = dev(x)
    ws, dws, dys, segs = [], [], [], []
    for i, t in enumerate(order):
        ws.append(synth.tensor(t, rows[i], H, 8460 + i))
        dws.append(dev(ws[-1]))
        dys.append(torch.full((rows[i],), float("nan"), dtype=torch.float32, device="cuda"))
        segs.append(K.segment(t, H, rows[i], [dws[-1].data_ptr()], dx.data_ptr(),
                              dys[-1].data_ptr()))
    print(f"mixed q4k/q6k order={order}", flush=True)
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i, t in enumerate(order):
        got = dys[i].cpu().numpy()
        assert same_values(got, gpu_gemv(t, ws[i], x, rows[i], H)), (i, t)
        if i < 3:
            check_close(got, port.gemv(t, ws[i], x, rows[i], H, threads=8), f"seg {i}")


def test_segments_mixed_q4k_q6k_groups_and_add(port):
    """The Q4_K+Q6_K kernel with the other part forms: a Q4_K segment of
    three groups (separate weight bases, one x) with a residual add, a Q6_K
    segment of two groups each on its own x (x_stride), and a plain Q4_K
    one, in one list: every output equals its own single launch (with the
    add as one binary32 add after the row)."""
    H, N = 1024, 96
    r = synth.rng(8480)
    x = synth.gaussian(r, H)
    xs2 = np.stack([synth.gaussian(r, H) for _ in range(2)])
    add = synth.gaussian(r, 3 * N)
    wa = [synth.tensor(12, N, H, 8481 + g) for g in range(3)]
    wb = [synth.tensor(14, N, H, 8485 + g) for g in range(2)]
    wc = synth.tensor(12, 40, H, 8488)
    dx, dx2, dadd = dev(x), dev(xs2.reshape(-1)), dev(add)
    dwa, dwb, dwc = [dev(w) for w in wa], [dev(w) for w in wb], dev(wc)
    ya = torch.full((3 * N,), float("nan"), dtype=torch.float32, device="cuda")
    yb = torch.full((2 * N,), float("nan"), dtype=torch.float32, device="cuda")
    yc = torch.full((40,), float("nan"), dtype=torch.float32, device="cuda")
    segs = [K.segment(12, H, N, [d.data_ptr() for d in dwa], dx.data_ptr(), ya.data_ptr(),
                      add_ptr=dadd.data_ptr()),
            K.segment(14, H, N, [d.data_ptr() for d in dwb], dx2.data_ptr(), yb.data_ptr(),
                      x_stride=H),
            K.segment(12, H, 40, [dwc.data_ptr()], dx.data_ptr(), yc.data_ptr())]
    print("mixed q4k/q6k groups + add", flush=True)
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    got_a, got_b, got_c = ya.cpu().numpy(), yb.cpu().numpy(), yc.cpu().numpy()
    for g in range(3):
        want = gpu_gemv(12, wa[g], x, N, H, add=add[g * N:(g + 1) * N])
        assert same_values(got_a[g * N:(g + 1) * N], want), g
    for g in range(2):
        assert same_values(got_b[g * N:(g + 1) * N], gpu_gemv(14, wb[g], xs2[g], N, H)), g
    assert same_values(got_c, gpu_gemv(12, wc, x, 40, H))


def test_segments_groups_expert_slices(port):
    """MoE-style segments: groups with separate weight bases; gate/up share
    x, down uses one x per group (x_stride)."""
    H, F, E = 512, 768, 5
    r = np.random.default_rng(9)
    x = synth.gaussian(synth.rng(4), H)
    gate = [synth.tensor(12, F, H, 100 + e) for e in range(E)]
    down = [synth.tensor(12, H, F, 200 + e) for e in range(E)]
    a = np.stack([synth.gaussian(synth.rng(300 + e), F) for e in range(E)])
    dgate = [dev(g) for g in gate]
    ddown = [dev(d) for d in down]
    dx, da = dev(x), dev(a.reshape(-1))
    yg = torch.empty(E * F, dtype=torch.float32, device="cuda")
    yd = torch.empty(E * H, dtype=torch.float32, device="cuda")
    add = synth.gaussian(synth.rng(5), E * H)
    dadd = dev(add)
    segs = [K.segment(12, H, F, [t.data_ptr() for t in dgate], dx.data_ptr(), yg.data_ptr()),
            K.segment(12, F, H, [t.data_ptr() for t in ddown], da.data_ptr(), yd.data_ptr(),
                      x_stride=F, add_ptr=dadd.data_ptr())]
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    g_out = yg.cpu().numpy().reshape(E, F)
    d_out = yd.cpu().numpy().reshape(E, H)
    for e in range(E):
        check_close(g_out[e], port.gemv(12, gate[e], x, F, H), f"gate e{e}")
        check_close(d_out[e], port.gemv(12, down[e], a[e], H, F, add=add[e * H:(e + 1) * H]),
                    f"down e{e}")


def test_segments_same_x_other_stride(port):
    """Two multi-group segments on the same x pointer, K and group count but
    different x strides: the second must restage its own x rows, not reuse
    the first segment's (each output equals its own launch)."""
    H, F, G = 512, 256, 3
    xs = np.stack([synth.gaussian(synth.rng(640 + g), 2 * H) for g in range(G)]).reshape(-1)
    dx = dev(xs)
    ws = [[synth.tensor(12, F, H, 650 + 10 * i + g) for g in range(G)] for i in range(2)]
    dws = [[dev(w) for w in row] for row in ws]
    ys = [torch.empty(G * F, dtype=torch.float32, device="cuda") for _ in range(2)]
    strides = [H, 2 * H]                  # rows g*H (overlapping) and g*2H of the same buffer
    segs = [K.segment(12, H, F, [d.data_ptr() for d in dws[i]], dx.data_ptr(), ys[i].data_ptr(),
                      x_stride=strides[i]) for i in range(2)]
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i in range(2):
        got = ys[i].cpu().numpy().reshape(G, F)
        for g in range(G):
            xg = xs[g * strides[i]:g * strides[i] + H]
            assert same_values(got[g], gpu_gemv(12, ws[i][g], xg, F, H)), (i, g)
            check_close(got[g], port.gemv(12, ws[i][g], xg, F, H), f"stride {strides[i]} g{g}")


def test_segments_rejects_bad_input():
    bad = K.segment(12, 1000, 16, [0], 0, 0)
    with pytest.raises(RuntimeError):
        K.gemv_segments_dev([bad])


# ----------------------------------------------------- scaled-x window
# Q4_K, Q2_K and type 42 run on x scaled by 2^64 when every finite nonzero
# |x| lies in [2^-41, 2^52); otherwise the workgroups restage x unscaled and
# take the convert path.  Both must give the reference's values.
WINDOW_CASES = {
    "low-edge-in": [2.0 ** -41, -(2.0 ** -41)],
    "low-edge-out": [2.0 ** -42],
    "high-edge-in": [np.float32(2.0 ** 52) - np.float32(2.0 ** 28), -(2.0 ** 51)],
    "high-edge-out": [2.0 ** 52],
    "subnormal": [1e-40],
    "zeros-inf-nan": [0.0, -0.0, np.inf, np.nan],
}


@pytest.mark.parametrize("case", sorted(WINDOW_CASES))
@pytest.mark.parametrize("qtype", [12, 10, 42, 14])
def test_gemv_x_window_edges(port, qtype, case):
    N, Kd = 96, 1024
    w = synth.tensor(qtype, N, Kd, 500 + qtype)
    x = synth.gaussian(synth.rng(501), Kd)
    special = np.asarray(WINDOW_CASES[case], np.float32)
    x[7:7 + special.size] = special
    x[900:900 + special.size] = special[::-1]
    check_close(gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd),
                f"{K.TYPE_NAMES[qtype]} window {case}")


@pytest.mark.parametrize("scale", [2.0 ** -45, 2.0 ** -135])
@pytest.mark.parametrize("qtype", [12, 10, 42])
def test_gemv_x_all_below_window(port, qtype, scale):
    """Every x near 2^-45 (normal) or 2^-135 (subnormal): scaled products
    would fall below the binary32 normal range and lose bits or vanish, so
    only the unscaled fallback matches."""
    N, Kd = 64, 1024
    w = synth.tensor(qtype, N, Kd, 520 + qtype)
    x = (synth.gaussian(synth.rng(521), Kd).astype(np.float64) * scale).astype(np.float32)
    assert np.count_nonzero(x) > Kd // 2
    got, want = gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd)
    check_close(got, want, f"{K.TYPE_NAMES[qtype]} x ~ {scale:.1e}")
    # |y| is far below the 1e-6 floor of the relative bound, which then
    # cannot tell a wrong result; the binary64 sums of these few binary32
    # terms are exact, so the results must be bit-identical
    assert same_values(got, want), f"{K.TYPE_NAMES[qtype]} x ~ {scale:.1e} not bit-identical"


@pytest.mark.parametrize("where", [None, 5000, 9000])
@pytest.mark.parametrize("Kd", [6144, 12288])
@pytest.mark.parametrize("qtype", [14, 10, 42])
def test_gemv_x_staging_rounds(port, qtype, Kd, where, kq_env):
    """x longer than one staging round of the workgroup (256 lanes: 4096
    values per round for 16-value groups): two rounds (the second loaded
    with the first) and three, with an out-of-window x value in the second
    or third round (it must still switch every workgroup to the unscaled
    path)."""
    kq_env(KQ_WG_THREADS=256)
    N = 96
    w = synth.tensor(qtype, N, Kd, 540 + qtype)
    x = synth.gaussian(synth.rng(541), Kd)
    if where is not None and where < Kd:
        x[where] = 2.0 ** 60
    print(f"staging rounds type={qtype} K={Kd} big x at {where}", flush=True)
    check_close(gpu_gemv(qtype, w, x, N, Kd), port.gemv(qtype, w, x, N, Kd),
                f"{K.TYPE_NAMES[qtype]} K={Kd} rounds, x[{where}] = 2^60")


@pytest.mark.parametrize("wide", [False, True])
def test_segments_shared_x_across_types(port, wide):
    """Segments that share one x in different ways: sums recomputed from a
    scaled x (Q4_K -> type 42), Q6_K reading a scaled x, and -- with one x
    value outside the window -- every type on the unscaled fallback."""
    H = 1024
    x = synth.gaussian(synth.rng(600), H)
    if wide:
        x[33] = 2.0 ** 60
    specs = [(12, 256), (42, 192), (10, 128), (14, 320), (10, 64), (12, 96)]
    dx = dev(x)
    ws, dws, dys, segs = [], [], [], []
    for i, (t, N) in enumerate(specs):
        ws.append(synth.tensor(t, N, H, 610 + i))
        dws.append(dev(ws[-1]))
        dys.append(torch.empty(N, dtype=torch.float32, device="cuda"))
        segs.append(K.segment(t, H, N, [dws[-1].data_ptr()], dx.data_ptr(), dys[-1].data_ptr()))
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i, (t, N) in enumerate(specs):
        check_close(dys[i].cpu().numpy(), port.gemv(t, ws[i], x, N, H),
                    f"shared x seg {i} {K.TYPE_NAMES[t]} wide={wide}")


def test_segments_merged_same_input_parts(port):
    """Same-input single-tensor segments are merged into one row space of up
    to 4 parts of any sizes (then a new one starts); groups of 3 experts with
    one x each run as parts too.  Every output matches its own launch."""
    H = 768
    x = synth.gaussian(synth.rng(700), H)
    dx = dev(x)
    sizes = [100, 37, 300, 64, 5, 129]
    ws = [synth.tensor(12, n, H, 710 + i) for i, n in enumerate(sizes)]
    dws = [dev(w) for w in ws]
    dys = [torch.empty(n, dtype=torch.float32, device="cuda") for n in sizes]
    add = synth.gaussian(synth.rng(701), sizes[2])
    dadd = dev(add)
    segs = [K.segment(12, H, n, [dws[i].data_ptr()], dx.data_ptr(), dys[i].data_ptr(),
                      add_ptr=dadd.data_ptr() if i == 2 else None)
            for i, n in enumerate(sizes)]
    E, F = 3, 512
    ex = [synth.tensor(14, F, H, 720 + e) for e in range(E)]
    dex = [dev(t) for t in ex]
    xe = np.stack([synth.gaussian(synth.rng(730 + e), H) for e in range(E)])
    dxe = dev(xe.reshape(-1))
    ye = torch.empty(E * F, dtype=torch.float32, device="cuda")
    segs.append(K.segment(14, H, F, [t.data_ptr() for t in dex], dxe.data_ptr(), ye.data_ptr(),
                          x_stride=H))
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i, n in enumerate(sizes):
        got = dys[i].cpu().numpy()
        a = add if i == 2 else None
        assert same_values(got, gpu_gemv(12, ws[i], x, n, H, add=a)), f"part {i}"
        check_close(got, port.gemv(12, ws[i], x, n, H, add=a), f"merged part {i} ({n} rows)")
    got = ye.cpu().numpy().reshape(E, F)
    for e in range(E):
        check_close(got[e], port.gemv(14, ex[e], xe[e], F, H), f"expert part {e}")


# ------------------------------------------------------------ multi-stream
def gpu_multix(qtype, w, xs, N, Kd):
    B = xs.shape[0]
    dw, dx = dev(w), dev(xs.reshape(-1))
    dy = torch.empty(B * N, dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd, stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy().reshape(B, N)


@pytest.mark.parametrize("qtype", TYPES + [13, 11, 8])
@pytest.mark.parametrize("B,N,Kd", [(2, 300, 1024), (3, 129, 768), (8, 96, 3072),
                                    (16, 64, 1024), (19, 40, 2048)])
def test_multix_bit_identical_to_single_stream(port, qtype, B, N, Kd):
    """One weight pass for B streams (every block type, Q5_K / Q3_K / Q8_0
    included): every stream equals its own single-stream launch bit for
    bit, and the oracle within the bound."""
    w = synth.tensor(qtype, N, Kd, 800 + qtype + B)
    xs = np.stack([synth.gaussian(synth.rng(810 + s), Kd) for s in range(B)])
    got = gpu_multix(qtype, w, xs, N, Kd)
    for s in range(B):
        assert same_values(got[s], gpu_gemv(qtype, w, xs[s], N, Kd)), f"stream {s}"
    for s in (0, B - 1):
        check_close(got[s], port.gemv(qtype, w, xs[s], N, Kd), f"multix {K.TYPE_NAMES[qtype]} B={B} s={s}")


@pytest.mark.parametrize("qtype", [12, 10, 14, 13, 11, 8])
def test_multix_window_fallback(port, qtype):
    """One stream with a value outside the scaled window sends the launch to
    the exact path; every stream still equals its single-stream result."""
    N, Kd, B = 80, 1024, 4
    w = synth.tensor(qtype, N, Kd, 830 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(840 + s), Kd) for s in range(B)])
    xs[2, 17] = 2.0 ** 60
    got = gpu_multix(qtype, w, xs, N, Kd)
    for s in range(B):
        assert same_values(got[s], gpu_gemv(qtype, w, xs[s], N, Kd)), f"stream {s}"
        check_close(got[s], port.gemv(qtype, w, xs[s], N, Kd), f"multix window s={s}")


@pytest.mark.parametrize("qtype", [12, 10, 14, 42, 13, 11, 8])
def test_multix_tiled_window_fallback(port, qtype):
    """x too long to stage whole (tiles of a few chunks), with one stream
    outside the scaled window: the tiled exact path, still bit-identical."""
    N, Kd, B = 200, 5120, 8
    w = synth.tensor(qtype, N, Kd, 870 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(880 + s), Kd) for s in range(B)])
    xs[5, 4097] = -(2.0 ** 61)
    got = gpu_multix(qtype, w, xs, N, Kd)
    for s in range(B):
        assert same_values(got[s], gpu_gemv(qtype, w, xs[s], N, Kd)), f"stream {s}"
    check_close(got[5], port.gemv(qtype, w, xs[5], N, Kd), "tiled window s=5")


@pytest.mark.parametrize("qtype,B", [(12, 17), (12, 40), (12, 64), (12, 70), (13, 40), (11, 64),
                                     (8, 70)])
def test_multix_member_chunks(port, qtype, B):
    """More than 16 streams: members staged 16 at a time within one weight
    pass (and more than 64 in two launches)."""
    N, Kd = 100, 1024
    w = synth.tensor(qtype, N, Kd, 890 + B)
    xs = np.stack([synth.gaussian(synth.rng(900 + s), Kd) for s in range(B)])
    got = gpu_multix(qtype, w, xs, N, Kd)
    for s in range(B):
        assert same_values(got[s], gpu_gemv(qtype, w, xs[s], N, Kd)), f"stream {s}"


@pytest.mark.parametrize("tensor,B", [("gate", 8), ("down", 8), ("gate", 16), ("up", 16),
                                      ("down", 16), ("gate", 64), ("up", 64), ("down", 64),
                                      ("gate_q5k", 16), ("down_q3k", 16), ("down_q80", 64)])
def test_multix_27b_sampled(port, tensor, B):
    """27B gate / up (Q4_K 17408 x 5120) and down (Q6_K 5120 x 17408) with
    B = 8, 16 and 64 streams, the MULTISEQ shapes bench.py times (the
    planner picks other member chunks and x tiles at each B), and the same
    shapes as Q5_K, Q3_K and Q8_0: every stream against its single-stream
    launch bit for bit, and 256 sampled rows of two streams against the
    oracle."""
    qtype, N, Kd, seed = {"gate": (12, 17408, 5120, 850), "up": (12, 17408, 5120, 851),
                          "down": (14, 5120, 17408, 852), "gate_q5k": (13, 17408, 5120, 853),
                          "down_q3k": (11, 5120, 17408, 854),
                          "down_q80": (8, 5120, 17408, 855)}[tensor]
    w = synth.tensor(qtype, N, Kd, seed)
    xs = np.stack([synth.gaussian(synth.rng(860 + s), Kd) for s in range(B)])
    print(f"multix 27B {tensor} B={B}", flush=True)
    dw, dx = dev(w), dev(xs.reshape(-1))
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd,
                      stream=stream())
    d1 = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    for s in range(B):
        K.gemv_dev(qtype, dw.data_ptr(), dx.data_ptr() + 4 * s * Kd, d1.data_ptr() + 4 * s * N,
                   N, Kd, stream=stream())
    torch.cuda.synchronize()
    got = dy.cpu().numpy().reshape(B, N)
    single = d1.cpu().numpy().reshape(B, N)
    for s in range(B):
        assert same_values(got[s], single[s]), f"stream {s}"
    rows = np.random.default_rng(3 + B).choice(N, 256, replace=False)
    rb = K.lib().kq_row_bytes(qtype, Kd)
    sub = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    for s in (0, B - 3):
        check_close(got[s][rows], port.gemv(qtype, sub, xs[s], len(rows), Kd),
                    f"multix 27B {tensor} B={B} s={s}")
