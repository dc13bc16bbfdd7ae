"""GPU parity of the int8-activation mode (type | KQ_INT8_ACT, Q4_K, Q6_K,
Q5_K, Q3_K and Q8_0: the reference's SDOT path, stratum_linear.h:376-489)
against the CPU
oracle's restatement (oracle/kq_oracle.c ko_gemv_i8, pinned by
tests/test_oracle_i8.py).

Bars:
  * the quantizer (kq_quantize_x_q8_dev): int8 values, scales and sums
    bit-exact;
  * GEMV: within one binary32 ulp of the oracle's binary64-term order (the
    terms are identical; only the binary64 grouping differs), bit-identical
    count printed; on exactly quantizable inputs bit-exact; against the
    reference's order (q*_dot_row_sdot_f's binary32 lanes) within those
    lanes' rounding bound (K/64 + 3) 2^-24 sum|term|;
  * decomposition: segments, multix streams, launch shapes and the
    host-pointer switch (kq_linear_set_sdot) give the same bits as a single
    launch.
"""
import numpy as np
import pytest

import stratum_amd as K
from conftest import same_values
from i8_cases import reciprocal_groups
from stratum_amd import INT8_ACT, TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, synth

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
I8_TYPES = [TYPE_Q4_K, TYPE_Q6_K, TYPE_Q5_K, TYPE_Q3_K, TYPE_Q8_0]
GROUP = {TYPE_Q4_K: 32, TYPE_Q6_K: 16, TYPE_Q5_K: 32, TYPE_Q3_K: 32, TYPE_Q8_0: 32}


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


def check_ulp(got, want, what):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ulp = np.spacing(np.abs(want)).astype(np.float64)
    exact = int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
    print(f"{what}: max |d|/ulp {np.max(d / ulp):.2f}, bit-identical {exact}/{want.size}",
          flush=True)
    assert np.all(np.isfinite(got)), what
    assert np.all(d <= ulp), what


def check_lanes(got, port, qtype, w, x, N, Kd, what):
    yf, mag = port.gemv_i8(qtype, w, x, N, Kd, sdot_f=True, with_mag=True)
    d = np.abs(got.astype(np.float64) - yf.astype(np.float64))
    bound = (Kd / 64 + 3) * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(yf.astype(np.float64))
    print(f"{what}: vs sdot_f max d/bound {np.max(d / np.maximum(bound, 1e-300)):.3f}",
          flush=True)
    assert np.all(d <= bound), what


# -------------------------------------------------------------- quantizer
@pytest.mark.parametrize("G", [32, 16])
@pytest.mark.parametrize("Kd", [256, 5120, 17408])
def test_quantize_bit_exact(port, G, Kd):
    r = synth.rng(8000 + Kd + G)
    x = synth.gaussian(r, Kd) * np.float32(2.0)
    x[0:G] = 0.0                                    # a zero group
    x[G:G + 8] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5]   # ties
    x[G + 8:2 * G] = 0.25
    # groups where fl(x * fl(1 / scale)) and fl(x / scale) round apart
    rx, _ = reciprocal_groups(G, min(8, Kd // G - 2))
    x[2 * G:2 * G + rx.size] = rx
    dx = dev(x)
    ng = Kd // G
    xq = torch.empty(Kd, dtype=torch.int8, device="cuda")
    xs = torch.empty(ng, dtype=torch.float32, device="cuda")
    sm = torch.empty(ng, dtype=torch.int32, device="cuda")
    print(f"quantize G={G} K={Kd}", flush=True)
    K.quantize_x_q8_dev(dx.data_ptr(), Kd, G, xq.data_ptr(), xs.data_ptr(), sm.data_ptr(),
                        stream=stream())
    torch.cuda.synchronize()
    wq, ws = port.quantize_q8(x, G)
    assert np.array_equal(xq.cpu().numpy(), wq)
    assert same_values(xs.cpu().numpy(), ws)
    assert np.array_equal(sm.cpu().numpy(), wq.reshape(-1, G).astype(np.int32).sum(axis=1))


# ------------------------------------------------------------------- GEMV
@pytest.mark.parametrize("qtype", I8_TYPES)
@pytest.mark.parametrize("N,Kd", [(1, 256), (3, 512), (65, 768), (300, 1024), (129, 3072),
                                  (64, 6144)])
def test_gemv_shapes(port, qtype, N, Kd):
    w = synth.tensor(qtype, N, Kd, 8100 + N)
    x = synth.gaussian(synth.rng(8200 + Kd), Kd)
    print(f"int8 gemv type={qtype} N={N} K={Kd}", flush=True)
    got = gpu_gemv(qtype | INT8_ACT, w, x, N, Kd)
    check_ulp(got, port.gemv_i8(qtype, w, x, N, Kd), f"i8 {K.TYPE_NAMES[qtype]} {N}x{Kd}")
    check_lanes(got, port, qtype, w, x, N, Kd, f"i8 {K.TYPE_NAMES[qtype]} {N}x{Kd}")


def pow2_blocks(qtype, r, nblocks):
    b = synth.blocks(qtype, r, nblocks).reshape(nblocks, -1)
    f16 = lambda v: np.array([v], np.float16).view(np.uint8)   # noqa: E731
    if qtype in (TYPE_Q4_K, TYPE_Q5_K):
        b[:, 0:2] = f16(2.0 ** -10)
        b[:, 2:4] = f16(2.0 ** -12)
    elif qtype == TYPE_Q6_K:
        b[:, 208:210] = f16(2.0 ** -10)
    elif qtype == TYPE_Q3_K:
        b[:, 108:110] = f16(2.0 ** -10)
    else:
        b.reshape(nblocks, 8, 34)[:, :, 0:2] = f16(2.0 ** -10)
    return b.reshape(-1)


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_gemv_exact_inputs(port, qtype):
    """power-of-two d / dmin and exactly quantizable x: every step is exact,
    so y == fl(sum dequant(w) * x) bit for bit"""
    r = synth.rng(8300 + qtype)
    N, Kd, G = 200, 1024, GROUP[qtype]
    w = pow2_blocks(qtype, r, N * Kd // 256)
    k = r.integers(-127, 128, Kd).astype(np.int32)
    k.reshape(-1, G)[:, 3] = 127
    x = k.astype(np.float32) * np.float32(2.0 ** -7)
    deq = port.dequant(qtype, w, N, Kd).reshape(N, Kd).astype(np.float64)
    want = (deq * x.astype(np.float64)).sum(axis=1).astype(np.float32)
    assert same_values(gpu_gemv(qtype | INT8_ACT, w, x, N, Kd), want)


@pytest.mark.parametrize("qtype,N,Kd", [(TYPE_Q4_K, 6144, 5120), (TYPE_Q4_K, 17408, 5120),
                                        (TYPE_Q6_K, 5120, 17408), (TYPE_Q6_K, 1024, 5120),
                                        (TYPE_Q5_K, 17408, 5120), (TYPE_Q3_K, 17408, 5120),
                                        (TYPE_Q8_0, 5120, 17408)])
def test_gemv_config_shapes(port, qtype, N, Kd, kq_env):
    """27B-class shapes: sampled rows against the oracle, a bit-identical
    rerun and the same bits under 37 workgroups of 256 lanes."""
    w = synth.tensor(qtype, N, Kd, 8400 + N)
    x = synth.gaussian(synth.rng(8401), Kd)
    print(f"int8 config type={qtype} N={N} K={Kd}", flush=True)
    y = gpu_gemv(qtype | INT8_ACT, w, x, N, Kd)
    rows = np.unique(np.concatenate([np.random.default_rng(2).integers(0, N, 300), [0, N - 1]]))
    rb = K.lib().kq_row_bytes(qtype, Kd)
    wr = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    check_ulp(y[rows], port.gemv_i8(qtype, wr, x, rows.size, Kd), f"i8 config {qtype} {N}x{Kd}")
    assert same_values(gpu_gemv(qtype | INT8_ACT, w, x, N, Kd), y)
    kq_env(KQ_GRID=37, KQ_WG_THREADS=256)
    assert same_values(gpu_gemv(qtype | INT8_ACT, w, x, N, Kd), y)


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_gemv_add(port, qtype):
    N, Kd = 200, 2048
    w = synth.tensor(qtype, N, Kd, 8500)
    x = synth.gaussian(synth.rng(8501), Kd)
    add = synth.gaussian(synth.rng(8502), N)
    got = gpu_gemv(qtype | INT8_ACT, w, x, N, Kd, add=add)
    check_ulp(got, port.gemv_i8(qtype, w, x, N, Kd, add=add), f"i8 add {qtype}")
    assert same_values(got, add + gpu_gemv(qtype | INT8_ACT, w, x, N, Kd))


def test_segments_share_x_with_exact_path(port):
    """One x feeding int8 and exact segments of both types in one list: each
    output equals its own single launch (the staged x is re-staged when the
    layout changes)."""
    H = 1024
    x = synth.gaussian(synth.rng(8600), H)
    specs = [(TYPE_Q4_K | INT8_ACT, 256), (TYPE_Q4_K, 128), (TYPE_Q6_K | INT8_ACT, 96),
             (TYPE_Q4_K | INT8_ACT, 64), (TYPE_Q6_K, 80), (TYPE_Q6_K | INT8_ACT, 32)]
    dx = dev(x)
    ws, dws, dys, segs = [], [], [], []
    for i, (t, N) in enumerate(specs):
        ws.append(synth.tensor(t & 0xff, N, H, 8610 + i))
        dws.append(dev(ws[-1]))
        dys.append(torch.full((N,), float("nan"), dtype=torch.float32, device="cuda"))
        segs.append(K.segment(t, H, N, [dws[-1].data_ptr()], dx.data_ptr(), dys[-1].data_ptr()))
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i, (t, N) in enumerate(specs):
        got = dys[i].cpu().numpy()
        assert same_values(got, gpu_gemv(t, ws[i], x, N, H)), (i, t)
        if t & INT8_ACT:
            check_ulp(got, port.gemv_i8(t & 0xff, ws[i], x, N, H), f"seg {i}")


@pytest.mark.parametrize("order", [(12, 12, 14), (14, 12, 14, 14, 12)])
def test_segments_mixed_int8_q4k_q6k_one_launch(port, order):
    """Q4_K and Q6_K in the int8 mode in one segment list (a Q, K, V group
    with a Q6_K V): one launch of the mixed int8 kernel, as
    st_mixed_fused_sdot dispatches the group once (stratum_linear.h:
    1043-1085); each output equals its own single int8 launch."""
    H = 2048
    x = synth.gaussian(synth.rng(8650), H)
    rows = [512, 128, 160, 96, 64]
    dx = dev(x)
    ws, dws, dys, segs = [], [], [], []
    for i, t in enumerate(order):
        N = rows[i]
        ws.append(synth.tensor(t, N, H, 8660 + i))
        dws.append(dev(ws[-1]))
        dys.append(torch.full((N,), float("nan"), dtype=torch.float32, device="cuda"))
        segs.append(K.segment(t | INT8_ACT, H, N, [dws[-1].data_ptr()], dx.data_ptr(),
                              dys[-1].data_ptr()))
    K.gemv_segments_dev(segs, stream=stream())
    torch.cuda.synchronize()
    for i, t in enumerate(order):
        got = dys[i].cpu().numpy()
        assert same_values(got, gpu_gemv(t | INT8_ACT, ws[i], x, rows[i], H)), (i, t)
        check_ulp(got, port.gemv_i8(t, ws[i], x, rows[i], H), f"seg {i}")


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_segments_groups_strided_x(port, qtype):
    """A segment of several groups, each with its own x (x_stride), as the
    MoE-style multi-x form of the batch kernel."""
    H, N, G = 768, 48, 4
    xs = np.stack([synth.gaussian(synth.rng(8700 + g), H) for g in range(G)])
    ws = [synth.tensor(qtype, N, H, 8710 + g) for g in range(G)]
    dx = dev(xs.reshape(-1))
    dws = [dev(w) for w in ws]
    dy = torch.full((G * N,), float("nan"), dtype=torch.float32, device="cuda")
    seg = K.segment(qtype | INT8_ACT, H, N, [d.data_ptr() for d in dws], dx.data_ptr(),
                    dy.data_ptr(), x_stride=H)
    K.gemv_segments_dev([seg], stream=stream())
    torch.cuda.synchronize()
    y = dy.cpu().numpy().reshape(G, N)
    for g in range(G):
        assert same_values(y[g], gpu_gemv(qtype | INT8_ACT, ws[g], xs[g], N, H)), g


@pytest.mark.parametrize("qtype", [TYPE_Q5_K, TYPE_Q3_K, TYPE_Q8_0])
@pytest.mark.parametrize("B,N,Kd", [(5, 100, 1024), (2, 300, 768), (16, 64, 2048), (19, 40, 3072),
                                    (40, 96, 1024), (70, 33, 512), (8, 200, 17408)])
def test_multix_equals_single_stream(qtype, B, N, Kd):
    """The int8 types whose reference batches are per stream (Q5_K, Q3_K,
    Q8_0: st_linear_multix calls the single-stream form per stream): one
    weight pass of the multi-x kernel for all streams, each stream
    bit-identical to its single-stream result; ragged rows, member chunks
    past 16 and 64 streams, and rows of 272 chunks."""
    w = synth.tensor(qtype, N, Kd, 8800 + B)
    xs = np.stack([synth.gaussian(synth.rng(8801 + s), Kd) for s in range(B)])
    print(f"int8 multix type={qtype} B={B} N={N} K={Kd}", flush=True)
    dw, dx = dev(w), dev(xs.reshape(-1))
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype | INT8_ACT, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd,
                      stream=stream())
    torch.cuda.synchronize()
    ys = dy.cpu().numpy().reshape(B, N)
    for s in range(B):
        assert same_values(ys[s], gpu_gemv(qtype | INT8_ACT, w, xs[s], N, Kd)), s


@pytest.mark.parametrize("qtype", [TYPE_Q5_K, TYPE_Q3_K, TYPE_Q8_0])
def test_multix_edge_streams(qtype):
    """The int8 multi-x path of the per-stream types on edge inputs: rows
    of one super-block (K = 256) and a single row, a stream of zeros (scale
    0: every quantized value 0), a stream with 1e30 and subnormal values,
    and 65 streams (two launches): each stream bit-identical to its
    single-stream result."""
    for N, Kd, B in ((1, 256, 3), (37, 256, 65), (130, 512, 4)):
        w = synth.tensor(qtype, N, Kd, 8900 + N)
        xs = np.stack([synth.gaussian(synth.rng(8901 + s), Kd) for s in range(B)])
        xs[1] = 0.0
        xs[B - 1, ::7] = 1e30
        xs[B - 1, 3::11] = 1e-40
        print(f"int8 multix edges type={qtype} N={N} K={Kd} B={B}", flush=True)
        dw, dx = dev(w), dev(xs.reshape(-1))
        dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
        K.gemv_multix_dev(qtype | INT8_ACT, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd,
                          stream=stream())
        torch.cuda.synchronize()
        ys = dy.cpu().numpy().reshape(B, N)
        for s in range(B):
            assert same_values(ys[s], gpu_gemv(qtype | INT8_ACT, w, xs[s], N, Kd)), (N, Kd, s)


def test_host_abi_sdot_switch(port):
    """kq_linear_set_sdot routes the host-pointer entry points through the
    int8 mode for Q4_K, Q6_K, Q5_K, Q3_K and Q8_0 (as g_st.use_sdot does,
    stratum_linear.h:376-489) and leaves other types (Q2_K) alone;
    switching it off restores the exact path."""
    Kd = 1024
    specs = [(TYPE_Q4_K, 300), (TYPE_Q6_K, 200), (10, 64), (TYPE_Q5_K, 96), (TYPE_Q3_K, 80),
             (TYPE_Q8_0, 72)]
    parts, tensors, off = [], [], 0
    for i, (t, N) in enumerate(specs):
        wb = synth.tensor(t, N, Kd, 8900 + i)
        tensors.append((K.make_tensor(t, N, Kd, off, name=f"s{i}".encode()), wb, t, N))
        parts.append(wb)
        off += wb.size
    blob = np.concatenate(parts)
    K.WeightRegion(blob)
    x = synth.gaussian(synth.rng(8950), Kd)
    exact = [K.linear_dispatch(d, x, N, Kd) for d, _, _, N in tensors]
    prev = K.set_sdot(True)
    try:
        for (d, wb, t, N), ye in zip(tensors, exact):
            y = K.linear_dispatch(d, x, N, Kd)
            if t == 10:
                assert same_values(y, ye)
                continue
            assert same_values(y, gpu_gemv(t | INT8_ACT, wb, x, N, Kd)), t
            add = synth.gaussian(synth.rng(8960), N)
            assert same_values(K.linear_dispatch_add(d, x, add, N, Kd), add + y), t
            xs = [synth.gaussian(synth.rng(8970 + s), Kd) for s in range(3)]
            ys = K.linear_multix(d, xs, N, Kd)
            if t in (TYPE_Q4_K, TYPE_Q6_K):      # st_linear_multix's int8 arithmetic
                want = port.gemv_i8_multix(t, wb, np.stack(xs), N, Kd)
                for s in range(3):
                    assert same_values(ys[s], want[s]), (t, s)
                continue
            for s in range(3):
                assert same_values(ys[s], K.linear_dispatch(d, xs[s], N, Kd)), (t, s)
        (d0, _, _, n0), (d1, _, _, n1) = tensors[:2]
        g = K.q4k_group(x, Kd, (d0, n0), (d1, n1))
        assert same_values(g[0], K.linear_dispatch(d0, x, n0, Kd))
        assert same_values(g[1], K.linear_dispatch(d1, x, n1, Kd))
    finally:
        K.set_sdot(prev)
    for (d, _, _, N), ye in zip(tensors, exact):
        assert same_values(K.linear_dispatch(d, x, N, Kd), ye)


def test_refused_forms():
    """No matrix-core int8 form, and no int8 form of Q2_K, type 42, F16 or
    F32: refused with -1."""
    N, Kd = 64, 512
    w = dev(synth.tensor(TYPE_Q4_K, N, Kd, 9000))
    x = dev(synth.gaussian(synth.rng(9001), 2 * Kd))
    y = torch.empty(2 * N, dtype=torch.float32, device="cuda")
    L = K.lib()
    assert L.kq_gemv_multix_mfma_dev(TYPE_Q4_K | INT8_ACT, w.data_ptr(), x.data_ptr(),
                                     y.data_ptr(), 2, N, Kd, None) == -1
    assert L.kq_gemv_dev(10 | INT8_ACT, w.data_ptr(), x.data_ptr(), None, y.data_ptr(), N, Kd,
                         None) == -1
    for t in (10, 42, 0, 1):
        assert L.kq_row_bytes(t | INT8_ACT, Kd) == -1, t
    for t in (TYPE_Q5_K, TYPE_Q3_K, TYPE_Q8_0):
        assert L.kq_row_bytes(t | INT8_ACT, Kd) == L.kq_row_bytes(t, Kd)


# ------------------------------------ int8 MULTISEQ on the matrix cores
MX_TYPES = [TYPE_Q4_K, TYPE_Q6_K]


def gpu_multix_i8(qtype, dw, dx, B, N, Kd):
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype | INT8_ACT, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd,
                      stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy().reshape(B, N)


@pytest.mark.parametrize("qtype", MX_TYPES)
@pytest.mark.parametrize("B,N,Kd", [(2, 100, 1024), (5, 33, 512), (8, 130, 2048), (16, 64, 4096),
                                    (17, 70, 768), (33, 96, 1280), (64, 200, 2048)])
def test_multix_i8_matches_reference_pack(port, qtype, B, N, Kd):
    """Q4_K / Q6_K int8 MULTISEQ (B >= 2) on the matrix cores: every stream
    bit-identical to the oracle's restatement of the reference's
    q*_dot_rows2_sdot_multix_pack arithmetic (streams not a multiple of the
    wave's 8/16/32, rows not a multiple of 16 or 64)"""
    w = synth.tensor(qtype, N, Kd, 9100 + B)
    xs = np.stack([synth.gaussian(synth.rng(9110 + s), Kd) for s in range(B)])
    print(f"int8 mfma multix type={qtype} B={B} N={N} K={Kd}", flush=True)
    got = gpu_multix_i8(qtype, dev(w), dev(xs.reshape(-1)), B, N, Kd)
    want = port.gemv_i8_multix(qtype, w, xs, N, Kd)
    exact = int(np.sum(got.view(np.uint32) == want.view(np.uint32)))
    print(f"  bit-identical {exact}/{want.size}", flush=True)
    assert same_values(got, want)


@pytest.mark.parametrize("qtype,N,Kd,B", [(TYPE_Q4_K, 17408, 5120, 8), (TYPE_Q4_K, 17408, 5120, 16),
                                          (TYPE_Q4_K, 17408, 5120, 64), (TYPE_Q6_K, 5120, 17408, 16),
                                          (TYPE_Q6_K, 5120, 17408, 64)])
def test_multix_i8_27b_sampled(port, qtype, N, Kd, B):
    """configs[3] shapes (27B gate / down) at B = 8, 16, 64: 256 sampled rows
    of every stream bit-identical to the oracle's pack arithmetic, and two
    streams within the terms' rounding bound of the single-stream int8 form"""
    w = synth.tensor(qtype, N, Kd, 9200 + qtype)
    xs = np.stack([synth.gaussian(synth.rng(9210 + s), Kd) for s in range(B)])
    print(f"int8 mfma multix 27B type={qtype} B={B}", flush=True)
    dw, dx = dev(w), dev(xs.reshape(-1))
    got = gpu_multix_i8(qtype, dw, dx, B, N, Kd)
    rows = np.random.default_rng(5 + B).choice(N, 256, replace=False)
    rb = K.lib().kq_row_bytes(qtype, Kd)
    sub = np.concatenate([w[r * rb:(r + 1) * rb] for r in rows])
    want = port.gemv_i8_multix(qtype, sub, xs, rows.size, Kd)
    assert same_values(got[:, rows], want)
    for s in (0, B - 1):
        y1 = gpu_gemv(qtype | INT8_ACT, w, xs[s], N, Kd)
        _, mag = port.gemv_i8(qtype, sub, xs[s], rows.size, Kd, sdot_f=True, with_mag=True)
        d = np.abs(got[s, rows].astype(np.float64) - y1[rows].astype(np.float64))
        assert np.all(d <= 5 * 2.0 ** -24 * mag + np.spacing(np.abs(y1[rows]))), s


def test_multix_i8_repeatable_and_strided_launch_shapes(port):
    """two launches give the same bits; B = 1 stays the single-stream form"""
    qtype, N, Kd, B = TYPE_Q4_K, 300, 3072, 24
    w = synth.tensor(qtype, N, Kd, 9300)
    xs = np.stack([synth.gaussian(synth.rng(9310 + s), Kd) for s in range(B)])
    dw, dx = dev(w), dev(xs.reshape(-1))
    a = gpu_multix_i8(qtype, dw, dx, B, N, Kd)
    b = gpu_multix_i8(qtype, dw, dx, B, N, Kd)
    assert same_values(a, b)
    one = gpu_multix_i8(qtype, dw, dx, 1, N, Kd)
    assert same_values(one[0], gpu_gemv(qtype | INT8_ACT, w, xs[0], N, Kd))
