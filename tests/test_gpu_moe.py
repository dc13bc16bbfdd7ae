"""GPU parity of the MoE gather (through the C ABI): device top-k against
the oracle's moe_topk, and the routed expert GEMVs against the
single-stream GEMV of each selected slice (bit for bit) and the oracle
(within the GEMV bound), for one token and for batches whose tokens share
experts (stratum_arch_moe.inc.c:605-755, 817-1267)."""
import numpy as np
import pytest

import stratum_amd as K
from conftest import same_values
from oracle import oracle as O
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


def stream():
    return torch.cuda.current_stream().cuda_stream


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def softmax_rows(logits):
    z = logits - logits.max(axis=1, keepdims=True)
    p = np.exp(z.astype(np.float64))
    return (p / p.sum(axis=1, keepdims=True)).astype(np.float32)


def gpu_topk(probs, k):
    B, E = probs.shape
    dp = dev(probs)
    sel = torch.empty(B * k, dtype=torch.int32, device="cuda")
    selw = torch.empty(B * k, dtype=torch.float32, device="cuda")
    K.moe_topk_dev(dp.data_ptr(), B, E, k, sel.data_ptr(), selw.data_ptr(), stream())
    torch.cuda.synchronize()
    return sel.cpu().numpy().reshape(B, k), selw.cpu().numpy().reshape(B, k)


@pytest.mark.parametrize("B,E,k", [(16, 128, 8), (1, 128, 8), (5, 100, 6), (3, 4096, 8),
                                   (2, 5, 5), (4, 64, 1), (2, 1000, 8), (1, 1024, 16),
                                   (3, 1025, 4), (2, 192, 7)])
def test_topk_dev_matches_oracle(port, B, E, k):
    r = np.random.default_rng(B * 1000 + E + k)
    probs = softmax_rows(r.standard_normal((B, E)).astype(np.float32))
    sel, selw = gpu_topk(probs, k)
    for s in range(B):
        ws, ww = port.topk(probs[s], k)
        assert list(sel[s]) == ws, s
        assert same_values(selw[s], ww), s


@pytest.mark.parametrize("E", [200, 1000])
def test_topk_dev_ties_across_parts(port, E):
    """Wide router rows, where several lanes share one expert's comparisons:
    all-equal weights (the lowest ids win), repeated values spread over the
    whole row, and ineligible weights in between."""
    r = np.random.default_rng(E)
    rows = [np.full(E, 0.5 / E, np.float32),
            r.integers(0, 4, E).astype(np.float32) * 0.25,
            np.where(r.random(E) < 0.5, -1.5, r.integers(0, 3, E) * 0.5).astype(np.float32)]
    probs = np.stack(rows)
    for k in (1, 8, 16):
        sel, selw = gpu_topk(probs, k)
        for s in range(len(rows)):
            ws, ww = port.topk(probs[s], k)
            assert list(sel[s]) == ws, (E, s, k)
            assert same_values(selw[s], ww), (E, s, k)


def test_topk_dev_ties_and_ineligible(port):
    """Equal weights keep the lower expert first; weights <= -1 and NaN are
    never chosen; missing slots are (-1, -1.0f)."""
    rows = [
        np.array([0.1, 0.3, 0.3, 0.2, 0.3, 0.05] + [0.0] * 94, np.float32),
        np.full(100, 0.125, np.float32),
        np.array([-2.0, -1.0, -0.5, np.nan, 0.0, -0.0] + [-1.0] * 94, np.float32),
        np.array([-3.0] * 99 + [-1.0], np.float32),
    ]
    probs = np.stack(rows)
    for k in (1, 3, 8):
        sel, selw = gpu_topk(probs, k)
        for s in range(len(rows)):
            ws, ww = port.topk(probs[s], k)
            assert list(sel[s]) == ws, (s, k)
            assert same_values(selw[s], ww), (s, k)


def experts(qtype, n_exp, N_out, K_in, seed):
    """Stacked expert tensor: expert e's slice is rows [e*N_out, (e+1)*N_out)."""
    return synth.tensor(qtype, n_exp * N_out, K_in, seed)


def single(qtype, w_slice, x, N, K_in):
    dw, dx = dev(w_slice), dev(x)
    dy = torch.empty(N, dtype=torch.float32, device="cuda")
    K.gemv_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), N, K_in, stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy()


def run_moe(qtype, wts, sel, x, x_div, B, k, n_exp, N_out, K_in, stride=None, w_off=None):
    """kq_moe_gemv_dev over the stacked tensors wts (or one buffer with
    per-tensor offsets w_off and expert stride `stride`)."""
    nt = len(wts) if w_off is None else len(w_off)
    if w_off is None:
        dws = [dev(w) for w in wts]
        ptrs = [d.data_ptr() for d in dws]
        stride = N_out * K.lib().kq_row_bytes(qtype, K_in)
    else:
        dws = [dev(wts[0])]
        ptrs = [dws[0].data_ptr() + o for o in w_off]
    dx = dev(x)
    ys = [torch.full((B * k * N_out,), float("nan"), dtype=torch.float32, device="cuda")
          for _ in range(nt)]
    dsel = dev(np.asarray(sel, np.int32).reshape(-1))
    op = K.moe_op(qtype, N_out, K_in, ptrs, stride, dx.data_ptr(), x_div,
                  [y.data_ptr() for y in ys])
    K.moe_gemv_dev(op, dsel.data_ptr(), B, k, n_exp, stream())
    torch.cuda.synchronize()
    return [y.cpu().numpy().reshape(B * k, N_out) for y in ys]


def check_members(port, qtype, wts, sel, x, x_div, got, N_out, K_in, n_oracle=3):
    rb = K.lib().kq_row_bytes(qtype, K_in)
    sl = N_out * rb
    sel = np.asarray(sel).reshape(-1)
    checked = 0
    for t, w in enumerate(wts):
        for m, e in enumerate(sel):
            if e < 0:
                continue
            xm = x[(m // x_div) * K_in:(m // x_div + 1) * K_in]
            ws = w[e * sl:(e + 1) * sl]
            assert same_values(got[t][m], single(qtype, ws, xm, N_out, K_in)), (t, m, e)
            if checked < n_oracle:
                want = port.gemv(qtype, ws, xm, N_out, K_in)
                err = O.rel_err(got[t][m], want).max()
                assert err <= 1e-5, (t, m, e, err)
                checked += 1


@pytest.mark.parametrize("qtype", [12, 14])
def test_moe_one_token_gate_up_and_down(port, qtype):
    """Batch 1: gate and up (one x) in one launch, down (one activation per
    rank) in another; each rank's output equals its slice's single GEMV."""
    n_exp, H, F, k = 32, 512, 256, 8
    gate, up = experts(qtype, n_exp, F, H, 1), experts(qtype, n_exp, F, H, 2)
    down = experts(qtype, n_exp, H, F, 3)
    r = np.random.default_rng(4)
    sel = r.choice(n_exp, k, replace=False).astype(np.int32)
    x = synth.gaussian(r, H)
    got = run_moe(qtype, [gate, up], sel, x, k, 1, k, n_exp, F, H)
    check_members(port, qtype, [gate, up], sel, x, k, got, F, H)
    act = np.stack([synth.gaussian(r, F) for _ in range(k)]).reshape(-1)
    got = run_moe(qtype, [down], sel, act, 1, 1, k, n_exp, H, F)
    check_members(port, qtype, [down], sel, act, 1, got, H, F)


def run_routed(qtype, wts, probs, x, x_div, k, N_out, K_in):
    """kq_moe_gemv_routed_dev: top-k of probs ([E] or [B, E]) inside the
    launch; returns the outputs and the sel / selw it wrote."""
    probs2 = probs.reshape(-1, probs.shape[-1])
    B, E = probs2.shape
    dws = [dev(w) for w in wts]
    stride = N_out * K.lib().kq_row_bytes(qtype, K_in)
    dx, dp = dev(x), dev(np.ascontiguousarray(probs2).reshape(-1))
    ys = [torch.full((B * k * N_out,), float("nan"), dtype=torch.float32, device="cuda")
          for _ in wts]
    sel = torch.full((B * k,), -7, dtype=torch.int32, device="cuda")
    selw = torch.full((B * k,), 7.0, dtype=torch.float32, device="cuda")
    op = K.moe_op(qtype, N_out, K_in, [d.data_ptr() for d in dws], stride, dx.data_ptr(), x_div,
                  [y.data_ptr() for y in ys])
    K.moe_gemv_routed_dev(op, dp.data_ptr(), B, k, E, sel.data_ptr(), selw.data_ptr(), stream())
    torch.cuda.synchronize()
    return ([y.cpu().numpy().reshape(B * k, N_out) for y in ys], sel.cpu().numpy(),
            selw.cpu().numpy())


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("E,k,case", [(32, 8, "random"), (128, 8, "random"), (1000, 4, "random"),
                                      (64, 8, "ties"), (40, 16, "few-eligible")])
def test_moe_routed_one_token(port, qtype, E, k, case):
    """Routing inside the gate+up launch: sel / selw equal the device top-k
    (and the oracle's moe_topk), and every output equals the unrouted
    call's bit for bit; the down call then runs on the written sel."""
    H, F = 512, 256
    gate, up = experts(qtype, E, F, H, 11), experts(qtype, E, F, H, 12)
    r = np.random.default_rng(E + k)
    if case == "random":
        probs = softmax_rows(r.standard_normal((1, E)).astype(np.float32))[0]
    elif case == "ties":
        probs = (r.integers(0, 3, E) * 0.25).astype(np.float32)
    else:                                   # fewer eligible experts than k
        probs = np.full(E, -2.0, np.float32)
        probs[[3, 17, 30]] = [0.5, 0.25, 0.5]
    x = synth.gaussian(r, H)
    got, sel, selw = run_routed(qtype, [gate, up], probs, x, k, k, F, H)
    ws, ww = port.topk(probs, k)
    assert list(sel) == ws
    assert same_values(selw, ww)
    dsel, dselw = gpu_topk(probs[None, :], k)
    assert list(dsel[0]) == list(sel) and same_values(dselw[0], selw)
    want = run_moe(qtype, [gate, up], sel, x, k, 1, k, E, F, H)
    for t in range(2):
        for m in range(k):
            if sel[m] >= 0:
                assert same_values(got[t][m], want[t][m]), (t, m)
    check_members(port, qtype, [gate, up], sel, x, k, got, F, H)


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("B,E,k,case", [(16, 128, 8, "random"), (3, 32, 4, "ties"),
                                        (8, 40, 16, "few-eligible"), (64, 16, 2, "random")])
def test_moe_routed_batch(port, qtype, B, E, k, case):
    """Batches routed inside the gate+up launch: sel / selw equal the device
    top-k of every token, and every output equals the unrouted batch call's
    bit for bit; the down call then runs on the written sel."""
    H, F = 512, 256
    gate, up = experts(qtype, E, F, H, 31), experts(qtype, E, F, H, 32)
    r = np.random.default_rng(B * E + k)
    if case == "random":
        probs = softmax_rows(r.standard_normal((B, E)).astype(np.float32))
    elif case == "ties":
        probs = (r.integers(0, 3, (B, E)) * 0.25).astype(np.float32)
    else:                                   # fewer eligible experts than k in some tokens
        probs = softmax_rows(r.standard_normal((B, E)).astype(np.float32))
        probs[1] = -2.0
        probs[1, [3, 17, 30]] = [0.5, 0.25, 0.5]
        probs[5, :] = np.nan
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    got, sel, selw = run_routed(qtype, [gate, up], probs, x, k, k, F, H)
    dsel, dselw = gpu_topk(probs, k)
    assert np.array_equal(dsel.reshape(-1), sel) and same_values(dselw.reshape(-1), selw)
    for s_ in range(min(B, 4)):
        ws, ww = port.topk(probs[s_], k)
        assert list(sel[s_ * k:(s_ + 1) * k]) == ws
    want = run_moe(qtype, [gate, up], sel.reshape(B, k), x, k, B, k, E, F, H)
    for t in range(2):
        for m in range(B * k):
            if sel[m] >= 0:
                assert same_values(got[t][m], want[t][m]), (t, m)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    down = experts(qtype, E, H, F, 33)
    dn = run_moe(qtype, [down], sel.reshape(B, k), act, 1, B, k, E, H, F)
    check_members(port, qtype, [down], sel.reshape(B, k), act, 1, dn, H, F)


@pytest.mark.parametrize("grouping", ["in_launch", "group_launch"])
@pytest.mark.parametrize("qtype", [12, 14, 10, 13, 11, 8])
@pytest.mark.parametrize("B,n_exp", [(16, 32), (16, 128), (3, 8), (64, 16)])
def test_moe_batch_grouped(port, qtype, B, n_exp, grouping, kq_env):
    """Batches whose tokens share experts: each selected slice is streamed
    once for all its tokens; every member still equals its single GEMV.
    The expert runs are built inside the multi-x launch, or (forced) by the
    separate grouping launch."""
    if grouping == "group_launch":
        kq_env(KQ_MOE_GROUP_LAUNCH=1)
    H, F, k = 512, 256, min(8, n_exp)
    gate, up = experts(qtype, n_exp, F, H, 11), experts(qtype, n_exp, F, H, 12)
    down = experts(qtype, n_exp, H, F, 13)
    r = np.random.default_rng(B + n_exp)
    probs = softmax_rows(r.standard_normal((B, n_exp)).astype(np.float32))
    sel = np.stack([port.topk(probs[s], k)[0] for s in range(B)]).astype(np.int32)
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    got = run_moe(qtype, [gate, up], sel, x, k, B, k, n_exp, F, H)
    check_members(port, qtype, [gate, up], sel, x, k, got, F, H)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    got = run_moe(qtype, [down], sel, act, 1, B, k, n_exp, H, F)
    check_members(port, qtype, [down], sel, act, 1, got, H, F)


@pytest.mark.parametrize("grouping", ["in_launch", "group_launch"])
def test_moe_pack_layout_and_unselected_slots(port, grouping, kq_env):
    """Expert slices in a pack (gate|up|down per expert, stride = their sum),
    with some ranks unselected (sel -1): the selected ranks are exact."""
    if grouping == "group_launch":
        kq_env(KQ_MOE_GROUP_LAUNCH=1)
    qtype, n_exp, H, F, B, k = 12, 12, 512, 256, 6, 4
    rb_g = K.lib().kq_row_bytes(qtype, H)
    rb_d = K.lib().kq_row_bytes(qtype, F)
    gsl, dsl = F * rb_g, H * rb_d
    stride = 2 * gsl + dsl
    gate, up = experts(qtype, n_exp, F, H, 21), experts(qtype, n_exp, F, H, 22)
    down = experts(qtype, n_exp, H, F, 23)
    pack = np.concatenate([np.concatenate([gate[e * gsl:(e + 1) * gsl], up[e * gsl:(e + 1) * gsl],
                                           down[e * dsl:(e + 1) * dsl]]) for e in range(n_exp)])
    r = np.random.default_rng(24)
    sel = np.stack([r.choice(n_exp, k, replace=False) for _ in range(B)]).astype(np.int32)
    sel[1, 2:] = -1
    sel[4, 3] = -1
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    got = run_moe(qtype, [pack], sel, x, k, B, k, n_exp, F, H, stride=stride, w_off=[0, gsl])
    check_members(port, qtype, [gate, up], sel, x, k, got, F, H)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    got = run_moe(qtype, [pack], sel, act, 1, B, k, n_exp, H, F, stride=stride, w_off=[2 * gsl])
    check_members(port, qtype, [down], sel, act, 1, got, H, F)


@pytest.mark.parametrize("B", [1, 16])
def test_moe_config_routed_on_device(port, B):
    """The MoE configuration (128 experts, top-8, hidden 2048, expert ffn
    768, Q4_K): router probabilities -> device top-k -> gate/up gather, the
    selection feeding the GEMV without leaving the device; sampled members
    against the oracle and their single GEMVs."""
    qtype, n_exp, H, F, k = 12, 128, 2048, 768, 8
    gate, up = experts(qtype, n_exp, F, H, 31), experts(qtype, n_exp, F, H, 32)
    r = np.random.default_rng(33 + B)
    probs = softmax_rows(r.standard_normal((B, n_exp)).astype(np.float32))
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    dp = dev(probs)
    dsel = torch.empty(B * k, dtype=torch.int32, device="cuda")
    dselw = torch.empty(B * k, dtype=torch.float32, device="cuda")
    K.moe_topk_dev(dp.data_ptr(), B, n_exp, k, dsel.data_ptr(), dselw.data_ptr(), stream())
    dg, du, dx = dev(gate), dev(up), dev(x)
    ys = [torch.empty(B * k * F, dtype=torch.float32, device="cuda") for _ in range(2)]
    op = K.moe_op(qtype, F, H, [dg.data_ptr(), du.data_ptr()],
                  F * K.lib().kq_row_bytes(qtype, H), dx.data_ptr(), k, [y.data_ptr() for y in ys])
    K.moe_gemv_dev(op, dsel.data_ptr(), B, k, n_exp, stream())
    torch.cuda.synchronize()
    sel = dsel.cpu().numpy().reshape(B, k)
    for s in range(B):
        assert list(sel[s]) == port.topk(probs[s], k)[0]
    got = [y.cpu().numpy().reshape(B * k, F) for y in ys]
    members = [0, B * k - 1] if B > 1 else [0, 7]
    sl = F * K.lib().kq_row_bytes(qtype, H)
    for t, w in enumerate([gate, up]):
        for m in members:
            e = sel.reshape(-1)[m]
            xm = x[(m // k) * H:(m // k + 1) * H]
            ws = w[e * sl:(e + 1) * sl]
            assert same_values(got[t][m], single(qtype, ws, xm, F, H)), (t, m)
            assert O.rel_err(got[t][m], port.gemv(qtype, ws, xm, F, H)).max() <= 1e-5


@pytest.mark.parametrize("B", [1, 16])
def test_moe_config_full_layer_routed(port, B):
    """The MoE configuration as bench.py runs it: kq_moe_gemv_routed_dev for
    gate+up (top-k of the router weights inside the launch for B = 1, a
    top-k launch first for B = 16), then the down op (2048 x 768 per slice)
    through kq_moe_gemv_dev on the sel it wrote.  Every member of gate, up
    and down equals its own single-slice GEMV bit for bit; at least 4
    members per tensor are checked against the oracle; sel equals the
    oracle's moe_topk."""
    qtype, n_exp, H, F, k = 12, 128, 2048, 768, 8
    gate, up = experts(qtype, n_exp, F, H, 41), experts(qtype, n_exp, F, H, 42)
    down = experts(qtype, n_exp, H, F, 43)
    r = np.random.default_rng(44 + B)
    probs = softmax_rows(r.standard_normal((B, n_exp)).astype(np.float32))
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    got, sel, selw = run_routed(qtype, [gate, up], probs, x, k, k, F, H)
    for s_ in range(B):
        ws, ww = port.topk(probs[s_], k)
        assert list(sel[s_ * k:(s_ + 1) * k]) == ws, s_
        assert same_values(selw[s_ * k:(s_ + 1) * k], ww), s_
    check_members(port, qtype, [gate, up], sel, x, k, got, F, H, n_oracle=8)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    dn = run_moe(qtype, [down], sel.reshape(B, k), act, 1, B, k, n_exp, H, F)
    check_members(port, qtype, [down], sel, act, 1, dn, H, F, n_oracle=4)


# --------------------------------------------------- int8-activation mode
def check_ulp1(got, want, what):
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(d <= np.spacing(np.abs(want)).astype(np.float64)), what


def gpu_multix(qtype, w, xs, N, K_in):
    """kq_gemv_multix_dev over the rows of xs: [B, N]"""
    dw, dx = dev(w), dev(np.ascontiguousarray(xs, np.float32).reshape(-1))
    B = xs.shape[0]
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, K_in,
                      stream=stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy().reshape(B, N)


def check_i8_tickets(port, qtype, w, sel, x, x_div, got, N_out, K_in, n_exp, n_oracle=2):
    """Every member of an int8 batch (type | KQ_INT8_ACT) against the
    reference's tickets (moe_forward_b, stratum_arch_moe.inc.c:1136-1201,
    restated by oracle.moe_tickets): a ticket of two or more members of a
    Q4_K / Q6_K expert equals kq_gemv_multix_dev over the ticket's members
    (the multix pack arithmetic) bit for bit, and the oracle's restatement of
    that arithmetic on the first n_oracle such tickets; a ticket of one
    member, and every member of the other types, equals its slice's single
    int8 GEMV bit for bit.  Returns the ticket sizes seen."""
    qi = qtype | K.INT8_ACT
    rb = K.lib().kq_row_bytes(qtype, K_in)
    sl = N_out * rb
    xr = x.reshape(-1, K_in)
    sizes, packed = [], 0
    for e, mem in O.moe_tickets(np.asarray(sel).reshape(-1), n_exp):
        ws = w[e * sl:(e + 1) * sl]
        xs = np.stack([xr[m // x_div] for m in mem])
        sizes.append(len(mem))
        if len(mem) == 1 or qtype not in (12, 14):
            for i, m in enumerate(mem):
                assert same_values(got[m], single(qi, ws, xs[i], N_out, K_in)), (e, m)
            continue
        want = gpu_multix(qi, ws, xs, N_out, K_in)
        for i, m in enumerate(mem):
            assert same_values(got[m], want[i]), (e, m, len(mem))
        if packed < n_oracle:
            ref = port.gemv_i8_multix(qtype, ws, xs, N_out, K_in)
            assert same_values(want, ref), (e, len(mem))
            packed += 1
    return sizes


@pytest.mark.parametrize("qtype", [12, 14, 13, 11, 8])
@pytest.mark.parametrize("B", [1, 3])
def test_moe_int8_members(port, qtype, B):
    """The int8-activation mode (type | KQ_INT8_ACT).  Batch 1 is
    moe_forward_one_token's per-slice st_linear_dispatch under use_sdot
    (stratum_arch_moe.inc.c:596-603): every member bit-identical to its
    slice's single int8 GEMV and within one ulp of the oracle's int8 form.
    At B = 3, moe_forward_b's tickets (check_i8_tickets).  Gate and up
    routed in one launch, down on the written sel."""
    qi = qtype | K.INT8_ACT
    n_exp, H, F, k = 32, 512, 256, 8
    gate, up = experts(qtype, n_exp, F, H, 61), experts(qtype, n_exp, F, H, 62)
    down = experts(qtype, n_exp, H, F, 63)
    r = np.random.default_rng(64 + B + qtype)
    probs = softmax_rows(r.standard_normal((B, n_exp)).astype(np.float32))
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    print(f"moe int8 type={qtype} B={B}", flush=True)
    got, sel, selw = run_routed(qi, [gate, up], probs if B > 1 else probs[0], x, k, k, F, H)
    for s_ in range(B):
        ws, ww = port.topk(probs[s_], k)
        assert list(sel[s_ * k:(s_ + 1) * k]) == ws
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    dn = run_moe(qi, [down], sel.reshape(B, k), act, 1, B, k, n_exp, H, F)
    if B > 1:
        for t, w in enumerate((gate, up)):
            check_i8_tickets(port, qtype, w, sel, x, k, got[t], F, H, n_exp)
        check_i8_tickets(port, qtype, down, sel, act, 1, dn[0], H, F, n_exp)
        return
    rb = K.lib().kq_row_bytes(qtype, H)
    for t, w in enumerate((gate, up)):
        for m, e in enumerate(sel):
            xm = x[(m // k) * H:(m // k + 1) * H]
            ws_ = w[e * F * rb:(e + 1) * F * rb]
            assert same_values(got[t][m], single(qi, ws_, xm, F, H)), (t, m)
            if m < 3:
                check_ulp1(got[t][m], port.gemv_i8(qtype, ws_, xm, F, H), (t, m))
    rbd = K.lib().kq_row_bytes(qtype, F)
    for m, e in enumerate(sel):
        ws_ = down[e * H * rbd:(e + 1) * H * rbd]
        am = act[m * F:(m + 1) * F]
        assert same_values(dn[0][m], single(qi, ws_, am, H, F)), m
        if m < 3:
            check_ulp1(dn[0][m], port.gemv_i8(qtype, ws_, am, H, F), m)


def designed_sel(B, k, counts, n_exp, seed):
    """A selection [B, k] (distinct experts per token) in which expert e is
    chosen by counts[e] tokens; the other slots take experts past
    len(counts); ranks shuffled per token."""
    r = np.random.default_rng(seed)
    rows = [[] for _ in range(B)]
    for e, c in enumerate(counts):
        toks = sorted(range(B), key=lambda s: (len(rows[s]), r.random()))[:c]
        for s in toks:
            rows[s].append(e)
    rest = list(range(len(counts), n_exp))
    for s in range(B):
        extra = [int(e) for e in r.permutation(rest) if e not in rows[s]][:k - len(rows[s])]
        rows[s] += extra
        assert len(rows[s]) == k and len(set(rows[s])) == k
        r.shuffle(rows[s])
    return np.array(rows, np.int32)


@pytest.mark.parametrize("qtype", [12, 14])
def test_moe_int8_ticket_sizes(port, qtype):
    """Experts chosen by 1, 2, 7, 8, 9, 16 and 17 tokens (tickets 1, 2, 7,
    8, 8+1, 8+8, 8+8+1): a ticket of one member takes the single-stream int8
    form, a longer one the pack arithmetic over exactly its members; gate
    and up share x per token (x_div = k), down has one x per member; one
    slot left empty (sel -1) is not written."""
    n_exp, H, F, k, B = 48, 768, 512, 6, 20
    sel = designed_sel(B, k, [1, 2, 7, 8, 9, 16, 17], n_exp, 70 + qtype)
    hole = 3 * k + int(np.nonzero(sel[3] >= 7)[0][0])   # a slot of an unplanned expert
    sel.reshape(-1)[hole] = -1
    gate, up = experts(qtype, n_exp, F, H, 71), experts(qtype, n_exp, F, H, 72)
    down = experts(qtype, n_exp, H, F, 73)
    r = np.random.default_rng(74)
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    qi = qtype | K.INT8_ACT
    print(f"moe int8 tickets type={qtype}", flush=True)
    got = run_moe(qi, [gate, up], sel, x, k, B, k, n_exp, F, H)
    sizes = check_i8_tickets(port, qtype, gate, sel, x, k, got[0], F, H, n_exp, n_oracle=3)
    check_i8_tickets(port, qtype, up, sel, x, k, got[1], F, H, n_exp, n_oracle=1)
    assert {1, 2, 7, 8}.issubset(set(sizes)), sizes
    assert np.isnan(got[0][hole]).all()
    dn = run_moe(qi, [down], sel, act, 1, B, k, n_exp, H, F)
    check_i8_tickets(port, qtype, down, sel, act, 1, dn[0], H, F, n_exp, n_oracle=2)


def test_moe_int8_two_member_runs_wide_launch(port):
    """A Q4_K launch with two row blocks per workgroup (more runs' waves than
    the GPU holds at once), where runs of two members take the VALU form
    and runs of three or more the matrix-core form: experts chosen by 2, 2,
    1, 3, 4, 9 and 10 tokens (runs 8 + 1 and 8 + 2 among them); 1000 output rows (the last workgroup holds one row
    block, its last rows past N) of K = 768 (three super-blocks) and
    K = 2048 -- every member against its ticket."""
    n_exp, k, B = 48, 6, 20
    sel = designed_sel(B, k, [2, 2, 1, 3, 4, 9, 10], n_exp, 90)
    r = np.random.default_rng(91)
    for F, H in ((1000, 768), (1000, 2048)):
        gate = experts(12, n_exp, F, H, 92 + H)
        x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
        print(f"moe int8 two-member runs F={F} H={H}", flush=True)
        got = run_moe(12 | K.INT8_ACT, [gate, gate], sel, x, k, B, k, n_exp, F, H)
        sizes = check_i8_tickets(port, 12, gate, sel, x, k, got[0], F, H, n_exp, n_oracle=2)
        assert {1, 2, 3, 4, 8}.issubset(set(sizes)), sizes
        assert np.array_equal(got[0].view(np.uint32), got[1].view(np.uint32))


def test_moe_int8_config_b16(port):
    """configs[4] in the int8 mode at batch 16 (128 experts, top-8, hidden
    2048, expert ffn 768, Q4_K): routed gate+up, then down; every member
    against its ticket (check_i8_tickets)."""
    n_exp, H, F, k, B = 128, 2048, 768, 8, 16
    gate, up = experts(12, n_exp, F, H, 81), experts(12, n_exp, F, H, 82)
    down = experts(12, n_exp, H, F, 83)
    r = np.random.default_rng(84)
    probs = softmax_rows(r.standard_normal((B, n_exp)).astype(np.float32))
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    qi = 12 | K.INT8_ACT
    print("moe int8 configs[4] B=16", flush=True)
    got, sel, _ = run_routed(qi, [gate, up], probs, x, k, k, F, H)
    for s_ in range(B):
        assert list(sel[s_ * k:(s_ + 1) * k]) == port.topk(probs[s_], k)[0]
    sizes = check_i8_tickets(port, 12, gate, sel, x, k, got[0], F, H, n_exp)
    assert 1 in sizes and max(sizes) >= 2, sizes
    check_i8_tickets(port, 12, up, sel, x, k, got[1], F, H, n_exp, n_oracle=0)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    dn = run_moe(qi, [down], sel.reshape(B, k), act, 1, B, k, n_exp, H, F)
    check_i8_tickets(port, 12, down, sel, act, 1, dn[0], H, F, n_exp, n_oracle=1)


@pytest.mark.parametrize("qtype", [12, 14])
@pytest.mark.parametrize("H,F", [(4096, 256), (256, 12288)])
def test_moe_int8_tickets_long_rows(port, qtype, H, F):
    """Rows of 16 and 48 super-blocks (gate/up K = 4096, down K = 12288),
    where the ticket kernel splits each row over 2 and 4 waves (K-parts) and
    takes one row block per workgroup: every member against its ticket, with
    tickets of 1, 2, 7, 8 and 9 members."""
    n_exp, k, B = 16, 4, 12
    sel = designed_sel(B, k, [1, 2, 7, 9], n_exp, 90 + qtype)
    gate = experts(qtype, n_exp, F, H, 91)
    down = experts(qtype, n_exp, H, F, 93)
    r = np.random.default_rng(94)
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    qi = qtype | K.INT8_ACT
    print(f"moe int8 long rows type={qtype} H={H} F={F}", flush=True)
    got = run_moe(qi, [gate], sel, x, k, B, k, n_exp, F, H)
    sizes = check_i8_tickets(port, qtype, gate, sel, x, k, got[0], F, H, n_exp, n_oracle=2)
    assert {1, 2, 7, 8}.issubset(set(sizes)), sizes
    dn = run_moe(qi, [down], sel, act, 1, B, k, n_exp, H, F)
    check_i8_tickets(port, qtype, down, sel, act, 1, dn[0], H, F, n_exp, n_oracle=2)


@pytest.mark.parametrize("B,E,k", [(5, 1000, 1), (4, 4096, 8), (64, 32, 2)])
def test_moe_int8_tickets_shapes(port, B, E, k):
    """Int8 batches at the edges of the ticket cut: one rank per token
    (every member alone unless tokens share their expert), 4096 experts
    (the grouping's LDS tables at their largest), and 64 tokens over 32
    experts (tickets of eight and their remainders); Q4_K gate and up
    routed, then down on the written sel, against check_i8_tickets."""
    H, F = (256, 256) if E > 1024 else (512, 256)
    gate, up = experts(12, E, F, H, 101), experts(12, E, F, H, 102)
    down = experts(12, E, H, F, 103)
    r = np.random.default_rng(104 + B)
    probs = softmax_rows(r.standard_normal((B, E)).astype(np.float32))
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    qi = 12 | K.INT8_ACT
    print(f"moe int8 tickets B={B} E={E} k={k}", flush=True)
    if E <= 1024:
        got, sel, _ = run_routed(qi, [gate, up], probs, x, k, k, F, H)
    else:
        sel = np.stack([port.topk(probs[s], k)[0] for s in range(B)]).astype(np.int32).reshape(-1)
        got = run_moe(qi, [gate, up], sel.reshape(B, k), x, k, B, k, E, F, H)
    for s_ in range(B):
        assert list(sel[s_ * k:(s_ + 1) * k]) == port.topk(probs[s_], k)[0]
    for t, w in enumerate((gate, up)):
        check_i8_tickets(port, 12, w, sel, x, k, got[t], F, H, E, n_oracle=1)
    dn = run_moe(qi, [down], sel.reshape(B, k), act, 1, B, k, E, H, F)
    check_i8_tickets(port, 12, down, sel, act, 1, dn[0], H, F, E, n_oracle=1)


@pytest.mark.parametrize("qtype", [13, 11, 8])
@pytest.mark.parametrize("H,F,N_g", [(768, 512, 512), (256, 12288, 12288), (512, 256, 200)])
def test_moe_int8_per_stream_types(port, qtype, H, F, N_g):
    """Q5_K, Q3_K and Q8_0 batches in the int8 mode: st_linear_multix is per
    stream for them, so every member of every ticket equals its slice's
    single int8 GEMV bit for bit (each slice streamed once for its members).
    Experts chosen by 1, 2, 9 and 17 tokens with one slot left empty (sel
    -1, not written); rows of 4 to 192 chunks (down K = 12288), and a gate
    of 200 rows (a partial last row block, gate only)."""
    n_exp, k, B = 24, 4, 20
    sel = designed_sel(B, k, [1, 2, 9, 17], n_exp, 110 + qtype)
    hole = 5 * k + int(np.nonzero(sel[5] >= 4)[0][0])
    sel.reshape(-1)[hole] = -1
    gate = experts(qtype, n_exp, N_g, H, 111)
    r = np.random.default_rng(112 + qtype)
    x = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    qi = qtype | K.INT8_ACT
    print(f"moe int8 per-stream type={qtype} H={H} F={F} N={N_g}", flush=True)
    got = run_moe(qi, [gate], sel, x, k, B, k, n_exp, N_g, H)
    sizes = check_i8_tickets(port, qtype, gate, sel, x, k, got[0], N_g, H, n_exp)
    assert {1, 2, 8}.issubset(set(sizes)), sizes
    assert np.isnan(got[0][hole]).all()
    if N_g != F:
        return
    down = experts(qtype, n_exp, H, F, 113)
    act = np.stack([synth.gaussian(r, F) for _ in range(B * k)]).reshape(-1)
    dn = run_moe(qi, [down], sel, act, 1, B, k, n_exp, H, F)
    check_i8_tickets(port, qtype, down, sel, act, 1, dn[0], H, F, n_exp)
    assert np.isnan(dn[0][hole]).all()
