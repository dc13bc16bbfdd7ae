"""GPU parity of the MoE FFN step around the gather (kq_softmax_dev,
kq_swiglu_dev, kq_moe_combine_dev, the dense multi-stream router GEMV and
kq_moe_ffn_dev) against the CPU oracle (oracle/kq_oracle.c ko_softmax,
ko_swiglu, ko_moe_combine, ko_moe_ffn, pinned by
tests/test_oracle_moe_ffn.py).

Bars:
  * softmax and SwiGLU use the device expf (within one ulp of exp) where
    the reference calls libm's: every output within 4 binary32 ulps of the
    oracle's; exactly representable cases (equal logits, -inf, NaN, g = 0,
    large |g|) bit for bit;
  * combine: bit for bit (binary32 in rank order);
  * router GEMV (F32 / F16 rows): within one ulp of the oracle's binary64
    element-order sum; every stream of the multi-stream form bit-identical
    to its single-stream launch;
  * the whole step: each stage checked against the oracle applied to the
    device's own previous stage (GEMVs at their 1e-5 contract, bit-identical
    counts printed; combine bit for bit), sel identical to the oracle's
    top-k of the device's probabilities, and the final x within 1e-4 of
    the all-oracle chain relative to the largest FFN contribution.
"""
import numpy as np
import pytest

import stratum_amd as K
from conftest import same_values
from oracle import oracle as O
from stratum_amd import TYPE_F16, TYPE_F32, TYPE_Q4_K, synth

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


def ulps(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    sp = np.spacing(np.abs(b).astype(np.float32)).astype(np.float64)
    d = np.abs(a - b)
    d[np.isnan(a) & np.isnan(b)] = 0.0
    return d / sp


def gpu_softmax(x2d):
    d = dev(x2d.reshape(-1))
    K.softmax_dev(d.data_ptr(), x2d.shape[0], x2d.shape[1], stream())
    torch.cuda.synchronize()
    return d.cpu().numpy().reshape(x2d.shape)


def gpu_swiglu(g, u):
    dg, du = dev(g), dev(u)
    dy = torch.full(g.shape, float("nan"), dtype=torch.float32, device="cuda")
    K.swiglu_dev(dg.data_ptr(), du.data_ptr(), dy.data_ptr(), g.size, stream())
    torch.cuda.synchronize()
    return dy.cpu().numpy()


# ---------------------------------------------------------------- softmax
@pytest.mark.parametrize("B,E", [(1, 1), (1, 128), (16, 128), (4, 1000), (2, 4096)])
def test_softmax_within_ulps(port, B, E):
    r = synth.rng(9100 + E + B)
    x = (r.standard_normal((B, E)) * 4).astype(np.float32)
    print(f"softmax B={B} E={E}", flush=True)
    got, want = gpu_softmax(x), port.softmax(x)
    u = ulps(got, want)
    print(f"  max ulps {u.max():.1f}, bit-identical {int(np.sum(got == want))}/{got.size}",
          flush=True)
    assert u.max() <= 4.0


def test_softmax_exact_cases(port):
    ar = np.arange(128, dtype=np.float32)
    x = np.stack([np.full(128, 0.375, np.float32),
                  np.array([0.0, -np.inf] * 64, np.float32),
                  np.where(ar == 0, np.float32(np.nan), ar - 1),
                  np.where(ar == 127, np.float32(np.nan), ar)]).astype(np.float32)
    got = gpu_softmax(x)
    assert same_values(got, port.softmax(x))
    assert np.all(got[0] == np.float32(1 / 128))
    assert np.all(np.isnan(got[2])) and np.all(np.isnan(got[3]))


# ----------------------------------------------------------------- SwiGLU
@pytest.mark.parametrize("n", [1, 5, 768, 98304 + 3])
def test_swiglu_within_ulps(port, n):
    r = synth.rng(9200 + n)
    g = (r.standard_normal(n) * 4).astype(np.float32)
    u = r.standard_normal(n).astype(np.float32)
    got, want = gpu_swiglu(g, u), port.swiglu(g, u)
    uu = ulps(got, want)
    print(f"swiglu n={n}: max ulps {uu.max():.1f}, bit-identical "
          f"{int(np.sum(got == want))}/{n}", flush=True)
    assert uu.max() <= 4.0


def test_swiglu_exact_cases(port):
    g = np.array([0.0, 0.0, 100.0, 100.0, -100.0, 2.0, -0.0, 90.0], np.float32)
    u = np.array([5.0, -3.0, 0.25, -1.5, 3.0, 0.0, 1.0, 2.0], np.float32)
    assert same_values(gpu_swiglu(g, u), port.swiglu(g, u))


# ---------------------------------------------------------------- combine
@pytest.mark.parametrize("B,k,H", [(1, 8, 2048), (16, 8, 2048), (3, 2, 4)])
def test_combine_bit_exact(port, B, k, H):
    r = synth.rng(9300 + B)
    o = (r.standard_normal(B * k * H) * 3).astype(np.float32)
    sel = r.integers(0, 128, B * k).astype(np.int32)
    sel[::5] = -1
    selw = r.random(B * k).astype(np.float32)
    resid = r.standard_normal(B * H).astype(np.float32)
    do, ds, dw, dr = dev(o), dev(sel), dev(selw), dev(resid)
    dx = torch.full((B * H,), float("nan"), dtype=torch.float32, device="cuda")
    K.moe_combine_dev(do.data_ptr(), ds.data_ptr(), dw.data_ptr(), dr.data_ptr(), dx.data_ptr(),
                      B, k, H, stream())
    torch.cuda.synchronize()
    assert same_values(dx.cpu().numpy(), port.moe_combine(o, sel, selw, resid, B, k, H))
    # in place (x == resid)
    K.moe_combine_dev(do.data_ptr(), ds.data_ptr(), dw.data_ptr(), dr.data_ptr(), dr.data_ptr(),
                      B, k, H, stream())
    torch.cuda.synchronize()
    assert same_values(dr.cpu().numpy(), port.moe_combine(o, sel, selw, resid, B, k, H))


# ------------------------------------------------------------ dense router
@pytest.mark.parametrize("qtype", [TYPE_F32, TYPE_F16])
@pytest.mark.parametrize("B,N,Kd", [(16, 128, 2048), (9, 300, 1024), (3, 64, 5120)])
def test_dense_multix_equals_single(port, qtype, B, N, Kd):
    w = synth.tensor(qtype, N, Kd, 9400 + N)
    xs = np.stack([synth.gaussian(synth.rng(9401 + s), Kd) for s in range(B)])
    dw, dx = dev(w), dev(xs.reshape(-1))
    dy = torch.full((B * N,), float("nan"), dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(qtype, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), B, N, Kd, stream())
    torch.cuda.synchronize()
    ys = dy.cpu().numpy().reshape(B, N)
    for s in range(B):
        d1 = torch.full((N,), float("nan"), dtype=torch.float32, device="cuda")
        K.gemv_dev(qtype, dw.data_ptr(), dx.data_ptr() + 4 * s * Kd, d1.data_ptr(), N, Kd,
                   stream=stream())
        torch.cuda.synchronize()
        assert same_values(ys[s], d1.cpu().numpy()), s
    assert ulps(ys[0], port.gemv(qtype, w, xs[0], N, Kd)).max() <= 1.0


# --------------------------------------------------------- the whole step
def make_layer(H, F, E, k, seed, qtype=TYPE_Q4_K, router_type=TYPE_F32):
    rb_in = synth.row_bytes(qtype, H)
    rb_ff = synth.row_bytes(qtype, F)
    router = synth.tensor(router_type, E, H, seed)
    return {"n_embed": H, "n_ff": F, "n_experts": E, "k": k,
            "router_type": router_type, "router": router,
            "gate_type": qtype, "gate": synth.tensor(qtype, E * F, H, seed + 1),
            "up_type": qtype, "up": synth.tensor(qtype, E * F, H, seed + 2),
            "down_type": qtype, "down": synth.tensor(qtype, E * H, F, seed + 3),
            "gate_stride": F * rb_in, "up_stride": F * rb_in, "down_stride": H * rb_ff}


def run_step(d, xn, x0, B):
    H, F, E, k = d["n_embed"], d["n_ff"], d["n_experts"], d["k"]
    bufs = {n: dev(d[n]) for n in ("router", "gate", "up", "down")}
    f = K.KqMoeFfn()
    f.n_embed, f.n_ff, f.n_experts, f.k = H, F, E, k
    for n in ("router", "gate", "up", "down"):
        setattr(f, n, bufs[n].data_ptr())
        setattr(f, n + "_type", d[n + "_type"])
    f.gate_stride, f.up_stride, f.down_stride = d["gate_stride"], d["up_stride"], d["down_stride"]
    nbytes = K.moe_ffn_workspace_bytes(f, B)
    work = torch.full((nbytes // 4,), float("nan"), dtype=torch.float32, device="cuda")
    dxn, dx = dev(xn), dev(x0)
    sel = torch.full((B * k,), -7, dtype=torch.int32, device="cuda")
    selw = torch.full((B * k,), 7.0, dtype=torch.float32, device="cuda")
    K.moe_ffn_dev(f, dxn.data_ptr(), dx.data_ptr(), B, sel.data_ptr(), selw.data_ptr(),
                  work.data_ptr(), nbytes, stream())
    torch.cuda.synchronize()
    off = K.moe_ffn_workspace_offsets(f, B)
    wk = work.cpu().numpy()
    sizes = {"probs": B * E, "g": B * k * F, "u": B * k * F, "act": B * k * F, "ffo": B * k * H}
    out = {n: wk[off[n] // 4:off[n] // 4 + sizes[n]] for n in sizes}
    out.update(x=dx.cpu().numpy(), sel=sel.cpu().numpy(), selw=selw.cpu().numpy())
    # what the step ran, and the first word of the run-table region (the
    # run count when the gate+up launch stored its tables; the workspace was
    # filled with NaN bits before the call)
    out["path"] = K.moe_ffn_last_path()
    out["runs0"] = int(wk[off["runs"] // 4:off["runs"] // 4 + 1].view(np.int32)[0])
    return out


NAN_BITS = int(np.array([np.nan], np.float32).view(np.int32)[0])


@pytest.mark.parametrize("B", [1, 16])
def test_moe_ffn_step_config(port, B, kq_env):
    """128 experts, top-8, hidden 2048, expert ffn 768, Q4_K
    experts, F32 router.  Every stage's output is checked, so batch 1 runs
    the six-launch form (KQ_MOE_FFN_SPLIT), whose intermediates the
    three-launch form does not write; test_moe_ffn_fused_matches_split holds
    the two bit-identical."""
    H, F, E, k = 2048, 768, 128, 8
    d = make_layer(H, F, E, k, 9500)
    r = synth.rng(9501 + B)
    xn = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    x0 = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    print(f"moe ffn step B={B}", flush=True)
    kq_env(KQ_MOE_FFN_SPLIT=1)
    got = run_step(d, xn, x0, B)
    rb_in, rb_ff = synth.row_bytes(TYPE_Q4_K, H), synth.row_bytes(TYPE_Q4_K, F)
    # the router logits as the step computes them (the same dense kernel)
    dr, dxn = dev(d["router"]), dev(xn)
    dl = torch.empty(B * E, dtype=torch.float32, device="cuda")
    K.gemv_multix_dev(TYPE_F32, dr.data_ptr(), dxn.data_ptr(), dl.data_ptr(), B, E, H, stream())
    torch.cuda.synchronize()
    glog = dl.cpu().numpy()
    n_or = 0
    for s in range(B):
        xs = xn[s * H:(s + 1) * H]
        lg = glog[s * E:(s + 1) * E]
        assert ulps(lg, port.gemv(TYPE_F32, d["router"], xs, E, H)).max() <= 1.0, s
        p = got["probs"][s * E:(s + 1) * E]
        assert ulps(p, port.softmax(lg)).max() <= 4.0, s
        sel, selw = port.topk(p, k)
        assert list(got["sel"][s * k:(s + 1) * k]) == sel, s
        assert same_values(got["selw"][s * k:(s + 1) * k], selw), s
        for r_, e in enumerate(sel):
            m = s * k + r_
            g, u = got["g"][m * F:(m + 1) * F], got["u"][m * F:(m + 1) * F]
            a = got["act"][m * F:(m + 1) * F]
            assert ulps(a, port.swiglu(g, u)).max() <= 4.0, m
            if n_or < 6:      # the GEMV members against the oracle (1e-5 contract)
                gw = port.gemv(TYPE_Q4_K, d["gate"][e * F * rb_in:(e + 1) * F * rb_in], xs, F, H)
                uw = port.gemv(TYPE_Q4_K, d["up"][e * F * rb_in:(e + 1) * F * rb_in], xs, F, H)
                ow = port.gemv(TYPE_Q4_K, d["down"][e * H * rb_ff:(e + 1) * H * rb_ff], a, H, F)
                o = got["ffo"][m * H:(m + 1) * H]
                for name, gv, wv in (("gate", g, gw), ("up", u, uw), ("down", o, ow)):
                    rel = O.rel_err(gv, wv).max()
                    print(f"  member {m} {name}: max rel {rel:.2e}, bit-identical "
                          f"{int(np.sum(gv == wv))}/{wv.size}", flush=True)
                    assert rel <= 1e-5, (m, name)
                n_or += 1
    want_x = port.moe_combine(got["ffo"], got["sel"], got["selw"], x0, B, k, H)
    assert same_values(got["x"], want_x)
    full = port.moe_ffn(d, xn, x0, B)
    assert np.array_equal(full["sel"], got["sel"])
    contrib = np.abs(full["x"] - x0).max()
    err = np.abs(got["x"] - full["x"]).max()
    print(f"  end to end: max |x - x_oracle| {err:.3e} (largest FFN contribution {contrib:.3e})",
          flush=True)
    assert err <= 1e-4 * contrib


@pytest.mark.parametrize("case", ["config", "q6k_down", "parts16", "grid37", "e512", "wide_ff",
                                  "config_i8", "q6k_down_i8", "q5k", "q3k_i8", "q80_i8"])
def test_moe_ffn_fused_matches_split(port, case, kq_env):
    """Batch 1 in three launches (softmax and top-k inside the gate+up
    launch and SwiGLU in its epilogue; the rank-ordered combine plus residual
    in the down launch's epilogue) against the six-launch form: x, sel, selw
    and the activations bit-identical, and x against the oracle.  grid37 (37
    workgroups: the rows per part are not a multiple), e512 (512 experts:
    more than 256 logits) and wide_ff (n_ff 32x n_embed: a workgroup's gate
    and up outputs overflow the x region the fused epilogue keeps them in)
    take the six-launch form inside kq_moe_ffn_dev and must give the same
    bits too; kq_moe_ffn_last_path tells which form ran.  q5k takes Q5_K
    experts; the _i8 cases take the experts in the int8-activation mode
    (type | KQ_INT8_ACT), whose batch-1 step also runs in three launches;
    their values against the oracle's int8 forms are
    test_moe_ffn_step_int8's."""
    i8 = case.endswith("_i8")
    base = case[:-3] if i8 else case
    qtype = {"q5k": 13, "q3k": 11, "q80": 8}.get(base, TYPE_Q4_K)
    H, F, E, k = {"config": (2048, 768, 128, 8), "q6k_down": (1024, 512, 64, 4),
                  "parts16": (1024, 256, 32, 8), "grid37": (2048, 768, 128, 8),
                  "e512": (1024, 256, 512, 4), "wide_ff": (256, 8192, 16, 8),
                  "q5k": (1024, 512, 64, 4), "q3k": (1024, 512, 64, 4),
                  "q80": (1024, 512, 64, 4)}[base]
    d = make_layer(H, F, E, k, 9700, qtype=qtype)
    if base == "q6k_down":
        d["down_type"] = 14
        d["down"] = synth.tensor(14, E * H, F, 9704)
        d["down_stride"] = H * synth.row_bytes(14, F)
    if i8:
        for n in ("gate_type", "up_type", "down_type"):
            d[n] |= K.INT8_ACT
    r = synth.rng(9701)
    xn, x0 = synth.gaussian(r, H), synth.gaussian(r, H)
    if case == "grid37":
        kq_env(KQ_GRID=37)
    print(f"moe ffn fused vs split: {case}", flush=True)
    fused = run_step(d, xn, x0, 1)
    want_fused = base in ("config", "q6k_down", "parts16", "q5k", "q3k", "q80")
    assert bool(fused["path"] & K.FFN_FUSED_B1) == want_fused, fused["path"]
    kq_env(KQ_MOE_FFN_SPLIT=1)
    split = run_step(d, xn, x0, 1)
    assert not split["path"] & K.FFN_FUSED_B1
    for n in ("sel", "selw", "act", "x"):
        assert same_values(fused[n], split[n]), n
    if i8:
        return
    full = port.moe_ffn(d, xn, x0, 1)
    assert np.array_equal(full["sel"], fused["sel"])
    contrib = np.abs(full["x"] - x0).max()
    assert np.abs(fused["x"] - full["x"]).max() <= 1e-4 * contrib


@pytest.mark.parametrize("case", ["config_b16", "routed_b4", "q5k_b16", "q3k_routed_b4"])
def test_moe_ffn_batch_shared_runs_match_split(port, case, kq_env):
    """B > 1: the grouped gate+up launch stores its expert-run tables and
    the down launch loads them instead of grouping the selection again.
    config_b16 routes in a top-k launch first; routed_b4 (B E^2 <= 2^16)
    inside the gate+up launch; the q5k / q3k cases are the same with Q5_K
    and Q3_K experts.  Every output (gate, up, activations, down outputs,
    x, sel, selw) is bit-identical to the split form's (KQ_MOE_FFN_SPLIT,
    where each launch groups for itself), and x agrees with the oracle."""
    B, H, F, E, k, qt = {"config_b16": (16, 2048, 768, 128, 8, TYPE_Q4_K),
                         "routed_b4": (4, 1024, 512, 64, 4, TYPE_Q4_K),
                         "q5k_b16": (16, 2048, 768, 128, 8, 13),
                         "q3k_routed_b4": (4, 1024, 512, 64, 4, 11)}[case]
    d = make_layer(H, F, E, k, 9800, qtype=qt)
    r = synth.rng(9801)
    xn = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    x0 = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    print(f"moe ffn batch shared run tables vs split: {case}", flush=True)
    fused = run_step(d, xn, x0, B)
    # the tables were stored (run count written over the NaN fill) and the
    # down launch loaded them (Q4_K: its down plan cuts runs as gate+up's;
    # the q5k / q3k down plans may cut them otherwise and then regroup)
    assert fused["path"] & K.FFN_RUNS_STORED, fused["path"]
    if qt == TYPE_Q4_K:
        assert fused["path"] & K.FFN_RUNS_LOADED, fused["path"]
    assert fused["runs0"] != NAN_BITS and 0 < fused["runs0"] <= B * k, fused["runs0"]
    kq_env(KQ_MOE_FFN_SPLIT=1)
    split = run_step(d, xn, x0, B)
    assert not split["path"] & (K.FFN_RUNS_STORED | K.FFN_RUNS_LOADED)
    for n in ("sel", "selw", "g", "u", "act", "ffo", "x"):
        assert same_values(fused[n], split[n]), n
    full = port.moe_ffn(d, xn, x0, B)
    assert np.array_equal(full["sel"], fused["sel"])
    contrib = np.abs(full["x"] - x0).max()
    assert np.abs(fused["x"] - full["x"]).max() <= 1e-4 * contrib


@pytest.mark.parametrize("case", ["group_launch_b16", "e4096_b4", "e4096_b4_group_launch"])
def test_moe_ffn_never_grows_library_scratch(port, case, kq_env):
    """No allocation in the step, also where a launch groups the selection
    in a launch of its own: group_launch_b16 and e4096_b4_group_launch force
    that form (KQ_MOE_GROUP_LAUNCH); e4096_b4 is the largest expert count,
    routed by a separate top-k launch.  With the library's scratch emptied
    first (kq_linear_shutdown), kq_scratch_bytes() stays 0 across the step,
    the forced group records went to the workspace (KQ_FFN_GROUP_LAUNCH),
    and x agrees with the oracle (group_launch_b16: bit-identical to the
    step with the runs built in the launch)."""
    B, H, F, E, k = {"group_launch_b16": (16, 2048, 768, 128, 8),
                     "e4096_b4": (4, 256, 256, 4096, 8),
                     "e4096_b4_group_launch": (4, 256, 256, 4096, 8)}[case]
    forced = case != "e4096_b4"
    d = make_layer(H, F, E, k, 9900)
    r = synth.rng(9901)
    xn = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    x0 = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    print(f"moe ffn scratch: {case}", flush=True)
    if case == "group_launch_b16":
        base = run_step(d, xn, x0, B)
    if forced:
        kq_env(KQ_MOE_GROUP_LAUNCH=1)
    K.lib().kq_linear_shutdown()
    assert K.lib().kq_scratch_bytes() == 0
    got = run_step(d, xn, x0, B)
    assert K.lib().kq_scratch_bytes() == 0
    if forced:
        assert got["path"] & K.FFN_GROUP_LAUNCH, got["path"]
    if case == "group_launch_b16":
        for n in ("sel", "selw", "g", "u", "act", "ffo", "x"):
            assert same_values(got[n], base[n]), n
    full = port.moe_ffn(d, xn, x0, B)
    assert np.array_equal(full["sel"], got["sel"])
    contrib = np.abs(full["x"] - x0).max()
    assert np.abs(got["x"] - full["x"]).max() <= 1e-4 * contrib


@pytest.mark.parametrize("qtype,B", [(TYPE_Q4_K, 1), (TYPE_Q4_K, 3), (14, 3), (13, 3), (8, 3),
                                     (14, 1), (13, 1), (11, 1), (8, 1)])
def test_moe_ffn_step_int8(port, qtype, B):
    """The step with experts in the int8-activation mode (gate, up and down
    types | KQ_INT8_ACT; F32 router): sel is the oracle's top-k of the
    step's own probabilities; every gate, up and down member is
    bit-identical, on the step's own inputs, to its ticket's int8 call
    (moe_forward_b's tickets of at most 8 members, oracle.moe_tickets: for
    Q4_K / Q6_K a single int8 GEMV for a ticket of one, kq_gemv_multix_dev
    over the ticket otherwise; for Q5_K / Q8_0, whose multix is per stream,
    every member's single int8 GEMV; at B = 1 every ticket has one member);
    SwiGLU within 4 ulps and the combine bit for bit; the library's scratch
    stays empty across the step (the ticket batch's workspace is the
    step's)."""
    H, F, E, k = 1024, 512, 32, 4
    d = make_layer(H, F, E, k, 9950, qtype=qtype)
    qi = qtype | K.INT8_ACT
    d["gate_type"] = d["up_type"] = d["down_type"] = qi
    r = synth.rng(9951 + B)
    xn = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    x0 = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    print(f"moe ffn int8 type={qtype} B={B}", flush=True)
    K.lib().kq_linear_shutdown()                  # the step allocates nothing
    assert K.lib().kq_scratch_bytes() == 0
    got = run_step(d, xn, x0, B)
    assert K.lib().kq_scratch_bytes() == 0
    rb_in, rb_ff = synth.row_bytes(qtype, H), synth.row_bytes(qtype, F)

    def single(w, xv, N, Kd):
        dw, dx = dev(w), dev(xv)
        dy = torch.empty(N, dtype=torch.float32, device="cuda")
        K.gemv_dev(qi, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), N, Kd, stream=stream())
        torch.cuda.synchronize()
        return dy.cpu().numpy()
    def multix(w, xs, N, Kd):
        dw, dx = dev(w), dev(np.ascontiguousarray(xs).reshape(-1))
        dy = torch.empty(xs.shape[0] * N, dtype=torch.float32, device="cuda")
        K.gemv_multix_dev(qi, dw.data_ptr(), dx.data_ptr(), dy.data_ptr(), xs.shape[0], N, Kd,
                          stream=stream())
        torch.cuda.synchronize()
        return dy.cpu().numpy().reshape(xs.shape[0], N)

    def ticket(w, xs, N, Kd):
        # moe_forward_b's ticket: one member -> the single-stream form, more
        # -> the multix pack arithmetic over exactly those members (per
        # stream for the types without a pack)
        if len(xs) > 1 and qtype in (TYPE_Q4_K, 14):
            return multix(w, xs, N, Kd)
        return np.stack([single(w, xv, N, Kd) for xv in xs])
    for s in range(B):
        p = got["probs"][s * E:(s + 1) * E]
        sel, selw = port.topk(p, k)
        assert list(got["sel"][s * k:(s + 1) * k]) == sel, s
    # batch 1 runs in three launches (SwiGLU and the combine in the GEMV
    # epilogues), which write no gate, up or per-member down outputs: those
    # are then the tickets' own calls, and act and x are checked against them
    fused = bool(got["path"] & K.FFN_FUSED_B1)
    assert fused == (B == 1), got["path"]
    a = got["act"].reshape(B * k, F)
    xr = xn.reshape(B, H)
    g, u, o = (np.full((B * k, n), np.nan, np.float32) for n in (F, F, H))
    for e, mem in O.moe_tickets(got["sel"], E):
        xs = np.stack([xr[m // k] for m in mem])
        g[mem] = ticket(d["gate"][e * F * rb_in:(e + 1) * F * rb_in], xs, F, H)
        u[mem] = ticket(d["up"][e * F * rb_in:(e + 1) * F * rb_in], xs, F, H)
        o[mem] = ticket(d["down"][e * H * rb_ff:(e + 1) * H * rb_ff], a[mem], H, F)
    if not fused:
        assert same_values(got["g"].reshape(B * k, F), g)
        assert same_values(got["u"].reshape(B * k, F), u)
        assert same_values(got["ffo"].reshape(B * k, H), o)
    for m in range(B * k):
        assert ulps(a[m], port.swiglu(g[m], u[m])).max() <= 4.0
    assert same_values(got["x"], port.moe_combine(o.reshape(-1), got["sel"], got["selw"], x0, B,
                                                  k, H))


def test_moe_ffn_step_f16_router_mixed_types(port):
    """An F16 router and gate/up/down of different types (Q4_K gate/up,
    Q6_K down): gate and up still share one routed launch, down has its
    own type."""
    H, F, E, k, B = 1024, 512, 32, 4, 3
    d = make_layer(H, F, E, k, 9600, router_type=TYPE_F16)
    d["down_type"] = 14
    d["down"] = synth.tensor(14, E * H, F, 9604)
    d["down_stride"] = H * synth.row_bytes(14, F)
    r = synth.rng(9601)
    xn = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    x0 = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    got = run_step(d, xn, x0, B)
    full = port.moe_ffn(d, xn, x0, B)
    assert np.array_equal(full["sel"], got["sel"])
    assert same_values(got["x"], port.moe_combine(got["ffo"], got["sel"], got["selw"], x0, B, k,
                                                  H))
    contrib = np.abs(full["x"] - x0).max()
    assert np.abs(got["x"] - full["x"]).max() <= 1e-4 * contrib


def test_moe_ffn_refuses_short_workspace():
    H, F, E, k, B = 512, 256, 16, 4, 2
    f = K.KqMoeFfn()
    f.n_embed, f.n_ff, f.n_experts, f.k = H, F, E, k
    f.router_type = f.gate_type = f.up_type = f.down_type = TYPE_Q4_K
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    for n in ("router", "gate", "up", "down"):
        setattr(f, n, buf.data_ptr())
    f.gate_stride = f.up_stride = f.down_stride = 1 << 16
    need = K.moe_ffn_workspace_bytes(f, B)
    x = torch.zeros(B * H, dtype=torch.float32, device="cuda")
    sel = torch.zeros(B * k, dtype=torch.int32, device="cuda")
    rc = K.lib().kq_moe_ffn_dev(K.ctypes.byref(f), x.data_ptr(), x.data_ptr(), B, sel.data_ptr(),
                                sel.data_ptr(), buf.data_ptr(), need - 256, None)
    assert rc == -1 and b"workspace" in K.lib().kq_last_error()
