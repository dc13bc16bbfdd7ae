"""The MoE FFN step's restatement in oracle/kq_oracle.c, pinned on the CPU.

stratum_engine.h (softmax, SwiGLU) includes macOS-only headers and does
not build here, so these functions are pinned by closed forms and by
binary64 recomputation:

  * softmax (stratum_engine.h:395-423): equal logits give exactly 1/E for
    E a power of two; -inf logits give 0 and leave the rest exact; a NaN
    first value makes every output NaN (the scan keeps it as the max);
    shifting integer logits leaves every output unchanged; otherwise each
    output is within 2 ulp of the binary64 softmax of the binary32
    differences x - max, and the outputs sum to 1 within E ulps;
  * SwiGLU (stratum_engine.h:373-392): g = 0 and u = 0 give 0, large |g|
    gives g * u and -0, otherwise within 3 ulp of the binary64 formula;
  * combine (stratum_arch_moe.inc.c:728-743): rank order pinned by values
    whose binary32 sum depends on it, sel < 0 skipped, exact cases equal;
  * the whole step (:689-743): each stage equals the pinned pieces and the
    kq_gemv restatement on the selected slices at their expert strides.
"""
import numpy as np
import pytest

from stratum_amd import TYPE_F32, TYPE_Q4_K, synth


def ulps(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.abs(a - b) / np.spacing(np.abs(b).astype(np.float32)).astype(np.float64)


@pytest.mark.parametrize("E", [1, 2, 64, 128, 1024])
def test_softmax_equal_logits(port, E):
    p = port.softmax(np.full(E, 0.375, np.float32))
    assert np.all(p == np.float32(1.0 / E))


def test_softmax_equal_logits_three(port):
    p = port.softmax(np.full(3, -2.0, np.float32))
    assert np.all(p == np.float32(np.float32(1.0 / 3.0)))


def test_softmax_neg_inf_and_nan(port):
    x = np.array([0.0, -np.inf, 0.0, -np.inf], np.float32)
    assert list(port.softmax(x)) == [0.5, 0.0, 0.5, 0.0]
    assert np.all(np.isnan(port.softmax(np.array([np.nan, 1.0, 2.0], np.float32))))
    # a later NaN is skipped by the scan but its exp poisons the sum
    assert np.all(np.isnan(port.softmax(np.array([1.0, np.nan, 2.0], np.float32))))


def test_softmax_shift_invariance(port):
    r = synth.rng(7700)
    x = r.integers(-20, 20, 128).astype(np.float32)
    p0 = port.softmax(x)
    for c in (1.0, 64.0, -1000.0):
        assert np.array_equal(port.softmax(x + np.float32(c)), p0)


@pytest.mark.parametrize("E", [8, 128, 1000])
def test_softmax_against_binary64(port, E):
    r = synth.rng(7800 + E)
    x = (r.standard_normal((16, E)) * 3).astype(np.float32)
    p = port.softmax(x)
    z = (x - x.max(axis=1, keepdims=True)).astype(np.float64)   # the binary32 difference
    q = np.exp(z)
    q /= q.sum(axis=1, keepdims=True)
    assert np.max(ulps(p, q.astype(np.float32))) <= 2.0
    s = p.astype(np.float64).sum(axis=1)
    assert np.all(np.abs(s - 1.0) <= E * 2.0 ** -24)


def test_swiglu_closed_forms(port):
    g = np.array([0.0, 0.0, 100.0, 100.0, -100.0, 2.0], np.float32)
    u = np.array([5.0, -3.0, 0.25, -1.5, 3.0, 0.0], np.float32)
    y = port.swiglu(g, u)
    assert y[0] == 0.0 and y[1] == 0.0
    assert y[2] == np.float32(25.0) and y[3] == np.float32(-150.0)
    assert y[4] == 0.0 and np.signbit(y[4])
    assert y[5] == 0.0


def test_swiglu_against_binary64(port):
    r = synth.rng(7900)
    g = (r.standard_normal(1 << 16) * 4).astype(np.float32)
    u = r.standard_normal(1 << 16).astype(np.float32)
    y = port.swiglu(g, u)
    gd = g.astype(np.float64)
    want = (gd / (1.0 + np.exp(-gd))) * u.astype(np.float64)
    assert np.max(ulps(y, want.astype(np.float32))) <= 3.0


def test_combine_rank_order_and_skip(port):
    B, k, H = 2, 3, 4
    o = np.zeros((B * k, H), np.float32)
    o[0] = [2.0 ** 24, 1.0, 0.5, 7.0]
    o[1] = [1.0, 2.0 ** 24, 0.25, 7.0]
    o[2] = [-(2.0 ** 24), -(2.0 ** 24), 0.125, 9.0]
    o[3:] = 1.0
    sel = np.array([4, 9, 2, 1, -1, 3], np.int32)
    selw = np.array([1.0, 1.0, 1.0, 0.5, 8.0, 0.25], np.float32)
    resid = np.arange(B * H, dtype=np.float32)
    x = port.moe_combine(o.reshape(-1), sel, selw, resid, B, k, H).reshape(B, H)
    # ((0 + 2^24) + 1) + -2^24 = 0 in binary32; the reverse order gives 1
    assert x[0, 0] == resid[0] + 0.0
    # (1 + 2^24) + -2^24 = 0
    assert x[0, 1] == resid[1] + 0.0
    assert x[0, 2] == resid[2] + np.float32(0.875)
    assert x[0, 3] == resid[3] + 23.0
    # rank 1 of token 1 has sel -1 and is skipped
    assert np.all(x[1] == resid[4:] + np.float32(0.5 + 0.25))


def make_layer(H, F, E, k, seed, router_type=TYPE_F32, qtype=TYPE_Q4_K):
    rb_in = synth.row_bytes(qtype, H)
    rb_ff = synth.row_bytes(qtype, F)
    d = {"n_embed": H, "n_ff": F, "n_experts": E, "k": k,
         "router_type": router_type, "router": synth.tensor(router_type, E, H, seed),
         "gate_type": qtype, "gate": synth.tensor(qtype, E * F, H, seed + 1),
         "up_type": qtype, "up": synth.tensor(qtype, E * F, H, seed + 2),
         "down_type": qtype, "down": synth.tensor(qtype, E * H, F, seed + 3),
         "gate_stride": F * rb_in, "up_stride": F * rb_in, "down_stride": H * rb_ff}
    return d


@pytest.mark.parametrize("B", [1, 3])
def test_moe_ffn_stages(port, B):
    H, F, E, k = 512, 256, 16, 4
    d = make_layer(H, F, E, k, 8000)
    r = synth.rng(8001)
    xn = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    x0 = np.stack([synth.gaussian(r, H) for _ in range(B)]).reshape(-1)
    out = port.moe_ffn(d, xn, x0, B)
    rb_in, rb_ff = synth.row_bytes(TYPE_Q4_K, H), synth.row_bytes(TYPE_Q4_K, F)
    for s in range(B):
        xs = xn[s * H:(s + 1) * H]
        logits = port.gemv(TYPE_F32, d["router"], xs, E, H)
        p = port.softmax(logits)
        assert np.array_equal(out["probs"][s * E:(s + 1) * E], p)
        sel, selw = port.topk(p, k)
        assert list(out["sel"][s * k:(s + 1) * k]) == sel
        for r_, e in enumerate(sel):
            m = s * k + r_
            g = port.gemv(TYPE_Q4_K, d["gate"][e * F * rb_in:(e + 1) * F * rb_in], xs, F, H)
            u = port.gemv(TYPE_Q4_K, d["up"][e * F * rb_in:(e + 1) * F * rb_in], xs, F, H)
            assert np.array_equal(out["g"][m * F:(m + 1) * F], g)
            assert np.array_equal(out["u"][m * F:(m + 1) * F], u)
            a = port.swiglu(g, u)
            assert np.array_equal(out["act"][m * F:(m + 1) * F], a)
            o = port.gemv(TYPE_Q4_K, d["down"][e * H * rb_ff:(e + 1) * H * rb_ff], a, H, F)
            assert np.array_equal(out["ffo"][m * H:(m + 1) * H], o)
    want = port.moe_combine(out["ffo"], out["sel"], out["selw"], x0, B, k, H)
    assert np.array_equal(out["x"], want)
