"""The int8-activation restatement in oracle/kq_oracle.c, pinned on the CPU.

The reference's SDOT kernels (stratum_q4k_neon.h, stratum_q6k_neon.h) need
NEON and do not build here, so oracle/_ref cannot check this part.  What
pins it instead:

  * the quantizer against closed forms: groups whose largest |x| is
    127 * 2^e quantize exactly (scale 2^e, q = x / 2^e), halfway values
    round to even, zero groups give scale 0 and q 0, and for any x the
    rounding error is at most half a step;
  * the integer dots, group indexing and coefficients against the pinned
    dequantization: with power-of-two d / dmin and exactly quantizable x,
    every step is exact and the int8 GEMV must equal the binary64 sum of
    dequant(w) * x (a wrong group, scale or sign breaks this);
  * the reference's own test of the mode (quant_test.c:95-122): on its
    data (d = 0.01, dmin = 0.001, x uniform in [-0.5, 0.5)) the result is
    within 5e-2 relative of the exact dot;
  * the two summation orders (binary32 FMA lanes of q*_dot_row_sdot_f vs
    binary64 terms) within the lanes' rounding bound.
"""
import numpy as np
import pytest

from i8_cases import reciprocal_groups
from oracle import oracle as O
from stratum_amd import TYPE_Q3_K, TYPE_Q4_K, TYPE_Q5_K, TYPE_Q6_K, TYPE_Q8_0, synth

I8_TYPES = [TYPE_Q4_K, TYPE_Q6_K, TYPE_Q5_K, TYPE_Q3_K, TYPE_Q8_0]
GROUP = {TYPE_Q4_K: 32, TYPE_Q6_K: 16, TYPE_Q5_K: 32, TYPE_Q3_K: 32, TYPE_Q8_0: 32}


def exact_x(r, K, G, e):
    """x whose every group has max |x| = 127 * 2^e and values k * 2^e"""
    k = r.integers(-127, 128, K).astype(np.int32)
    k.reshape(-1, G)[:, r.integers(0, G)] = np.where(r.integers(0, 2, K // G) > 0, 127, -127)
    return (k.astype(np.float32) * np.float32(2.0 ** e)), k


@pytest.mark.parametrize("G", [32, 16])
def test_quantize_exact_groups(port, G):
    r = synth.rng(7100 + G)
    K = 1024
    x, k = exact_x(r, K, G, -7)
    xq, xs = port.quantize_q8(x, G)
    assert np.array_equal(xq.astype(np.int32), k)
    assert np.all(xs == np.float32(2.0 ** -7))


@pytest.mark.parametrize("G", [32, 16])
def test_quantize_halfway_zero_sign(port, G):
    K = 4 * G
    x = np.zeros(K, np.float32)
    g0 = x[0:G]
    g0[0] = 127.0
    g0[1:9] = [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5]   # ties to even
    x[G] = -127.0 * 4                                              # negative amax
    x[G + 1] = 3.0 * 4
    # group 2 stays zero; group 3: a denormal-free tiny group
    x[3 * G:4 * G] = np.float32(1e-30)
    xq, xs = port.quantize_q8(x, G)
    assert list(xq[0:9]) == [127, 0, 2, 2, 0, -2, -2, 126, -126]
    assert xs[0] == 1.0 and xs[1] == 4.0
    assert xq[G] == -127 and xq[G + 1] == 3
    assert xs[2] == 0.0 and not np.any(xq[2 * G:3 * G])
    assert np.all(xq[3 * G:4 * G] == 127)


@pytest.mark.parametrize("G", [32, 16])
def test_quantize_multiplies_by_the_rounded_reciprocal(port, G):
    """q = rne(fl(x * fl(1 / scale))) as the reference writes it
    (stratum_q4k_neon.h:262-276, stratum_q6k_neon.h:117-133), not
    rne(fl(x / scale)): on 24 inputs where the two round to different
    integers, the restatement gives the reciprocal form's value."""
    x, want = reciprocal_groups(G, 24)
    xq, xs = port.quantize_q8(x, G)
    got = xq.reshape(-1, G)[:, 1].astype(np.int32)
    assert np.array_equal(got, want)
    amax = x.reshape(-1, G)[:, 0]
    div = np.rint((x.reshape(-1, G)[:, 1] / (amax / np.float32(127.0))).astype(np.float32))
    assert np.all(div.astype(np.int32) != want)
    assert np.all(xq.reshape(-1, G)[:, 0] == 127)


@pytest.mark.parametrize("G", [32, 16])
def test_quantize_error_bound(port, G):
    r = synth.rng(7200 + G)
    K = 8192
    x = synth.gaussian(r, K) * np.float32(3.0)
    xq, xs = port.quantize_q8(x, G)
    amax = np.abs(x.reshape(-1, G)).max(axis=1)
    assert np.all(xs == amax / np.float32(127.0))
    step = np.repeat(xs.astype(np.float64), G)
    err = np.abs(xq.astype(np.float64) * step - x.astype(np.float64))
    assert np.all(err <= 0.5 * step * (1 + 2.0 ** -20))
    assert np.all(np.abs(xq.astype(np.int32)) <= 127)
    # the largest |x| of each group maps to +-127
    imax = np.abs(x.reshape(-1, G)).argmax(axis=1)
    top = xq.reshape(-1, G)[np.arange(K // G), imax].astype(np.int32)
    assert np.all(np.abs(top) == 127)


def pow2_blocks(qtype, r, nblocks, small=False):
    """random blocks with d = 2^-10 (and dmin = 2^-12), so every product is
    exact; small: scales (and mins) limited to 3 bits (Q3_K: sc - 32 in
    0..3; Q8_0: quants in -8..7), so that the reference's binary32 lanes
    stay exact too over one block"""
    b = synth.blocks(qtype, r, nblocks).reshape(nblocks, -1)
    f16 = lambda v: np.array([v], np.float16).view(np.uint8)   # noqa: E731
    if qtype in (TYPE_Q4_K, TYPE_Q5_K):
        b[:, 0:2] = f16(2.0 ** -10)
        b[:, 2:4] = f16(2.0 ** -12)
        if small:
            b[:, 4:16] = synth.pack_q4k_scales(r.integers(0, 8, (nblocks, 8)),
                                               r.integers(0, 8, (nblocks, 8)))
    elif qtype == TYPE_Q6_K:
        b[:, 208:210] = f16(2.0 ** -10)
        if small:
            b[:, 192:208] = r.integers(-4, 4, (nblocks, 16)).astype(np.int8).view(np.uint8)
    elif qtype == TYPE_Q3_K:
        b[:, 108:110] = f16(2.0 ** -10)
        if small:   # every 6-bit scale 32 + (0..3): low nibbles 0..3, top bits 2
            lo = r.integers(0, 4, (nblocks, 8, 2))
            b[:, 96:104] = (lo[:, :, 0] | (lo[:, :, 1] << 4)).astype(np.uint8)
            b[:, 104:108] = 0xAA
    else:            # Q8_0: eight 34-byte blocks per 256 weights
        u = b.reshape(nblocks, 8, 34)
        u[:, :, 0:2] = f16(2.0 ** -10)
        if small:
            u[:, :, 2:34] = r.integers(-8, 8, (nblocks, 8, 32)).astype(np.int8).view(np.uint8)
    return b.reshape(-1)


@pytest.mark.parametrize("qtype", I8_TYPES)
@pytest.mark.parametrize("case", ["wide", "small-f32-lanes", "small"])
def test_i8_exact_against_dequant(port, qtype, case):
    """exactly quantizable x and exact products: y == fl(sum dequant(w) * x).
    'wide' (random scales, two blocks) holds for the binary64 order only;
    'small' also for the reference's binary32 lanes (sdot_f)."""
    r = synth.rng(7300 + qtype + (0 if case == "wide" else 50))
    small = case != "wide"
    N, K = 24, 256 if small else 512
    w = pow2_blocks(qtype, r, N * K // 256, small)
    x, _ = exact_x(r, K, GROUP[qtype], -7)
    deq = port.dequant(qtype, w, N, K).reshape(N, K).astype(np.float64)
    want = (deq * x.astype(np.float64)).sum(axis=1)          # exact in binary64
    y = port.gemv_i8(qtype, w, x, N, K, sdot_f=case == "small-f32-lanes")
    assert np.array_equal(y, want.astype(np.float32))


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_i8_reference_quant_test_case(port, qtype):
    """quant_test.c's data and relation for each type's SDOT form, rel err
    <= 5e-2 against the exact dot: Q4_K :95-122, Q6_K :196-237, Q5_K
    :150-187 (d 0.01, dmin 0.001), Q3_K :245-275 (d 0.01), Q8_0 :45-88
    (d 0.01 + U(0, 1), random int8 quants); random bytes elsewhere.  The
    reference asserts the relation on one dot of its own seed; over several
    rows, the signed types (Q3_K, Q8_0) can cancel to a dot far below its
    terms, so the relative error is taken against max(|dot|, 0.1 sum |w x|)."""
    r = synth.rng(7400 + qtype)
    N, K = 8, 1024
    bb = K // 256 * synth.row_bytes(qtype, 256)
    b = r.integers(0, 256, (N * K // 256, bb // (K // 256)), dtype=np.uint8)
    f16 = lambda v: np.array(v, np.float16).view(np.uint8)   # noqa: E731
    if qtype in (TYPE_Q4_K, TYPE_Q5_K):
        b[:, 0:2] = f16([0.01])
        b[:, 2:4] = f16([0.001])
    elif qtype == TYPE_Q6_K:
        b[:, 208:210] = f16([0.01])
    elif qtype == TYPE_Q3_K:
        b[:, 108:110] = f16([0.01])
    else:
        u = b.reshape(-1, 8, 34)
        d = (0.01 + r.integers(0, 0x10000, (u.shape[0], 8)) / 65535.0).astype(np.float16)
        u[:, :, 0:2] = d.view(np.uint8).reshape(u.shape[0], 8, 2)
    w = b.reshape(-1)
    x = (r.integers(0, 0x10000, K) / 32768.0 - 0.5).astype(np.float32)
    deq = port.dequant(qtype, w, N, K).reshape(N, K).astype(np.float64)
    ref = (deq * x.astype(np.float64)).sum(axis=1).astype(np.float32)
    mag = (np.abs(deq) * np.abs(x.astype(np.float64))).sum(axis=1)
    for sdot_f in (True, False):
        y = port.gemv_i8(qtype, w, x, N, K, sdot_f=sdot_f)
        rel = np.abs(y - ref) / np.maximum(np.maximum(np.abs(ref), 0.1 * mag), 1e-6)
        assert rel.max() <= 5e-2, (sdot_f, rel.max())


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_i8_orders_within_lane_bound(port, qtype):
    r = synth.rng(7500 + qtype)
    N, K = 64, 4096
    w = synth.blocks(qtype, r, N * K // 256)
    x = synth.gaussian(r, K)
    yg = port.gemv_i8(qtype, w, x, N, K)
    yf, mag = port.gemv_i8(qtype, w, x, N, K, sdot_f=True, with_mag=True)
    d = np.abs(yg.astype(np.float64) - yf.astype(np.float64))
    bound = (K / 64 + 3) * 2.0 ** -24 * mag + 2.0 ** -24 * np.abs(yg.astype(np.float64))
    assert np.all(d <= bound)
    # int8 quantization error stays small against the exact fp32 path
    y32 = port.gemv(qtype, w, x, N, K)
    assert np.max(np.abs(yg - y32)) <= 5e-2 * np.max(np.abs(y32))


@pytest.mark.parametrize("qtype", I8_TYPES)
def test_i8_add(port, qtype):
    r = synth.rng(7600 + qtype)
    N, K = 16, 768
    w = synth.blocks(qtype, r, N * K // 256)
    x = synth.gaussian(r, K)
    add = synth.gaussian(r, N)
    y = port.gemv_i8(qtype, w, x, N, K)
    ya = port.gemv_i8(qtype, w, x, N, K, add=add)
    assert np.array_equal(ya, add + y)


# ------------------------------------------------- int8 MULTISEQ (pack form)
MX_TYPES = [TYPE_Q4_K, TYPE_Q6_K]


@pytest.mark.parametrize("qtype", MX_TYPES)
def test_i8_multix_exact_against_dequant(port, qtype):
    """the multix_pack arithmetic on exact inputs (power-of-two d / dmin,
    3-bit scales and mins, exactly quantizable x): every term is exact, so
    each stream's y == fl(sum dequant(w) * x)"""
    r = synth.rng(7700 + qtype)
    N, K, B = 20, 512, 3
    w = pow2_blocks(qtype, r, N * K // 256, small=True)
    xs = np.stack([exact_x(r, K, GROUP[qtype], -7 + s)[0] for s in range(B)])
    deq = port.dequant(qtype, w, N, K).reshape(N, K).astype(np.float64)
    want = (xs.astype(np.float64) @ deq.T).astype(np.float32)
    assert np.array_equal(port.gemv_i8_multix(qtype, w, xs, N, K), want)


@pytest.mark.parametrize("qtype", MX_TYPES)
def test_i8_multix_reference_relation(port, qtype):
    """quant_test.c:126-145 (Q4_K) / :228-238 (Q6_K): on the reference's
    data (d 0.01, dmin 0.001, x uniform in [-0.5, 0.5)), B = 4 streams of
    the pack form within 1e-4 relative of q*_dot_row_sdot_f (the
    single-stream lanes), and within 5e-2 of the exact dot (relative to
    max(|dot|, 0.1 sum |w x|), as random signed Q6_K rows can cancel)"""
    r = synth.rng(7800 + qtype)
    N, K, B = 8, 1024, 4
    b = r.integers(0, 256, (N * K // 256, 144 if qtype == TYPE_Q4_K else 210), dtype=np.uint8)
    if qtype == TYPE_Q4_K:
        b[:, 0:2] = np.array([0.01], np.float16).view(np.uint8)
        b[:, 2:4] = np.array([0.001], np.float16).view(np.uint8)
    else:
        b[:, 208:210] = np.array([0.01], np.float16).view(np.uint8)
    w = b.reshape(-1)
    xs = (r.integers(0, 0x10000, (B, K)) / 32768.0 - 0.5).astype(np.float32)
    ys = port.gemv_i8_multix(qtype, w, xs, N, K)
    deq = port.dequant(qtype, w, N, K).reshape(N, K).astype(np.float64)
    for s in range(B):
        fy = port.gemv_i8(qtype, w, xs[s], N, K, sdot_f=True)
        assert np.all(np.abs(ys[s] - fy) <= 1e-4 * np.maximum(np.abs(fy), 1e-6)), s
        ref = deq @ xs[s].astype(np.float64)
        mag = np.abs(deq) @ np.abs(xs[s].astype(np.float64))
        assert np.all(np.abs(ys[s] - ref) <= 5e-2 * np.maximum(np.abs(ref), 0.1 * mag)), s


@pytest.mark.parametrize("qtype", MX_TYPES)
def test_i8_multix_within_term_bound_of_binary64_terms(port, qtype):
    """each pack term rounds at most four times in binary32 (Q4_K; Q6_K's
    are binary64): against the exact-term binary64 order of the
    single-stream form the difference stays within 5 2^-24 sum|term| plus
    one ulp"""
    r = synth.rng(7900 + qtype)
    N, K, B = 48, 4096, 5
    w = synth.blocks(qtype, r, N * K // 256)
    xs = np.stack([synth.gaussian(r, K) for _ in range(B)])
    ys = port.gemv_i8_multix(qtype, w, xs, N, K)
    for s in range(B):
        yg = port.gemv_i8(qtype, w, xs[s], N, K)
        _, mag = port.gemv_i8(qtype, w, xs[s], N, K, sdot_f=True, with_mag=True)
        d = np.abs(ys[s].astype(np.float64) - yg.astype(np.float64))
        bound = 5 * 2.0 ** -24 * mag + np.spacing(np.abs(yg)).astype(np.float64)
        assert np.all(d <= bound), s


def test_moe_tickets_rule():
    """oracle.moe_tickets, moe_forward_b's expert tickets
    (stratum_arch_moe.inc.c:1136-1140, 1158-1178): a worked case, the cut
    at 8, and over random selections the invariants the reference's loops
    fix -- every chosen member in exactly one ticket of its expert, members
    in increasing order, experts in increasing order, every ticket but an
    expert's last holding exactly 8."""
    # B = 3, k = 2: members 0..5 choose experts 1,0 | 1,2 | 0,1
    assert O.moe_tickets([1, 0, 1, 2, 0, 1], 3) == [(0, [1, 4]), (1, [0, 2, 5]), (2, [3])]
    assert O.moe_tickets([-1, 2, -1], 4) == [(2, [1])]
    assert [len(m) for _, m in O.moe_tickets([5] * 19, 6)] == [8, 8, 3]
    rng = np.random.default_rng(11)
    for _ in range(50):
        B, k, E = int(rng.integers(1, 40)), int(rng.integers(1, 9)), int(rng.integers(8, 64))
        sel = np.stack([rng.choice(E, k, replace=False) for _ in range(B)]).reshape(-1)
        sel[rng.random(sel.size) < 0.05] = -1
        t = O.moe_tickets(sel, E)
        seen = sorted(m for _, mem in t for m in mem)
        assert seen == [m for m in range(sel.size) if sel[m] >= 0]
        assert [e for e, _ in t] == sorted(e for e, _ in t)
        for i, (e, mem) in enumerate(t):
            assert all(sel[m] == e for m in mem) and mem == sorted(mem) and 1 <= len(mem) <= 8
            if i + 1 < len(t) and t[i + 1][0] == e:
                assert len(mem) == 8 and mem[-1] < t[i + 1][1][0]
