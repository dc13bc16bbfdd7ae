"""Pins the CPU oracle (oracle/kq_oracle.c) before it is trusted.

Checks, per function of the oracle:
  * golden fixtures written by the reference's own compiled scalar code
    and converter (tests/golden/make_golden.py) -- bit-exact;
  * direct comparison with oracle/_ref (the reference headers compiled
    where they lie), when that build exists;
  * closed forms that a plausible slip (wrong nibble, wrong scale byte,
    transposed index, dropped min term) would break: exhaustive fp16 against
    numpy, known-answer rows built from known scales/mins/quants,
    x = e_i picks the dequantized weight i, type-42 layout of single
    weights, top-k tie rules.
"""
import numpy as np
import pytest

from conftest import GOLDEN_FILES, load_golden, same_values
from oracle import oracle as O
from stratum_amd import synth

TYPES = [12, 14, 10, 42, 13, 11, 8]
REF_TYPES = [12, 14, 10, 13, 11, 8]    # the types whose scalar routines _ref builds


# ------------------------------------------------------------ fp16 widening
def test_fp16_exhaustive_matches_numpy(port):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([port.fp16_to_fp32(int(v)) for v in h], np.float32)
    # (NaN payload bits are not compared: returning a float through ctypes
    # quiets signalling NaNs)
    assert same_values(got, want)


def test_fp16_exhaustive_matches_reference(port, ref):
    h = np.arange(65536, dtype=np.uint32)
    got = np.array([port.fp16_to_fp32(int(v)) for v in h], np.float32)
    want = np.array([ref.L.kqref_fp16_to_fp32(int(v)) for v in h], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------ scale decode
def test_q4k_scale_pack_roundtrip_exhaustive(port):
    """Every (scale, min) pair in every sub-block slot survives pack -> decode."""
    v = np.arange(64, dtype=np.uint8)
    sc_all, m_all = np.meshgrid(v, v, indexing="ij")
    sc_all, m_all = sc_all.reshape(-1), m_all.reshape(-1)
    import ctypes
    out_sc, out_m = ctypes.c_uint8(), ctypes.c_uint8()
    for j in range(8):
        sc = np.zeros((sc_all.size, 8), np.uint8)
        m = np.zeros((sc_all.size, 8), np.uint8)
        sc[:, j] = sc_all
        m[:, j] = m_all
        # neighbouring slots hold distinct values so a wrong byte shows up
        for k in range(8):
            if k != j:
                sc[:, k] = (7 * k + 3) % 64
                m[:, k] = (11 * k + 5) % 64
        packed = synth.pack_q4k_scales(sc, m)
        for i in range(sc_all.size):
            row = np.ascontiguousarray(packed[i])
            port.L.ko_q4k_scale_min(j, O._u8(row), ctypes.byref(out_sc), ctypes.byref(out_m))
            assert (out_sc.value, out_m.value) == (sc[i, j], m[i, j])


def scale_bytes_read(j):
    """The scale bytes q4k_get_scale_min reads for sub-block j
    (stratum_q4k.h:57-65): j < 4 reads bytes j and j + 4; j >= 4 reads
    j + 4, j - 4 and j."""
    return [j, j + 4] if j < 4 else [j + 4, j - 4, j]


@pytest.mark.parametrize("j", range(8))
def test_q4k_scale_decode_matches_reference_exhaustive(port, ref, j):
    """Every value of the bytes sub-block j reads (2^16 for j < 4, 2^24 for
    j >= 4), with the other nine or ten bytes fixed to zeros, to ones, and
    to a random pattern: the oracle equals the reference's own decode on
    all of them, and the result does not depend on the other bytes."""
    idx = scale_bytes_read(j)
    first = None
    for bg in (np.zeros(12, np.uint8), np.full(12, 0xff, np.uint8),
               np.random.default_rng(j).integers(0, 256, 12).astype(np.uint8)):
        got = O.scale_min_sweep(port.L.ko_q4k_scale_min_sweep, j, idx, bg)
        want = O.scale_min_sweep(ref.L.kqref_scale_min_sweep, j, idx, bg)
        assert np.array_equal(got, want), j
        if first is None:
            first = got
        assert np.array_equal(got, first), j
    # closed form of the decode on the first byte combinations: the 6-bit
    # fields, and for j >= 4 the nibble plus the top bits of bytes j-4 / j
    c = np.arange(first.shape[0], dtype=np.int64)
    b = [(c >> (8 * i)) & 0xff for i in range(len(idx))]
    if j < 4:
        sc, m = b[0] & 63, b[1] & 63
    else:
        sc = (b[0] & 15) | ((b[1] >> 6) << 4)
        m = (b[0] >> 4) | ((b[2] >> 6) << 4)
    assert np.array_equal(first[:, 0], sc) and np.array_equal(first[:, 1], m), j


def q3k_scale_bytes_read(g):
    """Bytes q3k_unpack_scales reads for scale g (stratum_q3k.h:17-28): the
    nibble from byte g%4 (+4 for words 1 and 3), the top two bits from
    byte 8 + g%4."""
    w, bi = g // 4, g % 4
    return [(4 if w & 1 else 0) + bi, 8 + bi]


@pytest.mark.parametrize("g", range(16))
def test_q3k_scale_decode_matches_reference_exhaustive(port, ref, g):
    """Every value of the two bytes Q3_K scale g reads, with the other ten
    fixed to zeros, ones and a random pattern: the oracle's decode equals
    the reference's q3k_unpack_scales and ignores the other bytes."""
    idx = q3k_scale_bytes_read(g)
    first = None
    for bg in (np.zeros(12, np.uint8), np.full(12, 0xff, np.uint8),
               np.random.default_rng(100 + g).integers(0, 256, 12).astype(np.uint8)):
        got = O.q3k_scale_sweep(port.L.ko_q3k_scale_sweep, g, idx, bg)
        want = O.q3k_scale_sweep(ref.L.kqref_q3k_scale_sweep, g, idx, bg)
        assert np.array_equal(got, want), g
        first = got if first is None else first
        assert np.array_equal(got, first), g
    c = np.arange(first.size)
    lo, hi = c & 0xff, c >> 8
    w = g // 4
    nib = (lo >> 4) if w & 2 else (lo & 15)
    assert np.array_equal(first, nib | (((hi >> (2 * w)) & 3) << 4)), g


# ------------------------------------------------------- golden fixtures
@pytest.mark.parametrize("qtype", TYPES)
def test_oracle_matches_golden(port, qtype):
    for case, d in load_golden(GOLDEN_FILES[qtype]).items():
        N, K = (int(v) for v in d["shape"])
        deq = port.dequant(qtype, d["w"], N, K)
        assert same_values(deq, d["deq"]), (qtype, case, "dequant")
        y = port.gemv(qtype, d["w"], d["x"], N, K)
        assert same_values(y, d["y"]), (qtype, case, "dot")


@pytest.mark.parametrize("qtype", REF_TYPES)
@pytest.mark.parametrize("K", [256, 768, 2048])
def test_oracle_matches_reference_random(port, ref, qtype, K):
    for seed in range(3):
        N = 33
        w = synth.tensor(qtype, N, K, seed)
        x = synth.gaussian(synth.rng(100 + seed), K)
        assert same_values(port.dequant(qtype, w, N, K), ref.dequant(qtype, w, N, K))
        assert same_values(port.gemv(qtype, w, x, N, K), ref.gemv(qtype, w, x, N, K))


@pytest.mark.parametrize("qtype", [12, 14, 10])
def test_oracle_add_is_one_binary32_add_after_the_row(port, ref, qtype):
    """st_linear_dispatch_add computes y[r] = add[r] + dot, the row's
    result rounded to binary32 first and then one binary32 addition
    (stratum_linear.h:566-600).  The oracle's add path must equal the
    reference's plain GEMV plus a numpy float32 add bit for bit; adding
    before the final rounding (in binary64) would differ on these inputs."""
    N, K = 257, 1024
    w = synth.tensor(qtype, N, K, 61)
    x = synth.gaussian(synth.rng(62), K)
    r = np.random.default_rng(63)
    # adds of every magnitude relative to the row results, so that the
    # rounding of the sum differs between the two orders on many rows
    add = (synth.gaussian(r, N) * np.float32(2.0) ** r.integers(-30, 30, N)).astype(np.float32)
    got = port.gemv(qtype, w, x, N, K, add=add)
    want = add + ref.gemv(qtype, w, x, N, K)
    assert same_values(got, want)
    # the other order (binary64 sum, rounded once) gives different bits
    fused = np.array([np.float32(np.float64(a) + port.L.ko_dot_row_f64(
        qtype, O._u8(np.ascontiguousarray(w[i * (w.size // N):(i + 1) * (w.size // N)])), K,
        O._f(x))) for i, a in enumerate(add)], np.float32)
    assert not same_values(fused, want)


def test_oracle_threads_do_not_change_results(port):
    w = synth.tensor(12, 300, 1024, 3)
    x = synth.gaussian(synth.rng(4), 1024)
    y1 = port.gemv(12, w, x, 300, 1024, threads=1)
    y8 = port.gemv(12, w, x, 300, 1024, threads=8)
    assert same_values(y1, y8)


# ----------------------------------------------------------- closed forms
@pytest.mark.parametrize("qtype", TYPES)
def test_unit_vector_picks_dequantized_weight(port, qtype):
    """dot(row, e_i) == dequant(row)[i] exactly: every other sub-block term
    is fl(d*0 - m*0) = 0 and the one product is q_i * 1."""
    K = 512
    w = synth.tensor(qtype, 1, K, 7)
    deq = port.dequant(qtype, w, 1, K)
    for i in list(range(0, K, 37)) + [K - 1]:
        x = np.zeros(K, np.float32)
        x[i] = 1.0
        assert port.gemv(qtype, w, x, 1, K)[0] == deq[i], (qtype, i)


def test_q4k_known_answer_from_construction(port):
    """Blocks built from KNOWN scales/mins/quants; expected dot with x = 1
    derived from those arrays, not from decoding the block."""
    r = np.random.default_rng(5)
    n = 64
    sc = r.integers(0, 64, (n, 8), dtype=np.uint8)
    m = r.integers(0, 64, (n, 8), dtype=np.uint8)
    q = r.integers(0, 16, (n, 8, 32), dtype=np.uint8)
    d = np.float16(0.0123)
    dmin = np.float16(0.00457)
    b = np.zeros((n, 144), np.uint8)
    b[:, 0:2] = np.array([d], np.float16).view(np.uint8)
    b[:, 2:4] = np.array([dmin], np.float16).view(np.uint8)
    b[:, 4:16] = synth.pack_q4k_scales(sc, m)
    for s in range(8):  # sub-block s: qs bytes 32*(s//2).., nibble s%2
        if s % 2 == 0:
            b[:, 16 + 32 * (s // 2):48 + 32 * (s // 2)] |= q[:, s, :]
        else:
            b[:, 16 + 32 * (s // 2):48 + 32 * (s // 2)] |= q[:, s, :] << 4
    x = np.ones(256, np.float32)
    got = port.gemv(12, np.ascontiguousarray(b.reshape(-1)), x, n, 256)
    f = np.float32
    for i in range(n):
        dot = 0.0
        for s in range(8):
            a = f(q[i, s].sum())                     # exact small-integer sum
            t = f(f(f(d) * f(sc[i, s])) * a) - f(f(f(dmin) * f(m[i, s])) * f(32.0))
            dot += float(t)
        assert got[i] == f(dot), i


def test_q6k_known_answer_from_construction(port):
    """Q6_K block from known 6-bit quants and int8 scales, x = 1."""
    r = np.random.default_rng(6)
    n = 32
    q = r.integers(0, 64, (n, 256), dtype=np.int64)     # by position
    sc = r.integers(-128, 128, (n, 16), dtype=np.int64)
    d = np.float16(0.0071)
    b = np.zeros((n, 210), np.uint8)
    for p in range(256):
        h, t, l = p // 128, (p % 128) // 32, p % 32
        lo = q[:, p] & 15
        hi = q[:, p] >> 4
        b[:, 64 * h + l + 32 * (t & 1)] |= (lo << (4 * (t >> 1))).astype(np.uint8)
        b[:, 128 + 32 * h + l] |= (hi << (2 * t)).astype(np.uint8)
    b[:, 192:208] = sc.astype(np.int8).view(np.uint8)
    b[:, 208:210] = np.array([d], np.float16).view(np.uint8)
    x = np.ones(256, np.float32)
    got = port.gemv(14, np.ascontiguousarray(b.reshape(-1)), x, n, 256)
    for i in range(n):
        dot = 0.0
        for h in range(2):
            for is_ in range(2):
                for t in range(4):
                    pos = [128 * h + 32 * t + 16 * is_ + l for l in range(16)]
                    a = float(np.float32((q[i, pos] - 32).sum()))
                    dot += float(d) * float(sc[i, 8 * h + is_ + 2 * t]) * a
        assert got[i] == np.float32(dot), i


def test_q2k_known_answer_from_construction(port):
    r = np.random.default_rng(8)
    n = 32
    q = r.integers(0, 4, (n, 256), dtype=np.int64)
    scb = r.integers(0, 256, (n, 16), dtype=np.int64)
    d, dmin = np.float16(0.0219), np.float16(0.0033)
    b = np.zeros((n, 84), np.uint8)
    for p in range(256):
        s, j, hl = p // 128, (p % 128) // 32, p % 32
        b[:, 16 + 32 * s + hl] |= (q[:, p] << (2 * j)).astype(np.uint8)
    b[:, 0:16] = scb.astype(np.uint8)
    b[:, 80:82] = np.array([d], np.float16).view(np.uint8)
    b[:, 82:84] = np.array([dmin], np.float16).view(np.uint8)
    x = np.ones(256, np.float32)
    f = np.float32
    got = port.gemv(10, np.ascontiguousarray(b.reshape(-1)), x, n, 256)
    for i in range(n):
        dot = 0.0
        for g in range(16):  # group g covers positions 16g..16g+15
            a = f(q[i, 16 * g:16 * g + 16].sum())
            dl = f(f(d) * f(scb[i, g] & 15))
            ml = f(f(dmin) * f(scb[i, g] >> 4))
            dot += float(f(dl * a) - f(ml * f(16.0)))
        assert got[i] == f(dot), i


# ------------------------------------------------------------ type 42
def test_nib_layout_single_weight(port):
    """One non-zero weight at position p lands in byte 16 + 16*(p//32) + p%16,
    low nibble for p%32 < 16 -- the reader layout of stratum_q2k_neon.h:265-291."""
    for p in [0, 5, 15, 16, 31, 32, 100, 127, 128, 200, 255]:
        b = np.zeros(84, np.uint8)
        s, j, hl = p // 128, (p % 128) // 32, p % 32
        b[16 + 32 * s + hl] = 3 << (2 * j)
        nib = port.q2k_to_nib(b)
        nz = np.nonzero(nib[16:144])[0]
        assert list(nz) == [16 * (p // 32) + p % 16], p
        v = nib[16 + nz[0]]
        assert v == (0x30 if p % 32 >= 16 else 0x03), p


def test_nib_matches_reference_converter_golden(port):
    for case, d in load_golden("q2k_nib").items():
        q2 = d["src"]
        assert np.array_equal(port.q2k_to_nib(q2), d["w"]), case
        assert np.array_equal(synth.q2k_to_nib(q2), d["w"]), case
        assert np.array_equal(port.nib_to_q2k(d["w"]), q2), case


def test_nib_roundtrip_and_value_identity(port):
    q2 = synth.tensor(10, 40, 1024, 11)
    nib = port.q2k_to_nib(q2)
    assert np.array_equal(port.nib_to_q2k(nib), q2)
    assert same_values(port.dequant(42, nib, 40, 1024), port.dequant(10, q2, 40, 1024))
    x = synth.gaussian(synth.rng(12), 1024)
    assert same_values(port.gemv(42, nib, x, 40, 1024), port.gemv(10, q2, x, 40, 1024))


# -------------------------------------------------------------- top-k
def test_topk_ties_keep_lower_id(port):
    w = np.array([0.1, 0.3, 0.3, 0.2, 0.3, 0.05], np.float32)
    sel, selw = port.topk(w, 3)
    assert sel == [1, 2, 4]
    sel, _ = port.topk(w, 4)
    assert sel == [1, 2, 4, 3]
    sel, _ = port.topk(np.full(8, 0.125, np.float32), 2)
    assert sel == [0, 1]


def test_topk_matches_sort(port):
    r = np.random.default_rng(3)
    for _ in range(200):
        w = r.standard_normal(128).astype(np.float32)
        sel, selw = port.topk(w, 8)
        order = sorted(range(128), key=lambda e: (-w[e], e))[:8]
        assert sel == order
        assert np.array_equal(selw, w[order])


# ------------------------------------------------------------ F16 / F32
# st_linear_f16 (stratum_linear.h:491-505) sums exact binary64 products in
# element order; F32 goes to cblas_sgemv (:508-512), restated as the same
# binary64 sum of exact products.  Neither builds here (the file needs
# Accelerate), so these pin the restatement by closed forms.
def _dense(qtype, vals):
    v = np.asarray(vals, np.float32)
    return (v.astype(np.float16).view(np.uint8) if qtype == 1 else v.view(np.uint8)).copy()


@pytest.mark.parametrize("qtype", [1, 0])
def test_dense_unit_vectors_and_integers(port, qtype):
    K = 512
    r = np.random.default_rng(7 + qtype)
    w = r.integers(-8, 8, (3, K)).astype(np.float32)
    w[1] *= np.float32(0.125)                 # exact in fp16 as well
    wb = _dense(qtype, w.reshape(-1))
    for i in (0, 1, 255, 256, K - 1):
        x = np.zeros(K, np.float32)
        x[i] = 1.0
        assert np.array_equal(port.gemv(qtype, wb, x, 3, K), w[:, i])
    x = r.integers(-100, 100, K).astype(np.float32)
    assert np.array_equal(port.gemv(qtype, wb, x, 3, K), (w.astype(np.float64) @ x).astype(np.float32))


@pytest.mark.parametrize("qtype", [1, 0])
def test_dense_sum_is_elementwise_binary64(port, qtype):
    """Random rows: the oracle equals a Python loop of exact binary64
    products added in element order, and differs from the correctly rounded
    sum (math.fsum) by less than one binary32 ulp; the fp16 decode is
    numpy's."""
    import math
    K = 1024
    r = np.random.default_rng(11 + qtype)
    w = (r.standard_normal((4, K)) * 0.05).astype(np.float32)
    wb = _dense(qtype, w.reshape(-1))
    wv = (wb.view(np.float16).astype(np.float64) if qtype == 1 else wb.view(np.float32).astype(np.float64))
    wv = wv.reshape(4, K)
    x = r.standard_normal(K).astype(np.float32)
    got = port.gemv(qtype, wb, x, 4, K)
    for rr in range(4):
        acc = 0.0
        for c in range(K):
            acc += float(wv[rr, c]) * float(x[c])
        assert got[rr] == np.float32(acc)
        exact = math.fsum(float(wv[rr, c]) * float(x[c]) for c in range(K))
        assert abs(float(got[rr]) - exact) <= np.spacing(np.float32(abs(exact)))
