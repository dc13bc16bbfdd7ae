"""MoE host logic through the C ABI (no GPU): expert-slice sizes and
descriptors, the .moep pack header checks and addressing, and the host
top-k, each against the oracle's restatement and closed-form values."""
import ctypes
import struct

import numpy as np
import pytest

import stratum_amd as K
from oracle import oracle as O

H, F, E = 2048, 768, 128          # the MoE configuration (hidden, expert ffn, experts)


def stacked(qtype, K_in, N_out, n_exp, offset=0):
    t = K.make_tensor(qtype, N_out, K_in, offset)
    t.n_dims = 3
    t.dims[2] = n_exp
    t.nelem = K_in * N_out * n_exp
    t.nbytes = n_exp * N_out * (K_in // 256) * K.BLOCK_BYTES[qtype]
    return t


def test_slice_bytes_known_values():
    """Q4_K gate/up slice of the MoE configuration: 768 rows x 8 blocks x
    144 B = 884,736 B; the expert span gate+up+down is 2,654,208 B."""
    g = stacked(12, H, F, E)
    d = stacked(12, F, H, E)
    assert K.moe_slice_bytes(g, H, F) == 884736
    assert K.moe_slice_bytes(g, H, F) * 2 + K.moe_slice_bytes(d, F, H) == 2654208


@pytest.mark.parametrize("qtype", [10, 12, 14, 42, 43, 44])
@pytest.mark.parametrize("sizes", ["set", "unset"])
def test_slice_bytes_matches_oracle(qtype, sizes):
    for K_in, N_out, n_exp in [(2048, 768, 128), (768, 2048, 64), (1024, 512, 3)]:
        t = K.make_tensor(qtype if qtype in K.BLOCK_BYTES else 12, N_out, K_in, 0)
        t.type = qtype
        t.nelem = K_in * N_out * n_exp if sizes == "set" else 0
        t.nbytes = (n_exp * N_out * (K_in // 256) * K.BLOCK_BYTES.get(qtype, 144)
                    if sizes == "set" else 0)
        want = O.moe_slice_bytes(qtype, t.nelem, t.nbytes, K_in, N_out)
        assert K.moe_slice_bytes(t, K_in, N_out) == want, (qtype, K_in, N_out)


def test_slice_bytes_w16_closed_form():
    """Types 43/44 (W16 experts): 2 B per weight + 8 B per 256 (+ 2 B per
    32 for 43), e.g. 768 x 2048: 3,145,728 + 49,152 (+ 98,304)."""
    t = K.make_tensor(12, F, H, 0)
    t.type = 43
    assert K.moe_slice_bytes(t, H, F) == 3145728 + 49152 + 98304
    t.type = 44
    assert K.moe_slice_bytes(t, H, F) == 3145728 + 49152


def test_bind_slice_in_stacked_tensor_and_pack():
    g = stacked(12, H, F, E, offset=1 << 20)
    sl = K.moe_slice_bytes(g, H, F)
    d = K.moe_bind_slice(g, 37, sl, F, H)
    assert d.offset == (1 << 20) + 37 * sl
    assert d.nbytes == sl and d.nelem == H * F and d.type == 12
    assert list(d.dims) == list(g.dims)
    base = 0x7f0000000000
    d2 = K.moe_bind_slice(g, 37, sl, F, H, slice_host=base + 123456, base=base)
    assert d2.offset == 123456


def build_pack(n_layers, n_exp, n_emb, n_ff, types, rng, data_off=4096):
    """A .moep file laid out as the reference's tools/moe_expert_pack.py
    describes it: '<4s8I4Q' header, zero padding to data_off, then for each
    layer and expert the gate|up|down slices."""
    gsb = n_ff * (n_emb // 256) * K.BLOCK_BYTES[types[0]]
    usb = n_ff * (n_emb // 256) * K.BLOCK_BYTES[types[1]]
    dsb = n_emb * (n_ff // 256) * K.BLOCK_BYTES[types[2]]
    hdr = struct.pack("<4s8I4Q", b"MOEP", 1, n_layers, n_exp, n_emb, n_ff, *types, gsb, usb,
                      dsb, data_off)
    assert len(hdr) == 68
    body = rng.integers(0, 256, n_layers * n_exp * (gsb + usb + dsb), dtype=np.uint8)
    blob = np.concatenate([np.frombuffer(hdr, np.uint8), np.zeros(data_off - 68, np.uint8), body])
    return blob, (gsb, usb, dsb)


def pack_tensors(n_emb, n_ff, n_exp, types):
    return (stacked(types[0], n_emb, n_ff, n_exp), stacked(types[1], n_emb, n_ff, n_exp),
            stacked(types[2], n_ff, n_emb, n_exp))


def test_pack_open_and_which():
    rng = np.random.default_rng(5)
    L_, E_, H_, F_ = 3, 5, 512, 256
    types = (12, 12, 14)
    blob, (gsb, usb, dsb) = build_pack(L_, E_, H_, F_, types, rng)
    gate, up, down = pack_tensors(H_, F_, E_, types)
    pk = K.moe_pack_open(blob, L_, E_, H_, F_, gate, up, down)
    assert pk.stride == gsb + usb + dsb and pk.data_off == 4096
    for li in range(L_):
        for e in range(E_):
            for which in range(3):
                off = K.moe_pack_which(pk, li, e, which)
                assert off == O.moe_pack_offset(4096, E_, gsb, usb, dsb, li, e, which)
    # the last slice ends exactly at the end of the file
    assert K.moe_pack_which(pk, L_ - 1, E_ - 1, 2) + dsb == blob.size


@pytest.mark.parametrize("defect", ["magic", "version", "layers", "type", "slice", "data_off",
                                    "truncated"])
def test_pack_open_rejects_mismatch(defect):
    """Each header test of moe_pack_load (stratum_arch_moe.inc.c:506-525)
    refuses the pack with -1 and a message (never exit())."""
    rng = np.random.default_rng(6)
    L_, E_, H_, F_ = 2, 3, 512, 256
    types = (12, 12, 14)
    blob, _ = build_pack(L_, E_, H_, F_, types, rng)
    gate, up, down = pack_tensors(H_, F_, E_, types)
    if defect == "magic":
        blob[0] = ord("X")
    elif defect == "version":
        blob[4] = 2
    elif defect == "layers":
        blob[8] = L_ + 1
    elif defect == "type":
        blob[24] = 14             # gate_type
    elif defect == "slice":
        blob[36] ^= 1             # gate_slice low byte
    elif defect == "data_off":
        blob[60:68] = np.frombuffer(struct.pack("<Q", 40), np.uint8)
    elif defect == "truncated":
        blob = blob[:-1].copy()
    with pytest.raises(RuntimeError, match="MOE_PACK"):
        K.moe_pack_open(blob, L_, E_, H_, F_, gate, up, down)


def test_topk_matches_oracle(port):
    r = np.random.default_rng(9)
    cases = [r.standard_normal(128).astype(np.float32) for _ in range(50)]
    p = np.exp(cases[0] - cases[0].max())
    cases.append((p / p.sum()).astype(np.float32))
    cases.append(np.array([0.1, 0.3, 0.3, 0.2, 0.3, 0.05], np.float32))      # ties
    cases.append(np.full(8, 0.125, np.float32))                              # all equal
    cases.append(np.array([-2.0, -1.0, -0.5, np.nan, 0.0, -0.0], np.float32))  # <= -1, NaN, zeros
    cases.append(np.array([-3.0, -1.0], np.float32))                          # nothing eligible
    for w in cases:
        for k in (1, 2, 4, 8):
            got = K.moe_topk(w, k)
            want = port.topk(w, k)
            assert got[0] == want[0], (w, k)
            assert np.array_equal(got[1], want[1]), (w, k)
