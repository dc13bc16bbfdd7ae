"""GGUF v3 index (kq_gguf_open), the type-42 file conversion and the MoE
pack byte check: host code, no GPU.

The parser is pinned against the reference's own gguf_open
(stratum_gguf.h:226-444, built into oracle/_ref through ref_harness.c):
  * tests/golden/gguf.npz holds 417 files -- the hostile cases of
    gguf_bounds_test.c and input_guards_test.c, a well-formed model and
    400 seeded corruptions of it -- with the reference's verdict and index
    per file; kq_gguf_open must give the same verdict and the same tensor
    types, offsets, element counts and byte sizes;
  * with oracle/_ref built, 2000 fresh corruptions are compared live.
The converter is pinned against the reference tool's output
(tools_gguf_nib_convert.c, oracle/_ref/nib_convert): byte-identical files,
from the fixture and live; the converted tensors dequantize to the same
values.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import gguf_build as G
import stratum_amd as K
from conftest import GOLDEN
from oracle import oracle as O
from stratum_amd import gguf as KG
from stratum_amd import synth

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
TOOL = os.path.join(ROOT, "stratum_amd", "kq_nib_convert")


def ours(buf: np.ndarray):
    """(counts, tensors) from kq_gguf_open, or None when it refuses"""
    try:
        ix = KG.Index(np.ascontiguousarray(buf, np.uint8))
    except RuntimeError:
        return None
    g = ix.g
    ts = [{"name": t.name, "type": t.type, "n_dims": t.n_dims,
           "dims": [t.dims[d] for d in range(t.n_dims)], "offset": t.offset,
           "nelem": t.nelem, "nbytes": t.nbytes} for t in ix.tensors()]
    out = (g.n_tensors, g.n_kv, g.body_offset, g.alignment), ts
    ix.close()
    return out


def load_corpus():
    z = np.load(os.path.join(GOLDEN, "gguf.npz"), allow_pickle=False)
    ends = np.cumsum(z["lens"])
    starts = ends - z["lens"]
    files = [z["blob"][s:e] for s, e in zip(starts, ends)]
    return z, files


# ---------------------------------------------------------------- parser
def test_corpus_matches_reference_verdicts_and_index():
    z, files = load_corpus()
    assert len(files) == 417
    n_acc = 0
    for i, f in enumerate(files):
        got = ours(f)
        assert (got is not None) == bool(z["accept"][i]), i
        if got is None:
            continue
        n_acc += 1
        assert tuple(got[0]) == tuple(int(v) for v in z["counts"][i]), i
        for j, t in enumerate(got[1][:8]):
            assert (t["type"], t["offset"], t["nelem"], t["nbytes"]) == (
                int(z["types"][i, j]), int(z["offsets"][i, j]), int(z["nelem"][i, j]),
                int(z["nbytes"][i, j])), (i, j)
    assert n_acc == int(z["accept"].sum())


def test_reference_test_cases():
    """the cases and expectations of gguf_bounds_test.c and input_guards_test.c"""
    six = b"\xab" * 16
    a = lambda b: ours(np.frombuffer(b, np.uint8))  # noqa: E731
    ok = a(G.bounds_case([4], 0, 0, six))
    assert ok and ok[1][0]["nelem"] == 4 and ok[1][0]["nbytes"] == 16
    assert a(G.bounds_case([1 << 62, 8], 0, 0, b"")) is None
    assert a(G.bounds_case([(2 ** 63 - 1) // 4 + 1], 0, 0, b"")) is None
    assert a(G.bounds_case([100], 12, 0, b"")) is None
    assert a(G.bounds_case([2 ** 64 - 1], 0, 0, b"")) is None
    unk = a(G.bounds_case([4], 99, 0, b""))
    assert unk and unk[1][0]["nbytes"] == -1
    assert a(G.bounds_case([4], 0, 0, six, nest_depth=2)) is not None
    assert a(G.bounds_case([4], 0, 0, six, nest_depth=64)) is None
    assert a(G.bounds_case([4], 0, 0, b"")) is None
    assert a(G.guards_case(1, 1, 0, 0, 512)) is not None
    assert a(G.guards_case(1, 1, 0, 2 ** 64 - 9, 512)) is None
    assert a(G.guards_case(1, 1, 100, 1 << 40, 512)) is None
    assert a(G.guards_case(1, 1, 100, 0, 512)) is not None
    assert a(G.guards_case(1, 1, 100, 512, 512)) is not None      # one past the end
    assert a(G.guards_case(1 << 40, 1, 0, 0, 512)) is None
    assert a(G.guards_case(1, 1 << 40, 0, 0, 512)) is None
    assert a(b"") is None and a(b"GGUF") is None and a(b"GGUF\x02\0\0\0" + b"\0" * 16) is None


def test_live_corruptions_match_reference(ref, tmp_path):
    if not ref.has_gguf:
        pytest.skip("oracle/_ref predates the gguf harness")
    r = synth.rng(77)
    base = G.model([("a", [512, 2], 12, synth.q4k_blocks(r, 4).tobytes()),
                    ("b", [256], 10, synth.q2k_blocks(r, 1).tobytes()),
                    ("c", [8], 0, bytes(32))],
                   [G.kv_str("general.name", "m"), G.kv_array_u32("x", [1, 2])], align=32)
    path = str(tmp_path / "f.gguf")
    for i, m in enumerate([base] + G.mutations(base, 2000, 78)):
        m.tofile(path)
        want = ref.gguf_open(path)
        got = ours(m)
        assert (got is None) == (want is None), i
        if got is not None:
            assert tuple(got[0]) == want[0], i
            for t, u in zip(got[1], want[1]):
                assert t["name"] == u["name"] and t["dims"] == u["dims"], i
                for k in ("type", "n_dims", "offset", "nelem", "nbytes"):
                    assert t[k] == u[k], (i, k)


def test_model_index_and_metadata():
    r = synth.rng(80)
    w4 = synth.q4k_blocks(r, 6).tobytes()
    ts = [("blk.0.attn_q.weight", [768, 2], 12, w4),
          ("norm", [40], 0, np.arange(40, dtype=np.float32).tobytes())]
    kvs = [G.kv_str("general.architecture", "qwen3"), G.kv_u32("qwen3.block_count", 28),
           G.kv_u64("qwen3.context_length", 1 << 40), G.kv_f32("qwen3.rope.freq_base", 1e6),
           G.kv_array_str("tok", ["a", "b"])]
    buf = G.model(ts, kvs, align=128)
    ix = KG.Index(buf)
    assert ix.g.alignment == 128 and ix.g.n_tensors == 2 and ix.g.n_kv == 6
    q = ix.find("blk.0.attn_q.weight")
    assert q is not None and q.type == 12 and q.nelem == 1536 and q.nbytes == 6 * 144
    assert q.offset % 128 == 0 and bytes(buf[q.offset:q.offset + q.nbytes]) == w4
    assert ix.find("missing") is None
    assert ix.string("general.architecture") == "qwen3"
    assert ix.u32("qwen3.block_count") == 28 and ix.u64("qwen3.block_count") == 28
    assert ix.u64("qwen3.context_length") == 1 << 40
    assert ix.u32("qwen3.context_length") == 0            # truncated as gguf_get_u32 does
    assert ix.f32("qwen3.rope.freq_base") == np.float32(1e6)
    assert ix.f32("qwen3.block_count") is None and ix.string("qwen3.block_count") is None
    assert ix.u32("general.alignment") == 128
    n = ix.find("norm")
    assert np.array_equal(np.frombuffer(bytes(buf[n.offset:n.offset + 160]), np.float32),
                          np.arange(40, dtype=np.float32))
    ix.close()


def test_descriptors_outlive_the_index_object():
    """tensors() and find() return copies that keep their Index (and the C
    memory their names point into) alive: dropping the Index object first
    leaves them valid."""
    import gc
    r = synth.rng(81)
    ts = [("blk.0.attn_q.weight", [768, 2], 12, synth.q4k_blocks(r, 6).tobytes()),
          ("norm", [40], 0, np.arange(40, dtype=np.float32).tobytes())]
    buf = G.model(ts, [G.kv_str("general.architecture", "qwen3")])
    got = KG.Index(buf).tensors()
    q = KG.Index(buf).find("blk.0.attn_q.weight")
    gc.collect()
    junk = [KG.Index(buf) for _ in range(4)]       # reuse freed memory, if any
    assert [t.name for t in got] == [b"blk.0.attn_q.weight", b"norm"]
    assert got[0].type == 12 and got[1].nelem == 40
    assert q.name == b"blk.0.attn_q.weight" and q.nbytes == 6 * 144
    del junk


def test_type_table():
    for t, (b, e) in {0: (4, 1), 1: (2, 1), 8: (34, 32), 10: (84, 256), 11: (110, 256),
                      12: (144, 256), 13: (176, 256), 14: (210, 256), 42: (148, 256),
                      30: (2, 1), 23: (136, 256)}.items():
        assert KG.type_size(t) == (b, e), t
    for t in (4, 5, 16, 31, 41, 45, 99, 2 ** 32 - 1):
        assert KG.type_size(t) == (0, 0), t


# ------------------------------------------------------------ converter
def test_nib_convert_matches_reference_fixture():
    z, _ = load_corpus()
    ix = KG.Index(np.ascontiguousarray(z["nib_in"]))
    out, n = ix.nib_convert()
    assert n == 2
    assert np.array_equal(out, z["nib_out"])


def test_nib_convert_values(port):
    """converted tensors: type 42, same values as the Q2_K source"""
    z, _ = load_corpus()
    src = np.ascontiguousarray(z["nib_in"])
    a, b = KG.Index(src), KG.Index(np.ascontiguousarray(z["nib_out"]))
    for t, u in zip(a.tensors(), b.tensors()):
        assert t.name == u.name and t.nelem == u.nelem
        if t.type == 10:
            assert u.type == 42 and u.nbytes == t.nelem // 256 * 148
            K_ = t.dims[0]
            N_ = t.nelem // K_
            d0 = port.dequant(10, src[t.offset:t.offset + t.nbytes], N_, K_)
            d1 = port.dequant(42, z["nib_out"][u.offset:u.offset + u.nbytes], N_, K_)
            assert np.array_equal(d0, d1)
        else:
            assert u.type == t.type
            assert np.array_equal(src[t.offset:t.offset + t.nbytes],
                                  z["nib_out"][u.offset:u.offset + u.nbytes])


def test_nib_convert_tool_matches_reference_tool(tmp_path):
    if not os.path.exists(O.NIBCONV_PATH):
        pytest.skip("oracle/_ref/nib_convert not built")
    if not os.path.exists(TOOL):
        pytest.skip("kq_nib_convert not built")
    r = synth.rng(90)
    buf = G.model([("x.weight", [256, 5], 10, synth.q2k_blocks(r, 5).tobytes()),
                   ("y.weight", [512, 1], 12, synth.q4k_blocks(r, 2).tobytes()),
                   ("z.weight", [256, 7], 10, synth.q2k_blocks(r, 7).tobytes())],
                  [G.kv_str("general.architecture", "llama")])
    src = tmp_path / "in.gguf"
    buf.tofile(src)
    subprocess.run([O.NIBCONV_PATH, str(src), str(tmp_path / "ref.gguf")], check=True,
                   capture_output=True)
    subprocess.run([TOOL, str(src), str(tmp_path / "ours.gguf")], check=True, capture_output=True)
    want = np.fromfile(tmp_path / "ref.gguf", np.uint8)
    assert np.array_equal(np.fromfile(tmp_path / "ours.gguf", np.uint8), want)
    out, n = KG.Index(buf).nib_convert()
    assert n == 2 and np.array_equal(out, want)


def test_nib_convert_refuses_unknown_size():
    buf = np.frombuffer(G.guards_case(1, 1, 100, 0, 512), np.uint8).copy()
    ix = KG.Index(buf)
    with pytest.raises(RuntimeError):
        ix.nib_convert()


# ------------------------------------------------------ MoE pack check
def make_pack(n_layers, E, H, F, seed):
    """stacked Q4_K expert tensors in one model blob and the .moep pack of
    them (header, then per layer and expert: gate | up | down)"""
    r = synth.rng(seed)
    sl_gu = F * (H // 256) * 144
    sl_d = H * (F // 256) * 144
    model = []
    descs = {"gate": [], "up": [], "down": []}
    off = 0
    for li in range(n_layers):
        for name, n_out, k_in in (("gate", F, H), ("up", F, H), ("down", H, F)):
            w = synth.tensor(12, E * n_out, k_in, seed + 10 * li + len(model))
            t = K.make_tensor(12, E * n_out, k_in, off, name=f"{li}.{name}".encode())
            t.dims[0], t.dims[1], t.dims[2], t.n_dims = k_in, n_out, E, 3
            t.nelem = E * n_out * k_in
            t.nbytes = w.size
            descs[name].append(t)
            model.append(w)
            off += w.size
    blob = np.concatenate(model)
    data_off = 4096
    hdr = K.KqMoePackHdr()
    hdr.magic = b"MOEP"
    hdr.version, hdr.n_layers, hdr.n_experts, hdr.n_embed, hdr.n_ff = 1, n_layers, E, H, F
    hdr.gate_type = hdr.up_type = hdr.down_type = 12
    hdr.gate_slice, hdr.up_slice, hdr.down_slice, hdr.data_off = sl_gu, sl_gu, sl_d, data_off
    stride = 2 * sl_gu + sl_d
    pack = np.zeros(data_off + n_layers * E * stride, np.uint8)
    pack[:ctypes.sizeof(hdr)] = np.frombuffer(bytes(hdr), np.uint8)
    for li in range(n_layers):
        for e in range(E):
            p = data_off + (li * E + e) * stride
            for name, sl in (("gate", sl_gu), ("up", sl_gu), ("down", sl_d)):
                t = descs[name][li]
                pack[p:p + sl] = blob[t.offset + e * sl:t.offset + (e + 1) * sl]
                p += sl
    return blob, pack, descs


def test_moe_pack_check_sampled_and_full():
    H, F, E, L = 512, 256, 6, 2
    blob, pack, d = make_pack(L, E, H, F, 9100)
    pk = K.moe_pack_open(pack, L, E, H, F, d["gate"][0], d["up"][0], d["down"][0])
    assert KG.moe_pack_check(pk, blob, d["gate"], d["up"], d["down"], H, F) == 2 * 3
    assert KG.moe_pack_check(pk, blob, d["gate"], d["up"], d["down"], H, F, full=True) == 2 * E
    # a byte changed in expert 1 (not sampled): the sampled check passes, the full one fails
    sl_gu = F * (H // 256) * 144
    stride = 2 * sl_gu + H * (F // 256) * 144
    bad = pack.copy()
    bad[4096 + 1 * stride + 17] ^= 1
    pk2 = K.moe_pack_open(bad, L, E, H, F, d["gate"][0], d["up"][0], d["down"][0])
    assert KG.moe_pack_check(pk2, blob, d["gate"], d["up"], d["down"], H, F) == 6
    assert KG.moe_pack_check(pk2, blob, d["gate"], d["up"], d["down"], H, F, full=True) == -1
    # a byte changed in layer 1, expert E/2, down: both fail
    bad = pack.copy()
    bad[4096 + (1 * E + E // 2) * stride + 2 * sl_gu + 5] ^= 0x80
    pk3 = K.moe_pack_open(bad, L, E, H, F, d["gate"][0], d["up"][0], d["down"][0])
    assert KG.moe_pack_check(pk3, blob, d["gate"], d["up"], d["down"], H, F) == -1
