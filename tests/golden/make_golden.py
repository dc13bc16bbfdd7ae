"""Write the golden fixtures for the k-quant GEMV path.

Run once in a container that has /root/reference (the outputs are
committed; the GPU box never runs this):

    make -C oracle && python tests/golden/make_golden.py

Expected values come ONLY from the reference's own code, compiled from its
sources where they lie by oracle/Makefile:
  * oracle/_ref/libkqref.so -- q{4,6,2,5,3}k_dequant_block_scalar,
    q{4,6,2,5,3}k_dot_row_scalar and q8_0_dequant_block_scalar /
    q8_0_dot_row_scalar (stratum_q4k.h, stratum_q6k.h, stratum_q2k.h,
    stratum_q5k.h, stratum_q3k.h, stratum_q8_0.h);
  * oracle/_ref/nib_convert -- tools_gguf_nib_convert.c, run on a small GGUF
    v3 file written here, for the type-42 bytes;
  * gguf_open (stratum_gguf.h:226-444, through ref_harness.c) on the GGUF
    corpus of gguf.npz: its verdict and index for every file.
Inputs are seeded numpy draws plus hand-built edge blocks.  Nothing from
the repo's own oracle (oracle/kq_oracle.c) is used, so the fixtures pin it.

Each fixture file <type>.npz holds, per case c:
  c_w (uint8 blocks), c_x (float32 [K]), c_shape ([N, K]),
  c_deq (float32 [N*K]), c_y (float32 [N]);
and for type 42 also c_src, the Q2_K bytes given to the converter.
gguf.npz holds the corpus files back to back (blob, lens), the reference's
accept flag, (n_tensors, n_kv, body_offset, alignment) and the first 8
tensors' type / offset / nelem / nbytes per file, and a small model before
(nib_in) and after (nib_out) the reference's type-42 converter.
"""
from __future__ import annotations

import hashlib
import os
import struct
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.abspath(os.path.join(HERE, "..", ".."))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402

Q2, Q4, Q6, NIB = 10, 12, 14, 42
Q5, Q3, Q80 = 13, 11, 8
BB = {Q2: 84, Q4: 144, Q6: 210, NIB: 148, Q5: 176, Q3: 110, Q80: 272}   # per 256 weights
# byte offsets of the fp16 d (and dmin) fields in a 256-weight unit
D_AT = {Q4: [0], Q5: [0], Q6: [208], Q2: [80], Q3: [108], Q80: [34 * q for q in range(8)]}
DMIN_AT = {Q4: 2, Q5: 2, Q2: 82}


def f16(v) -> np.ndarray:
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def rand_blocks(t: int, r: np.random.Generator, n: int) -> np.ndarray:
    """Field distributions of the benchmark configs (uniform bytes,
    fp16(|N(0,1)|*0.01) scales), drawn with numpy directly."""
    b = r.integers(0, 256, (n, BB[t]), dtype=np.uint8)
    if t == Q4:
        b[:, 0:2] = f16(np.abs(r.standard_normal(n)) * 0.01).view(np.uint8).reshape(n, 2)
        b[:, 2:4] = f16(np.abs(r.standard_normal(n)) * 0.01).view(np.uint8).reshape(n, 2)
    elif t == Q6:
        b[:, 208:210] = f16(np.abs(r.standard_normal(n)) * 0.01).view(np.uint8).reshape(n, 2)
    elif t == Q2:
        b[:, 80:82] = f16(np.abs(r.standard_normal(n)) * 0.01).view(np.uint8).reshape(n, 2)
        b[:, 82:84] = f16(np.abs(r.standard_normal(n)) * 0.01).view(np.uint8).reshape(n, 2)
    elif t in (Q5, Q3, Q80):
        for o in D_AT[t] + ([DMIN_AT[t]] if t in DMIN_AT else []):
            b[:, o:o + 2] = f16(np.abs(r.standard_normal(n)) * 0.01).view(np.uint8).reshape(n, 2)
    return b


# fp16 bit patterns exercised in the edge rows: 1.0, smallest and largest
# subnormal, largest normal, -0, -1, +inf, NaN, a negative normal, 0
EDGE_D = [0x3C00, 0x0001, 0x03FF, 0x7BFF, 0x8000, 0xBC00, 0x7C00, 0x7E00, 0xA8F5, 0x0000]


def edge_blocks(t: int, r: np.random.Generator) -> np.ndarray:
    n = len(EDGE_D)
    b = rand_blocks(t, r, n)
    for i, dv in enumerate(EDGE_D):
        mv = EDGE_D[(i + 3) % n]
        if t == Q4:
            b[i, 0:2] = np.frombuffer(struct.pack("<H", dv), np.uint8)
            b[i, 2:4] = np.frombuffer(struct.pack("<H", mv), np.uint8)
        elif t == Q6:
            b[i, 208:210] = np.frombuffer(struct.pack("<H", dv), np.uint8)
        elif t in (Q5, Q3, Q80):
            pass                 # set with the payloads below
        else:
            b[i, 80:82] = np.frombuffer(struct.pack("<H", dv), np.uint8)
            b[i, 82:84] = np.frombuffer(struct.pack("<H", mv), np.uint8)
    # extreme payloads: all-ones and all-zero quant/scale bytes
    if t == Q4:
        b[0, 4:] = 0xFF          # scales/mins 63, nibbles 15
        b[9, 4:] = 0x00
    elif t == Q6:
        b[0, 0:208] = 0xFF       # q = 63, scales -1
        b[1, 192:208] = 0x80     # scales -128
        b[2, 192:208] = 0x7F     # scales 127
        b[9, 0:208] = 0x00       # q = 0 -> -32, scales 0
    elif t in (Q5, Q3, Q80):
        for i, dv in enumerate(EDGE_D):
            for o in D_AT[t]:
                b[i, o:o + 2] = np.frombuffer(struct.pack("<H", dv), np.uint8)
            if t in DMIN_AT:
                b[i, DMIN_AT[t]:DMIN_AT[t] + 2] = np.frombuffer(
                    struct.pack("<H", EDGE_D[(i + 3) % n]), np.uint8)
        payload = [k for k in range(BB[t])
                   if all(not (o <= k < o + 2) for o in D_AT[t]) and
                   not (t in DMIN_AT and DMIN_AT[t] <= k < DMIN_AT[t] + 2)]
        b[0, payload] = 0xFF     # Q5_K: q 31, scales 63; Q3_K: q 3, scale 31; Q8_0: -1
        b[1, payload] = 0x80 if t == Q80 else 0x55
        b[9, payload] = 0x00     # Q3_K: q -4, scale -32
    else:
        b[0, 0:80] = 0xFF
        b[9, 0:80] = 0x00
    return b


def write_gguf(path: str, q2k: np.ndarray, N: int, K: int) -> int:
    """Minimal GGUF v3 with one Q2_K tensor; returns the data offset."""
    name = b"blk.0.ffn_gate.weight"
    hdr = b"GGUF" + struct.pack("<IQQ", 3, 1, 0)
    info = struct.pack("<Q", len(name)) + name + struct.pack("<IQQIQ", 2, K, N, Q2, 0)
    body = len(hdr) + len(info)
    body = (body + 31) & ~31
    with open(path, "wb") as f:
        f.write(hdr + info)
        f.write(b"\0" * (body - len(hdr) - len(info)))
        f.write(q2k.tobytes())
    return body


def reference_nib(q2k: np.ndarray, N: int, K: int) -> np.ndarray:
    """Run the reference converter (tools_gguf_nib_convert.c) on q2k."""
    with tempfile.TemporaryDirectory() as td:
        src, dst = os.path.join(td, "in.gguf"), os.path.join(td, "out.gguf")
        body = write_gguf(src, q2k, N, K)
        subprocess.run([O.NIBCONV_PATH, src, dst], check=True, capture_output=True)
        data = np.fromfile(dst, np.uint8)
    nbytes = N * (K // 256) * 148
    assert data.size == body + nbytes, (data.size, body, nbytes)
    # the converter rewrote the type field to 42
    return data[body:body + nbytes].copy()


def make_cases(t: int, ref: O.Ref):
    r = np.random.Generator(np.random.PCG64(0x5EED + t))
    tt = Q2 if t == NIB else t
    cases = {}
    # (name, N, K, block source, x source)
    specs = [
        ("edge", len(EDGE_D), 256, "edge", "special"),
        ("rand", 16, 1024, "rand", "normal"),
        ("wide", 4, 5120, "rand", "normal"),
        ("subx", 4, 256, "rand", "subnormal"),
    ]
    for name, N, K, bsrc, xsrc in specs:
        nb = N * K // 256
        w = edge_blocks(tt, r) if bsrc == "edge" else rand_blocks(tt, r, nb)
        w = np.ascontiguousarray(w.reshape(-1))
        x = r.standard_normal(K).astype(np.float32)
        if xsrc == "special":
            x[0], x[1], x[2], x[3], x[5] = 0.0, -0.0, 1e30, -1e-30, 3.0e7
        elif xsrc == "subnormal":
            x[::3] = np.float32(1e-40) * (1 + np.arange(x[::3].size, dtype=np.float32))
            x[1::3] *= np.float32(1e-38)
        deq = ref.dequant(tt, w, N, K)
        y = ref.gemv(tt, w, x, N, K)
        extra = {}
        if t == NIB:
            extra["src"] = w           # the Q2_K bytes the converter was given
            w = reference_nib(w, N, K)
        cases[name] = dict(w=w, x=x, shape=np.array([N, K], np.int64), deq=deq, y=y, **extra)
    return cases


def gguf_corpus():
    """The GGUF files of the parser fixture: the hostile cases of
    gguf_bounds_test.c and input_guards_test.c, a well-formed model and
    seeded corruptions of it."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_build as G
    six = b"\xab" * 16
    files = [
        G.bounds_case([4], 0, 0, six), G.bounds_case([1 << 62, 8], 0, 0, b""),
        G.bounds_case([(2 ** 63 - 1) // 4 + 1], 0, 0, b""), G.bounds_case([100], 12, 0, b""),
        G.bounds_case([2 ** 64 - 1], 0, 0, b""), G.bounds_case([4], 99, 0, b""),
        G.bounds_case([4], 0, 0, six, nest_depth=2), G.bounds_case([4], 0, 0, six, nest_depth=64),
        G.bounds_case([4], 0, 0, b""),
        G.guards_case(1, 1, 0, 0, 512), G.guards_case(1, 1, 0, 2 ** 64 - 9, 512),
        G.guards_case(1, 1, 100, 1 << 40, 512), G.guards_case(1, 1, 100, 0, 512),
        G.guards_case(1, 1, 100, 512, 512), G.guards_case(1 << 40, 1, 0, 0, 512),
        G.guards_case(1, 1 << 40, 0, 0, 512),
    ]
    r = np.random.Generator(np.random.PCG64(0x66))
    base = gguf_model(r)
    files.append(base.tobytes())
    files += [m.tobytes() for m in G.mutations(base, 400, 0x67)]
    return files


def gguf_model(r):
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import gguf_build as G
    ts = [("blk.0.attn_q.weight", [512, 4], Q4, rand_blocks(Q4, r, 8).tobytes()),
          ("blk.0.ffn_down.weight", [256, 2], Q6, rand_blocks(Q6, r, 2).tobytes()),
          ("blk.0.ffn_gate.weight", [256, 3], Q2, rand_blocks(Q2, r, 3).tobytes()),
          ("output_norm.weight", [40], 0, r.standard_normal(40).astype(np.float32).tobytes()),
          ("blk.0.ffn_up.weight", [256, 2], Q2, rand_blocks(Q2, r, 2).tobytes()),
          ("token_embd.weight", [16, 2], 1, r.standard_normal(32).astype(np.float16).tobytes())]
    kvs = [G.kv_str("general.architecture", "llama"), G.kv_u32("llama.block_count", 1),
           G.kv_u64("llama.context_length", 4096), G.kv_f32("llama.rope.freq_base", 1e6),
           G.kv_array_u32("tokenizer.ggml.token_type", [1, 2, 3]),
           G.kv_array_str("tokenizer.ggml.tokens", ["a", "bc", ""])]
    return G.model(ts, kvs, align=64)


def make_gguf_fixture(ref: O.Ref):
    """gguf.npz: every corpus file with the reference gguf_open's verdict and
    index (up to 8 tensors), and a model converted by the reference tool."""
    files = gguf_corpus()
    cap = 8
    n = len(files)
    accept = np.zeros(n, np.int8)
    counts = np.zeros((n, 4), np.uint64)
    types = np.zeros((n, cap), np.uint32)
    offs = np.zeros((n, cap), np.uint64)
    nelem = np.zeros((n, cap), np.int64)
    nbytes = np.zeros((n, cap), np.int64)
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "f.gguf")
        for i, fb in enumerate(files):
            with open(path, "wb") as f:
                f.write(fb)
            got = ref.gguf_open(path, cap)
            if got is None:
                continue
            accept[i] = 1
            counts[i] = got[0]
            for j, t in enumerate(got[1]):
                types[i, j], offs[i, j], nelem[i, j], nbytes[i, j] = (
                    t["type"], t["offset"], t["nelem"], t["nbytes"])
        r = np.random.Generator(np.random.PCG64(0x68))
        model = gguf_model(r)
        src, dst = os.path.join(td, "in.gguf"), os.path.join(td, "out.gguf")
        model.tofile(src)
        subprocess.run([O.NIBCONV_PATH, src, dst], check=True, capture_output=True)
        conv = np.fromfile(dst, np.uint8)
    lens = np.array([len(f) for f in files], np.int64)
    blob = np.frombuffer(b"".join(files), np.uint8)
    return dict(blob=blob, lens=lens, accept=accept, counts=counts, types=types, offsets=offs,
                nelem=nelem, nbytes=nbytes, nib_in=model, nib_out=conv)


def main() -> None:
    O.build()
    ref = O.ref()
    if ref is None or not os.path.exists(O.NIBCONV_PATH):
        sys.exit("oracle/_ref is not built: /root/reference is required to write fixtures")
    manifest = []
    for t, fname in [(Q4, "q4k"), (Q6, "q6k"), (Q2, "q2k"), (NIB, "q2k_nib"), (Q5, "q5k"),
                     (Q3, "q3k"), (Q80, "q8_0")]:
        cases = make_cases(t, ref)
        arrays = {f"{c}_{k}": v for c, d in cases.items() for k, v in d.items()}
        path = os.path.join(HERE, f"{fname}.npz")
        np.savez_compressed(path, **arrays)
        h = hashlib.sha256(open(path, "rb").read()).hexdigest()
        manifest.append(f"{fname}.npz {h} {os.path.getsize(path)}")
    path = os.path.join(HERE, "gguf.npz")
    np.savez_compressed(path, **make_gguf_fixture(ref))
    h = hashlib.sha256(open(path, "rb").read()).hexdigest()
    manifest.append(f"gguf.npz {h} {os.path.getsize(path)}")
    with open(os.path.join(HERE, "MANIFEST"), "w") as f:
        f.write("# sha256 and size of each fixture written by make_golden.py\n")
        f.write("\n".join(manifest) + "\n")
    print("\n".join(manifest))


if __name__ == "__main__":
    main()
