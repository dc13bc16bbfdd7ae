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
    v3 file written here, for the type-42 bytes.
Inputs are seeded numpy draws plus hand-built edge blocks.  Nothing from
the repo's own oracle (oracle/kq_oracle.c) is used, so the fixtures pin it.

Each fixture file <type>.npz holds, per case c:
  c_w (uint8 blocks), c_x (float32 [K]), c_shape ([N, K]),
  c_deq (float32 [N*K]), c_y (float32 [N]);
and for type 42 also c_src, the Q2_K bytes given to the converter.
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
    with open(os.path.join(HERE, "MANIFEST"), "w") as f:
        f.write("# sha256 and size of each fixture written by make_golden.py\n")
        f.write("\n".join(manifest) + "\n")
    print("\n".join(manifest))


if __name__ == "__main__":
    main()
