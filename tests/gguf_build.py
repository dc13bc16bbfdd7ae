"""GGUF v3 byte builders for the tests (test infrastructure).

`model()` lays out a well-formed file; `bounds_case()` and `guards_case()`
restate the hostile files of the reference's gguf_bounds_test.c:44-93 and
input_guards_test.c:38-63 (one tensor, or a header claiming n_tensors with
at most four infos written); `mutations()` derives corrupted variants of a
file by byte flips, truncations and field overwrites.
"""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)


def s_str(s: bytes) -> bytes:
    return struct.pack("<Q", len(s)) + s


def kv_u32(key: str, v: int) -> bytes:
    return s_str(key.encode()) + struct.pack("<II", U32, v)


def kv_u64(key: str, v: int) -> bytes:
    return s_str(key.encode()) + struct.pack("<IQ", U64, v)


def kv_f32(key: str, v: float) -> bytes:
    return s_str(key.encode()) + struct.pack("<If", F32, v)


def kv_str(key: str, v: str) -> bytes:
    return s_str(key.encode()) + struct.pack("<I", STRING) + s_str(v.encode())


def kv_array_u32(key: str, vals) -> bytes:
    return (s_str(key.encode()) + struct.pack("<IIQ", ARRAY, U32, len(vals)) +
            b"".join(struct.pack("<I", v) for v in vals))


def kv_array_str(key: str, vals) -> bytes:
    return (s_str(key.encode()) + struct.pack("<IIQ", ARRAY, STRING, len(vals)) +
            b"".join(s_str(v.encode()) for v in vals))


def tensor_info(name: str, dims, ttype: int, offset: int) -> bytes:
    return (s_str(name.encode()) + struct.pack("<I", len(dims)) +
            b"".join(struct.pack("<Q", d) for d in dims) + struct.pack("<IQ", ttype, offset))


def header(n_tensors: int, n_kv: int) -> bytes:
    return b"GGUF" + struct.pack("<IQQ", 3, n_tensors, n_kv)


def pad(b: bytes, align: int) -> bytes:
    return b + b"\0" * ((-len(b)) % align)


def model(tensors, kvs=(), align: int = 32) -> np.ndarray:
    """tensors: (name, dims, type, data bytes); data laid out aligned"""
    kv = list(kvs)
    if align != 32:
        kv = [kv_u32("general.alignment", align)] + kv
    infos, body, off = [], b"", 0
    for name, dims, ttype, data in tensors:
        off = (off + align - 1) // align * align
        body = body + b"\0" * (off - len(body))
        infos.append(tensor_info(name, dims, ttype, off))
        body += data
        off += len(data)
    idx = header(len(tensors), len(kv)) + b"".join(kv) + b"".join(infos)
    return np.frombuffer(pad(idx, align) + body, np.uint8).copy()


def bounds_case(dims, ttype: int, offset_field: int, data: bytes, nest_depth: int = -1) -> bytes:
    """make_file of gguf_bounds_test.c: general.alignment 32, optionally a
    `test.nested` array nest_depth arrays deep around an empty UINT8 array,
    one tensor "w", the data after 32-byte padding"""
    kv = kv_u32("general.alignment", 32)
    n_kv = 1
    if nest_depth >= 0:
        kv += s_str(b"test.nested") + struct.pack("<I", ARRAY)
        kv += struct.pack("<IQ", ARRAY, 1) * nest_depth + struct.pack("<IQ", U8, 0)
        n_kv = 2
    idx = header(1, n_kv) + kv + tensor_info("w", dims, ttype, offset_field)
    return pad(idx, 32) + data


def guards_case(n_tensors: int, n_kv: int, ttype: int, offset: int, body: int) -> bytes:
    """write_case of input_guards_test.c: one KV, min(n_tensors, 4) infos of a
    4 x 4 tensor, padding, `body` zero bytes"""
    infos = tensor_info("token_embd.weight", [4, 4], ttype, offset) * min(n_tensors, 4)
    idx = header(n_tensors, n_kv) + kv_u32("general.alignment", 32) + infos
    return pad(idx, 32) + b"\0" * body


def mutations(base: np.ndarray, n: int, seed: int):
    """n corrupted variants of base: byte flips, truncations, u64 fields
    overwritten with hostile values"""
    r = np.random.default_rng(seed)
    hostile = [0, 1, 2 ** 31, 2 ** 32 - 1, 2 ** 63 - 1, 2 ** 63, 2 ** 64 - 1, 2 ** 40, 255]
    out = []
    for i in range(n):
        b = base.copy()
        kind = i % 4
        if kind == 0:                      # flip a few header-region bytes
            for _ in range(int(r.integers(1, 4))):
                p = int(r.integers(0, min(len(b), 400)))
                b[p] ^= np.uint8(1 << int(r.integers(0, 8)))
        elif kind == 1:                    # truncate
            b = b[:int(r.integers(0, len(b)))].copy()
        elif kind == 2:                    # a hostile u64 at a random 8-byte slot
            p = int(r.integers(0, min(len(b), 400) - 8))
            v = hostile[int(r.integers(len(hostile)))]
            b[p:p + 8] = np.frombuffer(struct.pack("<Q", v), np.uint8)
        else:                              # a hostile u32
            p = int(r.integers(0, min(len(b), 400) - 4))
            v = hostile[int(r.integers(len(hostile)))] & 0xFFFFFFFF
            b[p:p + 4] = np.frombuffer(struct.pack("<I", v), np.uint8)
        out.append(b)
    return out
