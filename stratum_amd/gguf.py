"""GGUF v3 index, type-42 conversion and MoE pack check (include/kq_gguf.h).

The index is kq_gguf_open over a caller-owned buffer (a numpy uint8 array
or an mmap): tensor descriptors are kq_tensor with offsets from the start
of that buffer, ready for kq_linear_init(buffer) and kq_linear_dispatch.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import KqMoePack, KqTensor, _check, lib


class KqGgufKv(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("vtype", ctypes.c_uint32),
                ("bytes", ctypes.c_void_p), ("bytes_len", ctypes.c_size_t)]


class KqGguf(ctypes.Structure):
    _fields_ = [("base", ctypes.c_void_p), ("size", ctypes.c_size_t),
                ("version", ctypes.c_uint32), ("n_tensors", ctypes.c_uint64),
                ("n_kv", ctypes.c_uint64), ("kv", ctypes.POINTER(KqGgufKv)),
                ("tensors", ctypes.POINTER(KqTensor)), ("body_offset", ctypes.c_uint64),
                ("alignment", ctypes.c_uint64)]


def _bind(L):
    if getattr(L, "_gguf_bound", False):
        return L
    P = ctypes.c_void_p
    G = ctypes.POINTER(KqGguf)
    L.kq_gguf_open.argtypes = [P, ctypes.c_size_t, G]
    L.kq_gguf_close.argtypes = [G]
    L.kq_gguf_close.restype = None
    L.kq_gguf_find_tensor.argtypes = [G, ctypes.c_char_p]
    L.kq_gguf_find_tensor.restype = ctypes.POINTER(KqTensor)
    L.kq_gguf_find_kv.argtypes = [G, ctypes.c_char_p]
    L.kq_gguf_find_kv.restype = ctypes.POINTER(KqGgufKv)
    L.kq_gguf_get_u32.argtypes = [G, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint32)]
    L.kq_gguf_get_u64.argtypes = [G, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint64)]
    L.kq_gguf_get_f32.argtypes = [G, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float)]
    L.kq_gguf_get_string_dup.argtypes = [G, ctypes.c_char_p]
    L.kq_gguf_get_string_dup.restype = ctypes.c_void_p
    L.kq_gguf_type_size.argtypes = [ctypes.c_uint32, ctypes.POINTER(ctypes.c_int)]
    L.kq_gguf_nib_convert.argtypes = [G, P, ctypes.POINTER(ctypes.c_uint64)]
    L.kq_gguf_nib_convert.restype = ctypes.c_int64
    L.kq_q2k_to_nib_dev.argtypes = [P, P, ctypes.c_int64, P]
    TP = ctypes.POINTER(KqTensor)
    L.kq_moe_pack_check.argtypes = [ctypes.POINTER(KqMoePack), P, ctypes.c_int,
                                    ctypes.POINTER(TP), ctypes.POINTER(TP), ctypes.POINTER(TP),
                                    ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L._gguf_bound = True
    return L


def glib():
    return _bind(lib())


class Index:
    """An open index over `buf` (kept alive with it)."""

    def __init__(self, buf: np.ndarray):
        assert buf.dtype == np.uint8 and buf.flags["C_CONTIGUOUS"]
        self.buf = buf
        self.g = KqGguf()
        _check(glib().kq_gguf_open(buf.ctypes.data, buf.nbytes, ctypes.byref(self.g)),
               "kq_gguf_open")

    def close(self) -> None:
        if self.g.base:
            glib().kq_gguf_close(ctypes.byref(self.g))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # The descriptors kq_gguf_open builds live in C memory that
    # kq_gguf_close frees (names included).  tensors() and find() return
    # copies that hold a reference to this Index, so the C memory their
    # name pointers use stays alive as long as any of them does; close()
    # must not be called while they are still in use.
    def _own(self, t: KqTensor) -> KqTensor:
        c = KqTensor.from_buffer_copy(t)
        c._index = self
        return c

    def tensors(self) -> list[KqTensor]:
        return [self._own(self.g.tensors[i]) for i in range(self.g.n_tensors)]

    def find(self, name: str) -> KqTensor | None:
        p = glib().kq_gguf_find_tensor(ctypes.byref(self.g), name.encode())
        return self._own(p.contents) if p else None

    def u32(self, key: str) -> int | None:
        v = ctypes.c_uint32()
        return v.value if glib().kq_gguf_get_u32(ctypes.byref(self.g), key.encode(),
                                                 ctypes.byref(v)) == 0 else None

    def u64(self, key: str) -> int | None:
        v = ctypes.c_uint64()
        return v.value if glib().kq_gguf_get_u64(ctypes.byref(self.g), key.encode(),
                                                 ctypes.byref(v)) == 0 else None

    def f32(self, key: str) -> float | None:
        v = ctypes.c_float()
        return v.value if glib().kq_gguf_get_f32(ctypes.byref(self.g), key.encode(),
                                                 ctypes.byref(v)) == 0 else None

    def string(self, key: str) -> str | None:
        p = glib().kq_gguf_get_string_dup(ctypes.byref(self.g), key.encode())
        if not p:
            return None
        s = ctypes.string_at(p).decode()
        ctypes.CDLL(None).free(ctypes.c_void_p(p))
        return s

    def nib_convert(self) -> tuple[np.ndarray, int]:
        """(converted file bytes, number of Q2_K tensors converted)"""
        n = ctypes.c_uint64()
        L = glib()
        if L.kq_gguf_nib_convert(ctypes.byref(self.g), None, ctypes.byref(n)) < 0:
            raise RuntimeError(L.kq_last_error().decode(errors="replace"))
        out = np.zeros(n.value, np.uint8)
        c = L.kq_gguf_nib_convert(ctypes.byref(self.g), out.ctypes.data, ctypes.byref(n))
        if c < 0:
            raise RuntimeError(L.kq_last_error().decode(errors="replace"))
        return out, c


def type_size(t: int) -> tuple[int, int]:
    """(bytes per block, elements per block); (0, 0) for an unknown id"""
    e = ctypes.c_int()
    b = glib().kq_gguf_type_size(t, ctypes.byref(e))
    return b, e.value


def q2k_to_nib_dev(q2k_ptr: int, nib_ptr: int, nblocks: int, stream: int | None = None) -> None:
    _check(glib().kq_q2k_to_nib_dev(q2k_ptr, nib_ptr, nblocks, stream), "kq_q2k_to_nib_dev")


def moe_pack_check(pk, model: np.ndarray, gate, up, down, n_embed: int, n_ff: int,
                   full: bool = False) -> int:
    """kq_moe_pack_check; gate / up / down are per-layer KqTensor lists.
    Returns the experts checked, or -1 when a slice differs."""
    TP = ctypes.POINTER(KqTensor)
    arrs = [(TP * len(ts))(*[ctypes.pointer(t) for t in ts]) for ts in (gate, up, down)]
    return glib().kq_moe_pack_check(ctypes.byref(pk), model.ctypes.data, len(gate), arrs[0],
                                    arrs[1], arrs[2], n_embed, n_ff, int(full))
