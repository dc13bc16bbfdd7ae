"""MI355X-native k-quant GEMV: the stratum quantized-matvec hot path on gfx950.

The product is the C-ABI library ``libkqgemv.so`` built from
``stratum_amd/csrc`` (HIP kernels for gfx950 + a C host layer).  Its
declarations live in ``include/kq_gemv.h``.  This module only loads the
library with ctypes and gives Python callers (tests, bench.py) thin
wrappers with the reference's argument meaning:

  linear_dispatch(w, x, N, K)        st_linear_dispatch   (stratum_linear.h:526)
  linear_dispatch_add(w, x, add, ..) st_linear_dispatch_add (stratum_linear.h:568)
  linear_multix(w, xs, N, K)         st_linear_multix     (stratum_linear.h:715)
  q4k_group(x, K, (w, N), ...)       st_q4k_group         (stratum_linear.h:1086)

There is no CPU fallback: if the library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

TYPE_Q2_K = 10
TYPE_Q4_K = 12
TYPE_Q6_K = 14
TYPE_Q2K_NIB = 42

BLOCK_BYTES = {TYPE_Q2_K: 84, TYPE_Q4_K: 144, TYPE_Q6_K: 210, TYPE_Q2K_NIB: 148}
TYPE_NAMES = {TYPE_Q2_K: "Q2_K", TYPE_Q4_K: "Q4_K", TYPE_Q6_K: "Q6_K", TYPE_Q2K_NIB: "Q2K_NIB"}

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkqgemv.so")

# Every symbol include/kq_gemv.h declares (checked by tests/test_abi.py).
EXPORTS = (
    "kq_linear_init", "kq_register_region", "kq_device_ptr", "kq_linear_shutdown",
    "kq_last_error", "kq_linear_dispatch", "kq_linear_dispatch_add", "kq_linear_multix",
    "kq_q4k_group", "kq_gemv_dev", "kq_gemv_multix_dev", "kq_gemv_segments_dev",
    "kq_dequant_dev", "kq_row_bytes",
)

MAX_SEGMENTS = 8
MAX_GROUPS = 16


class KqSegment(ctypes.Structure):
    """kq_segment (include/kq_gemv.h): one segment of a batched launch."""

    _fields_ = [
        ("type", ctypes.c_int),
        ("K", ctypes.c_int),
        ("rows_per_group", ctypes.c_int),
        ("ngroups", ctypes.c_int),
        ("w", ctypes.c_void_p * MAX_GROUPS),
        ("x", ctypes.c_void_p),
        ("x_stride", ctypes.c_int),
        ("add", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
    ]


def segment(qtype: int, K: int, rows_per_group: int, w_ptrs, x_ptr: int, y_ptr: int,
            x_stride: int = 0, add_ptr: int | None = None) -> KqSegment:
    s = KqSegment()
    s.type = qtype
    s.K = K
    s.rows_per_group = rows_per_group
    s.ngroups = len(w_ptrs)
    for i, p in enumerate(w_ptrs):
        s.w[i] = p
    s.x = x_ptr
    s.x_stride = x_stride
    s.add = add_ptr
    s.y = y_ptr
    return s


class KqTensor(ctypes.Structure):
    """kq_tensor == GgufTensor layout (stratum_gguf.h:129-137)."""

    _fields_ = [
        ("name", ctypes.c_char_p),
        ("n_dims", ctypes.c_uint32),
        ("dims", ctypes.c_uint64 * 8),
        ("type", ctypes.c_uint32),
        ("offset", ctypes.c_uint64),
        ("nelem", ctypes.c_int64),
        ("nbytes", ctypes.c_int64),
    ]


def make_tensor(qtype: int, N: int, K: int, offset: int, name: bytes = b"w") -> KqTensor:
    """Descriptor of an N x K tensor at byte `offset` of the registered base.

    GGUF stores dims[0] = K (row length) and dims[1] = N (q6k_test.c:27-28).
    """
    t = KqTensor()
    t.name = name
    t.n_dims = 2
    t.dims[0] = K
    t.dims[1] = N
    t.type = qtype
    t.offset = offset
    t.nelem = N * K
    t.nbytes = N * (K // 256) * BLOCK_BYTES[qtype]
    return t


_LIB = None


def lib() -> ctypes.CDLL:
    """Load libkqgemv.so (raises if it was not built: no silent fallback)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is missing: run __graft_entry__.build() "
                          "(make -C stratum_amd/csrc)")
    L = ctypes.CDLL(LIB_PATH)
    P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_float)
    TP = ctypes.POINTER(KqTensor)
    FPP = ctypes.POINTER(F)
    L.kq_linear_init.argtypes = [P, ctypes.c_size_t]
    L.kq_register_region.argtypes = [P, ctypes.c_size_t]
    L.kq_device_ptr.argtypes = [P, ctypes.c_size_t]
    L.kq_device_ptr.restype = P
    L.kq_linear_shutdown.argtypes = []
    L.kq_linear_shutdown.restype = None
    L.kq_last_error.restype = ctypes.c_char_p
    L.kq_linear_dispatch.argtypes = [TP, F, F, I, I]
    L.kq_linear_dispatch_add.argtypes = [TP, F, F, F, I, I]
    L.kq_linear_multix.argtypes = [TP, FPP, FPP, I, I, I]
    L.kq_q4k_group.argtypes = [F, I, TP, F, I, TP, F, I, TP, F, I]
    L.kq_gemv_dev.argtypes = [I, P, P, P, P, I, I, P]
    L.kq_gemv_multix_dev.argtypes = [I, P, P, P, I, I, I, P]
    L.kq_dequant_dev.argtypes = [I, P, P, ctypes.c_int64, P]
    L.kq_gemv_segments_dev.argtypes = [ctypes.POINTER(KqSegment), I, P]
    L.kq_row_bytes.argtypes = [I, I]
    L.kq_row_bytes.restype = ctypes.c_int64
    _LIB = L
    return L


def _fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {lib().kq_last_error().decode()}")


class WeightRegion:
    """Host weight bytes registered with kq_linear_init (uploaded to HBM).

    Mirrors stratum_linear_init(mmap_base, mmap_size): tensor offsets are
    bytes from the start of `blob`.
    """

    def __init__(self, blob: np.ndarray):
        assert blob.dtype == np.uint8 and blob.flags["C_CONTIGUOUS"]
        self.blob = blob  # keep the host mapping alive
        _check(lib().kq_linear_init(blob.ctypes.data, blob.nbytes), "kq_linear_init")


def linear_dispatch(w: KqTensor, x: np.ndarray, N: int, K: int) -> np.ndarray:
    y = np.empty(N, np.float32)
    _check(lib().kq_linear_dispatch(ctypes.byref(w), _fptr(x), _fptr(y), N, K),
           "kq_linear_dispatch")
    return y


def linear_dispatch_add(w: KqTensor, x: np.ndarray, add: np.ndarray | None,
                        N: int, K: int) -> np.ndarray:
    y = np.empty(N, np.float32)
    addp = _fptr(add) if add is not None else None
    _check(lib().kq_linear_dispatch_add(ctypes.byref(w), _fptr(x), addp, _fptr(y), N, K),
           "kq_linear_dispatch_add")
    return y


def linear_multix(w: KqTensor, xs: list[np.ndarray], N: int, K: int) -> list[np.ndarray]:
    B = len(xs)
    ys = [np.empty(N, np.float32) for _ in range(B)]
    FP = ctypes.POINTER(ctypes.c_float)
    xa = (FP * B)(*[_fptr(x) for x in xs])
    ya = (FP * B)(*[_fptr(y) for y in ys])
    _check(lib().kq_linear_multix(ctypes.byref(w), xa, ya, B, N, K), "kq_linear_multix")
    return ys


def q4k_group(x: np.ndarray, K: int, *members: tuple[KqTensor, int]) -> list[np.ndarray]:
    assert len(members) in (2, 3)
    outs = [np.empty(N, np.float32) for _, N in members]
    args = []
    for i in range(3):
        if i < len(members):
            args += [ctypes.byref(members[i][0]), _fptr(outs[i]), members[i][1]]
        else:
            args += [None, None, 0]
    _check(lib().kq_q4k_group(_fptr(x), K, *args), "kq_q4k_group")
    return outs


def gemv_dev(qtype: int, w_ptr: int, x_ptr: int, y_ptr: int, N: int, K: int,
             add_ptr: int | None = None, stream: int | None = None) -> None:
    """Device-pointer GEMV (raw addresses, e.g. torch tensor .data_ptr())."""
    _check(lib().kq_gemv_dev(qtype, w_ptr, x_ptr, add_ptr, y_ptr, N, K, stream),
           "kq_gemv_dev")


def gemv_multix_dev(qtype: int, w_ptr: int, xs_ptr: int, ys_ptr: int, B: int, N: int,
                    K: int, stream: int | None = None) -> None:
    _check(lib().kq_gemv_multix_dev(qtype, w_ptr, xs_ptr, ys_ptr, B, N, K, stream),
           "kq_gemv_multix_dev")


def gemv_segments_dev(segs: list[KqSegment], stream: int | None = None) -> None:
    """One launch over up to 8 segments (kq_gemv_segments_dev)."""
    arr = (KqSegment * len(segs))(*segs)
    _check(lib().kq_gemv_segments_dev(arr, len(segs), stream), "kq_gemv_segments_dev")


def dequant_dev(qtype: int, w_ptr: int, y_ptr: int, nblocks: int,
                stream: int | None = None) -> None:
    _check(lib().kq_dequant_dev(qtype, w_ptr, y_ptr, nblocks, stream), "kq_dequant_dev")
