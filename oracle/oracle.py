"""ctypes access to the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker or as the timed CPU baseline.

  port()  -> oracle/liboracle.so      the repo's C restatement (kq_oracle.c)
  ref()   -> oracle/_ref/libkqref.so  the reference's own scalar headers
             compiled from /root/reference (None when not built)
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libkqref.so")
NIBCONV_PATH = os.path.join(HERE, "_ref", "nib_convert")

_F = ctypes.POINTER(ctypes.c_float)
_U8 = ctypes.POINTER(ctypes.c_uint8)


def build(quiet: bool = True) -> None:
    """make -C oracle (the reference part only where /root/reference exists)."""
    out = subprocess.run(["make", "-C", HERE], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def _u8(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_U8)


def _f(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_F)


class MoeFfnDesc(ctypes.Structure):
    """ko_moe_ffn_desc (oracle/kq_oracle.h)"""
    _fields_ = [("n_embed", ctypes.c_int), ("n_ff", ctypes.c_int), ("n_experts", ctypes.c_int),
                ("k", ctypes.c_int), ("router_type", ctypes.c_int), ("router", ctypes.c_void_p),
                ("gate_type", ctypes.c_int), ("up_type", ctypes.c_int),
                ("down_type", ctypes.c_int), ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p),
                ("down", ctypes.c_void_p), ("gate_stride", ctypes.c_int64),
                ("up_stride", ctypes.c_int64), ("down_stride", ctypes.c_int64)]


class Port:
    """The restatement in oracle/kq_oracle.c."""

    def __init__(self, path: str = PORT_PATH):
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        I = ctypes.c_int
        L.ko_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.ko_fp16_to_fp32.restype = ctypes.c_float
        L.ko_q4k_scale_min.argtypes = [I, _U8, _U8, _U8]
        L.ko_q4k_scale_min_sweep.argtypes = [I, ctypes.POINTER(I), I, _U8, _U8]
        L.ko_q4k_scale_min_sweep.restype = None
        L.ko_q3k_scale_sweep.argtypes = [I, ctypes.POINTER(I), I, _U8, _U8]
        L.ko_q3k_scale_sweep.restype = None
        L.ko_dequant_row.argtypes = [I, _U8, I, _F]
        L.ko_dot_row.argtypes = [I, _U8, I, _F]
        L.ko_dot_row.restype = ctypes.c_float
        L.ko_dot_row_f64.argtypes = [I, _U8, I, _F]
        L.ko_dot_row_f64.restype = ctypes.c_double
        L.ko_gemv.argtypes = [I, _U8, _F, _F, _F, I, I, I]
        L.ko_gemv_multix.argtypes = [I, _U8, _F, _F, I, I, I, I]
        L.ko_q2k_to_nib.argtypes = [_U8, _U8, ctypes.c_int64]
        L.ko_nib_to_q2k.argtypes = [_U8, _U8, ctypes.c_int64]
        L.ko_moe_topk.argtypes = [_F, I, I, ctypes.POINTER(ctypes.c_int), _F]
        L.ko_quantize_x_q8.argtypes = [_F, I, I, ctypes.POINTER(ctypes.c_int8), _F]
        L.ko_quantize_x_q8.restype = None
        L.ko_gemv_i8.argtypes = [I, _U8, _F, _F, _F, ctypes.POINTER(ctypes.c_double), I, I, I]
        L.ko_gemv_i8_multix.argtypes = [I, _U8, _F, _F, I, I, I]
        L.ko_softmax.argtypes = [_F, I]
        L.ko_softmax.restype = None
        L.ko_swiglu.argtypes = [_F, _F, _F, ctypes.c_int64]
        L.ko_swiglu.restype = None
        _I = ctypes.POINTER(ctypes.c_int)
        L.ko_moe_combine.argtypes = [_F, _I, _F, _F, _F, I, I, I]
        L.ko_moe_combine.restype = None
        L.ko_moe_ffn.argtypes = [ctypes.POINTER(MoeFfnDesc), _F, _F, I, _I, _F, _F, _F, _F, _F,
                                 _F]
        self.L = L

    def fp16_to_fp32(self, h: int) -> float:
        return self.L.ko_fp16_to_fp32(h)

    def dequant(self, qtype: int, w: np.ndarray, nrows: int, K: int) -> np.ndarray:
        y = np.empty(nrows * K, np.float32)
        rb = w.size // nrows
        for r in range(nrows):
            self.L.ko_dequant_row(qtype, _u8(w[r * rb:(r + 1) * rb]), K,
                                  y[r * K:(r + 1) * K].ctypes.data_as(_F))
        return y

    def gemv(self, qtype: int, w: np.ndarray, x: np.ndarray, N: int, K: int,
             add: np.ndarray | None = None, threads: int = 1) -> np.ndarray:
        y = np.empty(N, np.float32)
        rc = self.L.ko_gemv(qtype, _u8(w), _f(x), _f(add) if add is not None else None,
                            _f(y), N, K, threads)
        assert rc == 0
        return y

    def gemv_rows(self, qtype: int, w: np.ndarray, x: np.ndarray, rows, K: int) -> np.ndarray:
        """Oracle result for a subset of rows (large tensors)."""
        rb = (K // 256) * BLOCK_BYTES[qtype]
        out = np.empty(len(rows), np.float32)
        for i, r in enumerate(rows):
            seg = w[r * rb:(r + 1) * rb]
            out[i] = self.L.ko_dot_row(qtype, _u8(seg), K, _f(x))
        return out

    def gemv_multix(self, qtype, w, xs, N, K, threads=1):
        B = xs.shape[0]
        ys = np.empty((B, N), np.float32)
        assert self.L.ko_gemv_multix(qtype, _u8(w), _f(np.ascontiguousarray(xs)), _f(ys),
                                     B, N, K, threads) == 0
        return ys

    def q2k_to_nib(self, q2k: np.ndarray) -> np.ndarray:
        n = q2k.size // 84
        out = np.empty(n * 148, np.uint8)
        self.L.ko_q2k_to_nib(_u8(q2k), _u8(out), n)
        return out

    def nib_to_q2k(self, nib: np.ndarray) -> np.ndarray:
        n = nib.size // 148
        out = np.empty(n * 84, np.uint8)
        self.L.ko_nib_to_q2k(_u8(nib), _u8(out), n)
        return out

    def quantize_q8(self, x: np.ndarray, G: int):
        """(xq int8 [K], xscale float32 [K/G])"""
        xq = np.empty(x.size, np.int8)
        xs = np.empty(x.size // G, np.float32)
        self.L.ko_quantize_x_q8(_f(x), x.size, G, xq.ctypes.data_as(ctypes.POINTER(ctypes.c_int8)),
                                _f(xs))
        return xq, xs

    def gemv_i8(self, qtype, w, x, N, K, add=None, sdot_f=False, with_mag=False):
        """int8-activation GEMV: the GPU's order, or (sdot_f) the reference's"""
        y = np.empty(N, np.float32)
        mag = np.empty(N, np.float64) if with_mag else None
        rc = self.L.ko_gemv_i8(qtype, _u8(w), _f(x), _f(add) if add is not None else None, _f(y),
                               mag.ctypes.data_as(ctypes.POINTER(ctypes.c_double))
                               if with_mag else None, N, K, int(sdot_f))
        assert rc == 0
        return (y, mag) if with_mag else y

    def gemv_i8_multix(self, qtype, w, xs, N, K):
        """int8 MULTISEQ (the reference's multix_pack arithmetic): ys [B, N]"""
        xs = np.ascontiguousarray(xs, np.float32)
        B = xs.shape[0]
        ys = np.empty((B, N), np.float32)
        rc = self.L.ko_gemv_i8_multix(qtype, _u8(w), _f(xs), _f(ys), B, N, K)
        assert rc == 0
        return ys

    def softmax(self, x: np.ndarray) -> np.ndarray:
        """softmax of each row of x (copied)"""
        out = np.array(x, np.float32, copy=True, order="C")
        rows = out.reshape(-1, out.shape[-1])
        for r in rows:
            self.L.ko_softmax(_f(r), r.size)
        return out

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        y = np.empty_like(g)
        self.L.ko_swiglu(_f(g), _f(u), _f(y), g.size)
        return y

    def moe_combine(self, o, sel, selw, resid, B, k, H):
        x = np.empty(B * H, np.float32)
        s = np.ascontiguousarray(sel, np.int32)
        self.L.ko_moe_combine(_f(o), s.ctypes.data_as(ctypes.POINTER(ctypes.c_int)), _f(selw),
                              _f(resid), _f(x), B, k, H)
        return x

    def moe_ffn(self, d: dict, xn: np.ndarray, x: np.ndarray, B: int) -> dict:
        """the whole expert FFN step; d holds n_embed, n_ff, n_experts, k,
        router_type / router, gate_type / gate, up_type / up, down_type /
        down (uint8 arrays of all experts' slices) and the strides"""
        H, F, E, k = d["n_embed"], d["n_ff"], d["n_experts"], d["k"]
        desc = MoeFfnDesc()
        keep = []
        for name in ("router", "gate", "up", "down"):
            a = np.ascontiguousarray(d[name], np.uint8)
            keep.append(a)
            setattr(desc, name, a.ctypes.data)
            setattr(desc, name + "_type", d[name + "_type"])
        desc.n_embed, desc.n_ff, desc.n_experts, desc.k = H, F, E, k
        desc.gate_stride, desc.up_stride, desc.down_stride = (
            d["gate_stride"], d["up_stride"], d["down_stride"])
        out = {"x": np.array(x, np.float32, copy=True),
               "sel": np.empty(B * k, np.int32), "selw": np.empty(B * k, np.float32),
               "probs": np.empty(B * E, np.float32), "g": np.empty(B * k * F, np.float32),
               "u": np.empty(B * k * F, np.float32), "act": np.empty(B * k * F, np.float32),
               "ffo": np.empty(B * k * H, np.float32)}
        rc = self.L.ko_moe_ffn(ctypes.byref(desc), _f(xn), _f(out["x"]), B,
                               out["sel"].ctypes.data_as(ctypes.POINTER(ctypes.c_int)),
                               _f(out["selw"]), _f(out["probs"]), _f(out["g"]), _f(out["u"]),
                               _f(out["act"]), _f(out["ffo"]))
        assert rc == 0
        return out

    def topk(self, w: np.ndarray, k: int):
        sel = (ctypes.c_int * k)()
        selw = np.empty(k, np.float32)
        self.L.ko_moe_topk(_f(w), w.size, k, sel, _f(selw))
        return list(sel), selw


def scale_min_sweep(fn, j: int, idx, bg: np.ndarray) -> np.ndarray:
    """(sc, m) of sub-block j for every value of the scale bytes idx (the
    rest fixed to bg), through fn = ko_q4k_scale_min_sweep or its reference
    twin: array [256^len(idx), 2]."""
    n = 1 << (8 * len(idx))
    out = np.empty(2 * n, np.uint8)
    ia = (ctypes.c_int * len(idx))(*idx)
    fn(j, ia, len(idx), _u8(np.ascontiguousarray(bg, np.uint8)), _u8(out))
    return out.reshape(n, 2)


def q3k_scale_sweep(fn, g: int, idx, bg: np.ndarray) -> np.ndarray:
    """The Q3_K scale of group g for every value of the scale bytes idx,
    through fn = ko_q3k_scale_sweep or its reference twin."""
    n = 1 << (8 * len(idx))
    out = np.empty(n, np.uint8)
    ia = (ctypes.c_int * len(idx))(*idx)
    fn(g, ia, len(idx), _u8(np.ascontiguousarray(bg, np.uint8)), _u8(out))
    return out


class Ref:
    """The reference's own scalar routines (oracle/_ref/libkqref.so)."""

    def __init__(self, path: str = REF_PATH):
        L = ctypes.CDLL(path)
        I = ctypes.c_int
        L.kqref_fp16_to_fp32.argtypes = [ctypes.c_uint16]
        L.kqref_fp16_to_fp32.restype = ctypes.c_float
        L.kqref_scale_min.argtypes = [I, _U8, _U8, _U8]
        L.kqref_scale_min_sweep.argtypes = [I, ctypes.POINTER(I), I, _U8, _U8]
        L.kqref_scale_min_sweep.restype = None
        L.kqref_q3k_scale_sweep.argtypes = [I, ctypes.POINTER(I), I, _U8, _U8]
        L.kqref_q3k_scale_sweep.restype = None
        L.kqref_dequant_row.argtypes = [I, _U8, I, _F]
        L.kqref_dot_row.argtypes = [I, _U8, I, _F]
        L.kqref_dot_row.restype = ctypes.c_float
        L.kqref_gemv.argtypes = [I, _U8, _F, _F, I, I, I, I]
        self.has_gguf = hasattr(L, "kqref_gguf_open")
        if self.has_gguf:
            P = ctypes.c_void_p
            L.kqref_gguf_open.argtypes = [ctypes.c_char_p, P, I, P, P, P, P, P, P, P]
        self.L = L

    def gguf_open(self, path: str, cap: int = 64):
        """gguf_open on the file: None if refused, else (n_tensors, n_kv,
        body_offset, alignment) and per-tensor dicts (the first cap)."""
        counts = np.zeros(4, np.uint64)
        types = np.zeros(cap, np.uint32)
        ndims = np.zeros(cap, np.uint32)
        dims = np.zeros(8 * cap, np.uint64)
        offs = np.zeros(cap, np.uint64)
        nelem = np.zeros(cap, np.int64)
        nbytes = np.zeros(cap, np.int64)
        names = np.zeros(64 * cap, np.uint8)
        rc = self.L.kqref_gguf_open(path.encode(), counts.ctypes.data, cap, types.ctypes.data,
                                    ndims.ctypes.data, dims.ctypes.data, offs.ctypes.data,
                                    nelem.ctypes.data, nbytes.ctypes.data, names.ctypes.data)
        if rc != 0:
            return None
        n = int(counts[0])
        ts = []
        for i in range(min(n, cap)):
            nm = bytes(names[64 * i:64 * i + 64]).split(b"\0")[0]
            ts.append({"name": nm, "type": int(types[i]), "n_dims": int(ndims[i]),
                       "dims": [int(v) for v in dims[8 * i:8 * i + int(ndims[i])]],
                       "offset": int(offs[i]), "nelem": int(nelem[i]),
                       "nbytes": int(nbytes[i])})
        return tuple(int(c) for c in counts), ts

    def dequant(self, qtype: int, w: np.ndarray, nrows: int, K: int) -> np.ndarray:
        y = np.empty(nrows * K, np.float32)
        rb = w.size // nrows
        for r in range(nrows):
            assert self.L.kqref_dequant_row(qtype, _u8(w[r * rb:(r + 1) * rb]), K,
                                            y[r * K:(r + 1) * K].ctypes.data_as(_F)) == 0
        return y

    def gemv(self, qtype: int, w: np.ndarray, x: np.ndarray, N: int, K: int,
             threads: int = 1) -> np.ndarray:
        y = np.empty(N, np.float32)
        assert self.L.kqref_gemv(qtype, _u8(w), _f(x), _f(y), 1, N, K, threads) == 0
        return y

    def gemv_multix(self, qtype, w, xs, N, K, threads=1):
        B = xs.shape[0]
        ys = np.empty((B, N), np.float32)
        assert self.L.kqref_gemv(qtype, _u8(w), _f(np.ascontiguousarray(xs)), _f(ys),
                                 B, N, K, threads) == 0
        return ys


_port = None
_ref = None


def port() -> Port:
    global _port
    if _port is None:
        _port = Port()
    return _port


def ref() -> Ref | None:
    """The reference build, or None where /root/reference was not available."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        _ref = Ref()
    return _ref


# ------------------------------------------------------------ MoE addressing
# Integer restatements of the expert-slice and pack addressing (pure
# arithmetic, so plain Python).

# bytes per 256 weights (stratum_gguf.h:57-79)
BLOCK_BYTES = {0: 1024, 1: 512, 8: 272, 10: 84, 11: 110, 12: 144, 13: 176, 14: 210, 42: 148}


def moe_slice_bytes(qtype: int, nelem: int, nbytes: int, K_in: int, N_out: int) -> int:
    """stratum_arch_moe.inc.c:220-238."""
    if qtype == 43:
        return N_out * K_in * 2 + N_out * (K_in // 256) * 8 + N_out * (K_in // 32) * 2
    if qtype == 44:
        return N_out * K_in * 2 + N_out * (K_in // 256) * 8
    one = K_in * N_out
    if nbytes <= 0 or nelem <= 0:
        return one // 256 * BLOCK_BYTES[qtype]      # gguf_tensor_bytes of one slice
    e_all = max(1, nelem // one)
    return nbytes // e_all


def moe_pack_offset(data_off: int, n_experts: int, gate: int, up: int, down: int,
                    li: int, e: int, which: int) -> int:
    """moe_pack_which, stratum_arch_moe.inc.c:307-313 (stride = gate+up+down)."""
    off = data_off + (li * n_experts + e) * (gate + up + down)
    if which == 1:
        off += gate
    elif which == 2:
        off += gate + up
    return off


def moe_tickets(sel, n_experts: int, ch: int = 8):
    """The expert tickets of moe_forward_b (stratum_arch_moe.inc.c:1136-1140,
    1158-1178): member m = s * k + r with sel[m] >= 0 joins expert sel[m]'s
    list (tokens s in order, ranks r in order, i.e. increasing m), and each
    list is cut from its start into tickets of at most CH = 8 members, each
    one st_linear_multix call (stratum_arch_moe.inc.c:1194-1201).  Returns
    [(e, [m, ...]), ...] in increasing expert order."""
    lists = [[] for _ in range(n_experts)]
    for m, e in enumerate(int(v) for v in sel):
        if 0 <= e < n_experts:
            lists[e].append(m)
    return [(e, lst[j:j + ch]) for e, lst in enumerate(lists) for j in range(0, len(lst), ch)]


# ------------------------------------------------------------ tolerances
def rel_err(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Per-element |a-b| / max(|b|, 1e-6): ASSERT_REL of quant_test.c:34-43."""
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return np.abs(a - b) / np.maximum(np.abs(b), 1e-6)
