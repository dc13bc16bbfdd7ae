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
  moe_slice_bytes / moe_bind_slice   (stratum_arch_moe.inc.c:220-238, 327-337)
  moe_pack_open / moe_pack_which     (stratum_arch_moe.inc.c:245-313, 506-525)
  moe_topk, moe_topk_dev             moe_topk (stratum_arch_moe.inc.c:368-385)
  moe_gemv_dev(op, sel, B, k, E)     the routed expert GEMVs (:596-603, 808-815, 1135-1205)

There is no CPU fallback: if the library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

TYPE_F32 = 0
TYPE_F16 = 1
TYPE_Q8_0 = 8
TYPE_Q2_K = 10
TYPE_Q3_K = 11
TYPE_Q4_K = 12
TYPE_Q5_K = 13
TYPE_Q6_K = 14
TYPE_Q2K_NIB = 42
# int8-activation mode flag (KQ_INT8_ACT): TYPE_Q4_K | INT8_ACT, and likewise for
# Q6_K, Q5_K, Q3_K and Q8_0
INT8_ACT = 0x100

# bytes per 256 weights (stratum_gguf.h:57-79; Q8_0: eight 34-byte blocks)
BLOCK_BYTES = {TYPE_F32: 1024, TYPE_F16: 512, TYPE_Q8_0: 272, TYPE_Q2_K: 84, TYPE_Q3_K: 110,
               TYPE_Q4_K: 144, TYPE_Q5_K: 176, TYPE_Q6_K: 210, TYPE_Q2K_NIB: 148}
TYPE_NAMES = {TYPE_F32: "F32", TYPE_F16: "F16", TYPE_Q8_0: "Q8_0", TYPE_Q2_K: "Q2_K",
              TYPE_Q3_K: "Q3_K", TYPE_Q4_K: "Q4_K", TYPE_Q5_K: "Q5_K", TYPE_Q6_K: "Q6_K",
              TYPE_Q2K_NIB: "Q2K_NIB"}

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libkqgemv.so")

# Every symbol include/kq_gemv.h declares (checked by tests/test_abi.py).
EXPORTS = (
    "kq_linear_init", "kq_register_region", "kq_device_ptr", "kq_linear_shutdown",
    "kq_last_error", "kq_linear_dispatch", "kq_linear_dispatch_add", "kq_linear_multix",
    "kq_q4k_group", "kq_gemv_dev", "kq_gemv_multix_dev", "kq_gemv_segments_dev",
    "kq_dequant_dev", "kq_row_bytes", "kq_moe_slice_bytes", "kq_moe_bind_slice",
    "kq_moe_pack_open", "kq_moe_pack_which", "kq_moe_topk", "kq_moe_topk_dev",
    "kq_moe_gemv_dev", "kq_gemv_multix_mfma_dev", "kq_moe_gemv_routed_dev",
    "kq_tuning_reload", "kq_gemv_multix_mfma_noalloc_dev", "kq_linear_set_sdot",
    "kq_quantize_x_q8_dev", "kq_softmax_dev", "kq_swiglu_dev", "kq_moe_combine_dev",
    "kq_moe_ffn_workspace_bytes", "kq_moe_ffn_dev", "kq_gemv_multix_mfma_workspace_bytes",
    "kq_reserve_mfma_workspace", "kq_scratch_bytes", "kq_moe_ffn_last_path",
)
# include/kq_gguf.h (bound in stratum_amd/gguf.py)
GGUF_EXPORTS = (
    "kq_gguf_open", "kq_gguf_close", "kq_gguf_find_tensor", "kq_gguf_find_kv",
    "kq_gguf_get_u32", "kq_gguf_get_u64", "kq_gguf_get_f32", "kq_gguf_get_string_dup",
    "kq_gguf_type_size", "kq_gguf_nib_convert", "kq_q2k_to_nib_dev", "kq_moe_pack_check",
)

NOALLOC_SCRATCH_BYTES = 32 << 20   # KQ_NOALLOC_SCRATCH_BYTES

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


class KqMoePackHdr(ctypes.Structure):
    """kq_moe_pack_hdr == MoePackHdr (stratum_arch_moe.inc.c:245-259), packed."""

    _pack_ = 1
    _fields_ = [("magic", ctypes.c_char * 4)] + [
        (n, ctypes.c_uint32) for n in ("version", "n_layers", "n_experts", "n_embed", "n_ff",
                                       "gate_type", "up_type", "down_type")] + [
        (n, ctypes.c_uint64) for n in ("gate_slice", "up_slice", "down_slice", "data_off")]


class KqMoePack(ctypes.Structure):
    """kq_moe_pack: a validated pack mapping."""

    _fields_ = [("base", ctypes.c_void_p), ("size", ctypes.c_size_t)] + [
        (n, ctypes.c_uint64) for n in ("data_off", "gate_slice", "up_slice", "down_slice",
                                       "stride")] + [
        ("n_layers", ctypes.c_uint32), ("n_experts", ctypes.c_uint32)]


class KqMoeOp(ctypes.Structure):
    """kq_moe_op: one routed expert GEMV (gate+up, or down) of a layer."""

    _fields_ = [
        ("type", ctypes.c_int), ("n_out", ctypes.c_int), ("k_in", ctypes.c_int),
        ("ntensors", ctypes.c_int),
        ("w", ctypes.c_void_p * 2),
        ("expert_stride", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("x_div", ctypes.c_int),
        ("y", ctypes.c_void_p * 2),
    ]


class KqMoeFfn(ctypes.Structure):
    """kq_moe_ffn: one MoE layer's router and stacked expert tensors."""

    _fields_ = [
        ("n_embed", ctypes.c_int), ("n_ff", ctypes.c_int), ("n_experts", ctypes.c_int),
        ("k", ctypes.c_int), ("router_type", ctypes.c_int), ("router", ctypes.c_void_p),
        ("gate_type", ctypes.c_int), ("up_type", ctypes.c_int), ("down_type", ctypes.c_int),
        ("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p),
        ("gate_stride", ctypes.c_int64), ("up_stride", ctypes.c_int64),
        ("down_stride", ctypes.c_int64),
    ]


def moe_op(qtype: int, n_out: int, k_in: int, w_ptrs, expert_stride: int, x_ptr: int,
           x_div: int, y_ptrs) -> KqMoeOp:
    op = KqMoeOp()
    op.type, op.n_out, op.k_in, op.ntensors = qtype, n_out, k_in, len(w_ptrs)
    for i, p in enumerate(w_ptrs):
        op.w[i] = p
    for i, p in enumerate(y_ptrs):
        op.y[i] = p
    op.expert_stride = expert_stride
    op.x = x_ptr
    op.x_div = x_div
    return op


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
    L.kq_tuning_reload.argtypes = []
    L.kq_linear_dispatch.argtypes = [TP, F, F, I, I]
    L.kq_linear_dispatch_add.argtypes = [TP, F, F, F, I, I]
    L.kq_linear_multix.argtypes = [TP, FPP, FPP, I, I, I]
    L.kq_q4k_group.argtypes = [F, I, TP, F, I, TP, F, I, TP, F, I]
    L.kq_gemv_dev.argtypes = [I, P, P, P, P, I, I, P]
    L.kq_gemv_multix_dev.argtypes = [I, P, P, P, I, I, I, P]
    L.kq_gemv_multix_mfma_dev.argtypes = [I, P, P, P, I, I, I, P]
    L.kq_gemv_multix_mfma_noalloc_dev.argtypes = [I, P, P, P, I, I, I, P]
    L.kq_gemv_multix_mfma_workspace_bytes.argtypes = [I, I, I, I]
    L.kq_gemv_multix_mfma_workspace_bytes.restype = ctypes.c_int64
    L.kq_reserve_mfma_workspace.argtypes = [ctypes.c_int64]
    L.kq_scratch_bytes.argtypes = []
    L.kq_scratch_bytes.restype = ctypes.c_int64
    L.kq_dequant_dev.argtypes = [I, P, P, ctypes.c_int64, P]
    L.kq_linear_set_sdot.argtypes = [I]
    L.kq_softmax_dev.argtypes = [P, I, I, P]
    L.kq_swiglu_dev.argtypes = [P, P, P, ctypes.c_int64, P]
    L.kq_moe_combine_dev.argtypes = [P, P, P, P, P, I, I, I, P]
    L.kq_moe_ffn_workspace_bytes.argtypes = [ctypes.POINTER(KqMoeFfn), I]
    L.kq_moe_ffn_workspace_bytes.restype = ctypes.c_int64
    L.kq_moe_ffn_dev.argtypes = [ctypes.POINTER(KqMoeFfn), P, P, I, P, P, P, ctypes.c_int64, P]
    L.kq_moe_ffn_last_path.argtypes = []
    L.kq_quantize_x_q8_dev.argtypes = [P, I, I, P, P, P, P]
    L.kq_gemv_segments_dev.argtypes = [ctypes.POINTER(KqSegment), I, P]
    L.kq_row_bytes.argtypes = [I, I]
    L.kq_row_bytes.restype = ctypes.c_int64
    L.kq_moe_slice_bytes.argtypes = [TP, I, I]
    L.kq_moe_slice_bytes.restype = ctypes.c_int64
    L.kq_moe_bind_slice.argtypes = [TP, TP, I, ctypes.c_int64, I, I, P, P]
    L.kq_moe_bind_slice.restype = None
    L.kq_moe_pack_open.argtypes = [P, ctypes.c_size_t, I, I, I, I, TP, TP, TP,
                                   ctypes.POINTER(KqMoePack)]
    L.kq_moe_pack_which.argtypes = [ctypes.POINTER(KqMoePack), I, I, I]
    L.kq_moe_pack_which.restype = P
    L.kq_moe_topk.argtypes = [F, I, I, ctypes.POINTER(ctypes.c_int), F]
    L.kq_moe_topk.restype = None
    L.kq_moe_topk_dev.argtypes = [P, I, I, I, P, P, P]
    L.kq_moe_gemv_dev.argtypes = [ctypes.POINTER(KqMoeOp), P, I, I, I, P]
    L.kq_moe_gemv_routed_dev.argtypes = [ctypes.POINTER(KqMoeOp), P, I, I, I, P, P, P]
    _LIB = L
    return L


def reload_tuning() -> None:
    """Re-read the KQ_* launch-shape overrides (kq_tuning_reload)."""
    lib().kq_tuning_reload()


def _fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().kq_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed: {msg}")


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


def quantize_x_q8_dev(x_ptr: int, K: int, group: int, xq_ptr: int, xscale_ptr: int,
                      xsum_ptr: int | None = None, stream: int | None = None) -> None:
    """int8 quantizer of the int8-activation mode (kq_quantize_x_q8_dev)."""
    _check(lib().kq_quantize_x_q8_dev(x_ptr, K, group, xq_ptr, xscale_ptr, xsum_ptr, stream),
           "kq_quantize_x_q8_dev")


def set_sdot(on: bool) -> bool:
    """use_sdot for the host-pointer entry points; returns the previous setting."""
    return bool(lib().kq_linear_set_sdot(int(on)))


def gemv_multix_dev(qtype: int, w_ptr: int, xs_ptr: int, ys_ptr: int, B: int, N: int,
                    K: int, stream: int | None = None) -> None:
    _check(lib().kq_gemv_multix_dev(qtype, w_ptr, xs_ptr, ys_ptr, B, N, K, stream),
           "kq_gemv_multix_dev")


def gemv_multix_mfma_dev(qtype: int, w_ptr: int, xs_ptr: int, ys_ptr: int, B: int, N: int,
                         K: int, stream: int | None = None) -> None:
    """Matrix-core multi-stream GEMV (tolerance path, Q4_K / Q6_K)."""
    _check(lib().kq_gemv_multix_mfma_dev(qtype, w_ptr, xs_ptr, ys_ptr, B, N, K, stream),
           "kq_gemv_multix_mfma_dev")


def gemv_segments_dev(segs: list[KqSegment], stream: int | None = None) -> None:
    """One launch over up to 8 segments (kq_gemv_segments_dev)."""
    arr = (KqSegment * len(segs))(*segs)
    _check(lib().kq_gemv_segments_dev(arr, len(segs), stream), "kq_gemv_segments_dev")


def dequant_dev(qtype: int, w_ptr: int, y_ptr: int, nblocks: int,
                stream: int | None = None) -> None:
    _check(lib().kq_dequant_dev(qtype, w_ptr, y_ptr, nblocks, stream), "kq_dequant_dev")


def moe_slice_bytes(t: KqTensor, K_in: int, N_out: int) -> int:
    return lib().kq_moe_slice_bytes(ctypes.byref(t), K_in, N_out)


def moe_bind_slice(t: KqTensor, e: int, slice_bytes: int, N_out: int, K_in: int,
                   slice_host: int | None = None, base: int | None = None) -> KqTensor:
    d = KqTensor()
    lib().kq_moe_bind_slice(ctypes.byref(d), ctypes.byref(t), e, slice_bytes, N_out, K_in,
                            slice_host, base)
    return d


def moe_pack_open(blob: np.ndarray, n_layers: int, n_experts: int, n_embed: int, n_ff: int,
                  gate: KqTensor, up: KqTensor, down: KqTensor) -> KqMoePack:
    pk = KqMoePack()
    _check(lib().kq_moe_pack_open(blob.ctypes.data, blob.nbytes, n_layers, n_experts, n_embed,
                                  n_ff, ctypes.byref(gate), ctypes.byref(up), ctypes.byref(down),
                                  ctypes.byref(pk)), "kq_moe_pack_open")
    return pk


def moe_pack_which(pk: KqMoePack, li: int, e: int, which: int) -> int:
    """Byte offset from the pack base of (layer li, expert e, tensor which)."""
    return lib().kq_moe_pack_which(ctypes.byref(pk), li, e, which) - pk.base


def moe_topk(w: np.ndarray, k: int) -> tuple[list[int], np.ndarray]:
    sel = (ctypes.c_int * k)()
    selw = np.empty(k, np.float32)
    lib().kq_moe_topk(_fptr(w), len(w), k, sel, _fptr(selw))
    return list(sel), selw


def moe_topk_dev(probs_ptr: int, B: int, E: int, k: int, sel_ptr: int, selw_ptr: int,
                 stream: int | None = None) -> None:
    _check(lib().kq_moe_topk_dev(probs_ptr, B, E, k, sel_ptr, selw_ptr, stream),
           "kq_moe_topk_dev")


def moe_gemv_dev(op: KqMoeOp, sel_ptr: int, B: int, k: int, E: int,
                 stream: int | None = None) -> None:
    _check(lib().kq_moe_gemv_dev(ctypes.byref(op), sel_ptr, B, k, E, stream), "kq_moe_gemv_dev")


def moe_gemv_routed_dev(op: KqMoeOp, probs_ptr: int, B: int, k: int, E: int, sel_ptr: int,
                        selw_ptr: int, stream: int | None = None) -> None:
    """B tokens: top-k of probs[B][E] inside the launch that runs op (written
    to sel / selw), then op on the selected experts (kq_moe_gemv_routed_dev)."""
    _check(lib().kq_moe_gemv_routed_dev(ctypes.byref(op), probs_ptr, B, k, E, sel_ptr, selw_ptr,
                                        stream), "kq_moe_gemv_routed_dev")


def softmax_dev(x_ptr: int, B: int, E: int, stream: int | None = None) -> None:
    _check(lib().kq_softmax_dev(x_ptr, B, E, stream), "kq_softmax_dev")


def swiglu_dev(g_ptr: int, u_ptr: int, y_ptr: int, n: int, stream: int | None = None) -> None:
    _check(lib().kq_swiglu_dev(g_ptr, u_ptr, y_ptr, n, stream), "kq_swiglu_dev")


def moe_combine_dev(o_ptr: int, sel_ptr: int, selw_ptr: int, resid_ptr: int, x_ptr: int, B: int,
                    k: int, H: int, stream: int | None = None) -> None:
    _check(lib().kq_moe_combine_dev(o_ptr, sel_ptr, selw_ptr, resid_ptr, x_ptr, B, k, H, stream),
           "kq_moe_combine_dev")


def moe_ffn_workspace_bytes(f: KqMoeFfn, B: int) -> int:
    n = lib().kq_moe_ffn_workspace_bytes(ctypes.byref(f), B)
    if n < 0:
        msg = lib().kq_last_error().decode(errors="replace")
        raise RuntimeError(f"kq_moe_ffn_workspace_bytes failed: {msg}")
    return n


# kq_moe_ffn_last_path bits (include/kq_gemv.h)
FFN_FUSED_B1, FFN_RUNS_STORED, FFN_RUNS_LOADED, FFN_GROUP_LAUNCH = 1, 2, 4, 8


def moe_ffn_workspace_offsets(f: KqMoeFfn, B: int) -> dict:
    """Offsets of probs, g, u, act, ffo and the run tables ("runs") in the
    step's workspace (the layout kq_moe_ffn_dev uses: in that order, each
    256-byte aligned; the grouping records follow the run tables)."""
    bk = B * f.k
    sizes = [("probs", B * f.n_experts * 4), ("g", bk * f.n_ff * 4), ("u", bk * f.n_ff * 4),
             ("act", bk * f.n_ff * 4), ("ffo", bk * f.n_embed * 4)]
    out, t = {}, 0
    for name, n in sizes:
        out[name] = t
        t += (n + 255) // 256 * 256
    out["runs"] = t
    return out


def moe_ffn_last_path() -> int:
    """What the last kq_moe_ffn_dev call ran (FFN_* bits)."""
    return int(lib().kq_moe_ffn_last_path())


def moe_ffn_dev(f: KqMoeFfn, xn_ptr: int, x_ptr: int, B: int, sel_ptr: int, selw_ptr: int,
                work_ptr: int, work_bytes: int, stream: int | None = None) -> None:
    _check(lib().kq_moe_ffn_dev(ctypes.byref(f), xn_ptr, x_ptr, B, sel_ptr, selw_ptr, work_ptr,
                                work_bytes, stream), "kq_moe_ffn_dev")
