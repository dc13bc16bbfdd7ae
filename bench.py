#!/usr/bin/env python3
"""k-quant GEMV on one MI355X: HBM GB/s, fraction of peak, µs per layer set.

Workload (where the >=70 % north-star target is
quoted): the seven batch-1 matvecs of one 27B-class dense decode layer,
hidden 5120 --
  Q 5120->6144, K/V 5120->1024, O 6144->5120, gate/up 5120->17408 in Q4_K,
  down 17408->5120 in Q6_K --
on seeded synthetic super-blocks and x ~ N(0,1) (stratum_amd.synth).

A step is one pass over the layer set as a decode loop issues it: one
kq_gemv_segments_dev launch per group of matvecs that share an input and
have no dependency between them -- [Q, K, V], [O], [gate, up], [down] --
each launch reading its weights from HBM.  (The 7-launch form, one
kq_gemv_dev per tensor as the reference calls st_linear_dispatch, is timed
too and reported as "separate_launches".)  Four device copies of the
layer's weights (860 MB) are rotated so no step finds its weights in the
256 MB MALL or the L2s.

value = algorithmic bytes of the layer set / measured time per step, with
algorithmic bytes per matvec = N*(K/256)*block_bytes + 4K + 4N.  Before the
W warm-up steps the step runs untimed for 50 ms (clock_ramp_ms): an idle
GPU needs ~20 ms of sustained work to reach its clocks, as a running decode
loop has.
roofline: the dominant launch ([gate, up], kernel kq_segs_kernel<1, 1, false>)
timed per launch with HIP events on the stream it runs on; traffic from
profiles/traffic.json (rocprofv3 FETCH_SIZE / WRITE_SIZE, calibrated).
cpu_baseline: the reference's own scalar routines (oracle/_ref) -- or the
repo's restatement when that build is absent -- on the host cores, over a
bounded number of passes of the same layer set.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import stratum_amd as KQ  # noqa: E402
from stratum_amd import synth  # noqa: E402

METRIC = "k-quant GEMV HBM GB/s + % of peak (1 GPU); µs per decode-layer matvec set"
PEAK_HBM_GBS = 8000.0

# name, type, N (rows), K (row length), activation
LAYER_27B = [
    ("attn_q", KQ.TYPE_Q4_K, 6144, 5120, "h"),
    ("attn_k", KQ.TYPE_Q4_K, 1024, 5120, "h"),
    ("attn_v", KQ.TYPE_Q4_K, 1024, 5120, "h"),
    ("attn_output", KQ.TYPE_Q4_K, 5120, 6144, "attn"),
    ("ffn_gate", KQ.TYPE_Q4_K, 17408, 5120, "h"),
    ("ffn_up", KQ.TYPE_Q4_K, 17408, 5120, "h"),
    ("ffn_down", KQ.TYPE_Q6_K, 5120, 17408, "ff"),
]
X_LEN = {"h": 5120, "attn": 6144, "ff": 17408}
# launches of one step: matvecs that share x and do not depend on each other
GROUPS = [
    ("attn_qkv", ["attn_q", "attn_k", "attn_v"]),
    ("attn_output", ["attn_output"]),
    ("ffn_gate_up", ["ffn_gate", "ffn_up"]),
    ("ffn_down", ["ffn_down"]),
]
DOMINANT = "ffn_gate_up"
DOMINANT_KERNEL = "kq_segs_kernel<1, 1, false>"
COPIES = 4


def algo_bytes(qtype: int, N: int, K: int, B: int = 1) -> int:
    return N * (K // 256) * KQ.BLOCK_BYTES[qtype] + 4 * K * B + 4 * N * B


# CPU share of one GPU on the GPU boxes: worker pools are sized to it
BOX_CPU_SHARE = 16


def physical_cores() -> int:
    """Physical cores among the CPUs this process may run on (hyperthread
    siblings counted once), from /proc/cpuinfo."""
    try:
        cpus = os.sched_getaffinity(0)
    except AttributeError:
        return os.cpu_count() or 1
    cores, cpu = set(), None
    try:
        phys = core = None
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "processor":
                cpu, phys, core = int(v), None, None
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
                if cpu in cpus:
                    cores.add((phys, core))
    except OSError:
        pass
    return len(cores) if cores else len(cpus)


def host_cores() -> int:
    """Threads for the CPU baselines: every physical core, at most the box's
    CPU share for one GPU."""
    return max(1, min(BOX_CPU_SHARE, physical_cores()))


def cpu_baseline(weights: dict, xs: dict) -> dict:
    """Reference scalar GEMV (oracle/_ref) over whole passes of the layer set,
    on all physical cores (at most the box's share) and on one thread."""
    from oracle import oracle as O
    impl, kind = O.ref(), "reference"
    if impl is None:
        impl, kind = O.port(), "port"
    cores = host_cores()
    set_bytes = sum(algo_bytes(t, N, K) for _, t, N, K, _ in LAYER_27B)

    def timed_passes(threads: int, budget_s: float):
        def one_pass():
            for name, t, N, K, xn in LAYER_27B:
                impl.gemv(t, weights[name], xs[xn], N, K, threads=threads)
        t0 = time.perf_counter()
        one_pass()                               # also warms the page cache
        first = time.perf_counter() - t0
        passes = max(1, min(200, int(budget_s / max(first, 1e-3))))
        t0 = time.perf_counter()
        for _ in range(passes):
            one_pass()
        return passes, (time.perf_counter() - t0) / passes

    passes, dt = timed_passes(cores, 6.0)
    passes1, dt1 = timed_passes(1, 6.0)
    return {
        "value": round(set_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": kind,
        "sample": (f"{passes} passes of the full 27B layer set (7 matvecs, "
                   f"{set_bytes / 1e6:.1f} MB) with the scalar routines "
                   f"q4k_dot_row_scalar / q6k_dot_row_scalar on {cores} threads "
                   f"(64-row tickets; {physical_cores()} physical cores available, "
                   f"at most {BOX_CPU_SHARE} used: the box's CPU share per GPU); "
                   f"{dt * 1e6:.0f} µs per layer set"),
        "us_per_layer_set": round(dt * 1e6, 1),
        "physical_cores": physical_cores(),
        "single_thread": {"value": round(set_bytes / dt1 / 1e9, 3), "unit": "GB/s", "cores": 1,
                          "us_per_layer_set": round(dt1 * 1e6, 1),
                          "sample": f"{passes1} passes of the same layer set on 1 thread"},
    }


def load_traffic() -> dict | None:
    path = os.path.join(ROOT, "profiles", "traffic.json")
    if not os.path.exists(path):
        return None
    return json.load(open(path)).get(DOMINANT)


# ---------------------------------------------------------------- other configs
# The other benchmark configurations, timed in the same run: weights rotated
# over enough device copies that each pass reads HBM (>= 600 MB rotating
# set), HIP events on the launch stream.
QWEN06B = [  # name, type, N, K, activation (hidden 1024, q 2048, ffn 3072)
    ("attn_q", KQ.TYPE_Q4_K, 2048, 1024, "h"),
    ("attn_k", KQ.TYPE_Q4_K, 1024, 1024, "h"),
    ("attn_v", KQ.TYPE_Q4_K, 1024, 1024, "h"),
    ("attn_output", KQ.TYPE_Q4_K, 1024, 2048, "attn"),
    ("ffn_gate", KQ.TYPE_Q4_K, 3072, 1024, "h"),
    ("ffn_up", KQ.TYPE_Q4_K, 3072, 1024, "h"),
    ("ffn_down", KQ.TYPE_Q6_K, 1024, 3072, "ff"),
]
QWEN06B_GROUPS = [["attn_q", "attn_k", "attn_v"], ["attn_output"], ["ffn_gate", "ffn_up"],
                  ["ffn_down"]]
ROTATE_BYTES = 600 << 20


RAMP_MS = 50.0   # untimed work before any timing: the GPU's clocks take ~20 ms to ramp up


def ramp(torch, fn, ms=RAMP_MS):
    """Runs fn untimed for `ms` of wall time.  After an idle period the GPU
    needs about 20 ms of sustained work to reach its clocks (measured: the
    27B layer set runs at ~69 us per step after 1.4 ms of warm-up and ~64 us
    after 20 ms or more), and a decode loop runs continuously."""
    t0, i = time.perf_counter(), 0
    while (time.perf_counter() - t0) * 1e3 < ms:
        fn(i)
        i += 1
        if i % 32 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    return i


def _events_us(torch, stream, fn, reps, warmup=3):
    ramp(torch, fn, 20.0)
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(reps):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) * 1e3 / reps


def _copies(torch, host: np.ndarray, min_copies: int = 3):
    n = max(min_copies, -(-ROTATE_BYTES // max(1, host.size)))
    d = torch.from_numpy(host).cuda()
    return [d] + [d.clone() for _ in range(n - 1)]


def _check(L, rc):
    if rc != 0:
        raise RuntimeError(L.kq_last_error().decode())


MFMA_F16_PEAK_TFLOPS = 2500.0

# the CPU baseline beside each other configuration (cleared by --no-cpu-baseline)
CPU = {"on": True}


def cpu_impl(qtype: int):
    """The reference's scalar routines (oracle/_ref) for the types it runs on
    x86 (its type-42 kernel is NEON only), else the repo's restatement."""
    from oracle import oracle as O
    r = O.ref()
    if r is not None and qtype in (KQ.TYPE_Q2_K, KQ.TYPE_Q4_K, KQ.TYPE_Q6_K):
        return r, "reference"
    return O.port(), "port"


def cpu_us(fn, min_s: float = 0.3, max_n: int = 50) -> float:
    """Mean host time of fn over at least min_s (after one untimed call)."""
    fn()
    t0, n = time.perf_counter(), 0
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= min_s or n >= max_n:
            return dt / n * 1e6


def cpu_entry(us: float, kind: str, what: str) -> dict:
    return {"us": round(us, 1), "cores": host_cores(), "kind": kind, "sample": what}


def multiseq_mfma(L, torch, stream, host_w) -> dict:
    """configs[3] on the matrix cores (kq_gemv_multix_mfma_dev, B >= 16).

    Time per call with HIP events on the launch stream; TFLOP/s counts the
    product's 2*N*K*B flops; mfma_util counts the fp16 MFMA flops the kernel
    issues (two planes of x, times hi and lo of the weights for Q6_K, streams
    padded to 16) against the dense fp16 peak.
    Tolerance: every output against the exact multi-x path (bit-identical to
    the reference's scalar routine in the GPU tests): max |a-b|/max(|b|,1e-6),
    the fraction within 1e-5, and max |a-b| / sum_k |w_k x_k| (the error
    relative to the magnitude of the terms, |W| from the device dequant)."""
    sh = stream.cuda_stream
    res = {}
    for name, t, N, K in (("ffn_gate", 12, 17408, 5120), ("ffn_up", 12, 17408, 5120),
                          ("ffn_down", 14, 5120, 17408)):
        cm = _copies(torch, host_w[name])
        wabs = torch.empty(N * K, dtype=torch.float32, device="cuda")
        _check(L, L.kq_dequant_dev(t, cm[0].data_ptr(), wabs.data_ptr(), N * K // 256, sh))
        wabs = wabs.view(N, K).abs_()
        for B in (16, 32, 64):
            xs = torch.from_numpy(np.stack([synth.gaussian(synth.rng(3900 + s), K)
                                            for s in range(B)])).cuda()
            ym = torch.empty(B * N, dtype=torch.float32, device="cuda")
            ye = torch.empty(B * N, dtype=torch.float32, device="cuda")
            us = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_multix_mfma_dev(
                t, cm[i % len(cm)].data_ptr(), xs.data_ptr(), ym.data_ptr(), B, N, K, sh)),
                20)
            _check(L, L.kq_gemv_multix_mfma_dev(t, cm[0].data_ptr(), xs.data_ptr(),
                                                ym.data_ptr(), B, N, K, sh))
            _check(L, L.kq_gemv_multix_dev(t, cm[0].data_ptr(), xs.data_ptr(), ye.data_ptr(),
                                           B, N, K, sh))
            mag = torch.matmul(xs.abs(), wabs.t()).reshape(-1)
            torch.cuda.synchronize()
            d = (ym - ye).abs()
            rel = d / ye.abs().clamp_min(1e-6)
            nb = algo_bytes(t, N, K, B)
            flops = 2.0 * N * K * B
            issued = (2 if t == 12 else 4) * 2.0 * N * K * ((B + 15) // 16 * 16)
            res[f"{name}_B{B}"] = {
                "us_per_call": round(us, 2), "us_per_stream": round(us / B, 2),
                "GB/s": round(nb / us / 1e3, 1), "TFLOP/s": round(flops / us / 1e6, 2),
                "mfma_util": round(issued / us / 1e6 / MFMA_F16_PEAK_TFLOPS, 4),
                "max_rel_err_vs_exact": float(f"{rel.max().item():.3e}"),
                "frac_within_1e-5": round((rel <= 1e-5).float().mean().item(), 5),
                "max_err_over_mag": float(f"{(d / mag.clamp_min(1e-30)).max().item():.3e}")}
            del xs, ym, ye, mag, d, rel
        del cm, wabs
    return res


MFMA_I8_PEAK_TOPS = 5000.0


def multiseq_int8(L, torch, stream, host_w) -> dict:
    """configs[3] in the int8-activation mode: kq_gemv_multix_dev(type |
    KQ_INT8_ACT), which for Q4_K / Q6_K at B >= 2 computes st_linear_multix's
    use_sdot arithmetic (the reference's multix_pack: a binary32 term per
    Q4_K sub-block, binary64 per Q6_K 16-group, summed in binary64) with the
    integer dots on the matrix cores (v_mfma_i32_16x16x64_i8).
    Time per call (quantization launch included) with HIP events; TOP/s
    counts the product's 2*N*K*B integer ops; mfma_util the int8 MFMA ops
    the kernel issues (operand rows masked to one sub-block (Q4_K) or one
    16-run (Q6_K) of the 64 k-values: 2x and 4x the product's) against the
    dense int8 peak.  Distance to the single-stream int8 form
    (kq_gemv_dev(type | KQ_INT8_ACT)): max |a - b| / max(|b|, 1e-6)."""
    sh = stream.cuda_stream
    res = {}
    for name, t, N, K in (("ffn_gate", 12, 17408, 5120), ("ffn_up", 12, 17408, 5120),
                          ("ffn_down", 14, 5120, 17408)):
        cm = _copies(torch, host_w[name])
        for B in (8, 16, 32, 64):
            xs = torch.from_numpy(np.stack([synth.gaussian(synth.rng(4100 + s), K)
                                            for s in range(B)])).cuda()
            ym = torch.empty(B * N, dtype=torch.float32, device="cuda")
            us = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_multix_dev(
                t | KQ.INT8_ACT, cm[i % len(cm)].data_ptr(), xs.data_ptr(), ym.data_ptr(), B,
                N, K, sh)), 20)
            _check(L, L.kq_gemv_multix_dev(t | KQ.INT8_ACT, cm[0].data_ptr(), xs.data_ptr(),
                                           ym.data_ptr(), B, N, K, sh))
            y1 = torch.empty(N, dtype=torch.float32, device="cuda")
            _check(L, L.kq_gemv_dev(t | KQ.INT8_ACT, cm[0].data_ptr(), xs.data_ptr(), None,
                                    y1.data_ptr(), N, K, sh))
            torch.cuda.synchronize()
            rel = ((ym[:N] - y1).abs() / y1.abs().clamp_min(1e-6)).max().item()
            ops = 2.0 * N * K * B
            issued = ops * (2 if t == 12 else 4) * ((B + 7) // 8 * 8) / B
            nb = algo_bytes(t, N, K, B)
            res[f"{name}_B{B}"] = {
                "us_per_call": round(us, 2), "us_per_stream": round(us / B, 2),
                "GB/s": round(nb / us / 1e3, 1), "TOP/s": round(ops / us / 1e6, 2),
                "mfma_util": round(issued / us / 1e6 / MFMA_I8_PEAK_TOPS, 4),
                "max_rel_vs_single_stream_int8": float(f"{rel:.3e}")}
            del xs, ym, y1
        del cm
    return res


def cfg1(L, torch, stream, host_w) -> dict:
    """one Q4_K GEMV, W 1024 x 1024 (4096 blocks), batch 1."""
    sh = stream.cuda_stream
    w = synth.tensor(KQ.TYPE_Q4_K, 1024, 1024, 3000)
    cw = _copies(torch, w)
    xh = synth.gaussian(synth.rng(3001), 1024)
    x = torch.from_numpy(xh).cuda()
    y = torch.empty(1024, dtype=torch.float32, device="cuda")
    us = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_dev(
        12, cw[i % len(cw)].data_ptr(), x.data_ptr(), None, y.data_ptr(), 1024, 1024, sh)), 200)
    nb = algo_bytes(12, 1024, 1024)
    res = {"us_per_call": round(us, 2), "bytes": nb, "GB/s": round(nb / us / 1e3, 1)}
    if CPU["on"]:
        impl, kind = cpu_impl(12)
        res["cpu"] = cpu_entry(cpu_us(lambda: impl.gemv(12, w, xh, 1024, 1024,
                                                        threads=host_cores())), kind,
                               "one call of the same GEMV")
    return res


def cfg2(L, torch, stream, host_w) -> dict:
    """Qwen3-0.6B layer set (4 launches) and the LM head."""
    sh = stream.cuda_stream
    spec = {n: (t, N, K, xn) for n, t, N, K, xn in QWEN06B}
    xl = {"h": 1024, "attn": 2048, "ff": 3072}
    hw = {n: synth.tensor(t, N, K, 3100 + i) for i, (n, t, N, K, _) in enumerate(QWEN06B)}
    offs, tot = {}, 0
    for n in hw:
        offs[n] = tot
        tot += (hw[n].size + 255) // 256 * 256
    blob = np.zeros(tot, np.uint8)
    for n in hw:
        blob[offs[n]:offs[n] + hw[n].size] = hw[n]
    cb = _copies(torch, blob)
    xqh = {k: synth.gaussian(synth.rng(3200 + j), n) for j, (k, n) in enumerate(xl.items())}
    xq = {k: torch.from_numpy(v).cuda() for k, v in xqh.items()}
    yq = {n: torch.empty(N, dtype=torch.float32, device="cuda") for n, _, N, _, _ in QWEN06B}
    arrs = []
    for c in cb:
        per = []
        for members in QWEN06B_GROUPS:
            segs = [KQ.segment(spec[m][0], spec[m][2], spec[m][1], [c.data_ptr() + offs[m]],
                               xq[spec[m][3]].data_ptr(), yq[m].data_ptr()) for m in members]
            per.append(((KQ.KqSegment * len(segs))(*segs), len(segs)))
        arrs.append(per)

    def qstep(i):
        for arr, n in arrs[i % len(arrs)]:
            _check(L, L.kq_gemv_segments_dev(arr, n, sh))
    us = _events_us(torch, stream, qstep, 100)
    nb = sum(algo_bytes(t, N, K) for _, t, N, K, _ in QWEN06B)
    res = {"us_per_layer_set": round(us, 2), "bytes": nb, "GB/s": round(nb / us / 1e3, 1),
           "launches": len(QWEN06B_GROUPS)}
    del cb, arrs
    lm = synth.tensor(KQ.TYPE_Q6_K, 151936, 1024, 3300)
    cl = _copies(torch, lm)
    ylm = torch.empty(151936, dtype=torch.float32, device="cuda")
    us = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_dev(
        14, cl[i % len(cl)].data_ptr(), xq["h"].data_ptr(), None, ylm.data_ptr(), 151936, 1024,
        sh)), 50)
    nb = algo_bytes(14, 151936, 1024)
    res["lm_head_q6k"] = {"us_per_call": round(us, 2), "bytes": nb, "GB/s": round(nb / us / 1e3, 1)}
    if CPU["on"]:
        impl, kind = cpu_impl(12)
        res["cpu"] = cpu_entry(cpu_us(lambda: [impl.gemv(t, hw[n], xqh[xn], N, K, threads=host_cores())
                                               for n, t, N, K, xn in QWEN06B]), kind,
                               "the 7 matvecs of the layer set")
        res["lm_head_q6k"]["cpu"] = cpu_entry(
            cpu_us(lambda: impl.gemv(14, lm, xqh["h"], 151936, 1024, threads=host_cores())), kind,
            "one LM-head GEMV")
    return res


def cfg3(L, torch, stream, host_w) -> dict:
    """configs[2] extra: gate + up as Q2_K and as type 42 (one launch of two tensors)."""
    sh = stream.cuda_stream
    res = {}
    q2 = [synth.tensor(KQ.TYPE_Q2_K, 17408, 5120, 3400 + i) for i in range(2)]
    for t, name in ((KQ.TYPE_Q2_K, "q2k"), (KQ.TYPE_Q2K_NIB, "type42")):
        ws = q2 if t == KQ.TYPE_Q2_K else [
            np.concatenate([synth.q2k_to_nib(q[j:j + 84 * 20000]) for j in range(0, q.size, 84 * 20000)])
            for q in q2]
        both = np.concatenate(ws)
        cg = _copies(torch, both)
        xgh = synth.gaussian(synth.rng(3500), 5120)
        xg = torch.from_numpy(xgh).cuda()
        yg = [torch.empty(17408, dtype=torch.float32, device="cuda") for _ in range(2)]
        half = ws[0].size
        arrs = []
        for c in cg:
            segs = [KQ.segment(t, 5120, 17408, [c.data_ptr() + j * half], xg.data_ptr(),
                               yg[j].data_ptr()) for j in range(2)]
            arrs.append((KQ.KqSegment * 2)(*segs))
        us = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_segments_dev(
            arrs[i % len(arrs)], 2, sh)), 50)
        nb = 2 * algo_bytes(t, 17408, 5120)
        res[name] = {"us_per_launch": round(us, 2), "bytes": nb, "GB/s": round(nb / us / 1e3, 1)}
        if CPU["on"]:
            impl, kind = cpu_impl(t)
            res[name]["cpu"] = cpu_entry(
                cpu_us(lambda: [impl.gemv(t, wj, xgh, 17408, 5120, threads=host_cores())
                                for wj in ws]), kind, "gate and up (two GEMVs)")
        del cg, arrs
    return res


def cfg4(L, torch, stream, host_w) -> dict:
    """MULTISEQ, B streams with one weight pass (27B gate / up /
    down), exact path (each stream bit-identical to its single-stream result)."""
    sh = stream.cuda_stream
    res = {}
    for name, t, N, K in (("ffn_gate", 12, 17408, 5120), ("ffn_up", 12, 17408, 5120),
                          ("ffn_down", 14, 5120, 17408)):
        cm = _copies(torch, host_w[name])
        for B in (8, 16, 64):
            xsh = np.stack([synth.gaussian(synth.rng(3600 + s), K) for s in range(B)])
            xs = torch.from_numpy(xsh).cuda()
            ysb = torch.empty(B * N, dtype=torch.float32, device="cuda")
            us = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_multix_dev(
                t, cm[i % len(cm)].data_ptr(), xs.data_ptr(), ysb.data_ptr(), B, N, K, sh)),
                10 if B == 64 else 20)
            nb = algo_bytes(t, N, K, B)
            res[f"{name}_B{B}"] = {"us_per_call": round(us, 2), "us_per_stream": round(us / B, 2),
                                   "GB/s": round(nb / us / 1e3, 1),
                                   "TFLOP/s": round(2.0 * N * K * B / us / 1e6, 2)}
            if CPU["on"]:
                impl, kind = cpu_impl(t)
                res[f"{name}_B{B}"]["cpu"] = cpu_entry(
                    cpu_us(lambda: impl.gemv_multix(t, host_w[name], xsh, N, K,
                                                    threads=host_cores()), min_s=0.2, max_n=5),
                    kind, f"one call of {B} streams (the scalar routine per stream)")
        del cm
    return res


def cfg5(L, torch, stream, host_w) -> dict:
    """MoE gather, 128 experts, top-8, hidden 2048, expert ffn
    768, Q4_K; a step is top-k on the device, gate+up, down (batch 1: the
    top-k inside the gate+up launch, kq_moe_gemv_routed_dev).

    Past the MALL: the selected slices change from step to step.  Step i
    takes routing set i % MOE_SETS on weight copy (i // MOE_SETS) % 3: at
    batch 1 the sets select disjoint experts (set j: experts 8j .. 8j+7,
    by logits raised by 10), at batch 16 they are independent N(0,1)
    logits.  One rotation then reads 48 x 21 MB = 1 GB (batch 1) or about
    3 x 16 x 215 MB (batch 16) of distinct slices, 4x the 256 MB MALL.  The
    FFN step routes from its own router GEMV, so it cycles MOE_SETS
    different normed inputs the same way."""
    sh = stream.cuda_stream
    E, H, F, k = 128, 2048, 768, 8
    MOE_SETS, NCOPY = 16, 3
    rbg, rbd = L.kq_row_bytes(12, H), L.kq_row_bytes(12, F)
    gsl, dsl = F * rbg, H * rbd
    ex = [synth.tensor(12, E * F, H, 3700), synth.tensor(12, E * F, H, 3701),
          synth.tensor(12, E * H, F, 3702)]
    stacked = np.concatenate(ex)
    cm = _copies(torch, stacked, NCOPY)[:NCOPY]
    from oracle import oracle as O
    port = O.port()
    res = {}
    for B in (1, 16):
        r = np.random.default_rng(3800 + B)
        lg = r.standard_normal((MOE_SETS, B, E)).astype(np.float32)
        if B == 1:
            for j in range(MOE_SETS):
                lg[j, 0, 8 * j:8 * j + 8] += 10.0
        p = np.exp(lg - lg.max(2, keepdims=True))
        ph = (p / p.sum(2, keepdims=True)).astype(np.float32)
        probs = torch.from_numpy(ph.reshape(-1)).cuda()
        xmh = np.stack([synth.gaussian(r, H) for _ in range(MOE_SETS * B)])
        acth = np.stack([synth.gaussian(r, F) for _ in range(B * k)])
        xm = torch.from_numpy(xmh.reshape(-1)).cuda()
        act = torch.from_numpy(acth).cuda()
        sel = torch.empty(B * k, dtype=torch.int32, device="cuda")
        selw = torch.empty(B * k, dtype=torch.float32, device="cuda")
        yg, yu = (torch.empty(B * k * F, device="cuda") for _ in range(2))
        yd = torch.empty(B * k * H, device="cuda")
        # the experts each routing set selects (moe_topk per token)
        sets = [sorted({e for s in range(B) for e in port.topk(ph[j, s], k)[0]})
                for j in range(MOE_SETS)]
        distinct = float(np.mean([len(t) for t in sets]))
        ops = []
        for c in cm:
            base = c.data_ptr()
            ops.append([(KQ.moe_op(12, F, H, [base, base + E * gsl], gsl,
                                   xm.data_ptr() + 4 * j * B * H, k,
                                   [yg.data_ptr(), yu.data_ptr()]),
                         KQ.moe_op(12, H, F, [base + 2 * E * gsl], dsl, act.data_ptr(), 1,
                                   [yd.data_ptr()]))
                        for j in range(MOE_SETS)])

        def moe_step(i):
            j = i % MOE_SETS
            gu, dn = ops[(i // MOE_SETS) % NCOPY][j]
            # routed inside the gate+up launch
            _check(L, L.kq_moe_gemv_routed_dev(ctypes.byref(gu), probs.data_ptr() + 4 * j * B * E,
                                               B, k, E, sel.data_ptr(), selw.data_ptr(), sh))
            _check(L, L.kq_moe_gemv_dev(ctypes.byref(dn), sel.data_ptr(), B, k, E, sh))
        us = _events_us(torch, stream, moe_step, 2 * MOE_SETS * NCOPY)
        # the same step in the int8-activation mode (Q4_K | KQ_INT8_ACT)
        def as_int8(op):
            o = KQ.KqMoeOp.from_buffer_copy(op)
            o.type = 12 | KQ.INT8_ACT
            return o
        ops8 = [[(as_int8(gu), as_int8(dn)) for gu, dn in per] for per in ops]

        def moe_step8(i):
            j = i % MOE_SETS
            gu, dn = ops8[(i // MOE_SETS) % NCOPY][j]
            _check(L, L.kq_moe_gemv_routed_dev(ctypes.byref(gu), probs.data_ptr() + 4 * j * B * E,
                                               B, k, E, sel.data_ptr(), selw.data_ptr(), sh))
            _check(L, L.kq_moe_gemv_dev(ctypes.byref(dn), sel.data_ptr(), B, k, E, sh))
        us8 = _events_us(torch, stream, moe_step8, 2 * MOE_SETS * NCOPY)
        nb = distinct * (2 * gsl + dsl) + 4 * (B * H + 2 * B * k * F + B * k * F + B * k * H)
        per_rot = sum(len(t) for t in sets) * NCOPY * (2 * gsl + dsl)
        res[f"B{B}"] = {"us_per_layer": round(us, 2), "distinct_experts": round(distinct, 2),
                        "bytes": int(nb), "GB/s": round(nb / us / 1e3, 1),
                        "launches": 2 if B * ((E + 63) // 64 * 64) ** 2 <= 1 << 16 else 3,
                        "route": "kq_moe_gemv_routed_dev",
                        "rotation": f"{MOE_SETS} routing sets x {NCOPY} weight copies: "
                                    f"{per_rot / 2 ** 20:.0f} MiB of selected slices per "
                                    "rotation",
                        "int8": {"us_per_layer": round(us8, 2), "GB/s": round(nb / us8 / 1e3, 1),
                                 "what": "the same gather with Q4_K | KQ_INT8_ACT"}}
        # the whole expert FFN step (kq_moe_ffn_dev): F32 router GEMV, softmax,
        # routed gate+up, SwiGLU, down, rank-ordered combine + residual
        router = torch.from_numpy(synth.tensor(KQ.TYPE_F32, E, H, 3703)).cuda()
        ffns = []
        for c in cm:
            f = KQ.KqMoeFfn()
            f.n_embed, f.n_ff, f.n_experts, f.k = H, F, E, k
            f.router_type, f.router = KQ.TYPE_F32, router.data_ptr()
            f.gate_type = f.up_type = f.down_type = 12
            f.gate, f.up, f.down = c.data_ptr(), c.data_ptr() + E * gsl, c.data_ptr() + 2 * E * gsl
            f.gate_stride, f.up_stride, f.down_stride = gsl, gsl, dsl
            ffns.append(f)
        wbytes = KQ.moe_ffn_workspace_bytes(ffns[0], B)
        work = torch.empty(wbytes, dtype=torch.uint8, device="cuda")
        xres = torch.from_numpy(np.stack([synth.gaussian(r, H) for _ in range(B)])).cuda()

        def ffn_step(i):
            j = i % MOE_SETS
            _check(L, L.kq_moe_ffn_dev(ctypes.byref(ffns[(i // MOE_SETS) % NCOPY]),
                                       xm.data_ptr() + 4 * j * B * H, xres.data_ptr(), B,
                                       sel.data_ptr(), selw.data_ptr(), work.data_ptr(), wbytes,
                                       sh))
        fus = _events_us(torch, stream, ffn_step, 2 * MOE_SETS * NCOPY)
        # the same step in the int8-activation mode (the reference's default
        # arithmetic, use_sdot: expert GEMVs as Q4_K | KQ_INT8_ACT)
        ffns8 = []
        for f in ffns:
            f8 = KQ.KqMoeFfn.from_buffer_copy(f)
            f8.gate_type = f8.up_type = f8.down_type = 12 | KQ.INT8_ACT
            ffns8.append(f8)
        wbytes8 = KQ.moe_ffn_workspace_bytes(ffns8[0], B)
        work8 = torch.empty(wbytes8, dtype=torch.uint8, device="cuda")

        def ffn_step8(i):
            j = i % MOE_SETS
            _check(L, L.kq_moe_ffn_dev(ctypes.byref(ffns8[(i // MOE_SETS) % NCOPY]),
                                       xm.data_ptr() + 4 * j * B * H, xres.data_ptr(), B,
                                       sel.data_ptr(), selw.data_ptr(), work8.data_ptr(), wbytes8,
                                       sh))
        fus8 = _events_us(torch, stream, ffn_step8, 2 * MOE_SETS * NCOPY)
        res[f"B{B}"]["ffn_step"] = {
            "us_per_layer": round(fus, 2),
            "int8_us_per_layer": round(fus8, 2),
            "what": "router GEMV (F32 128x2048), softmax, routed gate+up, SwiGLU, down, "
                    f"combine + residual; {MOE_SETS} normed inputs x {NCOPY} weight copies; "
                    "int8: the same step with the expert GEMVs as Q4_K | KQ_INT8_ACT"}
        del work8
        del work, router
        if CPU["on"]:
            impl, kind = cpu_impl(12)
            rb = (rbg, rbg, rbd)
            sl = (gsl, gsl, dsl)
            pr = ph[0]

            def cpu_layer():
                for s in range(B):            # moe_topk per token, then the selected slices
                    es, _ = port.topk(pr[s], k)
                    for rr, e in enumerate(es):
                        m = s * k + rr
                        for ti, (nout, kin, xv) in enumerate(((F, H, xmh[s]), (F, H, xmh[s]),
                                                              (H, F, acth[m]))):
                            off = e * sl[ti]
                            impl.gemv(12, ex[ti][off:off + nout * rb[ti]], xv, nout, kin,
                                      threads=host_cores())
            res[f"B{B}"]["cpu"] = cpu_entry(cpu_us(cpu_layer, min_s=0.2, max_n=10), kind,
                                            "top-k and the selected gate, up and down slices")
    del cm
    return res


# bench.py --only NAME runs one of these (the keys of other_configs' result)
def cfg_int8(L, torch, stream, host_w) -> dict:
    """configs[2] in the int8-activation mode (type | KQ_INT8_ACT, the
    reference's SDOT path): the same four launches of the 27B layer set,
    weights rotated over device copies.  Tolerance: within one binary32 ulp
    of the binary64-term order, and within the binary32 lanes' rounding
    bound of q*_dot_row_sdot_f (tests/test_gpu_int8.py)."""
    sh = stream.cuda_stream
    spec = {name: (t, N, K, xn) for name, t, N, K, xn in LAYER_27B}
    xs_host = {k: synth.gaussian(synth.rng(2000 + j), n) for j, (k, n) in enumerate(X_LEN.items())}
    xs = {k: torch.from_numpy(v).cuda() for k, v in xs_host.items()}
    ys = {name: torch.empty(N, dtype=torch.float32, device="cuda") for name, _, N, _, _ in LAYER_27B}
    offs, total = {}, 0
    for name, *_ in LAYER_27B:
        offs[name] = total
        total += (host_w[name].size + 255) // 256 * 256
    blob = np.zeros(total, np.uint8)
    for name, *_ in LAYER_27B:
        blob[offs[name]:offs[name] + host_w[name].size] = host_w[name]
    copies = _copies(torch, blob, COPIES)
    arrs = {}
    for flag in (KQ.INT8_ACT, 0):
        arrs[flag] = []
        for c in copies:
            per_group = []
            for gname, members in GROUPS:
                segs = [KQ.segment(spec[m][0] | flag, spec[m][2], spec[m][1],
                                   [c.data_ptr() + offs[m]], xs[spec[m][3]].data_ptr(),
                                   ys[m].data_ptr()) for m in members]
                per_group.append(((KQ.KqSegment * len(segs))(*segs), len(segs)))
            arrs[flag].append(per_group)

    def launch(ci, g, flag=KQ.INT8_ACT):
        arr, n = arrs[flag][ci % len(arrs[flag])][g]
        _check(L, L.kq_gemv_segments_dev(arr, n, sh))

    res = {}
    set_bytes = sum(algo_bytes(t, N, K) for _, t, N, K, _ in LAYER_27B)
    for flag, key in ((KQ.INT8_ACT, "layer_set"), (0, "layer_set_exact_same_process")):
        us = _events_us(torch, stream,
                        lambda i: [launch(i, g, flag) for g in range(len(GROUPS))], 100)
        res[key] = {"us_per_layer_set": round(us, 2), "bytes": set_bytes,
                    "GB/s": round(set_bytes / us / 1e3, 1)}
    del arrs
    # per launch: each group's weights rotated over >= ROTATE_BYTES of copies
    # (so every launch reads HBM, not the MALL), both modes in one process
    for gname, members in GROUPS:
        goff, gtot = {}, 0
        for m in members:
            goff[m] = gtot
            gtot += (host_w[m].size + 255) // 256 * 256
        gblob = np.zeros(gtot, np.uint8)
        for m in members:
            gblob[goff[m]:goff[m] + host_w[m].size] = host_w[m]
        gc = _copies(torch, gblob, COPIES)
        nb = sum(algo_bytes(spec[m][0], spec[m][1], spec[m][2]) for m in members)
        res[gname] = {"bytes": nb, "copies_rotated": len(gc)}
        for flag, key in ((KQ.INT8_ACT, "int8"), (0, "exact")):
            garr = []
            for c in gc:
                segs = [KQ.segment(spec[m][0] | flag, spec[m][2], spec[m][1],
                                   [c.data_ptr() + goff[m]], xs[spec[m][3]].data_ptr(),
                                   ys[m].data_ptr()) for m in members]
                garr.append(((KQ.KqSegment * len(segs))(*segs), len(segs)))

            def go(i):
                arr, n = garr[i % len(garr)]
                _check(L, L.kq_gemv_segments_dev(arr, n, sh))
            gus = _events_us(torch, stream, go, 100)
            res[gname][key] = {"us": round(gus, 2), "GB/s": round(nb / gus / 1e3, 1)}
        del gc
    if CPU["on"]:
        from oracle import oracle as O
        port = O.port()
        res["layer_set"]["cpu"] = cpu_entry(
            cpu_us(lambda: [port.gemv_i8(spec[m][0], host_w[m], xs_host[spec[m][3]], spec[m][1],
                                         spec[m][2], sdot_f=True) for m, *_ in LAYER_27B],
                   min_s=0.5, max_n=3),
            "port", "the seven matvecs in q*_dot_row_sdot_f's order, one thread")
        res["layer_set"]["cpu"]["cores"] = 1
    del copies
    # the other SDOT types (st_linear_q5k / _q3k / _q8_0 under use_sdot) on
    # the 27B gate shape, int8 against the exact path, weights rotated
    N, K = 17408, 5120
    xg = xs["h"]
    yt = torch.empty(N, dtype=torch.float32, device="cuda")
    for t, tname in ((KQ.TYPE_Q5_K, "Q5_K"), (KQ.TYPE_Q3_K, "Q3_K"), (KQ.TYPE_Q8_0, "Q8_0")):
        tc = _copies(torch, synth.tensor(t, N, K, 4200 + t), COPIES)
        nb = algo_bytes(t, N, K)
        res[f"{tname}_17408x5120"] = {"bytes": nb}
        for flag, key in ((KQ.INT8_ACT, "int8"), (0, "exact")):
            tus = _events_us(torch, stream, lambda i: _check(L, L.kq_gemv_dev(
                t | flag, tc[i % len(tc)].data_ptr(), xg.data_ptr(), None, yt.data_ptr(), N, K,
                sh)), 50)
            res[f"{tname}_17408x5120"][key] = {"us": round(tus, 2), "GB/s": round(nb / tus / 1e3, 1)}
        del tc
    return res


OTHER = {"cfg1_q4k_1024x1024": cfg1, "cfg2_qwen3_0.6b": cfg2, "cfg3_gate_up_q2k_type42": cfg3,
         "cfg4_multiseq_exact": cfg4, "cfg4_multiseq_mfma": multiseq_mfma,
         "cfg4_multiseq_int8": multiseq_int8,
         "cfg5_moe_128e_top8": cfg5, "cfg3_int8_activations": cfg_int8}


def _hbm_frac(o) -> None:
    """Adds hbm_frac = GB/s / 8000 next to every algorithmic-bytes rate."""
    if isinstance(o, dict):
        if "GB/s" in o:
            o["hbm_frac"] = round(o["GB/s"] / PEAK_HBM_GBS, 4)
        for v in o.values():
            _hbm_frac(v)


def other_configs(L, torch, stream, host_w, only=None) -> dict:
    out = {}
    for name, fn in OTHER.items():
        if only is None or name == only:
            out[name] = fn(L, torch, stream, host_w)
            torch.cuda.synchronize()
            torch.cuda.empty_cache()
    _hbm_frac(out)
    return out


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--skip-separate", action="store_true",
                    help="do not time the 7-launch form (profiling runs: then every "
                         "kq_segs_kernel<1, 1, false> dispatch is the dominant launch)")
    ap.add_argument("--main-only", action="store_true",
                    help="time only the 27B layer set (skip BASELINE's other configurations)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run 5 copies of 64 MiB (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--only", choices=sorted(OTHER),
                    help="run only this one of BASELINE's other configurations and print its "
                         "figures (profiling runs of one path)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} was asked for): every box here has one GPU, and the "
              f"row split across GPUs is a design, not code.", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    L = KQ.lib()  # fails loudly when the HIP library is missing

    # ---- inputs: one seeded copy on the host, COPIES rotated on the device
    spec = {name: (t, N, K, xn) for name, t, N, K, xn in LAYER_27B}
    host_w, offs, total = {}, {}, 0
    for i, (name, t, N, K, _) in enumerate(LAYER_27B):
        host_w[name] = synth.tensor(t, N, K, seed=1000 + i)
        offs[name] = total
        total += (host_w[name].size + 255) // 256 * 256
    blob = np.zeros(total, np.uint8)
    for name, *_ in LAYER_27B:
        blob[offs[name]:offs[name] + host_w[name].size] = host_w[name]
    dev0 = torch.from_numpy(blob).cuda()
    copies = [dev0] + [dev0.clone() for _ in range(COPIES - 1)]
    xs_host = {k: synth.gaussian(synth.rng(2000 + j), n) for j, (k, n) in enumerate(X_LEN.items())}
    xs = {k: torch.from_numpy(v).cuda() for k, v in xs_host.items()}
    ys = {name: torch.empty(N, dtype=torch.float32, device="cuda") for name, _, N, _, _ in LAYER_27B}
    stream = torch.cuda.current_stream()
    sh = stream.cuda_stream
    CPU["on"] = not args.no_cpu_baseline
    if args.only:
        del copies, dev0
        res = other_configs(L, torch, stream, host_w, only=args.only)
        print(json.dumps({"only": args.only, "data": "synthetic (seeded k-quant super-blocks, "
                          "x ~ N(0,1))", "figures": res[args.only]}), flush=True)
        return 0

    # segment arrays of every (copy, group), built once
    seg_arrays = []
    for c in copies:
        per_group = []
        for _, members in GROUPS:
            segs = [KQ.segment(spec[m][0], spec[m][2], spec[m][1], [c.data_ptr() + offs[m]],
                               xs[spec[m][3]].data_ptr(), ys[m].data_ptr()) for m in members]
            per_group.append(((KQ.KqSegment * len(segs))(*segs), len(segs)))
        seg_arrays.append(per_group)

    def launch_group(copy_i, g):
        arr, n = seg_arrays[copy_i][g]
        if L.kq_gemv_segments_dev(arr, n, sh) != 0:
            raise RuntimeError(L.kq_last_error().decode())

    def step(i):
        for g in range(len(GROUPS)):
            launch_group(i % COPIES, g)

    def step_separate(i):
        c = copies[i % COPIES]
        for name, t, N, K, xn in LAYER_27B:
            if L.kq_gemv_dev(t, c.data_ptr() + offs[name], xs[xn].data_ptr(), None,
                             ys[name].data_ptr(), N, K, sh) != 0:
                raise RuntimeError(L.kq_last_error().decode())

    def timed(fn, steps, warmup):
        ramp(torch, fn)
        for i in range(warmup):
            fn(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        w0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            fn(i)
        e1.record(stream)
        enqueue_s = time.perf_counter() - w0
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps, enqueue_s / steps * 1e3

    set_bytes = sum(algo_bytes(t, N, K) for _, t, N, K, _ in LAYER_27B)
    ms_per_step, enq_ms = timed(step, args.steps, args.warmup)
    gbs = set_bytes / (ms_per_step * 1e-3) / 1e9
    sep_ms, sep_enq_ms = (None, None) if args.skip_separate else \
        timed(step_separate, args.steps, args.warmup)

    # ---- per-launch durations: HIP events on the launch stream around
    # kernel_reps back-to-back launches of one group, each group's weights
    # rotated over enough device copies (>= ROTATE_BYTES) that every launch
    # reads them from HBM, not from the 256 MB MALL
    per_launch = {}
    for g, (gname, members) in enumerate(GROUPS):
        goff, gtot = {}, 0
        for m in members:
            goff[m] = gtot
            gtot += (host_w[m].size + 255) // 256 * 256
        gblob = np.zeros(gtot, np.uint8)
        for m in members:
            gblob[goff[m]:goff[m] + host_w[m].size] = host_w[m]
        gcopies = _copies(torch, gblob, COPIES)
        garr = []
        for c in gcopies:
            segs = [KQ.segment(spec[m][0], spec[m][2], spec[m][1], [c.data_ptr() + goff[m]],
                               xs[spec[m][3]].data_ptr(), ys[m].data_ptr()) for m in members]
            garr.append(((KQ.KqSegment * len(segs))(*segs), len(segs)))

        def launch_copy(i):
            arr, n = garr[i % len(garr)]
            if L.kq_gemv_segments_dev(arr, n, sh) != 0:
                raise RuntimeError(L.kq_last_error().decode())
        ramp(torch, launch_copy, 20.0)
        for i in range(4):
            launch_copy(i)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for i in range(args.kernel_reps):
            launch_copy(i + 1)
        b.record(stream)
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / args.kernel_reps
        nbytes = sum(algo_bytes(spec[m][0], spec[m][1], spec[m][2]) for m in members)
        per_launch[gname] = {"us": round(us, 2), "bytes": nbytes,
                             "GB/s": round(nbytes / (us * 1e-6) / 1e9, 1),
                             "copies_rotated": len(gcopies)}
        del gcopies, garr
    dom = per_launch[DOMINANT]
    achieved = dom["bytes"] / (dom["us"] * 1e-6) / 1e9
    tr = load_traffic()
    traffic = tr.get("hbm_bytes_per_launch") if tr else None

    if args.copy_calibration:
        src = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()

    out = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded k-quant super-blocks, x ~ N(0,1))",
        "config": {
            "workload": "27B-class dense decode layer matvec set, batch 1 (BASELINE configs[2]): "
                        "Q/K/V/O/gate/up Q4_K, down Q6_K, hidden 5120, ffn 17408; launches "
                        "[Q,K,V] [O] [gate,up] [down]",
            "layer_set_bytes": set_bytes,
            "weight_copies_rotated": COPIES,
            "launches_per_step": len(GROUPS),
        },
        "us_per_layer_set": round(ms_per_step * 1e3, 2),
        "clock_ramp_ms": RAMP_MS,
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "host_enqueue_us_per_step": round(enq_ms * 1e3, 1),
        "separate_launches": None if sep_ms is None else {
            "launches_per_step": len(LAYER_27B),
            "us_per_layer_set": round(sep_ms * 1e3, 2),
            "GB/s": round(set_bytes / (sep_ms * 1e-3) / 1e9, 1),
            "host_enqueue_us_per_step": round(sep_enq_ms * 1e3, 1)},
        "per_launch": per_launch,
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
            "kernel": f"{DOMINANT_KERNEL}: ffn_gate + ffn_up (Q4_K 2 x 17408x5120) in one launch",
        },
        "cpu_baseline": None,
    }
    if not args.main_only:
        del copies, seg_arrays
        out["other_configs"] = other_configs(L, torch, stream, host_w)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(host_w, xs_host)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
