#!/usr/bin/env python3
"""k-quant GEMV on one MI355X: HBM GB/s, fraction of peak, µs per layer set.

Workload (where the ≥70 % north-star target is
quoted): the seven batch-1 matvecs of one 27B-class dense decode layer,
hidden 5120 --
  Q 5120->6144, K/V 5120->1024, O 6144->5120, gate/up 5120->17408 in Q4_K,
  down 17408->5120 in Q6_K --
on seeded synthetic super-blocks and x ~ N(0,1) (stratum_amd.synth).
A step is one pass over the layer set: 7 GEMV launches, each reading its
weights from HBM.  Four device copies of the layer's weights (860 MB) are
rotated so no step finds its weights in the 256 MB MALL or the L2s.

value = algorithmic bytes of the layer set / measured time per step, with
algorithmic bytes per matvec = N*(K/256)*block_bytes + 4K + 4N.
roofline: the dominant kernel (ffn_gate, Q4_K 17408x5120) timed per launch
with HIP events on the stream it runs on.
cpu_baseline: the reference's own scalar routines (oracle/_ref) -- or the
repo's restatement when that build is absent -- on the host cores, over a
bounded number of passes of the same layer set.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""
from __future__ import annotations

import argparse
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
DOMINANT = "ffn_gate"
COPIES = 4


def algo_bytes(qtype: int, N: int, K: int, B: int = 1) -> int:
    return N * (K // 256) * KQ.BLOCK_BYTES[qtype] + 4 * K * B + 4 * N * B


def host_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(weights: dict, xs: dict) -> dict:
    """Reference scalar GEMV (oracle/_ref) over whole passes of the layer set."""
    from oracle import oracle as O
    impl, kind = O.ref(), "reference"
    if impl is None:
        impl, kind = O.port(), "port"
    cores = host_cores()
    set_bytes = sum(algo_bytes(t, N, K) for _, t, N, K, _ in LAYER_27B)

    def one_pass():
        for name, t, N, K, xn in LAYER_27B:
            impl.gemv(t, weights[name], xs[xn], N, K, threads=cores)

    t0 = time.perf_counter()
    one_pass()                                   # also warms the page cache
    first = time.perf_counter() - t0
    passes = max(1, min(200, int(8.0 / max(first, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(passes):
        one_pass()
    dt = (time.perf_counter() - t0) / passes
    return {
        "value": round(set_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": kind,
        "sample": (f"{passes} passes of the full 27B layer set (7 matvecs, "
                   f"{set_bytes / 1e6:.1f} MB) with the scalar routines "
                   f"q4k_dot_row_scalar / q6k_dot_row_scalar on {cores} threads "
                   f"(64-row tickets); {dt * 1e6:.0f} µs per layer set"),
        "us_per_layer_set": round(dt * 1e6, 1),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--kernel-reps", type=int, default=100)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path "
              f"(--gpus {args.gpus} was asked for); the row split across GPUs is "
              f"described in DESIGN.md.", file=sys.stderr)
        return 2

    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    KQ.lib()  # fails loudly when the HIP library is missing

    # ---- inputs: one seeded copy on the host, COPIES rotated on the device
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
    L = KQ.lib()
    plan = [(t, N, K, offs[name], xs[xn].data_ptr(), ys[name].data_ptr(), name)
            for name, t, N, K, xn in LAYER_27B]

    def launch(copy, t, N, K, off, xp, yp):
        rc = L.kq_gemv_dev(t, copy.data_ptr() + off, xp, None, yp, N, K, sh)
        if rc != 0:
            raise RuntimeError(L.kq_last_error().decode())

    def step(i):
        c = copies[i % COPIES]
        for t, N, K, off, xp, yp, _ in plan:
            launch(c, t, N, K, off, xp, yp)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(args.steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_per_step = e0.elapsed_time(e1) / args.steps
    set_bytes = sum(algo_bytes(t, N, K) for _, t, N, K, _ in LAYER_27B)
    gbs = set_bytes / (ms_per_step * 1e-3) / 1e9

    # ---- per-kernel durations (events around each launch, same stream)
    per_kernel = {}
    for t, N, K, off, xp, yp, name in plan:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(args.kernel_reps)]
        for i in range(4):
            launch(copies[i % COPIES], t, N, K, off, xp, yp)
        for i, (a, b) in enumerate(evs):
            a.record(stream)
            launch(copies[(i + 1) % COPIES], t, N, K, off, xp, yp)
            b.record(stream)
        torch.cuda.synchronize()
        us = float(np.mean([a.elapsed_time(b) for a, b in evs])) * 1e3
        per_kernel[name] = {"us": round(us, 2),
                            "GB/s": round(algo_bytes(t, N, K) / (us * 1e-6) / 1e9, 1)}
    dom = next(x for x in LAYER_27B if x[0] == DOMINANT)
    dom_us = per_kernel[DOMINANT]["us"]
    achieved = algo_bytes(dom[1], dom[2], dom[3]) / (dom_us * 1e-6) / 1e9
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("q4k_gemv_27b_gate", {}).get("hbm_bytes_per_launch")

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
        "data": "synthetic",
        "config": {
            "workload": "27B-class dense decode layer matvec set, batch 1 (BASELINE configs[2]): "
                        "Q/K/V/O/gate/up Q4_K, down Q6_K, hidden 5120, ffn 17408",
            "layer_set_bytes": set_bytes,
            "weight_copies_rotated": COPIES,
            "launches_per_step": len(LAYER_27B),
        },
        "us_per_layer_set": round(ms_per_step * 1e3, 2),
        "pct_of_peak": round(100.0 * gbs / PEAK_HBM_GBS, 2),
        "per_kernel": per_kernel,
        "roofline": {
            "bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": round(achieved / PEAK_HBM_GBS, 4), "traffic": traffic,
            "kernel": "kq_gemv_kernel<Q4_K> ffn_gate 17408x5120",
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(host_w, xs_host)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
