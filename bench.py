"""Benchmark driver (one JSON line on stdout).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads:
  qmv-config0  BASELINE config 0: affine 4-bit g64 QMV, W [4096, 2048],
               x [1, 2048].  A step is one QMV launch over a fresh weight copy:
               the timed loop rotates through >= 2 GiB of distinct weight
               copies so the 256 MB Infinity Cache cannot serve repeats.

Timing uses HIP events recorded on the stream the kernels are launched on.
The CPU baseline is the C oracle (oracle/liboracle.so, a restatement of the
reference arithmetic) timed on this host's cores over a bounded sample.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))

HBM_PEAK_GBS = 8000.0
METRIC = "batch-8 decode tok/s (aggregate) + QMV/MoE achieved HBM GB/s vs 8 TB/s peak"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def qweight_bytes(n: int, k: int, bits: int, gs: int) -> int:
    return n * k * bits // 8 + 4 * n * (k // gs)


def bench_qmv_config0(mx, args):
    from oracle import oracle as orc

    n, k, bits, gs, m = 4096, 2048, 4, 64, 1
    wbytes = qweight_bytes(n, k, bits, gs)
    alg_bytes = wbytes + 2 * m * k + 2 * m * n  # weights + x + y, counted once per launch
    copies = max(2, int(np.ceil(2 * 1024**3 / wbytes)))
    log(f"qmv-config0: {copies} weight copies ({copies * wbytes / 1e9:.2f} GB) for MALL rotation")
    ws = [mx.QWeight.random(n, k, bits, gs, seed=100 + 17 * i) for i in range(copies)]
    x = mx.DeviceArray.from_numpy(orc.fill_bf16(m * k, 101, 1, 1.0, 0.0).reshape(m, k))
    y = mx.DeviceArray((m, n), np.uint16)
    stream = C.c_void_p()
    mx.check(mx.lib.mx_stream_create(C.byref(stream)))
    qcs = [w.c() for w in ws]

    def launch(i):
        mx.check(mx.lib.mx_qmv(C.byref(qcs[i % copies]), x.ptr, m, y.ptr, stream))

    for i in range(args.warmup):
        launch(i)
    mx.check(mx.lib.mx_stream_sync(stream))
    e0, e1 = C.c_void_p(), C.c_void_p()
    mx.check(mx.lib.mx_event_create(C.byref(e0)))
    mx.check(mx.lib.mx_event_create(C.byref(e1)))
    mx.check(mx.lib.mx_device_sync())
    t0 = time.perf_counter()
    mx.check(mx.lib.mx_event_record(e0, stream))
    for i in range(args.steps):
        launch(args.warmup + i)
    mx.check(mx.lib.mx_event_record(e1, stream))
    ms = C.c_float()
    mx.check(mx.lib.mx_event_elapsed_ms(e0, e1, C.byref(ms)))
    mx.check(mx.lib.mx_device_sync())
    wall = time.perf_counter() - t0
    avg_s = ms.value / 1e3 / args.steps
    achieved = alg_bytes / avg_s / 1e9
    log(f"qmv-config0: {avg_s * 1e6:.2f} us/launch (events), wall {wall * 1e3:.1f} ms")

    # correctness of the measured kernel on the last copy
    codes, s, b = orc.random_qweight(n, k, bits, gs, seed=100 + 17 * ((args.warmup + args.steps - 1) % copies))
    want = orc.qmv(codes, s, b, k, bits, gs, x.numpy())
    if not (y.numpy() == want).all():
        raise SystemExit("bench: QMV output differs from oracle")

    cpu = cpu_baseline_qmv(orc, codes, s, b, k, bits, gs, x.numpy(), alg_bytes)
    return {
        "metric": METRIC,
        "value": round(achieved, 2),
        "unit": "GB/s",
        "ms_per_step": avg_s * 1e3,
        "dtype": "u4 codes x bf16 -> fp32 acc",
        "config": {"workload": "qmv-config0", "n": n, "k": k, "bits": bits, "group_size": gs,
                   "rows": m, "mall_rotation_copies": copies},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }


def cpu_baseline_qmv(orc, codes, s, b, k, bits, gs, x, alg_bytes, budget_s=10.0):
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        orc.qmv(codes, s, b, k, bits, gs, x)
        reps += 1
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(alg_bytes / dt / 1e9, 3), "unit": "GB/s", "cores": orc.num_threads(),
            "kind": "port",
            "sample": f"{reps} oracle QMVs of the same config-0 matrix in {budget_s:.0f}s (OpenMP)"}


WORKLOADS = {"qmv-config0": bench_qmv_config0}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="qmv-config0", choices=sorted(WORKLOADS))
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); multi-GPU runs are "
              "not part of this build", file=sys.stderr)
        raise SystemExit(2)
    from conftest import load_mx

    mx = load_mx()
    res = WORKLOADS[args.workload](mx, args)
    out = {
        "metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": res["dtype"], "data": "synthetic (seeded counter-based generator)",
        "config": res["config"], "roofline": res["roofline"], "cpu_baseline": res["cpu_baseline"],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
