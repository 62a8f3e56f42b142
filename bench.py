"""Benchmark driver (one JSON line on stdout, progress on stderr).

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]

Workloads:
  config3-b8-decode (default)  benchmark config 3: the full synthetic hybrid
      model (48 layers, 3:1 GatedDeltaNet : gated attention, 512-expert top-10
      MoE with a shared expert, hc = 4 hyper-connections, vocab 151936, 4-bit
      weights with 5-bit expert down and 8-bit embedding/head), 8 slots
      prefilled with seeded uniform-random prompts of ragged lengths 10..2048
      (512-token chunks on the matrix cores; --block-prefill: the exact
      eight-token blocks), then batched greedy decode of all 8 rows per step (rows at their own
      offsets).  A step = one decode token for each of the 8 rows; W + K = 256
      steps per row by default.  value = aggregate tok/s over the K timed steps.
  qmv-config0  benchmark config 0: one affine 4-bit g64 QMV [4096, 2048] per
      step, rotating >= 2 GiB of weight copies so the 256 MB Infinity Cache
      cannot serve repeats; value = achieved GB/s.
  gdn-prefill-config1  benchmark config 1 prefill: the chunked GatedDeltaNet
      scan over T = 2048 tokens of one sequence (16 key / 32 value heads, head
      dim 128, config-1 inputs); a step = one whole scan (prep + chunk walk);
      value = tokens/s.  Roofline: fp32 matrix-core FLOPs of the chunked
      algorithm per scan over the scan time (MI355X fp32 MFMA 157.3 TFLOP/s);
      the sequential GPU scan (mx_gdn_scan) is timed beside it.
  gdn-decode-config1  benchmark config 1 decode: one fast-mode GatedDeltaNet
      step (mx_gdn_recurrence_fast) at B = 1, 2, 4, 8 rows over a rotated 1 GiB
      fp32 state arena; value = B = 8 rows per second, roofline = state and
      q/k/v/y bytes over the step time.
  moe-config2  benchmark config 2: the decode MoE sublayer (router projection,
      routing, gathered expert gate/up and down, slot sum into the residual
      streams) at B = 1..8 rows; 32 rotated input batches; value = B = 8 rows
      per second, roofline = router + shared + distinct experts' bytes.
  prefill-config3  chunked prefill of one 2048-token prompt on the config-3
      model (512-token chunks on the matrix cores); value = prompt tokens/s.
  mtp-config4  benchmark config 4: MTP speculative generation (depth 3) on the
      mixed-width config-3 model, batch 1, 4096-token prompt, 256 tokens, timed
      against plain greedy decoding of the same prompt.

Timing: the decode loop is bracketed by device synchronisation (the engine
synchronises once per step to read the tokens, as the reference's eval does).
Config 3 times the exact mode by default: the exact-integer kernels, whose
tokens, routing and every layer output equal the CPU oracle's bit for bit
(tests/test_config3_gpu.py).  `--fast` times the bf16 matrix-core mode
instead; the other mode is always timed beside the headline one.
The roofline object is the MoE expert gate/up kernel (the step's dominant
kernel), in the form the step launches: algorithmic bytes (distinct experts'
weights + the shared expert) over its duration, from HIP events on the
engine's stream around the 48 layers' gate/up launches run back to back on
the routing of the last step (each launch reads its own layer's weights from
HBM).  `traffic` is the measured HBM bytes per launch from the committed
rocprofv3 counter summary of that kernel
(profiles/config3-b8-decode-exact_hbm-traffic.md, or
profiles/config3-b8-decode_hbm-traffic.md for --fast).
The CPU baseline is the C oracle (oracle/, a restatement of the reference
arithmetic) timed on this host: for config 3, one whole batch-8 step on the
engine's weights and caches, whose next tokens must equal the exact engine's
for the same step; for the component workloads, a bounded sample.
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

HBM_PEAK_GBS = 8000.0
METRIC = "batch-8 decode tok/s (aggregate) + QMV/MoE achieved HBM GB/s vs 8 TB/s peak"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def to_bf16(x) -> np.ndarray:
    """float32 -> bf16 bits, round to nearest even (synthetic inputs)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def load_package():
    """Import rust-mlx_amd (a hyphenated directory) as module rust_mlx_amd."""
    import importlib.util

    if "rust_mlx_amd" in sys.modules:
        return sys.modules["rust_mlx_amd"]
    spec = importlib.util.spec_from_file_location(
        "rust_mlx_amd", os.path.join(ROOT, "rust-mlx_amd", "__init__.py"))
    mod = importlib.util.module_from_spec(spec)
    sys.modules["rust_mlx_amd"] = mod
    spec.loader.exec_module(mod)
    return mod


# --------------------------------------------------------------- config 3 --
def bench_config3(mx, args):
    cfg = dict(mx.CONFIG3)
    cfg["max_context"] = 2048 + args.warmup + args.steps + 16
    rows = 8
    t0 = time.perf_counter()
    eng = mx.Engine(cfg)
    exact = not args.fast
    eng.set_flags(eager=args.eager, exact=exact)
    log(f"config3: engine built in {time.perf_counter() - t0:.1f}s "
        f"({cfg['layers']} layers, {cfg['experts']} experts)")
    rng = np.random.default_rng(3000)
    lengths = rng.integers(10, 2049, rows)
    nxt = np.zeros(rows, np.uint32)
    t0 = time.perf_counter()
    for s in range(rows):
        prompt = rng.integers(0, cfg["vocab"], lengths[s])
        if args.synthetic_context:
            eng.fill_slot(s, int(lengths[s]), seed=4000 + s)
            nxt[s] = prompt[-1]
        else:
            nxt[s] = eng.prefill(s, prompt, chunked=not args.block_prefill)
    prefill_s = time.perf_counter() - t0
    prefill_mode = ("synthetic" if args.synthetic_context else
                    "exact 8-token blocks" if args.block_prefill else f"{mx.PREFILL_CHUNK}-token chunks")
    log(f"config3: {'filled' if args.synthetic_context else 'prefilled'} {int(lengths.sum())} "
        f"context positions (lengths {[int(x) for x in lengths]}) in {prefill_s:.2f}s "
        f"({prefill_mode}, {lengths.sum() / prefill_s:.0f} positions/s)")
    slots = list(range(rows))
    toks = nxt
    # one profiled (eager, instrumented) step: expert-kernel timing and bytes
    toks, prof = eng.profile_step(slots, toks)
    for _ in range(max(args.warmup - 1, 0)):
        toks = eng.decode_batch(slots, toks, equal=False)
    mx.check(mx.lib.mx_device_sync())
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks = eng.decode_batch(slots, toks, equal=False)
    mx.check(mx.lib.mx_device_sync())
    dt = time.perf_counter() - t0
    tok_s = rows * args.steps / dt
    ms_step = dt / args.steps * 1e3
    log(f"config3: {args.steps} steps x {rows} rows in {dt:.3f}s -> {tok_s:.1f} tok/s, "
        f"{ms_step:.3f} ms/step")
    # the other mode timed the same way on the same rows (exact: the
    # exact-integer kernels the CPU oracle reproduces bit for bit; fast: the
    # bf16 matrix-core kernels, within tolerance of it)
    exact_steps = max(args.steps // 4, 4)
    eng.set_flags(exact=not exact, eager=args.eager)
    for _ in range(2):
        toks = eng.decode_batch(slots, toks, equal=False)
    mx.check(mx.lib.mx_device_sync())
    t0 = time.perf_counter()
    for _ in range(exact_steps):
        toks = eng.decode_batch(slots, toks, equal=False)
    mx.check(mx.lib.mx_device_sync())
    other_dt = (time.perf_counter() - t0) / exact_steps
    other_tok_s = rows / other_dt
    eng.set_flags(exact=exact, eager=args.eager)
    log(f"config3: {'fast' if exact else 'exact'} mode {exact_steps} steps: "
        f"{other_tok_s:.1f} tok/s, {other_dt * 1e3:.3f} ms/step")
    # the reference's batching policy (src/bin/server/batch.rs:274-289): only
    # rows at equal offsets share a decode step (mx_engine_decode_batch); the
    # ragged rows here all differ, so each row steps alone
    toks = np.asarray(toks, np.uint32).copy()
    groups = {}
    for i, s_ in enumerate(slots):
        groups.setdefault(eng.offset(s_), []).append(i)
    ref_steps = max(args.steps // 8, 4)
    for _ in range(2):
        for idx in groups.values():
            toks[idx] = eng.decode_batch([slots[i] for i in idx], toks[idx], equal=True)
    mx.check(mx.lib.mx_device_sync())
    t0 = time.perf_counter()
    for _ in range(ref_steps):
        for idx in groups.values():
            toks[idx] = eng.decode_batch([slots[i] for i in idx], toks[idx], equal=True)
    mx.check(mx.lib.mx_device_sync())
    ref_tok_s = rows * ref_steps / (time.perf_counter() - t0)
    log(f"config3: reference batching policy ({len(groups)} equal-offset groups per step): "
        f"{ref_tok_s:.1f} tok/s over {ref_steps} steps")
    # a second profiled step after the timed loop (longer contexts), then the
    # expert kernels of all 48 layers back to back on that step's routing
    _, prof2 = eng.profile_step(slots, toks)
    reps = [eng.time_experts(rows) for _ in range(EXPERT_REPS)]
    et = dict(reps[0])
    et["gate_up_ms"] = sum(r["gate_up_ms"] for r in reps) / len(reps)
    et["down_ms"] = sum(r["down_ms"] for r in reps) / len(reps)
    gu_gbs = et["gate_up_bytes"] / (et["gate_up_ms"] * 1e-3) / 1e9
    dn_gbs = et["down_bytes"] / (et["down_ms"] * 1e-3) / 1e9
    layers = prof["layers"]
    gu_us = et["gate_up_ms"] / et["launches"] * 1e3
    gu_launch_bytes = et["gate_up_bytes"] / et["launches"]
    step_bytes = prof2["step_bytes"]
    step_frac = step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS
    log(f"config3: expert gate/up {gu_gbs:.0f} GB/s ({gu_us:.1f} us/launch avg), "
        f"down {dn_gbs:.0f} GB/s; distinct experts/layer {prof2['distinct_experts'] / layers:.1f}; "
        f"step bytes {step_bytes / 1e9:.2f} GB -> {step_frac * 100:.1f}% of HBM roofline per step")
    positions = [eng.offset(s) for s in slots]
    cpu = None
    if not args.no_cpu_baseline:
        cpu, cpu_next = cpu_baseline_config3(mx, eng, cfg, slots, toks, positions)
        # the engine's own step on the same rows, tokens and caches
        eng_next = np.asarray(eng.decode_batch(slots, toks, equal=False), np.uint32)
        same = bool((np.asarray(cpu_next, np.uint32).reshape(-1)[:rows] == eng_next).all())
        log(f"cpu baseline: oracle next tokens {'equal' if same else 'DIFFER FROM'} the engine's")
        if exact and not same:
            raise SystemExit("bench: the oracle's step and the exact engine step disagree")
        cpu["tokens_equal_engine"] = same
    eng.close()
    return {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "ms_per_step": ms_step,
        "dtype": step_dtype(exact, "u4/u5/u8"),
        "config": {
            "workload": "config3-b8-decode", "model": "synthetic hybrid GDN/attention MoE",
            "layers": cfg["layers"], "hidden": cfg["hidden"], "experts": cfg["experts"],
            "top_k": cfg["top_k"], "vocab": cfg["vocab"], "global_batch": rows,
            "prompt_lengths": [int(x) for x in lengths], "parallelism": "single GPU",
            "rows_at_own_offsets": True,
            "step_bytes_gb": round(step_bytes / 1e9, 3),
            "step_hbm_roofline_frac": round(step_frac, 4),
            "distinct_experts_per_layer": round(prof2["distinct_experts"] / layers, 2),
            "expert_down_gbs": round(dn_gbs, 1),
            "prefill_s": round(prefill_s, 2),
            "prefill_positions": int(lengths.sum()),
            "context": "synthetic" if args.synthetic_context else "prefilled",
            "prefill": prefill_mode,
            "mode": "exact" if exact else "fast",
            ("fast_tok_s" if exact else "exact_tok_s"): round(other_tok_s, 2),
            "reference_policy_tok_s": round(ref_tok_s, 2),
            "reference_policy_groups": len(groups),
        },
        "roofline": {"bound": "hbm",
                     "kernel": (("xq_gate_up_kernel<4, 16, 3, true> (exact-integer expert gate/up + "
                                 "SwiGLU over the plan's work items, the form the step launches)")
                                if exact else
                                ("gate_up_persist_kernel<4, 16, 4, 2, 0> (route-taking form; the "
                                 "step launches the self-routing <4, 16, 4, 2, 8>)")) +
                               f"; timing: HIP events on the engine stream around the {layers} "
                               f"layers' launches run back to back on the last step's routing, "
                               f"mean of {EXPERT_REPS} such runs, divided by {layers}",
                     "achieved": round(gu_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": measured_traffic("config3-b8-decode-exact_hbm-traffic.md" if exact
                                                 else "config3-b8-decode_hbm-traffic.md"),
                     "algorithmic_bytes_per_launch": int(gu_launch_bytes),
                     "us_per_launch": round(gu_us, 2)},
        "cpu_baseline": cpu,
    }


# back-to-back runs of the 48 expert gate/up (and down) launches averaged for
# the roofline figure
EXPERT_REPS = 4


def step_dtype(exact: bool, widths: str) -> str:
    """The arithmetic the timed step computes in, by mode."""
    if exact:
        return (f"affine {widths} codes; bf16 activations as exact integers on a per-group grid "
                "(int8 matrix-core digits, exact int32 sums), fp64 group combination, one fp32 "
                "rounding; fp32 GDN state")
    return (f"affine {widths} codes x bf16 matrix-core products -> fp32 sums; bf16 activations; "
            "fp32 GDN state")


def measured_traffic(summary: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3
    counter summary (FETCH_SIZE + WRITE_SIZE, copy-calibrated), or None."""
    path = os.path.join(ROOT, "profiles", summary)
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch ="):
            return int(line.split("=")[1])
    return None


def cpu_baseline_config3(mx, eng, cfg, slots, toks, positions):
    """The oracle runs one whole batch-8 decode step (all layers, the mixer and
    the head, the engine's weights and caches read back from the device) at
    the rows' real positions, and its next tokens are checked against the
    engine's for the same step."""
    from oracle.model import Model
    from oracle import oracle as orc

    def fetch(name, dtype, shape):
        return eng.read(name, dtype, shape)

    t0 = time.perf_counter()
    model = Model(cfg, fetch)
    # the engine's caches (the oracle keeps them in the same layout)
    model.state[...] = eng.read("cache.gdn_state", np.float32, model.state.shape)
    model.conv[...] = eng.read("cache.conv_state", np.uint16, model.conv.shape)
    model.k[...] = eng.read("cache.k", np.uint16, model.k.shape)
    model.v[...] = eng.read("cache.v", np.uint16, model.v.shape)
    log(f"cpu baseline: fetched {cfg['layers']} layers and the caches in "
        f"{time.perf_counter() - t0:.1f}s")
    for s, p in zip(slots, positions):
        model.offsets[s] = p
    t0 = time.perf_counter()
    nxt = model.decode_rows(slots, list(toks))
    step_s = time.perf_counter() - t0
    tok_s = len(slots) / step_s
    log(f"cpu baseline: one step {step_s:.1f}s -> {tok_s:.4f} tok/s")
    del model
    return {"value": round(tok_s, 5), "unit": "tok/s", "cores": orc.num_threads(), "kind": "port",
            "sample": f"one whole batch-8 decode step ({cfg['layers']} layers + mixer + head) "
                      f"= {step_s:.1f}s"}, nxt


# ---------------------------------------------------------------- config 0 --
def qweight_bytes(n: int, k: int, bits: int, gs: int) -> int:
    return n * k * bits // 8 + 4 * n * (k // gs)


def bench_qmv_config0(mx, args):
    """Config 0: one affine 4-bit g64 QMV [4096, 2048] x 1 row per step, over
    rotated weight copies.  Headline: the exact-integer kernel (mx_xq, the
    engine's exact mode, bit-exact with the oracle's mxo_xq); the fixed-order
    VALU kernel (mx_qmv, bit-exact with the oracle's mxo_qmv) and the bf16
    matrix-core kernel (mx_qmm) are timed beside it."""
    n, k, bits, gs, m = 4096, 2048, 4, 64, 1
    wbytes = qweight_bytes(n, k, bits, gs)
    alg_bytes = wbytes + 2 * m * k + 2 * m * n
    copies = max(2, int(np.ceil(2 * 1024**3 / wbytes)))
    log(f"qmv-config0: {copies} weight copies ({copies * wbytes / 1e9:.2f} GB) for MALL rotation")
    ws = [mx.QWeight.random(n, k, bits, gs, seed=100 + 17 * i) for i in range(copies)]
    x = mx.DeviceArray((m, k), np.uint16)
    mx.fill_bf16(x, 101, 1, 1.0, 0.0)
    ys = {name: mx.DeviceArray((m, n), np.uint16) for name in ("xq", "qmv", "qmm")}
    stream = C.c_void_p()
    mx.check(mx.lib.mx_stream_create(C.byref(stream)))
    qcs = [w.c() for w in ws]
    fns = {"xq": mx.lib.mx_xq, "qmv": mx.lib.mx_qmv, "qmm": mx.lib.mx_qmm}
    per = {}
    for name, fn in fns.items():
        y = ys[name]

        def launch(i, fn=fn, y=y):
            mx.check(fn(C.byref(qcs[i % copies]), x.ptr, m, y.ptr, stream))

        for i in range(args.warmup):
            launch(i)
        mx.check(mx.lib.mx_stream_sync(stream))
        sec = timed_launches(mx, stream, lambda i: launch(args.warmup + i), args.steps)
        per[name] = {"us": round(sec * 1e6, 3), "gbs": round(alg_bytes / sec / 1e9, 2)}
        log(f"qmv-config0: {name} {sec * 1e6:.2f} us/launch (events), "
            f"{alg_bytes / sec / 1e9:.0f} GB/s")
    avg_s = per["xq"]["us"] * 1e-6
    achieved = alg_bytes / avg_s / 1e9
    cpu = None
    if not args.no_cpu_baseline:
        # CPU baseline leg: the oracle checks each kernel's last launch bit for
        # bit, then repeats the exact-integer QMV for about 10 s
        from oracle import oracle as orc

        seed = 100 + 17 * ((args.warmup + args.steps - 1) % copies)
        codes, s, b = orc.random_qweight(n, k, bits, gs, seed=seed)
        xh = x.numpy()
        if not (ys["xq"].numpy() == orc.f32_to_bf16(orc.xq(codes, s, b, k, bits, xh))).all():
            raise SystemExit("bench: exact-integer QMV differs from the oracle")
        if not (ys["qmv"].numpy() == orc.qmv(codes, s, b, k, bits, gs, xh)).all():
            raise SystemExit("bench: fixed-order QMV differs from the oracle")
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            orc.xq(codes, s, b, k, bits, xh)
            reps += 1
        cpu_dt = (time.perf_counter() - t0) / reps
        cpu = {"value": round(alg_bytes / cpu_dt / 1e9, 3), "unit": "GB/s",
               "cores": orc.num_threads(), "kind": "port",
               "sample": f"{reps} oracle exact-integer QMVs of the config-0 matrix in 10s"}
    return {
        "metric": METRIC, "value": round(achieved, 2), "unit": "GB/s", "ms_per_step": avg_s * 1e3,
        "dtype": "u4 codes x bf16 activations on a per-group integer grid -> exact int32 sums, "
                 "fp64 group combination",
        "config": {"workload": "qmv-config0", "n": n, "k": k, "bits": bits, "group_size": gs,
                   "rows": m, "mall_rotation_copies": copies, "kernels": per},
        "roofline": {"bound": "hbm", "kernel": "xq_dense_kernel (mx_xq, exact-integer)",
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": cpu,
    }


# --------------------------------------------------------------- config 1 --
FP32_MFMA_PEAK_TFLOPS = 157.3


def prefill_flops(t: int, hv: int) -> float:
    """fp32-equivalent FLOPs of the chunked scan per sequence: per 64-token
    chunk and value head, K K^T and Q K^T (2 x 64x64x128), W and U (2 x
    64x64x128), D = U - W S and (gamma Q) S (2 x 64x128x128), P D (64x64x128)
    and K'^T D (128x64x128), 2 FLOPs per multiply-add."""
    c, d = 64, 128
    per_chunk = 2 * (2 * c * c * d + 2 * c * c * d + 2 * c * d * d + c * c * d + d * c * d)
    return per_chunk * ((t + c - 1) // c) * hv


def gdn_config1_inputs(rows, hk, hv, seed):
    """Config-1 style scan inputs: L2-normalised q, k; beta = sigmoid(N(0,1));
    g = exp(-softplus(N(0,1)) * A) with A ~ U(0, 16) per head."""
    rng = np.random.default_rng(seed)

    def l2n(x):
        return x / np.linalg.norm(x, axis=-1, keepdims=True)

    q = to_bf16(l2n(rng.standard_normal((rows, hk, 128))).astype(np.float32))
    k = to_bf16(l2n(rng.standard_normal((rows, hk, 128))).astype(np.float32))
    v = to_bf16(rng.standard_normal((rows, hv, 128)).astype(np.float32))
    beta = to_bf16((1 / (1 + np.exp(-rng.standard_normal((rows, hv))))).astype(np.float32))
    A = rng.uniform(0, 16, hv)
    g = np.exp(-np.log1p(np.exp(rng.standard_normal((rows, hv)))) * A).astype(np.float32)
    return q, k, v, g, beta


def bench_gdn_prefill_config1(mx, args):
    hk, hv, t = 16, 32, 2048
    q, k, v, g, beta = gdn_config1_inputs(t, hk, hv, 2048)
    state0 = np.zeros((1, hv, 128, 128), np.float32)
    slots = np.zeros(1, np.int32)
    dims = mx.GdnDimsC(hk, hv, 128, 128, 4)
    dq, dk, dv_, dg, db, dsl, dst = (mx.DeviceArray.from_numpy(np.ascontiguousarray(a))
                                     for a in (q, k, v, g, beta, slots, state0))
    y = mx.DeviceArray((t, hv, 128), np.uint16)
    ws = mx.DeviceArray((mx.lib.mx_gdn_prefill_workspace_bytes(1, hv, t),), np.uint8)
    stream = C.c_void_p()
    mx.check(mx.lib.mx_stream_create(C.byref(stream)))

    def chunked():
        mx.check(mx.lib.mx_gdn_prefill_chunked(dq.ptr, dk.ptr, dv_.ptr, dg.ptr, db.ptr,
                                               C.byref(dims), 1, t, dsl.ptr, dst.ptr, y.ptr,
                                               ws.ptr, stream))

    def sequential():
        mx.check(mx.lib.mx_gdn_scan(dq.ptr, dk.ptr, dv_.ptr, dg.ptr, db.ptr, C.byref(dims), 1, t,
                                    dsl.ptr, dst.ptr, None, y.ptr, stream))

    def timed(fn, n):
        e0, e1 = C.c_void_p(), C.c_void_p()
        mx.check(mx.lib.mx_event_create(C.byref(e0)))
        mx.check(mx.lib.mx_event_create(C.byref(e1)))
        mx.check(mx.lib.mx_device_sync())
        mx.check(mx.lib.mx_event_record(e0, stream))
        for _ in range(n):
            fn()
        mx.check(mx.lib.mx_event_record(e1, stream))
        ms = C.c_float()
        mx.check(mx.lib.mx_stream_sync(stream))
        mx.check(mx.lib.mx_event_elapsed_ms(e0, e1, C.byref(ms)))
        return ms.value / 1e3 / n

    chunked()
    mx.check(mx.lib.mx_stream_sync(stream))
    err = cpu = None
    if not args.no_cpu_baseline:
        # CPU baseline leg: one sequential oracle scan of the same input,
        # timed, and the checker of the first chunked scan's state
        from oracle import oracle as orc

        t0 = time.perf_counter()
        y_w, st_w, _ = orc.gdn_scan(q, k, v, g, beta, hk, hv, 1, t, slots, state0)
        cpu_s = time.perf_counter() - t0
        err = float(np.abs(dst.numpy() - st_w).max() / np.abs(st_w).max())
        log(f"gdn-prefill-config1: state max rel err vs oracle {err:.2e}; oracle (sequential, "
            f"{orc.num_threads()} threads) {cpu_s:.2f} s")
        if err > 1e-4:
            raise SystemExit("bench: chunked prefill state differs from the oracle")
        cpu = {"value": round(t / cpu_s, 1), "unit": "tok/s", "cores": orc.num_threads(),
               "kind": "port", "sample": f"one sequential oracle scan of the same T={t} input "
                                         f"({cpu_s:.2f}s)"}
    for _ in range(args.warmup):
        chunked()
    avg = timed(chunked, args.steps)
    seq = timed(sequential, max(1, min(5, args.steps)))
    flops = prefill_flops(t, hv)
    tflops = flops / avg / 1e12
    log(f"gdn-prefill-config1: chunked {avg * 1e6:.1f} us/scan ({t / avg:.0f} tok/s, "
        f"{tflops:.2f} TFLOP/s); sequential GPU scan {seq * 1e6:.1f} us")
    return {
        "metric": METRIC, "value": round(t / avg, 1), "unit": "tok/s", "ms_per_step": avg * 1e3,
        "dtype": "bf16 q/k/v -> fp32 state, fp32 matrix-core products",
        "config": {"workload": "gdn-prefill-config1", "t": t, "batch": 1, "key_heads": hk,
                   "value_heads": hv, "head_dim": 128, "chunk": 64,
                   "sequential_gpu_scan_us": round(seq * 1e6, 1),
                   "state_rel_err_vs_oracle": None if err is None else float(f"{err:.3e}")},
        "roofline": {"bound": "mfma", "kernel": "chunk_prep_kernel + chunk_scan_kernel",
                     "achieved": round(tflops, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / FP32_MFMA_PEAK_TFLOPS, 4),
                     "traffic": None},
        "cpu_baseline": cpu,
    }


def timed_launches(mx, stream, fn, n):
    """Average seconds per call of fn() over n calls, HIP events on `stream`
    (the stream the kernels are launched on)."""
    e0, e1 = C.c_void_p(), C.c_void_p()
    mx.check(mx.lib.mx_event_create(C.byref(e0)))
    mx.check(mx.lib.mx_event_create(C.byref(e1)))
    mx.check(mx.lib.mx_device_sync())
    mx.check(mx.lib.mx_event_record(e0, stream))
    for i in range(n):
        fn(i)
    mx.check(mx.lib.mx_event_record(e1, stream))
    ms = C.c_float()
    mx.check(mx.lib.mx_stream_sync(stream))
    mx.check(mx.lib.mx_event_elapsed_ms(e0, e1, C.byref(ms)))
    mx.check(mx.lib.mx_event_destroy(e0))
    mx.check(mx.lib.mx_event_destroy(e1))
    return ms.value / 1e3 / n


# per row: fp32 state read + written (2 Hv Dk Dv 4) plus q, k, v (8192 bf16),
# y (4096 bf16), g (32 fp32) and beta (32 bf16)
GDN_DECODE_BYTES_PER_ROW = 2 * 32 * 128 * 128 * 4 + 16384 + 8192 + 128 + 64


def bench_gdn_decode_config1(mx, args):
    """Config 1 decode: one fast-mode GatedDeltaNet step (q/k L2 norm, beta,
    decay, delta rule, gated RMS norm) for B = 1, 2, 4, 8 rows, each row on its
    own slot of a 1 GiB fp32 state arena (rotated so the 256 MB last-level cache
    cannot serve repeats).  `value` is the B = 8 step's rows per second."""
    hk, hv, d = 16, 32, 128
    slots_n = 512  # 2 MiB of state per slot
    dims = mx.GdnDimsC(hk, hv, d, d, 4)
    rng = np.random.default_rng(1001)
    rows_max = 8
    conv = to_bf16(rng.standard_normal((rows_max, 2 * hk * d + hv * d)).astype(np.float32))
    z = to_bf16(rng.standard_normal((rows_max, hv * d)).astype(np.float32))
    a = to_bf16(rng.standard_normal((rows_max, hv)).astype(np.float32))
    b = to_bf16(rng.standard_normal((rows_max, hv)).astype(np.float32))
    a_log = np.log(rng.uniform(1e-3, 16, hv)).astype(np.float32)  # A ~ U(0, 16)
    dt = to_bf16(rng.uniform(-1, 1, hv).astype(np.float32))
    norm_w = to_bf16(rng.uniform(0.5, 1.5, d).astype(np.float32))
    eps = 1e-6
    zab = np.ascontiguousarray(np.concatenate([z, a, b], axis=1))
    dconv, dzab = mx.DeviceArray.from_numpy(conv), mx.DeviceArray.from_numpy(zab)
    dal, ddt, dnw = (mx.DeviceArray.from_numpy(v) for v in (a_log, dt, norm_w))
    state = mx.DeviceArray((slots_n, hv, d, d), np.float32, zero=True)
    lists = np.arange(slots_n * rows_max, dtype=np.int32).reshape(-1, rows_max) % slots_n
    dlists = mx.DeviceArray.from_numpy(np.ascontiguousarray(lists))
    y = mx.DeviceArray((rows_max, hv * d), np.uint16)
    stream = C.c_void_p()
    mx.check(mx.lib.mx_stream_create(C.byref(stream)))
    zp = dzab.ptr

    def launch(rows, i):
        lst = dlists.ptr + 4 * rows * (i % (slots_n // rows))  # `rows` consecutive slots
        mx.check(mx.lib.mx_gdn_recurrence_fast(dconv.ptr, conv.shape[1], zp, zp + 2 * hv * d,
                                               zp + 2 * (hv * d + hv), zab.shape[1], dal.ptr,
                                               ddt.ptr, dnw.ptr, eps, C.byref(dims), rows, 1,
                                               lst, state.ptr, None, y.ptr, stream))

    # one B = 8 step from the zero state: the CPU baseline leg checks it
    launch(rows_max, 0)
    mx.check(mx.lib.mx_stream_sync(stream))
    got_st = np.empty((rows_max, hv, d, d), np.float32)
    mx.check(mx.lib.mx_memcpy_dtoh(got_st.ctypes.data, state.ptr, got_st.nbytes))
    got_y = bf16_to_f32(y.numpy()).astype(np.float64)
    per_b = {}
    for rows in (1, 2, 4, 8):
        for i in range(args.warmup):
            launch(rows, i)
        sec = timed_launches(mx, stream, lambda i, r=rows: launch(r, args.warmup + i), args.steps)
        gbs = rows * GDN_DECODE_BYTES_PER_ROW / sec / 1e9
        per_b[rows] = {"us": round(sec * 1e6, 2), "rows_per_s": round(rows / sec, 1),
                       "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"gdn-decode-config1: B={rows} {sec * 1e6:.2f} us/step, {gbs:.0f} GB/s")
    b8 = per_b[8]
    cpu = st_err = None
    if not args.no_cpu_baseline:
        # CPU baseline leg: the oracle's B = 8 step from the zero state checks
        # the GPU's first step, then repeats for about 10 s
        from oracle import oracle as orc

        st0 = np.zeros((rows_max, hv, d, d), np.float32)
        sl = np.arange(rows_max, dtype=np.int32)
        t0 = time.perf_counter()
        y_w, st_w, _ = orc.gdn_recurrence(conv, z, a, b, a_log, dt, norm_w, eps, hk, hv, rows_max,
                                          1, sl, st0)
        cpu_once = time.perf_counter() - t0
        st_err = float(np.abs(got_st - st_w).max() / np.abs(st_w).max())
        want_y = bf16_to_f32(y_w).astype(np.float64)
        y_ok = bool(np.all(np.abs(got_y - want_y) <= 2e-2 * np.abs(want_y) + 1e-2))
        log(f"gdn-decode-config1: B=8 state max rel err vs oracle {st_err:.2e}, "
            f"y within tolerance {y_ok}")
        if st_err > 1e-4 or not y_ok:
            raise SystemExit("bench: GDN decode step differs from the oracle")
        reps, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < 10.0:
            orc.gdn_recurrence(conv, z, a, b, a_log, dt, norm_w, eps, hk, hv, rows_max, 1, sl, st0)
            reps += 1
        cpu_dt = (time.perf_counter() - t0) / reps
        cpu = {"value": round(rows_max / cpu_dt, 2), "unit": "tok/s", "cores": orc.num_threads(),
               "kind": "port", "sample": f"{reps} oracle B=8 steps in 10s (first {cpu_once:.3f}s)"}
    return {
        "metric": METRIC, "value": b8["rows_per_s"], "unit": "tok/s (rows stepped per second)",
        "ms_per_step": b8["us"] / 1e3,
        "dtype": "bf16 q/k/v/z -> fp32 state and arithmetic",
        "config": {"workload": "gdn-decode-config1", "key_heads": hk, "value_heads": hv,
                   "head_dim": d, "state_slots_rotated": slots_n,
                   "per_batch": {str(k): v for k, v in per_b.items()},
                   "state_rel_err_vs_oracle": None if st_err is None else float(f"{st_err:.3e}")},
        "roofline": {"bound": "hbm", "kernel": "recurrence_fast_kernel (B=8)",
                     "achieved": b8["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": b8["frac"], "traffic": None,
                     "algorithmic_bytes_per_launch": 8 * GDN_DECODE_BYTES_PER_ROW},
        "cpu_baseline": cpu,
    }


def bench_moe_config2(mx, args):
    """Config 2: the sparse MoE block at decode for B = 1..8 rows: the router
    projection (512 experts + the shared-expert gate, 4-bit), routing (softmax,
    top-10, renormalisation) inside the expert gate/up kernel, the 4-bit
    gate/up and 5-bit down projections of the selected and shared experts, and
    the slot sum written into 4 residual streams (the decode step's MoE
    sublayer).  32 input batches rotate so that consecutive calls select
    different experts.  Bytes per call: router + shared expert + U distinct
    experts x (2 q(512,2048,4) + q(2048,512,5)), U counted per input batch."""
    E, H, I, k = 512, 2048, 512, 10
    n_x = 32
    gate = mx.QBank.random(E, I, H, 4, 64, 2001)
    up = mx.QBank.random(E, I, H, 4, 64, 2002)
    down = mx.QBank.random(E, H, I, 5, 64, 2003)
    sg = mx.QWeight.random(I, H, 4, 64, 2004)
    su = mx.QWeight.random(I, H, 4, 64, 2005)
    sd = mx.QWeight.random(H, I, 5, 64, 2006)
    router = mx.QWeight.random(E + 1, H, 4, 64, 2007)
    dx = mx.DeviceArray((n_x, 8, H), np.uint16)
    dres = mx.DeviceArray((8, 4, H), np.uint16)
    dhg = mx.DeviceArray((8, 4), np.uint16)
    for arr, seed, base in ((dx, 2008, 0.0), (dres, 2009, 0.0), (dhg, 2010, 1.0)):
        mx.fill_bf16(arr, seed, 1, 1.0, base)
    logits = mx.DeviceArray((8, E + 1), np.uint16)
    ids = mx.DeviceArray((8, k), np.uint32)
    sc = mx.DeviceArray((8, k), np.uint16)
    fa = mx.DeviceArray((8,), np.uint16)
    ws = mx.DeviceArray((mx.lib.mx_moe_workspace_bytes(8, 16, I),), np.uint8)
    qb = [bk.c() for bk in (gate, up, down)]
    qs = [w.c() for w in (sg, su, sd)]
    rc = router.c()
    stream = C.c_void_p()
    mx.check(mx.lib.mx_stream_create(C.byref(stream)))

    def launch(rows, i):
        xp = dx.ptr + 2 * 8 * H * (i % n_x)
        mx.check(mx.lib.mx_qmm(C.byref(rc), xp, rows, logits.ptr, stream))
        mx.check(mx.lib.mx_moe_routed_experts_hc_mfma(
            logits.ptr, E + 1, logits.ptr + 2 * E, E + 1, E, xp, rows, k, 4, C.byref(qb[0]),
            C.byref(qb[1]), C.byref(qb[2]), C.byref(qs[0]), C.byref(qs[1]), C.byref(qs[2]),
            ws.ptr, ids.ptr, sc.ptr, fa.ptr, dhg.ptr, dres.ptr, stream))

    ex_bytes = 2 * qweight_bytes(I, H, 4, 64) + qweight_bytes(H, I, 5, 64)
    fixed_bytes = qweight_bytes(E + 1, H, 4, 64) + ex_bytes  # router + shared expert
    # one B = 8 block whose routing the CPU baseline leg checks; then the
    # distinct experts of every input batch
    launch(8, 0)
    mx.check(mx.lib.mx_stream_sync(stream))
    first = (logits.numpy(), ids.numpy(), sc.numpy(), fa.numpy())
    per_b = {}
    for rows in range(1, 9):
        distinct = []
        for i in range(n_x):
            launch(rows, i)
            mx.check(mx.lib.mx_stream_sync(stream))
            distinct.append(len(np.unique(ids.numpy()[:rows])))
        u = float(np.mean(distinct))
        for i in range(args.warmup):
            launch(rows, i)
        sec = timed_launches(mx, stream, lambda i, r=rows: launch(r, args.warmup + i), args.steps)
        alg = fixed_bytes + u * ex_bytes
        gbs = alg / sec / 1e9
        per_b[rows] = {"us": round(sec * 1e6, 2), "distinct_experts": round(u, 2),
                       "bytes": int(alg), "gbs": round(gbs, 1),
                       "frac": round(gbs / HBM_PEAK_GBS, 4), "rows_per_s": round(rows / sec, 1)}
        log(f"moe-config2: B={rows} {sec * 1e6:.2f} us/block, U={u:.1f}, {gbs:.0f} GB/s")
    b8 = per_b[8]
    cpu = None if args.no_cpu_baseline else moe_cpu_baseline(gate, up, down, sg, su, sd, router,
                                                             dx.numpy(), first)
    return {
        "metric": METRIC, "value": b8["rows_per_s"], "unit": "tok/s (rows per second)",
        "ms_per_step": b8["us"] / 1e3,
        "dtype": "affine u4 (gate/up, router) / u5 (down) codes x bf16 matrix-core products "
                 "-> fp32 sums (fast mode)",
        "config": {"workload": "moe-config2", "experts": E, "top_k": k, "hidden": H,
                   "inter": I, "shared_inter": I, "rotated_input_batches": n_x,
                   "per_batch": {str(b_): v for b_, v in per_b.items()}},
        "roofline": {"bound": "hbm",
                     "kernel": "router dense_kernel + gate_up_persist_kernel + down_hc_kernel (B=8)",
                     "achieved": b8["gbs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": b8["frac"], "traffic": None,
                     "algorithmic_bytes_per_launch": b8["bytes"]},
        "cpu_baseline": cpu,
    }


def moe_cpu_baseline(gate, up, down, sg, su, sd, router, xs, first):
    """The oracle's B = 8 MoE block (router QMV, route, experts, slot sum),
    repeated for about 10 s on this host, after it checks the routing of the
    GPU's first block (`first`: its router logits, ids, scores and shared
    factors) bit for bit."""
    from oracle import oracle as orc

    E, H, k = gate.experts, gate.k, 10
    lg, ids_g, sc_g, fa_g = first
    ids_w, sc_w, fa_w = orc.moe_route(lg[:, :E], lg[:, E], k)
    if not ((ids_g == ids_w).all() and (sc_g == sc_w).all() and (fa_g == fa_w).all()):
        raise SystemExit("bench: MoE routing differs from the oracle")
    n_x = xs.shape[0]
    # the oracle's structs view host arrays: keep the arrays alive beside them
    host_b = [bk.host() for bk in (gate, up, down)]
    host_s = [w.host() for w in (sg, su, sd)]
    hb = [orc.qbank(*a, E, bk.n, bk.k, bk.bits, 64) for a, bk in zip(host_b, (gate, up, down))]
    hs = [orc.qw(*a, w.n, w.k, w.bits, 64) for a, w in zip(host_s, (sg, su, sd))]
    rcodes, rs, rb = router.host()
    reps, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < 10.0 or reps == 0:
        x8 = xs[reps % n_x]
        lgc = orc.qmv(rcodes, rs, rb, H, 4, 64, x8)
        i_c, s_c, f_c = orc.moe_route(lgc[:, :E], lgc[:, E], k)
        p = orc.moe_experts(x8, i_c, s_c, k, hb[0], hb[1], hb[2], hs[0], hs[1], hs[2], H)
        orc.moe_reduce(p, k)
        reps += 1
    cpu_dt = (time.perf_counter() - t0) / reps
    return {"value": round(8 / cpu_dt, 2), "unit": "tok/s", "cores": orc.num_threads(),
            "kind": "port", "sample": f"{reps} oracle B=8 MoE blocks (router, route, experts, "
                                      f"slot sum) in {reps * cpu_dt:.1f}s"}


def bench_mtp_config4(mx, args):
    """Config 4: MTP speculative generation on the config-3 model with per-layer
    widths {4,5,6,8} from the seeded schedule and one draft layer: batch 1, a
    4096-token prompt (prefilled in 512-token matrix-core chunks, the draft
    layer's prompt pass too; --block-prefill: exact eight-token blocks), 256
    generated tokens, draft depth 3 (4-token verify
    blocks, greedy acceptance, state and KV rollback).  Timed against plain
    greedy decoding (depth 0) of the same prompt; each figure is the generate
    call minus the same call stopped after its first token (prompt and drafter
    prefill).  Random weights make drafts rarely right: the acceptance rate is
    reported, and the tokens must equal plain greedy decoding's.  Exact mode
    unless --fast."""
    n_tok, ctx, depth = 256, 4096, 3
    cfg = dict(mx.CONFIG3, mixed_bits=1, mtp=1, max_slots=2,
               max_context=ctx + n_tok + 64)
    eng = mx.Engine(cfg)
    exact = not args.fast
    eng.set_flags(exact=exact, eager=args.eager, chunked_generate=not args.block_prefill)
    prompt = np.random.default_rng(4004).integers(0, cfg["vocab"], ctx)
    res = {}
    for d in (0, depth):
        eng.reset(0)
        t0 = time.perf_counter()
        eng.generate(0, prompt, 1, depth=d)
        t_first = time.perf_counter() - t0
        eng.reset(0)
        t0 = time.perf_counter()
        toks, st = eng.generate(0, prompt, n_tok + 1, depth=d)
        t_all = time.perf_counter() - t0
        res[d] = (toks, st, t_all - t_first, t_first)
        log(f"mtp-config4: depth {d}: {n_tok} tokens in {t_all - t_first:.3f}s after a "
            f"{t_first:.2f}s prompt; rounds {st['rounds']}, accepted {st['accepted']}/{st['drafted']}")
    if not (res[0][0] == res[depth][0]).all():
        raise SystemExit("bench: speculative tokens differ from greedy decoding")
    toks, st, dt, t_first = res[depth]
    _, _, dt0, _ = res[0]
    ms_round = dt / max(st["rounds"], 1) * 1e3
    tok_per_round = n_tok / max(st["rounds"], 1)
    # one more verify round at the end of the generated context: the caches
    # as they stand (read by the CPU leg first), one profiled verify block of
    # depth + 1 tokens (its algorithmic bytes), a commit, and the bytes of the
    # round's depth draft-layer steps (depth - 1 drafts before the block and
    # one resynchronisation after it)
    pos = eng.offset(0)
    block = [int(t) for t in toks[-(depth + 1):]]
    cpu_model = None
    if not args.no_cpu_baseline:
        cpu_model = mtp_cpu_model(mx, eng, cfg, pos)
    pred, vprof = eng.profile_verify(0, block)
    eng.commit(0, 1)
    draft_b = eng.draft_bytes(pos)
    round_bytes = vprof["step_bytes"] + depth * draft_b
    gbs = round_bytes / (ms_round * 1e-3) / 1e9
    log(f"mtp-config4: verify block {vprof['step_bytes'] / 1e9:.3f} GB "
        f"({vprof['distinct_experts'] / max(vprof['layers'], 1):.1f} distinct experts/layer), "
        f"draft step {draft_b / 1e9:.3f} GB; round {round_bytes / 1e9:.3f} GB in {ms_round:.3f} ms "
        f"-> {gbs:.0f} GB/s")
    cpu = None
    if cpu_model is not None:
        cpu = mtp_cpu_round(cpu_model, block, pred, depth, tok_per_round, exact)
        del cpu_model
    eng.close()
    return {
        "metric": METRIC, "value": round(n_tok / dt, 2), "unit": "tok/s", "ms_per_step": dt / n_tok * 1e3,
        "dtype": step_dtype(exact, "u4/u5/u6/u8"),
        "config": {"workload": "mtp-config4", "model": "synthetic hybrid GDN/attention MoE, mixed widths",
                   "batch": 1, "context": ctx, "generated": n_tok, "draft_depth": depth,
                   "rounds": st["rounds"], "drafted": st["drafted"], "accepted": st["accepted"],
                   "ms_per_round": round(ms_round, 3),
                   "verify_block_bytes_gb": round(vprof["step_bytes"] / 1e9, 4),
                   "draft_step_bytes_gb": round(draft_b / 1e9, 4),
                   "round_bytes_gb": round(round_bytes / 1e9, 4),
                   "greedy_decode_tok_s": round(n_tok / dt0, 2), "prompt_s": round(t_first, 2),
                   "prompt_prefill": "exact 8-token blocks" if args.block_prefill
                                     else f"{mx.PREFILL_CHUNK}-token chunks",
                   "tokens_equal_greedy": True, "mode": "exact" if exact else "fast"},
        "roofline": {"bound": "hbm",
                     "kernel": f"whole verify round, graph-replayed: one {depth + 1}-token verify "
                               f"block through all {cfg['layers']} layers + {depth} MTP draft-layer "
                               "steps with the greedy head",
                     "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes_per_round": int(round_bytes),
                     "ms_per_round": round(ms_round, 3)},
        "cpu_baseline": cpu,
    }


def mtp_cpu_model(mx, eng, cfg, pos):
    """The oracle model on the engine's weights (mixed widths, the MTP layer)
    and its caches as they stand, slot 0 at position pos."""
    from oracle.model import Model

    t0 = time.perf_counter()
    model = Model(cfg, lambda name, dtype, shape: eng.read(name, dtype, shape))
    model.state[...] = eng.read("cache.gdn_state", np.float32, model.state.shape)
    model.conv[...] = eng.read("cache.conv_state", np.uint16, model.conv.shape)
    model.k[...] = eng.read("cache.k", np.uint16, model.k.shape)
    model.v[...] = eng.read("cache.v", np.uint16, model.v.shape)
    model.offsets[0] = pos
    log(f"cpu baseline: fetched {cfg['layers']} layers + the MTP layer and the caches in "
        f"{time.perf_counter() - t0:.1f}s")
    return model


def mtp_cpu_round(model, block, pred, depth, tok_per_round, exact):
    """One verify round on the CPU oracle: the same verify block as the
    engine's (its predictions must equal the engine's in exact mode), a
    commit, and depth draft-layer steps on the block's hidden streams."""
    from oracle import oracle as orc

    t0 = time.perf_counter()
    cpu_pred = np.asarray(model.verify(0, block), np.uint32)
    hid = model.hidden.copy()
    model.commit(0, 1)
    pos = model.offsets[0]
    for i in range(depth):
        model.mtp_step(0, [block[-1]], pos + i, hid[-1:])
    round_s = time.perf_counter() - t0
    same = bool((cpu_pred == np.asarray(pred, np.uint32)).all())
    log(f"cpu baseline: one verify round {round_s:.1f}s; verify predictions "
        f"{'equal' if same else 'DIFFER FROM'} the engine's")
    if exact and not same:
        raise SystemExit("bench: the oracle's verify block and the exact engine's disagree")
    return {"value": round(tok_per_round / round_s, 5), "unit": "tok/s", "cores": orc.num_threads(),
            "kind": "port", "tokens_equal_engine": same,
            "sample": f"one whole verify round ({len(block)}-token verify block through all layers "
                      f"+ commit + {depth} MTP draft steps) = {round_s:.1f}s, at the engine's "
                      f"{tok_per_round:.2f} tokens per round"}


# ------------------------------------------------------- copy calibration --
COPY_BYTES = 256 << 20


def bench_copy_calibration(mx, args):
    """Device-to-device copies of 256 MiB (the runtime's copy kernel): the
    reference point that scales rocprofv3's FETCH_SIZE / WRITE_SIZE counters to
    bytes (a copy fetches and writes exactly COPY_BYTES)."""
    src = mx.DeviceArray((COPY_BYTES,), np.uint8)
    dst = mx.DeviceArray((COPY_BYTES,), np.uint8)
    stream = C.c_void_p()
    mx.check(mx.lib.mx_stream_create(C.byref(stream)))
    for _ in range(args.warmup):
        mx.check(mx.lib.mx_memcpy_dtod(dst.ptr, src.ptr, COPY_BYTES, stream))
    mx.check(mx.lib.mx_stream_sync(stream))
    t0 = time.perf_counter()
    for _ in range(args.steps):
        mx.check(mx.lib.mx_memcpy_dtod(dst.ptr, src.ptr, COPY_BYTES, stream))
    mx.check(mx.lib.mx_stream_sync(stream))
    dt = (time.perf_counter() - t0) / args.steps
    gbs = 2 * COPY_BYTES / dt / 1e9
    log(f"copy-calibration: {COPY_BYTES >> 20} MiB copy in {dt * 1e6:.1f} us ({gbs:.0f} GB/s read+write)")
    return {"metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "ms_per_step": dt * 1e3,
            "dtype": "u8", "config": {"workload": "copy-calibration", "bytes": COPY_BYTES},
            "roofline": {"bound": "hbm", "kernel": "runtime copy", "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": 2 * COPY_BYTES},
            "cpu_baseline": None}


def model_weight_bytes(eng, cfg):
    """Bytes of every layer weight of the engine (projections, expert banks,
    hyper-connections; not the embedding or the head)."""
    total = 0
    for i in range(cfg["layers"]):
        p = f"layers.{i}"
        mats = [".attn_hc.down", ".attn_hc.up", ".mlp_hc.down", ".mlp_hc.up", ".moe.router",
                ".moe.gate", ".moe.up", ".moe.down", ".moe.shared_gate", ".moe.shared_up",
                ".moe.shared_down"]
        attn = (i % cfg["attn_every"]) == cfg["attn_every"] - 1
        mats += [".attn.in", ".attn.out"] if attn else [".gdn.in", ".gdn.out"]
        for m in mats:
            for part in (".codes", ".scales", ".biases"):
                total += eng.tensor_bytes(p + m + part)
    return total


def bench_prefill_config3(mx, args):
    """Chunked prefill on the config-3 model: a step = one 2048-token prompt of
    one slot through mx_engine_prefill_chunked (four 512-token chunks: the
    projections as matrix-core GEMMs, routes grouped by expert, causal
    attention over each chunk, the GDN layers through the chunked scan).
    value = prompt tokens/s.  Roofline: a chunk of 512 tokens routes 5120
    tokens over 512 experts, so every expert's weights stream once per chunk
    (at least); the bound is every layer weight once per chunk at 8 TB/s.  The
    exact eight-token block prefill (mx_engine_prefill) of 256 tokens is timed
    beside it."""
    cfg = dict(mx.CONFIG3, max_slots=2, max_context=2048 + 64)
    eng = mx.Engine(cfg)
    eng.set_flags(eager=args.eager)
    rng = np.random.default_rng(5005)
    t = 2048
    prompt = rng.integers(0, cfg["vocab"], t)
    for _ in range(max(args.warmup, 1)):
        eng.reset(0)
        eng.prefill(0, prompt[:256], chunked=True)
    mx.check(mx.lib.mx_device_sync())
    t0 = time.perf_counter()
    for _ in range(args.steps):
        eng.reset(0)
        eng.prefill(0, prompt, chunked=True)
    mx.check(mx.lib.mx_device_sync())
    dt = (time.perf_counter() - t0) / args.steps
    tok_s = t / dt
    chunk = mx.PREFILL_CHUNK
    chunks = (t + chunk - 1) // chunk
    wbytes = model_weight_bytes(eng, cfg)
    gbs = wbytes * chunks / dt / 1e9
    block_tok_s = None
    if not args.eager:  # profiled (eager) runs trace the chunked prefill alone
        eng.reset(1)
        eng.set_flags(exact=True)
        t0 = time.perf_counter()
        eng.prefill(1, prompt[:256])
        block_tok_s = 256 / (time.perf_counter() - t0)
    log(f"prefill-config3: {t} tokens in {dt * 1e3:.1f} ms -> {tok_s:.0f} tok/s "
        f"({dt / chunks * 1e3:.2f} ms per {chunk}-token chunk; layer weights {wbytes / 1e9:.2f} GB "
        f"once per chunk -> {gbs:.0f} GB/s)"
        + (f"; exact 8-token blocks: {block_tok_s:.0f} tok/s" if block_tok_s else ""))
    eng.close()
    return {"metric": "chunked prefill tok/s (one 2048-token prompt, config-3 model)",
            "value": round(tok_s, 1), "unit": "tok/s", "ms_per_step": dt * 1e3,
            "dtype": "u4/u5 codes x bf16 on the bf16 matrix cores, fp32 sums",
            "config": {"workload": "prefill-config3", "prompt": t, "chunk": chunk,
                       "layers": cfg["layers"], "experts": cfg["experts"],
                       "ms_per_chunk": round(dt / chunks * 1e3, 3),
                       "block_prefill_tok_s": round(block_tok_s, 1) if block_tok_s else None},
            "roofline": {"bound": "hbm",
                         "kernel": f"whole chunk: every layer weight once per {chunk}-token chunk",
                         "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "algorithmic_bytes_per_chunk": int(wbytes)},
            "cpu_baseline": None}


WORKLOADS = {"config3-b8-decode": bench_config3, "qmv-config0": bench_qmv_config0,
             "gdn-prefill-config1": bench_gdn_prefill_config1,
             "gdn-decode-config1": bench_gdn_decode_config1, "moe-config2": bench_moe_config2,
             "mtp-config4": bench_mtp_config4, "copy-calibration": bench_copy_calibration,
             "prefill-config3": bench_prefill_config3}
DEFAULTS = {"config3-b8-decode": (240, 16), "qmv-config0": (2000, 200),
            "gdn-prefill-config1": (50, 5), "gdn-decode-config1": (200, 20),
            "moe-config2": (200, 20), "mtp-config4": (1, 0), "copy-calibration": (10, 2),
            "prefill-config3": (3, 1)}


def short_kernel_name(name: str) -> str:
    """A kernel's name without namespaces, return type and argument list."""
    import re
    name = name.replace("mx::(anonymous namespace)::", "").replace("void ", "")
    m = re.match(r"([\w]+(?:<[^>]*>)?)", name)
    return m.group(1) if m else name[:60]


def summarize_trace(path: str, line_path=None, kernel="xq_gate_up_kernel") -> None:
    """Markdown summary of a rocprofv3 kernel trace of this script
    (`--kernel-trace --output-format csv`, the *_kernel_trace.csv file):

    * every run of >= 16 launches of `kernel` each starting within 5 us of
      the previous one's end (the back-to-back launches behind the roofline
      figure; inside a step a layer's other kernels separate them, also when
      the trace was filtered to `kernel` alone), with the mean kernel duration
      and first-start-to-last-end span per launch; with `line_path` (the JSON
      line the same run printed), `frac` recomputed from the trace's mean
      beside the line's own;
    * when the trace holds whole eager steps: one step (the kernels after the
      third launch of the greedy head up to and including the fourth) by
      kernel and grid, with the hyper-connection kernels (norm, 8192-deep
      down projection, up-mix) summed."""
    import csv
    import gzip
    import io
    fh = gzip.open(path) if path.endswith(".gz") else open(path, "rb")
    rows = list(csv.DictReader(io.TextIOWrapper(fh, "utf-8")))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))

    def dur(r):
        return (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3

    names = [short_kernel_name(r["Kernel_Name"]) for r in rows]
    mine = [k for k, nm in enumerate(names) if nm.startswith(kernel)]
    runs, i = [], 0
    while i < len(mine):
        j = i + 1
        while (j < len(mine) and mine[j] == mine[j - 1] + 1 and
               int(rows[mine[j]]["Start_Timestamp"]) - int(rows[mine[j - 1]]["End_Timestamp"]) < 5000):
            j += 1
        if j - i >= 16:
            runs.append((mine[i], mine[j - 1] + 1))
        i = j
    print(f"## Back-to-back launches of `{kernel}`\n")
    print("| run | kernel | launches | mean us | span us / launch |")
    print("|---:|---|---:|---:|---:|")
    all_d = []
    for n, (i, j) in enumerate(runs):
        d = [dur(r) for r in rows[i:j]]
        all_d += d
        span = (int(rows[j - 1]["End_Timestamp"]) - int(rows[i]["Start_Timestamp"])) / 1e3
        print(f"| {n} | `{names[i]}` | {j - i} | {sum(d) / len(d):.2f} | {span / (j - i):.2f} |")
    if all_d:
        mean = sum(all_d) / len(all_d)
        print(f"\nmean over {len(all_d)} back-to-back launches: {mean:.2f} us")
        if line_path:
            line = None
            for text in open(line_path):
                text = text.strip()
                if text.startswith("{"):
                    line = json.loads(text)
            rf = line["roofline"]
            b = rf["algorithmic_bytes_per_launch"]
            frac = b / (mean * 1e-6) / 1e9 / rf["peak"]
            print(f"algorithmic bytes per launch (the line's): {b}")
            print(f"frac from the trace: {frac:.4f}; the line's frac: {rf['frac']} "
                  f"(us_per_launch {rf['us_per_launch']}); ratio {frac / rf['frac']:.4f}")
    heads = [k for k, nm in enumerate(names) if nm.startswith(("xq_head_kernel", "head_kernel"))]
    if len(heads) < 4:
        return
    a, b = heads[2], heads[3]
    step = rows[a + 1:b + 1]
    groups = {}
    for r, nm in zip(step, names[a + 1:b + 1]):
        wg = int(r["Workgroup_Size_X"])
        grid = (int(r["Grid_Size_X"]) // wg, int(r["Grid_Size_Y"]) // int(r["Workgroup_Size_Y"]),
                int(r["Grid_Size_Z"]) // int(r["Workgroup_Size_Z"]))
        groups.setdefault((nm, grid, wg), []).append(dur(r))
    tot = sum(sum(v) for v in groups.values())
    span = (int(step[-1]["End_Timestamp"]) - int(step[0]["Start_Timestamp"])) / 1e3
    print(f"\n## One step\n\n{len(step)} launches, {tot / 1e3:.3f} ms of kernel time, "
          f"{span / 1e3:.3f} ms first start to last end\n")
    print("| kernel | workgroups (x, y, z) | threads | calls/step | avg us | ms/step | share |")
    print("|---|---|---:|---:|---:|---:|---:|")
    for (nm, grid, wg), v in sorted(groups.items(), key=lambda kv: -sum(kv[1])):
        print(f"| `{nm}` | {grid} | {wg} | {len(v)} | {sum(v) / len(v):.1f} | "
              f"{sum(v) / 1e3:.3f} | {sum(v) / tot * 100:.1f} % |")
    hc = [(k, v) for k, v in groups.items()
          if k[0].startswith(("hc_norm_kernel", "xq_upmix_kernel", "xq_dense_kernel<4, 1,"))]
    hc_us = sum(sum(v) for _, v in hc)
    print(f"\nhyper-connection family (norm + HC down + up-mix): "
          f"{sum(len(v) for _, v in hc)} launches, {hc_us / 1e3:.3f} ms per step")


def summarize_kernels(path: str) -> None:
    """Markdown table of a rocprofv3 kernel trace grouped by kernel and grid
    (workgroups): launches, average and total duration.  Weight fills of
    engine creation and runtime copies are left out."""
    import collections
    import csv

    agg = collections.defaultdict(lambda: [0, 0.0])
    with open(path) as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if name.startswith("mx::(anonymous namespace)::fill") or "rocclr" in name:
                continue
            key = (short_kernel_name(name), int(r["Grid_Size_X"]) // int(r["Workgroup_Size_X"]),
                   int(r["Grid_Size_Y"]), int(r["Grid_Size_Z"]))
            agg[key][0] += 1
            agg[key][1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    rows = sorted(agg.items(), key=lambda kv: -kv[1][1])
    print("| kernel | workgroups (x, y, z) | launches | avg us | total ms |")
    print("|---|---|---:|---:|---:|")
    for (name, gx, gy, gz), (n, us) in rows:
        print(f"| `{name}` | ({gx}, {gy}, {gz}) | {n} | {us / n:.1f} | {us / 1e3:.2f} |")


def summarize_counters(fetch_csv: str, write_csv: str, fetch_scale: float, write_scale: float,
                       kernel="xq_gate_up_kernel") -> None:
    """Markdown table of HBM bytes per dispatch from two rocprofv3 `--pmc`
    runs of this script (FETCH_SIZE, then WRITE_SIZE; the
    *_counter_collection.csv files): per (kernel, grid size), the median
    counter over its dispatches times the copy calibration (bytes per KiB
    the counter reports for a device copy of known size, the
    copy-calibration workload), then `traffic_bytes_per_launch` of `kernel`
    (fetched + written) as the roofline's `traffic` reads it."""
    import csv
    import gzip
    import io
    import statistics

    def load(path, counter):
        out = {}
        fh = gzip.open(path) if path.endswith(".gz") else open(path, "rb")
        for r in csv.DictReader(io.TextIOWrapper(fh, "utf-8")):
            if r["Counter_Name"] == counter:
                key = (short_kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]))
                out.setdefault(key, []).append(float(r["Counter_Value"]))
        return out

    f, w = load(fetch_csv, "FETCH_SIZE"), load(write_csv, "WRITE_SIZE")
    fs, ws = fetch_scale * 1024, write_scale * 1024
    print("| kernel | grid (threads) | dispatches | fetched MB | written MB |")
    print("|---|---:|---:|---:|---:|")
    for key in sorted(f, key=lambda k: -statistics.median(f[k])):
        fm = statistics.median(f[key]) * fs / 1e6
        wm = statistics.median(w.get(key, [0.0])) * ws / 1e6
        if fm + wm >= 0.01:
            print(f"| `{key[0]}` | {key[1]} | {len(f[key])} | {fm:.2f} | {wm:.3f} |")
    tops = [k for k in f if k[0].startswith(kernel)]
    if tops:
        key = max(tops, key=lambda k: statistics.median(f[k]))  # the batch-8 grid
        tb = statistics.median(f[key]) * fs + statistics.median(w.get(key, [0.0])) * ws
        print(f"\ntraffic_bytes_per_launch = {int(tb)}")


def summarize_pmc(paths, kernels=("xq_gate_up_kernel", "xq_down_kernel", "xq_head_kernel")) -> None:
    """Markdown table of every counter in rocprofv3 `--pmc` runs of this script
    (their *_counter_collection.csv files, one pass each): per kernel name
    prefix in `kernels`, its largest grid (the batch-8 step's), the median of
    each counter over that grid's dispatches."""
    import csv
    import gzip
    import io
    import statistics

    vals = {}  # (short name, grid) -> counter -> values
    for path in paths:
        fh = gzip.open(path) if path.endswith(".gz") else open(path, "rb")
        for r in csv.DictReader(io.TextIOWrapper(fh, "utf-8")):
            key = (short_kernel_name(r["Kernel_Name"]), int(r["Grid_Size"]))
            vals.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(
                float(r["Counter_Value"]))
    picked = []
    for prefix in kernels:
        keys = [k for k in vals if k[0].startswith(prefix)]
        if keys:
            picked.append(max(keys, key=lambda k: k[1]))
    counters = sorted({c for k in picked for c in vals[k]})
    print("| counter | " + " | ".join(f"`{k[0]}` ({k[1]} threads)" for k in picked) + " |")
    print("|---|" + "---:|" * len(picked))
    for c in counters:
        cells = []
        for k in picked:
            v = vals[k].get(c)
            cells.append(f"{statistics.median(v):.6g}" if v else "")
        print(f"| {c} | " + " | ".join(cells) + " |")
    print("\n| dispatches | " + " | ".join(
        str(max(len(v) for v in vals[k].values())) for k in picked) + " |")


def main() -> None:
    if len(sys.argv) >= 3 and sys.argv[1] == "--summarize-pmc":
        # no device work: medians of every counter of rocprofv3 --pmc runs
        # (optionally `--kernels a,b,c`: the kernel name prefixes to report)
        args = sys.argv[2:]
        if "--kernels" in args:
            i = args.index("--kernels")
            summarize_pmc(args[:i] + args[i + 2:], tuple(args[i + 1].split(",")))
        else:
            summarize_pmc(args)
        return
    if len(sys.argv) >= 6 and sys.argv[1] == "--summarize-counters":
        # no device work: summarise two rocprofv3 counter runs of this script
        summarize_counters(sys.argv[2], sys.argv[3], float(sys.argv[4]), float(sys.argv[5]),
                           *(sys.argv[6:7]))
        return
    if len(sys.argv) >= 3 and sys.argv[1] == "--summarize-kernels":
        # no device work: group a rocprofv3 kernel trace by kernel and grid
        summarize_kernels(sys.argv[2])
        return
    if len(sys.argv) >= 3 and sys.argv[1] == "--summarize-trace":
        # no device work: summarise a rocprofv3 kernel trace of an earlier run
        summarize_trace(sys.argv[2], sys.argv[3] if len(sys.argv) > 3 else None,
                        *(sys.argv[4:5]))
        return
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--workload", default="config3-b8-decode", choices=sorted(WORKLOADS))
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel eagerly instead of replaying captured HIP graphs "
                         "(same kernels; used under rocprofv3, whose kernel trace does not "
                         "follow graph replays)")
    ap.add_argument("--synthetic-context", action="store_true",
                    help="give the rows random caches of the prompt lengths instead of "
                         "prefilling them (profiling runs: the decode step's cost depends on "
                         "the context length only)")
    ap.add_argument("--block-prefill", action="store_true",
                    help="config3 / mtp-config4: prefill the contexts (prompt) in exact eight-token blocks "
                         "(mx_engine_prefill) instead of 512-token matrix-core chunks "
                         "(mx_engine_prefill_chunked)")
    ap.add_argument("--fast", action="store_true",
                    help="config3: time the bf16 matrix-core kernels (within tolerance of the "
                         "oracle, not bit-exact) as the headline path, and the exact path "
                         "beside it")
    ap.add_argument("--exact", action="store_true",
                    help="config3: the exact-integer kernels (bit-exact with the oracle) as "
                         "the headline path, the matrix-core path beside it (the default)")
    ap.add_argument("--no-cpu-baseline", action="store_true",
                    help="skip the oracle CPU baseline (profiling runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): this build runs on a "
              "single MI355X and has no multi-GPU path", file=sys.stderr)
        raise SystemExit(2)
    steps, warmup = DEFAULTS[args.workload]
    args.steps = steps if args.steps is None else args.steps
    args.warmup = warmup if args.warmup is None else args.warmup
    mx = load_package()
    res = WORKLOADS[args.workload](mx, args)
    out = {
        "metric": res["metric"], "value": res["value"], "unit": res["unit"], "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": res["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": res["dtype"], "data": "synthetic (seeded counter-based generator, random-init weights)",
        "config": res["config"], "roofline": res["roofline"], "cpu_baseline": res["cpu_baseline"],
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
