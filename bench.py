#!/usr/bin/env python3
"""Benchmark of the GGUF dequant-fused quantized linear on one MI355X.

Workload ("C3"): Qwen-27B-like UD-Q4_K_XL mix, decode GEMV
at batch 1, 2, 8 and 16 — Q4_K gate/up 34816x5120 and qkv 7168x5120, Q6_K down
5120x17408 and o_proj 5120x6144, weights quantized from seeded N(0, 0.02),
activations fp16 N(0, 1). One step = for each batch size, each projection's Q8_1
activation preparation and its GEMV (rows <= 8: kai_fused_mmvq, 16:
kai_fused_mmq_run), i.e. 16 projections. value = weight bytes streamed per step /
step time (GB/s); inputs are resident in HBM.

Measurement: every step is a replay of a captured HIP graph; 3 copies of the
weights (660 MB) rotate so the 256 MB Infinity Cache never holds the working set.
The roofline object covers the dominant kernel, the Q4_K gate/up GEMV (100 MB of
wire bytes per launch), timed by HIP events around replays of a graph of those
launches alone (8 rounds of the 3 copies per graph). The prefill leg (configs[3],
M=2048) reports TOPS. The CPU baseline times the oracle (the C restatement of the
reference arithmetic) on a bounded sample on the host cores.
"""
import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
COPIES = 3
ROUNDS = 8  # rounds of the copies per timed graph, so graph-launch overhead is amortised


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=60)
    p.add_argument("--warmup", type=int, default=6)
    p.add_argument("--batches", default="1,2,8,16")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-prefill", action="store_true", help="skip the prefill leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--kernel-sample", action="store_true",
                   help="counter-collection run: a 256 MiB device copy (calibration) and the dominant "
                        "GEMV on each weight copy, eager launches only")
    return p.parse_args()


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see DESIGN.md for how the op would shard)", file=sys.stderr)
        sys.exit(2)
    import torch

    from kaillm_amd import native
    from kaillm_amd.formats import Q4_K, Q6_K, quantize, weight_bytes

    lib = native.library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    batches = [int(b) for b in args.batches.split(",")]
    if args.kernel_sample:
        kernel_sample(lib, dev, batches)
        return

    mats = [  # name, type, n, k
        ("gate_up", Q4_K, 34816, 5120),
        ("qkv", Q4_K, 7168, 5120),
        ("down", Q6_K, 5120, 17408),
        ("o_proj", Q6_K, 5120, 6144),
    ]
    rng = np.random.default_rng(2)
    t0 = time.time()
    weights = {}
    for i, (name, qtype, n, k) in enumerate(mats):
        g = torch.Generator(device=dev).manual_seed(1000 + i)
        w32 = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32).mul_(0.02).cpu().numpy()
        packed = torch.from_numpy(quantize(w32, qtype)).to(dev)
        del w32
        weights[name] = [packed] + [packed.clone() for _ in range(COPIES - 1)]
    print(f"[bench] weights quantized and uploaded in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    stream = torch.cuda.Stream(device=dev)
    max_m = max(batches)
    xs = {name: torch.from_numpy(rng.standard_normal((max_m, k)).astype(np.float16)).to(dev)
          for name, _, _, k in mats}
    outs = {name: torch.empty((max_m, n), dtype=torch.float32, device=dev) for name, _, n, _ in mats}
    acts = {name: torch.empty(lib.kai_fused_activation_bytes(max_m, k, 0), dtype=torch.uint8, device=dev)
            for name, _, _, k in mats}
    groups = {}
    for name, qtype, n, k in mats:
        for c in range(COPIES):
            groups[(name, c)] = ((ctypes.c_void_p * 1)(weights[name][c].data_ptr()),
                                 (ctypes.c_int * 1)(qtype), (ctypes.c_int64 * 1)(n))
    # scratch of the batched entry at the largest batch (its size query, as the reference's
    # callers do)
    mmq_ws = {}
    for name, qtype, n, k in mats:
        ptrs, types, rows = groups[(name, 0)]
        size = lib.kai_fused_mmq_workspace(0, types, rows, 1, k, max_m, 1) if max_m > 8 else 0
        mmq_ws[name] = torch.empty(max(size, 1), dtype=torch.uint8, device=dev)

    def projection(name, qtype, n, k, m, copy, s):
        x = xs[name][:m]
        if m <= 8:
            native.check(lib, lib.kai_fused_prepare(x.data_ptr(), 2, m, k, k, acts[name].data_ptr(), 0, s))
            native.check(lib, lib.kai_fused_mmvq(weights[name][copy].data_ptr(), qtype, n, k, m,
                                                 acts[name].data_ptr(), 0, outs[name].data_ptr(), 0, n, s))
        else:
            ptrs, types, rows = groups[(name, copy)]
            native.check(lib, lib.kai_fused_mmq_run(ptrs, types, rows, 1, x.data_ptr(), 2, k, k, m,
                                                    outs[name].data_ptr(), 0, 0, mmq_ws[name].data_ptr(),
                                                    mmq_ws[name].numel(), 0, s))

    def capture(fn):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            fn()  # warm once outside capture (module/code-object loading)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=stream):
                fn()
        return g

    def step_fn(copy_base):
        def fn():
            s = torch.cuda.current_stream().cuda_stream
            for bi, m in enumerate(batches):
                for name, qtype, n, k in mats:
                    projection(name, qtype, n, k, m, (copy_base + bi) % COPIES, s)
        return fn

    step_graphs = [capture(step_fn(c)) for c in range(COPIES)]
    step_bytes = sum(weight_bytes(q, n, k) for _, q, n, k in mats) * len(batches)

    def timed(graphs, reps):
        for i in range(args.warmup):
            graphs[i % len(graphs)].replay()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        for i in range(reps):
            graphs[i % len(graphs)].replay()
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / reps  # ms per replay

    with torch.cuda.stream(stream):
        ms_step = timed(step_graphs, args.steps)
    print(f"[bench] step {ms_step * 1e3:.1f} us for {step_bytes / 1e6:.1f} MB of weights", file=sys.stderr, flush=True)

    # Dominant kernel: Q4_K gate/up GEMV at every batch size, copies rotating.
    name, qtype, n, k = mats[0]
    per_m = {}
    for m in batches:
        x = xs[name][:m]
        s0 = torch.cuda.current_stream().cuda_stream
        # the activation is prepared once outside the graph; the graph holds only GEMVs
        with torch.cuda.stream(stream):
            native.check(lib, lib.kai_fused_prepare(x.data_ptr(), 2, m, k, k, acts[name].data_ptr(), 0,
                                                    stream.cuda_stream))
        del s0

        def gemv_fn(m=m):
            def fn():
                s = torch.cuda.current_stream().cuda_stream
                for c in [c for _ in range(ROUNDS) for c in range(COPIES)]:
                    if m <= 8:
                        native.check(lib, lib.kai_fused_mmvq(weights[name][c].data_ptr(), qtype, n, k, m,
                                                             acts[name].data_ptr(), 0, outs[name].data_ptr(), 0, n, s))
                    else:
                        projection(name, qtype, n, k, m, c, s)
            return fn
        g = capture(gemv_fn())
        with torch.cuda.stream(stream):
            ms = timed([g], max(10, args.steps)) / (ROUNDS * COPIES)
        per_m[m] = ms
    wb = weight_bytes(qtype, n, k)
    avg_ms = float(np.mean([per_m[m] for m in batches]))
    achieved = wb / (avg_ms * 1e-3) / 1e9
    by_m = {str(m): {"us": round(per_m[m] * 1e3, 2), "GB/s": round(wb / (per_m[m] * 1e-3) / 1e9, 1)}
            for m in batches}
    print(f"[bench] Q4_K gate/up GEMV per batch: {by_m}", file=sys.stderr, flush=True)

    prefill = None
    if not args.no_prefill:
        m = 2048
        xp = torch.from_numpy(rng.standard_normal((m, k)).astype(np.float16)).to(dev)
        outp = torch.empty((m, n), dtype=torch.float32, device=dev)
        ptrs, types, rows = groups[(name, 0)]
        size = lib.kai_fused_mmq_workspace(0, types, rows, 1, k, m, 1)
        scratch = torch.empty(size, dtype=torch.uint8, device=dev)

        def prefill_fn():
            s = torch.cuda.current_stream().cuda_stream
            native.check(lib, lib.kai_fused_mmq_run(ptrs, types, rows, 1, xp.data_ptr(), 2, k, k, m,
                                                    outp.data_ptr(), 0, 0, scratch.data_ptr(), size, 0, s))
        g = capture(prefill_fn)
        with torch.cuda.stream(stream):
            ms = timed([g], 5)
        tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
        prefill = {"config": "Q4_K 34816x5120, M=2048 (configs[3])", "ms": round(ms, 3),
                   "TOPS": round(tops, 2), "frac_int8_peak": round(tops / INT8_PEAK_TOPS, 4)}
        print(f"[bench] prefill {prefill}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(weights[name][0], qtype, n, k, args.cpu_seconds)

    # HBM bytes per launch of the same kernels, from the FETCH_SIZE / WRITE_SIZE counter runs
    # (scaled by a plain copy's readings) summarised in profiles/.
    traffic = None
    tfile = ROOT / "profiles" / "gemv_q4k_34816x5120_traffic.json"
    if tfile.exists():
        tb = json.loads(tfile.read_text())["by_batch"]
        if all(str(m) in tb for m in batches):
            traffic = round(float(np.mean([tb[str(m)]["bytes"] for m in batches])))

    result = {
        "metric": "weight-stream HBM GB/s (% of peak) for Q4_K GEMV b1-16; prefill int8 TOPS",
        "value": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic: weights quantized from seeded N(0,0.02), activations fp16 N(0,1)",
        "config": {"workload": "C3 Qwen-27B-like Q4_K/Q6_K decode GEMV, batch " + args.batches,
                   "matrices": {nm: [n_, k_] for nm, _, n_, k_ in mats},
                   "step_weight_bytes": step_bytes, "weight_copies": COPIES},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "kernel": "Q4_K gate/up GEMV 34816x5120 (mean over batch " + args.batches + ")",
                     "bytes_per_launch": wb, "avg_launch_us": round(avg_ms * 1e3, 2), "by_batch": by_m},
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def kernel_sample(lib, dev, batches):
    """Eager launches for rocprofv3 --pmc runs: FETCH_SIZE / WRITE_SIZE of a plain copy of
    known size (the calibration) next to those of the Q4_K gate/up GEMV per batch size."""
    import torch

    from kaillm_amd import native
    from kaillm_amd.formats import Q4_K, quantize

    n, k = 34816, 5120
    g = torch.Generator(device=dev).manual_seed(1000)
    w32 = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32).mul_(0.02).cpu().numpy()
    packed = torch.from_numpy(quantize(w32, Q4_K)).to(dev)
    copies = [packed] + [packed.clone() for _ in range(COPIES - 1)]
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((max(batches), k)).astype(np.float16)).to(dev)
    out = torch.empty((max(batches), n), dtype=torch.float32, device=dev)
    act = torch.empty(lib.kai_fused_activation_bytes(max(batches), k, 0), dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    types, rows = (ctypes.c_int * 1)(Q4_K), (ctypes.c_int64 * 1)(n)
    for m in batches:
        if m <= 8:
            native.check(lib, lib.kai_fused_prepare(x.data_ptr(), 2, m, k, k, act.data_ptr(), 0, s))
            for c in copies:
                native.check(lib, lib.kai_fused_mmvq(c.data_ptr(), Q4_K, n, k, m, act.data_ptr(), 0,
                                                     out.data_ptr(), 0, n, s))
        else:
            size = lib.kai_fused_mmq_workspace(0, types, rows, 1, k, m, 1)
            scratch = torch.empty(size, dtype=torch.uint8, device=dev)
            for c in copies:
                ptrs = (ctypes.c_void_p * 1)(c.data_ptr())
                native.check(lib, lib.kai_fused_mmq_run(ptrs, types, rows, 1, x.data_ptr(), 2, k, k, m,
                                                        out.data_ptr(), 0, 0, scratch.data_ptr(), size, 0, s))
    torch.cuda.synchronize()
    print(f"[bench] kernel sample: 3 copies of {src.numel()} bytes, Q4_K {n}x{k} GEMV x{COPIES} "
          f"at batch {batches}", flush=True)


def cpu_baseline(w_dev, qtype, n, k, seconds):
    """Oracle GEMV (the C restatement of the reference arithmetic) on host cores."""
    sys.path.insert(0, str(ROOT / "tests"))
    import _oracle as O

    cores = len(os.sched_getaffinity(0))
    rows = min(n, 4096)
    w = w_dev[:rows].cpu().numpy()
    x = np.random.default_rng(5).standard_normal((1, k)).astype(np.float16)
    act = O.prepare(x)
    out = np.empty((1, rows), dtype=np.float32)
    o = O.lib()
    reps, t0 = 0, time.perf_counter()
    while True:
        assert o.oracle_mul_mat_f32(qtype, O._p(w), rows, k, 1, O._p(act), 0, O._p(out), rows, cores) == 0
        reps += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = (time.perf_counter() - t0) / reps
    wb = rows * (k // 256) * 144
    return {"value": round(wb / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle_mul_mat_f32 Q4_K {rows}x{k} rows of gate/up, M=1, {reps} calls in {seconds:.0f}s, "
                      f"{dt * 1e3:.2f} ms/call"}


if __name__ == "__main__":
    main()
