#!/usr/bin/env python3
"""Benchmark of the GGUF dequant-fused quantized linear on one MI355X.

Headline workload ("C3"): Qwen-27B-like UD-Q4_K_XL mix at batch
1, 2, 8 and 16 — Q4_K gate/up 34816x5120 and qkv 7168x5120, Q6_K down 5120x17408 and
o_proj 5120x6144, weights quantized from seeded N(0, 0.02), activations fp16 N(0, 1). One
step = for each batch size, each projection's activation preparation and its product
(rows <= 8: kai_fused_prepare + kai_fused_mmvq; 16: kai_fused_mmq_run), 16 projections.
value = weight bytes streamed per step / step time (GB/s); inputs are resident in HBM.

Every timing is a replay of a captured HIP graph, HIP events on the replay stream, with
rotating weight copies totalling >= 600 MB so the 256 MB Infinity Cache never holds the
working set.

* ``roofline``: every C3 matrix at every batch, kernel only where the API allows it (batch
  1-8: kai_fused_mmvq with the activation prepared once outside the graph; batch 16:
  kai_fused_mmq_run, whose operand preparation runs inside the call); weight bytes per launch
  over the mean launch time. The headline fields are those of the dominant launch (the longest
  kernel-only one), with its HBM traffic from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE
  summary of that matrix.
* ``legs``: every BASELINE config as whole calls (preparation included, as a caller sees
  them): C1, C2 and C5 decode, C3 per matrix and batch, C4 spec-verify (M=80, GB/s) and
  prefill (M=512, 2048, TOPS), C5 batch 16 and prefill. Each leg names its kernel. TOPS count
  2·M·N·K ops; ``frac`` is against the dense int8 MFMA peak the target is set on, and the legs on
  the folded fp16 GEMM also give ``fp16_frac``, against the fp16 MFMA peak of the pipe they use.
* ``cpu_baseline``: the oracle (the C restatement of the reference arithmetic) on a bounded
  sample, on the host cores, with the CPU model and thread count.
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
FP16_PEAK_TFLOPS = 2500.0
ROTATION_BYTES = 600e6   # weight copies per matrix: at least this many bytes in rotation
MIN_COPIES = 3

# BASELINE.json configs as (config, matrix, type, n, k, batches). tests/test_gpu_bench_routes.py
# generates its full-size oracle cases from these tables, so every timed route has a parity test.
Q4_0, Q8_0, Q2_K, Q4_K, Q6_K, IQ3_S = 2, 8, 10, 12, 14, 21
C3_BATCHES = (1, 2, 8, 16)
C3 = [("gate_up", Q4_K, 34816, 5120), ("qkv", Q4_K, 7168, 5120), ("down", Q6_K, 5120, 17408),
      ("o_proj", Q6_K, 5120, 6144)]
LEGS = [
    ("C1", "plumbing", Q8_0, 2048, 2048, (1,)),
    ("C2", "gate_up", Q4_0, 16384, 2048, (1, 2, 4, 8)),
    ("C2", "down", Q4_0, 2048, 8192, (1, 2, 4, 8)),
    ("C2", "qkv", Q4_0, 3072, 2048, (1, 2, 4, 8)),
    ("C4", "gate_up", Q4_K, 34816, 5120, (80, 512, 2048)),
    ("C4", "down", Q4_K, 5120, 17408, (80, 512, 2048)),
    ("C5", "gate_up Q2_K", Q2_K, 34816, 5120, (1, 16, 2048)),
    ("C5", "down Q2_K", Q2_K, 5120, 17408, (1, 16, 2048)),
    ("C5", "gate_up IQ3_S", IQ3_S, 34816, 5120, (1, 16, 2048)),
    ("C5", "down IQ3_S", IQ3_S, 5120, 17408, (1, 16, 2048)),
]
NAMES = {Q4_0: "Q4_0", Q8_0: "Q8_0", Q2_K: "Q2_K", Q4_K: "Q4_K", Q6_K: "Q6_K", IQ3_S: "IQ3_S"}
def gemv_max_rows(qtype, k):  # kai_launch.h gemv_max_rows
    return {Q4_0: 8, Q8_0: 8, Q4_K: 4, Q6_K: 3 if k >= 12288 else 4, IQ3_S: 4, Q2_K: 3}[qtype]


def persistent(n, image=False, cus=256):
    """kai_mmqd.cuh mmqd_suits for the benched shapes (all fit its LDS): whole 16-row sets per
    workgroup keep the workgroups busy for at least 90 % (85 % over the small-M image) of the
    longest one's time."""
    sets = (n + 15) // 16
    wgs = min(sets, cus)
    return sets * 20 >= (17 if image else 18) * wgs * -(-sets // wgs)


def gemv_rows(qtype, n, k):  # kai_abi.hip run_decode
    if persistent(n):  # kai_launch.h gemv_rows_before_persistent
        if qtype == Q4_0 and (n + 15) // 16 < 256:
            return 8
        return {Q4_0: 6, Q8_0: 6, Q4_K: 3, Q2_K: 2}.get(qtype, gemv_max_rows(qtype, k))
    return gemv_max_rows(qtype, k)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=60)
    p.add_argument("--warmup", type=int, default=6)
    p.add_argument("--batches", default=",".join(map(str, C3_BATCHES)))
    p.add_argument("--legs", default="all", help="'all', 'none', or a comma list of C1,C2,C3,C4,C5")
    p.add_argument("--reps", type=int, default=8, help="graph replays per leg")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--kernel-sample", action="store_true",
                   help="counter-collection run: a 256 MiB device copy (calibration) and the decode "
                        "kernels of one C3 matrix on each weight copy, eager launches only")
    p.add_argument("--sample-matrix", default="gate_up", choices=[c[0] for c in C3],
                   help="the C3 matrix of --kernel-sample")
    p.add_argument("--peaks", action="store_true",
                   help="measure this device's ceilings instead (MFMA rate per kind, LDS reads, HBM copy)")
    return p.parse_args()


def kernel_name(qtype, m, n, k):
    if m > 16:
        if qtype in (Q4_K, Q4_0, Q8_0, IQ3_S, Q2_K):  # kai_launch.h mmq_uses_h
            return "fp16 folded-operand GEMM (kai_fused_mmq_run: fp16 image + mmqh_kernel)"
        return "int8 MMQ (kai_fused_mmq_run: GGML MMQ planes + mmq_kernel)"
    if m > 8:
        if persistent(n, image=True):
            return "persistent int8 GEMM (kai_fused_mmq_run: GGML MMQ image + mmqd_kernel)"
        return "small-M int8 GEMM (kai_fused_mmq_run: GGML MMQ image + mmqs_kernel + reduction)"
    if m <= gemv_rows(qtype, n, k):
        return "v_dot4 GEMV (mmvq_kernel)"
    if persistent(n):
        return "persistent paired int8 GEMM (mmqd_kernel)"
    if (n + 15) // 16 < 512 and k >= 32 * 256:  # kai_mmq.cuh launch_mmq_type: K pieces
        return "paired int8 MMQ tile with K pieces across workgroups (mmq_kernel, PAIR)"
    return "paired int8 MMQ tile (mmq_kernel, PAIR)"


class Runner:
    """Weights (rotating copies), inputs, outputs and scratch of the projections benched."""

    def __init__(self, lib, dev, torch, max_m):
        self.lib, self.dev, self.torch = lib, dev, torch
        self.weights, self.groups, self.ws = {}, {}, {}
        self.max_m = max_m
        self.stream = torch.cuda.Stream(device=dev)
        self.rng = np.random.default_rng(2)
        self.x, self.out, self.act = {}, {}, {}

    def add(self, key, qtype, n, k, seed, max_m):
        from kaillm_amd.formats import quantize, weight_bytes
        torch = self.torch
        if key in self.weights:
            return
        g = torch.Generator(device=self.dev).manual_seed(seed)
        w32 = torch.randn((n, k), generator=g, device=self.dev, dtype=torch.float32).mul_(0.02).cpu().numpy()
        packed = torch.from_numpy(quantize(w32, qtype)).to(self.dev)
        del w32
        copies = max(MIN_COPIES, int(np.ceil(ROTATION_BYTES / weight_bytes(qtype, n, k))))
        self.weights[key] = [packed] + [packed.clone() for _ in range(copies - 1)]
        self.groups[key] = [((ctypes.c_void_p * 1)(w.data_ptr()), (ctypes.c_int * 1)(qtype), (ctypes.c_int64 * 1)(n))
                            for w in self.weights[key]]
        if k not in self.x or self.x[k].shape[0] < max_m:
            self.x[k] = torch.from_numpy(self.rng.standard_normal((max_m, k)).astype(np.float16)).to(self.dev)
        if n not in self.out or self.out[n].numel() < max_m * n:
            self.out[n] = torch.empty(max_m * n, dtype=torch.float32, device=self.dev)
        if k not in self.act or self.act[k].numel() < self.lib.kai_fused_activation_bytes(8, k, 0):
            self.act[k] = torch.empty(self.lib.kai_fused_activation_bytes(8, k, 0), dtype=torch.uint8,
                                      device=self.dev)

    def workspace(self, key, k, m):
        """The batched entry's scratch for this matrix at m rows (kai_fused_mmq_workspace per
        shape, as a caller keeps it: its size is not monotonic in m, since split-K sums can make
        a smaller product need more)."""
        if (key, m) not in self.ws:
            size = self.lib.kai_fused_mmq_workspace(0, self.groups[key][0][1], self.groups[key][0][2], 1, k, m, 1)
            if size == 0:
                raise RuntimeError(self.lib.current_direct_error().decode())
            self.ws[(key, m)] = self.torch.empty(size, dtype=self.torch.uint8, device=self.dev)
        return self.ws[(key, m)]

    def call(self, key, qtype, n, k, m, copy, s, prepare=True):
        """One projection: preparation + product (decode), or one batched call."""
        from kaillm_amd import native
        lib, x = self.lib, self.x[k][:m]
        if m <= 8:
            if prepare:
                native.check(lib, lib.kai_fused_prepare(x.data_ptr(), 2, m, k, k, self.act[k].data_ptr(), 0, s))
            native.check(lib, lib.kai_fused_mmvq(self.weights[key][copy].data_ptr(), qtype, n, k, m,
                                                 self.act[k].data_ptr(), 0, self.out[n].data_ptr(), 0, n, s))
        else:
            ptrs, types, rows = self.groups[key][copy]
            ws = self.workspace(key, k, m)
            native.check(lib, lib.kai_fused_mmq_run(ptrs, types, rows, 1, x.data_ptr(), 2, k, k, m,
                                                    self.out[n].data_ptr(), 0, 0, ws.data_ptr(), ws.numel(), 0, s))

    def capture(self, fn):
        torch = self.torch
        g = torch.cuda.CUDAGraph()
        with torch.cuda.stream(self.stream):
            fn()  # once outside capture (code-object loading, LDS attributes)
            torch.cuda.synchronize()
            with torch.cuda.graph(g, stream=self.stream):
                fn()
        return g

    def timed(self, graphs, reps, warmup):
        """ms per replay (HIP events on the replay stream)."""
        torch = self.torch
        with torch.cuda.stream(self.stream):
            for i in range(warmup):
                graphs[i % len(graphs)].replay()
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record(self.stream)
            for i in range(reps):
                graphs[i % len(graphs)].replay()
            end.record(self.stream)
            torch.cuda.synchronize()
        return start.elapsed_time(end) / reps

    def per_launch_us(self, key, qtype, n, k, m, reps, warmup, prepare=True, budget_ms=40.0):
        """Mean time of one call, from a graph of calls over every weight copy (rounds of the
        copies until the graph holds about budget_ms of work)."""
        copies = len(self.weights[key])
        one = self.timed([self.capture(lambda: self.call(key, qtype, n, k, m, 0, self.stream.cuda_stream,
                                                         prepare))], 3, 1)
        rounds = max(1, min(int(budget_ms / max(one * copies, 1e-3)), 2000 // copies))
        seq = [c for _ in range(rounds) for c in range(copies)]

        def fn():
            s = self.torch.cuda.current_stream().cuda_stream
            for c in seq:
                self.call(key, qtype, n, k, m, c, s, prepare)
        return self.timed([self.capture(fn)], reps, warmup) / len(seq) * 1e3


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(see DESIGN.md for how the op would shard)", file=sys.stderr)
        sys.exit(2)
    import torch

    from kaillm_amd import native
    from kaillm_amd.formats import weight_bytes

    lib = native.library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    batches = [int(b) for b in args.batches.split(",")]
    if args.kernel_sample:
        kernel_sample(lib, dev, batches, args.sample_matrix)
        return
    if args.peaks:
        print(json.dumps(measure_peaks(lib, dev)), flush=True)
        return
    chosen = set(("C1,C2,C3,C4,C5" if args.legs == "all" else "" if args.legs == "none" else args.legs).split(","))

    t0 = time.time()
    r = Runner(lib, dev, torch, max(batches))
    for i, (name, qtype, n, k) in enumerate(C3):
        r.add(("C3", name), qtype, n, k, 1000 + i, max(batches))
    print(f"[bench] C3 weights quantized and uploaded in {time.time() - t0:.1f}s", file=sys.stderr, flush=True)

    # ---- headline: the C3 decode step
    def step_fn(base):
        def fn():
            s = torch.cuda.current_stream().cuda_stream
            for bi, m in enumerate(batches):
                for name, qtype, n, k in C3:
                    key = ("C3", name)
                    r.call(key, qtype, n, k, m, (base + bi) % len(r.weights[key]), s)
        return fn
    step_graphs = [r.capture(step_fn(c)) for c in range(MIN_COPIES)]
    step_bytes = sum(weight_bytes(q, n, k) for _, q, n, k in C3) * len(batches)
    ms_step = r.timed(step_graphs, args.steps, args.warmup)
    print(f"[bench] step {ms_step * 1e3:.1f} us for {step_bytes / 1e6:.1f} MB of weights", file=sys.stderr,
          flush=True)

    # ---- roofline: every C3 launch, kernel only for the decode batches (activation prepared
    # once outside the graph); batch 16 is a whole kai_fused_mmq_run call
    by_launch = {}
    for name, qtype, n, k in C3:
        key = ("C3", name)
        wb = weight_bytes(qtype, n, k)
        for m in batches:
            if m <= 8:
                x = r.x[k][:m]
                native.check(lib, lib.kai_fused_prepare(x.data_ptr(), 2, m, k, k, r.act[k].data_ptr(), 0,
                                                        torch.cuda.current_stream().cuda_stream))
                torch.cuda.synchronize()
            us = r.per_launch_us(key, qtype, n, k, m, max(10, args.steps // 4), 2, prepare=False)
            gbs = wb / (us * 1e-6) / 1e9
            by_launch[f"{name} b{m}"] = {"us": round(us, 2), "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                                         "kernel": kernel_name(qtype, m, n, k), "bytes": wb,
                                         "timed": "kernel only" if m <= 8 else "whole call (preparation inside)"}
    dom_name = max((kk for kk, v in by_launch.items() if v["timed"] == "kernel only"), key=lambda kk: by_launch[kk]["us"])
    dom = by_launch[dom_name]
    dmat, dm = dom_name.split(" b")
    achieved = dom["GB/s"]
    roof = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
            "kernel": f"{dom_name}: {dom['kernel']} (the longest kernel-only launch of the step)",
            "bytes_per_launch": dom["bytes"], "avg_launch_us": dom["us"], "by_launch": by_launch}
    tfile = ROOT / "profiles" / f"decode_traffic_{dmat}.json"
    if tfile.exists():
        tb = json.loads(tfile.read_text()).get("by_batch", {})
        if dm in tb:
            roof["traffic"] = tb[dm]["bytes"]
            roof["traffic_source"] = f"profiles/{tfile.name} (rocprofv3 FETCH_SIZE/WRITE_SIZE, not this run)"
    print(f"[bench] roofline {by_launch}", file=sys.stderr, flush=True)

    # ---- per-config legs: whole calls
    legs = []

    def leg(cfg, mname, qtype, n, k, m, key):
        us = r.per_launch_us(key, qtype, n, k, m, args.reps, 2)
        wbytes = weight_bytes(qtype, n, k)
        entry = {"config": cfg, "matrix": f"{mname} {NAMES[qtype]} {n}x{k}", "m": m, "us": round(us, 2),
                 "kernel": kernel_name(qtype, m, n, k), "includes": "activation preparation"}
        if m >= 512:
            tops = 2.0 * m * n * k / (us * 1e-6) / 1e12
            entry.update({"TOPS": round(tops, 1), "frac": round(tops / INT8_PEAK_TOPS, 4), "bound": "mfma int8"})
            if "fp16" in entry["kernel"]:
                entry.update({"fp16_frac": round(tops / FP16_PEAK_TFLOPS, 4), "bound": "mfma fp16"})
        else:
            gbs = wbytes / (us * 1e-6) / 1e9
            entry.update({"GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4), "bound": "hbm"})
        legs.append(entry)
        print(f"[bench] leg {entry}", file=sys.stderr, flush=True)

    if "C3" in chosen:
        for name, qtype, n, k in C3:
            for m in batches:
                leg("C3", name, qtype, n, k, m, ("C3", name))
    for i, (cfg, mname, qtype, n, k, ms) in enumerate(LEGS):
        if cfg not in chosen:
            continue
        key = (cfg, mname)
        r.add(key, qtype, n, k, 2000 + i, max(ms))
        for m in ms:
            leg(cfg, mname, qtype, n, k, m, key)
        del r.weights[key], r.groups[key]
        for wkey in [w for w in r.ws if w[0] == key]:
            del r.ws[wkey]
        torch.cuda.empty_cache()

    cpu = None if args.no_cpu else cpu_baseline(r.weights[("C3", "gate_up")][0], Q4_K, 34816, 5120, args.cpu_seconds)

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
        "config": {"workload": "C3 Qwen-27B-like Q4_K/Q6_K decode, batch " + args.batches,
                   "matrices": {nm: [n_, k_] for nm, _, n_, k_ in C3},
                   "step_weight_bytes": step_bytes,
                   "weight_copies": {nm: len(r.weights[("C3", nm)]) for nm, _, _, _ in C3}},
        "roofline": roof,
        "legs": legs,
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


def kernel_sample(lib, dev, batches, matrix="gate_up"):
    """Eager launches for rocprofv3 --pmc runs: FETCH_SIZE / WRITE_SIZE of a plain copy of
    known size (the calibration) next to those of one C3 matrix's decode kernels per batch."""
    import torch

    from kaillm_amd import native
    from kaillm_amd.formats import quantize

    _, qtype, n, k = next(c for c in C3 if c[0] == matrix)
    g = torch.Generator(device=dev).manual_seed(1000)
    w32 = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32).mul_(0.02).cpu().numpy()
    packed = torch.from_numpy(quantize(w32, qtype)).to(dev)
    copies = [packed] + [packed.clone() for _ in range(MIN_COPIES - 1)]
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    x = torch.from_numpy(np.random.default_rng(2).standard_normal((max(batches), k)).astype(np.float16)).to(dev)
    out = torch.empty((max(batches), n), dtype=torch.float32, device=dev)
    act = torch.empty(lib.kai_fused_activation_bytes(max(batches), k, 0), dtype=torch.uint8, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    types, rows = (ctypes.c_int * 1)(qtype), (ctypes.c_int64 * 1)(n)
    for m in batches:
        if m <= 8:
            native.check(lib, lib.kai_fused_prepare(x.data_ptr(), 2, m, k, k, act.data_ptr(), 0, s))
            for c in copies:
                native.check(lib, lib.kai_fused_mmvq(c.data_ptr(), qtype, n, k, m, act.data_ptr(), 0,
                                                     out.data_ptr(), 0, n, s))
        else:
            size = lib.kai_fused_mmq_workspace(0, types, rows, 1, k, m, 1)
            scratch = torch.empty(size, dtype=torch.uint8, device=dev)
            for c in copies:
                ptrs = (ctypes.c_void_p * 1)(c.data_ptr())
                native.check(lib, lib.kai_fused_mmq_run(ptrs, types, rows, 1, x.data_ptr(), 2, k, k, m,
                                                        out.data_ptr(), 0, 0, scratch.data_ptr(), size, 0, s))
    torch.cuda.synchronize()
    print(f"[bench] kernel sample: 3 copies of {src.numel()} bytes, {matrix} {NAMES[qtype]} {n}x{k} x{MIN_COPIES} "
          f"at batch {batches}", flush=True)


PEAK_KINDS = {0: "f16 v_mfma_f32_32x32x16_f16", 1: "f16 v_mfma_f32_16x16x32_f16", 2: "f16 v_mfma_f32_32x32x8_f16",
              3: "int8 v_mfma_i32_32x32x32_i8", 4: "int8 v_mfma_i32_16x16x64_i8"}


def measure_peaks(lib, dev):
    """This device's ceilings, each kernel timed with HIP events on one stream (kai_peaks.h):
    dense MFMA rate per instruction kind at one and at two waves per SIMD (4 independent
    accumulation chains per wave), LDS read bandwidth, and a 2 GiB STREAM-style copy (bytes
    read plus written)."""
    import torch

    from kaillm_amd import native

    props = torch.cuda.get_device_properties(dev)
    cus = props.multi_processor_count
    s = torch.cuda.current_stream()
    guard = torch.zeros(1024, dtype=torch.float32, device=dev)

    def timed(fn, reps=5):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        best = float("inf")
        for _ in range(reps):
            e0.record(s)
            fn()
            e1.record(s)
            torch.cuda.synchronize()
            best = min(best, e0.elapsed_time(e1) * 1e-3)
        return best

    out = {"device": props.name, "cus": cus, "mfma": {}, "method": "best of 5 timed launches after one warm-up"}
    iters = 20000
    for kind, name in PEAK_KINDS.items():
        ops = lib.kai_peak_mfma_ops(kind)
        for threads in (256, 512):  # 1 and 2 waves per SIMD, one workgroup per CU
            blocks = 4 * cus
            t = timed(lambda: native.check(lib, lib.kai_peak_mfma(kind, iters, blocks, threads, guard.data_ptr(),
                                                                  s.cuda_stream)))
            tops = ops * 4 * iters * (threads // 64) * blocks / t / 1e12
            out["mfma"][f"{name} ({threads // 256} wave/SIMD)"] = round(tops, 1)
    lds_iters = 20000
    blocks, threads = 4 * cus, 1024
    t = timed(lambda: native.check(lib, lib.kai_peak_lds(lds_iters, blocks, threads, guard.data_ptr(),
                                                         s.cuda_stream)))
    lds_bytes = lds_iters * 4 * 16 * threads * blocks
    out["lds_read_TBps"] = round(lds_bytes / t / 1e12, 2)
    out["lds_read_bytes_per_cu_clk_at_2400MHz"] = round(lds_bytes / t / cus / 2.4e9, 1)
    n = 1 << 31
    src = torch.empty(n, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    best = {}
    for blocks in (cus * 8, cus * 16, cus * 32):
        t = timed(lambda: native.check(lib, lib.kai_peak_copy(src.data_ptr(), dst.data_ptr(), n, blocks,
                                                              s.cuda_stream)))
        best[blocks] = round(2 * n / t / 1e9, 1)
    out["hbm_copy_GBps"] = max(best.values())
    out["hbm_copy_by_grid"] = best
    torch.cuda.synchronize()
    return out


def cpu_model():
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(w_dev, qtype, n, k, seconds):
    """The oracle's GEMV (the C restatement of the reference arithmetic, OpenMP over rows) on
    the host cores: a bounded sample of the gate/up matrix at M=1."""
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
    return {"value": round(wb / dt / 1e9, 3), "unit": "GB/s", "cores": cores, "threads": cores, "kind": "port",
            "cpu_model": cpu_model(), "build": o.oracle_build_info().decode(),
            "sample": f"oracle_mul_mat_f32 Q4_K {rows}x{k} rows of gate/up, M=1, {reps} calls in {seconds:.0f}s, "
                      f"{dt * 1e3:.2f} ms/call"}


if __name__ == "__main__":
    main()
