"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-configs] [--no-cpu]

A step is one batch-1 decode pass over the Qwen2.5-7B Q4_K_M-style projection
mix (benchmark config 2): gate and up (Q4_K 18944x3584), down (Q6_K
3584x18944) and lm_head (Q6_K 152064x3584).  Weights are seeded synthetic
blocks resident in HBM; two full copies of the step (1.16 GB) alternate, so
no step is served from the 256 MB Infinity Cache.  Prints ONE JSON line:
  value      whole-step algorithmic HBM bytes / step time, in GB/s, with the
             weights in the aligned device layout (repacked once at load time,
             outside the timed region, as a loader does; fq_gemv_packed)
  gguf       the same step through the operator path on the unmodified GGUF
             bytes (fq_matmul_transB, what ops::matmul_transB reaches)
  per_kernel each matrix alone, launches rotating over >= 512 MB of distinct
             copies (HBM-clean), HIP events on the launch stream
  roofline   the dominant kernel (lm_head), algorithmic bytes per launch over
             its average launch time
  configs    every benchmark configuration (0-4) and the Qwen2.5-7B Q4_0
             shapes, each with the reference CPU path timed on a row sample
             (--no-configs skips them)
  cpu_baseline  the reference's own AVX2+OpenMP ops::matmul_transB (compiled
             from its sources into oracle/_ref) on the same step, on this
             host's cores.
"""
from __future__ import annotations

import argparse
import copy
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_FP16_TFLOPS = 2500.0
METRIC = "batch-1 quant GEMV µs + achieved HBM GB/s (% of peak) at 7B shapes"

# (name, dtype, N, K) of config 2
CFG2 = [("gate", 4, 18944, 3584), ("up", 4, 18944, 3584), ("down", 13, 3584, 18944),
        ("lm_head", 13, 152064, 3584)]


def alg_bytes(dtype, N, K, M=1):
    from forge_amd.formats import fmt
    return fmt(dtype).matrix_bytes(N, K) + 4 * M * K + 4 * M * N


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=300)
    p.add_argument("--warmup", type=int, default=100)
    p.add_argument("--no-configs", action="store_true",
                   help="skip the per-configuration lines (configs 0-4, Q4_0 7B shapes)")
    p.add_argument("--formats", action="store_true",
                   help="also time the five formats outside the configs (stderr)")
    p.add_argument("--shape", action="append", default=[], metavar="DTYPE:NxK[:M]",
                   help="only time these shapes (e.g. q4_0:152064x3584:1), GGUF and, for "
                        "M = 1, aligned layout; one JSON line each on stdout")
    p.add_argument("--fused", action="append", default=[], metavar="DTYPE:NxK",
                   help="only time the fused gate/up (aligned, two GEMVs, GGUF) at these "
                        "shapes; one JSON line each on stdout")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--warm-seconds", type=float, default=0.2,
                   help="graph replays before each per-config timing (clock ramp)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--layout", choices=("packed", "gguf"), default="packed",
                   help="device weight layout of the headline value: aligned repack "
                        "(default) or GGUF bytes")
    p.add_argument("--kernel-launch", choices=("graph", "stream"), default="graph",
                   help="per_kernel timing: launches replayed from one HIP graph (default) "
                        "or launched back to back from the host")
    p.add_argument("--graph", action="store_true",
                   help="replay each step as one captured HIP graph instead of four launches")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="before the timed region, copy MIB MiB device-to-device three times "
                        "(a plain copy kernel of known size for scaling HBM byte counters)")
    return p.parse_args()


def cpu_threads():
    """Threads for the CPU baseline: the CPUs this process may run on, at most
    16 (the host share a one-GPU job is granted on the GPU boxes)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_info():
    """CPU model and core counts of this host (from /proc/cpuinfo)."""
    model, cores = None, set()
    phys = core = None
    try:
        for line in open("/proc/cpuinfo"):
            k, _, v = line.partition(":")
            k, v = k.strip(), v.strip()
            if k == "model name" and model is None:
                model = v
            elif k == "physical id":
                phys = v
            elif k == "core id":
                core = v
                cores.add((phys, core))
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return {"cpu_model": model, "physical_cores_host": len(cores) or None,
            "logical_cpus_available": avail}


def cpu_baseline(host_w, host_x, budget_s):
    """Time the reference CPU path on the same config-2 step: at the job's
    thread count (the headline baseline) and on one thread."""
    import oracle
    if not oracle.have_ref():
        return None
    L = oracle.load_ref()
    outs = [np.empty((1, N), np.float32) for (_, _, N, _) in CFG2]
    total = sum(alg_bytes(dt, N, K) for (_, dt, N, K) in CFG2)

    def measure(threads, seconds):
        def step():
            for (name, dt, N, K), w, y in zip(CFG2, host_w, outs):
                rc = L.fqr_matmul_transB(dt, oracle._p(host_x[K]), oracle._p(w), oracle._p(y),
                                         1, K, N, threads)
                if rc != 0:
                    raise RuntimeError(f"reference matmul_transB failed on {name}")

        step()  # warm-up (page-in, OpenMP pool)
        times = []
        t_end = time.perf_counter() + seconds
        while time.perf_counter() < t_end or len(times) < 3:
            t0 = time.perf_counter()
            step()
            times.append(time.perf_counter() - t0)
        return statistics.median(times), len(times)

    threads = cpu_threads()
    med, n = measure(threads, budget_s)
    med1, n1 = measure(1, budget_s / 3)
    info = cpu_info()
    return {
        "value": round(total / med / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"reference ops::matmul_transB (AVX2+OpenMP, oracle/_ref) on the full "
                   f"config-2 step, median of {n} steps in ~{budget_s:.0f} s: "
                   f"{med * 1e3:.2f} ms/step on {threads} threads; one thread "
                   f"{med1 * 1e3:.2f} ms/step ({total / med1 / 1e9:.2f} GB/s, {n1} steps)"),
        "ms_per_step": round(med * 1e3, 3),
        "one_thread_ms_per_step": round(med1 * 1e3, 3),
        **info,
        "threads_note": ("a one-GPU job on the GPU boxes is granted 16 host CPUs; the "
                         "baseline uses min(16, CPUs available)"),
    }


def cpu_config(dtype, w_np, N, K, M, budget_s=1.0):
    """The reference CPU path (oracle/_ref, AVX2 + OpenMP) on a bounded row
    sample of one config: the first rows of the same weights, median over
    ~budget_s, scaled to all N rows (the reference parallelises over rows)."""
    import oracle
    from forge_amd import synth
    if not oracle.have_ref():
        return None
    threads = cpu_threads()
    L = oracle.load_ref()
    x = np.ascontiguousarray(synth.make_x(M, K, 1))
    # about 2^27 multiply-adds per call, at least 64 rows (all when fewer)
    rows = max(min(N, 64), min(N, (1 << 27) // max(1, M * K)))
    w = np.ascontiguousarray(w_np[:rows])
    y = np.empty((M, rows), np.float32)

    def call():
        if L.fqr_matmul_transB(dtype, oracle._p(x), oracle._p(w), oracle._p(y), M, K, rows,
                               threads) != 0:
            raise RuntimeError("reference matmul_transB failed")

    call()
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    us = statistics.median(times) * 1e6 * N / rows
    return {"cpu_ref_us": round(us, 1), "cpu_rows": rows, "cpu_threads": threads}


WARM_SECONDS = 0.2


def time_config(name, dtype, N, K, M, reps=20, pool_bytes=600 << 20, packed=False, cpu=False,
                w_np=None):
    """Average per-call device time of one matmul shape.  `reps` calls over
    rotated weight copies (>= 600 MB, so calls stream from HBM) are captured
    in one HIP graph, so host launch cost does not hide small kernels; the
    graph is replayed and timed with events on its stream."""
    import torch
    from forge_amd import ops, synth
    nb = alg_bytes(dtype, N, K, M) - 4 * M * K - 4 * M * N
    copies = max(2, -(-pool_bytes // nb))
    if w_np is None:
        w_np = synth.make_weights(dtype, N, K, seed=N + K)
    base = torch.from_numpy(w_np.reshape(-1)).cuda()
    ws = [ops.QWeight(base if i == 0 else base.clone(), dtype, N, K) for i in range(copies)]
    if packed:
        ws = [ops.pack_weights(w) for w in ws]
    x = torch.from_numpy(synth.make_x(M, K, 1)).cuda()
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    from forge_amd import _lib
    L = _lib.lib()

    def call(w, stream):
        if packed:
            st = L.fq_gemv_packed(dtype, x.data_ptr(), w.data.data_ptr(), None, 0, y.data_ptr(),
                                  K, N, stream)
        else:
            st = L.fq_matmul_transB(dtype, x.data_ptr(), w.data.data_ptr(), None, 0, 0,
                                    y.data_ptr(), M, K, N, stream)
        if st != 0:
            raise RuntimeError(f"fq_matmul_transB failed with status {st} on {name}")

    # the library keeps its scratch per stream: warm up on the capture stream
    # so nothing is allocated while capturing
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    for i in range(copies):
        call(ws[i], side.cuda_stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        for r in range(reps):
            call(ws[r % copies], side.cuda_stream)
    # replays for ~0.2 s first: the GPU idles while the host makes the
    # weights, and its clocks need that long to come back up
    t_end = time.perf_counter() + WARM_SECONDS
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(10):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (10 * reps)
    b = alg_bytes(dtype, N, K, M)
    line = {"config": name, "layout": "packed" if packed else "gguf", "M": M, "N": N, "K": K,
            "us": round(us, 2),
            "GBs": round(b / us / 1e3, 1), "pct_hbm": round(100 * b / us / 1e3 / PEAK_HBM_GBS, 1)}
    if M > 32:
        tf = 2.0 * M * N * K / us / 1e6
        line["TFLOPs"] = round(tf, 1)
        line["pct_fp16_mfma"] = round(100 * tf / PEAK_FP16_TFLOPS, 2)
    if cpu and not packed:
        c = cpu_config(dtype, w_np, N, K, M)
        if c:
            line.update(c)
            line["gpu_speedup"] = round(c["cpu_ref_us"] / us, 1)
    del g, ws, base
    torch.cuda.empty_cache()
    return line


class StepRunner:
    """The config-2 step on one weight layout: launches on one side stream
    (also the capture stream for --graph)."""

    def __init__(self, layout, host_w, host_x):
        import torch
        from forge_amd import _lib, ops
        self.L = _lib.lib()
        self.packed = layout == "packed"
        self.layout = layout
        self.sets = []
        for _ in range(2):  # two full copies of the step alternate
            ws = [ops.QWeight(torch.from_numpy(w.reshape(-1)).cuda(), dt, N, K)
                  for w, (_, dt, N, K) in zip(host_w, CFG2)]
            self.sets.append([ops.pack_weights(w) for w in ws] if self.packed else ws)
            del ws
        torch.cuda.synchronize()
        self.xs = {K: torch.from_numpy(v).cuda() for K, v in host_x.items()}
        self.ys = [torch.empty((N,), dtype=torch.float32, device="cuda") for (_, _, N, _) in CFG2]
        self.side = torch.cuda.Stream()
        self.side.wait_stream(torch.cuda.current_stream())

    def launch(self, i, w):
        (name, dt, N, K) = CFG2[i]
        st = self.side.cuda_stream
        if self.packed:
            rc = self.L.fq_gemv_packed(dt, self.xs[K].data_ptr(), w.data.data_ptr(), None, 0,
                                       self.ys[i].data_ptr(), K, N, st)
        else:  # the operator path: ops::matmul_transB's device branch
            rc = self.L.fq_matmul_transB(dt, self.xs[K].data_ptr(), w.data.data_ptr(), None, 0,
                                         0, self.ys[i].data_ptr(), 1, K, N, st)
        if rc != 0:
            raise RuntimeError(f"GEMV ({name}, {self.layout}) failed with status {rc}")

    def time_steps(self, steps, warmup, graph=False):
        """ms per step over `steps` steps after `warmup` untimed ones: HIP
        events on the launch stream around the whole region."""
        import torch
        nk = len(CFG2)
        # steps for ~WARM_SECONDS first (not counted as warm-up steps): the GPU
        # idles while the host makes the weights, and its clocks need that
        # long to come back up
        t_end = time.perf_counter() + WARM_SECONDS
        s = 0
        while time.perf_counter() < t_end:
            for i in range(nk):
                self.launch(i, self.sets[s % 2][i])
            s += 1
            if s % 16 == 0:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
        for s in range(warmup):
            for i in range(nk):
                self.launch(i, self.sets[s % 2][i])
        torch.cuda.synchronize()
        graphs = []
        if graph:
            for c in range(2):
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.side):
                    for i in range(nk):
                        self.launch(i, self.sets[c][i])
                graphs.append(g)
            for g in graphs:
                g.replay()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        with torch.cuda.stream(self.side):
            t0.record()
            for s in range(steps):
                if graphs:
                    graphs[s % 2].replay()
                else:
                    for i in range(nk):
                        self.launch(i, self.sets[s % 2][i])
            t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / steps

    def time_kernels(self, launches=100, pool_bytes=512 << 20, graph=True, reps=5):
        """Average launch time of each matrix alone: `reps` x `launches`
        back-to-back launches rotating over >= pool_bytes of distinct copies
        of that matrix
        (so every launch streams from HBM, not the Infinity Cache).  With
        `graph` the launches are captured in one HIP graph and replayed, so
        the host's dispatch gaps between back-to-back launches (a few µs each)
        are not counted as kernel time; events on the launch stream either
        way."""
        import torch
        out = {}
        for i, (name, dt, N, K) in enumerate(CFG2):
            nb = alg_bytes(dt, N, K) - 4 * K - 4 * N
            copies = [self.sets[0][i], self.sets[1][i]]
            while len(copies) * nb < pool_bytes:
                w = copies[len(copies) % 2]
                c = copy.copy(w)
                c.data = w.data.clone()
                copies.append(c)
            for c in copies:
                self.launch(i, c)
            torch.cuda.synchronize()
            g = None
            if graph:
                g = torch.cuda.CUDAGraph()
                with torch.cuda.graph(g, stream=self.side):
                    for s in range(launches):
                        self.launch(i, copies[s % len(copies)])
            # replays (or launches) for ~WARM_SECONDS before the timed region,
            # as for the per-config timings: clocks ramp back up after the
            # host-side copies
            t_end = time.perf_counter() + WARM_SECONDS
            while True:
                if g is not None:
                    g.replay()
                else:
                    for s in range(launches):
                        self.launch(i, copies[s % len(copies)])
                torch.cuda.synchronize()
                if time.perf_counter() >= t_end:
                    break
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            with torch.cuda.stream(self.side):
                e0.record()
                for _ in range(reps):
                    if g is not None:
                        g.replay()
                    else:
                        for s in range(launches):
                            self.launch(i, copies[s % len(copies)])
                e1.record()
            torch.cuda.synchronize()
            del g
            us = e0.elapsed_time(e1) * 1e3 / (reps * launches)
            b = alg_bytes(dt, N, K)
            out[name] = {"us": round(us, 2), "GBs": round(b / us / 1e3, 1),
                         "pct_hbm": round(100 * b / us / 1e3 / PEAK_HBM_GBS, 1),
                         "alg_bytes": b, "rotation_copies": len(copies)}
            del copies
            torch.cuda.empty_cache()
        return out

    def free(self):
        import torch
        self.sets = []
        torch.cuda.synchronize()
        torch.cuda.empty_cache()


def main():
    global WARM_SECONDS
    args = parse()
    WARM_SECONDS = args.warm_seconds
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this hot path is single-GPU by design "
              "(sharding the rows across GPUs is a design, not implemented); "
              "run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from forge_amd import synth

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)

    if args.shape or args.fused:
        from forge_amd import formats as F
        if args.copy_calibration:
            copy_calibration(args.copy_calibration)
        names = {f.name.lower(): dt for dt, f in F.FORMATS.items()}
        for spec in args.fused:
            parts = spec.split(":")
            N, K = (int(v) for v in parts[1].lower().split("x"))
            print(json.dumps(time_fused(spec, names[parts[0].lower()], N, K)), flush=True)
        for spec in args.shape:
            parts = spec.split(":")
            dt = names[parts[0].lower()]
            N, K = (int(v) for v in parts[1].lower().split("x"))
            M = int(parts[2]) if len(parts) > 2 else 1
            w_np = synth.make_weights(dt, N, K, seed=N + K)
            line = time_config(spec, dt, N, K, M, cpu=not args.no_cpu, w_np=w_np)
            if M == 1 and dt in (F.Q4_0, F.Q4_1, F.Q8_0, F.Q4_K, F.Q6_K):
                pk = time_config(spec, dt, N, K, M, packed=True, w_np=w_np)
                line["packed_us"] = pk["us"]
                line["packed_pct_hbm"] = pk["pct_hbm"]
            print(json.dumps(line), flush=True)
        return

    # ---- inputs: seeded blocks, two device copies of the whole step per layout
    host_w = [synth.make_weights(dt, N, K, seed=2000 + i) for i, (_, dt, N, K) in enumerate(CFG2)]
    host_x = {K: synth.make_x(1, K, seed=2100 + K) for K in {K for (_, _, _, K) in CFG2}}
    step_bytes = sum(alg_bytes(dt, N, K) for (_, dt, N, K) in CFG2)
    other = "gguf" if args.layout == "packed" else "packed"
    results = {}
    for layout in (args.layout, other):
        r = StepRunner(layout, host_w, host_x)
        if layout == args.layout and args.copy_calibration:
            copy_calibration(args.copy_calibration)
        ms = r.time_steps(args.steps, args.warmup, graph=args.graph)
        kern = r.time_kernels(graph=args.kernel_launch == "graph")
        results[layout] = (ms, kern)
        r.free()
        del r

    ms_per_step, per_kernel = results[args.layout]
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    lm = per_kernel["lm_head"]
    packed = args.layout == "packed"
    roofline = {"bound": "hbm", "achieved": lm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(lm["GBs"] / PEAK_HBM_GBS, 4),
                "traffic": measured_traffic() if packed else None,
                "kernel": ("gemvp_kernel<Q6_K>, aligned layout" if packed
                           else "gemvp_kernel<Q6_K, GGUF slices>")
                + " (lm_head 152064x3584, M=1)",
                "alg_bytes_per_launch": lm["alg_bytes"]}
    g_ms, g_kern = results[other]
    g_value = step_bytes / (g_ms * 1e-3) / 1e9
    alt = {"layout": other,
           "entry_point": "fq_matmul_transB" if other == "gguf" else "fq_gemv_packed",
           "ms_per_step": round(g_ms, 4), "value": round(g_value, 1),
           "pct_hbm_peak": round(100 * g_value / PEAK_HBM_GBS, 1), "per_kernel": g_kern}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(host_w, host_x, args.cpu_seconds)

    configs = None
    if not args.no_configs:
        configs = all_configs(cpu=not args.no_cpu)

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("GGUF Q4_K/Q6_K integer codes x fp32 activations carried as three int8 limbs "
                  "per 32-element unit under one power-of-two scale (about 2^-21 of the "
                  "unit's max); exact int32 dot products, fp32 block scales and accumulation"),
        "data": "synthetic (seeded GGUF blocks: fp16 scales |N(0,0.02)|, uniform codes; x~N(0,1))",
        "config": {"workload": "cfg2: Qwen2.5-7B Q4_K_M decode projections at M=1 "
                               "(gate,up Q4_K 18944x3584; down Q6_K 3584x18944; "
                               "lm_head Q6_K 152064x3584)",
                   "M": 1, "layout": args.layout,
                   "entry_point": "fq_gemv_packed" if packed else "fq_matmul_transB",
                   "launch": "hip_graph" if args.graph else "stream",
                   "step_alg_bytes": step_bytes,
                   "pct_hbm_peak": round(100 * value / PEAK_HBM_GBS, 1),
                   "per_kernel": per_kernel,
                   "per_kernel_launch": "hip_graph" if args.kernel_launch == "graph" else "stream"},
        other: alt,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "configs": configs,
    }
    print(json.dumps(out), flush=True)

    if args.formats:
        for line in format_lines(cpu=not args.no_cpu):
            print(json.dumps(line), file=sys.stderr, flush=True)


def copy_calibration(mib):
    """Three device-to-device copies of `mib` MiB: a plain copy kernel of known
    size, for scaling the HBM byte counters of the same profiler run."""
    import torch
    src = torch.ones(mib << 18, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst
    torch.cuda.empty_cache()


def measured_traffic():
    """HBM bytes per lm_head launch from the committed rocprofv3 --pmc runs
    (the JSON block of profiles/lm_head_q6k_traffic.md), or None when not
    measured."""
    path = os.path.join(ROOT, "profiles", "lm_head_q6k_traffic.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(block).get("hbm_bytes_per_launch")
    except (OSError, ValueError, IndexError):
        return None


def time_fused(name, dtype, N, K, reps=20, pool_bytes=600 << 20):
    """Average device time of the fused gate/up (fq_ffn_up_fused_packed, one
    launch) next to the two separate packed GEMVs and to the operator path's
    fq_ffn_up_fused on the GGUF bytes, all HIP-graph replays."""
    import torch
    from forge_amd import _lib, ops, synth
    L = _lib.lib()
    nb = 2 * (alg_bytes(dtype, N, K) - 4 * K - 4 * N)
    copies = max(2, -(-pool_bytes // nb))
    pairs = []
    for c in range(copies):
        g = ops.QWeight.from_numpy(synth.make_weights(dtype, N, K, seed=3 * c), dtype, N, K)
        u = ops.QWeight.from_numpy(synth.make_weights(dtype, N, K, seed=3 * c + 1), dtype, N, K)
        pairs.append((ops.pack_weights(g), ops.pack_weights(u), g, u))
        del g, u
    x = torch.from_numpy(synth.make_x(1, K, 1)).cuda()
    y = torch.empty(N, device="cuda")
    y2 = torch.empty(N, device="cuda")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())

    def fused(p, st):
        assert L.fq_ffn_up_fused_packed(dtype, x.data_ptr(), p[0].data.data_ptr(),
                                        p[1].data.data_ptr(), y.data_ptr(), K, N, st) == 0

    def separate(p, st):
        for w, out in ((p[0], y), (p[1], y2)):
            assert L.fq_gemv_packed(dtype, x.data_ptr(), w.data.data_ptr(), None, 0,
                                    out.data_ptr(), K, N, st) == 0

    def gguf_fused(p, st):  # the operator path: fq_ffn_up_fused on the GGUF bytes
        assert L.fq_ffn_up_fused(dtype, x.data_ptr(), p[2].data.data_ptr(), p[3].data.data_ptr(),
                                 y.data_ptr(), 1, K, N, st) == 0

    out = {"config": name, "M": 1, "N": N, "K": K, "op": "ffn_up_fused (gate+up+SiLU)"}
    for label, fn in (("fused_us", fused), ("two_gemv_us", separate),
                      ("gguf_fused_us", gguf_fused)):
        for p in pairs:
            fn(p, side.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            for r in range(reps):
                fn(pairs[r % copies], side.cuda_stream)
        t_end = time.perf_counter() + WARM_SECONDS  # clocks back up after the host-side setup
        while time.perf_counter() < t_end:
            g.replay()
            torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(10):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        out[label] = round(e0.elapsed_time(e1) * 1e3 / (10 * reps), 2)
        del g
    b = 2 * alg_bytes(dtype, N, K) - 4 * K
    out["fused_GBs"] = round(b / out["fused_us"] / 1e3, 1)
    out["fused_pct_hbm"] = round(100 * b / out["fused_us"] / 1e3 / PEAK_HBM_GBS, 1)
    del pairs
    torch.cuda.empty_cache()
    return out


def all_configs(cpu=False):
    """Every benchmark configuration on the operator path (fq_matmul_transB on
    GGUF bytes; M = 1 rows also on the aligned layout), plus the Qwen2.5-7B
    Q4_0 shapes of the reference's published decode workload, each beside the
    reference CPU path on a row sample.  Compact keys: us, GBs, pct_hbm (of
    8 TB/s); M = 512 adds TFLOPs and pct_fp16_mfma (of 2.5 PFLOP/s dense, two
    fp16 MFMAs issued per product)."""
    Q4_0, Q8_0, Q4_K, Q6_K = 2, 7, 4, 13
    lines = []

    def add(name, dt, N, K, M, packed_too=False, reps=20):
        from forge_amd import synth
        w_np = synth.make_weights(dt, N, K, seed=N + K)
        line = time_config(name, dt, N, K, M, reps=reps, cpu=cpu, w_np=w_np)
        if packed_too:
            pk = time_config(name, dt, N, K, M, reps=reps, packed=True, w_np=w_np)
            line["packed_us"] = pk["us"]
            line["packed_pct_hbm"] = pk["pct_hbm"]
        lines.append(line)

    add("cfg0", Q4_0, 5632, 2048, 1, packed_too=True)
    for dt in (Q4_0, Q8_0):
        for n, N, K in [("q", 2048, 2048), ("k", 256, 2048), ("o", 2048, 2048),
                        ("gate", 5632, 2048), ("down", 2048, 5632)]:
            add(f"cfg1-{n}-{'q4_0' if dt == Q4_0 else 'q8_0'}", dt, N, K, 1)
    for n, dt, N, K in [("gate", Q4_K, 18944, 3584), ("down", Q6_K, 3584, 18944),
                        ("lm_head", Q6_K, 152064, 3584)]:
        add(f"cfg2-{n}", dt, N, K, 1, packed_too=True)
    for M in (1, 2, 3, 4, 8, 16):
        add("cfg3", Q4_K, 14336, 4096, M, packed_too=M == 1)
    for dt in (Q8_0, Q4_0):
        for N in (4096, 14336):
            add(f"cfg4-{'q8_0' if dt == Q8_0 else 'q4_0'}", dt, N, 4096, 512, reps=10)
    # the reference's published workload: Qwen2.5-7B in Q4_0
    for n, N, K in [("up", 18944, 3584), ("down", 3584, 18944), ("lm_head", 152064, 3584)]:
        add(f"q4_0-7b-{n}", Q4_0, N, K, 1, packed_too=True)
    lines.append(time_fused("cfg2-gate+up", Q4_K, 18944, 3584))
    return lines


def format_lines(cpu=False):
    """The formats outside the benchmark configs, at the 7B gate shape."""
    lines = []
    for name, dt in (("q5_0", 8), ("q5_1", 9), ("q3_k", 11), ("q5_k", 12), ("iq4_nl", 17)):
        for M in (1, 8):
            lines.append(time_config(f"fmt-{name}", dt, 18944, 3584, M, cpu=cpu))
    return lines


if __name__ == "__main__":
    main()
