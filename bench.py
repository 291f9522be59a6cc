"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs]

A step is one batch-1 decode pass over the Qwen2.5-7B Q4_K_M-style projection
mix (benchmark config 2): gate and up (Q4_K 18944x3584), down (Q6_K
3584x18944) and lm_head (Q6_K 152064x3584), each one fq_gemv_packed call
through the C ABI (--layout gguf: fq_gemv on the unmodified GGUF bytes).
Weights are seeded synthetic blocks, repacked once into the aligned device
layout at load time (outside the timed region, as a loader does) and resident
in HBM; two full copies (1.16 GB) alternate between steps so no step can be
served from the 256 MB Infinity Cache.  Prints ONE JSON line:
  value      whole-step algorithmic HBM bytes / step time, in GB/s
  roofline   the dominant kernel (lm_head), algorithmic bytes per launch over
             its average launch time (K launches back to back, HIP events on
             the launch stream around them)
  cpu_baseline  the reference's own AVX2+OpenMP ops::matmul_transB (compiled
             from its sources into oracle/_ref) on the same step, on this
             host's cores.
--configs additionally prints per-config lines (configs 0-4) to stderr, each
with the reference CPU path timed on a row sample of the same weights
(skipped with --no-cpu).
"""
from __future__ import annotations

import argparse
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
    p.add_argument("--configs", action="store_true", help="also time configs 0-4 (stderr)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--layout", choices=("packed", "gguf"), default="packed",
                   help="device weight layout: aligned repack (default) or GGUF bytes")
    p.add_argument("--graph", action="store_true",
                   help="replay each step as one captured HIP graph instead of four launches")
    p.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                   help="before the timed region, copy MIB MiB device-to-device three times "
                        "(a plain copy kernel of known size for scaling HBM byte counters)")
    return p.parse_args()


def cpu_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_baseline(host_w, host_x, budget_s):
    """Time the reference CPU path on the same config-2 step."""
    import oracle
    if not oracle.have_ref():
        return None
    threads = cpu_threads()
    L = oracle.load_ref()
    outs = [np.empty((1, N), np.float32) for (_, _, N, _) in CFG2]

    def step():
        for (name, dt, N, K), w, y in zip(CFG2, host_w, outs):
            rc = L.fqr_matmul_transB(dt, oracle._p(host_x[K]), oracle._p(w), oracle._p(y),
                                     1, K, N, threads)
            if rc != 0:
                raise RuntimeError(f"reference matmul_transB failed on {name}")

    step()  # warm-up (page-in, OpenMP pool)
    times = []
    t_end = time.perf_counter() + budget_s
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    total = sum(alg_bytes(dt, N, K) for (_, dt, N, K) in CFG2)
    return {
        "value": round(total / med / 1e9, 2),
        "unit": "GB/s",
        "cores": threads,
        "kind": "reference",
        "sample": (f"reference ops::matmul_transB (AVX2+OpenMP, oracle/_ref) on the full "
                   f"config-2 step, median of {len(times)} steps in ~{budget_s:.0f} s; "
                   f"{med * 1e3:.2f} ms/step"),
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


def time_config(name, dtype, N, K, M, reps=20, pool_bytes=600 << 20, packed=False, cpu=False):
    """Average per-call device time of one matmul shape.  `reps` calls over
    rotated weight copies (>= 600 MB, so calls stream from HBM) are captured
    in one HIP graph, so host launch cost does not hide small kernels; the
    graph is replayed and timed with events on its stream."""
    import torch
    from forge_amd import ops, synth
    nb = alg_bytes(dtype, N, K, M) - 4 * M * K - 4 * M * N
    copies = max(2, -(-pool_bytes // nb))
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
    g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(3):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / (3 * reps)
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


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this hot path is single-GPU by design "
              "(sharding the rows across GPUs is a design, not implemented); "
              "run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    from forge_amd import ops, synth

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)

    # ---- inputs: seeded blocks, two device copies of the whole step
    host_w = [synth.make_weights(dt, N, K, seed=2000 + i) for i, (_, dt, N, K) in enumerate(CFG2)]
    host_x = {K: synth.make_x(1, K, seed=2100 + K) for K in {K for (_, _, _, K) in CFG2}}
    packed = args.layout == "packed"
    sets = []
    for c in range(2):
        ws = [ops.QWeight(torch.from_numpy(w.reshape(-1)).cuda(), dt, N, K)
              for w, (_, dt, N, K) in zip(host_w, CFG2)]
        sets.append([ops.pack_weights(w) for w in ws] if packed else ws)
        del ws
    torch.cuda.synchronize()
    xs = {K: torch.from_numpy(v).cuda() for K, v in host_x.items()}
    ys = [torch.empty((N,), dtype=torch.float32, device="cuda") for (_, _, N, _) in CFG2]

    from forge_amd import _lib
    L = _lib.lib()
    # every launch goes to one side stream, which is also the capture stream
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    stream = side.cuda_stream

    def launch(i, s):
        (name, dt, N, K) = CFG2[i]
        w = sets[s][i]
        if packed:
            st = L.fq_gemv_packed(dt, xs[K].data_ptr(), w.data.data_ptr(), None, 0,
                                  ys[i].data_ptr(), K, N, stream)
        else:
            st = L.fq_gemv(dt, xs[K].data_ptr(), w.data.data_ptr(), ys[i].data_ptr(), K, N,
                           stream)
        if st != 0:
            raise RuntimeError(f"GEMV ({name}, {args.layout}) failed with status {st}")

    for s in range(args.warmup):
        for i in range(len(CFG2)):
            launch(i, s % 2)
    torch.cuda.synchronize()
    if args.copy_calibration:
        src = torch.ones(args.copy_calibration << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # ---- timed region: K steps, HIP events on the launch stream around the
    # whole region.  The step's four kernels are launched one by one; --graph
    # replays each step as one captured HIP graph instead (measured no faster
    # on MI355X for these launch sizes).
    nk = len(CFG2)
    graphs = []
    if args.graph:
        for c in range(2):
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g, stream=side):
                for i in range(nk):
                    launch(i, c)
            graphs.append(g)
        for g in graphs:
            g.replay()
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        t_start.record()
        for s in range(args.steps):
            if graphs:
                graphs[s % 2].replay()
            else:
                for i in range(nk):
                    launch(i, s % 2)
        t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / args.steps

    # ---- per-kernel average launch time: each matrix alone, K launches back
    # to back (alternating the two weight copies), events around the loop
    kern_us = []
    for i in range(nk):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        launch(i, 1)
        with torch.cuda.stream(side):
            e0.record()
            for s in range(args.steps):
                launch(i, s % 2)
            e1.record()
        torch.cuda.synchronize()
        kern_us.append(e0.elapsed_time(e1) * 1e3 / args.steps)

    step_bytes = sum(alg_bytes(dt, N, K) for (_, dt, N, K) in CFG2)
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    per_kernel = {}
    for (name, dt, N, K), us in zip(CFG2, kern_us):
        b = alg_bytes(dt, N, K)
        per_kernel[name] = {"us": round(us, 2), "GBs": round(b / us / 1e3, 1),
                            "pct_hbm": round(100 * b / us / 1e3 / PEAK_HBM_GBS, 1),
                            "alg_bytes": b}
    lm = per_kernel["lm_head"]
    roofline = {"bound": "hbm", "achieved": lm["GBs"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(lm["GBs"] / PEAK_HBM_GBS, 4), "traffic": measured_traffic(),
                "kernel": ("gemvp_kernel<Q6_K>" if packed else "gemv1r_kernel<Q6_K>")
                + " (lm_head 152064x3584, M=1)",
                "alg_bytes_per_launch": lm["alg_bytes"]}

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(host_w, host_x, args.cpu_seconds)

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
        "dtype": "fp32 activations x GGUF Q4_K/Q6_K weights (fp32 accumulate)",
        "data": "synthetic (seeded GGUF blocks: fp16 scales |N(0,0.02)|, uniform codes; x~N(0,1))",
        "config": {"workload": "cfg2: Qwen2.5-7B Q4_K_M decode projections at M=1 "
                               "(gate,up Q4_K 18944x3584; down Q6_K 3584x18944; "
                               "lm_head Q6_K 152064x3584)",
                   "M": 1, "layout": args.layout,
                   "launch": "hip_graph" if args.graph else "stream",
                   "step_alg_bytes": step_bytes,
                   "pct_hbm_peak": round(100 * value / PEAK_HBM_GBS, 1),
                   "per_kernel": per_kernel},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)

    if args.configs:
        for line in all_configs(cpu=not args.no_cpu):
            print(json.dumps(line), file=sys.stderr, flush=True)


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
    launch) next to the two separate packed GEMVs, both HIP-graph replays."""
    import torch
    from forge_amd import _lib, ops, synth
    L = _lib.lib()
    nb = 2 * (alg_bytes(dtype, N, K) - 4 * K - 4 * N)
    copies = max(2, -(-pool_bytes // nb))
    pairs = []
    for c in range(copies):
        g = ops.QWeight.from_numpy(synth.make_weights(dtype, N, K, seed=3 * c), dtype, N, K)
        u = ops.QWeight.from_numpy(synth.make_weights(dtype, N, K, seed=3 * c + 1), dtype, N, K)
        pairs.append((ops.pack_weights(g), ops.pack_weights(u)))
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

    out = {"config": name, "M": 1, "N": N, "K": K, "op": "ffn_up_fused (gate+up+SiLU)"}
    for label, fn in (("fused_us", fused), ("two_gemv_us", separate)):
        for p in pairs:
            fn(p, side.cuda_stream)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            for r in range(reps):
                fn(pairs[r % copies], side.cuda_stream)
        g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(3):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        out[label] = round(e0.elapsed_time(e1) * 1e3 / (3 * reps), 2)
        del g
    b = 2 * alg_bytes(dtype, N, K) - 4 * K
    out["fused_GBs"] = round(b / out["fused_us"] / 1e3, 1)
    out["fused_pct_hbm"] = round(100 * b / out["fused_us"] / 1e3 / PEAK_HBM_GBS, 1)
    del pairs
    torch.cuda.empty_cache()
    return out


def all_configs(cpu=False):
    Q4_0, Q8_0, Q4_K, Q6_K = 2, 7, 4, 13
    lines = []
    for pk in (False, True):
        lines.append(time_config("cfg0", Q4_0, 5632, 2048, 1, packed=pk, cpu=cpu))
        for dt in (Q4_0, Q8_0):
            for n, N, K in [("q", 2048, 2048), ("k", 256, 2048), ("o", 2048, 2048),
                            ("gate", 5632, 2048), ("down", 2048, 5632)]:
                lines.append(time_config(f"cfg1-{n}-{'q4_0' if dt == Q4_0 else 'q8_0'}", dt, N,
                                         K, 1, packed=pk, cpu=cpu))
        for n, dt, N, K in [("gate", Q4_K, 18944, 3584), ("down", Q6_K, 3584, 18944),
                            ("lm_head", Q6_K, 152064, 3584)]:
            lines.append(time_config(f"cfg2-{n}", dt, N, K, 1, packed=pk, cpu=cpu))
    lines.append(time_fused("cfg2-gate+up", Q4_K, 18944, 3584))
    lines.append(time_fused("cfg1-gate+up-q4_0", Q4_0, 5632, 2048))
    lines.append(time_config("cfg3", Q4_K, 14336, 4096, 1, packed=True))
    for M in (1, 2, 4, 8, 16):
        lines.append(time_config("cfg3", Q4_K, 14336, 4096, M, cpu=cpu))
    for dt in (Q8_0, Q4_0):
        for N in (4096, 14336):
            lines.append(time_config(f"cfg4-{'q8_0' if dt == Q8_0 else 'q4_0'}", dt, N, 4096, 512,
                                     reps=10, cpu=cpu))
    # the formats outside the benchmark configs, at the 7B gate shape (GGUF layout)
    for name, dt in (("q5_0", 8), ("q5_1", 9), ("q3_k", 11), ("q5_k", 12), ("iq4_nl", 17)):
        for M in (1, 8):
            lines.append(time_config(f"fmt-{name}", dt, 18944, 3584, M, cpu=cpu))
    return lines


if __name__ == "__main__":
    main()
