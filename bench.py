"""Benchmark of the quantized-matmul hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs]

A step is one batch-1 decode pass over the Qwen2.5-7B Q4_K_M-style projection
mix (benchmark config 2): gate and up (Q4_K 18944x3584), down (Q6_K
3584x18944) and lm_head (Q6_K 152064x3584), each one fq_gemv call through
the C ABI.  Weights are seeded synthetic blocks resident in HBM; two full
copies (1.16 GB) alternate between steps so no step can be served from the
256 MB Infinity Cache.  Prints ONE JSON line:
  value      whole-step algorithmic HBM bytes / step time, in GB/s
  roofline   the dominant kernel (lm_head), algorithmic bytes per launch over
             its average launch time (HIP events on the launch stream)
  cpu_baseline  the reference's own AVX2+OpenMP ops::matmul_transB (compiled
             from its sources into oracle/_ref) on the same step, on this
             host's cores.
--configs additionally prints per-config lines (configs 0-4) to stderr.
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
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--configs", action="store_true", help="also time configs 0-4 (stderr)")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
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


def time_config(name, dtype, N, K, M, reps=40, pool_bytes=600 << 20):
    """Median per-call device time of one matmul shape over rotated copies."""
    import torch
    from forge_amd import ops, synth
    nb = alg_bytes(dtype, N, K, M) - 4 * M * K - 4 * M * N
    copies = max(2, -(-pool_bytes // nb))
    w_np = synth.make_weights(dtype, N, K, seed=N + K)
    base = torch.from_numpy(w_np.reshape(-1)).cuda()
    ws = [ops.QWeight(base if i == 0 else base.clone(), dtype, N, K) for i in range(copies)]
    x = torch.from_numpy(synth.make_x(M, K, 1)).cuda()
    for i in range(copies):
        ops.matmul_transB(x, ws[i])
    torch.cuda.synchronize()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(reps)]
    for r in range(reps):
        ev[r][0].record()
        ops.matmul_transB(x, ws[r % copies])
        ev[r][1].record()
    torch.cuda.synchronize()
    us = statistics.median(a.elapsed_time(b) * 1e3 for a, b in ev)
    b = alg_bytes(dtype, N, K, M)
    line = {"config": name, "M": M, "N": N, "K": K, "us": round(us, 2),
            "GBs": round(b / us / 1e3, 1), "pct_hbm": round(100 * b / us / 1e3 / PEAK_HBM_GBS, 1)}
    if M > 32:
        tf = 2.0 * M * N * K / us / 1e6
        line["TFLOPs"] = round(tf, 1)
        line["pct_fp16_mfma"] = round(100 * tf / PEAK_FP16_TFLOPS, 2)
    del ws, base
    torch.cuda.empty_cache()
    return line


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this hot path is single-GPU by design "
              "(row-sharding across GPUs is described in DESIGN.md, not implemented); "
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
    sets = []
    for c in range(2):
        sets.append([ops.QWeight(torch.from_numpy(w.reshape(-1)).cuda(), dt, N, K)
                     for w, (_, dt, N, K) in zip(host_w, CFG2)])
    xs = {K: torch.from_numpy(v).cuda() for K, v in host_x.items()}
    ys = [torch.empty((N,), dtype=torch.float32, device="cuda") for (_, _, N, _) in CFG2]

    from forge_amd import _lib
    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def launch(i, s):
        (name, dt, N, K) = CFG2[i]
        w = sets[s][i]
        st = L.fq_gemv(dt, xs[K].data_ptr(), w.data.data_ptr(), ys[i].data_ptr(), K, N, stream)
        if st != 0:
            raise RuntimeError(f"fq_gemv({name}) failed with status {st}")

    for s in range(args.warmup):
        for i in range(len(CFG2)):
            launch(i, s % 2)
    torch.cuda.synchronize()

    # ---- timed region: K steps, HIP events around every launch
    nk = len(CFG2)
    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(nk)] for _ in range(args.steps)]
    t_start, t_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for s in range(args.steps):
        for i in range(nk):
            ev[s][i][0].record()
            launch(i, s % 2)
            ev[s][i][1].record()
    t_end.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_end)
    ms_per_step = total_ms / args.steps
    kern_us = [statistics.mean(ev[s][i][0].elapsed_time(ev[s][i][1]) * 1e3
                               for s in range(args.steps)) for i in range(nk)]

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
                "kernel": "gemv_kernel<Q6_K> (lm_head 152064x3584, M=1)",
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
                   "M": 1, "step_alg_bytes": step_bytes,
                   "pct_hbm_peak": round(100 * value / PEAK_HBM_GBS, 1),
                   "per_kernel": per_kernel},
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)

    if args.configs:
        for line in all_configs():
            print(json.dumps(line), file=sys.stderr, flush=True)


def measured_traffic():
    """HBM bytes per lm_head launch from the committed rocprofv3 --pmc runs
    (profiles/lm_head_q6k_traffic.json), or None when not measured."""
    path = os.path.join(ROOT, "profiles", "lm_head_q6k_traffic.json")
    if not os.path.exists(path):
        return None
    try:
        with open(path) as f:
            return json.load(f).get("hbm_bytes_per_launch")
    except (OSError, ValueError):
        return None


def all_configs():
    Q4_0, Q8_0, Q4_K, Q6_K = 2, 7, 4, 13
    lines = [time_config("cfg0", Q4_0, 5632, 2048, 1)]
    for dt in (Q4_0, Q8_0):
        for n, N, K in [("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
                        ("gate", 5632, 2048), ("up", 5632, 2048), ("down", 2048, 5632)]:
            lines.append(time_config(f"cfg1-{n}-{'q4_0' if dt == Q4_0 else 'q8_0'}", dt, N, K, 1))
    for n, dt, N, K in [("gate", Q4_K, 18944, 3584), ("down", Q6_K, 3584, 18944),
                        ("lm_head", Q6_K, 152064, 3584)]:
        lines.append(time_config(f"cfg2-{n}", dt, N, K, 1))
    for M in (1, 2, 4, 8, 16):
        lines.append(time_config("cfg3", Q4_K, 14336, 4096, M))
    for dt in (Q8_0, Q4_0):
        for N in (4096, 14336):
            lines.append(time_config(f"cfg4-{'q8_0' if dt == Q8_0 else 'q4_0'}", dt, N, 4096, 512,
                                     reps=10))
    return lines


if __name__ == "__main__":
    main()
