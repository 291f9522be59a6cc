"""Summarise a rocprofv3 kernel trace per kernel launch shape.

    python -m forge_amd.profsum <prefix>_kernel_trace.csv [--title TEXT]
    python -m forge_amd.profsum --traffic FETCH.csv WRITE.csv --copy-mib MIB \
        --kernel NAME_PREFIX --grid G --lds B

rocprofv3's own ``--stats`` table averages every launch of one kernel symbol,
but one template instance serves several matrices (the Q6_K GEMV runs both
down 3584x18944 and lm_head 152064x3584).  This groups the dispatches by
(kernel, grid, work-group, LDS bytes) instead -- LDS bytes follow the row
length K -- and prints a Markdown table of calls and durations in µs.
"""
from __future__ import annotations

import argparse
import collections
import csv
import statistics


def summarise(path: str):
    groups = collections.OrderedDict()
    for r in csv.DictReader(open(path)):
        key = (r["Kernel_Name"], int(r["Grid_Size_X"]), int(r["Workgroup_Size_X"]),
               int(r["LDS_Block_Size"]), int(r["VGPR_Count"]), int(r["Scratch_Size"]))
        groups.setdefault(key, []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    rows = []
    for (name, grid, wg, lds, vgpr, scratch), d in groups.items():
        rows.append({"kernel": name, "grid": grid, "wg": wg, "lds": lds, "vgpr": vgpr,
                     "scratch": scratch, "calls": len(d), "avg_us": statistics.mean(d),
                     "median_us": statistics.median(d), "min_us": min(d), "max_us": max(d)})
    rows.sort(key=lambda r: -r["avg_us"] * r["calls"])
    return rows


def short(name: str) -> str:
    name = name.replace("fq::(anonymous namespace)::", "").replace("void ", "")
    return name.split("(")[0] if "(" in name else name


def counter_groups(path: str):
    """Mean counter value per (kernel, grid, LDS bytes) of a --pmc CSV."""
    g = collections.defaultdict(list)
    for r in csv.DictReader(open(path)):
        g[(short(r["Kernel_Name"]), int(r["Grid_Size"]), int(r["LDS_Block_Size"]))].append(
            float(r["Counter_Value"]))
    return {k: statistics.mean(v) for k, v in g.items()}


def traffic(fetch_csv, write_csv, copy_mib, kernel, grid, lds):
    """HBM bytes per launch of one kernel shape from FETCH_SIZE and WRITE_SIZE
    (KiB per dispatch), each scaled by what the same counter reads for the
    plain device-to-device copy of copy_mib MiB that ran in the same process
    (it reads and writes copy_mib MiB)."""
    f, w = counter_groups(fetch_csv), counter_groups(write_csv)
    kib = copy_mib * 1024.0

    def copy_val(path):
        # the calibration copy is by far the largest single copy dispatch
        # (copies of other sizes share its kernel name and grid, so group
        # means would mix them in)
        return max(float(r["Counter_Value"]) for r in csv.DictReader(open(path))
                   if "copy" in r["Kernel_Name"].lower())

    cf, cw = copy_val(fetch_csv) / kib, copy_val(write_csv) / kib
    key = [k for k in f if k[0].startswith(kernel) and k[1] == grid and k[2] == lds]
    if len(key) != 1:
        raise SystemExit(f"kernel shape not found uniquely: {key}")
    k = key[0]
    fetch_b = f[k] * 1024.0 / cf
    write_b = w[k] * 1024.0 / cw
    return {"kernel": k[0], "grid": grid, "lds": lds,
            "fetch_kib_raw": round(f[k], 1), "write_kib_raw": round(w[k], 1),
            "fetch_scale": round(cf, 5), "write_scale": round(cw, 5),
            "fetch_bytes": int(fetch_b), "write_bytes": int(write_b),
            "hbm_bytes_per_launch": int(fetch_b + write_b)}


def counters(path: str, match: str = ""):
    """Average each counter per dispatch, grouped by (kernel, grid, LDS bytes)
    -- the rocprofv3 --pmc counter_collection.csv, one row per (dispatch,
    counter), values already summed over the chip's instances."""
    agg = collections.OrderedDict()
    for r in csv.DictReader(open(path)):
        if match and match not in r["Kernel_Name"]:
            continue
        key = (r["Kernel_Name"], int(r["Grid_Size"]), int(r["LDS_Block_Size"]))
        d = agg.setdefault(key, {})
        tot, n = d.get(r["Counter_Name"], (0.0, 0))
        d[r["Counter_Name"]] = (tot + float(r["Counter_Value"]), n + 1)
    rows = []
    for (name, grid, lds), d in agg.items():
        rows.append({"kernel": name, "grid": grid, "lds": lds,
                     "dispatches": max(n for _, n in d.values()),
                     **{c: tot / n for c, (tot, n) in sorted(d.items())}})
    return rows


def _agg(path: str):
    """{(short kernel name, grid, LDS): {counter: mean per dispatch}} of a --pmc CSV."""
    agg = collections.OrderedDict()
    for r in csv.DictReader(open(path)):
        key = (short(r["Kernel_Name"]), int(r["Grid_Size"]), int(r["LDS_Block_Size"]))
        d = agg.setdefault(key, {})
        tot, n = d.get(r["Counter_Name"], (0.0, 0))
        d[r["Counter_Name"]] = (tot + float(r["Counter_Value"]), n + 1)
    return {k: {c: t / n for c, (t, n) in d.items()} for k, d in agg.items()}


def shape_table(runs, copy_mib: float, match: str):
    """One row per (shape, kernel) from per-shape --pmc runs.

    runs: "SPEC=DIR" items, SPEC = DTYPE:NxK[:M] (the bench --shape spec) or
    fused:DTYPE:NxK, DIR holding that shape's pass CSVs (*_counter_collection.csv,
    any number of passes; the FETCH_SIZE / WRITE_SIZE passes must include the
    --copy-calibration copy).  Derived columns:
      HBM/alg   (FETCH_SIZE + WRITE_SIZE bytes, each scaled by the copy's
                reading) / algorithmic bytes of the call
      VALU/B    SQ_INSTS_VALU (wave instructions) per weight byte
      VALU%     SQ_ACTIVE_INST_VALU / SQ_WAVE_CYCLES
      wait%     SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (waves waiting on a dependency)
      TA%       TA_TA_BUSY_sum / (GRBM_GUI_ACTIVE / 8 XCDs x 256 CUs): the
                address unit's busy share
      MFMA%     SQ_VALU_MFMA_BUSY_CYCLES / (cycles x 1024 SIMDs)
      cycles    GRBM_GUI_ACTIVE / 8 (GPU cycles per XCD for the dispatch,
                including the profiler's per-dispatch overhead)
    Runtime and torch kernels (the copy calibration, fills) are left out.
    """
    import glob
    import os
    from forge_amd.formats import FORMATS
    names = {f.name.lower(): dt for dt, f in FORMATS.items()}
    print("| shape | kernel | grid | cycles | HBM/alg | VALU/B | VALU% | wait% | TA% | MFMA% |")
    print("|---|---|---:|---:|---:|---:|---:|---:|---:|---:|")
    for item in runs:
        spec, d = item.split("=", 1)
        parts = spec.split(":")
        fused = parts[0] == "fused"
        if fused:
            parts = parts[1:]
        dt = names[parts[0].lower()]
        N, K = (int(v) for v in parts[1].lower().split("x"))
        M = int(parts[2]) if len(parts) > 2 else 1
        f = FORMATS[dt]
        wbytes = f.matrix_bytes(N, K) * (2 if fused else 1)
        alg = wbytes + 4 * M * K + 4 * M * N
        merged = {}
        kib = copy_mib * 1024.0
        scale = {}
        for path in sorted(glob.glob(os.path.join(d, "*_counter_collection.csv"))):
            for k, c in _agg(path).items():
                merged.setdefault(k, {}).update(c)
            for r in csv.DictReader(open(path)):
                if "copy" in r["Kernel_Name"].lower() and r["Counter_Name"] in ("FETCH_SIZE", "WRITE_SIZE"):
                    scale[r["Counter_Name"]] = max(scale.get(r["Counter_Name"], 0.0),
                                                   float(r["Counter_Value"]))
        for (name, grid, lds), c in merged.items():
            if match not in name or name.startswith(("at::", "__amd")):
                continue
            hbm = ""
            if "FETCH_SIZE" in c and "WRITE_SIZE" in c and scale.get("FETCH_SIZE") and scale.get("WRITE_SIZE"):
                b = (c["FETCH_SIZE"] / (scale["FETCH_SIZE"] / kib) +
                     c["WRITE_SIZE"] / (scale["WRITE_SIZE"] / kib)) * 1024.0
                hbm = f"{b / alg:.3f}"
            cyc = c.get("GRBM_GUI_ACTIVE", 0.0) / 8.0
            def ratio(a, b, pct=True):
                if a in c and b in c and c[b] > 0:
                    return f"{100 * c[a] / c[b]:.0f}" if pct else f"{c[a] / c[b]:.3f}"
                return ""
            valub = f"{c['SQ_INSTS_VALU'] / wbytes:.4f}" if "SQ_INSTS_VALU" in c else ""
            ta = (f"{100 * c['TA_TA_BUSY_sum'] / (cyc * 256):.0f}"
                  if "TA_TA_BUSY_sum" in c and cyc > 0 else "")
            mf = (f"{100 * c['SQ_VALU_MFMA_BUSY_CYCLES'] / (cyc * 1024):.0f}"
                  if "SQ_VALU_MFMA_BUSY_CYCLES" in c and cyc > 0 else "")
            print(f"| {spec} | `{name}` | {grid} | {cyc:.0f} | {hbm} | "
                  f"{valub} | {ratio('SQ_ACTIVE_INST_VALU', 'SQ_WAVE_CYCLES')} | "
                  f"{ratio('SQ_WAIT_INST_ANY', 'SQ_WAVE_CYCLES')} | {ta} | {mf} |")


def main():
    p = argparse.ArgumentParser()
    p.add_argument("--counters", metavar="COUNTER_CSV",
                   help="average --pmc counters per dispatch and kernel shape")
    p.add_argument("--match", default="", help="with --counters: kernel name substring")
    p.add_argument("trace", nargs="?")
    p.add_argument("--title", default="")
    p.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    p.add_argument("--copy-mib", type=float, default=448)
    p.add_argument("--kernel", default="gemvp_kernel<13")
    p.add_argument("--grid", type=int, default=0)
    p.add_argument("--lds", type=int, default=0)
    p.add_argument("--shapes", nargs="+", metavar="SPEC=DIR",
                   help="per-shape --pmc run directories: one table of derived ratios")
    a = p.parse_args()
    if a.shapes:
        shape_table(a.shapes, a.copy_mib, a.match)
        return
    if a.counters:
        for r in counters(a.counters, a.match):
            print(f"- `{short(r.pop('kernel'))}` grid {r.pop('grid')} LDS {r.pop('lds')} "
                  f"({r.pop('dispatches')} dispatches): " +
                  ", ".join(f"{k} {v:.0f}" for k, v in r.items()))
        return
    if a.traffic:
        import json
        print(json.dumps(traffic(a.traffic[0], a.traffic[1], a.copy_mib, a.kernel, a.grid,
                                 a.lds), indent=1))
        return
    if a.title:
        print(f"# {a.title}\n")
    print("| kernel | grid | wg | LDS B | VGPR | scratch | calls | avg µs | median µs | min µs | max µs |")
    print("|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|")
    for r in summarise(a.trace):
        print(f"| `{short(r['kernel'])}` | {r['grid']} | {r['wg']} | {r['lds']} | {r['vgpr']} | "
              f"{r['scratch']} | {r['calls']} | {r['avg_us']:.2f} | {r['median_us']:.2f} | "
              f"{r['min_us']:.2f} | {r['max_us']:.2f} |")


if __name__ == "__main__":
    main()
