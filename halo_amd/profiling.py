"""Summaries of rocprofv3 output for this library's kernels.

    python -m halo_amd.profiling stats <kernel_stats.csv> [--match NAME]
        per-kernel call count and average / min / max duration (us) from a
        `rocprofv3 --kernel-trace --stats --output-format csv` run.

    python -m halo_amd.profiling traffic --fetch <counter_collection.csv> --write <counter_collection.csv>
                                         --kernel NAME --copy-bytes N [--out FILE]
        HBM bytes per dispatch of the kernels matching NAME, from one `--pmc FETCH_SIZE` run and one
        `--pmc WRITE_SIZE` run (KiB per dispatch). Each counter is scaled by what it reads for a plain
        device-to-device copy of N bytes in the same run (the copy reads N and writes N bytes), so the
        result is in bytes whatever the counters' unit and sampling.

    python -m halo_amd.profiling counters <counter_collection.csv> [--match NAME]
        per kernel, the median over its dispatches of every counter of a `rocprofv3 --pmc ...
        --output-format csv` run, with the dispatch count and the kernel's VGPR / LDS figures.

The traffic summary is a small JSON file that bench.py reports as `roofline.traffic`.
"""
from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys
from collections import defaultdict

COPY_KERNEL_HINTS = ("copy", "Copy")


def _short(name: str) -> str:
    """Kernel name without the return type and argument list (templates kept)."""
    name = name.replace("(anonymous namespace)", "{anon}")
    if name.startswith("void "):
        name = name[5:]
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            return name[:i]
    return name


def kernel_stats(path: str, match: str | None = None) -> list[dict]:
    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r.get("Name") or r.get("KernelName") or ""
            if match and match not in name:
                continue
            calls = int(r["Calls"])
            rows.append({"kernel": _short(name), "calls": calls,
                         "avg_us": float(r["AverageNs"]) / 1e3, "min_us": float(r["MinNs"]) / 1e3,
                         "max_us": float(r["MaxNs"]) / 1e3, "total_ms": float(r["TotalDurationNs"]) / 1e6,
                         "percent": float(r.get("Percentage", 0.0))})
    return rows


def counter_per_dispatch(path: str, counter: str) -> dict[str, list[float]]:
    """Kernel name -> the counter's value for each dispatch (in file order)."""
    out: dict[str, list[float]] = defaultdict(list)
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            out[r["Kernel_Name"]].append(float(r["Counter_Value"]))
    return out


def _pick(per: dict[str, list[float]], match: str) -> tuple[str, list[float]]:
    hits = [(k, v) for k, v in per.items() if match in k]
    if not hits:
        raise SystemExit(f"no kernel matching {match!r}: {sorted(per)}")
    # the most-dispatched match (the timed kernel rather than a one-off warm-up shape)
    return max(hits, key=lambda kv: len(kv[1]))


def traffic(fetch_csv: str, write_csv: str, kernel: str, copy_bytes: int) -> dict:
    fetch = counter_per_dispatch(fetch_csv, "FETCH_SIZE")
    write = counter_per_dispatch(write_csv, "WRITE_SIZE")
    kname, kf = _pick(fetch, kernel)
    _, kw = _pick(write, kernel)
    copies_f = [v for k, vs in fetch.items() if any(h in k for h in COPY_KERNEL_HINTS) for v in vs]
    copies_w = [v for k, vs in write.items() if any(h in k for h in COPY_KERNEL_HINTS) for v in vs]
    if not copies_f or not copies_w:
        raise SystemExit("no copy kernel in the counter files: run the profiled command with a calibration copy")
    # the calibration copies are the largest copy dispatches of the run
    cf = statistics.median(sorted(copies_f)[-4:])
    cw = statistics.median(sorted(copies_w)[-4:])
    scale_f = copy_bytes / cf   # bytes per counter unit, FETCH_SIZE
    scale_w = copy_bytes / cw   # bytes per counter unit, WRITE_SIZE
    f_units = statistics.median(kf)
    w_units = statistics.median(kw)
    return {
        "kernel": _short(kname),
        "dispatches": len(kf),
        "fetch_counter_median": f_units,
        "write_counter_median": w_units,
        "copy_bytes": copy_bytes,
        "copy_fetch_counter": cf,
        "copy_write_counter": cw,
        "fetch_scale_bytes_per_unit": scale_f,
        "write_scale_bytes_per_unit": scale_w,
        "fetch_bytes": f_units * scale_f,
        "write_bytes": w_units * scale_w,
        "traffic_bytes": f_units * scale_f + w_units * scale_w,
    }


def counters(path: str, match: str | None = None) -> list[dict]:
    per: dict[str, dict[str, list[float]]] = defaultdict(lambda: defaultdict(list))
    meta: dict[str, dict] = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            name = r["Kernel_Name"]
            if match and match not in name:
                continue
            per[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
            meta[name] = {"grid": r.get("Grid_Size"), "workgroup": r.get("Workgroup_Size"),
                          "vgpr": r.get("VGPR_Count"), "agpr": r.get("Accum_VGPR_Count"), "lds": r.get("LDS_Block_Size")}
    out = []
    for name, cs in per.items():
        n = max(len(v) for v in cs.values())
        out.append({"kernel": _short(name), "dispatches": n, **meta[name],
                    "counters": {c: statistics.median(v) for c, v in sorted(cs.items())}})
    return sorted(out, key=lambda d: -d["dispatches"])


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m halo_amd.profiling")
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--match")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--out")
    c = sub.add_parser("counters")
    c.add_argument("csv")
    c.add_argument("--match")
    a = ap.parse_args(argv)
    if a.cmd == "counters":
        for k in counters(a.csv, a.match):
            print(f"{k['kernel']}: {k['dispatches']} dispatches, grid {k['grid']}, workgroup {k['workgroup']}, "
                  f"vgpr {k['vgpr']}, agpr {k['agpr']}, lds {k['lds']}")
            for cn, v in k["counters"].items():
                print(f"    {cn:34s} {v:18,.0f}")
        return 0
    if a.cmd == "stats":
        for r in kernel_stats(a.csv, a.match):
            print(f"{r['calls']:8d}  avg {r['avg_us']:10.3f} us  min {r['min_us']:10.3f}  max {r['max_us']:10.3f}  "
                  f"{r['percent']:6.2f}%  {r['kernel']}")
        return 0
    res = traffic(a.fetch, a.write, a.kernel, a.copy_bytes)
    text = json.dumps(res, indent=1)
    if a.out:
        with open(a.out, "w") as f:
            f.write(text + "\n")
    print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
