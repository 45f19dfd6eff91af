"""Summaries of rocprofv3 output (CSV mode) for the Library-read kernels.

    python -m kv_skill_v2_amd.profiling stats  <kernel_stats.csv> [--match decode_read_kernel]
    python -m kv_skill_v2_amd.profiling traffic <fetch counter_collection.csv> <write counter_collection.csv>
        --kernel decode_read_kernel --copy-bytes 1073741824 [--json out.json]

`traffic` averages FETCH_SIZE and WRITE_SIZE (KiB per dispatch) over the dispatches of the
kernel, and scales each by what the same counter reads for the device-to-device blit copy of
known size that `bench.py --calibration-copy-mib` launches after the workload (expected:
copy_bytes read, copy_bytes written).
"""

from __future__ import annotations

import argparse
import csv
import json
import statistics
import sys


def _short(name: str, width: int = 60) -> str:
    return name if len(name) <= width else name[: width - 3] + "..."


def kernel_stats(path: str, match: str | None = None, top: int = 12) -> list[dict]:
    rows = list(csv.DictReader(open(path)))
    out = []
    for r in rows:
        if match and match not in r["Name"]:
            continue
        out.append({"name": r["Name"], "calls": int(r["Calls"]), "avg_us": float(r["AverageNs"]) / 1e3,
                    "min_us": float(r["MinNs"]) / 1e3, "max_us": float(r["MaxNs"]) / 1e3,
                    "pct": float(r["Percentage"])})
    return out[:top]


def _counter(path: str, counter: str) -> list[tuple[str, float]]:
    rows = list(csv.DictReader(open(path)))
    return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows if r["Counter_Name"] == counter]


def _copy_kernel(vals: list[tuple[str, float]], copy_bytes: int) -> float:
    """The calibration copy: the three largest dispatches of the device-to-device blit kernel
    (`__amd_rocclr_copyBuffer`) that `bench.py --calibration-copy-mib` launches after the workload.
    Other kernels with "copy" in their names (dtype conversions while the synthetic inputs are
    built) move other byte counts and are never taken.  A reading below 1/16 of the copy's size
    means the calibration copy is not in the file."""
    cands = sorted(v for n, v in vals if "copyBuffer" in n)
    if len(cands) < 3 or cands[-1] * 1024.0 * 16 < copy_bytes:
        raise SystemExit("no calibration copy dispatches of that size found "
                         "(run bench.py with --calibration-copy-mib)")
    return statistics.median(cands[-3:])


def traffic(fetch_csv: str, write_csv: str, kernel: str, copy_bytes: int) -> dict:
    """Scaled HBM bytes per launch of `kernel`; a comma-separated list sums the per-dispatch means
    of each kernel (the kernels one step launches once each)."""
    f = _counter(fetch_csv, "FETCH_SIZE")
    w = _counter(write_csv, "WRITE_SIZE")
    fetch_scale = copy_bytes / (_copy_kernel(f, copy_bytes) * 1024.0)
    write_scale = copy_bytes / (_copy_kernel(w, copy_bytes) * 1024.0)
    per, fetch_b, write_b, disp = {}, 0.0, 0.0, 0
    for name in kernel.split(","):
        fk = [v for n, v in f if name in n]
        wk = [v for n, v in w if name in n]
        if not fk or not wk:
            raise SystemExit(f"kernel {name!r} not found in the counter files")
        fb = statistics.mean(fk) * 1024.0 * fetch_scale
        wb = statistics.mean(wk) * 1024.0 * write_scale
        per[name] = {"fetch_bytes": fb, "write_bytes": wb, "dispatches": len(fk)}
        fetch_b, write_b, disp = fetch_b + fb, write_b + wb, max(disp, len(fk))
    return {"kernel": kernel, "fetch_bytes": fetch_b, "write_bytes": write_b,
            "bytes_per_launch": fetch_b + write_b, "fetch_scale": fetch_scale,
            "write_scale": write_scale, "dispatches": disp, "per_kernel": per}


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--match")
    t = sub.add_parser("traffic")
    t.add_argument("fetch_csv")
    t.add_argument("write_csv")
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--json")
    t.add_argument("--source", default="")
    a = ap.parse_args(argv)
    if a.cmd == "stats":
        print(f"{'kernel':60s} {'calls':>6s} {'avg us':>10s} {'min us':>10s} {'max us':>10s} {'%':>6s}")
        for r in kernel_stats(a.csv, a.match):
            print(f"{_short(r['name']):60s} {r['calls']:6d} {r['avg_us']:10.2f} {r['min_us']:10.2f} "
                  f"{r['max_us']:10.2f} {r['pct']:6.2f}")
    else:
        res = traffic(a.fetch_csv, a.write_csv, a.kernel, a.copy_bytes)
        res["source"] = a.source
        print(json.dumps(res, indent=1))
        if a.json:
            with open(a.json, "w") as fh:
                json.dump(res, fh, indent=1)
    return 0


if __name__ == "__main__":
    sys.exit(main())
