"""Summaries of rocprofv3 CSV output (--output-format csv).

    python rocprof_summary.py stats <run_kernel_stats.csv> [--top N]
    python rocprof_summary.py traffic --fetch DIR --write DIR --kernel NAME
                                      --copy-bytes B [--record JSON --source FILE]

`stats` prints the per-kernel table of a --kernel-trace --stats run.

`traffic` turns two counter passes (--pmc FETCH_SIZE, then --pmc
WRITE_SIZE; both report KiB per dispatch) into HBM bytes per launch of one
kernel.  Each counter is scaled by what it reads for the largest
device-to-device copy in the same run (`copy-bytes` read and written), so the
figure is in bytes the memory system actually moved.  With --record, the
result is stored under the kernel's name together with its source file and
that file's SHA-256, so that a later benchmark uses it only while the kernel
is unchanged.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
from pathlib import Path


def short(name: str) -> str:
    if "::" in name:
        name = name.split("::", 1)[1]
    return name.split("(")[0]


def stats(path: str, top: int) -> str:
    rows = list(csv.DictReader(open(path)))
    out = [f"{'kernel':32s} {'calls':>7s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'total_ms':>9s} {'pct':>6s}"]
    for r in rows[:top]:
        out.append(f"{short(r['Name'])[:32]:32s} {int(r['Calls']):7d} {float(r['AverageNs']) / 1e3:9.2f} "
                   f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f} "
                   f"{float(r['TotalDurationNs']) / 1e6:9.2f} {float(r['Percentage']):6.2f}")
    return "\n".join(out)


def counter_rows(run_dir: str):
    files = sorted(Path(run_dir).rglob("*counter_collection.csv"))
    if not files:
        raise SystemExit(f"no counter_collection.csv under {run_dir}")
    return [r for f in files for r in csv.DictReader(open(f))]


def per_dispatch_kib(rows, kernel: str):
    """(mean KiB per dispatch of `kernel`, dispatches, mean KiB of the largest copy)."""
    k = [float(r["Counter_Value"]) for r in rows if short(r["Kernel_Name"]) == kernel]
    copies = [r for r in rows if "copyBuffer" in r["Kernel_Name"]]
    if not k or not copies:
        raise SystemExit(f"kernel {kernel!r} or the calibration copy is missing")
    big = max(int(r["Grid_Size"]) for r in copies)
    c = [float(r["Counter_Value"]) for r in copies if int(r["Grid_Size"]) == big]
    return sum(k) / len(k), len(k), sum(c) / len(c)


def traffic(args) -> str:
    fk, fn, fc = per_dispatch_kib(counter_rows(args.fetch), args.kernel)
    wk, wn, wc = per_dispatch_kib(counter_rows(args.write), args.kernel)
    f_scale = args.copy_bytes / (fc * 1024.0)
    w_scale = args.copy_bytes / (wc * 1024.0)
    fetch_b, write_b = fk * 1024.0 * f_scale, wk * 1024.0 * w_scale
    total = fetch_b + write_b
    lines = [
        f"kernel {args.kernel}: {fn} dispatches (FETCH_SIZE pass), {wn} (WRITE_SIZE pass)",
        f"FETCH_SIZE {fk:.1f} KiB/dispatch; copy of {args.copy_bytes} B reads {fc:.1f} KiB -> scale {f_scale:.4f}",
        f"WRITE_SIZE {wk:.1f} KiB/dispatch; copy of {args.copy_bytes} B reads {wc:.1f} KiB -> scale {w_scale:.4f}",
        f"HBM bytes per launch: fetch {fetch_b:.0f} + write {write_b:.0f} = {total:.0f}",
    ]
    if args.record:
        rec_path = Path(args.record)
        rec = json.loads(rec_path.read_text()) if rec_path.exists() else {}
        src = Path(args.source)
        rec[args.kernel] = {"source": src.name, "bytes_per_launch": round(total),
                         "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
                         "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
                         "source_sha256": hashlib.sha256(src.read_bytes()).hexdigest()}
        rec_path.write_text(json.dumps(rec, indent=1, sort_keys=True) + "\n")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--top", type=int, default=20)
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-bytes", type=int, default=1 << 30)
    t.add_argument("--record")
    t.add_argument("--source")
    args = ap.parse_args()
    print(stats(args.csv, args.top) if args.cmd == "stats" else traffic(args))


if __name__ == "__main__":
    main()
