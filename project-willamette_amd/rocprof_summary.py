"""Summaries of rocprofv3 CSV output (--output-format csv).

    python rocprof_summary.py stats <run_kernel_stats.csv> [--top N]
    python rocprof_summary.py traffic --fetch DIR --write DIR --kernel NAME
                                      --copy-bytes B [--record JSON --source FILE]

`stats` prints the per-kernel table of a --kernel-trace --stats run.

`roles` splits a --kernel-trace run's dispatches (run_kernel_trace.csv) of
the decode step into per-role averages: every dispatch gets the name of its
kernel plus its ordinal since the last dispatch of the `--anchor` kernel (the
first kernel of a layer), so the same kernel launched twice per layer shows
as two rows; the mean gap between a dispatch's start and the previous one's
end is printed beside it.

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


def roles(path: str, anchor: str, skip: int) -> str:
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    first = next((i for i, r in enumerate(rows) if anchor in r["Kernel_Name"]), None)
    if first is None:
        raise SystemExit(f"no dispatch of {anchor!r}")
    acc, order = {}, []
    k, prev_end, n_anchor = 0, None, 0
    for r in rows[first:]:
        name = short(r["Kernel_Name"])
        start, end = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if anchor in r["Kernel_Name"]:
            k, n_anchor = 0, n_anchor + 1
        role = f"{name} #{k}"
        k += 1
        gap = (start - prev_end) if prev_end is not None else 0
        prev_end = end
        if n_anchor <= skip:
            continue
        if role not in acc:
            acc[role] = []
            order.append(role)
        acc[role].append((end - start, gap))
    out = [f"{'role (kernel #ordinal in layer)':44s} {'calls':>6s} {'avg_us':>8s} {'min_us':>8s} "
           f"{'gap_us':>7s}"]
    for role in order:
        v = acc[role]
        d = [x[0] for x in v]
        g = [x[1] for x in v]
        out.append(f"{role[:44]:44s} {len(v):6d} {sum(d) / len(d) / 1e3:8.2f} {min(d) / 1e3:8.2f} "
                   f"{sum(g) / len(g) / 1e3:7.2f}")
    return "\n".join(out)


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
    r = sub.add_parser("roles")
    r.add_argument("csv")
    r.add_argument("--anchor", required=True, help="substring of the first kernel of a layer")
    r.add_argument("--skip", type=int, default=0, help="layers to skip (warm-up)")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-bytes", type=int, default=1 << 30)
    t.add_argument("--record")
    t.add_argument("--source")
    args = ap.parse_args()
    if args.cmd == "stats":
        print(stats(args.csv, args.top))
    elif args.cmd == "roles":
        print(roles(args.csv, args.anchor, args.skip))
    else:
        print(traffic(args))


if __name__ == "__main__":
    main()
