"""Summaries of rocprofv3 CSV output (--output-format csv).

    python rocprof_summary.py stats <run_kernel_stats.csv> [--top N]
    python rocprof_summary.py traffic --fetch DIR --write DIR --kernel NAME
                                      --copy-bytes B [--record JSON --source FILE]
    python rocprof_summary.py mfma --pmc DIR --trace run_kernel_trace.csv

`stats` prints the per-kernel table of a --kernel-trace --stats run.

`roles` splits a --kernel-trace run's dispatches (run_kernel_trace.csv) of
the decode step into per-role averages: every dispatch gets the name of its
kernel plus its ordinal since the last dispatch of the `--anchor` kernel (the
first kernel of a layer), so the same kernel launched twice per layer shows
as two rows; the mean gap between a dispatch's start and the previous one's
end is printed beside it.

`traffic-roles` does the same for the decode step: the dispatches of each
pass are put in order and named by role as in `roles` (--names maps
"kernel #ordinal" to a role name, "a #1+b #2" adding two kernels into one
role), and each role's bytes per launch are recorded under "decode:<role>".

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
    """(mean KiB per dispatch of `kernel`, dispatches, mean KiB of a calibration
    copy).  The calibration copies are the largest device-to-device copies
    after the run's last other dispatch (the probe ends with them; earlier
    copies, such as weight uploads, and the small copies of a decode step's
    results are not calibration)."""
    k = [float(r["Counter_Value"]) for r in rows if short(r["Kernel_Name"]) == kernel]
    rows = sorted(rows, key=lambda r: int(r["Dispatch_Id"]))
    last_other = max((i for i, r in enumerate(rows) if "copyBuffer" not in r["Kernel_Name"]), default=-1)
    tail = rows[last_other + 1:]
    big = max((int(r["Grid_Size"]) for r in tail), default=0)
    c = [float(r["Counter_Value"]) for r in tail if int(r["Grid_Size"]) == big]
    if not k or not c:
        raise SystemExit(f"kernel {kernel!r} or the calibration copy is missing")
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


def role_kib(rows, anchor: str, skip: int):
    """Mean KiB per dispatch of every 'kernel #ordinal' role after `skip`
    layers, dispatches in Dispatch_Id order."""
    rows = sorted(rows, key=lambda r: int(r["Dispatch_Id"]))
    first = next((i for i, r in enumerate(rows) if anchor in r["Kernel_Name"]), None)
    if first is None:
        raise SystemExit(f"no dispatch of {anchor!r}")
    acc, k, n_anchor = {}, 0, 0
    for r in rows[first:]:
        if anchor in r["Kernel_Name"]:
            k, n_anchor = 0, n_anchor + 1
        role = f"{short(r['Kernel_Name'])} #{k}"
        k += 1
        if n_anchor > skip:
            acc.setdefault(role, []).append(float(r["Counter_Value"]))
    return {role: sum(v) / len(v) for role, v in acc.items()}


def traffic_roles(args) -> str:
    frows, wrows = counter_rows(args.fetch), counter_rows(args.write)
    _, _, fc = per_dispatch_kib(frows, short(next(r["Kernel_Name"] for r in frows)))
    _, _, wc = per_dispatch_kib(wrows, short(next(r["Kernel_Name"] for r in wrows)))
    f_scale = args.copy_bytes / (fc * 1024.0)
    w_scale = args.copy_bytes / (wc * 1024.0)
    fk = role_kib(frows, args.anchor, args.skip)
    wk = role_kib(wrows, args.anchor, args.skip)
    names = dict(n.split("=", 1) for n in args.names)
    lines = [f"copy of {args.copy_bytes} B: FETCH_SIZE scale {f_scale:.4f}, WRITE_SIZE scale {w_scale:.4f}",
             f"{'role':12s} {'kernel #ordinal':36s} {'fetch_B':>12s} {'write_B':>10s} {'total_B':>12s}"]
    rec = {}
    if args.record:
        rec_path = Path(args.record)
        rec = json.loads(rec_path.read_text()) if rec_path.exists() else {}
    for key, role in names.items():
        parts = key.split("+")  # several kernels making one role: their bytes add up
        for k in parts:
            if k not in fk or k not in wk:
                raise SystemExit(f"no dispatches of {k!r}")
        fb = sum(fk[k] for k in parts) * 1024.0 * f_scale
        wb = sum(wk[k] for k in parts) * 1024.0 * w_scale
        lines.append(f"{role:12s} {key:36s} {fb:12.0f} {wb:10.0f} {fb + wb:12.0f}")
        if args.record:
            src = Path(args.source)
            rec["decode:" + role] = {"source": src.name, "bytes_per_launch": round(fb + wb),
                                     "fetch_bytes": round(fb), "write_bytes": round(wb),
                                     "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4),
                                     "source_sha256": hashlib.sha256(src.read_bytes()).hexdigest()}
    if args.record:
        Path(args.record).write_text(json.dumps(rec, indent=1, sort_keys=True) + "\n")
    return "\n".join(lines)


def mfma(args) -> str:
    """Per kernel of a --pmc SQ_INSTS_VALU_MFMA_MOPS_I8 SQ_VALU_MFMA_BUSY_CYCLES
    pass, with durations from a --kernel-trace run of the same command: int8
    MFMA operations per dispatch (the counter counts units of 512), the MFMA
    busy cycles per SIMD (the counter sums over every SIMD), and their share
    of the kernel's duration at the given clock."""
    rows = counter_rows(args.pmc)
    ops, busy = {}, {}
    for r in rows:
        k = short(r["Kernel_Name"])
        if r["Counter_Name"] == "SQ_INSTS_VALU_MFMA_MOPS_I8":
            ops.setdefault(k, []).append(float(r["Counter_Value"]) * 512)
        elif r["Counter_Name"] == "SQ_VALU_MFMA_BUSY_CYCLES":
            busy.setdefault(k, []).append(float(r["Counter_Value"]))
    dur = {}
    for r in csv.DictReader(open(args.trace)):
        dur.setdefault(short(r["Kernel_Name"]), []).append(
            (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    out = [f"{'kernel':24s} {'dispatches':>10s} {'GOP/disp':>9s} {'us/disp':>8s} {'TOP/s':>8s} "
           f"{'of peak':>8s} {'MFMA busy/SIMD us':>18s} {'busy share':>10s}"]
    for k in sorted(ops):
        if not any(ops[k]):
            continue
        o = sum(ops[k]) / len(ops[k])
        b = sum(busy.get(k, [0])) / max(len(busy.get(k, [1])), 1) / args.simds / (args.clock_ghz * 1e3)
        d = sum(dur.get(k, [0])) / max(len(dur.get(k, [1])), 1)
        tops = o / (d * 1e-6) / 1e12 if d else 0.0
        out.append(f"{k[:24]:24s} {len(ops[k]):10d} {o / 1e9:9.2f} {d:8.2f} {tops:8.1f} "
                   f"{tops / args.peak_tops:8.3f} {b:18.2f} {b / d if d else 0:10.3f}")
    return "\n".join(out)


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
    tr = sub.add_parser("traffic-roles")
    tr.add_argument("--fetch", required=True)
    tr.add_argument("--write", required=True)
    tr.add_argument("--anchor", required=True)
    tr.add_argument("--skip", type=int, default=0)
    tr.add_argument("--names", nargs="+", required=True,
                    help="'kernel #ordinal=role' pairs ('a #1+b #2=role' adds kernels up)")
    tr.add_argument("--copy-bytes", type=int, default=1 << 30)
    tr.add_argument("--record")
    tr.add_argument("--source")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--kernel", required=True)
    t.add_argument("--copy-bytes", type=int, default=1 << 30)
    t.add_argument("--record")
    t.add_argument("--source")
    m = sub.add_parser("mfma")
    m.add_argument("--pmc", required=True, help="run directory of the counter pass")
    m.add_argument("--trace", required=True, help="run_kernel_trace.csv of the same command")
    m.add_argument("--simds", type=int, default=1024)
    m.add_argument("--clock-ghz", type=float, default=2.4)
    m.add_argument("--peak-tops", type=float, default=5000.0)
    args = ap.parse_args()
    if args.cmd == "mfma":
        print(mfma(args))
        return
    if args.cmd == "stats":
        print(stats(args.csv, args.top))
    elif args.cmd == "roles":
        print(roles(args.csv, args.anchor, args.skip))
    elif args.cmd == "traffic-roles":
        print(traffic_roles(args))
    else:
        print(traffic(args))


if __name__ == "__main__":
    main()
