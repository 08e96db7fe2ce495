"""Summaries of rocprofv3 output for the hot-path kernels.

    python -m redpanda_amd.profiling stats  <kernel_stats.csv> --cmd "<command>" > out.md
    python -m redpanda_amd.profiling traffic --fetch <pmc_fetch.csv> --write <pmc_write.csv> \
        --calib-bytes 1073741824 --out traffic.json
    python -m redpanda_amd.profiling valu <pmc_valu.csv> --out valu.json

`traffic` turns two counter passes (FETCH_SIZE, then WRITE_SIZE, each in KiB
per dispatch) into HBM bytes per dispatch for every kernel, scaled by what
the same counters read for a plain streaming kernel of known size: the
single torch.neg dispatch of `bench.py --profile-pass`, which reads and
writes `calib_bytes` each (on gfx950 the raw FETCH_SIZE of such a dispatch
reads about half its bytes, WRITE_SIZE about all of them).  Kernels are
keyed by their function name without template arguments (e.g.
`scan_bwd_kernel`).
"""

import argparse
import collections
import csv
import json
import re
import sys

CALIB_MARK = "neg_kernel"  # substring of the calibration dispatch's full name


def _template_args(kernel_name):
    """Top-level template arguments of a demangled kernel name."""
    start = kernel_name.find("<")
    if start < 0:
        return []
    depth, cur, args = 0, [], []
    for ch in kernel_name[start:]:
        if ch == "<":
            depth += 1
            if depth == 1:
                continue
        elif ch == ">":
            depth -= 1
            if depth == 0:
                args.append("".join(cur).strip())
                break
        elif ch == "," and depth == 1:
            args.append("".join(cur).strip())
            cur = []
            continue
        cur.append(ch)
    return args


def short_name(kernel_name):
    """`void rp::scan_bwd_kernel<8, 5, ...>(rp::ScanParams, ...)` -> `scan_bwd_kernel`.
    The step tile kernel's rank-1 instantiation (template argument RANK1,
    the sixth, true) is `step_tile_kernel[rank1]`, and its shared-state
    instantiation (SHARED, the seventh) carries `[shared]`, so the forms'
    counters stay apart."""
    name = kernel_name
    depth, out = 0, []
    for ch in name:  # drop template arguments
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif depth == 0:
            out.append(ch)
    name = "".join(out).split("(")[0]
    name = name.replace("void ", "").strip()
    name = re.sub(r"^.*::", "", name)
    if name == "step_tile_kernel":
        args = _template_args(kernel_name)
        if len(args) >= 6 and args[5] in ("true", "1"):
            name += "[rank1]"
        if len(args) >= 7 and args[6] in ("true", "1"):
            name += "[shared]"
    return name


def counter_means(path, counter):
    """Mean counter value per dispatch by short kernel name, and the
    calibration dispatch's value (summed, in case there are several)."""
    acc = collections.defaultdict(list)
    calib = 0.0
    with open(path) as fh:
        for row in csv.DictReader(fh):
            if row["Counter_Name"] != counter:
                continue
            if CALIB_MARK in row["Kernel_Name"]:
                calib += float(row["Counter_Value"])
            else:
                acc[short_name(row["Kernel_Name"])].append(float(row["Counter_Value"]))
    return {k: sum(v) / len(v) for k, v in acc.items()}, calib


def traffic(fetch_csv, write_csv, calib_bytes):
    fetch, f_cal = counter_means(fetch_csv, "FETCH_SIZE")
    write, w_cal = counter_means(write_csv, "WRITE_SIZE")
    if f_cal <= 0 or w_cal <= 0:
        raise SystemExit("no calibration dispatch in the counter files (run bench.py "
                         "--profile-pass under rocprofv3 --pmc)")
    f_scale = calib_bytes / (f_cal * 1024.0)
    w_scale = calib_bytes / (w_cal * 1024.0)
    out = {"calibration": {"dispatch": "torch.neg over calib_bytes",
                           "bytes_each_way": calib_bytes,
                           "fetch_kib": f_cal, "write_kib": w_cal,
                           "fetch_scale": f_scale, "write_scale": w_scale},
           "kernels": {}}
    for k in sorted(set(fetch) | set(write)):
        fb = fetch.get(k, 0.0) * 1024.0 * f_scale
        wb = write.get(k, 0.0) * 1024.0 * w_scale
        out["kernels"][k] = {"fetch_bytes": fb, "write_bytes": wb, "bytes": fb + wb}
    return out


def valu(csv_path):
    """Mean VALU wave-instructions (and transcendental ones) per dispatch by
    kernel, from a pass with SQ_INSTS_VALU / SQ_INSTS_VALU_TRANS_F32."""
    acc = collections.defaultdict(lambda: collections.defaultdict(list))
    with open(csv_path) as fh:
        for row in csv.DictReader(fh):
            if CALIB_MARK in row["Kernel_Name"]:
                continue
            acc[short_name(row["Kernel_Name"])][row["Counter_Name"]].append(float(row["Counter_Value"]))
    out = {}
    for k, ctrs in acc.items():
        out[k] = {name: sum(v) / len(v) for name, v in ctrs.items()}
    return {"counters": "mean per dispatch; wave-instructions summed over the device",
            "kernels": out}


def stats_markdown(csv_path, cmd, title, top=None):
    rows = list(csv.DictReader(open(csv_path)))
    rows.sort(key=lambda r: -float(r["TotalDurationNs"]))
    if top:
        rows = rows[:top]
    lines = [f"# {title}", "", "Command (repo root, one MI355X):", "", f"    {cmd}", "",
             "| kernel | calls | avg (us) | min (us) | max (us) | share |",
             "|---|---|---|---|---|---|"]
    for r in rows:
        name = r["Name"]
        if len(name) > 90:
            name = name[:87] + "..."
        lines.append(f"| `{name}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                     f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                     f"{float(r['Percentage']):.1f}% |")
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="action", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--cmd", required=True)
    s.add_argument("--title", default="rocprofv3 kernel statistics")
    s.add_argument("--top", type=int, default=None, help="only the N kernels with most total time")
    t = sub.add_parser("traffic")
    t.add_argument("--fetch", required=True)
    t.add_argument("--write", required=True)
    t.add_argument("--calib-bytes", type=int, default=1 << 30)
    t.add_argument("--out")
    v = sub.add_parser("valu")
    v.add_argument("csv")
    v.add_argument("--out")
    a = ap.parse_args(argv)
    if a.action == "stats":
        sys.stdout.write(stats_markdown(a.csv, a.cmd, a.title, a.top))
    elif a.action == "valu":
        text = json.dumps(valu(a.csv), indent=1, sort_keys=True)
        if a.out:
            with open(a.out, "w") as fh:
                fh.write(text + "\n")
        else:
            print(text)
    else:
        res = traffic(a.fetch, a.write, a.calib_bytes)
        text = json.dumps(res, indent=1, sort_keys=True)
        if a.out:
            with open(a.out, "w") as fh:
                fh.write(text + "\n")
        else:
            print(text)


if __name__ == "__main__":
    main()
