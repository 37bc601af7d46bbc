"""Summaries of rocprofv3 CSV output for the decode engine (text only, a few KB).

    python -m qwen_hip.rocprof_summary steps <run_kernel_trace.csv> [--last N] [--boundary NAME]
    python -m qwen_hip.rocprof_summary pmc <run_counter_collection.csv> --kernel SUBSTR
                                           --copy-bytes B --copies C [--last N]

``steps``: decode steps are the intervals between consecutive
``decode_finish_kernel`` dispatches (one per graph replay; ``spec_accept_kernel``
for speculative verify steps, via ``--boundary``); prints, for the
last N steps, each kernel's launches per step, average duration and share of
the step, and the step-to-step time.

``pmc``: average of one counter (``FETCH_SIZE`` or ``WRITE_SIZE``, KiB per
dispatch) over the dispatches whose name contains SUBSTR (with ``--last N`` only the last N of
them, in dispatch order: the profile sample's own launches), next to the same
counter over the largest copy dispatches (``C`` copies of ``B`` bytes each way: the runtime's
``copyBuffer`` blits, else any copy-like kernel), and the scale factor ``B / (copy KiB * 1024)`` that turns the
counter into bytes.
"""

from __future__ import annotations

import argparse
import csv
import re
import statistics
from collections import defaultdict


def _short(name: str) -> str:
    name = re.sub(r"\(anonymous namespace\)::", "", name)
    name = re.sub(r"\(.*\)$", "", name)  # drop the parameter list
    return name.strip()


def _rows(path):
    with open(path, newline="") as f:
        return list(csv.DictReader(f))


def steps(path: str, last: int, boundary: str = "decode_finish_kernel") -> str:
    rows = _rows(path)
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if boundary in r["Kernel_Name"]]
    if len(marks) < 2:
        return "no decode steps found"
    marks = marks[-(last + 1):]
    n = len(marks) - 1
    per = defaultdict(list)
    shape = {}
    for a, b in zip(marks[:-1], marks[1:]):
        for r in rows[a + 1:b + 1]:
            k = _short(r["Kernel_Name"])
            per[k].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
            gx = int(r.get("Grid_Size_X", r.get("Grid_Size", 0)) or 0)
            gy = int(r.get("Grid_Size_Y", 1) or 1)
            gz = int(r.get("Grid_Size_Z", 1) or 1)
            wx = int(r.get("Workgroup_Size_X", r.get("Workgroup_Size", 1)) or 1)
            wy = int(r.get("Workgroup_Size_Y", 1) or 1)
            wz = int(r.get("Workgroup_Size_Z", 1) or 1)
            shape[k] = f"{(gx // wx) * (gy // wy) * (gz // wz)} x {wx * wy * wz}"
    span = (int(rows[marks[-1]]["Start_Timestamp"]) - int(rows[marks[0]]["Start_Timestamp"])) / 1e3 / n
    busy = sum(sum(v) for v in per.values()) / n
    out = [f"Decode steps analysed: the last {n} (between consecutive `{boundary}` dispatches); "
           f"{sum(len(v) for v in per.values()) // n} kernels per step; step-to-step {span:.1f} us; "
           f"kernel busy time {busy:.1f} us per step.", "",
           "| share | per step | avg us | workgroups x threads | kernel |", "|---:|---:|---:|---|---|"]
    for k, v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        out.append(f"| {100 * sum(v) / n / span:.1f}% | {len(v) // n} | {statistics.mean(v):.2f} | "
                   f"{shape[k]} | `{k}` |")
    return "\n".join(out)


def pmc(path: str, kernel: str, copy_bytes: int, copies: int, last: int = 0) -> str:
    rows = _rows(path)
    per = defaultdict(float)
    names = {}
    counter = None
    for r in rows:
        d = int(r["Dispatch_Id"])
        per[d] += float(r["Counter_Value"])
        names[d] = _short(r["Kernel_Name"])
        counter = r["Counter_Name"]
    target = [per[d] for d in sorted(per) if kernel in names[d]]
    if last > 0:   # only the last N dispatches (the profile sample), not engine set-up at other shapes
        target = target[-last:]
    # the runtime's blit copy when present (other large elementwise kernels, such as a masked
    # fill of a KV-sized tensor, would otherwise pass for the calibration copy)
    copy_like = sorted(((per[d], d) for d in per if "copyBuffer" in names[d]), reverse=True) or \
        sorted(((per[d], d) for d in per if re.search(r"copy|elementwise|Copy", names[d])), reverse=True)
    copy_vals = [v for v, _ in copy_like[:copies]]
    lines = [f"counter {counter}: {len(target)} dispatches of `{kernel}`"]
    if target:
        lines.append(f"  kernel avg {statistics.mean(target):.1f} KiB/dispatch (min {min(target):.1f}, "
                     f"max {max(target):.1f})")
    if copy_vals:
        cavg = statistics.mean(copy_vals)
        factor = copy_bytes / (cavg * 1024.0)
        lines.append(f"  copy of {copy_bytes} B each way: {cavg:.1f} KiB/dispatch over {len(copy_vals)} "
                     f"dispatches (`{names[copy_like[0][1]]}`); scale factor {factor:.4f}")
        if target:
            lines.append(f"  kernel bytes/dispatch (scaled): {statistics.mean(target) * 1024.0 * factor:.0f}")
    return "\n".join(lines)


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("steps")
    s.add_argument("csv")
    s.add_argument("--last", type=int, default=32)
    s.add_argument("--boundary", default="decode_finish_kernel")
    p = sub.add_parser("pmc")
    p.add_argument("csv")
    p.add_argument("--kernel", required=True)
    p.add_argument("--copy-bytes", type=int, required=True)
    p.add_argument("--copies", type=int, default=3)
    p.add_argument("--last", type=int, default=0, help="average only the last N dispatches of the kernel")
    a = ap.parse_args()
    print(steps(a.csv, a.last, a.boundary) if a.cmd == "steps" else pmc(a.csv, a.kernel, a.copy_bytes, a.copies, a.last))


if __name__ == "__main__":
    main()
