#!/usr/bin/env python3
"""Summarize a rocprofv3 kernel trace (CSV) per kernel and launch shape.

One template instance of a kernel can run at several shapes in one program
(the Q8_0 GEMV serves every projection of a decode round), so dispatches
are grouped by (kernel, grid, workgroup) and reported with their count and
mean / min / max duration, as a Markdown table sorted by total time.

usage: prof_summary.py <kernel_trace.csv> [--top N] [--match SUBSTRING]
"""
from __future__ import annotations

import argparse
import csv
import re
import sys
from collections import defaultdict


def short_name(name: str) -> str:
    """Kernel name without the argument list; template arguments kept."""
    name = name.strip().replace("(anonymous namespace)::", "")
    depth, out = 0, []
    for ch in name:
        if ch == "(" and depth == 0:
            break
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        out.append(ch)
    s = "".join(out)
    s = re.sub(r"^void\s+", "", s)
    s = s.replace("lfm3amd::", "")
    return s


def summarize(path: str, top: int, match: str | None):
    groups = defaultdict(list)
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = short_name(row["Kernel_Name"])
            if match and match not in name:
                continue
            grid = tuple(int(row.get(f"Grid_Size_{a}", 1) or 1) for a in "XYZ")
            wg = tuple(int(row.get(f"Workgroup_Size_{a}", 1) or 1) for a in "XYZ")
            dur = (int(row["End_Timestamp"]) - int(row["Start_Timestamp"])) / 1000.0
            groups[(name, grid, wg)].append(dur)
    rows = []
    for (name, grid, wg), d in groups.items():
        blocks = tuple(g // w for g, w in zip(grid, wg))
        rows.append((sum(d), name, blocks, wg, len(d), sum(d) / len(d), min(d), max(d)))
    rows.sort(reverse=True)
    total = sum(r[0] for r in rows)
    print(f"source: {path}")
    print(f"dispatches: {sum(r[4] for r in rows)}, kernel time: {total / 1000.0:.3f} ms")
    print()
    print("| kernel | workgroups (x,y,z) | threads | calls | mean us | min us | max us | total ms | % |")
    print("|---|---|---|---|---|---|---|---|---|")
    for tot, name, blocks, wg, n, mean, lo, hi in rows[:top]:
        print(f"| `{name}` | {blocks} | {wg[0] * wg[1] * wg[2]} | {n} | {mean:.2f} | {lo:.2f} | "
              f"{hi:.2f} | {tot / 1000.0:.3f} | {100.0 * tot / total:.1f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--top", type=int, default=40)
    ap.add_argument("--match", default=None)
    a = ap.parse_args()
    summarize(a.trace, a.top, a.match)


if __name__ == "__main__":
    sys.exit(main())
