#!/usr/bin/env python3
"""Summarize rocprofv3 output per kernel and launch shape.

One template instance of a kernel can run at several shapes in one program
(the Q8_0 GEMV serves every projection of a decode round), so dispatches
are grouped by (kernel, grid, workgroup).

Kernel trace: count and mean / min / max duration per group, as a Markdown
table sorted by total time.

HBM traffic (--fetch and --write, the counter_collection.csv files of two
`rocprofv3 --pmc FETCH_SIZE` and `--pmc WRITE_SIZE` runs of one program):
mean KiB per dispatch of each group, and bytes scaled by what the same
counter reads for a plain copy of --copy-bytes (the group whose name holds
--copy-match with the largest reading): scale = copy bytes / counter bytes,
so the copy reads and writes exactly its size.

Runs of one kernel (--chunk N with --match and --blocks): its dispatches
in start order, after the first --skip K, cut into consecutive runs of N,
with each run's mean
duration, for a program that launches one kernel at several arguments one
after another (a batch-size sweep).

usage: prof_summary.py <kernel_trace.csv> [--top N] [--match SUBSTRING]
       prof_summary.py <kernel_trace.csv> --match NAME --blocks X --chunk N [--skip K]
       prof_summary.py --fetch F.csv --write W.csv --copy-bytes B [--match S]
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


def chunks(path: str, match: str, blocks: int, size: int, skip: int):
    runs = []
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            name = short_name(row["Kernel_Name"])
            wg = int(row.get("Workgroup_Size_X", 1) or 1)
            if name != match or int(row.get("Grid_Size_X", 1) or 1) // wg != blocks:
                continue
            start, end = int(row["Start_Timestamp"]), int(row["End_Timestamp"])
            runs.append((start, (end - start) / 1000.0))
    runs.sort()
    total = len(runs)
    runs = runs[skip:]
    print(f"source: {path}")
    print(f"`{match}`, {blocks} workgroups: {total} dispatches; after the first {skip}, "
          f"runs of {size}")
    print()
    print("| run | dispatches | mean us | min us | max us |")
    print("|---|---|---|---|---|")
    for i in range(0, len(runs), size):
        d = [x[1] for x in runs[i:i + size]]
        print(f"| {i // size} | {len(d)} | {sum(d) / len(d):.2f} | {min(d):.2f} | {max(d):.2f} |")
    d = [x[1] for x in runs]
    if d:
        print(f"| all | {len(d)} | {sum(d) / len(d):.2f} | {min(d):.2f} | {max(d):.2f} |")


def counter_groups(path: str, counter: str):
    """Mean value of `counter` per dispatch, by (kernel, blocks, threads)."""
    groups = defaultdict(list)
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] != counter:
                continue
            grid, wg = int(row["Grid_Size"]), int(row["Workgroup_Size"])
            key = (short_name(row["Kernel_Name"]), grid // max(wg, 1), wg)
            groups[key].append(float(row["Counter_Value"]))
    return {k: (len(v), sum(v) / len(v)) for k, v in groups.items()}


def traffic(fetch_csv: str, write_csv: str, copy_bytes: int, copy_match: str,
            match: str | None, top: int):
    fetch = counter_groups(fetch_csv, "FETCH_SIZE")
    write = counter_groups(write_csv, "WRITE_SIZE")
    copies = [k for k in fetch if copy_match in k[0] and k in write]
    if not copies:
        raise SystemExit(f"no dispatch of a kernel named like {copy_match!r} in both runs")
    ck = max(copies, key=lambda k: fetch[k][1])
    fscale = copy_bytes / (fetch[ck][1] * 1024.0)
    wscale = copy_bytes / (write[ck][1] * 1024.0)
    print(f"fetch: {fetch_csv}")
    print(f"write: {write_csv}")
    print(f"calibration: `{ck[0]}` {ck[1]} x {ck[2]}, {fetch[ck][0]} dispatches of "
          f"{copy_bytes} bytes: FETCH_SIZE {fetch[ck][1]:.1f} KiB, WRITE_SIZE "
          f"{write[ck][1]:.1f} KiB; scale fetch {fscale:.4f}, write {wscale:.4f}")
    print()
    print("| kernel | workgroups | threads | calls | FETCH_SIZE KiB | WRITE_SIZE KiB | "
          "scaled read MB | scaled write MB |")
    print("|---|---|---|---|---|---|---|---|")
    rows = []
    for k, (n, f) in fetch.items():
        if match and match not in k[0]:
            continue
        w = write.get(k, (0, 0.0))[1]
        rows.append((f + w, k, n, f, w))
    rows.sort(reverse=True)
    for _, k, n, f, w in rows[:top]:
        print(f"| `{k[0]}` | {k[1]} | {k[2]} | {n} | {f:.1f} | {w:.1f} | "
              f"{f * 1024 * fscale / 1e6:.3f} | {w * 1024 * wscale / 1e6:.3f} |")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace", nargs="?")
    ap.add_argument("--top", type=int, default=40)
    ap.add_argument("--match", default=None)
    ap.add_argument("--fetch", default=None)
    ap.add_argument("--write", default=None)
    ap.add_argument("--copy-bytes", type=int, default=0)
    ap.add_argument("--copy-match", default="copyBuffer")
    ap.add_argument("--blocks", type=int, default=0)
    ap.add_argument("--chunk", type=int, default=0)
    ap.add_argument("--skip", type=int, default=0)
    a = ap.parse_args()
    if a.fetch or a.write:
        if not (a.fetch and a.write and a.copy_bytes > 0):
            ap.error("--fetch, --write and --copy-bytes go together")
        traffic(a.fetch, a.write, a.copy_bytes, a.copy_match, a.match, a.top)
    elif a.trace and a.chunk > 0:
        if not (a.match and a.blocks > 0):
            ap.error("--chunk needs --match (the exact short kernel name) and --blocks")
        chunks(a.trace, a.match, a.blocks, a.chunk, a.skip)
    elif a.trace:
        summarize(a.trace, a.top, a.match)
    else:
        ap.error("a kernel trace CSV, or --fetch/--write")


if __name__ == "__main__":
    sys.exit(main())
