"""Summarise a rocprofv3 kernel trace by kernel and launch grid.

``rocprofv3 --stats`` aggregates by kernel name only; one GEMM template serves
several shapes, so this groups dispatches by (name, grid) to give per-shape
average durations. Reads either the CSV trace (``--output-format csv``:
``*_kernel_trace.csv``) or the SQLite database rocprofv3 writes by default.

Usage: python -m inferc_amd.profsum <trace.csv | results.db> [--top N]
"""
from __future__ import annotations

import argparse
import csv
import sqlite3
import sys
from collections import defaultdict


def _short(name: str, width: int = 96) -> str:
    name = name.replace("ih::(anonymous namespace)::", "")
    return name if len(name) <= width else name[: width - 3] + "..."


def load(path: str):
    rows = []
    if path.endswith(".db"):
        con = sqlite3.connect(path)
        for name, gx, gy, gz, wx, start, end in con.execute(
                "select name, grid_x, grid_y, grid_z, workgroup_x, start, end from kernels"):
            rows.append((name, (gx, gy, gz), wx, (end - start) / 1e3))
    else:
        with open(path, newline="") as f:
            for r in csv.DictReader(f):
                grid = (int(r["Grid_Size_X"]), int(r["Grid_Size_Y"]), int(r["Grid_Size_Z"]))
                rows.append((r["Kernel_Name"], grid, int(r["Workgroup_Size_X"]),
                             (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3))
    return rows


def summarize(rows, top: int = 25) -> str:
    agg = defaultdict(list)
    for name, grid, wg, us in rows:
        agg[(name, grid, wg)].append(us)
    total = sum(us for *_, us in rows) or 1.0
    lines = [f"{'calls':>6} {'avg_us':>9} {'min_us':>9} {'total_us':>11} {'pct':>5}  "
             f"{'grid(x,y,z)/wg':<24} kernel"]
    for (name, grid, wg), v in sorted(agg.items(), key=lambda kv: -sum(kv[1]))[:top]:
        g = f"{grid[0]},{grid[1]},{grid[2]}/{wg}"
        lines.append(f"{len(v):6d} {sum(v) / len(v):9.2f} {min(v):9.2f} {sum(v):11.1f} "
                     f"{100 * sum(v) / total:5.1f}  {g:<24} {_short(name)}")
    return "\n".join(lines)


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--top", type=int, default=25)
    a = ap.parse_args(argv)
    print(summarize(load(a.trace), a.top))
    return 0


if __name__ == "__main__":
    sys.exit(main())
