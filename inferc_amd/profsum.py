"""Summarise a rocprofv3 kernel trace by kernel and launch grid.

``rocprofv3 --stats`` aggregates by kernel name only; one GEMM template serves
several shapes, so this groups dispatches by (name, grid) to give per-shape
average durations. Reads either the CSV trace (``--output-format csv``:
``*_kernel_trace.csv``) or the SQLite database rocprofv3 writes by default.

Usage: python -m inferc_amd.profsum <trace.csv | results.db> [--top N]
       python -m inferc_amd.profsum --traffic FETCH.csv WRITE.csv --copy-bytes B
       python -m inferc_amd.profsum --mfma MFMA.csv [--simds 1024] [--xcc 8]

The ``--traffic`` form reads two ``rocprofv3 --pmc FETCH_SIZE`` /
``--pmc WRITE_SIZE`` counter CSVs of the same program, takes the largest
``__amd_rocclr_copyBuffer`` dispatch (a device copy of ``B`` bytes) as the
calibration (counter KiB that a copy of known size reads), and prints every
other kernel's mean per-dispatch HBM bytes scaled by that factor.

The ``--mfma`` form reads one ``rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_F32
SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE`` CSV and prints per (kernel, grid):
the fp32 MFMA FLOPs the counter saw (MOPS x 512) per dispatch, the dispatch's
duration (its timestamps) and the FLOP rate over it, the MFMA busy fraction
SQ_VALU_MFMA_BUSY_CYCLES / (simds x GRBM_GUI_ACTIVE / xcc) (the busy counter
is summed over every SIMD, the GUI counter over every XCC), the same busy
count over simds x duration x clock (busy%d), and the engine clock that
GRBM_GUI_ACTIVE / xcc over the duration implies. On dispatches of a few us
the GUI counter also covers time outside the dispatch's timestamps (the
implied clock exceeds the engine's), so busy%d is the figure for them;
dispatches of one template and grid are split by their FLOP count.
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


def _counter_means(path: str):
    per = defaultdict(list)
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            per[(r["Kernel_Name"], int(r["Grid_Size"]))].append(float(r["Counter_Value"]))
    return per


def traffic(fetch_csv: str, write_csv: str, copy_bytes: int) -> dict:
    """Per-(kernel, grid) mean fetch/write KiB and calibrated HBM bytes."""
    out = {}
    scales = {}
    for tag, path in (("fetch", fetch_csv), ("write", write_csv)):
        per = _counter_means(path)
        copies = [max(v) for (n, _), v in per.items() if "copyBuffer" in n]
        if not copies:
            raise SystemExit(f"{path}: no copy dispatch to calibrate against")
        scales[tag] = copy_bytes / 1024.0 / max(copies)
        for (name, grid), v in per.items():
            if "copyBuffer" in name:
                continue
            e = out.setdefault((name, grid), {"dispatches": len(v)})
            e[f"{tag}_kib"] = sum(v) / len(v)
    for e in out.values():
        e["bytes"] = 1024.0 * (e.get("fetch_kib", 0.0) * scales["fetch"] +
                               e.get("write_kib", 0.0) * scales["write"])
    return {"fetch_scale": scales["fetch"], "write_scale": scales["write"], "kernels": out}


def mfma(path: str, simds: int, xcc: int, clock_mhz: float) -> list[dict]:
    """Per-(kernel, grid) means of the MFMA counters and derived rates."""
    per = defaultdict(lambda: defaultdict(dict))
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            key = (r["Kernel_Name"], int(r["Grid_Size"]))
            d = per[key][r.get("Dispatch_Id") or r["Correlation_Id"]]
            d[r["Counter_Name"]] = float(r["Counter_Value"])
            d["us"] = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    # one template and grid can serve several shapes (the encoder's out-proj
    # and FFN-down both write 128 x 768): split a group by its FLOP count
    groups = defaultdict(list)
    for (name, grid), ds in per.items():
        for d in ds.values():
            fl = 512.0 * d.get("SQ_INSTS_VALU_MFMA_MOPS_F32", 0.0)
            groups[(name, grid, float(f"{fl:.3e}"))].append(d)
    out = []
    for (name, grid, _), ds in groups.items():
        n = len(ds)
        mean = lambda k: sum(d.get(k, 0.0) for d in ds) / n  # noqa: E731
        us, gui = mean("us"), mean("GRBM_GUI_ACTIVE")
        flops = 512.0 * mean("SQ_INSTS_VALU_MFMA_MOPS_F32")
        busy = mean("SQ_VALU_MFMA_BUSY_CYCLES")
        cyc = gui / xcc
        out.append({"kernel": name, "grid": grid, "dispatches": n, "us": us, "flops": flops,
                    "tflops": flops / (us * 1e-6) / 1e12 if us > 0 else 0.0,
                    "mfma_busy": busy / (simds * cyc) if cyc > 0 else 0.0,
                    "mfma_busy_dur": busy / (simds * us * clock_mhz) if us > 0 else 0.0,
                    "clock_mhz": cyc / us if us > 0 else 0.0})
    return sorted(out, key=lambda e: -e["us"] * e["dispatches"])


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("trace", nargs="?")
    ap.add_argument("--top", type=int, default=25)
    ap.add_argument("--traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"))
    ap.add_argument("--copy-bytes", type=int, default=64 << 20)
    ap.add_argument("--mfma", metavar="MFMA_CSV")
    ap.add_argument("--simds", type=int, default=1024, help="SIMDs on the device (256 CUs x 4)")
    ap.add_argument("--xcc", type=int, default=8, help="XCCs summed by GRBM_GUI_ACTIVE")
    ap.add_argument("--clock-mhz", type=float, default=2280.0,
                    help="engine clock for the duration-based busy fraction")
    a = ap.parse_args(argv)
    if a.mfma:
        rows = mfma(a.mfma, a.simds, a.xcc, a.clock_mhz)
        print(f"{'disp':>5} {'avg_us':>8} {'MFMA_GFLOP':>11} {'TFLOP/s':>8} {'busy%':>6} "
              f"{'busy%d':>6} {'clk_MHz':>8} {'grid':>9}  kernel")
        for e in rows[:a.top]:
            print(f"{e['dispatches']:5d} {e['us']:8.2f} {e['flops'] / 1e9:11.4f} "
                  f"{e['tflops']:8.2f} {100 * e['mfma_busy']:6.1f} "
                  f"{100 * e['mfma_busy_dur']:6.1f} {e['clock_mhz']:8.0f} "
                  f"{e['grid']:>9}  {_short(e['kernel'])}")
        return 0
    if a.traffic:
        t = traffic(a.traffic[0], a.traffic[1], a.copy_bytes)
        print(f"calibration: FETCH_SIZE x{t['fetch_scale']:.4f}, "
              f"WRITE_SIZE x{t['write_scale']:.4f} (copy of {a.copy_bytes} bytes)")
        print(f"{'dispatches':>10} {'fetch_KiB':>11} {'write_KiB':>11} {'HBM_bytes':>13}  "
              f"{'grid':>8}  kernel")
        for (name, grid), e in sorted(t["kernels"].items(), key=lambda kv: -kv[1]["bytes"]):
            print(f"{e['dispatches']:10d} {e.get('fetch_kib', 0):11.1f} "
                  f"{e.get('write_kib', 0):11.1f} {e['bytes']:13.0f}  {grid:>8}  {_short(name)}")
        return 0
    if not a.trace:
        ap.error("a trace file is required")
    print(summarize(load(a.trace), a.top))
    return 0


if __name__ == "__main__":
    sys.exit(main())
