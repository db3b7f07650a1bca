"""Host-side mirror of ``inferc::prof`` (src/profiler/profiler.h:40-89) over
the C-ABI, and the ``inferc compare`` table (src/cli/main.cpp:481-593).

:class:`Profiler` owns an ``inferc_profiler``: the host-clock calls
(begin/end iteration and op) behave as the reference's, and the executor and
GPT-2 decoder record into it with device times
(:meth:`inferc_amd.rt.Executor.run_profiled`,
:meth:`inferc_amd.rt.Gpt2Decoder.generate_profiled`). :meth:`Profiler.to_json`
returns the reference's report schema (profiler.cc:138-176), so two reports
(for instance the reference's CPU profile and this backend's) can be set side
by side with :func:`compare_table`.

Usage: ``python -m inferc_amd.profiler compare <a.json> <b.json>``.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import sys
from typing import Sequence

from . import lib as L
from .lib import check

_D = C.c_double
STAT_KEYS = ("mean", "p50", "p95", "min", "max")


def _sample(v: Sequence[float]):
    arr = (_D * max(1, len(v)))(*[float(x) for x in v])
    return arr, len(v)


def percentile(v: Sequence[float], p: float) -> float:
    """prof::Percentile (profiler.cc:25-37): numpy's default linear
    interpolation between closest ranks; 0 for an empty sample."""
    arr, n = _sample(v)
    out = _D()
    check(L.load_library().inferc_profile_percentile(arr, n, p, C.byref(out)))
    return out.value


def stats_from(v: Sequence[float]) -> dict[str, float]:
    """prof::StatsFrom (profiler.cc:39-49): mean, p50, p95, min, max."""
    arr, n = _sample(v)
    out = (_D * 5)()
    check(L.load_library().inferc_profile_stats(arr, n, out))
    return dict(zip(STAT_KEYS, out))


class Profiler:
    """prof::Profiler (profiler.h:40-85)."""

    def __init__(self):
        self._lib = L.load_library()
        h = C.c_void_p()
        check(self._lib.inferc_profiler_create(C.byref(h)))
        self.handle = h.value

    def begin_iteration(self) -> None:
        check(self._lib.inferc_profiler_begin_iteration(self.handle))

    def end_iteration(self) -> None:
        check(self._lib.inferc_profiler_end_iteration(self.handle))

    def begin_op(self, op_type: str, node_name: str = "") -> None:
        check(self._lib.inferc_profiler_begin_op(self.handle, op_type.encode(),
                                                 node_name.encode()))

    def end_op(self, activation_bytes_after: int = 0) -> None:
        check(self._lib.inferc_profiler_end_op(self.handle, activation_bytes_after))

    def record_op(self, op_type: str, node_name: str, ms: float,
                  activation_bytes_after: int = 0) -> None:
        """Adds a finished op timed by the caller."""
        check(self._lib.inferc_profiler_record_op(self.handle, op_type.encode(),
                                                  node_name.encode(), ms,
                                                  activation_bytes_after))

    def set_track_activation_bytes(self, on: bool) -> None:
        check(self._lib.inferc_profiler_set_track_activation_bytes(self.handle, int(on)))

    def snapshot_peak_rss(self) -> None:
        check(self._lib.inferc_profiler_snapshot_peak_rss(self.handle))

    def iterations(self) -> int:
        n = C.c_int64()
        check(self._lib.inferc_profiler_iteration_count(self.handle, C.byref(n)))
        return n.value

    def total_stats(self) -> dict[str, float]:
        out = (_D * 5)()
        check(self._lib.inferc_profiler_total_stats(self.handle, out))
        return dict(zip(STAT_KEYS, out))

    def to_json(self, backend: str, model: str = "") -> str:
        """Profiler::ToJson (profiler.cc:138-176)."""
        n = C.c_size_t()
        b, m = backend.encode(), model.encode()
        check(self._lib.inferc_profiler_to_json(self.handle, b, m, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        check(self._lib.inferc_profiler_to_json(self.handle, b, m, buf, n.value + 1, C.byref(n)))
        return buf.value.decode()

    def report(self, backend: str, model: str = "") -> dict:
        return json.loads(self.to_json(backend, model))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.inferc_profiler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def compare_table(a: dict, b: dict, top: int = 12) -> str:
    """The ``inferc compare`` report (main.cpp:481-593): totals of both
    profiles, which is faster, then the op types of either report ordered by
    the larger of their two mean per-iteration times, with the ratio b/a.
    ``calls/iter`` is taken from the first report where it has the op."""
    def bn(j):
        return j.get("backend", "?")

    def tot(j, k):
        return float(j.get("total", {}).get(k, 0.0))

    out = ["", "=== inferc compare ===", f"  model: {a.get('model', '?')}", ""]
    out.append(f"{'backend':<20}{'iters':>8}{'mean(ms)':>11}{'p50(ms)':>11}{'p95(ms)':>11}"
               f"{'min(ms)':>11}{'max(ms)':>11}{'RSS(MB)':>10}")
    out.append("-" * 93)
    for j in (a, b):
        out.append(f"{bn(j):<20}{int(j.get('iterations', 0)):>8}"
                   + "".join(f"{tot(j, k):>11.2f}" for k in
                             ("mean_ms", "p50_ms", "p95_ms", "min_ms", "max_ms"))
                   + f"{j.get('peak_rss_bytes', 0) / (1024.0 * 1024.0):>10.1f}")
    am, bm = tot(a, "mean_ms"), tot(b, "mean_ms")
    if am > 0 and bm > 0:
        faster = am < bm
        f = bm / am if faster else am / bm
        out += ["", f"  {bn(a)} is {f:.2f}x {'faster' if faster else 'slower'} than {bn(b)} "
                    "(mean total)"]
    if "per_op_type" in a or "per_op_type" in b:
        out += ["", f"Top ops by mean total time per iter (ratio = {bn(b)}/{bn(a)}):"]
        out.append(f"{'op_type':<20}{'calls/iter':>11}{(bn(a) + '(ms)')[:15]:>16}"
                   f"{(bn(b) + '(ms)')[:15]:>16}{'ratio':>10}")
        out.append("-" * 73)
        rows: dict[str, list] = {}
        for slot, j in enumerate((a, b)):
            for op, val in j.get("per_op_type", {}).items():
                r = rows.setdefault(op, [0, 0.0, 0.0])
                r[1 + slot] = float(val.get("total_ms", {}).get("mean_ms", 0.0))
                calls = int(val.get("calls_per_iter", 0))
                if slot == 0 or r[0] == 0:
                    r[0] = calls
        order = sorted(rows.items(), key=lambda kv: -max(kv[1][1], kv[1][2]))
        for op, (calls, x, y) in order[:top]:
            line = f"{op:<20}{calls:>11}{x:>16.3f}{y:>16.3f}"
            if x > 0 and y > 0:
                r = y / x
                line += f"{r:>10.{3 if r < 1.0 else 2}f}"
            else:
                line += f"{'—':>10}"
            out.append(line)
    out.append("")
    return "\n".join(out)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description="inferc profile reports")
    sub = ap.add_subparsers(dest="cmd", required=True)
    c = sub.add_parser("compare", help="side-by-side table of two profile JSON files")
    c.add_argument("a")
    c.add_argument("b")
    args = ap.parse_args(argv)
    with open(args.a) as fa, open(args.b) as fb:
        a, b = json.load(fa), json.load(fb)
    print(compare_table(a, b))
    return 0


if __name__ == "__main__":
    sys.exit(main())
