"""The native profiler (no GPU): prof::Percentile / StatsFrom known answers
from the reference's tests (tests/profiler_test.cc:14-40), the record and
error behaviour of prof::Profiler (:42-95), its JSON report schema (:97-121,
src/profiler/profiler.cc:138-176), a dry-run executor's profiled pass with
the reference's live-activation-byte accounting (src/runtime/executor.cc:
112-119), and the `inferc compare` table (src/cli/main.cpp:481-593)."""
from __future__ import annotations

import json
import time

import numpy as np
import pytest

from inferc_amd import lib as L
from inferc_amd import profiler as P
from inferc_amd.rt import Executor, Graph


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not L.library_path().exists():
        from inferc_amd.build import build

        build()


# ---------------------------------------------------------------- statistics

def test_percentile_known_answers():
    v = [1, 2, 3, 4, 5]
    assert P.percentile(v, 0) == 1.0
    assert P.percentile(v, 100) == 5.0
    assert P.percentile(v, 50) == 3.0
    assert P.percentile(v, 25) == 2.0
    assert P.percentile(v, 75) == 4.0
    assert P.percentile([10, 20, 30, 40], 50) == 25.0


def test_stats_from_known_answers():
    s = P.stats_from([2.0, 4.0, 6.0, 8.0])
    assert (s["mean"], s["min"], s["max"], s["p50"]) == (5.0, 2.0, 8.0, 5.0)
    # rank 0.95 * 3 = 2.85 -> 6 + 0.85 * (8 - 6)
    assert s["p95"] == pytest.approx(7.7, abs=1e-12)
    assert P.stats_from([]) == dict.fromkeys(P.STAT_KEYS, 0.0)
    assert P.stats_from([3.5]) == dict.fromkeys(P.STAT_KEYS, 3.5)


@pytest.mark.parametrize("n", [2, 3, 7, 50])
def test_percentile_matches_numpy_linear(n):
    """numpy's default percentile is the same type-7 rule; unsorted input."""
    v = np.random.default_rng(n).standard_normal(n) * 10
    for p in (0, 1, 5, 12.5, 33.3, 50, 77, 95, 99, 100):
        assert P.percentile(list(v), p) == pytest.approx(np.percentile(v, p), rel=1e-12,
                                                         abs=1e-12)
    s = P.stats_from(list(v))
    assert s["mean"] == pytest.approx(v.mean(), rel=1e-12)
    assert (s["min"], s["max"]) == (v.min(), v.max())


def test_percentile_planted_nearest_rank_differs():
    """A nearest-rank percentile (no interpolation) would give 20 or 30 for
    the median of {10,20,30,40}; the interpolated answer is pinned at 25."""
    v = [40, 10, 30, 20]
    assert P.percentile(v, 50) == 25.0
    assert P.percentile(v, 50) not in (20.0, 30.0)


# ---------------------------------------------------------------- records

def test_records_iterations_and_ops():
    p = P.Profiler()
    for _ in range(5):
        p.begin_iteration()
        p.begin_op("MatMul", "n0")
        time.sleep(200e-6)
        p.end_op(1024)
        p.begin_op("Add", "n1")
        time.sleep(100e-6)
        p.end_op(2048)
        p.end_iteration()
    assert p.iterations() == 5
    r = p.report("inferc-hip")
    assert r["op_counts"] == {"MatMul": 1, "Add": 1}
    assert r["activation_bytes_peak"] == 2048
    assert r["total"]["min_ms"] > 0
    assert r["per_op_type"]["MatMul"]["total_ms"]["min_ms"] >= 0.2
    # the ops sit inside their iteration
    ops = r["per_op_type"]["MatMul"]["total_ms"]["mean_ms"] + \
        r["per_op_type"]["Add"]["total_ms"]["mean_ms"]
    assert ops <= r["total"]["mean_ms"]


def test_begin_op_twice_and_end_op_without_begin_fail():
    p = P.Profiler()
    p.begin_iteration()
    p.begin_op("A", "a")
    with pytest.raises(RuntimeError, match="another op is in flight"):
        p.begin_op("B", "b")
    q = P.Profiler()
    q.begin_iteration()
    with pytest.raises(RuntimeError, match="EndOp called without BeginOp"):
        q.end_op(0)
    with pytest.raises(RuntimeError, match="EndIteration without BeginIteration"):
        P.Profiler().end_iteration()


def test_per_op_type_stats_are_over_per_iteration_sums():
    """Known op times: MatMul sums per iteration are 3, 7, 11 and Add 0.5, 1.5,
    2.5, so the per-op-type statistics are those of the sums, with counts
    taken from the first iteration."""
    p = P.Profiler()
    times = [(1.0, 2.0, 0.5), (3.0, 4.0, 1.5), (5.0, 6.0, 2.5)]
    for i, (m0, m1, a) in enumerate(times):
        p.begin_iteration()
        p.record_op("MatMul", "m0", m0, 100 * i)
        p.record_op("Add", "a0", a, 700)
        p.record_op("MatMul", "m1", m1, 50)
        p.end_iteration()
    r = p.report("x")
    mm = r["per_op_type"]["MatMul"]
    assert mm["calls_per_iter"] == 2
    sums = [3.0, 7.0, 11.0]
    assert mm["total_ms"] == {"mean_ms": 7.0, "p50_ms": 7.0,
                              "p95_ms": pytest.approx(np.percentile(sums, 95), abs=1e-12),
                              "min_ms": 3.0, "max_ms": 11.0}
    ad = r["per_op_type"]["Add"]["total_ms"]
    assert (ad["mean_ms"], ad["min_ms"], ad["max_ms"]) == (1.5, 0.5, 2.5)
    assert r["op_counts"] == {"Add": 1, "MatMul": 2}
    assert r["activation_bytes_peak"] == 700
    with pytest.raises(RuntimeError, match="in flight"):
        p.begin_iteration()
        p.begin_op("X")
        p.record_op("Y", "", 1.0)


def test_json_round_trips_expected_keys():
    p = P.Profiler()
    for _ in range(3):
        p.begin_iteration()
        p.begin_op("MatMul", "m0")
        time.sleep(50e-6)
        p.end_op(512)
        p.end_iteration()
    p.snapshot_peak_rss()
    s = p.to_json("inferc-baseline", "models/distilbert.onnx")
    j = json.loads(s)
    assert sorted(j) == ["activation_bytes_peak", "backend", "iterations", "model",
                         "op_counts", "peak_rss_bytes", "per_op_type", "total"]
    assert j["backend"] == "inferc-baseline"
    assert j["model"] == "models/distilbert.onnx"
    assert j["iterations"] == 3
    assert sorted(j["total"]) == ["max_ms", "mean_ms", "min_ms", "p50_ms", "p95_ms"]
    assert j["per_op_type"]["MatMul"]["calls_per_iter"] == 1
    assert j["op_counts"]["MatMul"] == 1
    assert j["peak_rss_bytes"] > 0
    assert j["activation_bytes_peak"] == 512
    # the layout of the reference's dump(2): sorted keys, two-space indent
    assert s == json.dumps(j, indent=2, sort_keys=True, ensure_ascii=False)


def test_empty_report_and_string_escaping():
    p = P.Profiler()
    name = 'q"uote\\back\nline\ttab\x01é'
    j = json.loads(p.to_json(name, "m"))
    assert j["backend"] == name
    assert j["iterations"] == 0
    assert j["per_op_type"] == {} and j["op_counts"] == {}
    assert j["total"] == {"mean_ms": 0.0, "p50_ms": 0.0, "p95_ms": 0.0, "min_ms": 0.0,
                          "max_ms": 0.0}
    assert j["activation_bytes_peak"] == 0


def test_json_numbers_round_trip_exactly():
    p = P.Profiler()
    vals = [0.1, 1.0 / 3.0, 1e-7, 123456.789, 2.0 ** -30, 5e300]
    p.begin_iteration()
    for i, v in enumerate(vals):
        p.record_op(f"op{i}", "", v)
    p.end_iteration()
    j = p.report("b")
    for i, v in enumerate(vals):
        assert j["per_op_type"][f"op{i}"]["total_ms"]["mean_ms"] == v


def test_json_buffer_too_small_is_an_error():
    import ctypes as C
    p = P.Profiler()
    n = C.c_size_t()
    lib = L.load_library()
    assert lib.inferc_profiler_to_json(p.handle, b"b", b"m", None, 0, C.byref(n)) == L.OK
    buf = C.create_string_buffer(int(n.value))
    with pytest.raises(RuntimeError, match="too small"):
        L.check(lib.inferc_profiler_to_json(p.handle, b"b", b"m", buf, n.value, C.byref(n)))


# ---------------------------------------------------------------- executor

def _plumbing_graph() -> Graph:
    g = Graph()
    g.add_initializer("one", np.array(1, np.int64))
    g.add_initializer("zero", np.array(0, np.int64))
    g.add_node("Shape", ["x"], ["s"], name="shape")
    g.add_node("Gather", ["s", "one"], ["n"], axis=0, name="gather")
    g.add_node("Range", ["zero", "n", "one"], ["r"], name="range")
    g.add_node("Unsqueeze", ["r"], ["r2"], axes=[0, 2], name="unsq")
    g.add_node("Reshape", ["x", "s"], ["x2"], name="reshape")
    g.add_node("Squeeze", ["r2"], ["r3"], axes=[0], name="sq")
    g.add_output("x2")
    g.add_output("r3")
    return g


def test_dry_executor_profiled_pass_counts_live_activation_bytes():
    """Live bytes after each node = the input plus every output so far, views
    at their logical size (executor.cc:112-119): x f32[4,9,2] 288, then
    s i64[3] 24, n 8, r i64[9] 72, r2 72, x2 288, r3 72 -> peak 824."""
    ex = Executor.dry(_plumbing_graph())
    ex.set_input("x", np.zeros((4, 9, 2), np.float32))
    p = P.Profiler()
    for _ in range(2):
        ex.run_profiled(p)
    j = p.report("inferc-hip-dry", "plumbing")
    assert j["iterations"] == 2
    assert j["op_counts"] == {"Shape": 1, "Gather": 1, "Range": 1, "Unsqueeze": 1,
                              "Reshape": 1, "Squeeze": 1}
    assert j["activation_bytes_peak"] == 288 + 24 + 8 + 72 + 72 + 288 + 72
    assert all(v["total_ms"]["max_ms"] == 0.0 for v in j["per_op_type"].values())
    q = P.Profiler()
    q.set_track_activation_bytes(False)
    ex.run_profiled(q)
    assert q.report("b")["activation_bytes_peak"] == 0


def test_dry_executor_profile_counts_fused_encoder_ops():
    from inferc_amd import graphs

    cfg = graphs.small_encoder_cfg()
    g = graphs.encoder_graph(cfg, graphs.encoder_weights(cfg, 3))
    ex = Executor.dry(g)
    ids, mask = graphs.encoder_inputs(cfg, 2, 9)
    ex.set_input("input_ids", ids)
    ex.set_input("attention_mask", mask)
    p = P.Profiler()
    ex.run_profiled(p)
    counts = p.report("b")["op_counts"]
    assert sum(counts.values()) == ex.node_count()
    assert counts["FusedAttention"] == cfg["layers"]
    assert counts["FusedQKV"] == cfg["layers"]
    assert counts["FusedMatMulAddGELU"] == cfg["layers"]


# ---------------------------------------------------------------- compare

def _report(backend, total, ops, rss=0, iters=10):
    return {"backend": backend, "model": "distilbert.onnx", "iterations": iters,
            "total": {"mean_ms": total, "p50_ms": total, "p95_ms": total, "min_ms": total,
                      "max_ms": total},
            "per_op_type": {op: {"calls_per_iter": c, "total_ms": {"mean_ms": m}}
                            for op, (c, m) in ops.items()},
            "op_counts": {op: c for op, (c, _) in ops.items()},
            "peak_rss_bytes": rss, "activation_bytes_peak": 0}


def test_compare_table():
    a = _report("inferc-hip", 0.5, {"MatMul": (12, 0.2), "FusedAttention": (6, 0.1)},
                rss=3 * 1024 * 1024)
    b = _report("inferc-cpu", 2.0, {"MatMul": (24, 1.5), "Softmax": (6, 0.3)})
    t = P.compare_table(a, b)
    lines = t.splitlines()
    assert "  model: distilbert.onnx" in lines
    assert "  inferc-hip is 4.00x faster than inferc-cpu (mean total)" in lines
    row = {ln.split()[0]: ln.split() for ln in lines if ln[:1].isalpha() and
           len(ln.split()) == 5 and ln.split()[1].isdigit()}
    assert row["MatMul"] == ["MatMul", "12", "0.200", "1.500", "7.50"]
    assert row["FusedAttention"][4] == "—" and row["Softmax"][1] == "6"
    # ordered by the larger of the two means
    names = [ln.split()[0] for ln in lines if ln.split() and ln.split()[0] in row]
    assert names == ["MatMul", "Softmax", "FusedAttention"]
    rss = [ln for ln in lines if ln.startswith("inferc-hip")][0].split()[-1]
    assert rss == "3.0"
    t2 = P.compare_table(b, a)
    assert "  inferc-cpu is 4.00x slower than inferc-hip (mean total)" in t2.splitlines()
    assert any(ln.split()[:1] == ["MatMul"] and ln.split()[4] == "0.133"
               for ln in t2.splitlines() if len(ln.split()) == 5)


def test_compare_cli(tmp_path, capsys):
    a = tmp_path / "a.json"
    b = tmp_path / "b.json"
    a.write_text(json.dumps(_report("x", 1.0, {"Add": (1, 0.5)})))
    b.write_text(json.dumps(_report("y", 3.0, {"Add": (1, 1.0)})))
    assert P.main(["compare", str(a), str(b)]) == 0
    out = capsys.readouterr().out
    assert "x is 3.00x faster than y" in out
