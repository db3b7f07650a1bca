"""Host-side behaviour of bench.py that needs no GPU: the refusal of runs on
more than one GPU, and the accounting of the untimed warm-up before a timed
region."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import bench

ROOT = Path(__file__).resolve().parents[1]


def _run(args, env=None):
    return subprocess.run([sys.executable, str(ROOT / "bench.py"), *args], capture_output=True,
                          text=True, timeout=120, env=env)


def test_more_than_one_gpu_is_refused():
    r = _run(["--gpus", "2"])
    assert r.returncode == 2
    assert "one GPU" in r.stderr
    assert r.stdout == ""


def test_a_distributed_launch_is_refused():
    env = dict(os.environ, WORLD_SIZE="2")
    r = _run([], env)
    assert r.returncode == 2
    assert "WORLD_SIZE" in r.stderr


class _Timer:
    """The two timer calls of a context, returning a fixed GPU time."""

    def __init__(self, ms: float):
        self.ms = ms
        self.open = False

    def timer_start(self) -> None:
        assert not self.open
        self.open = True

    def timer_stop(self) -> float:
        assert self.open
        self.open = False
        return self.ms


def test_warm_up_stops_once_the_gpu_time_is_spent():
    calls = []
    bench.warm_up(_Timer(7.0), lambda: calls.append(1), 60.0)
    assert len(calls) == 9  # 8 calls spend 56 ms, the 9th reaches 63


def test_warm_up_of_zero_runs_nothing():
    calls = []
    bench.warm_up(_Timer(1.0), lambda: calls.append(1), 0.0)
    assert calls == []
