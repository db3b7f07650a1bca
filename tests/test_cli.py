"""The inferc commands (src/cli/main.cpp): inspect, compare and the argument
errors of run/decode without a GPU; run and decode end to end on the GPU
against torch's outputs for the exported fixture models."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest

from inferc_amd import cli
from inferc_amd import lib as L

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    if not L.library_path().exists():
        from inferc_amd.build import build

        build()


def test_inspect_prints_the_summary(capsys):
    assert cli.main(["inspect", str(GOLDEN / "gpt2_tiny_past.onnx")]) == 0
    out = capsys.readouterr().out.splitlines()
    assert out[0] == "Model: main_graph"
    assert "Inputs (6):" in out and "Outputs (5):" in out
    assert any(ln.startswith("  present.1.value") for ln in out)
    assert cli.main(["inspect", "/no/such/file.onnx"]) == 1


def test_argument_errors(capsys, tmp_path):
    assert cli.main(["run"]) == 2
    assert cli.main(["run", "m.onnx", "--input-ids", "a"]) == 2
    assert "required" in capsys.readouterr().err
    assert cli.main(["run", "m.onnx", "--input-ids", "a", "--attention-mask", "b"]) == 2
    assert "--output and/or --profile" in capsys.readouterr().err
    assert cli.main(["run", "m.onnx", "--bogus"]) == 2
    assert "unknown arg" in capsys.readouterr().err
    assert cli.main(["decode", "--model", "a.onnx"]) == 2
    dec = ["decode", "--model", "a.onnx", "--past-model", "b.onnx", "--prompt-ids", "p.bin",
           "--output", "o.bin"]
    assert cli.main(dec + ["--device", "x"]) == 2
    assert "integers" in capsys.readouterr().err
    for flag in ("--no-gemv", "--no-fold", "--no-optimize"):
        assert cli.main(dec + ["--int4", flag]) == 2
        assert "graph executor" in capsys.readouterr().err
    assert cli.main(dec + ["--no-such-flag"]) == 2
    assert cli.main(["compare", "only_one.json"]) == 2
    assert cli.main(["nope"]) == 1


def test_compare(capsys, tmp_path):
    rep = {"backend": "x", "model": "m", "iterations": 2,
           "total": {"mean_ms": 1.0, "p50_ms": 1.0, "p95_ms": 1.0, "min_ms": 1.0, "max_ms": 1.0},
           "per_op_type": {"MatMul": {"calls_per_iter": 3, "total_ms": {"mean_ms": 0.5}}},
           "op_counts": {"MatMul": 3}, "peak_rss_bytes": 0, "activation_bytes_peak": 0}
    a, b = tmp_path / "a.json", tmp_path / "b.json"
    a.write_text(json.dumps(rep))
    b.write_text(json.dumps(dict(rep, backend="y", total=dict(rep["total"], mean_ms=2.0))))
    assert cli.main(["compare", str(a), str(b)]) == 0
    assert "x is 2.00x faster than y (mean total)" in capsys.readouterr().out


@pytest.mark.gpu
def test_run_writes_logits_and_profile(ctx, tmp_path, capsys):
    io = np.load(GOLDEN / "distilbert_tiny_io.npz")
    ids, mask = tmp_path / "ids.bin", tmp_path / "mask.bin"
    io["ids_a"].astype(np.int64).tofile(ids)
    io["mask_a"].astype(np.int64).tofile(mask)
    out, prof = tmp_path / "logits.bin", tmp_path / "prof.json"
    assert cli.main(["run", str(GOLDEN / "distilbert_tiny.onnx"), "--input-ids", str(ids),
                     "--attention-mask", str(mask), "--shape", "2,16", "--output", str(out),
                     "--profile", str(prof), "-n", "3", "--warmup", "1"]) == 0
    got = np.fromfile(out, np.float32).reshape(2, 2)
    assert np.max(np.abs(got - io["logits_a"])) <= 1e-4
    rep = json.loads(prof.read_text())
    assert rep["iterations"] == 3 and rep["op_counts"]["FusedAttention"] == 2
    assert "values:" in capsys.readouterr().out


@pytest.mark.gpu
def test_decode_two_graphs_matches_torch(ctx, tmp_path):
    """`inferc decode --model prefill --past-model with_past`: the prefill
    graph's present.* seed the device KV cache; tokens equal torch's greedy
    generation with its cache."""
    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    ids, out, prof = tmp_path / "prompt.bin", tmp_path / "toks.bin", tmp_path / "dec.json"
    io["prompt"].astype(np.int64).tofile(ids)
    assert cli.main(["decode", "--model", str(GOLDEN / "gpt2_tiny_prefill.onnx"),
                     "--past-model", str(GOLDEN / "gpt2_tiny_past.onnx"),
                     "--prompt-ids", str(ids), "--max-tokens", "12", "--output", str(out),
                     "--profile", str(prof)]) == 0
    np.testing.assert_array_equal(np.fromfile(out, np.int64), io["gen_tokens"])
    rep = json.loads(prof.read_text())
    assert rep["iterations"] == 11 and rep["op_counts"]["FusedAttentionPast"] == 2


@pytest.mark.gpu
@pytest.mark.parametrize("flags", [["--no-gemv"], ["--no-fold"], ["--no-gemv", "--no-fold"],
                                   ["--device", "0"], ["--native"]])
def test_decode_flags_keep_the_tokens(ctx, tmp_path, flags):
    """The reference's ablation flags (--no-gemv: the one-row GEMV route off,
    main.cpp:718,727; --no-fold: FoldConstantTranspose, RecognizeLayerNorm
    and RecognizeGeluTanh left out, :719,756-775) change how the graphs run,
    not the greedy tokens; --native runs the same weights on the native
    decoder."""
    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    ids, out = tmp_path / "prompt.bin", tmp_path / "toks.bin"
    io["prompt"].astype(np.int64).tofile(ids)
    assert cli.main(["decode", "--model", str(GOLDEN / "gpt2_tiny_prefill.onnx"),
                     "--past-model", str(GOLDEN / "gpt2_tiny_past.onnx"),
                     "--prompt-ids", str(ids), "--max-tokens", "12", "--output", str(out)]
                    + flags) == 0
    np.testing.assert_array_equal(np.fromfile(out, np.int64), io["gen_tokens"])
    assert ctx.gemv_decode_enabled()


@pytest.mark.gpu
def test_decode_int4_needs_the_gpt2_small_row_lengths(ctx, tmp_path, capsys):
    """--int4 on a model whose projections the int4 decode GEMV does not
    cover (hidden 64 here; it needs hidden 768, ffn 3072) fails cleanly with
    exit code 1. The int4 route itself is checked at GPT-2-small shape in
    test_gpu_onnx.py."""
    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    ids, out = tmp_path / "prompt.bin", tmp_path / "toks.bin"
    io["prompt"].astype(np.int64).tofile(ids)
    assert cli.main(["decode", "--model", str(GOLDEN / "gpt2_tiny_prefill.onnx"),
                     "--past-model", str(GOLDEN / "gpt2_tiny_past.onnx"),
                     "--prompt-ids", str(ids), "--max-tokens", "4", "--output", str(out),
                     "--int4"]) == 1
    assert "hidden 768, ffn 3072" in capsys.readouterr().err
