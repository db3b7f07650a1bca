"""End-to-end GPU parity: the executor running the fused DistilBERT graph and
the GPT-2 greedy decoder against the CPU oracle on identical seeded inputs
(BASELINE configs 1 and 4). Logits within 1e-4 max-abs-diff; greedy token
sequences bit-exact."""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from inferc_amd import graphs, rt
from inferc_amd.profiler import Profiler

pytestmark = pytest.mark.gpu


def _encoder(ctx, cfg, seed):
    w = graphs.encoder_weights(cfg, seed)
    ex = rt.Executor(ctx, graphs.encoder_graph(cfg, w))
    return w, ex


def test_encoder_small_ragged_and_graph_replay(ctx):
    cfg = graphs.small_encoder_cfg()
    w, ex = _encoder(ctx, cfg, 21)
    ids, mask = graphs.encoder_inputs(cfg, 3, 40, ragged=True)
    ref = O.encoder_forward(cfg, w, ids, mask)
    outs = [ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"]
            for _ in range(4)]  # eager, capture, replay, replay
    assert outs[0].shape == (3, 2)
    np.testing.assert_allclose(outs[0], ref, atol=1e-4)
    for o in outs[1:]:
        np.testing.assert_array_equal(o, outs[0])
    ex.set_graph_mode(False)
    np.testing.assert_array_equal(
        ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"], outs[0])
    # a new input shape re-plans
    ids2, mask2 = graphs.encoder_inputs(cfg, 2, 17, seed=8)
    np.testing.assert_allclose(
        ex.run({"input_ids": ids2, "attention_mask": mask2}, ["logits"])["logits"],
        O.encoder_forward(cfg, w, ids2, mask2), atol=1e-4)


def test_encoder_recordings_of_several_signatures(ctx):
    """The executor keeps a recording per input signature (up to four): runs
    that alternate between batch shapes replay each shape's recording, with
    that shape's outputs, after runs of the others; a larger shape, whose
    pass grows the buffers, makes the recordings naming the old ones stale
    instead of replaying them; a fifth signature evicts the least recently
    used. Every run against the oracle."""
    cfg = graphs.small_encoder_cfg()
    w, ex = _encoder(ctx, cfg, 22)
    shapes = {"a": (2, 24), "b": (3, 40), "c": (1, 16), "d": (2, 8), "e": (1, 40)}
    inputs = {k: graphs.encoder_inputs(cfg, B, S, ragged=True, seed=30 + i)
              for i, (k, (B, S)) in enumerate(shapes.items())}
    refs = {k: O.encoder_forward(cfg, w, *inputs[k]) for k in shapes}
    for k in "aaa" "bbb" "aaa" "bab" "ccc" "abc" "ddd" "eee" "abcde" "edcba":
        ids, mask = inputs[k]
        out = ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"]
        assert out.shape == (shapes[k][0], 2), k
        np.testing.assert_allclose(out, refs[k], atol=1e-4, err_msg=k)
    ex.close()


def test_encoder_unsupported_op_raises(ctx):
    g = rt.Graph()
    g.add_node("NonZero", ["x"], ["y"])
    g.add_output("y")
    ex = rt.Executor(ctx, g)
    ex.set_input("x", np.ones(3, np.float32))
    with pytest.raises(RuntimeError, match="unsupported op 'NonZero'"):
        ex.run_async()


def test_executor_folds_add_into_layernorm_and_gathers_by_view(ctx):
    """Add(x[B,S,H], table[positions]) -> LayerNorm runs as one LayerNorm with
    a residual repeated over the batch, and the Gather of rows 2..S+1 of the
    table (host-known Range indices) is a view; checked against numpy."""
    B, S, H = 3, 5, 96
    rng = np.random.default_rng(120)
    table = rng.standard_normal((16, H)).astype(np.float32)
    gamma = rng.standard_normal(H).astype(np.float32)
    beta = rng.standard_normal(H).astype(np.float32)
    x = rng.standard_normal((B, S, H)).astype(np.float32)
    g = rt.Graph()
    g.add_initializer("table", table)
    g.add_initializer("gamma", gamma)
    g.add_initializer("beta", beta)
    g.add_initializer("start", np.array(2, np.int64))
    g.add_initializer("stop", np.array(S + 2, np.int64))
    g.add_initializer("one", np.array(1, np.int64))
    g.add_node("Range", ["start", "stop", "one"], ["pos"])
    g.add_node("Unsqueeze", ["pos"], ["pos2"], axes=[0])
    g.add_node("Gather", ["table", "pos2"], ["pe"], axis=0)
    g.add_node("Add", ["x", "pe"], ["s"])
    g.add_node("FusedLayerNorm", ["s", "gamma", "beta"], ["y"], epsilon=1e-12)
    g.add_output("y")
    ex = rt.Executor(ctx, g)
    got = ex.run({"x": x}, ["y"])["y"]
    s = x.astype(np.float64) + table[2:S + 2][None].astype(np.float64)
    mu = s.mean(-1, keepdims=True)
    var = ((s - mu) ** 2).mean(-1, keepdims=True)
    ref = (s - mu) / np.sqrt(var + 1e-12) * gamma + beta
    assert np.max(np.abs(got - ref)) <= 1e-4


def _check_device_profile(rep, iters):
    assert rep["iterations"] == iters
    per = rep["per_op_type"]
    # device op times sit inside the iteration's wall clock
    assert sum(v["total_ms"]["mean_ms"] for v in per.values()) <= rep["total"]["mean_ms"]
    assert rep["total"]["min_ms"] > 0


def test_executor_profiled_runs(ctx):
    """Profiled eager passes (Executor::Run with a profiler): device time per
    node, the node counts of the fused graph, the dry run's activation bytes,
    and outputs that still match the oracle; the graph captured before the
    profiled passes and one captured after a new shape both replay correctly."""
    cfg = graphs.small_encoder_cfg()
    w, ex = _encoder(ctx, cfg, 31)
    ids, mask = graphs.encoder_inputs(cfg, 3, 40, ragged=True)
    feeds = {"input_ids": ids, "attention_mask": mask}
    ref = O.encoder_forward(cfg, w, ids, mask)
    first = [ex.run(feeds, ["logits"])["logits"] for _ in range(2)]  # eager, capture
    rep = ex.profile(feeds, iters=5, warmup=1, backend="inferc-hip", model="small-encoder",
                     track_activation_bytes=True)
    print({k: round(v["total_ms"]["mean_ms"], 4) for k, v in rep["per_op_type"].items()},
          "total", round(rep["total"]["mean_ms"], 4))
    np.testing.assert_array_equal(ex.output("logits"), first[0])
    np.testing.assert_allclose(first[0], ref, atol=1e-4)
    np.testing.assert_array_equal(ex.run(feeds, ["logits"])["logits"], first[0])  # replay
    _check_device_profile(rep, 5)
    assert rep["peak_rss_bytes"] > 0  # snapshot taken by profile() (main.cpp:382)
    assert sum(rep["op_counts"].values()) == ex.node_count()
    for op in ("FusedQKV", "FusedAttention", "FusedMatMulAddGELU", "FusedGemmEpilogue"):
        assert rep["per_op_type"][op]["total_ms"]["min_ms"] > 0, op
    assert rep["per_op_type"]["Shape"]["total_ms"]["max_ms"] < 0.05
    dry = rt.Executor.dry(graphs.encoder_graph(cfg, w))
    for k, v in feeds.items():
        dry.set_input(k, v)
    pd = Profiler()
    dry.run_profiled(pd)
    assert rep["activation_bytes_peak"] == pd.report("d")["activation_bytes_peak"] > 0
    # a new input shape, profiled first, then eager + capture + replay
    ids2, mask2 = graphs.encoder_inputs(cfg, 2, 17, seed=5)
    feeds2 = {"input_ids": ids2, "attention_mask": mask2}
    rep2 = ex.profile(feeds2, iters=2, warmup=0)
    _check_device_profile(rep2, 2)
    ref2 = O.encoder_forward(cfg, w, ids2, mask2)
    for _ in range(3):
        np.testing.assert_allclose(ex.run(feeds2, ["logits"])["logits"], ref2, atol=1e-4)


def _decode_counts(layers, embed):
    c = {"LayerNorm+QKV": layers, "AttentionDecode": layers,
         "MatMul+Bias+Residual": 2 * layers, "LayerNorm+MatMulAddGELU": layers,
         "LayerNorm+LMHead+ArgMax": 1}
    if embed:
        c["Embedding"] = 1
    return c


def test_gpt2_small_generate_profiled(ctx):
    cfg = graphs.small_gpt2_cfg()
    w = graphs.gpt2_weights(cfg, 24)
    prompt = graphs.gpt2_prompt(cfg, 7)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=32)
    p = Profiler()
    toks_p = dec.generate_profiled(prompt, 12, p)
    toks, _, _ = dec.generate(prompt, 12)
    np.testing.assert_array_equal(toks_p, toks)
    np.testing.assert_array_equal(toks, O.gpt2_generate(cfg, w, prompt, 12)[0])
    rep = p.report("inferc-decode-hip")
    _check_device_profile(rep, 11)
    assert rep["op_counts"] == _decode_counts(cfg["layers"], embed=True)
    assert all(v["total_ms"]["min_ms"] > 0 for v in rep["per_op_type"].values())


@pytest.mark.parametrize("B,ragged", [(1, False), (32, False), (32, True)])
def test_distilbert_encoder_config1(ctx, B, ragged):
    """6 layers, H 768, 12x64, FFN 3072, S=128."""
    cfg = graphs.DISTILBERT
    w, ex = _encoder(ctx, cfg, 1)
    ids, mask = graphs.encoder_inputs(cfg, B, 128, ragged=ragged)
    got = ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"]
    ref = O.encoder_forward(cfg, w, ids, mask)
    assert got.shape == (B, 2)
    assert np.max(np.abs(got - ref)) <= 1e-4, np.max(np.abs(got - ref))
    again = ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"]
    np.testing.assert_array_equal(again, got)


@pytest.mark.parametrize("B,S,ragged", [(1, 1, False), (1, 77, True), (3, 200, True)])
def test_distilbert_encoder_odd_sequence_lengths(ctx, B, S, ragged):
    """The config-1 encoder off its S = 128: one token (every product a
    single row), 77 tokens (row counts off the tile grid) and 3 x 200 ragged
    rows (the large-M GEMM forms, attention over 200 keys); logits within
    1e-4 of the oracle, and a second run bit-identical."""
    cfg = graphs.DISTILBERT
    w, ex = _encoder(ctx, cfg, 1)
    ids, mask = graphs.encoder_inputs(cfg, B, S, seed=11, ragged=ragged)
    got = ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"]
    ref = O.encoder_forward(cfg, w, ids, mask)
    assert got.shape == (B, 2)
    assert np.max(np.abs(got - ref)) <= 1e-4, np.max(np.abs(got - ref))
    again = ex.run({"input_ids": ids, "attention_mask": mask}, ["logits"])["logits"]
    np.testing.assert_array_equal(again, got)


def test_gpt2_small_generate_and_forward(ctx):
    cfg = graphs.small_gpt2_cfg()
    w = graphs.gpt2_weights(cfg, 22)
    prompt = graphs.gpt2_prompt(cfg, 9)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=64)
    toks, steps, logits = dec.generate(prompt, 20, want_step_ms=True, want_logits=True)
    ref_toks, ref_logits, margins = O.gpt2_generate(cfg, w, prompt, 20)
    np.testing.assert_array_equal(toks, ref_toks)
    np.testing.assert_allclose(logits, ref_logits, atol=1e-4)
    assert steps.shape == (19,) and np.all(steps > 0)
    np.testing.assert_allclose(dec.forward(prompt), O.gpt2_forward(cfg, w, prompt), atol=1e-4)
    # a second generate on the same model reuses the captured step
    toks2, _, _ = dec.generate(prompt, 20)
    np.testing.assert_array_equal(toks2, toks)
    with pytest.raises(RuntimeError, match="exceed the KV cache"):
        dec.generate(prompt, 60)
    with pytest.raises(RuntimeError, match="out of range"):
        dec.generate(np.array([cfg["vocab"]], np.int64), 2)


@pytest.fixture(scope="module")
def gpt2_full():
    cfg = graphs.GPT2_SMALL
    return cfg, graphs.gpt2_weights(cfg, 2)


def test_gpt2_forward_logits_config4(ctx, gpt2_full):
    cfg, w = gpt2_full
    prompt = graphs.gpt2_prompt(cfg, 32)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=160)
    got = dec.forward(prompt)
    ref = O.gpt2_forward(cfg, w, prompt)
    assert np.max(np.abs(got - ref)) <= 1e-4, np.max(np.abs(got - ref))


def test_gpt2_int4_decode_matches_oracle_on_dequantised_weights(ctx, gpt2_full):
    """int4 weight-only decode (inferc_gpt2_use_int4) against the oracle GPT-2
    run on the same weights dequantised by the numpy statement of the
    quantiser: greedy tokens bit-exact, last logits and the prefill forward
    within 1e-4."""
    cfg, w = gpt2_full
    wq = graphs.gpt2_int4_dequantized(cfg, w)
    prompt = graphs.gpt2_prompt(cfg, 16)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=64)
    dec.use_int4()
    dec.use_int4()  # a second call changes nothing
    toks, steps, logits = dec.generate(prompt, 24, want_step_ms=True, want_logits=True)
    ref_toks, ref_logits, margins = O.gpt2_generate(cfg, wq, prompt, 24)
    print(f"int4: min top-2 margin {margins.min():.3e}; max |dlogit| "
          f"{np.max(np.abs(logits - ref_logits)):.3e}; ms/token {steps.mean():.4f}")
    np.testing.assert_array_equal(toks, ref_toks)
    assert np.max(np.abs(logits - ref_logits)) <= 1e-4
    got = dec.forward(prompt)
    assert np.max(np.abs(got - O.gpt2_forward(cfg, wq, prompt))) <= 1e-4
    toks2, _, _ = dec.generate(prompt, 24)
    np.testing.assert_array_equal(toks2, toks)
    p = Profiler()
    np.testing.assert_array_equal(dec.generate_profiled(prompt, 8, p), toks[:8])
    rep = p.report("inferc-decode-int4")
    _check_device_profile(rep, 7)
    assert rep["op_counts"] == _decode_counts(cfg["layers"], embed=False)


def test_gpt2_int4_rejects_other_shapes(ctx):
    cfg = graphs.small_gpt2_cfg()
    dec = rt.Gpt2Decoder(ctx, cfg, graphs.gpt2_weights(cfg, 23), max_t=16)
    with pytest.raises(RuntimeError, match="hidden 768, ffn 3072"):
        dec.use_int4()


def test_gpt2_generate_profiled_config4(ctx, gpt2_full):
    """Profiled decode steps of GPT-2 small (fp32 GEMV path): tokens equal
    generate()'s, one iteration per step, the step's fused launch groups."""
    cfg, w = gpt2_full
    prompt = graphs.gpt2_prompt(cfg, 32)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=64)
    p = Profiler()
    toks_p = dec.generate_profiled(prompt, 10, p)
    toks, _, _ = dec.generate(prompt, 10)
    np.testing.assert_array_equal(toks_p, toks)
    rep = p.report("inferc-decode-hip", "gpt2")
    print({k: round(v["total_ms"]["mean_ms"], 4) for k, v in rep["per_op_type"].items()},
          "total", round(rep["total"]["mean_ms"], 4))
    _check_device_profile(rep, 9)
    assert rep["op_counts"] == _decode_counts(cfg["layers"], embed=False)


@pytest.mark.parametrize("int4", [False, True])
def test_gpt2_decode_fills_the_cache_exactly(ctx, gpt2_full, int4):
    """GPT-2 small (the step's fast kernels): prompt 32 and 9 tokens on a
    40-position cache, so the last step attends over every slot; tokens equal
    the oracle's (on the dequantised weights for int4), and one token more is
    refused before anything runs."""
    cfg, w = gpt2_full
    prompt = graphs.gpt2_prompt(cfg, 32)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=40)
    ref_w = w
    if int4:
        dec.use_int4()
        ref_w = graphs.gpt2_int4_dequantized(cfg, w)
    toks, _, logits = dec.generate(prompt, 9, want_logits=True)
    ref_toks, ref_logits, _ = O.gpt2_generate(cfg, ref_w, prompt, 9)
    np.testing.assert_array_equal(toks, ref_toks)
    assert np.max(np.abs(logits - ref_logits)) <= 1e-4
    with pytest.raises(RuntimeError, match="exceed the KV cache"):
        dec.generate(prompt, 10)
    np.testing.assert_array_equal(dec.generate(prompt, 9)[0], toks)


@pytest.mark.parametrize("n_prompt,n_tok", [(1, 6), (1, 1), (4, 1)])
def test_gpt2_decode_one_token_prompt_and_no_decode_step(ctx, gpt2_full, n_prompt, n_tok):
    """A one-token prompt (the prefill is a single row), and a generate of one
    token (the prefill's arg-max alone, no decode step replayed): tokens and
    the last logits against the oracle."""
    cfg, w = gpt2_full
    prompt = graphs.gpt2_prompt(cfg, n_prompt)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=16)
    toks, steps, logits = dec.generate(prompt, n_tok, want_step_ms=True, want_logits=True)
    ref_toks, ref_logits, _ = O.gpt2_generate(cfg, w, prompt, n_tok)
    np.testing.assert_array_equal(toks, ref_toks)
    assert np.max(np.abs(logits - ref_logits)) <= 1e-4
    assert steps.shape == (n_tok - 1,)


def test_gpt2_small_cfg_decode_fills_the_cache_exactly(ctx):
    """The general step kernels (a model off the GPT-2-small shape): prompt 5
    and 12 tokens on a 16-position cache."""
    cfg = graphs.small_gpt2_cfg()
    w = graphs.gpt2_weights(cfg, 25)
    prompt = graphs.gpt2_prompt(cfg, 5)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=16)
    toks, _, logits = dec.generate(prompt, 12, want_logits=True)
    ref_toks, ref_logits, _ = O.gpt2_generate(cfg, w, prompt, 12)
    np.testing.assert_array_equal(toks, ref_toks)
    np.testing.assert_allclose(logits, ref_logits, atol=1e-4)
    with pytest.raises(RuntimeError, match="exceed the KV cache"):
        dec.generate(prompt, 13)


def test_gpt2_greedy_decode_config4_bit_exact(ctx, gpt2_full):
    """prompt 32, 128 generated tokens, sequence bit-exact."""
    cfg, w = gpt2_full
    prompt = graphs.gpt2_prompt(cfg, 32)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=160)
    toks, steps, logits = dec.generate(prompt, 128, want_step_ms=True, want_logits=True)
    ref_toks, ref_logits, margins = O.gpt2_generate(cfg, w, prompt, 128)
    print(f"min top-2 margin {margins.min():.3e}; max |dlogit| "
          f"{np.max(np.abs(logits - ref_logits)):.3e}; ms/token {steps.mean():.4f}")
    np.testing.assert_array_equal(toks, ref_toks)
    assert np.max(np.abs(logits - ref_logits)) <= 1e-4
