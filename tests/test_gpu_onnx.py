"""Exported ONNX models end to end on the GPU: read by the protobuf-free
reader, optionally optimized by the pass pipeline, run by the executor, and
compared with the logits torch computed for the same models and inputs
(tests/golden/make_onnx_fixtures.py). The unoptimized graphs exercise the
generic ops (decomposed LayerNorm and GELU, unfused attention with
Transpose / batched MatMul / Softmax, the mask arithmetic); the optimized
ones the fused kernels. Tolerance 1e-4 on the logits."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from inferc_amd import rt

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def _run_model(ctx, name, optimize, sets):
    g = rt.Graph.from_onnx(GOLDEN / f"{name}.onnx")
    counts = g.optimize() if optimize else None
    ex = rt.Executor(ctx, g)
    io = np.load(GOLDEN / f"{name}_io.npz")
    for tag in sets:
        feeds = {"input_ids": io[f"ids_{tag}"], "attention_mask": io[f"mask_{tag}"]}
        ref = io[f"logits_{tag}"]
        outs = [ex.run(feeds, ["logits"])["logits"] for _ in range(3)]  # eager, capture, replay
        err = float(np.max(np.abs(outs[0] - ref)))
        print(f"{name} optimize={optimize} set={tag}: max|dlogit| {err:.3e}")
        assert outs[0].shape == ref.shape
        assert err <= 1e-4
        for o in outs[1:]:
            np.testing.assert_array_equal(o, outs[0])
    return counts, ex


@pytest.mark.parametrize("optimize", [False, True])
def test_exported_distilbert(ctx, optimize):
    counts, ex = _run_model(ctx, "distilbert_tiny", optimize, ["a", "b"])
    if optimize:
        assert counts["recognize_attention_additive"] == 2


@pytest.mark.parametrize("optimize", [False, True])
def test_exported_gpt2(ctx, optimize):
    _run_model(ctx, "gpt2_tiny", optimize, ["a", "b"])


def _past_feeds(io):
    feeds = {"input_ids": io["step_ids"], "attention_mask": np.ones((1, 8), np.int64)}
    for k in range(4):
        feeds[f"past_key_values.{k // 2}.{'key' if k % 2 == 0 else 'value'}"] = io[f"past_{k}"]
    return feeds


@pytest.mark.parametrize("optimize,bound", [(False, False), (True, False), (True, True)])
def test_exported_gpt2_with_past_step(ctx, optimize, bound):
    """One decode step of the with-past graph over torch's 7-token cache:
    logits and present.* against torch (1e-4). Bound to a KV cache (which
    holds the FusedAttentionPast nodes the passes make) the past data seeds
    the cache and present.* are read back through the cache."""
    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    g = rt.Graph.from_onnx(GOLDEN / "gpt2_tiny_past.onnx")
    if optimize:
        assert g.optimize()["recognize_attention_additive"] == 2
    ex = rt.Executor(ctx, g)
    if bound:
        ex.bind_kv_cache(32)
    outs = ["logits"] + [f"present.{k // 2}.{'key' if k % 2 == 0 else 'value'}" for k in range(4)]
    got = ex.run(_past_feeds(io), outs)
    err = float(np.max(np.abs(got["logits"] - io["step_logits"])))
    print(f"with-past step optimize={optimize} bound={bound}: max|dlogit| {err:.3e}")
    assert err <= 1e-4
    for k in range(4):
        ref = io[f"present_{k}"]
        assert got[outs[1 + k]].shape == ref.shape
        np.testing.assert_allclose(got[outs[1 + k]], ref, atol=1e-4)


def test_decode_feedback_matches_host_steps(ctx):
    """Decode mode with the token fed back on the device (steps replayed back
    to back, tokens read once at the end) against the same decode mode one
    step at a time through the host (a profiler forces that path) and
    against walking every step with grown shapes: the same tokens, and the
    same last logits bit for bit; run_steps reports one device time per
    step; decode_tokens refuses positions past the cache."""
    from inferc_amd.profiler import Profiler

    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    dec = rt.OnnxDecoder(ctx, GOLDEN / "gpt2_tiny_past.onnx", max_t=32)
    ms: list = []
    fed = dec.generate(io["prompt"], 12, step_ms=ms)
    fed_logits = dec.logits()
    host = dec.generate(io["prompt"], 12, profiler=Profiler())
    host_logits = dec.logits()
    walked = dec.generate(io["prompt"], 12, decode_mode=False)
    np.testing.assert_array_equal(fed, io["gen_tokens"])
    np.testing.assert_array_equal(host, fed)
    np.testing.assert_array_equal(walked, fed)
    np.testing.assert_array_equal(fed_logits, host_logits)
    assert len(ms) == 11 and all(m > 0 for m in ms)
    with pytest.raises(RuntimeError, match="past the KV cache"):
        dec.ex.decode_tokens(30, 4)
    dec.close()


def test_decode_mode_token_out_of_range(ctx):
    """In decode mode the token and position embedding rows are one kernel:
    a token id out of the vocabulary still fails the step as Gather does on
    the host (embedding.cc:63), in the planning pass and in a replay, and the
    steps after it run clean."""
    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    dec = rt.OnnxDecoder(ctx, GOLDEN / "gpt2_tiny_past.onnx", max_t=32)
    prompt = np.asarray(io["prompt"], np.int64).reshape(1, -1)
    n = prompt.shape[1]
    tok = dec._step(prompt, n)
    dec._enter_decode(n)
    for bad in (True, False, False, True, False):  # planning pass, recording, replays
        if bad:
            with pytest.raises(RuntimeError, match="index out of range"):
                dec._decode_step(2 ** 40)
        else:
            tok = dec._decode_step(tok)
            assert 0 <= tok < dec.logits().shape[-1]
    dec.ex.set_decode_position(-1)
    dec.close()


def test_onnx_decoder_greedy_tokens_match_torch(ctx):
    """`inferc decode` over the exported with-past graph with the device KV
    cache: the 12 greedy tokens equal torch's generation with its own cache
    (bit-exact), the last step's logits within 1e-4."""
    io = np.load(GOLDEN / "gpt2_tiny_past_io.npz")
    dec = rt.OnnxDecoder(ctx, GOLDEN / "gpt2_tiny_past.onnx", max_t=32)
    toks = dec.generate(io["prompt"], 12)
    np.testing.assert_array_equal(toks, io["gen_tokens"])
    err = float(np.max(np.abs(dec.logits()[0, -1] - io["gen_last_logits"])))
    print(f"onnx decode: tokens {toks.tolist()}; last max|dlogit| {err:.3e}")
    assert err <= 1e-4
    # a second generation restarts at past length 0 and repeats itself
    np.testing.assert_array_equal(dec.generate(io["prompt"], 12), toks)
    with pytest.raises(RuntimeError, match="exceed the KV cache"):
        dec.generate(io["prompt"], 40)
    # a shape-only past longer than what the cache holds is refused
    ex = dec.ex
    ex.set_input("input_ids", np.array([[1]], np.int64))
    ex.set_input("attention_mask", np.ones((1, 30), np.int64))
    for i in dec.past:
        ex.set_input_shape(i["name"], np.float32, [1, 4, 29, 16])
    with pytest.raises(RuntimeError, match="KV cache holds"):
        ex.run_async()


def test_gpt2_small_with_past_graph_decode_config4(ctx):
    """`inferc decode` over the exported with-past graph at GPT-2-small shape
    (prompt 32, 128 greedy tokens): the structure-only
    export with the config's seeded weights bound (graphs.gpt2_bind_weights),
    the pass pipeline, the device KV cache. Tokens bit-exact against the CPU
    oracle on the same weights (main.cpp:700-936; argmax rule :875-879)."""
    import oracle as O
    from inferc_amd import graphs

    cfg = graphs.GPT2_SMALL
    w = graphs.gpt2_weights(cfg, 2)
    g = rt.Graph.from_onnx(GOLDEN / "gpt2_small_past_noparams.onnx")
    graphs.gpt2_bind_weights(g, cfg, w)
    prompt = graphs.gpt2_prompt(cfg, 32)
    dec = rt.OnnxDecoder(ctx, g, max_t=160)
    assert dec.counts["recognize_attention_additive"] == 12
    ms: list = []
    toks = dec.generate(prompt, 128, step_ms=ms)
    ref, _, margins = O.gpt2_generate(cfg, w, prompt, 128)
    print(f"with-past graph: {np.mean(ms):.3f} ms/token; min top-2 margin {margins.min():.3e}")
    np.testing.assert_array_equal(toks, ref)
    assert len(ms) == 127
    dec.close()


def test_gpt2_small_with_past_graph_fills_the_cache_exactly(ctx):
    """The with-past graph at GPT-2-small shape in decode mode (the native
    attention kernel on the graph's cache) with prompt 32 and 9 tokens on a
    40-position cache: the last step attends over every slot. Tokens equal
    the oracle's; one token more is refused, and the decoder still generates
    the same tokens after the refusal."""
    import oracle as O
    from inferc_amd import graphs

    cfg = graphs.GPT2_SMALL
    w = graphs.gpt2_weights(cfg, 2)
    g = rt.Graph.from_onnx(GOLDEN / "gpt2_small_past_noparams.onnx")
    graphs.gpt2_bind_weights(g, cfg, w)
    prompt = graphs.gpt2_prompt(cfg, 32)
    dec = rt.OnnxDecoder(ctx, g, max_t=40)
    toks = dec.generate(prompt, 9)
    ref, _, _ = O.gpt2_generate(cfg, w, prompt, 9)
    np.testing.assert_array_equal(toks, ref)
    with pytest.raises(RuntimeError, match="exceed the KV cache"):
        dec.generate(prompt, 10)
    np.testing.assert_array_equal(dec.generate(prompt, 9), toks)
    dec.close()


@pytest.mark.parametrize("n_prompt,n_tok", [(1, 6), (1, 1)])
def test_gpt2_small_with_past_graph_one_token_prompt(ctx, n_prompt, n_tok):
    """The with-past graph at GPT-2-small shape with a one-token prompt (an
    empty past on the first step), and a generate of one token (the prompt
    step alone): tokens against the oracle."""
    import oracle as O
    from inferc_amd import graphs

    cfg = graphs.GPT2_SMALL
    w = graphs.gpt2_weights(cfg, 2)
    g = rt.Graph.from_onnx(GOLDEN / "gpt2_small_past_noparams.onnx")
    graphs.gpt2_bind_weights(g, cfg, w)
    prompt = graphs.gpt2_prompt(cfg, n_prompt)
    dec = rt.OnnxDecoder(ctx, g, max_t=16)
    toks = dec.generate(prompt, n_tok)
    ref, _, _ = O.gpt2_generate(cfg, w, prompt, n_tok)
    np.testing.assert_array_equal(toks, ref)
    dec.close()


def test_gpt2_small_graph_on_the_native_decoder_int4(ctx):
    """`inferc decode --int4`'s route at GPT-2-small shape: the exported
    with-past graph with config 4's weights bound, read back by parameter
    name into the native decoder (Gpt2Decoder.from_graph), switched to int4
    weight-only projections; tokens bit-exact against the CPU oracle on the
    dequantised weights."""
    import oracle as O
    from inferc_amd import graphs

    cfg = graphs.GPT2_SMALL
    w = graphs.gpt2_weights(cfg, 2)
    g = rt.Graph.from_onnx(GOLDEN / "gpt2_small_past_noparams.onnx")
    graphs.gpt2_bind_weights(g, cfg, w)
    prompt = graphs.gpt2_prompt(cfg, 16)
    dec = rt.Gpt2Decoder.from_graph(ctx, g, max_t=48)
    dec.use_int4()
    toks, _, _ = dec.generate(prompt, 16)
    ref, _, _ = O.gpt2_generate(cfg, graphs.gpt2_int4_dequantized(cfg, w), prompt, 16)
    np.testing.assert_array_equal(toks, ref)
    dec.close()


@pytest.mark.gpu
@pytest.mark.parametrize("P,S,fill", [(0, 40, -3.4028234663852886e38), (29, 1, -3.4028234663852886e38),
                                      (300, 3, float("-inf")), (150, 2, -1e4)])
def test_attention_past_head_dim_64_vs_float64(ctx, P, S, fill):
    """FusedAttentionPast at head_dim 64 (the cache attention's 8-wave form):
    keys past 256 (several chunks per wave), a per-row mask, a row whose
    first 64 keys are all masked (with fill = -inf those chunks score -inf
    throughout and must leave the running softmax alone), against float64
    (attention.cc:59-98 with the cached keys first)."""
    B, nH, dh = 2, 2, 64
    H, T = nH * dh, P + S
    rng = np.random.default_rng(P + S)
    q, k, v = (rng.standard_normal((B, S, H)).astype(np.float32) for _ in range(3))
    pk, pv = (rng.standard_normal((B, nH, P, dh)).astype(np.float32) for _ in range(2))
    mask = rng.random((B, 1, S, T)) < 0.3
    mask[:, :, :, -1] = False                      # every row keeps a key
    mask[0, 0, 0, :min(64, T - 1)] = True          # whole leading chunks masked
    g = rt.Graph()
    for name, shape in (("q", q.shape), ("k", k.shape), ("v", v.shape)):
        g.add_input(name, np.float32, shape)
    if P:
        g.add_input("pk", np.float32, pk.shape)
        g.add_input("pv", np.float32, pv.shape)
    g.add_input("mask", np.bool_, mask.shape)
    g.add_node("FusedAttentionPast", ["q", "k", "v", "pk" if P else "", "pv" if P else "", "mask"],
               ["ctx", "present_k", "present_v"], head_dim=dh, fill=fill)
    g.add_output("ctx")
    ex = rt.Executor(ctx, g)
    feeds = {"q": q, "k": k, "v": v, "mask": mask}
    if P:
        feeds.update(pk=pk, pv=pv)
    got = ex.run(feeds, ["ctx"])["ctx"]
    ex.close()
    heads = lambda x: x.reshape(B, S, nH, dh).transpose(0, 2, 1, 3).astype(np.float64)
    K = np.concatenate([pk.astype(np.float64), heads(k)], axis=2)
    V = np.concatenate([pv.astype(np.float64), heads(v)], axis=2)
    s = heads(q) @ K.transpose(0, 1, 3, 2) / np.sqrt(dh)
    s = np.where(mask, fill, s)
    s = s - s.max(axis=-1, keepdims=True)
    e = np.exp(s)
    ref = (e / e.sum(axis=-1, keepdims=True)) @ V
    ref = ref.transpose(0, 2, 1, 3).reshape(B, S, H)
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-5)
