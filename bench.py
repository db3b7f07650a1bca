#!/usr/bin/env python3
"""Benchmark of inferc's runtime hot path on one MI355X (gfx950).

Primary metric: "encoder fwd ms (b1,s128) + GPT-2 decode
ms/token; % MFMA/HBM roofline". `value` is the DistilBERT-shape encoder
forward latency at batch 1, seq 128 (config 1), one step = one forward of the
fused graph through the executor, inputs already resident in HBM, its launches
enqueued on the stream per forward, timed with HIP events on the context
stream. The encoder's steps follow the roofline kernel's measurement, whose
untimed replays bring the GPU to its sustained clocks; every other timed
region is preceded by untimed work of its own for the same reason. The same JSON line
carries the GPT-2 greedy-decode ms/token (config 4), the other configs
(encoder b=32, FFN+LN, QKV+MHA, int4 GEMV) under "extra", the roofline of the
dominant kernel of the primary workload, and the CPU oracle timed on this
host's cores as the CPU baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "encoder fwd ms (b1,s128) + GPT-2 decode ms/token; % MFMA/HBM roofline"
PEAK_FP32_TFLOPS = 157.3
PEAK_HBM_GBPS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# GPU time of untimed work before a timed region that follows host-side set-up:
# after an idle gap MI355X needs ~30 ms of sustained work to return to its
# sustained clocks (the FFN+LN graph at M=4096 runs 0.40 ms on its first
# forwards and 0.35 ms from ~30 ms on; the roofline GEMM 12.4 us, then 11.45).
WARM_MS = 60.0


def warm_up(ctx, fn, warm_ms: float) -> None:
    """Untimed calls of fn (each enqueues GPU work) until the GPU has spent
    warm_ms in them."""
    spent = 0.0
    while spent < warm_ms:
        ctx.timer_start()
        fn()
        spent += ctx.timer_stop()


def time_executor(ctx, ex, steps: int, warmup: int, warm_ms: float = 0.0) -> float:
    """ms per executor run: `warmup` untimed runs (at least 2: the first run of
    an input signature plans it), then untimed runs for warm_ms of GPU time,
    then `steps` timed runs with HIP events on the context stream."""
    for _ in range(max(warmup, 2)):
        ex.run_async()
    ctx.sync()
    if warm_ms > 0:
        warm_up(ctx, ex.run_async, warm_ms)
    ctx.timer_start()
    for _ in range(steps):
        ex.run_async()
    return ctx.timer_stop() / steps


def time_replays(ctx, cap, launches_per_replay: int, total_launches: int) -> float:
    """ms per launch of a captured sequence, replayed back to back so the
    GPU, not host submission, sets the pace."""
    return time_replay_windows(ctx, cap, launches_per_replay, total_launches, 1)[1]


def time_replay_windows(ctx, cap, launches_per_replay: int, total_launches: int,
                        windows: int) -> tuple[float, float]:
    """(min, mean) ms per launch over `windows` equal timing windows of
    back-to-back replays, after untimed replays for WARM_MS of GPU time; the
    sequence is closed afterwards."""
    cap.replay()
    ctx.sync()
    warm_up(ctx, cap.replay, WARM_MS)
    replays = max(2, total_launches // (launches_per_replay * windows))
    per = []
    for _ in range(windows):
        ctx.timer_start()
        for _ in range(replays):
            cap.replay()
        per.append(ctx.timer_stop() / (replays * launches_per_replay))
    cap.close()
    return min(per), sum(per) / len(per)


def encoder_flops(cfg: dict, B: int, S: int) -> float:
    H, F, L = cfg["hidden"], cfg["ffn"], cfg["layers"]
    M = B * S
    per_layer = 2 * M * H * 3 * H + 2 * M * H * H + 4 * M * H * F + 4 * B * S * S * H
    return float(L * per_layer)


def device_inputs(ctx, ex, arrays: dict):
    from inferc_amd import rt

    keep = []
    for name, arr in arrays.items():
        t = rt.Tensor.from_numpy(ctx, arr)
        ex.set_input_device(name, t)
        keep.append(t)
    return keep


def prepare_encoder(ctx, B: int, weights=None):
    """The encoder's executor at batch B, seq 128, with its inputs resident in
    HBM, dispatching eagerly: every run enqueues its launches on the stream.
    Replaying a captured HIP graph of the same launches measured 2-12% slower
    on the GPU for every executor workload here (encoder b=1 0.301 against
    0.295 ms, with 0.13 ms of host time per eager run)."""
    from inferc_amd import graphs, rt

    cfg = graphs.DISTILBERT
    w = weights if weights is not None else graphs.encoder_weights(cfg, 1)
    ex = rt.Executor(ctx, graphs.encoder_graph(cfg, w))
    ex.set_graph_mode(False)
    ids, mask = graphs.encoder_inputs(cfg, B, 128)
    keep = device_inputs(ctx, ex, {"input_ids": ids, "attention_mask": mask})
    return ex, keep, w


def bench_encoder(ctx, B: int, steps: int, warmup: int, weights=None, warm_ms: float = 0.0,
                  prepared=None):
    ex, keep, w = prepared if prepared is not None else prepare_encoder(ctx, B, weights)
    ms = time_executor(ctx, ex, steps, warmup, warm_ms)
    out = ex.output("logits")
    del keep
    ex.close()
    return ms, out, w


def ffn_ln_graph(M: int, seed: int = 3):
    """Config 2: LN_{1e-12}(GELU(X W1 + b1) W2 + b2), X [M,768]."""
    from inferc_amd import graphs, rt

    g = rt.Graph()
    n = graphs.normal
    g.add_initializer("w1", n(seed, "w1", (768, 3072)))
    g.add_initializer("b1", n(seed, "b1", (3072,)))
    g.add_initializer("w2", n(seed, "w2", (3072, 768)))
    g.add_initializer("b2", n(seed, "b2", (768,)))
    g.add_initializer("g", np.ones(768, np.float32))
    g.add_initializer("b", np.zeros(768, np.float32))
    g.add_node("FusedMatMulAddGELU", ["x", "w1", "b1"], ["f"])
    g.add_node("MatMul", ["f", "w2"], ["y_mm"])
    g.add_node("Add", ["y_mm", "b2"], ["y"])
    g.add_node("FusedLayerNorm", ["y", "g", "b"], ["out"], epsilon=1e-12)
    g.add_output("out")
    x = graphs.normal(seed, f"x{M}", (M, 768), std=1.0)
    return g, x


def qkv_mha_graph(S: int, seed: int = 4):
    """Config 3: FusedQKV + FusedAttention, B=32, valid length U[16,S]."""
    from inferc_amd import graphs, rt

    B = 32
    g = rt.Graph()
    for i, nm in enumerate(("wq", "wk", "wv")):
        g.add_initializer(nm, graphs.normal(seed, nm, (768, 768)))
        g.add_initializer("b" + nm[1], graphs.normal(seed, "b" + nm[1], (768,)))
    g.add_node("FusedQKV", ["x", "wq", "bq", "wk", "bk", "wv", "bv"], ["q", "k", "v"])
    g.add_node("FusedAttention", ["q", "k", "v", "mask"], ["ctx"], head_dim=64,
               fill=graphs.FILL_MIN)
    g.add_output("ctx")
    x = graphs.normal(seed, f"x{S}", (B, S, 768), std=1.0)
    lens = graphs.rng_for(seed, f"lens{S}").integers(16, S + 1, size=B)
    mask = (np.arange(S)[None, :] >= lens[:, None]).reshape(B, 1, 1, S)
    return g, x, mask.astype(np.bool_), lens


def bench_graph(ctx, g, inputs: dict, steps: int, warmup: int) -> float:
    """A config graph through the executor, dispatched eagerly as the encoder
    is, timed after WARM_MS of untimed runs."""
    from inferc_amd import rt

    ex = rt.Executor(ctx, g)
    ex.set_graph_mode(False)
    keep = device_inputs(ctx, ex, inputs)
    ms = time_executor(ctx, ex, steps, warmup, WARM_MS)
    del keep
    ex.close()
    return ms


def bench_decode(ctx, max_tokens: int = 128, prompt_len: int = 32, int4: bool = False,
                 warm: bool = True):
    """Config 4 (int4=False), or the same model switched to int4 weight-only
    decode (inferc_gpt2_use_int4). warm=False times the first generate (the
    --decode-only mode for kernel traces: under the tracer, a run that
    replayed one step graph over two generates died in the tracer)."""
    from inferc_amd import graphs, rt

    cfg = graphs.GPT2_SMALL
    w = graphs.gpt2_weights(cfg, 2)
    dec = rt.Gpt2Decoder(ctx, cfg, w, max_t=prompt_len + max_tokens)
    if int4:
        dec.use_int4()
    prompt = graphs.gpt2_prompt(cfg, prompt_len)
    # An untimed generate of the same length (the step graph is captured in
    # it, and the GPU returns to its sustained clocks after the weight upload),
    # then one generate whose every post-prefill step is timed
    # (main.cpp:863-872).
    if warm:
        dec.generate(prompt, max_tokens)
    toks, steps, _ = dec.generate(prompt, max_tokens, want_step_ms=True)
    dec.close()
    return float(np.mean(steps)), float(np.median(steps)), float(np.min(steps)), toks, w, prompt


GPT2_SMALL_PAST_ONNX = ROOT / "tests" / "golden" / "gpt2_small_past_noparams.onnx"


def bench_onnx_decode(ctx, weights, prompt, max_tokens: int = 128):
    """`inferc decode` over the exported with-past graph of GPT-2-small (the
    reference's own caller, main.cpp:700-936): the structure-only export with
    the config-4 weights bound, the pass pipeline, the device KV cache. The
    post-prompt steps run in the executor's decode mode (past length on the
    device, one recorded step replayed, each greedy token fed back on the
    device); an untimed generate of the same length records the step first.
    ms/token is each post-prompt step's time as main.cpp:863-872 times Run,
    device time between HIP events."""
    from inferc_amd import graphs, rt

    g = rt.Graph.from_onnx(str(GPT2_SMALL_PAST_ONNX))
    graphs.gpt2_bind_weights(g, graphs.GPT2_SMALL, weights)
    dec = rt.OnnxDecoder(ctx, g, max_t=len(prompt) + max_tokens)
    ms: list = []
    # untimed: plans and allocates the executor's buffers, records the step,
    # and returns the GPU to its sustained clocks
    dec.generate(prompt, max_tokens)
    toks = dec.generate(prompt, max_tokens, step_ms=ms)
    nodes = dec.ex.node_count()
    counts = dec.counts
    dec.close()
    return {"ms_per_token": round(float(np.mean(ms)), 4), "p50": round(float(np.median(ms)), 4),
            "min": round(float(np.min(ms)), 4), "timed_steps": len(ms),
            "nodes_after_fusion": nodes, "fusions": counts}, toks


def gpt2_bytes_per_token(cfg: dict, mean_ctx: float, int4: bool = False) -> float:
    H, F, V, L = cfg["hidden"], cfg["ffn"], cfg["vocab"], cfg["layers"]
    weights = L * (3 * H * H + H * H + 2 * H * F) + V * H
    rows = L * (3 * H + H + F + H) + V  # one int4 scale per weight row
    small = L * (3 * H + H + F + H + 4 * H) + 2 * H + H * 2  # biases, LN, wpe row
    kv = L * 2 * H * mean_ctx
    if int4:
        return weights / 2.0 + 4.0 * (rows + small + kv + H)  # + the embedding row
    return 4.0 * (weights + small + kv)


def bench_int4(ctx, batch: int, copies: int = 5, reps: int = 240):
    """Config 5: all 49 GPT-2-small matrices in one grouped launch; `copies`
    weight sets (>= 316 MB, beyond the 256 MB Infinity Cache) are rotated so
    every launch streams its weights from HBM. `ms` is the minimum over 6
    timing windows, as the reference reports its int4 GEMV (min of 6,
    bench/amx/int4_gemv_amx.cc:558-566); `ms_mean` is the mean over all of
    them."""
    from inferc_amd import graphs, rt

    shapes = graphs.int4_matrices()
    sets = []
    for c in range(copies):
        mats = []
        for i, (N, K) in enumerate(shapes):
            W, s = graphs.int4_weights(N, K, 100 + c, f"b{i}")
            x = graphs.normal(200 + c, f"x{i}_{batch}", (batch, K), std=1.0)
            mats.append((rt.Tensor.from_numpy(ctx, W), rt.Tensor.from_numpy(ctx, s),
                         rt.Tensor.from_numpy(ctx, x), rt.Tensor.empty(ctx, (batch, N)), K))
        sets.append(mats)
    for mats in sets:
        rt.int4_gemv_grouped(ctx, mats, batch)  # uploads + caches each table
    per_graph = 4 * copies
    cap = ctx.capture(lambda: [rt.int4_gemv_grouped(ctx, sets[r % copies], batch)
                               for r in range(per_graph)])
    ms, ms_mean = time_replay_windows(ctx, cap, per_graph, reps, 6)
    n_w = sum(N * K for N, K in shapes)
    n_rows = sum(N for N, _ in shapes)
    int4_bytes = n_w // 2
    compulsory = int4_bytes + 4 * n_rows + 4 * batch * sum(K for _, K in shapes) + \
        4 * batch * n_rows
    return {"ms": ms, "ms_mean": ms_mean, "int4_bytes": int4_bytes, "compulsory_bytes": compulsory,
            "gbps_compulsory": compulsory / (ms * 1e-3) / 1e9,
            "gbps_int4_only": int4_bytes / (ms * 1e-3) / 1e9,
            "hbm_frac": compulsory / (ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
            "copies_rotated": copies}


# The kernel with the most time per encoder forward at b=1: the FFN-down
# GEMM with its residual (6 launches per forward), on the small-M template
# gemm_f32_ksplit<16,48,16,2> with K split over two blocks per tile,
# Y = X[128,3072] W[3072,768] + b + residual.
ROOF_M, ROOF_N, ROOF_K = 128, 768, 3072
ROOF_KERNEL = "gemm_f32_ksplit<16,48,16,2>, K split over 2 blocks per tile"


def _roofline_operands(ctx):
    from inferc_amd import graphs, rt

    M, N, K = ROOF_M, ROOF_N, ROOF_K
    x = rt.Tensor.from_numpy(ctx, graphs.normal(9, "rx", (M, K), 1.0))
    w = rt.Tensor.from_numpy(ctx, graphs.normal(9, "rw", (K, N)))
    b = rt.Tensor.from_numpy(ctx, graphs.normal(9, "rb", (N,)))
    r = rt.Tensor.from_numpy(ctx, graphs.normal(9, "rr", (M, N), 1.0))
    y = rt.Tensor.empty(ctx, (M, N))
    lib = ctx._lib

    def launch():
        from inferc_amd import lib as L

        L.check(lib.inferc_hip_gemm_f32(ctx.handle, 0, 0, M, N, K, C.c_float(1.0), x.ptr, K,
                                        w.ptr, N, C.c_float(1.0), b.ptr, L.C_ROW, 0, r.ptr, N,
                                        L.ACT_NONE, y.ptr, N))

    return launch, (x, w, b, r, y)


def roofline_kernel(ctx, reps: int = 400):
    """Roofline of the dominant kernel of the primary workload: the residual
    GEMM template at the encoder's FFN-down shape (M=128, N=768, K=3072,
    bias row + residual epilogue), launched through the C-ABI, timed with
    HIP events on the context stream over back-to-back replays of a captured
    sequence of 20 launches (the stream the kernel runs on), after WARM_MS of
    untimed replays."""
    M, N, K = ROOF_M, ROOF_N, ROOF_K
    launch, keep = _roofline_operands(ctx)
    launch()
    per_graph = 20
    cap = ctx.capture(lambda: [launch() for _ in range(per_graph)])
    ms = time_replays(ctx, cap, per_graph, reps)
    del keep
    flops = 2.0 * M * N * K
    achieved = flops / (ms * 1e-3) / 1e12
    traffic = None
    tf = ROOT / "profiles" / "traffic.json"
    if tf.exists():
        traffic = json.loads(tf.read_text()).get("gemm_residual_ffn_down_b1")
    return {"bound": "mfma", "achieved": round(achieved, 3), "peak": PEAK_FP32_TFLOPS,
            "unit": "TFLOP/s", "frac": round(achieved / PEAK_FP32_TFLOPS, 4),
            "traffic": traffic,
            "kernel": f"{ROOF_KERNEL} (residual GEMM at the encoder's FFN-down shape)",
            "shape": [M, N, K], "algorithmic_flops_per_launch": flops,
            "algorithmic_bytes_per_launch": 4 * (M * K + K * N + N + 2 * M * N),
            "avg_launch_us": round(ms * 1e3, 3)}


def _chain_us(ctx, launches) -> float:
    """Per-launch time of a captured chain of dependent launches (stream
    order), from back-to-back replays timed with HIP events."""
    for f in launches:
        f()
    ctx.sync()
    cap = ctx.capture(lambda: [f() for f in launches])
    for _ in range(3):
        cap.replay()
    ms = time_replays(ctx, cap, len(launches), 20 * len(launches))
    cap.close()
    return round(ms * 1e3, 3)


def launch_floors(ctx) -> dict:
    """What one dependent launch of the batch-1 decode step costs, by kind.

    Each figure is the per-launch time of a captured chain of the same launch
    (a graph replay, as the decode step runs):
      - floor: a 4-row GEMV (one block), the cost of a dependent launch;
      - the decode step's GEMV shapes through inferc_hip_gemv_f32 (plain: no
        LayerNorm prologue, bias or residual), warm (one matrix, cache
        resident) and cold (distinct matrices, together past the 256 MB
        Infinity Cache, so every launch streams from HBM);
      - decode attention (12 heads of 64, 12 layers' caches) at several key
        counts t, through inferc_hip_kv_append_attend_f32.
    `step_model_ms` sums one layer's cold launches (attention at the run's
    mean t) over 12 layers plus the LM head and one floor launch for the
    step's tail, to set beside the measured ms/token."""
    lib = ctx._lib
    rng = np.random.default_rng(7)
    out = {}
    x = rt_tensor(ctx, rng.standard_normal(3072, dtype=np.float32))
    y = ctx.malloc(4 * 50304)

    def gemv(N, K, w):
        return lambda: check_rc(lib, lib.inferc_hip_gemv_f32(
            ctx.handle, N, K, w, x.ptr, None, None, 0.0, None, None, 0, y))

    src = rt_tensor(ctx, (rng.standard_normal((3072, 3072), dtype=np.float32) * 0.02))
    out["floor_us"] = _chain_us(ctx, [gemv(4, 768, src.ptr)] * 60)
    shapes = {"qkv": (2304, 768), "out_proj": (768, 768), "ffn_up": (3072, 768),
              "ffn_down": (768, 3072), "lm_head": (50257, 768)}
    for name, (N, K) in shapes.items():
        nbytes = 4 * N * K
        n_cold = max(4, -(-600_000_000 // nbytes))
        mats = []
        for _ in range(n_cold):
            p = ctx.malloc(nbytes)
            for off in range(0, nbytes, src.nbytes):
                check_rc(lib, lib.inferc_hip_d2d(ctx.handle, p + off, src.ptr,
                                                 min(src.nbytes, nbytes - off)))
            mats.append(p)
        warm = _chain_us(ctx, [gemv(N, K, mats[0])] * min(n_cold, 60))
        cold = _chain_us(ctx, [gemv(N, K, p) for p in mats])
        for p in mats:
            ctx.free(p)
        out[name] = {"warm_us": warm, "cold_us": cold, "mb": round(nbytes / 1e6, 2),
                     "cold_hbm_gbps": round(nbytes / (cold * 1e-6) / 1e9, 1)}
    nH, D, T = 12, 64, 160
    caches = [(rt_tensor(ctx, rng.standard_normal((nH, T, D), dtype=np.float32)),
               rt_tensor(ctx, rng.standard_normal((nH, T, D), dtype=np.float32)))
              for _ in range(12)]
    qkv = rt_tensor(ctx, rng.standard_normal(3 * nH * D, dtype=np.float32))
    att = ctx.malloc(4 * nH * D)
    out["attention_us"] = {}
    for t in (1, 33, 96, 160):
        pos = rt_tensor(ctx, np.array([t - 1], np.int64))

        def attn(kc, vc, pos=pos):
            return lambda: check_rc(lib, lib.inferc_hip_kv_append_attend_f32(
                ctx.handle, nH, D, T, pos.ptr, qkv.ptr, qkv.ptr + 4 * nH * D,
                qkv.ptr + 8 * nH * D, kc.ptr, vc.ptr, att))
        out["attention_us"][str(t)] = _chain_us(ctx, [attn(kc, vc) for kc, vc in caches] * 5)
    ctx.free(att)
    ctx.free(y)
    a = out["attention_us"]
    attn_mean = (a["33"] + a["160"]) / 2.0  # the bench run's keys go 33 .. 160
    layer = sum(out[k]["cold_us"] for k in ("qkv", "out_proj", "ffn_up", "ffn_down")) + attn_mean
    out["step_model_ms"] = round((12 * layer + out["lm_head"]["cold_us"] + out["floor_us"]) / 1e3, 4)
    out["step_launches"] = 62
    out["launch_floor_ms"] = round(62 * out["floor_us"] / 1e3, 4)
    return out


def rt_tensor(ctx, arr):
    from inferc_amd import rt
    return rt.Tensor.from_numpy(ctx, arr)


def check_rc(lib, rc: int) -> None:
    if rc != 0:
        raise RuntimeError(f"inferc_hip call failed ({rc}): "
                           f"{lib.inferc_hip_last_error().decode(errors='replace')}")


COUNTER_PARTS = ("encoder", "roofline", "int4", "decode")


def counters_workload(ctx, parts=COUNTER_PARTS) -> dict:
    """For rocprofv3 --pmc runs: eager dispatches of the kernels the counter
    summaries cover, then one 64 MiB device copy whose FETCH_SIZE /
    WRITE_SIZE calibrate the counters (the copy moves 64 MiB each way).
    - encoder: 3 forwards at b=1 and 1 at b=32 (graph mode off);
    - roofline: 10 launches of the roofline kernel;
    - int4: 3 launches of the 49-matrix int4 GEMV at B=1 and at B=8 on each
      of 5 weight copies (316 MB per rotation, so weights stream from HBM);
    - decode: 8-token greedy decodes, fp32 and int4 (steps replayed from the
      step graph)."""
    from inferc_amd import graphs, rt
    from inferc_amd.lib import check

    if "encoder" in parts:
        cfg = graphs.DISTILBERT
        w = graphs.encoder_weights(cfg, 1)
        for B, n in ((1, 3), (32, 1)):
            ex = rt.Executor(ctx, graphs.encoder_graph(cfg, w))
            ex.set_graph_mode(False)
            ids, mask = graphs.encoder_inputs(cfg, B, 128)
            keep = device_inputs(ctx, ex, {"input_ids": ids, "attention_mask": mask})
            for _ in range(n):
                ex.run_async()
            ctx.sync()
            del keep
            ex.close()
    if "roofline" in parts:
        launch, keep = _roofline_operands(ctx)
        for _ in range(10):
            launch()
        ctx.sync()
        del keep
    shapes = graphs.int4_matrices()
    for B in ((1, 8) if "int4" in parts else ()):
        sets = []
        for c in range(5):
            mats = []
            for i, (N, K) in enumerate(shapes):
                W, s = graphs.int4_weights(N, K, 100 + c, f"b{i}")
                mats.append((rt.Tensor.from_numpy(ctx, W), rt.Tensor.from_numpy(ctx, s),
                             rt.Tensor.from_numpy(ctx, graphs.normal(200 + c, f"x{i}_{B}",
                                                                     (B, K), std=1.0)),
                             rt.Tensor.empty(ctx, (B, N)), K))
            sets.append(mats)
        for _ in range(3):
            for mats in sets:
                rt.int4_gemv_grouped(ctx, mats, B)
        ctx.sync()
        del sets
    if "decode" in parts:
        gcfg = graphs.GPT2_SMALL
        dec = rt.Gpt2Decoder(ctx, gcfg, graphs.gpt2_weights(gcfg, 2), max_t=64)
        prompt = graphs.gpt2_prompt(gcfg, 32)
        dec.generate(prompt, 8)
        dec.use_int4()
        dec.generate(prompt, 8)
        dec.close()
    nbytes = 64 << 20
    src, dst = rt.Tensor.empty(ctx, (nbytes // 4,)), rt.Tensor.empty(ctx, (nbytes // 4,))
    ctx.sync()
    check(ctx._lib.inferc_hip_d2d(ctx.handle, dst.ptr, src.ptr, nbytes))
    ctx.sync()
    return {"copy_bytes": nbytes, "parts": list(parts),
            "roofline_shape": [ROOF_M, ROOF_N, ROOF_K]}


def cpu_info() -> dict:
    """CPU model name, physical cores (distinct (package, core) pairs in
    /proc/cpuinfo), logical CPUs and the CPUs this process may run on."""
    model, cores = "unknown", set()
    try:
        for block in Path("/proc/cpuinfo").read_text().split("\n\n"):
            kv = {}
            for line in block.splitlines():
                if ":" in line:
                    k, v = line.split(":", 1)
                    kv[k.strip()] = v.strip()
            if "model name" in kv:
                model = kv["model name"]
            if "core id" in kv:
                cores.add((kv.get("physical id", "0"), kv["core id"]))
    except OSError:
        pass
    return {"model": model, "physical_cores": len(cores) or None,
            "logical_cpus": os.cpu_count(), "usable_cpus": len(os.sched_getaffinity(0))}


def _time_cpu(fn, budget_s: float, max_n: int = 1000,
              min_n: int = 1, warm: bool = True) -> tuple[float, float, int]:
    """(min, mean) seconds of fn over as many calls as fit in budget_s (at
    least min_n, at most max_n, after one untimed call unless warm is
    False)."""
    if warm:
        fn()
    ts = []
    t_end = time.perf_counter() + budget_s
    while len(ts) < min_n or (time.perf_counter() < t_end and len(ts) < max_n):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return min(ts), sum(ts) / len(ts), len(ts)


def cpu_decode_ms_per_token(cfg, w, prompt, steps: int) -> float:
    """Mean ms of the oracle GPT-2's greedy decode steps after `prompt`, each
    step timed by the oracle itself around its forward and LM head
    (main.cpp:863-872); the prefill is not timed."""
    import oracle as O

    return float(np.mean(O.gpt2_decode_step_ms(cfg, w, prompt, 1 + steps)))


def cpu_baseline(enc_w, gpt2_w, full: bool) -> dict:
    """The C oracle (this repo's restatement of inferc's CPU kernels) timed on
    the host's cores, all cores (OpenMP default) and 1 thread, on bounded
    samples of every config: encoder b1 (the `value` workload) and b32,
    FFN+LN M=128/1024/4096, QKV+MHA S=128/512, GPT-2 decode steps at cache
    lengths 32-47 and 144-159 (config 4 spans 32-159), and the 49-matrix
    int4 GEMV at B=1 and B=8 with GB/s as streamed int4 bytes / best time
    (bench/amx/int4_gemv_amx.cc:556-567). The 1-thread encoder b32 row is
    one cold forward (about 9 s of work)."""
    import oracle as O
    from inferc_amd import graphs

    info = cpu_info()
    all_t = O.num_threads()
    cfg = graphs.DISTILBERT
    ids1, mask1 = graphs.encoder_inputs(cfg, 1, 128)
    res = {"threads_all": all_t, "cpu": info, "configs": {}}
    c = res["configs"]

    def timed(name, fn, budget_all, budget_1, warm_1=True):
        row = {}
        for th, budget in ((all_t, budget_all), (1, budget_1)):
            if budget is None:
                continue
            O.set_num_threads(th)
            try:
                best, mean, n = _time_cpu(fn, budget, warm=th == all_t or warm_1)
            finally:
                O.set_num_threads(all_t)
            key = "all" if th == all_t else "1t"
            row[key] = {"ms": round(mean * 1e3, 3), "ms_min": round(best * 1e3, 3), "n": n}
        c[name] = row
        return row

    log("  cpu: encoder b1 s128")
    timed("encoder_b1_s128", lambda: O.encoder_forward(cfg, enc_w, ids1, mask1), 6.0, 2.0)
    if full:
        ids32, mask32 = graphs.encoder_inputs(cfg, 32, 128)
        log("  cpu: encoder b32 s128")
        timed("encoder_b32_s128", lambda: O.encoder_forward(cfg, enc_w, ids32, mask32), 2.0,
              0.0, warm_1=False)
        ones, zeros = np.ones(768, np.float32), np.zeros(768, np.float32)
        for M in (128, 1024, 4096):
            g, x = ffn_ln_graph(M)
            w1, b1, w2, b2 = (g.initializer(n) for n in ("w1", "b1", "w2", "b2"))

            def ffn(x=x, w1=w1, b1=b1, w2=w2, b2=b2):
                f = O.fused_matmul_add_gelu(x, w1, b1)
                return O.layernorm(O.add_bcast(O.matmul(f, w2), b2), ones, zeros, 1e-12)

            log(f"  cpu: ffn+ln M={M}")
            timed(f"ffn_ln_m{M}", ffn, 2.0, 1.0)
        for S in (128, 512):
            g, xq, mask, _ = qkv_mha_graph(S)
            qw = [g.initializer(n) for n in ("wq", "bq", "wk", "bk", "wv", "bv")]
            x2 = xq.reshape(-1, 768)

            def qkv_mha(x2=x2, qw=qw, mask=mask, S=S):
                q, k, v = O.fused_qkv(x2, *qw)
                return O.fused_attention(q.reshape(32, S, 768), k.reshape(32, S, 768),
                                         v.reshape(32, S, 768), mask, 64, graphs.FILL_MIN)

            log(f"  cpu: qkv+mha S={S}")
            timed(f"qkv_mha_b32_s{S}", qkv_mha, 2.0, 1.0, warm_1=False)
        gcfg = graphs.GPT2_SMALL
        dec = {}
        for lo, steps_all, steps_1 in ((32, 15, 6), (144, 15, 6)):
            prompt = graphs.gpt2_prompt(gcfg, lo, seed=11)
            log(f"  cpu: gpt2 decode, cache {lo}..{lo + steps_all}")
            row = {}
            for th, steps in ((all_t, steps_all), (1, steps_1)):
                O.set_num_threads(th)
                try:
                    ms = cpu_decode_ms_per_token(gcfg, gpt2_w, prompt, steps)
                finally:
                    O.set_num_threads(all_t)
                row["all" if th == all_t else "1t"] = {"ms_per_token": round(ms, 3),
                                                       "steps": steps}
            dec[f"cache_{lo}_{lo + steps_all}"] = row
        c["gpt2_decode"] = dec
        shapes = graphs.int4_matrices()
        mats = [graphs.int4_weights(N, K, 100, f"b{i}") for i, (N, K) in enumerate(shapes)]
        int4_bytes = sum(N * K for N, K in shapes) // 2
        for B in (1, 8):
            xs = [graphs.normal(200, f"x{i}_{B}", (B, K), std=1.0)
                  for i, (_, K) in enumerate(shapes)]

            def sweep():
                for (W, sc), xb, (_, K) in zip(mats, xs, shapes):
                    O.int4_gemv_f32acc(W, sc, xb, K)

            log(f"  cpu: int4 GEMV sweep B={B}")
            row = {}
            for th in (all_t, 1):
                reps = 6 if th == all_t else 2  # best of 6, as int4_gemv_amx.cc:558-566
                O.set_num_threads(th)
                try:
                    best, mean, n = _time_cpu(sweep, 0.0, reps, reps)
                finally:
                    O.set_num_threads(all_t)
                row["all" if th == all_t else "1t"] = {
                    "ms_min": round(best * 1e3, 3), "n": n,
                    "gbps_int4": round(int4_bytes / best / 1e9, 2)}
            c[f"int4_gemv_b{B}"] = row
    return res


def cpu_profile_encoder(weights, B: int = 1, S: int = 128, iters: int = 3):
    """The CPU baseline's per-op profile in the same JSON schema: the oracle's
    encoder forward replayed op by op through the oracle's per-op functions
    under the native profiler's host clock, one op record per op of the
    executor's fused graph (embedding Gathers, the embedding Add folded into
    its LayerNorm, per layer FusedQKV, FusedAttention, the MatMul + bias +
    residual epilogue GEMMs, LayerNorms and FusedMatMulAddGELU, then the two
    classifier Gemms). The last pass's logits are checked against the
    oracle's own encoder forward."""
    import oracle as O
    from inferc_amd import graphs
    from inferc_amd.profiler import Profiler

    cfg = graphs.DISTILBERT
    H, L, nh = cfg["hidden"], cfg["layers"], cfg["heads"]
    eps = cfg["eps"]
    w = [np.ascontiguousarray(t, np.float32) for t in weights]
    ids, amask = graphs.encoder_inputs(cfg, B, S)
    p = Profiler()
    p.set_track_activation_bytes(False)

    def op(kind, name, fn, *a):
        p.begin_op(kind, name)
        r = fn(*a)
        p.end_op(0)
        return r

    def gemm_res(x, wt, b, res):
        return O.add_bcast(O.add_bcast(O.sgemm(x, wt), b), res)

    for _ in range(iters):
        p.begin_iteration()
        tok = op("Gather", "word_embeddings", O.gather_rows, w[0], ids.reshape(-1))
        pos = op("Gather", "position_embeddings", O.gather_rows, w[1], np.arange(S))
        h = op("FusedLayerNorm", "embeddings.LayerNorm",
               lambda: O.layernorm(O.add_bcast(tok.reshape(B, S, H), pos), w[2], w[3], eps))
        mask = (amask == 0).reshape(B, 1, 1, S)
        for l in range(L):
            lw = w[4 + 16 * l: 4 + 16 * (l + 1)]
            x2 = h.reshape(B * S, H)
            q, k, v = op("FusedQKV", f"l{l}.qkv", O.fused_qkv, x2, *lw[0:6])
            c = op("FusedAttention", f"l{l}.attn", O.fused_attention, q.reshape(B, S, H),
                   k.reshape(B, S, H), v.reshape(B, S, H), mask, H // nh, -3.4028234663852886e38)
            t = op("FusedGemmEpilogue", f"l{l}.out_lin", gemm_res, c.reshape(B * S, H), lw[6],
                   lw[7], x2)
            h1 = op("FusedLayerNorm", f"l{l}.sa_layer_norm", O.layernorm, t, lw[8], lw[9], eps)
            f = op("FusedMatMulAddGELU", f"l{l}.ffn.lin1", O.fused_matmul_add_gelu, h1, lw[10],
                   lw[11])
            t = op("FusedGemmEpilogue", f"l{l}.ffn.lin2", gemm_res, f, lw[12], lw[13], h1)
            h = op("FusedLayerNorm", f"l{l}.output_layer_norm", O.layernorm, t, lw[14], lw[15],
                   eps).reshape(B, S, H)
        tw = w[4 + 16 * L:]
        cls = np.ascontiguousarray(h[:, 0, :])
        pre = op("Gemm", "pre_classifier", lambda: np.maximum(
            O.gemm(cls, tw[0], tw[1], trans_b=True), np.float32(0)))
        logits = op("Gemm", "classifier", O.gemm, pre, tw[2], tw[3], 1.0, 1.0, False, True)
        p.end_iteration()
    p.snapshot_peak_rss()
    ref = O.encoder_forward(cfg, weights, ids, amask)
    err = float(np.max(np.abs(logits - ref)))
    if err > 1e-5:
        raise RuntimeError(f"per-op CPU replay differs from the oracle encoder by {err}")
    return p.report(f"oracle-cpu-{O.num_threads()}t", "distilbert_encoder_b1_s128")


def write_profiles(ctx, out_dir: str, enc_w) -> None:
    """--profile-dir: per-op profiles in the reference's JSON schema of the
    encoder (b1 s128, executor, device times per node), its CPU baseline
    replay, and the GPT-2 decode steps; plus the `inferc compare` table of
    the two encoder profiles."""
    from inferc_amd import graphs, rt
    from inferc_amd.profiler import Profiler, compare_table

    d = Path(out_dir)
    d.mkdir(parents=True, exist_ok=True)
    cfg = graphs.DISTILBERT
    ex = rt.Executor(ctx, graphs.encoder_graph(cfg, enc_w))
    ids, mask = graphs.encoder_inputs(cfg, 1, 128)
    hip = ex.profile({"input_ids": ids, "attention_mask": mask}, iters=20, warmup=3,
                     backend="inferc-hip-gfx950", model="distilbert_encoder_b1_s128")
    ex.close()
    (d / "encoder_b1_s128.hip.json").write_text(json.dumps(hip, indent=2, sort_keys=True))
    log("  encoder profile written")
    cpu = cpu_profile_encoder(enc_w)
    (d / "encoder_b1_s128.cpu.json").write_text(json.dumps(cpu, indent=2, sort_keys=True))
    table = compare_table(hip, cpu)
    (d / "encoder_b1_s128.compare.txt").write_text(table)
    log(table)
    gcfg = graphs.GPT2_SMALL
    dec = rt.Gpt2Decoder(ctx, gcfg, graphs.gpt2_weights(gcfg, 2), max_t=160)
    for int4 in (False, True):
        if int4:
            dec.use_int4()
        p = Profiler()
        dec.generate_profiled(graphs.gpt2_prompt(gcfg, 32), 33, p)
        name = "gpt2_decode_int4" if int4 else "gpt2_decode"
        rep = p.report("inferc-decode-hip" + ("-int4" if int4 else ""), name)
        (d / f"{name}.hip.json").write_text(json.dumps(rep, indent=2, sort_keys=True))
        log(f"  {name} profile written")
    dec.close()


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true", help="primary workload and roofline only")
    ap.add_argument("--counters", nargs="*", choices=COUNTER_PARTS, default=None,
                    help="eager dispatches of the profiled kernels (all parts, or the "
                         "ones named) + a calibration copy (for rocprofv3 --pmc runs)")
    ap.add_argument("--roofline-only", action="store_true",
                    help="the roofline kernel's timed replays only, printed as JSON")
    ap.add_argument("--encoder-only", type=int, nargs="?", const=1, default=None,
                    metavar="B", help="the encoder forward at batch B only, as text")
    ap.add_argument("--decode-only", nargs="?", const="both", choices=["fp32", "int4", "both"],
                    help="GPT-2 decode only (fp32 weights, int4 weights or both), one "
                         "generate each, printed as text (for rocprofv3 --kernel-trace runs)")
    ap.add_argument("--int4-only", action="store_true",
                    help="the 49-matrix int4 GEMV at batch 1 and 8 only, printed as JSON")
    ap.add_argument("--floors", action="store_true",
                    help="per-launch cost of dependent launch chains (launch floor, decode "
                         "GEMV shapes warm and cold, decode attention by key count), as JSON")
    ap.add_argument("--profile-dir", default=None,
                    help="also write per-op profiles (reference JSON schema) to this folder")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); "
              "multi-GPU runs are out of scope", file=sys.stderr)
        return 2
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: launched with WORLD_SIZE > 1; one GPU only", file=sys.stderr)
        return 2

    from inferc_amd import graphs, rt

    ctx = rt.Context(0)
    if args.counters is not None:
        print(json.dumps(counters_workload(ctx, tuple(args.counters) or COUNTER_PARTS)),
              flush=True)
        ctx.close()
        return 0
    if args.floors:
        print(json.dumps(launch_floors(ctx)), flush=True)
        ctx.close()
        return 0
    if args.int4_only:
        print(json.dumps({f"int4_gemv_b{B}": bench_int4(ctx, B) for B in (1, 8)}), flush=True)
        ctx.close()
        return 0
    if args.roofline_only:
        print(json.dumps(roofline_kernel(ctx)), flush=True)
        ctx.close()
        return 0
    if args.encoder_only is not None:
        ms, _, _ = bench_encoder(ctx, args.encoder_only, args.steps, args.warmup,
                                 warm_ms=WARM_MS)
        print(f"encoder b{args.encoder_only} s128: {ms:.4f} ms/forward", flush=True)
        ctx.close()
        return 0
    if args.decode_only:
        for int4 in {"fp32": (False,), "int4": (True,), "both": (False, True)}[args.decode_only]:
            mean, p50, _, _, _, _ = bench_decode(ctx, int4=int4, warm=False)
            print(f"gpt2 decode {'int4' if int4 else 'fp32'}: {mean:.4f} ms/token "
                  f"(p50 {p50:.4f})", flush=True)
        ctx.close()
        return 0
    extra = {}
    # The encoder is set up first; the roofline kernel's replays (WARM_MS
    # untimed, then the timed ones) run next, and the encoder's W warmup and K
    # timed forwards follow them with no idle gap, at sustained clocks.
    enc1 = prepare_encoder(ctx, 1)
    log("roofline kernel")
    roof = roofline_kernel(ctx)
    log(f"  {roof['avg_launch_us']} us, {roof['achieved']} TFLOP/s")
    log("encoder b1 s128")
    ms_b1, _, enc_w = bench_encoder(ctx, 1, args.steps, args.warmup, prepared=enc1)
    fl_b1 = encoder_flops(graphs.DISTILBERT, 1, 128)
    extra["encoder_b1_s128"] = {"ms": round(ms_b1, 4), "gflop": round(fl_b1 / 1e9, 3),
                                "mfma_frac_fp32": round(fl_b1 / (ms_b1 * 1e-3) / 1e12 /
                                                        PEAK_FP32_TFLOPS, 4)}
    log(f"  {ms_b1:.4f} ms/forward")

    dec = None
    if not args.quick:
        log("encoder b32 s128")
        ms_b32, _, _ = bench_encoder(ctx, 32, max(20, args.steps // 5), 3, enc_w, WARM_MS)
        fl_b32 = encoder_flops(graphs.DISTILBERT, 32, 128)
        extra["encoder_b32_s128"] = {"ms": round(ms_b32, 4), "gflop": round(fl_b32 / 1e9, 2),
                                     "tflops": round(fl_b32 / (ms_b32 * 1e-3) / 1e12, 2),
                                     "mfma_frac_fp32": round(fl_b32 / (ms_b32 * 1e-3) / 1e12 /
                                                             PEAK_FP32_TFLOPS, 4)}
        log(f"  {ms_b32:.4f} ms/forward")
        for M in (128, 1024, 4096):
            g, x = ffn_ln_graph(M)
            ms = bench_graph(ctx, g, {"x": x}, max(10, args.steps // 2), 3)
            fl = 4.0 * M * 768 * 3072
            extra[f"ffn_ln_m{M}"] = {"ms": round(ms, 4), "tflops": round(fl / (ms * 1e-3) / 1e12, 2),
                                     "mfma_frac_fp32": round(fl / (ms * 1e-3) / 1e12 /
                                                             PEAK_FP32_TFLOPS, 4)}
            log(f"  ffn+ln M={M}: {ms:.4f} ms")
        for S in (128, 512):
            g, x, mask, _ = qkv_mha_graph(S)
            ms = bench_graph(ctx, g, {"x": x, "mask": mask}, max(10, args.steps // 2), 3)
            fl = 2.0 * 32 * S * 768 * 2304 + 4.0 * 32 * 12 * S * S * 64
            extra[f"qkv_mha_b32_s{S}"] = {"ms": round(ms, 4),
                                          "tflops_dense": round(fl / (ms * 1e-3) / 1e12, 2),
                                          "mfma_frac_fp32": round(fl / (ms * 1e-3) / 1e12 /
                                                                  PEAK_FP32_TFLOPS, 4)}
            log(f"  qkv+mha S={S}: {ms:.4f} ms")
        log("gpt2 decode")
        d_mean, d_p50, d_min, toks, gw, prompt = bench_decode(ctx)
        bpt = gpt2_bytes_per_token(graphs.GPT2_SMALL, 32 + 64)
        dec = {"ms_per_token": round(d_mean, 4), "p50": round(d_p50, 4),
               "min": round(d_min, 4), "tokens_per_s": round(1e3 / d_mean, 1),
               "prompt": 32, "generated": 128, "timed_steps": 127,
               "bytes_per_token": int(bpt),
               "hbm_gbps": round(bpt / (d_mean * 1e-3) / 1e9, 1),
               "hbm_frac": round(bpt / (d_mean * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"  {d_mean:.4f} ms/token")
        log("gpt2 decode over the exported with-past graph")
        od, otoks = bench_onnx_decode(ctx, gw, prompt)
        od["tokens_match_native"] = bool(np.array_equal(otoks, toks))
        extra["gpt2_decode_onnx_with_past"] = od
        log(f"  {od['ms_per_token']:.4f} ms/token, tokens match: {od['tokens_match_native']}")
        log("gpt2 decode, int4 weight-only")
        i_mean, i_p50, i_min, _, _, _ = bench_decode(ctx, int4=True)
        ibpt = gpt2_bytes_per_token(graphs.GPT2_SMALL, 32 + 64, int4=True)
        extra["gpt2_decode_int4"] = {
            "ms_per_token": round(i_mean, 4), "p50": round(i_p50, 4), "min": round(i_min, 4),
            "tokens_per_s": round(1e3 / i_mean, 1), "bytes_per_token": int(ibpt),
            "hbm_gbps": round(ibpt / (i_mean * 1e-3) / 1e9, 1),
            "hbm_frac": round(ibpt / (i_mean * 1e-3) / 1e9 / PEAK_HBM_GBPS, 4)}
        log(f"  {i_mean:.4f} ms/token")
        for B in (1, 8):
            log(f"int4 grouped GEMV B={B}")
            r = bench_int4(ctx, B)
            extra[f"int4_gemv_b{B}"] = {k: (round(v, 4) if isinstance(v, float) else v)
                                        for k, v in r.items()}
            log(f"  {r['ms'] * 1e3:.2f} us, {r['gbps_compulsory']:.0f} GB/s")

    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle)")
        gpt2_w = None if args.quick else gw
        cb = cpu_baseline(enc_w, gpt2_w, full=not args.quick)
        b1 = cb["configs"]["encoder_b1_s128"]
        thr = cb["threads_all"]
        cpu = {"value": b1["all"]["ms"], "unit": "ms", "cores": thr, "kind": "port",
               "sample": (f"{b1['all']['n']} encoder forwards at b1 s128 on {thr} OpenMP "
                          f"threads ({b1['1t']['n']} on 1 thread) of the C oracle; other "
                          "configs in `configs`, each on a bounded sample (see its n / "
                          "steps)"),
               "value_1_thread": b1["1t"]["ms"], "cpu": cb["cpu"], "configs": cb["configs"]}
        log(f"  {cpu['value']:.2f} ms/forward on {thr} threads, {cpu['value_1_thread']:.2f} on 1")

    if args.profile_dir:
        log(f"per-op profiles -> {args.profile_dir}")
        write_profiles(ctx, args.profile_dir, enc_w)

    line = {
        "metric": METRIC,
        "value": round(ms_b1, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_b1, 4),
        "higher_is_better": False,
        "scaling": "strong",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded random-init weights of the DistilBERT / GPT-2-small shapes)",
        "config": {"workload": "distilbert_encoder_fwd_b1_s128", "batch": 1, "seq_len": 128,
                   "layers": 6, "hidden": 768, "heads": 12, "ffn": 3072},
        "gpt2_decode": dec,
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
