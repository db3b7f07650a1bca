"""`inferc` commands over the gfx950 backend (src/cli/main.cpp): the callers
of the runtime hot path, with the reference's arguments and outputs.

  inspect <model.onnx>                      CmdInspect (main.cpp:119-158): the model summary
  run <model.onnx> --input-ids BIN --attention-mask BIN [--output BIN]
      [--shape B,S] [--profile JSON] [-n N] [--warmup N] [--name LABEL]
      [--no-optimize]                       DoRun / CmdRun (main.cpp:324-465)
  decode --model M --past-model M --prompt-ids BIN --max-tokens N
      --output BIN [--profile JSON] [--no-gemv] [--no-fold] [--no-optimize]
      [--device N] [--native | --int4]      CmdDecode (main.cpp:700-936)
  compare <a.json> <b.json>                 CmdCompare (main.cpp:595-611)

`run` reads int64 ids/mask files of shape B,S, loads the ONNX model with the
protobuf-free reader, applies the fusion pass pipeline (the reference runs
graphs `inferc optimize` already rewrote; --no-optimize runs the graph as
exported), executes it on the GPU and writes the first output's float32
bytes. `decode` runs the prefill graph over the prompt and the with-past
graph for each further token with the KV cache on the device, and writes the
int64 tokens. Profiles are the reference's JSON schema with device per-op
times.

decode flags: --no-gemv (main.cpp:718,727) turns the one-row GEMV route of
the graph executor off, --no-fold (main.cpp:719,756-775) leaves out the
passes the reference's flag skips (FoldConstantTranspose, RecognizeLayerNorm,
RecognizeGeluTanh); both are the reference's ablation baselines. Beyond the
reference: --device N picks the GPU, --native runs the model the with-past
graph describes (its weights read by parameter name) on the native decoder
(one captured step per token), and --int4 does the same with int4
weight-only projections (inferc_gpt2_use_int4).

Usage: python -m inferc_amd <command> ...
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np


def _err(msg: str) -> int:
    print(msg, file=sys.stderr)
    return 2


def cmd_inspect(args: list[str]) -> int:
    if len(args) != 1:
        return _err("usage: inferc inspect <model.onnx>")
    from . import rt

    try:
        print(rt.onnx_summary(Path(args[0]).read_bytes(), text=True), end="")
    except (OSError, RuntimeError) as e:
        print(f"inferc inspect: failed to parse '{args[0]}': {e}", file=sys.stderr)
        return 1
    return 0


def _opts(args: list[str], flags: set[str], valued: set[str]):
    """Flags, valued options and positionals; an unknown option is an error
    (main.cpp:447-450)."""
    o, pos, i = {}, [], 0
    while i < len(args):
        a = args[i]
        if a in flags:
            o[a] = True
        elif a in valued:
            if i + 1 >= len(args):
                raise ValueError(f"missing value for {a}")
            o[a] = args[i + 1]
            i += 1
        elif a.startswith("--"):
            raise ValueError(f"unknown arg '{a}'")
        else:
            pos.append(a)
        i += 1
    return o, pos


def cmd_run(args: list[str]) -> int:
    try:
        o, pos = _opts(args, {"--no-optimize"},
                       {"--input-ids", "--attention-mask", "--shape", "--output", "-n", "--warmup",
                        "--profile", "--name"})
    except ValueError as e:
        return _err(f"inferc: {e}")
    if len(pos) != 1:
        return _err("usage: inferc run <model.onnx> --input-ids <bin> --attention-mask <bin> "
                    "[--output <bin>] [--shape B,S] [--profile <out.json>] [-n <iters>] "
                    "[--warmup <n>]")
    if "--input-ids" not in o or "--attention-mask" not in o:
        return _err("inferc run: --input-ids and --attention-mask required")
    if "--output" not in o and "--profile" not in o:
        return _err("inferc run: must provide --output and/or --profile")
    try:
        B, S = (int(x) for x in o.get("--shape", "1,128").split(","))
    except ValueError:
        return _err("inferc run: --shape must be 'B,S' (e.g. 1,128)")
    from . import rt

    ids = np.fromfile(o["--input-ids"], np.int64)
    mask = np.fromfile(o["--attention-mask"], np.int64)
    if ids.size != B * S or mask.size != B * S:
        return _err(f"inferc run: ids/mask files must hold {B * S} int64 values")
    try:
        g = rt.Graph.from_onnx(pos[0])
    except RuntimeError as e:
        print(f"inferc run: failed to parse '{pos[0]}': {e}", file=sys.stderr)
        return 1
    counts = None if "--no-optimize" in o else g.optimize()
    if counts:
        print("inferc run: fused " + ", ".join(f"{k} {v}" for k, v in counts.items() if v))
    ctx = rt.Context(0)
    ex = rt.Executor(ctx, g)
    feeds = {"input_ids": ids.reshape(B, S), "attention_mask": mask.reshape(B, S)}
    out_name = g.to_dict()["outputs"][0]
    warmup, iters = max(int(o.get("--warmup", 0)), 0), max(int(o.get("-n", 1)), 1)
    try:
        for _ in range(warmup):
            ex.run(feeds, [])
        if "--profile" in o:
            backend = o.get("--name") or ("inferc-hip-optimized" if counts else "inferc-hip")
            rep = ex.profile(feeds, iters=iters, warmup=0, backend=backend, model=pos[0])
            Path(o["--profile"]).write_text(json.dumps(rep, indent=2, sort_keys=True))
            t = rep["total"]
            print(f"inferc run: profile -> {o['--profile']} (mean {t['mean_ms']:.3f} ms, "
                  f"p50 {t['p50_ms']:.3f} ms, {iters} iters)")
        else:
            t0 = time.perf_counter()
            for _ in range(iters):
                ex.run_async()
            ctx.sync()
            ms = (time.perf_counter() - t0) * 1e3 / max(iters, 1)
            print(f"inferc run: {iters} iters, {ms:.3f} ms/iter")
        logits = ex.output(out_name)
    except RuntimeError as e:
        print(f"inferc run: executor failed: {e}", file=sys.stderr)
        return 1
    print(f"inferc run: {out_name} {logits.dtype}{list(logits.shape)}"
          + (f" -> {o['--output']}" if "--output" in o else ""))
    if "--output" in o:
        logits.astype(np.float32).tofile(o["--output"])
    if logits.size <= 16:
        print("  values: " + " ".join(f"{v:g}" for v in logits.reshape(-1)))
    return 0


def cmd_decode(args: list[str]) -> int:
    try:
        o, pos = _opts(args, {"--no-optimize", "--no-gemv", "--no-fold", "--native", "--int4"},
                       {"--model", "--past-model", "--prompt-ids", "--max-tokens", "--output",
                        "--profile", "--max-t", "--device"})
    except ValueError as e:
        return _err(f"inferc decode: {e}")
    need = ("--model", "--past-model", "--prompt-ids", "--output")
    if pos or any(k not in o for k in need):
        return _err("usage: inferc decode --model <gpt2.onnx> --past-model <gpt2_with_past.onnx>\n"
                    "                     --prompt-ids <bin> --max-tokens N --output <bin>")
    try:
        max_tokens = int(o.get("--max-tokens", 32))
        device = int(o.get("--device", 0))
    except ValueError:
        return _err("inferc decode: --max-tokens and --device take integers")
    if max_tokens <= 0:
        return _err("inferc decode: missing required args")
    native = "--native" in o or "--int4" in o
    if native and ("--no-gemv" in o or "--no-fold" in o or "--no-optimize" in o):
        return _err("inferc decode: --no-gemv, --no-fold and --no-optimize apply to the graph "
                    "executor, not to --native/--int4")
    from . import rt
    from .profiler import Profiler

    prompt = np.fromfile(o["--prompt-ids"], np.int64)
    if prompt.size == 0:
        print("inferc decode: empty prompt", file=sys.stderr)
        return 1
    max_t = int(o.get("--max-t", prompt.size + max_tokens))
    try:
        ctx = rt.Context(device)
    except RuntimeError as e:
        print(f"inferc decode: device {device}: {e}", file=sys.stderr)
        return 1
    try:
        prof = Profiler() if "--profile" in o else None
        if prof is not None:
            prof.set_track_activation_bytes(False)
        if native:
            toks, el = _decode_native(ctx, o, prompt, max_tokens, max_t, prof)
        else:
            ctx.set_gemv_decode("--no-gemv" not in o)
            skip = rt.OnnxDecoder.FOLD_PASSES if "--no-fold" in o else ()
            dec = rt.OnnxDecoder(ctx, o["--past-model"], max_t=max_t, prefill=o["--model"],
                                 optimize="--no-optimize" not in o, skip_passes=skip)
            t0 = time.perf_counter()
            toks = dec.generate(prompt, max_tokens, profiler=prof)
            el = time.perf_counter() - t0
    except (RuntimeError, ValueError) as e:
        print(f"inferc decode: {e}", file=sys.stderr)
        return 1
    toks.astype(np.int64).tofile(o["--output"])
    print(f"inferc decode: generated {toks.size} tokens -> {o['--output']}")
    print("  tokens: " + " ".join(str(int(t)) for t in toks))
    print(f"  {el * 1e3 / max(toks.size, 1):.2f} ms/token (host wall clock, prompt included)")
    if prof is not None and toks.size > 1:
        rep = prof.report("inferc-decode-hip", o["--past-model"])
        Path(o["--profile"]).write_text(json.dumps(rep, indent=2, sort_keys=True))
        print(f"  decode profile -> {o['--profile']}")
    return 0


def _decode_native(ctx, o: dict, prompt: np.ndarray, max_tokens: int, max_t: int, prof):
    """--native / --int4: the GPT-2 the with-past graph holds, on the native
    decoder; returns (tokens, seconds)."""
    from . import rt

    dec = rt.Gpt2Decoder.from_graph(ctx, o["--past-model"], max_t)
    try:
        if "--int4" in o:
            dec.use_int4()
        t0 = time.perf_counter()
        if prof is not None:
            toks = dec.generate_profiled(prompt, max_tokens, prof)
        else:
            toks, _, _ = dec.generate(prompt, max_tokens)
        return toks, time.perf_counter() - t0
    finally:
        dec.close()


def cmd_compare(args: list[str]) -> int:
    if len(args) != 2:
        return _err("usage: inferc compare <a.json> <b.json>")
    from .profiler import compare_table

    try:
        a, b = (json.loads(Path(p).read_text()) for p in args)
    except (OSError, ValueError) as e:
        print(f"inferc compare: {e}", file=sys.stderr)
        return 1
    print(compare_table(a, b))
    return 0


COMMANDS = {"inspect": cmd_inspect, "run": cmd_run, "decode": cmd_decode, "compare": cmd_compare}


def main(argv: list[str] | None = None) -> int:
    argv = sys.argv[1:] if argv is None else argv
    if not argv or argv[0] in ("-h", "--help"):
        print(__doc__)
        return 0
    fn = COMMANDS.get(argv[0])
    if fn is None:
        print(f"inferc: unknown command '{argv[0]}'", file=sys.stderr)
        print(__doc__)
        return 1
    return fn(argv[1:])


if __name__ == "__main__":
    sys.exit(main())
