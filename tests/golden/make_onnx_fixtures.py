"""Writes the exported-model fixtures of the ONNX reader / pass / executor
tests:

  distilbert_tiny.onnx + distilbert_tiny_io.npz
      DistilBertForSequenceClassification (2 layers, dim 64, 4 heads, FFN 128,
      vocab 97), eager attention, exported by torch.onnx (TorchScript
      exporter, opset 13, dynamic batch/sequence) as transformers exports
      DistilBERT; the npz holds two input sets (one with padding) and the
      logits torch computes for them in float32.
  gpt2_tiny.onnx + gpt2_tiny_io.npz
      GPT2LMHeadModel (2 layers, dim 64, 4 heads, vocab 101), eager
      attention, no KV cache, inputs input_ids + attention_mask as the
      reference's GPT-2 decoder model takes them, dynamic batch/sequence; the
      npz holds token ids, masks and torch's float32 logits.
  gpt2_tiny_past.onnx + gpt2_tiny_past_io.npz
      The same GPT-2 as a with-past decoder: inputs input_ids, attention_mask
      and past_key_values.{i}.key/value [batch, heads, past, head_dim];
      outputs logits and present.{i}.key/value. The npz holds one step over a
      7-token prompt's cache (past tensors, step logits and presents) and
      torch's greedy generation of 12 tokens from that prompt with its KV
      cache (first-maximum argmax) and the last step's logits.
  gpt2_tiny_prefill.onnx
      The same GPT-2 as the reference's prefill decoder model: inputs
      input_ids and attention_mask, outputs logits and present.{i}.key/value
      (the first graph of `inferc decode --model`).
  gpt2_small_past_noparams.onnx
      GPT-2-small (12 layers, dim 768, 12 heads, vocab 50257, 1024 positions)
      as the same with-past decoder, exported with export_params=False: the
      graph's structure only, every parameter a named graph input
      (inner.transformer.*), plus the LM head's folded transpose of the tied
      wte as one [768, 50257] input. No weights are stored (450 KB); the
      bench binds seeded weights to these inputs (graphs.gpt2_bind_weights).

Every parameter is drawn at random (biases and LayerNorm weights included),
so the exporter's deduplication of equal initializers does not fire.
The exporter's only use of the `onnx` package (absent here) is inserting
custom-op functions, which these models do not have; that step is skipped.

Usage: python tests/golden/make_onnx_fixtures.py
"""
from __future__ import annotations

import io
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent


def _export(model, args, input_names, output_names, dynamic_axes,
            export_params: bool = True) -> bytes:
    from torch.onnx._internal.torchscript_exporter import onnx_proto_utils as opu

    opu._add_onnxscript_fn = lambda model_bytes, custom_opsets: model_bytes
    f = io.BytesIO()
    torch.onnx.export(model, args, f, input_names=input_names, output_names=output_names,
                      dynamic_axes=dynamic_axes, opset_version=13, dynamo=False,
                      do_constant_folding=True, export_params=export_params)
    return f.getvalue()


def _randomize(model, seed: int) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in model.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.2)
        for name, p in model.named_parameters():
            if "LayerNorm" in name or "layer_norm" in name or ".ln_" in name:
                if name.endswith("weight"):
                    p.add_(1.0)


def distilbert() -> None:
    from transformers import DistilBertConfig, DistilBertForSequenceClassification

    cfg = DistilBertConfig(vocab_size=97, dim=64, n_layers=2, n_heads=4, hidden_dim=128,
                           max_position_embeddings=64, num_labels=2)
    cfg._attn_implementation = "eager"
    m = DistilBertForSequenceClassification(cfg).eval()
    _randomize(m, 11)
    rng = np.random.default_rng(5)
    ids_a = rng.integers(0, 97, (2, 16)).astype(np.int64)
    mask_a = np.ones((2, 16), np.int64)
    mask_a[1, 11:] = 0  # a padded row
    ids_b = rng.integers(0, 97, (3, 9)).astype(np.int64)
    mask_b = np.ones((3, 9), np.int64)
    mask_b[0, 5:] = 0
    data = _export(m, (torch.from_numpy(ids_a), torch.from_numpy(mask_a)),
                   ["input_ids", "attention_mask"], ["logits"],
                   {"input_ids": {0: "batch", 1: "sequence"},
                    "attention_mask": {0: "batch", 1: "sequence"}, "logits": {0: "batch"}})
    (OUT / "distilbert_tiny.onnx").write_bytes(data)
    with torch.no_grad():
        la = m(torch.from_numpy(ids_a), attention_mask=torch.from_numpy(mask_a)).logits.numpy()
        lb = m(torch.from_numpy(ids_b), attention_mask=torch.from_numpy(mask_b)).logits.numpy()
    np.savez(OUT / "distilbert_tiny_io.npz", ids_a=ids_a, mask_a=mask_a, logits_a=la,
             ids_b=ids_b, mask_b=mask_b, logits_b=lb)


def gpt2() -> None:
    from transformers import GPT2Config, GPT2LMHeadModel

    cfg = GPT2Config(vocab_size=101, n_positions=64, n_embd=64, n_layer=2, n_head=4,
                     use_cache=False)
    cfg._attn_implementation = "eager"
    m = GPT2LMHeadModel(cfg).eval()
    _randomize(m, 12)
    rng = np.random.default_rng(6)
    ids = rng.integers(0, 101, (1, 12)).astype(np.int64)
    ids2 = rng.integers(0, 101, (2, 7)).astype(np.int64)

    class Logits(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, input_ids, attention_mask):
            return self.inner(input_ids=input_ids, attention_mask=attention_mask,
                              use_cache=False).logits

    w = Logits(m).eval()
    mask = np.ones_like(ids)
    mask2 = np.ones_like(ids2)
    data = _export(w, (torch.from_numpy(ids), torch.from_numpy(mask)),
                   ["input_ids", "attention_mask"], ["logits"],
                   {"input_ids": {0: "batch", 1: "sequence"},
                    "attention_mask": {0: "batch", 1: "sequence"},
                    "logits": {0: "batch", 1: "sequence"}})
    (OUT / "gpt2_tiny.onnx").write_bytes(data)
    with torch.no_grad():
        la = w(torch.from_numpy(ids), torch.from_numpy(mask)).numpy()
        lb = w(torch.from_numpy(ids2), torch.from_numpy(mask2)).numpy()
    np.savez(OUT / "gpt2_tiny_io.npz", ids_a=ids, mask_a=mask, logits_a=la, ids_b=ids2,
             mask_b=mask2, logits_b=lb)
    gpt2_past(m, cfg)


def _past_wrapper(m, L):
    from transformers.cache_utils import DynamicCache

    class Past(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, input_ids, attention_mask, *past):
            cache = DynamicCache()
            for i in range(L):
                cache.update(past[2 * i], past[2 * i + 1], i)
            out = self.inner(input_ids=input_ids, attention_mask=attention_mask,
                             past_key_values=cache, use_cache=True)
            pres = []
            for i in range(L):
                pres += [out.past_key_values.layers[i].keys, out.past_key_values.layers[i].values]
            return (out.logits, *pres)

    return Past(m).eval()


def _past_io(L):
    names_in = ["input_ids", "attention_mask"] + [
        f"past_key_values.{i}.{kv}" for i in range(L) for kv in ("key", "value")]
    names_out = ["logits"] + [f"present.{i}.{kv}" for i in range(L) for kv in ("key", "value")]
    dyn = {"input_ids": {0: "batch", 1: "sequence"},
           "attention_mask": {0: "batch", 1: "total_sequence"}, "logits": {0: "batch", 1: "sequence"}}
    for nm in names_in[2:]:
        dyn[nm] = {0: "batch", 2: "past_sequence"}
    for nm in names_out[1:]:
        dyn[nm] = {0: "batch", 2: "total_sequence"}
    return names_in, names_out, dyn


def gpt2_small_structure() -> None:
    """GPT-2-small with-past decoder, structure only (export_params=False)."""
    from transformers import GPT2Config, GPT2LMHeadModel

    cfg = GPT2Config(vocab_size=50257, n_positions=1024, n_embd=768, n_layer=12, n_head=12,
                     use_cache=True)
    cfg._attn_implementation = "eager"
    m = GPT2LMHeadModel(cfg).eval()
    _randomize(m, 13)  # distinct values: no parameter is merged with another
    L, nh, dh = cfg.n_layer, cfg.n_head, cfg.n_embd // cfg.n_head
    names_in, names_out, dyn = _past_io(L)
    ex = (torch.tensor([[5]], dtype=torch.int64), torch.ones(1, 4, dtype=torch.int64),
          *[torch.zeros(1, nh, 3, dh) for _ in range(2 * L)])
    data = _export(_past_wrapper(m, L), ex, names_in, names_out, dyn, export_params=False)
    (OUT / "gpt2_small_past_noparams.onnx").write_bytes(data)


def gpt2_past(m, cfg) -> None:
    L = cfg.n_layer
    w = _past_wrapper(m, L)
    nh, dh = cfg.n_head, cfg.n_embd // cfg.n_head
    names_in, names_out, dyn = _past_io(L)
    ex_ids = torch.tensor([[5]], dtype=torch.int64)
    ex_mask = torch.ones(1, 4, dtype=torch.int64)
    ex_past = [torch.zeros(1, nh, 3, dh) for _ in range(2 * L)]
    data = _export(w, (ex_ids, ex_mask, *ex_past), names_in, names_out, dyn)
    (OUT / "gpt2_tiny_past.onnx").write_bytes(data)

    class Prefill(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, input_ids, attention_mask):
            out = self.inner(input_ids=input_ids, attention_mask=attention_mask, use_cache=True)
            pres = []
            for i in range(L):
                pres += [out.past_key_values.layers[i].keys, out.past_key_values.layers[i].values]
            return (out.logits, *pres)

    dyn_p = {"input_ids": {0: "batch", 1: "sequence"}, "attention_mask": {0: "batch", 1: "sequence"},
             "logits": {0: "batch", 1: "sequence"}}
    for nm in names_out[1:]:
        dyn_p[nm] = {0: "batch", 2: "sequence"}
    data = _export(Prefill(m).eval(), (torch.tensor([[1, 2, 3]]), torch.ones(1, 3, dtype=torch.int64)),
                   ["input_ids", "attention_mask"], names_out, dyn_p)
    (OUT / "gpt2_tiny_prefill.onnx").write_bytes(data)

    rng = np.random.default_rng(7)
    prompt = rng.integers(0, cfg.vocab_size, (1, 7)).astype(np.int64)
    out = {}
    with torch.no_grad():
        # one step over the prompt's cache
        r = m(input_ids=torch.from_numpy(prompt), use_cache=True)
        past = []
        for i in range(L):
            past += [r.past_key_values.layers[i].keys.clone(),
                     r.past_key_values.layers[i].values.clone()]
        step = np.array([[int(rng.integers(0, cfg.vocab_size))]], np.int64)
        res = w(torch.from_numpy(step), torch.ones(1, 8, dtype=torch.int64), *past)
        out["step_ids"] = step
        for k in range(2 * L):
            out[f"past_{k}"] = past[k].numpy()
            out[f"present_{k}"] = res[1 + k].numpy()
        out["step_logits"] = res[0].numpy()
        # greedy generation with the KV cache
        toks = []
        r = m(input_ids=torch.from_numpy(prompt), use_cache=True)
        cache = r.past_key_values
        nxt = int(np.argmax(r.logits[0, -1].numpy()))
        toks.append(nxt)
        for _ in range(11):
            r = m(input_ids=torch.tensor([[nxt]]), past_key_values=cache, use_cache=True)
            cache = r.past_key_values
            nxt = int(np.argmax(r.logits[0, -1].numpy()))
            toks.append(nxt)
        out["gen_tokens"] = np.array(toks, np.int64)
        out["gen_last_logits"] = r.logits[0, -1].numpy()
    np.savez(OUT / "gpt2_tiny_past_io.npz", prompt=prompt, **out)


if __name__ == "__main__":
    torch.manual_seed(0)
    distilbert()
    gpt2()
    gpt2_small_structure()
    for p in sorted(OUT.glob("*_tiny*")):
        print(p.name, p.stat().st_size)
