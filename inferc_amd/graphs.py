"""Synthetic models for the hot path: seeded weights and the fused graphs the
reference's passes would hand to the executor.

No ONNX models, protobuf or network exist here, so the DistilBERT encoder is
emitted directly as the post-``inferc optimize`` graph (pass order of
src/cli/main.cpp:270-276; per-layer op sequence of SESSIONS.md:559 /
correctness_test.cc:131-144), including the integer shape plumbing a real
export carries (Shape -> Gather -> Range for the position ids, Equal ->
Unsqueeze for the attention mask). GPT-2 weights follow HF GPT-2's layout
([in, out] Conv1D weights, tied LM head).

Seeds: every tensor is drawn from ``numpy.random.default_rng`` seeded by
``(base_seed, crc32(tensor name))``, so any tensor can be regenerated alone
and the CPU oracle and the GPU always see identical bytes.
"""
from __future__ import annotations

import zlib

import numpy as np

DISTILBERT = dict(layers=6, hidden=768, heads=12, ffn=3072, vocab=30522, max_pos=512,
                  n_classes=2, eps=1e-12)
GPT2_SMALL = dict(layers=12, hidden=768, heads=12, ffn=3072, vocab=50257, max_pos=1024,
                  eps=1e-5)
FILL_MIN = float(np.finfo(np.float32).min)  # torch.finfo(float32).min of the exports


def rng_for(seed: int, name: str) -> np.random.Generator:
    return np.random.default_rng([seed, zlib.crc32(name.encode())])


def normal(seed: int, name: str, shape, std: float = 0.02) -> np.ndarray:
    g = rng_for(seed, name)
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(np.float32)


def encoder_weights(cfg: dict, seed: int = 1) -> list[np.ndarray]:
    """Weights in the order of orc_encoder_forward / the graph below."""
    H, F, V, P, C = cfg["hidden"], cfg["ffn"], cfg["vocab"], cfg["max_pos"], cfg["n_classes"]
    w = [normal(seed, "word_emb", (V, H)), normal(seed, "pos_emb", (P, H)),
         np.ones(H, np.float32), np.zeros(H, np.float32)]
    for l in range(cfg["layers"]):
        p = f"l{l}."
        w += [normal(seed, p + "wq", (H, H)), normal(seed, p + "bq", (H,)),
              normal(seed, p + "wk", (H, H)), normal(seed, p + "bk", (H,)),
              normal(seed, p + "wv", (H, H)), normal(seed, p + "bv", (H,)),
              normal(seed, p + "wo", (H, H)), normal(seed, p + "bo", (H,)),
              np.ones(H, np.float32), np.zeros(H, np.float32),
              normal(seed, p + "w1", (H, F)), normal(seed, p + "b1", (F,)),
              normal(seed, p + "w2", (F, H)), normal(seed, p + "b2", (H,)),
              np.ones(H, np.float32), np.zeros(H, np.float32)]
    w += [normal(seed, "pre_w", (H, H)), normal(seed, "pre_b", (H,)),
          normal(seed, "cls_w", (C, H)), normal(seed, "cls_b", (C,))]
    return w


def encoder_inputs(cfg: dict, B: int, S: int, seed: int = 7, ragged: bool = False):
    """token ids U[0, vocab) and an all-ones mask (or, if ragged, a valid
    prefix of U[1, S] per row)."""
    g = rng_for(seed, f"enc_inputs_{B}_{S}")
    ids = g.integers(0, cfg["vocab"], size=(B, S), dtype=np.int64)
    mask = np.ones((B, S), np.int64)
    if ragged:
        lens = g.integers(1, S + 1, size=B)
        for b in range(B):
            mask[b, lens[b]:] = 0
    return ids, mask


def encoder_graph(cfg: dict, weights: list[np.ndarray]):
    """The fused DistilBERT graph for :class:`inferc_amd.rt.Executor`."""
    from .rt import Graph

    g = Graph()
    H, L = cfg["hidden"], cfg["layers"]
    hd = H // cfg["heads"]
    names = ["word_emb", "pos_emb", "emb_ln_g", "emb_ln_b"]
    for l in range(L):
        p = f"l{l}."
        names += [p + n for n in ("wq", "bq", "wk", "bk", "wv", "bv", "wo", "bo", "ln1_g",
                                  "ln1_b", "w1", "b1", "w2", "b2", "ln2_g", "ln2_b")]
    names += ["pre_w", "pre_b", "cls_w", "cls_b"]
    for n, w in zip(names, weights):
        g.add_initializer(n, w)
    g.add_initializer("c_zero_i64", np.array(0, np.int64))
    g.add_initializer("c_one_i64", np.array(1, np.int64))
    g.add_initializer("c_one_vec", np.array([1], np.int64))
    g.add_initializer("c_cls_idx", np.array(0, np.int64))
    # embeddings: word + position, position ids from the input's shape
    g.add_node("Gather", ["word_emb", "input_ids"], ["we"], axis=0)
    g.add_node("Shape", ["input_ids"], ["ids_shape"])
    g.add_node("Gather", ["ids_shape", "c_one_i64"], ["seq_len"], axis=0)
    g.add_node("Range", ["c_zero_i64", "seq_len", "c_one_i64"], ["pos_range"])
    g.add_node("Unsqueeze", ["pos_range"], ["position_ids"], axes=[0])
    g.add_node("Gather", ["pos_emb", "position_ids"], ["pe"], axis=0)
    g.add_node("Add", ["we", "pe"], ["emb"])
    g.add_node("FusedLayerNorm", ["emb", "emb_ln_g", "emb_ln_b"], ["h0"], epsilon=cfg["eps"])
    # mask cond = (attention_mask == 0) as [B,1,1,S]
    g.add_node("Equal", ["attention_mask", "c_zero_i64"], ["mask_eq"])
    g.add_node("Unsqueeze", ["mask_eq"], ["mask_cond"], axes=[1, 2])
    h = "h0"
    for l in range(L):
        p = f"l{l}."
        g.add_node("FusedQKV", [h, p + "wq", p + "bq", p + "wk", p + "bk", p + "wv", p + "bv"],
                   [p + "q", p + "k", p + "v"])
        g.add_node("FusedAttention", [p + "q", p + "k", p + "v", "mask_cond"], [p + "ctx"],
                   head_dim=hd, fill=FILL_MIN)
        g.add_node("MatMul", [p + "ctx", p + "wo"], [p + "o_mm"])
        g.add_node("Add", [p + "o_mm", p + "bo"], [p + "o"])
        g.add_node("Add", [p + "o", h], [p + "sa_res"])
        g.add_node("FusedLayerNorm", [p + "sa_res", p + "ln1_g", p + "ln1_b"], [p + "h1"],
                   epsilon=cfg["eps"])
        g.add_node("FusedMatMulAddGELU", [p + "h1", p + "w1", p + "b1"], [p + "ff"])
        g.add_node("MatMul", [p + "ff", p + "w2"], [p + "ff2_mm"])
        g.add_node("Add", [p + "ff2_mm", p + "b2"], [p + "ff2"])
        g.add_node("Add", [p + "ff2", p + "h1"], [p + "ff_res"])
        g.add_node("FusedLayerNorm", [p + "ff_res", p + "ln2_g", p + "ln2_b"], [p + "h2"],
                   epsilon=cfg["eps"])
        h = p + "h2"
    g.add_node("Gather", [h, "c_cls_idx"], ["cls"], axis=1)
    g.add_node("Gemm", ["cls", "pre_w", "pre_b"], ["pre"], transB=1)
    g.add_node("Relu", ["pre"], ["pre_act"])
    g.add_node("Gemm", ["pre_act", "cls_w", "cls_b"], ["logits"], transB=1)
    g.add_output("logits")
    return g


def gpt2_weights(cfg: dict, seed: int = 2) -> list[np.ndarray]:
    """Weights in the order of include/inferc_hip.h (inferc_gpt2_create)."""
    H, F, V, P = cfg["hidden"], cfg["ffn"], cfg["vocab"], cfg["max_pos"]
    w = [normal(seed, "wte", (V, H)), normal(seed, "wpe", (P, H))]
    for l in range(cfg["layers"]):
        p = f"h{l}."
        w += [np.ones(H, np.float32), np.zeros(H, np.float32),
              normal(seed, p + "attn_w", (H, 3 * H)), normal(seed, p + "attn_b", (3 * H,)),
              normal(seed, p + "proj_w", (H, H)), normal(seed, p + "proj_b", (H,)),
              np.ones(H, np.float32), np.zeros(H, np.float32),
              normal(seed, p + "fc_w", (H, F)), normal(seed, p + "fc_b", (F,)),
              normal(seed, p + "fcproj_w", (F, H)), normal(seed, p + "fcproj_b", (H,))]
    w += [np.ones(H, np.float32), np.zeros(H, np.float32)]
    return w


def int4_quantize_rows_np(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Per-row symmetric int4 quantisation in numpy (fp32 arithmetic):
    s_r = max|w_r| / 7, q = clip(rint(w / s_r), -8, 7), 0 for an all-zero
    row. Returns (q as int8 [N, K], s [N]); the dequantised row is s_r * q."""
    w = np.ascontiguousarray(w, np.float32)
    s = (np.abs(w).max(axis=1) / np.float32(7)).astype(np.float32)
    safe = np.where(s > 0, s, np.float32(1))[:, None]
    q = np.where(s[:, None] > 0, np.rint(w / safe), np.float32(0))
    return np.clip(q, -8, 7).astype(np.int8), s


def gpt2_int4_dequantized(cfg: dict, w: list[np.ndarray]) -> list[np.ndarray]:
    """The weights of an int4 weight-only GPT-2 (inferc_gpt2_use_int4), as
    fp32 values: every projection quantised per output feature (a column of
    the [K, N] matrix) and the tied wte per vocabulary row; biases, LayerNorm
    and wpe unchanged."""
    out = [a.copy() for a in w]

    def deq_rows(m):  # rows of m are the quantised rows
        q, s = int4_quantize_rows_np(m)
        return (s[:, None] * q.astype(np.float32)).astype(np.float32)

    out[0] = deq_rows(w[0])
    for l in range(cfg["layers"]):
        base = 2 + 12 * l
        for off in (2, 4, 8, 10):
            out[base + off] = np.ascontiguousarray(deq_rows(w[base + off].T).T)
    return out


def gpt2_bind_weights(graph, cfg: dict, weights: list[np.ndarray]) -> None:
    """Binds `weights` (the order of gpt2_weights) to a GPT-2 graph exported
    without parameters: each parameter input (inner.transformer.wte.weight,
    .h.{l}.ln_1.weight, ..., .ln_f.bias) becomes an initializer of that name,
    and the one [hidden, vocab] input, the LM head's folded transpose of the
    tied wte, becomes wte^T (the initializer FoldConstantTranspose makes,
    constant_fold.cc:12-54). Fails on any parameter input it cannot place."""
    H, V, L = cfg["hidden"], cfg["vocab"], cfg["layers"]
    p = "inner.transformer."
    names = {p + "wte.weight": weights[0], p + "wpe.weight": weights[1],
             p + "ln_f.weight": weights[2 + 12 * L], p + "ln_f.bias": weights[3 + 12 * L]}
    parts = ["ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
             "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
             "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight", "mlp.c_proj.bias"]
    for l in range(L):
        for k, part in enumerate(parts):
            names[f"{p}h.{l}.{part}"] = weights[2 + 12 * l + k]
    bound = 0
    for i in graph.to_dict()["inputs"]:
        nm, shape = i["name"], list(i["shape"])
        if nm in names:
            arr = names[nm]
        elif shape == [H, V]:
            arr = np.ascontiguousarray(weights[0].T)
        else:
            if nm.startswith(p) or nm.startswith("onnx::"):
                raise ValueError(f"gpt2_bind_weights: no weight for input {nm} {shape}")
            continue
        if list(arr.shape) != shape:
            raise ValueError(f"gpt2_bind_weights: {nm} is {shape}, weight is {list(arr.shape)}")
        graph.add_initializer(nm, np.ascontiguousarray(arr, np.float32))
        bound += 1
    if bound != len(names) + 1:
        raise ValueError(f"gpt2_bind_weights: bound {bound} of {len(names) + 1} parameters")


def gpt2_weights_from_graph(graph) -> tuple[dict, list[np.ndarray]]:
    """The config and weights (the order of gpt2_weights) of an exported HF
    GPT-2 graph, read from its initializers by parameter name
    (<prefix>transformer.wte.weight, .h.{l}.ln_1.weight, ..., .ln_f.bias):
    what the native decoder (inferc_gpt2_create) needs to run the model the
    graph describes. Heads come from the past_key_values.* inputs of a
    with-past graph ([batch, heads, past, head_dim]); the LayerNorm epsilon
    from the graph's fused LayerNorms (1e-5, GPT-2's, if none is fused)."""
    d = graph.to_dict()
    names = {i["name"] for i in d["initializers"]}
    wte = [n for n in names if n.endswith("transformer.wte.weight")]
    if len(wte) != 1:
        raise ValueError("gpt2_weights_from_graph: no single transformer.wte.weight initializer")
    p = wte[0][:-len("wte.weight")]
    get = graph.initializer
    L = 0
    while f"{p}h.{L}.ln_1.weight" in names:
        L += 1
    if L == 0:
        raise ValueError("gpt2_weights_from_graph: no transformer.h.0 parameters")
    heads = [i["shape"][1] for i in d["inputs"] if i["name"].startswith("past_key_values.")
             and len(i["shape"]) == 4]
    if not heads or heads[0] <= 0:
        raise ValueError("gpt2_weights_from_graph: head count needs the with-past graph's "
                         "past_key_values.* inputs")
    eps = [float(n["attrs"]["epsilon"]) for n in d["nodes"]
           if n["op"] == "FusedLayerNorm" and "epsilon" in n.get("attrs", {})]
    w = [get(p + "wte.weight"), get(p + "wpe.weight")]
    parts = ["ln_1.weight", "ln_1.bias", "attn.c_attn.weight", "attn.c_attn.bias",
             "attn.c_proj.weight", "attn.c_proj.bias", "ln_2.weight", "ln_2.bias",
             "mlp.c_fc.weight", "mlp.c_fc.bias", "mlp.c_proj.weight", "mlp.c_proj.bias"]
    for l in range(L):
        w += [get(f"{p}h.{l}.{part}") for part in parts]
    w += [get(p + "ln_f.weight"), get(p + "ln_f.bias")]
    V, H = w[0].shape
    cfg = dict(layers=L, hidden=int(H), heads=int(heads[0]), ffn=int(w[10].shape[1]),
               vocab=int(V), max_pos=int(w[1].shape[0]), eps=eps[0] if eps else 1e-5)
    return cfg, [np.ascontiguousarray(a, np.float32) for a in w]


def gpt2_prompt(cfg: dict, n: int, seed: int = 3) -> np.ndarray:
    return rng_for(seed, f"prompt_{n}").integers(0, cfg["vocab"], size=n, dtype=np.int64)


def small_encoder_cfg() -> dict:
    """A reduced DistilBERT-shape config (head_dim 64) for fast tests."""
    return dict(layers=2, hidden=128, heads=2, ffn=256, vocab=1000, max_pos=64, n_classes=2,
                eps=1e-12)


def small_gpt2_cfg() -> dict:
    return dict(layers=2, hidden=128, heads=2, ffn=512, vocab=2000, max_pos=128, eps=1e-5)


def int4_matrices(layers: int = 12, hidden: int = 768, ffn: int = 3072, vocab: int = 50257):
    """(N, K) of the GPT-2-small weight volume: per layer QKV, out, FC, FC-proj
    as [out, in], plus the LM head."""
    mats = []
    for _ in range(layers):
        mats += [(3 * hidden, hidden), (hidden, hidden), (ffn, hidden), (hidden, ffn)]
    mats.append((vocab, hidden))
    return mats


def int4_weights(N: int, K: int, seed: int, tag: str):
    """Symmetric int4 q ~ U{-8..7} packed 2/byte (low nibble = even k) and
    scales ~ U(0.001, 0.05)."""
    g = rng_for(seed, f"int4_{tag}_{N}_{K}")
    W = g.integers(0, 256, size=(N, K // 2), dtype=np.uint8)
    s = g.uniform(0.001, 0.05, size=N).astype(np.float32)
    return W, s
