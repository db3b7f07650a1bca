"""Python binding of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Loads ``oracle/build/liboracle.so`` (built by ``make -C oracle``) and exposes
numpy wrappers of the C restatement in ``oracle.c`` / ``oracle_blas.c``. Only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package; the product library never does.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np


_DIR = Path(__file__).resolve().parent
# ORACLE_LIB selects another build of the same sources (the sanitized one)
_LIB = Path(os.environ.get("ORACLE_LIB", _DIR / "build" / "liboracle.so"))
_lib = None

F = C.POINTER(C.c_float)
I64 = C.POINTER(C.c_int64)
U8 = C.POINTER(C.c_uint8)
i64 = C.c_int64
f32 = C.c_float


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(_DIR)], check=True)
    return _LIB


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not _LIB.exists():
        build()
    lib = C.CDLL(str(_LIB))
    sig = {
        "orc_num_threads": ([], C.c_int),
        "orc_set_num_threads": ([C.c_int], None),
        "orc_parallel_blocks": ([i64, i64, i64, I64, I64], i64),
        "orc_sgemm": ([C.c_int, C.c_int, i64, i64, i64, f32, F, i64, F, i64, f32, F, i64], None),
        "orc_matmul": ([i64, i64, i64, i64, F, i64, F, i64, F], None),
        "orc_gemm": ([C.c_int, C.c_int, i64, i64, i64, f32, F, F, f32, F, C.c_int, F], None),
        "orc_fused_matmul_add_gelu": ([i64, i64, i64, F, F, F, F], None),
        "orc_fused_qkv": ([i64, i64, i64, F, F, F, F, F, F, F, F, F, F], None),
        "orc_fused_attention": ([i64, i64, i64, i64, F, F, F, U8, I64, f32, F], None),
        "orc_layernorm": ([i64, i64, F, F, F, f32, F], None),
        "orc_gelu": ([i64, F, F], None),
        "orc_gelu_tanh": ([i64, F, F], None),
        "orc_relu": ([i64, F, F], None),
        "orc_softmax": ([i64, i64, i64, F, F], None),
        "orc_add_bcast": ([i64, F, F, i64, F], None),
        "orc_gather_rows": ([i64, i64, F, I64, i64, F], C.c_int),
        "orc_split": ([i64, i64, i64, i64, I64, F, C.POINTER(F)], None),
        "orc_concat": ([i64, i64, i64, I64, C.POINTER(F), F], None),
        "orc_argmax": ([i64, F], i64),
        "orc_int4_gemv_per_row": ([U8, F, F, F, i64, i64], None),
        "orc_int4_gemv_per_row_batched": ([U8, F, F, F, i64, i64, i64], None),
        "orc_int4_gemv_per_tensor": ([U8, f32, F, F, i64, i64], None),
        "orc_int4_unpack": ([U8, F, i64, i64, F], None),
        "orc_int4_gemv_f32acc": ([U8, F, F, F, i64, i64, i64], None),
        "orc_sgemv_rows": ([i64, i64, F, F, F], None),
        "orc_encoder_forward": ([C.c_void_p, C.POINTER(F), i64, i64, I64, I64, F], C.c_int),
        "orc_gpt2_generate": ([C.c_void_p, C.POINTER(F), I64, i64, i64, I64, F, F], C.c_int),
        "orc_gpt2_generate_timed": ([C.c_void_p, C.POINTER(F), I64, i64, i64, I64, F, F,
                                     C.POINTER(C.c_double)], C.c_int),
        "orc_gpt2_forward": ([C.c_void_p, C.POINTER(F), I64, i64, F], C.c_int),
    }
    for name, (args, res) in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def _f(a: np.ndarray):
    return a.ctypes.data_as(F)


def _c32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return load().orc_num_threads()


def set_num_threads(n: int) -> None:
    load().orc_set_num_threads(n)


def parallel_blocks(n: int, grain: int, max_threads: int) -> list[tuple[int, int]]:
    """par::ParallelFor's [begin, end) blocks (src/util/parallel.cc:49-72)."""
    cap = max(1, max_threads)
    b = np.zeros(cap, np.int64)
    e = np.zeros(cap, np.int64)
    k = load().orc_parallel_blocks(n, grain, max_threads, b.ctypes.data_as(I64),
                                   e.ctypes.data_as(I64))
    return list(zip(b[:k].tolist(), e[:k].tolist()))


def sgemm(a, b, trans_a=False, trans_b=False, alpha=1.0, beta=0.0, c=None):
    a, b = _c32(a), _c32(b)
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    out = np.zeros((M, N), np.float32) if c is None else _c32(c).copy()
    load().orc_sgemm(int(trans_a), int(trans_b), M, N, K, alpha, _f(a), a.shape[1], _f(b),
                     b.shape[1], beta, _f(out), N)
    return out


def gemm(a, b, c=None, alpha=1.0, beta=1.0, trans_a=False, trans_b=False):
    a, b = _c32(a), _c32(b)
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    N = b.shape[0] if trans_b else b.shape[1]
    kind, cp = 0, None
    if c is not None:
        c = _c32(c)
        kind = 2 if c.size == M * N else (1 if c.ndim == 1 and c.shape[0] == N else 3)
        cp = _f(c)
    out = np.empty((M, N), np.float32)
    load().orc_gemm(int(trans_a), int(trans_b), M, N, K, alpha, _f(a), _f(b), beta, cp, kind,
                    _f(out))
    return out


def matmul(a, b):
    a, b = _c32(a), _c32(b)
    M, K = a.shape[-2:]
    N = b.shape[-1]
    ab, bb = a.shape[:-2], b.shape[:-2]
    ob = np.broadcast_shapes(ab, bb)
    batch = int(np.prod(ob)) if ob else 1
    na = int(np.prod(ab)) if ab else 1
    nb = int(np.prod(bb)) if bb else 1
    out = np.empty(tuple(ob) + (M, N), np.float32)
    load().orc_matmul(batch, M, N, K, _f(a), 0 if na == 1 else M * K, _f(b),
                      0 if nb == 1 else K * N, _f(out))
    return out


def fused_matmul_add_gelu(x, w, b):
    x, w, b = _c32(x), _c32(w), _c32(b)
    K, N = w.shape
    M = x.size // K
    out = np.empty(x.shape[:-1] + (N,), np.float32)
    load().orc_fused_matmul_add_gelu(M, N, K, _f(x), _f(w), _f(b), _f(out))
    return out


def fused_qkv(x, wq, bq, wk, bk, wv, bv):
    x = _c32(x)
    ws = [_c32(t) for t in (wq, bq, wk, bk, wv, bv)]
    K = x.shape[-1]
    M = x.size // K
    N = ws[0].shape[1]
    outs = [np.empty(x.shape[:-1] + (N,), np.float32) for _ in range(3)]
    load().orc_fused_qkv(M, K, N, _f(x), *[_f(t) for t in ws], *[_f(o) for o in outs])
    return outs


def mask_strides(mask_shape):
    s = [0, 0, 0, 0]
    st = 1
    r = len(mask_shape)
    for i in range(r - 1, -1, -1):
        od = 4 - (r - i)
        if od >= 0:
            s[od] = 0 if mask_shape[i] == 1 else st
        st *= mask_shape[i]
    return s


def fused_attention(q, k, v, mask, head_dim, fill):
    q, k, v = _c32(q), _c32(k), _c32(v)
    B, S, H = q.shape
    out = np.empty_like(q)
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        ms = (C.c_int64 * 4)(*mask_strides(m.shape))
        mp = m.ctypes.data_as(U8)
    else:
        ms, mp = None, None
    load().orc_fused_attention(B, S, H, head_dim, _f(q), _f(k), _f(v), mp, ms, fill, _f(out))
    return out


def layernorm(x, g, b, eps):
    x = _c32(x)
    feat = x.shape[-1]
    out = np.empty_like(x)
    load().orc_layernorm(x.size // feat, feat, _f(x), _f(_c32(g)), _f(_c32(b)), eps, _f(out))
    return out


def gelu(x):
    x = _c32(x)
    out = np.empty_like(x)
    load().orc_gelu(x.size, _f(x), _f(out))
    return out


def gelu_tanh(x):
    x = _c32(x)
    out = np.empty_like(x)
    load().orc_gelu_tanh(x.size, _f(x), _f(out))
    return out


def softmax(x, axis=-1):
    x = _c32(x)
    r = x.ndim
    axis = axis + r if axis < 0 else axis
    outer = int(np.prod(x.shape[:axis])) if axis else 1
    inner = int(np.prod(x.shape[axis + 1:])) if axis + 1 < r else 1
    out = np.empty_like(x)
    load().orc_softmax(outer, x.shape[axis], inner, _f(x), _f(out))
    return out


def add_bcast(a, b):
    a, b = _c32(a), _c32(b)
    out = np.empty_like(a)
    load().orc_add_bcast(a.size, _f(a), _f(b), b.size, _f(out))
    return out


def gather_rows(table, idx):
    table = _c32(table)
    idx = np.ascontiguousarray(idx, dtype=np.int64)
    out = np.empty(idx.shape + table.shape[1:], np.float32)
    rc = load().orc_gather_rows(table.shape[0], table.size // table.shape[0], _f(table),
                                idx.ctypes.data_as(I64), idx.size, _f(out))
    if rc != 0:
        raise RuntimeError("Gather: index out of range")
    return out


def split(x, axis, sizes):
    x = _c32(x)
    r = x.ndim
    axis = axis + r if axis < 0 else axis
    outer = int(np.prod(x.shape[:axis])) if axis else 1
    inner = int(np.prod(x.shape[axis + 1:])) if axis + 1 < r else 1
    outs = []
    for s in sizes:
        shp = list(x.shape)
        shp[axis] = s
        outs.append(np.empty(shp, np.float32))
    ptrs = (F * len(outs))(*[_f(o) for o in outs])
    load().orc_split(outer, x.shape[axis], inner, len(sizes), (C.c_int64 * len(sizes))(*sizes),
                     _f(x), ptrs)
    return outs


def concat(parts, axis):
    parts = [_c32(p) for p in parts]
    r = parts[0].ndim
    axis = axis + r if axis < 0 else axis
    shp = list(parts[0].shape)
    shp[axis] = sum(p.shape[axis] for p in parts)
    outer = int(np.prod(shp[:axis])) if axis else 1
    inner = int(np.prod(shp[axis + 1:])) if axis + 1 < r else 1
    out = np.empty(shp, np.float32)
    sizes = (C.c_int64 * len(parts))(*[p.shape[axis] for p in parts])
    ptrs = (F * len(parts))(*[_f(p) for p in parts])
    load().orc_concat(outer, inner, len(parts), sizes, ptrs, _f(out))
    return out


def argmax(x) -> int:
    x = _c32(x)
    return int(load().orc_argmax(x.size, _f(x)))


def _u8(a):
    return np.ascontiguousarray(a, dtype=np.uint8)


def int4_gemv_per_row(W, scales, x, K):
    W, scales, x = _u8(W), _c32(scales), _c32(x)
    N = scales.size
    B = x.size // K
    out = np.empty((B, N), np.float32)
    load().orc_int4_gemv_per_row_batched(W.ctypes.data_as(U8), _f(scales), _f(x), _f(out), N, K,
                                         B)
    return out


def int4_gemv_per_tensor(W, scale, x, N, K):
    W, x = _u8(W), _c32(x)
    out = np.empty(N, np.float32)
    load().orc_int4_gemv_per_tensor(W.ctypes.data_as(U8), scale, _f(x), _f(out), N, K)
    return out


def int4_unpack(W, scales, K):
    W, scales = _u8(W), _c32(scales)
    N = scales.size
    out = np.empty((N, K), np.float32)
    load().orc_int4_unpack(W.ctypes.data_as(U8), _f(scales), N, K, _f(out))
    return out


def int4_gemv_f32acc(W, scales, x, K):
    W, scales, x = _u8(W), _c32(scales), _c32(x)
    N = scales.size
    B = x.size // K
    out = np.empty((B, N), np.float32)
    load().orc_int4_gemv_f32acc(W.ctypes.data_as(U8), _f(scales), _f(x), _f(out), N, K, B)
    return out


def sgemv_rows(W, x):
    W, x = _c32(W), _c32(x)
    out = np.empty(W.shape[0], np.float32)
    load().orc_sgemv_rows(W.shape[0], W.shape[1], _f(W), _f(x), _f(out))
    return out


class _EncCfg(C.Structure):
    _fields_ = [("layers", C.c_int64), ("hidden", C.c_int64), ("heads", C.c_int64),
                ("ffn", C.c_int64), ("vocab", C.c_int64), ("max_pos", C.c_int64),
                ("n_classes", C.c_int64), ("eps", C.c_float)]


class _Gpt2Cfg(C.Structure):
    _fields_ = [("layers", C.c_int64), ("hidden", C.c_int64), ("heads", C.c_int64),
                ("ffn", C.c_int64), ("vocab", C.c_int64), ("max_pos", C.c_int64),
                ("eps", C.c_float)]


def _wptrs(weights):
    ws = [_c32(w) for w in weights]
    return ws, (F * len(ws))(*[_f(w) for w in ws])


def encoder_forward(cfg: dict, weights, ids, mask):
    ids = np.ascontiguousarray(ids, dtype=np.int64)
    mask = np.ascontiguousarray(mask, dtype=np.int64)
    B, S = ids.shape
    ws, ptrs = _wptrs(weights)
    c = _EncCfg(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["ffn"], cfg["vocab"],
                cfg["max_pos"], cfg["n_classes"], cfg["eps"])
    out = np.empty((B, cfg["n_classes"]), np.float32)
    rc = load().orc_encoder_forward(C.byref(c), ptrs, B, S, ids.ctypes.data_as(I64),
                                    mask.ctypes.data_as(I64), _f(out))
    if rc != 0:
        raise RuntimeError("encoder_forward: bad token id or sequence too long")
    return out


def gpt2_generate(cfg: dict, weights, prompt, max_tokens):
    p = np.ascontiguousarray(prompt, dtype=np.int64)
    ws, ptrs = _wptrs(weights)
    c = _Gpt2Cfg(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["ffn"], cfg["vocab"],
                 cfg["max_pos"], cfg["eps"])
    toks = np.empty(max_tokens, np.int64)
    logits = np.empty(cfg["vocab"], np.float32)
    margins = np.empty(max_tokens, np.float32)
    rc = load().orc_gpt2_generate(C.byref(c), ptrs, p.ctypes.data_as(I64), p.size, max_tokens,
                                  toks.ctypes.data_as(I64), _f(logits), _f(margins))
    if rc != 0:
        raise RuntimeError("gpt2_generate: bad token id or sequence too long")
    return toks, logits, margins


def gpt2_decode_step_ms(cfg: dict, weights, prompt, max_tokens) -> np.ndarray:
    """Wall time in ms of each of the max_tokens - 1 decode steps after the
    prompt (the step's forward and LM head; main.cpp:863-872)."""
    p = np.ascontiguousarray(prompt, dtype=np.int64)
    ws, ptrs = _wptrs(weights)
    c = _Gpt2Cfg(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["ffn"], cfg["vocab"],
                 cfg["max_pos"], cfg["eps"])
    toks = np.empty(max_tokens, np.int64)
    ms = np.zeros(max(1, max_tokens - 1), np.float64)
    rc = load().orc_gpt2_generate_timed(C.byref(c), ptrs, p.ctypes.data_as(I64), p.size,
                                        max_tokens, toks.ctypes.data_as(I64), None, None,
                                        ms.ctypes.data_as(C.POINTER(C.c_double)))
    if rc != 0:
        raise RuntimeError("gpt2_generate: bad token id or sequence too long")
    return ms[: max_tokens - 1]


def gpt2_forward(cfg: dict, weights, ids):
    i = np.ascontiguousarray(ids, dtype=np.int64)
    ws, ptrs = _wptrs(weights)
    c = _Gpt2Cfg(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["ffn"], cfg["vocab"],
                 cfg["max_pos"], cfg["eps"])
    out = np.empty((i.size, cfg["vocab"]), np.float32)
    rc = load().orc_gpt2_forward(C.byref(c), ptrs, i.ctypes.data_as(I64), i.size, _f(out))
    if rc != 0:
        raise RuntimeError("gpt2_forward: bad token id or sequence too long")
    return out
