"""The oracle's threading (row a20: par::ParallelFor, src/util/parallel.cc:49-72).

- The block partition restated in oracle.c (orc_parallel_blocks) against
  hand-worked cases of the reference's arithmetic and the properties that
  pin it: the blocks tile [0, n) in order, at most max_threads and at most
  ceil(n / grain) of them, all of one size but the last (grain bounds the
  block count only: chunks may be smaller than grain).
- The counterpart of the reference's one concurrency pin, Parallel.
  MatchesSerial (tests/kernels_test.cc:192-206): every OpenMP-parallel
  oracle kernel gives byte-identical output on 1 thread and on 8.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle as O
from inferc_amd import graphs


# (n, grain, max_threads) -> blocks, worked by hand from parallel.cc:53-71:
# blocks = min(T, max(1, ceil(n/grain))), chunk = ceil(n/blocks).
KATS = [
    ((10, 3, 4), [(0, 3), (3, 6), (6, 9), (9, 10)]),  # 4 blocks, chunk 3
    ((10, 3, 2), [(0, 5), (5, 10)]),                   # capped at 2 threads
    ((100, 64, 8), [(0, 50), (50, 100)]),              # ceil(100/64) = 2 blocks
    ((5, 0, 8), [(0, 1), (1, 2), (2, 3), (3, 4), (4, 5)]),  # grain 0: 8 blocks, 3 empty
    ((7, 100, 8), [(0, 7)]),                           # below the grain: serial
    ((9, 1, 4), [(0, 3), (3, 6), (6, 9)]),             # chunk 3 leaves block 4 empty
    ((1, 1, 1), [(0, 1)]),
    ((0, 1, 4), []),
    ((-3, 1, 4), []),
]


@pytest.mark.parametrize("args,blocks", KATS)
def test_parallel_blocks_kats(args, blocks):
    assert O.parallel_blocks(*args) == blocks


@pytest.mark.parametrize("n", [1, 2, 3, 17, 64, 100, 1023, 4096, 50257])
@pytest.mark.parametrize("grain", [0, 1, 7, 64, 1000])
@pytest.mark.parametrize("threads", [1, 3, 8, 16])
def test_parallel_blocks_tile_the_range(n, grain, threads):
    b = O.parallel_blocks(n, grain, threads)
    assert b[0][0] == 0 and b[-1][1] == n
    assert all(x[1] == y[0] for x, y in zip(b, b[1:]))  # contiguous, ordered
    assert all(lo < hi for lo, hi in b)
    assert len(b) <= max(1, threads)
    if grain > 0:
        assert len(b) <= -(-n // grain)
    sizes = [hi - lo for lo, hi in b]
    assert max(sizes) - min(sizes[:-1] or sizes) == 0  # equal chunks but the last


def test_parallel_blocks_planted_floor_chunk_is_caught():
    """chunk = floor(n / blocks) (a plausible slip) drops the tail."""
    def floor_chunk(n, grain, t):
        blocks = min(max(1, t), max(1, -(-n // grain) if grain > 0 else t))
        chunk = n // blocks
        return [(i * chunk, min(n, i * chunk + chunk)) for i in range(blocks)
                if i * chunk < min(n, i * chunk + chunk)]
    assert floor_chunk(10, 3, 4) != O.parallel_blocks(10, 3, 4)
    assert floor_chunk(10, 3, 4)[-1][1] != 10


def _both(fn):
    """fn() on 1 thread and on 8, restoring the thread count."""
    keep = O.num_threads()
    try:
        O.set_num_threads(1)
        a = fn()
        O.set_num_threads(8)
        b = fn()
    finally:
        O.set_num_threads(keep)
    return a, b


def _same(a, b):
    if isinstance(a, (tuple, list)):
        assert len(a) == len(b)
        for x, y in zip(a, b):
            _same(x, y)
        return
    a, b = np.asarray(a), np.asarray(b)
    assert a.dtype == b.dtype and a.shape == b.shape
    assert a.tobytes() == b.tobytes()


def _r(shape, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(shape) * scale).astype(np.float32)


KERNELS = {
    "sgemm": lambda: [O.sgemm(_r((97, 131), 1), _r((131, 75), 2), ta, tb)
                      if not (ta or tb) else
                      O.sgemm(_r((131, 97) if ta else (97, 131), 1),
                              _r((75, 131) if tb else (131, 75), 2), ta, tb)
                      for ta in (False, True) for tb in (False, True)],
    "gemm": lambda: O.gemm(_r((33, 64), 3), _r((48, 64), 4), _r(48, 5), 0.5, 2.0, False, True),
    "ffn_gelu": lambda: O.fused_matmul_add_gelu(_r((70, 96), 6), _r((96, 200), 7, 0.1),
                                                _r(200, 8)),
    "qkv": lambda: O.fused_qkv(_r((40, 64), 9), *[_r(s, 10 + i, 0.1) for i, s in
                                                  enumerate([(64, 64), 64] * 3)]),
    "attention": lambda: O.fused_attention(
        _r((3, 37, 128), 20), _r((3, 37, 128), 21), _r((3, 37, 128), 22),
        (np.arange(37)[None, :] >= np.array([37, 20, 5])[:, None]).reshape(3, 1, 1, 37),
        64, -3.0e38),
    "layernorm": lambda: O.layernorm(_r((300, 768), 23, 3.0), _r(768, 24), _r(768, 25), 1e-12),
    "softmax": lambda: [O.softmax(_r((4, 96), 26), -1), O.softmax(_r((6, 5, 7), 27), 1)],
    "add": lambda: O.add_bcast(_r((4, 96), 28), _r((1, 96), 29)),
    "gelus": lambda: [O.gelu(_r(10000, 30, 3.0)), O.gelu_tanh(_r(10000, 31, 3.0))],
    "int4_per_row": lambda: O.int4_gemv_per_row(*graphs.int4_weights(3000, 768, 32, "par"),
                                                _r((3, 768), 33), 768),
    "int4_f32acc": lambda: O.int4_gemv_f32acc(*graphs.int4_weights(3000, 768, 32, "par"),
                                              _r((3, 768), 33), 768),
    "sgemv": lambda: O.sgemv_rows(_r((5000, 768), 34, 0.02), _r(768, 35)),
}


@pytest.mark.parametrize("name", sorted(KERNELS))
def test_oracle_kernels_parallel_matches_serial(name):
    _same(*_both(KERNELS[name]))


def test_oracle_models_parallel_matches_serial():
    cfg = graphs.small_encoder_cfg()
    w = graphs.encoder_weights(cfg, 5)
    ids, mask = graphs.encoder_inputs(cfg, 2, 24, ragged=True)
    _same(*_both(lambda: O.encoder_forward(cfg, w, ids, mask)))
    gcfg = graphs.small_gpt2_cfg()
    gw = graphs.gpt2_weights(gcfg, 6)
    prompt = graphs.gpt2_prompt(gcfg, 8)
    _same(*_both(lambda: O.gpt2_generate(gcfg, gw, prompt, 6)))
