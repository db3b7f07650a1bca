"""Host-side mirror of inferc's kernel API (namespace ``inferc::rt``) over the
gfx950 C-ABI.

Names, argument meaning and error behaviour follow the reference headers:
``src/kernels/{matmul,fused_matmul_add_gelu,attention,activation,embedding,
movement}.h`` and ``src/runtime/{tensor,executor}.h``. Tensors live on the
device (:class:`Tensor`); every function enqueues on the context's stream and
returns a new tensor, as the reference's functions return a new
``rt::Tensor``. Errors raise :class:`~inferc_amd.lib.HipError`, a
``RuntimeError`` — the reference throws ``std::runtime_error``.
"""
from __future__ import annotations

import ctypes as C
import time
from typing import Sequence

import numpy as np

from . import lib as L
from .lib import HipError, check

_NP2DT = {
    np.dtype(np.float32): L.DT_F32,
    np.dtype(np.uint8): L.DT_U8,
    np.dtype(np.bool_): L.DT_BOOL,
    np.dtype(np.int32): L.DT_I32,
    np.dtype(np.int64): L.DT_I64,
}
_DT2NP = {v: k for k, v in _NP2DT.items()}


def _c_order(arr, dtype=None) -> np.ndarray:
    """C-contiguous view/copy that keeps 0-d arrays 0-d (np.ascontiguousarray
    would promote a scalar to shape (1,))."""
    return np.asarray(arr, dtype=dtype, order="C")


def _i64_array(vals: Sequence[int]):
    arr = (C.c_int64 * max(1, len(vals)))(*vals)
    return arr


class Context:
    """One device + one HIP stream (``inferc_hip_ctx``)."""

    def __init__(self, device: int = 0):
        self._lib = L.load_library()
        h = C.c_void_p()
        check(self._lib.inferc_hip_create(device, C.byref(h)))
        self.handle = h.value
        self.device = device

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.inferc_hip_destroy(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def sync(self) -> None:
        check(self._lib.inferc_hip_sync(self.handle))

    def reserve_workspace(self, nbytes: int) -> None:
        check(self._lib.inferc_hip_reserve_workspace(self.handle, nbytes))

    def set_gemv_decode(self, enabled: bool) -> None:
        """rt::SetGemvDecodeEnabled (src/kernels/matmul.cc:56-61) for this
        context: one-row products with a transposed B take the GEMV route."""
        check(self._lib.inferc_hip_set_gemv_decode(self.handle, int(bool(enabled))))

    def gemv_decode_enabled(self) -> bool:
        v = C.c_int()
        check(self._lib.inferc_hip_gemv_decode_enabled(self.handle, C.byref(v)))
        return bool(v.value)

    def malloc(self, nbytes: int) -> int:
        p = C.c_void_p()
        check(self._lib.inferc_hip_malloc(self.handle, nbytes, C.byref(p)))
        return p.value or 0

    def free(self, ptr: int) -> None:
        check(self._lib.inferc_hip_free(self.handle, ptr))

    def timer_start(self) -> None:
        check(self._lib.inferc_hip_timer_start(self.handle))

    def timer_stop(self) -> float:
        ms = C.c_float()
        check(self._lib.inferc_hip_timer_stop(self.handle, C.byref(ms)))
        return float(ms.value)

    def capture(self, fn) -> "Capture":
        """Records the kernels `fn()` enqueues into a replayable HIP graph.
        Run `fn` once beforehand so nothing allocates during capture."""
        check(self._lib.inferc_hip_capture_begin(self.handle))
        h = C.c_void_p()
        try:
            fn()
        finally:
            rc = self._lib.inferc_hip_capture_end(self.handle, C.byref(h))
        check(rc)
        return Capture(self, h.value)


class Capture:
    """A recorded sequence of entry points (inferc_hip_capture)."""

    def __init__(self, ctx: Context, handle: int):
        self.ctx = ctx
        self.handle = handle

    def replay(self) -> None:
        check(self.ctx._lib.inferc_hip_capture_replay(self.handle))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx._lib.inferc_hip_capture_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Tensor:
    """Device tensor: dtype + shape over a device allocation (rt::Tensor,
    src/runtime/tensor.h:23-74). Always contiguous row-major."""

    def __init__(self, ctx: Context, shape, dtype, ptr: int | None = None, owned: bool = True):
        self.ctx = ctx
        self.shape = tuple(int(d) for d in shape)
        self.dtype = np.dtype(dtype)
        if self.dtype not in _NP2DT:
            raise HipError(L.ERR_UNSUPPORTED, f"unsupported dtype {self.dtype}")
        self.owned = ptr is None
        self.ptr = ctx.malloc(max(self.nbytes, 4)) if ptr is None else ptr
        if ptr is not None:
            self.owned = owned

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.numel * self.dtype.itemsize

    @property
    def rank(self) -> int:
        return len(self.shape)

    @property
    def dt_code(self) -> int:
        return _NP2DT[self.dtype]

    @staticmethod
    def empty(ctx: Context, shape, dtype=np.float32) -> "Tensor":
        return Tensor(ctx, shape, dtype)

    @staticmethod
    def from_numpy(ctx: Context, arr) -> "Tensor":
        a = _c_order(arr)
        t = Tensor(ctx, a.shape, a.dtype)
        if a.nbytes:
            check(ctx._lib.inferc_hip_h2d(ctx.handle, t.ptr, a.ctypes.data, a.nbytes))
        return t

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=self.dtype)
        if out.nbytes:
            check(self.ctx._lib.inferc_hip_d2h(self.ctx.handle, out.ctypes.data, self.ptr,
                                               out.nbytes))
        return out

    def view(self, shape) -> "Tensor":
        """Reshape without copying (the buffer stays owned by self)."""
        t = Tensor(self.ctx, shape, self.dtype, ptr=self.ptr, owned=False)
        if t.numel != self.numel:
            raise HipError(L.ERR_SHAPE, f"view: {self.shape} -> {t.shape} changes element count")
        t._base = self
        return t

    def free(self) -> None:
        if self.owned and self.ptr and self.ctx.handle:
            self.ctx.free(self.ptr)
        self.ptr = 0
        self.owned = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def _ctx_of(*ts: Tensor) -> Context:
    return ts[0].ctx


def _need_f32(t: Tensor, who: str) -> None:
    if t.dtype != np.float32:
        raise HipError(L.ERR_UNSUPPORTED, f"{who}: float32 only")


# ----------------------------------------------------------------- products

def Gemm(a: Tensor, b: Tensor, c: Tensor | None = None, alpha: float = 1.0, beta: float = 1.0,
         trans_a: bool = False, trans_b: bool = False, residual: Tensor | None = None,
         act: int = L.ACT_NONE) -> Tensor:
    """alpha*op(A)*op(B) + beta*C (src/kernels/matmul.cc:161-228)."""
    if a.rank != 2 or b.rank != 2:
        raise HipError(L.ERR_SHAPE, "Gemm: 2D inputs only")
    _need_f32(a, "Gemm")
    _need_f32(b, "Gemm")
    M = a.shape[1] if trans_a else a.shape[0]
    K = a.shape[0] if trans_a else a.shape[1]
    Kb = b.shape[1] if trans_b else b.shape[0]
    N = b.shape[0] if trans_b else b.shape[1]
    if K != Kb:
        raise HipError(L.ERR_SHAPE, "Gemm: K mismatch")
    ctx = a.ctx
    out = Tensor.empty(ctx, (M, N))
    c_kind, ldc, cptr = L.C_NONE, 0, None
    if c is not None and beta != 0.0:
        if c.numel == M * N:
            c_kind, ldc = L.C_FULL, N
        elif c.rank == 1 and c.shape[0] == N:
            c_kind = L.C_ROW
        elif c.numel == 1:
            c_kind = L.C_SCALAR
        else:
            raise HipError(L.ERR_SHAPE, "Gemm: unsupported C shape for broadcast")
        cptr = c.ptr
    check(ctx._lib.inferc_hip_gemm_f32(
        ctx.handle, int(trans_a), int(trans_b), M, N, K, alpha, a.ptr, a.shape[1], b.ptr,
        b.shape[1], beta, cptr, c_kind, ldc, residual.ptr if residual else None,
        N if residual else 0, act, out.ptr, N))
    return out


def MatMul(a: Tensor, b: Tensor) -> Tensor:
    """numpy-semantics MatMul (src/kernels/matmul.cc:63-159): batch dims
    broadcast when one side has a single batch slice."""
    _need_f32(a, "MatMul")
    _need_f32(b, "MatMul")
    a_1d, b_1d = a.rank == 1, b.rank == 1
    ash = (1,) + a.shape if a_1d else a.shape
    bsh = b.shape + (1,) if b_1d else b.shape
    M, K = ash[-2], ash[-1]
    Kb, N = bsh[-2], bsh[-1]
    if K != Kb:
        raise HipError(L.ERR_SHAPE, "MatMul: inner dim mismatch (K!=K)")
    ab, bb = ash[:-2], bsh[:-2]
    ob = np.broadcast_shapes(ab, bb)
    batch = int(np.prod(ob, dtype=np.int64)) if ob else 1
    na = int(np.prod(ab, dtype=np.int64)) if ab else 1
    nb = int(np.prod(bb, dtype=np.int64)) if bb else 1
    if na not in (1, batch) or nb not in (1, batch):
        raise HipError(L.ERR_UNSUPPORTED, "MatMul: partial batch broadcast is not supported")
    ctx = a.ctx
    out_shape = tuple(ob) + (M, N)
    out = Tensor.empty(ctx, out_shape)
    check(ctx._lib.inferc_hip_matmul_f32(ctx.handle, batch, M, N, K, a.ptr,
                                         0 if na == 1 else M * K, b.ptr,
                                         0 if nb == 1 else K * N, out.ptr))
    if a_1d:
        out_shape = out_shape[:-2] + out_shape[-1:]
    if b_1d:
        out_shape = out_shape[:-1]
    return out.view(out_shape) if (a_1d or b_1d) else out


def FusedMatMulAddGELU(x: Tensor, w: Tensor, bias: Tensor) -> Tensor:
    """Y = GELU(X @ W + bias) (src/kernels/fused_matmul_add_gelu.cc:13-80)."""
    if w.rank != 2:
        raise HipError(L.ERR_SHAPE, "FusedMatMulAddGELU: W must be 2D [K, N]")
    if bias.rank != 1:
        raise HipError(L.ERR_SHAPE, "FusedMatMulAddGELU: bias must be 1D [N]")
    if x.rank < 2:
        raise HipError(L.ERR_SHAPE, "FusedMatMulAddGELU: X must be at least 2D")
    K, N = w.shape
    if x.shape[-1] != K:
        raise HipError(L.ERR_SHAPE, "FusedMatMulAddGELU: K mismatch between X and W")
    if bias.shape[0] != N:
        raise HipError(L.ERR_SHAPE, "FusedMatMulAddGELU: bias size must equal N")
    M = x.numel // K
    ctx = x.ctx
    out = Tensor.empty(ctx, x.shape[:-1] + (N,))
    check(ctx._lib.inferc_hip_fused_matmul_add_gelu_f32(ctx.handle, M, N, K, x.ptr, w.ptr,
                                                         bias.ptr, out.ptr))
    return out


def FusedQKVProjection(x: Tensor, wq: Tensor, bq: Tensor, wk: Tensor, bk: Tensor, wv: Tensor,
                       bv: Tensor) -> list[Tensor]:
    """{X Wq + bq, X Wk + bk, X Wv + bv} (src/kernels/attention.cc:102-141)."""
    _need_f32(x, "FusedQKV")
    K = x.shape[-1]
    M = x.numel // K
    N = wq.shape[1]
    for w, b in ((wq, bq), (wk, bk), (wv, bv)):
        if w.shape != (K, N) or b.numel != N:
            raise HipError(L.ERR_SHAPE, "FusedQKV: projections must be [K,N] with bias [N]")
    ctx = x.ctx
    outs = [Tensor.empty(ctx, x.shape[:-1] + (N,)) for _ in range(3)]
    check(ctx._lib.inferc_hip_fused_qkv_f32(ctx.handle, M, K, N, x.ptr, wq.ptr, bq.ptr, wk.ptr,
                                            bk.ptr, wv.ptr, bv.ptr, outs[0].ptr, outs[1].ptr,
                                            outs[2].ptr))
    return outs


# ---------------------------------------------------------------- attention

def mask_strides(mask_shape: Sequence[int]) -> list[int]:
    """Strides of a mask right-aligned against [B,nH,S,S], 0 on broadcast axes
    (src/kernels/attention.cc:17-29)."""
    s = [0, 0, 0, 0]
    st = 1
    r = len(mask_shape)
    for i in range(r - 1, -1, -1):
        od = 4 - (r - i)
        if od >= 0:
            s[od] = 0 if mask_shape[i] == 1 else st
        st *= mask_shape[i]
    return s


def FusedAttention(q: Tensor, k: Tensor, v: Tensor, mask_cond: Tensor | None, head_dim: int,
                   fill: float) -> Tensor:
    """Multi-head attention over [B,S,H] (src/kernels/attention.cc:32-100)."""
    _need_f32(q, "FusedAttention")
    if q.rank != 3:
        raise HipError(L.ERR_SHAPE, "FusedAttention: expect [B,S,H]")
    B, S, H = q.shape
    ctx = q.ctx
    out = Tensor.empty(ctx, (B, S, H))
    mptr, ms = None, None
    if mask_cond is not None and mask_cond.rank > 0 and mask_cond.numel > 0:
        mptr = mask_cond.ptr
        ms = _i64_array(mask_strides(mask_cond.shape))
    check(ctx._lib.inferc_hip_fused_attention_f32(ctx.handle, B, S, H, head_dim, q.ptr, k.ptr,
                                                  v.ptr, mptr, ms, fill, out.ptr))
    return out


# ------------------------------------------------------- normalisation, etc.

def LayerNorm(x: Tensor, scale: Tensor, bias: Tensor, eps: float = 1e-12,
              normalized_dims: int = 1, residual: Tensor | None = None) -> Tensor:
    """LayerNorm over the last `normalized_dims` axes (activation.cc:103-150)."""
    _need_f32(x, "LayerNorm")
    if normalized_dims < 1 or normalized_dims > x.rank:
        raise HipError(L.ERR_ARG, "LayerNorm: bad normalized_dims")
    feat = int(np.prod(x.shape[x.rank - normalized_dims:], dtype=np.int64))
    if scale.numel != feat or bias.numel != feat:
        raise HipError(L.ERR_SHAPE, "LayerNorm: scale/bias size mismatch with feature dim")
    ctx = x.ctx
    out = Tensor.empty(ctx, x.shape)
    check(ctx._lib.inferc_hip_layernorm_f32(ctx.handle, x.numel // feat, feat, x.ptr,
                                            residual.ptr if residual else None, scale.ptr,
                                            bias.ptr, eps, out.ptr))
    return out


def _act(x: Tensor, act: int, who: str) -> Tensor:
    _need_f32(x, who)
    out = Tensor.empty(x.ctx, x.shape)
    check(x.ctx._lib.inferc_hip_activation_f32(x.ctx.handle, x.numel, x.ptr, act, out.ptr))
    return out


def Gelu(x: Tensor) -> Tensor:
    """x*0.5*(1+erf(x/sqrt2)) (src/kernels/activation.cc:15-29)."""
    return _act(x, L.ACT_GELU_ERF, "Gelu")


def GeluTanh(x: Tensor) -> Tensor:
    """GPT-2 tanh GELU (src/kernels/activation.cc:31-50)."""
    return _act(x, L.ACT_GELU_TANH, "GeluTanh")


def Relu(x: Tensor) -> Tensor:
    return _act(x, L.ACT_RELU, "Relu")


def Softmax(x: Tensor, axis: int = -1) -> Tensor:
    """Stable softmax along `axis` (src/kernels/activation.cc:52-101)."""
    _need_f32(x, "Softmax")
    r = x.rank
    if axis < 0:
        axis += r
    if axis < 0 or axis >= r:
        raise HipError(L.ERR_ARG, "Softmax: axis out of range")
    outer = int(np.prod(x.shape[:axis], dtype=np.int64)) if axis else 1
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64)) if axis + 1 < r else 1
    out = Tensor.empty(x.ctx, x.shape)
    check(x.ctx._lib.inferc_hip_softmax_f32(x.ctx.handle, outer, x.shape[axis], inner, x.ptr,
                                            out.ptr))
    return out


def Add(a: Tensor, b: Tensor) -> Tensor:
    """Broadcast add for the hot path's forms: equal shapes, a row/suffix
    broadcast, or a scalar (src/kernels/elementwise.cc:225)."""
    _need_f32(a, "Add")
    _need_f32(b, "Add")
    big, small = (a, b) if a.numel >= b.numel else (b, a)
    shape = np.broadcast_shapes(a.shape, b.shape)
    if int(np.prod(shape, dtype=np.int64)) != big.numel:
        raise HipError(L.ERR_UNSUPPORTED, "Add: only suffix broadcasts are supported")
    trail = small.shape
    while trail and trail[0] == 1:
        trail = trail[1:]
    if small.numel != big.numel and tuple(big.shape[len(big.shape) - len(trail):]) != trail:
        raise HipError(L.ERR_UNSUPPORTED, "Add: only suffix broadcasts are supported")
    out = Tensor.empty(a.ctx, shape)
    check(a.ctx._lib.inferc_hip_add_f32(a.ctx.handle, big.numel, big.ptr, small.ptr,
                                        small.numel, out.ptr))
    return out


def Gather(data: Tensor, idx: Tensor, axis: int = 0) -> Tensor:
    """Row gather along axis 0 with int64 indices (src/kernels/embedding.cc:9-72).
    Out-of-range indices raise, as the reference does."""
    if axis != 0:
        raise HipError(L.ERR_UNSUPPORTED, "Gather: axis 0 only on this path")
    _need_f32(data, "Gather")
    if idx.dtype != np.int64:
        raise HipError(L.ERR_ARG, "Gather: indices must be int64")
    ctx = data.ctx
    rows = data.shape[0]
    row_len = data.numel // rows if rows else 0
    out = Tensor.empty(ctx, tuple(idx.shape) + tuple(data.shape[1:]))
    flag = Tensor.from_numpy(ctx, np.zeros(1, np.int32))
    check(ctx._lib.inferc_hip_gather_f32(ctx.handle, rows, row_len, data.ptr, idx.ptr,
                                         idx.numel, out.ptr, flag.ptr))
    if flag.numpy()[0]:
        raise HipError(L.ERR_ARG, "Gather: index out of range")
    return out


def Split(x: Tensor, axis: int, sizes: Sequence[int]) -> list[Tensor]:
    """src/kernels/movement.cc:391-431."""
    _need_f32(x, "Split")
    r = x.rank
    if axis < 0:
        axis += r
    if axis < 0 or axis >= r:
        raise HipError(L.ERR_ARG, "Split: axis out of range")
    outer = int(np.prod(x.shape[:axis], dtype=np.int64)) if axis else 1
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64)) if axis + 1 < r else 1
    outs = []
    for s in sizes:
        shp = list(x.shape)
        shp[axis] = s
        outs.append(Tensor.empty(x.ctx, shp))
    ptrs = (C.c_void_p * max(1, len(outs)))(*[o.ptr for o in outs])
    check(x.ctx._lib.inferc_hip_split_f32(x.ctx.handle, outer, x.shape[axis], inner, len(sizes),
                                          _i64_array(list(sizes)), x.ptr, ptrs))
    return outs


def Concat(parts: Sequence[Tensor], axis: int) -> Tensor:
    """src/kernels/movement.cc:142-189."""
    if not parts:
        raise HipError(L.ERR_ARG, "Concat: no inputs")
    r = parts[0].rank
    if axis < 0:
        axis += r
    shp = list(parts[0].shape)
    shp[axis] = sum(p.shape[axis] for p in parts)
    outer = int(np.prod(shp[:axis], dtype=np.int64)) if axis else 1
    inner = int(np.prod(shp[axis + 1:], dtype=np.int64)) if axis + 1 < r else 1
    out = Tensor.empty(parts[0].ctx, shp)
    ptrs = (C.c_void_p * len(parts))(*[p.ptr for p in parts])
    check(out.ctx._lib.inferc_hip_concat_f32(out.ctx.handle, outer, inner, len(parts),
                                             _i64_array([p.shape[axis] for p in parts]), ptrs,
                                             out.ptr))
    return out


def Argmax(x: Tensor) -> int:
    """First index of the maximum (src/cli/main.cpp:875-879)."""
    _need_f32(x, "Argmax")
    out = Tensor.empty(x.ctx, (1,), np.int64)
    check(x.ctx._lib.inferc_hip_argmax_f32(x.ctx.handle, x.numel, x.ptr, out.ptr))
    return int(out.numpy()[0])


# ------------------------------------------------------------- decode GEMVs

def Gemv(w_nk: Tensor, x: Tensor, bias: Tensor | None = None, residual: Tensor | None = None,
         act: int = L.ACT_NONE, ln: tuple[Tensor, Tensor, float] | None = None) -> Tensor:
    """y = act(W x + bias + residual), W [N,K] (the transB=1 sgemv route of
    src/kernels/matmul.cc:207-216); `ln` = (gamma, beta, eps) normalises x first."""
    _need_f32(w_nk, "Gemv")
    N, K = w_nk.shape
    if x.numel != K:
        raise HipError(L.ERR_SHAPE, "Gemv: x length != K")
    out = Tensor.empty(x.ctx, (N,))
    g, b, eps = (ln[0].ptr, ln[1].ptr, ln[2]) if ln else (None, None, 0.0)
    check(x.ctx._lib.inferc_hip_gemv_f32(x.ctx.handle, N, K, w_nk.ptr, x.ptr, g, b, eps,
                                         bias.ptr if bias else None,
                                         residual.ptr if residual else None, act, out.ptr))
    return out


def Int4Unpack(w: Tensor, scales: Tensor, K: int) -> Tensor:
    """out[r,k] = s_r * float(nib - 8) (bench/amx/int4_gemv_amx.cc:258-271)."""
    N = scales.numel
    out = Tensor.empty(w.ctx, (N, K))
    check(w.ctx._lib.inferc_hip_int4_unpack(w.ctx.handle, N, K, w.ptr, scales.ptr, out.ptr))
    return out


def Int4Gemv(w: Tensor, scales: Tensor, x: Tensor, K: int) -> Tensor:
    """y[b] = W_deq x[b] for x [B,K] (int4_gemv_amx.cc:258-356)."""
    N = scales.numel
    B = x.numel // K
    out = Tensor.empty(w.ctx, (B, N))
    check(w.ctx._lib.inferc_hip_int4_gemv(w.ctx.handle, N, K, w.ptr, scales.ptr, B, x.ptr,
                                          out.ptr))
    return out


def int4_quantize_rows(w: np.ndarray, lib=None) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Per-row symmetric int4 quantisation of w [N, K] on the host (no GPU):
    returns (packed [N, K/2] uint8, scales [N] fp32, dequantised [N, K] fp32)."""
    from . import lib as L
    w = _c_order(w, np.float32)
    N, K = w.shape
    packed = np.empty((N, K // 2), np.uint8)
    scales = np.empty(N, np.float32)
    deq = np.empty((N, K), np.float32)
    lb = lib or L.load_library()
    check(lb.inferc_int4_quantize_rows(N, K, w.ctypes.data, packed.ctypes.data,
                                       scales.ctypes.data, deq.ctypes.data))
    return packed, scales, deq


def int4_gemv_grouped(ctx: Context, mats: Sequence[tuple[Tensor, Tensor, Tensor, Tensor, int]],
                      batch: int) -> None:
    """One launch over many int4 GEMVs; each entry is (W, scales, x, y, K)."""
    n = len(mats)
    Ns = _i64_array([m[1].numel for m in mats])
    Ks = _i64_array([m[4] for m in mats])
    W = (C.c_void_p * n)(*[m[0].ptr for m in mats])
    S = (C.c_void_p * n)(*[m[1].ptr for m in mats])
    X = (C.c_void_p * n)(*[m[2].ptr for m in mats])
    Y = (C.c_void_p * n)(*[m[3].ptr for m in mats])
    check(ctx._lib.inferc_hip_int4_gemv_grouped(ctx.handle, n, Ns, Ks, W, S, batch, X, Y))


def KvAppendAttend(q: Tensor, k_new: Tensor, v_new: Tensor, k_cache: Tensor, v_cache: Tensor,
                   pos: Tensor, n_heads: int, head_dim: int, max_t: int) -> Tensor:
    """Append K/V at *pos and attend over positions <= pos."""
    out = Tensor.empty(q.ctx, (n_heads * head_dim,))
    check(q.ctx._lib.inferc_hip_kv_append_attend_f32(q.ctx.handle, n_heads, head_dim, max_t,
                                                      pos.ptr, q.ptr, k_new.ptr, v_new.ptr,
                                                      k_cache.ptr, v_cache.ptr, out.ptr))
    return out


# ----------------------------------------------------------------- executor

# inferc_graph_optimize's pass order and count slots
PASSES = ("fold_constant_transpose", "recognize_attention", "recognize_attention_additive",
          "fuse_qkv_projection", "recognize_layernorm", "recognize_gelu", "recognize_gelu_tanh",
          "fuse_matmul_add_gelu")


def onnx_summary(src, text: bool = False):
    """SummarizeModel (dict) or PrintSummary (text) of an ONNX model
    (src/frontend/onnx_loader.cc:113-210), from a path or bytes."""
    import json
    lib = L.load_library()
    b = bytes(src) if isinstance(src, (bytes, bytearray, memoryview)) else open(src, "rb").read()
    n = C.c_size_t()
    check(lib.inferc_onnx_summary(b, len(b), int(text), None, 0, C.byref(n)))
    buf = C.create_string_buffer(n.value + 1)
    check(lib.inferc_onnx_summary(b, len(b), int(text), buf, n.value + 1, C.byref(n)))
    s = buf.value.decode()
    return s if text else json.loads(s)


class Graph:
    """Host IR of (fused) nodes as the reference's passes leave it
    (src/ir/graph.h:45-97)."""

    def __init__(self):
        self._lib = L.load_library()
        h = C.c_void_p()
        check(self._lib.inferc_graph_create(C.byref(h)))
        self.handle = h.value
        self.op_types: list[str] = []

    def add_initializer(self, name: str, arr: np.ndarray) -> None:
        a = _c_order(arr)
        dt = _NP2DT[a.dtype]
        shape = _i64_array(list(a.shape))
        check(self._lib.inferc_graph_add_initializer(self.handle, name.encode(), dt, a.ndim, shape,
                                                     a.ctypes.data if a.nbytes else None))

    def add_node(self, op_type: str, inputs: Sequence[str], outputs: Sequence[str],
                 name: str = "", **attrs) -> None:
        ins = (C.c_char_p * max(1, len(inputs)))(*[s.encode() for s in inputs])
        outs = (C.c_char_p * max(1, len(outputs)))(*[s.encode() for s in outputs])
        parts = []
        for k, v in attrs.items():
            if isinstance(v, (list, tuple)):
                v = ",".join(str(int(e)) for e in v)
            elif isinstance(v, float):
                v = repr(float(v))
            parts.append(f"{k}={v}")
        check(self._lib.inferc_graph_add_node(self.handle, op_type.encode(),
                                              (name or f"{op_type}_{len(self.op_types)}").encode(),
                                              len(inputs), ins, len(outputs), outs,
                                              ";".join(parts).encode()))
        self.op_types.append(op_type)

    def add_output(self, name: str) -> None:
        check(self._lib.inferc_graph_add_output(self.handle, name.encode()))

    def add_input(self, name: str, dtype, shape: Sequence[int]) -> None:
        """A declared graph input (-1 for a symbolic dim)."""
        check(self._lib.inferc_graph_add_input(self.handle, name.encode(),
                                               _NP2DT[np.dtype(dtype)], len(shape),
                                               _i64_array(list(shape))))

    def add_tensor_attr(self, attr: str, arr: np.ndarray) -> None:
        """A tensor-valued attribute on the most recently added node."""
        a = _c_order(arr)
        check(self._lib.inferc_graph_add_tensor_attr(self.handle, attr.encode(), _NP2DT[a.dtype],
                                                     a.ndim, _i64_array(list(a.shape)),
                                                     a.ctypes.data if a.nbytes else None))

    def add_constant(self, out: str, arr, name: str = "") -> None:
        """An ONNX Constant node whose `value` attribute holds `arr`."""
        self.add_node("Constant", [], [out], name=name)
        self.add_tensor_attr("value", np.asarray(arr))

    @classmethod
    def from_onnx(cls, src) -> "Graph":
        """LoadOnnx + ConvertOnnxToIR (src/frontend/onnx_loader.cc:107-111,
        onnx_to_ir.cc:87-144) from a path or the model's bytes."""
        g = cls.__new__(cls)
        g._lib = L.load_library()
        g.op_types = []
        h = C.c_void_p()
        if isinstance(src, (bytes, bytearray, memoryview)):
            b = bytes(src)
            check(g._lib.inferc_onnx_load_bytes(b, len(b), C.byref(h)))
        else:
            check(g._lib.inferc_onnx_load(str(src).encode(), C.byref(h)))
        g.handle = h.value
        g.op_types = [n["op"] for n in g.to_dict()["nodes"]]
        return g

    def to_dict(self) -> dict:
        """The graph's structure: name, inputs, outputs, initializers (name,
        dtype, shape, bytes) and nodes (op, name, domain, inputs, outputs,
        attrs as text, tensor_attrs)."""
        import json
        n = C.c_size_t()
        check(self._lib.inferc_graph_to_json(self.handle, None, 0, C.byref(n)))
        buf = C.create_string_buffer(n.value + 1)
        check(self._lib.inferc_graph_to_json(self.handle, buf, n.value + 1, C.byref(n)))
        return json.loads(buf.value.decode(errors="replace"))

    def initializer(self, name: str) -> np.ndarray:
        dt, rank = C.c_int(), C.c_int()
        shape = (C.c_int64 * 8)()
        check(self._lib.inferc_graph_get_initializer(self.handle, name.encode(), C.byref(dt),
                                                     C.byref(rank), shape, None, 0))
        out = np.empty(tuple(shape[i] for i in range(rank.value)), dtype=_DT2NP[dt.value])
        check(self._lib.inferc_graph_get_initializer(self.handle, name.encode(), C.byref(dt),
                                                     C.byref(rank), shape, out.ctypes.data,
                                                     out.nbytes))
        return out

    def run_pass(self, name: str) -> int:
        """One fusion pass by name (see PASSES); returns its match count."""
        c = C.c_int()
        check(self._lib.inferc_graph_run_pass(self.handle, name.encode(), C.byref(c)))
        self.op_types = [n["op"] for n in self.to_dict()["nodes"]]
        return c.value

    def optimize(self) -> dict[str, int]:
        """The pass pipeline of `inferc optimize` (src/cli/main.cpp:265-271);
        returns each pass's match count."""
        counts = (C.c_int * len(PASSES))()
        check(self._lib.inferc_graph_optimize(self.handle, counts))
        self.op_types = [n["op"] for n in self.to_dict()["nodes"]]
        return dict(zip(PASSES, counts))

    def close(self) -> None:
        if getattr(self, "handle", None):
            self._lib.inferc_graph_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class _NoDevice:
    """Stands in for a Context in a dry-run executor (no device calls)."""

    def __init__(self):
        self._lib = L.load_library()
        self.handle = None


class Executor:
    """rt::Executor (src/runtime/executor.h:24-41) on the device.

    ``Executor.dry(graph)`` builds a device-free executor whose run() only
    plans: shape inference, host shape plumbing and peephole fusion."""

    def __init__(self, ctx: Context, graph: Graph, _dry: bool = False):
        self.ctx = ctx
        h = C.c_void_p()
        if _dry:
            check(ctx._lib.inferc_executor_create_dry(graph.handle, C.byref(h)))
        else:
            check(ctx._lib.inferc_executor_create(ctx.handle, graph.handle, C.byref(h)))
        self.handle = h.value

    @classmethod
    def dry(cls, graph: Graph) -> "Executor":
        return cls(_NoDevice(), graph, _dry=True)

    def node_count(self) -> int:
        n = C.c_int()
        check(self.ctx._lib.inferc_executor_node_count(self.handle, C.byref(n)))
        return n.value

    def output_shape(self, name: str) -> tuple[tuple[int, ...], np.dtype]:
        dt, rank = C.c_int(), C.c_int()
        shape = (C.c_int64 * 8)()
        check(self.ctx._lib.inferc_executor_output_info(self.handle, name.encode(), C.byref(dt),
                                                        C.byref(rank), shape))
        return tuple(shape[i] for i in range(rank.value)), _DT2NP[dt.value]

    def set_graph_mode(self, enabled: bool) -> None:
        check(self.ctx._lib.inferc_executor_set_graph_mode(self.handle, int(enabled)))

    def set_input(self, name: str, arr: np.ndarray) -> None:
        a = _c_order(arr)
        check(self.ctx._lib.inferc_executor_set_input(
            self.handle, name.encode(), _NP2DT[a.dtype], a.ndim, _i64_array(list(a.shape)),
            a.ctypes.data if a.nbytes else None))

    def set_input_device(self, name: str, t: Tensor) -> None:
        check(self.ctx._lib.inferc_executor_set_input_device(
            self.handle, name.encode(), t.dt_code, t.rank, _i64_array(list(t.shape)), t.ptr))

    def run_async(self) -> None:
        check(self.ctx._lib.inferc_executor_run(self.handle))

    def output(self, name: str) -> np.ndarray:
        dt, rank = C.c_int(), C.c_int()
        shape = (C.c_int64 * 8)()
        check(self.ctx._lib.inferc_executor_output_info(self.handle, name.encode(), C.byref(dt),
                                                        C.byref(rank), shape))
        out = np.empty(tuple(shape[i] for i in range(rank.value)), dtype=_DT2NP[dt.value])
        check(self.ctx._lib.inferc_executor_get_output(self.handle, name.encode(),
                                                       out.ctypes.data, out.nbytes))
        return out

    def run(self, inputs: dict[str, np.ndarray], outputs: Sequence[str]) -> dict[str, np.ndarray]:
        """Executor::Run: bind inputs, run, return the named outputs."""
        for k, v in inputs.items():
            self.set_input(k, v)
        self.run_async()
        return {o: self.output(o) for o in outputs}

    def bind_kv_cache(self, max_t: int) -> None:
        """Keeps the K/V of every FusedAttentionPast node in a device cache of
        max_t positions (0 unbinds); see inferc_executor_bind_kv_cache."""
        check(self.ctx._lib.inferc_executor_bind_kv_cache(self.handle, max_t))

    def set_decode_position(self, length: int, mask_input: str | None = None) -> None:
        """Decode mode (inferc_executor_set_decode_position): the KV caches
        hold `length` positions, counted on the device; every run is one step
        with the past given by shape with length 0 and an all-ones mask of
        the new positions. A negative length leaves decode mode."""
        check(self.ctx._lib.inferc_executor_set_decode_position(
            self.handle, int(length), mask_input.encode() if mask_input else None))

    def decode_position(self) -> int:
        v = C.c_int64()
        check(self.ctx._lib.inferc_executor_decode_position(self.handle, C.byref(v)))
        return v.value

    def set_decode_feedback(self, logits: str | None, ids: str = "input_ids",
                            first_token: int = 0) -> None:
        """In decode mode, every run feeds the greedy token of `logits` back
        as input `ids` on the device and records it by position
        (inferc_executor_set_decode_feedback); None turns it off."""
        check(self.ctx._lib.inferc_executor_set_decode_feedback(
            self.handle, logits.encode() if logits else None, ids.encode(), int(first_token)))

    def run_steps(self, steps: int, timed: bool = True) -> list[float] | None:
        """`steps` runs back to back (inferc_executor_run_steps); with timed,
        waits and returns each run's device ms from HIP events."""
        if not timed:
            check(self.ctx._lib.inferc_executor_run_steps(self.handle, int(steps), None))
            return None
        ms = (C.c_float * max(1, int(steps)))()
        check(self.ctx._lib.inferc_executor_run_steps(self.handle, int(steps), ms))
        return [float(ms[i]) for i in range(int(steps))]

    def decode_tokens(self, first_pos: int, n: int) -> np.ndarray:
        """The fed-back tokens at positions first_pos .. first_pos + n - 1."""
        out = np.zeros(max(0, int(n)), np.int64)
        check(self.ctx._lib.inferc_executor_decode_tokens(
            self.handle, int(first_pos), int(n),
            out.ctypes.data_as(C.POINTER(C.c_int64))))
        return out

    def set_input_shape(self, name: str, dtype, shape: Sequence[int]) -> None:
        """An input that carries only its shape (a past the KV cache holds)."""
        check(self.ctx._lib.inferc_executor_set_input_shape(
            self.handle, name.encode(), _NP2DT[np.dtype(dtype)], len(shape),
            _i64_array(list(shape))))

    def output_device(self, name: str) -> "Tensor":
        """A borrowed device view of an output (valid until the next run)."""
        shape, dt = self.output_shape(name)
        p = C.c_void_p()
        check(self.ctx._lib.inferc_executor_output_device(self.handle, name.encode(),
                                                          C.byref(p)))
        return Tensor(self.ctx, shape, dt, ptr=p.value, owned=False)

    def output_argmax(self, name: str) -> int:
        """Index of the first maximum of the output's last row, on the device."""
        idx = C.c_int64()
        check(self.ctx._lib.inferc_executor_output_argmax(self.handle, name.encode(),
                                                          C.byref(idx)))
        return idx.value

    def device_bytes(self) -> dict[str, int]:
        """Device bytes held: uploaded initializers, transposed copies of
        [K, N] weights read by one-row products, activation arena."""
        a, b, c = C.c_int64(), C.c_int64(), C.c_int64()
        check(self.ctx._lib.inferc_executor_device_bytes(self.handle, C.byref(a), C.byref(b),
                                                         C.byref(c)))
        return {"initializers": a.value, "transposed_copies": b.value, "arena": c.value}

    def run_profiled(self, profiler) -> None:
        """Executor::Run(inputs, profiler) (src/runtime/executor.cc:98-125,
        349-354): one eager pass recorded as one profiler iteration, each
        node's time measured between HIP events on the stream."""
        check(self.ctx._lib.inferc_executor_run_profiled(self.handle, profiler.handle))

    def profile(self, inputs: dict[str, np.ndarray], iters: int = 10, warmup: int = 3,
                backend: str = "inferc-hip", model: str = "",
                track_activation_bytes: bool = False) -> dict:
        """The profiled loop of `inferc run --profile` (src/cli/main.cpp:355-424):
        `warmup` unprofiled runs, `iters` profiled ones, peak RSS, then the
        report in the reference's JSON schema (as a dict)."""
        from .profiler import Profiler
        for k, v in inputs.items():
            self.set_input(k, v)
        for _ in range(warmup):
            self.run_async()
        p = Profiler()
        p.set_track_activation_bytes(track_activation_bytes)
        for _ in range(iters):
            self.run_profiled(p)
        p.snapshot_peak_rss()
        return p.report(backend, model)

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx._lib.inferc_executor_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


# -------------------------------------------------------------------- GPT-2

def _optimize(g: Graph, skip: Sequence[str] = ()) -> dict[str, int]:
    """The pass pipeline in its order, leaving out the passes named in
    `skip` (their count is 0)."""
    bad = set(skip) - set(PASSES)
    if bad:
        raise HipError(L.ERR_ARG, f"unknown pass(es): {sorted(bad)}")
    if not skip:
        return g.optimize()
    return {p: (0 if p in skip else g.run_pass(p)) for p in PASSES}


class OnnxDecoder:
    """Greedy decode over an exported GPT-2 with-past graph (`inferc decode`,
    src/cli/main.cpp:700-936) with the KV cache on the device.

    The reference runs two graphs and, between steps, renames every
    present.* output to the next step's past_key_values.* input (main.cpp:
    831-836, 883-888), so each step copies the whole cache through the host.
    Here the pass pipeline turns each layer's attention into a
    FusedAttentionPast node, the executor keeps its K/V in a device cache
    (bind_kv_cache), and each step passes the past inputs by shape only: the
    prompt is the first step (past length 0), then one token per step.
    Argmax (first maximum, main.cpp:875-879) runs on the device."""

    # the passes `inferc decode --no-fold` leaves out (main.cpp:756-775)
    FOLD_PASSES = ("fold_constant_transpose", "recognize_layernorm", "recognize_gelu_tanh")

    def __init__(self, ctx: Context, with_past, max_t: int, prefill=None, optimize: bool = True,
                 skip_passes: Sequence[str] = ()):
        self.graph = with_past if isinstance(with_past, Graph) else Graph.from_onnx(with_past)
        self.counts = _optimize(self.graph, skip_passes) if optimize else None
        self.prefill_ex = None
        if prefill is not None:
            pg = prefill if isinstance(prefill, Graph) else Graph.from_onnx(prefill)
            if optimize:
                _optimize(pg, skip_passes)
            self.prefill_ex = Executor(ctx, pg)
        d = self.graph.to_dict()
        self.past = [i for i in d["inputs"] if i["name"].startswith("past_key_values.")]
        if not self.past:
            raise HipError(L.ERR_ARG, "graph has no past_key_values.* inputs")
        for i in self.past:
            if len(i["shape"]) != 4 or i["shape"][1] <= 0 or i["shape"][3] <= 0:
                raise HipError(L.ERR_SHAPE, f"{i['name']}: expected [batch, heads, past, head_dim]")
        self.max_t = max_t
        self.ex = Executor(ctx, self.graph)
        self.ex.bind_kv_cache(max_t)

    def _step(self, ids: np.ndarray, total: int, seed=None, profiler=None) -> int:
        self.ex.set_input("input_ids", ids)
        self.ex.set_input("attention_mask", np.ones((1, total), np.int64))
        past = total - ids.shape[1]
        for i in self.past:
            if seed is not None:
                self.ex.set_input_device(i["name"], seed[i["name"]])
            else:
                self.ex.set_input_shape(i["name"], np.float32,
                                        [1, i["shape"][1], past, i["shape"][3]])
        if profiler is not None:
            self.ex.run_profiled(profiler)
        else:
            self.ex.run_async()
        return self.ex.output_argmax("logits")

    def _decode_step(self, tok: int, profiler=None) -> int:
        """One step in the executor's decode mode: only the token changes."""
        self.ex.set_input("input_ids", np.array([[tok]], np.int64))
        if profiler is not None:
            self.ex.run_profiled(profiler)
        else:
            self.ex.run_async()
        return self.ex.output_argmax("logits")

    def _enter_decode(self, length: int) -> None:
        """Decode mode with the caches holding `length` positions: the past
        inputs by shape with length 0, the new position's mask."""
        self.ex.set_decode_position(length, "attention_mask")
        for i in self.past:
            self.ex.set_input_shape(i["name"], np.float32, [1, i["shape"][1], 0, i["shape"][3]])
        self.ex.set_input("attention_mask", np.ones((1, 1), np.int64))

    def generate(self, prompt: np.ndarray, max_tokens: int, profiler=None,
                 step_ms: list | None = None, decode_mode: bool = True) -> np.ndarray:
        """Greedy tokens. With a prefill graph the prompt runs there
        (main.cpp:786-828) and its present.* seed the cache on the first
        step, device to device; without one the prompt is the with-past
        graph's first step. The steps after the prompt (after the first step
        past it with a prefill graph, which seeds the cache) run in the
        executor's decode mode (inferc_executor_set_decode_position), where
        they replay one recorded step back to back, each step's greedy token
        fed back on the device as the next one's input (set_decode_feedback;
        with a profiler, one step at a time through the host instead);
        decode_mode=False walks every step with its grown shapes instead.
        `profiler` records each post-prompt step as one iteration
        (main.cpp:846-872). `step_ms`, when given, receives each post-prompt
        step's time in ms (the step timer of main.cpp:863-872 around Run):
        host wall time for the steps run one at a time, device time between
        HIP events for the fed-back ones."""
        p = np.asarray(prompt, np.int64).reshape(1, -1)
        n = p.shape[1]
        if n + max_tokens - 1 > self.max_t:
            raise HipError(L.ERR_SHAPE, "prompt + generated tokens exceed the KV cache (max_t)")
        seed = None
        if self.prefill_ex is not None:
            pe = self.prefill_ex
            pe.set_input("input_ids", p)
            pe.set_input("attention_mask", np.ones((1, n), np.int64))
            pe.run_async()
            toks = [pe.output_argmax("logits")]
            seed = {i["name"]: pe.output_device(i["name"].replace("past_key_values.", "present."))
                    for i in self.past}
        else:
            toks = [self._step(p, n)]
        self.ex.set_decode_position(-1)
        # the first step in decode mode: the one after the prompt, or with a
        # prefill graph the one after the step that seeds the cache
        first = 1 if seed is None else 2
        if decode_mode and first == 1 and max_tokens > 1:
            self._enter_decode(n)
        for k in range(1, max_tokens):
            t0 = time.perf_counter()
            if decode_mode and k >= first and profiler is None:
                # the remaining steps on the device, each one's token fed back
                # as the next one's input; per-step device times by events
                self.ex.set_decode_feedback("logits", "input_ids", toks[-1])
                ms = self.ex.run_steps(max_tokens - k, timed=True)
                toks.extend(int(t) for t in self.ex.decode_tokens(n + k, max_tokens - k))
                if step_ms is not None:
                    step_ms.extend(ms)
                break
            if decode_mode and k >= first:
                toks.append(self._decode_step(toks[-1], profiler))
            else:
                toks.append(self._step(np.array([[toks[-1]]], np.int64), n + k, seed=seed,
                                       profiler=profiler))
                if decode_mode and k + 1 < max_tokens:
                    self._enter_decode(n + k)  # the caches now hold n + k positions
            if step_ms is not None:
                step_ms.append((time.perf_counter() - t0) * 1e3)
            seed = None
        self.ex.set_decode_position(-1)
        return np.array(toks, np.int64)

    def logits(self) -> np.ndarray:
        return self.ex.output("logits")

    def close(self) -> None:
        """Frees the executors (weights, arena, KV caches)."""
        for ex in (self.ex, self.prefill_ex):
            if ex is not None:
                ex.close()
        self.prefill_ex = None


class Gpt2Config(C.Structure):
    _fields_ = [("layers", C.c_int64), ("hidden", C.c_int64), ("heads", C.c_int64),
                ("ffn", C.c_int64), ("vocab", C.c_int64), ("max_pos", C.c_int64),
                ("eps", C.c_float)]


class Gpt2Decoder:
    """Greedy decode with a device KV cache (`inferc decode`,
    src/cli/main.cpp:700-936). `weights` follows the order documented in
    include/inferc_hip.h (fp32 numpy arrays)."""

    def __init__(self, ctx: Context, cfg: dict, weights: Sequence[np.ndarray], max_t: int):
        self.ctx = ctx
        self.cfg = cfg
        self._w = [_c_order(w, np.float32) for w in weights]
        ptrs = (C.c_void_p * len(self._w))(*[w.ctypes.data for w in self._w])
        c = Gpt2Config(cfg["layers"], cfg["hidden"], cfg["heads"], cfg["ffn"], cfg["vocab"],
                       cfg["max_pos"], cfg["eps"])
        h = C.c_void_p()
        check(ctx._lib.inferc_gpt2_create(ctx.handle, C.byref(c), ptrs, max_t, C.byref(h)))
        self.handle = h.value
        self._w = None  # uploaded; host copies no longer needed

    def generate(self, prompt: np.ndarray, max_tokens: int, want_step_ms: bool = False,
                 want_logits: bool = False):
        p = _c_order(prompt, np.int64)
        toks = np.empty(max_tokens, np.int64)
        steps = np.empty(max(1, max_tokens - 1), np.float32) if want_step_ms else None
        logits = np.empty(self.cfg["vocab"], np.float32) if want_logits else None
        fp = C.POINTER(C.c_float)
        check(self.ctx._lib.inferc_gpt2_generate(
            self.handle, p.ctypes.data_as(C.POINTER(C.c_int64)), p.size, max_tokens,
            toks.ctypes.data_as(C.POINTER(C.c_int64)),
            steps.ctypes.data_as(fp) if steps is not None else None,
            logits.ctypes.data_as(fp) if logits is not None else None))
        return toks, (steps[:max_tokens - 1] if steps is not None else None), logits

    def generate_profiled(self, prompt: np.ndarray, max_tokens: int, profiler) -> np.ndarray:
        """generate() with every decode step recorded as one profiler
        iteration of fused launch groups (main.cpp:846-872); the steps run
        eagerly, so their totals include launch overhead that the replayed
        step graph of generate() avoids. Returns the tokens."""
        p = _c_order(prompt, np.int64)
        toks = np.empty(max_tokens, np.int64)
        check(self.ctx._lib.inferc_gpt2_generate_profiled(
            self.handle, p.ctypes.data_as(C.POINTER(C.c_int64)), p.size, max_tokens,
            toks.ctypes.data_as(C.POINTER(C.c_int64)), profiler.handle))
        return toks

    @classmethod
    def from_graph(cls, ctx: Context, graph, max_t: int) -> "Gpt2Decoder":
        """The GPT-2 an exported with-past graph (a Graph or an ONNX path)
        describes, its weights read by parameter name
        (graphs.gpt2_weights_from_graph), on the native decoder."""
        from . import graphs

        own = not isinstance(graph, Graph)
        g = Graph.from_onnx(graph) if own else graph
        try:
            if not any(n["op"] == "FusedLayerNorm" for n in g.to_dict()["nodes"]):
                g.run_pass("recognize_layernorm")  # the epsilon attribute, for the config
            cfg, w = graphs.gpt2_weights_from_graph(g)
        finally:
            if own:
                g.close()
        return cls(ctx, cfg, w, max_t)

    def use_int4(self) -> None:
        """int4 weight-only decode (irreversible): see inferc_gpt2_use_int4."""
        check(self.ctx._lib.inferc_gpt2_use_int4(self.handle))

    def forward(self, ids: np.ndarray) -> np.ndarray:
        i = _c_order(ids, np.int64)
        out = np.empty((i.size, self.cfg["vocab"]), np.float32)
        check(self.ctx._lib.inferc_gpt2_forward(self.handle, i.ctypes.data_as(C.POINTER(C.c_int64)),
                                                i.size,
                                                out.ctypes.data_as(C.POINTER(C.c_float))))
        return out

    def close(self) -> None:
        if getattr(self, "handle", None):
            self.ctx._lib.inferc_gpt2_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
