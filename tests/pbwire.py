"""Minimal ONNX protobuf writer and reader for the tests, written from the
protobuf encoding spec and onnx.proto's field numbers, independently of the
library's C++ reader: models built here check the reader, and the reader's
view of exported models is checked against the decoder here.

Writer: `model(graph(...), ...)` with `node`, `tensor`, `value_info`, `attr_*`
helpers returns serialized ModelProto bytes. Reader: `decode_graph(bytes)`
returns node op types, node count and initializer bytes.
"""
from __future__ import annotations

import struct

import numpy as np

# TensorProto.DataType
FLOAT, UINT8, INT8, INT32, INT64, BOOL, DOUBLE = 1, 2, 3, 6, 7, 9, 11
_NP = {np.dtype(np.float32): FLOAT, np.dtype(np.uint8): UINT8, np.dtype(np.int8): INT8,
       np.dtype(np.int32): INT32, np.dtype(np.int64): INT64, np.dtype(np.bool_): BOOL,
       np.dtype(np.float64): DOUBLE}


def varint(v: int) -> bytes:
    v &= (1 << 64) - 1  # negative int64 -> two's complement, 10 bytes
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def key(field: int, wire: int) -> bytes:
    return varint(field << 3 | wire)


def f_varint(field: int, v: int) -> bytes:
    return key(field, 0) + varint(v)


def f_bytes(field: int, b: bytes | str) -> bytes:
    if isinstance(b, str):
        b = b.encode()
    return key(field, 2) + varint(len(b)) + b


def f_float(field: int, x: float) -> bytes:
    return key(field, 5) + struct.pack("<f", x)


def f_packed_varints(field: int, vals) -> bytes:
    return f_bytes(field, b"".join(varint(int(v)) for v in vals))


def tensor(name: str, arr=None, dtype=None, dims=None, typed: bool = False,
           packed: bool = True) -> bytes:
    """TensorProto: raw_data by default; `typed` stores float_data /
    int32_data / int64_data / double_data instead (packed or one record per
    value)."""
    a = np.asarray(arr)
    dt = dtype if dtype is not None else _NP[a.dtype]
    out = b""
    for d in (a.shape if dims is None else dims):
        out += f_varint(1, d)
    out += f_varint(2, dt) + f_bytes(8, name)
    if not typed:
        return out + f_bytes(9, np.ascontiguousarray(a).tobytes())
    flat = a.reshape(-1)
    if dt == FLOAT:
        if packed:
            return out + f_bytes(4, flat.astype("<f4").tobytes())
        return out + b"".join(f_float(4, float(x)) for x in flat)
    if dt == DOUBLE:
        return out + f_bytes(10, flat.astype("<f8").tobytes())
    field = 7 if dt == INT64 else 5
    vals = [int(x) for x in flat]
    if packed:
        return out + f_packed_varints(field, vals)
    return out + b"".join(f_varint(field, v) for v in vals)


def attr_int(name: str, v: int) -> bytes:
    return f_bytes(1, name) + f_varint(20, 2) + f_varint(3, v)


def attr_float(name: str, v: float) -> bytes:
    return f_bytes(1, name) + f_varint(20, 1) + f_float(2, v)


def attr_ints(name: str, vals) -> bytes:
    return f_bytes(1, name) + f_varint(20, 7) + f_packed_varints(8, vals)


def attr_floats(name: str, vals) -> bytes:
    return f_bytes(1, name) + f_varint(20, 6) + b"".join(f_float(7, float(v)) for v in vals)


def attr_string(name: str, s: str) -> bytes:
    return f_bytes(1, name) + f_varint(20, 3) + f_bytes(4, s)


def attr_tensor(name: str, t: bytes) -> bytes:
    return f_bytes(1, name) + f_varint(20, 4) + f_bytes(5, t)


def node(op: str, inputs, outputs, name: str = "", attrs=(), domain: str = "") -> bytes:
    out = b"".join(f_bytes(1, i) for i in inputs) + b"".join(f_bytes(2, o) for o in outputs)
    if name:
        out += f_bytes(3, name)
    out += f_bytes(4, op)
    out += b"".join(f_bytes(5, a) for a in attrs)
    if domain:
        out += f_bytes(7, domain)
    return out


def value_info(name: str, elem: int, dims) -> bytes:
    """ValueInfoProto with a tensor type; a str dim is a dim_param."""
    shape = b""
    for d in dims:
        dim = f_bytes(2, d) if isinstance(d, str) else f_varint(1, d)
        shape += f_bytes(1, dim)
    tt = f_varint(1, elem) + f_bytes(2, shape)
    return f_bytes(1, name) + f_bytes(2, f_bytes(1, tt))


def graph(name: str, nodes=(), inits=(), inputs=(), outputs=()) -> bytes:
    return (b"".join(f_bytes(1, n) for n in nodes) + f_bytes(2, name) +
            b"".join(f_bytes(5, t) for t in inits) + b"".join(f_bytes(11, i) for i in inputs) +
            b"".join(f_bytes(12, o) for o in outputs))


def model(g: bytes | None, ir_version: int = 7, producer: str = "", producer_version: str = "",
          opset: int = 13) -> bytes:
    out = f_varint(1, ir_version)
    if producer:
        out += f_bytes(2, producer)
    if producer_version:
        out += f_bytes(3, producer_version)
    if g is not None:
        out += f_bytes(7, g)
    out += f_bytes(8, f_bytes(1, "") + f_varint(2, opset))
    return out


# ------------------------------------------------------------------ reader

def _fields(b: bytes):
    i, n = 0, len(b)
    while i < n:
        k, i = _read_varint(b, i)
        f, w = k >> 3, k & 7
        if w == 0:
            v, i = _read_varint(b, i)
        elif w == 1:
            v, i = b[i:i + 8], i + 8
        elif w == 5:
            v, i = b[i:i + 4], i + 4
        elif w == 2:
            ln, i = _read_varint(b, i)
            v, i = b[i:i + ln], i + ln
        else:
            raise ValueError(f"wire type {w}")
        yield f, w, v


def _read_varint(b: bytes, i: int):
    r = s = 0
    while True:
        c = b[i]
        i += 1
        r |= (c & 0x7F) << s
        s += 7
        if c < 0x80:
            return r, i


_ELEM = {1: 4, 2: 1, 3: 1, 4: 2, 5: 2, 6: 4, 7: 8, 9: 1, 10: 2, 11: 8, 12: 4, 13: 8, 16: 2}


def decode_graph(model_bytes: bytes) -> dict:
    """Node op types in order, and initializer count / total bytes (dims x
    element size, as the loader's summary counts them)."""
    g = next(v for f, w, v in _fields(model_bytes) if f == 7)
    ops, n_init, init_bytes = [], 0, 0
    for f, w, v in _fields(g):
        if f == 1:
            ops.append(next(v2.decode() for f2, w2, v2 in _fields(v) if f2 == 4))
        elif f == 5:
            dims, dt = [], 0
            for f2, w2, v2 in _fields(v):
                if f2 == 1 and w2 == 0:
                    dims.append(v2)
                elif f2 == 1 and w2 == 2:
                    j = 0
                    while j < len(v2):
                        d, j = _read_varint(v2, j)
                        dims.append(d)
                elif f2 == 2:
                    dt = v2
            n_init += 1
            init_bytes += int(np.prod(dims, dtype=np.int64)) * _ELEM.get(dt, 0)
    return {"ops": ops, "node_count": len(ops), "initializer_count": n_init,
            "initializer_total_bytes": init_bytes}
