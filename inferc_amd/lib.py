"""ctypes declarations of the C-ABI in ``include/inferc_hip.h``.

Each entry point is declared with its exact argument types so that a wrong
call fails in ctypes rather than on the device. Every function returns an
``inferc_status``; :func:`check` turns a non-zero status into :class:`HipError`
carrying the library's thread-local message (the reference's kernels throw
``std::runtime_error`` with a message, e.g. src/kernels/attention.cc:35-39).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

_PKG = Path(__file__).resolve().parent
_LIB_NAME = "libinferc_hip.so"

OK, ERR_ARG, ERR_SHAPE, ERR_HIP, ERR_OOM, ERR_UNSUPPORTED, ERR_STATE = range(7)
STATUS_NAMES = {
    OK: "OK", ERR_ARG: "ERR_ARG", ERR_SHAPE: "ERR_SHAPE", ERR_HIP: "ERR_HIP",
    ERR_OOM: "ERR_OOM", ERR_UNSUPPORTED: "ERR_UNSUPPORTED", ERR_STATE: "ERR_STATE",
}
ACT_NONE, ACT_GELU_ERF, ACT_GELU_TANH, ACT_RELU = range(4)
C_NONE, C_ROW, C_FULL, C_SCALAR = range(4)
DT_F32, DT_U8, DT_I32, DT_I64, DT_BOOL = 1, 2, 6, 7, 9


class HipError(RuntimeError):
    """A non-zero status from the backend, with its message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(code, code)}: {message}")
        self.code = code
        self.message = message


def library_path() -> Path:
    return Path(os.environ.get("INFERC_HIP_LIB", _PKG / _LIB_NAME))


_lib: C.CDLL | None = None

vp = C.c_void_p
i64 = C.c_int64
i32 = C.c_int
f32 = C.c_float
sz = C.c_size_t
P = C.POINTER

# name -> argtypes (all return int status unless listed in _RESTYPE)
_SIGS = {
    "inferc_hip_abi_version": [],
    "inferc_hip_device_count": [P(i32)],
    "inferc_hip_create": [i32, P(vp)],
    "inferc_hip_destroy": [vp],
    "inferc_hip_reserve_workspace": [vp, sz],
    "inferc_hip_set_gemv_decode": [vp, C.c_int],
    "inferc_hip_gemv_decode_enabled": [vp, P(C.c_int)],
    "inferc_hip_malloc": [vp, sz, P(vp)],
    "inferc_hip_free": [vp, vp],
    "inferc_hip_h2d": [vp, vp, vp, sz],
    "inferc_hip_d2h": [vp, vp, vp, sz],
    "inferc_hip_d2d": [vp, vp, vp, sz],
    "inferc_hip_sync": [vp],
    "inferc_hip_timer_start": [vp],
    "inferc_hip_timer_stop": [vp, P(f32)],
    "inferc_hip_capture_begin": [vp],
    "inferc_hip_capture_end": [vp, P(vp)],
    "inferc_hip_capture_replay": [vp],
    "inferc_hip_capture_destroy": [vp],
    "inferc_hip_gemm_f32": [vp, i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp, i32,
                            i64, vp, i64, i32, vp, i64],
    "inferc_hip_gemm_f32_noalloc": [vp, i32, i32, i64, i64, i64, f32, vp, i64, vp, i64, f32, vp,
                                    i32, i64, vp, i64, i32, vp, i64],
    "inferc_hip_matmul_f32": [vp, i64, i64, i64, i64, vp, i64, vp, i64, vp],
    "inferc_hip_fused_matmul_add_gelu_f32": [vp, i64, i64, i64, vp, vp, vp, vp],
    "inferc_hip_fused_qkv_f32": [vp, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp, vp, vp, vp],
    "inferc_hip_fused_attention_f32": [vp, i64, i64, i64, i64, vp, vp, vp, vp, P(i64), f32, vp],
    "inferc_hip_layernorm_f32": [vp, i64, i64, vp, vp, vp, vp, f32, vp],
    "inferc_hip_activation_f32": [vp, i64, vp, i32, vp],
    "inferc_hip_softmax_f32": [vp, i64, i64, i64, vp, vp],
    "inferc_hip_add_f32": [vp, i64, vp, vp, i64, vp],
    "inferc_hip_gather_f32": [vp, i64, i64, vp, vp, i64, vp, vp],
    "inferc_hip_split_f32": [vp, i64, i64, i64, i64, P(i64), vp, P(vp)],
    "inferc_hip_concat_f32": [vp, i64, i64, i64, P(i64), P(vp), vp],
    "inferc_hip_argmax_f32": [vp, i64, vp, vp],
    "inferc_hip_gemv_f32": [vp, i64, i64, vp, vp, vp, vp, f32, vp, vp, i32, vp],
    "inferc_hip_int4_unpack": [vp, i64, i64, vp, vp, vp],
    "inferc_hip_int4_gemv": [vp, i64, i64, vp, vp, i64, vp, vp],
    "inferc_hip_int4_gemv_grouped": [vp, i64, P(i64), P(i64), P(vp), P(vp), i64, P(vp), P(vp)],
    "inferc_hip_kv_append_attend_f32": [vp, i64, i64, i64, vp, vp, vp, vp, vp, vp, vp],
    "inferc_graph_create": [P(vp)],
    "inferc_graph_destroy": [vp],
    "inferc_graph_add_initializer": [vp, C.c_char_p, i32, i32, P(i64), vp],
    "inferc_graph_add_node": [vp, C.c_char_p, C.c_char_p, i32, P(C.c_char_p), i32,
                              P(C.c_char_p), C.c_char_p],
    "inferc_graph_add_output": [vp, C.c_char_p],
    "inferc_graph_add_input": [vp, C.c_char_p, i32, i32, P(i64)],
    "inferc_graph_add_tensor_attr": [vp, C.c_char_p, i32, i32, P(i64), vp],
    "inferc_graph_to_json": [vp, vp, sz, P(sz)],
    "inferc_graph_get_initializer": [vp, C.c_char_p, P(i32), P(i32), P(i64), vp, sz],
    "inferc_graph_run_pass": [vp, C.c_char_p, P(i32)],
    "inferc_graph_optimize": [vp, P(i32)],
    "inferc_onnx_load": [C.c_char_p, P(vp)],
    "inferc_onnx_load_bytes": [C.c_char_p, sz, P(vp)],
    "inferc_onnx_summary": [C.c_char_p, sz, i32, vp, sz, P(sz)],
    "inferc_onnx_element_bytes": [i32, P(i64)],
    "inferc_executor_create": [vp, vp, P(vp)],
    "inferc_executor_destroy": [vp],
    "inferc_executor_create_dry": [vp, P(vp)],
    "inferc_executor_node_count": [vp, P(i32)],
    "inferc_executor_set_input": [vp, C.c_char_p, i32, i32, P(i64), vp],
    "inferc_executor_set_input_device": [vp, C.c_char_p, i32, i32, P(i64), vp],
    "inferc_executor_run": [vp],
    "inferc_executor_output_info": [vp, C.c_char_p, P(i32), P(i32), P(i64)],
    "inferc_executor_get_output": [vp, C.c_char_p, vp, sz],
    "inferc_executor_set_graph_mode": [vp, i32],
    "inferc_executor_run_profiled": [vp, vp],
    "inferc_executor_bind_kv_cache": [vp, i64],
    "inferc_executor_set_input_shape": [vp, C.c_char_p, i32, i32, P(i64)],
    "inferc_executor_output_argmax": [vp, C.c_char_p, P(i64)],
    "inferc_executor_device_bytes": [vp, P(i64), P(i64), P(i64)],
    "inferc_executor_set_decode_position": [vp, i64, C.c_char_p],
    "inferc_executor_decode_position": [vp, P(i64)],
    "inferc_executor_set_decode_feedback": [vp, C.c_char_p, C.c_char_p, i64],
    "inferc_executor_run_steps": [vp, i64, P(C.c_float)],
    "inferc_executor_decode_tokens": [vp, i64, i64, P(i64)],
    "inferc_executor_output_device": [vp, C.c_char_p, P(vp)],
    "inferc_profiler_create": [P(vp)],
    "inferc_profiler_destroy": [vp],
    "inferc_profiler_begin_iteration": [vp],
    "inferc_profiler_end_iteration": [vp],
    "inferc_profiler_begin_op": [vp, C.c_char_p, C.c_char_p],
    "inferc_profiler_end_op": [vp, i64],
    "inferc_profiler_record_op": [vp, C.c_char_p, C.c_char_p, C.c_double, i64],
    "inferc_profiler_set_track_activation_bytes": [vp, i32],
    "inferc_profiler_snapshot_peak_rss": [vp],
    "inferc_profiler_iteration_count": [vp, P(i64)],
    "inferc_profiler_total_stats": [vp, P(C.c_double)],
    "inferc_profiler_to_json": [vp, C.c_char_p, C.c_char_p, vp, sz, P(sz)],
    "inferc_profile_percentile": [P(C.c_double), i64, C.c_double, P(C.c_double)],
    "inferc_profile_stats": [P(C.c_double), i64, P(C.c_double)],
    "inferc_gpt2_create": [vp, vp, P(vp), i64, P(vp)],
    "inferc_gpt2_destroy": [vp],
    "inferc_gpt2_use_int4": [vp],
    "inferc_int4_quantize_rows": [i64, i64, vp, vp, vp, vp],
    "inferc_gpt2_generate": [vp, P(i64), i64, i64, P(i64), P(f32), P(f32)],
    "inferc_gpt2_forward": [vp, P(i64), i64, P(f32)],
    "inferc_gpt2_generate_profiled": [vp, P(i64), i64, i64, P(i64), vp],
}

EXPORTED = sorted(list(_SIGS) + ["inferc_hip_last_error"])


def load_library() -> C.CDLL:
    """Loads and declares the backend library (once). Raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    path = library_path()
    if not path.exists():
        raise HipError(ERR_STATE, f"{path} is not built; run `python -m inferc_amd.build`")
    lib = C.CDLL(str(path))
    lib.inferc_hip_last_error.restype = C.c_char_p
    lib.inferc_hip_last_error.argtypes = []
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    _lib = lib
    return lib


def last_error() -> str:
    msg = load_library().inferc_hip_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> None:
    if status != OK:
        raise HipError(status, last_error())
