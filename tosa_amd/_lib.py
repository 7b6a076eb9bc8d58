"""ctypes declarations of the C ABI in include/tosa_mi355x.h."""

from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libtosa_mi355x.so")
_LIB = None

# schema/tosa.fbs:26-46
DTYPE_NAMES = [
    "UNKNOWN", "BOOL", "INT4", "INT8", "INT16", "INT32", "INT48", "FP32", "FP16", "BF16", "SHAPE",
    "FP8E4M3", "FP8E5M2", "FP6E2M3", "FP6E3M2", "FP4E2M1", "FP8UE8M0", "INT64", "MXINT8",
]
DTYPE_CODE = {n: i for i, n in enumerate(DTYPE_NAMES)}
DTYPE_NAME = {i: n for i, n in enumerate(DTYPE_NAMES)}

STATUS_NAMES = {
    0: "Ok", 1: "Deserialize", 2: "UnsupportedOp", 3: "TensorNotFound", 4: "DTypeMismatch",
    5: "ShapeMismatch", 6: "Broadcast", 7: "GraphError", 8: "ControlFlow", 9: "Io", 10: "Device",
    11: "InvalidArgument",
}


class TosaError(RuntimeError):
    """An error returned by the library; `kind` is the reference's Error
    variant name (src/error.rs:4-31), or Device / InvalidArgument."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, str(status))
        super().__init__(f"{self.kind}: {message}")


P = ctypes.c_void_p
PRE_OP = ctypes.CFUNCTYPE(None, P, ctypes.c_uint32, ctypes.c_size_t, ctypes.POINTER(P), ctypes.c_size_t)
POST_OP = ctypes.CFUNCTYPE(None, P, ctypes.c_uint32, ctypes.c_size_t, ctypes.POINTER(P), ctypes.c_size_t,
                           ctypes.POINTER(P), ctypes.c_size_t)
ON_ALLOC = ctypes.CFUNCTYPE(None, P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                            ctypes.c_uint32, ctypes.c_size_t)
ON_FREE = ctypes.CFUNCTYPE(None, P, ctypes.c_char_p, ctypes.c_size_t)


class HookCallbacks(ctypes.Structure):
    _fields_ = [
        ("user", P), ("pre_op", PRE_OP), ("post_op", POST_OP), ("on_tensor_alloc", ON_ALLOC),
        ("on_tensor_free", ON_FREE), ("needs_sync", ctypes.c_int), ("reads_data", ctypes.c_int),
    ]


class RescaleI32(ctypes.Structure):
    """tosa_rescale_i32 (include/tosa_mi355x.h)."""
    _fields_ = [
        ("multiplier", P), ("shift", P), ("channels", ctypes.c_int32), ("double_round", ctypes.c_int32),
        ("output_dtype", ctypes.c_uint32), ("output_zp", ctypes.c_int32), ("has_clamp", ctypes.c_int32),
        ("clamp_min", ctypes.c_int32), ("clamp_max", ctypes.c_int32),
    ]


_I64P = ctypes.POINTER(ctypes.c_int64)
_I32P = ctypes.POINTER(ctypes.c_int32)
_CONV2D_I8_ARGS = [P, _I64P, P, _I64P, P, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32, _I32P, _I32P, _I32P,
                   ctypes.POINTER(RescaleI32), P, _I64P, P, P]

# name -> (restype, argtypes); every function declared in include/tosa_mi355x.h
SIGNATURES = {
    "tosa_last_error": (ctypes.c_char_p, []),
    "tosa_op_name": (ctypes.c_char_p, [ctypes.c_uint32]),
    "tosa_dtype_name": (ctypes.c_char_p, [ctypes.c_uint32]),
    "tosa_graph_from_flatbuffer": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(P)]),
    "tosa_graph_free": (None, [P]),
    "tosa_graph_num_operators": (ctypes.c_size_t, [P]),
    "tosa_graph_operator": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint32),
                                           ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]),
    "tosa_graph_operator_input": (ctypes.c_char_p, [P, ctypes.c_size_t, ctypes.c_size_t]),
    "tosa_graph_operator_output": (ctypes.c_char_p, [P, ctypes.c_size_t, ctypes.c_size_t]),
    "tosa_graph_num_tensors": (ctypes.c_size_t, [P]),
    "tosa_graph_tensor": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_char_p),
                                         ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32),
                                         ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]),
    "tosa_graph_num_inputs": (ctypes.c_size_t, [P]),
    "tosa_graph_num_outputs": (ctypes.c_size_t, [P]),
    "tosa_graph_input": (ctypes.c_char_p, [P, ctypes.c_size_t]),
    "tosa_graph_output": (ctypes.c_char_p, [P, ctypes.c_size_t]),
    "tosa_tensor_from_host": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                                             ctypes.c_uint32, P, ctypes.c_size_t, ctypes.POINTER(P)]),
    "tosa_tensor_from_device": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                                               ctypes.c_uint32, P, ctypes.c_size_t, ctypes.POINTER(P)]),
    "tosa_tensor_to_host": (ctypes.c_int, [P, P, ctypes.c_size_t]),
    "tosa_tensor_device_ptr": (ctypes.c_int, [P, ctypes.POINTER(P)]),
    "tosa_tensor_name": (ctypes.c_char_p, [P]),
    "tosa_tensor_dtype": (ctypes.c_uint32, [P]),
    "tosa_tensor_rank": (ctypes.c_int, [P]),
    "tosa_tensor_shape": (ctypes.c_int, [P, ctypes.POINTER(ctypes.c_int64), ctypes.c_int]),
    "tosa_tensor_size_bytes": (ctypes.c_size_t, [P]),
    "tosa_tensor_data_bytes": (ctypes.c_size_t, [P]),
    "tosa_tensor_free": (None, [P]),
    "tosa_hook_new_callbacks": (P, [ctypes.POINTER(HookCallbacks)]),
    "tosa_hook_new_noop": (P, []),
    "tosa_hook_new_stats": (P, []),
    "tosa_hook_new_flops": (P, []),
    "tosa_hook_new_trace": (P, []),
    "tosa_hook_new_set": (P, []),
    "tosa_hookset_add": (ctypes.c_int, [P, P]),
    "tosa_hookset_len": (ctypes.c_size_t, [P]),
    "tosa_hookset_get": (P, [P, ctypes.c_size_t]),
    "tosa_hook_free": (None, [P]),
    "tosa_stats_total_ops": (ctypes.c_uint64, [P]),
    "tosa_stats_peak_memory": (ctypes.c_size_t, [P]),
    "tosa_stats_current_memory": (ctypes.c_size_t, [P]),
    "tosa_stats_num_ops": (ctypes.c_size_t, [P]),
    "tosa_stats_op": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_char_p),
                                     ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_double),
                                     ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    "tosa_stats_summary": (ctypes.c_size_t, [P, ctypes.c_char_p, ctypes.c_size_t]),
    "tosa_flops_total": (ctypes.c_uint64, [P]),
    "tosa_flops_for": (ctypes.c_uint64, [P, ctypes.c_char_p]),
    "tosa_trace_len": (ctypes.c_size_t, [P]),
    "tosa_trace_entry": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(ctypes.c_char_p),
                                        ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t),
                                        ctypes.POINTER(ctypes.c_size_t)]),
    "tosa_trace_shape": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.c_int, ctypes.c_size_t,
                                        ctypes.POINTER(ctypes.c_int64), ctypes.c_int, ctypes.POINTER(ctypes.c_int)]),
    "tosa_run": (ctypes.c_int, [P, ctypes.POINTER(P), ctypes.c_size_t, P, ctypes.POINTER(P),
                                ctypes.POINTER(ctypes.c_size_t)]),
    "tosa_outputs_free": (None, [P, ctypes.c_size_t]),
    "tosa_outputs_array_free": (None, [P]),
    "tosa_run_graph": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(P), ctypes.c_size_t, ctypes.POINTER(P),
                                      ctypes.POINTER(ctypes.c_size_t)]),
    "tosa_run_graph_with_stats": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(P), ctypes.c_size_t,
                                                 ctypes.POINTER(P), ctypes.POINTER(ctypes.c_size_t),
                                                 ctypes.POINTER(P)]),
    "tosa_run_graph_with_hooks": (ctypes.c_int, [P, ctypes.c_size_t, ctypes.POINTER(P), ctypes.c_size_t, P,
                                                 ctypes.POINTER(P), ctypes.POINTER(ctypes.c_size_t)]),
    "tosa_set_option": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int]),
    "tosa_get_option": (ctypes.c_int, [ctypes.c_char_p]),
    "tosa_set_stream": (ctypes.c_int, [P]),
    "tosa_synchronize": (ctypes.c_int, []),
    "tosa_device_count": (ctypes.c_int, []),
    "tosa_conv2d_i8": (ctypes.c_int, _CONV2D_I8_ARGS),
    "tosa_conv2d_i8_noalloc": (ctypes.c_int, _CONV2D_I8_ARGS),
    "tosa_matmul_i8": (ctypes.c_int, [P, ctypes.POINTER(ctypes.c_int64), P, ctypes.POINTER(ctypes.c_int64),
                                      ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(RescaleI32), P,
                                      ctypes.POINTER(ctypes.c_int64), P, P]),
}


def loaded() -> bool:
    return _LIB is not None


def _bind_process_hip_runtime():
    """Make this process use one HIP runtime. PyTorch-ROCm ships its own
    libamdhip64 (soname libamdhip64.so.7, but loaded by torch as
    "libamdhip64.so" from its own directory); if ours were loaded first, a
    later `import torch` would bring in a second runtime and the two would
    contend for the device. Loading torch's copy first, globally, makes this
    library bind to it too (same soname), and torch then reuses the same file."""
    import importlib.util
    spec = importlib.util.find_spec("torch")
    if spec is None or not spec.submodule_search_locations:
        return
    for d in spec.submodule_search_locations:
        hip = os.path.join(d, "lib", "libamdhip64.so")
        if os.path.exists(hip):
            ctypes.CDLL(hip, mode=ctypes.RTLD_GLOBAL)
            return


def lib():
    """The loaded library. Raises if it was not built: there is no fallback."""
    global _LIB
    if _LIB is None:
        _bind_process_hip_runtime()
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m tosa_amd.build` "
                "(the MI355X path has no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(status: int):
    if status != 0:
        raise TosaError(status, lib().tosa_last_error().decode(errors="replace"))


def OP_NAME(code: int) -> str:
    return lib().tosa_op_name(code).decode()
