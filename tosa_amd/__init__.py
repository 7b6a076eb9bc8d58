"""tosa_amd: the MI355X execution path of a TOSA graph interpreter.

Python face of `libtosa_mi355x.so` (C ABI in `include/tosa_mi355x.h`),
mirroring the reference crate's public API (src/lib.rs:1-43):
`run_graph`, `run_graph_with_stats`, `run_graph_with_hooks`, `Interpreter`,
`Tensor`, and the hooks `InterpreterHook`, `HookSet`, `StatsCollector`,
`FlopCounter`, `OpTrace`, `NoopHook`. Every operator runs as a gfx950 kernel;
there is no host fallback, and importing fails loudly when the library has
not been built.
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

from . import _lib
from ._lib import DTYPE_CODE, DTYPE_NAME, OP_NAME, TosaError, check, lib  # noqa: F401

__all__ = [
    "Tensor", "Interpreter", "run_graph", "run_graph_with_stats", "run_graph_with_hooks",
    "InterpreterHook", "HookSet", "StatsCollector", "FlopCounter", "OpTrace", "NoopHook",
    "TosaError", "set_option", "get_option", "set_stream", "synchronize", "device_count",
]

# Element storage of each TOSA type on the host side of the ABI.
_NP_STORAGE = {
    "BOOL": np.uint8, "INT4": np.int8, "INT8": np.int8, "INT16": np.int16, "INT32": np.int32,
    "INT48": np.int64, "INT64": np.int64, "SHAPE": np.int64, "FP32": np.float32, "FP16": np.uint16,
    "BF16": np.uint16, "FP8E4M3": np.uint8, "FP8E5M2": np.uint8,
}


def _np_storage(dtype: str):
    try:
        return _NP_STORAGE[dtype]
    except KeyError:
        raise TosaError(4, f"no host storage for dtype {dtype}") from None


class Tensor:
    """A named, shaped tensor held in GPU memory (src/tensor.rs:228-250)."""

    __slots__ = ("_h", "_owned", "_keep")

    def __init__(self, handle, owned=True, keep=None):
        self._h = handle
        self._owned = owned
        self._keep = keep

    @classmethod
    def from_numpy(cls, name: str, array, dtype: str) -> "Tensor":
        """Copy host elements. `array` holds the element storage of `dtype`
        (BF16/FP16 as uint16 bit patterns are also accepted as float16 for FP16)."""
        a = np.asarray(array)
        st = _np_storage(dtype)
        if dtype == "FP16" and a.dtype == np.float16:
            a = a.view(np.uint16)
        a = a.astype(st, copy=False)
        if not a.flags.c_contiguous:
            a = a.copy(order="C")  # keeps rank 0, unlike np.ascontiguousarray
        shape = (ctypes.c_int64 * max(1, a.ndim))(*a.shape)
        h = ctypes.c_void_p()
        check(lib().tosa_tensor_from_host(name.encode(), shape, a.ndim, DTYPE_CODE[dtype],
                                          a.ctypes.data_as(ctypes.c_void_p), a.nbytes, ctypes.byref(h)))
        return cls(h)

    @classmethod
    def from_device(cls, name: str, shape, dtype: str, ptr: int, nbytes: int, keep=None) -> "Tensor":
        """Wrap device memory (e.g. a torch tensor's data_ptr()) without a copy;
        `keep` is held to keep the owner alive."""
        shape = tuple(int(d) for d in shape)
        s = (ctypes.c_int64 * max(1, len(shape)))(*shape)
        h = ctypes.c_void_p()
        check(lib().tosa_tensor_from_device(name.encode(), s, len(shape), DTYPE_CODE[dtype],
                                            ctypes.c_void_p(ptr), nbytes, ctypes.byref(h)))
        return cls(h, keep=keep)

    # The library module is bound as a default argument: at interpreter exit
    # module globals may already be cleared when the last objects go.
    def __del__(self, _l=_lib):
        if getattr(self, "_owned", False) and self._h and _l.loaded():
            _l.lib().tosa_tensor_free(self._h)
            self._h = None

    @property
    def name(self) -> str:
        return lib().tosa_tensor_name(self._h).decode()

    @property
    def dtype(self) -> str:
        return DTYPE_NAME[lib().tosa_tensor_dtype(self._h)]

    @property
    def shape(self) -> list:
        r = lib().tosa_tensor_rank(self._h)
        dims = (ctypes.c_int64 * max(1, r))()
        check(lib().tosa_tensor_shape(self._h, dims, r))
        return [int(dims[i]) for i in range(r)]

    def element_count(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return max(1, n)

    def size_bytes(self) -> int:
        return lib().tosa_tensor_size_bytes(self._h)

    def device_ptr(self) -> int:
        p = ctypes.c_void_p()
        check(lib().tosa_tensor_device_ptr(self._h, ctypes.byref(p)))
        return p.value or 0

    def numpy(self) -> np.ndarray:
        """The elements in their host storage format (synchronises)."""
        st = _np_storage(self.dtype)
        shape = self.shape
        out = np.empty(shape, dtype=st)
        check(lib().tosa_tensor_to_host(self._h, out.ctypes.data_as(ctypes.c_void_p), out.nbytes))
        return out

    def __repr__(self):
        return f"Tensor({self.name!r}, {self.dtype}, {self.shape})"


# ---------------------------------------------------------------------------
# Hooks (src/stats.rs)
# ---------------------------------------------------------------------------

class _Hook:
    """Owner of a native hook handle."""

    _handle = None
    _borrowed = False

    def _native(self):
        return self._handle

    def __del__(self, _l=_lib):
        if self._handle and not self._borrowed and _l.loaded():
            _l.lib().tosa_hook_free(self._handle)
            self._handle = None


class NoopHook(_Hook):
    def __init__(self):
        self._handle = lib().tosa_hook_new_noop()


class StatsCollector(_Hook):
    """Per-operator counts, host-timed durations and element counts; peak memory."""

    def __init__(self, handle=None):
        self._handle = handle or lib().tosa_hook_new_stats()

    @property
    def total_ops_executed(self) -> int:
        return lib().tosa_stats_total_ops(self._handle)

    @property
    def peak_memory_bytes(self) -> int:
        return lib().tosa_stats_peak_memory(self._handle)

    @property
    def current_memory_bytes(self) -> int:
        return lib().tosa_stats_current_memory(self._handle)

    @property
    def op_stats(self) -> dict:
        out = {}
        L = lib()
        for i in range(L.tosa_stats_num_ops(self._handle)):
            name = ctypes.c_char_p()
            cnt, tin, tout = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
            sec = ctypes.c_double()
            check(L.tosa_stats_op(self._handle, i, ctypes.byref(name), ctypes.byref(cnt), ctypes.byref(sec),
                                  ctypes.byref(tin), ctypes.byref(tout)))
            out[name.value.decode()] = {"count": cnt.value, "total_time": sec.value,
                                        "total_input_elements": tin.value, "total_output_elements": tout.value}
        return out

    def summary(self) -> str:
        L = lib()
        n = L.tosa_stats_summary(self._handle, None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        L.tosa_stats_summary(self._handle, buf, n + 1)
        return buf.value.decode()


class FlopCounter(_Hook):
    def __init__(self):
        self._handle = lib().tosa_hook_new_flops()

    @property
    def total_flops(self) -> int:
        return lib().tosa_flops_total(self._handle)

    def flops_for(self, op: str) -> int:
        return lib().tosa_flops_for(self._handle, op.encode())


class OpTrace(_Hook):
    def __init__(self):
        self._handle = lib().tosa_hook_new_trace()

    @property
    def entries(self) -> list:
        L = lib()
        out = []
        for i in range(L.tosa_trace_len(self._handle)):
            op = ctypes.c_char_p()
            idx, ni, no = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
            check(L.tosa_trace_entry(self._handle, i, ctypes.byref(op), ctypes.byref(idx), ctypes.byref(ni),
                                     ctypes.byref(no)))

            def shapes(which, count):
                res = []
                for j in range(count):
                    dims = (ctypes.c_int64 * 8)()
                    r = ctypes.c_int()
                    check(L.tosa_trace_shape(self._handle, i, which, j, dims, 8, ctypes.byref(r)))
                    res.append([int(dims[k]) for k in range(r.value)])
                return res

            out.append({"op": op.value.decode(), "op_index": idx.value,
                        "input_shapes": shapes(0, ni.value), "output_shapes": shapes(1, no.value), "elapsed": 0.0})
        return out


class InterpreterHook(_Hook):
    """Base class for user hooks: override pre_op / post_op / on_tensor_alloc /
    on_tensor_free. Tensor arguments are `Tensor` views valid during the call.
    Set `needs_sync` to see each operator's kernels finished in post_op, and
    `reads_data` if the hook reads tensor values (this disables fusion)."""

    needs_sync = False
    reads_data = False

    def __init__(self):
        cb = _lib.HookCallbacks()

        def views(ptr, n):
            return [Tensor(ctypes.c_void_p(ptr[i]), owned=False) for i in range(n)]

        self._cbs = (
            _lib.PRE_OP(lambda u, op, idx, ins, n: self.pre_op(op, idx, views(ins, n))),
            _lib.POST_OP(lambda u, op, idx, ins, ni, outs, no: self.post_op(op, idx, views(ins, ni), views(outs, no))),
            _lib.ON_ALLOC(lambda u, name, shape, rank, dt, b: self.on_tensor_alloc(
                name.decode(), [shape[i] for i in range(rank)], DTYPE_NAME[dt], b)),
            _lib.ON_FREE(lambda u, name, b: self.on_tensor_free(name.decode(), b)),
        )
        cb.pre_op, cb.post_op, cb.on_tensor_alloc, cb.on_tensor_free = self._cbs
        cb.needs_sync = int(self.needs_sync)
        cb.reads_data = int(self.reads_data)
        self._handle = lib().tosa_hook_new_callbacks(ctypes.byref(cb))

    def pre_op(self, op: int, op_index: int, inputs: list):
        pass

    def post_op(self, op: int, op_index: int, inputs: list, outputs: list):
        pass

    def on_tensor_alloc(self, name: str, shape: list, dtype: str, nbytes: int):
        pass

    def on_tensor_free(self, name: str, nbytes: int):
        pass


class HookSet(_Hook):
    """Dispatches to every added hook, in insertion order (src/stats.rs:19-76)."""

    def __init__(self):
        self._handle = lib().tosa_hook_new_set()
        self._members = []

    def add(self, hook: _Hook):
        check(lib().tosa_hookset_add(self._handle, hook._handle))
        hook._borrowed = True
        self._members.append(hook)  # keeps Python callbacks alive

    def hooks(self) -> list:
        return list(self._members)


# ---------------------------------------------------------------------------
# Interpreter (src/interpreter.rs:104-148) and the convenience API
# ---------------------------------------------------------------------------

def _inputs(inputs):
    if isinstance(inputs, dict):
        inputs = list(inputs.values())
    arr = (ctypes.c_void_p * max(1, len(inputs)))(*[t._h for t in inputs])
    return arr, len(inputs), list(inputs)


def _outputs(ptr, n):
    res = {}
    arr = ctypes.cast(ptr, ctypes.POINTER(ctypes.c_void_p))
    for i in range(n):
        t = Tensor(ctypes.c_void_p(arr[i]))
        res[t.name] = t
    # free only the array: the handles now belong to the Tensor objects
    lib().tosa_outputs_array_free(ptr)
    return res


class Interpreter:
    def __init__(self, handle):
        self._h = handle

    @classmethod
    def from_flatbuffer(cls, data: bytes) -> "Interpreter":
        h = ctypes.c_void_p()
        buf = (ctypes.c_uint8 * max(1, len(data))).from_buffer_copy(bytes(data) or b"\0")
        check(lib().tosa_graph_from_flatbuffer(buf, len(data), ctypes.byref(h)))
        return cls(h)

    def __del__(self, _l=_lib):
        if getattr(self, "_h", None) and _l.loaded():
            _l.lib().tosa_graph_free(self._h)
            self._h = None

    def graph(self) -> dict:
        """The main block: operators (code, name, inputs, outputs), tensors, inputs, outputs."""
        L = lib()
        ops = []
        for i in range(L.tosa_graph_num_operators(self._h)):
            code, ni, no = ctypes.c_uint32(), ctypes.c_size_t(), ctypes.c_size_t()
            check(L.tosa_graph_operator(self._h, i, ctypes.byref(code), ctypes.byref(ni), ctypes.byref(no)))
            ops.append({"op": code.value, "name": OP_NAME(code.value),
                        "inputs": [L.tosa_graph_operator_input(self._h, i, j).decode() for j in range(ni.value)],
                        "outputs": [L.tosa_graph_operator_output(self._h, i, j).decode() for j in range(no.value)]})
        tensors = []
        for i in range(L.tosa_graph_num_tensors(self._h)):
            name = ctypes.c_char_p()
            dt = ctypes.c_uint32()
            shape = (ctypes.c_int32 * 16)()
            rank, has = ctypes.c_int(), ctypes.c_int()
            check(L.tosa_graph_tensor(self._h, i, ctypes.byref(name), ctypes.byref(dt), shape, 16, ctypes.byref(rank),
                                      ctypes.byref(has)))
            tensors.append({"name": name.value.decode(), "dtype": DTYPE_NAME.get(dt.value, "UNKNOWN"),
                            "shape": [shape[k] for k in range(rank.value)], "has_data": bool(has.value)})
        return {
            "operators": ops, "tensors": tensors,
            "inputs": [L.tosa_graph_input(self._h, i).decode() for i in range(L.tosa_graph_num_inputs(self._h))],
            "outputs": [L.tosa_graph_output(self._h, i).decode() for i in range(L.tosa_graph_num_outputs(self._h))],
        }

    def run(self, inputs, hook: _Hook | None = None) -> dict:
        arr, n, _keep = _inputs(inputs)
        out = ctypes.c_void_p()
        nout = ctypes.c_size_t()
        check(lib().tosa_run(self._h, arr, n, hook._native() if hook else None, ctypes.byref(out),
                             ctypes.byref(nout)))
        return _outputs(out, nout.value)


def _graph_buf(data: bytes):
    return (ctypes.c_uint8 * max(1, len(data))).from_buffer_copy(bytes(data) or b"\0")


def run_graph(data: bytes, inputs) -> dict:
    """src/lib.rs:20-24"""
    arr, n, _keep = _inputs(inputs)
    out, nout = ctypes.c_void_p(), ctypes.c_size_t()
    check(lib().tosa_run_graph(_graph_buf(data), len(data), arr, n, ctypes.byref(out), ctypes.byref(nout)))
    return _outputs(out, nout.value)


def run_graph_with_stats(data: bytes, inputs):
    """src/lib.rs:26-34: (outputs, StatsCollector)"""
    arr, n, _keep = _inputs(inputs)
    out, nout, st = ctypes.c_void_p(), ctypes.c_size_t(), ctypes.c_void_p()
    check(lib().tosa_run_graph_with_stats(_graph_buf(data), len(data), arr, n, ctypes.byref(out),
                                          ctypes.byref(nout), ctypes.byref(st)))
    return _outputs(out, nout.value), StatsCollector(st)


def run_graph_with_hooks(data: bytes, inputs, hooks: _Hook) -> dict:
    """src/lib.rs:36-43"""
    arr, n, _keep = _inputs(inputs)
    out, nout = ctypes.c_void_p(), ctypes.c_size_t()
    check(lib().tosa_run_graph_with_hooks(_graph_buf(data), len(data), arr, n, hooks._native(), ctypes.byref(out),
                                          ctypes.byref(nout)))
    return _outputs(out, nout.value)


def set_option(key: str, value: int):
    check(lib().tosa_set_option(key.encode(), int(value)))


def get_option(key: str) -> int:
    return lib().tosa_get_option(key.encode())


def set_stream(stream_ptr: int | None):
    """Run this thread's work on a HIP stream (e.g. torch.cuda.current_stream().cuda_stream)."""
    check(lib().tosa_set_stream(ctypes.c_void_p(stream_ptr or 0)))


def conv2d_i8(x_ptr, x_shape, w_ptr, w_shape, bias_ptr, bias_len, input_zp=0, weight_zp=0, pad=(0, 0, 0, 0),
              stride=(1, 1), dilation=(1, 1), rescale=None, out_ptr=0, device_error=0, stream=0, no_alloc=False):
    """Op-level int8 CONV2D on device buffers (tosa_conv2d_i8): x NHWC and w
    OHWI int8, bias int32, out NHWC (int32, or the rescale's type), given as
    device addresses; returns the output shape. `rescale` is None or a dict
    with multiplier, shift (sequences of 1 or OC values), double_round,
    output_dtype ("INT8"/"INT16"/"INT32"), output_zp and optional clamp
    (lo, hi). Enqueued on `stream` (0: this thread's stream); REQUIRE
    failures go to the device word at `device_error` (0: the stream's own,
    reported by synchronize()). `no_alloc`: tosa_conv2d_i8_noalloc (workspace in
    the per-GPU static array; `stream` 0 is then HIP's null stream)."""
    xs = (ctypes.c_int64 * 4)(*x_shape)
    ws = (ctypes.c_int64 * 4)(*w_shape)
    pd = (ctypes.c_int32 * 4)(*pad)
    st = (ctypes.c_int32 * 2)(*stride)
    dl = (ctypes.c_int32 * 2)(*dilation)
    os_ = (ctypes.c_int64 * 4)()
    keep = []
    rs_p = _rescale_arg(rescale, keep)
    fn = lib().tosa_conv2d_i8_noalloc if no_alloc else lib().tosa_conv2d_i8
    check(fn(ctypes.c_void_p(x_ptr), xs, ctypes.c_void_p(w_ptr), ws, ctypes.c_void_p(bias_ptr), int(bias_len),
             int(input_zp), int(weight_zp), pd, st, dl, rs_p, ctypes.c_void_p(out_ptr), os_,
             ctypes.c_void_p(device_error or 0), ctypes.c_void_p(stream or 0)))
    del keep
    return tuple(os_)


def _rescale_arg(rescale, keep):
    if rescale is None:
        return None
    m = np.ascontiguousarray(np.asarray(rescale["multiplier"], dtype=np.int32).reshape(-1))
    sh = np.ascontiguousarray(np.asarray(rescale["shift"], dtype=np.int8).reshape(-1))
    keep += [m, sh]
    clamp = rescale.get("clamp")
    rs = _lib.RescaleI32(m.ctypes.data, sh.ctypes.data, len(m), int(bool(rescale.get("double_round", True))),
                         DTYPE_CODE[rescale.get("output_dtype", "INT8")], int(rescale.get("output_zp", 0)),
                         int(clamp is not None), int(clamp[0]) if clamp else 0, int(clamp[1]) if clamp else 0)
    return ctypes.pointer(rs)


def matmul_i8(a_ptr, a_shape, b_ptr, b_shape, a_zp=0, b_zp=0, rescale=None, out_ptr=0, device_error=0, stream=0):
    """Op-level int8 MATMUL on device buffers (tosa_matmul_i8): a [N,H,C] and
    b [N,C,W] int8, out [N,H,W] (int32, or the rescale's type), given as
    device addresses; returns the output shape. `rescale` as for conv2d_i8
    (1 or W multiplier/shift values); `device_error` and `stream` as there."""
    as_ = (ctypes.c_int64 * 3)(*a_shape)
    bs = (ctypes.c_int64 * 3)(*b_shape)
    os_ = (ctypes.c_int64 * 3)()
    keep = []
    rs_p = _rescale_arg(rescale, keep)
    check(lib().tosa_matmul_i8(ctypes.c_void_p(a_ptr), as_, ctypes.c_void_p(b_ptr), bs, int(a_zp), int(b_zp), rs_p,
                               ctypes.c_void_p(out_ptr), os_, ctypes.c_void_p(device_error or 0),
                               ctypes.c_void_p(stream or 0)))
    del keep
    return tuple(os_)


def synchronize():
    check(lib().tosa_synchronize())


def device_count() -> int:
    return lib().tosa_device_count()
