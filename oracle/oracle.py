"""CPU oracle: ctypes binding of `tosa_oracle.c` and a reference-order graph runner.

TEST INFRASTRUCTURE ONLY. Imported by `tests/`, `__graft_entry__.smoke()` and
`bench.py`'s CPU-baseline leg as the checker; the product package
`tosa_amd/` never imports it.

`run_block()` executes a parsed `.tosa` main block the way the reference
interpreter does (src/interpreter.rs:154-245): a ready queue seeded in
operator order, CONST always ready, a full rescan after each operator. Each
operator's arithmetic is delegated to the C restatement; CLAMP, ADD,
RESHAPE, TRANSPOSE, CONST, IDENTITY, MAX_POOL2D and CAST, which are plain
data movement, a window maximum or one integer/float operation per element,
are restated here with numpy (MATMUL_T as MATMUL on B rearranged).

Values are held widened, as the reference does: every integer type as int64,
every float type as float32 holding a value exactly representable in its
TOSA type, BOOL as bool.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from collections import deque

import numpy as np

try:
    from . import tosa_reader as fb
except ImportError:  # loaded as a top-level module
    import tosa_reader as fb

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB = None

F32, F16, BF16, FP8E4M3, FP8E5M2 = 0, 1, 2, 3, 4
FMT = {"FP32": F32, "FP16": F16, "BF16": BF16, "FP8E4M3": FP8E4M3, "FP8E5M2": FP8E5M2}
FACC = {"FP32": 0, "FP16": 1, "BF16": 2}           # convolution accumulators (accum.rs)
MM_FACC = {"FP32": 0, "FP16": 3, "BF16": 4}        # MATMUL: unrounded product (accum.rs:94-123)
INT_TYPES = ("INT4", "INT8", "INT16", "INT32", "INT48", "INT64", "SHAPE")
FLOAT_TYPES = ("FP32", "FP16", "BF16", "FP8E4M3", "FP8E5M2")
INT_RANGE = {"INT4": (-8, 7), "INT8": (-128, 127), "INT16": (-32768, 32767),
             "INT32": (-(2 ** 31), 2 ** 31 - 1), "INT48": (-(2 ** 47), 2 ** 47 - 1)}
BITS = {"INT8": 8, "INT16": 16, "INT32": 32, "INT48": 48}


class OracleError(RuntimeError):
    """A condition under which the reference returns an error."""


def build():
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _LIB
    if _LIB is None:
        path = os.path.join(_HERE, "liboracle.so")
        if not os.path.exists(path):
            build()
        L = ctypes.CDLL(path)
        P = ctypes.c_void_p
        i32, i64 = ctypes.c_int32, ctypes.c_int64
        L.orc_reciprocal_scale.argtypes = [i32, P]
        L.orc_reciprocal_scale.restype = i32
        L.orc_apply_scale_32.argtypes = [i32, i32, i32, ctypes.c_int, P]
        L.orc_apply_scale_16.argtypes = [i64, ctypes.c_int16, i32, P]
        L.orc_conv2d_int.argtypes = [P, P, P, ctypes.c_int] + [ctypes.c_int] * 7 + [P, P, P, i64, i64, ctypes.c_int, P]
        L.orc_conv2d_float.argtypes = [P, P, P, ctypes.c_int] + [ctypes.c_int] * 7 + [P, P, P, ctypes.c_float,
                                                                                    ctypes.c_float, ctypes.c_int, ctypes.c_int, P]
        L.orc_depthwise_int.argtypes = L.orc_conv2d_int.argtypes
        L.orc_depthwise_float.argtypes = L.orc_conv2d_float.argtypes
        L.orc_matmul_int.argtypes = [P, P] + [ctypes.c_int] * 4 + [i64, i64, ctypes.c_int, P]
        L.orc_matmul_float.argtypes = [P, P] + [ctypes.c_int] * 4 + [ctypes.c_int, P]
        L.orc_avg_pool_int.argtypes = [P] + [ctypes.c_int] * 4 + [P, P, P, i64, i64, i64, i64, P]
        L.orc_avg_pool_float.argtypes = [P] + [ctypes.c_int] * 4 + [P, P, P, ctypes.c_int, P]
        L.orc_rescale.argtypes = [P, i64, P, P, i64] + [ctypes.c_int] * 7 + [i64, i64, P]
        L.orc_conv3d.argtypes = [ctypes.c_int] + [P] * 6 + [ctypes.c_int] * 10 + [P, P, P, i64, i64, ctypes.c_int,
                                                                                 ctypes.c_int, P, P]
        L.orc_transpose_conv2d.argtypes = [ctypes.c_int] + [P] * 6 + [ctypes.c_int] * 8 + [P, P, i64, i64,
                                                                                         ctypes.c_int, ctypes.c_int,
                                                                                         P, P]
        L.orc_encode_array.argtypes = [ctypes.c_int, P, i64, P]
        L.orc_decode_array.argtypes = [ctypes.c_int, P, i64, P]
        L.orc_round_array.argtypes = [ctypes.c_int, P, i64, P]
        _LIB = L
    return _LIB


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------------------
# Codecs
# ---------------------------------------------------------------------------

def decode(dtype: str, raw: np.ndarray) -> np.ndarray:
    """Stored elements of `dtype` (bf16/fp8 as bit patterns) -> widened values."""
    if dtype in INT_TYPES:
        return raw.astype(np.int64)
    if dtype == "BOOL":
        return raw.astype(np.bool_)
    if dtype == "FP32":
        return raw.astype(np.float32)
    src = np.ascontiguousarray(raw.view(np.uint16) if dtype in ("FP16", "BF16") else raw.astype(np.uint8))
    out = np.empty(src.size, dtype=np.float32)
    lib().orc_decode_array(FMT[dtype], _p(src), src.size, _p(out))
    return out.reshape(raw.shape)


def encode(dtype: str, vals: np.ndarray) -> np.ndarray:
    """Widened values -> stored elements of `dtype` (RNE for floats, wrap for ints)."""
    if dtype in ("INT4",):
        return (((vals.astype(np.int64) & 0xF) ^ 0x8) - 0x8).astype(np.int8)
    if dtype in INT_TYPES:
        v = vals.astype(np.int64)
        if dtype == "INT48":
            return ((v << 16) >> 16)
        return v.astype(fb.np_dtype(dtype))
    if dtype == "BOOL":
        return vals.astype(np.bool_)
    v = np.ascontiguousarray(vals, dtype=np.float32)
    if dtype == "FP32":
        return v.copy()
    out = np.empty(v.size, dtype=np.uint16 if dtype in ("FP16", "BF16") else np.uint8)
    lib().orc_encode_array(FMT[dtype], _p(v), v.size, _p(out))
    if dtype == "FP16":
        out = out.view(np.float16)
    return out.reshape(vals.shape)


def round_to(dtype: str, vals: np.ndarray) -> np.ndarray:
    """`round_to` (src/ops/common.rs:100-108) elementwise."""
    v = np.ascontiguousarray(vals, dtype=np.float32)
    if dtype not in FMT or dtype == "FP32":
        return v.copy()
    out = np.empty_like(v)
    lib().orc_round_array(FMT[dtype], _p(v), v.size, _p(out))
    return out


# ---------------------------------------------------------------------------
# Operators (each cites the reference function it restates)
# ---------------------------------------------------------------------------

class T:
    """A tensor: TOSA dtype, shape and widened values (flat)."""

    def __init__(self, dtype, shape, vals):
        self.dtype = dtype
        self.shape = list(shape)
        self.vals = np.ascontiguousarray(vals).reshape(-1)

    def array(self):
        return self.vals.reshape(self.shape) if self.shape else self.vals.reshape(())


def conv2d(x: T, w: T, bias: T, in_zp, w_zp, pad, stride, dilation, acc_type, out_t, depthwise=False) -> T:
    """CONV2D / DEPTHWISE_CONV2D: src/ops/conv.rs:398-500."""
    L = lib()
    n, ih, iw, ic = x.shape
    if depthwise:
        kh, kw, c, m = w.shape
        oc = c * m
    else:
        oc, kh, kw, _ = w.shape
    oh = (ih - 1 + pad[0] + pad[1] - (kh - 1) * dilation[0]) // stride[0] + 1
    ow = (iw - 1 + pad[2] + pad[3] - (kw - 1) * dilation[1]) // stride[1] + 1
    pad_a = np.array(pad, dtype=np.int32)
    st = np.array(stride, dtype=np.int32)
    dl = np.array(dilation, dtype=np.int32)
    count = n * oh * ow * oc
    if acc_type in ("INT32", "INT48"):
        out = np.empty(count, dtype=np.int64)
        xv = np.ascontiguousarray(x.vals, dtype=np.int64)
        wv = np.ascontiguousarray(w.vals, dtype=np.int64)
        bv = np.ascontiguousarray(bias.vals, dtype=np.int64)
        fn = L.orc_depthwise_int if depthwise else L.orc_conv2d_int
        dims = (n, ih, iw, c, m, kh, kw) if depthwise else (n, ih, iw, ic, oc, kh, kw)
        fn(_p(xv), _p(wv), _p(bv), bv.size, *dims, _p(pad_a), _p(st), _p(dl), int(in_zp), int(w_zp),
           0 if acc_type == "INT32" else 1, _p(out))
    else:
        out = np.empty(count, dtype=np.float32)
        xv = np.ascontiguousarray(x.vals, dtype=np.float32)
        wv = np.ascontiguousarray(w.vals, dtype=np.float32)
        bv = np.ascontiguousarray(bias.vals, dtype=np.float32)
        fn = L.orc_depthwise_float if depthwise else L.orc_conv2d_float
        dims = (n, ih, iw, c, m, kh, kw) if depthwise else (n, ih, iw, ic, oc, kh, kw)
        fn(_p(xv), _p(wv), _p(bv), bv.size, *dims, _p(pad_a), _p(st), _p(dl), float(in_zp), float(w_zp),
           FACC[acc_type], FMT[out_t], _p(out))
    return T(out_t, [n, oh, ow, oc], out)


def matmul(a: T, b: T, a_zp, b_zp, out_t) -> T:
    """MATMUL: src/ops/matmul.rs:98-174."""
    L = lib()
    n, h, c = a.shape
    w = b.shape[2]
    if out_t in ("INT32", "INT48"):
        out = np.empty(n * h * w, dtype=np.int64)
        av = np.ascontiguousarray(a.vals, dtype=np.int64)
        bv = np.ascontiguousarray(b.vals, dtype=np.int64)
        L.orc_matmul_int(_p(av), _p(bv), n, h, c, w, int(a_zp), int(b_zp), 0 if out_t == "INT32" else 1, _p(out))
    else:
        av = round_to(out_t, a.vals)   # operands converted to the output type (matmul.rs:160-162)
        bv = round_to(out_t, b.vals)
        out = np.empty(n * h * w, dtype=np.float32)
        L.orc_matmul_float(_p(av), _p(bv), n, h, c, w, MM_FACC[out_t], _p(out))
    return T(out_t, [n, h, w], out)


def _conv_operands(x: T, w: T, bias: T, acc_type):
    """Operand arrays of the C convolutions: the integer branch takes int64
    values, the float one float32 (the accumulator kind and output format
    come from acc_type and the bias type, src/ops/conv.rs:475-496)."""
    if acc_type in ("INT32", "INT48"):
        cast = lambda t: np.ascontiguousarray(t.vals, dtype=np.int64)  # noqa: E731
        return 1, (cast(x), cast(w), cast(bias), None, None, None), 0 if acc_type == "INT32" else 1, 0
    cast = lambda t: np.ascontiguousarray(t.vals, dtype=np.float32)  # noqa: E731
    return 0, (None, None, None, cast(x), cast(w), cast(bias)), FACC[acc_type], FMT[bias.dtype]


def conv3d(x: T, w: T, bias: T, in_zp, w_zp, pad, stride, dilation, acc_type) -> T:
    """CONV3D: src/ops/conv.rs:505-511 (ConvNd with three spatial dimensions,
    :92-181) through eval_conv (:398-500)."""
    L = lib()
    n, id_, ih, iw, ic = x.shape
    oc, kd, kh, kw, _ = w.shape
    ext = lambda i, a, b, k, d, s: (i - 1 + a + b - (k - 1) * d) // s + 1  # noqa: E731
    od = ext(id_, pad[0], pad[1], kd, dilation[0], stride[0])
    oh = ext(ih, pad[2], pad[3], kh, dilation[1], stride[1])
    ow = ext(iw, pad[4], pad[5], kw, dilation[2], stride[2])
    is_int, ops_, kind, fmt = _conv_operands(x, w, bias, acc_type)
    count = n * od * oh * ow * oc
    out_i = np.empty(count, dtype=np.int64) if is_int else None
    out_f = None if is_int else np.empty(count, dtype=np.float32)
    arr = lambda v, t: np.ascontiguousarray(v, dtype=t)  # noqa: E731
    pd, st, dl = arr(pad, np.int32), arr(stride, np.int32), arr(dilation, np.int32)
    L.orc_conv3d(is_int, *[_p(a) if a is not None else None for a in ops_], len(bias.vals), n, id_, ih, iw, ic, oc,
                 kd, kh, kw, _p(pd), _p(st), _p(dl), int(in_zp) if is_int else 0, int(w_zp) if is_int else 0, kind,
                 fmt, _p(out_i) if is_int else None, None if is_int else _p(out_f))
    return T(bias.dtype, [n, od, oh, ow, oc], out_i if is_int else out_f)


def transpose_conv2d(x: T, w: T, bias: T, in_zp, w_zp, out_pad, stride, acc_type) -> T:
    """TRANSPOSE_CONV2D: src/ops/conv.rs:526-532 (Transpose, :268-372) through
    eval_conv (:398-500)."""
    L = lib()
    n, ih, iw, ic = x.shape
    oc, kh, kw, _ = w.shape
    oh = (ih - 1) * stride[0] + out_pad[0] + out_pad[1] + kh
    ow = (iw - 1) * stride[1] + out_pad[2] + out_pad[3] + kw
    is_int, ops_, kind, fmt = _conv_operands(x, w, bias, acc_type)
    count = n * oh * ow * oc
    out_i = np.empty(count, dtype=np.int64) if is_int else None
    out_f = None if is_int else np.empty(count, dtype=np.float32)
    op_ = np.ascontiguousarray(out_pad, dtype=np.int32)
    st = np.ascontiguousarray(stride, dtype=np.int32)
    L.orc_transpose_conv2d(is_int, *[_p(a) if a is not None else None for a in ops_], len(bias.vals), n, ih, iw, ic,
                           oc, kh, kw, _p(op_), _p(st), int(in_zp) if is_int else 0, int(w_zp) if is_int else 0,
                           kind, fmt, _p(out_i) if is_int else None, None if is_int else _p(out_f))
    return T(bias.dtype, [n, oh, ow, oc], out_i if is_int else out_f)


def matmul_t(a: T, b: T, a_zp, b_zp, out_t) -> T:
    """MATMUL_T: src/ops/matmul.rs:180-182, eval (:98-174) with b [D,W,C], D = N
    or 1 (broadcast, Dims::b_index :74-77): MATMUL on b laid out [N,C,W]."""
    bt = b.array().transpose(0, 2, 1)
    if bt.shape[0] != a.shape[0]:
        bt = np.broadcast_to(bt, (a.shape[0],) + bt.shape[1:])
    return matmul(a, T(b.dtype, list(bt.shape), np.ascontiguousarray(bt).reshape(-1)), a_zp, b_zp, out_t)


def max_pool2d(x: T, kernel, stride, pad, nan_mode) -> T:
    """MAX_POOL2D: src/ops/pool.rs:233-286; windows as for_each_window
    (:77-104, padding positions skipped, (ky, kx) order); integers fold
    i64::max from the type's minimum, floats nan_max (common.rs:155-177:
    ties keep the running value) from the type's lowest value, or from NaN
    under IGNORE."""
    n, ih, iw, c = x.shape
    oh = (ih + pad[0] + pad[1] - kernel[0]) // stride[0] + 1
    ow = (iw + pad[2] + pad[3] - kernel[1]) // stride[1] + 1
    xa = x.array()
    oy = np.arange(oh) * stride[0] - pad[0]
    ox = np.arange(ow) * stride[1] - pad[2]
    is_int = x.dtype in INT_TYPES
    ignore = nan_mode == 2
    if is_int:
        m = np.full((n, oh, ow, c), INT_RANGE[x.dtype][0], dtype=np.int64)
    else:
        init = np.float32(np.nan) if ignore else np.float32(-448.0 if x.dtype == "FP8E4M3" else -np.inf)
        m = np.full((n, oh, ow, c), init, dtype=np.float32)
    for ky in range(kernel[0]):
        y = oy + ky
        vy = (y >= 0) & (y < ih)
        for kx in range(kernel[1]):
            xx = ox + kx
            vx = (xx >= 0) & (xx < iw)
            valid = (vy[:, None] & vx[None, :])[None, :, :, None]
            v = xa[:, np.clip(y, 0, ih - 1)][:, :, np.clip(xx, 0, iw - 1)]
            if is_int:
                nm = np.maximum(m, v)
            else:
                with np.errstate(invalid="ignore"):
                    either = np.isnan(m) | np.isnan(v)
                    picked = np.where(np.isnan(m), v, m) if ignore else np.float32(np.nan)
                    nm = np.where(either, picked, np.where(m >= v, m, v)).astype(np.float32)
            m = np.where(valid, nm, m)
    out = m.reshape(-1)
    return T(x.dtype, [n, oh, ow, c], out if is_int else round_to(x.dtype, out))


def _wrap(dtype, v):
    """int_data's truncation to an integer type (src/ops/common.rs:110-122)."""
    bits = {"INT8": 8, "INT16": 16, "INT32": 32}.get(dtype)
    v = v.astype(np.int64)
    if bits is None:
        return v
    return ((v + (1 << (bits - 1))) & ((1 << bits) - 1)) - (1 << (bits - 1))


def cast(x: T, to) -> T:
    """CAST: src/ops/type_conv.rs:45-80 (float_to_int :34-43: saturation
    bounds taken in the input's precision, otherwise round half to even;
    integers reach floats through FP32; int to int wraps)."""
    frm, v = x.dtype, x.vals
    if frm == "BOOL":
        out = v.astype(np.float32) if to == "FP32" else _wrap(to, v.astype(np.int64))
    elif to == "BOOL":
        out = v != 0
    elif frm in INT_TYPES:
        out = _wrap(to, v) if to in INT_TYPES else round_to(to, v.astype(np.int64).astype(np.float32))
    elif to in INT_TYPES:
        lo, hi = INT_RANGE.get(to, (-(2 ** 63), 2 ** 63 - 1))
        f = v.astype(np.float32)
        hi_r = round_to(frm, np.array([hi], dtype=np.float32))[0]
        lo_r = round_to(frm, np.array([lo], dtype=np.float32))[0]
        with np.errstate(invalid="ignore"):
            r = np.where(np.isnan(f), 0.0, np.rint(f)).astype(np.float64)
            out = np.where(f >= hi_r, hi, np.where(f <= lo_r, lo, r)).astype(np.int64)
        out = _wrap(to, out)
    else:
        out = round_to(to, v.astype(np.float32))
    return T(to, x.shape, out)


def avg_pool2d(x: T, in_zp, out_zp, kernel, stride, pad, acc_type) -> T:
    """AVG_POOL2D: src/ops/pool.rs:164-231."""
    L = lib()
    n, ih, iw, c = x.shape
    oh = (ih + pad[0] + pad[1] - kernel[0]) // stride[0] + 1
    ow = (iw + pad[2] + pad[3] - kernel[1]) // stride[1] + 1
    k = np.array(kernel, dtype=np.int32)
    st = np.array(stride, dtype=np.int32)
    pd = np.array(pad, dtype=np.int32)
    if x.dtype in INT_TYPES:
        lo, hi = INT_RANGE[x.dtype]
        out = np.empty(n * oh * ow * c, dtype=np.int64)
        xv = np.ascontiguousarray(x.vals, dtype=np.int64)
        if L.orc_avg_pool_int(_p(xv), n, ih, iw, c, _p(k), _p(st), _p(pd), int(in_zp), int(out_zp), lo, hi, _p(out)):
            raise OracleError("AVG_POOL2D: apply_scale_32 REQUIRE failure")
    else:
        out = np.empty(n * oh * ow * c, dtype=np.float32)
        xv = np.ascontiguousarray(x.vals, dtype=np.float32)
        L.orc_avg_pool_float(_p(xv), n, ih, iw, c, _p(k), _p(st), _p(pd), FMT[acc_type], _p(out))
        out = round_to(x.dtype, out)   # float_data(in_t, ...) (pool.rs:227)
    return T(x.dtype, [n, oh, ow, c], out)


def rescale(x: T, mult: T, shift: T, in_zp, out_zp, out_t, scale32, rounding_mode, per_channel,
            input_unsigned, output_unsigned) -> T:
    """RESCALE: src/ops/type_conv.rs:111-191 (per-element part :171-188)."""
    L = lib()
    xv = np.ascontiguousarray(x.vals, dtype=np.int64)
    mv = np.ascontiguousarray(mult.vals, dtype=np.int64)
    sv = np.ascontiguousarray(shift.vals, dtype=np.int64)
    channels = x.shape[-1] if per_channel else 1
    out = np.empty(xv.size, dtype=np.int64)
    st = L.orc_rescale(_p(xv), xv.size, _p(mv), _p(sv), channels, int(per_channel), int(scale32), int(rounding_mode),
                       BITS[x.dtype], BITS[out_t], int(input_unsigned), int(output_unsigned), int(in_zp), int(out_zp),
                       _p(out))
    if st:
        raise OracleError("RESCALE: REQUIRE failure")
    return T(out_t, x.shape, out)


def clamp(x: T, lo, hi) -> T:
    """CLAMP: src/ops/elementwise.rs:319-343 (`min(max(x, lo), hi)`; NaN modes are
    not exercised by integer data, and for floats max/min follow nan_max/nan_min)."""
    if x.dtype in INT_TYPES:
        return T(x.dtype, x.shape, np.minimum(np.maximum(x.vals, lo), hi))
    raise NotImplementedError


def add(a: T, b: T, out_shape) -> T:
    """ADD: src/ops/elementwise.rs:395-397 with broadcasting (:57-107); int
    lanes wrap to the type (:138-145), float results are rounded to it."""
    av = np.broadcast_to(a.array(), out_shape)
    bv = np.broadcast_to(b.array(), out_shape)
    if a.dtype in INT_TYPES:
        s = (av.astype(np.int64) + bv.astype(np.int64))
        if a.dtype == "INT32":
            s = s.astype(np.int32).astype(np.int64)
        return T(a.dtype, out_shape, s)
    s = (av.astype(np.float32) + bv.astype(np.float32)).astype(np.float32)
    return T(a.dtype, out_shape, round_to(a.dtype, s.reshape(-1)))


# ---------------------------------------------------------------------------
# Graph runner
# ---------------------------------------------------------------------------

def _single(t: T):
    return t.vals.reshape(-1)[0]


def _float_minmax(dtype, raw):
    v = fb.decode_raw(dtype, raw, 1)
    return float(decode(dtype, v)[0])


def run_block(block: fb.Block, inputs: dict, order: list | None = None) -> dict:
    """Run `block` on `inputs` (name -> T) in the reference's ready-queue order;
    the executed operator indices are appended to `order` when given."""
    defs = {t.name: t for t in block.tensors}
    tensors = dict(inputs)
    ops = block.operators
    available = set(tensors)

    def ready(o):
        return o.op == "CONST" or all(i in available for i in o.inputs)

    q = deque(i for i, o in enumerate(ops) if ready(o))
    done = [False] * len(ops)
    while q:
        i = q.popleft()
        if done[i]:
            continue
        _eval(ops[i], tensors, defs)
        if order is not None:
            order.append(i)
        done[i] = True
        available.update(ops[i].outputs)
        for j, o in enumerate(ops):
            if not done[j] and ready(o) and j not in q:
                q.append(j)
    if not all(done):
        raise OracleError("could not execute all ops")
    return {n: tensors[n] for n in block.outputs if n in tensors}


def _eval(o, tensors, defs):
    out_name = o.outputs[0] if o.outputs else None
    decl = defs.get(out_name)
    g = [tensors[n] for n in o.inputs]
    a = o.attr
    if o.op in ("CONST", "CONST_SHAPE"):
        d = defs[out_name]
        shape = [max(s, 0) for s in d.shape]
        cnt = int(np.prod(shape)) if shape else 1
        raw = fb.decode_raw(d.dtype, d.data, cnt)
        r = T(d.dtype, shape, decode(d.dtype, raw))
    elif o.op == "IDENTITY":
        r = T(g[0].dtype, g[0].shape, g[0].vals.copy())
    elif o.op == "RESHAPE":
        r = T(g[0].dtype, [int(v) for v in g[1].vals], g[0].vals.copy())
    elif o.op == "TRANSPOSE":
        arr = g[0].array().transpose(a["perms"])
        r = T(g[0].dtype, list(arr.shape), arr.reshape(-1))
    elif o.op in ("CONV2D", "DEPTHWISE_CONV2D"):
        acc = fb.DTYPE_NAMES[a["acc_type"]]
        r = conv2d(g[0], g[1], g[2], _single(g[3]), _single(g[4]), a["pad"], a["stride"], a["dilation"],
                   acc, g[2].dtype, depthwise=(o.op == "DEPTHWISE_CONV2D"))
    elif o.op == "MATMUL":
        out_t = decl.dtype if decl else {"INT8": "INT32", "INT16": "INT48", "FP16": "FP16"}.get(g[0].dtype, "FP32")
        r = matmul(g[0], g[1], _single(g[2]), _single(g[3]), out_t)
    elif o.op == "CONV3D":
        r = conv3d(g[0], g[1], g[2], _single(g[3]), _single(g[4]), a["pad"], a["stride"], a["dilation"],
                   fb.DTYPE_NAMES[a["acc_type"]])
    elif o.op == "TRANSPOSE_CONV2D":
        r = transpose_conv2d(g[0], g[1], g[2], _single(g[3]), _single(g[4]), a["out_pad"], a["stride"],
                             fb.DTYPE_NAMES[a["acc_type"]])
    elif o.op == "MATMUL_T":
        # default_output (src/ops/matmul.rs:53-61)
        dflt = {"INT8": "INT32", "INT16": "INT48", "FP16": "FP16", "FP8E4M3": "FP16", "FP8E5M2": "FP16"}
        out_t = decl.dtype if decl else dflt.get(g[0].dtype, "FP32")
        r = matmul_t(g[0], g[1], _single(g[2]), _single(g[3]), out_t)
    elif o.op == "MAX_POOL2D":
        r = max_pool2d(g[0], a["kernel"], a["stride"], a["pad"], a["nan_mode"])
    elif o.op == "CAST":
        r = cast(g[0], decl.dtype)
    elif o.op == "AVG_POOL2D":
        r = avg_pool2d(g[0], _single(g[1]), _single(g[2]), a["kernel"], a["stride"], a["pad"],
                       fb.DTYPE_NAMES[a["acc_type"]])
    elif o.op == "RESCALE":
        out_t = decl.dtype if decl else "INT32"
        r = rescale(g[0], g[1], g[2], _single(g[3]), _single(g[4]), out_t, a["scale32"], a["rounding_mode"],
                    a["per_channel"], a["input_unsigned"], a["output_unsigned"])
    elif o.op == "CLAMP":
        x = g[0]
        if x.dtype in INT_TYPES:
            lo = int(decode(x.dtype, fb.decode_raw(x.dtype, a["min_val"], 1))[0])
            hi = int(decode(x.dtype, fb.decode_raw(x.dtype, a["max_val"], 1))[0])
            r = clamp(x, lo, hi)
        else:
            lo = _float_minmax(x.dtype, a["min_val"])
            hi = _float_minmax(x.dtype, a["max_val"])
            v = x.vals.astype(np.float32)
            ignore = a["nan_mode"] == 2
            # nan_max(x, lo) then nan_min(., hi) (src/ops/common.rs:156-177)
            m = np.where(np.isnan(v), (lo if ignore else np.nan), np.where(v >= lo, v, lo)).astype(np.float32)
            m = np.where(np.isnan(m), (hi if ignore else np.nan), np.where(m < hi, m, hi)).astype(np.float32)
            r = T(x.dtype, x.shape, round_to(x.dtype, m))
    elif o.op == "ADD":
        shape = list(np.broadcast_shapes(tuple(g[0].shape), tuple(g[1].shape)))
        r = add(g[0], g[1], shape)
    else:
        raise OracleError(f"oracle does not restate {o.op}")
    tensors[out_name] = r
