"""GPU parity of the op-level entry tosa_conv2d_i8 (no graph) against the
oracle, bit for bit, on caller-owned device buffers; its checks and error
reporting; and agreement with the graph path on the same operands.

The oracle restates eval_conv's integer branch (src/ops/conv.rs:398-474),
eval_rescale (src/ops/type_conv.rs:111-191) and eval_clamp
(src/ops/elementwise.rs:328-334); each case below picks the parameters one
kernel path depends on: the stride-1 3x3 halo kernel (packed weights), the
tiled kernel (stride 2, asymmetric padding, dilation), the 1x1 pointwise
kernel, the int32 output without RESCALE, per-tensor and per-channel
RESCALE, SINGLE and DOUBLE rounding, INT16 output with CLAMP, a weight zero
point, a bias of one value, and a RESCALE whose output zero point the fused
epilogue cannot fold (then the int32 result and the standalone RESCALE
kernel run).
"""

import zlib

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.test_gpu_conv_fast import build, oracle_run, run

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

NP = {"INT8": np.int8, "INT16": np.int16, "INT32": np.int32}


def dev(a):
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.uint8).reshape(-1).copy()).cuda()
    return t, t.data_ptr()


def oracle_conv(x, w, bias, zx, zw, pad, stride, dil, rescale):
    acc = O.conv2d(O.T("INT8", list(x.shape), x), O.T("INT8", list(w.shape), w),
                   O.T("INT32", list(bias.shape), bias), zx, zw, list(pad), list(stride), list(dil), "INT32", "INT32")
    if rescale is None:
        return acc.vals.astype(np.int64).reshape(acc.shape)
    ch = len(rescale["multiplier"])
    y = O.rescale(acc, O.T("INT32", [ch], np.asarray(rescale["multiplier"], np.int64)),
                  O.T("INT8", [ch], np.asarray(rescale["shift"], np.int64)), 0, rescale["output_zp"],
                  rescale["output_dtype"], True, 3 if rescale["double_round"] else 1, ch > 1, False, False)
    if rescale.get("clamp"):
        y = O.clamp(y, *rescale["clamp"])
    return y.vals.astype(np.int64).reshape(acc.shape)


def call(x, w, bias, zx, zw, pad, stride, dil, rescale, device_error=0):
    xt, xp = dev(x)
    wt, wp = dev(w)
    bt, bp = dev(bias)
    shape = T.conv2d_i8(xp, x.shape, wp, w.shape, bp, bias.size, zx, zw, pad, stride, dil, rescale, 0)
    out_t = rescale["output_dtype"] if rescale else "INT32"
    out = torch.empty(int(np.prod(shape)) * np.dtype(NP[out_t]).itemsize, dtype=torch.uint8, device="cuda")
    got_shape = T.conv2d_i8(xp, x.shape, wp, w.shape, bp, bias.size, zx, zw, pad, stride, dil, rescale,
                            out.data_ptr(), device_error)
    T.synchronize()
    torch.cuda.synchronize()
    assert got_shape == shape
    return out.cpu().numpy().view(NP[out_t]).reshape(shape).astype(np.int64)


# (n, ih, iw, ic, oc, k, pad, stride, dil)
GEOMS = {
    "halo3x3": (2, 14, 14, 128, 96, 3, (1, 1, 1, 1), (1, 1), (1, 1)),
    "tiled_s2": (2, 18, 15, 64, 64, 3, (0, 1, 1, 1), (2, 2), (1, 1)),
    "dilated": (1, 12, 13, 64, 32, 3, (2, 2, 2, 2), (1, 1), (2, 2)),
    "pointwise": (3, 9, 10, 32, 48, 1, (0, 0, 0, 0), (1, 1), (1, 1)),
}
RESCALES = ["none", "channel_double", "tensor_single_i16_clamp", "unfolded_zp"]


def make_case(geom, mode, seed):
    n, ih, iw, ic, oc, k, pad, stride, dil = GEOMS[geom]
    r = np.random.default_rng(seed)
    x = r.integers(-128, 128, (n, ih, iw, ic)).astype(np.int8)
    w = r.integers(-128, 128, (oc, k, k, ic)).astype(np.int8)
    zx = int(r.integers(-128, 128))
    zw = int(r.integers(-20, 20)) if geom == "tiled_s2" else 0
    bias = r.integers(-2 ** 20, 2 ** 20, 1 if geom == "dilated" else oc).astype(np.int32)
    rescale = None
    if mode == "channel_double":
        rescale = dict(multiplier=r.integers(2 ** 30, 2 ** 31, oc), shift=r.integers(33, 41, oc), double_round=True,
                       output_dtype="INT8", output_zp=int(r.integers(-128, 128)))
    elif mode == "tensor_single_i16_clamp":
        rescale = dict(multiplier=[int(r.integers(2 ** 28, 2 ** 30))], shift=[36], double_round=False,
                       output_dtype="INT16", output_zp=0, clamp=(-3000, 2500))
    elif mode == "unfolded_zp":
        # |zp| 2^shift above 2^60: the table cannot fold the zero point.
        rescale = dict(multiplier=r.integers(2 ** 30, 2 ** 31, oc), shift=r.integers(52, 56, oc), double_round=True,
                       output_dtype="INT8", output_zp=100)
        bias = (bias.astype(np.int64) * 0 + 2 ** 28).astype(np.int32)  # large enough to reach the output
    return x, w, bias, zx, zw, pad, stride, dil, rescale


@pytest.mark.parametrize("mode", RESCALES)
@pytest.mark.parametrize("geom", list(GEOMS))
def test_conv2d_i8_matches_oracle(geom, mode):
    args = make_case(geom, mode, zlib.crc32(f"{geom}:{mode}".encode()))
    got = call(*args)
    assert np.array_equal(got, oracle_conv(*args))


def test_conv2d_i8_matches_graph_path():
    x, w, bias, zx, zw, pad, stride, dil, rescale = make_case("halo3x3", "channel_double", 5)
    got = call(x, w, bias, zx, zw, pad, stride, dil, rescale)
    graph, out = build(x, w, bias, zx, zw, list(pad), list(stride), list(dil),
                       rescale=(np.asarray(rescale["multiplier"]), np.asarray(rescale["shift"]),
                                rescale["output_zp"], True, True))
    g = run(graph, {"x": (x, "INT8")})[out].numpy().astype(np.int64)
    assert np.array_equal(got, g.reshape(got.shape))
    assert np.array_equal(got, oracle_run(graph, {"x": (x, "INT8")})[out].vals.reshape(got.shape))


def test_conv2d_i8_repeated_calls_reuse_nothing_stale():
    # Same shapes, new weights, bias and parameters each call: derived data
    # (table, packed weights) is rebuilt per call.
    for seed in range(3):
        args = make_case("halo3x3", "channel_double", 100 + seed)
        assert np.array_equal(call(*args), oracle_conv(*args)), seed


def test_conv2d_i8_range_require_reported():
    # Shift 24 with a bias far outside [-2^23, 2^23): apply_scale_32's range
    # REQUIRE fails, reported in the caller's device word, or by
    # synchronize() through the stream's word.
    r = np.random.default_rng(3)
    x = r.integers(-128, 128, (1, 6, 28, 64)).astype(np.int8)
    w = r.integers(-128, 128, (32, 3, 3, 64)).astype(np.int8)
    bias = np.zeros(32, np.int32)
    bias[7] = 2 ** 26
    rescale = dict(multiplier=[2 ** 20] * 32, shift=[24] * 32, double_round=True, output_dtype="INT8", output_zp=0)
    xt, xp = dev(x)
    wt, wp = dev(w)
    bt, bp = dev(bias)
    out = torch.empty(1 * 6 * 28 * 32, dtype=torch.uint8, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()  # the zero fill ran on torch's stream, the call runs on the library's
    T.conv2d_i8(xp, x.shape, wp, w.shape, bp, 32, 0, 0, (1, 1, 1, 1), (1, 1), (1, 1), rescale, out.data_ptr(),
                err.data_ptr())
    T.synchronize()
    torch.cuda.synchronize()
    assert int(err.item()) != 0
    T.conv2d_i8(xp, x.shape, wp, w.shape, bp, 32, 0, 0, (1, 1, 1, 1), (1, 1), (1, 1), rescale, out.data_ptr())
    with pytest.raises(T.TosaError):
        T.synchronize()
    T.synchronize()  # cleared


def test_conv2d_i8_rejects_bad_arguments():
    x = np.zeros((1, 8, 8, 64), np.int8)
    w = np.zeros((32, 3, 3, 64), np.int8)
    bias = np.zeros(32, np.int32)
    xt, xp = dev(x)
    wt, wp = dev(w)
    bt, bp = dev(bias)
    out = torch.empty(8 * 8 * 32 * 4, dtype=torch.uint8, device="cuda")
    ok = dict(pad=(1, 1, 1, 1), stride=(1, 1), dilation=(1, 1))

    def status(xs=x.shape, ws=w.shape, blen=32, zx=0, zw=0, pad=ok["pad"], stride=ok["stride"],
               dil=ok["dilation"], rescale=None, x_ptr=xp):
        try:
            T.conv2d_i8(x_ptr, xs, wp, ws, bp, blen, zx, zw, pad, stride, dil, rescale, out.data_ptr())
            return "OK"
        except T.TosaError as e:
            return e.kind

    assert status() == "OK"
    assert status(ws=(32, 3, 3, 48)) == "ShapeMismatch"          # weight channels
    assert status(blen=5) == "ShapeMismatch"                     # bias length
    assert status(stride=(0, 1)) == "GraphError"                 # ERROR_IF
    assert status(pad=(-1, 0, 0, 0)) == "GraphError"
    assert status(pad=(0, 0, 0, 0), stride=(2, 2)) == "GraphError"  # inexact output extent
    assert status(zx=200) == "DTypeMismatch"
    assert status(xs=(1, 8, 8, 48), ws=(32, 3, 3, 48)) == "UnsupportedOp"  # channels for the fast kernels
    assert status(x_ptr=xp + 1) == "UnsupportedOp"               # alignment
    bad = dict(multiplier=[1 << 30] * 32, shift=[70] * 32, double_round=True, output_dtype="INT8", output_zp=0)
    assert status(rescale=bad) == "GraphError"                   # apply_scale_32 parameters
    two = dict(multiplier=[1 << 30] * 2, shift=[35] * 2, double_round=True, output_dtype="INT8", output_zp=0)
    assert status(rescale=two) == "GraphError"                   # channel count
    zp16 = dict(multiplier=[1 << 30], shift=[35], double_round=True, output_dtype="INT16", output_zp=3)
    assert status(rescale=zp16) == "GraphError"                  # zero point of a 16-bit output
