"""GPU parity of MATMUL_T, CONV3D, TRANSPOSE_CONV2D, MAX_POOL2D and CAST at
sizes beyond the reference's fixtures, against the oracle (bit for bit), and
of the paths no fixture reaches: MATMUL_T int8 on the tiled pointwise kernel
(16-aligned channels; B per batch and B shared by every batch; zero points;
a fused RESCALE) and bf16 MATMUL_T on the dedicated GEMM (fp32 reassociation
bound 2 K u sum|a b|, computed in float64).
"""

import zlib

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.test_gpu_conv_fast import oracle_run, run
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu


def rng_for(*key):
    return np.random.default_rng(zlib.crc32(repr(key).encode()))


def same(got, ref):
    return np.array_equal(np.asarray(got).reshape(-1).astype(np.int64), np.asarray(ref).reshape(-1).astype(np.int64))


def matmul_t_graph(n, h, c, w, d, azp, bzp, rescale=None):
    g = GraphBuilder()
    g.input("a", [n, h, c], "INT8")
    g.input("b", [d, w, c], "INT8")
    g.const("az", np.array([azp]), "INT8")
    g.const("bz", np.array([bzp]), "INT8")
    g.tensor("acc", [n, h, w], "INT32")
    g.op("MATMUL_T", ["a", "b", "az", "bz"], ["acc"])
    out = "acc"
    if rescale is not None:
        mult, shift, ozp = rescale
        g.const("m", np.asarray(mult, np.int32), "INT32")
        g.const("s", np.asarray(shift, np.int8), "INT8")
        g.const("iz", np.array([0]), "INT32")
        g.const("oz", np.array([ozp]), "INT8")
        g.tensor("q", [n, h, w], "INT8")
        g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["q"], scale32=1, rounding_mode="DOUBLE_ROUND",
             per_channel=int(len(mult) > 1))
        out = "q"
    return g.build([out]), out


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("d", [4, 1])
def test_matmul_t_int8_tiled(d, fused):
    n, h, c, w = 4, 72, 128, 96
    r = rng_for("mmt", d, fused)
    a = r.integers(-128, 128, (n, h, c)).astype(np.int8)
    b = r.integers(-128, 128, (d, w, c)).astype(np.int8)
    rescale = (r.integers(2 ** 30, 2 ** 31, w), r.integers(33, 40, w), -7) if fused else None
    graph, out = matmul_t_graph(n, h, c, w, d, -5, 3, rescale)
    ins = {"a": (a, "INT8"), "b": (b, "INT8")}
    ref = oracle_run(graph, ins)[out].vals
    assert same(run(graph, ins)[out].numpy(), ref)
    assert same(run(graph, ins, fusion=False)[out].numpy(), ref)


def test_matmul_t_bf16_gemm():
    n, h, c, w = 2, 64, 128, 96
    r = rng_for("mmt_bf16")
    a32 = r.standard_normal((n, h, c)).astype(np.float32)
    b32 = r.standard_normal((1, w, c)).astype(np.float32)
    a, b = O.encode("BF16", a32), O.encode("BF16", b32)
    g = GraphBuilder()
    g.input("a", [n, h, c], "BF16")
    g.input("b", [1, w, c], "BF16")
    g.const("az", np.array([0], np.uint16), "BF16")
    g.const("bz", np.array([0], np.uint16), "BF16")
    g.tensor("y", [n, h, w], "FP32")
    g.op("MATMUL_T", ["a", "b", "az", "bz"], ["y"])
    got = run(g.build(["y"]), {"a": (a, "BF16"), "b": (b, "BF16")})["y"].numpy().astype(np.float64)
    av = O.decode("BF16", a).astype(np.float64)
    bv = O.decode("BF16", b).astype(np.float64)[0]
    exact = av @ bv.T
    bound = 2 * c * 2.0 ** -24 * (np.abs(av) @ np.abs(bv).T)
    assert (np.abs(got - exact) <= bound).all()


def conv_nd_graph(kind, x, w, bias, zx, zw, **attr):
    g = GraphBuilder()
    g.input("x", list(x.shape), "INT8")
    g.const("w", w, "INT8")
    g.const("b", bias, "INT32")
    g.const("zx", np.array([zx]), "INT8")
    g.const("zw", np.array([zw]), "INT8")
    if kind == "CONV3D":
        ext = [(x.shape[1 + i] - 1 + attr["pad"][2 * i] + attr["pad"][2 * i + 1] - (w.shape[1 + i] - 1) *
                attr["dilation"][i]) // attr["stride"][i] + 1 for i in range(3)]
        shape = [x.shape[0]] + ext + [w.shape[0]]
    else:
        op_, st = attr["out_pad"], attr["stride"]
        shape = [x.shape[0], (x.shape[1] - 1) * st[0] + op_[0] + op_[1] + w.shape[1],
                 (x.shape[2] - 1) * st[1] + op_[2] + op_[3] + w.shape[2], w.shape[0]]
    g.tensor("y", shape, "INT32")
    g.op(kind, ["x", "w", "b", "zx", "zw"], ["y"], acc_type="INT32", **attr)
    return g.build(["y"])


def test_conv3d_int8():
    r = rng_for("conv3d")
    x = r.integers(-128, 128, (2, 6, 11, 9, 16)).astype(np.int8)
    w = r.integers(-128, 128, (8, 3, 3, 2, 16)).astype(np.int8)
    bias = r.integers(-2 ** 20, 2 ** 20, 8).astype(np.int32)
    graph = conv_nd_graph("CONV3D", x, w, bias, -3, 2, pad=[1, 1, 1, 1, 0, 1], stride=[1, 2, 1],
                          dilation=[2, 1, 1])
    ins = {"x": (x, "INT8")}
    assert same(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals)


@pytest.mark.parametrize("out_pad", [(0, 1, 0, 1), (-1, 0, -2, 1)])
def test_transpose_conv2d_int8(out_pad):
    r = rng_for("tconv", out_pad)
    x = r.integers(-128, 128, (2, 7, 6, 32)).astype(np.int8)
    w = r.integers(-128, 128, (16, 3, 4, 32)).astype(np.int8)
    bias = r.integers(-2 ** 20, 2 ** 20, 16).astype(np.int32)
    graph = conv_nd_graph("TRANSPOSE_CONV2D", x, w, bias, 5, -1, out_pad=list(out_pad), stride=[2, 3])
    ins = {"x": (x, "INT8")}
    assert same(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals)


def pool_graph(x, dt, kernel, stride, pad, nan_mode):
    n, ih, iw, c = x.shape
    oh = (ih + pad[0] + pad[1] - kernel[0]) // stride[0] + 1
    ow = (iw + pad[2] + pad[3] - kernel[1]) // stride[1] + 1
    g = GraphBuilder()
    g.input("x", list(x.shape), dt)
    g.tensor("y", [n, oh, ow, c], dt)
    g.op("MAX_POOL2D", ["x"], ["y"], kernel=kernel, stride=stride, pad=pad, nan_mode=nan_mode)
    return g.build(["y"])


def test_max_pool2d_int8_large():
    x = rng_for("mp8").integers(-128, 128, (8, 56, 56, 64)).astype(np.int8)
    graph = pool_graph(x, "INT8", [3, 3], [2, 2], [0, 1, 0, 1], "PROPAGATE")
    ins = {"x": (x, "INT8")}
    assert same(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals)


@pytest.mark.parametrize("mode", ["PROPAGATE", "IGNORE"])
def test_max_pool2d_bf16_nan_modes(mode):
    r = rng_for("mpbf", mode)
    v = r.standard_normal((2, 17, 19, 24)).astype(np.float32)
    v[r.random(v.shape) < 0.05] = np.nan
    v[r.random(v.shape) < 0.05] = 0.0
    v[r.random(v.shape) < 0.05] = -0.0
    x = O.encode("BF16", v)
    graph = pool_graph(x, "BF16", [2, 3], [1, 2], [1, 0, 1, 1], mode)
    ins = {"x": (x, "BF16")}
    got = run(graph, ins)["y"].numpy().view(np.uint16).reshape(-1)
    ref = O.encode("BF16", oracle_run(graph, ins)["y"].vals).view(np.uint16).reshape(-1)
    nan_g, nan_r = np.isnan(O.decode("BF16", got)), np.isnan(O.decode("BF16", ref))
    assert np.array_equal(nan_g, nan_r)
    assert np.array_equal(got[~nan_g], ref[~nan_r])  # bit patterns: the sign of zero included


@pytest.mark.parametrize("pair", [("FP32", "INT8"), ("FP32", "INT16"), ("BF16", "INT32"), ("FP16", "INT16"),
                                  ("FP32", "BF16"), ("FP32", "FP8E4M3"), ("FP16", "FP8E5M2"), ("INT32", "FP16"),
                                  ("INT16", "INT8"), ("INT32", "INT64"), ("FP32", "BOOL")])
def test_cast_large(pair):
    frm, to = pair
    r = rng_for("cast", pair)
    shape = (3, 257, 129)
    if frm in ("INT16", "INT32"):
        lim = 2 ** 15 if frm == "INT16" else 2 ** 31
        v = r.integers(-lim, lim, shape)
        x = v.astype(np.int16 if frm == "INT16" else np.int32)
    else:
        v = (r.standard_normal(shape) * np.float32(3e4 if "INT" in to else 100)).astype(np.float32)
        v.reshape(-1)[:6] = [0.5, 1.5, 2.5, -2.5, np.inf, -np.inf]
        if to not in ("INT8", "INT16", "INT32"):
            v.reshape(-1)[6] = np.nan
        x = O.encode(frm, v)
    g = GraphBuilder()
    g.input("x", list(shape), frm)
    g.tensor("y", list(shape), to)
    g.op("CAST", ["x"], ["y"])
    graph = g.build(["y"])
    ins = {"x": (x, frm)}
    got = run(graph, ins)["y"].numpy()
    ref = oracle_run(graph, ins)["y"]
    if to in ("INT8", "INT16", "INT32", "INT64", "BOOL"):
        assert same(got, ref.vals)
    else:
        # bit patterns (the sign of zero included); NaNs compared as NaN
        gv = O.decode(to, got.reshape(-1))
        rv = ref.vals.astype(np.float32)
        nan = np.isnan(rv)
        assert np.array_equal(np.isnan(gv), nan)
        assert np.array_equal(O.encode(to, gv)[~nan].view(np.uint8), O.encode(to, rv)[~nan].view(np.uint8))


# int16 on the int8 MFMA kernels: each int16 operand split into two int8
# halves, partial products combined in int64 and clamped to 48 bits.
@pytest.mark.parametrize("geom", [((2, 14, 14, 64), 64, 3, [1, 1, 1, 1], [1, 1]),
                                  ((2, 16, 17, 64), 48, 3, [0, 1, 1, 1], [2, 2]),
                                  ((3, 9, 10, 48), 32, 1, [0, 0, 0, 0], [1, 1])])
@pytest.mark.parametrize("rescale16", [False, True, "clamp"])
def test_conv2d_int16_split(geom, rescale16):
    xs, oc, k, pad, stride = geom
    r = rng_for("conv_i16", geom)
    x = r.integers(-2 ** 15, 2 ** 15, xs).astype(np.int16)
    x.reshape(-1)[:4] = [-2 ** 15, 2 ** 15 - 1, 0, -1]
    w = r.integers(-128, 128, (oc, k, k, xs[3])).astype(np.int8)
    bias = r.integers(-2 ** 40, 2 ** 40, oc)
    oh = (xs[1] + pad[0] + pad[1] - k) // stride[0] + 1
    ow = (xs[2] + pad[2] + pad[3] - k) // stride[1] + 1
    g = GraphBuilder()
    g.input("x", list(xs), "INT16")
    g.const("w", w, "INT8")
    g.const("b", bias, "INT48")
    g.const("zx", np.array([0]), "INT16")
    g.const("zw", np.array([-7]), "INT8")
    g.tensor("y", [xs[0], oh, ow, oc], "INT48")
    g.op("CONV2D", ["x", "w", "b", "zx", "zw"], ["y"], pad=pad, stride=stride, dilation=[1, 1], acc_type="INT48")
    out = "y"
    if rescale16:
        # INT48 -> INT16 through apply_scale_16, per channel, as an int16 network requantises
        g.const("m", r.integers(2 ** 14, 2 ** 15, oc).astype(np.int16), "INT16")
        g.const("s", r.integers(34, 40, oc).astype(np.int8), "INT8")
        g.const("iz", np.array([0]), "INT48")
        g.const("oz", np.array([0]), "INT16")
        g.tensor("q", [xs[0], oh, ow, oc], "INT16")
        g.op("RESCALE", ["y", "m", "s", "iz", "oz"], ["q"], scale32=0, rounding_mode="SINGLE_ROUND", per_channel=1)
        out = "q"
        if rescale16 == "clamp":
            g.tensor("qc", [xs[0], oh, ow, oc], "INT16")
            g.op("CLAMP", ["q"], ["qc"], min_val=(-20000).to_bytes(2, "little", signed=True) + bytes(6),
                 max_val=(15000).to_bytes(2, "little", signed=True) + bytes(6))
            out = "qc"
    graph = g.build([out])
    ins = {"x": (x, "INT16")}
    got = run(graph, ins)[out].numpy()
    assert same(got, oracle_run(graph, ins)[out].vals)
    if rescale16:
        # the combine and RESCALE as one kernel, and as two
        assert np.array_equal(got, run(graph, ins, fusion=False)[out].numpy())


def test_conv2d_int16_benchmark_layer():
    # The benchmark's int16 layer ([N,28,28,128] x [128,3,3,128] into INT48,
    # per-channel RESCALE to int16) at two images: every output against the
    # oracle.
    from tosa_amd import workloads as W
    graph, ins, info = W.conv_i16(n=2)
    assert same(run(graph, ins)[info["out"]].numpy(), oracle_run(graph, ins)[info["out"]].vals)


@pytest.mark.parametrize("kind,d", [("MATMUL", 2), ("MATMUL_T", 2), ("MATMUL_T", 1)])
def test_matmul_int16_split(kind, d):
    n, h, c, w = 2, 64, 128, 96
    r = rng_for("mm_i16", kind, d)
    a = r.integers(-2 ** 15, 2 ** 15, (n, h, c)).astype(np.int16)
    bshape = (n, c, w) if kind == "MATMUL" else (d, w, c)
    b = r.integers(-2 ** 15, 2 ** 15, bshape).astype(np.int16)
    a.reshape(-1)[:c] = -2 ** 15   # a row of extremes against B's first column
    b.reshape(-1)[:2] = [-2 ** 15, 2 ** 15 - 1]
    g = GraphBuilder()
    g.input("a", [n, h, c], "INT16")
    g.input("b", list(bshape), "INT16")
    g.const("az", np.array([0]), "INT16")
    g.const("bz", np.array([0]), "INT16")
    g.tensor("y", [n, h, w], "INT48")
    g.op(kind, ["a", "b", "az", "bz"], ["y"])
    graph = g.build(["y"])
    ins = {"a": (a, "INT16"), "b": (b, "INT16")}
    assert same(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals)


def test_matmul_int16_rescale_fused():
    # INT48 MATMUL followed by a per-column RESCALE to int16 (apply_scale_16)
    # and a CLAMP: the combine and the RESCALE run as one kernel; the result
    # must match the oracle and the unfused run.
    n, h, c, w = 2, 40, 128, 48
    r = rng_for("mm_i16_rescale")
    a = r.integers(-2 ** 15, 2 ** 15, (n, h, c)).astype(np.int16)
    b = r.integers(-2 ** 15, 2 ** 15, (n, c, w)).astype(np.int16)
    g = GraphBuilder()
    g.input("a", [n, h, c], "INT16")
    g.input("b", [n, c, w], "INT16")
    g.const("az", np.array([0]), "INT16")
    g.const("bz", np.array([0]), "INT16")
    g.tensor("y", [n, h, w], "INT48")
    g.op("MATMUL", ["a", "b", "az", "bz"], ["y"])
    g.const("m", r.integers(2 ** 14, 2 ** 15, w).astype(np.int16), "INT16")
    g.const("s", r.integers(30, 36, w).astype(np.int8), "INT8")
    g.const("iz", np.array([0]), "INT48")
    g.const("oz", np.array([0]), "INT16")
    g.tensor("q", [n, h, w], "INT16")
    g.op("RESCALE", ["y", "m", "s", "iz", "oz"], ["q"], scale32=0, rounding_mode="SINGLE_ROUND", per_channel=1)
    g.tensor("qc", [n, h, w], "INT16")
    g.op("CLAMP", ["q"], ["qc"], min_val=(-20000).to_bytes(2, "little", signed=True) + bytes(6),
         max_val=(15000).to_bytes(2, "little", signed=True) + bytes(6))
    graph = g.build(["qc"])
    ins = {"a": (a, "INT16"), "b": (b, "INT16")}
    got = run(graph, ins)["qc"].numpy()
    assert same(got, oracle_run(graph, ins)["qc"].vals)
    assert np.array_equal(got, run(graph, ins, fusion=False)["qc"].numpy())
