"""GPU parity of the quantised residual folded into a pointwise convolution's
epilogue (conv_i8_kernel with the residual stage, tosa_amd/csrc/kernels/
conv_i8.hip; the convolution's launch held back until the residual's ADD in
tosa_amd/csrc/ops.cpp) against the oracle, bit for bit, and against the same
graph run unfused.

The block is the MobileNetV2 residual: a 1x1 CONV2D + RESCALE to int8 (y),
RESCALE(y) and RESCALE(skip) to int32, ADD, RESCALE to int8. The cases pick
what the fold depends on: reductions on the 64- and 128-byte staging paths;
pixel counts that leave the last tile partial; 16 to 160 channels (24 and 20
leave a channel tile partial; 18, not a multiple of 4, takes the residual
kernel instead; 128 channels over few and over many pixels, where the
convolution alone would take a tile without room for the residual stage);
y as the
ADD's first or second operand; per-tensor and per-channel parameters, single
and double rounding, input and output zero points; a final shift below 32
(apply_scale_32's value-range REQUIRE checked per value: passing, and
failing).
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.test_gpu_workloads import oracle_run, run, same_int
from tosa_amd import workloads as W
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu

CASES = [
    # n, h, w, k, c, y first, out shifts, double (a, b, out), per-channel (a, b, out)
    (2, 7, 9, 144, 24, True, (38, 44), (False, False, True), (True, False, True)),
    (2, 7, 9, 144, 32, True, (38, 44), (False, False, True), (True, False, True)),
    (1, 28, 28, 192, 64, False, (40, 46), (True, True, True), (True, True, False)),
    (3, 5, 11, 384, 160, True, (36, 42), (False, True, False), (False, True, True)),
    (2, 14, 14, 96, 16, False, (42, 48), (True, False, True), (True, True, True)),
    (1, 9, 13, 576, 96, True, (30, 32), (True, True, True), (True, True, True)),
    (2, 9, 10, 160, 20, False, (38, 44), (True, False, True), (False, True, True)),
    (1, 6, 7, 144, 18, True, (38, 44), (False, False, True), (True, False, True)),
    (1, 16, 16, 128, 128, False, (38, 44), (True, True, True), (True, False, True)),
    (2, 128, 128, 64, 128, True, (38, 44), (False, True, True), (True, True, False)),
]


def _graph(case, rng):
    n, h, w, k, c, y_first, (slo, shi), dbl, pc = CASES[case]
    shape = (n, h, w, c)
    x = rng.integers(-128, 128, size=(n, h, w, k)).astype(np.int8)
    skip = rng.integers(-128, 128, size=shape).astype(np.int8)
    wt = rng.integers(-128, 128, size=(c, 1, 1, k)).astype(np.int8)
    bias = rng.integers(-2 ** 20, 2 ** 20, size=c).astype(np.int32)
    zx, zy, zs, zo = (int(v) for v in rng.integers(-100, 100, 4))
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.input("skip", shape, "INT8")
    g.const("w", wt, "INT8")
    g.const("bias", bias, "INT32")
    g.const("zx", np.array([zx]), "INT8")
    g.const("zw", np.array([0]), "INT8")
    g.tensor("acc", list(shape), "INT32")
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["acc"], pad=[0, 0, 0, 0], stride=[1, 1], dilation=[1, 1],
         acc_type="INT32")
    W._rescale(g, "acc", g.tensor("y", shape, "INT8"), c, rng.integers(2 ** 30, 2 ** 31, c),
               rng.integers(38, 44, c), "INT32", "INT8", 0, zy, True, True, "ry")
    ca, cb, co = (c if pc[0] else 1), (c if pc[1] else 1), (c if pc[2] else 1)
    W._rescale(g, "y", g.tensor("ya", shape, "INT32"), c, rng.integers(2 ** 30, 2 ** 31, ca),
               rng.integers(12, 22, ca), "INT8", "INT32", zy, 0, dbl[0], pc[0], "r1")
    W._rescale(g, "skip", g.tensor("sb", shape, "INT32"), c, rng.integers(2 ** 30, 2 ** 31, cb),
               rng.integers(12, 22, cb), "INT8", "INT32", zs, 0, dbl[1], pc[1], "r2")
    g.tensor("sum", list(shape), "INT32")
    g.op("ADD", ["ya", "sb"] if y_first else ["sb", "ya"], ["sum"])
    W._rescale(g, "sum", g.tensor("out", shape, "INT8"), c, rng.integers(2 ** 30, 2 ** 31, co),
               rng.integers(slo, shi, co), "INT32", "INT8", 0, zo, dbl[2], pc[2], "r3")
    return g.build(["out"]), {"x": (x, "INT8"), "skip": (skip, "INT8")}


@pytest.mark.parametrize("case", range(len(CASES)))
def test_residual_fused_conv(case):
    graph, ins = _graph(case, np.random.default_rng(4100 + case))
    ref = oracle_run(graph, ins)["out"].vals
    got = run(graph, ins)["out"].numpy()
    assert same_int(got, ref)
    assert np.array_equal(got, run(graph, ins, fusion=False)["out"].numpy())


def test_residual_fused_repeated_runs():
    # One interpreter, several runs: the held-back launch and the cached
    # residual constants serve every run.
    graph, ins = _graph(2, np.random.default_rng(4200))
    ref = oracle_run(graph, ins)["out"].vals
    interp = T.Interpreter.from_flatbuffer(graph)
    for _ in range(3):
        out = interp.run([T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in ins.items()])
        assert same_int(out["out"].numpy(), ref)


def test_residual_fused_range_require_failure():
    # A final shift of 8 with the sums far beyond 2^7: apply_scale_32's
    # value-range REQUIRE fails for some element, on the device as in the
    # oracle.
    n, h, w, k, c = 1, 6, 8, 144, 32
    rng = np.random.default_rng(4300)
    shape = (n, h, w, c)
    x = rng.integers(-128, 128, size=(n, h, w, k)).astype(np.int8)
    skip = rng.integers(-128, 128, size=shape).astype(np.int8)
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.input("skip", shape, "INT8")
    g.const("w", rng.integers(-128, 128, size=(c, 1, 1, k)).astype(np.int8), "INT8")
    g.const("bias", np.zeros(c, np.int32), "INT32")
    g.const("zx", np.array([0]), "INT8")
    g.const("zw", np.array([0]), "INT8")
    g.tensor("acc", list(shape), "INT32")
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["acc"], pad=[0, 0, 0, 0], stride=[1, 1], dilation=[1, 1],
         acc_type="INT32")
    W._rescale(g, "acc", g.tensor("y", shape, "INT8"), c, [2 ** 30] * c, [40] * c, "INT32", "INT8", 0, 0, True,
               True, "ry")
    W._rescale(g, "y", g.tensor("ya", shape, "INT32"), c, [2 ** 30], [10], "INT8", "INT32", 0, 0, False, False, "r1")
    W._rescale(g, "skip", g.tensor("sb", shape, "INT32"), c, [2 ** 30], [10], "INT8", "INT32", 0, 0, False, False,
               "r2")
    g.tensor("sum", list(shape), "INT32")
    g.op("ADD", ["ya", "sb"], ["sum"])
    W._rescale(g, "sum", g.tensor("out", shape, "INT8"), c, [2 ** 30], [8], "INT32", "INT8", 0, 0, False, False, "r3")
    graph = g.build(["out"])
    ins = {"x": (x, "INT8"), "skip": (skip, "INT8")}
    with pytest.raises(O.OracleError):
        oracle_run(graph, ins)
    with pytest.raises(T.TosaError) as e:
        run(graph, ins)
    assert e.value.kind == "GraphError"
