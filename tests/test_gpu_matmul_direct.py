"""GPU parity of the one-kernel int8 MATMUL (matmul_i8_kernel in
tosa_amd/csrc/kernels/conv_i8.hip: A and B copied to LDS as they lie, B's
column fragments read with LDS transpose reads, the zero-point terms from the
fragments) against the oracle, bit for bit.

The kernel takes C a multiple of 128 and W a multiple of 16. The cases pick
what its indexing depends on: workgroups of 64 and of 128 rows (option
matmul_rows); H below, at and past the row tile (rows of the last tile
re-read row H - 1 and are not stored); W below, at and past the 128-column
tile (the last column piece re-reads the final 16 columns); one to five and
eight 128-byte stages (rings of three and of four LDS buffers); every combination of zero and nonzero zero points (row
sums of A, column sums of B, both, neither); int32 output and the fused
RESCALE to int8 and int16 with per-tensor and per-channel parameters, an
output zero point and a CLAMP; shifts below 32 (apply_scale_32's value-range
REQUIRE checked per value, passing and failing). Results of the fused and
unfused graphs must agree as well.
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.test_gpu_workloads import oracle_run, run, same_int
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu

DIMS = [
    # batch, h, c, w
    (1, 1, 128, 16),
    (2, 64, 128, 128),
    (3, 100, 256, 208),
    (1, 7, 384, 1040),
    (2, 130, 1024, 144),
    (1, 200, 512, 96),
    (2, 33, 640, 48),
]


@pytest.fixture(params=[64, 128], autouse=True)
def tile_rows(request):
    T.set_option("matmul_rows", request.param)
    assert T.get_option("matmul_rows") == request.param
    yield request.param
    T.set_option("matmul_rows", 128)
ZPS = [(0, 0), (-7, 2), (127, -128), (0, 5), (-3, 0)]


def _graph(a, b, azp, bzp, rescale=None, out_dtype="INT8", clamp=None):
    batch, h, _ = a.shape
    w = b.shape[2]
    g = GraphBuilder()
    g.input("a", a.shape, "INT8")
    g.input("b", b.shape, "INT8")
    g.const("az", np.array([azp]), "INT8")
    g.const("bz", np.array([bzp]), "INT8")
    g.tensor("acc", [batch, h, w], "INT32")
    g.op("MATMUL", ["a", "b", "az", "bz"], ["acc"])
    if rescale is None:
        return g.build(["acc"]), "acc"
    mult, shift, ozp, double, per_channel = rescale
    g.const("m", np.asarray(mult, np.int32).reshape(-1), "INT32")
    g.const("s", np.asarray(shift, np.int8).reshape(-1), "INT8")
    g.const("iz", np.array([0]), "INT32")
    g.const("oz", np.array([ozp]), out_dtype)
    g.tensor("y", [batch, h, w], out_dtype)
    g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["y"], scale32=1,
         rounding_mode="DOUBLE_ROUND" if double else "SINGLE_ROUND", per_channel=int(per_channel))
    if clamp is None:
        return g.build(["y"]), "y"
    g.tensor("yc", [batch, h, w], out_dtype)
    width = {"INT8": 1, "INT16": 2}[out_dtype]
    lo = int(clamp[0]).to_bytes(width, "little", signed=True) + bytes(8 - width)
    hi = int(clamp[1]).to_bytes(width, "little", signed=True) + bytes(8 - width)
    g.op("CLAMP", ["y"], ["yc"], min_val=lo, max_val=hi)
    return g.build(["yc"]), "yc"


def _operands(dims, seed):
    batch, h, c, w = dims
    rng = np.random.default_rng(seed)
    a = rng.integers(-128, 128, size=(batch, h, c)).astype(np.int8)
    b = rng.integers(-128, 128, size=(batch, c, w)).astype(np.int8)
    return rng, a, b


@pytest.mark.parametrize("dims", DIMS)
def test_matmul_direct_int32(dims):
    _, a, b = _operands(dims, 500 + sum(dims))
    ins = {"a": (a, "INT8"), "b": (b, "INT8")}
    for azp, bzp in ZPS:
        graph, out = _graph(a, b, azp, bzp)
        assert same_int(run(graph, ins)[out].numpy(), oracle_run(graph, ins)[out].vals), (azp, bzp)


@pytest.mark.parametrize("dims", DIMS[1:])
@pytest.mark.parametrize("mode", ["i8_tensor", "i8_channel_clamp", "i16_channel"])
def test_matmul_direct_rescale(dims, mode):
    rng, a, b = _operands(dims, 700 + sum(dims) + len(mode))
    w = dims[3]
    per_channel = mode != "i8_tensor"
    n = w if per_channel else 1
    out_dtype = "INT16" if mode == "i16_channel" else "INT8"
    rs = (rng.integers(2 ** 30, 2 ** 31, size=n), rng.integers(32, 42, size=n),
          0 if out_dtype == "INT16" else int(rng.integers(-128, 128)), mode != "i16_channel", per_channel)
    clamp = (-90, 100) if mode == "i8_channel_clamp" else None
    ins = {"a": (a, "INT8"), "b": (b, "INT8")}
    for azp, bzp in ZPS[:3]:
        graph, out = _graph(a, b, azp, bzp, rs, out_dtype, clamp)
        got = run(graph, ins)[out].numpy()
        assert np.array_equal(got, run(graph, ins, fusion=False)[out].numpy()), (azp, bzp)
        assert same_int(got, oracle_run(graph, ins)[out].vals), (azp, bzp)


def test_matmul_direct_range_checked():
    # Shift 24 with a small multiplier: the sums stay far inside 2^23, the
    # table cannot rule the REQUIRE out (no weight sums for a B input).
    rng, a, b = _operands((2, 70, 256, 160), 901)
    rs = (rng.integers(2 ** 10, 2 ** 11, size=160), np.full(160, 24), 3, True, True)
    ins = {"a": (a // 16, "INT8"), "b": (b // 16, "INT8")}
    graph, out = _graph(a // 16, b // 16, -1, 1, rs)
    assert same_int(run(graph, ins)[out].numpy(), oracle_run(graph, ins)[out].vals)


def test_matmul_direct_range_require_failure():
    # Full-range operands at shift 12: |acc| reaches far beyond 2^11, so
    # apply_scale_32's REQUIRE fails on the device and the run reports it.
    rng, a, b = _operands((1, 64, 128, 32), 902)
    rs = (np.full(32, 2 ** 10), np.full(32, 12), 0, True, True)
    graph, out = _graph(a, b, 0, 0, rs)
    ins = {"a": (a, "INT8"), "b": (b, "INT8")}
    with pytest.raises(O.OracleError):
        oracle_run(graph, ins)
    with pytest.raises(T.TosaError) as e:
        run(graph, ins)
    assert e.value.kind == "GraphError"
