"""GPU parity of the op-level entry tosa_matmul_i8 (no graph) against the
oracle, bit for bit, on caller-owned device buffers; its checks; and
agreement with the graph path on the same operands.

The oracle restates eval_matmul's integer branch (src/ops/matmul.rs:98-153)
and eval_rescale (src/ops/type_conv.rs:111-191). The cases pick what the
one-kernel MATMUL depends on: rows below, at and past the 128-row workgroup;
columns below and past the 128-column tile; one and several 128-byte
stages; zero and nonzero zero points; int32 output, per-channel DOUBLE_ROUND
to int8, per-tensor SINGLE_ROUND to int16 with a CLAMP.
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.test_gpu_opapi import NP, dev
from tests.test_gpu_workloads import run, same_int
from tosa_amd import workloads as W
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")

# (n, h, c, w, a_zp, b_zp)
SHAPES = [
    (1, 7, 128, 16, 0, 0),
    (2, 128, 256, 144, -7, 2),
    (3, 130, 384, 208, 127, -128),
    (1, 64, 1024, 1040, 5, 0),
]
MODES = ["none", "channel_double", "tensor_single_i16_clamp"]


def _case(shape, mode, seed):
    n, h, c, w, za, zb = shape
    r = np.random.default_rng(seed)
    a = r.integers(-128, 128, (n, h, c)).astype(np.int8)
    b = r.integers(-128, 128, (n, c, w)).astype(np.int8)
    rescale = None
    if mode == "channel_double":
        rescale = dict(multiplier=r.integers(2 ** 30, 2 ** 31, w), shift=r.integers(36, 44, w), double_round=True,
                       output_dtype="INT8", output_zp=int(r.integers(-128, 128)))
    elif mode == "tensor_single_i16_clamp":
        rescale = dict(multiplier=[int(r.integers(2 ** 28, 2 ** 30))], shift=[36], double_round=False,
                       output_dtype="INT16", output_zp=0, clamp=(-3000, 2500))
    return a, b, za, zb, rescale


def _oracle(a, b, za, zb, rescale):
    acc = O.matmul(O.T("INT8", list(a.shape), a), O.T("INT8", list(b.shape), b), za, zb, "INT32")
    if rescale is None:
        return acc.vals.astype(np.int64).reshape(acc.shape)
    ch = len(rescale["multiplier"])
    y = O.rescale(acc, O.T("INT32", [ch], np.asarray(rescale["multiplier"], np.int64)),
                  O.T("INT8", [ch], np.asarray(rescale["shift"], np.int64)), 0, rescale["output_zp"],
                  rescale["output_dtype"], True, 3 if rescale["double_round"] else 1, ch > 1, False, False)
    if rescale.get("clamp"):
        y = O.clamp(y, *rescale["clamp"])
    return y.vals.astype(np.int64).reshape(acc.shape)


def _call(a, b, za, zb, rescale):
    at, ap = dev(a)
    bt, bp = dev(b)
    shape = T.matmul_i8(ap, a.shape, bp, b.shape, za, zb, rescale, 0)
    assert shape == (a.shape[0], a.shape[1], b.shape[2])
    out_t = rescale["output_dtype"] if rescale else "INT32"
    out = torch.empty(int(np.prod(shape)) * np.dtype(NP[out_t]).itemsize, dtype=torch.uint8, device="cuda")
    assert T.matmul_i8(ap, a.shape, bp, b.shape, za, zb, rescale, out.data_ptr()) == shape
    T.synchronize()
    torch.cuda.synchronize()
    return out.cpu().numpy().view(NP[out_t]).reshape(shape).astype(np.int64)


@pytest.mark.parametrize("mode", MODES)
@pytest.mark.parametrize("shape", SHAPES)
def test_matmul_i8_matches_oracle(shape, mode):
    a, b, za, zb, rescale = _case(shape, mode, 6100 + sum(shape[:4]) + len(mode))
    assert np.array_equal(_call(a, b, za, zb, rescale), _oracle(a, b, za, zb, rescale))


def test_matmul_i8_matches_graph_path():
    a, b, za, zb, rescale = _case(SHAPES[1], "channel_double", 6200)
    g = GraphBuilder()
    g.input("a", a.shape, "INT8")
    g.input("b", b.shape, "INT8")
    g.const("az", np.array([za]), "INT8")
    g.const("bz", np.array([zb]), "INT8")
    g.tensor("acc", [a.shape[0], a.shape[1], b.shape[2]], "INT32")
    g.op("MATMUL", ["a", "b", "az", "bz"], ["acc"])
    W._rescale(g, "acc", g.tensor("y", [a.shape[0], a.shape[1], b.shape[2]], "INT8"), b.shape[2],
               rescale["multiplier"], rescale["shift"], "INT32", "INT8", 0, rescale["output_zp"], True, True, "rs")
    graph = g.build(["y"])
    ref = run(graph, {"a": (a, "INT8"), "b": (b, "INT8")})["y"].numpy()
    assert same_int(_call(a, b, za, zb, rescale), ref.reshape(-1))


def test_matmul_i8_rejects_bad_arguments():
    a = np.zeros((2, 16, 128), np.int8)
    b = np.zeros((2, 128, 32), np.int8)
    at, ap = dev(a)
    bt, bp = dev(b)
    out = torch.empty(2 * 16 * 32 * 4, dtype=torch.uint8, device="cuda")

    def status(a_shape=a.shape, b_shape=b.shape, za=0, zb=0, rescale=None):
        try:
            T.matmul_i8(ap, a_shape, bp, b_shape, za, zb, rescale, out.data_ptr())
            return "OK"
        except T.TosaError as e:
            return e.kind

    assert status() == "OK"
    assert status(b_shape=(2, 64, 32)) == "ShapeMismatch"     # C differs
    assert status(b_shape=(1, 128, 32)) == "ShapeMismatch"    # batch differs
    assert status(a_shape=(2, 16, 0)) == "ShapeMismatch"      # empty dimension
    assert status(za=200) == "DTypeMismatch"                  # not an int8 value
    assert status(a_shape=(2, 16, 64), b_shape=(2, 64, 32)) == "UnsupportedOp"  # C % 128
    assert status(b_shape=(2, 128, 24)) == "UnsupportedOp"    # W % 16
    bad = dict(multiplier=[1 << 30, 1 << 30], shift=[36, 36], double_round=True, output_dtype="INT8", output_zp=0)
    assert status(rescale=bad) == "GraphError"                # 2 multipliers for 32 columns
    T.synchronize()
