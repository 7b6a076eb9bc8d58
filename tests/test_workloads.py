"""CPU checks of the in-memory graph writer and the benchmark workloads."""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from oracle import tosa_reader as fb
from tosa_amd import workloads as W
from tosa_amd.tosa_writer import GraphBuilder, encode_values

BUILDERS = [
    ("conv_rescale", W.conv_rescale, {}),
    ("conv_rescale_resnet", W.conv_rescale, {"n": 2, "h": 28, "w": 28, "cin": 128, "cout": 128}),
    ("matmul_rescale", W.matmul_rescale, {"batch": 2, "h": 16, "c": 64, "w": 32}),
    ("depthwise", W.depthwise, {"n": 1, "h": 16, "w": 16, "c": 16}),
    ("avg_pool", W.avg_pool, {"n": 2, "c": 64}),
    ("mobilenet_v2", W.mobilenet_v2, {"n": 1}),
    ("float_conv", W.float_conv, {"n": 1, "h": 6, "w": 6, "cin": 16, "cout": 8}),
    ("float_matmul", W.float_matmul, {"batch": 1, "h": 8, "c": 16, "w": 8}),
    ("conv_i16", W.conv_i16, {"n": 1, "h": 6, "w": 6, "cin": 64, "cout": 16}),
]


@pytest.mark.parametrize("name,fn,kw", BUILDERS, ids=[b[0] for b in BUILDERS])
def test_writer_output_reads_back_identically(name, fn, kw):
    graph, ins, info = fn(**kw)
    blk = fb.main_block(graph)
    prod = T.Interpreter.from_flatbuffer(graph).graph()
    assert [o["name"] for o in prod["operators"]] == [o.op for o in blk.operators]
    assert [o["inputs"] for o in prod["operators"]] == [o.inputs for o in blk.operators]
    assert [(t["name"], t["dtype"], t["shape"]) for t in prod["tensors"]] == \
        [(t.name, t.dtype, t.shape) for t in blk.tensors]
    assert prod["inputs"] == list(ins)
    for n, (a, dt) in ins.items():
        assert blk.tensor(n).shape == list(a.shape) and blk.tensor(n).dtype == dt
    assert info["ops"] > 0


def test_mobilenet_v2_structure():
    graph, _, info = W.mobilenet_v2(n=1)
    ops = [o.op for o in fb.main_block(graph).operators]
    assert ops.count("CONV2D") == 35 and ops.count("DEPTHWISE_CONV2D") == 17
    assert ops.count("CLAMP") == 35 and ops.count("ADD") == 10
    assert ops.count("AVG_POOL2D") == 1 and ops.count("MATMUL") == 1 and ops.count("RESHAPE") == 1
    # 300.8 M MAC per image (SURVEY-level count incl. the FC layer)
    assert 2.9e8 < info["macs"] < 3.1e8


def test_const_encoding_matches_reference_decoder():
    rng = np.random.default_rng(0)
    cases = [("INT4", rng.integers(-8, 8, size=7)), ("INT48", rng.integers(-2 ** 47, 2 ** 47, size=5)),
             ("INT16", rng.integers(-2 ** 15, 2 ** 15, size=9)), ("FP32", rng.standard_normal(4).astype(np.float32)),
             ("SHAPE", np.array([1, 64, 1280]))]
    for dt, vals in cases:
        raw = encode_values(vals, dt)
        back = fb.decode_raw(dt, raw, vals.size)
        assert np.array_equal(back.astype(vals.dtype), vals), dt


def test_small_graph_runs_in_oracle():
    g = GraphBuilder()
    g.input("x", [1, 5, 5, 8], "INT8")
    x = np.arange(200, dtype=np.int64).reshape(1, 5, 5, 8) % 256 - 128
    g.const("w", np.ones((4, 3, 3, 8), np.int8), "INT8")
    g.const("b", np.zeros(4, np.int32), "INT32")
    g.const("zx", np.array([0]), "INT8")
    g.const("zw", np.array([0]), "INT8")
    g.tensor("y", [1, 5, 5, 4], "INT32")
    g.op("CONV2D", ["x", "w", "b", "zx", "zw"], ["y"], pad=[1, 1, 1, 1], stride=[1, 1], dilation=[1, 1],
         acc_type="INT32")
    blk = fb.main_block(g.build(["y"]))
    y = O.run_block(blk, {"x": O.T("INT8", x.shape, x)})["y"].vals.reshape(1, 5, 5, 4)
    xp = np.pad(x, ((0, 0), (1, 1), (1, 1), (0, 0)))
    want = sum(xp[:, i:i + 5, j:j + 5, :].sum(-1) for i in range(3) for j in range(3))
    assert np.array_equal(y[..., 0], want)
