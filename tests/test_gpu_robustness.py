"""Caching and sharing hazards of the device path.

* A tensor wrapped around caller-owned device memory may be rewritten by
  the caller between runs. Every operand of a run must then be read afresh:
  zero points, RESCALE multipliers and shifts, biases and weights that are
  graph inputs (not CONSTs) must not come from a cache of an earlier run.
* One Interpreter may serve several host threads at once (the graph is
  borrowed immutably, src/interpreter.rs:122-147): the first use of its
  constants, and the data derived from them, must be safe under concurrency.
"""

import threading

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from oracle import tosa_reader as fb
from tosa_amd import workloads as W
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu


def oracle_run(graph, ins):
    blk = fb.main_block(graph)
    return O.run_block(blk, {n: O.T(dt, list(a.shape), O.decode(dt, a)) for n, (a, dt) in ins.items()})


def conv_rescale_all_inputs(n=2, h=9, w=11, cin=64, cout=32):
    """CONV2D + per-channel RESCALE whose weight, bias, zero points,
    multiplier and shift are all graph inputs."""
    g = GraphBuilder()
    g.input("x", [n, h, w, cin], "INT8")
    g.input("w", [cout, 3, 3, cin], "INT8")
    g.input("bias", [cout], "INT32")
    g.input("zx", [1], "INT8")
    g.input("zw", [1], "INT8")
    g.tensor("acc", [n, h, w, cout], "INT32")
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["acc"], pad=[1, 1, 1, 1], stride=[1, 1], dilation=[1, 1],
         acc_type="INT32")
    g.input("m", [cout], "INT32")
    g.input("s", [cout], "INT8")
    g.const("izp", np.array([0]), "INT32")
    g.input("ozp", [1], "INT8")
    g.tensor("y", [n, h, w, cout], "INT8")
    g.op("RESCALE", ["acc", "m", "s", "izp", "ozp"], ["y"], scale32=1, rounding_mode="DOUBLE_ROUND", per_channel=1)
    return g.build(["y"])


def draw(seed, n=2, h=9, w=11, cin=64, cout=32):
    r = np.random.default_rng(seed)
    return {
        "x": (r.integers(-128, 128, (n, h, w, cin)).astype(np.int8), "INT8"),
        "w": (r.integers(-128, 128, (cout, 3, 3, cin)).astype(np.int8), "INT8"),
        "bias": (r.integers(-2 ** 15, 2 ** 15, cout).astype(np.int32), "INT32"),
        "zx": (np.array([r.integers(-128, 128)], np.int8), "INT8"),
        "zw": (np.array([r.integers(-128, 128)], np.int8), "INT8"),
        "m": (r.integers(2 ** 30, 2 ** 31, cout).astype(np.int32), "INT32"),
        "s": (r.integers(34, 41, cout).astype(np.int8), "INT8"),
        "ozp": (np.array([r.integers(-128, 128)], np.int8), "INT8"),
    }


def test_rewritten_device_operands_are_read_each_run():
    torch = pytest.importorskip("torch")
    graph = conv_rescale_all_inputs()
    interp = T.Interpreter.from_flatbuffer(graph)
    first = draw(1)
    bufs, handles = {}, []
    for name, (a, dt) in first.items():
        bufs[name] = torch.from_numpy(a.copy().view(np.uint8).reshape(-1)).cuda()
        handles.append(T.Tensor.from_device(name, a.shape, dt, bufs[name].data_ptr(), a.nbytes, keep=bufs[name]))
    torch.cuda.synchronize()
    for seed in (1, 2, 3):
        vals = draw(seed)
        # Rewrite every operand in place (seed 1 holds what was wrapped).
        for name, (a, _) in vals.items():
            bufs[name].copy_(torch.from_numpy(a.copy().view(np.uint8).reshape(-1)))
        torch.cuda.synchronize()
        got = interp.run(handles)["y"].numpy()
        ref = oracle_run(graph, vals)["y"]
        assert np.array_equal(got.reshape(-1).astype(np.int64), ref.vals), seed
        # The same values handed over from host memory to a fresh interpreter.
        fresh = T.Interpreter.from_flatbuffer(graph).run(
            [T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in vals.items()])["y"].numpy()
        assert np.array_equal(got, fresh), seed


def test_rewritten_float_bias_is_read_each_run():
    torch = pytest.importorskip("torch")
    n, h, w, cin, cout = 1, 6, 7, 32, 16
    g = GraphBuilder()
    g.input("x", [n, h, w, cin], "BF16")
    g.input("w", [cout, 3, 3, cin], "BF16")
    g.input("bias", [cout], "FP32")
    g.const("zx", np.array([0], np.uint16), "BF16")
    g.const("zw", np.array([0], np.uint16), "BF16")
    g.tensor("y", [n, h, w, cout], "FP32")
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["y"], pad=[1, 1, 1, 1], stride=[1, 1], dilation=[1, 1],
         acc_type="FP32")
    graph = g.build(["y"])
    r = np.random.default_rng(7)
    bf = lambda a: O.encode("BF16", a.astype(np.float32))  # noqa: E731
    x = bf(r.standard_normal((n, h, w, cin)))
    wt = bf(r.standard_normal((cout, 3, 3, cin)))
    interp = T.Interpreter.from_flatbuffer(graph)
    bias_dev = torch.zeros(cout, dtype=torch.float32, device="cuda")
    ins = [T.Tensor.from_numpy("x", x, "BF16"), T.Tensor.from_numpy("w", wt, "BF16"),
           T.Tensor.from_device("bias", [cout], "FP32", bias_dev.data_ptr(), 4 * cout, keep=bias_dev)]
    for seed in range(3):
        b = np.random.default_rng(100 + seed).standard_normal(cout).astype(np.float32) * 10
        bias_dev.copy_(torch.from_numpy(b))
        torch.cuda.synchronize()
        got = interp.run(ins)["y"].numpy()
        fresh = T.Interpreter.from_flatbuffer(graph).run(
            [T.Tensor.from_numpy("x", x, "BF16"), T.Tensor.from_numpy("w", wt, "BF16"),
             T.Tensor.from_numpy("bias", b, "FP32")])["y"].numpy()
        assert np.array_equal(got.view(np.uint32), fresh.view(np.uint32)), seed


def test_host_inputs_uploaded_without_waiting():
    # Runs fed from host memory, issued back to back in deferred mode (the
    # uploads go through pinned staging and do not wait for the stream),
    # each checked afterwards.
    graph, _, _ = W.conv_rescale(n=2, h=12, w=10, cin=64, cout=64)
    interp = T.Interpreter.from_flatbuffer(graph)
    xs = [np.random.default_rng(s).integers(-128, 128, (2, 12, 10, 64)).astype(np.int8) for s in range(6)]
    old = T.get_option("deferred")
    T.set_option("deferred", 1)
    try:
        outs = [interp.run([T.Tensor.from_numpy("x", x, "INT8")]) for x in xs]
        T.synchronize()
    finally:
        T.set_option("deferred", old)
    for x, o in zip(xs, outs):
        ref = oracle_run(graph, {"x": (x, "INT8")})["y"]
        assert np.array_equal(o["y"].numpy().reshape(-1).astype(np.int64), ref.vals)


@pytest.mark.parametrize("workload", ["conv_rescale", "mobilenet_v2"])
def test_two_threads_share_one_interpreter(workload):
    if workload == "conv_rescale":
        graph, _, _ = W.conv_rescale(n=2, h=14, w=14, cin=64, cout=64)
        shape, name = (2, 14, 14, 64), "x"
    else:
        graph, _, _ = W.mobilenet_v2(n=1)
        shape, name = (1, 224, 224, 3), "input"
    out_name = fb.main_block(graph).outputs[0]
    xs = [np.random.default_rng(50 + k).integers(-128, 128, shape).astype(np.int8) for k in range(4)]
    refs = [oracle_run(graph, {name: (x, "INT8")})[out_name].vals for x in xs]
    # A fresh interpreter: the threads race on the first use of its constants.
    interp = T.Interpreter.from_flatbuffer(graph)
    start = threading.Barrier(2)
    errors, done = [], []

    def work(k):
        try:
            start.wait()
            for i in range(6):
                j = (k + 2 * i) % 4
                got = interp.run([T.Tensor.from_numpy(name, xs[j], "INT8")])[out_name].numpy()
                if not np.array_equal(got.reshape(-1).astype(np.int64), refs[j]):
                    errors.append((k, i, j))
                done.append((k, i))
        except Exception as e:  # reported below
            errors.append((k, repr(e)))

    threads = [threading.Thread(target=work, args=(k,)) for k in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors
    assert len(done) == 12
