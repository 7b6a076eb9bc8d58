"""The reference's public-API and hook tests (tests/integration.rs:64-186), run
through the C ABI on the GPU, plus the scheduling order against the oracle's
restatement of the reference's ready queue."""

import dataclasses
import os

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.helpers import GOLDEN, Case

pytestmark = pytest.mark.gpu


def load_case(name):
    return Case(os.path.join(GOLDEN, "networks", name))


def inputs(c):
    return [T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in c.inputs().items()]


def operator_count(c):
    return len(c.block.operators)


def test_run_graph_matches_reference():
    # integration.rs:64-75
    c = load_case("tf_add_f32")
    out = T.run_graph(c.graph, inputs(c))
    exp = c.expected()
    assert len(out) == len(exp)
    for n, (e, _) in exp.items():
        assert out[n].shape == list(e.shape)
        assert np.array_equal(out[n].numpy().view(np.uint32), e.view(np.uint32))


def test_stats_collector_counts_every_operator():
    # integration.rs:92-103
    c = load_case("mobilenet_like")
    ops = operator_count(c)
    out, stats = T.run_graph_with_stats(c.graph, inputs(c))
    assert len(out) == 1
    assert stats.total_ops_executed == ops
    assert sum(s["count"] for s in stats.op_stats.values()) == ops
    assert "CONV2D" in stats.op_stats
    assert stats.peak_memory_bytes > 0
    assert "CONV2D" in stats.summary()
    assert stats.summary().startswith(f"Total ops executed: {ops}\nPeak memory: ")


def test_op_trace_records_every_operator_once():
    # integration.rs:105-121
    c = load_case("conv_matmul")
    trace = T.OpTrace()
    T.run_graph_with_hooks(c.graph, inputs(c), trace)
    seen = sorted(e["op_index"] for e in trace.entries)
    assert seen == list(range(operator_count(c)))
    for e in trace.entries:
        op = c.block.operators[e["op_index"]]
        assert e["op"] == op.op
        assert len(e["output_shapes"]) == len(op.outputs)


def test_flop_counter_matches_operator_shapes():
    # integration.rs:123-152
    c = load_case("conv_matmul")
    trace = T.OpTrace()
    T.run_graph_with_hooks(c.graph, inputs(c), trace)
    flops = T.FlopCounter()
    T.run_graph_with_hooks(c.graph, inputs(c), flops)

    def expected(op):
        tot = 0
        for e in trace.entries:
            if e["op"] != op:
                continue
            i, w, o = e["input_shapes"][0], e["input_shapes"][1], e["output_shapes"][0]
            tot += 2 * int(np.prod(i[:3])) * w[2] if op == "MATMUL" else 2 * int(np.prod(o)) * int(np.prod(w[1:]))
        return tot

    for op in ("MATMUL", "CONV2D"):
        assert expected(op) > 0
        assert flops.flops_for(op) == expected(op)


class CallCounter(T.InterpreterHook):
    def __init__(self):
        super().__init__()
        self.pre = 0
        self.post = 0

    def pre_op(self, op, idx, ins):
        self.pre += 1

    def post_op(self, op, idx, ins, outs):
        self.post += 1


def test_hookset_dispatches_to_every_hook():
    # integration.rs:169-186
    c = load_case("mobilenet_like")
    ops = operator_count(c)
    counters = [CallCounter(), CallCounter()]
    hooks = T.HookSet()
    for h in counters:
        hooks.add(h)
    hooks.add(T.StatsCollector())
    assert len(hooks.hooks()) == 3
    out = T.run_graph_with_hooks(c.graph, inputs(c), hooks)
    assert len(out) == 1
    for h in counters:
        assert (h.pre, h.post) == (ops, ops)


class Recorder(T.InterpreterHook):
    """Records the hook call sequence, and reads every output's values."""
    reads_data = True

    def __init__(self):
        super().__init__()
        self.calls = []
        self.values = {}

    def pre_op(self, op, idx, ins):
        self.calls.append(("pre", idx, [t.name for t in ins]))

    def post_op(self, op, idx, ins, outs):
        self.calls.append(("post", idx, [t.name for t in outs]))
        for t in outs:
            self.values[t.name] = t.numpy()

    def on_tensor_alloc(self, name, shape, dtype, nbytes):
        self.calls.append(("alloc", name, nbytes))


@pytest.mark.parametrize("name", ["conv_matmul", "mobilenet_like", "tflite_conv2d_qi8"])
def test_operator_order_and_hook_sequence_match_reference(name):
    c = load_case(name)
    order = []
    ins = {n: O.T(dt, list(a.shape), O.decode(dt, a)) for n, (a, dt) in c.inputs().items()}
    every = dataclasses.replace(c.block, outputs=[o for op in c.block.operators for o in op.outputs])
    ref = O.run_block(every, ins, order)
    rec = Recorder()
    T.Interpreter.from_flatbuffer(c.graph).run(inputs(c), rec)
    got = [x[1] for x in rec.calls if x[0] == "pre"]
    assert got == order
    # pre_op, then one on_tensor_alloc per output, then post_op; never on_tensor_free
    i = 0
    for idx in order:
        assert rec.calls[i][:2] == ("pre", idx)
        i += 1
        for out in c.block.operators[idx].outputs:
            assert rec.calls[i][0] == "alloc" and rec.calls[i][1] == out
            i += 1
        assert rec.calls[i][:2] == ("post", idx)
        i += 1
    assert i == len(rec.calls)
    # A data-reading hook sees every intermediate with the reference's values.
    for n, t in ref.items():
        exp = O.encode(t.dtype, t.array())
        assert np.array_equal(np.asarray(rec.values[n]).reshape(-1).view(np.uint8),
                              np.asarray(exp).reshape(-1).view(np.uint8)), n


def test_fused_intermediates_are_materialised_on_request():
    """With fusion on, the int32 CONV2D result of tflite_conv2d_qi8 is never
    written by the fused kernel; a hook reading it after the run still gets
    the reference's values."""
    c = load_case("tflite_conv2d_qi8")

    class Keep(T.InterpreterHook):
        def __init__(self):
            super().__init__()
            self.keep = {}

        def post_op(self, op, idx, ins, outs):
            for t in outs:
                assert t.device_ptr() != 0
                self.keep[t.name] = t.numpy()  # forces the recomputation

    k = Keep()
    out = T.Interpreter.from_flatbuffer(c.graph).run(inputs(c), k)
    exp, _ = c.expected()["TosaOutput_0"]
    assert np.array_equal(out["TosaOutput_0"].numpy(), exp)
    ins = {n: O.T(dt, list(a.shape), O.decode(dt, a)) for n, (a, dt) in c.inputs().items()}
    every = dataclasses.replace(c.block, outputs=["layer_7"])
    ref = O.run_block(every, ins)["layer_7"]
    assert np.array_equal(k.keep["layer_7"].reshape(-1).astype(np.int64), ref.vals)


def test_interpreter_runs_repeatedly():
    # One Interpreter, many runs (src/interpreter.rs:122: the graph is borrowed).
    c = load_case("tflite_conv2d_qi8")
    interp = T.Interpreter.from_flatbuffer(c.graph)
    exp, _ = c.expected()["TosaOutput_0"]
    for _ in range(3):
        out = interp.run(inputs(c))
        assert np.array_equal(out["TosaOutput_0"].numpy(), exp)


def test_device_resident_inputs():
    torch = pytest.importorskip("torch")
    c = load_case("tflite_conv2d_qi8")
    (name, (a, dt)), = c.inputs().items()
    dev = torch.from_numpy(a.copy()).cuda()
    torch.cuda.synchronize()
    t = T.Tensor.from_device(name, a.shape, dt, dev.data_ptr(), a.nbytes, keep=dev)
    out = T.Interpreter.from_flatbuffer(c.graph).run([t])
    exp, _ = c.expected()["TosaOutput_0"]
    assert np.array_equal(out["TosaOutput_0"].numpy(), exp)
