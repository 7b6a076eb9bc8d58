"""Host-side tests of the product library (no GPU needed).

* the shared library loads and exports every function include/*.h declares;
* its FlatBuffer reader agrees with the oracle's independent reader on every
  golden graph;
* malformed buffers, missing inputs and every ERROR_IF golden case are
  rejected, with the error raised by host-side validation (before any device
  work), as the reference's `tests/conformance.rs:251-261` requires;
* without a GPU a valid graph fails loudly with a device error: there is no
  host fallback.
"""

import glob
import os
import re
import subprocess

import numpy as np
import pytest

import tosa_amd as T
from tests.helpers import ROOT, Case, case_dirs, case_id

HEADERS = glob.glob(os.path.join(ROOT, "include", "*.h"))


def declared_functions():
    names = set()
    for h in HEADERS:
        text = open(h).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"typedef\s+struct\s*\{.*?\}\s*\w+\s*;", "", text, flags=re.S)
        for m in re.finditer(r"\b(tosa_\w+)\s*\(", text):
            names.add(m.group(1))
    return sorted(names)


def test_headers_exist():
    assert HEADERS, "include/*.h must declare the C ABI"


def test_library_exports_every_declared_symbol():
    lib = os.path.join(ROOT, "tosa_amd", "libtosa_mi355x.so")
    out = subprocess.run(["nm", "-D", "--defined-only", lib], capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.strip()}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    assert len(declared_functions()) > 40


def test_python_binding_declares_every_symbol():
    from tosa_amd import _lib
    assert set(declared_functions()) == set(_lib.SIGNATURES)
    T.lib()  # binds every signature


GRAPHS = case_dirs("conformance") + case_dirs("networks")


@pytest.mark.parametrize("d", GRAPHS[::3], ids=case_id)
def test_reader_matches_oracle_reader(d):
    c = Case(d)
    info = T.Interpreter.from_flatbuffer(c.graph).graph()
    blk = c.block
    assert [o["name"] for o in info["operators"]] == [o.op for o in blk.operators]
    assert [o["inputs"] for o in info["operators"]] == [o.inputs for o in blk.operators]
    assert [o["outputs"] for o in info["operators"]] == [o.outputs for o in blk.operators]
    assert [(t["name"], t["dtype"], t["shape"], t["has_data"]) for t in info["tensors"]] == \
        [(t.name, t.dtype, t.shape, t.data is not None) for t in blk.tensors]
    assert info["inputs"] == blk.inputs and info["outputs"] == blk.outputs


def test_run_graph_rejects_invalid_flatbuffer():
    # tests/integration.rs:86-90
    for data in (b"not a tosa flatbuffer", b""):
        with pytest.raises(T.TosaError) as e:
            T.run_graph(data, [])
        assert e.value.kind == "Deserialize"
    good = Case(case_dirs("networks")[0]).graph
    for cut in (8, 16, 64, len(good) // 2):
        with pytest.raises(T.TosaError):
            T.Interpreter.from_flatbuffer(good[:cut]).run([])


def _tensors(case):
    return [T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in case.inputs().items()]


def test_run_graph_rejects_missing_input():
    # tests/integration.rs:77-84: the ADD never becomes ready
    c = Case(os.path.join(ROOT, "tests", "golden", "networks", "tf_add_f32"))
    ins = _tensors(c)[1:]
    with pytest.raises(T.TosaError) as e:
        T.run_graph(c.graph, ins)
    assert e.value.kind == "GraphError" and "stuck" in str(e.value)


ERROR_IF = [d for d in case_dirs("conformance") if Case(d).expected_failure]


@pytest.mark.parametrize("d", ERROR_IF, ids=case_id)
def test_error_if_cases_are_rejected_by_validation(d):
    c = Case(d)
    with pytest.raises(T.TosaError) as e:
        T.Interpreter.from_flatbuffer(c.graph).run(_tensors(c))
    # Rejected by the graph/operator checks, not by a missing GPU.
    assert e.value.kind not in ("Device", "InvalidArgument"), str(e.value)


def test_tensor_host_round_trip():
    for dt, arr in (("INT8", np.arange(-5, 5, dtype=np.int8)), ("INT48", np.array([-(2 ** 47), 2 ** 47 - 1])),
                    ("BF16", np.array([0x3F80, 0xC000], dtype=np.uint16)), ("FP32", np.linspace(0, 1, 7, dtype=np.float32)),
                    ("INT32", np.zeros((0, 3), dtype=np.int32)), ("BOOL", np.array(True)),
                    ("INT8", np.int8(-3))):
        t = T.Tensor.from_numpy("t", arr, dt)
        assert t.dtype == dt and t.shape == list(arr.shape)
        assert np.array_equal(t.numpy(), arr.astype(t.numpy().dtype))
    assert T.Tensor.from_numpy("s", np.int32(3), "INT32").size_bytes() == 4
    assert T.Tensor.from_numpy("z", np.zeros((0,), np.int32), "INT32").size_bytes() == 4  # max(1, 0) elements


def test_constant_only_graph_runs_without_device():
    c = Case(os.path.join(ROOT, "tests", "golden", "conformance", "const", "const_0_i8"))
    out = T.run_graph(c.graph, [])
    exp, _ = c.expected()["const-0"]
    assert np.array_equal(out["const-0"].numpy(), exp)


@pytest.mark.skipif(T.device_count() > 0, reason="checks the behaviour without a GPU")
def test_no_host_fallback_without_gpu():
    c = Case(os.path.join(ROOT, "tests", "golden", "networks", "tflite_conv2d_qi8"))
    with pytest.raises(T.TosaError) as e:
        T.run_graph(c.graph, _tensors(c))
    assert e.value.kind == "Device"


def test_options_round_trip():
    assert T.get_option("fusion") in (0, 1)
    old = T.get_option("strict_float")
    T.set_option("strict_float", 1)
    assert T.get_option("strict_float") == 1
    T.set_option("strict_float", old)
    with pytest.raises(T.TosaError):
        T.set_option("no_such_option", 1)


@pytest.mark.parametrize("key,default,values", [
    ("conv_rows", 1, [(0, 0), (2, 2), (4, 1), (7, 1), (1, 1)]),
    ("matmul_rows", 128, [(64, 64), (128, 128), (100, 128), (0, 128)]),
])
def test_kernel_tiling_options(key, default, values):
    # Process-wide tiling choices: documented values are kept, others map to
    # the default kind (any nonzero conv_rows value other than 2 is 1;
    # any matmul_rows value other than 64 is 128).
    assert T.get_option(key) == default
    try:
        for value, kept in values:
            T.set_option(key, value)
            assert T.get_option(key) == kept, (value, kept)
    finally:
        T.set_option(key, default)
    assert T.get_option(key) == default


def test_interpreter_replans_for_each_input_name_set():
    # One Interpreter, runs alternating between complete and incomplete input
    # sets: the ready queue's starting state is kept per set of input names,
    # so each run must see its own set (tests/integration.rs:77-84 for the
    # stuck case).
    c = Case(os.path.join(ROOT, "tests", "golden", "networks", "tf_add_f32"))
    interp = T.Interpreter.from_flatbuffer(c.graph)
    for complete in (False, True, False, True):
        ins = _tensors(c) if complete else _tensors(c)[1:]
        if complete and T.device_count() > 0:
            assert set(interp.run(ins)) == set(c.expected())
            continue
        with pytest.raises(T.TosaError) as e:
            interp.run(ins)
        if complete:  # the ADD became ready and reached the device check
            assert e.value.kind == "Device", str(e.value)
        else:
            assert e.value.kind == "GraphError" and "stuck" in str(e.value)


def test_identity_graph_reruns_with_other_input_names():
    from tosa_amd.tosa_writer import GraphBuilder
    g = GraphBuilder()
    g.input("x", [2, 3], "INT8")
    g.tensor("y", [2, 3], "INT8")
    g.op("IDENTITY", ["x"], ["y"])
    interp = T.Interpreter.from_flatbuffer(g.build(["y"]))
    x = np.arange(6, dtype=np.int8).reshape(2, 3)
    for name in ("x", "q", "x"):
        if name == "x":
            out = interp.run([T.Tensor.from_numpy("x", x, "INT8")])
            assert np.array_equal(out["y"].numpy(), x)
        else:
            with pytest.raises(T.TosaError) as e:
                interp.run([T.Tensor.from_numpy(name, x, "INT8")])
            assert "stuck" in str(e.value)
