"""Every positive golden case of the hot-path operators and the networks, run
through the C ABI on the GPU and compared with the reference model's output.

Integer outputs: bit-exact. Float outputs: bit-exact everywhere except where
the MFMA kernels legitimately reorder the fp32 accumulation (bf16/fp16 CONV2D
and MATMUL with fp32 accumulators); there the tolerance is

    |y - y_ref| <= 2 K u * sum_k |a_k b_k| + u |bias| + 2 ulp_out(|y_ref|)

with u = 2^-24 (fp32 unit roundoff), K the reduction length and ulp_out the
spacing of the output format at |y_ref| (zero for fp32 outputs). In strict
float mode the same cases must be bit-exact.
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.helpers import Case, case_dirs, case_id, float_values, mismatches

pytestmark = pytest.mark.gpu

POSITIVE = [d for d in case_dirs("conformance") + case_dirs("networks") if not Case(d).expected_failure]


def run_product(c, strict=False, fusion=True):
    old = (T.get_option("strict_float"), T.get_option("fusion"))
    T.set_option("strict_float", int(strict))
    T.set_option("fusion", int(fusion))
    try:
        ins = [T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in c.inputs().items()]
        return T.Interpreter.from_flatbuffer(c.graph).run(ins)
    finally:
        T.set_option("strict_float", old[0])
        T.set_option("fusion", old[1])


def mfma_float_op(c):
    """The single CONV2D/MATMUL/MATMUL_T of a case that runs on float MFMA, or None."""
    if c.tested_op() not in ("CONV2D", "MATMUL", "MATMUL_T"):
        return None
    op = [o for o in c.block.operators if o.op in ("CONV2D", "MATMUL", "MATMUL_T")][0]
    a, b = (c.defs[op.inputs[0]].dtype, c.defs[op.inputs[1]].dtype)
    if (a, b) not in (("BF16", "BF16"), ("FP16", "FP16")):
        return None
    if op.op == "CONV2D" and op.attr.get("acc_type") != 7:  # FP32 accumulator
        return None
    if op.op in ("MATMUL", "MATMUL_T") and c.defs[op.outputs[0]].dtype != "FP32":
        return None
    return op


def ulp(dtype, v):
    v = np.abs(v)
    if dtype == "FP16":
        e = np.floor(np.log2(np.maximum(v, 2.0 ** -14)))
        return 2.0 ** (e - 10)
    if dtype == "BF16":
        e = np.floor(np.log2(np.maximum(v, 2.0 ** -126)))
        return 2.0 ** (e - 7)
    return np.zeros_like(v)


def tolerance(c, op, exp_vals, out_dt):
    """Per-element bound from the oracle run on |a| and |b|."""
    ins = {n: O.T(dt, list(a.shape), np.abs(O.decode(dt, a))) for n, (a, dt) in c.inputs().items()}
    blk = c.block
    tensors = dict(ins)
    for o in blk.operators:  # constants, with absolute values
        if o.op == "CONST":
            d = c.defs[o.outputs[0]]
            shape = [max(s, 0) for s in d.shape]
            raw = O.fb.decode_raw(d.dtype, d.data, int(np.prod(shape)) if shape else 1)
            v = O.decode(d.dtype, raw)
            tensors[o.outputs[0]] = O.T(d.dtype, shape, np.abs(v) if d.dtype in O.FLOAT_TYPES else v)
    g = [tensors[n] for n in op.inputs]
    if op.op == "CONV2D":
        z = O.T("FP32", [1], np.zeros(1, np.float32))
        w = g[1]
        K = w.shape[1] * w.shape[2] * w.shape[3]
        s = O.conv2d(g[0], w, O.T("FP32", [1], np.zeros(1, np.float32)), 0.0, 0.0, op.attr["pad"],
                     op.attr["stride"], op.attr["dilation"], "FP32", "FP32")
        bias = np.abs(O.decode(g[2].dtype, O.encode(g[2].dtype, g[2].vals)) if g[2].dtype in O.FLOAT_TYPES else g[2].vals)
        bias = np.broadcast_to(bias, (s.shape[-1],)) if bias.size == 1 else bias
        absum = s.vals.reshape(-1, s.shape[-1]).astype(np.float64)
        bterm = np.abs(bias.astype(np.float64))[None, :]
        del z
    else:
        K = g[0].shape[2]
        s = (O.matmul_t if op.op == "MATMUL_T" else O.matmul)(g[0], g[1], 0, 0, "FP32")
        absum = s.vals.astype(np.float64).reshape(-1, 1)
        bterm = 0.0
    u = 2.0 ** -24
    bound = 2 * K * u * absum + u * bterm
    return bound.reshape(-1) + 2 * ulp(out_dt, exp_vals)


@pytest.mark.parametrize("d", POSITIVE, ids=case_id)
def test_golden_case_on_gpu(d):
    c = Case(d)
    out = run_product(c)
    op = mfma_float_op(c)
    for n, (exp, dt) in c.expected().items():
        got = out[n]
        assert got.shape == list(exp.shape), n
        g = got.numpy()
        if op is not None and dt in ("FP32", "FP16", "BF16"):
            gv, ev = float_values(g, dt), float_values(exp, dt)
            tol = tolerance(c, op, ev, dt)
            same_nan = np.isnan(gv) == np.isnan(ev)
            ok = same_nan & (np.isnan(ev) | (np.abs(gv - ev) <= tol) | (gv == ev))
            assert ok.all(), f"{n}: {(~ok).sum()} outside tolerance; first {np.nonzero(~ok)[0][:5]}"
        else:
            bad = mismatches(g, exp, dt)
            assert bad.size == 0, f"{n}: {bad.size} of {exp.size} differ, first at {bad[:5]}"


STRICT = [d for d in POSITIVE if mfma_float_op(Case(d)) is not None]


@pytest.mark.parametrize("d", STRICT, ids=case_id)
def test_strict_float_mode_is_bit_exact(d):
    c = Case(d)
    out = run_product(c, strict=True)
    for n, (exp, dt) in c.expected().items():
        bad = mismatches(out[n].numpy(), exp, dt)
        assert bad.size == 0, f"{n}: {bad.size} differ"


NETWORKS = case_dirs("networks")


@pytest.mark.parametrize("d", NETWORKS, ids=case_id)
def test_networks_without_fusion(d):
    c = Case(d)
    out = run_product(c, fusion=False)
    for n, (exp, dt) in c.expected().items():
        assert mismatches(out[n].numpy(), exp, dt).size == 0
