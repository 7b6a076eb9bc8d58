"""GPU parity of the int8 MFMA convolution with the table-driven epilogue
(tosa_amd/csrc/kernels/conv_i8.hip) against the oracle, bit for bit.

The sweep covers the kernel's template variants: tap-uniform stages of 64 and
128 bytes (IC a multiple of 64 / 128) and 1x1 stride-1 convolutions over any
IC that is a multiple of 16; channel tiles of 16/32/64/128 with ragged output
channel counts; pixel counts that are not a multiple of the tile; nonzero
input and weight zero points; int32, and RESCALE to int8/int16/int32 with
per-channel and per-tensor SINGLE/DOUBLE rounding, shifts below 32 (where
apply_scale_32's value-range REQUIRE is live), output zero points, a fused
CLAMP, and biases near +-2^31 so the accumulator wraps.
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from oracle import tosa_reader as fb
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu


def oracle_run(graph, ins):
    blk = fb.main_block(graph)
    return O.run_block(blk, {n: O.T(dt, list(a.shape), O.decode(dt, a)) for n, (a, dt) in ins.items()})


def run(graph, ins, fusion=True):
    old = T.get_option("fusion")
    T.set_option("fusion", int(fusion))
    try:
        return T.run_graph(graph, [T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in ins.items()])
    finally:
        T.set_option("fusion", old)


def build(x, w, bias, zx, zw, pad, stride, dil, rescale=None, out_dtype="INT8", clamp=None, bias_input=False):
    n, ih, iw, _ = x.shape
    oc, kh, kw, _ = w.shape
    oh = (ih - 1 + pad[0] + pad[1] - (kh - 1) * dil[0]) // stride[0] + 1
    ow = (iw - 1 + pad[2] + pad[3] - (kw - 1) * dil[1]) // stride[1] + 1
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("w", w, "INT8")
    if bias_input:
        g.input("b", bias.shape, "INT32")
    else:
        g.const("b", bias, "INT32")
    g.const("zx", np.array([zx]), "INT8")
    g.const("zw", np.array([zw]), "INT8")
    g.tensor("acc", [n, oh, ow, oc], "INT32")
    g.op("CONV2D", ["x", "w", "b", "zx", "zw"], ["acc"], pad=list(pad), stride=list(stride), dilation=list(dil),
         acc_type="INT32")
    out = "acc"
    if rescale is not None:
        mult, shift, ozp, dbl, pc = rescale
        g.const("m", np.asarray(mult, np.int32), "INT32")
        g.const("s", np.asarray(shift, np.int8), "INT8")
        g.const("iz", np.array([0]), "INT32")
        g.const("oz", np.array([ozp]), out_dtype)
        g.tensor("q", [n, oh, ow, oc], out_dtype)
        g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["q"], scale32=1,
             rounding_mode="DOUBLE_ROUND" if dbl else "SINGLE_ROUND", per_channel=int(pc))
        out = "q"
        if clamp is not None:
            g.tensor("c", [n, oh, ow, oc], out_dtype)
            width = {"INT8": 1, "INT16": 2, "INT32": 4}[out_dtype]
            lo = int(clamp[0]).to_bytes(width, "little", signed=True) + bytes(8 - width)
            hi = int(clamp[1]).to_bytes(width, "little", signed=True) + bytes(8 - width)
            g.op("CLAMP", ["q"], ["c"], min_val=lo, max_val=hi)
            out = "c"
    return g.build([out]), out


def check(graph, out, ins):
    ref = oracle_run(graph, ins)[out]
    for fusion in (True, False):
        got = run(graph, ins, fusion)[out].numpy()
        assert np.array_equal(got.reshape(-1).astype(np.int64), ref.vals.reshape(-1).astype(np.int64)), fusion


TAPS = [(3, 3, 64), (3, 3, 128), (5, 5, 64), (1, 3, 192), (3, 1, 256), (3, 3, 256), (2, 2, 128), (1, 1, 64)]
OCS = [8, 16, 24, 40, 64, 96, 128, 130, 200, 256]


@pytest.mark.parametrize("seed", range(20))
def test_fast_conv_taps(seed):
    rng = np.random.default_rng(5000 + seed)
    kh, kw, ic = TAPS[seed % len(TAPS)]
    oc = OCS[(seed * 3) % len(OCS)]
    n, ih, iw = int(rng.integers(1, 3)), int(rng.integers(5, 15)), int(rng.integers(5, 15))
    stride = [int(rng.integers(1, 3)), int(rng.integers(1, 3))]
    dil = [int(rng.integers(1, 3)), 1]
    pad = [int(v) for v in rng.integers(0, 3, size=4)]
    for d, (i, k) in enumerate(((ih, kh), (iw, kw))):
        full = i - 1 + pad[2 * d] + pad[2 * d + 1] - (k - 1) * dil[d]
        if full < 0:
            pad[2 * d + 1] += -full
            full = 0
        pad[2 * d + 1] += (-full) % stride[d]
    x = rng.integers(-128, 128, size=(n, ih, iw, ic)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, kh, kw, ic)).astype(np.int8)
    bias = (rng.integers(2 ** 31 - 2 ** 20, 2 ** 31, size=oc) * rng.choice([-1, 1], size=oc)).astype(np.int32)
    zx = int(rng.integers(-128, 128))
    zw = int(rng.integers(-128, 128)) if seed % 3 else 0
    mode = seed % 4
    if mode == 0:
        graph, out = build(x, w, bias, zx, zw, pad, stride, dil)
    else:
        out_dtype = ["INT8", "INT16", "INT32"][seed % 3]
        ozp = int(rng.integers(-128, 128)) if out_dtype == "INT8" else 0
        pc = mode != 3
        cnt = oc if pc else 1
        rs = (rng.integers(0, 2 ** 31, size=cnt), rng.integers(40, 56, size=cnt), ozp, bool(mode == 1), pc)
        # CLAMP takes int8 and int16 only (src/ops/elementwise.rs:327).
        clamp = (-20, 100) if seed % 5 == 0 and out_dtype != "INT32" else None
        graph, out = build(x, w, bias, zx, zw, pad, stride, dil, rescale=rs, out_dtype=out_dtype, clamp=clamp)
    check(graph, out, {"x": (x, "INT8")})


PW_IC = [16, 32, 48, 96, 144, 160, 64, 320]


@pytest.mark.parametrize("seed", range(16))
def test_fast_conv_pointwise(seed):
    rng = np.random.default_rng(6000 + seed)
    ic = PW_IC[seed % len(PW_IC)]
    oc = OCS[(seed * 7) % len(OCS)]
    n, h, w_ = int(rng.integers(1, 4)), int(rng.integers(3, 20)), int(rng.integers(3, 20))
    x = rng.integers(-128, 128, size=(n, h, w_, ic)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, 1, 1, ic)).astype(np.int8)
    bias = rng.integers(-2 ** 31, 2 ** 31, size=oc).astype(np.int32)
    zx = int(rng.integers(-128, 128))
    zw = int(rng.integers(-5, 6)) if seed % 2 else 0
    dbl = bool(seed % 2)
    # Shifts from 20 upwards: below 32 the value-range REQUIRE is live, so the
    # accumulators are kept small (weights in [-2, 2]) for those seeds.
    if seed % 4 == 3:
        w = rng.integers(-2, 3, size=(oc, 1, 1, ic)).astype(np.int8)
        bias = rng.integers(-1000, 1000, size=oc).astype(np.int32)
        shift = rng.integers(24, 32, size=oc)
    else:
        shift = rng.integers(36, 50, size=oc)
    rs = (rng.integers(2 ** 30, 2 ** 31, size=oc), shift, int(rng.integers(-16, 17)), dbl, True)
    clamp = (int(rng.integers(-128, 0)), 127) if seed % 3 == 0 else None
    graph, out = build(x, w, bias, zx, zw, [0, 0, 0, 0], [1, 1], [1, 1], rescale=rs, clamp=clamp)
    check(graph, out, {"x": (x, "INT8")})


def test_fast_conv_table_cache_and_runtime_bias():
    """The same interpreter run twice (the second run uses the cached
    epilogue table), and a bias that is a graph input (never cached)."""
    rng = np.random.default_rng(77)
    x = rng.integers(-128, 128, size=(2, 9, 9, 128)).astype(np.int8)
    w = rng.integers(-128, 128, size=(64, 3, 3, 128)).astype(np.int8)
    bias = rng.integers(-2 ** 20, 2 ** 20, size=64).astype(np.int32)
    rs = (rng.integers(2 ** 30, 2 ** 31, size=64), rng.integers(30, 40, size=64), 5, True, True)
    graph, out = build(x, w, bias, -3, 0, [1, 1, 1, 1], [1, 1], [1, 1], rescale=rs)
    ins = {"x": (x, "INT8")}
    ref = oracle_run(graph, ins)[out].vals
    interp = T.Interpreter.from_flatbuffer(graph)
    for _ in range(3):
        got = interp.run([T.Tensor.from_numpy("x", x, "INT8")])[out].numpy()
        assert np.array_equal(got.reshape(-1).astype(np.int64), ref.astype(np.int64))

    graph2, out2 = build(x, w, bias, -3, 0, [1, 1, 1, 1], [1, 1], [1, 1], rescale=rs, bias_input=True)
    interp2 = T.Interpreter.from_flatbuffer(graph2)
    for b in (bias, bias + 12345):
        ins2 = {"x": (x, "INT8"), "b": (b.astype(np.int32), "INT32")}
        ref2 = oracle_run(graph2, ins2)[out2].vals
        got = interp2.run([T.Tensor.from_numpy(k, a, dt) for k, (a, dt) in ins2.items()])[out2].numpy()
        assert np.array_equal(got.reshape(-1).astype(np.int64), ref2.astype(np.int64))


def test_fast_conv_require_failure():
    """A shift below 32 with accumulators outside [-2^(s-1), 2^(s-1)) is
    apply_scale_32's REQUIRE failure: the run reports GraphError."""
    rng = np.random.default_rng(78)
    x = rng.integers(-128, 128, size=(1, 8, 8, 64)).astype(np.int8)
    w = rng.integers(-128, 128, size=(32, 3, 3, 64)).astype(np.int8)
    bias = np.zeros(32, np.int32)
    rs = (np.full(32, 2 ** 30), np.full(32, 8), 0, False, True)
    graph, out = build(x, w, bias, 0, 0, [1, 1, 1, 1], [1, 1], [1, 1], rescale=rs)
    with pytest.raises(T.TosaError) as e:
        run(graph, {"x": (x, "INT8")})
    assert e.value.kind == "GraphError"
    with pytest.raises(O.OracleError):
        oracle_run(graph, {"x": (x, "INT8")})


# Stride-1 shapes that take the halo-tiled kernel: output rows of 14..56
# pixels so a workgroup tile holds >= 112 pixels; IC 512 with a 28-wide image
# needs two halo passes of 256 channels.
HALO = [
    # n, h, w, ic, oc, kh, kw, dil, pad
    (2, 28, 28, 128, 128, 3, 3, (1, 1), (1, 1, 1, 1)),
    (1, 14, 14, 256, 256, 3, 3, (1, 1), (1, 1, 1, 1)),
    (1, 30, 20, 64, 40, 5, 5, (1, 1), (2, 2, 2, 2)),
    (2, 17, 23, 192, 130, 1, 3, (1, 1), (0, 0, 1, 1)),
    (1, 23, 17, 128, 64, 3, 1, (2, 1), (2, 2, 0, 0)),
    (1, 28, 28, 512, 96, 3, 3, (1, 1), (1, 1, 1, 1)),
    (1, 29, 31, 64, 200, 2, 2, (1, 2), (0, 1, 1, 0)),
    (3, 16, 16, 320, 24, 3, 3, (2, 2), (2, 2, 2, 2)),
    (2, 12, 12, 32, 48, 3, 3, (1, 1), (1, 1, 1, 1)),
    (1, 9, 40, 96, 136, 3, 3, (1, 1), (1, 1, 1, 1)),
    (1, 5, 250, 32, 32, 1, 3, (1, 1), (0, 0, 1, 1)),
    (1, 14, 14, 160, 256, 3, 3, (1, 1), (0, 2, 1, 1)),
]


@pytest.mark.parametrize("case", range(len(HALO)))
@pytest.mark.parametrize("mode", ["i32", "rescale_i8", "rescale_i16_zw"])
def test_fast_conv_halo(case, mode):
    n, h, w_, ic, oc, kh, kw, dil, pad = HALO[case]
    rng = np.random.default_rng(7000 + 10 * case + len(mode))
    oh = h - 1 + pad[0] + pad[1] - (kh - 1) * dil[0] + 1
    ow = w_ - 1 + pad[2] + pad[3] - (kw - 1) * dil[1] + 1
    assert oh > 0 and ow > 0
    x = rng.integers(-128, 128, size=(n, h, w_, ic)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, kh, kw, ic)).astype(np.int8)
    bias = (rng.integers(2 ** 31 - 2 ** 20, 2 ** 31, size=oc) * rng.choice([-1, 1], size=oc)).astype(np.int32)
    zx = int(rng.integers(-128, 128))
    zw = int(rng.integers(-128, 128)) if mode.endswith("zw") else 0
    if mode == "i32":
        graph, out = build(x, w, bias, zx, zw, pad, [1, 1], list(dil))
    else:
        out_dtype = "INT16" if "i16" in mode else "INT8"
        ozp = 0 if out_dtype == "INT16" else int(rng.integers(-128, 128))
        rs = (rng.integers(2 ** 30, 2 ** 31, size=oc), rng.integers(38, 50, size=oc), ozp, case % 2 == 0, True)
        clamp = (-100, 90) if case % 3 == 0 else None
        graph, out = build(x, w, bias, zx, zw, pad, [1, 1], list(dil), rescale=rs, out_dtype=out_dtype, clamp=clamp)
    check(graph, out, {"x": (x, "INT8")})


# Convolutions whose input channels the tiled kernels do not take directly
# (a 3-channel stem, 24-channel 1x1 expansions, strided 1x1): materialised
# im2col, then the pointwise kernel.
IM2COL = [
    # n, h, w, ic, oc, kh, kw, stride, dil
    (2, 24, 24, 3, 32, 3, 3, (2, 2), (1, 1)),
    (1, 13, 11, 24, 144, 1, 1, (1, 1), (1, 1)),
    (2, 9, 10, 8, 40, 3, 3, (1, 1), (1, 1)),
    (1, 17, 15, 5, 7, 5, 3, (2, 1), (1, 2)),
    (2, 12, 12, 40, 96, 3, 3, (2, 2), (1, 1)),
    (1, 10, 14, 12, 130, 2, 2, (1, 1), (2, 1)),
    (3, 8, 8, 32, 24, 1, 1, (2, 2), (1, 1)),
    (1, 30, 7, 1, 16, 7, 1, (1, 1), (1, 1)),
]


@pytest.mark.parametrize("case", range(len(IM2COL)))
@pytest.mark.parametrize("mode", ["i32", "rescale_i8", "rescale_i8_zw"])
def test_im2col_conv(case, mode):
    n, h, w_, ic, oc, kh, kw, stride, dil = IM2COL[case]
    rng = np.random.default_rng(8000 + 10 * case + len(mode))
    pad = [int(v) for v in rng.integers(0, 2, size=4)]
    for d, (i, k) in enumerate(((h, kh), (w_, kw))):
        full = i - 1 + pad[2 * d] + pad[2 * d + 1] - (k - 1) * dil[d]
        if full < 0:
            pad[2 * d + 1] += -full
            full = 0
        pad[2 * d + 1] += (-full) % stride[d]
    x = rng.integers(-128, 128, size=(n, h, w_, ic)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, kh, kw, ic)).astype(np.int8)
    bias = (rng.integers(2 ** 31 - 2 ** 20, 2 ** 31, size=oc) * rng.choice([-1, 1], size=oc)).astype(np.int32)
    zx = int(rng.integers(-128, 128))
    zw = int(rng.integers(-128, 128)) if mode == "i32" or mode.endswith("zw") else 0
    if mode == "i32":
        graph, out = build(x, w, bias, zx, zw, pad, list(stride), list(dil))
    else:
        rs = (rng.integers(2 ** 30, 2 ** 31, size=oc), rng.integers(36, 48, size=oc), int(rng.integers(-128, 128)),
              case % 2 == 0, True)
        clamp = (-60, 100) if case % 3 == 0 else None
        graph, out = build(x, w, bias, zx, zw, pad, list(stride), list(dil), rescale=rs, clamp=clamp)
    check(graph, out, {"x": (x, "INT8")})


def matmul_graph(a, b, azp, bzp, b_const, rescale=None, clamp=None):
    batch, h, c = a.shape
    w = b.shape[2]
    g = GraphBuilder()
    g.input("a", a.shape, "INT8")
    if b_const:
        g.const("b", b, "INT8")
    else:
        g.input("b", b.shape, "INT8")
    g.const("az", np.array([azp]), "INT8")
    g.const("bz", np.array([bzp]), "INT8")
    g.tensor("acc", [batch, h, w], "INT32")
    g.op("MATMUL", ["a", "b", "az", "bz"], ["acc"])
    out = "acc"
    if rescale is not None:
        mult, shift, ozp, dbl, pc = rescale
        g.const("m", np.asarray(mult, np.int32), "INT32")
        g.const("s", np.asarray(shift, np.int8), "INT8")
        g.const("iz", np.array([0]), "INT32")
        g.const("oz", np.array([ozp]), "INT8")
        g.tensor("q", [batch, h, w], "INT8")
        g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["q"], scale32=1,
             rounding_mode="DOUBLE_ROUND" if dbl else "SINGLE_ROUND", per_channel=int(pc))
        out = "q"
        if clamp is not None:
            g.tensor("c", [batch, h, w], "INT8")
            lo = int(clamp[0]).to_bytes(1, "little", signed=True) + bytes(7)
            hi = int(clamp[1]).to_bytes(1, "little", signed=True) + bytes(7)
            g.op("CLAMP", ["q"], ["c"], min_val=lo, max_val=hi)
            out = "c"
    return g.build([out]), out


# Batched int8 MATMUL with C a multiple of 16: B transposed on the device,
# then the pointwise kernel with one grid slice per batch.
MATMUL = [
    # batch, h, c, w
    (2, 64, 1280, 1000),
    (3, 100, 16, 48),
    (1, 33, 48, 100),
    (4, 129, 256, 130),
    (2, 7, 32, 1),
    (8, 64, 64, 64),
    (1, 200, 1024, 16),
]


@pytest.mark.parametrize("case", range(len(MATMUL)))
@pytest.mark.parametrize("mode", ["i32_input_b", "i32_const_b", "rescale_const_b", "rescale_input_b"])
def test_matmul_tiled(case, mode):
    batch, h, c, w = MATMUL[case]
    rng = np.random.default_rng(9000 + 10 * case + len(mode))
    a = rng.integers(-128, 128, size=(batch, h, c)).astype(np.int8)
    b = rng.integers(-128, 128, size=(batch, c, w)).astype(np.int8)
    azp, bzp = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    b_const = "const_b" in mode
    if mode.startswith("i32"):
        graph, out = matmul_graph(a, b, azp, bzp, b_const)
    else:
        pc = case % 2 == 0
        cnt = w if pc else 1
        rs = (rng.integers(2 ** 30, 2 ** 31, size=cnt), rng.integers(38, 50, size=cnt), int(rng.integers(-128, 128)),
              case % 3 == 0, pc)
        graph, out = matmul_graph(a, b, azp, bzp, b_const, rescale=rs, clamp=(-50, 120) if case % 2 else None)
    ins = {"a": (a, "INT8")}
    if not b_const:
        ins["b"] = (b, "INT8")
    ref = oracle_run(graph, ins)[out]
    for fusion in (True, False):
        got = run(graph, ins, fusion)[out].numpy()
        assert np.array_equal(got.reshape(-1).astype(np.int64), ref.vals.reshape(-1).astype(np.int64)), fusion


def dw_graph(x, w, bias, zx, zw, pad, stride, rescale):
    n, ih, iw, c = x.shape
    kh, kw = w.shape[:2]
    oh = (ih - 1 + pad[0] + pad[1] - (kh - 1)) // stride[0] + 1
    ow = (iw - 1 + pad[2] + pad[3] - (kw - 1)) // stride[1] + 1
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("w", w, "INT8")
    g.const("b", bias, "INT32")
    g.const("zx", np.array([zx]), "INT8")
    g.const("zw", np.array([zw]), "INT8")
    g.tensor("acc", [n, oh, ow, c], "INT32")
    g.op("DEPTHWISE_CONV2D", ["x", "w", "b", "zx", "zw"], ["acc"], pad=list(pad), stride=list(stride),
         dilation=[1, 1], acc_type="INT32")
    mult, shift, ozp = rescale
    g.const("m", np.asarray(mult, np.int32), "INT32")
    g.const("s", np.asarray(shift, np.int8), "INT8")
    g.const("iz", np.array([0]), "INT32")
    g.const("oz", np.array([ozp]), "INT8")
    g.tensor("q", [n, oh, ow, c], "INT8")
    g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["q"], scale32=1, rounding_mode="DOUBLE_ROUND", per_channel=1)
    return g.build(["q"])


@pytest.mark.parametrize("c", [16, 32, 48, 96])
def test_depthwise_range_checked_shifts(c):
    """Shifts from 16 to 31 on the MFMA depthwise kernel: the value-range
    REQUIRE is live; small weights keep every value inside it."""
    rng = np.random.default_rng(400 + c)
    x = rng.integers(-128, 128, size=(2, 9, 11, c)).astype(np.int8)
    w = rng.integers(-2, 3, size=(3, 3, c, 1)).astype(np.int8)
    bias = rng.integers(-1000, 1000, size=c).astype(np.int32)
    rs = (rng.integers(2 ** 30, 2 ** 31, size=c), rng.integers(16, 32, size=c), 3)
    graph = dw_graph(x, w, bias, -5, 0, [1, 1, 1, 1], [1, 1], rs)
    ins = {"x": (x, "INT8")}
    ref = oracle_run(graph, ins)["q"].vals
    for fusion in (True, False):
        got = run(graph, ins, fusion)["q"].numpy()
        assert np.array_equal(got.reshape(-1).astype(np.int64), ref.reshape(-1).astype(np.int64)), fusion


def test_depthwise_range_require_failure():
    rng = np.random.default_rng(401)
    x = rng.integers(-128, 128, size=(1, 8, 8, 32)).astype(np.int8)
    w = rng.integers(-128, 128, size=(3, 3, 32, 1)).astype(np.int8)
    graph = dw_graph(x, w, np.zeros(32, np.int32), 0, 0, [1, 1, 1, 1], [1, 1],
                     (np.full(32, 2 ** 30), np.full(32, 6), 0))
    with pytest.raises(O.OracleError):
        oracle_run(graph, {"x": (x, "INT8")})
    with pytest.raises(T.TosaError) as e:
        run(graph, {"x": (x, "INT8")})
    assert e.value.kind == "GraphError"


# Images of at least 28 x 28 take the LDS-tiled depthwise kernel (every
# channel of a tile of output rows per workgroup).
DW_LDS = [
    # n, h, w, c, kh, kw, stride, dil, pad, zw, shifts
    (1, 28, 28, 16, 3, 3, (1, 1), (1, 1), (1, 1, 1, 1), 0, (36, 44)),
    (2, 30, 29, 48, 3, 3, (2, 2), (1, 1), (0, 1, 0, 0), 3, (36, 44)),
    (1, 32, 40, 64, 3, 3, (1, 1), (2, 2), (2, 2, 2, 2), -2, (36, 44)),
    (2, 28, 31, 32, 1, 3, (1, 1), (1, 1), (0, 0, 1, 1), 0, (20, 32)),
    (1, 28, 28, 96, 2, 2, (1, 2), (1, 1), (0, 1, 0, 0), 4, (36, 44)),
    (1, 56, 56, 144, 3, 3, (2, 2), (1, 1), (0, 1, 0, 1), -1, (36, 44)),
    (1, 29, 33, 960, 3, 3, (1, 1), (1, 1), (1, 1, 1, 1), 2, (36, 44)),
]


@pytest.mark.parametrize("case", range(len(DW_LDS)))
def test_depthwise_lds_tiles(case):
    n, h, w_, c, kh, kw, stride, dil, pad, zw, (slo, shi) = DW_LDS[case]
    rng = np.random.default_rng(500 + case)
    oh = (h - 1 + pad[0] + pad[1] - (kh - 1) * dil[0]) // stride[0] + 1
    ow = (w_ - 1 + pad[2] + pad[3] - (kw - 1) * dil[1]) // stride[1] + 1
    assert (h - 1 + pad[0] + pad[1] - (kh - 1) * dil[0]) % stride[0] == 0
    assert (w_ - 1 + pad[2] + pad[3] - (kw - 1) * dil[1]) % stride[1] == 0
    x = rng.integers(-128, 128, size=(n, h, w_, c)).astype(np.int8)
    small = slo < 32
    w = rng.integers(-2, 3, size=(kh, kw, c, 1)).astype(np.int8) if small else \
        rng.integers(-128, 128, size=(kh, kw, c, 1)).astype(np.int8)
    bias = rng.integers(-1000, 1000, size=c).astype(np.int32) if small else \
        rng.integers(-2 ** 20, 2 ** 20, size=c).astype(np.int32)
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("w", w, "INT8")
    g.const("b", bias, "INT32")
    g.const("zx", np.array([int(rng.integers(-128, 128))]), "INT8")
    g.const("zw", np.array([zw]), "INT8")
    g.tensor("acc", [n, oh, ow, c], "INT32")
    g.op("DEPTHWISE_CONV2D", ["x", "w", "b", "zx", "zw"], ["acc"], pad=list(pad), stride=list(stride),
         dilation=list(dil), acc_type="INT32")
    g.const("m", rng.integers(2 ** 30, 2 ** 31, size=c).astype(np.int32), "INT32")
    g.const("s", rng.integers(slo, shi, size=c).astype(np.int8), "INT8")
    g.const("iz", np.array([0]), "INT32")
    g.const("oz", np.array([int(rng.integers(-20, 20))]), "INT8")
    g.tensor("q", [n, oh, ow, c], "INT8")
    g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["q"], scale32=1, rounding_mode="DOUBLE_ROUND", per_channel=1)
    for out in ("q", "acc"):
        graph = g.build([out])
        ins = {"x": (x, "INT8")}
        ref = oracle_run(graph, ins)[out].vals
        for fusion in (True, False):
            got = run(graph, ins, fusion)[out].numpy()
            assert np.array_equal(got.reshape(-1).astype(np.int64), ref.reshape(-1).astype(np.int64)), (out, fusion)


# The epilogue table proves apply_scale_32's range REQUIRE unfailable when
# every channel with a shift below 32 has |bias| + max|x - zx| sum|w - zw|
# below 2^(shift-1); the kernels then skip the per-value check. Channel 0 is
# built to meet that bound exactly at one output pixel (every product at
# max|x - zx| |w - zw|): with the bound at 2^(shift-1) - 1 the table proves
# the range and the result must equal the oracle's; with the bias one higher
# the value is 2^(shift-1), the REQUIRE fails and the kernel must report it.
RANGE_EDGE = [
    # kind, n, h, w, ic, oc, k, stride, pad, zx, zw
    ("halo", 1, 28, 28, 64, 64, 3, 1, 1, 5, 3),
    ("tiled", 1, 17, 17, 64, 32, 3, 2, 1, 0, 0),
    ("pointwise", 1, 16, 16, 64, 48, 1, 1, 0, -7, 2),
    ("depthwise_lds", 1, 28, 28, 32, 32, 3, 1, 1, 4, -2),
    ("depthwise", 2, 9, 9, 16, 16, 3, 1, 1, 0, 0),
]


def _range_edge(case, over, bias_input=False):
    kind, n, h, w_, ic, oc, k, stride, pad, zx, zw = RANGE_EDGE[case]
    rng = np.random.default_rng(900 + case)
    dw = kind.startswith("depthwise")
    K = k * k * (1 if dw else ic)
    # The input value that attains max|x - zx|, and the weight step that
    # makes its product positive.
    xe, step = (-128, -1) if 128 + zx >= 127 - zx else (127, 1)
    xmax = abs(xe - zx)
    s = int(np.floor(np.log2(xmax * K))) if K * xmax < 2 ** 14 else 17
    T = 2 ** (s - 1)
    na = (T - 1) // xmax
    assert 0 < na <= K
    b0 = T - 1 - na * xmax
    x = rng.integers(-128, 128, size=(n, h, w_, ic)).astype(np.int8)
    cy, cx = h // 2, w_ // 2
    x[0, cy - k // 2:cy + k // 2 + 1, cx - k // 2:cx + k // 2 + 1, :] = xe
    # Rows of K weights per channel: channel 0 has na active entries, the
    # others fewer, with random signs.
    rows = np.full((oc, K), zw, np.int64)
    rows[0, :na] = zw + step
    for c in range(1, oc):
        m = int(rng.integers(0, na))
        rows[c, rng.choice(K, size=m, replace=False)] = zw + rng.choice([-1, 1], size=m)
    bias = rng.integers(-50, 50, size=oc).astype(np.int32)
    bias[0] = b0 + (1 if over else 0)
    rs = (np.full(oc, 2 ** (s - 7) if s > 7 else 1), np.full(oc, s), 0, False, True)
    if dw:
        w = rows.T.reshape(k, k, ic, 1).astype(np.int8)
        graph = dw_graph(x, w, bias, zx, zw, [pad] * 4, [stride] * 2, (rs[0], rs[1], 0))
        out = "q"
    else:
        w = rows.reshape(oc, k, k, ic).astype(np.int8)
        graph, out = build(x, w, bias, zx, zw, [pad] * 4, [stride] * 2, [1, 1], rescale=rs, bias_input=bias_input)
    ins = {"x": (x, "INT8")}
    if bias_input:
        ins["b"] = (bias, "INT32")
    return graph, out, ins


@pytest.mark.parametrize("case", range(len(RANGE_EDGE)))
def test_range_bound_proved(case):
    graph, out, ins = _range_edge(case, over=False)
    check(graph, out, ins)


@pytest.mark.parametrize("case", range(len(RANGE_EDGE)))
def test_range_bound_exceeded(case):
    graph, out, ins = _range_edge(case, over=True)
    with pytest.raises(O.OracleError):
        oracle_run(graph, ins)
    with pytest.raises(T.TosaError) as e:
        run(graph, ins)
    assert e.value.kind == "GraphError"


@pytest.mark.parametrize("case", [0, 1, 2])
def test_range_bound_runtime_bias(case):
    """A bias that is a graph input keeps the table uncached: the per-value
    check stays on, values inside the range pass."""
    graph, out, ins = _range_edge(case, over=False, bias_input=True)
    check(graph, out, ins)


# 1x1 convolutions with K <= 64, N a multiple of 32, at least 4096 pixels
# and an int8 RESCALE take the streaming pointwise kernel: every
# channel-tile count (TA 1-4, and N past 128 in several blocks), one and two
# reduction steps (K = 16 and 48 leave a zero-filled half step), nonzero
# weight zero points, shifts below 32 (range check live), a fused CLAMP and
# pixel counts that are not a multiple of 32; (N = 24, K = 32) stays on the
# tiled kernel. K % 16 == 8 cases read each row as 8-byte halves.
PWS = [
    # n, h, w, ic, oc
    (1, 64, 64, 16, 96),
    (2, 48, 47, 32, 32),
    (1, 65, 67, 48, 64),
    (3, 40, 40, 64, 192),
    (1, 70, 64, 32, 384),
    (2, 50, 41, 16, 128),
    (1, 80, 80, 64, 160),
    (2, 48, 47, 32, 24),
    # K % 16 == 8: 8-byte row halves, N a multiple of 16 in one-tile blocks
    (2, 48, 47, 24, 144),
    (1, 70, 64, 40, 48),
    (1, 64, 66, 56, 16),
    (3, 40, 40, 24, 32),
]


@pytest.mark.parametrize("case", range(len(PWS)))
def test_pointwise_stream(case):
    n, h, w_, ic, oc = PWS[case]
    rng = np.random.default_rng(9300 + case)
    x = rng.integers(-128, 128, size=(n, h, w_, ic)).astype(np.int8)
    zx = int(rng.integers(-128, 128))
    zw = int(rng.integers(-5, 6)) if case % 2 else 0
    if case % 3 == 2:
        w = rng.integers(-2, 3, size=(oc, 1, 1, ic)).astype(np.int8)
        bias = rng.integers(-1000, 1000, size=oc).astype(np.int32)
        shift = rng.integers(24, 32, size=oc)
    else:
        w = rng.integers(-128, 128, size=(oc, 1, 1, ic)).astype(np.int8)
        bias = rng.integers(-2 ** 31, 2 ** 31, size=oc).astype(np.int32)
        shift = rng.integers(36, 50, size=oc)
    rs = (rng.integers(2 ** 30, 2 ** 31, size=oc), shift, int(rng.integers(-16, 17)), bool(case % 2), True)
    clamp = (int(rng.integers(-128, 0)), 100) if case % 3 == 0 else None
    graph, out = build(x, w, bias, zx, zw, [0, 0, 0, 0], [1, 1], [1, 1], rescale=rs, clamp=clamp)
    check(graph, out, {"x": (x, "INT8")})


# 3x3 convolutions over 3 input channels with a RESCALE to int8 and at least
# 4096 output pixels take the stem kernel (im2col built in LDS): strides 1
# and 2, paddings 0-2 per side, 32-96 output channels.
STEM = [
    # n, h, w, stride, (pt, pb, pl, pr), oc
    (4, 64, 64, 2, (1, 1, 1, 1), 32),
    (2, 48, 48, 1, (1, 1, 1, 1), 64),
    (2, 70, 68, 1, (2, 2, 0, 0), 32),
    (8, 48, 48, 2, (2, 1, 2, 1), 96),
    (1, 130, 128, 2, (0, 1, 0, 1), 32),
]


@pytest.mark.parametrize("case", range(len(STEM)))
@pytest.mark.parametrize("zw_on", [False, True])
def test_stem_conv(case, zw_on):
    n, h, w_, s, pad, oc = STEM[case]
    rng = np.random.default_rng(9700 + 2 * case + int(zw_on))
    pad = list(pad)
    for d, i in enumerate((h, w_)):
        full = i - 1 + pad[2 * d] + pad[2 * d + 1] - 2
        pad[2 * d + 1] -= full % s  # exact output size: trim the far side
    x = rng.integers(-128, 128, size=(n, h, w_, 3)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, 3, 3, 3)).astype(np.int8)
    bias = rng.integers(-2 ** 20, 2 ** 20, size=oc).astype(np.int32)
    zx = int(rng.integers(-128, 128))
    zw = int(rng.integers(-100, 100)) if zw_on else 0
    rs = (rng.integers(2 ** 30, 2 ** 31, size=oc), rng.integers(30, 40, size=oc), int(rng.integers(-20, 20)),
          case % 2 == 0, True)
    clamp = (0, 100) if case % 2 else None
    graph, out = build(x, w, bias, zx, zw, pad, [s, s], [1, 1], rescale=rs, clamp=clamp)
    check(graph, out, {"x": (x, "INT8")})
