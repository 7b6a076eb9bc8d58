"""GPU parity of the benchmark configurations and randomized sweeps of the
kernels' code paths, against the oracle.

Integer results are compared bit for bit. Where the oracle would take too
long at full size, it checks batch/image subsets of the full-size GPU run
(each output image depends on its input image only), plus size-independent
properties. Float MFMA results are held to the bound stated in
test_gpu_conformance.py; at full size the fp32 reference is torch on the GPU.
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from oracle import tosa_reader as fb
from tosa_amd import workloads as W
from tosa_amd.tosa_writer import GraphBuilder

pytestmark = pytest.mark.gpu


def run(graph, ins, fusion=True):
    old = T.get_option("fusion")
    T.set_option("fusion", int(fusion))
    try:
        return T.run_graph(graph, [T.Tensor.from_numpy(n, a, dt) for n, (a, dt) in ins.items()])
    finally:
        T.set_option("fusion", old)


def oracle_run(graph, ins, outputs=None):
    blk = fb.main_block(graph)
    if outputs:
        import dataclasses
        blk = dataclasses.replace(blk, outputs=outputs)
    return O.run_block(blk, {n: O.T(dt, list(a.shape), O.decode(dt, a)) for n, (a, dt) in ins.items()})


def same_int(got, ref):
    return np.array_equal(np.asarray(got).reshape(-1).astype(np.int64), np.asarray(ref).reshape(-1).astype(np.int64))


# ---------------------------------------------------------------------------
# Benchmark configurations
# ---------------------------------------------------------------------------

def test_cfg1_conv_rescale_full_size():
    graph, ins, _ = W.conv_rescale()
    ref = oracle_run(graph, ins)["y"]
    for fusion in (True, False):
        assert same_int(run(graph, ins, fusion)["y"].numpy(), ref.vals)


@pytest.mark.parametrize("shape", [(64, 28, 28, 128, 128), (64, 14, 14, 256, 256)])
def test_resnet_scale_conv_rescale(shape):
    # Every image of the batch against the oracle (C loops, a few seconds).
    n, h, w, cin, cout = shape
    graph, ins, _ = W.conv_rescale(n=n, h=h, w=w, cin=cin, cout=cout)
    y = run(graph, ins)["y"].numpy()
    ref = oracle_run(graph, ins)["y"]
    assert same_int(y, ref.vals)


def _exact_matmul_i32(a, b, azp, bzp):
    """sum_k (a - azp)(b - bzp) per batch through float64 GEMMs: every partial
    sum is an integer below 2^53 (|terms| <= 255 * 255, K <= 2^20), so the
    result is exact; then wrapped to int32 as the reference's AccI32."""
    af = a.astype(np.float64) - azp
    bf = b.astype(np.float64) - bzp
    out = np.matmul(af, bf)
    return ((out.astype(np.int64) + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int64)


def test_cfg2_matmul_rescale():
    graph, ins, _ = W.matmul_rescale()
    y = run(graph, ins)["y"].numpy()
    yi = run(graph, ins, fusion=False)["y"].numpy()
    assert np.array_equal(y, yi)
    a, b = ins["a"][0], ins["b"][0]
    # Batch 0 through the oracle's own MATMUL + RESCALE.
    g1, _, _ = W.matmul_rescale(batch=1)
    ref0 = oracle_run(g1, {"a": (a[:1], "INT8"), "b": (b[:1], "INT8")})["y"]
    assert same_int(y[0], ref0.vals)
    # Every batch: exact accumulators, then the oracle's RESCALE.
    acc = _exact_matmul_i32(a, b, -7, 2)
    r = O.rescale(O.T("INT32", list(acc.shape), acc), O.T("INT32", [1], np.array([1518500250])),
                  O.T("INT8", [1], np.array([38])), 0, 0, "INT8", True, 1, False, False, False)
    assert same_int(y, r.vals)
    # The exact accumulators agree with the oracle's on batch 0.
    acc_ref = oracle_run(g1, {"a": (a[:1], "INT8"), "b": (b[:1], "INT8")}, outputs=["acc"])["acc"]
    assert same_int(acc[0], acc_ref.vals)


def test_cfg3_depthwise_and_avg_pool():
    graph, ins, _ = W.depthwise()
    y = run(graph, ins)["y"].numpy()
    assert same_int(y, oracle_run(graph, ins)["y"].vals)  # all 32 images
    graph, ins, _ = W.avg_pool()
    assert same_int(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals)


def test_cfg4_mobilenet_v2_end_to_end():
    graph2, ins2, _ = W.mobilenet_v2(n=2)
    ref = oracle_run(graph2, ins2)["logits"]
    ref2 = np.asarray(ref.vals).reshape(2, 1000)
    for fusion in (True, False):
        got = run(graph2, ins2, fusion)["logits"].numpy()
        assert same_int(got, ref.vals), fusion
    graph64, ins64, _ = W.mobilenet_v2(n=64)
    x64 = ins64["input"][0]
    # Images 0 and 1 of the 64-image input are the 2-image input (the same
    # seeded stream), so their logits must be the same.
    assert np.array_equal(x64[:2], ins2["input"][0])
    got64 = run(graph64, ins64)["logits"].numpy()
    assert got64.shape == (1, 64, 1000)
    assert same_int(got64[0, :2], ref.vals)
    # Every batch position: the two checked images tiled 32 times must give
    # their oracle logits in all 64 rows.
    tiled = np.ascontiguousarray(np.tile(ins2["input"][0], (32, 1, 1, 1)))
    got_t = run(graph64, {"input": (tiled, "INT8")})["logits"].numpy().reshape(64, 1000)
    for i in range(64):
        assert same_int(got_t[i], ref2[i % 2]), i
    # Every image of the real input: a batch in reversed order gives the
    # reversed logits (each image lands on other tiles), and eight images
    # spread over the batch match the oracle.
    got_r = run(graph64, {"input": (np.ascontiguousarray(x64[::-1]), "INT8")})["logits"].numpy().reshape(64, 1000)
    assert np.array_equal(got_r, got64.reshape(64, 1000)[::-1])
    pick = [2, 9, 18, 27, 36, 45, 54, 63]
    g8, _, _ = W.mobilenet_v2(n=8)
    ref8 = oracle_run(g8, {"input": (np.ascontiguousarray(x64[pick]), "INT8")})["logits"]
    assert same_int(got64.reshape(64, 1000)[pick], ref8.vals)


def _torch_conv_ref(x_bits, w_bits, bias, dtype, pad):
    import torch
    td = torch.bfloat16 if dtype == "BF16" else torch.float16
    x = torch.from_numpy(x_bits.view(np.int16)).view(td).float().cuda().permute(0, 3, 1, 2)
    w = torch.from_numpy(w_bits.view(np.int16)).view(td).float().cuda().permute(0, 3, 1, 2)
    absy = torch.nn.functional.conv2d(x.abs(), w.abs(), padding=pad)
    y = torch.nn.functional.conv2d(x.double(), w.double(), padding=pad)
    y = y + torch.from_numpy(bias).double().cuda()[None, :, None, None]
    return y.permute(0, 2, 3, 1).cpu().numpy(), absy.permute(0, 2, 3, 1).double().cpu().numpy()


@pytest.mark.parametrize("dtype", ["BF16", "FP16"])
@pytest.mark.parametrize("k,cout", [(3, 128), (1, 512)])
def test_cfg5_float_conv(dtype, k, cout):
    graph, ins, _ = W.float_conv(dtype=dtype, k=k, cout=cout)
    y = run(graph, ins)["y"].numpy()
    blk = fb.main_block(graph)
    wt = fb.decode_raw(dtype, blk.tensor("w").data, int(np.prod(blk.tensor("w").shape))).reshape(blk.tensor("w").shape)
    bias = fb.decode_raw("FP32", blk.tensor("bias").data, cout)
    exact, absy = _torch_conv_ref(ins["x"][0], wt, bias, dtype, k // 2)
    K = k * k * 128
    bound = 2 * K * 2.0 ** -24 * absy + 2.0 ** -24 * np.abs(bias) + 1e-30
    assert np.all(np.abs(y.astype(np.float64) - exact) <= bound)


def test_cfg5_bf16_matmul():
    import torch
    graph, ins, _ = W.float_matmul()
    y = run(graph, ins)["y"].numpy()
    a = torch.from_numpy(ins["a"][0].view(np.int16)).view(torch.bfloat16).float().cuda()
    b = torch.from_numpy(ins["b"][0].view(np.int16)).view(torch.bfloat16).float().cuda()
    exact = torch.bmm(a.double(), b.double()).cpu().numpy()
    absy = torch.bmm(a.abs(), b.abs()).double().cpu().numpy()
    bound = 2 * 2048 * 2.0 ** -24 * absy
    assert np.all(np.abs(y.astype(np.float64) - exact) <= bound)


# ---------------------------------------------------------------------------
# Randomized sweeps over the kernels' code paths
# ---------------------------------------------------------------------------

def conv_graph(x, w, bias, zx, zw, pad, stride, dil, depthwise=False, rescale=None, clamp=None, wdtype="INT8"):
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("w", w, wdtype)
    g.const("b", bias, "INT32")
    g.const("zx", np.array([zx]), "INT8")
    g.const("zw", np.array([zw]), wdtype)
    n, ih, iw, c = x.shape
    if depthwise:
        kh, kw, _, m = w.shape
        oc = c * m
    else:
        oc, kh, kw, _ = w.shape
    oh = (ih - 1 + pad[0] + pad[1] - (kh - 1) * dil[0]) // stride[0] + 1
    ow = (iw - 1 + pad[2] + pad[3] - (kw - 1) * dil[1]) // stride[1] + 1
    g.tensor("acc", [n, oh, ow, oc], "INT32")
    g.op("DEPTHWISE_CONV2D" if depthwise else "CONV2D", ["x", "w", "b", "zx", "zw"], ["acc"], pad=list(pad),
         stride=list(stride), dilation=list(dil), acc_type="INT32")
    out = "acc"
    if rescale is not None:
        mult, shift, ozp, dbl, pc = rescale
        g.const("m", np.asarray(mult, np.int32), "INT32")
        g.const("s", np.asarray(shift, np.int8), "INT8")
        g.const("iz", np.array([0]), "INT32")
        g.const("oz", np.array([ozp]), "INT8")
        g.tensor("q", [n, oh, ow, oc], "INT8")
        g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["q"], scale32=1,
             rounding_mode="DOUBLE_ROUND" if dbl else "SINGLE_ROUND", per_channel=int(pc))
        out = "q"
        if clamp is not None:
            g.tensor("c", [n, oh, ow, oc], "INT8")
            g.op("CLAMP", ["q"], ["c"], min_val=bytes([clamp[0] & 0xFF] + [0] * 7),
                 max_val=bytes([clamp[1] & 0xFF] + [0] * 7))
            out = "c"
    return g.build([out]), out


def exact_pads(rng, ih, iw, kh, kw, stride, dil):
    pad = [int(v) for v in rng.integers(0, 3, size=4)]
    for d, (i, k) in enumerate(((ih, kh), (iw, kw))):
        full = i - 1 + pad[2 * d] + pad[2 * d + 1] - (k - 1) * dil[d]
        if full < 0:
            pad[2 * d + 1] += -full
            full = 0
        pad[2 * d + 1] += (-full) % stride[d]
    return pad


IC = [1, 3, 5, 8, 16, 24, 33, 64, 96, 144]
OC = [1, 7, 16, 24, 33, 64, 100, 128, 200]


@pytest.mark.parametrize("seed", range(24))
def test_conv2d_int8_sweep(seed):
    rng = np.random.default_rng(1000 + seed)
    ic, oc = IC[seed % len(IC)], OC[(seed * 7) % len(OC)]
    n, ih, iw = int(rng.integers(1, 4)), int(rng.integers(4, 13)), int(rng.integers(4, 13))
    kh, kw = [(1, 1), (3, 3), (5, 5), (1, 3), (3, 1)][seed % 5]
    stride = [int(rng.integers(1, 3)), int(rng.integers(1, 3))]
    dil = [int(rng.integers(1, 3)), 1]
    pad = exact_pads(rng, ih, iw, kh, kw, stride, dil)
    i4 = seed % 6 == 5
    x = rng.integers(-128, 128, size=(n, ih, iw, ic)).astype(np.int8)
    w = rng.integers(-8, 8, size=(oc, kh, kw, ic)) if i4 else rng.integers(-128, 128, size=(oc, kh, kw, ic))
    bias = rng.integers(2 ** 31 - 2 ** 20, 2 ** 31, size=oc) * rng.choice([-1, 1], size=oc)  # forces wrap
    zx = int(rng.integers(-128, 128))
    zw = 0 if i4 else int(rng.integers(-128, 128))
    rs = None
    if seed % 2 == 0:
        rs = (rng.integers(0, 2 ** 31, size=oc), rng.integers(32, 50, size=oc), int(rng.integers(-128, 128)),
              bool(seed % 4 == 0), True)
    clamp = (-20, 100) if seed % 8 == 0 else None
    graph, out = conv_graph(x, w.astype(np.int8), bias.astype(np.int32), zx, zw, pad, stride, dil, rescale=rs,
                            clamp=clamp, wdtype="INT4" if i4 else "INT8")
    ins = {"x": (x, "INT8")}
    ref = oracle_run(graph, ins)[out]
    for fusion in (True, False):
        assert same_int(run(graph, ins, fusion)[out].numpy(), ref.vals), (fusion, ic, oc, kh, kw, stride, dil, pad)


@pytest.mark.parametrize("seed", range(16))
def test_depthwise_int8_sweep(seed):
    rng = np.random.default_rng(2000 + seed)
    c = [4, 8, 12, 144, 3, 5, 32, 96][seed % 8]
    m = 1 if seed % 5 else 2
    kh, kw = [(3, 3), (1, 1), (1, 3), (3, 1), (2, 2), (5, 5)][seed % 6]
    n, ih, iw = 2, int(rng.integers(4, 14)), int(rng.integers(4, 14))
    stride = [int(rng.integers(1, 3)), int(rng.integers(1, 3))]
    dil = [int(rng.integers(1, 3)), int(rng.integers(1, 3))]
    pad = exact_pads(rng, ih, iw, kh, kw, stride, dil)
    x = rng.integers(-128, 128, size=(n, ih, iw, c)).astype(np.int8)
    w = rng.integers(-128, 128, size=(kh, kw, c, m)).astype(np.int8)
    bias = (rng.integers(-2 ** 31, 2 ** 31, size=c * m)).astype(np.int32)
    zx, zw = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    rs = (rng.integers(0, 2 ** 31, size=c * m), rng.integers(33, 45, size=c * m), 3, True, True) if seed % 2 else None
    graph, out = conv_graph(x, w, bias, zx, zw, pad, stride, dil, depthwise=True, rescale=rs)
    ins = {"x": (x, "INT8")}
    ref = oracle_run(graph, ins)[out]
    for fusion in (True, False):
        assert same_int(run(graph, ins, fusion)[out].numpy(), ref.vals), (fusion, c, m, kh, kw)


@pytest.mark.parametrize("dims", [(1, 1, 1, 1), (2, 17, 40, 9), (3, 64, 128, 100), (1, 130, 257, 65),
                                  (2, 5, 3, 300), (4, 33, 64, 1000)])
def test_matmul_int8_sweep(dims):
    batch, h, c, w = dims
    rng = np.random.default_rng(sum(dims))
    a = rng.integers(-128, 128, size=(batch, h, c)).astype(np.int8)
    b = rng.integers(-128, 128, size=(batch, c, w)).astype(np.int8)
    for azp, bzp in ((0, 0), (-7, 2), (127, -128)):
        g = GraphBuilder()
        g.input("a", a.shape, "INT8")
        g.input("b", b.shape, "INT8")
        g.const("az", np.array([azp]), "INT8")
        g.const("bz", np.array([bzp]), "INT8")
        g.tensor("y", [batch, h, w], "INT32")
        g.op("MATMUL", ["a", "b", "az", "bz"], ["y"])
        graph = g.build(["y"])
        ins = {"a": (a, "INT8"), "b": (b, "INT8")}
        assert same_int(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals), (azp, bzp)


def test_rescale_modes_sweep():
    rng = np.random.default_rng(5)
    for in_t, out_t, scale32, rnd, pc, iu, ou in [
        ("INT32", "INT8", 1, "DOUBLE_ROUND", 1, 0, 0), ("INT32", "INT16", 1, "SINGLE_ROUND", 0, 0, 0),
        ("INT8", "INT32", 1, "SINGLE_ROUND", 1, 0, 0), ("INT16", "INT8", 0, "SINGLE_ROUND", 1, 0, 0),
        ("INT8", "INT8", 1, "INEXACT_ROUND", 1, 0, 0), ("INT8", "INT16", 1, "DOUBLE_ROUND", 0, 0, 1),
        ("INT16", "INT8", 1, "SINGLE_ROUND", 0, 1, 0), ("INT48", "INT32", 0, "SINGLE_ROUND", 1, 0, 0)]:
        shape = (3, 5, 8)
        lo, hi = {"INT8": (-128, 128), "INT16": (-2 ** 15, 2 ** 15), "INT32": (-2 ** 28, 2 ** 28),
                  "INT48": (-2 ** 40, 2 ** 40)}[in_t]
        x = rng.integers(lo, hi, size=shape)
        ch = shape[-1] if pc else 1
        mult = rng.integers(1, 2 ** 31 if scale32 else 2 ** 15, size=ch)
        shift = rng.integers(20 if in_t in ("INT32", "INT48") else 8, 40, size=ch)
        izp = int(rng.integers(-128, 128)) if in_t == "INT8" and not iu else 0
        ozp = int(rng.integers(-128, 128)) if out_t == "INT8" and not ou else 0
        g = GraphBuilder()
        g.input("x", shape, in_t)
        g.const("m", mult, "INT32" if scale32 else "INT16")
        g.const("s", shift, "INT8")
        g.const("iz", np.array([izp]), in_t)
        g.const("oz", np.array([ozp]), out_t)
        g.tensor("y", shape, out_t)
        g.op("RESCALE", ["x", "m", "s", "iz", "oz"], ["y"], scale32=scale32, rounding_mode=rnd, per_channel=pc,
             input_unsigned=iu, output_unsigned=ou)
        graph = g.build(["y"])
        st = {"INT8": np.int8, "INT16": np.int16, "INT32": np.int32, "INT48": np.int64}[in_t]
        ins = {"x": (x.astype(st), in_t)}
        try:
            ref = oracle_run(graph, ins)["y"].vals
        except O.OracleError:
            with pytest.raises(T.TosaError):
                run(graph, ins)["y"].numpy()
            continue
        got = run(graph, ins)["y"].numpy()
        refs = O.encode(out_t, ref)
        assert np.array_equal(got.reshape(-1), np.asarray(refs).reshape(-1)), (in_t, out_t, rnd)


def test_require_failure_is_reported():
    """A RESCALE whose input exceeds [-2^(s-1), 2^(s-1)) fails, fused or not,
    and in deferred mode at the next synchronize."""
    x = np.full((1, 4, 4, 8), 100, np.int8)
    w = np.full((8, 1, 1, 8), 100, np.int8)
    rs = (np.full(8, 2 ** 30), np.full(8, 3), 0, False, True)  # shift 3: |value| must be < 4
    graph, out = conv_graph(x, w, np.zeros(8, np.int32), 0, 0, [0, 0, 0, 0], [1, 1], [1, 1], rescale=rs)
    ins = {"x": (x, "INT8")}
    with pytest.raises(O.OracleError):
        oracle_run(graph, ins)
    for fusion in (True, False):
        with pytest.raises(T.TosaError) as e:
            run(graph, ins, fusion)
        assert e.value.kind == "GraphError"
    T.set_option("deferred", 1)
    try:
        r = run(graph, ins)
        with pytest.raises(T.TosaError):
            T.synchronize()
        T.synchronize()  # the error was cleared
        del r
    finally:
        T.set_option("deferred", 0)


def test_residual_fusion_matches_unfused():
    rng = np.random.default_rng(11)
    shape = (2, 7, 9, 24)
    a = rng.integers(-128, 128, size=shape).astype(np.int8)
    b = rng.integers(-128, 128, size=shape).astype(np.int8)
    g = GraphBuilder()
    g.input("a", shape, "INT8")
    g.input("b", shape, "INT8")
    W._rescale(g, "a", g.tensor("ra", shape, "INT32"), 24, rng.integers(2 ** 30, 2 ** 31, 24), [20] * 24, "INT8",
               "INT32", -5, 0, False, True, "x1")
    W._rescale(g, "b", g.tensor("rb", shape, "INT32"), 24, [2 ** 30], [21], "INT8", "INT32", 7, 0, False, False, "x2")
    g.tensor("s", shape, "INT32")
    g.op("ADD", ["ra", "rb"], ["s"])
    W._rescale(g, "s", g.tensor("y", shape, "INT8"), 24, rng.integers(2 ** 30, 2 ** 31, 24), [42] * 24, "INT32",
               "INT8", 0, 3, True, True, "x3")
    graph = g.build(["y"])
    ins = {"a": (a, "INT8"), "b": (b, "INT8")}
    ref = oracle_run(graph, ins)["y"].vals
    for fusion in (True, False):
        assert same_int(run(graph, ins, fusion)["y"].numpy(), ref), fusion


# (channels, input shifts, output shift range, double rounding of a/b/out,
# per-channel a/b/out): shifts >= 9 on the int8 inputs take the residual
# kernel whose REQUIREs are settled on the host; a shift of 8 falls back to
# the per-element kernel.
RESIDUAL = [
    (24, 20, (34, 40), (False, False, True), (True, False, True)),
    (32, 9, (44, 50), (True, True, True), (True, True, False)),
    (96, 12, (42, 47), (False, True, False), (False, True, True)),
    (160, 30, (24, 30), (True, False, True), (True, True, True)),
    (8, 8, (46, 50), (False, False, False), (True, True, True)),
    (1024, 16, (38, 43), (True, True, True), (True, True, True)),
]


@pytest.mark.parametrize("case", range(len(RESIDUAL)))
def test_residual_paths(case):
    c, sin, (slo, shi), dbl, pc = RESIDUAL[case]
    rng = np.random.default_rng(300 + case)
    shape = (3, 5, 7, c)
    a = rng.integers(-128, 128, size=shape).astype(np.int8)
    b = rng.integers(-128, 128, size=shape).astype(np.int8)
    g = GraphBuilder()
    g.input("a", shape, "INT8")
    g.input("b", shape, "INT8")
    ca, cb, co = (c if pc[0] else 1), (c if pc[1] else 1), (c if pc[2] else 1)
    # A shift of 8 admits |a - za| < 128 only: zero input zero points there.
    za, zb = (int(v) for v in rng.integers(-128, 128, 2)) if sin >= 9 else (0, 0)
    W._rescale(g, "a", g.tensor("ra", shape, "INT32"), c, rng.integers(2 ** 30, 2 ** 31, ca), [sin] * ca, "INT8",
               "INT32", za, 0, dbl[0], pc[0], "x1")
    W._rescale(g, "b", g.tensor("rb", shape, "INT32"), c, rng.integers(2 ** 30, 2 ** 31, cb),
               rng.integers(sin, sin + 3, cb), "INT8", "INT32", zb, 0, dbl[1], pc[1], "x2")
    g.tensor("s", shape, "INT32")
    g.op("ADD", ["ra", "rb"], ["s"])
    W._rescale(g, "s", g.tensor("y", shape, "INT8"), c, rng.integers(2 ** 30, 2 ** 31, co),
               rng.integers(slo, shi, co), "INT32", "INT8", 0, int(rng.integers(-128, 128)),
               dbl[2], pc[2], "x3")
    graph = g.build(["y"])
    ins = {"a": (a, "INT8"), "b": (b, "INT8")}
    ref = oracle_run(graph, ins)["y"].vals
    for fusion in (True, False):
        assert same_int(run(graph, ins, fusion)["y"].numpy(), ref), fusion


def test_residual_range_require():
    """An output shift below 32 whose sums fall outside [-2^(s-1), 2^(s-1))
    is apply_scale_32's REQUIRE failure, reported as GraphError."""
    shape = (2, 4, 4, 16)
    a = np.full(shape, 100, np.int8)
    g = GraphBuilder()
    g.input("a", shape, "INT8")
    g.input("b", shape, "INT8")
    W._rescale(g, "a", g.tensor("ra", shape, "INT32"), 16, [2 ** 30], [10], "INT8", "INT32", 0, 0, False, False, "x1")
    W._rescale(g, "b", g.tensor("rb", shape, "INT32"), 16, [2 ** 30], [10], "INT8", "INT32", 0, 0, False, False, "x2")
    g.tensor("s", shape, "INT32")
    g.op("ADD", ["ra", "rb"], ["s"])
    W._rescale(g, "s", g.tensor("y", shape, "INT8"), 16, [2 ** 30], [6], "INT32", "INT8", 0, 0, False, False, "x3")
    graph = g.build(["y"])
    ins = {"a": (a, "INT8"), "b": (a, "INT8")}
    with pytest.raises(O.OracleError):
        oracle_run(graph, ins)
    for fusion in (True, False):
        with pytest.raises(T.TosaError) as e:
            run(graph, ins, fusion)
        assert e.value.kind == "GraphError"


@pytest.mark.parametrize("c", [3, 8, 1280])
def test_avg_pool_int8_paths(c):
    rng = np.random.default_rng(c)
    for k, s, pad in (((3, 3), (1, 1), [1, 1, 1, 1]), ((7, 7), (7, 7), [0, 0, 0, 0]), ((2, 3), (2, 1), [0, 1, 1, 1])):
        ih, iw = 7, 7
        if (ih + pad[0] + pad[1] - k[0]) % s[0] or (iw + pad[2] + pad[3] - k[1]) % s[1]:
            continue
        x = rng.integers(-128, 128, size=(2, ih, iw, c)).astype(np.int8)
        g = GraphBuilder()
        g.input("x", x.shape, "INT8")
        g.const("iz", np.array([-1]), "INT8")
        g.const("oz", np.array([2]), "INT8")
        oh = (ih + pad[0] + pad[1] - k[0]) // s[0] + 1
        ow = (iw + pad[2] + pad[3] - k[1]) // s[1] + 1
        g.tensor("y", [2, oh, ow, c], "INT8")
        g.op("AVG_POOL2D", ["x", "iz", "oz"], ["y"], kernel=list(k), stride=list(s), pad=pad, acc_type="INT32")
        graph = g.build(["y"])
        ins = {"x": (x, "INT8")}
        assert same_int(run(graph, ins)["y"].numpy(), oracle_run(graph, ins)["y"].vals), (k, s, pad)


# ---------------------------------------------------------------------------
# bf16 / fp16 GEMM kernel (K a multiple of 64): batched MATMUL with B as
# [K][N] and 1x1 CONV2D with the float epilogue. fp32 accumulation in another
# order than the reference's: |y - exact| <= 2 K 2^-24 sum|a b| (+ the output
# rounding and the bias add for narrow outputs).
# ---------------------------------------------------------------------------
def _f16_to_torch(bits, dtype):
    import torch
    t = torch.from_numpy(bits.view(np.int16))
    return t.view(torch.bfloat16 if dtype == "BF16" else torch.float16).double()


@pytest.mark.parametrize("dtype", ["BF16", "FP16"])
@pytest.mark.parametrize("dims", [(2, 300, 128, 264), (1, 64, 1280, 1000), (3, 257, 64, 8), (1, 512, 192, 520)])
def test_gemm_f16_matmul(dtype, dims):
    import torch
    batch, h, c, w = dims
    r = np.random.default_rng(sum(dims) + len(dtype))
    a = W._normal(r, (batch, h, c), dtype)
    b = W._normal(r, (batch, c, w), dtype)
    g = GraphBuilder()
    g.input("a", a.shape, dtype)
    g.input("b", b.shape, dtype)
    g.const("az", np.array([0], np.uint16), dtype)
    g.const("bz", np.array([0], np.uint16), dtype)
    g.tensor("y", [batch, h, w], "FP32")
    g.op("MATMUL", ["a", "b", "az", "bz"], ["y"])
    y = run(g.build(["y"]), {"a": (a, dtype), "b": (b, dtype)})["y"].numpy().astype(np.float64)
    ta, tb = _f16_to_torch(a, dtype), _f16_to_torch(b, dtype)
    exact = torch.bmm(ta, tb).numpy()
    absy = torch.bmm(ta.abs(), tb.abs()).numpy()
    assert np.all(np.abs(y - exact) <= 2 * c * 2.0 ** -24 * absy), np.abs(y - exact).max()


@pytest.mark.parametrize("dtype,out_dtype", [("BF16", "FP32"), ("FP16", "FP32"), ("BF16", "BF16"), ("FP16", "FP16")])
@pytest.mark.parametrize("shape", [(2, 13, 17, 128, 200), (1, 28, 28, 64, 512), (3, 5, 7, 256, 24)])
def test_gemm_f16_conv1x1(dtype, out_dtype, shape):
    import torch
    n, h, w_, cin, cout = shape
    r = np.random.default_rng(sum(shape) + len(dtype) + len(out_dtype))
    x = W._normal(r, (n, h, w_, cin), dtype)
    wt = W._normal(r, (cout, 1, 1, cin), dtype)
    g = GraphBuilder()
    g.input("x", x.shape, dtype)
    g.const("w", wt, dtype)
    if out_dtype == "FP32":
        bias = r.standard_normal(cout).astype(np.float32)
        g.const("bias", bias, "FP32")
        bias_f = bias.astype(np.float64)
    else:
        bias_bits = W._normal(r, (cout,), out_dtype)
        g.const("bias", bias_bits, out_dtype)
        bias_f = _f16_to_torch(bias_bits, out_dtype).numpy()
    g.const("zx", np.array([0], np.uint16), dtype)
    g.const("zw", np.array([0], np.uint16), dtype)
    g.tensor("y", [n, h, w_, cout], out_dtype)
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["y"], pad=[0, 0, 0, 0], stride=[1, 1], dilation=[1, 1],
         acc_type="FP32")
    got = run(g.build(["y"]), {"x": (x, dtype)})["y"].numpy()
    if out_dtype != "FP32":
        got = _f16_to_torch(got.view(np.uint16), out_dtype).numpy()
    got = got.astype(np.float64).reshape(-1, cout)
    tx = _f16_to_torch(x, dtype).reshape(-1, cin)
    tw = _f16_to_torch(wt, dtype).reshape(cout, cin)
    acc = (tx @ tw.T).numpy()
    absy = (tx.abs() @ tw.abs().T).numpy()
    exact = acc + bias_f
    u = {"FP32": 0.0, "BF16": 2.0 ** -8, "FP16": 2.0 ** -11}[out_dtype]
    bound = 2 * cin * 2.0 ** -24 * absy + 2.0 ** -24 * np.abs(exact) + 2 * u * (np.abs(acc) + np.abs(exact)) + 1e-30
    assert np.all(np.abs(got - exact) <= bound), np.abs(got - exact).max()


# Stride-1 bf16/fp16 convolutions on the halo kernel's float variant: 3x3 and
# other taps, padding, dilation, ragged output channels, and fp32 / bf16 /
# fp16 outputs. The small shapes take the 64-channel one-tile layout, the
# last one the 128-channel layout; the cfg5 workload test above takes the
# 64-channel two-tile layout.
FLOAT_HALO = [
    # n, h, w, cin, cout, kh, kw, pad, dil
    (2, 28, 28, 128, 128, 3, 3, (1, 1, 1, 1), (1, 1)),
    (1, 14, 14, 256, 200, 3, 3, (1, 1, 1, 1), (1, 1)),
    (2, 20, 30, 64, 96, 5, 5, (2, 2, 2, 2), (1, 1)),
    (1, 16, 40, 48, 40, 1, 3, (0, 0, 1, 1), (1, 1)),
    (3, 12, 12, 32, 64, 3, 3, (2, 2, 2, 2), (2, 2)),
    (1, 9, 61, 16, 136, 2, 2, (0, 1, 1, 0), (1, 1)),
    (43, 4, 4, 16, 384, 3, 3, (1, 1, 1, 1), (1, 1)),
]


@pytest.mark.parametrize("dtype,out_dtype", [("BF16", "FP32"), ("FP16", "FP32"), ("BF16", "BF16"), ("FP16", "FP16")])
@pytest.mark.parametrize("case", range(len(FLOAT_HALO)))
def test_float_halo_conv(dtype, out_dtype, case):
    import torch
    n, h, w_, cin, cout, kh, kw, pad, dil = FLOAT_HALO[case]
    r = np.random.default_rng(8100 + 10 * case + len(dtype) + len(out_dtype))
    oh = h - 1 + pad[0] + pad[1] - (kh - 1) * dil[0] + 1
    ow = w_ - 1 + pad[2] + pad[3] - (kw - 1) * dil[1] + 1
    x = W._normal(r, (n, h, w_, cin), dtype)
    wt = W._normal(r, (cout, kh, kw, cin), dtype)
    g = GraphBuilder()
    g.input("x", x.shape, dtype)
    g.const("w", wt, dtype)
    if out_dtype == "FP32":
        bias = r.standard_normal(cout).astype(np.float32)
        g.const("bias", bias, "FP32")
        bias_f = bias.astype(np.float64)
    else:
        bias_bits = W._normal(r, (cout,), out_dtype)
        g.const("bias", bias_bits, out_dtype)
        bias_f = _f16_to_torch(bias_bits, out_dtype).numpy()
    g.const("zx", np.array([0], np.uint16), dtype)
    g.const("zw", np.array([0], np.uint16), dtype)
    g.tensor("y", [n, oh, ow, cout], out_dtype)
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["y"], pad=list(pad), stride=[1, 1], dilation=list(dil),
         acc_type="FP32")
    got = run(g.build(["y"]), {"x": (x, dtype)})["y"].numpy()
    if out_dtype != "FP32":
        got = _f16_to_torch(got.view(np.uint16), out_dtype).numpy()
    got = got.astype(np.float64)
    tx = _f16_to_torch(x, dtype).permute(0, 3, 1, 2)
    tw = _f16_to_torch(wt, dtype).permute(0, 3, 1, 2)
    xp = torch.nn.functional.pad(tx, (pad[2], pad[3], pad[0], pad[1]))
    acc = torch.nn.functional.conv2d(xp, tw, dilation=dil).permute(0, 2, 3, 1).numpy()
    absy = torch.nn.functional.conv2d(xp.abs(), tw.abs(), dilation=dil).permute(0, 2, 3, 1).numpy()
    exact = acc + bias_f
    K = kh * kw * cin
    u = {"FP32": 0.0, "BF16": 2.0 ** -8, "FP16": 2.0 ** -11}[out_dtype]
    bound = 2 * K * 2.0 ** -24 * absy + 2.0 ** -24 * np.abs(exact) + 2 * u * (np.abs(acc) + np.abs(exact)) + 1e-30
    assert np.all(np.abs(got - exact) <= bound), np.abs(got - exact).max()
