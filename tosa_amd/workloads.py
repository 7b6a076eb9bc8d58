"""Synthetic TOSA graphs of the benchmark workloads, with seeded random data.

Each builder returns (graph bytes, {input name: (array, dtype)}, info). Values
are drawn from numpy's PCG64 with seed 1000*config + tensor index, so tests,
the benchmark and the CPU baseline see identical inputs.

Workloads:
  conv_rescale   int8 CONV2D + per-channel DOUBLE_ROUND RESCALE to int8
                 (x U[-128,127], zx=-3; w U, zw=0; bias U[-2^15,2^15];
                 multiplier U[2^30, 2^31), shift U[30,40], output zp 5)
  matmul_rescale int8 batched MATMUL + per-tensor SINGLE_ROUND RESCALE
  depthwise      int8 DEPTHWISE_CONV2D 3x3 stride 2 + per-channel RESCALE
  avg_pool       int8 AVG_POOL2D
  mobilenet_v2   int8 MobileNetV2-style graph (stem, 17 inverted residual
                 blocks, head, global pool, fully connected MATMUL)
  float_conv / float_matmul   bf16/fp16 CONV2D and MATMUL, fp32 accumulators
"""

from __future__ import annotations

import math

import numpy as np

from .tosa_writer import GraphBuilder


def rng(cfg: int, idx: int) -> np.random.Generator:
    return np.random.default_rng(1000 * cfg + idx)


def i8(r, shape):
    return r.integers(-128, 128, size=shape, dtype=np.int64).astype(np.int8)


def _rescale(g, src, dst, shape_last, mult, shift, in_dtype, out_dtype, in_zp, out_zp, double, per_channel, tag):
    m = g.const(f"{tag}_m", np.asarray(mult, np.int32).reshape(-1), "INT32")
    s = g.const(f"{tag}_s", np.asarray(shift, np.int8).reshape(-1), "INT8")
    iz = g.const(f"{tag}_izp", np.array([in_zp]), in_dtype)
    oz = g.const(f"{tag}_ozp", np.array([out_zp]), out_dtype)
    g.op("RESCALE", [src, m, s, iz, oz], [dst], scale32=1, rounding_mode="DOUBLE_ROUND" if double else "SINGLE_ROUND",
         per_channel=int(per_channel))
    return dst


def conv_rescale(n=1, h=56, w=56, cin=64, cout=64, k=3, stride=1, pad=(1, 1, 1, 1), cfg=1, zx=-3, zw=0, ozp=5):
    """CONV2D + per-channel RESCALE (the first benchmark config at its default
    sizes; ResNet-scale layers with other sizes)."""
    x = i8(rng(cfg, 0), (n, h, w, cin))
    wt = i8(rng(cfg, 1), (cout, k, k, cin))
    bias = rng(cfg, 2).integers(-2 ** 15, 2 ** 15 + 1, size=cout).astype(np.int32)
    mult = rng(cfg, 3).integers(2 ** 30, 2 ** 31, size=cout).astype(np.int64)
    shift = rng(cfg, 4).integers(30, 41, size=cout).astype(np.int8)
    oh = (h - 1 + pad[0] + pad[1] - (k - 1)) // stride + 1
    ow = (w - 1 + pad[2] + pad[3] - (k - 1)) // stride + 1
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("w", wt, "INT8")
    g.const("bias", bias, "INT32")
    g.const("zx", np.array([zx]), "INT8")
    g.const("zw", np.array([zw]), "INT8")
    g.tensor("acc", [n, oh, ow, cout], "INT32")
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["acc"], pad=list(pad), stride=[stride, stride],
         dilation=[1, 1], acc_type="INT32")
    g.tensor("y", [n, oh, ow, cout], "INT8")
    _rescale(g, "acc", "y", cout, mult, shift, "INT32", "INT8", 0, ozp, True, True, "rs")
    macs = n * oh * ow * cout * k * k * cin
    info = {"macs": macs, "ops": 2 * macs, "bytes": x.nbytes + wt.nbytes + n * oh * ow * cout + cout * 9,
            "out": "y", "shape": [n, oh, ow, cout]}
    return g.build(["y"]), {"x": (x, "INT8")}, info


def matmul_rescale(batch=8, h=512, c=1024, w=1024, cfg=2, azp=-7, bzp=2):
    a = i8(rng(cfg, 0), (batch, h, c))
    b = i8(rng(cfg, 1), (batch, c, w))
    g = GraphBuilder()
    g.input("a", a.shape, "INT8")
    g.input("b", b.shape, "INT8")
    g.const("azp", np.array([azp]), "INT8")
    g.const("bzp", np.array([bzp]), "INT8")
    g.tensor("acc", [batch, h, w], "INT32")
    g.op("MATMUL", ["a", "b", "azp", "bzp"], ["acc"])
    g.tensor("y", [batch, h, w], "INT8")
    _rescale(g, "acc", "y", w, [1518500250], [38], "INT32", "INT8", 0, 0, False, False, "rs")
    macs = batch * h * c * w
    info = {"macs": macs, "ops": 2 * macs, "bytes": a.nbytes + b.nbytes + batch * h * w, "out": "y"}
    return g.build(["y"]), {"a": (a, "INT8"), "b": (b, "INT8")}, info


def depthwise(n=32, h=112, w=112, c=144, stride=2, pad=(0, 1, 0, 1), cfg=3):
    x = i8(rng(cfg, 0), (n, h, w, c))
    wt = i8(rng(cfg, 1), (3, 3, c, 1))
    bias = rng(cfg, 2).integers(-2 ** 15, 2 ** 15 + 1, size=c).astype(np.int32)
    mult = rng(cfg, 3).integers(2 ** 30, 2 ** 31, size=c).astype(np.int64)
    shift = rng(cfg, 4).integers(30, 41, size=c).astype(np.int8)
    oh = (h - 1 + pad[0] + pad[1] - 2) // stride + 1
    ow = (w - 1 + pad[2] + pad[3] - 2) // stride + 1
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("w", wt, "INT8")
    g.const("bias", bias, "INT32")
    g.const("zx", np.array([0]), "INT8")
    g.const("zw", np.array([0]), "INT8")
    g.tensor("acc", [n, oh, ow, c], "INT32")
    g.op("DEPTHWISE_CONV2D", ["x", "w", "bias", "zx", "zw"], ["acc"], pad=list(pad), stride=[stride, stride],
         dilation=[1, 1], acc_type="INT32")
    g.tensor("y", [n, oh, ow, c], "INT8")
    _rescale(g, "acc", "y", c, mult, shift, "INT32", "INT8", 0, 5, True, True, "rs")
    macs = n * oh * ow * c * 9
    info = {"macs": macs, "ops": 2 * macs, "bytes": x.nbytes + n * oh * ow * c + wt.nbytes + 9 * c, "out": "y"}
    return g.build(["y"]), {"x": (x, "INT8")}, info


def avg_pool(n=32, h=7, w=7, c=1280, k=7, stride=7, cfg=3, izp=-1, ozp=2):
    x = i8(rng(cfg, 10), (n, h, w, c))
    oh = (h - k) // stride + 1
    ow = (w - k) // stride + 1
    g = GraphBuilder()
    g.input("x", x.shape, "INT8")
    g.const("izp", np.array([izp]), "INT8")
    g.const("ozp", np.array([ozp]), "INT8")
    g.tensor("y", [n, oh, ow, c], "INT8")
    g.op("AVG_POOL2D", ["x", "izp", "ozp"], ["y"], kernel=[k, k], stride=[stride, stride], pad=[0, 0, 0, 0],
         acc_type="INT32")
    info = {"ops": x.size, "bytes": x.nbytes + n * oh * ow * c, "out": "y"}
    return g.build(["y"]), {"x": (x, "INT8")}, info


# ---------------------------------------------------------------------------
# int8 MobileNetV2-style graph
# ---------------------------------------------------------------------------

MOBILENET_V2_BLOCKS = [(1, 16, 1, 1), (6, 24, 2, 2), (6, 32, 3, 2), (6, 64, 4, 2), (6, 96, 3, 1), (6, 160, 3, 2),
                       (6, 320, 1, 1)]


class _Net:
    def __init__(self, g: GraphBuilder, cfg: int):
        self.g = g
        self.cfg = cfg
        self.k = 0  # tensor counter, also the seed index
        self.macs = 0
        self.bytes = 0

    def r(self):
        self.k += 1
        return rng(self.cfg, self.k)

    def name(self, p):
        self.k += 1
        return f"{p}{self.k}"

    def requant(self, fan_in, channels):
        """Per-channel (multiplier, shift) for an int32 sum of `fan_in` products
        of roughly uniform int8 values, aimed at an output spread of ~32."""
        r = self.r()
        mult = r.integers(2 ** 30, 2 ** 31, size=channels)
        sigma = 73.0 * 73.0 * math.sqrt(fan_in)
        shift = np.clip(np.round(np.log2(mult * sigma / 32.0)), 2, 62).astype(np.int8)
        return mult, shift

    def conv(self, x, xzp, shape, cout, k, stride, depthwise=False, clamp=True):
        n, h, w, cin = shape
        if stride == 2:
            pad = [0, 1, 0, 1] if k == 3 else [0, 0, 0, 0]
        else:
            pad = [k // 2] * 4
        oh = (h - 1 + pad[0] + pad[1] - (k - 1)) // stride + 1
        ow = (w - 1 + pad[2] + pad[3] - (k - 1)) // stride + 1
        g = self.g
        r = self.r()
        if depthwise:
            wt = r.integers(-128, 128, size=(k, k, cin, 1)).astype(np.int8)
            cout = cin
            op = "DEPTHWISE_CONV2D"
            fan_in = k * k
        else:
            wt = r.integers(-128, 128, size=(cout, k, k, cin)).astype(np.int8)
            op = "CONV2D"
            fan_in = k * k * cin
        wzp = int(self.r().integers(-4, 5))
        bias = self.r().integers(-2 ** 12, 2 ** 12, size=cout).astype(np.int32)
        wn, bn, zxn, zwn = (self.name("w"), self.name("b"), self.name("zx"), self.name("zw"))
        g.const(wn, wt, "INT8")
        g.const(bn, bias, "INT32")
        g.const(zxn, np.array([xzp]), "INT8")
        g.const(zwn, np.array([wzp]), "INT8")
        acc = g.tensor(self.name("acc"), [n, oh, ow, cout], "INT32")
        g.op(op, [x, wn, bn, zxn, zwn], [acc], pad=pad, stride=[stride, stride], dilation=[1, 1], acc_type="INT32")
        mult, shift = self.requant(fan_in, cout)
        ozp = int(self.r().integers(-16, 17))
        y = g.tensor(self.name("q"), [n, oh, ow, cout], "INT8")
        _rescale(g, acc, y, cout, mult, shift, "INT32", "INT8", 0, ozp, True, True, self.name("rs"))
        self.macs += n * oh * ow * cout * fan_in
        self.bytes += n * h * w * cin + n * oh * ow * cout + wt.size
        if clamp:
            # CLAMP in place of ReLU6: from the zero point up.
            c = g.tensor(self.name("c"), [n, oh, ow, cout], "INT8")
            g.op("CLAMP", [y], [c], min_val=bytes([ozp & 0xFF] + [0] * 7), max_val=bytes([127] + [0] * 7))
            y = c
        return y, ozp, [n, oh, ow, cout]

    def residual(self, a, azp, b, bzp, shape):
        g = self.g
        n, h, w, c = shape
        outs = []
        for src, zp in ((a, azp), (b, bzp)):
            m = self.r().integers(2 ** 30, 2 ** 31, size=1)
            t = g.tensor(self.name("r"), shape, "INT32")
            _rescale(g, src, t, c, m, [20], "INT8", "INT32", zp, 0, False, False, self.name("rr"))
            outs.append(t)
        s = g.tensor(self.name("sum"), shape, "INT32")
        g.op("ADD", outs, [s])
        ozp = int(self.r().integers(-16, 17))
        y = g.tensor(self.name("res"), shape, "INT8")
        m = self.r().integers(2 ** 30, 2 ** 31, size=1)
        _rescale(g, s, y, c, m, [42], "INT32", "INT8", 0, ozp, True, False, self.name("ro"))
        self.bytes += 3 * n * h * w * c
        return y, ozp


def mobilenet_v2(n=64, cfg=4, classes=1000):
    """int8 MobileNetV2-style graph: input [n,224,224,3]."""
    g = GraphBuilder("mobilenet_v2")
    net = _Net(g, cfg)
    x = i8(rng(cfg, 0), (n, 224, 224, 3))
    xzp = int(rng(cfg, 999).integers(-128, 128))
    g.input("input", x.shape, "INT8")
    y, zp, shape = net.conv("input", xzp, list(x.shape), 32, 3, 2)
    cin = 32
    for t, c, reps, s in MOBILENET_V2_BLOCKS:
        for i in range(reps):
            stride = s if i == 0 else 1
            inp, inp_zp, inp_shape = y, zp, shape
            h = y
            hzp, hshape = zp, shape
            if t != 1:
                h, hzp, hshape = net.conv(h, hzp, hshape, cin * t, 1, 1)
            h, hzp, hshape = net.conv(h, hzp, hshape, None, 3, stride, depthwise=True)
            h, hzp, hshape = net.conv(h, hzp, hshape, c, 1, 1, clamp=False)
            if stride == 1 and cin == c:
                h, hzp = net.residual(inp, inp_zp, h, hzp, hshape)
            y, zp, shape = h, hzp, hshape
            cin = c
    y, zp, shape = net.conv(y, zp, shape, 1280, 1, 1)
    pooled = g.tensor("pooled", [n, 1, 1, 1280], "INT8")
    g.const("pool_izp", np.array([zp]), "INT8")
    g.const("pool_ozp", np.array([zp]), "INT8")
    g.op("AVG_POOL2D", [y, "pool_izp", "pool_ozp"], [pooled], kernel=[7, 7], stride=[7, 7], pad=[0, 0, 0, 0],
         acc_type="INT32")
    g.const_shape("flat_shape", [1, n, 1280])
    flat = g.tensor("flat", [1, n, 1280], "INT8")
    g.op("RESHAPE", [pooled, "flat_shape"], [flat])
    fc = rng(cfg, 998).integers(-128, 128, size=(1, 1280, classes)).astype(np.int8)
    g.const("fc_w", fc, "INT8")
    g.const("fc_azp", np.array([zp]), "INT8")
    g.const("fc_bzp", np.array([0]), "INT8")
    g.tensor("logits", [1, n, classes], "INT32")
    g.op("MATMUL", [flat, "fc_w", "fc_azp", "fc_bzp"], ["logits"])
    net.macs += n * 1280 * classes
    info = {"macs": net.macs, "ops": 2 * net.macs, "bytes": net.bytes, "out": "logits", "images": n}
    return g.build(["logits"]), {"input": (x, "INT8")}, info


# ---------------------------------------------------------------------------
# bf16 / fp16
# ---------------------------------------------------------------------------

def _normal(r, shape, dtype):
    import torch  # RNE conversion to bf16/fp16
    v = torch.from_numpy(r.standard_normal(size=shape).astype(np.float32))
    t = v.to(torch.bfloat16 if dtype == "BF16" else torch.float16)
    return t.view(torch.int16).numpy().view(np.uint16)


def float_conv(dtype="BF16", n=64, h=28, w=28, cin=128, cout=128, k=3, cfg=5, out_dtype="FP32"):
    pad = [k // 2] * 4
    x = _normal(rng(cfg, 0), (n, h, w, cin), dtype)
    wt = _normal(rng(cfg, 1 if k == 3 else 2), (cout, k, k, cin), dtype)
    bias = rng(cfg, 3).standard_normal(cout).astype(np.float32)
    g = GraphBuilder()
    g.input("x", x.shape, dtype)
    g.const("w", wt, dtype)
    if out_dtype == "FP32":
        g.const("bias", bias, "FP32")
    else:
        g.const("bias", _normal(rng(cfg, 3), (cout,), out_dtype), out_dtype)
    g.const("zx", np.array([0], np.uint16), dtype)
    g.const("zw", np.array([0], np.uint16), dtype)
    g.tensor("y", [n, h, w, cout], out_dtype)
    g.op("CONV2D", ["x", "w", "bias", "zx", "zw"], ["y"], pad=pad, stride=[1, 1], dilation=[1, 1], acc_type="FP32")
    macs = n * h * w * cout * k * k * cin
    es = 4 if out_dtype == "FP32" else 2
    info = {"macs": macs, "ops": 2 * macs, "bytes": x.nbytes + wt.nbytes + n * h * w * cout * es, "out": "y"}
    return g.build(["y"]), {"x": (x, dtype)}, info


def conv_i16(n=64, h=28, w=28, cin=128, cout=128, k=3, cfg=6):
    """int16 x int8 CONV2D into INT48 (the reference's i16 conv path) with
    the per-channel RESCALE to int16 an int16 network requantises with
    (apply_scale_16): the ResNet-scale layer at 16-bit activations."""
    r = rng(cfg, 0)
    x = r.integers(-2 ** 15, 2 ** 15, (n, h, w, cin)).astype(np.int16)
    wt = i8(rng(cfg, 1), (cout, k, k, cin))
    # Sums of ~1152 products of uniform int16 and int8 values spread to
    # ~2^25.5; multiplier ~2^14.5 and shifts 27-30 bring them to ~2^12.
    bias = rng(cfg, 2).integers(-2 ** 24, 2 ** 24, cout)
    mult = rng(cfg, 3).integers(2 ** 14, 2 ** 15, cout).astype(np.int16)
    shift = rng(cfg, 4).integers(27, 31, cout).astype(np.int8)
    pad = [k // 2] * 4
    g = GraphBuilder()
    g.input("x", x.shape, "INT16")
    g.const("w", wt, "INT8")
    g.const("b", bias, "INT48")
    g.const("zx", np.array([0]), "INT16")
    g.const("zw", np.array([0]), "INT8")
    g.tensor("acc", [n, h, w, cout], "INT48")
    g.op("CONV2D", ["x", "w", "b", "zx", "zw"], ["acc"], pad=pad, stride=[1, 1], dilation=[1, 1], acc_type="INT48")
    g.const("m", mult, "INT16")
    g.const("s", shift, "INT8")
    g.const("iz", np.array([0]), "INT48")
    g.const("oz", np.array([0]), "INT16")
    g.tensor("y", [n, h, w, cout], "INT16")
    g.op("RESCALE", ["acc", "m", "s", "iz", "oz"], ["y"], scale32=0, rounding_mode="SINGLE_ROUND", per_channel=1)
    macs = n * h * w * cout * k * k * cin
    info = {"macs": macs, "ops": 2 * macs, "bytes": x.nbytes + wt.nbytes + n * h * w * cout * 2, "out": "y"}
    return g.build(["y"]), {"x": (x, "INT16")}, info


def float_matmul(dtype="BF16", batch=16, h=2048, c=2048, w=2048, cfg=5):
    a = _normal(rng(cfg, 10), (batch, h, c), dtype)
    b = _normal(rng(cfg, 11), (batch, c, w), dtype)
    g = GraphBuilder()
    g.input("a", a.shape, dtype)
    g.input("b", b.shape, dtype)
    g.const("azp", np.array([0], np.uint16), dtype)
    g.const("bzp", np.array([0], np.uint16), dtype)
    g.tensor("y", [batch, h, w], "FP32")
    g.op("MATMUL", ["a", "b", "azp", "bzp"], ["y"])
    macs = batch * h * c * w
    info = {"macs": macs, "ops": 2 * macs, "bytes": a.nbytes + b.nbytes + batch * h * w * 4, "out": "y"}
    return g.build(["y"]), {"a": (a, dtype), "b": (b, dtype)}, info
