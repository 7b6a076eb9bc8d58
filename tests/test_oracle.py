"""Pins the CPU oracle (oracle/) before anything is checked against it.

* every positive golden case of the hot-path operators and the networks,
  bit-exact (expected outputs come from ARM's TOSA reference model);
* the reference's own known-answer test for reciprocal_scale/apply_scale_32
  (src/ops/quant.rs:38-48);
* apply_scale_32 single rounding against exact rational round-half-up;
* the f16/bf16/fp8 codecs against independent converters (numpy, torch);
* integer CONV2D / DEPTHWISE_CONV2D / MATMUL against a vectorised numpy
  brute force (a different formulation: shifted windows, int64, mod 2^32).
"""

import ctypes
from fractions import Fraction

import numpy as np
import pytest

from oracle import oracle as O
from oracle import tosa_reader as fb
from tests.helpers import Case, case_dirs, case_id, mismatches

POSITIVE = [d for d in case_dirs("conformance") + case_dirs("networks") if not Case(d).expected_failure]


@pytest.mark.parametrize("d", POSITIVE, ids=case_id)
def test_oracle_matches_golden(d):
    c = Case(d)
    ins = {n: O.T(dt, list(a.shape), O.decode(dt, a)) for n, (a, dt) in c.inputs().items()}
    outs = O.run_block(c.block, ins)
    for n, (exp, dt) in c.expected().items():
        got = outs[n]
        assert list(exp.shape) == got.shape
        g = O.encode(dt, got.vals.reshape(got.shape) if got.shape else got.vals.reshape(()))
        bad = mismatches(g, exp, dt)
        assert bad.size == 0, f"{n}: {bad.size} of {exp.size} differ, first at {bad[:5]}"


def _scale32(v, m, s, dbl=False):
    out = ctypes.c_int32()
    st = O.lib().orc_apply_scale_32(v, m, s, int(dbl), ctypes.byref(out))
    return None if st else out.value


def test_reciprocal_scale_divides():
    # src/ops/quant.rs:38-48
    for count in range(1, 65):
        sh = ctypes.c_int32()
        m = O.lib().orc_reciprocal_scale(count, ctypes.byref(sh))
        for s in (-1000, -7, 0, 5, 999):
            q = _scale32(s, m, sh.value)
            assert abs(q - s / count) <= 0.5 + 1e-9, (s, count, q)


def test_apply_scale_32_is_round_half_up():
    rng = np.random.default_rng(7)
    for _ in range(20000):
        s = int(rng.integers(2, 63))
        m = int(rng.integers(0, 2 ** 31))
        lim = min(2 ** 31, 2 ** (s - 1))
        v = int(rng.integers(-lim, lim))
        got = _scale32(v, m, s)
        exact = Fraction(v * m, 2 ** s) + Fraction(1, 2)
        want = exact.numerator // exact.denominator  # floor
        if -(2 ** 31) <= want < 2 ** 31:
            assert got == want, (v, m, s)
        else:
            assert got is None


def test_apply_scale_32_require_failures():
    assert _scale32(0, -1, 10) is None           # negative multiplier
    assert _scale32(0, 1, 1) is None             # shift below 2
    assert _scale32(0, 1, 63) is None            # shift above 62
    assert _scale32(2 ** 9, 1, 10) is None       # value outside [-2^(s-1), 2^(s-1))
    assert _scale32(-(2 ** 9), 1, 10) == 0
    assert _scale32(2 ** 30, 2 ** 31 - 1, 2) is None  # result exceeds int32


def _random_f32(n, seed):
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)
    special = np.array([0, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0x477FE000, 0x477FF000, 0x477FEFFF,
                        0x33000000, 0x33000001, 0x387FC000, 0x7F7FFFFF, 0x00000001, 0x7F7F8000], dtype=np.uint32)
    return np.concatenate([b, special]).view(np.float32)


def test_f16_codec_matches_numpy():
    x = _random_f32(1 << 20, 1)
    # Also sweep the range that maps onto f16 finely.
    x = np.concatenate([x, (np.random.default_rng(2).standard_normal(1 << 18) * 3e4).astype(np.float32),
                        np.ldexp(np.random.default_rng(3).random(1 << 16), -24).astype(np.float32)])
    got = O.encode("FP16", x).view(np.uint16)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all(got[nan] & 0x3FF)
    # decode is exact
    h = np.arange(1 << 16, dtype=np.uint16)
    dec = O.decode("FP16", h)
    ref = h.view(np.float16).astype(np.float32)
    ok = np.isnan(ref)
    assert np.array_equal(dec[~ok], ref[~ok]) and np.all(np.isnan(dec[ok]))


def test_bf16_codec_matches_torch():
    torch = pytest.importorskip("torch")
    x = _random_f32(1 << 20, 4)
    got = O.encode("BF16", x).view(np.uint16)
    want = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    nan = np.isnan(x)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7F80) == 0x7F80) and np.all(got[nan] & 0x7F)


@pytest.mark.parametrize("fmt", ["FP8E4M3", "FP8E5M2"])
def test_fp8_codec_matches_torch(fmt):
    torch = pytest.importorskip("torch")
    td = torch.float8_e4m3fn if fmt == "FP8E4M3" else torch.float8_e5m2
    x = np.concatenate([_random_f32(1 << 18, 5), (np.random.default_rng(6).standard_normal(1 << 16) * 300).astype(np.float32)])
    got = O.encode(fmt, x)
    want = torch.from_numpy(x.copy()).to(td).view(torch.uint8).numpy()
    nan_x = np.isnan(x)
    dec_w = torch.from_numpy(want.copy()).view(td).float().numpy()
    dec_g = O.decode(fmt, got)
    same = (got == want) | (np.isnan(dec_w) & np.isnan(dec_g))
    assert same[~nan_x].all()
    assert np.isnan(dec_g[nan_x]).all()
    codes = np.arange(256, dtype=np.uint8)
    a = O.decode(fmt, codes)
    b = torch.from_numpy(codes.copy()).view(td).float().numpy()
    assert np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)])


# ---------------------------------------------------------------------------
# Integer brute force
# ---------------------------------------------------------------------------

def conv_bruteforce(x, w, bias, zx, zw, pad, stride, dil, depthwise=False):
    """NHWC int64 conv by shifted windows: taps outside the input are masked
    out, which equals skipping them."""
    n, ih, iw, c = x.shape
    if depthwise:
        kh, kw, _, m = w.shape
        oc = c * m
    else:
        oc, kh, kw, _ = w.shape
    oh = (ih - 1 + pad[0] + pad[1] - (kh - 1) * dil[0]) // stride[0] + 1
    ow = (iw - 1 + pad[2] + pad[3] - (kw - 1) * dil[1]) // stride[1] + 1
    xs = x.astype(np.int64) - zx
    ws = w.astype(np.int64) - zw
    acc = np.zeros((n, oh, ow, oc), dtype=np.int64)
    oy = np.arange(oh)[:, None]
    ox = np.arange(ow)[None, :]
    for ky in range(kh):
        for kx in range(kw):
            iy = oy * stride[0] + ky * dil[0] - pad[0]
            ix = ox * stride[1] + kx * dil[1] - pad[2]
            valid = (iy >= 0) & (iy < ih) & (ix >= 0) & (ix < iw)
            win = xs[:, np.clip(iy, 0, ih - 1), np.clip(ix, 0, iw - 1), :] * valid[None, :, :, None]
            if depthwise:
                acc += (win[..., :, None] * ws[ky, kx][None, None, None]).reshape(n, oh, ow, oc)
            else:
                acc += np.einsum("nyxc,oc->nyxo", win, ws[:, ky, kx, :])
    acc = acc + bias.astype(np.int64)
    return ((acc + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int64)


@pytest.mark.parametrize("seed", range(12))
def test_conv2d_int_matches_bruteforce(seed):
    rng = np.random.default_rng(100 + seed)
    n, ih, iw, ic, oc = 2, int(rng.integers(3, 9)), int(rng.integers(3, 9)), int(rng.integers(1, 9)), int(rng.integers(1, 7))
    kh, kw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    dil = [int(rng.integers(1, 3)), int(rng.integers(1, 3))]
    stride = [int(rng.integers(1, 3)), int(rng.integers(1, 3))]
    pad = [int(v) for v in rng.integers(0, 3, size=4)]
    # make the extents exact
    for d, (i, k) in enumerate(((ih, kh), (iw, kw))):
        full = i - 1 + pad[2 * d] + pad[2 * d + 1] - (k - 1) * dil[d]
        if full < 0:
            pad[2 * d + 1] += -full
            full = 0
        pad[2 * d + 1] += (-full) % stride[d]
    x = rng.integers(-128, 128, size=(n, ih, iw, ic))
    w = rng.integers(-128, 128, size=(oc, kh, kw, ic))
    bias = rng.integers(-2 ** 31, 2 ** 31, size=oc)
    zx, zw = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    got = O.conv2d(O.T("INT8", x.shape, x), O.T("INT8", w.shape, w), O.T("INT32", bias.shape, bias), zx, zw,
                   pad, stride, dil, "INT32", "INT32")
    want = conv_bruteforce(x, w, bias, zx, zw, pad, stride, dil)
    assert got.shape == list(want.shape)
    assert np.array_equal(got.vals.reshape(want.shape), want)


def wrap32(v):
    return ((v + 2 ** 31) % 2 ** 32 - 2 ** 31).astype(np.int64)


@pytest.mark.parametrize("seed", range(8))
def test_conv3d_int_matches_bruteforce(seed):
    # Depth slices of CONV3D are CONV2Ds: the 3-D sum equals the sum over kd
    # of 2-D brute-force convolutions of the matching input depth slices.
    rng = np.random.default_rng(700 + seed)
    n, idp, ih, iw, ic, oc = 2, int(rng.integers(2, 6)), int(rng.integers(3, 7)), int(rng.integers(3, 7)), \
        int(rng.integers(1, 6)), int(rng.integers(1, 5))
    kd, kh, kw = int(rng.integers(1, 4)), int(rng.integers(1, 4)), int(rng.integers(1, 4))
    stride = [int(v) for v in rng.integers(1, 3, size=3)]
    dil = [int(v) for v in rng.integers(1, 3, size=3)]
    pad = [int(v) for v in rng.integers(0, 3, size=6)]
    for d, (i, k) in enumerate(((idp, kd), (ih, kh), (iw, kw))):
        full = i - 1 + pad[2 * d] + pad[2 * d + 1] - (k - 1) * dil[d]
        if full < 0:
            pad[2 * d + 1] += -full
            full = 0
        pad[2 * d + 1] += (-full) % stride[d]
    x = rng.integers(-128, 128, size=(n, idp, ih, iw, ic))
    w = rng.integers(-128, 128, size=(oc, kd, kh, kw, ic))
    bias = rng.integers(-2 ** 31, 2 ** 31, size=oc)
    zx, zw = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    got = O.conv3d(O.T("INT8", x.shape, x), O.T("INT8", w.shape, w), O.T("INT32", bias.shape, bias), zx, zw,
                   pad, stride, dil, "INT32")
    od = (idp - 1 + pad[0] + pad[1] - (kd - 1) * dil[0]) // stride[0] + 1
    oh = (ih - 1 + pad[2] + pad[3] - (kh - 1) * dil[1]) // stride[1] + 1
    ow = (iw - 1 + pad[4] + pad[5] - (kw - 1) * dil[2]) // stride[2] + 1
    want = None
    for z in range(od):
        plane = np.zeros((n, oh, ow, oc), dtype=np.int64)
        for k in range(kd):
            iz = z * stride[0] + k * dil[0] - pad[0]
            if not 0 <= iz < idp:
                continue
            # a 2-D convolution of this depth slice with the k-th kernel plane
            # (zero bias, unwrapped: the sum is wrapped once at the end)
            c2 = conv_bruteforce(x[:, iz], w[:, k], np.zeros(oc, np.int64), zx, zw, pad[2:], stride[1:], dil[1:])
            plane = plane + c2
        acc = np.asarray(plane, dtype=np.int64) + bias.astype(np.int64)
        want = acc[:, None] if want is None else np.concatenate([want, acc[:, None]], axis=1)
    # conv_bruteforce wraps each partial sum to int32; wrapping is additive mod 2^32
    assert np.array_equal(wrap32(got.vals), wrap32(want.reshape(-1)))
    assert got.shape == [n, od] + list(want.shape[2:])


@pytest.mark.parametrize("seed", range(8))
def test_transpose_conv2d_int_matches_scatter_form(seed):
    # The reference gathers (output reads input where (o - pad - k) / s is
    # exact); the scatter form adds every input pixel's products into output
    # (i s + k + pad), dropping what falls outside a cropped (negative pad)
    # output.
    rng = np.random.default_rng(800 + seed)
    n, ih, iw, ic, oc = 2, int(rng.integers(2, 6)), int(rng.integers(2, 6)), int(rng.integers(1, 6)), \
        int(rng.integers(1, 5))
    kh, kw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
    stride = [int(rng.integers(1, 4)), int(rng.integers(1, 4))]
    out_pad = [int(rng.integers(-kh + 1, 3)), int(rng.integers(-kh + 1, 3)), int(rng.integers(-kw + 1, 3)),
               int(rng.integers(-kw + 1, 3))]
    oh = (ih - 1) * stride[0] + out_pad[0] + out_pad[1] + kh
    ow = (iw - 1) * stride[1] + out_pad[2] + out_pad[3] + kw
    if oh < 1 or ow < 1:
        pytest.skip("empty output for this draw")
    x = rng.integers(-128, 128, size=(n, ih, iw, ic))
    w = rng.integers(-128, 128, size=(oc, kh, kw, ic))
    bias = rng.integers(-2 ** 31, 2 ** 31, size=oc)
    zx, zw = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    got = O.transpose_conv2d(O.T("INT8", x.shape, x), O.T("INT8", w.shape, w), O.T("INT32", bias.shape, bias), zx,
                             zw, out_pad, stride, "INT32")
    want = np.zeros((n, oh, ow, oc), dtype=np.int64)
    xs, ws = x.astype(np.int64) - zx, w.astype(np.int64) - zw
    for y in range(ih):
        for xx in range(iw):
            for ky in range(kh):
                for kx in range(kw):
                    oy, ox = y * stride[0] + ky + out_pad[0], xx * stride[1] + kx + out_pad[2]
                    if 0 <= oy < oh and 0 <= ox < ow:
                        want[:, oy, ox, :] += xs[:, y, xx, :] @ ws[:, ky, kx, :].T
    want += bias.astype(np.int64)
    assert got.shape == [n, oh, ow, oc]
    assert np.array_equal(got.vals, wrap32(want.reshape(-1)))


def test_max_pool_and_cast_known_answers():
    # MAX_POOL2D: padding never wins (a window of negatives next to the pad
    # keeps its own maximum), ties keep the running value (-0 before +0), NaN
    # per mode; CAST: saturation at the FP16-rounded INT16 bound 32768 and
    # round half to even.
    x = np.array([-5.0, -3.0, -0.0, 0.0, np.nan, 2.0], np.float32).reshape(1, 1, 6, 1)
    t = O.T("FP32", [1, 1, 6, 1], x.reshape(-1))
    prop = O.max_pool2d(t, [1, 2], [1, 2], [0, 0, 0, 0], 1).vals
    ign = O.max_pool2d(t, [1, 2], [1, 2], [0, 0, 0, 0], 2).vals
    assert prop[0] == -3.0 and np.signbit(prop[1]) and np.isnan(prop[2])
    assert ign[0] == -3.0 and ign[2] == 2.0
    padded = O.max_pool2d(O.T("INT8", [1, 1, 2, 1], np.array([-7, -9])), [1, 2], [1, 1], [0, 0, 1, 0], 1).vals
    assert list(padded) == [-7, -7]
    h = O.T("FP16", [6], np.array([32767.0, 40000.0, -40000.0, 2.5, 3.5, -2.5], np.float32))
    assert list(O.cast(h, "INT16").vals) == [32767, 32767, -32768, 2, 4, -2]
    assert list(O.cast(O.T("INT32", [2], np.array([300, -129])), "INT8").vals) == [44, 127]


@pytest.mark.parametrize("seed", range(8))
def test_depthwise_int_matches_bruteforce(seed):
    rng = np.random.default_rng(200 + seed)
    n, ih, iw, c, m = 2, 7, 6, int(rng.integers(1, 6)), int(rng.integers(1, 3))
    kh, kw = 3, int(rng.integers(1, 4))
    stride, dil, pad = [1, 2], [1, 1], [1, 1, 0, 0]
    full = iw - 1 + pad[2] + pad[3] - (kw - 1) * dil[1]
    pad[3] += (-full) % stride[1]
    x = rng.integers(-128, 128, size=(n, ih, iw, c))
    w = rng.integers(-128, 128, size=(kh, kw, c, m))
    bias = rng.integers(-2 ** 31, 2 ** 31, size=c * m)
    zx, zw = int(rng.integers(-128, 128)), int(rng.integers(-128, 128))
    got = O.conv2d(O.T("INT8", x.shape, x), O.T("INT8", w.shape, w), O.T("INT32", bias.shape, bias), zx, zw,
                   pad, stride, dil, "INT32", "INT32", depthwise=True)
    want = conv_bruteforce(x, w, bias, zx, zw, pad, stride, dil, depthwise=True)
    assert np.array_equal(got.vals.reshape(want.shape), want)


def test_matmul_int_matches_numpy():
    rng = np.random.default_rng(9)
    a = rng.integers(-128, 128, size=(3, 17, 40))
    b = rng.integers(-128, 128, size=(3, 40, 9))
    got = O.matmul(O.T("INT8", a.shape, a), O.T("INT8", b.shape, b), -7, 2, "INT32")
    want = np.matmul(a - (-7), b - 2)
    want = (want + 2 ** 31) % 2 ** 32 - 2 ** 31
    assert np.array_equal(got.vals.reshape(want.shape), want)
    # wrap: a sum beyond int32 must wrap, not saturate
    a = np.full((1, 1, 4096), 127)
    b = np.full((1, 4096, 1), 127)
    got = O.matmul(O.T("INT8", a.shape, a), O.T("INT8", b.shape, b), -128, -128, "INT32")
    assert got.vals[0] == ((4096 * 255 * 255 + 2 ** 31) % 2 ** 32 - 2 ** 31)


def test_reader_rejects_truncated_buffers():
    data = Case(case_dirs("networks")[0]).graph
    for cut in (0, 4, 7, 16, len(data) // 2):
        with pytest.raises(Exception):
            fb.main_block(data[:cut])
