"""tosa_conv2d_i8_noalloc (workspace in the per-GPU static scratch array)
against tosa_conv2d_i8 (workspace from the stream's pool), bit for bit,
through the C ABI: two calls in a row, the second on a smaller input (the
array keeps the first call's contents), then calls without a RESCALE, the
size limit and the device_error requirement.
"""

import numpy as np
import pytest

import tosa_amd as T
from tests.test_gpu_opapi import NP, dev, make_case, oracle_conv

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")


def run_both(x, w, bias, zx, zw, pad, stride, dil, rescale):
    xt, xp = dev(x)
    wt, wp = dev(w)
    bt, bp = dev(bias)
    shape = T.conv2d_i8(xp, x.shape, wp, w.shape, bp, bias.size, zx, zw, pad, stride, dil, rescale, 0)
    out_t = rescale["output_dtype"] if rescale else "INT32"
    nbytes = int(np.prod(shape)) * np.dtype(NP[out_t]).itemsize
    outs, errs = [], []
    for no_alloc in (False, True):
        out = torch.full((nbytes,), 0x5A, dtype=torch.uint8, device="cuda")
        err = torch.zeros(1, dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()  # the fills above ran on torch's stream
        got = T.conv2d_i8(xp, x.shape, wp, w.shape, bp, bias.size, zx, zw, pad, stride, dil, rescale,
                          out.data_ptr(), err.data_ptr() if rescale else 0, 0, no_alloc=no_alloc)
        assert got == shape
        torch.cuda.synchronize()
        T.synchronize()
        outs.append(out.cpu().numpy().view(NP[out_t]).reshape(shape).astype(np.int64))
        errs.append(int(err.item()))
    return outs, errs


def test_noalloc_matches_pool_entry_twice_then_smaller():
    # First a 3x3 halo-kernel call, then a smaller strided one: the second
    # call's table and packed weights overwrite the first's in the array.
    first = make_case("halo3x3", "channel_double", 7)
    second = make_case("tiled_s2", "tensor_single_i16_clamp", 8)
    assert first[0].size > second[0].size
    for args in (first, second):
        (pool, noalloc), errs = run_both(*args)
        assert np.array_equal(noalloc, pool)
        assert np.array_equal(noalloc, oracle_conv(*args))
        assert errs == [0, 0]


def test_noalloc_without_rescale_and_unfolded_zero_point():
    for geom, mode in (("pointwise", "none"), ("dilated", "unfolded_zp"), ("halo3x3", "none")):
        args = make_case(geom, mode, 11)
        (pool, noalloc), _ = run_both(*args)
        assert np.array_equal(noalloc, pool), (geom, mode)


def test_noalloc_limits():
    # A RESCALE the fused epilogue cannot take needs the int32 result in the
    # workspace: 8x32x32 pixels x 128 channels x 4 bytes = 4 MiB, beyond the
    # array. The pool entry takes the same call.
    r = np.random.default_rng(21)
    x = r.integers(-128, 128, (8, 32, 32, 64)).astype(np.int8)
    w = r.integers(-128, 128, (128, 1, 1, 64)).astype(np.int8)
    bias = np.full(128, 2 ** 28, np.int32)
    rescale = dict(multiplier=r.integers(2 ** 30, 2 ** 31, 128), shift=r.integers(52, 56, 128), double_round=True,
                   output_dtype="INT8", output_zp=100)
    xt, xp = dev(x)
    wt, wp = dev(w)
    bt, bp = dev(bias)
    out = torch.zeros(8 * 32 * 32 * 128, dtype=torch.uint8, device="cuda")
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    args = (xp, x.shape, wp, w.shape, bp, 128, -5, 0, (0, 0, 0, 0), (1, 1), (1, 1), rescale, out.data_ptr())
    with pytest.raises(T.TosaError) as e:
        T.conv2d_i8(*args, err.data_ptr(), 0, no_alloc=True)
    assert e.value.kind == "InvalidArgument" and "at most" in str(e.value)
    T.conv2d_i8(*args, err.data_ptr())
    T.synchronize()
    got = out.cpu().numpy().view(np.int8).reshape(8, 32, 32, 128).astype(np.int64)
    assert np.array_equal(got, oracle_conv(x, w, bias, -5, 0, (0, 0, 0, 0), (1, 1), (1, 1), rescale))
    assert int(err.item()) == 0
    # A RESCALE without device_error is refused.
    small = make_case("pointwise", "channel_double", 3)
    x8, w8, b8 = small[0], small[1], small[2]
    xt, xp = dev(x8)
    wt, wp = dev(w8)
    bt, bp = dev(b8)
    with pytest.raises(T.TosaError) as e:
        T.conv2d_i8(xp, x8.shape, wp, w8.shape, bp, b8.size, small[3], small[4], small[5], small[6], small[7],
                    small[8], out.data_ptr(), 0, 0, no_alloc=True)
    assert e.value.kind == "InvalidArgument" and "device_error" in str(e.value)
