"""GPU parity of the row-tile int8 3x3 convolution (conv_i8_rows_kernel in
tosa_amd/csrc/kernels/conv_i8.hip) against the oracle, bit for bit.

The kernel takes 3x3 stride-1 CONV2D with 128 input channels, output rows of
17-30 pixels and output channels a multiple of 64; producer waves issue the
MFMAs and hand each phase's accumulators through LDS to consumer waves that
run the epilogue. The cases pick what its
indexing depends on: 128-channel workgroups (CB 4) and 64-channel ones with
two waves along the rows (CB 2, also with three channel tiles); row counts
that leave the last row tile partial; the narrowest (17) and widest (30)
rows; asymmetric and zero padding (halo positions from the zero-point fill);
int32 output (the fused epilogue's pass-through, and the unfused graph),
RESCALE to int8 and int16 with per-channel and per-tensor SINGLE/DOUBLE
rounding and output zero points, a fused CLAMP, and shifts below 32 with
biases the table cannot prove safe (apply_scale_32's value-range REQUIRE
checked per value: passing, and failing). The halo kernel (option
conv_rows 0) and 64-channel workgroups (conv_rows 2) must give the same bits.
"""

import numpy as np
import pytest

import tosa_amd as T
from oracle import oracle as O
from tests.test_gpu_conv_fast import build, check, oracle_run, run

pytestmark = pytest.mark.gpu

ROWS = [
    # n, h, w, oc, pad
    (2, 28, 28, 128, (1, 1, 1, 1)),
    (1, 20, 20, 64, (1, 1, 1, 1)),
    (3, 30, 30, 192, (1, 1, 1, 1)),
    (1, 19, 19, 128, (0, 0, 0, 0)),
    (2, 16, 26, 256, (1, 0, 2, 1)),
    (1, 9, 30, 320, (1, 1, 1, 1)),
]


def _case(case, mode):
    n, h, w_, oc, pad = ROWS[case]
    rng = np.random.default_rng(9100 + 10 * case + len(mode))
    x = rng.integers(-128, 128, size=(n, h, w_, 128)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, 3, 3, 128)).astype(np.int8)
    zx = int(rng.integers(-128, 128))
    if mode == "i32":
        bias = (rng.integers(2 ** 31 - 2 ** 20, 2 ** 31, size=oc) * rng.choice([-1, 1], size=oc)).astype(np.int32)
        return build(x, w, bias, zx, 0, pad, [1, 1], [1, 1]), x
    if mode == "range_checked":
        # Shift 24: |bias| + max|x - zx| sum|w| exceeds 2^23, so the table
        # cannot rule the REQUIRE out; the actual sums stay far inside.
        bias = rng.integers(-2 ** 20, 2 ** 20, size=oc).astype(np.int32)
        rs = (rng.integers(2 ** 13, 2 ** 14, size=oc), np.full(oc, 24), int(rng.integers(-128, 128)), True, True)
        return build(x, w, bias, zx, 0, pad, [1, 1], [1, 1], rescale=rs), x
    bias = (rng.integers(2 ** 31 - 2 ** 20, 2 ** 31, size=oc) * rng.choice([-1, 1], size=oc)).astype(np.int32)
    out_dtype = "INT16" if mode == "rescale_i16" else "INT8"
    ozp = 0 if out_dtype == "INT16" else int(rng.integers(-128, 128))
    per_channel = case % 2 == 0
    mult = rng.integers(2 ** 30, 2 ** 31, size=oc if per_channel else 1)
    shift = rng.integers(38, 50, size=oc if per_channel else 1)
    rs = (mult, shift, ozp, case % 3 != 1, per_channel)
    clamp = (-100, 90) if case % 3 == 0 else None
    return build(x, w, bias, zx, 0, pad, [1, 1], [1, 1], rescale=rs, out_dtype=out_dtype, clamp=clamp), x


@pytest.mark.parametrize("case", range(len(ROWS)))
@pytest.mark.parametrize("mode", ["i32", "rescale_i8", "rescale_i16", "range_checked"])
def test_rows_conv(case, mode):
    (graph, out), x = _case(case, mode)
    ins = {"x": (x, "INT8")}
    assert T.get_option("conv_rows") == 1
    check(graph, out, ins)


@pytest.mark.parametrize("case", [0, 2, 4])
@pytest.mark.parametrize("other", [0, 2])
def test_rows_matches_other_kernels(case, other):
    # conv_rows 0: the halo kernel; 2: the row-tile kernel at 64-channel
    # workgroups for channel counts that allow 128.
    (graph, out), x = _case(case, "rescale_i8")
    ins = {"x": (x, "INT8")}
    rows = run(graph, ins)[out].numpy()
    T.set_option("conv_rows", other)
    try:
        assert T.get_option("conv_rows") == other
        alt = run(graph, ins)[out].numpy()
    finally:
        T.set_option("conv_rows", 1)
    assert np.array_equal(rows, alt)


def test_rows_range_require_failure():
    # One channel's bias alone is beyond 2^23 at shift 24: apply_scale_32's
    # REQUIRE fails on the device and the run reports it.
    n, h, w_, oc, pad = ROWS[0]
    rng = np.random.default_rng(77)
    x = rng.integers(-128, 128, size=(n, h, w_, 128)).astype(np.int8)
    w = rng.integers(-128, 128, size=(oc, 3, 3, 128)).astype(np.int8)
    bias = rng.integers(-2 ** 20, 2 ** 20, size=oc).astype(np.int32)
    bias[37] = 2 ** 23 + 2 ** 22
    rs = (np.full(oc, 2 ** 13), np.full(oc, 24), 0, True, True)
    graph, out = build(x, w, bias, 3, 0, pad, [1, 1], [1, 1], rescale=rs)
    ins = {"x": (x, "INT8")}
    with pytest.raises(O.OracleError):
        oracle_run(graph, ins)
    with pytest.raises(T.TosaError) as e:
        run(graph, ins)
    assert e.value.kind == "GraphError"
