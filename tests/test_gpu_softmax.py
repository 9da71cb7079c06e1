"""GPU parity of sile_hip_softmax_rows and sile_hip_reduce_rows against the CPU
oracle on the up-cast fp32 inputs.

softmax tolerance: |g - r| <= 1e-6 + 1e-2 |r| per element for 16-bit outputs
(the north star's 1e-2 relative bound; the absolute part is lowered from 2e-2
to 1e-6 because every softmax output is below 2e-2 at these widths, which
would make a 2e-2 bound vacuous), 1e-4 relative for fp32 outputs.
"""
import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import (assert_close, assert_same_bits, bf16_round, f16_round,
                           max_fold_probe_rows, rng, say)

pytestmark = pytest.mark.gpu


def _softmax_gpu(hip, x_bits, in_t, out_t, rows, cols, ldx=None, ldy=None):
    ldx = ldx or cols
    ldy = ldy or cols
    dx = hip.DeviceBuffer.from_array(x_bits)
    ob = 4 if out_t == hip.F32 else 2
    dy = hip.DeviceBuffer(rows * ldy * ob)
    dy.fill_bytes(0)
    hip.softmax_rows(in_t, out_t, rows, cols, dx.ptr, ldx, dy.ptr, ldy)
    hip.synchronize()
    if out_t == hip.F32:
        y = dy.download(np.float32, (rows, ldy))
    elif out_t == hip.F16:
        y = dy.download(np.uint16, (rows, ldy)).view(np.float16).astype(np.float32)
    else:
        y = cpuref.f32_from_bf16(dy.download(np.uint16, (rows, ldy)))
    return y[:, :cols]


def test_softmax_f16_config2_full(hip):
    """[8192, 8192] fp16, N(0, 4) seed 3, every element checked."""
    say("softmax f16 8192x8192")
    x = (rng(3).normal(size=(8192, 8192)) * 2.0).astype(np.float32)
    xb, xf = f16_round(x)
    got = _softmax_gpu(hip, xb, hip.F16, hip.F16, 8192, 8192)
    ref = cpuref.softmax_rows(xf)
    assert_close(got, ref, atol=1e-6, rtol=1e-2, what="softmax f16 8192")
    assert np.all(np.abs(got.astype(np.float64).sum(axis=1) - 1.0) < 5e-3)
    np.testing.assert_array_equal(got.argmax(axis=1), ref.argmax(axis=1))


@pytest.mark.parametrize("cols", [512, 1024, 2048, 4096, 8192, 100, 3000, 1, 257, 6100, 8000,
                                  13, 32, 128, 200, 256, 9000, 16384, 20000, 32768, 50000,
                                  70000, 1 << 20])
@pytest.mark.parametrize("dt", ["f16", "bf16", "f32", "f16_f32"])
def test_softmax_widths_and_types(hip, cols, dt):
    """Every kernel of the row softmax: kL lanes per row (up to 32 chunks),
    a wave per row (whole or masked last chunk), a workgroup per row (exact
    widths, masked up to 1024 x 8 chunks), and two passes beyond."""
    rows = 37
    say(f"softmax {dt} {rows}x{cols}")
    x = (rng(cols).normal(size=(rows, cols)) * 2.0).astype(np.float32)
    if dt == "f16":
        xb, xf = f16_round(x)
        in_t = out_t = hip.F16
    elif dt == "bf16":
        xb, xf = bf16_round(x)
        in_t = out_t = hip.BF16
    elif dt == "f16_f32":
        xb, xf = f16_round(x)
        in_t, out_t = hip.F16, hip.F32
    else:
        xb = xf = x
        in_t = out_t = hip.F32
    got = _softmax_gpu(hip, xb, in_t, out_t, rows, cols)
    ref = cpuref.softmax_rows(xf)
    if out_t == hip.F32 and cols >= 1 << 20:
        # The reference's strictly sequential fp32 row sum drifts over 2^20
        # positive terms (1.2e-3 relative here); the kernel's sum is held to
        # the exact softmax instead, and the oracle's drift is bounded.
        x64 = xf.astype(np.float64)
        e = np.exp(x64 - x64.max(axis=1, keepdims=True))
        exact = e / e.sum(axis=1, keepdims=True)
        assert_close(got, exact, atol=1e-30, rtol=1e-4, what=f"softmax {dt} vs exact")
        assert_close(ref, exact, atol=1e-30, rtol=3e-3, what="oracle's sequential-sum drift")
    elif out_t == hip.F32:
        assert_close(got, ref, atol=1e-30, rtol=1e-4, what=f"softmax {dt}")
    else:
        rtol = 1e-2
        assert_close(got, ref, atol=1e-6, rtol=rtol, what=f"softmax {dt}")


@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("rows,cols", [(1001, 128), (77, 33), (5, 4), (300, 250)])
def test_softmax_narrow_rows_many(hip, dt, rows, cols):
    """Rows of up to 32 chunks share waves (256 / kL rows per workgroup): row
    counts that leave the last workgroup and wave partly empty, padded
    leading dimensions, every element against the oracle."""
    say(f"softmax narrow {dt} {rows}x{cols}")
    ld = cols + (8 if dt == "f16" else 4) - cols % (8 if dt == "f16" else 4)
    x = (rng(rows + cols).normal(size=(rows, ld)) * 2.0).astype(np.float32)
    if dt == "f16":
        xb, xf = f16_round(x)
        t = hip.F16
    else:
        xb = xf = x
        t = hip.F32
    got = _softmax_gpu(hip, xb, t, t, rows, cols, ldx=ld, ldy=ld)
    ref = cpuref.softmax_rows(np.ascontiguousarray(xf[:, :cols]))
    if dt == "f32":
        assert_close(got, ref, atol=1e-30, rtol=1e-4, what="narrow f32")
    else:
        assert_close(got, ref, atol=1e-6, rtol=1e-2, what="narrow f16")


@pytest.mark.parametrize("cols", [20000, 70000])
def test_softmax_wide_rows_with_minus_inf(hip, cols):
    """Wide rows with -inf runs (masked scores): a row whose first 60 % is
    -inf, a row with one finite entry at its end, a row of -inf save one
    entry in the middle; the workgroup-per-row kernels (in registers, and
    the two-pass one with its running max starting at -inf) give exp 0 there
    and the oracle's values elsewhere."""
    say(f"softmax f32 wide rows with -inf, cols={cols}")
    rows = 4
    x = (rng(cols).normal(size=(rows, cols)) * 2.0).astype(np.float32)
    x[0, : int(0.6 * cols)] = -np.inf
    x[1, :-1] = -np.inf
    x[2, :] = -np.inf
    x[2, cols // 2] = 3.0
    got = _softmax_gpu(hip, x, hip.F32, hip.F32, rows, cols)
    ref = cpuref.softmax_rows(x)
    assert np.isfinite(got).all()
    assert got[1, -1] == 1.0 and got[2, cols // 2] == 1.0
    assert_close(got, ref, atol=1e-30, rtol=1e-4, what="wide -inf")


def test_softmax_padded_rows(hip):
    say("softmax f16 padded leading dimensions")
    rows, cols = 20, 1024
    x = (rng(8).normal(size=(rows, cols + 24)) * 2).astype(np.float32)
    xb, xf = f16_round(x)
    got = _softmax_gpu(hip, xb, hip.F16, hip.F16, rows, cols, ldx=cols + 24, ldy=cols + 8)
    assert_close(got, cpuref.softmax_rows(np.ascontiguousarray(xf[:, :cols])), atol=1e-6,
                 rtol=1e-2, what="padded")


def test_softmax_extremes(hip):
    say("softmax f32 extremes")
    x = np.zeros((4, 512), np.float32)
    x[1] = 7.0                      # constant row -> exactly 1/512
    x[2, 17] = 80.0                 # one dominant entry
    x[3] = np.linspace(-60, 60, 512)
    got = _softmax_gpu(hip, x, hip.F32, hip.F32, 4, 512)
    ref = cpuref.softmax_rows(x)
    np.testing.assert_array_equal(got[1], np.float32(1 / 512))
    assert got[2, 17] == pytest.approx(1.0, rel=1e-6)
    assert_close(got, ref, atol=1e-30, rtol=1e-4, what="extremes")


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("cols", [8192, 1000, 13, 4, 100, 256, 2048, 4096, 16384, 65537,
                                  (1 << 20) + 5])
def test_reduce_rows(hip, dt, cols):
    """Row max (bit-identical to the reference's fold) and row sum (within
    1e-5 of the row's absolute sum) for every kernel: kL lanes per row up to
    32 chunks, a wave per row, a 1024-thread workgroup per row for few wide
    rows (16384, and 65537 with a ragged end)."""
    rows = 41
    say(f"reduce_rows {dt} {rows}x{cols}")
    x = rng(cols + 1).normal(size=(rows, cols)).astype(np.float32) * 3
    if dt == "f16":
        xb, xf = f16_round(x)
        t = hip.F16
    elif dt == "bf16":
        xb, xf = bf16_round(x)
        t = hip.BF16
    else:
        xb = xf = x
        t = hip.F32
    dx = hip.DeviceBuffer.from_array(xb)
    dout = hip.DeviceBuffer(rows * 4)
    hip.reduce_rows(hip.REDUCE_MAX, t, rows, cols, dx.ptr, cols, dout.ptr)
    hip.synchronize()
    # the max is the reference's fold from x0, bit for bit
    np.testing.assert_array_equal(dout.download(np.float32, (rows,)),
                                  cpuref.reduce_rows(xf, cpuref.REDUCE_MAX))
    hip.reduce_rows(hip.REDUCE_SUM, t, rows, cols, dx.ptr, cols, dout.ptr)
    hip.synchronize()
    ref = cpuref.reduce_rows(xf, cpuref.REDUCE_SUM)
    scale = np.abs(xf).sum(axis=1)
    got = dout.download(np.float32, (rows,))
    assert np.all(np.abs(got - ref) <= 1e-5 * scale), np.max(np.abs(got - ref) / scale)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("rows,cols", [(5001, 4096), (3, 8192), (16411, 8192)])
def test_softmax_many_ragged_rows(hip, dt, rows, cols):
    """Many rows, row counts that are not a multiple of the 4 rows of a
    workgroup, and fewer rows than a workgroup: every row written exactly once."""
    say(f"softmax rows {dt} {rows}x{cols}")
    x = (rng(rows + cols).normal(size=(rows, cols)) * 2.0).astype(np.float32)
    xb, xf = f16_round(x) if dt == "f16" else bf16_round(x)
    t = hip.F16 if dt == "f16" else hip.BF16
    got = _softmax_gpu(hip, xb, t, t, rows, cols)
    assert_close(got, cpuref.softmax_rows(xf), atol=1e-6, rtol=1e-2, what=f"softmax {dt}")


@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("cols", [1000, 5000])
def test_softmax_masked_tail_padded(hip, dt, cols):
    """Widths that end inside a lane's chunk (the one-pass kernel's masked last
    chunk) in wider row pitches: the row is right and the pitch padding of y
    keeps its fill."""
    rows, ldx, ldy = 9, cols + 16, cols + 8
    say(f"softmax {dt} {rows}x{cols} ldx={ldx} ldy={ldy}")
    x = (rng(cols + 5).normal(size=(rows, ldx)) * 2.0).astype(np.float32)
    if dt == "f16":
        xb, xf = f16_round(x)
        t, ob, fill = hip.F16, 2, np.uint16(0xABCD)
    else:
        xb = xf = x
        t, ob, fill = hip.F32, 4, np.uint32(0xABCDEF01)
    dx = hip.DeviceBuffer.from_array(xb)
    dy = hip.DeviceBuffer(rows * ldy * ob)
    dy.upload(np.full((rows, ldy), fill))
    hip.softmax_rows(t, t, rows, cols, dx.ptr, ldx, dy.ptr, ldy)
    hip.synchronize()
    raw = dy.download(np.uint16 if ob == 2 else np.uint32, (rows, ldy))
    got = raw.view(np.float16).astype(np.float32) if ob == 2 else raw.view(np.float32)
    ref = cpuref.softmax_rows(np.ascontiguousarray(xf[:, :cols]))
    if dt == "f16":
        assert_close(got[:, :cols], ref, atol=1e-6, rtol=1e-2, what="masked tail")
    else:
        assert_close(got[:, :cols], ref, atol=1e-30, rtol=1e-4, what="masked tail")
    assert (raw[:, cols:] == fill).all()


@pytest.mark.parametrize("rows,cols,ldx", [(33, 20, 20), (100, 1000, 1000), (64, 1024, 1028),
                                           (31, 4100, 4100), (70, 8192, 8192), (5, 12288, 12300),
                                           (40, 18, 18), (9, 1003, 1003), (7, 16, 16), (3, 3, 3),
                                           (8, 8190, 8190), (4, 65537, 65537), (3, 600, 603),
                                           (1, 17, 17), (6, 2049, 2051), (3, (1 << 20) + 3, (1 << 20) + 3)])
def test_reduce_rows_fused_sum_bit_exact(hip, rows, cols, ldx):
    """sile_hip_reduce_rows_fused_sum against the oracle's fused vec4 order,
    bit for bit: rows past 16 columns run the chunked kernel (window sums in
    parallel, one chain per row; blocks of 256 windows double-buffered,
    ragged last block, row pitch past cols, rows not a multiple of 4; with
    16-byte loads for aligned multiples of 4, element loads otherwise, the
    last window reading the next row's first elements and the last row's
    running past the buffer), rows of up to 16 the one-lane-per-row kernel."""
    say(f"fused row sum {rows}x{cols} ldx={ldx}")
    x = rng(rows * cols).normal(size=(rows, ldx)).astype(np.float32) * np.float32(3.0)
    x[:, :cols:7] = -0.0
    want = cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4, cols=cols)
    dx = hip.DeviceBuffer.from_array(x)
    dout = hip.DeviceBuffer(rows * 4)
    dout.fill_bytes(0xFF)
    hip.reduce_rows_fused_sum(rows, cols, dx.ptr, ldx, x.size, dout.ptr)
    hip.synchronize()
    got = dout.download(np.float32, (rows,))
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def test_reduce_rows_fused_sum_order_probes(hip):
    """Closed forms the chunked kernel must keep: [1, 1, 2^24, 0] windows give
    2^24 + 2 per window order (a pairwise tree gives 2^24), rows of -0.0 past
    16 columns sum to +0.0 (the loop starts from 0.0f), and a row of ones of
    width 4 k sums to 4 k."""
    big = np.float32(2.0 ** 24)
    rows, cols = 3, 2048
    x = np.zeros((rows, cols), np.float32)
    x[0, 0:4] = [1.0, 1.0, big, 0.0]
    x[1, :] = -0.0
    x[2, :] = 1.0
    dx = hip.DeviceBuffer.from_array(x)
    dout = hip.DeviceBuffer(rows * 4)
    hip.reduce_rows_fused_sum(rows, cols, dx.ptr, cols, x.size, dout.ptr)
    hip.synchronize()
    got = dout.download(np.float32, (rows,))
    want = cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    assert got[0] == big + 2 and not np.signbit(got[1]) and got[1] == 0.0 and got[2] == cols


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("cols,pitch_pad", [
    (13, 0), (100, 0), (256, 0),   # kL lanes per row (f32 up to 128, 16-bit up to 256)
    (1000, 0), (6000, 0),          # a wave per row, 16-byte chunks
    (2048, 0), (4096, 0), (8192, 0),  # a row per 256- or 512-thread workgroup (2 chunks a thread)
    (1000, 1), (37, 1),            # a wave per row, element loads (pitch not 16-byte aligned)
    (16384, 0), (65537, 0),        # a 1024-thread workgroup per row
])
def test_reduce_rows_max_follows_the_fold(hip, dt, cols, pitch_pad):
    """Row max with NaN, -inf and +0 / -0 ties, bit-exact against the oracle's
    fold (reduce.rs:10-30) through every max kernel; NaN matches NaN."""
    x = max_fold_probe_rows(cols, cols + pitch_pad)
    rows = x.shape[0]
    ldx = cols + pitch_pad
    say(f"reduce_rows max special values {dt} {rows}x{cols} ldx={ldx}")
    xp = np.full((rows, ldx), 7.0, np.float32)
    xp[:, :cols] = x
    if dt == "f16":
        xb, xf = f16_round(xp)
        t = hip.F16
    elif dt == "bf16":
        xb, xf = bf16_round(xp)
        t = hip.BF16
    else:
        xb = xf = xp
        t = hip.F32
    dx = hip.DeviceBuffer.from_array(xb)
    dout = hip.DeviceBuffer(rows * 4)
    hip.reduce_rows(hip.REDUCE_MAX, t, rows, cols, dx.ptr, ldx, dout.ptr)
    hip.synchronize()
    got = dout.download(np.float32, (rows,))
    ref = cpuref.reduce_rows(np.ascontiguousarray(xf), cpuref.REDUCE_MAX, cols=cols)
    assert np.isnan(ref[0]) and not np.isnan(ref[1])
    assert_same_bits(got, ref, what=f"row max {dt} {cols}")
