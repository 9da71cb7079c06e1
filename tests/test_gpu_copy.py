"""sile_hip_copy_rows: a byte-exact 2-D copy (the row softmax's access pattern
without its arithmetic), for 16-byte-aligned rows (128-bit path) and for any
other row length or pitch (byte path); bytes past each row stay untouched."""
import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import rng, say

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("rows,row_bytes,ldx,ldy", [
    (8192, 16384, 16384, 16384),   # the softmax workload's rows
    (37, 16 * 1025, 16 * 1030, 16 * 1025),  # longer than one pass of 16 chunks x 64 lanes
    (5, 48, 64, 80),
    (9, 1001, 1003, 1010),         # byte path
    (1, 15, 15, 15),
    (3, 4096 * 16 + 48, 4096 * 16 + 48, 4096 * 16 + 48),  # contiguous: one flat run, ragged end
])
def test_copy_rows(hip, rows, row_bytes, ldx, ldy):
    say(f"copy_rows {rows} x {row_bytes} B, pitches {ldx} / {ldy}")
    x = rng(rows + row_bytes).integers(0, 256, size=(rows, ldx), dtype=np.uint8)
    y0 = np.full((rows, ldy), 0xA5, np.uint8)
    dx, dy = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(y0)
    hip.copy_rows(rows, row_bytes, dx.ptr, ldx, dy.ptr, ldy)
    hip.synchronize()
    got = dy.download(np.uint8, (rows, ldy))
    np.testing.assert_array_equal(got[:, :row_bytes], x[:, :row_bytes])
    assert (got[:, row_bytes:] == 0xA5).all()


@pytest.mark.parametrize("dt", ["f32", "f16", "bf16"])
@pytest.mark.parametrize("rows,cols,ldy", [
    (8192, 8192, 8192),   # contiguous: the flat 16-byte path
    (37, 1000, 1003),     # pitched: element stores
    (5, 13, 13),          # rows not a multiple of 16 bytes
    (3, 4104, 4104),      # contiguous, flat run with a ragged end
])
@pytest.mark.parametrize("value", [0.1, -3.0e38, 7.0])
def test_fill_rows(hip, dt, rows, cols, ldy, value):
    """The store of a splat tile: every element of [rows, cols] becomes value
    rounded to nearest even in the element type (f16 / bf16 bits as numpy and
    the oracle round; -3e38 overflows f16 to -inf); the pitch padding stays."""
    say(f"fill_rows {dt} {rows}x{cols} ldy={ldy} value={value}")
    if dt == "f32":
        t, want = hip.F32, np.float32(value).view(np.uint32)
        y0 = np.full((rows, ldy), 0xA5A5A5A5, np.uint32)
    else:
        t = hip.F16 if dt == "f16" else hip.BF16
        with np.errstate(over="ignore"):
            want = (np.float16(np.float32(value)).view(np.uint16) if dt == "f16"
                    else cpuref.bf16_from_f32(np.array([value], np.float32))[0])
        y0 = np.full((rows, ldy), 0xA5A5, np.uint16)
    dy = hip.DeviceBuffer.from_array(y0)
    hip.fill_rows(t, rows, cols, value, dy.ptr, ldy)
    hip.synchronize()
    got = dy.download(y0.dtype, y0.shape)
    assert (got[:, :cols] == want).all(), (got[0, :4], want)
    assert (got[:, cols:] == y0[:, cols:]).all()
