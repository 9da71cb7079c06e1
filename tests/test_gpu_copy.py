"""sile_hip_copy_rows: a byte-exact 2-D copy (the row softmax's access pattern
without its arithmetic), for 16-byte-aligned rows (128-bit path) and for any
other row length or pitch (byte path); bytes past each row stay untouched."""
import numpy as np
import pytest

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
