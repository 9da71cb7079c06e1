"""sile_hip_launch_tiles_noalloc against sile_hip_launch_tiles through the C
ABI: the same kernel (vec_add<4> of crates/sile/tests/backend_vec_add.rs:3-9,
built into the library's dsl code object) on the same inputs, compared
element for element (integer-valued floats: exact), on two calls in a row,
the second with a smaller input, so the second call's tables overwrite the
first's in the shared device array.  Also: tables beyond the array's 512
entries are a Shape error before any device work."""
import ctypes
import os

import numpy as np
import pytest

from tests.helpers import say

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def vec_add(hip):
    path = os.path.join(os.path.dirname(hip.LIB_PATH), "_build", "dsl.hsaco")
    image = open(path, "rb").read()
    mod = ctypes.c_void_p()
    hip.call("sile_hip_module_load", image, len(image), ctypes.byref(mod))
    fn = ctypes.c_void_p()
    hip.call("sile_hip_module_get", mod, b"sile_tiles_vec_add4", ctypes.byref(fn))
    yield fn
    hip.call("sile_hip_module_unload", mod)


def _launch(hip, entry, fn, n, seed):
    """c = a + b over n elements (n / 4 programs of 4) through `entry`."""
    r = np.random.default_rng(seed)
    a = r.integers(-1000, 1000, n).astype(np.float32)
    b = r.integers(-1000, 1000, n).astype(np.float32)
    bufs = [hip.DeviceBuffer.from_array(t) for t in (a, b, np.full(n, -7.0, np.float32))]
    grid = (ctypes.c_uint32 * 3)(n // 4, 1, 1)
    hip.call(entry, fn, hip._ptr_array([x.ptr for x in bufs]), 3, hip._i64_array([n, n, n]), 3,
             grid, 64, None)
    out = bufs[2].download(np.float32, (n,))
    for x in bufs:
        x.close()
    return out, a + b


@pytest.mark.parametrize("sizes", [(4096, 64), (1 << 20, 16)])
def test_noalloc_launch_matches_launch_tiles(hip, vec_add, sizes):
    for i, n in enumerate(sizes):
        say(f"launch_tiles_noalloc vec_add n={n} (call {i + 1} of {len(sizes)})")
        got, want = _launch(hip, "sile_hip_launch_tiles_noalloc", vec_add, n, seed=n)
        ref, _ = _launch(hip, "sile_hip_launch_tiles", vec_add, n, seed=n)
        np.testing.assert_array_equal(got, ref)
        np.testing.assert_array_equal(got, want)


def test_noalloc_launch_rejects_oversized_tables(hip, vec_add):
    say("launch_tiles_noalloc table limit")
    bufs = hip._ptr_array([0] * 3)
    shapes = hip._i64_array([4] * 510)
    grid = (ctypes.c_uint32 * 3)(1, 1, 1)
    rc = hip.status("sile_hip_launch_tiles_noalloc", vec_add, bufs, 3, shapes, 510, grid, 64, None)
    assert rc == 5 and "exceed" in hip.last_error()
