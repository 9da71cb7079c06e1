"""sile_hip_launch_tiles_noalloc against sile_hip_launch_tiles through the C
ABI: the same kernel (vec_add<4> of crates/sile/tests/backend_vec_add.rs:3-9,
built into the library's dsl code object) on the same inputs, compared
element for element (integer-valued floats: exact), on two calls in a row,
the second with a smaller input, so the second call's tables overwrite the
first's in the shared device array.  Also: tables beyond the array's 512
entries are a Shape error before any device work; a call on a stream that is
being captured into a graph is refused (the launch is synchronous); and two
host threads calling at once on one device, with different sizes, each get
their own result (the calls take the shared array in turn)."""
import ctypes
import os
import threading

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


def test_noalloc_launch_refuses_a_capturing_stream(hip, vec_add):
    say("launch_tiles_noalloc on a capturing stream")
    st = hip.Stream()
    n = 256
    bufs = [hip.DeviceBuffer.from_array(np.zeros(n, np.float32)) for _ in range(3)]
    x = np.arange(64 * 64, dtype=np.float32).reshape(64, 64)
    dx, dout = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer(64 * 4)
    grid = (ctypes.c_uint32 * 3)(n // 4, 1, 1)
    with hip.Graph(st) as g:
        rc = hip.status("sile_hip_launch_tiles_noalloc", vec_add,
                        hip._ptr_array([b.ptr for b in bufs]), 3, hip._i64_array([n, n, n]), 3,
                        grid, 64, st.handle)
        err = hip.last_error()
        # one captured op, so the graph is not empty
        hip.reduce_rows(hip.REDUCE_MAX, hip.F32, 64, 64, dx.ptr, 64, dout.ptr, st)
    assert rc == 2 and "capturing" in err, (rc, err)
    g.launch()
    st.synchronize()
    np.testing.assert_array_equal(dout.download(np.float32, (64,)), x.max(axis=1))
    g.close()
    st.close()


def test_noalloc_launch_two_threads(hip, vec_add):
    """Two host threads, different sizes, many calls each at once: every
    call's output is its own a + b."""
    say("launch_tiles_noalloc from two threads")
    errors = []

    def worker(n, seed):
        try:
            for i in range(20):
                got, want = _launch(hip, "sile_hip_launch_tiles_noalloc", vec_add, n, seed + i)
                np.testing.assert_array_equal(got, want)
        except Exception as e:  # reported by the main thread
            errors.append(e)

    ts = [threading.Thread(target=worker, args=(n, s)) for n, s in ((1 << 16, 100), (4096, 200))]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errors, errors
