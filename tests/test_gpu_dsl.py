"""GPU parity of sile's DSL kernels run through the C ABI with the
sile_kernel_<name> convention, against the CPU oracle and the reference's own
fixtures.  matmul and the parallel_reduce tile sums are bit-exact; softmax
is within fp32 tolerance (device exp, tree sum)."""
import json
import os

import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import assert_close, rng, say

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_fixtures.json")


@pytest.fixture(scope="module")
def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


def run_matmul(hip, a, b, c_init, grid, bm, bn, bk):
    da, db, dc = (hip.DeviceBuffer.from_array(t) for t in (a, b, c_init))
    shapes = [*a.shape, *b.shape, *c_init.shape]
    hip.kernel_matmul([da.ptr, db.ptr, dc.ptr], int(np.prod(grid)), shapes, bm, bn, bk)
    return dc.download(np.float32, c_init.shape)


def test_matmul_reference_fixture(hip, fixtures):
    fx = fixtures["matmul_4x4"]
    say("dsl matmul 4x4 reference fixture")
    a = np.array(fx["a"]["data"], np.float32).reshape(fx["a"]["shape"])
    b = np.array(fx["b"]["data"], np.float32).reshape(fx["b"]["shape"])
    c = np.zeros((4, 4), np.float32)
    got = run_matmul(hip, a, b, c, fx["grid"], fx["bm"], fx["bn"], fx["bk"])
    np.testing.assert_array_equal(got.ravel(), np.array(fx["expected"], np.float32))


@pytest.mark.parametrize("grid", [(2, 1, 1), (4, 1, 1), (100, 1, 1), (2, 2, 1)])
def test_matmul_launch_semantics(hip, grid):
    say(f"dsl matmul launch semantics grid={grid}")
    a = rng(7).integers(-4, 5, size=(4, 5)).astype(np.float32)
    b = rng(8).integers(-4, 5, size=(5, 4)).astype(np.float32)
    c0 = np.full((4, 4), -1.5, np.float32)
    ref = cpuref.kernel_matmul(a, b, c0.copy(), grid, 2, 2, 2)
    got = run_matmul(hip, a, b, c0, grid, 2, 2, 2)
    np.testing.assert_array_equal(got, ref)


def test_matmul_config1_512_bit_exact(hip):
    """fp32 GEMM 512^3, U(-1,1) seeds 1/2, 32x32 tiles."""
    say("dsl matmul 512^3 BM=BN=BK=32")
    a = rng(1).uniform(-1, 1, size=(512, 512)).astype(np.float32)
    b = rng(2).uniform(-1, 1, size=(512, 512)).astype(np.float32)
    grid = (16, 16, 1)
    ref = cpuref.kernel_matmul(a, b, np.zeros((512, 512), np.float32), grid, 32, 32, 32)
    got = run_matmul(hip, a, b, np.zeros((512, 512), np.float32), grid, 32, 32, 32)
    np.testing.assert_array_equal(got, ref)


def test_matmul_odd_tiles_bit_exact(hip):
    say("dsl matmul ragged 100x70x45 BM=32 BN=16 BK=8")
    a = rng(3).normal(size=(100, 45)).astype(np.float32)
    b = rng(4).normal(size=(45, 70)).astype(np.float32)
    c0 = np.full((100, 70), 9.0, np.float32)
    grid = (3 * 4, 1, 1)
    ref = cpuref.kernel_matmul(a, b, c0.copy(), grid, 32, 16, 8)
    got = run_matmul(hip, a, b, c0, grid, 32, 16, 8)
    np.testing.assert_array_equal(got, ref)


def run_softmax(hip, x, y0, grid, bm, bn):
    dx, dy = hip.DeviceBuffer.from_array(x), hip.DeviceBuffer.from_array(y0)
    hip.kernel_softmax([dx.ptr, dy.ptr], int(np.prod(grid)), [*x.shape, *y0.shape], bm, bn)
    return dy.download(np.float32, y0.shape)


def test_softmax_reference_fixture(hip, fixtures):
    fx = fixtures["softmax_4x8"]
    say("dsl softmax 4x8 reference fixture")
    x = np.array(fx["x"]["data"], np.float32).reshape(fx["x"]["shape"])
    y = run_softmax(hip, x, np.zeros_like(x), fx["grid"], fx["bm"], fx["bn"])
    assert np.all(np.abs(y.sum(axis=1) - fx["expected_row_sum"]) < fx["tolerance_abs"])
    ref = cpuref.kernel_softmax(x, np.zeros_like(x), fx["grid"], fx["bm"], fx["bn"])
    assert_close(y, ref, atol=1e-7, rtol=1e-4, what="softmax fixture")


@pytest.mark.parametrize("shape,bm,bn,grid", [
    ((64, 256), 4, 256, (16, 1, 1)),
    ((64, 256), 2, 64, (128, 1, 1)),    # BN < row width: per-tile normalisation
    ((30, 100), 7, 100, (3, 1, 1)),     # ragged: last 2 rows not covered
    ((8, 3000), 1, 3000, (8, 1, 1)),
])
def test_softmax_tiles(hip, shape, bm, bn, grid):
    say(f"dsl softmax {shape} BM={bm} BN={bn} grid={grid}")
    x = (rng(5).normal(size=shape) * 2).astype(np.float32)
    y0 = np.full(shape, -3.0, np.float32)
    ref = cpuref.kernel_softmax(x, y0.copy(), grid, bm, bn)
    got = run_softmax(hip, x, y0, grid, bm, bn)
    # fp32 relative tolerance 1e-4 (north star); untouched cells must stay bit-equal
    assert_close(got, ref, atol=1e-30, rtol=1e-4, what="dsl softmax")
    np.testing.assert_array_equal(got[ref == -3.0], -3.0)


@pytest.mark.parametrize("name", ["parallel_reduce_ones", "parallel_reduce_arange"])
def test_parallel_reduce_reference_fixtures(hip, fixtures, name):
    fx = fixtures[name]
    say(f"dsl parallel_reduce {name}")
    n = fx["a"]["shape"][0]
    a = (np.full(n, fx["a"]["fill"], np.float32) if "fill" in fx["a"]
         else np.arange(fx["a"]["arange_from"], fx["a"]["arange_from"] + n, dtype=np.float32))
    da = hip.DeviceBuffer.from_array(a)
    dout = hip.DeviceBuffer.from_array(np.zeros(1, np.float32))
    programs = int(np.prod(fx["grid"]))
    dpart = hip.DeviceBuffer(programs * 4)
    hip.kernel_parallel_reduce([da.ptr, dout.ptr], programs, [n, 1], fx["tile"], partials=dpart.ptr)
    got = dout.download(np.float32, (1,))[0]
    if "tolerance_abs" in fx:
        assert abs(got - fx["expected"]) < fx["tolerance_abs"]
    else:
        assert abs(got - fx["expected"]) <= fx["tolerance_rel"] * fx["expected"]
    # per-program tile sums are bit-identical to the CPU backend's vec4 order
    parts = dpart.download(np.float32, (programs,))
    np.testing.assert_array_equal(parts, cpuref.parallel_reduce_partials(a, programs, fx["tile"]))


@pytest.mark.parametrize("tile", [17, 18, 19, 20, 1003])
def test_parallel_reduce_ones_closed_form(hip, tile):
    """Ones: the reference's loop form reads ceil(TILE/4) windows (into the
    next tile) and re-adds the TILE % 4 tail: TILE = 18 gives 16 + 4 + 2 = 22
    per program; the last program's window runs past a (0.0f): 20."""
    say(f"dsl parallel_reduce ones tile={tile}")
    programs = 25
    a = np.ones(programs * tile, np.float32)
    da = hip.DeviceBuffer.from_array(a)
    dout = hip.DeviceBuffer.from_array(np.zeros(1, np.float32))
    dpart = hip.DeviceBuffer(programs * 4)
    hip.kernel_parallel_reduce([da.ptr, dout.ptr], programs, [a.size, 1], tile, partials=dpart.ptr)
    parts = dpart.download(np.float32, (programs,))
    rem = tile % 4
    interior = 4 * ((tile + 3) // 4) + rem if rem else tile
    last = 4 * (tile // 4) + 2 * rem
    np.testing.assert_array_equal(parts[:-1], interior)
    assert parts[-1] == last
    if tile == 18:
        assert (interior, last) == (22, 20)
    assert dout.download(np.float32, (1,))[0] == interior * (programs - 1) + last


@pytest.mark.parametrize("tile,pad", [(3, 5), (12, 5), (16, 5), (1000, 5), (1003, 5), (1003, 0),
                                      (17, 0), (17, 2), (20, 0), (2052, 3), (4096, 0), (5003, 1),
                                      (5003, 0)])
def test_parallel_reduce_partials_random(hip, tile, pad):
    """pad = elements of a past the last tile: the last program's final
    window reads them (pad >= 4 - TILE % 4) or runs past a."""
    say(f"dsl parallel_reduce random tile={tile} pad={pad}")
    programs = 37
    a = rng(tile).normal(size=programs * tile + pad).astype(np.float32)
    da = hip.DeviceBuffer.from_array(a)
    dout = hip.DeviceBuffer.from_array(np.zeros(1, np.float32))
    dpart = hip.DeviceBuffer(programs * 4)
    hip.kernel_parallel_reduce([da.ptr, dout.ptr], programs, [a.size, 1], tile, partials=dpart.ptr)
    parts = dpart.download(np.float32, (programs,))
    np.testing.assert_array_equal(parts, cpuref.parallel_reduce_partials(a, programs, tile))
    total = dout.download(np.float32, (1,))[0]
    assert_close(total, parts.astype(np.float64).sum(), atol=1e-3, rtol=1e-5, what="atomic total")


def test_generic_tile_launch_vec_add(hip):
    """sile_hip_module_load / module_get / launch_tiles on a code object built
    here, with the reference's vec_add fixture (1 + 2 = 3,
    crates/sile/tests/backend_vec_add.rs:11-25)."""
    import ctypes
    import os
    say("generic launch_tiles vec_add")
    path = os.path.join(os.path.dirname(hip.LIB_PATH), "_build", "dsl.hsaco")
    image = open(path, "rb").read()
    mod = ctypes.c_void_p()
    hip.call("sile_hip_module_load", image, len(image), ctypes.byref(mod))
    fn = ctypes.c_void_p()
    hip.call("sile_hip_module_get", mod, b"sile_tiles_vec_add4", ctypes.byref(fn))
    with pytest.raises(hip.SileError) as e:
        hip.call("sile_hip_module_get", mod, b"no_such_kernel", ctypes.byref(ctypes.c_void_p()))
    assert e.value.kind == "Compile"
    a, b = np.ones(16, np.float32), np.full(16, 2.0, np.float32)
    bufs = [hip.DeviceBuffer.from_array(t) for t in (a, b, np.zeros(16, np.float32))]
    grid = (ctypes.c_uint32 * 3)(4, 1, 1)
    hip.call("sile_hip_launch_tiles", fn, hip._ptr_array([x.ptr for x in bufs]), 3,
             hip._i64_array([16, 16, 16]), 3, grid, 64, None)
    np.testing.assert_array_equal(bufs[2].download(np.float32, (16,)), 3.0)
    hip.call("sile_hip_module_unload", mod)
