"""GPU parity of the seeded tile MMA (the reference's MmaF lowered with an
accumulator that is a loaded tile or a constant splat, mma.rs:25-739) against
the oracle's cpuref_mma_f32: bit-exact, through sile_hip_mma_f32 and through
the Tile IR router (splat seeds, an accumulator loaded from another buffer or
from c itself, and the mlp example's gemm)."""
import numpy as np
import pytest

from oracle import cpuref
from tests import tile_ir_text as T
from tests.helpers import rng, say

pytestmark = pytest.mark.gpu


def _mma(hip, a, b, b_col, acc, acc_value, m, n, k, bk=0, in_place=False):
    da = hip.DeviceBuffer.from_array(a)
    db = hip.DeviceBuffer.from_array(b)
    if in_place:
        dc = hip.DeviceBuffer.from_array(acc)
        accp, ld_acc = dc.ptr, n
    else:
        dc = hip.DeviceBuffer(m * n * 4)
        dc.fill_bytes(0xFF)
        dacc = hip.DeviceBuffer.from_array(acc) if acc is not None else None
        accp, ld_acc = (dacc.ptr, n) if dacc is not None else (None, 0)
    hip.mma_f32(m, n, k, da.ptr, k, db.ptr, b.shape[1], hip.COL_MAJOR if b_col else hip.ROW_MAJOR,
                accp, ld_acc, acc_value, dc.ptr, n, bk)
    hip.synchronize()
    return dc.download(np.float32, (m, n))


@pytest.mark.parametrize("m,n,k", [(200, 300, 150), (512, 512, 512), (2048, 2000, 40),
                                   (1024, 1040, 96)])
@pytest.mark.parametrize("seed", ["splat", "tile", "in_place"])
@pytest.mark.parametrize("b_col", [False, True])
def test_mma_bit_exact(hip, m, n, k, seed, b_col):
    say(f"mma f32 {m}x{n}x{k} seed={seed} b_col={b_col}")
    r = rng(m + n + k)
    a = r.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = r.uniform(-1, 1, size=(n, k) if b_col else (k, n)).astype(np.float32)
    d = r.uniform(-4, 4, size=(m, n)).astype(np.float32)
    if seed == "splat":
        got = _mma(hip, a, b, b_col, None, 1.5, m, n, k)
        ref = cpuref.mma_f32(a, b, acc_value=1.5, b_col_major=b_col)
    else:
        got = _mma(hip, a, b, b_col, d, 0.0, m, n, k, in_place=seed == "in_place")
        ref = cpuref.mma_f32(a, b, acc=d, b_col_major=b_col)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_mma_truncated_k_and_signed_zeros(hip):
    """K' = 0 (bk > K) returns the seed bit for bit, -0.0 included; with
    products that are all -0.0 the chain stays -0.0, so the padding the kernel
    stages past K' (inside its last k-tile) must add -0.0, not +0.0."""
    m, n, k = 70, 90, 21
    say(f"mma f32 signed zeros {m}x{n}x{k}")
    d = rng(5).uniform(-1, 1, size=(m, n)).astype(np.float32)
    d[::3] = -0.0
    a = rng(6).uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng(7).uniform(-1, 1, size=(k, n)).astype(np.float32)
    got = _mma(hip, a, b, False, d, 0.0, m, n, k, bk=64)
    np.testing.assert_array_equal(got.view(np.uint32), d.view(np.uint32))
    az = np.full((m, k), -0.0, np.float32)
    bp = np.abs(b) + 1.0
    got = _mma(hip, az, bp, False, None, -0.0, m, n, k)
    ref = cpuref.mma_f32(az, bp, acc_value=-0.0)
    assert np.signbit(ref).all()
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    for bk in (8, 16):  # K' = 16 and 16: the last k-tile holds padding
        got = _mma(hip, a, b, False, d, 0.0, m, n, k, bk=bk)
        ref = cpuref.mma_f32(a, b, acc=d, bk=bk)
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))


def _expected_tiles(full, c0, programs, bm, bn):
    """c0 with the tiles of programs pid < min(programs, total) replaced by
    the full result's (the CPU wrapper's pid decode)."""
    out = c0.copy()
    tiles_n = c0.shape[1] // bn
    total = (c0.shape[0] // bm) * tiles_n
    for pid in range(min(programs, total)):
        g0, g1 = pid // tiles_n, pid % tiles_n
        sl = (slice(g0 * bm, g0 * bm + bm), slice(g1 * bn, g1 * bn + bn))
        out[sl] = full[sl]
    return out


def _route_run(hip, text, arrays, programs, out_index):
    shapes = [dd for x in arrays for dd in x.shape]
    route = hip.tile_ir_route(text, shapes, programs)
    assert route.kind == hip.ROUTE_MATMUL, (route.name, route.reason)
    bufs = [hip.DeviceBuffer.from_array(x) for x in arrays]
    hip.tile_ir_launch(route, [x.ptr for x in bufs], shapes, programs)
    return bufs[out_index].download(np.float32, arrays[out_index].shape)


@pytest.mark.parametrize("m,n,k,bm,bn,bk,programs", [
    (256, 192, 160, 32, 32, 32, 48),     # every tile: the register-tiled kernel
    (96, 80, 70, 32, 16, 8, 11),         # 11 of 15 tiles, K' = 64: the per-program kernel
])
@pytest.mark.parametrize("form", ["splat", "tile_d", "tile_c", "mlp"])
def test_routed_tile_mma_bit_exact(hip, m, n, k, bm, bn, bk, programs, form):
    say(f"tile ir mma {form} {m}x{n}x{k} tiles {bm}/{bn}/{bk} programs={programs}")
    r = rng(31)
    a = r.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = r.uniform(-1, 1, size=(k, n)).astype(np.float32)
    d = r.uniform(-2, 2, size=(m, n)).astype(np.float32)
    c0 = np.full((m, n), 7.0, np.float32)
    if form == "splat":
        got = _route_run(hip, T.matmul(bm, bn, bk, splat=1.5), [a, b, c0], programs, 2)
        full = cpuref.mma_f32(a, b, acc_value=1.5, bk=bk)
    elif form == "tile_d":
        got = _route_run(hip, T.matmul_acc(bm, bn, bk, src="d"), [a, b, d, c0], programs, 3)
        full = cpuref.mma_f32(a, b, acc=d, bk=bk)
    elif form == "tile_c":
        c0 = d.copy()
        got = _route_run(hip, T.matmul_acc(bm, bn, bk, src="c"), [a, b, c0], programs, 2)
        full = cpuref.mma_f32(a, b, acc=d, bk=bk)
    else:
        got = _route_run(hip, T.mlp_gemm(bm, bn, bk), [a, b, c0], programs, 2)
        full = cpuref.mma_f32(a, b, acc_value=0.0, bk=bk)
        # the mlp gemm is the canonical matmul's arithmetic
        np.testing.assert_array_equal(
            _expected_tiles(full, c0, programs, bm, bn),
            cpuref.kernel_matmul(a, b, c0.copy(), (programs, 1, 1), bm, bn, bk))
    want = _expected_tiles(full, c0, programs, bm, bn)
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
