"""The matvec program of crates/sile/examples/mlp.rs:26-44 on the GPU:
sile_hip_matvec_f32 directly and through the Tile IR router, bit for bit
against the oracle's restatement (oracle/sile_cpuref.c cpuref_dsl_matvec_f32:
per tile a sequential sum of rounded products, the tiles added to the seed in
order), and the example's whole pipeline (gemm -> matvec -> relu) against its
own host check (tolerance 1e-3, mlp.rs:104-140)."""
import ctypes

import numpy as np
import pytest

from oracle import cpuref
from tests import tile_ir_text as T
from tests.helpers import assert_close, assert_same_bits, rng, say
from tests.test_llir import PLANS, text

pytestmark = pytest.mark.gpu


def _matvec(hip, x, y, bk, m=None, k=None, seed=0.0, x_off=0, y_off=0):
    """Runs sile_hip_matvec_f32 on rows 0..m of x (copied to the device at a
    byte offset of x_off / y_off elements, to reach the unaligned path)."""
    m = x.shape[0] if m is None else m
    k = x.shape[1] if k is None else k
    xb = np.concatenate([np.zeros(x_off, np.float32), x.ravel()])
    yb = np.concatenate([np.zeros(y_off, np.float32), y])
    dx, dy = hip.DeviceBuffer.from_array(xb), hip.DeviceBuffer.from_array(yb)
    out = hip.DeviceBuffer.from_array(np.full(m + 3, 5.0, np.float32))
    hip.matvec_f32(m, k, bk, dx.ptr + 4 * x_off, x.shape[1], dy.ptr + 4 * y_off, out.ptr, seed)
    hip.synchronize()
    got = out.download(np.float32, (m + 3,))
    for b in (dx, dy, out):
        b.close()
    np.testing.assert_array_equal(got[m:], 5.0)   # nothing past row m is written
    return got[:m]


@pytest.mark.parametrize("m,k,bk,ldx,x_off", [
    (64, 64, 8, 64, 0),          # the mlp example's shape, 16-byte path
    (100, 23, 5, 23, 0),         # BK not a multiple of 4, K truncated to 20
    (7, 1000, 32, 1003, 0),      # row pitch not a multiple of 4: element loads
    (33, 8192, 32, 8192, 0),     # 256 tiles a row: four rounds of 64 lanes
    (5, 300, 1, 300, 0),         # one element a tile: 300 carried adds
    (9, 640, 64, 640, 1),        # x one element past an aligned address
    (3, 12, 16, 12, 0),          # BK > K: no tile, the seed
    (4096, 256, 16, 256, 0),     # many rows, 1024 workgroups
    # tiles of 1 .. 16 16-byte chunks: coalesced spans, chains carried across lanes
    (64, 300, 4, 300, 0),        # 75 tiles: a partial last span of 44 elements
    (16, 1000, 16, 1000, 0),     # 62 tiles, K truncated to 992
    (16, 4096, 64, 4096, 0),     # 16 lanes a tile
    (8, 8200, 8, 8204, 0),       # pitch > K, 1025 tiles
    # BK 4 and 8: eight rows a wave
    (13, 1000, 8, 1000, 0),      # a wave with 5 rows past m
    (37, 520, 4, 520, 0),        # 130 tiles, a partial last span
])
def test_matvec_matches_the_oracle_bit_for_bit(hip, m, k, bk, ldx, x_off):
    say(f"matvec m={m} k={k} bk={bk} ldx={ldx} x_off={x_off}")
    r = rng(m + k + bk)
    x = r.normal(size=(m, ldx)).astype(np.float32)
    x[:, k:] = np.nan                       # past K: never read
    kp = (k // bk) * bk
    x[:, kp:k] = np.nan                     # past the last whole tile: never added
    y = r.normal(size=max(kp, 1)).astype(np.float32)
    for seed in (0.0, 1.25):
        got = _matvec(hip, x, y, bk, m=m, k=k, seed=seed, x_off=x_off)
        want = cpuref.dsl_matvec_f32(x, y, bk, m=m, k=k, seed=seed)
        assert_same_bits(got, want, what=f"matvec seed {seed}")


def test_matvec_order_probes(hip):
    """The closed forms that pin the oracle's order hold on the device too."""
    say("matvec order probes")
    big = np.float32(2 ** 24)
    ones = np.ones(4, np.float32)
    row = np.array([[big, 1, 1, 1]], np.float32)
    assert _matvec(hip, row, ones, 4)[0] == big           # sequential in a tile
    assert _matvec(hip, row, ones, 1)[0] == big           # tiles in order
    assert _matvec(hip, np.ones((1, 2), np.float32), ones[:2], 1, seed=big)[0] == big
    a = np.float32(1 + 2 ** -12)                          # no fused multiply-add
    assert _matvec(hip, np.array([[1.0, a]], np.float32),
                   np.array([-(1 + 2 ** -11), a], np.float32), 2)[0] == 0.0
    z = _matvec(hip, np.array([[-0.0]], np.float32), np.ones(1, np.float32), 1)
    assert z[0] == 0.0 and not np.signbit(z[0])


def test_matvec_rejects_bad_arguments(hip):
    x = hip.DeviceBuffer(64)
    for args, code in [((4, 4, 0), 5), ((4, 4, -2), 5), ((-1, 4, 2), 5)]:
        rc = hip.status("sile_hip_matvec_f32", *args, x.ptr, 4, x.ptr, ctypes.c_float(0.0), x.ptr,
                        None)
        assert rc == code, (args, rc)
    rc = hip.status("sile_hip_matvec_f32", 4, 8, 2, x.ptr, 4, x.ptr, ctypes.c_float(0.0), x.ptr,
                    None)
    assert rc == 5 and "leading dimension" in hip.last_error()
    assert hip.status("sile_hip_matvec_f32", 0, 8, 2, None, 8, None, ctypes.c_float(0.0), None,
                      None) == 0
    x.close()


def _route_run(hip, text_, arrays, programs):
    shapes = [d for a in arrays for d in a.shape]
    route = hip.tile_ir_route(text_, shapes, programs)
    assert route.kind == hip.ROUTE_MATVEC, route.reason
    bufs = [hip.DeviceBuffer.from_array(a) for a in arrays]
    hip.tile_ir_launch(route, [b.ptr for b in bufs], shapes, programs)
    out = [b.download(np.float32, a.shape) for a, b in zip(arrays, bufs)]
    for b in bufs:
        b.close()
    return out


@pytest.mark.parametrize("bm,bk,m,k,programs,passes", [
    (32, 8, 64, 64, 2, True),      # the mlp example (mlp.rs:68-89)
    (16, 5, 100, 23, 3, False),    # fewer programs than row tiles, K truncated
    (64, 32, 8192, 8192, 128, True),
])
def test_matvec_route_matches_the_oracle(hip, bm, bk, m, k, programs, passes):
    say(f"tile ir matvec BM={bm} BK={bk} {m}x{k} programs={programs}")
    r = rng(bm + bk + m)
    x = r.uniform(-1, 1, size=(m, k)).astype(np.float32)
    y = r.uniform(-1, 1, size=k).astype(np.float32)
    z = np.full(m, 9.0, np.float32)
    _, _, got = _route_run(hip, T.matvec(bm, bk, passes=passes), [x, y, z], programs)
    rows = programs * bm
    assert_same_bits(got[:rows], cpuref.dsl_matvec_f32(x, y, bk, m=rows), what="routed matvec")
    np.testing.assert_array_equal(got[rows:], 9.0)


def test_mlp_example_pipeline(hip):
    """crates/sile/examples/mlp.rs main: out0 = x @ w0 (the gemm kernel,
    routed), out1 = out0 @ w1 (the matvec kernel, routed), relu in place (the
    generated LLIR relu over [8] tiles), at dim 64 with the example's tiles;
    bit for bit against the oracle's chain and within the example's own 1e-3
    of its sequential host loops."""
    say("mlp example pipeline dim=64")
    dim = 64
    r = rng(64)
    x_in = r.uniform(0, 1, size=(dim, dim)).astype(np.float32)
    w0 = r.uniform(0, 1, size=(dim, dim)).astype(np.float32)
    w1 = r.uniform(-1, 1, size=dim).astype(np.float32)
    shapes0 = [dim, dim, dim, dim, dim, dim]
    g = hip.tile_ir_route(T.mlp_gemm(32, 32, 8), shapes0, 4)
    assert g.kind == hip.ROUTE_MATMUL, g.reason
    mv = hip.tile_ir_route(T.matvec(32, 8), [dim, dim, dim, dim], 2)
    assert mv.kind == hip.ROUTE_MATVEC, mv.reason
    dx, dw0, dw1 = (hip.DeviceBuffer.from_array(a) for a in (x_in, w0, w1))
    dout0 = hip.DeviceBuffer.from_array(np.zeros((dim, dim), np.float32))
    dout1 = hip.DeviceBuffer.from_array(np.zeros(dim, np.float32))
    hip.tile_ir_launch(g, [dx.ptr, dw0.ptr, dout0.ptr], shapes0, 4)
    hip.tile_ir_launch(mv, [dout0.ptr, dw1.ptr, dout1.ptr], [dim, dim, dim, dim], 2)
    relu = hip.LlirKernel(text("relu"), PLANS["relu"])
    relu([dout1.ptr], [dim], (dim // 8, 1, 1))
    hip.synchronize()
    got = dout1.download(np.float32, (dim,))
    relu.close()
    for b in (dx, dw0, dw1, dout0, dout1):
        b.close()
    # the oracle's chain: canonical matmul, the matvec program, relu x >= 0 ? x : 0
    out0 = np.zeros((dim, dim), np.float32)
    cpuref.kernel_matmul(x_in, w0, out0, (2, 2, 1), 32, 32, 8)
    out1 = cpuref.dsl_matvec_f32(out0, w1, 8)
    want = np.where(out1 >= 0, out1, np.float32(0.0)).astype(np.float32)
    assert_same_bits(got, want, what="mlp pipeline vs oracle")
    # the example's own host check: sequential f32 loops, |gpu - cpu| < 1e-3
    host0 = np.zeros((dim, dim), np.float32)
    for i in range(dim):
        for j in range(dim):
            s = np.float32(0.0)
            for kk in range(dim):
                s = np.float32(s + x_in[i, kk] * w0[kk, j])
            host0[i, j] = s
    host1 = np.zeros(dim, np.float32)
    for i in range(dim):
        s = np.float32(0.0)
        for kk in range(dim):
            s = np.float32(s + host0[i, kk] * w1[kk])
        host1[i] = s
    host1 = np.maximum(host1, 0.0)
    assert_close(got, host1, atol=1e-3, rtol=0.0, what="mlp example host check")
