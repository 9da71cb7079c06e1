"""GPU parity of the Tile IR pattern router: each DSL kernel's printed Tile IR
is routed (sile_hip_tile_ir_route) and launched (sile_hip_tile_ir_launch)
through the C ABI, and compared with the reference's fixtures and the CPU
oracle of the same kernel with the same grid.  Bars: matmul bit-exact (the
exact-order tile kernel); row max and row sum bit-exact (the sum in the fused
load + reduce vec4 order); softmax |g - r| <= 1e-6 + 1e-5 |r| (device exp,
tree sums; the reference test bounds row sums by 1e-4); the atomic sum of
ones exact."""
import json
import os

import numpy as np
import pytest

from oracle import cpuref
from tests import tile_ir_text as T
from tests.helpers import assert_close, assert_same_bits, max_fold_probe_rows, rng, say

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def fixtures():
    with open(os.path.join(GOLDEN, "reference_fixtures.json")) as f:
        return json.load(f)


def _golden_text(name):
    with open(os.path.join(GOLDEN, "tile_ir", name)) as f:
        return f.read()


def _run(hip, text, arrays, programs, want_kind):
    """Routes `text` for these arrays and grid, launches, returns the arrays back."""
    shapes = [d for a in arrays for d in a.shape]
    route = hip.tile_ir_route(text, shapes, programs)
    assert route.kind == want_kind, (route.name, route.reason)
    bufs = [hip.DeviceBuffer.from_array(a) for a in arrays]
    hip.tile_ir_launch(route, [b.ptr for b in bufs], shapes, programs)
    return [b.download(np.float32, a.shape) for a, b in zip(arrays, bufs)]


def test_matmul_reference_fixture(hip, fixtures):
    fx = fixtures["matmul_4x4"]
    say("tile ir matmul 4x4 reference fixture")
    a = np.array(fx["a"]["data"], np.float32).reshape(fx["a"]["shape"])
    b = np.array(fx["b"]["data"], np.float32).reshape(fx["b"]["shape"])
    c = np.zeros((4, 4), np.float32)
    _, _, got = _run(hip, _golden_text("matmul_2x2x2.tir"), [a, b, c], int(np.prod(fx["grid"])),
                     hip.ROUTE_MATMUL)
    np.testing.assert_array_equal(got.ravel(), np.array(fx["expected"], np.float32))


@pytest.mark.parametrize("m,n,k,bm,bn,bk,programs", [
    (512, 512, 512, 32, 32, 32, 256),
    (96, 80, 70, 32, 16, 8, 11),        # K truncated to 64, 11 of 15 tiles
    (64, 64, 64, 16, 32, 16, 1000),     # more programs than tiles
])
def test_matmul_bit_exact(hip, m, n, k, bm, bn, bk, programs):
    say(f"tile ir matmul {m}x{n}x{k} tiles {bm}/{bn}/{bk} programs={programs}")
    a = rng(1).uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = rng(2).uniform(-1, 1, size=(k, n)).astype(np.float32)
    c0 = np.full((m, n), 7.0, np.float32)
    ref = cpuref.kernel_matmul(a, b, c0.copy(), (programs, 1, 1), bm, bn, bk)
    _, _, got = _run(hip, T.matmul(bm, bn, bk), [a, b, c0], programs, hip.ROUTE_MATMUL)
    np.testing.assert_array_equal(got, ref)


@pytest.mark.parametrize("name", ["softmax_2x8.tir", "softmax_2x8_unfused.tir"])
def test_softmax_reference_fixture(hip, fixtures, name):
    fx = fixtures["softmax_4x8"]
    say(f"tile ir softmax reference fixture {name}")
    x = np.array(fx["x"]["data"], np.float32).reshape(fx["x"]["shape"])
    y = np.zeros_like(x)
    programs = int(np.prod(fx["grid"]))
    _, got = _run(hip, _golden_text(name), [x, y], programs, hip.ROUTE_SOFTMAX_ROWS)
    np.testing.assert_allclose(got.sum(axis=1), fx["expected_row_sum"], atol=fx["tolerance_abs"])
    ref = cpuref.kernel_softmax(x, np.zeros_like(x), fx["grid"], fx["bm"], fx["bn"])
    assert_close(got, ref, atol=1e-6, rtol=1e-5, what=name)


@pytest.mark.parametrize("rows,cols,bm,bn,programs,kind", [
    (1024, 8192, 1, 8192, 1024, "rows"),   # config 2 width, one row per program
    (64, 1000, 4, 1000, 10, "rows"),       # 10 of 16 row bands
    (64, 512, 2, 128, 256, "tiles"),       # 4 column tiles per band: the tile kernel
    (32, 96, 4, 64, 8, "rows"),            # y one tile plus 32 untouched columns
])
def test_softmax_routes_match_the_oracle(hip, rows, cols, bm, bn, programs, kind):
    say(f"tile ir softmax {rows}x{cols} BM={bm} BN={bn} programs={programs}")
    x = (rng(3).normal(size=(rows, cols)) * 2).astype(np.float32)
    y0 = np.full((rows, cols), -3.0, np.float32)
    want = hip.ROUTE_SOFTMAX_ROWS if kind == "rows" else hip.ROUTE_SOFTMAX_TILES
    _, got = _run(hip, T.softmax(bm, bn), [x, y0.copy()], programs, want)
    ref = cpuref.kernel_softmax(x, y0.copy(), (programs, 1, 1), bm, bn)
    assert_close(got, ref, atol=1e-6, rtol=1e-5, what="softmax")
    # elements no program owns keep their values
    untouched = ref == -3.0
    np.testing.assert_array_equal(got[untouched], y0[untouched])


@pytest.mark.parametrize("op", ["sum", "max"])
@pytest.mark.parametrize("rows,cols,bm,bn,programs,out_rank", [
    (64, 1000, 4, 1000, 16, 2),
    (64, 1000, 4, 960, 9, 1),   # first 960 columns, 9 of 16 row bands
    (256, 8192, 1, 8192, 256, 2),
    (40, 1003, 2, 1003, 20, 2),  # last window of each row reads the next row; the
                                 # buffer's last row reads past x (0.0f)
    (40, 1003, 2, 1001, 7, 1),   # windows read the row's own columns 1001..1003
    (16, 18, 4, 17, 4, 2),       # 17 wide: one window of 1 + 3 elements past
    (16, 12, 4, 7, 4, 2),        # unrolled form, 1 window and a tail of 3
    (8, 3, 1, 3, 8, 2),          # below 4: the plain fold
])
def test_row_reduce_matches_the_oracle(hip, op, rows, cols, bm, bn, programs, out_rank):
    """The route is the reference's fused load + reduce: the max bit-exact,
    the sum bit-exact in its vec4 window order (over-read included)."""
    say(f"tile ir row_{op} {rows}x{cols} BM={bm} BN={bn} programs={programs} rank={out_rank}")
    x = (rng(5).normal(size=(rows, cols)) * 3).astype(np.float32)
    yshape = (rows, 1) if out_rank == 2 else (rows,)
    y0 = np.full(yshape, 11.0, np.float32)
    _, got = _run(hip, T.row_reduce(bm, bn, op, out_rank), [x, y0.copy()], programs,
                  hip.ROUTE_REDUCE_ROWS)
    got = got.reshape(rows)
    n = programs * bm
    ref = cpuref.reduce_rows(x, cpuref.REDUCE_MAX if op == "max" else cpuref.REDUCE_SUM_VEC4,
                             cols=bn)
    np.testing.assert_array_equal(got[:n], ref[:n])
    np.testing.assert_array_equal(got[n:], 11.0)


def test_row_sum_route_ones_closed_form(hip):
    """Rows of ones, 18 wide: every row but the buffer's last adds 16 + 4 + 2
    = 22; the last row's window runs past x: 16 + 2 + 2 = 20."""
    say("tile ir row_sum ones 18 wide")
    rows, cols = 12, 18
    x = np.ones((rows, cols), np.float32)
    y0 = np.zeros((rows, 1), np.float32)
    _, got = _run(hip, T.row_reduce(4, cols, "sum", 2), [x, y0], rows // 4, hip.ROUTE_REDUCE_ROWS)
    np.testing.assert_array_equal(got[:-1, 0], 22.0)
    assert got[-1, 0] == 20.0


def test_parallel_reduce_reference_fixture(hip, fixtures):
    fx = fixtures["parallel_reduce_ones"]
    say("tile ir parallel_reduce reference fixture")
    a = np.ones(fx["a"]["shape"], np.float32)
    out = np.zeros(1, np.float32)
    programs = int(np.prod(fx["grid"]))
    _, got = _run(hip, _golden_text("parallel_reduce_1000.tir"), [a, out], programs,
                  hip.ROUTE_ATOMIC_REDUCE)
    assert got[0] == fx["expected"]


@pytest.mark.parametrize("cols,bm", [(1000, 4), (8192, 1), (100, 2)])
def test_row_max_route_follows_the_fold(hip, cols, bm):
    """The routed row max on rows with NaN, -inf and +0 / -0 ties is the
    reference's fold from x0 bit for bit (NaN matches NaN)."""
    x = max_fold_probe_rows(cols, 3 * cols)
    rows = x.shape[0] - x.shape[0] % bm
    x = np.ascontiguousarray(x[:rows])
    say(f"tile ir row_max special values {rows}x{cols} BM={bm}")
    y0 = np.full((rows, 1), 11.0, np.float32)
    _, got = _run(hip, T.row_reduce(bm, cols, "max", 2), [x, y0], rows // bm,
                  hip.ROUTE_REDUCE_ROWS)
    assert_same_bits(got.reshape(rows), cpuref.reduce_rows(x, cpuref.REDUCE_MAX),
                     what="routed row max")


@pytest.mark.parametrize("bm,bn,d,n_q,s_k,programs,passes", [
    (32, 64, 128, 256, 512, 8, True),
    (16, 32, 64, 96, 200, 5, False),   # keys truncated to 192; 5 of 6 query tiles
    (64, 16, 48, 64, 64, 1, True),
])
def test_attention_route_matches_the_oracle(hip, bm, bn, d, n_q, s_k, programs, passes):
    """The DSL attention loop (K transposed, no mask), routed and launched:
    within fp32 tolerance (|g - r| <= 1e-5 + 1e-4 |r|) of the oracle's
    statement of the same program and of the oracle's non-causal attention
    over the keys the program reads (whole BN blocks, K = kt^T); rows no
    program owns stay untouched."""
    say(f"tile ir attention BM={bm} BN={bn} D={d} n_q={n_q} S={s_k} programs={programs}")
    scale = 1 / np.sqrt(d)
    r = rng(bm + bn + d)
    q = r.normal(size=(n_q, d)).astype(np.float32)
    kt = r.normal(size=(d, s_k)).astype(np.float32)
    v = r.normal(size=(s_k, d)).astype(np.float32)
    o0 = np.full((n_q, d), 11.0, np.float32)
    *_, got = _run(hip, T.attention(bm, bn, d, scale, passes=passes), [q, kt, v, o0], programs,
                   hip.ROUTE_ATTENTION)
    rows = programs * bm
    ref = cpuref.dsl_attention_f32(q, kt, v, bn, np.float32(scale), np.float32(-1e30), n_q=rows)
    assert_close(got[:rows], ref, atol=1e-5, rtol=1e-4, what="routed attention")
    n_keys = (s_k // bn) * bn
    assert rows <= n_keys
    qq = np.zeros((n_keys, d), np.float32)
    qq[:rows] = q[:rows]
    fwd = cpuref.attention_fwd(qq, np.ascontiguousarray(kt[:, :n_keys].T),
                               np.ascontiguousarray(v[:n_keys]), np.float32(scale), causal=False,
                               q_end=rows)[:rows]
    assert_close(got[:rows], fwd, atol=1e-5, rtol=1e-4, what="routed attention vs attention_fwd")
    np.testing.assert_array_equal(got[rows:], 11.0)
