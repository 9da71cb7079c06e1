"""GPU runs of kernels generated from LLIR (tests/golden/llir/, hand-written in
the reference's printed form) through sile_hip_llir_compile + module_load +
sile_hip_launch_llir, against the reference's fixtures and the CPU oracle.
vec_add, relu and matmul are bit-exact (the matmul in the canonical order,
compiled without contraction); softmax is within 1e-6 relative of the oracle
(device expf against the host's), parallel_reduce within float rounding of
the atomic order."""
import json
import os

import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import assert_close, rng, say
from tests.test_llir import PLANS, text

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_fixtures.json")


@pytest.fixture(scope="module")
def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def kernels(hip):
    ks = {name: hip.LlirKernel(text(name), plan) for name, plan in PLANS.items()}
    yield ks
    for k in ks.values():
        k.close()


def _run(hip, kern, arrays, grid):
    bufs = [hip.DeviceBuffer.from_array(a) for a in arrays]
    shapes = [d for a in arrays for d in a.shape]
    kern([b.ptr for b in bufs], shapes, grid)
    return [b.download(a.dtype, a.shape) for b, a in zip(bufs, arrays)]


def test_vec_add(hip, kernels, fixtures):
    fx = fixtures["vec_add"]
    say("llir vec_add fixture and 4096 random")
    a = np.full(16, fx["a_fill"], np.float32)
    b = np.full(16, fx["b_fill"], np.float32)
    c = _run(hip, kernels["vec_add"], [a, b, np.zeros(16, np.float32)], (4, 1, 1))[2]
    np.testing.assert_array_equal(c, fx["expected_fill"])
    a, b = rng(1).normal(size=4096).astype(np.float32), rng(2).normal(size=4096).astype(np.float32)
    c = _run(hip, kernels["vec_add"], [a, b, np.zeros(4096, np.float32)], (1024, 1, 1))[2]
    np.testing.assert_array_equal(c, a + b)


def test_relu(hip, kernels, fixtures):
    fx = fixtures["relu_8"]
    say("llir relu fixture")
    x = _run(hip, kernels["relu"], [np.array(fx["x"], np.float32)], (1, 1, 1))[0]
    np.testing.assert_array_equal(x, np.array(fx["expected"], np.float32))


def test_matmul(hip, kernels, fixtures):
    fx = fixtures["matmul_4x4"]
    say("llir matmul 4x4 fixture and 64x40x48 bit-exact")
    a = np.array(fx["a"]["data"], np.float32).reshape(fx["a"]["shape"])
    b = np.array(fx["b"]["data"], np.float32).reshape(fx["b"]["shape"])
    c = _run(hip, kernels["matmul"], [a, b, np.zeros((4, 4), np.float32)], (4, 1, 1))[2]
    np.testing.assert_array_equal(c.ravel(), np.array(fx["expected"], np.float32))
    a = rng(3).uniform(-1, 1, size=(64, 41)).astype(np.float32)   # K' = 40 (BK = 2)
    b = rng(4).uniform(-1, 1, size=(41, 48)).astype(np.float32)
    grid = (32 * 24, 1, 1)
    got = _run(hip, kernels["matmul"], [a, b, np.zeros((64, 48), np.float32)], grid)[2]
    ref = np.zeros((64, 48), np.float32)
    cpuref.kernel_matmul(a, b, ref, grid, 2, 2, 2)
    np.testing.assert_array_equal(got, ref)


def test_softmax(hip, kernels, fixtures):
    fx = fixtures["softmax_4x8"]
    say("llir softmax fixture and [64, 8] random")
    x = np.array(fx["x"]["data"], np.float32).reshape(fx["x"]["shape"])
    y = _run(hip, kernels["softmax"], [x, np.zeros_like(x)], tuple(fx["grid"]))[1]
    np.testing.assert_allclose(y.sum(axis=1), fx["expected_row_sum"], atol=fx["tolerance_abs"])
    x = rng(5).normal(scale=2.0, size=(64, 8)).astype(np.float32)
    y = _run(hip, kernels["softmax"], [x, np.zeros_like(x)], (32, 1, 1))[1]
    ref = np.zeros_like(x)
    cpuref.kernel_softmax(x, ref, (32, 1, 1), 2, 8)
    assert_close(y, ref, atol=1e-7, rtol=1e-6, what="llir softmax")


def test_parallel_reduce(hip, kernels):
    say("llir parallel_reduce: 100000 ones and 1600 random")
    x = np.ones(100000, np.float32)
    out = _run(hip, kernels["parallel_reduce"], [x, np.zeros(1, np.float32)], (6250, 1, 1))[1]
    assert out[0] == 100000.0
    x = rng(6).uniform(0, 1, size=1600).astype(np.float32)
    out = _run(hip, kernels["parallel_reduce"], [x, np.zeros(1, np.float32)], (100, 1, 1))[1]
    parts = cpuref.parallel_reduce_partials(x, 100, 16)
    assert_close(out[0], parts.astype(np.float64).sum(), atol=1e-3, rtol=1e-5, what="llir reduce")


# ---- one workgroup per program (loops of >= 256 iterations spread over lanes) ----

from tests.helpers import assert_same_bits, max_fold_probe_rows  # noqa: E402
from tests.test_llir import parallel_reduce_llir, softmax_llir, vec_add_llir  # noqa: E402

# row_max<BN>: out[pid] = the fold from x[pid][0] over the row's BN columns
# (reduce.rs:10-30), one row per program, written in the printed LLIR form
ROW_MAX_LLIR = """\
define void @row_max(ptr addrspace(1) %x, ptr addrspace(1) %out, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %x [rank=2, shape_offset=0, elem=f32]
  ; sile.param %out [rank=1, shape_offset=2, elem=f32]
  ; sile.param %__sile_shapes [elem=i64]
bb0:
  %__shape_x = getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0
  %ldx_p = getelementptr i64, ptr addrspace(4) %__shape_x, i64 1
  %ldx = load i64, ptr addrspace(4) %ldx_p
  %pid = call i32 @llvm.nvvm.ctaid.x()
  %xrow = mul %pid, %ldx
  %x0p = getelementptr f32, ptr addrspace(1) %x, i64 %xrow
  %x0 = load f32, ptr addrspace(1) %x0p
  br label %rm_header ; args(1, %x0)
rm_header:
  ; args(%c: i64, %mx: f32)
  %cond = icmp slt %c, BN
  br i1 %cond, label %rm_body, label %rm_done
rm_body:
  %xi = add %xrow, %c
  %xp = getelementptr f32, ptr addrspace(1) %x, i64 %xi
  %xv = load f32, ptr addrspace(1) %xp
  %gt = fcmp ogt %xv, %mx
  %mx_next = select i1 %gt, f32 %xv, f32 %mx
  %c_next = add %c, 1
  br label %rm_header ; args(%c_next, %mx_next)
rm_done:
  %op = getelementptr f32, ptr addrspace(1) %out, i64 %pid
  store f32 %mx, ptr addrspace(1) %op
  ret void
}
"""


@pytest.mark.parametrize("rows,bm,bn", [(64, 4, 8192), (10, 2, 300), (8, 1, 1000)])
def test_spread_softmax(hip, rows, bm, bn):
    """softmax<BM, BN> with its loops spread over a 1024-lane workgroup per
    program: within 1e-7 + 1e-5 |r| of the oracle's tile semantics (the row
    sum is a tree over lanes instead of one chain; the max is the fold)."""
    say(f"llir spread softmax<{bm}, {bn}> over [{rows}, {bn}]")
    kern = hip.LlirKernel(softmax_llir(bm, bn), (1, bm, bn))
    x = rng(bm + bn).normal(scale=2.0, size=(rows, bn)).astype(np.float32)
    grid = (rows // bm, 1, 1)
    y = _run(hip, kern, [x, np.zeros_like(x)], grid)[1]
    ref = np.zeros_like(x)
    cpuref.kernel_softmax(x, ref, grid, bm, bn)
    assert_close(y, ref, atol=1e-7, rtol=1e-5, what="llir spread softmax")
    kern.close()


@pytest.mark.parametrize("bn", [4096, 1000])
def test_spread_max_fold_is_bit_exact(hip, bn):
    """The spread max fold (lane partials with their first iteration, merged
    by value then iteration, then against x0) equals the sequential fold bit
    for bit on rows with NaN, -inf and +0 / -0 ties."""
    x = max_fold_probe_rows(bn, bn + 7)
    rows = x.shape[0]
    say(f"llir spread row max over [{rows}, {bn}]")
    kern = hip.LlirKernel(ROW_MAX_LLIR.replace("BN", str(bn)), (1, 1, 1))
    out = _run(hip, kern, [x, np.full(rows, 5.0, np.float32)], (rows, 1, 1))[1]
    assert_same_bits(out, cpuref.reduce_rows(x, cpuref.REDUCE_MAX), what="spread row max")
    kern.close()


def test_spread_reduce_and_vec_add(hip):
    say("llir spread parallel_reduce<4096> and vec_add<4096>")
    kern = hip.LlirKernel(parallel_reduce_llir(4096), None)
    x = np.ones(1 << 20, np.float32)
    out = _run(hip, kern, [x, np.zeros(1, np.float32)], (256, 1, 1))[1]
    assert out[0] == float(1 << 20)   # one atomic add per program, sums of ones exact
    x = rng(8).uniform(0, 1, size=1 << 16).astype(np.float32)
    out = _run(hip, kern, [x, np.zeros(1, np.float32)], (16, 1, 1))[1]
    assert_close(out[0], x.astype(np.float64).sum(), atol=1e-2, rtol=1e-5, what="spread reduce")
    kern.close()
    kern = hip.LlirKernel(vec_add_llir(4096), (2, 1, 4096))
    a = rng(9).integers(-1000, 1000, 1 << 16).astype(np.float32)
    b = rng(10).integers(-1000, 1000, 1 << 16).astype(np.float32)
    c = _run(hip, kern, [a, b, np.zeros_like(a)], (16, 1, 1))[2]
    np.testing.assert_array_equal(c, a + b)
    kern.close()


# ---- LLIR in the reference's loop shapes (tests/llir_shapes.py) ----

from tests import llir_shapes  # noqa: E402


@pytest.mark.parametrize("rows,bm,bn", [(64, 4, 8192), (10, 2, 300), (8, 1, 1000), (6, 2, 8)])
def test_reference_shaped_softmax(hip, rows, bm, bn):
    """softmax<BM, BN> in the reference's loop shapes (a loop nest and a
    private tile per op; reductions from element 0): spread over a
    1024-lane workgroup per program (one program a lane at BN = 8), within
    1e-7 + 1e-5 |r| of the oracle's tile semantics."""
    say(f"llir reference-shaped softmax<{bm}, {bn}> over [{rows}, {bn}]")
    kern = hip.LlirKernel(llir_shapes.softmax(bm, bn), (1, bm, bn))
    x = rng(bm * bn + 3).normal(scale=2.0, size=(rows, bn)).astype(np.float32)
    grid = (rows // bm, 1, 1)
    y = _run(hip, kern, [x, np.zeros_like(x)], grid)[1]
    ref = np.zeros_like(x)
    cpuref.kernel_softmax(x, ref, grid, bm, bn)
    assert_close(y, ref, atol=1e-7, rtol=1e-5, what="reference-shaped softmax")
    kern.close()


@pytest.mark.parametrize("bn", [4096, 1000])
def test_reference_shaped_row_max_is_bit_exact(hip, bn):
    """The row max in the reference's shapes (the reduction's element 0 read
    from the LDS copy its lane wrote, the rest folded over the lanes) equals
    the sequential fold bit for bit on rows with NaN, -inf and +0 / -0 ties."""
    x = max_fold_probe_rows(bn, bn + 11)
    rows = x.shape[0]
    say(f"llir reference-shaped row max over [{rows}, {bn}]")
    kern = hip.LlirKernel(llir_shapes.row_max(bn), (1, 1, 1))
    out = _run(hip, kern, [x, np.full(rows, 5.0, np.float32)], (rows, 1, 1))[1]
    assert_same_bits(out, cpuref.reduce_rows(x, cpuref.REDUCE_MAX), what="reference-shaped row max")
    kern.close()


@pytest.mark.parametrize("fused", [False, True])
def test_reference_shaped_vec_add(hip, fused):
    say(f"llir reference-shaped vec_add<4096> and <8>, fused={fused}")
    gen = llir_shapes.vec_add_fused if fused else llir_shapes.vec_add
    for tile, n in ((4096, 1 << 16), (8, 4096)):
        kern = hip.LlirKernel(gen(tile), (2, 1, tile))
        a = rng(tile).integers(-1000, 1000, n).astype(np.float32)
        b = rng(tile + 1).integers(-1000, 1000, n).astype(np.float32)
        c = _run(hip, kern, [a, b, np.zeros_like(a)], (n // tile, 1, 1))[2]
        np.testing.assert_array_equal(c, a + b)
        kern.close()


@pytest.mark.parametrize("bm,bn,bk,m,n,k", [
    (64, 64, 8, 128, 192, 72),    # 4096 cells a program, nine k tiles
    (64, 64, 8, 64, 64, 75),      # K truncated to 72 (whole BK tiles)
    (32, 32, 8, 64, 64, 64),      # the mlp example's gemm tiles
    (16, 32, 4, 48, 96, 20),      # 512 cells a program
    (128, 64, 8, 256, 128, 40),   # 8192 cells: two jammed groups of four a lane
    (96, 32, 8, 96, 64, 24),      # 3072 cells: one group of three
    (32, 96, 8, 64, 192, 16),     # the same, the column per cell (96 does not divide 1024)
    (24, 64, 8, 48, 128, 16),     # 1536 cells: slot form, a partial slot, rows in scalar registers
    (256, 128, 4, 256, 256, 8),   # 32768 cells: the strided form, rows in scalar registers
])
def test_canonical_matmul_nest(hip, bm, bn, bk, m, n, k):
    """The canonical matmul's LLIR with its row x column nest spread over the
    lanes (each cell's k loop serial on one lane): bit for bit the oracle's
    canonical order."""
    say(f"llir canonical matmul<{bm}, {bn}, {bk}> {m}x{n}x{k}")
    kern = hip.LlirKernel(llir_shapes.matmul(bm, bn, bk), (2, bm, bn))
    r = rng(m + n + k)
    a = r.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = r.uniform(-1, 1, size=(k, n)).astype(np.float32)
    grid = (m // bm, n // bn, 1)
    c = _run(hip, kern, [a, b, np.zeros((m, n), np.float32)], (grid[0] * grid[1], 1, 1))[2]
    want = np.zeros((m, n), np.float32)
    cpuref.kernel_matmul(a, b, want, grid, bm, bn, bk)
    assert_same_bits(c, want, what="llir canonical matmul")
    kern.close()


@pytest.mark.parametrize("by", ["row", "col"])
def test_nest_with_a_trip_count_per_cell(hip, by):
    """The canonical matmul with its k loop bounded by the cell's row or
    column (tests/test_llir.py triangular_matmul): bounded by the column the
    lane's cells still run jammed, bounded by the row one slot at a time;
    both bit for bit a numpy restatement of the loops (each cell a
    sequential sum of rounded products over k < its bound)."""
    from tests.test_llir import triangular_matmul
    say(f"llir canonical matmul<64, 64, 8> with k < {by}")
    kern = hip.LlirKernel(triangular_matmul(64, 64, 8, by), (2, 64, 64))
    m, n, k = 128, 128, 72
    r = rng(91 if by == "row" else 92)
    a = r.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = r.uniform(-1, 1, size=(k, n)).astype(np.float32)
    c = _run(hip, kern, [a, b, np.zeros((m, n), np.float32)], (4, 1, 1))[2]
    kern.close()
    want = np.zeros((m, n), np.float32)
    for row in range(m):
        for col0 in range(0, n, 64):
            s = np.zeros(64, np.float32)
            for kk in range(k):
                # the bound is the cell's row / column inside its 64 x 64 tile
                live = (np.full(64, row % 64) if by == "row" else np.arange(64)) > kk
                s = np.where(live, s + a[row, kk] * b[kk, col0:col0 + 64], s).astype(np.float32)
            want[row, col0:col0 + 64] = s
    assert_same_bits(c, want, what=f"llir k < {by}")


@pytest.mark.parametrize("t", [32, 64])   # 64: the nest whose spread copy is jammed
def test_canonical_matmul_nest_in_order_when_rows_overlap(hip, t):
    """With ldc < BN the rows of the C tile overlap: the nest then runs in
    order on lane 0, so the last write of each element is the sequential
    one (one program, planned on a; numpy restatement of the loops)."""
    say(f"llir canonical matmul<{t}, {t}, 8>, ldc 16: the in-order path")
    kern = hip.LlirKernel(llir_shapes.matmul(t, t, 8), (0, t, 16))
    r = rng(77 + t)
    a = r.integers(-4, 5, size=(t, 16)).astype(np.float32)
    b = r.integers(-4, 5, size=(16, t)).astype(np.float32)
    crows = (t - 1) + (t - 1) // 16 + 2     # holds element (t - 1) * 16 + t - 1
    c = _run(hip, kern, [a, b, np.zeros((crows, 16), np.float32)], (1, 1, 1))[2]
    want = np.zeros((crows, 16), np.float32).ravel()
    for row in range(t):
        for col in range(t):
            s = np.float32(0.0)
            for kk in range(16):
                s = np.float32(s + np.float32(a[row, kk] * b[kk, col]))
            want[row * 16 + col] = s
    np.testing.assert_array_equal(c.ravel(), want)
    kern.close()


@pytest.mark.parametrize("bm,bn,bk,grid", [(32, 32, 16, (2, 3)), (64, 64, 8, (1, 2)), (16, 16, 32, (3, 2)),
                                          (48, 32, 8, (2, 2)),    # 1536 cells: a partial second slot
                                          (128, 128, 4, (1, 2))])  # 16 accumulator slots a lane, jammed
def test_tile_mma_nest(hip, bm, bn, bk, grid):
    """Tiles loaded, a zero accumulator, the tile MMA nest (mma.rs) and the
    store, every nest spread over the lanes: bit for bit the canonical order
    (sum from 0.0, products rounded, k in order)."""
    m, n = grid[0] * bm, grid[1] * bn
    say(f"llir tile mma<{bm}, {bn}, {bk}> {m}x{n}x{bk}")
    kern = hip.LlirKernel(llir_shapes.mma_program(bm, bn, bk), (2, bm, bn))
    r = rng(bm * bn + bk)
    a = r.uniform(-1, 1, size=(m, bk)).astype(np.float32)
    b = r.uniform(-1, 1, size=(bk, n)).astype(np.float32)
    c = _run(hip, kern, [a, b, np.zeros((m, n), np.float32)], (grid[0] * grid[1], 1, 1))[2]
    want = np.zeros((m, n), np.float32)
    cpuref.kernel_matmul(a, b, want, (*grid, 1), bm, bn, bk)
    assert_same_bits(c, want, what="llir tile mma")
    kern.close()


@pytest.mark.parametrize("bm,bn,is_max", [(64, 1024, True), (64, 1024, False), (20, 300, True),
                                          (33, 512, False)])
def test_reference_shaped_column_reduce(hip, bm, bn, is_max):
    """Reductions along axis 0 in the reference's shape (a column a lane,
    rows folded in order from row 0): bit for bit the left fold, with NaN,
    -inf and +0 / -0 columns for the max."""
    say(f"llir column {'max' if is_max else 'sum'} over [{bm}, {bn}] tiles")
    progs = 3
    x = rng(bm + bn).normal(size=(bm, bn * progs)).astype(np.float32)
    if is_max:
        probe = max_fold_probe_rows(bm, bm + 5)        # rows become columns
        k = min(probe.shape[0], bn * progs)
        x[:, :k] = probe[:k].T
    kern = hip.LlirKernel(llir_shapes.col_reduce(bm, bn, is_max), (1, 1, bn))
    out = _run(hip, kern, [x, np.full(bn * progs, 7.0, np.float32)], (progs, 1, 1))[1]
    acc = x[0].copy()
    for i in range(1, bm):
        acc = np.where(x[i] > acc, x[i], acc) if is_max else (acc + x[i]).astype(np.float32)
    assert_same_bits(out, acc.astype(np.float32), what="reference-shaped column reduce")
    kern.close()


@pytest.mark.parametrize("gen", ["fused_mma_loop", "mma_k_loop"])
@pytest.mark.parametrize("bm,bn,bk,m,n,k", [(32, 32, 8, 64, 96, 64), (64, 64, 16, 128, 64, 48),
                                            (4, 4, 2, 8, 8, 6)])
def test_k_tile_loop_with_a_carried_accumulator(hip, gen, bm, bn, bk, m, n, k):
    """K-tile loops carrying the accumulator tile (fused: the MMA reads a and
    b from their buffers and updates the tile in place, starting from the
    splat; unfused: loaded tiles, the MMA into a result tile that is carried
    on): bit for bit the canonical order (one sequential sum over all k)."""
    say(f"llir {gen}<{bm}, {bn}, {bk}> {m}x{n}x{k}")
    kern = hip.LlirKernel(getattr(llir_shapes, gen)(bm, bn, bk), (2, bm, bn))
    r = rng(m * n + k)
    a = r.uniform(-1, 1, size=(m, k)).astype(np.float32)
    b = r.uniform(-1, 1, size=(k, n)).astype(np.float32)
    grid = (m // bm, n // bn, 1)
    c = _run(hip, kern, [a, b, np.zeros((m, n), np.float32)], (grid[0] * grid[1], 1, 1))[2]
    want = np.zeros((m, n), np.float32)
    cpuref.kernel_matmul(a, b, want, grid, bm, bn, bk)
    assert_same_bits(c, want, what=f"llir {gen}")
    kern.close()


def test_memcpy_round_trip(hip):
    """Each program copies its 4 elements of x into a private tile and from
    there into y (memcpy both ways): y equals x bit for bit."""
    from tests.test_llir import MEMCPY_LLIR
    say("llir memcpy buffer -> tile -> buffer")
    kern = hip.LlirKernel(MEMCPY_LLIR, None)
    x = rng(5).normal(size=4096).astype(np.float32)
    x[7] = -0.0
    x[9] = np.nan
    y = _run(hip, kern, [x, np.zeros_like(x)], (1024, 1, 1))[1]
    assert_same_bits(y, x, what="memcpy round trip")
    kern.close()


def test_every_operation_runs(hip):
    """Each binary op, compare predicate, cast and select of the printed form
    on a = 7.75, b = -2.5 gives the C targets' value (casts convert, `sdiv`
    truncates toward zero, `and` / `or` are bitwise, booleans widen to 0/1)."""
    from tests.test_llir import OPS_EXPECTED, ops_llir
    say("llir every operation")
    kern = hip.LlirKernel(ops_llir(), None)
    x = np.array([7.75, -2.5], np.float32)
    out = _run(hip, kern, [x, np.full(20, 99.0, np.float32)], (1, 1, 1))[1]
    assert_same_bits(out, np.array(OPS_EXPECTED, np.float32), what="llir operations")
    kern.close()
