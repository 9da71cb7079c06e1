"""Pins the CPU oracle (oracle/sile_cpuref.c) before it is trusted as the checker.

Each check is chosen so that a plausible mistake in the restatement (a dropped
K truncation, a transposed operand, a wrong program-id decode, FMA
contraction, a reordered sum, a wrong rounding mode) fails at least one of:
  * the reference's own literal fixtures (tests/golden/reference_fixtures.json),
  * closed forms (exact integer GEMMs, constant-row softmax, n(n+1)/2),
  * brute force / float64 recomputation on small inputs,
  * order-sensitivity probes showing the exact-order claims are not vacuous.
"""
import json
import os

import numpy as np
import pytest

from oracle import cpuref
from tests.helpers import assert_close, rng

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "reference_fixtures.json")


@pytest.fixture(scope="module")
def fixtures():
    with open(GOLDEN) as f:
        return json.load(f)


# ---------------------------------------------------------------- matmul (a1, a3)

def test_matmul_reference_fixture(fixtures):
    fx = fixtures["matmul_4x4"]
    a = np.array(fx["a"]["data"], np.float32).reshape(fx["a"]["shape"])
    b = np.array(fx["b"]["data"], np.float32).reshape(fx["b"]["shape"])
    c = np.array(fx["c_init"]["data"], np.float32).reshape(fx["c_init"]["shape"])
    cpuref.kernel_matmul(a, b, c, fx["grid"], fx["bm"], fx["bn"], fx["bk"])
    np.testing.assert_array_equal(c.ravel(), np.array(fx["expected"], np.float32))


def test_matmul_program_decode_and_guard():
    # grid smaller than the tile count: only pids 0..1 run -> tiles (0,0), (0,1)
    a = np.arange(16, dtype=np.float32).reshape(4, 4)
    b = np.eye(4, dtype=np.float32)
    c = np.full((4, 4), -7.0, np.float32)
    cpuref.kernel_matmul(a, b, c, (2, 1, 1), 2, 2, 2)
    np.testing.assert_array_equal(c[:2], a[:2])
    np.testing.assert_array_equal(c[2:], -7.0)
    # grid larger than the tile count: extra programs are skipped
    c = np.zeros((4, 4), np.float32)
    cpuref.kernel_matmul(a, b, c, (100, 1, 1), 2, 2, 2)
    np.testing.assert_array_equal(c, a)
    # tile count truncates: c[5,5] with BM=BN=2 covers rows/cols 0..3 only
    c = np.full((5, 5), 3.0, np.float32)
    a5 = np.ones((5, 4), np.float32)
    b5 = np.ones((4, 5), np.float32)
    cpuref.kernel_matmul(a5, b5, c, (4, 1, 1), 2, 2, 2)
    np.testing.assert_array_equal(c[:4, :4], 4.0)
    np.testing.assert_array_equal(c[4, :], 3.0)
    np.testing.assert_array_equal(c[:, 4], 3.0)
    assert cpuref.total_tiles([5, 5], 2, 2) == 4
    assert cpuref.total_tiles([7], 1, 3) == 7


def test_matmul_k_truncation():
    # K = 5, BK = 2 -> k runs over 0..3 only (canonical_matmul.rs:58-73)
    a = rng(11).integers(-3, 4, size=(4, 5)).astype(np.float32)
    b = rng(12).integers(-3, 4, size=(5, 4)).astype(np.float32)
    c = np.zeros((4, 4), np.float32)
    cpuref.kernel_matmul(a, b, c, (4, 1, 1), 2, 2, 2)
    np.testing.assert_array_equal(c, a[:, :4] @ b[:4, :])
    assert not np.array_equal(c, a @ b)


def test_matmul_integer_closed_form():
    # integer data: every partial sum is an exact fp32 integer, so any order gives a @ b
    a = rng(1).integers(-8, 9, size=(64, 96)).astype(np.float32)
    b = rng(2).integers(-8, 9, size=(96, 32)).astype(np.float32)
    c = np.zeros((64, 32), np.float32)
    cpuref.kernel_matmul(a, b, c, (64 // 16 * 32 // 8, 1, 1), 16, 8, 32)
    np.testing.assert_array_equal(c, (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))


def _sequential_f32_gemm(a, b):
    """Independent numpy statement of the canonical order: a fp32 running sum
    over k, each step rounding the product and then the add."""
    s = np.zeros((a.shape[0], b.shape[1]), np.float32)
    for k in range(a.shape[1]):
        p = (a[:, k:k + 1] * b[k:k + 1, :]).astype(np.float32)
        s = (s + p).astype(np.float32)
    return s


def test_matmul_exact_order_random():
    a = rng(1).uniform(-1, 1, size=(64, 128)).astype(np.float32)
    b = rng(2).uniform(-1, 1, size=(128, 64)).astype(np.float32)
    c = np.zeros((64, 64), np.float32)
    cpuref.kernel_matmul(a, b, c, (4, 1, 1), 32, 32, 32)
    ref = _sequential_f32_gemm(a, b)
    np.testing.assert_array_equal(c, ref)
    # the order is observable: a float64 sum rounded once, or an FMA chain,
    # differs in the last bits for random data (so the equality above pins it)
    f64 = (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32)
    assert not np.array_equal(c, f64)
    fma = np.zeros_like(ref)
    for k in range(a.shape[1]):
        fma = (fma.astype(np.float64) + a[:, k:k + 1].astype(np.float64) * b[k:k + 1, :]).astype(np.float32)
    assert not np.array_equal(c, fma)
    assert_close(c, f64, atol=1e-5, rtol=1e-4, what="fp64 sanity")


def test_gemm_nt_matches_kernel_matmul():
    a = rng(3).uniform(-1, 1, size=(96, 160)).astype(np.float32)
    b = rng(4).uniform(-1, 1, size=(160, 64)).astype(np.float32)
    c = np.zeros((96, 64), np.float32)
    cpuref.kernel_matmul(a, b, c, (1000, 1, 1), 32, 32, 32)
    c2 = cpuref.gemm_nt(a, np.ascontiguousarray(b.T), bk=32)
    np.testing.assert_array_equal(c, c2)
    # sampling: every 2nd row tile of 32 rows
    c3 = np.full((96, 64), np.nan, np.float32)
    cpuref.gemm_nt(a, np.ascontiguousarray(b.T), bk=32, bm=32, row_tile_step=2, out=c3)
    np.testing.assert_array_equal(c3[0:32], c[0:32])
    np.testing.assert_array_equal(c3[64:96], c[64:96])
    assert np.isnan(c3[32:64]).all()


# ---------------------------------------------------------------- reduce (a4, a5, a8)

def test_reduce_rows_max_and_sequential_sum():
    x = rng(5).normal(size=(33, 77)).astype(np.float32)
    np.testing.assert_array_equal(cpuref.reduce_rows(x, cpuref.REDUCE_MAX), x.max(axis=1))
    seq = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]  # left fold from element 0
    np.testing.assert_array_equal(cpuref.reduce_rows(x, cpuref.REDUCE_SUM), seq)


def test_reduce_rows_max_special_values():
    """The reference's ReduceMax folds acc = x0; acc = (x > acc) ? x : acc
    (reduce.rs:10-30), which fixes these cases: NaN at column 0 gives NaN, a
    NaN later never replaces acc, an all -inf row gives -inf, and of a +0 / -0
    tie the first in row order is kept.  numpy's max (NaN-propagating, tie
    sign unspecified) differs on them, so each case is a closed form."""
    nan, inf = np.float32(np.nan), np.float32(np.inf)
    rows = [
        ([nan, 1, 2, 3], nan),
        ([1, nan, 3, 2], 3.0),
        ([nan] * 4, nan),
        ([-inf] * 4, -inf),
        ([-inf, nan, nan, nan], -inf),
        ([-1, -0.0, 0.0, -2], -0.0),
        ([-1, 0.0, -0.0, -2], 0.0),
        ([-0.0, -5, 0.0, 0.0], -0.0),
        ([nan, inf, 0.0, -inf], nan),
        ([5, inf, nan, inf], inf),
    ]
    x = np.array([r for r, _ in rows], np.float32)
    got = cpuref.reduce_rows(x, cpuref.REDUCE_MAX)
    for (_, want), g in zip(rows, got):
        want = np.float32(want)
        if np.isnan(want):
            assert np.isnan(g)
        else:
            assert g.view(np.uint32) == want.view(np.uint32), (g, want)


def _ones_vec4_sum(extent, past_end):
    """Closed form of the reference's fused vec4 sum over a row of ones
    (fused_reduce.rs:1182-1256 with single_axis.rs:180-260): the loop form
    (extent > 16) runs ceil(extent/4) windows of 4 and then re-adds the
    extent % 4 elements of the partial last window in the scalar tail; a
    window element past the buffer's end counts 0 (`past_end`), otherwise it
    is the next element of the buffer (1 here).  The unrolled form (extent
    <= 16) reads extent/4 windows and the tail once: exactly `extent`."""
    if extent <= 16:
        return float(extent)
    rem = extent % 4
    if rem == 0:
        return float(extent)
    windows = 4 * ((extent + 3) // 4) if not past_end else 4 * (extent // 4) + rem
    return float(windows + rem)


@pytest.mark.parametrize("tile", [4, 7, 16, 17, 18, 19, 20, 21, 1000, 1003])
def test_parallel_reduce_vec4_ones_closed_form(tile):
    """TILE = 18 over ones: every program but the last reads 2 elements of
    the next tile in its last window and re-adds 2 in the tail: 16 + 4 + 2 =
    22; the last program's window runs past the buffer (0.0f there): 16 + 2
    + 2 = 20."""
    programs = 9
    a = np.ones(programs * tile, np.float32)
    parts = cpuref.parallel_reduce_partials(a, programs, tile)
    interior, last = _ones_vec4_sum(tile, False), _ones_vec4_sum(tile, True)
    np.testing.assert_array_equal(parts[:-1], interior)
    assert parts[-1] == last
    if tile == 18:
        assert (interior, last) == (22.0, 20.0)
    out = np.zeros(1, np.float32)
    cpuref.kernel_parallel_reduce(a, out, (programs, 1, 1), tile)
    assert out[0] == interior * (programs - 1) + last


@pytest.mark.parametrize("cols", [5, 17, 18, 19, 33])
def test_reduce_rows_vec4_ones_closed_form(cols):
    """Rows of a [rows, cols] buffer: the last window of a row reads the next
    row's first elements; only the last row's reads past the buffer."""
    x = np.ones((5, cols), np.float32)
    got = cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4)
    np.testing.assert_array_equal(got[:-1], _ones_vec4_sum(cols, False))
    assert got[-1] == _ones_vec4_sum(cols, True)
    # inside a wider pitch the window reads the row's own padding (ones here)
    xp = np.ones((3, cols + 8), np.float32)
    np.testing.assert_array_equal(cpuref.reduce_rows(xp, cpuref.REDUCE_SUM_VEC4, cols=cols),
                                  _ones_vec4_sum(cols, False))
    xp[:, cols:] = 0.0
    np.testing.assert_array_equal(cpuref.reduce_rows(xp, cpuref.REDUCE_SUM_VEC4, cols=cols),
                                  _ones_vec4_sum(cols, True))


def test_vec4_grouping_and_start_probes():
    """Inputs whose result fixes the grouping, each chosen so a plausible
    other order gives a different float:
      [1, 1, 2^24, 0]           ((v0+v1)+v2)+v3 = 2^24+2; a pairwise tree 2^24
      [2^24,0,0,0, 1,1,0,0]     chunk sums added: 2^24+2; an element-wise fold 2^24
      16 x -0.0                 unrolled start at chunk 0: -0.0
      20 x -0.0                 loop start at +0.0f: +0.0"""
    f = np.float32
    big = f(2.0 ** 24)
    x = np.array([[1, 1, big, 0]], np.float32)
    assert cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4)[0] == big + 2
    x = np.array([[big, 0, 0, 0, 1, 1, 0, 0]], np.float32)
    assert cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4)[0] == big + 2
    assert cpuref.reduce_rows(x, cpuref.REDUCE_SUM)[0] == big
    z = cpuref.reduce_rows(np.full((1, 16), -0.0, np.float32), cpuref.REDUCE_SUM_VEC4)[0]
    assert z == 0.0 and np.signbit(z)
    z = cpuref.reduce_rows(np.full((1, 20), -0.0, np.float32), cpuref.REDUCE_SUM_VEC4)[0]
    assert z == 0.0 and not np.signbit(z)
    # loop form, 17 wide: the last window adds x[16] with 3 elements of the
    # next row; the tail adds x[16] again
    x = np.zeros((2, 17), np.float32)
    x[0, 16] = 1.0
    x[1, :3] = 100.0
    assert cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4)[0] == 302.0


@pytest.mark.parametrize("cols", [4, 7, 16, 17, 1000, 1003])
def test_reduce_rows_vec4_fp64_sanity(cols):
    x = rng(cols).normal(size=(4, cols + 4)).astype(np.float32) * np.float32(1e3)
    x[:, cols:] = 0.0  # the loop's over-read lands on zeros: the row sum itself
    got = cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4, cols=cols)
    ref = x[:, :cols].astype(np.float64).sum(axis=1)
    tail = (cols % 4) if cols > 16 else 0   # the re-added elements
    ref += x[:, (cols // 4) * 4:cols].astype(np.float64).sum(axis=1) if tail else 0.0
    assert_close(got, ref, atol=1e-2, rtol=1e-5, what="vec4 sum vs fp64")


def test_vec4_order_is_observable():
    x = rng(9).normal(size=(64, 1000)).astype(np.float32) * np.float32(1e3)
    v = cpuref.reduce_rows(x, cpuref.REDUCE_SUM_VEC4)
    s = cpuref.reduce_rows(x, cpuref.REDUCE_SUM)
    assert not np.array_equal(v, s)


def test_parallel_reduce_reference_fixtures(fixtures):
    fx = fixtures["parallel_reduce_ones"]
    a = np.full(fx["a"]["shape"], fx["a"]["fill"], np.float32)
    out = np.zeros(1, np.float32)
    cpuref.kernel_parallel_reduce(a, out, fx["grid"], fx["tile"])
    assert abs(out[0] - fx["expected"]) < fx["tolerance_abs"]
    fx = fixtures["parallel_reduce_arange"]
    n = fx["a"]["shape"][0]
    a = np.arange(fx["a"]["arange_from"], fx["a"]["arange_from"] + n, dtype=np.float32)
    out = np.zeros(1, np.float32)
    cpuref.kernel_parallel_reduce(a, out, fx["grid"], fx["tile"])
    assert abs(out[0] - fx["expected"]) <= fx["tolerance_rel"] * fx["expected"]
    assert fx["expected"] == n * (n + 1) / 2


def test_parallel_reduce_partials_order():
    """A program's tile of the rank-1 buffer is summed as a row of the same
    buffer viewed [programs, TILE] (the windows read on into the next tile),
    whose order the closed-form probes above pin; TILE < 4 is the plain
    fold from element 0."""
    a = rng(13).normal(size=3003).astype(np.float32)
    for tile in (1000, 1001, 12):
        progs = a.size // tile
        parts = cpuref.parallel_reduce_partials(a[:progs * tile], progs, tile)
        rows = cpuref.reduce_rows(a[:progs * tile].reshape(progs, tile), cpuref.REDUCE_SUM_VEC4)
        np.testing.assert_array_equal(parts, rows)
    tiny = cpuref.parallel_reduce_partials(a[:6], 2, 3)  # TILE < 4: plain fold
    np.testing.assert_array_equal(tiny, np.add.accumulate(a[:6].reshape(2, 3), axis=1, dtype=np.float32)[:, -1])


# ---------------------------------------------------------------- softmax (a6, a7)

def test_softmax_reference_fixture(fixtures):
    fx = fixtures["softmax_4x8"]
    x = np.array(fx["x"]["data"], np.float32).reshape(fx["x"]["shape"])
    y = np.zeros_like(x)
    cpuref.kernel_softmax(x, y, fx["grid"], fx["bm"], fx["bn"])
    assert np.all(np.abs(y.sum(axis=1) - fx["expected_row_sum"]) < fx["tolerance_abs"])
    # every row is 0..7 shifted, so every row is the same softmax
    np.testing.assert_array_equal(y, np.tile(y[0], (4, 1)))


def test_softmax_closed_forms():
    x = np.full((3, 64), 5.25, np.float32)
    y = cpuref.softmax_rows(x)
    np.testing.assert_array_equal(y, np.float32(1.0 / 64))
    # one dominant entry: exp(-inf-like) underflows to 0, the max gets exactly 1
    x = np.zeros((1, 16), np.float32)
    x[0, 5] = 200.0
    y = cpuref.softmax_rows(x)
    assert y[0, 5] == 1.0 and np.all(np.delete(y[0], 5) == 0.0)


def test_softmax_fp64_and_tile_semantics():
    x = (rng(3).normal(size=(8, 256)) * 2).astype(np.float32)
    y = cpuref.softmax_rows(x)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    assert_close(y, e / e.sum(axis=1, keepdims=True), atol=1e-9, rtol=1e-5, what="fp64")
    # shift invariance is exact up to fp32 rounding of x - m
    y2 = cpuref.softmax_rows(x + np.float32(3.0))
    assert_close(y2, y, atol=1e-9, rtol=1e-5, what="shift")
    # the DSL kernel over [BM, BN] tiles: with BN < row width each tile is
    # normalised on its own, as the reference program does
    yt = np.zeros_like(x)
    cpuref.kernel_softmax(x, yt, (8 * 2, 1, 1), 1, 128)
    np.testing.assert_array_equal(yt[:, :128], cpuref.softmax_rows(x[:, :128]))
    np.testing.assert_array_equal(yt[:, 128:], cpuref.softmax_rows(x[:, 128:]))


# ---------------------------------------------------------------- attention (a9)

def _attn_fp64(q, k, v, scale, causal):
    q, k, v = (t.astype(np.float64) for t in (q, k, v))
    s = q @ k.T * scale
    if causal:
        s = np.where(np.tril(np.ones_like(s, dtype=bool)), s, -np.inf)
    s = s - s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ v) / p.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("causal", [True, False])
def test_attention_fp64(causal):
    q, k, v = (rng(20 + i).normal(size=(96, 32)).astype(np.float32) for i in range(3))
    o = cpuref.attention_fwd(q, k, v, 1 / np.sqrt(32), causal=causal)
    assert_close(o, _attn_fp64(q, k, v, 1 / np.sqrt(32), causal), atol=1e-5, rtol=1e-4, what="attn")


def test_attention_closed_forms():
    s, d = 64, 16
    q, k = (rng(30 + i).normal(size=(s, d)).astype(np.float32) for i in range(2))
    # constant V rows -> every output row is that constant (weights sum to 1)
    v = np.tile(rng(32).normal(size=(1, d)).astype(np.float32), (s, 1))
    o = cpuref.attention_fwd(q, k, v, 0.25, causal=True)
    assert_close(o, v, atol=1e-6, rtol=1e-6, what="const V")
    # query 0 sees only key 0: p = exp(0) = 1, l = 1, so o[0] = v[0] exactly
    v = rng(33).normal(size=(s, d)).astype(np.float32)
    o = cpuref.attention_fwd(q, k, v, 0.25, causal=True)
    np.testing.assert_array_equal(o[0], v[0])
    # zero keys -> uniform weights over the visible prefix: o[i] = mean(v[0..i])
    o = cpuref.attention_fwd(q, np.zeros_like(k), v, 0.25, causal=True)
    means = np.cumsum(v.astype(np.float64), axis=0) / np.arange(1, s + 1)[:, None]
    assert_close(o, means, atol=1e-6, rtol=1e-5, what="uniform")
    # causality: keys/values after row i do not change row i
    k2, v2 = k.copy(), v.copy()
    k2[40:] = 100.0
    v2[40:] = -100.0
    o2 = cpuref.attention_fwd(q, k2, v2, 0.25, causal=True)
    np.testing.assert_array_equal(o2[:40], cpuref.attention_fwd(q, k, v, 0.25)[:40])
    # row sampling computes exactly the requested rows
    part = cpuref.attention_fwd(q, k, v, 0.25, q_begin=10, q_end=20)
    full = cpuref.attention_fwd(q, k, v, 0.25)
    np.testing.assert_array_equal(part[10:20], full[10:20])
    assert np.all(part[:10] == 0) and np.all(part[20:] == 0)


def _dsl_attn_fp64(q, kt, v, scale, n_keys):
    s = (q.astype(np.float64) @ kt[:, :n_keys].astype(np.float64)) * scale
    s -= s.max(axis=1, keepdims=True)
    p = np.exp(s)
    return (p @ v[:n_keys].astype(np.float64)) / p.sum(axis=1, keepdims=True)


@pytest.mark.parametrize("n_q,d,s_k,bn,m0", [
    (48, 32, 256, 32, -1.0e30),
    (17, 64, 200, 64, -1.0e30),   # keys truncated to 192 = 3 whole blocks
    (8, 16, 96, 16, 0.0),         # an initial max inside the score range
    (5, 128, 64, 64, -3.0),
])
def test_dsl_attention_fp64(n_q, d, s_k, bn, m0):
    """The DSL program's online softmax equals softmax(Q K^T scale) V over the
    first (s_k / bn) * bn keys for any initial max the scores do not
    underflow against."""
    r = rng(n_q + d + s_k)
    q = r.normal(size=(n_q, d)).astype(np.float32)
    kt = r.normal(size=(d, s_k)).astype(np.float32)
    v = r.normal(size=(s_k, d)).astype(np.float32)
    scale = 1 / np.sqrt(d)
    o = cpuref.dsl_attention_f32(q, kt, v, bn, scale, m0)
    assert_close(o, _dsl_attn_fp64(q, kt, v, scale, (s_k // bn) * bn), atol=1e-5, rtol=1e-4,
                 what="dsl attention")


def test_dsl_attention_closed_forms():
    r = rng(40)
    n_q, d, s_k, bn = 16, 32, 100, 32
    q = r.normal(size=(n_q, d)).astype(np.float32)
    kt = r.normal(size=(d, s_k)).astype(np.float32)
    v = r.normal(size=(s_k, d)).astype(np.float32)
    # keys past the last whole block never enter, however large their scores
    kt2, v2 = kt.copy(), v.copy()
    kt2[:, 96:] = 50.0
    v2[96:] = 1e6
    np.testing.assert_array_equal(cpuref.dsl_attention_f32(q, kt2, v2, bn, 0.2, -1e30),
                                  cpuref.dsl_attention_f32(q, kt, v, bn, 0.2, -1e30))
    # an initial max above every score: every p and alpha-weighted sum is 0,
    # so each output is 0 / 0
    assert np.isnan(cpuref.dsl_attention_f32(q, kt, v, bn, 0.2, 1e30)).all()
    # one block, constant V rows: every output row is that row
    vc = np.tile(v[:1], (s_k, 1))
    assert_close(cpuref.dsl_attention_f32(q, kt, vc, bn, 0.2, -1e30), vc[:n_q], atol=1e-6,
                 rtol=1e-6, what="const V")
    # the non-causal attention oracle on the same keys (K = kt^T), 3 blocks
    k96 = np.ascontiguousarray(kt[:, :96].T)
    qq = np.zeros((96, d), np.float32)
    qq[:n_q] = q
    o_ref = cpuref.attention_fwd(qq, k96, v[:96], 0.2, causal=False, q_end=n_q)[:n_q]
    assert_close(cpuref.dsl_attention_f32(q, kt, v, bn, 0.2, -1e30), o_ref, atol=1e-6,
                 rtol=1e-5, what="vs attention_fwd")



# ---------------------------------------------------------------- matvec (mlp.rs)

@pytest.mark.parametrize("m,k,bk", [(7, 64, 8), (33, 100, 3), (5, 1000, 32), (4, 9, 1)])
def test_dsl_matvec_fp64(m, k, bk):
    """The matvec program equals x[:, :K'] @ y[:K'] for K' = (k / bk) * bk,
    within fp32 rounding of the sequential sums."""
    r = rng(m + k + bk)
    x = r.normal(size=(m, k)).astype(np.float32)
    y = r.normal(size=k).astype(np.float32)
    kp = (k // bk) * bk
    want = x[:, :kp].astype(np.float64) @ y[:kp].astype(np.float64)
    bound = 1e-6 * (np.abs(x[:, :kp]).astype(np.float64) @ np.abs(y[:kp]) + 1)
    got = cpuref.dsl_matvec_f32(x, y, bk)
    assert np.all(np.abs(got - want) <= bound), np.max(np.abs(got - want) / bound)


def test_dsl_matvec_exact_and_order():
    """Closed forms that pin the program's order of operations
    (fused_reduce.rs:189-293 inside a tile, the carried add across tiles)."""
    big = np.float32(2 ** 24)
    # integer-valued rows: exact
    r = rng(5)
    x = r.integers(-8, 9, size=(6, 48)).astype(np.float32)
    y = r.integers(-8, 9, size=48).astype(np.float32)
    np.testing.assert_array_equal(cpuref.dsl_matvec_f32(x, y, 16), (x @ y).astype(np.float32))
    ones = np.ones(4, np.float32)
    row = np.array([[big, 1, 1, 1]], np.float32)
    # one tile: sequential from element 0 gives 2^24 (each + 1 rounds back);
    # a pairwise tree would give 2^24 + 2, the reverse order 2^24 + 4
    assert cpuref.dsl_matvec_f32(row, ones, 4)[0] == big
    # four tiles of one: the partials 2^24, 1, 1, 1 added to the seed in order
    assert cpuref.dsl_matvec_f32(row, ones, 1)[0] == big
    # the seed comes first: 2^24 + 1 + 1 = 2^24 (partials first would give 2^24 + 2)
    assert cpuref.dsl_matvec_f32(np.ones((1, 2), np.float32), ones[:2], 1, seed=big)[0] == big
    # products rounded on their own: (1 + 2^-12)^2 rounds to 1 + 2^-11, which
    # cancels the first product exactly; a fused multiply-add would leave 2^-24
    a = np.float32(1 + 2 ** -12)
    x2 = np.array([[1.0, a]], np.float32)
    y2 = np.array([-(1 + 2 ** -11), a], np.float32)
    assert cpuref.dsl_matvec_f32(x2, y2, 2)[0] == 0.0
    # K truncated to whole tiles: what lies past them never enters
    x3 = np.array([[1, 2, 3, 4, 5, 6, np.nan, np.inf]], np.float32)
    assert cpuref.dsl_matvec_f32(x3, np.ones(8, np.float32), 3, k=8)[0] == 21.0
    # no whole tile: the seed
    assert cpuref.dsl_matvec_f32(x3, np.ones(8, np.float32), 9, seed=2.5)[0] == 2.5
    # -0.0 products: +0.0 once added to the +0.0 seed, -0.0 from a -0.0 seed
    z = cpuref.dsl_matvec_f32(np.array([[-0.0]], np.float32), np.ones(1, np.float32), 1)
    assert z[0] == 0.0 and not np.signbit(z[0])
    z = cpuref.dsl_matvec_f32(np.array([[-0.0]], np.float32), np.ones(1, np.float32), 1, seed=-0.0)
    assert np.signbit(z[0])

# ---------------------------------------------------------------- number formats

def _e4m3_table():
    vals = []
    for code in range(256):
        s, e, m = code >> 7, (code >> 3) & 15, code & 7
        if e == 15 and m == 7:
            vals.append(np.nan)
            continue
        mag = m * 2.0 ** -9 if e == 0 else (1 + m / 8) * 2.0 ** (e - 7)
        vals.append(-mag if s else mag)
    return np.array(vals)


def test_e4m3_decode_table():
    table = _e4m3_table()
    got = cpuref.e4m3_decode(np.arange(256, dtype=np.uint8))
    finite = ~np.isnan(table)
    np.testing.assert_array_equal(got[finite], table[finite].astype(np.float32))
    assert np.isnan(got[0x7F]) and np.isnan(got[0xFF])
    assert got[0x7E] == 448.0 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6 and got[0x38] == 1.0


def test_e4m3_encode_round_trip_and_rne():
    codes = np.array([c for c in range(256) if c not in (0x7F, 0xFF)], np.uint8)
    vals = cpuref.e4m3_decode(codes)
    back = cpuref.e4m3_encode(vals)
    np.testing.assert_array_equal(back, codes)
    # brute-force nearest-even against the table for random values
    table = _e4m3_table()
    pos = np.array([c for c in range(0, 0x7F)])  # positive finite codes, ascending value
    x = np.abs(rng(40).normal(size=20000) * 60).astype(np.float32)
    x = np.concatenate([x, ((table[pos][1:] + table[pos][:-1]) / 2).astype(np.float32)])  # exact midpoints
    got = cpuref.e4m3_encode(x)
    for xi, gi in zip(x, got):
        if xi >= 448:
            assert gi == 0x7E
            continue
        d = np.abs(table[pos] - xi)
        best = np.flatnonzero(d == d.min())
        want = best[0] if len(best) == 1 else best[np.argmin(pos[best] & 1)]  # tie -> even mantissa
        assert gi == pos[want], (xi, gi, pos[want])
    assert cpuref.e4m3_encode(np.array([1e6, -1e6], np.float32)).tolist() == [0x7E, 0xFE]
    # the division form q = rne_sat(x / s) is used for the per-tensor scale
    assert cpuref.e4m3_encode(np.array([3.0], np.float32), 0.5)[0] == cpuref.e4m3_encode(np.array([6.0], np.float32))[0]


def test_bf16_rne():
    x = rng(41).normal(size=50000).astype(np.float32)
    x = np.concatenate([x, np.array([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -0.0, np.inf], np.float32)])
    got = cpuref.bf16_from_f32(x)
    bits = x.view(np.uint32).astype(np.uint64)
    lo = (bits >> 16).astype(np.uint64)
    with np.errstate(invalid="ignore"):
        cand_lo = (lo << 16).astype(np.uint32).view(np.float32).astype(np.float64)
        cand_hi = ((lo + 1) << 16).astype(np.uint32).view(np.float32).astype(np.float64)
        xd = x.astype(np.float64)
        d_lo, d_hi = np.abs(xd - cand_lo), np.abs(cand_hi - xd)
    want = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, lo + 1, np.where(lo % 2 == 0, lo, lo + 1)))
    finite = np.isfinite(x)
    np.testing.assert_array_equal(got[finite], want[finite].astype(np.uint16))
    assert got[-1] == 0x7F80 and got[-2] == 0x8000
    assert got[-4] == 0x3F80 and got[-3] == 0x3F82  # ties to even


# ---------------------------------------------------------------- seeded tile MMA (a2)

def test_mma_seed_zero_is_the_canonical_matmul():
    a = rng(21).uniform(-1, 1, size=(64, 96)).astype(np.float32)
    b = rng(22).uniform(-1, 1, size=(96, 48)).astype(np.float32)
    c = np.zeros((64, 48), np.float32)
    cpuref.kernel_matmul(a, b, c, (1000, 1, 1), 16, 16, 32)
    np.testing.assert_array_equal(cpuref.mma_f32(a, b, acc_value=0.0, bk=32), c)
    np.testing.assert_array_equal(cpuref.mma_f32(a, np.ascontiguousarray(b.T), b_col_major=True,
                                                 bk=32), c)


def test_mma_integer_seeds_are_exact():
    r = rng(23)
    a = r.integers(-8, 9, size=(40, 30)).astype(np.float32)
    b = r.integers(-8, 9, size=(30, 20)).astype(np.float32)
    d = r.integers(-1000, 1000, size=(40, 20)).astype(np.float32)
    want = d.astype(np.int64) + a.astype(np.int64) @ b.astype(np.int64)
    np.testing.assert_array_equal(cpuref.mma_f32(a, b, acc=d), want.astype(np.float32))
    want = 7 + a.astype(np.int64) @ b.astype(np.int64)
    np.testing.assert_array_equal(cpuref.mma_f32(a, b, acc_value=7.0), want.astype(np.float32))
    # K truncation: only k < (30 // 8) * 8 = 24 contributes
    want = d.astype(np.int64) + a[:, :24].astype(np.int64) @ b[:24].astype(np.int64)
    np.testing.assert_array_equal(cpuref.mma_f32(a, b, acc=d, bk=8), want.astype(np.float32))


def test_mma_seed_starts_the_chain():
    """Seed 2^24 then two products of 1: the chain from the seed gives
    (2^24 + 1) + 1 = 2^24 (each add rounds to even); adding the seed after the
    products would give 2^24 + 2."""
    a = np.ones((1, 2), np.float32)
    b = np.ones((2, 1), np.float32)
    big = np.float32(2.0 ** 24)
    assert cpuref.mma_f32(a, b, acc_value=big)[0, 0] == big
    assert cpuref.mma_f32(a, b, acc=np.full((1, 1), big, np.float32))[0, 0] == big


def test_mma_signed_zero_seeds():
    a = np.zeros((2, 3), np.float32)
    b = np.zeros((3, 2), np.float32)
    z = cpuref.mma_f32(a, b, acc_value=-0.0, bk=4)   # K' = 0: the seed itself
    assert (z == 0).all() and np.signbit(z).all()
    z = cpuref.mma_f32(a, b, acc_value=-0.0)         # -0.0 + (+0.0) = +0.0
    assert (z == 0).all() and not np.signbit(z).any()
