"""The Tile IR pattern router on the CPU (no GPU needed): the printed Tile IR
fixtures, which kernel each DSL kernel routes to for given shapes and grids,
the detector's rejections (the conditions of the reference's
CanonicalMatmulPlan::detect, canonical_matmul.rs:446-666) and parse errors."""
import os

import numpy as np
import pytest

from sile_amd import _abi as hip
from tests import tile_ir_text as T

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "tile_ir")


def _route(text, shapes, grid):
    return hip.tile_ir_route(text, shapes, grid)


def test_fixtures_match_the_derivation():
    from tests.golden.make_tile_ir_fixtures import FIXTURES
    for name, text in FIXTURES.items():
        with open(os.path.join(GOLDEN, name)) as f:
            assert f.read() == text, name


def test_vec_add_text_has_what_the_reference_print_test_asserts():
    # crates/sile/tests/tile_ir_print.rs:77-89 (lowering only) and :166-168 (after the passes)
    printed = T.vec_add(4, passes=False)
    for s in ["module {", "entry @vec_add(", 'kind = "launch.index", dim = 0', "load_ptr_tko",
              "addf", "store_ptr_tko", ", [%5, %3] {shape = [1, 4], stride_dim = 0}", "return",
              "tile<1x4xf32>", "tile<ptr<f32>>"]:
        assert s in printed, s
    for s in ['kind = "sile.program_id"', "sile.get_tile_block_id_dim", "dim = 1"]:
        assert s not in printed, s
    fused = T.vec_add(2)
    assert "map addf(load_ptr_tko(" in fused
    for s in ["= addf ", "= load_ptr_tko %0", "= load_ptr_tko %1"]:
        assert s not in fused, s


def test_matmul_routes_to_the_exact_tile_kernel():
    r = _route(T.matmul(32, 32, 32), [512, 512, 512, 512, 512, 512], 256)
    assert r.kind == hip.ROUTE_MATMUL
    assert (r.tile_m, r.tile_n, r.tile_k) == (32, 32, 32)
    assert list(r.buffer) == [0, 1, 2, -1] and list(r.shape_offset) == [0, 2, 4, -1]
    assert r.seed_from_tile == 0 and r.seed_value == 0.0
    r = _route(T.matmul(2, 2, 2), [4, 4, 4, 4, 4, 4], 4)
    assert r.kind == hip.ROUTE_MATMUL and (r.tile_m, r.tile_n, r.tile_k) == (2, 2, 2)


@pytest.mark.parametrize("passes", [True, False])
def test_softmax_routes(passes):
    # one column tile per row band -> the row softmax over run * BM rows
    r = _route(T.softmax(2, 8, passes), [4, 8, 4, 8], 2)
    assert r.kind == hip.ROUTE_SOFTMAX_ROWS and (r.rows, r.cols) == (4, 8)
    # fewer programs than tiles: only their rows
    r = _route(T.softmax(2, 8, passes), [4, 8, 4, 8], 1)
    assert r.kind == hip.ROUTE_SOFTMAX_ROWS and (r.rows, r.cols) == (2, 8)
    # y wider than the tile but less than two tiles: still one column tile
    r = _route(T.softmax(2, 8, passes), [4, 12, 4, 12], 2)
    assert r.kind == hip.ROUTE_SOFTMAX_ROWS and (r.rows, r.cols) == (4, 8)
    # two column tiles per row band -> the tile kernel
    r = _route(T.softmax(2, 4, passes), [4, 8, 4, 8], 4)
    assert r.kind == hip.ROUTE_SOFTMAX_TILES and (r.tile_m, r.tile_n) == (2, 4)
    # x narrower than a tile row: the tile kernel (which rejects the shapes)
    r = _route(T.softmax(2, 8, passes), [4, 6, 4, 8], 2)
    assert r.kind == hip.ROUTE_SOFTMAX_TILES


def test_row_reduce_routes():
    r = _route(T.row_reduce(4, 64, "sum"), [16, 64, 16, 1], 4)
    assert r.kind == hip.ROUTE_REDUCE_ROWS and r.reduce_op == hip.REDUCE_SUM
    assert (r.rows, r.cols) == (16, 64)
    r = _route(T.row_reduce(4, 64, "max", out_rank=1), [16, 100, 16], 3)
    assert r.kind == hip.ROUTE_REDUCE_ROWS and r.reduce_op == hip.REDUCE_MAX
    assert (r.rows, r.cols) == (12, 64)
    r = _route(T.row_reduce(1, 64), [16, 64, 16, 1], 16)
    assert r.kind == hip.ROUTE_REDUCE_ROWS and (r.rows, r.cols) == (16, 64)
    # more than one output column: every column tile re-reduces the same x columns
    r = _route(T.row_reduce(4, 64), [16, 64, 16, 2], 8)
    assert r.kind == hip.ROUTE_NONE and b"more than one column" in r.reason
    # rank-1 output: 16 programs of 4 rows would write past y[16]
    r = _route(T.row_reduce(4, 64, "max", out_rank=1), [64, 64, 16], 16)
    assert r.kind == hip.ROUTE_NONE and b"past" in r.reason
    # x narrower than the tile
    r = _route(T.row_reduce(4, 64), [16, 32, 16, 1], 4)
    assert r.kind == hip.ROUTE_NONE


def test_parallel_reduce_routes():
    r = _route(T.parallel_reduce(1000), [100000, 1], 100)
    assert r.kind == hip.ROUTE_ATOMIC_REDUCE and r.tile_n == 1000


@pytest.mark.parametrize("passes", [True, False])
def test_vec_add_has_no_route(passes):
    r = _route(T.vec_add(4, passes), [8, 8, 8], 2)
    assert r.kind == hip.ROUTE_NONE
    why = r.reason.decode()
    for d in ("matmul:", "softmax:", "row reduce:", "atomic reduce:", "attention:", "matvec:"):
        assert d in why
    assert list(r.buffer) == [-1, -1, -1, -1]


MATMUL_MUTATIONS = {
    # each breaks one condition of CanonicalMatmulPlan::detect
    "k seed 1": ("%8 = constant <i64: 0>", "%8 = constant <i64: 1>"),
    "step 2": ("%20 = constant <i64: 1>", "%20 = constant <i64: 2>"),
    "bound k <= n": ('cmpi "lt"', 'cmpi "le"'),
    "bound multiply": ("divi %10, %11", "muli %10, %11"),
    "shape dim 0": ("sile.shape_dim %9 {dim = 1}", "sile.shape_dim %9 {dim = 0}"),
    "bk differs from mma k": ("%11 = constant <i64: 32>", "%11 = constant <i64: 16>"),
    "a loaded from b": ("%16 = load_ptr_tko %0,", "%16 = load_ptr_tko %1,"),
    "b walked by n, k": ("load_ptr_tko %1, [%14, %4]", "load_ptr_tko %1, [%4, %14]"),
    "store at swapped launch": ("store_ptr_tko %2, %22, [%3, %4]", "store_ptr_tko %2, %22, [%4, %3]"),
    "store of the seed": ("store_ptr_tko %2, %22,", "store_ptr_tko %2, %5,"),
}


@pytest.mark.parametrize("name", sorted(MATMUL_MUTATIONS))
def test_matmul_detector_rejections(name):
    old, new = MATMUL_MUTATIONS[name]
    text = T.matmul(32, 32, 32)
    assert old in text
    r = _route(text.replace(old, new), [64, 64, 64, 64, 64, 64], 4)
    assert r.kind == hip.ROUTE_NONE, name
    assert b"matmul:" in r.reason


def test_matmul_launch_dims_must_be_row_0_col_1():
    # both tiles from launch indices, but rows from dim 1: the detector of the
    # reference fires; the exact-order kernel decodes (0, 1), so no route
    text = T.matmul(32, 32, 32).replace('"__launch_idx0", kind = "launch.index", dim = 0',
                                        '"__launch_idx0", kind = "launch.index", dim = 2')
    r = _route(text, [64, 64, 64, 64, 64, 64], 4)
    assert r.kind == hip.ROUTE_NONE and b"not (0, 1)" in r.reason


def test_softmax_detector_rejections():
    base = T.softmax(2, 8)
    for old, new in [("exp(subf(", "negf(subf("),
                     ('combiner = "max"', 'combiner = "sum"'),
                     ("map divf(%9,", "map mulf(%9,"),
                     ("store_ptr_tko %1, %13, [%3, %4]", "store_ptr_tko %1, %13, [%4, %3]")]:
        assert old in base
        r = _route(base.replace(old, new), [4, 8, 4, 8], 2)
        assert r.kind == hip.ROUTE_NONE, old


def test_buffer_order_follows_the_parameters():
    # the same softmax with y declared first: operands map to buffer 1 (x) and 0 (y)
    text = T.softmax(2, 8)
    text = text.replace('%0 {sym_name = "x", rank = 2} : tile<ptr<f32>>,\n'
                        '    %1 {sym_name = "y", rank = 2} : tile<ptr<f32>>,',
                        '%1 {sym_name = "y", rank = 2} : tile<ptr<f32>>,\n'
                        '    %0 {sym_name = "x", rank = 2} : tile<ptr<f32>>,')
    r = _route(text, [6, 8, 4, 8], 2)  # y [6, 8], x [4, 8]
    assert r.kind == hip.ROUTE_SOFTMAX_ROWS
    assert list(r.buffer)[:2] == [1, 0] and list(r.shape_offset)[:2] == [2, 0]
    assert (r.rows, r.cols) == (4, 8)
    # three programs would read rows 4 and 5 of x [4, 8]: not the row kernel's domain
    assert _route(text, [6, 8, 4, 8], 3).kind == hip.ROUTE_SOFTMAX_TILES


@pytest.mark.parametrize("text,why", [
    ("", "incomplete"),
    ("module {\n  entry @k(\n  ) {\n    ^bb0:  // entry\n      %1 = frob %0 : none\n"
     "      return\n  }\n}\n", "unknown op"),
    ("module {\n  entry @k(\n  ) {\n    ^bb0:  // entry\n      cf.br ^bb7\n  }\n}\n",
     "unknown block"),
    ("module {\n  entry @k(\n  ) {\n    ^bb0:\n      return\n  }\n}\n", "no entry"),
    ("module {\n  entry @k(\n  ) {\n    ^bb0:  // entry\n      %1 = constant <i64: 0> : tile<i64>\n"
     "  }\n}\n", "terminator"),
])
def test_malformed_text_is_a_compile_error(text, why):
    with pytest.raises(hip.SileError) as e:
        _route(text, [], 1)
    assert e.value.kind == "Compile"
    assert why in str(e.value)


def test_shape_count_must_match_the_buffers():
    with pytest.raises(hip.SileError) as e:
        _route(T.matmul(2, 2, 2), [4, 4, 4, 4, 4], 4)
    assert e.value.kind == "Shape"
    with pytest.raises(hip.SileError) as e:
        _route(T.matmul(2, 2, 2), [4, 4, 4, -4, 4, 4], 4)
    assert e.value.kind == "Shape"


def test_launch_of_no_route_is_unsupported():
    r = _route(T.vec_add(4), [8, 8, 8], 2)
    with pytest.raises(hip.SileError) as e:
        hip.tile_ir_launch(r, [0, 0, 0], [8, 8, 8], 2)
    assert e.value.kind == "UnsupportedBackend"


def test_launch_rejects_other_shapes_or_grid():
    r = _route(T.softmax(2, 8), [4, 8, 4, 8], 2)
    with pytest.raises(hip.SileError) as e:
        hip.tile_ir_launch(r, [0, 0], [8, 8, 8, 8], 2)
    assert e.value.kind == "Shape"
    with pytest.raises(hip.SileError) as e:
        hip.tile_ir_launch(r, [0, 0], [4, 8, 4, 8], 1)
    assert e.value.kind == "Shape"


# ---------------------------------------------------------------- seeded tile MMA forms

@pytest.mark.parametrize("splat", [1.5, -0.0, 3.0])
def test_matmul_with_a_splat_seed_routes(splat):
    """A splat other than 0.0 fails the reference's canonical detector but is
    the same MMA loop with a LoopCarriedSplat seed: routed with its value."""
    r = _route(T.matmul(32, 32, 32, splat=splat), [512, 512, 512, 512, 512, 512], 256)
    assert r.kind == hip.ROUTE_MATMUL, r.reason
    assert r.seed_from_tile == 0 and r.seed_value == splat
    assert np.signbit(np.float32(r.seed_value)) == np.signbit(np.float32(splat))


@pytest.mark.parametrize("src", ["d", "c"])
def test_matmul_with_a_loaded_accumulator_routes(src):
    if src == "d":
        shapes = [64, 96, 96, 48, 64, 48, 64, 48]   # a, b, d, c
        want_buf, want_off = [0, 1, 3, 2], [0, 2, 6, 4]
    else:
        shapes = [64, 96, 96, 48, 64, 48]           # a, b, c (the seed is c itself)
        want_buf, want_off = [0, 1, 2, 2], [0, 2, 4, 4]
    r = _route(T.matmul_acc(16, 16, 32, src=src), shapes, 12)
    assert r.kind == hip.ROUTE_MATMUL, r.reason
    assert r.seed_from_tile == 1
    assert list(r.buffer) == want_buf and list(r.shape_offset) == want_off


def test_mlp_gemm_routes():
    """crates/sile/examples/mlp.rs:6-23 hoists the k-tile count out of the loop."""
    r = _route(T.mlp_gemm(32, 32, 8), [64, 64, 64, 64, 64, 64], 4)
    assert r.kind == hip.ROUTE_MATMUL, r.reason
    assert (r.tile_m, r.tile_n, r.tile_k) == (32, 32, 8) and r.seed_value == 0.0


def test_loaded_accumulator_must_be_the_programs_tile():
    text = T.matmul_acc(16, 16, 32, src="d").replace(
        "%7 = load_ptr_tko %2, [%4, %5]", "%7 = load_ptr_tko %2, [%5, %4]")
    r = _route(text, [64, 96, 96, 48, 64, 48, 64, 48], 12)
    assert r.kind == hip.ROUTE_NONE and b"accumulator tile" in r.reason


ATTN = dict(bm=32, bn=64, d=128, scale=0.08838834764831845)


def _attn_shapes(n_q=256, s_k=512, d=128, ldq=None, ldv=None):
    return [n_q, ldq or d, d, s_k, s_k, ldv or d, n_q, d]


@pytest.mark.parametrize("passes", [True, False])
def test_attention_routes(passes):
    """The DSL's attention loop routes to the fp32 attention kernel with the
    scale and initial max read from the text; programs * BM queries and
    (S / BN) * BN keys."""
    text = T.attention(**ATTN, passes=passes)
    r = _route(text, _attn_shapes(), 8)
    assert r.kind == hip.ROUTE_ATTENTION, r.reason
    assert (r.tile_m, r.tile_n, r.tile_k) == (32, 64, 128)
    assert list(r.buffer) == [0, 1, 2, 3] and list(r.shape_offset) == [0, 2, 4, 6]
    assert r.attn_scale == np.float32(ATTN["scale"]) and r.attn_m0 == np.float32(-1e30)
    assert (r.rows, r.cols) == (256, 512)
    # fewer programs than query tiles; keys truncated to whole BN blocks
    r = _route(text, _attn_shapes(s_k=500), 3)
    assert r.kind == hip.ROUTE_ATTENTION and (r.rows, r.cols) == (96, 448)
    # another initial max and no scale multiply
    t2 = T.attention(16, 32, 64, 1.0, m0=5.0, passes=passes)
    r = _route(t2.replace("mulf(%30, constant(1.0))", "mulf(constant(1.0), %30)"),
               _attn_shapes(n_q=64, s_k=96, d=64), 4)
    assert r.kind == hip.ROUTE_ATTENTION and r.attn_m0 == -5.0 and r.attn_scale == 1.0


def test_attention_route_declines_uncovered_shapes():
    text = T.attention(**ATTN)
    for shapes, why in [([256, 128, 128, 512, 512, 128, 256, 256], b"column tile"),
                        ([100, 128, 128, 512, 512, 128, 256, 128], b"query tiles"),
                        ([256, 128, 128, 512, 400, 128, 256, 128], b"key tiles"),
                        ([256, 128, 64, 512, 512, 128, 256, 128], b"key tiles")]:
        r = _route(text, shapes, 8)
        assert r.kind == hip.ROUTE_NONE and why in r.reason, (shapes, r.reason)


ATTN_MUTATIONS = {
    # each breaks one condition of the attention program
    "max not ge": ('cmpf("ge", %26, %33)', 'cmpf("gt", %26, %33)'),
    "max keeps the row max": ("select(cmpf(\"ge\", %26, %33), %26, %33)",
                              "select(cmpf(\"ge\", %26, %33), %33, %26)"),
    "reduce sum as max": ('combiner = "max", input_shape = [32, 64]} : tile<32x1xf32>\n      %34',
                          'combiner = "sum", input_shape = [32, 64]} : tile<32x1xf32>\n      %34'),
    "p without the shift": ("map exp(subf(%32, broadcast(%34, src_shape=[32, 1])))",
                            "map exp(subf(%32, broadcast(%26, src_shape=[32, 1])))"),
    "alpha reversed": ("map exp(subf(%26, %34))", "map exp(subf(%34, %26))"),
    "l not rescaled": ("map addf(mulf(%24, %39), %41)", "map addf(mulf(%24, %24), %41)"),
    "acc not rescaled": ("map mulf(%25, broadcast(%39,", "map mulf(%25, broadcast(%34,"),
    "v walked by (0, j)": ("load_ptr_tko %2, [%23, %27]", "load_ptr_tko %2, [%27, %23]"),
    "kt walked by (j, 0)": ("load_ptr_tko %1, [%27, %23]", "load_ptr_tko %1, [%23, %27]"),
    "score seed 1": ("%29 = constant <f32: 0.0>", "%29 = constant <f32: 1.0>"),
    "l starts at 1": ("cf.br ^bb1(%6, %8, %12, %10)", "cf.br ^bb1(%6, %10, %12, %8)"),
    "output not divided": ("map divf(%52, broadcast(%51,", "map mulf(%52, broadcast(%51,"),
    "bound from q": ("%19 = sile.shape_dim %18 {dim = 1}", "%19 = sile.shape_dim %5 {dim = 1}"),
    "bound BN differs": ("%20 = constant <i64: 64>", "%20 = constant <i64: 32>"),
    "store at swapped launch": ("[%4, %57] {shape = [32, 128]", "[%57, %4] {shape = [32, 128]"),
}


@pytest.mark.parametrize("name", sorted(ATTN_MUTATIONS))
def test_attention_detector_rejections(name):
    old, new = ATTN_MUTATIONS[name]
    text = T.attention(**ATTN)
    assert old in text, name
    r = _route(text.replace(old, new), _attn_shapes(), 8)
    assert r.kind == hip.ROUTE_NONE, name
    assert b"attention:" in r.reason


# ---------------------------------------------------------------- matvec (mlp.rs)

def _mv_shapes(m=64, k=64, ky=None, mz=None):
    """x [m, k], y [ky], z [mz]."""
    return [m, k, ky if ky is not None else k, mz if mz is not None else m]


@pytest.mark.parametrize("passes", [True, False])
def test_matvec_routes(passes):
    """The mlp example's matvec loop routes to the matvec kernel: rows =
    programs * BM, K = shape(x)[1], BK and the seed from the text."""
    r = _route(T.matvec(32, 8, passes=passes), _mv_shapes(), 2)
    assert r.kind == hip.ROUTE_MATVEC, r.reason
    assert (r.tile_m, r.tile_k, r.rows, r.cols) == (32, 8, 64, 64)
    assert list(r.buffer[:3]) == [0, 1, 2] and list(r.shape_offset[:3]) == [0, 2, 3]
    assert r.seed_value == 0.0
    # fewer programs than row tiles; K not a multiple of BK; another seed
    r = _route(T.matvec(16, 5, passes=passes, seed=1.5), _mv_shapes(m=100, k=23, ky=20, mz=96), 3)
    assert r.kind == hip.ROUTE_MATVEC, r.reason
    assert (r.rows, r.cols, r.tile_k, r.seed_value) == (48, 23, 5, 1.5)
    # the factors in the other order (a program that loads y first)
    t = T.matvec(32, 8, passes=passes)
    if passes:
        t = t.replace("map mulf(load_ptr_tko(%0, [%3, %13], shape=[32, 8], stride_dim=1), "
                      "broadcast(load_ptr_tko(%1, [%17, %13], shape=[1, 8], stride_dim=0), "
                      "src_shape=[1, 8]))",
                      "map mulf(broadcast(load_ptr_tko(%1, [%17, %13], shape=[1, 8], "
                      "stride_dim=0), src_shape=[1, 8]), load_ptr_tko(%0, [%3, %13], "
                      "shape=[32, 8], stride_dim=1))")
    else:
        t = t.replace("%20 = mulf %15, %19", "%20 = mulf %19, %15")
    t = t.replace("addf(%14, %21)", "addf(%21, %14)").replace("addf %14, %21", "addf %21, %14")
    assert _route(t, _mv_shapes(), 2).kind == hip.ROUTE_MATVEC


def test_matvec_route_declines_uncovered_shapes():
    text = T.matvec(32, 8)
    for shapes, grid, why in [(_mv_shapes(m=32, mz=64), 2, b"x does not cover"),
                              (_mv_shapes(mz=48), 2, b"past the rank-1 output"),
                              (_mv_shapes(ky=56), 2, b"y does not cover")]:
        r = _route(text, shapes, grid)
        assert r.kind == hip.ROUTE_NONE and why in r.reason, (shapes, r.reason)
    # y may be longer than K; the grid may exceed z's tiles only within z
    assert _route(text, _mv_shapes(ky=100), 2).kind == hip.ROUTE_MATVEC


MATVEC_MUTATIONS = {
    # each breaks one condition of the matvec program
    "reduce max": ('combiner = "sum"', 'combiner = "max"'),
    "reduce axis 0": ("axis = 1, combiner", "axis = 0, combiner"),
    "acc times partial": ("map addf(%14, %21)", "map mulf(%14, %21)"),
    "acc dropped": ("map addf(%14, %21)", "map addf(%21, %21)"),
    "sum not product": ("%20 = map mulf(", "%20 = map addf("),
    "x walked by (k, pid)": ("load_ptr_tko(%0, [%3, %13]", "load_ptr_tko(%0, [%13, %3]"),
    "y not broadcast": ("broadcast(load_ptr_tko(%1, [%17, %13], shape=[1, 8], stride_dim=0), "
                        "src_shape=[1, 8])",
                        "load_ptr_tko(%1, [%17, %13], shape=[32, 8], stride_dim=0)"),
    "y at row 1": ("%17 = constant <i64: 0>", "%17 = constant <i64: 1>"),
    "bound BK differs": ("%7 = constant <i64: 8>", "%7 = constant <i64: 4>"),
    "bound from y": ("%6 = sile.shape_dim %5 {dim = 1}", "%6 = sile.shape_dim %16 {dim = 1}"),
    "step 2": ("%23 = constant <i64: 1>", "%23 = constant <i64: 2>"),
    "seed not a splat": ("cf.br ^bb1(%11, %4)", "cf.br ^bb1(%11, %11)"),
    "store at [pid, 0]": ("[%27, %3] {shape = [1, 32]", "[%3, %27] {shape = [1, 32]"),
    "stored value not acc": ("store_ptr_tko %2, %25,", "store_ptr_tko %2, %27,"),
    "counter from 1": ("%11 = constant <i64: 0>", "%11 = constant <i64: 1>"),
}


@pytest.mark.parametrize("name", sorted(MATVEC_MUTATIONS))
def test_matvec_detector_rejections(name):
    old, new = MATVEC_MUTATIONS[name]
    text = T.matvec(32, 8)
    assert old in text, name
    r = _route(text.replace(old, new, 1), _mv_shapes(), 2)
    assert r.kind == hip.ROUTE_NONE, name
    assert b"matvec:" in r.reason
