"""Printed Tile IR of the DSL kernels on the hot path, as the reference's
HIR -> Tile IR lowering and its default Tile IR passes produce it.

The reference is Rust and cannot run here, so each text is derived by hand:
the lowering (crates/sile-tile-ir/src/lower.rs) gives every emitted op and
every parameter it creates (`__launch_idx<d>`, `__shape_<buf>`) the next value
id in emission order; the passes are canonicalize_shape, canonicalize_tile_ops,
pointwise_fusion, tile_expr_cse and dce
(crates/sile-tile-ir/src/passes/mod.rs:31-42); the printer is
crates/sile-tile-ir/src/print.rs:5-354.  The vec_add text carries every
substring that crates/sile/tests/tile_ir_print.rs asserts, which pins the
numbering procedure on the one kernel the reference prints in its tests.
`passes=False` gives the text before the passes.

The kernels (DSL source as in crates/sile/examples/*.rs):
  matmul<BM,BN,BK>      crates/sile/examples/matmul.rs:3-19 (splat seeds other
                        than 0.0: `sile::constant(v, [BM, BN])`)
  matmul_acc<BM,BN,BK>  not in the reference: the matmul with its accumulator
                        loaded from a tile (`d.load_tile` or `c.load_tile`)
  gemm<BM,BN,BK>        crates/sile/examples/mlp.rs:6-23
  matvec<BM,BK>         crates/sile/examples/mlp.rs:26-44
  softmax<BM,BN>        crates/sile/examples/softmax.rs:3-16
  parallel_reduce<TILE> crates/sile/examples/parallel_reduce.rs:3-9
  vec_add<TILE>         crates/sile/examples/vec_add.rs:3-14
  attention<BM,BN,D>    not in the reference (it has no attention kernel): the
                        DSL program below, non-causal (the DSL has no iota or
                        select on indices), K given transposed as kt [D, S]
  row_reduce<BM,BN>     not in the reference: `let pid = tile::id().0;
                        let t = x.load_tile([BM, BN], [pid, 0]);
                        y.store(sile::reduce_{sum,max}(t, 1));` with y
                        `[BM, 1]` (rank 2) or `[BM]` (rank 1)
"""
import numpy as np


def _param_buf(v, name, rank):
    return f'%{v} {{sym_name = "{name}", rank = {rank}}} : tile<ptr<f32>>'


def _param_launch(v, dim):
    return f'%{v} {{sym_name = "__launch_idx{dim}", kind = "launch.index", dim = {dim}}} : tile<i64>'


def _param_shape(v, src, name, rank):
    return (f'%{v} {{sym_name = "__shape_{name}", kind = "shape.desc", source = %{src}}} : '
            f'shape_desc<{rank}>')


def _tile(r, c):
    return f"tile<{r}x{c}xf32>"


def _module(name, params, blocks):
    """blocks: [(header, [lines...])]; the first block is the entry."""
    out = ["module {", f"  entry @{name}("]
    for i, p in enumerate(params):
        out.append(f"    {p}{',' if i + 1 < len(params) else ''}")
    out.append("  ) {")
    for i, (header, lines) in enumerate(blocks):
        out.append(f"    {header}:{'  // entry' if i == 0 else ''}")
        out.extend(f"      {ln}" for ln in lines)
    out += ["  }", "}"]
    return "\n".join(out) + "\n"


def _fmt_float(x):
    # print.rs:348-354: integral values print with one decimal
    return f"{x:.1f}" if float(x).is_integer() else repr(float(x))


def matmul(bm, bn, bk, splat=0.0):
    """Canonical matmul: entry -> header(k, acc) -> body -> exit with one store."""
    params = [_param_buf(0, "a", 2), _param_buf(1, "b", 2), _param_buf(2, "c", 2),
              _param_launch(3, 0), _param_launch(4, 1),
              _param_shape(9, 0, "a", 2), _param_shape(17, 1, "b", 2), _param_shape(23, 2, "c", 2)]
    acc = _tile(bm, bn)
    blocks = [
        ("^bb0", [f"%5 = constant <f32: {_fmt_float(splat)}> : {acc}",
                  "%8 = constant <i64: 0> : tile<i64>",
                  "cf.br ^bb1(%8, %5)"]),
        (f"^bb1(%6: tile<i64>, %7: {acc})",
         ["%10 = sile.shape_dim %9 {dim = 1} : tile<i64>",
          f"%11 = constant <i64: {bk}> : tile<i64>",
          "%12 = divi %10, %11 : tile<i64>",
          '%13 = cmpi "lt" %6, %12 : tile<i64>',
          "cf.cond_br %13, ^bb2(%6, %7), ^bb3(%7)"]),
        (f"^bb2(%14: tile<i64>, %15: {acc})",
         [f"%16 = load_ptr_tko %0, [%3, %14] {{shape = [{bm}, {bk}], stride_dim = 1}} : "
          f"{_tile(bm, bk)}",
          f"%18 = load_ptr_tko %1, [%14, %4] {{shape = [{bk}, {bn}], stride_dim = 1}} : "
          f"{_tile(bk, bn)}",
          f"%19 = mmaf %16, %18, %15 {{m = {bm}, n = {bn}, k = {bk}}} : {acc}",
          "%20 = constant <i64: 1> : tile<i64>",
          "%21 = addi %14, %20 : tile<i64>",
          "cf.br ^bb1(%21, %19)"]),
        (f"^bb3(%22: {acc})",
         [f"%24 = store_ptr_tko %2, %22, [%3, %4] {{shape = [{bm}, {bn}], stride_dim = 1}} : none",
          "return"]),
    ]
    return _module("matmul", params, blocks)


def matmul_acc(bm, bn, bk, src="d"):
    """C = D + A.B as a tile MMA whose accumulator starts from a loaded tile:
    `let mut acc = d.load_tile([BM, BN], [m, n]); for k in 0..a.shape()[1] / BK
    { acc = sile::mma(a.load_tile(..), b.load_tile(..), acc) } c.store(acc)`,
    with d a fourth parameter (src="d") or c itself (src="c", C += A.B in
    place).  The accumulator seed is a tile, so the reference lowers the mma
    through its general tile-MMA path (mma.rs:25-739, init :213-229)."""
    acc = _tile(bm, bn)
    if src == "c":
        params = [_param_buf(0, "a", 2), _param_buf(1, "b", 2), _param_buf(2, "c", 2),
                  _param_launch(3, 0), _param_launch(4, 1), _param_shape(5, 2, "c", 2),
                  _param_shape(10, 0, "a", 2), _param_shape(18, 1, "b", 2)]
        seed_buf = "%2"
    else:
        params = [_param_buf(0, "a", 2), _param_buf(1, "b", 2), _param_buf(2, "d", 2),
                  _param_buf(3, "c", 2), _param_launch(4, 0), _param_launch(5, 1),
                  _param_shape(6, 2, "d", 2), _param_shape(10, 0, "a", 2),
                  _param_shape(18, 1, "b", 2), _param_shape(24, 3, "c", 2)]
        seed_buf = "%2"
    m_idx, n_idx = ("%3", "%4") if src == "c" else ("%4", "%5")
    out = "%2" if src == "c" else "%3"
    blocks = [
        ("^bb0", [f"%7 = load_ptr_tko {seed_buf}, [{m_idx}, {n_idx}] {{shape = [{bm}, {bn}], "
                  f"stride_dim = 1}} : {acc}",
                  "%9 = constant <i64: 0> : tile<i64>",
                  "cf.br ^bb1(%9, %7)"]),
        (f"^bb1(%11: tile<i64>, %12: {acc})",
         ["%13 = sile.shape_dim %10 {dim = 1} : tile<i64>",
          f"%14 = constant <i64: {bk}> : tile<i64>",
          "%15 = divi %13, %14 : tile<i64>",
          '%16 = cmpi "lt" %11, %15 : tile<i64>',
          "cf.cond_br %16, ^bb2(%11, %12), ^bb3(%12)"]),
        (f"^bb2(%19: tile<i64>, %20: {acc})",
         [f"%17 = load_ptr_tko %0, [{m_idx}, %19] {{shape = [{bm}, {bk}], stride_dim = 1}} : "
          f"{_tile(bm, bk)}",
          f"%21 = load_ptr_tko %1, [%19, {n_idx}] {{shape = [{bk}, {bn}], stride_dim = 1}} : "
          f"{_tile(bk, bn)}",
          f"%22 = mmaf %17, %21, %20 {{m = {bm}, n = {bn}, k = {bk}}} : {acc}",
          "%23 = constant <i64: 1> : tile<i64>",
          "%25 = addi %19, %23 : tile<i64>",
          "cf.br ^bb1(%25, %22)"]),
        (f"^bb3(%26: {acc})",
         [f"%27 = store_ptr_tko {out}, %26, [{m_idx}, {n_idx}] {{shape = [{bm}, {bn}], "
          f"stride_dim = 1}} : none",
          "return"]),
    ]
    return _module("matmul_acc", params, blocks)


def mlp_gemm(bm, bn, bk):
    """The gemm kernel of crates/sile/examples/mlp.rs:6-23: the canonical
    matmul except that `let k_tiles = x.shape()[1] / BK;` is computed once
    before the loop, so the bound's division sits in the entry block and the
    reference's CanonicalMatmulPlan::detect (canonical_matmul.rs:511-534,
    which looks for it in the loop header) declines it; the general tile-MMA
    lowering (LoopCarriedSplat seed 0.0) gives the same per-cell chain.  The
    loop's block parameters take their value ids before the start constant
    (lower.rs:266-283)."""
    acc = _tile(bm, bn)
    params = [_param_buf(0, "x", 2), _param_buf(1, "y", 2), _param_buf(2, "z", 2),
              _param_launch(3, 0), _param_launch(4, 1), _param_shape(6, 0, "x", 2),
              _param_shape(17, 1, "y", 2), _param_shape(23, 2, "z", 2)]
    blocks = [
        ("^bb0", [f"%5 = constant <f32: 0.0> : {acc}",
                  "%7 = sile.shape_dim %6 {dim = 1} : tile<i64>",
                  f"%8 = constant <i64: {bk}> : tile<i64>",
                  "%9 = divi %7, %8 : tile<i64>",
                  "%12 = constant <i64: 0> : tile<i64>",
                  "cf.br ^bb1(%12, %5)"]),
        (f"^bb1(%10: tile<i64>, %11: {acc})",
         ['%13 = cmpi "lt" %10, %9 : tile<i64>',
          "cf.cond_br %13, ^bb2(%10, %11), ^bb3(%11)"]),
        (f"^bb2(%14: tile<i64>, %15: {acc})",
         [f"%16 = load_ptr_tko %0, [%3, %14] {{shape = [{bm}, {bk}], stride_dim = 1}} : "
          f"{_tile(bm, bk)}",
          f"%18 = load_ptr_tko %1, [%14, %4] {{shape = [{bk}, {bn}], stride_dim = 1}} : "
          f"{_tile(bk, bn)}",
          f"%19 = mmaf %16, %18, %15 {{m = {bm}, n = {bn}, k = {bk}}} : {acc}",
          "%20 = constant <i64: 1> : tile<i64>",
          "%21 = addi %14, %20 : tile<i64>",
          "cf.br ^bb1(%21, %19)"]),
        (f"^bb3(%22: {acc})",
         [f"%24 = store_ptr_tko %2, %22, [%3, %4] {{shape = [{bm}, {bn}], stride_dim = 1}} : none",
          "return"]),
    ]
    return _module("gemm", params, blocks)


def matvec(bm, bk, passes=True, seed=0.0):
    """The matvec kernel of crates/sile/examples/mlp.rs:26-44:

        let m_idx = tile::id().0;
        let mut acc = sile::constant(SEED, [BM]);
        let k_tiles = x.shape()[1] / BK;
        for k_idx in 0..k_tiles {
            let tile_x = x.load_tile([BM, BK], [m_idx, k_idx]);
            let tile_y = y.load_tile([BK], [k_idx]).broadcast(&[BM, BK]);
            let partial = sile::reduce_sum(tile_x * tile_y, 1);
            acc = acc + partial;
        }
        z.store(acc);

    x rank 2, y and z rank 1.  The [BM] constant is a [1, BM] tile and the
    rank-1 loads are [1, BK] at [0, k] (lower.rs:514-546, 946-967); the loop
    carries acc (find_loop_carried_vars keeps the names defined before the
    loop, lower.rs:253-260, 448-465); y's shape descriptor is created at its
    load in the body, z's at the store, which writes [1, BM] at [0, pid]
    (lower.rs:777-821).  After the passes the product, the broadcast and both
    single-use loads fold into one map (pointwise_fusion.rs:5-235; the loads
    left standing and the broadcast map are dead, dce), and the carried add
    becomes a map of two values."""
    acc = _tile(1, bm)
    params = [_param_buf(0, "x", 2), _param_buf(1, "y", 1), _param_buf(2, "z", 1),
              _param_launch(3, 0), _param_shape(5, 0, "x", 2), _param_shape(16, 1, "y", 1),
              _param_shape(26, 2, "z", 1)]
    entry = [f"%4 = constant <f32: {_fmt_float(seed)}> : {acc}",
             "%6 = sile.shape_dim %5 {dim = 1} : tile<i64>",
             f"%7 = constant <i64: {bk}> : tile<i64>",
             "%8 = divi %6, %7 : tile<i64>",
             "%11 = constant <i64: 0> : tile<i64>",
             "cf.br ^bb1(%11, %4)"]
    header = (f"^bb1(%9: tile<i64>, %10: {acc})",
              ['%12 = cmpi "lt" %9, %8 : tile<i64>',
               "cf.cond_br %12, ^bb2(%9, %10), ^bb3(%10)"])
    reduce = (f'%21 = reduce %20 {{axis = 1, combiner = "sum", input_shape = [{bm}, {bk}]}} : '
              f"{_tile(bm, 1)}")
    tail = ["%23 = constant <i64: 1> : tile<i64>", "%24 = addi %13, %23 : tile<i64>",
            "cf.br ^bb1(%24, %22)"]
    if passes:
        body = ["%17 = constant <i64: 0> : tile<i64>",
                f"%20 = map mulf(load_ptr_tko(%0, [%3, %13], shape=[{bm}, {bk}], stride_dim=1), "
                f"broadcast(load_ptr_tko(%1, [%17, %13], shape=[1, {bk}], stride_dim=0), "
                f"src_shape=[1, {bk}])) {{shape = [{bm}, {bk}]}} : {_tile(bm, bk)}",
                reduce,
                f"%22 = map addf(%14, %21) {{shape = [1, {bm}]}} : {acc}"] + tail
    else:
        body = [f"%15 = load_ptr_tko %0, [%3, %13] {{shape = [{bm}, {bk}], stride_dim = 1}} : "
                f"{_tile(bm, bk)}",
                "%17 = constant <i64: 0> : tile<i64>",
                f"%18 = load_ptr_tko %1, [%17, %13] {{shape = [1, {bk}], stride_dim = 0}} : "
                f"{_tile(1, bk)}",
                f"%19 = broadcast %18 {{shape = [{bm}, {bk}]}} : {_tile(bm, bk)}",
                f"%20 = mulf %15, %19 : {_tile(bm, bk)}",
                reduce,
                f"%22 = addf %14, %21 : {acc}"] + tail
    exit_ = ["%27 = constant <i64: 0> : tile<i64>",
             f"%28 = store_ptr_tko %2, %25, [%27, %3] {{shape = [1, {bm}], stride_dim = 0}} : none",
             "return"]
    return _module("matvec", params, [("^bb0", entry), header,
                                      (f"^bb2(%13: tile<i64>, %14: {acc})", body),
                                      (f"^bb3(%25: {acc})", exit_)])


def softmax(bm, bn, passes=True):
    params = [_param_buf(0, "x", 2), _param_buf(1, "y", 2), _param_shape(2, 0, "x", 2),
              _param_launch(3, 0), _param_launch(4, 1), _param_shape(12, 1, "y", 2)]
    t, col = _tile(bm, bn), _tile(bm, 1)
    load = f"%5 = load_ptr_tko %0, [%3, %4] {{shape = [{bm}, {bn}], stride_dim = 1}} : {t}"
    rmax = f'%6 = reduce %5 {{axis = 1, combiner = "max", input_shape = [{bm}, {bn}]}} : {col}'
    rsum = f'%10 = reduce %9 {{axis = 1, combiner = "sum", input_shape = [{bm}, {bn}]}} : {col}'
    store = f"%14 = store_ptr_tko %1, %13, [%3, %4] {{shape = [{bm}, {bn}], stride_dim = 1}} : none"
    if passes:
        lines = [load, rmax,
                 f"%9 = map exp(subf(%5, broadcast(%6, src_shape=[{bm}, 1]))) "
                 f"{{shape = [{bm}, {bn}]}} : {t}",
                 rsum,
                 f"%13 = map divf(%9, broadcast(%10, src_shape=[{bm}, 1])) "
                 f"{{shape = [{bm}, {bn}]}} : {t}",
                 store, "return"]
    else:
        lines = [load, rmax,
                 f"%7 = broadcast %6 {{shape = [{bm}, {bn}]}} : {t}",
                 f"%8 = subf %5, %7 : {t}",
                 f"%9 = exp %8 : {t}",
                 rsum,
                 f"%11 = broadcast %10 {{shape = [{bm}, {bn}]}} : {t}",
                 f"%13 = divf %9, %11 : {t}",
                 store, "return"]
    return _module("softmax", params, [("^bb0", lines)])


def row_reduce(bm, bn, op="sum", out_rank=2):
    """row_reduce<BM,BN> (see the module docstring); op 'sum' or 'max'."""
    params = [_param_buf(0, "x", 2), _param_buf(1, "y", out_rank), _param_launch(2, 0),
              _param_shape(3, 0, "x", 2), _param_shape(6, 1, "y", out_rank)]
    lines = ["%4 = constant <i64: 0> : tile<i64>",
             f"%5 = load_ptr_tko %0, [%2, %4] {{shape = [{bm}, {bn}], stride_dim = 1}} : "
             f"{_tile(bm, bn)}",
             f'%7 = reduce %5 {{axis = 1, combiner = "{op}", input_shape = [{bm}, {bn}]}} : '
             f"{_tile(bm, 1)}"]
    if out_rank == 2:
        # the store's column is launch index 1 for a tile larger than 1x1
        # (lower.rs:790-800), a constant 0 otherwise
        if bm > 1:
            params.append(_param_launch(8, 1))
        else:
            lines.append("%8 = constant <i64: 0> : tile<i64>")
        lines.append(f"%9 = store_ptr_tko %1, %7, [%2, %8] {{shape = [{bm}, 1], stride_dim = 1}} "
                     ": none")
        if bm == 1:
            # CSE folds the second constant 0 into %4
            lines.pop(-2)
            lines[-1] = lines[-1].replace("[%2, %8]", "[%2, %4]")
    else:
        lines.append(f"%9 = store_ptr_tko %1, %7, [%4, %2] {{shape = [{bm}, 1], stride_dim = 0}} "
                     ": none")
    lines.append("return")
    return _module(f"row_{op}", params, [("^bb0", lines)])


def parallel_reduce(tile):
    params = [_param_buf(0, "a", 1), _param_buf(1, "out", 1), _param_launch(2, 0),
              _param_shape(3, 0, "a", 1), _param_shape(7, 1, "out", 1)]
    lines = ["%4 = constant <i64: 0> : tile<i64>",
             f"%5 = load_ptr_tko %0, [%4, %2] {{shape = [1, {tile}], stride_dim = 0}} : "
             f"{_tile(1, tile)}",
             f'%6 = reduce %5 {{axis = 1, combiner = "sum", input_shape = [1, {tile}]}} : '
             f"{_tile(1, 1)}",
             "%10 = extract %6[%4, %4] : tile<f32>",
             "%13 = sile.atomic_add %1, %10, [%4, %4] {stride_dim = 0} : none",
             "return"]
    return _module("parallel_reduce", params, [("^bb0", lines)])


def vec_add(tile, passes=True):
    params = [_param_buf(0, "a", 1), _param_buf(1, "b", 1), _param_buf(2, "c", 1),
              _param_launch(3, 0), _param_shape(4, 0, "a", 1), _param_shape(7, 1, "b", 1),
              _param_shape(10, 2, "c", 1)]
    t = _tile(1, tile)
    if passes:
        lines = ["%5 = constant <i64: 0> : tile<i64>",
                 f"%11 = map addf(load_ptr_tko(%0, [%5, %3], shape=[1, {tile}], stride_dim=0), "
                 f"load_ptr_tko(%1, [%5, %3], shape=[1, {tile}], stride_dim=0)) "
                 f"{{shape = [1, {tile}]}} : {t}",
                 f"%13 = store_ptr_tko %2, %11, [%5, %3] {{shape = [1, {tile}], stride_dim = 0}} "
                 ": none",
                 "return"]
    else:
        lines = ["%5 = constant <i64: 0> : tile<i64>",
                 f"%6 = load_ptr_tko %0, [%5, %3] {{shape = [1, {tile}], stride_dim = 0}} : {t}",
                 "%8 = constant <i64: 0> : tile<i64>",
                 f"%9 = load_ptr_tko %1, [%8, %3] {{shape = [1, {tile}], stride_dim = 0}} : {t}",
                 f"%11 = addf %6, %9 : {t}",
                 "%12 = constant <i64: 0> : tile<i64>",
                 f"%13 = store_ptr_tko %2, %11, [%12, %3] {{shape = [1, {tile}], stride_dim = 0}} "
                 ": none",
                 "return"]
    return _module("vec_add", params, [("^bb0", lines)])


def attention(bm, bn, d, scale, m0=1.0e30, passes=True):
    """attention<BM, BN, D> in the DSL (a negative literal does not parse in
    the DSL, crates/sile-macros/src/frontend/parse.rs:407-470, so the initial
    max is the tile difference constant(0.0) - constant(m0)):

        let pid = tile::id().0;
        let qt = q.load_tile([BM, D], [pid, 0]);
        let mut m = sile::constant(0.0, [BM, 1]) - sile::constant(M0, [BM, 1]);
        let mut l = sile::constant(0.0, [BM, 1]);
        let mut acc = sile::constant(0.0, [BM, D]);
        for j in 0..kt.shape()[1] / BN {
            let s = sile::mma(qt, kt.load_tile([D, BN], [0, j]), sile::constant(0.0, [BM, BN]))
                * sile::constant(SCALE, [BM, BN]);
            let m_new = sile::max_tile(m, sile::reduce_max(s, 1));
            let p = sile::exp(s - m_new.broadcast([BM, BN]));
            let alpha = sile::exp(m - m_new);
            l = l * alpha + sile::reduce_sum(p, 1);
            acc = sile::mma(p, v.load_tile([BN, D], [j, 0]), acc * alpha.broadcast([BM, D]));
            m = m_new;
        }
        o.store(acc / l.broadcast([BM, D]));

    The loop carries l, acc, m in the order the body first assigns them
    (find_loop_carried_vars, crates/sile-tile-ir/src/lower.rs:446-465);
    max_tile is a select map at lowering (lower.rs:619-641).  After the
    passes: single-use splats and pointwise chains fold into maps (the scale
    into s's map, both constants into m's initial map), CSE merges the second
    i64 0 of each block and the entry's second [BM, 1] zero splat into the
    first, DCE drops the folded values."""
    f32 = np.float32
    m0s, sc = _fmt_float(float(f32(m0))), _fmt_float(float(f32(scale)))
    col, acc_t, s_t = _tile(bm, 1), _tile(bm, d), _tile(bm, bn)
    params = [_param_buf(0, "q", 2), _param_buf(1, "kt", 2), _param_buf(2, "v", 2),
              _param_buf(3, "o", 2), _param_launch(4, 0), _param_shape(5, 0, "q", 2),
              _param_shape(18, 1, "kt", 2), _param_shape(43, 2, "v", 2),
              _param_shape(54, 3, "o", 2), _param_launch(57, 1)]
    load_q = (f"%7 = load_ptr_tko %0, [%4, %6] {{shape = [{bm}, {d}], stride_dim = 1}} : "
              f"{acc_t}")
    header = (f"^bb1(%13: tile<i64>, %14: {col}, %15: {acc_t}, %16: {col})",
              ["%19 = sile.shape_dim %18 {dim = 1} : tile<i64>",
               f"%20 = constant <i64: {bn}> : tile<i64>",
               "%21 = divi %19, %20 : tile<i64>",
               '%22 = cmpi "lt" %13, %21 : tile<i64>',
               "cf.cond_br %22, ^bb2(%13, %14, %15, %16), ^bb3(%14, %15, %16)"])
    body_hdr = f"^bb2(%23: tile<i64>, %24: {col}, %25: {acc_t}, %26: {col})"
    exit_hdr = f"^bb3(%51: {col}, %52: {acc_t}, %53: {col})"
    load_kt = (f"%28 = load_ptr_tko %1, [%27, %23] {{shape = [{d}, {bn}], stride_dim = 1}} : "
               f"{_tile(d, bn)}")
    mma_s = f"%30 = mmaf %7, %28, %29 {{m = {bm}, n = {bn}, k = {d}}} : {s_t}"
    rmax = (f'%33 = reduce %32 {{axis = 1, combiner = "max", input_shape = [{bm}, {bn}]}} : '
            f"{col}")
    m_new = (f'%34 = map select(cmpf("ge", %26, %33), %26, %33) {{shape = [{bm}, 1]}} : '
             f"{col}")
    rsum = (f'%41 = reduce %37 {{axis = 1, combiner = "sum", input_shape = [{bm}, {bn}]}} : '
            f"{col}")
    mma_pv = f"%48 = mmaf %37, %45, %47 {{m = {bm}, n = {d}, k = {bn}}} : {acc_t}"
    store = (f"%58 = store_ptr_tko %3, %56, [%4, %57] {{shape = [{bm}, {d}], stride_dim = 1}} "
             ": none")
    if passes:
        entry = ["%6 = constant <i64: 0> : tile<i64>", load_q,
                 f"%8 = constant <f32: 0.0> : {col}",
                 f"%10 = map subf(constant(0.0), constant({m0s})) {{shape = [{bm}, 1]}} : {col}",
                 f"%12 = constant <f32: 0.0> : {acc_t}",
                 "cf.br ^bb1(%6, %8, %12, %10)"]
        body = ["%27 = constant <i64: 0> : tile<i64>", load_kt,
                f"%29 = constant <f32: 0.0> : {s_t}", mma_s,
                f"%32 = map mulf(%30, constant({sc})) {{shape = [{bm}, {bn}]}} : {s_t}",
                rmax, m_new,
                f"%37 = map exp(subf(%32, broadcast(%34, src_shape=[{bm}, 1]))) "
                f"{{shape = [{bm}, {bn}]}} : {s_t}",
                f"%39 = map exp(subf(%26, %34)) {{shape = [{bm}, 1]}} : {col}",
                rsum,
                f"%42 = map addf(mulf(%24, %39), %41) {{shape = [{bm}, 1]}} : {col}",
                f"%45 = load_ptr_tko %2, [%23, %27] {{shape = [{bn}, {d}], stride_dim = 1}} : "
                f"{_tile(bn, d)}",
                f"%47 = map mulf(%25, broadcast(%39, src_shape=[{bm}, 1])) "
                f"{{shape = [{bm}, {d}]}} : {acc_t}",
                mma_pv,
                "%49 = constant <i64: 1> : tile<i64>",
                "%50 = addi %23, %49 : tile<i64>",
                "cf.br ^bb1(%50, %42, %48, %34)"]
        exit_ = [f"%56 = map divf(%52, broadcast(%51, src_shape=[{bm}, 1])) "
                 f"{{shape = [{bm}, {d}]}} : {acc_t}", store, "return"]
    else:
        entry = ["%6 = constant <i64: 0> : tile<i64>", load_q,
                 f"%8 = constant <f32: 0.0> : {col}",
                 f"%9 = constant <f32: {m0s}> : {col}",
                 f"%10 = subf %8, %9 : {col}",
                 f"%11 = constant <f32: 0.0> : {col}",
                 f"%12 = constant <f32: 0.0> : {acc_t}",
                 "%17 = constant <i64: 0> : tile<i64>",
                 "cf.br ^bb1(%17, %11, %12, %10)"]
        body = ["%27 = constant <i64: 0> : tile<i64>", load_kt,
                f"%29 = constant <f32: 0.0> : {s_t}", mma_s,
                f"%31 = constant <f32: {sc}> : {s_t}",
                f"%32 = mulf %30, %31 : {s_t}",
                rmax, m_new,
                f"%35 = broadcast %34 {{shape = [{bm}, {bn}]}} : {s_t}",
                f"%36 = subf %32, %35 : {s_t}",
                f"%37 = exp %36 : {s_t}",
                f"%38 = subf %26, %34 : {col}",
                f"%39 = exp %38 : {col}",
                f"%40 = mulf %24, %39 : {col}",
                rsum,
                f"%42 = addf %40, %41 : {col}",
                "%44 = constant <i64: 0> : tile<i64>",
                f"%45 = load_ptr_tko %2, [%23, %44] {{shape = [{bn}, {d}], stride_dim = 1}} : "
                f"{_tile(bn, d)}",
                f"%46 = broadcast %39 {{shape = [{bm}, {d}]}} : {acc_t}",
                f"%47 = mulf %25, %46 : {acc_t}",
                mma_pv,
                "%49 = constant <i64: 1> : tile<i64>",
                "%50 = addi %23, %49 : tile<i64>",
                "cf.br ^bb1(%50, %42, %48, %34)"]
        exit_ = [f"%55 = broadcast %51 {{shape = [{bm}, {d}]}} : {acc_t}",
                 f"%56 = divf %52, %55 : {acc_t}", store, "return"]
    return _module("attention", params, [("^bb0", entry), header, (body_hdr, body),
                                         (exit_hdr, exit_)])
