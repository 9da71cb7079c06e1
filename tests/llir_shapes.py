"""LLIR in the loop shapes of the reference's Tile IR -> LLIR lowering, in its
printed form (crates/sile-llvm-ir/src/print.rs), for tests of the generated
code on those shapes.

The shapes follow the reference's emitters, not this repository's
hand-written fixtures:
- a tile is a private alloca `[rows x [cols x f32]]`, addressed by
  `getelementptr <tile type>, ptr addrspace(5) %t, i64 row, i64 col`
  (core/emit/alloc.rs:8-32, insts/memory.rs:6-21);
- a tile loop over rows x cols is `lower_nested_tile_loop`
  (core/emit/tile_loops.rs:16-40): one column loop for rows == 1, one row loop
  for cols == 1, else the 2-D nest of tile_loops/grid.rs:7-130 (row header,
  column header carrying the row, body, row latch); every header passes its
  values on to a body block with parameters of its own;
- a reduction along the columns of more than 16 elements is a row loop whose
  body reads the row's first element, then a reduce loop from index 1 with
  the accumulator as a block parameter and an exit block receiving the final
  value (tile_compute/reduce.rs:279-374, tile_loops/single_axis.rs:85-153);
  the max combines with `fcmp ogt next, acc; select` (reduce.rs:10-30);
- buffer elements are addressed `tile_origin + row * stride + col` from the
  shape table (tile_memory.rs:150-318);
- value names are a prefix and a counter, block names a prefix and a block
  counter (core/block.rs:36-48, 101-122).

Which fusions the reference's passes apply before lowering is not modelled:
each tile op here is its own loop nest over its own tile.  The functions are
test inputs (no reference output is reproduced byte for byte)."""


class _Fn:
    def __init__(self, name, params):
        """params: (name, rank, shape_offset) of f32 buffers, in order."""
        self.name = name
        self.params = params
        self.nv = 0
        self.nb = 0
        self.blocks = []          # [name, params, lines, term]
        self.cur = self.new_block("entry", [])

    def val(self, prefix="v"):
        self.nv += 1
        return f"%{prefix}{self.nv}"

    def new_block(self, prefix, params):
        name = f"{prefix}_{self.nb}"
        self.nb += 1
        ps = [(self.val(p), t) for p, t in params]
        blk = [name, ps, [], None]
        self.blocks.append(blk)
        return blk

    def emit(self, text, prefix="v"):
        r = self.val(prefix)
        self.cur[2].append(f"{r} = {text}")
        return r

    def stmt(self, text):
        self.cur[2].append(text)

    def term(self, text):
        self.cur[3] = text

    def switch(self, blk):
        self.cur = blk

    def text(self):
        out = ["define void @%s(%s) {" % (self.name, ", ".join(
            [f"ptr addrspace(1) %{n}" for n, _, _ in self.params] +
            ["ptr addrspace(4) %__sile_shapes"]))]
        for n, rank, off in self.params:
            out.append(f"  ; sile.param %{n} [rank={rank}, shape_offset={off}, elem=f32]")
        out.append("  ; sile.param %__sile_shapes [elem=i64]")
        for name, ps, lines, term in self.blocks:
            out.append(f"{name}:")
            if ps:
                out.append("  ; args(%s)" % ", ".join(f"{p}: {t}" for p, t in ps))
            out += ["  " + x for x in lines]
            out.append("  " + term)
        out.append("}")
        return "\n".join(out) + "\n"


def _tile_loop(f, prefix, rows, cols, body):
    """lower_nested_tile_loop: body(row, col) appends the body's instructions."""
    if rows == 1 or cols == 1:
        axis = "col" if rows == 1 else "row"
        n = cols if rows == 1 else rows
        header = f.new_block(f"{prefix}_{axis}_header", [(f"loop_{axis}", "i64")])
        blk = f.new_block(f"{prefix}_body", [(f"loop_{axis}", "i64")])
        cont = f.new_block(f"{prefix}_continue", [])
        f.term(f"br label %{header[0]} ; args(0)")
        f.switch(header)
        i = header[1][0][0]
        c = f.emit(f"icmp slt {i}, {n}")
        f.term(f"br i1 {c}, label %{blk[0]}, label %{cont[0]} ; true_args({i})")
        f.switch(blk)
        bi = blk[1][0][0]
        body(0, bi) if rows == 1 else body(bi, 0)
        nx = f.emit(f"add {bi}, 1")
        f.term(f"br label %{header[0]} ; args({nx})")
        f.switch(cont)
        return
    rh = f.new_block(f"{prefix}_row_header", [("loop_row", "i64")])
    ch = f.new_block(f"{prefix}_col_header", [("loop_row", "i64"), ("loop_col", "i64")])
    blk = f.new_block(f"{prefix}_body", [("loop_row", "i64"), ("loop_col", "i64")])
    latch = f.new_block(f"{prefix}_row_latch", [("loop_row", "i64")])
    cont = f.new_block(f"{prefix}_continue", [])
    f.term(f"br label %{rh[0]} ; args(0)")
    f.switch(rh)
    r = rh[1][0][0]
    c = f.emit(f"icmp slt {r}, {rows}")
    f.term(f"br i1 {c}, label %{ch[0]}, label %{cont[0]} ; true_args({r}, 0)")
    f.switch(ch)
    cr, cc = ch[1][0][0], ch[1][1][0]
    c = f.emit(f"icmp slt {cc}, {cols}")
    f.term(f"br i1 {c}, label %{blk[0]}, label %{latch[0]} ; true_args({cr}, {cc}) ; false_args({cr})")
    f.switch(blk)
    br, bc = blk[1][0][0], blk[1][1][0]
    body(br, bc)
    nx = f.emit(f"add {bc}, 1")
    f.term(f"br label %{ch[0]} ; args({br}, {nx})")
    f.switch(latch)
    nr = f.emit(f"add {latch[1][0][0]}, 1")
    f.term(f"br label %{rh[0]} ; args({nr})")
    f.switch(cont)


def _tile_gep(f, tile, rows, cols, r, c):
    return f.emit(f"getelementptr [{rows} x [{cols} x f32]], ptr addrspace(5) {tile}, i64 {r}, i64 {c}")


def _tile_load(f, tile, rows, cols, r, c):
    p = _tile_gep(f, tile, rows, cols, r, c)
    return f.emit(f"load f32, ptr addrspace(5) {p}")


def _tile_store(f, tile, rows, cols, r, c, v):
    p = _tile_gep(f, tile, rows, cols, r, c)
    f.stmt(f"store f32 {v}, ptr addrspace(5) {p}")


def _reduce_rows(f, prefix, src, rows, cols, dst, is_max):
    """A reduction along axis 1 of a [rows x cols] tile into dst [rows x 1],
    cols > 16: reduce.rs lower_single_row_reduce_loop + lower_reduce_extent_loop
    (rows == 1 takes the single-column form with one column)."""
    axis = "col" if rows == 1 else "row"
    header = f.new_block(f"{prefix}_{axis}_header", [(f"loop_{axis}", "i64")])
    blk = f.new_block(f"{prefix}_{axis}_body", [(f"loop_{axis}", "i64")])
    cont = f.new_block(f"{prefix}_continue", [])
    f.term(f"br label %{header[0]} ; args(0)")
    f.switch(header)
    i = header[1][0][0]
    c = f.emit(f"icmp slt {i}, {1 if rows == 1 else rows}")
    f.term(f"br i1 {c}, label %{blk[0]}, label %{cont[0]} ; true_args({i})")
    f.switch(blk)
    row = 0 if rows == 1 else blk[1][0][0]
    col = blk[1][0][0] if rows == 1 else 0
    init = _tile_load(f, src, rows, cols, row, 0)
    rh = f.new_block(f"{prefix}_reduce_header", [("reduce_idx", "i64"), ("reduce_acc", "f32")])
    rb = f.new_block(f"{prefix}_reduce_body", [("reduce_idx", "i64"), ("reduce_acc", "f32")])
    rx = f.new_block(f"{prefix}_reduce_exit", [("final_acc", "f32")])
    f.term(f"br label %{rh[0]} ; args(1, {init})")
    f.switch(rh)
    hi, ha = rh[1][0][0], rh[1][1][0]
    c = f.emit(f"icmp slt {hi}, {cols}")
    f.term(f"br i1 {c}, label %{rb[0]}, label %{rx[0]} ; true_args({hi}, {ha}) ; false_args({ha})")
    f.switch(rb)
    bi, ba = rb[1][0][0], rb[1][1][0]
    nxt = _tile_load(f, src, rows, cols, row, bi)
    if is_max:
        gt = f.emit(f"fcmp ogt {nxt}, {ba}")
        acc = f.emit(f"select i1 {gt}, f32 {nxt}, f32 {ba}")
    else:
        acc = f.emit(f"fadd {ba}, {nxt}")
    ni = f.emit(f"add {bi}, 1")
    f.term(f"br label %{rh[0]} ; args({ni}, {acc})")
    f.switch(rx)
    _tile_store(f, dst, rows, 1, row, col, rx[1][0][0])
    nx = f.emit(f"add {blk[1][0][0]}, 1")
    f.term(f"br label %{header[0]} ; args({nx})")
    f.switch(cont)


def softmax(bm, bn):
    """softmax<BM, BN> over x, y [rows, BN·k] (crates/sile/tests/backend_softmax.rs:3-37):
    per program the row tile [BM, BN] at (pid, 0): load, row max, exp(x - max),
    row sum, divide, store, each its own loop nest over its own tile."""
    f = _Fn("softmax", [("x", 2, 0), ("y", 2, 2)])
    sx = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    sy = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 2")
    pid = f.emit("call i32 @llvm.nvvm.ctaid.x()")

    def origin(shape_desc):
        rb = f.emit(f"mul {pid}, {bm}")
        cb = f.emit(f"mul 0, {bn}")
        sp = f.emit(f"getelementptr i64, ptr addrspace(4) {shape_desc}, i64 1")
        stride = f.emit(f"load i64, ptr addrspace(4) {sp}")
        ro = f.emit(f"mul {rb}, {stride}")
        return f.emit(f"add {ro}, {cb}"), stride

    tiles = {}
    for t, cols in (("x", bn), ("m", 1), ("e", bn), ("s", 1), ("y", bn)):
        tiles[t] = f.emit(f"alloca [{bm} x [{cols} x f32]], addrspace(5)")
    xo, xs = origin(sx)

    def load_body(r, c):
        ro = f.emit(f"mul {r}, {xs}")
        wr = f.emit(f"add {xo}, {ro}")
        i = f.emit(f"add {wr}, {c}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %x, i64 {i}")
        v = f.emit(f"load f32, ptr addrspace(1) {p}")
        _tile_store(f, tiles["x"], bm, bn, r, c, v)
    _tile_loop(f, "tile_load", bm, bn, load_body)
    _reduce_rows(f, "tile_reduce_max", tiles["x"], bm, bn, tiles["m"], True)

    def exp_body(r, c):
        xv = _tile_load(f, tiles["x"], bm, bn, r, c)
        mv = _tile_load(f, tiles["m"], bm, 1, r, 0)
        d = f.emit(f"fsub {xv}, {mv}")
        ex = f.emit(f"call f32 @llvm.exp.f32(f32 {d})")
        _tile_store(f, tiles["e"], bm, bn, r, c, ex)
    _tile_loop(f, "tile_map_exp", bm, bn, exp_body)
    _reduce_rows(f, "tile_reduce_sum", tiles["e"], bm, bn, tiles["s"], False)

    def div_body(r, c):
        ev = _tile_load(f, tiles["e"], bm, bn, r, c)
        sv = _tile_load(f, tiles["s"], bm, 1, r, 0)
        q = f.emit(f"fdiv {ev}, {sv}")
        _tile_store(f, tiles["y"], bm, bn, r, c, q)
    _tile_loop(f, "tile_map_div", bm, bn, div_body)
    yo, ys = origin(sy)

    def store_body(r, c):
        v = _tile_load(f, tiles["y"], bm, bn, r, c)
        ro = f.emit(f"mul {r}, {ys}")
        wr = f.emit(f"add {yo}, {ro}")
        i = f.emit(f"add {wr}, {c}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %y, i64 {i}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {p}")
    _tile_loop(f, "tile_store", bm, bn, store_body)
    f.term("ret void")
    return f.text()


def vec_add(tile):
    """vec_add<TILE> over rank-1 a, b, c (crates/sile/examples/vec_add.rs): the
    tiles [1, TILE] at pid, loaded, added, stored (tile_memory.rs: rank-1
    buffers take `pid * TILE + row * TILE + col`)."""
    f = _Fn("vec_add", [("a", 1, 0), ("b", 1, 1), ("c", 1, 2)])
    pid = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    ta = f.emit(f"alloca [1 x [{tile} x f32]], addrspace(5)")
    tb = f.emit(f"alloca [1 x [{tile} x f32]], addrspace(5)")
    tc = f.emit(f"alloca [1 x [{tile} x f32]], addrspace(5)")

    def index(r, c):
        base = f.emit(f"mul {pid}, {tile}")
        ro = f.emit(f"mul {r}, {tile}")
        eo = f.emit(f"add {ro}, {c}")
        return f.emit(f"add {base}, {eo}")

    for buf, t in (("a", ta), ("b", tb)):
        def load_body(r, c, buf=buf, t=t):
            p = f.emit(f"getelementptr f32, ptr addrspace(1) %{buf}, i64 {index(r, c)}")
            v = f.emit(f"load f32, ptr addrspace(1) {p}")
            _tile_store(f, t, 1, tile, r, c, v)
        _tile_loop(f, "tile_load", 1, tile, load_body)

    def add_body(r, c):
        x = _tile_load(f, ta, 1, tile, r, c)
        y = _tile_load(f, tb, 1, tile, r, c)
        _tile_store(f, tc, 1, tile, r, c, f.emit(f"fadd {x}, {y}"))
    _tile_loop(f, "tile_map", 1, tile, add_body)

    def store_body(r, c):
        v = _tile_load(f, tc, 1, tile, r, c)
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %c, i64 {index(r, c)}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {p}")
    _tile_loop(f, "tile_store", 1, tile, store_body)
    f.term("ret void")
    return f.text()


def row_max(bn):
    """The row max of x [rows, BN] into out [rows] (the DSL's reduce_max along
    axis 1 of a [1, BN] tile per program, reduce.rs:10-30): load, reduce
    (single-column form: the output tile is [1 x 1]), store."""
    f = _Fn("row_max", [("x", 2, 0), ("out", 1, 2)])
    sx = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    pid = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    tx = f.emit(f"alloca [1 x [{bn} x f32]], addrspace(5)")
    tm = f.emit("alloca [1 x [1 x f32]], addrspace(5)")
    sp = f.emit(f"getelementptr i64, ptr addrspace(4) {sx}, i64 1")
    stride = f.emit(f"load i64, ptr addrspace(4) {sp}")
    ro = f.emit(f"mul {pid}, {stride}")

    def load_body(r, c):
        rs = f.emit(f"mul {r}, {stride}")
        wr = f.emit(f"add {ro}, {rs}")
        i = f.emit(f"add {wr}, {c}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %x, i64 {i}")
        _tile_store(f, tx, 1, bn, r, c, f.emit(f"load f32, ptr addrspace(1) {p}"))
    _tile_loop(f, "tile_load", 1, bn, load_body)
    _reduce_rows(f, "tile_reduce_max", tx, 1, bn, tm, True)

    def store_body(r, c):
        v = _tile_load(f, tm, 1, 1, r, c)
        base = f.emit(f"mul {pid}, 1")
        i = f.emit(f"add {base}, {c}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %out, i64 {i}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {p}")
    _tile_loop(f, "tile_store", 1, 1, store_body)
    f.term("ret void")
    return f.text()


def matmul(bm, bn, bk):
    """The canonical matmul's LLIR (crates/sile-tile-ir/src/passes/lowering/
    canonical_matmul.rs:24-444): c[tile] = a[rows] @ b[:, cols] over
    k < (lda / BK) * BK for program (m, n): a row x column nest of
    BM x BN cells, each a k loop carrying (k, sum, a_index, b_index) from
    (0, 0.0, a_tile_base + row * lda, col_tile_origin + col), then the store
    at c_tile_base + row * ldc + col."""
    f = _Fn("matmul", [("a", 2, 0), ("b", 2, 2), ("c", 2, 4)])
    sa = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    sb = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 2")
    sc = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 4")
    m = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    n = f.emit("call i32 @llvm.nvvm.ctaid.y()")

    def dim1(desc):
        p = f.emit(f"getelementptr i64, ptr addrspace(4) {desc}, i64 1")
        return f.emit(f"load i64, ptr addrspace(4) {p}")
    lda, ldb, ldc = dim1(sa), dim1(sb), dim1(sc)
    kt = f.emit(f"sdiv {lda}, {bk}")
    klim = f.emit(f"mul {kt}, {bk}")
    row0 = f.emit(f"mul {m}, {bm}")
    col0 = f.emit(f"mul {n}, {bn}")
    abase = f.emit(f"mul {row0}, {lda}")
    crow = f.emit(f"mul {row0}, {ldc}")
    cbase = f.emit(f"add {crow}, {col0}")
    rh = f.new_block("matmul_row_header", [("loop_row", "i64")])
    ch = f.new_block("matmul_col_header", [("loop_row", "i64"), ("loop_col", "i64")])
    ci = f.new_block("matmul_cell_init", [("loop_row", "i64"), ("loop_col", "i64")])
    kp = [("loop_row", "i64"), ("loop_col", "i64"), ("loop_k", "i64"), ("loop_sum", "f32"),
          ("loop_a_index", "i64"), ("loop_b_index", "i64")]
    kh = f.new_block("matmul_k_header", kp)
    kb = f.new_block("matmul_k_body", kp)
    st = f.new_block("matmul_store", [("loop_row", "i64"), ("loop_col", "i64"), ("loop_sum", "f32")])
    rl = f.new_block("matmul_row_latch", [("loop_row", "i64")])
    cont = f.new_block("matmul_continue", [])
    f.term(f"br label %{rh[0]} ; args(0)")
    f.switch(rh)
    r = rh[1][0][0]
    c = f.emit(f"icmp slt {r}, {bm}")
    f.term(f"br i1 {c}, label %{ch[0]}, label %{cont[0]} ; true_args({r}, 0)")
    f.switch(ch)
    cr, cc = ch[1][0][0], ch[1][1][0]
    c = f.emit(f"icmp slt {cc}, {bn}")
    f.term(f"br i1 {c}, label %{ci[0]}, label %{rl[0]} ; true_args({cr}, {cc}) ; false_args({cr})")
    f.switch(ci)
    ir, ic = ci[1][0][0], ci[1][1][0]
    aro = f.emit(f"mul {ir}, {lda}")
    a0 = f.emit(f"add {abase}, {aro}")
    b0 = f.emit(f"add {col0}, {ic}")
    f.term(f"br label %{kh[0]} ; args({ir}, {ic}, 0, 0.0, {a0}, {b0})")
    f.switch(kh)
    hr, hc, hk, hs, ha, hb = (p for p, _ in kh[1])
    c = f.emit(f"icmp slt {hk}, {klim}")
    f.term(f"br i1 {c}, label %{kb[0]}, label %{st[0]} ; true_args({hr}, {hc}, {hk}, {hs}, {ha}, {hb})"
           f" ; false_args({hr}, {hc}, {hs})")
    f.switch(kb)
    br_, bc, bkk, bs, ba, bb = (p for p, _ in kb[1])
    ap = f.emit(f"getelementptr f32, ptr addrspace(1) %a, i64 {ba}")
    av = f.emit(f"load f32, ptr addrspace(1) {ap}")
    bp = f.emit(f"getelementptr f32, ptr addrspace(1) %b, i64 {bb}")
    bv = f.emit(f"load f32, ptr addrspace(1) {bp}")
    prod = f.emit(f"fmul {av}, {bv}")
    ns = f.emit(f"fadd {bs}, {prod}")
    nk = f.emit(f"add {bkk}, 1")
    na = f.emit(f"add {ba}, 1")
    nb = f.emit(f"add {bb}, {ldb}")
    f.term(f"br label %{kh[0]} ; args({br_}, {bc}, {nk}, {ns}, {na}, {nb})")
    f.switch(st)
    sr, scol, ssum = (p for p, _ in st[1])
    cro = f.emit(f"mul {sr}, {ldc}")
    crb = f.emit(f"add {cbase}, {cro}")
    cix = f.emit(f"add {crb}, {scol}")
    cp = f.emit(f"getelementptr f32, ptr addrspace(1) %c, i64 {cix}")
    f.stmt(f"store f32 {ssum}, ptr addrspace(1) {cp}")
    nc = f.emit(f"add {scol}, 1")
    f.term(f"br label %{ch[0]} ; args({sr}, {nc})")
    f.switch(rl)
    nr = f.emit(f"add {rl[1][0][0]}, 1")
    f.term(f"br label %{rh[0]} ; args({nr})")
    f.switch(cont)
    f.term("ret void")
    return f.text()


def mma_program(bm, bn, bk):
    """c[tile (m, n)] = a[rows of m, :BK] @ b[:BK, cols of n] through tiles:
    loads of a [BM x BK] and b [BK x BN] (2-D tile loops), a zero
    accumulator (tile_memory.rs:22-47 fill loop), the MMA nest of
    tile_compute/mma.rs:25-260 (per cell: sum from acc[row][col], k loop over
    BK of a[row][k] * b[k][col], store into the result tile), then the
    store loop into c."""
    f = _Fn("mma", [("a", 2, 0), ("b", 2, 2), ("c", 2, 4)])
    sa = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    sb = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 2")
    sc = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 4")
    m = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    n = f.emit("call i32 @llvm.nvvm.ctaid.y()")
    ta = f.emit(f"alloca [{bm} x [{bk} x f32]], addrspace(5)")
    tb = f.emit(f"alloca [{bk} x [{bn} x f32]], addrspace(5)")
    tacc = f.emit(f"alloca [{bm} x [{bn} x f32]], addrspace(5)")
    tdst = f.emit(f"alloca [{bm} x [{bn} x f32]], addrspace(5)")

    def origin(desc, rt, ct, rows, cols):
        rb = f.emit(f"mul {rt}, {rows}")
        cb = f.emit(f"mul {ct}, {cols}")
        p = f.emit(f"getelementptr i64, ptr addrspace(4) {desc}, i64 1")
        stride = f.emit(f"load i64, ptr addrspace(4) {p}")
        ro = f.emit(f"mul {rb}, {stride}")
        return f.emit(f"add {ro}, {cb}"), stride

    def load(buf, desc, tile, rows, cols, rt, ct):
        o, stride = origin(desc, rt, ct, rows, cols)

        def body(r, c):
            ro = f.emit(f"mul {r}, {stride}")
            wr = f.emit(f"add {o}, {ro}")
            i = f.emit(f"add {wr}, {c}")
            p = f.emit(f"getelementptr f32, ptr addrspace(1) %{buf}, i64 {i}")
            _tile_store(f, tile, rows, cols, r, c, f.emit(f"load f32, ptr addrspace(1) {p}"))
        _tile_loop(f, "tile_load", rows, cols, body)
    load("a", sa, ta, bm, bk, m, 0)
    load("b", sb, tb, bk, bn, 0, n)
    _tile_loop(f, "tile_fill", bm, bn, lambda r, c: _tile_store(f, tacc, bm, bn, r, c, "0.0"))
    # the MMA nest (mma.rs:25-260)
    rh = f.new_block("tile_mma_row_header", [("loop_row", "i64")])
    ch = f.new_block("tile_mma_col_header", [("loop_row", "i64"), ("loop_col", "i64")])
    ib = f.new_block("tile_mma_init", [("loop_row", "i64"), ("loop_col", "i64")])
    kp = [("loop_row", "i64"), ("loop_col", "i64"), ("loop_k", "i64"), ("loop_sum", "f32")]
    kh = f.new_block("tile_mma_k_header", kp)
    kb = f.new_block("tile_mma_k_body", kp)
    st = f.new_block("tile_mma_store", [("loop_row", "i64"), ("loop_col", "i64"), ("loop_sum", "f32")])
    rl = f.new_block("tile_mma_row_latch", [("loop_row", "i64")])
    cont = f.new_block("tile_mma_continue", [])
    f.term(f"br label %{rh[0]} ; args(0)")
    f.switch(rh)
    r = rh[1][0][0]
    c = f.emit(f"icmp slt {r}, {bm}")
    f.term(f"br i1 {c}, label %{ch[0]}, label %{cont[0]} ; true_args({r}, 0)")
    f.switch(ch)
    cr, cc = ch[1][0][0], ch[1][1][0]
    c = f.emit(f"icmp slt {cc}, {bn}")
    f.term(f"br i1 {c}, label %{ib[0]}, label %{rl[0]} ; true_args({cr}, {cc}) ; false_args({cr})")
    f.switch(ib)
    ir, ic = ib[1][0][0], ib[1][1][0]
    s0 = _tile_load(f, tacc, bm, bn, ir, ic)
    f.term(f"br label %{kh[0]} ; args({ir}, {ic}, 0, {s0})")
    f.switch(kh)
    hr, hc, hk, hs = (p for p, _ in kh[1])
    c = f.emit(f"icmp slt {hk}, {bk}")
    f.term(f"br i1 {c}, label %{kb[0]}, label %{st[0]} ; true_args({hr}, {hc}, {hk}, {hs})"
           f" ; false_args({hr}, {hc}, {hs})")
    f.switch(kb)
    br_, bc, bkk, bs = (p for p, _ in kb[1])
    lhs = _tile_load(f, ta, bm, bk, br_, bkk)
    rhs = _tile_load(f, tb, bk, bn, bkk, bc)
    prod = f.emit(f"fmul {lhs}, {rhs}")
    ns = f.emit(f"fadd {bs}, {prod}")
    nk = f.emit(f"add {bkk}, 1")
    f.term(f"br label %{kh[0]} ; args({br_}, {bc}, {nk}, {ns})")
    f.switch(st)
    sr, scol, ssum = (p for p, _ in st[1])
    _tile_store(f, tdst, bm, bn, sr, scol, ssum)
    nc = f.emit(f"add {scol}, 1")
    f.term(f"br label %{ch[0]} ; args({sr}, {nc})")
    f.switch(rl)
    nr = f.emit(f"add {rl[1][0][0]}, 1")
    f.term(f"br label %{rh[0]} ; args({nr})")
    f.switch(cont)
    o, stride = origin(sc, m, n, bm, bn)

    def store_body(r, c):
        v = _tile_load(f, tdst, bm, bn, r, c)
        ro = f.emit(f"mul {r}, {stride}")
        wr = f.emit(f"add {o}, {ro}")
        i = f.emit(f"add {wr}, {c}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %c, i64 {i}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {p}")
    _tile_loop(f, "tile_store", bm, bn, store_body)
    f.term("ret void")
    return f.text()


def col_reduce(bm, bn, is_max):
    """out[pid * BN + c] = the reduction over the BM rows of column c of the
    tile x[0:BM, pid * BN : (pid + 1) * BN] (reduce_max / reduce_sum along
    axis 0, tile_compute/reduce.rs:160-277: a column loop whose body reads
    row 0, then a reduce loop over rows 1.., then stores), out rank 1."""
    f = _Fn("col_reduce", [("x", 2, 0), ("out", 1, 2)])
    sx = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    pid = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    tx = f.emit(f"alloca [{bm} x [{bn} x f32]], addrspace(5)")
    tr = f.emit(f"alloca [1 x [{bn} x f32]], addrspace(5)")
    rb = f.emit(f"mul 0, {bm}")
    cb = f.emit(f"mul {pid}, {bn}")
    sp = f.emit(f"getelementptr i64, ptr addrspace(4) {sx}, i64 1")
    stride = f.emit(f"load i64, ptr addrspace(4) {sp}")
    ro = f.emit(f"mul {rb}, {stride}")
    origin = f.emit(f"add {ro}, {cb}")

    def load_body(r, c):
        rs = f.emit(f"mul {r}, {stride}")
        wr = f.emit(f"add {origin}, {rs}")
        i = f.emit(f"add {wr}, {c}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %x, i64 {i}")
        _tile_store(f, tx, bm, bn, r, c, f.emit(f"load f32, ptr addrspace(1) {p}"))
    _tile_loop(f, "tile_load", bm, bn, load_body)
    prefix = "tile_reduce"
    header = f.new_block(f"{prefix}_col_header", [("loop_col", "i64")])
    blk = f.new_block(f"{prefix}_col_body", [("loop_col", "i64")])
    cont = f.new_block(f"{prefix}_continue", [])
    f.term(f"br label %{header[0]} ; args(0)")
    f.switch(header)
    i = header[1][0][0]
    c = f.emit(f"icmp slt {i}, {bn}")
    f.term(f"br i1 {c}, label %{blk[0]}, label %{cont[0]} ; true_args({i})")
    f.switch(blk)
    col = blk[1][0][0]
    init = _tile_load(f, tx, bm, bn, 0, col)
    rh = f.new_block(f"{prefix}_reduce_header", [("reduce_idx", "i64"), ("reduce_acc", "f32")])
    rbk = f.new_block(f"{prefix}_reduce_body", [("reduce_idx", "i64"), ("reduce_acc", "f32")])
    rx = f.new_block(f"{prefix}_reduce_exit", [("final_acc", "f32")])
    f.term(f"br label %{rh[0]} ; args(1, {init})")
    f.switch(rh)
    hi, ha = rh[1][0][0], rh[1][1][0]
    c = f.emit(f"icmp slt {hi}, {bm}")
    f.term(f"br i1 {c}, label %{rbk[0]}, label %{rx[0]} ; true_args({hi}, {ha}) ; false_args({ha})")
    f.switch(rbk)
    bi, ba = rbk[1][0][0], rbk[1][1][0]
    nxt = _tile_load(f, tx, bm, bn, bi, col)
    if is_max:
        gt = f.emit(f"fcmp ogt {nxt}, {ba}")
        acc = f.emit(f"select i1 {gt}, f32 {nxt}, f32 {ba}")
    else:
        acc = f.emit(f"fadd {ba}, {nxt}")
    ni = f.emit(f"add {bi}, 1")
    f.term(f"br label %{rh[0]} ; args({ni}, {acc})")
    f.switch(rx)
    _tile_store(f, tr, 1, bn, 0, col, rx[1][0][0])
    nx = f.emit(f"add {col}, 1")
    f.term(f"br label %{header[0]} ; args({nx})")
    f.switch(cont)

    def store_body(r, c):
        v = _tile_load(f, tr, 1, bn, r, c)
        base = f.emit(f"mul {pid}, {bn}")
        ro2 = f.emit(f"mul {r}, {bn}")
        eo = f.emit(f"add {ro2}, {c}")
        i = f.emit(f"add {base}, {eo}")
        p = f.emit(f"getelementptr f32, ptr addrspace(1) %out, i64 {i}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {p}")
    _tile_loop(f, "tile_store", 1, bn, store_body)
    f.term("ret void")
    return f.text()


def vec_add_fused(tile):
    """vec_add<TILE> as the reference lowers it after fusion (no tile allocas,
    crates/sile/tests/llvm_ir_lowering.rs:58-78): one column loop loading
    a and b at pid * TILE + col, adding, storing c."""
    f = _Fn("vec_add", [("a", 1, 0), ("b", 1, 1), ("c", 1, 2)])
    pid = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    base = f.emit(f"mul {pid}, {tile}")

    def body(r, c):
        ro = f.emit(f"mul {r}, {tile}")
        eo = f.emit(f"add {ro}, {c}")
        i = f.emit(f"add {base}, {eo}")
        pa = f.emit(f"getelementptr f32, ptr addrspace(1) %a, i64 {i}")
        va = f.emit(f"load f32, ptr addrspace(1) {pa}")
        pb = f.emit(f"getelementptr f32, ptr addrspace(1) %b, i64 {i}")
        vb = f.emit(f"load f32, ptr addrspace(1) {pb}")
        s = f.emit(f"fadd {va}, {vb}")
        pc = f.emit(f"getelementptr f32, ptr addrspace(1) %c, i64 {i}")
        f.stmt(f"store f32 {s}, ptr addrspace(1) {pc}")
    _tile_loop(f, "tile_map", 1, tile, body)
    f.term("ret void")
    return f.text()


def fused_mma_loop(bm, bn, bk):
    """c[tile (m, n)] = sum over K tiles of a[rows, k tile] @ b[k tile, cols],
    with the accumulator tile carried through the K-tile loop as a block
    parameter (a pointer) and the MMA fused with its loads
    (tile_compute/mma.rs:262-739: per cell, the first K tile starts from the
    splat 0.0, later ones from the accumulator; the k loop reads a and b from
    their buffers; the cell's sum goes back into the accumulator), then the
    store loop into c.  K = lda, whole BK tiles."""
    f = _Fn("fused_mma", [("a", 2, 0), ("b", 2, 2), ("c", 2, 4)])
    sa = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    sb = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 2")
    sc = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 4")
    m = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    n = f.emit("call i32 @llvm.nvvm.ctaid.y()")

    def dim1(desc):
        p = f.emit(f"getelementptr i64, ptr addrspace(4) {desc}, i64 1")
        return f.emit(f"load i64, ptr addrspace(4) {p}")
    lda, ldb, ldc = dim1(sa), dim1(sb), dim1(sc)
    ktiles = f.emit(f"sdiv {lda}, {bk}")
    acc0 = f.emit(f"alloca [{bm} x [{bn} x f32]], addrspace(5)")
    tty = f"[{bm} x [{bn} x f32]]"
    lh = f.new_block("loop_header", [("kt", "i64"), ("acc", "ptr addrspace(5)")])
    lb = f.new_block("loop_body", [("kt", "i64"), ("acc", "ptr addrspace(5)")])
    lx = f.new_block("loop_exit", [("acc", "ptr addrspace(5)")])
    f.term(f"br label %{lh[0]} ; args(0, {acc0})")
    f.switch(lh)
    kt, acc = lh[1][0][0], lh[1][1][0]
    c = f.emit(f"icmp slt {kt}, {ktiles}")
    f.term(f"br i1 {c}, label %{lb[0]}, label %{lx[0]} ; true_args({kt}, {acc}) ; false_args({acc})")
    f.switch(lb)
    bkt, bacc = lb[1][0][0], lb[1][1][0]
    # tile origins (compute_rank2_tile_origin, mma.rs:741-784)
    arb = f.emit(f"mul {m}, {bm}")
    acb = f.emit(f"mul {bkt}, {bk}")
    aro = f.emit(f"mul {arb}, {lda}")
    aorg = f.emit(f"add {aro}, {acb}")
    brb = f.emit(f"mul {bkt}, {bk}")
    bcb = f.emit(f"mul {n}, {bn}")
    bro = f.emit(f"mul {brb}, {ldb}")
    borg = f.emit(f"add {bro}, {bcb}")
    rh = f.new_block("tile_mma_row_header", [("loop_row", "i64")])
    ch = f.new_block("tile_mma_col_header", [("loop_row", "i64"), ("loop_col", "i64")])
    ib = f.new_block("tile_mma_init", [("loop_row", "i64"), ("loop_col", "i64")])
    zp = [("loop_row", "i64"), ("loop_col", "i64"), ("loop_a_index", "i64"), ("loop_b_index", "i64")]
    zb = f.new_block("tile_mma_init_zero", zp)
    ldb_ = f.new_block("tile_mma_init_load", zp)
    kp = [("loop_row", "i64"), ("loop_col", "i64"), ("loop_k", "i64"), ("loop_sum", "f32"),
          ("loop_a_index", "i64"), ("loop_b_index", "i64")]
    kh = f.new_block("tile_mma_k_header", kp)
    kb = f.new_block("tile_mma_k_body", kp)
    st = f.new_block("tile_mma_store", [("loop_row", "i64"), ("loop_col", "i64"), ("loop_sum", "f32")])
    rl = f.new_block("tile_mma_row_latch", [("loop_row", "i64")])
    cont = f.new_block("tile_mma_continue", [])
    f.term(f"br label %{rh[0]} ; args(0)")
    f.switch(rh)
    r = rh[1][0][0]
    c = f.emit(f"icmp slt {r}, {bm}")
    f.term(f"br i1 {c}, label %{ch[0]}, label %{cont[0]} ; true_args({r}, 0)")
    f.switch(ch)
    cr, cc = ch[1][0][0], ch[1][1][0]
    c = f.emit(f"icmp slt {cc}, {bn}")
    f.term(f"br i1 {c}, label %{ib[0]}, label %{rl[0]} ; true_args({cr}, {cc}) ; false_args({cr})")
    f.switch(ib)
    ir, ic = ib[1][0][0], ib[1][1][0]
    aro2 = f.emit(f"mul {ir}, {lda}")
    a0 = f.emit(f"add {aorg}, {aro2}")
    b0 = f.emit(f"add {borg}, {ic}")
    first = f.emit(f"icmp eq {bkt}, 0")
    f.term(f"br i1 {first}, label %{zb[0]}, label %{ldb_[0]} ; true_args({ir}, {ic}, {a0}, {b0})"
           f" ; false_args({ir}, {ic}, {a0}, {b0})")
    f.switch(zb)
    zr, zc, za, zbi = (p for p, _ in zb[1])
    f.term(f"br label %{kh[0]} ; args({zr}, {zc}, 0, 0.0, {za}, {zbi})")
    f.switch(ldb_)
    lr, lc, la, lbi = (p for p, _ in ldb_[1])
    gp = f.emit(f"getelementptr {tty}, ptr addrspace(5) {bacc}, i64 {lr}, i64 {lc}")
    s0 = f.emit(f"load f32, ptr addrspace(5) {gp}")
    f.term(f"br label %{kh[0]} ; args({lr}, {lc}, 0, {s0}, {la}, {lbi})")
    f.switch(kh)
    hr, hc, hk, hs, ha, hb = (p for p, _ in kh[1])
    c = f.emit(f"icmp slt {hk}, {bk}")
    f.term(f"br i1 {c}, label %{kb[0]}, label %{st[0]} ; true_args({hr}, {hc}, {hk}, {hs}, {ha}, {hb})"
           f" ; false_args({hr}, {hc}, {hs})")
    f.switch(kb)
    br_, bc, bkk, bs, ba, bb = (p for p, _ in kb[1])
    ap = f.emit(f"getelementptr f32, ptr addrspace(1) %a, i64 {ba}")
    av = f.emit(f"load f32, ptr addrspace(1) {ap}")
    bp = f.emit(f"getelementptr f32, ptr addrspace(1) %b, i64 {bb}")
    bv = f.emit(f"load f32, ptr addrspace(1) {bp}")
    prod = f.emit(f"fmul {av}, {bv}")
    ns = f.emit(f"fadd {bs}, {prod}")
    nk = f.emit(f"add {bkk}, 1")
    na = f.emit(f"add {ba}, 1")
    nb = f.emit(f"add {bb}, {ldb}")
    f.term(f"br label %{kh[0]} ; args({br_}, {bc}, {nk}, {ns}, {na}, {nb})")
    f.switch(st)
    sr, scol, ssum = (p for p, _ in st[1])
    dp = f.emit(f"getelementptr {tty}, ptr addrspace(5) {bacc}, i64 {sr}, i64 {scol}")
    f.stmt(f"store f32 {ssum}, ptr addrspace(5) {dp}")
    nc = f.emit(f"add {scol}, 1")
    f.term(f"br label %{ch[0]} ; args({sr}, {nc})")
    f.switch(rl)
    nr = f.emit(f"add {rl[1][0][0]}, 1")
    f.term(f"br label %{rh[0]} ; args({nr})")
    f.switch(cont)
    nkt = f.emit(f"add {bkt}, 1")
    f.term(f"br label %{lh[0]} ; args({nkt}, {bacc})")
    f.switch(lx)
    xacc = lx[1][0][0]
    crb = f.emit(f"mul {m}, {bm}")
    ccb = f.emit(f"mul {n}, {bn}")
    cro = f.emit(f"mul {crb}, {ldc}")
    corg = f.emit(f"add {cro}, {ccb}")

    def store_body(r, c):
        p = f.emit(f"getelementptr {tty}, ptr addrspace(5) {xacc}, i64 {r}, i64 {c}")
        v = f.emit(f"load f32, ptr addrspace(5) {p}")
        ro = f.emit(f"mul {r}, {ldc}")
        wr = f.emit(f"add {corg}, {ro}")
        i = f.emit(f"add {wr}, {c}")
        q = f.emit(f"getelementptr f32, ptr addrspace(1) %c, i64 {i}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {q}")
    _tile_loop(f, "tile_store", bm, bn, store_body)
    f.term("ret void")
    return f.text()


def mma_k_loop(bm, bn, bk):
    """The unfused form of a K-tile loop: the accumulator tile is a block
    parameter (a pointer) that starts at a zero-filled tile and is then the
    MMA's result tile: each iteration loads a [BM x BK] and b [BK x BN] tiles
    (2-D tile loops), runs the MMA nest of mma.rs:25-260 from acc into the
    result tile, and carries the result; the exit stores it into c."""
    f = _Fn("mma_k_loop", [("a", 2, 0), ("b", 2, 2), ("c", 2, 4)])
    sa = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 0")
    sb = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 2")
    sc = f.emit("getelementptr i64, ptr addrspace(4) %__sile_shapes, i64 4")
    m = f.emit("call i32 @llvm.nvvm.ctaid.x()")
    n = f.emit("call i32 @llvm.nvvm.ctaid.y()")

    def dim1(desc):
        p = f.emit(f"getelementptr i64, ptr addrspace(4) {desc}, i64 1")
        return f.emit(f"load i64, ptr addrspace(4) {p}")
    lda, ldb, ldc = dim1(sa), dim1(sb), dim1(sc)
    ktiles = f.emit(f"sdiv {lda}, {bk}")
    tty = f"[{bm} x [{bn} x f32]]"
    ta = f.emit(f"alloca [{bm} x [{bk} x f32]], addrspace(5)")
    tb = f.emit(f"alloca [{bk} x [{bn} x f32]], addrspace(5)")
    t0 = f.emit(f"alloca {tty}, addrspace(5)")
    td = f.emit(f"alloca {tty}, addrspace(5)")
    _tile_loop(f, "tile_fill", bm, bn, lambda r, c: _tile_store(f, t0, bm, bn, r, c, "0.0"))
    lh = f.new_block("loop_header", [("kt", "i64"), ("acc", "ptr addrspace(5)")])
    lb = f.new_block("loop_body", [("kt", "i64"), ("acc", "ptr addrspace(5)")])
    lx = f.new_block("loop_exit", [("acc", "ptr addrspace(5)")])
    f.term(f"br label %{lh[0]} ; args(0, {t0})")
    f.switch(lh)
    kt, acc = lh[1][0][0], lh[1][1][0]
    c = f.emit(f"icmp slt {kt}, {ktiles}")
    f.term(f"br i1 {c}, label %{lb[0]}, label %{lx[0]} ; true_args({kt}, {acc}) ; false_args({acc})")
    f.switch(lb)
    bkt, bacc = lb[1][0][0], lb[1][1][0]

    def load(buf, tile, rows, cols, rt, ct, stride):
        rb = f.emit(f"mul {rt}, {rows}")
        cb = f.emit(f"mul {ct}, {cols}")
        ro = f.emit(f"mul {rb}, {stride}")
        o = f.emit(f"add {ro}, {cb}")

        def body(r, c):
            rs = f.emit(f"mul {r}, {stride}")
            wr = f.emit(f"add {o}, {rs}")
            i = f.emit(f"add {wr}, {c}")
            p = f.emit(f"getelementptr f32, ptr addrspace(1) %{buf}, i64 {i}")
            _tile_store(f, tile, rows, cols, r, c, f.emit(f"load f32, ptr addrspace(1) {p}"))
        _tile_loop(f, "tile_load", rows, cols, body)
    load("a", ta, bm, bk, m, bkt, lda)
    load("b", tb, bk, bn, bkt, n, ldb)
    rh = f.new_block("tile_mma_row_header", [("loop_row", "i64")])
    ch = f.new_block("tile_mma_col_header", [("loop_row", "i64"), ("loop_col", "i64")])
    ib = f.new_block("tile_mma_init", [("loop_row", "i64"), ("loop_col", "i64")])
    kp = [("loop_row", "i64"), ("loop_col", "i64"), ("loop_k", "i64"), ("loop_sum", "f32")]
    kh = f.new_block("tile_mma_k_header", kp)
    kb = f.new_block("tile_mma_k_body", kp)
    st = f.new_block("tile_mma_store", [("loop_row", "i64"), ("loop_col", "i64"), ("loop_sum", "f32")])
    rl = f.new_block("tile_mma_row_latch", [("loop_row", "i64")])
    cont = f.new_block("tile_mma_continue", [])
    f.term(f"br label %{rh[0]} ; args(0)")
    f.switch(rh)
    r = rh[1][0][0]
    c = f.emit(f"icmp slt {r}, {bm}")
    f.term(f"br i1 {c}, label %{ch[0]}, label %{cont[0]} ; true_args({r}, 0)")
    f.switch(ch)
    cr, cc = ch[1][0][0], ch[1][1][0]
    c = f.emit(f"icmp slt {cc}, {bn}")
    f.term(f"br i1 {c}, label %{ib[0]}, label %{rl[0]} ; true_args({cr}, {cc}) ; false_args({cr})")
    f.switch(ib)
    ir, ic = ib[1][0][0], ib[1][1][0]
    gp = f.emit(f"getelementptr {tty}, ptr addrspace(5) {bacc}, i64 {ir}, i64 {ic}")
    s0 = f.emit(f"load f32, ptr addrspace(5) {gp}")
    f.term(f"br label %{kh[0]} ; args({ir}, {ic}, 0, {s0})")
    f.switch(kh)
    hr, hc, hk, hs = (p for p, _ in kh[1])
    c = f.emit(f"icmp slt {hk}, {bk}")
    f.term(f"br i1 {c}, label %{kb[0]}, label %{st[0]} ; true_args({hr}, {hc}, {hk}, {hs})"
           f" ; false_args({hr}, {hc}, {hs})")
    f.switch(kb)
    br_, bc, bkk, bs = (p for p, _ in kb[1])
    lhs = _tile_load(f, ta, bm, bk, br_, bkk)
    rhs = _tile_load(f, tb, bk, bn, bkk, bc)
    prod = f.emit(f"fmul {lhs}, {rhs}")
    ns = f.emit(f"fadd {bs}, {prod}")
    nk = f.emit(f"add {bkk}, 1")
    f.term(f"br label %{kh[0]} ; args({br_}, {bc}, {nk}, {ns})")
    f.switch(st)
    sr, scol, ssum = (p for p, _ in st[1])
    _tile_store(f, td, bm, bn, sr, scol, ssum)
    nc = f.emit(f"add {scol}, 1")
    f.term(f"br label %{ch[0]} ; args({sr}, {nc})")
    f.switch(rl)
    nr = f.emit(f"add {rl[1][0][0]}, 1")
    f.term(f"br label %{rh[0]} ; args({nr})")
    f.switch(cont)
    nkt = f.emit(f"add {bkt}, 1")
    f.term(f"br label %{lh[0]} ; args({nkt}, {td})")
    f.switch(lx)
    xacc = lx[1][0][0]
    crb = f.emit(f"mul {m}, {bm}")
    ccb = f.emit(f"mul {n}, {bn}")
    cro = f.emit(f"mul {crb}, {ldc}")
    corg = f.emit(f"add {cro}, {ccb}")

    def store_body(r, c):
        p = f.emit(f"getelementptr {tty}, ptr addrspace(5) {xacc}, i64 {r}, i64 {c}")
        v = f.emit(f"load f32, ptr addrspace(5) {p}")
        ro = f.emit(f"mul {r}, {ldc}")
        wr = f.emit(f"add {corg}, {ro}")
        i = f.emit(f"add {wr}, {c}")
        q = f.emit(f"getelementptr f32, ptr addrspace(1) %c, i64 {i}")
        f.stmt(f"store f32 {v}, ptr addrspace(1) {q}")
    _tile_loop(f, "tile_store", bm, bn, store_body)
    f.term("ret void")
    return f.text()
