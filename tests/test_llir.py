"""Generic HIP code generation for sile's LLIR (printed form,
crates/sile-llvm-ir/src/print.rs): translation and hiprtc compilation on the
CPU, no GPU needed.  The LLIR inputs under tests/golden/llir/ are written by
hand in that printed form (the reference's own lowering cannot run here: it is
Rust); the GPU tests in test_gpu_llir.py run what is compiled here against the
oracle and the reference's fixtures."""
import os

import pytest

from sile_amd import _abi as hip

LLIR = os.path.join(os.path.dirname(__file__), "golden", "llir")

# name -> tile plan (output parameter index, rows, cols) or None
PLANS = {
    "vec_add": (2, 1, 4),
    "relu": (0, 1, 8),
    "matmul": (2, 2, 2),
    "softmax": (1, 2, 8),
    "parallel_reduce": None,
}


def text(name):
    with open(os.path.join(LLIR, name + ".llir")) as f:
        return f.read()


@pytest.mark.parametrize("name", sorted(PLANS))
def test_translates_and_compiles(name):
    image, kernel = hip.llir_compile(text(name), PLANS[name])
    assert kernel == f"sile_kernel_{name}"
    # an ELF code object or a clang offload bundle holding one
    assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    assert len(image) > 1000


def test_generated_source_follows_the_cpu_codegen():
    src = hip.llir_to_hip(text("matmul"), PLANS["matmul"])
    # per-program body + wrapper, as crates/sile-backend/src/cpu/codegen.rs:433-555
    assert "void sile_llvm_ir_matmul(" in src
    assert 'extern "C" __global__' in src and "sile_kernel_matmul(void** buffers" in src
    # rank-2 output tile plan: tiles_n = shape(c)[1] / 2, total = shape(c)[0] / 2 * tiles_n
    assert "sile_tiles_n = shapes[5] / 2;" in src
    assert "sile_total_tiles = (shapes[4] / 2) * sile_tiles_n;" in src
    assert "g0 = sile_pid / sile_tiles_n, g1 = sile_pid % sile_tiles_n" in src
    # block ids are the tile coordinates, the accumulation is mul then add
    assert "v_m = sile_gid_0;" in src and "v_n = sile_gid_1;" in src
    assert "v_prod = v_av * v_bv;" in src and "v_acc_next = v_acc + v_prod;" in src
    sm = hip.llir_to_hip(text("softmax"), PLANS["softmax"])
    assert "expf(v_d)" in sm and "(v_gt) ? (v_xv) : (v_mx)" in sm
    # the tile's storage, its pointer decayed to a row pointer, an element gep
    # indexing [row][col] (the backends' C form, cpu/codegen.rs:601-664)
    assert "float v_tile_storage[2][8];" in sm and "float (*v_tile)[8] = v_tile_storage;" in sm
    assert "&(v_tile[v_r][v_e])" in sm
    pr = hip.llir_to_hip(text("parallel_reduce"), None)
    assert "llir_vec_load_4(v_x, v_off)" in pr and "atomicAdd(v_o, v_acc)" in pr
    # no tile plan, rank-1 last buffer: total tiles = shape of the first buffer
    assert "sile_total_tiles = shapes[0];" in pr


def test_branch_arguments_are_assigned_in_parallel():
    """Block arguments take the values of the branch's operands as they were
    before the branch (SSA): swapping two loop-carried values works."""
    src = hip.llir_to_hip("""define void @swap(ptr addrspace(1) %o, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %o [rank=1, shape_offset=0, elem=f32]
bb0:
  br label %loop ; args(0, 1.0, 2.0)
loop:
  ; args(%i: i64, %x: f32, %y: f32)
  %c = icmp slt %i, 3
  br i1 %c, label %body, label %done
body:
  %n = add %i, 1
  br label %loop ; args(%n, %y, %x)
done:
  %p = getelementptr f32, ptr addrspace(1) %o, i64 0
  store f32 %x, ptr addrspace(1) %p
  ret void
}
""", None)
    # the body, entered only from its header, runs inside a C loop there
    body = src[src.index("L_v_loop:"):src.index("L_v_done:")]
    assert "#pragma unroll 4\n  for (;;) {" in body and "if (!(v_c)) break;" in body
    assert "L_v_body:" not in src
    # every new value is read before any loop variable is written
    assert "float t1 = v_y;" in body and "float t2 = v_x;" in body
    assert body.index("float t2 = v_x;") < body.index("v_x = t1;") < body.index("v_y = t2;")


@pytest.mark.parametrize("bad,msg", [
    ("define void @f() {\nbb0:\n  %x = frobnicate 1, 2\n  ret void\n}\n", "unknown instruction"),
    ("define void @f() {\nbb0:\n  br label %nowhere\n}\n", "unknown block"),
    ("define void @f() {\nbb0:\n  ret void\n", "missing closing"),
    ("define void @f() {\nbb0:\n  br label %b ; args(1)\nb:\n  ret void\n}\n", "arguments for 0"),
    ("define void @f() {\nbb0:\n  %a = add 1, 2\n  %a = add 1, 2\n  ret void\n}\n", "defined twice"),
    ("hello\n", "expected 'define'"),
])
def test_malformed_llir_is_a_compile_error(bad, msg):
    with pytest.raises(hip.SileError) as e:
        hip.llir_to_hip(bad, None)
    assert e.value.kind == "Compile" and msg in str(e.value)


def test_tile_plan_must_name_a_shaped_parameter():
    with pytest.raises(hip.SileError) as e:
        hip.llir_to_hip(text("vec_add"), (3, 1, 4))  # %__sile_shapes has no shape ABI
    assert e.value.kind == "Compile"
    with pytest.raises(hip.SileError) as e:
        hip.llir_to_hip(text("vec_add"), (2, 0, 4))
    assert e.value.kind == "Shape"


def _fn(body, name="contract"):
    return ("define void @" + name + "(ptr addrspace(4) %__sile_shapes) {\n"
            "  ; sile.param %__sile_shapes [elem=i64]\n" + body + "}\n")


def test_switch_terminator_is_rejected():
    # crates/sile-backend/tests/compile.rs:23-57: every target rejects switch
    src = _fn("entry:\n  switch i64 0, label %exit [1 , label %exit]\nexit:\n  ret void\n")
    with pytest.raises(hip.SileError) as e:
        hip.llir_to_hip(src)
    assert e.value.kind == "Compile"
    assert "does not support switch terminators" in str(e.value)


def test_tile_helper_and_unknown_calls_are_rejected():
    # crates/sile-backend/src/verify.rs:31-40 (tile helpers, every target) and
    # crates/sile-backend/tests/compile.rs:81-103 (other calls, the Metal target;
    # the generated HIP defines no helpers either)
    for callee, why in [("tile_load", "does not allow tile helper calls"),
                        ("unknown_helper", "does not support LLVM IR call instructions")]:
        src = _fn(f"entry:\n  call void @{callee}()\n  ret void\n")
        with pytest.raises(hip.SileError) as e:
            hip.llir_to_hip(src)
        assert e.value.kind == "Compile" and why in str(e.value), str(e.value)


def test_thread_id_is_allowed_and_is_zero():
    # crates/sile-backend/tests/compile.rs:105-131: the C target allows thread_id
    # (one program per thread, so it is 0); so does the HIP target
    src = _fn("entry:\n  %tid = call i32 @llvm.nvvm.tid.x()\n  ret void\n")
    out = hip.llir_to_hip(src)
    assert "v_tid = 0;" in out


# ---- one workgroup per program: loops spread over the lanes ----

def softmax_llir(bm, bn):
    """The softmax fixture at BM rows and BN columns per program."""
    t = text("softmax")
    for old, new in [("[2 x [8 x f32]]", f"[{bm} x [{bn} x f32]]"), ("mul %m, 2", f"mul %m, {bm}"),
                     ("icmp slt %r, 2", f"icmp slt %r, {bm}"), ("icmp slt %c, 8", f"icmp slt %c, {bn}"),
                     ("icmp slt %e, 8", f"icmp slt %e, {bn}"), ("icmp slt %q, 8", f"icmp slt %q, {bn}")]:
        assert old in t
        t = t.replace(old, new)
    return t


def parallel_reduce_llir(tile):
    t = text("parallel_reduce")
    for old, new in [("mul %pid, 16", f"mul %pid, {tile}"), ("icmp slt %i, 16", f"icmp slt %i, {tile}")]:
        assert old in t
        t = t.replace(old, new)
    return t


def vec_add_llir(tile):
    t = text("vec_add")
    assert t.count(", 4") >= 2
    return t.replace("mul %pid, 4", f"mul %pid, {tile}").replace("icmp slt %i, 4",
                                                                  f"icmp slt %i, {tile}")


def test_the_fixtures_keep_one_program_per_lane():
    """Loops of fewer than 256 iterations are not spread: the five fixtures'
    code is unchanged (64 programs a workgroup, no workgroup folds)."""
    for name in PLANS:
        src = hip.llir_to_hip(text(name), PLANS[name])
        assert "__launch_bounds__(64)" in src and "coop_" not in src, name


def test_long_loops_spread_over_the_workgroup():
    src = hip.llir_to_hip(softmax_llir(4, 8192), (1, 4, 8192))
    assert "__launch_bounds__(1024)" in src and "sile_pid = (long long)blockIdx.x;" in src
    # the row loop (4 iterations, loops inside) stays on every lane; the max,
    # exp + sum and divide loops are spread, 8 iterations a lane: the slot
    # form (iteration k W + l on lane l, fully unrolled)
    assert src.count("for (int coop_k = 0; coop_k < 8; ++coop_k) {") == 3
    assert src.count("const long long coop_it = (long long)coop_k * 1024LL + (long long)threadIdx.x;") == 3
    # bounds checked only where a slot can cross them: the max loop starts at 1
    assert src.count("if (coop_it < 1LL) continue;") == 1 and "coop_it >= 8192" not in src
    assert "int coop_i0 = INT_MAX;" in src and "coop_red_j, coop_rb);" in src
    assert "coop_wg_first_max(coop_p0, coop_i0" in src        # the max fold, from x0
    assert "v_sum = coop_init1 + coop_wg_sum(coop_p1" in src or \
           "v_sum = coop_init0 + coop_wg_sum(coop_p0" in src  # the sum of exp
    # the tile is only touched at [r, e] by the spread loops: per-lane slices
    assert "float v_tile_storage[4][8];" in src and "__shared__ float v_tile" not in src
    assert "&(v_tile[v_r][coop_k])" in src
    # x is never written: the max loop keeps each lane's x values, the exp
    # loop takes them (its iteration 0, which the max loop starting at 1 did
    # not run, loads)
    assert "coop_cache0[coop_k] = v_xv;" in src
    # (the max loop ran iterations 1 .. 8191: constants the unrolled slots fold)
    assert ("if (coop_ok0 && coop_it >= 1 && coop_it < 8192) v_xev = coop_cache0[coop_k]; "
            "else v_xev = *(v_xep);") in src
    assert "coop_tag0 = (long long)v_xrow;" in src and "coop_tag0 == (long long)v_xrow;" in src
    # past 16 iterations a lane: the strided form, tiles sliced by e / W, no cache
    wide = hip.llir_to_hip(softmax_llir(1, 32768), (1, 1, 32768))
    assert wide.count("for (long long coop_it = coop_start + (long long)threadIdx.x") == 3
    assert wide.count("#pragma unroll 8") == 3 and "coop_cache" not in wide
    assert "&(v_tile[v_r][(v_e) / 1024LL])" in wide
    # a barrier after a spread loop only where another lane's later access may
    # conflict: the divide loop stores y; the max loop reads x (never written)
    # and the exp loop writes the lanes' own slices, so neither needs one
    body = src[src.index("L_v_bb0:"):]
    assert body.count("__syncthreads();") == 1 and "__syncthreads();\n  goto L_v_sm_row_latch;" in body
    # one barrier a workgroup fold (its LDS exchange alternates halves)
    assert src.count("__syncthreads();") == 3 and "int coop_rb = 0;" in src
    pr = hip.llir_to_hip(parallel_reduce_llir(4096), None)
    assert "coop_wg_sum" in pr and "if (threadIdx.x == 0) atomicAdd(v_o, v_acc);" in pr
    # the reduce loop only reads x: the fold's own barrier, none after the loop
    assert pr[pr.index("L_v_bb0:"):].count("__syncthreads();") == 0
    va = hip.llir_to_hip(vec_add_llir(4096), (2, 1, 4096))
    assert "__launch_bounds__(1024)" in va
    # the add loop stores c: a barrier after it
    assert va[va.index("L_v_bb0:"):].count("__syncthreads();") == 1
    # buffers keep the global address space (global, not flat, loads and stores)
    assert "__attribute__((address_space(1))) float* __restrict__ v_a" in va
    assert "= (__attribute__((address_space(1))) float* )buffers[0];" in va
    for t, plan in ((softmax_llir(4, 8192), (1, 4, 8192)), (parallel_reduce_llir(4096), None),
                    (vec_add_llir(4096), (2, 1, 4096))):
        image, _ = hip.llir_compile(t, plan)
        assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


@pytest.mark.parametrize("name,old,new", [
    # a store to the same element every iteration (not one per iteration)
    ("vec_add", "%pc = getelementptr f32, ptr addrspace(1) %c, i64 %idx",
     "%pc = getelementptr f32, ptr addrspace(1) %c, i64 %base"),
    # a carried value that is not a sum or a max fold
    ("parallel_reduce", "%acc_next = fadd %acc, %s", "%acc_next = fmul %acc, %s"),
    # the loop's bound is not a constant
    ("parallel_reduce", "icmp slt %i, 4096", "icmp slt %i, %base"),
])
def test_loops_that_cannot_be_spread_stay_serial(name, old, new):
    t = vec_add_llir(4096) if name == "vec_add" else parallel_reduce_llir(4096)
    assert old in t
    src = hip.llir_to_hip(t.replace(old, new), (2, 1, 4096) if name == "vec_add" else None)
    assert "__launch_bounds__(64)" in src and "coop_" not in src


# ---- LLIR in the reference's loop shapes (tests/llir_shapes.py) ----

from tests import llir_shapes  # noqa: E402


def test_reference_loop_shapes_spread():
    """The reference's lowering passes a loop header's values on to a body
    block with parameters of its own, carries the row through the column
    header of a 2-D nest, indexes tiles [row, col] and starts a reduction
    from the row's element 0 read before its loop: those loops spread like
    the hand-written form."""
    src = hip.llir_to_hip(llir_shapes.softmax(4, 8192), (1, 4, 8192))
    assert "__launch_bounds__(1024)" in src
    # load, exp, divide and store column loops and the two reduce loops, in
    # the slot form; the row loops stay on every lane
    assert src.count("for (int coop_k = 0; coop_k < 8; ++coop_k) {") == 6
    # body parameters were replaced by the header's values, and the column
    # header's row (passed the row header's row or itself) by that row
    assert "v_loop_row18" not in src and "v_reduce_acc39" not in src
    assert "v_loop_row16" not in src
    # x, exp and y tiles are per-lane slices; the [4 x 1] max and sum tiles
    # (read at [row, 0] outside the loops) live in LDS
    for t in ("v_v4", "v_v6", "v_v8"):
        assert f"float {t}_storage[4][8];" in src and f"float (*{t})[8] = {t}_storage;" in src
    for t in ("v_v5", "v_v7"):
        assert f"__shared__ float {t}_storage[4][1];" in src
    # a reduction's element 0 comes from an LDS copy that the lane storing it
    # writes, between barriers around the storing loop
    assert "if (coop_it == 0LL) v_v4_sh0[v_loop_row15] = v_v27;" in src
    assert "v_v34 = &(v_v4_sh0[v_loop_row31]);" in src
    assert "__syncthreads();\n  {\n    const long long coop_start = v_loop_col17;" in src
    # loops of 8 iterations: one program a lane, tiles in registers
    small = hip.llir_to_hip(llir_shapes.softmax(2, 8), (1, 2, 8))
    assert "__launch_bounds__(64)" in small and "coop_" not in small
    assert "float (*v_v4)[8] = v_v4_storage;" in small
    va = hip.llir_to_hip(llir_shapes.vec_add(4096), (2, 1, 4096))
    assert "__launch_bounds__(1024)" in va and va.count("coop_k < 4;") == 4
    fused = hip.llir_to_hip(llir_shapes.vec_add_fused(4096), (2, 1, 4096))
    assert "__launch_bounds__(1024)" in fused and fused.count("coop_k < 4;") == 1
    rm = hip.llir_to_hip(llir_shapes.row_max(4096), (1, 1, 1))
    assert "coop_wg_first_max" in rm and "v_v3_sh0" in rm
    for t, plan in ((llir_shapes.softmax(4, 8192), (1, 4, 8192)), (llir_shapes.softmax(1, 1000), (1, 1, 1000)),
                    (llir_shapes.vec_add(4096), (2, 1, 4096)), (llir_shapes.row_max(4096), (1, 1, 1))):
        image, _ = hip.llir_compile(t, plan)
        assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


def test_gep_indexes_the_tile_dimensions():
    """A tile's gep takes an index for each dimension, [row][col], on the
    storage decayed to a row pointer (crates/sile-backend/src/cpu/codegen.rs
    gep_private_ptrs_do_not_materialize_fake_storage_bindings); a gep with
    fewer indices gives the sub-array, decayed; more indices than dimensions
    are rejected."""
    t = """define void @g(ptr addrspace(1) %o, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %o [rank=1, shape_offset=0, elem=f32]
  ; sile.param %__sile_shapes [elem=i64]
bb0:
  %tile = alloca [2 x [2 x f32]], addrspace(5)
  %elt = getelementptr [2 x [2 x f32]], ptr addrspace(5) %tile, i64 0, i64 1
  store f32 3.0, ptr addrspace(5) %elt
  %row = getelementptr [2 x [2 x f32]], ptr addrspace(5) %tile, i64 0
  %e2 = getelementptr [2 x f32], ptr addrspace(5) %row, i64 1
  %v = load f32, ptr addrspace(5) %e2
  %op = getelementptr f32, ptr addrspace(1) %o, i64 0
  store f32 %v, ptr addrspace(1) %op
  ret void
}
"""
    src = hip.llir_to_hip(t, None)
    assert "float v_tile_storage[2][2];" in src and "float (*v_tile)[2] = v_tile_storage;" in src
    assert "v_elt = &(v_tile[(0LL)][(1LL)]);" in src
    assert "v_row = (v_tile[(0LL)]);" in src and "v_e2 = &(v_row[(1LL)]);" in src
    image, _ = hip.llir_compile(t, None)
    assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
    bad = t.replace("i64 0, i64 1\n", "i64 0, i64 0, i64 1\n")
    with pytest.raises(hip.SileError, match="indexes past the array levels"):
        hip.llir_to_hip(bad, None)


def triangular_matmul(bm, bn, bk, by):
    """The canonical matmul's LLIR with the k loop's bound replaced by the
    cell's row or column (`k < row` / `k < col`): a trip count that differs
    between cells."""
    t = llir_shapes.matmul(bm, bn, bk)
    old = "%v45 = icmp slt %loop_k26, %v13"
    assert t.count(old) == 1
    return t.replace(old, "%v45 = icmp slt %loop_k26, " + ("%loop_row24" if by == "row" else "%loop_col25"))


def test_jam_needs_branches_alike_for_a_lanes_cells():
    """Mutations of the jam's rule: a lane's four cells of a 64 x 64 nest
    share their column (64 divides 1024) but not their row, so a k loop
    bounded by the column still runs them jammed, and one bounded by the row
    (each cell's own trip count) runs them one slot at a time."""
    by_col = hip.llir_to_hip(triangular_matmul(64, 64, 8, "col"), (2, 64, 64))
    assert "for (int coop_g = 0; coop_g < 1; ++coop_g) {" in by_col
    assert "v_v45 = v_loop_k26 < v_loop_col21;" in by_col
    by_row = hip.llir_to_hip(triangular_matmul(64, 64, 8, "row"), (2, 64, 64))
    assert "coop_g" not in by_row and "__s0" not in by_row
    assert "for (int coop_k = 0; coop_k < 4; ++coop_k) {" in by_row
    assert "v_v45 = v_loop_k26 < v_loop_row19;" in by_row


@pytest.mark.parametrize("bm,bn", [(16, 64), (32, 32), (64, 64), (128, 64), (64, 128), (32, 96),
                                   (96, 32), (24, 64), (128, 128), (256, 64), (48, 32), (8, 8)])
def test_nest_shapes_translate(bm, bn):
    """Every nest generator of tests/llir_shapes.py translates at tile shapes
    that take each form (one program a lane, slot form with and without a
    partial slot, jammed groups of two to four with the column shared or per
    slot, the strided form), and the canonical and MMA-loop forms compile.
    (The MMA forms keep one program a lane where their tiles pass the LDS
    budget: 256 x 64 accumulator and result tiles.)"""
    for gen in ("matmul", "mma_program", "fused_mma_loop", "mma_k_loop"):
        for bk in (4, 16):
            src = hip.llir_to_hip(getattr(llir_shapes, gen)(bm, bn, bk), (2, bm, bn))
            if gen != "matmul":
                continue
            cells = bm * bn
            assert ("__launch_bounds__(1024)" in src) == (cells >= 256), (bm, bn, bk)
            jammed = cells % 1024 == 0 and 2 <= cells // 1024 <= 16
            assert ("coop_g" in src) == jammed, (bm, bn, bk)
    for gen in ("matmul", "mma_k_loop"):
        image, _ = hip.llir_compile(getattr(llir_shapes, gen)(bm, bn, 8), (2, bm, bn))
        assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


def test_two_dimensional_nests_spread():
    """The canonical matmul's row x column nest (canonical_matmul.rs:24-444)
    and the tile MMA's (tile_compute/mma.rs:25-260) have a region of blocks
    for a body (cell init, the k loop, the store): iteration row * BN + col
    runs the region on one lane, the k loop stays serial on it.  A buffer
    store at `row * ldc + col` spreads when ldc >= BN at run time (lane 0
    runs the nest in order otherwise); nests take the slot form, and a tile
    touched only at [row, col] by unguarded nests of its shape is split over
    the lanes.  With every slot of every lane full and the region's branches
    alike for all of a lane's cells, a lane's cells run jammed, four at a
    time: what depends on the row or column per slot, the rest once."""
    mm = hip.llir_to_hip(llir_shapes.matmul(64, 64, 8), (2, 64, 64))
    assert "__launch_bounds__(1024)" in mm
    assert "const bool coop_par = true && v_v11 >= 64LL;\n    if (coop_par) {" in mm
    # spread: 4 cells a lane, jammed; 64 columns divide the workgroup, so a
    # lane's cells share their column (and the b element of each k); a
    # wave's 64 cells share their row, read as the wave's first lane's
    assert "for (int coop_g = 0; coop_g < 1; ++coop_g) {" in mm
    assert ("const long long coop_it__s0 = (long long)(coop_g * 4 + 0) * 1024LL + "
            "(long long)threadIdx.x;\n"
            "    v_loop_col21 = coop_it__s0 % 64LL;\n"
            "    v_loop_row19__s0 = (long long)__builtin_amdgcn_readfirstlane((int)(coop_it__s0 / 64LL));\n") in mm
    assert ("const long long coop_it__s3 = (long long)(coop_g * 4 + 3) * 1024LL + "
            "(long long)threadIdx.x;\n"
            "    v_loop_row19__s3 = (long long)__builtin_amdgcn_readfirstlane((int)(coop_it__s3 / 64LL));\n") in mm
    assert "v_v51__s3 = v_loop_sum27__s3 + v_v50__s3;" in mm   # a sum per cell
    assert "v_v50__s3 = v_v47__s3 * v_v49;" in mm              # one b element
    assert "v_v54 = v_loop_b_index29 + v_v9;" in mm and "v_v54__s" not in mm
    assert mm.count("v_v52 = v_loop_k26 + (1LL);") == 2         # the k counter once a copy
    # a cell's k loop, in both copies, unrolled 16 times (loads in flight)
    assert mm.count("#pragma unroll 16\n  for (;;) {") == 2 and "#pragma unroll 4\n" not in mm
    assert "goto coop_next0p;" in mm and "L_v_matmul_k_header_4_n0p:;" in mm
    # in order on lane 0 when ldc < BN
    assert ("} else if (threadIdx.x == 0) {\n"
            "    for (long long coop_it = 0; coop_it < 4096LL; ++coop_it) {\n"
            "    v_loop_row19 = coop_it / 64LL; v_loop_col21 = coop_it % 64LL;\n"
            "  goto L_v_matmul_cell_init_3_n0s;") in mm
    assert "goto coop_next0s;" in mm and "L_v_matmul_k_header_4_n0s:;" in mm
    # the k loop's carried row and column were the nest's own
    assert "v_loop_row22" not in mm and "v_loop_col23" not in mm
    small = hip.llir_to_hip(llir_shapes.matmul(8, 8, 8), (2, 8, 8))   # 64 cells: a lane each
    assert "__launch_bounds__(64)" in small and "coop_" not in small
    # 96 columns do not divide the workgroup: the column per slot as well
    odd = hip.llir_to_hip(llir_shapes.matmul(32, 96, 8), (2, 32, 96))
    assert "for (int coop_g = 0; coop_g < 1; ++coop_g) {" in odd
    assert "__s2 = coop_it__s2 / 96LL; v_loop_col21__s2 = coop_it__s2 % 96LL;" in odd
    # a partial slot (1536 cells): the slot form with its bound check, no jam
    part = hip.llir_to_hip(llir_shapes.matmul(48, 32, 8), (2, 48, 32))
    assert "for (int coop_k = 0; coop_k < 2; ++coop_k) {" in part
    assert "if (coop_it >= 1536LL) continue;" in part and "coop_g" not in part
    mma64 = hip.llir_to_hip(llir_shapes.mma_program(64, 64, 16), (2, 64, 64))
    assert "float v_v8_storage[4];" in mma64
    assert "v_v62__s2 = &(v_v8[(coop_g * 4 + 2)]);" in mma64   # slot coop_g * 4 + k
    mma = hip.llir_to_hip(llir_shapes.mma_program(32, 32, 16), (2, 32, 32))
    assert "__launch_bounds__(1024)" in mma
    # the accumulator (filled and read at [row, col] by unguarded slot-form
    # nests): one slot a lane; a and b (read at [row, k] / [k, col]) and the
    # result (read by the guarded store nest) in LDS
    assert "float v_v8_storage[1];" in mma and "v_v8 = v_v8_storage;" in mma
    assert "__shared__ float v_v6_storage[32][16];" in mma
    assert "__shared__ float v_v9_storage[32][32];" in mma
    assert mma.count("for (int coop_k = 0; coop_k < 1; ++coop_k) {") == 5
    for t, plan in ((llir_shapes.matmul(64, 64, 8), (2, 64, 64)),
                    (llir_shapes.matmul(48, 32, 8), (2, 48, 32)),
                    (llir_shapes.mma_program(64, 64, 16), (2, 64, 64)),
                    (llir_shapes.mma_program(32, 32, 16), (2, 32, 32))):
        image, _ = hip.llir_compile(t, plan)
        assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


def test_lone_column_loops_with_a_region_spread():
    """A reduction along axis 0 is a column loop whose body holds a reduce
    loop over the rows (tile_compute/reduce.rs:160-277): each column runs on
    one lane (its reduce loop serial, in order); the tile read at [row, col]
    stays the lane's column slice."""
    src = hip.llir_to_hip(llir_shapes.col_reduce(64, 1024, True), (1, 1, 1024))
    assert "__launch_bounds__(1024)" in src
    assert "    v_loop_col27 = coop_it;\n  goto L_v_tile_reduce_col_body_7_n0;" in src
    assert "v_v38 = &(v_v3[v_reduce_idx32][coop_k]);" in src
    assert "float v_v3_storage[64][1];" in src
    image, _ = hip.llir_compile(llir_shapes.col_reduce(20, 300, False), (1, 1, 300))
    assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


def test_tiles_carried_through_a_loop():
    """A tile carried through the K-tile loop is a pointer block parameter
    (`ptr addrspace(5)`, no pointee in the printed form): it takes the tile
    type from its geps or from the alloca passed to it, and is declared as
    the backends' tile pointer.  The fused MMA passes the same tile back (the
    parameter is that alloca); the unfused one passes its result tile."""
    fused = hip.llir_to_hip(llir_shapes.fused_mma_loop(32, 32, 8), (2, 32, 32))
    assert "__launch_bounds__(1024)" in fused and "v_acc" not in fused
    unfused = hip.llir_to_hip(llir_shapes.mma_k_loop(32, 32, 8), (2, 32, 32))
    assert "float (*v_acc29)[32];" in unfused
    assert "v_v93 = &(v_acc29[v_loop_row74][v_loop_col76]);" in unfused
    for t, plan in ((llir_shapes.fused_mma_loop(32, 32, 8), (2, 32, 32)),
                    (llir_shapes.mma_k_loop(32, 32, 8), (2, 32, 32)),
                    (llir_shapes.mma_k_loop(4, 4, 2), (2, 4, 4))):
        image, _ = hip.llir_compile(t, plan)
        assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


MEMCPY_LLIR = """define void @cp(ptr addrspace(1) %x, ptr addrspace(1) %y, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %x [rank=1, shape_offset=0, elem=f32]
  ; sile.param %y [rank=1, shape_offset=1, elem=f32]
  ; sile.param %__sile_shapes [elem=i64]
bb0:
  %pid = call i32 @llvm.nvvm.ctaid.x()
  %t = alloca [1 x [4 x f32]], addrspace(5)
  %off = mul %pid, 4
  %src = getelementptr f32, ptr addrspace(1) %x, i64 %off
  %dst = getelementptr [1 x [4 x f32]], ptr addrspace(5) %t, i64 0, i64 0
  call void @llvm.memcpy.inline(ptr addrspace(5) %dst, ptr addrspace(1) %src, i64 16, i1 false)
  %d2 = getelementptr f32, ptr addrspace(1) %y, i64 %off
  call void @llvm.memcpy.inline(ptr addrspace(1) %d2, ptr addrspace(5) %dst, i64 16, i1 false)
  ret void
}
"""


def test_memcpy_between_buffers_and_tiles():
    """`llvm.memcpy.inline` as the reference prints it (print.rs:209-216: dst,
    src, a byte count, and a volatile flag the C targets ignore) between a
    global buffer and a private tile: `__builtin_memcpy`, compiled."""
    src = hip.llir_to_hip(MEMCPY_LLIR, None)
    assert "__builtin_memcpy(v_dst, v_src, (16LL));" in src
    assert "__builtin_memcpy(v_d2, v_dst, (16LL));" in src
    image, _ = hip.llir_compile(MEMCPY_LLIR, None)
    assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")


# every binary op, compare predicate, cast and select the printed form has
# (crates/sile-llvm-ir/src/print.rs:217-247), on a = 7.75, b = -2.5; the C
# targets' semantics (emit.rs:112-177): casts are C conversions, `sdiv`
# truncates, `and` / `or` are bitwise
OPS_LLIR = """define void @ops(ptr addrspace(1) %x, ptr addrspace(1) %o, ptr addrspace(4) %__sile_shapes) {
  ; sile.param %x [rank=1, shape_offset=0, elem=f32]
  ; sile.param %o [rank=1, shape_offset=1, elem=f32]
  ; sile.param %__sile_shapes [elem=i64]
bb0:
  %pa = getelementptr f32, ptr addrspace(1) %x, i64 0
  %a = load f32, ptr addrspace(1) %pa
  %pb = getelementptr f32, ptr addrspace(1) %x, i64 1
  %b = load f32, ptr addrspace(1) %pb
  %fs = fsub %a, %b
  %fm = fmul %a, %b
  %fd = fdiv %a, %b
  %ia = fptosi %a to i64
  %ib = fptosi %b to i64
  %q = sdiv %ia, %ib
  %d = sub %ia, %ib
  %m = mul %ia, %ib
  %an = and %ia, %ib
  %or = or %ia, %ib
  %c1 = icmp slt %ib, %ia
  %c2 = icmp sle %ia, %ia
  %c3 = icmp sgt %ib, %ia
  %c4 = icmp sge %ia, %ib
  %c5 = icmp eq %q, -3
  %c6 = icmp ne %q, -3
  %f1 = fcmp olt %b, %a
  %f2 = fcmp ole %a, %a
  %f3 = fcmp oge %b, %a
  %cc = and %c1, %c3
  %co = or %c1, %c3
  %sel = select i1 %c3, f32 %a, f32 %b
  br label %out ; args(%fs, %fm, %fd, %q, %d, %m, %an, %or, %c1, %c2, %c3, %c4, %c5, %c6, %f1, %f2, %f3, %cc, %co, %sel)
out:
  ; args(%v0: f32, %v1: f32, %v2: f32, %v3: i64, %v4: i64, %v5: i64, %v6: i64, %v7: i64, %v8: i1, %v9: i1, %v10: i1, %v11: i1, %v12: i1, %v13: i1, %v14: i1, %v15: i1, %v16: i1, %v17: i1, %v18: i1, %v19: f32)
OUT_STORES
  ret void
}
"""


def ops_llir():
    lines = []
    for k in range(20):
        v = f"%v{k}"
        if 3 <= k <= 7:
            lines.append(f"  %w{k} = sitofp {v} to f32")
            v = f"%w{k}"
        elif 8 <= k <= 18:
            lines.append(f"  %z{k} = zext {v} to i64")
            lines.append(f"  %w{k} = sitofp %z{k} to f32")
            v = f"%w{k}"
        lines.append(f"  %p{k} = getelementptr f32, ptr addrspace(1) %o, i64 {k}")
        lines.append(f"  store f32 {v}, ptr addrspace(1) %p{k}")
    return OPS_LLIR.replace("OUT_STORES\n", "\n".join(lines) + "\n")


OPS_EXPECTED = [10.25, 7.75 * -2.5, 7.75 / -2.5, -3, 9, -14, 7 & -2, 7 | -2,
                1, 1, 0, 1, 1, 0, 1, 1, 0, 0, 1, -2.5]


def test_every_operation_translates():
    src = hip.llir_to_hip(ops_llir(), None)
    for line in ("v_q = v_ia / v_ib;", "v_an = v_ia & v_ib;", "v_or = v_ia | v_ib;",
                 "v_c2 = v_ia <= v_ia;", "v_c4 = v_ia >= v_ib;", "v_c5 = v_q == (-3LL);",
                 "v_c6 = v_q != (-3LL);", "v_f3 = v_b >= v_a;", "v_ia = v_a;",
                 "v_sel = (v_c3) ? (v_a) : (v_b);"):
        assert line in src, line
    image, _ = hip.llir_compile(ops_llir(), None)
    assert image[:4] == b"\x7fELF" or image.startswith(b"__CLANG_OFFLOAD_BUNDLE__")
