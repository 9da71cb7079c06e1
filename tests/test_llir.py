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
    assert "float v_tile_storage[2][8];" in sm and "&(v_tile[(0LL)][v_r][v_e])" in sm
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
    body = src[src.index("L_v_body:"):src.index("L_v_done:")]
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
