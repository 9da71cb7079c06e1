"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/sile_hip.h declares, and rejects bad arguments on the host before any
device work (no GPU needed)."""
import os
import re
import subprocess

import pytest

from sile_amd import _abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sile_hip.h")


def declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sile_hip_\w+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ["sile_hip_init", "sile_hip_malloc", "sile_hip_module_load", "sile_hip_launch_tiles",
                 "sile_hip_kernel_matmul", "sile_hip_kernel_softmax",
                 "sile_hip_kernel_parallel_reduce", "sile_hip_gemm", "sile_hip_softmax_rows",
                 "sile_hip_reduce_rows", "sile_hip_flash_attn_fwd", "sile_hip_last_error"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    declared = set(declared_functions())
    assert declared <= exported, sorted(declared - exported)
    # nothing but the C ABI leaks out of the library
    assert all(name.startswith("sile_hip_") for name in exported), sorted(exported)
    # and the ctypes binding covers the same set
    assert declared == set(_abi.SIGNATURES), sorted(declared ^ set(_abi.SIGNATURES))


def test_integration_binding_declares_every_function():
    """The Rust FFI block of the integration guide names exactly the functions
    the header declares, so a maintainer copying it binds the whole ABI."""
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    block = text[text.index("## 3. FFI declarations"):text.index("## 4.")]
    bound = set(re.findall(r"pub fn (sile_hip_\w+)\s*\(", block))
    assert bound == set(declared_functions()), sorted(bound ^ set(declared_functions()))


def test_library_loads_and_reports_version():
    lib = _abi.lib()
    assert b"gfx950" in lib.sile_hip_version()
    assert lib.sile_hip_last_error() is not None


def test_no_gpu_is_unsupported_backend():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    assert _abi.status("sile_hip_init", 0) == 2
    assert "no HIP device" in _abi.last_error()
    n = _abi.device_count()
    assert n == 0


NULL = None


@pytest.mark.parametrize("args,code", [
    # unsupported dtype pair -> UnsupportedBackend
    ((_abi.F16, _abi.BF16, _abi.F32, 256, 256, 64), 2),
    # negative K -> Shape (any K' >= 0 is accepted)
    ((_abi.F8E4M3, _abi.F8E4M3, _abi.BF16, 256, 256, -1), 5),
])
def test_gemm_host_validation(args, code):
    a_t, b_t, c_t, m, n, k = args
    rc = _abi.status("sile_hip_gemm", a_t, b_t, c_t, m, n, k, 16, k, _abi.ROW_MAJOR, 16, k,
                     _abi.COL_MAJOR, 16, n, 1.0, 1.0, 0, NULL)
    assert rc == code, _abi.last_error()


@pytest.mark.parametrize("m,n", [(100, 256), (256, 258), (1, 1)])
def test_small_gemm_shapes_need_aligned_operands(m, n):
    """Shapes below one 256 x 256 tile take the any-shape MFMA kernel, which
    still needs 16-byte aligned A and B rows (checked before any device work)."""
    rc = _abi.status("sile_hip_gemm", _abi.BF16, _abi.BF16, _abi.BF16, m, n, 64, 16, 68,
                     _abi.ROW_MAJOR, 16, 64, _abi.COL_MAJOR, 16, n, 1.0, 1.0, 0, NULL)
    assert rc == 5 and "aligned" in _abi.last_error()


def test_gemm_rejects_unaligned_a_and_unknown_b_layout():
    rc = _abi.status("sile_hip_gemm", _abi.BF16, _abi.BF16, _abi.BF16, 256, 256, 64, 16, 64,
                     _abi.ROW_MAJOR, 16, 256, 7, 16, 256, 1.0, 1.0, 0, NULL)
    assert rc == 2 and "layout" in _abi.last_error()
    # row-major B: A's rows must still be 16-byte aligned (checked before device work)
    rc = _abi.status("sile_hip_gemm", _abi.BF16, _abi.BF16, _abi.BF16, 256, 256, 64, 16, 66,
                     _abi.ROW_MAJOR, 16, 256, _abi.ROW_MAJOR, 16, 256, 1.0, 1.0, 0, NULL)
    assert rc == 5 and "aligned" in _abi.last_error()
    # row-major B narrower than N
    rc = _abi.status("sile_hip_gemm", _abi.BF16, _abi.BF16, _abi.BF16, 256, 256, 64, 16, 64,
                     _abi.ROW_MAJOR, 16, 200, _abi.ROW_MAJOR, 16, 256, 1.0, 1.0, 0, NULL)
    assert rc == 5 and "leading dimension" in _abi.last_error()
    rc = _abi.status("sile_hip_gemm", _abi.BF16, _abi.BF16, _abi.BF16, 256, 256, 64, 18, 64,
                     _abi.ROW_MAJOR, 16, 64, _abi.COL_MAJOR, 16, 256, 1.0, 1.0, 0, NULL)
    assert rc == 5 and "aligned" in _abi.last_error()


@pytest.mark.parametrize("a_t,m,n,tile,splits,needle", [
    (_abi.BF16, 256, 256, 64, 0, "tile must be"),        # not a tile size
    (_abi.BF16, 256, 256, 256, 65, "splits must be"),    # too many ranges
    (_abi.BF16, 256, 256, 0, -1, "splits must be"),
    (_abi.BF16, 200, 512, 256, 0, "256 x 256 tiles need"),   # M below the forced tile
    (_abi.F8E4M3, 200, 512, 256, 0, "256 x 256 tiles need"),
    (_abi.BF16, 512, 258, 128, 0, "128 x 128 tiles need"),   # N not a multiple of 4
])
def test_gemm_tiled_host_validation(a_t, m, n, tile, splits, needle):
    """A forced tile size or split the shape cannot take is a Shape error,
    raised before any device work."""
    c_t = _abi.BF16
    rc = _abi.status("sile_hip_gemm_tiled", a_t, a_t, c_t, m, n, 64, 16, 64, _abi.ROW_MAJOR,
                     16, 64, _abi.COL_MAJOR, 16, n, 1.0, 1.0, 0, tile, splits, NULL)
    assert rc == 5 and needle in _abi.last_error(), _abi.last_error()


def test_dsl_kernel_host_validation():
    bufs = (_abi.ctypes.c_void_p * 3)(16, 16, 16)
    # wrong shape count
    shapes = _abi._i64_array([4, 4, 4, 4])
    assert _abi.status("sile_hip_kernel_matmul", bufs, 4, 1, shapes, 4, 2, 2, 2, NULL) == 5
    # shapes that do not cover the programs' tiles (a has too few rows)
    shapes = _abi._i64_array([2, 4, 4, 4, 4, 4])
    assert _abi.status("sile_hip_kernel_matmul", bufs, 4, 1, shapes, 6, 2, 2, 2, NULL) == 5
    assert "do not cover" in _abi.last_error()
    # BK = 0
    shapes = _abi._i64_array([4, 4, 4, 4, 4, 4])
    assert _abi.status("sile_hip_kernel_matmul", bufs, 4, 1, shapes, 6, 2, 2, 0, NULL) == 5
    # zero programs is a no-op that succeeds without a device
    assert _abi.status("sile_hip_kernel_matmul", bufs, 0, 1, shapes, 6, 2, 2, 2, NULL) == 0
    # parallel_reduce reading past the input
    shapes = _abi._i64_array([1000, 1])
    assert _abi.status("sile_hip_kernel_parallel_reduce", bufs, 11, 1, shapes, 2, 100, NULL, NULL) == 5
    # softmax: y shape that does not cover x's tiles
    shapes = _abi._i64_array([2, 8, 4, 8])
    assert _abi.status("sile_hip_kernel_softmax", bufs, 2, 1, shapes, 4, 2, 8, NULL) == 5


def test_op_host_validation():
    assert _abi.status("sile_hip_softmax_rows", _abi.F8E4M3, _abi.F16, 4, 4, 16, 4, 16, 4, NULL) == 2
    assert _abi.status("sile_hip_softmax_rows", _abi.F16, _abi.F16, 4, 0, 16, 4, 16, 4, NULL) == 5
    assert _abi.status("sile_hip_softmax_rows", _abi.F16, _abi.F16, 4, 8, 16, 4, 16, 8, NULL) == 5
    assert _abi.status("sile_hip_reduce_rows", 7, _abi.F32, 4, 4, 16, 4, 16, NULL) == 2
    assert _abi.status("sile_hip_flash_attn_fwd", _abi.F32, 1, 1, 128, 128, 16, 16, 16, 16,
                       1.0, 1, NULL) == 2
    assert _abi.status("sile_hip_flash_attn_fwd", _abi.F16, 1, 1, 128, 512, 16, 16, 16, 16,
                       1.0, 1, NULL) == 2
    assert _abi.status("sile_hip_launch_tiles", None, None, 0, None, 0, None, 1, NULL) == 3
    # the no-allocation launch: no function, and tables past its 512 entries
    assert _abi.status("sile_hip_launch_tiles_noalloc", None, None, 0, None, 0, None, 1,
                       NULL) == 3
    grid = (_abi.ctypes.c_uint32 * 3)(1, 1, 1)
    rc = _abi.status("sile_hip_launch_tiles_noalloc", 16, _abi._ptr_array([16] * 3), 3,
                     _abi._i64_array([4] * 510), 510, grid, 64, NULL)
    assert rc == 5 and "exceed" in _abi.last_error()


def test_32bit_buffer_range_guards():
    # a 256-row panel of A past 2 GiB (lda = 5M bf16 elements)
    lda = 5_000_000
    rc = _abi.status("sile_hip_gemm", _abi.BF16, _abi.BF16, _abi.BF16, 256, 256, 64, 16, lda,
                     _abi.ROW_MAJOR, 16, 64, _abi.COL_MAJOR, 16, 256, 1.0, 1.0, 0, NULL)
    assert rc == 5 and "panel" in _abi.last_error()
    # one head's K past 2 GiB (S = 2^23, D = 128)
    rc = _abi.status("sile_hip_flash_attn_fwd", _abi.F16, 1, 1, 1 << 23, 128, 16, 16, 16, 16,
                     1.0, 1, NULL)
    assert rc == 5 and "sequence" in _abi.last_error()


def test_graph_capture_rejects_the_null_stream():
    """Capture needs a stream of its own (checked before any HIP call)."""
    rc = _abi.status("sile_hip_graph_begin", NULL)
    assert rc == 5 and "null stream" in _abi.last_error()
    rc = _abi.status("sile_hip_graph_launch", NULL, NULL)
    assert rc == 5 and "graph is NULL" in _abi.last_error()
