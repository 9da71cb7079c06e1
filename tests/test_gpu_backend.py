"""GPU: the reference's own backend tests, run through HipBackend.execute_llir
(sile_amd.backend) the way `KernelLauncher::apply` drives a backend
(crates/sile/src/kernel_launcher.rs:55-72): host tensors in, the kernel's
LLIR (and Tile IR) and grid, only the Output parameters copied back.  Each
kernel runs through the router (Tile IR given) and through generated code
(LLIR only).  Fixtures: tests/golden/reference_fixtures.json."""
import json
import os

import numpy as np
import pytest

from sile_amd import _abi
from sile_amd.backend import HipBackend, LaunchConfig, ParamKind
from tests import tile_ir_text as T
from tests.helpers import say
from tests.test_llir import PLANS, text

pytestmark = pytest.mark.gpu

IN, OUT = ParamKind.INPUT, ParamKind.OUTPUT
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


@pytest.fixture(scope="module")
def fx():
    with open(os.path.join(GOLDEN, "reference_fixtures.json")) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def backend(hip):
    b = HipBackend(0)
    yield b
    b.close()


def _tir(name):
    with open(os.path.join(GOLDEN, "tile_ir", name)) as f:
        return f.read()


@pytest.mark.parametrize("routed", [True, False])
def test_vec_add(backend, fx, routed):
    """crates/sile/tests/backend_vec_add.rs:11-25: 1 + 2 = 3 elementwise."""
    f = fx["vec_add"]
    say(f"backend vec_add routed={routed}")
    a = np.full(16, f["a_fill"], np.float32)
    b = np.full(16, f["b_fill"], np.float32)
    c = np.zeros(16, np.float32)
    backend.execute_llir(text("vec_add"), [IN, IN, OUT], [a, b, c], LaunchConfig((4, 1, 1)),
                         tile_ir=_tir("vec_add_4.tir") if routed else None,
                         plan=PLANS["vec_add"])
    np.testing.assert_array_equal(c, np.full(16, f["expected_fill"], np.float32))
    assert backend.last_route == _abi.ROUTE_NONE   # no hand-written pattern: generated code


@pytest.mark.parametrize("routed", [True, False])
def test_matmul(backend, fx, routed):
    """crates/sile/tests/backend_matmul.rs:21-72: the 4x4 integer GEMM, exact."""
    f = fx["matmul_4x4"]
    say(f"backend matmul routed={routed}")
    a = np.array(f["a"]["data"], np.float32).reshape(f["a"]["shape"])
    b = np.array(f["b"]["data"], np.float32).reshape(f["b"]["shape"])
    c = np.zeros((4, 4), np.float32)
    backend.execute_llir(text("matmul"), [IN, IN, OUT], [a, b, c], LaunchConfig(tuple(f["grid"])),
                         tile_ir=_tir("matmul_2x2x2.tir") if routed else None,
                         plan=PLANS["matmul"])
    np.testing.assert_array_equal(c.ravel(), np.array(f["expected"], np.float32))
    assert backend.last_route == (_abi.ROUTE_MATMUL if routed else _abi.ROUTE_NONE)


@pytest.mark.parametrize("routed", [True, False])
def test_softmax(backend, fx, routed):
    """crates/sile/tests/backend_softmax.rs:17-38: every row sums to 1."""
    f = fx["softmax_4x8"]
    say(f"backend softmax routed={routed}")
    x = np.array(f["x"]["data"], np.float32).reshape(f["x"]["shape"])
    x0 = x.copy()
    y = np.zeros_like(x)
    backend.execute_llir(text("softmax"), [IN, OUT], [x, y], LaunchConfig(tuple(f["grid"])),
                         tile_ir=_tir("softmax_2x8.tir") if routed else None,
                         plan=PLANS["softmax"])
    np.testing.assert_allclose(y.sum(axis=1), f["expected_row_sum"], atol=f["tolerance_abs"])
    np.testing.assert_array_equal(x, x0)
    assert backend.last_route == (_abi.ROUTE_SOFTMAX_ROWS if routed else _abi.ROUTE_NONE)


@pytest.mark.parametrize("routed", [True, False])
def test_parallel_reduce(backend, fx, routed):
    """crates/sile/tests/backend_parallel_reduce.rs:11-29: 100000 ones sum to
    100000 (tile 1000 routed; the generated kernel's LLIR has tile 16)."""
    f = fx["parallel_reduce_ones"]
    say(f"backend parallel_reduce routed={routed}")
    x = np.full(f["a"]["shape"], f["a"]["fill"], np.float32)
    out = np.zeros(1, np.float32)
    if routed:
        backend.execute_llir(text("parallel_reduce"), [IN, OUT], [x, out],
                             LaunchConfig(tuple(f["grid"])), tile_ir=_tir("parallel_reduce_1000.tir"))
        assert backend.last_route == _abi.ROUTE_ATOMIC_REDUCE
    else:
        backend.execute_llir(text("parallel_reduce"), [IN, OUT], [x, out],
                             LaunchConfig((x.size // 16, 1, 1)))
        assert backend.last_route == _abi.ROUTE_NONE
    assert abs(out[0] - f["expected"]) <= f["tolerance_abs"]


def test_relu(backend, fx):
    """crates/sile/tests/llvm_ir_cpu_runtime.rs:105-141: relu in place (the
    one parameter is the output)."""
    f = fx["relu_8"]
    say("backend relu")
    x = np.array(f["x"], np.float32)
    backend.execute_llir(text("relu"), [OUT], [x], LaunchConfig((1, 1, 1)), plan=PLANS["relu"])
    np.testing.assert_array_equal(x, np.array(f["expected"], np.float32))


def test_only_outputs_are_copied_back(backend, fx):
    """As MetalBackend (crates/sile-backend/src/metal/mod.rs:160-169): the
    kernel writes C on the device, but C marked Input, or past the end of
    param_kinds, stays as the host had it."""
    f = fx["matmul_4x4"]
    say("backend copy-back")
    a = np.array(f["a"]["data"], np.float32).reshape(f["a"]["shape"])
    b = np.array(f["b"]["data"], np.float32).reshape(f["b"]["shape"])
    for kinds in ([IN, IN, IN], [IN, IN]):
        c = np.full((4, 4), 7.0, np.float32)
        backend.execute_llir(text("matmul"), kinds, [a, b, c], LaunchConfig(tuple(f["grid"])),
                             tile_ir=_tir("matmul_2x2x2.tir"))
        np.testing.assert_array_equal(c, np.full((4, 4), 7.0, np.float32))


def test_generated_kernels_are_kept(backend):
    """A second call with the same LLIR reuses the compiled code object."""
    say("backend kernel cache")
    n = len(backend._kernels)
    for _ in range(2):
        y = np.zeros(8, np.float32)
        backend.execute_llir(text("relu"), [OUT], [y], (1, 1, 1), plan=PLANS["relu"])
    assert len(backend._kernels) <= n + 1
