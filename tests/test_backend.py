"""CPU-side checks of sile_amd.backend, the host mirror of sile's backend
plugin (no GPU needed): its types, that it fails loudly without a device,
and that it rejects arguments sile's KernelArg cannot hold before any
device work."""
import os

import numpy as np
import pytest

from sile_amd import _abi
from sile_amd.backend import HipBackend, LaunchConfig, ParamKind


def test_param_kinds_and_launch_config():
    assert [int(k) for k in ParamKind] == [0, 1]
    assert LaunchConfig().grid == (1, 1, 1)


def test_no_device_fails_loudly():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(_abi.SileError) as e:
        HipBackend()
    assert e.value.kind == "UnsupportedBackend"


def _unbound():
    # the argument checks run before any device call
    return HipBackend.__new__(HipBackend)


@pytest.mark.parametrize("arg,kind", [(np.zeros(4, np.float64), "UnsupportedBackend"),
                                      (np.zeros(4, np.float16), "UnsupportedBackend"),
                                      ([0.0] * 4, "UnsupportedBackend"),
                                      (np.zeros((4, 4), np.float32)[:, ::2], "Shape")])
def test_rejects_what_kernel_arg_cannot_hold(arg, kind):
    with pytest.raises(_abi.SileError) as e:
        _unbound().execute_llir("", [ParamKind.OUTPUT], [arg], LaunchConfig((1, 1, 1)))
    assert e.value.kind == kind


@pytest.mark.parametrize("grid", [(1, 1), (1, -1, 1), (1, 1, 1, 1)])
def test_rejects_bad_grids(grid):
    with pytest.raises(_abi.SileError) as e:
        _unbound().execute_llir("", [], [], grid)
    assert e.value.kind == "Shape"
