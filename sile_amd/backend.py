"""sile's backend plugin for the HIP device, on the host side.

The reference runs a kernel's LLIR on host tensors through a backend object:
`CpuBackend::execute_llir(func, args, launch, stream)`
(crates/sile-backend/src/cpu/mod.rs:136-145) and
`MetalBackend::execute_llir(func, param_kinds, args, launch, stream)`
(crates/sile-backend/src/metal/mod.rs:65-76, body :104-172).  The Metal one
copies every argument to the device (:117-125), runs one threadgroup per
program, waits for completion (:158) and copies back only the arguments whose
ParamKind is Output (:160-169); an argument past the end of `param_kinds` is
not an output.  `HipBackend.execute_llir` keeps that contract over
libsile_hip:

* arguments are the reference's KernelArg, f32 tensors with a shape
  (crates/sile-core/src/kernel.rs:8-14): here C-contiguous float32 numpy
  arrays; outputs are written back into them in place, as the reference
  writes through `mut_ptr`;
* the launch is LaunchConfig.grid (crates/sile-core/src/kernel.rs:3-6); the
  program count is the product of its three dimensions, as in the CPU
  backend's LLIR mode (cpu/mod.rs:108-112);
* given the kernel's Tile IR as well, the pattern router
  (`sile_hip_tile_ir_route`) picks a hand-written kernel when the IR is one
  of its patterns; otherwise the LLIR is compiled to a gfx950 code object
  (`sile_hip_llir_compile`).  A compiled LLIR is kept for later calls with
  the same text and plan, where the reference compiles on every call;
* the call returns after the device has finished, as `apply` does
  (crates/sile/src/kernel_launcher.rs:55-72);
* failures raise SileError, whose `kind` is the sile_core::Error variant
  (crates/sile-core/src/error.rs:1-13).

There is no CPU fallback: without the library or a device every call fails.
"""
from __future__ import annotations

import enum
from dataclasses import dataclass

import numpy as np

from . import _abi

_CALL = "HipBackend.execute_llir"


class ParamKind(enum.IntEnum):
    """A kernel parameter's role: `&T` is Input, `&mut T` is Output
    (crates/sile-macros/src/frontend/lower.rs:10-14)."""

    INPUT = 0
    OUTPUT = 1


@dataclass(frozen=True)
class LaunchConfig:
    """crates/sile-core/src/kernel.rs:3-6."""

    grid: tuple = (1, 1, 1)


class HipBackend:
    """The HIP counterpart of CpuBackend / MetalBackend on device `ordinal`."""

    def __init__(self, ordinal: int = 0):
        _abi.init(ordinal)
        self._kernels: dict = {}
        # route kind of the last call (sile_route_kind; 0: the LLIR was compiled)
        self.last_route = None

    def execute_llir(self, llir: str, param_kinds, args, launch, stream=None, tile_ir=None,
                     plan=None) -> None:
        """Runs the kernel whose printed LLIR is `llir` (and, when given, whose
        printed Tile IR is `tile_ir`) over `args` with `launch`; copies the
        Output arguments back into their arrays.  `plan` is the LLIR's tile
        plan (output parameter, rows, cols) when it has one."""
        grid = tuple(int(g) for g in (launch.grid if isinstance(launch, LaunchConfig) else launch))
        if len(grid) != 3 or min(grid) < 0:
            raise _abi.SileError(5, f"grid must be three non-negative extents, got {grid}", _CALL)
        for i, a in enumerate(args):
            if not isinstance(a, np.ndarray) or a.dtype != np.float32:
                raise _abi.SileError(2, f"argument {i} is not a float32 tensor (sile's "
                                        "KernelArg holds f32 data)", _CALL)
            if not a.flags.c_contiguous:
                raise _abi.SileError(5, f"argument {i} is not contiguous", _CALL)
        shapes = [int(d) for a in args for d in a.shape]
        programs = grid[0] * grid[1] * grid[2]
        bufs = []
        try:
            for a in args:
                bufs.append(_abi.DeviceBuffer.from_array(a))
            ptrs = [b.ptr for b in bufs]
            route = None
            if tile_ir is not None:
                r = _abi.tile_ir_route(tile_ir, shapes, programs)
                route = r if r.kind != 0 else None
            if route is not None:
                _abi.tile_ir_launch(route, ptrs, shapes, programs, stream)
                self.last_route = route.kind
            else:
                key = (llir, None if plan is None else tuple(plan))
                kernel = self._kernels.get(key)
                if kernel is None:
                    kernel = self._kernels[key] = _abi.LlirKernel(llir, plan)
                kernel(ptrs, shapes, grid, stream)
                self.last_route = 0
            if stream is None:
                _abi.synchronize()
            else:
                stream.synchronize()
            for i, (buf, a) in enumerate(zip(bufs, args)):
                if i < len(param_kinds) and param_kinds[i] == ParamKind.OUTPUT:
                    a[...] = buf.download(np.float32, a.shape)
        finally:
            for b in bufs:
                b.close()

    def close(self) -> None:
        for k in self._kernels.values():
            k.close()
        self._kernels = {}
