"""ctypes binding of libsile_hip.so (the C ABI declared in include/sile_hip.h).

This is the Python caller of the drop-in boundary: tests, bench.py and the
host mirror of sile's backend plugin (sile_amd.backend) go through it.  There is no
fallback: if the library is missing, loading raises immediately.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libsile_hip.so")

# Status codes (include/sile_hip.h) and the sile_core::Error variant each maps
# to (crates/sile-core/src/error.rs:1-13).
SILE_OK = 0
STATUS_NAMES = {
    1: "InvalidDevice",
    2: "UnsupportedBackend",
    3: "Compile",
    4: "Io",
    5: "Shape",
    6: "Runtime",
}

F32, F16, BF16, F8E4M3 = 0, 1, 2, 3
ROW_MAJOR, COL_MAJOR = 0, 1
REDUCE_MAX, REDUCE_SUM = 0, 1

_DTYPE_BYTES = {F32: 4, F16: 2, BF16: 2, F8E4M3: 1}


class SileError(RuntimeError):
    """A failed libsile_hip call: `kind` is the sile_core::Error variant name."""

    def __init__(self, status: int, message: str, call: str):
        self.status = status
        self.kind = STATUS_NAMES.get(status, f"status{status}")
        super().__init__(f"{call}: {self.kind}: {message}")


_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t


class DeviceProps(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("gcn_arch", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("memory_bus_width", ctypes.c_int32),
        ("total_global_mem", ctypes.c_int64),
        ("l2_cache_bytes", ctypes.c_int64),
        ("lds_per_block", ctypes.c_int64),
    ]


ROUTE_NONE, ROUTE_MATMUL, ROUTE_SOFTMAX_ROWS, ROUTE_SOFTMAX_TILES, ROUTE_REDUCE_ROWS, \
    ROUTE_ATOMIC_REDUCE, ROUTE_ATTENTION, ROUTE_MATVEC = range(8)
ROUTE_NAMES = {ROUTE_NONE: "none", ROUTE_MATMUL: "matmul", ROUTE_SOFTMAX_ROWS: "softmax_rows",
               ROUTE_SOFTMAX_TILES: "softmax_tiles", ROUTE_REDUCE_ROWS: "reduce_rows",
               ROUTE_ATOMIC_REDUCE: "atomic_reduce", ROUTE_ATTENTION: "attention",
               ROUTE_MATVEC: "matvec"}


class Route(ctypes.Structure):
    """sile_hip_route: the kernel the Tile IR router picked for one launch."""
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("reduce_op", ctypes.c_int32),
        ("buffer", ctypes.c_int32 * 4),
        ("shape_offset", ctypes.c_int32 * 4),
        ("rank", ctypes.c_int32 * 4),
        ("num_buffers", ctypes.c_int32),
        ("seed_from_tile", ctypes.c_int32),
        ("seed_value", ctypes.c_float),
        ("attn_scale", ctypes.c_float),
        ("attn_m0", ctypes.c_float),
        ("num_shapes", ctypes.c_int64),
        ("operand_shapes", ctypes.c_int64 * 8),
        ("num_threadgroups", ctypes.c_int64),
        ("tile_m", ctypes.c_int64),
        ("tile_n", ctypes.c_int64),
        ("tile_k", ctypes.c_int64),
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("reason", ctypes.c_char * 512),
    ]

    @property
    def name(self) -> str:
        return ROUTE_NAMES.get(self.kind, f"kind{self.kind}")


# name -> argtypes (every function returns int status unless listed in _RESTYPE)
SIGNATURES = {
    "sile_hip_init": [_I32],
    "sile_hip_device_count": [ctypes.POINTER(_I32)],
    "sile_hip_device_info": [_I32, ctypes.POINTER(DeviceProps)],
    "sile_hip_device_synchronize": [],
    "sile_hip_last_error": [],
    "sile_hip_version": [],
    "sile_hip_malloc": [ctypes.POINTER(_P), _SZ],
    "sile_hip_free": [_P],
    "sile_hip_memcpy_htod": [_P, _P, _SZ],
    "sile_hip_memcpy_dtoh": [_P, _P, _SZ],
    "sile_hip_memcpy_dtod": [_P, _P, _SZ],
    "sile_hip_memset": [_P, _I32, _SZ],
    "sile_hip_stream_create": [ctypes.POINTER(_P)],
    "sile_hip_stream_destroy": [_P],
    "sile_hip_stream_synchronize": [_P],
    "sile_hip_event_create": [ctypes.POINTER(_P)],
    "sile_hip_event_destroy": [_P],
    "sile_hip_event_record": [_P, _P],
    "sile_hip_event_synchronize": [_P],
    "sile_hip_event_elapsed_ms": [ctypes.POINTER(_F32), _P, _P],
    "sile_hip_module_load": [_P, _SZ, ctypes.POINTER(_P)],
    "sile_hip_module_unload": [_P],
    "sile_hip_module_get": [_P, ctypes.c_char_p, ctypes.POINTER(_P)],
    "sile_hip_launch_tiles": [_P, _P, _I64, _P, _I64, _P, ctypes.c_uint32, _P],
    "sile_hip_launch_tiles_noalloc": [_P, _P, _I64, _P, _I64, _P, ctypes.c_uint32, _P],
    "sile_hip_llir_to_hip": [ctypes.c_char_p, _I64, _I64, _I64, _P, _SZ, ctypes.POINTER(_SZ)],
    "sile_hip_llir_compile": [ctypes.c_char_p, _I64, _I64, _I64, ctypes.POINTER(_P),
                              ctypes.POINTER(_SZ), _P, _SZ],
    "sile_hip_llir_free_code": [_P],
    "sile_hip_launch_llir": [_P, _P, _I64, _P, _I64, _P, _P],
    "sile_hip_kernel_matmul": [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _P],
    "sile_hip_kernel_softmax": [_P, _I64, _I64, _P, _I64, _I64, _I64, _P],
    "sile_hip_kernel_parallel_reduce": [_P, _I64, _I64, _P, _I64, _I64, _P, _P],
    "sile_hip_gemm": [_I32, _I32, _I32, _I64, _I64, _I64, _P, _I64, _I32, _P, _I64, _I32, _P,
                      _I64, _F32, _F32, _I64, _P],
    "sile_hip_graph_begin": [_P],
    "sile_hip_graph_end": [_P, ctypes.POINTER(_P)],
    "sile_hip_graph_launch": [_P, _P],
    "sile_hip_graph_destroy": [_P],
    "sile_hip_gemm_tiled": [_I32, _I32, _I32, _I64, _I64, _I64, _P, _I64, _I32, _P, _I64, _I32,
                            _P, _I64, _F32, _F32, _I64, _I32, _I32, _P],
    "sile_hip_mma_f32": [_I64, _I64, _I64, _P, _I64, _P, _I64, _I32, _P, _I64, _F32, _P, _I64, _I64,
                         _P],
    "sile_hip_softmax_rows": [_I32, _I32, _I64, _I64, _P, _I64, _P, _I64, _P],
    "sile_hip_reduce_rows": [_I32, _I32, _I64, _I64, _P, _I64, _P, _P],
    "sile_hip_reduce_rows_fused_sum": [_I64, _I64, _P, _I64, _I64, _P, _P],
    "sile_hip_copy_rows": [_I64, _I64, _P, _I64, _P, _I64, _P],
    "sile_hip_fill_rows": [_I32, _I64, _I64, _F32, _P, _I64, _P],
    "sile_hip_flash_attn_fwd": [_I32, _I64, _I64, _I64, _I64, _P, _P, _P, _P, _F32, _I32, _P],
    "sile_hip_attention_f32_kt": [_I64, _I64, _I64, _P, _I64, _P, _I64, _P, _I64, _P, _I64, _F32,
                                  _F32, _P],
    "sile_hip_matvec_f32": [_I64, _I64, _I64, _P, _I64, _P, _F32, _P, _P],
    "sile_hip_tile_ir_route": [ctypes.c_char_p, _P, _I64, _I64, ctypes.POINTER(Route)],
    "sile_hip_tile_ir_launch": [ctypes.POINTER(Route), _P, _I64, _P, _I64, _I64, _P],
}
_RESTYPE = {"sile_hip_last_error": ctypes.c_char_p, "sile_hip_version": ctypes.c_char_p,
            "sile_hip_llir_free_code": None}

_lib = None


def lib() -> ctypes.CDLL:
    """Loads libsile_hip.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m sile_amd.build` "
                "(the HIP path has no fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, argtypes in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = argtypes
            fn.restype = _RESTYPE.get(name, ctypes.c_int)
        _lib = L
    return _lib


def last_error() -> str:
    return lib().sile_hip_last_error().decode()


def call(name: str, *args) -> None:
    """Calls a status-returning entry point; raises SileError on failure."""
    rc = getattr(lib(), name)(*args)
    if rc != SILE_OK:
        raise SileError(rc, last_error(), name)


def status(name: str, *args) -> int:
    """Calls an entry point and returns its raw status (for error-path tests)."""
    return getattr(lib(), name)(*args)


# ---------------------------------------------------------------------------
# device, memory, streams, events
# ---------------------------------------------------------------------------

def init(ordinal: int = 0) -> None:
    call("sile_hip_init", ordinal)


def device_count() -> int:
    n = _I32(0)
    call("sile_hip_device_count", ctypes.byref(n))
    return n.value


def device_info(ordinal: int = 0) -> dict:
    p = DeviceProps()
    call("sile_hip_device_info", ordinal, ctypes.byref(p))
    return {
        "name": p.name.decode(), "gcn_arch": p.gcn_arch.decode(),
        "compute_units": p.compute_units, "clock_khz": p.clock_khz,
        "memory_clock_khz": p.memory_clock_khz, "memory_bus_width": p.memory_bus_width,
        "total_global_mem": p.total_global_mem, "l2_cache_bytes": p.l2_cache_bytes,
        "lds_per_block": p.lds_per_block,
    }


def synchronize() -> None:
    call("sile_hip_device_synchronize")


class DeviceBuffer:
    """An HBM allocation from sile_hip_malloc, freed on close()/GC."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = _P()
        call("sile_hip_malloc", ctypes.byref(p), self.nbytes)
        self.ptr = p.value or 0

    @classmethod
    def from_array(cls, arr: np.ndarray) -> "DeviceBuffer":
        arr = np.ascontiguousarray(arr)
        buf = cls(arr.nbytes)
        buf.upload(arr)
        return buf

    def upload(self, arr: np.ndarray) -> None:
        arr = np.ascontiguousarray(arr)
        assert arr.nbytes <= self.nbytes
        call("sile_hip_memcpy_htod", self.ptr, arr.ctypes.data, arr.nbytes)

    def download(self, dtype, shape) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        call("sile_hip_memcpy_dtoh", out.ctypes.data, self.ptr, out.nbytes)
        return out

    def fill_bytes(self, value: int) -> None:
        call("sile_hip_memset", self.ptr, value, self.nbytes)

    def close(self) -> None:
        if self.ptr and _lib is not None:
            call("sile_hip_free", self.ptr)
        self.ptr = 0

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Stream:
    def __init__(self):
        p = _P()
        call("sile_hip_stream_create", ctypes.byref(p))
        self.handle = p.value

    def synchronize(self) -> None:
        call("sile_hip_stream_synchronize", self.handle)

    def close(self) -> None:
        if self.handle:
            call("sile_hip_stream_destroy", self.handle)
            self.handle = None


class Graph:
    """A captured sequence of op calls on `stream` (sile_hip_graph_begin /
    end), replayed by launch()."""

    def __init__(self, stream: "Stream"):
        self.stream = stream
        self.handle = None

    def __enter__(self):
        call("sile_hip_graph_begin", self.stream.handle)
        return self

    def __exit__(self, exc_type, exc, tb):
        p = _P()
        rc = lib().sile_hip_graph_end(self.stream.handle, ctypes.byref(p))
        if exc_type is None:
            if rc != SILE_OK:
                raise SileError(rc, last_error(), "sile_hip_graph_end")
            self.handle = p.value
        elif rc == SILE_OK and p.value:
            # the body raised: capture ended cleanly, but the graph is not kept
            lib().sile_hip_graph_destroy(p)
        return False

    def launch(self, stream: "Stream | None" = None) -> None:
        call("sile_hip_graph_launch", self.handle, (stream or self.stream).handle)

    def close(self) -> None:
        if self.handle:
            call("sile_hip_graph_destroy", self.handle)
            self.handle = None


class Event:
    def __init__(self):
        p = _P()
        call("sile_hip_event_create", ctypes.byref(p))
        self.handle = p.value

    def record(self, stream: "Stream | None" = None) -> None:
        call("sile_hip_event_record", self.handle, stream.handle if stream else None)

    def synchronize(self) -> None:
        call("sile_hip_event_synchronize", self.handle)

    def elapsed_ms(self, end: "Event") -> float:
        ms = _F32(0.0)
        call("sile_hip_event_elapsed_ms", ctypes.byref(ms), self.handle, end.handle)
        return float(ms.value)

    def close(self) -> None:
        if self.handle:
            call("sile_hip_event_destroy", self.handle)
            self.handle = None


def _sh(stream) -> "int | None":
    return None if stream is None else stream.handle


def _ptr_array(ptrs):
    return (ctypes.c_void_p * len(ptrs))(*ptrs)


def _i64_array(vals):
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


# ---------------------------------------------------------------------------
# DSL kernels with the sile_kernel_<name> ABI
# ---------------------------------------------------------------------------

def kernel_matmul(bufs, num_threadgroups, shapes, bm, bn, bk, stream=None, threads_per_group=1):
    call("sile_hip_kernel_matmul", _ptr_array(bufs), num_threadgroups, threads_per_group,
         _i64_array(shapes), len(shapes), bm, bn, bk, _sh(stream))


def kernel_softmax(bufs, num_threadgroups, shapes, bm, bn, stream=None, threads_per_group=1):
    call("sile_hip_kernel_softmax", _ptr_array(bufs), num_threadgroups, threads_per_group,
         _i64_array(shapes), len(shapes), bm, bn, _sh(stream))


def kernel_parallel_reduce(bufs, num_threadgroups, shapes, tile, partials=0, stream=None,
                           threads_per_group=1):
    call("sile_hip_kernel_parallel_reduce", _ptr_array(bufs), num_threadgroups,
         threads_per_group, _i64_array(shapes), len(shapes), tile, partials or None, _sh(stream))


# ---------------------------------------------------------------------------
# generic code generation for LLIR text
# ---------------------------------------------------------------------------

def _plan(plan):
    """(output_param, rows, cols) or None (the CPU wrapper's fallbacks)."""
    return (-1, 0, 0) if plan is None else tuple(int(x) for x in plan)


def llir_to_hip(text: str, plan=None) -> str:
    """The HIP C++ that sile_hip_llir_compile builds from `text`."""
    p = _plan(plan)
    n = _SZ(0)
    call("sile_hip_llir_to_hip", text.encode(), *p, None, 0, ctypes.byref(n))
    buf = ctypes.create_string_buffer(n.value + 1)
    call("sile_hip_llir_to_hip", text.encode(), *p, ctypes.cast(buf, _P), n.value + 1, None)
    return buf.value.decode()


def llir_compile(text: str, plan=None) -> "tuple[bytes, str]":
    """gfx950 code object and kernel name for `text` (hiprtc; no GPU needed)."""
    p = _plan(plan)
    code, size = _P(), _SZ(0)
    name = ctypes.create_string_buffer(256)
    call("sile_hip_llir_compile", text.encode(), *p, ctypes.byref(code), ctypes.byref(size),
         ctypes.cast(name, _P), 256)
    try:
        image = ctypes.string_at(code.value, size.value)
    finally:
        lib().sile_hip_llir_free_code(code)
    return image, name.value.decode()


class LlirKernel:
    """A kernel generated from LLIR text, loaded on the current device."""

    def __init__(self, text: str, plan=None):
        self.image, self.name = llir_compile(text, plan)
        self.module, self.fn = _P(), _P()
        call("sile_hip_module_load", self.image, len(self.image), ctypes.byref(self.module))
        call("sile_hip_module_get", self.module, self.name.encode(), ctypes.byref(self.fn))

    def __call__(self, bufs, shapes, grid, stream=None):
        g = (ctypes.c_uint32 * 3)(*grid)
        call("sile_hip_launch_llir", self.fn, _ptr_array(bufs), len(bufs), _i64_array(shapes),
             len(shapes), g, _sh(stream))

    def close(self):
        if self.module.value and _lib is not None:
            call("sile_hip_module_unload", self.module)
            self.module = _P()


# ---------------------------------------------------------------------------
# Tile IR pattern router
# ---------------------------------------------------------------------------

def tile_ir_route(text: str, shapes, num_threadgroups: int) -> Route:
    """The kernel the router picks for `text` launched with `num_threadgroups`
    programs over buffers of `shapes` (no GPU needed)."""
    r = Route()
    call("sile_hip_tile_ir_route", text.encode(), _i64_array(shapes), len(shapes),
         num_threadgroups, ctypes.byref(r))
    return r


def tile_ir_launch(route: Route, bufs, shapes, num_threadgroups: int, stream=None) -> None:
    call("sile_hip_tile_ir_launch", ctypes.byref(route), _ptr_array(bufs), len(bufs),
         _i64_array(shapes), len(shapes), num_threadgroups, _sh(stream))


# ---------------------------------------------------------------------------
# op entry points (asynchronous on the stream)
# ---------------------------------------------------------------------------

def gemm(a_type, b_type, c_type, m, n, k, a, lda, a_layout, b, ldb, b_layout, c, ldc,
         scale_a=1.0, scale_b=1.0, bk=0, stream=None, tile=0, splits=0):
    """sile_hip_gemm; tile / splits other than 0 force the tile size and the
    K split (sile_hip_gemm_tiled)."""
    if tile or splits:
        call("sile_hip_gemm_tiled", a_type, b_type, c_type, m, n, k, a, lda, a_layout, b, ldb,
             b_layout, c, ldc, scale_a, scale_b, bk, tile, splits, _sh(stream))
    else:
        call("sile_hip_gemm", a_type, b_type, c_type, m, n, k, a, lda, a_layout, b, ldb,
             b_layout, c, ldc, scale_a, scale_b, bk, _sh(stream))


def mma_f32(m, n, k, a, lda, b, ldb, b_layout, acc, ld_acc, acc_value, c, ldc, bk=0, stream=None):
    call("sile_hip_mma_f32", m, n, k, a, lda, b, ldb, b_layout, acc, ld_acc, acc_value, c, ldc, bk,
         _sh(stream))


def softmax_rows(in_type, out_type, rows, cols, x, ldx, y, ldy, stream=None):
    call("sile_hip_softmax_rows", in_type, out_type, rows, cols, x, ldx, y, ldy, _sh(stream))


def reduce_rows(op, in_type, rows, cols, x, ldx, out, stream=None):
    call("sile_hip_reduce_rows", op, in_type, rows, cols, x, ldx, out, _sh(stream))


def reduce_rows_fused_sum(rows, cols, x, ldx, x_len, out, stream=None):
    call("sile_hip_reduce_rows_fused_sum", rows, cols, x, ldx, x_len, out, _sh(stream))


def fill_rows(dtype, rows, cols, value, y, ldy, stream=None):
    call("sile_hip_fill_rows", dtype, rows, cols, value, y, ldy, _sh(stream))


def copy_rows(rows, row_bytes, x, ldx_bytes, y, ldy_bytes, stream=None):
    call("sile_hip_copy_rows", rows, row_bytes, x, ldx_bytes, y, ldy_bytes, _sh(stream))


def flash_attn_fwd(dtype, batch, heads, seq_len, head_dim, q, k, v, o, scale, causal=True,
                   stream=None):
    call("sile_hip_flash_attn_fwd", dtype, batch, heads, seq_len, head_dim, q, k, v, o, scale,
         1 if causal else 0, _sh(stream))


def attention_f32_kt(n_q, n_k, head_dim, q, ldq, kt, ldkt, v, ldv, o, ldo, scale, m0,
                     stream=None):
    call("sile_hip_attention_f32_kt", n_q, n_k, head_dim, q, ldq, kt, ldkt, v, ldv, o, ldo, scale,
         m0, _sh(stream))


def matvec_f32(m, k, bk, x, ldx, y, out, seed=0.0, stream=None):
    call("sile_hip_matvec_f32", m, k, bk, x, ldx, y, seed, out, _sh(stream))


def dtype_bytes(t: int) -> int:
    return _DTYPE_BYTES[t]
