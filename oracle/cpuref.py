"""ctypes view of the CPU oracle (oracle/sile_cpuref.c).

TEST INFRASTRUCTURE ONLY: the checker the HIP path is compared against.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module.  Nothing in the product (sile_amd/) may import it.

Every function here is a thin numpy-facing wrapper; the arithmetic lives in
the C file, which cites the reference source it restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SRC = os.path.join(HERE, "sile_cpuref.c")
BUILD_DIR = os.path.join(HERE, "_build")
LIB_PATH = os.path.join(BUILD_DIR, "libsile_cpuref.so")

# The reference compiles its generated C with `cc -shared -fPIC -O2 -fopenmp -lm`
# and no -march (crates/sile-backend/src/cpu/mod.rs:83); -ffp-contract=off makes
# the absence of FMA contraction explicit.
CFLAGS = ["-shared", "-fPIC", "-O2", "-fopenmp", "-ffp-contract=off", "-Wall"]


def build() -> str:
    """Compile the oracle library in-tree and return its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    tmp = LIB_PATH + ".tmp"
    subprocess.run(["gcc", *CFLAGS, "-o", tmp, SRC, "-lm"], check=True)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


_lib = None

_P = ctypes.c_void_p
_I64 = ctypes.c_int64


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.cpuref_total_tiles.restype = _I64
        L.cpuref_total_tiles.argtypes = [_I64, _P, _I64, _I64]
        L.cpuref_kernel_matmul.argtypes = [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64]
        L.cpuref_kernel_softmax.argtypes = [_P, _I64, _I64, _P, _I64, _I64, _I64]
        L.cpuref_kernel_parallel_reduce.argtypes = [_P, _I64, _I64, _P, _I64, _I64]
        L.cpuref_parallel_reduce_partials.argtypes = [_P, _P, _I64, _I64, _I64]
        L.cpuref_gemm_nt.argtypes = [_P, _P, _P] + [_I64] * 9
        L.cpuref_mma_f32.argtypes = [_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, ctypes.c_int,
                                     _I64, ctypes.c_float, _I64, _I64]
        L.cpuref_reduce_rows.argtypes = [ctypes.c_int, _P, _P, _I64, _I64, _I64, _I64]
        L.cpuref_softmax_rows.argtypes = [_P, _P, _I64, _I64, _I64, _I64]
        L.cpuref_attention_fwd.argtypes = [_P, _P, _P, _P, _I64, _I64, ctypes.c_float,
                                           ctypes.c_int, _I64, _I64]
        L.cpuref_dsl_attention_f32.argtypes = [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64,
                                               _I64, _I64, ctypes.c_float, ctypes.c_float,
                                               _I64, _I64]
        L.cpuref_dsl_matvec_f32.argtypes = [_P, _I64, _P, _P, _I64, _I64, _I64, ctypes.c_float]
        L.cpuref_bf16_from_f32.argtypes = [_P, _P, _I64]
        L.cpuref_f32_from_bf16.argtypes = [_P, _P, _I64]
        L.cpuref_e4m3_encode.argtypes = [_P, _P, _I64, ctypes.c_float]
        L.cpuref_e4m3_decode.argtypes = [_P, _P, _I64, ctypes.c_float]
        L.cpuref_num_threads.restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def num_threads() -> int:
    return int(lib().cpuref_num_threads())


def total_tiles(out_shape, rows: int, cols: int) -> int:
    shp = np.asarray(out_shape, dtype=np.int64)
    return int(lib().cpuref_total_tiles(len(out_shape), _ptr(shp), rows, cols))


def _buffers(*arrays):
    arr = (ctypes.c_void_p * len(arrays))(*[_ptr(a) for a in arrays])
    return arr


def kernel_matmul(a, b, c, grid, bm, bn, bk):
    """sile_kernel_matmul on host arrays; c is updated in place (only the tiles
    a program covers are written, as in the reference)."""
    a, b = _f32(a), _f32(b)
    assert c.dtype == np.float32 and c.flags.c_contiguous
    shapes = np.array([*a.shape, *b.shape, *c.shape], dtype=np.int64)
    n_tg = int(np.prod(grid))
    lib().cpuref_kernel_matmul(_buffers(a, b, c), n_tg, 1, _ptr(shapes), len(shapes), bm, bn, bk)
    return c


def kernel_softmax(x, y, grid, bm, bn):
    x = _f32(x)
    assert y.dtype == np.float32 and y.flags.c_contiguous
    shapes = np.array([*x.shape, *y.shape], dtype=np.int64)
    n_tg = int(np.prod(grid))
    lib().cpuref_kernel_softmax(_buffers(x, y), n_tg, 1, _ptr(shapes), len(shapes), bm, bn)
    return y


def kernel_parallel_reduce(a, out, grid, tile):
    a = _f32(a)
    assert out.dtype == np.float32 and out.flags.c_contiguous
    shapes = np.array([*a.shape, *out.shape], dtype=np.int64)
    n_tg = int(np.prod(grid))
    lib().cpuref_kernel_parallel_reduce(_buffers(a, out), n_tg, 1, _ptr(shapes), len(shapes), tile)
    return out


def parallel_reduce_partials(a, programs, tile):
    """Each program's tile sum over the 1-D buffer a (programs * tile <= a.size)."""
    a = _f32(a)
    assert a.ndim == 1 and programs * tile <= a.size
    out = np.zeros(programs, dtype=np.float32)
    lib().cpuref_parallel_reduce_partials(_ptr(a), _ptr(out), programs, tile, a.size)
    return out


def gemm_nt(a, bt, bk=0, bm=1, row_tile_step=1, out=None):
    """C = A . B with A [M,K] row-major and B given as B^T [N,K] row-major."""
    a, bt = _f32(a), _f32(bt)
    m, k = a.shape
    n = bt.shape[0]
    c = np.zeros((m, n), dtype=np.float32) if out is None else out
    lib().cpuref_gemm_nt(_ptr(a), _ptr(bt), _ptr(c), m, n, k, k, k, n, bk, bm, row_tile_step)
    return c


def mma_f32(a, b, acc=None, acc_value=0.0, bk=0, b_col_major=False, out=None):
    """The seeded tile-MMA chain over a whole [M, N] result: C = fold from
    acc (or the constant acc_value) through A[r][k] * B[k][c] in increasing k.
    b is [K, N] row-major, or [N, K] when b_col_major."""
    a, b = _f32(a), _f32(b)
    m, k = a.shape
    n = b.shape[0] if b_col_major else b.shape[1]
    c = np.zeros((m, n), dtype=np.float32) if out is None else out
    accp, ld_acc = None, 0
    if acc is not None:
        acc = _f32(acc)
        accp, ld_acc = _ptr(acc), acc.shape[1]
    lib().cpuref_mma_f32(_ptr(a), _ptr(b), accp, _ptr(c), m, n, k, k, b.shape[1], int(b_col_major),
                         ld_acc, float(acc_value), c.shape[1], bk)
    return c


REDUCE_MAX, REDUCE_SUM, REDUCE_SUM_VEC4 = 0, 1, 2


def reduce_rows(x, op, cols=None):
    """Reduces the first `cols` columns (default: all) of every row of the
    [rows, ldx] buffer x.  For REDUCE_SUM_VEC4 a window of the reference's
    vec4 loop that runs past a row reads the buffer's next elements, and
    0.0f past the end of x."""
    x = _f32(x)
    rows, ldx = x.shape
    cols = ldx if cols is None else cols
    assert 0 < cols <= ldx
    out = np.zeros(rows, dtype=np.float32)
    lib().cpuref_reduce_rows(op, _ptr(x), _ptr(out), rows, cols, ldx, x.size)
    return out


def softmax_rows(x):
    x = _f32(x)
    rows, cols = x.shape
    y = np.empty_like(x)
    lib().cpuref_softmax_rows(_ptr(x), _ptr(y), rows, cols, cols, cols)
    return y


def attention_fwd(q, k, v, scale, causal=True, q_begin=0, q_end=None, out=None):
    """One (batch, head) slice: q, k, v are [S, D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    s, d = q.shape
    if q_end is None:
        q_end = s
    o = np.zeros((s, d), dtype=np.float32) if out is None else out
    lib().cpuref_attention_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), s, d, float(scale),
                               1 if causal else 0, q_begin, q_end)
    return o


def dsl_matvec_f32(x, y, bk, m=None, k=None, seed=0.0):
    """The matvec program (crates/sile/examples/mlp.rs:26-44) over rows 0..m of
    x [*, ldx] and y; k defaults to x's column count (the loop runs k / bk
    whole tiles).  Returns out [m]."""
    x, y = _f32(x), _f32(y)
    m = x.shape[0] if m is None else m
    k = x.shape[1] if k is None else k
    out = np.zeros(m, dtype=np.float32)
    lib().cpuref_dsl_matvec_f32(_ptr(x), x.shape[1], _ptr(y), _ptr(out), m, k, bk, float(seed))
    return out


def dsl_attention_f32(q, kt, v, bn, scale, m0, d=None, n_q=None, s_k=None):
    """The DSL attention program (K transposed, no mask) over rows 0..n_q of
    q [*, ldq], kt [D, ldkt], v [*, ldv]; keys 0 .. (s_k / bn) * bn, where s_k
    defaults to kt's column count.  Returns o [n_q, d]."""
    q, kt, v = _f32(q), _f32(kt), _f32(v)
    d = kt.shape[0] if d is None else d
    n_q = q.shape[0] if n_q is None else n_q
    s_k = kt.shape[1] if s_k is None else s_k
    o = np.zeros((n_q, d), dtype=np.float32)
    lib().cpuref_dsl_attention_f32(_ptr(q), q.shape[1], _ptr(kt), kt.shape[1], _ptr(v),
                                   v.shape[1], _ptr(o), d, d, s_k, bn, float(scale), float(m0),
                                   0, n_q)
    return o


def bf16_from_f32(x) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().cpuref_bf16_from_f32(_ptr(x), _ptr(out), x.size)
    return out


def f32_from_bf16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    out = np.empty(x.shape, dtype=np.float32)
    lib().cpuref_f32_from_bf16(_ptr(x), _ptr(out), x.size)
    return out


def e4m3_encode(x, scale=1.0) -> np.ndarray:
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint8)
    lib().cpuref_e4m3_encode(_ptr(x), _ptr(out), x.size, float(scale))
    return out


def e4m3_decode(q, scale=1.0) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(q.shape, dtype=np.float32)
    lib().cpuref_e4m3_decode(_ptr(q), _ptr(out), q.size, float(scale))
    return out
